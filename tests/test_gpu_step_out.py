"""GPU parity of attn.linearOut with the step's merge folded in (g4_attn_step_run_out): after the
attention pass of a prepared step, one launch merges every entry's partial records, writes attnOut
and multiplies it by the entry's o_proj weight (src/engine.ts:2096 after the attention block of
:2056-2094).

Bars: attnOut and the projected rows are bit-identical to the two-launch path it replaces
(g4_attn_step_run_merge, then g4_linear_f16 over attnOut), the rows are bit-identical to the
oracle's matmul_quant.wgsl restatement over that attnOut, and attnOut is within max-abs 2e-3 of the
oracle's reference chain. Cases cover the fused form (entries of 2..8 parts, group 8 and 4,
head_dim 256 and 512, several entries with mixed part counts) and the fallback forms (one part,
more than 8 parts, two kv heads).
"""
import numpy as np
import pytest
import torch

from conftest import announce
from g4attn import ops
from oracle import oracle as orc
from test_gpu_linear import t_u16, weights
from test_gpu_step import TOL, Layer

pytestmark = pytest.mark.gpu

H = 1536  # E2B hidden size: o_proj rows


def bits(t):
    return t.cpu().numpy().view(np.uint32)


def run_case(dev, layers, nqh, nkh, hd, seed, rows=H, check_oracle=True):
    entries = [L.entry() for L in layers]
    arr = ops.make_step_entries(entries, nqh, nkh, hd)
    ws = torch.empty(ops.step_workspace_bytes(len(entries), nqh, nkh, hd), dtype=torch.uint8, device=dev)
    plan = ops.attn_step_prepare(arr, nqh, nkh, hd, ws)
    n = nqh * hd
    wo = [weights(seed + i, rows, n, 0.02) for i in range(len(layers))]
    dwo = [t_u16(w, dev) for w in wo]
    # the path being replaced: attention, merge launch, one projection per entry
    ops.attn_step_run_attention(plan)
    ops.attn_step_run_merge(plan)
    y_ref = [torch.empty(rows, device=dev) for _ in layers]
    for L, w, y in zip(layers, dwo, y_ref):
        ops.linear_f16(L.out, n, [(w, y, rows)])
    torch.cuda.synchronize()
    attn_ref = [L.out.clone() for L in layers]
    # the fused path, twice on the same plan (the step and its records are rewritten each time)
    for rep in range(2):
        for L in layers:
            L.out.fill_(float("nan"))
        y = [torch.full((rows,), float("nan"), device=dev) for _ in layers]
        ops.attn_step_run_attention(plan)
        ops.attn_step_run_out(plan, n, [(w, yy, rows) for w, yy in zip(dwo, y)])
        torch.cuda.synchronize()
        for i, L in enumerate(layers):
            np.testing.assert_array_equal(bits(L.out), bits(attn_ref[i]), err_msg=f"attnOut entry {i} rep {rep}")
            np.testing.assert_array_equal(bits(y[i]), bits(y_ref[i]), err_msg=f"o_proj entry {i} rep {rep}")
    for i, L in enumerate(layers):
        got = attn_ref[i].cpu().numpy()
        np.testing.assert_array_equal(bits(y[i]), orc.matmul_quant(got, wo[i], rows, n).view(np.uint32),
                                      err_msg=f"o_proj entry {i} vs oracle matmulQuant")
        if check_oracle:
            want, _, _ = L.expected()
            err = float(np.abs(got - want).max())
            assert err <= TOL, f"entry {i}: attnOut max-abs {err}"
    return plan


CASES = [  # (label, [(seq, window, theta, divisor)], nqh, nkh, hd)
    ("local W512 (8 parts)", [(513, 512, 1e4, 0)], 8, 1, 256),
    ("one part", [(1, 0, 1e4, 0)], 8, 1, 256),
    ("3 tiles", [(70, 0, 1e6, 1)], 8, 1, 256),
    ("global 8193 (over 8 parts)", [(8193, 0, 1e6, 1)], 8, 1, 256),
    ("head_dim 512, 7 parts", [(200, 0, 1e6, 1)], 8, 1, 512),
    ("head_dim 512 local", [(513, 512, 1e4, 0)], 8, 1, 512),
    ("three entries", [(513, 512, 1e4, 0), (100, 0, 1e6, 1), (40, 0, 1e4, 0)], 8, 1, 256),
    ("group 4", [(513, 512, 1e4, 0)], 4, 1, 256),
    ("group 4 head_dim 512", [(200, 0, 1e6, 1)], 4, 1, 512),
    ("two kv heads", [(513, 512, 1e4, 0)], 8, 2, 256),
]


@pytest.mark.parametrize("label,specs,nqh,nkh,hd", CASES, ids=[c[0] for c in CASES])
def test_step_out_matches_merge_then_linear(dev, label, specs, nqh, nkh, hd):
    announce(f"attnStepOut {label}")
    layers = [Layer(dev, 7100 + 17 * i + s[0], *s, nqh=nqh, nkh=nkh, hd=hd) for i, s in enumerate(specs)]
    run_case(dev, layers, nqh, nkh, hd, seed=90 + len(specs) + hd)


def test_step_out_many_entries(dev):
    """A stack step of 28 local and 7 global entries (6 and 4 parts) with one projection each, one launch."""
    announce("attnStepOut 35 entries")
    specs = [(513 if i % 5 != 4 else 300, 512 if i % 5 != 4 else 0, 1e4 if i % 5 != 4 else 1e6, i % 5 == 4)
             for i in range(35)]
    layers = [Layer(dev, 9100 + 31 * i, s[0], s[1], s[2], int(s[3])) for i, s in enumerate(specs)]
    run_case(dev, layers, 8, 1, 256, seed=300, rows=256, check_oracle=False)


def test_step_out_rejects_mismatched_segments(dev):
    announce("attnStepOut argument errors")
    L = Layer(dev, 4242, 513, 512, 1e4, 0)
    arr = ops.make_step_entries([L.entry()], 8, 1, 256)
    ws = torch.empty(ops.step_workspace_bytes(1, 8, 1, 256), dtype=torch.uint8, device=dev)
    plan = ops.attn_step_prepare(arr, 8, 1, 256, ws)
    w = t_u16(weights(1, 16, 2048), dev)
    y = torch.empty(16, device=dev)
    with pytest.raises(RuntimeError, match="weight segments"):
        ops.attn_step_run_out(plan, 2048, [(w, y, 16), (w, y, 16)])
    torch.cuda.synchronize()
