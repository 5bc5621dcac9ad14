"""g4_attn_decode_noalloc (no workspace, no allocation: split partials in the library's fixed
device array) against g4_attn_decode (caller's workspace), through the C ABI.

The two use the same kernels and, on this GPU, the same split size, so the outputs must be
bit-identical; both are also checked against the oracle's reference chain within max-abs 2e-3.
Two calls in a row on the shared array, the second with a smaller input, show that a call does
not depend on what the previous one left there.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from g4attn import ops
from g4attn.abi import G4Error
from helpers import cache_f16, max_abs, unit_q
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL = 2e-3


def t_f32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def t_u16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)


def case(dev, seed, nqh, nkh, hd, seq, win):
    kc, vc = cache_f16(seed, seq, nkh, hd), cache_f16(seed + 1, seq, nkh, hd)
    q = unit_q(seed + 2, nqh, hd)
    d = dict(q=t_f32(q, dev), k=t_u16(kc, dev), v=t_u16(vc, dev))
    want = orc.attention_chain(q, orc.f16_bits_to_f32(kc), orc.f16_bits_to_f32(vc), nqh, nkh, hd, seq, 1.0, win)
    return d, want


def run_both(dev, d, nqh, nkh, hd, seq, win):
    ws = torch.empty(ops.decode_workspace_bytes(nqh, nkh, hd, seq), dtype=torch.uint8, device=dev)
    ref = torch.full((nqh * hd,), float("nan"), dtype=torch.float32, device=dev)
    got = torch.full((nqh * hd,), float("nan"), dtype=torch.float32, device=dev)
    ops.attn_decode(d["q"], d["k"], d["v"], ref, ws, nqh, nkh, hd, seq, 1.0, win)
    ops.attn_decode_noalloc(d["q"], d["k"], d["v"], got, nqh, nkh, hd, seq, 1.0, win)
    torch.cuda.synchronize()
    return ref.cpu().numpy(), got.cpu().numpy()


@pytest.mark.parametrize("first,second", [
    ((8, 1, 256, 40000, 0), (8, 1, 256, 3000, 512)),   # many splits, then fewer on the same array
    ((8, 1, 512, 20000, 0), (8, 2, 512, 700, 0)),      # head_dim 512, then two kv heads
    ((8, 1, 256, 131072, 0), (4, 1, 256, 5000, 0)),    # 512 splits (the array's limit), then a smaller group
])
def test_noalloc_matches_workspace_entry_point(dev, first, second):
    for label, (nqh, nkh, hd, seq, win) in (("first", first), ("second", second)):
        announce(f"attnDecodeNoAlloc {label}: nqh={nqh} nkh={nkh} hd={hd} seq={seq} win={win}")
        d, want = case(dev, 100 + seq + hd, nqh, nkh, hd, seq, win)
        ref, got = run_both(dev, d, nqh, nkh, hd, seq, win)
        assert np.isfinite(got).all(), f"{label}: non-finite output"
        np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32), err_msg=label)
        err = max_abs(got, want)
        assert err <= TOL, f"{label}: max-abs {err}"
        print(f"noalloc {label} seq={seq} hd={hd}: bit-identical to attnDecode, err {err:.2e}", flush=True)


def test_noalloc_rejects_beyond_scratch(dev):
    d, _ = case(dev, 5, 16, 2, 256, 64, 0)
    out = torch.empty(16 * 256, dtype=torch.float32, device=dev)
    with pytest.raises(G4Error, match="scratch"):
        ops.attn_decode_noalloc(d["q"], d["k"], d["v"], out, 16, 2, 256, 64)
