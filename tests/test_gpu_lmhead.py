"""GPU parity of the sampling head (lmHead -> logitSoftcap -> argmax, src/engine.ts:2223-2255) against
the oracle, and the end-to-end top-1 of a decode step.

The reference-shaped kernels and the fused lm head evaluate matmul_quant.wgsl's summation order and
logit_softcap.wgsl's expression, so logits are compared bit for bit; the top-1 index must equal the
oracle's argmax.wgsl restatement exactly, ties included (the tie cases are built from duplicated
weight rows, which give bitwise-equal logits).
"""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import closed_form as cf
from oracle import oracle as orc
from g4attn import ops

pytestmark = pytest.mark.gpu


def weights(seed, M, N, scale=0.05):
    w = (np.random.default_rng(seed).standard_normal((M, N), dtype=np.float32) * scale).astype(np.float16)
    return w.view(np.uint16)


def t_f32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def t_u16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)


def bits32(t):
    return t.cpu().numpy().view(np.uint32)


def oracle_head(x, wbits, M, N, cap):
    logits = orc.matmul_quant(x, wbits, M, N)
    if cap > 0:
        logits = orc.logit_softcap(logits, cap)
    return logits, orc.argmax(logits)


def run_fused(dev, x, wbits, M, N, cap, want_logits=True):
    ws = torch.empty(ops.lm_head_workspace_bytes(M, N, cap), dtype=torch.uint8, device=dev)
    logits = torch.full((M,), float("nan"), device=dev) if want_logits else None
    res = torch.full((1,), -1, dtype=torch.int32, device=dev)
    ops.lm_head_argmax(t_f32(x, dev), t_u16(wbits, dev), logits, res, ws, M, N, cap)
    torch.cuda.synchronize()
    return logits, int(res.cpu().item())


@pytest.mark.parametrize("M,N", [(1000, 1536), (300, 300), (70000, 256), (5, 17)])
def test_matmul_quant_bits(dev, M, N):
    announce(f"matmulQuant M={M} N={N}")
    x = np.random.default_rng(N).standard_normal(N, dtype=np.float32)
    w = weights(M + N, M, N)
    want = orc.matmul_quant(x, w, M, N)
    out = torch.full((M,), float("nan"), device=dev)
    ops.matmul_quant_f16(t_f32(x, dev), t_u16(w, dev), out, M, N)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits32(out), want.view(np.uint32))


@pytest.mark.parametrize("size", [1000, 262144])
def test_logit_softcap_bits(dev, size):
    announce(f"logitSoftcap size={size}")
    x = np.random.default_rng(size).standard_normal(size, dtype=np.float32) * 400.0  # past the +-15 clamp
    x[:4] = [np.inf, -np.inf, np.nan, 0.0]
    want = orc.logit_softcap(x, 30.0)
    d = t_f32(x, dev)
    ops.logit_softcap(d, size, 30.0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits32(d), want.view(np.uint32))


def tie_cases():
    rng = np.random.default_rng(11)
    cases = []
    for trial in range(6):
        n = [300, 1000, 4096, 262144, 7, 65537][trial]
        x = rng.integers(-3, 4, size=n).astype(np.float32)
        if trial == 4:
            x[:] = np.nan
        if trial == 5:
            x[rng.integers(0, n, size=n // 4)] = np.float32(-1e30)
        cases.append(x)
    x = np.zeros(256, np.float32)
    x[[1, 4]] = 3.0  # the tree keeps residue 4
    cases.append(x)
    return cases


@pytest.mark.parametrize("case", range(7))
def test_argmax_reference_kernel(dev, case):
    x = tie_cases()[case]
    announce(f"argmax case={case} n={x.size}")
    res = torch.full((1,), -1, dtype=torch.int32, device=dev)
    ops.argmax(t_f32(x, dev), res, x.size)
    torch.cuda.synchronize()
    got = int(res.cpu().item())
    assert got == orc.argmax(x) == cf.argmax_rule(x)


@pytest.mark.parametrize("M,N,cap", [(4096 + 37, 1536, 30.0), (1000, 2048, 0.0), (64, 1024, 30.0),
                                     (65536 + 13, 2560, 30.0), (3, 1280, 30.0)])
def test_lm_head_fused_bits(dev, M, N, cap):
    """Logits bit-identical to matmulQuant (+ logitSoftcap); top-1 equal to the oracle's argmax."""
    announce(f"lmHead fused M={M} N={N} cap={cap}")
    x = np.random.default_rng(M).standard_normal(N, dtype=np.float32)
    w = weights(M * 7 + N, M, N)
    want_logits, want_idx = oracle_head(x, w, M, N, cap)
    logits, idx = run_fused(dev, x, w, M, N, cap)
    np.testing.assert_array_equal(bits32(logits), want_logits.view(np.uint32))
    assert idx == want_idx
    _, idx2 = run_fused(dev, x, w, M, N, cap, want_logits=False)  # logits not written: same top-1
    assert idx2 == want_idx


@pytest.mark.parametrize("rows,cap", [([1, 4], 30.0), ([600, 700], 30.0), ([3, 259, 515], 0.0),
                                      ([9, 6, 4000], 0.0)])
def test_lm_head_ties(dev, rows, cap):
    """Duplicated weight rows give bitwise-equal logits: the winner follows argmax.wgsl's tie rule
    (first index per residue, residues through the tree)."""
    announce(f"lmHead ties rows={rows} cap={cap}")
    M, N = 5000, 1536
    x = np.random.default_rng(5).standard_normal(N, dtype=np.float32)
    w = weights(17, M, N).reshape(M, N).copy()
    top = (np.sign(x) * 0.2).astype(np.float16).view(np.uint16)  # aligned with x: far above every other row
    for r in rows:
        w[r] = top
    want_logits, want_idx = oracle_head(x, w, M, N, cap)
    assert want_idx == cf.argmax_rule(want_logits)
    logits, idx = run_fused(dev, x, w, M, N, cap)
    np.testing.assert_array_equal(bits32(logits), want_logits.view(np.uint32))
    assert idx == want_idx and idx in rows


def test_lm_head_softcap_clamp_ties(dev):
    """Logits past 15 * cap all soft-cap to exactly cap: a many-way tie settled by the rule."""
    announce("lmHead clamp ties")
    M, N = 3000, 1024
    x = np.full(N, 1.0, np.float32)
    w = weights(23, M, N, scale=0.01).reshape(M, N).copy()
    rng = np.random.default_rng(3)
    big = rng.choice(M, size=40, replace=False)
    w[big] = np.float16(1.0).view(np.uint16)  # logit 1024 > 15 * 30
    want_logits, want_idx = oracle_head(x, w, M, N, 30.0)
    assert (want_logits == 30.0).sum() >= 40
    logits, idx = run_fused(dev, x, w, M, N, 30.0)
    np.testing.assert_array_equal(bits32(logits), want_logits.view(np.uint32))
    assert idx == want_idx == cf.argmax_rule(want_logits)


def test_lm_head_no_candidate(dev):
    """Every logit at or below the shader's -1e30 start: index 0; one row above it wins."""
    announce("lmHead no candidate")
    M, N = 1000, 1024
    x = np.zeros(N, np.float32)
    x[0] = -1e32
    w = np.zeros((M, N), np.float16)
    w[:, 0] = 1.0
    wb = w.view(np.uint16)
    _, idx = run_fused(dev, x, wb, M, N, 0.0)
    assert idx == 0 == oracle_head(x, wb, M, N, 0.0)[1]
    w[777, 0] = -1.0
    wb = w.view(np.uint16)
    _, idx = run_fused(dev, x, wb, M, N, 0.0)
    assert idx == 777 == oracle_head(x, wb, M, N, 0.0)[1]


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_top1_end_to_end(dev, seed):
    """P3: one decode step end to end. A local and a global layer go through the one-launch step
    (norms, RoPE, KV store, attention); the global layer's attnOut feeds a synthetic lm head
    (vocab 32768 x 2048, softcap 30) and the fused argmax. The oracle runs the reference's six kernels,
    matmulQuant, logitSoftcap and argmax. The top-1 must be equal, and the oracle's margin between the
    first and second logit must exceed the largest logit difference (so equality is not luck)."""
    from test_gpu_step import HD, NQH, Layer, run_step

    announce(f"top-1 end to end seed={seed}")
    local = Layer(dev, 9000 + seed, 1000, 512, 1e4, 0)
    glob = Layer(dev, 9100 + seed, 3000, 0, 1e6, 1)
    run_step(dev, [local.entry(), glob.entry(inv_freq=True)])
    want_out, _, _ = glob.expected()
    M, N = 32768, NQH * HD
    w = weights(500 + seed, M, N, scale=0.03)
    want_logits, want_idx = oracle_head(want_out, w, M, N, 30.0)
    ws = torch.empty(ops.lm_head_workspace_bytes(M, N, 30.0), dtype=torch.uint8, device=dev)
    logits = torch.empty(M, device=dev)
    res = torch.full((1,), -1, dtype=torch.int32, device=dev)
    ops.lm_head_argmax(glob.out, t_u16(w, dev), logits, res, ws, M, N, 30.0)
    torch.cuda.synchronize()
    got_logits = logits.cpu().numpy()
    diff = float(np.abs(got_logits - want_logits).max())
    srt = np.sort(want_logits)
    margin = float(srt[-1] - srt[-2])
    print(f"seed={seed} top1={want_idx} margin={margin:.3e} max logit diff={diff:.3e}")
    assert int(res.cpu().item()) == want_idx
    assert margin > 2 * diff
