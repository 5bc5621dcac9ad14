"""GPU parity of the f16 projections either side of the attention block (attn.linearQKV,
src/engine.ts:2045-2051; attn.linearOut, :2096) against the oracle's matmul_quant.wgsl restatement:
bit-identical rows, one or several weight matrices per launch. And one producer layer end to end:
normed hidden state -> q/k/v projections -> the one-launch step (norms, RoPE, KV store, attention)
-> o_proj, against the oracle's matmulQuant x3 -> six reference kernels -> matmulQuant.
"""
import numpy as np
import pytest
import torch

from conftest import announce
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


@pytest.mark.parametrize("N,rows", [(1536, [2048, 256, 256]), (2048, [1536]), (4096, [1536]), (1024, [1]),
                                    (1536, [3, 1, 262, 5]), (2560, [4096, 512, 512]), (3072, [777])])
def test_linear_bits(dev, N, rows):
    announce(f"linear N={N} rows={rows}")
    x = np.random.default_rng(N).standard_normal(N, dtype=np.float32)
    ws = [weights(N + 31 * i + r, r, N) for i, r in enumerate(rows)]
    outs = [torch.full((r,), float("nan"), device=dev) for r in rows]
    ops.linear_f16(t_f32(x, dev), N, [(t_u16(w, dev), o, r) for w, o, r in zip(ws, outs, rows)])
    torch.cuda.synchronize()
    for i, (w, o, r) in enumerate(zip(ws, outs, rows)):
        want = orc.matmul_quant(x, w, r, N)
        np.testing.assert_array_equal(o.cpu().numpy().view(np.uint32), want.view(np.uint32), err_msg=f"segment {i}")


@pytest.mark.parametrize("seq,win,theta,div,hd", [(1000, 512, 1e4, 0, 256), (3000, 0, 1e6, 1, 512)])
def test_producer_layer_end_to_end(dev, seq, win, theta, div, hd):
    """E2B shapes: hidden 1536, 8 query heads and 1 kv head of head_dim hd."""
    from test_gpu_step import Layer, run_step

    announce(f"producer layer seq={seq} hd={hd}")
    H, NQH, NKH = 1536, 8, 1
    L = Layer(dev, 4000 + seq, seq, win, theta, div, hd=hd)
    x = np.random.default_rng(seq).standard_normal(H, dtype=np.float32)
    wq, wk, wv = weights(1, NQH * hd, H, 0.03), weights(2, NKH * hd, H, 0.03), weights(3, NKH * hd, H, 0.03)
    wo = weights(4, H, NQH * hd, 0.02)
    # the layer's raw projections come from the GEMV (the step reads them in place)
    ops.linear_f16(t_f32(x, dev), H, [(t_u16(wq, dev), L.d["q"], NQH * hd), (t_u16(wk, dev), L.d["k"], NKH * hd),
                                      (t_u16(wv, dev), L.d["v"], NKH * hd)])
    torch.cuda.synchronize()
    L.q = orc.matmul_quant(x, wq, NQH * hd, H)
    L.k = orc.matmul_quant(x, wk, NKH * hd, H)
    L.v = orc.matmul_quant(x, wv, NKH * hd, H)
    for name, arr in (("q", L.q), ("k", L.k), ("v", L.v)):
        np.testing.assert_array_equal(L.d[name].cpu().numpy().view(np.uint32), arr.view(np.uint32), err_msg=name)
    want_attn, kb, vb = L.expected()
    run_step(dev, [L.entry(inv_freq=True)], hd=hd)
    y = torch.empty(H, device=dev)
    ops.linear_f16(L.out, NQH * hd, [(t_u16(wo, dev), y, H)])
    torch.cuda.synchronize()
    want_y = orc.matmul_quant(want_attn, wo, H, NQH * hd)
    got_attn = L.out.cpu().numpy()
    assert np.abs(got_attn - want_attn).max() <= 2e-3
    # o_proj of the GPU's attnOut is bit-identical to the oracle's matmulQuant of the same vector
    np.testing.assert_array_equal(y.cpu().numpy().view(np.uint32),
                                  orc.matmul_quant(got_attn, wo, H, NQH * hd).view(np.uint32))
    err = float(np.abs(y.cpu().numpy() - want_y).max())
    bound = 2e-3 * float(np.abs(orc.f16_bits_to_f32(wo)).reshape(H, -1).sum(axis=1).max())
    print(f"producer layer seq={seq} hd={hd}: |y - oracle| {err:.2e} (bound {bound:.2e})")
    assert err <= bound
