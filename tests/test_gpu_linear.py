"""GPU parity of the projections either side of the attention block (attn.linearQKV,
src/engine.ts:2045-2051; attn.linearOut, :2096) against the oracle's matmul_quant.wgsl,
matmul_q8.wgsl and matmul_q4k.wgsl restatements: bit-identical rows, one or several weight matrices
per launch, and the reference-shaped matmulQ8 / matmulQ4K kernels likewise. And one producer layer end to end:
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


def q8_weights(seed, M, N):
    rng = np.random.default_rng(seed)
    q = rng.integers(-128, 128, size=(M, N)).astype(np.int8)
    sc = (rng.random((M, N // 32)) * 0.002 + 1e-4).astype(np.float16).view(np.uint16)
    return q, sc


def q4k_weights(seed, M, N):
    rng = np.random.default_rng(seed)
    nib = rng.integers(0, 16, size=(M * N // 8, 8)).astype(np.uint32)
    words = (nib << (4 * np.arange(8, dtype=np.uint32))).sum(axis=1, dtype=np.uint64).astype(np.uint32)
    sb = N // 256
    meta = np.concatenate([(rng.random((M, sb, 8)) * 0.01).astype(np.float16),
                           (rng.standard_normal((M, sb, 8)) * 0.05).astype(np.float16)], axis=2)
    return words, meta.view(np.uint16)


def t_i8(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int8)).to(dev)


def t_u32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(dev)


@pytest.mark.parametrize("fmt,M,N", [("q8", 1000, 1536), ("q8", 70000, 256), ("q8", 5, 96), ("q4k", 1000, 1536),
                                     ("q4k", 70000, 256), ("q4k", 3, 4096)])
def test_matmul_quantized_reference_kernels(dev, fmt, M, N):
    """matmulQ8 / matmulQ4K as the engine dispatches them (one workgroup per row; a 2D grid above 65535 rows)."""
    announce(f"matmul {fmt} M={M} N={N}")
    x = np.random.default_rng(N + M).standard_normal(N, dtype=np.float32)
    out = torch.full((M,), float("nan"), device=dev)
    if fmt == "q8":
        q, sc = q8_weights(M + N, M, N)
        ops.matmul_q8(t_f32(x, dev), t_i8(q, dev), t_u16(sc, dev), out, M, N)
        want = orc.matmul_q8(x, q, sc, M, N)
    else:
        w, meta = q4k_weights(M + N, M, N)
        ops.matmul_q4k(t_f32(x, dev), t_u32(w, dev), t_u16(meta, dev), out, M, N)
        want = orc.matmul_q4k(x, w, meta, M, N)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("fmt", ["q8", "q4k"])
@pytest.mark.parametrize("N,rows", [(1536, [2048, 256, 256]), (2048, [1536]), (4096, [1536]), (1024, [1]),
                                    (1536, [3, 1, 262, 5]), (3072, [777])])
def test_linear_quant_bits(dev, fmt, N, rows):
    """The fused projections with q8 / q4k weights: each row bit-identical to matmulQ8 / matmulQ4K."""
    announce(f"linear {fmt} N={N} rows={rows}")
    x = np.random.default_rng(N + 5).standard_normal(N, dtype=np.float32)
    segs, wants = [], []
    outs = [torch.full((r,), float("nan"), device=dev) for r in rows]
    for i, (r, o) in enumerate(zip(rows, outs)):
        if fmt == "q8":
            q, sc = q8_weights(N + 17 * i + r, r, N)
            segs.append((t_i8(q, dev), t_u16(sc, dev), o, r))
            wants.append(orc.matmul_q8(x, q, sc, r, N))
        else:
            w, meta = q4k_weights(N + 17 * i + r, r, N)
            segs.append((t_u32(w, dev), t_u16(meta, dev), o, r))
            wants.append(orc.matmul_q4k(x, w, meta, r, N))
    ops.linear_quant(t_f32(x, dev), N, fmt, segs)
    torch.cuda.synchronize()
    for i, (o, want) in enumerate(zip(outs, wants)):
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
