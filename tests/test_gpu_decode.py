"""GPU parity of the fused decode kernels (attnScore -> softmax -> attnOutput in
one flash-decoding pass) against the oracle's reference chain.

Both sides read bit-identical f16 K/V (the oracle gets them widened to f32,
as the WGSL binds f32 caches) and identical post-RoPE q. Tolerance: max-abs
2e-3 on attnOut (f16 KV, f32 accumulate); the measured error is printed and
is expected to be around 1e-6.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from g4attn import e2b, ops, synth
from helpers import cache_f16, cache_f16_torch, max_abs, unit_q
from oracle import closed_form as cf
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL = 2e-3


def t_f32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def t_u16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)


def run_decode(dev, q, kc, vc, nqh, nkh, hd, seq, win, scale=1.0, max_seq=None):
    ws = torch.empty(ops.decode_workspace_bytes(nqh, nkh, hd, max_seq or seq), dtype=torch.uint8, device=dev)
    out = torch.full((nqh * hd,), float("nan"), dtype=torch.float32, device=dev)
    kd = kc if isinstance(kc, torch.Tensor) else t_u16(kc, dev)
    vd = vc if isinstance(vc, torch.Tensor) else t_u16(vc, dev)
    ops.attn_decode(t_f32(q, dev), kd, vd, out, ws, nqh, nkh, hd, seq, scale, win)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def oracle_chain(q, kc_bits, vc_bits, nqh, nkh, hd, seq, win, scale=1.0):
    kf = orc.f16_bits_to_f32(kc_bits)
    vf = orc.f16_bits_to_f32(vc_bits)
    return orc.attention_chain(q, kf, vf, nqh, nkh, hd, seq, scale, win), kf, vf


EDGE_SEQS = [1, 2, 31, 32, 33, 100, 127, 128, 129, 255, 257, 511, 512, 513, 1000, 4097, 8193]


@pytest.mark.parametrize("seq", EDGE_SEQS)
@pytest.mark.parametrize("win", [0, 512])
def test_decode_matches_reference_chain(dev, seq, win):
    nqh, nkh, hd = 8, 1, 256
    announce(f"attnDecode seq={seq} win={win}")
    kc, vc = cache_f16(1000 + seq, seq, nkh, hd), cache_f16(2000 + seq, seq, nkh, hd)
    q = unit_q(3000 + seq, nqh, hd)
    want, kf, vf = oracle_chain(q, kc, vc, nqh, nkh, hd, seq, win)
    got = run_decode(dev, q, kc, vc, nqh, nkh, hd, seq, win)
    err = max_abs(got, want)
    err64 = max_abs(got, cf.sdpa(q, kf, vf, nqh, nkh, hd, seq, 1.0, win))
    print(f"seq={seq} win={win} max|gpu-oracle|={err:.2e} max|gpu-fp64|={err64:.2e}")
    assert np.isfinite(got).all()
    assert err <= TOL and err64 <= TOL


@pytest.mark.parametrize("nqh,nkh", [(16, 2), (4, 1), (8, 8), (2, 1)])
def test_decode_gqa_groups(dev, nqh, nkh):
    hd, seq, win = 256, 777, 0
    announce(f"attnDecode gqa nqh={nqh} nkh={nkh}")
    kc, vc = cache_f16(5, seq, nkh, hd), cache_f16(6, seq, nkh, hd)
    q = unit_q(7, nqh, hd)
    want, _, _ = oracle_chain(q, kc, vc, nqh, nkh, hd, seq, win)
    got = run_decode(dev, q, kc, vc, nqh, nkh, hd, seq, win)
    err = max_abs(got, want)
    print(f"nqh={nqh} nkh={nkh} err={err:.2e}")
    assert err <= TOL


def test_decode_scale_and_peaked(dev):
    """A non-unit scale, a query equal to a cached key (near one-hot softmax) and q = 0 (uniform)."""
    nqh, nkh, hd, seq = 8, 1, 256, 1500
    announce("attnDecode scale/peaked/uniform")
    kc, vc = cache_f16(8, seq, nkh, hd), cache_f16(9, seq, nkh, hd)
    kf = orc.f16_bits_to_f32(kc).reshape(seq, hd)
    q = unit_q(10, nqh, hd).reshape(nqh, hd)
    q[1] = kf[1234] * 4.0
    q[2] = 0.0
    q = q.ravel()
    for scale in (1.0, 0.0625):
        want, _, vf = oracle_chain(q, kc, vc, nqh, nkh, hd, seq, 0, scale)
        got = run_decode(dev, q, kc, vc, nqh, nkh, hd, seq, 0, scale)
        err = max_abs(got, want)
        print(f"scale={scale} err={err:.2e}")
        assert err <= TOL
    got = run_decode(dev, q, kc, vc, nqh, nkh, hd, seq, 0, 1.0).reshape(nqh, hd)
    np.testing.assert_allclose(got[2], vf.reshape(seq, hd).mean(axis=0), atol=1e-5)  # q = 0: mean of V


def test_decode_deterministic(dev):
    nqh, nkh, hd, seq = 8, 1, 256, 20000
    announce("attnDecode determinism")
    kc, vc = cache_f16(31, seq, nkh, hd), cache_f16(32, seq, nkh, hd)
    q = unit_q(33, nqh, hd)
    a = run_decode(dev, q, kc, vc, nqh, nkh, hd, seq, 0)
    b = run_decode(dev, q, kc, vc, nqh, nkh, hd, seq, 0)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def test_decode_long_context_131072(dev):
    """Long-context global decode: 131072 keys, split across the GPU, LSE merge."""
    nqh, nkh, hd, seq = 8, 1, 256, 131072
    announce("attnDecode seq=131072 (long context)")
    kd = cache_f16_torch(20261205, seq, nkh, hd, dev)
    vd = cache_f16_torch(20261205 + 7, seq, nkh, hd, dev)
    q = unit_q(20261205 + 11, nqh, hd)
    got = run_decode(dev, q, kd.view(torch.int16), vd.view(torch.int16), nqh, nkh, hd, seq, 0)
    kc = kd.view(torch.int16).cpu().numpy().view(np.uint16)
    vc = vd.view(torch.int16).cpu().numpy().view(np.uint16)
    want, _, _ = oracle_chain(q, kc, vc, nqh, nkh, hd, seq, 0)
    err = max_abs(got, want)
    print(f"seq=131072 err={err:.2e}")
    assert err <= TOL


def stack_entries(dev, nl, seq, hd=256, nqh=8, nkh=1, seed=20261202):
    """One token's 35-layer E2B-shaped stack: per-layer caches and queries."""
    cfg = e2b.AttnConfig(num_layers=nl)
    layers = []
    for il in range(nl):
        kd = cache_f16_torch(seed + 100 * il, seq, nkh, hd, dev)
        vd = cache_f16_torch(seed + 100 * il + 1, seq, nkh, hd, dev)
        q = unit_q(seed + 100 * il + 2, nqh, hd)
        win = e2b.sliding_window(il, cfg) if nl == 35 else (512 if il % 5 != 4 else 0)
        layers.append((t_f32(q, dev), kd.view(torch.int16), vd.view(torch.int16),
                       torch.full((nqh * hd,), float("nan"), device=dev), seq, win, 1.0))
    return layers


@pytest.mark.parametrize("seq", [2049, 8193])
def test_decode_many_layer_stack(dev, seq):
    """35 layers (7 global, 28 local W=512) of one token in one launch, each vs the oracle."""
    nqh, nkh, hd, nl = 8, 1, 256, 35
    announce(f"attnDecodeMany 35-layer stack seq={seq}")
    layers = stack_entries(dev, nl, seq)
    entries = ops.make_entries(layers, nqh, nkh, hd)
    total = sum(min(seq, w) if w else seq for (*_, s, w, _sc) in layers)
    ws = torch.empty(ops.decode_many_workspace_bytes(nl, nqh, nkh, hd, total), dtype=torch.uint8, device=dev)
    ops.attn_decode_many(entries, nqh, nkh, hd, ws)
    torch.cuda.synchronize()
    worst = 0.0
    for il, (q, kd, vd, out, s, win, sc) in enumerate(layers):
        kc, vc = kd.cpu().numpy().view(np.uint16), vd.cpu().numpy().view(np.uint16)
        want, _, _ = oracle_chain(q.cpu().numpy(), kc, vc, nqh, nkh, hd, seq, win)
        err = max_abs(out.cpu().numpy(), want)
        worst = max(worst, err)
        assert err <= TOL, f"layer {il}: {err}"
    print(f"35-layer stack seq={seq} worst err={worst:.2e}")


def test_decode_many_ragged_batch(dev):
    """Ragged batch: independent sequences with their own caches and lengths."""
    nqh, nkh, hd = 8, 1, 256
    lens = [int(x) for x in synth.ragged_lengths(20261203, 12, 1, 5000)] + [1, 32, 33, 4096]
    announce(f"attnDecodeMany ragged batch lens={lens}")
    items = []
    for b, L in enumerate(lens):
        kd = cache_f16_torch(500 + b, L, nkh, hd, dev)
        vd = cache_f16_torch(600 + b, L, nkh, hd, dev)
        q = unit_q(700 + b, nqh, hd)
        items.append((t_f32(q, dev), kd.view(torch.int16), vd.view(torch.int16),
                      torch.full((nqh * hd,), float("nan"), device=dev), L, 0, 1.0))
    entries = ops.make_entries(items, nqh, nkh, hd)
    ws = torch.empty(ops.decode_many_workspace_bytes(len(items), nqh, nkh, hd, sum(lens)), dtype=torch.uint8,
                     device=dev)
    plan = ops.attn_decode_many_prepare(entries, nqh, nkh, hd, ws)
    for rep in range(2):  # a prepared plan can be replayed
        for it in items:
            it[3].fill_(float("nan"))
        ops.attn_decode_many_run(plan)
        torch.cuda.synchronize()
        for b, (q, kd, vd, out, L, win, sc) in enumerate(items):
            kc, vc = kd.cpu().numpy().view(np.uint16), vd.cpu().numpy().view(np.uint16)
            want, _, _ = oracle_chain(q.cpu().numpy(), kc, vc, nqh, nkh, hd, L, 0)
            err = max_abs(out.cpu().numpy(), want)
            assert err <= TOL, f"seq {b} (len {L}) rep {rep}: {err}"


def test_decode_rejects_bad_shapes(dev):
    """Argument errors are rejected on the host, before any launch."""
    from g4attn.abi import G4Error

    q = torch.zeros(8 * 128, device=dev)
    kc = torch.zeros(10 * 128, dtype=torch.int16, device=dev)
    out = torch.zeros(8 * 128, device=dev)
    with pytest.raises(G4Error, match="head_dim"):
        ops.attn_decode(q, kc, kc, out, None, 8, 1, 128, 10)
    q = torch.zeros(8 * 256, device=dev)
    kc = torch.zeros(4000 * 256, dtype=torch.int16, device=dev)
    out = torch.zeros(8 * 256, device=dev)
    with pytest.raises(G4Error, match="workspace"):
        ops.attn_decode(q, kc, kc, out, None, 8, 1, 256, 4000)
    with pytest.raises(ValueError):
        ops.attn_decode(q, kc, kc, out, None, 8, 1, 256, 4001)  # cache smaller than seq_len rows


@pytest.mark.parametrize("seq,win", [(1, 0), (33, 0), (513, 512), (4097, 0), (20000, 0), (1000, 512)])
def test_decode_head_dim_512(dev, seq, win):
    """E2B global layers have head_dim 512: attnDecode at 512 against the oracle's chain and fp64 SDPA."""
    nqh, nkh, hd = 8, 1, 512
    announce(f"attnDecode hd=512 seq={seq} win={win}")
    kc, vc = cache_f16(4000 + seq, seq, nkh, hd), cache_f16(5000 + seq, seq, nkh, hd)
    q = unit_q(6000 + seq, nqh, hd)
    want, kf, vf = oracle_chain(q, kc, vc, nqh, nkh, hd, seq, win)
    got = run_decode(dev, q, kc, vc, nqh, nkh, hd, seq, win)
    err = max_abs(got, want)
    err64 = max_abs(got, cf.sdpa(q, kf, vf, nqh, nkh, hd, seq, 1.0, win))
    print(f"hd=512 seq={seq} win={win} max|gpu-oracle|={err:.2e} max|gpu-fp64|={err64:.2e}")
    assert np.isfinite(got).all()
    assert err <= TOL and err64 <= TOL


def test_decode_many_head_dim_512_ragged(dev):
    """attnDecodeMany at head_dim 512: a ragged batch of global-layer sequences, GQA 4:1 and 8:1 shapes."""
    for nqh, nkh in [(8, 1), (8, 2)]:
        hd = 512
        lens = [1, 77, 3000, 9000, 512]
        announce(f"attnDecodeMany hd=512 nqh={nqh} nkh={nkh} lens={lens}")
        items = []
        for b, L in enumerate(lens):
            kd = cache_f16_torch(800 + b, L, nkh, hd, dev)
            vd = cache_f16_torch(900 + b, L, nkh, hd, dev)
            q = unit_q(1000 + b, nqh, hd)
            items.append((t_f32(q, dev), kd.view(torch.int16), vd.view(torch.int16),
                          torch.full((nqh * hd,), float("nan"), device=dev), L, 0, 1.0))
        entries = ops.make_entries(items, nqh, nkh, hd)
        ws = torch.empty(ops.decode_many_workspace_bytes(len(items), nqh, nkh, hd, sum(lens)), dtype=torch.uint8,
                         device=dev)
        ops.attn_decode_many(entries, nqh, nkh, hd, ws)
        torch.cuda.synchronize()
        for b, (q, kd, vd, out, L, win, sc) in enumerate(items):
            kc, vc = kd.cpu().numpy().view(np.uint16), vd.cpu().numpy().view(np.uint16)
            want, _, _ = oracle_chain(q.cpu().numpy(), kc, vc, nqh, nkh, hd, L, 0)
            err = max_abs(out.cpu().numpy(), want)
            assert err <= TOL, f"nkh={nkh} seq {b} (len {L}): {err}"
