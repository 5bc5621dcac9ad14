"""GPU parity of the six reference kernels and the fused prep against the oracle.

These kernels evaluate the same f32 expressions as the oracle (no FMA
contraction, correctly rounded sqrt/division, f64-evaluated pow/sin/cos/exp),
so the bar is bit equality on identical inputs.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from g4attn import e2b, ops, synth
from helpers import EPS, cache_f16, f16_weight_bits
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

ROPE_FREQS = np.array(e2b.rope_freqs_f16_bits(256), dtype=np.uint16)


def t_f32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def t_u16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy().view(np.uint32 if t.dtype == torch.float32 else np.uint16)


NORM_ROPE_CASES = [
    # (num_heads, head_dim, position, theta, apply_divisor)
    (8, 256, 0, 1e4, 0),
    (8, 256, 14, 1e4, 0),
    (8, 256, 512, 1e4, 0),
    (1, 256, 8192, 1e6, 1),
    (8, 256, 32768, 1e6, 1),
    (8, 256, 131071, 1e6, 1),
    (8, 512, 4096, 1e6, 1),
    (2, 64, 77, 1e4, 0),
]


@pytest.mark.parametrize("nh,hd,pos,theta,div", NORM_ROPE_CASES)
def test_fused_per_head_norm_rope_bits(dev, nh, hd, pos, theta, div):
    announce(f"fusedPerHeadNormRope nh={nh} hd={hd} pos={pos} theta={theta} div={div}")
    x = synth.normal(101 + pos, nh * hd) * 3.0
    w = f16_weight_bits(7, hd)
    want = orc.fused_per_head_norm_rope(x, w, ROPE_FREQS, nh, hd, EPS, pos, theta, div)
    d = t_f32(x, dev)
    ops.fused_per_head_norm_rope(d, t_u16(w, dev), t_u16(ROPE_FREQS, dev), nh, hd, EPS, pos, theta, div)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(d), want.view(np.uint32))


@pytest.mark.parametrize("theta,div,hd", [(1e4, 0, 256), (1e6, 1, 256), (1e6, 0, 512), (5e5, 1, 64)])
def test_rope_inv_freq_bits(dev, theta, div, hd):
    announce(f"ropeInvFreq theta={theta} div={div} hd={hd}")
    rf = ROPE_FREQS if hd // 2 <= ROPE_FREQS.size else np.resize(ROPE_FREQS, hd // 2)
    want = orc.rope_inv_freq(theta, hd, div, rf)
    got = ops.rope_inv_freq(theta, hd, div, t_u16(rf, dev) if div else None)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(got), want.view(np.uint32))


@pytest.mark.parametrize("nh,hd", [(1, 256), (1, 512), (4, 256), (3, 100)])
def test_v_norm_bits(dev, nh, hd):
    announce(f"perHeadRmsNormNoWeight nh={nh} hd={hd}")
    x = synth.normal(55 + hd, nh * hd) * 5.0
    want = orc.per_head_rms_norm_no_weight(x, nh, hd, EPS)
    d = t_f32(x, dev)
    ops.per_head_rms_norm_no_weight(d, nh, hd, EPS)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(d), want.view(np.uint32))


def test_kv_cache_store_bits(dev):
    announce("kvCacheStore")
    nkh, hd, max_seq, pos = 2, 256, 64, 37
    k = synth.normal(1, nkh * hd) * 2
    v = synth.normal(2, nkh * hd) * 2
    kc = torch.zeros(max_seq * nkh * hd, dtype=torch.int16, device=dev)
    vc = torch.zeros_like(kc)
    ops.kv_cache_store(t_f32(k, dev), t_f32(v, dev), kc, vc, nkh, hd, pos, max_seq)
    torch.cuda.synchronize()
    kb, vb = bits(kc).reshape(max_seq, -1), bits(vc).reshape(max_seq, -1)
    np.testing.assert_array_equal(kb[pos], orc.f32_to_f16_bits(k))
    np.testing.assert_array_equal(vb[pos], orc.f32_to_f16_bits(v))
    mask = np.ones(max_seq, bool)
    mask[pos] = False
    assert not kb[mask].any() and not vb[mask].any()


CHAIN_CASES = [
    # (nqh, nkh, hd, seq_len, window)
    (8, 1, 256, 513, 512),
    (8, 1, 256, 1, 0),
    (8, 1, 256, 512, 512),
    (8, 1, 256, 2049, 0),
    (8, 2, 128, 300, 64),
    (4, 4, 64, 700, 0),
]


@pytest.mark.parametrize("nqh,nkh,hd,seq,win", CHAIN_CASES)
def test_score_softmax_output_bits(dev, nqh, nkh, hd, seq, win):
    announce(f"attnScore/softmax/attnOutput nqh={nqh} nkh={nkh} hd={hd} seq={seq} win={win}")
    kc = cache_f16(11 + seq, seq, nkh, hd)
    vc = cache_f16(12 + seq, seq, nkh, hd)
    q = synth.rms_normalize_rows(synth.normal(13, nqh * hd).reshape(nqh, hd)).ravel()
    kf, vf = orc.f16_bits_to_f32(kc), orc.f16_bits_to_f32(vc)
    s_want = orc.attn_score(q, kf, nqh, nkh, hd, seq, 1.0, win)
    p_want = orc.softmax(s_want, nqh, seq)
    o_want = orc.attn_output(p_want, vf, nqh, nkh, hd, seq)
    qd, kd, vd = t_f32(q, dev), t_u16(kc, dev), t_u16(vc, dev)
    sc = torch.empty(nqh * seq, dtype=torch.float32, device=dev)
    out = torch.empty(nqh * hd, dtype=torch.float32, device=dev)
    ops.attn_score(qd, kd, sc, nqh, nkh, hd, seq, 1.0, win)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(sc), s_want.view(np.uint32))
    ops.softmax(sc, nqh, seq)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(sc), p_want.view(np.uint32))
    ops.attn_output(sc, vd, out, nqh, nkh, hd, seq)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(out), o_want.view(np.uint32))


PREP_CASES = [
    # (nqh, nkh, hd, pos, theta, div, store)
    (8, 1, 256, 512, 1e4, 0, True),
    (8, 1, 256, 8192, 1e6, 1, True),
    (8, 1, 256, 131071, 1e6, 1, True),
    (8, 1, 512, 100, 1e6, 1, True),
    (8, 1, 256, 700, 1e4, 0, False),
    (8, 2, 256, 3, 1e4, 0, True),
]


@pytest.mark.parametrize("nqh,nkh,hd,pos,theta,div,store", PREP_CASES)
def test_prep_matches_reference_sequence(dev, nqh, nkh, hd, pos, theta, div, store):
    announce(f"attnPrep nqh={nqh} nkh={nkh} hd={hd} pos={pos} div={div} store={store}")
    max_seq = pos + 3
    q = synth.normal(21, nqh * hd) * 2
    k = synth.normal(22, nkh * hd) * 2
    v = synth.normal(23, nkh * hd) * 2
    qw, kw = f16_weight_bits(24, hd), f16_weight_bits(25, hd)
    # reference order (src/engine.ts:2056-2091): vNorm, normRope Q, normRope K, store
    v_want = orc.per_head_rms_norm_no_weight(v, nkh, hd, EPS)
    q_want = orc.fused_per_head_norm_rope(q, qw, ROPE_FREQS, nqh, hd, EPS, pos, theta, div)
    k_want = orc.fused_per_head_norm_rope(k, kw, ROPE_FREQS, nkh, hd, EPS, pos, theta, div)
    qd, kd, vd = t_f32(q, dev), t_f32(k, dev), t_f32(v, dev)
    kc = torch.zeros(max_seq * nkh * hd, dtype=torch.int16, device=dev)
    vc = torch.zeros_like(kc)
    ops.attn_prep(qd, kd, vd, t_u16(qw, dev), t_u16(kw, dev), t_u16(ROPE_FREQS, dev), kc, vc, nqh, nkh, hd, EPS,
                  pos, theta, div, pos, max_seq, store_kv=store)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(qd), q_want.view(np.uint32))
    if store:
        np.testing.assert_array_equal(bits(kd), k_want.view(np.uint32))
        np.testing.assert_array_equal(bits(vd), v_want.view(np.uint32))
        kb, vb = bits(kc).reshape(max_seq, -1), bits(vc).reshape(max_seq, -1)
        np.testing.assert_array_equal(kb[pos], orc.f32_to_f16_bits(k_want))
        np.testing.assert_array_equal(vb[pos], orc.f32_to_f16_bits(v_want))
        assert not kb[:pos].any() and not kb[pos + 1:].any()
    else:
        np.testing.assert_array_equal(bits(kd), k.view(np.uint32))
        assert not bits(kc).any()
