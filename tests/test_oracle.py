"""Pins the oracle (oracle/wgsl_ref.c) against independent evidence, on the CPU.

Each restated WGSL kernel is checked against at least one of: the
reference's own fixture (public/ref/layer_0_detail.npz, HF bf16 dumps of
Gemma-4-E2B layer 0), a library routine (numpy float16 casts, transformers'
Gemma4RMSNorm / apply_rotary_pos_emb, torch's SDPA), an fp64 closed form
(oracle/closed_form.py), invariants, or brute force on tiny shapes. The
checks are chosen so a plausible slip (dropped eps, sum instead of mean,
interleaved instead of rotate-half pairs, a sign, a window off by one, a
score head-stride of MAX_SEQ, the GQA head map) fails one of them.
"""
import numpy as np
import pytest
import torch

from conftest import GOLDEN
from g4attn import e2b, synth
from oracle import closed_form as cf

EPS = 1e-6
ROPE_FREQS = np.array(e2b.rope_freqs_f16_bits(256), dtype=np.uint16)
ONES = lambda n: np.full(n, 0x3C00, dtype=np.uint16)  # noqa: E731


# ---- f16 conversions: exhaustive against numpy's IEEE float16 -------------------------

def test_f16_to_f32_exhaustive(oracle):
    allbits = np.arange(65536, dtype=np.uint16)
    got = oracle.f16_bits_to_f32(allbits)
    want = allbits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    np.testing.assert_array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_rne(oracle):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(4.0),
        (rng.standard_normal(50000) * 1e-5).astype(np.float32),  # f16 subnormal range
        np.array([65504, 65519.996, 65520, 1e9, -65520, 2**-24, 2**-25, 2**-25 * 1.0000001, 3 * 2**-26,
                  6.1035156e-05, 0.0, -0.0, np.inf, -np.inf], dtype=np.float32),
        # exact ties between adjacent f16 values (round half to even)
        (np.arange(1024, 2048, dtype=np.float32) + 0.5) * np.float32(2**-10),
    ])
    got = oracle.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)


# ---- per-head RMSNorm ------------------------------------------------------------

@pytest.mark.parametrize("nh,hd", [(8, 256), (1, 512), (3, 100), (2, 4)])
def test_v_norm_closed_form(oracle, nh, hd):
    x = synth.normal(1 + hd, nh * hd) * 7.0
    got = oracle.per_head_rms_norm_no_weight(x, nh, hd, EPS)
    np.testing.assert_allclose(got, cf.rms_norm(x, None, EPS, hd), rtol=2e-6, atol=1e-7)
    # HF Gemma4RMSNorm(with_scale=False) as a library routine
    from transformers.models.gemma4.modeling_gemma4 import Gemma4RMSNorm
    hf = Gemma4RMSNorm(hd, eps=EPS, with_scale=False)(torch.from_numpy(x.reshape(nh, hd).astype(np.float64)))
    np.testing.assert_allclose(got, hf.numpy().ravel(), rtol=2e-6, atol=1e-7)


def test_v_norm_scale_invariant_and_unit_rms(oracle):
    x = synth.normal(5, 256)
    a = oracle.per_head_rms_norm_no_weight(x, 1, 256, 0.0)
    b = oracle.per_head_rms_norm_no_weight(x * 1024.0, 1, 256, 0.0)
    np.testing.assert_allclose(a, b, rtol=1e-6)
    assert abs(np.sqrt(np.mean(a.astype(np.float64) ** 2)) - 1.0) < 1e-6


def test_v_norm_real_model_fixture(oracle):
    """Gemma-4-E2B layer 0: v_proj -> v_norm (weightless) from the reference's HF dump."""
    d = np.load(GOLDEN / "layer0_attn.npz")
    got = oracle.per_head_rms_norm_no_weight(d["v_proj"], 1, 256, EPS)
    ref = d["v_norm"].ravel()
    rel = np.max(np.abs(got - ref)) / np.max(np.abs(ref))
    assert rel < 2e-3, rel  # bf16 source: ~5e-4
    # eps matters at the 1e-6 level only; mean (not sum) of squares matters at 16x
    bad = d["v_proj"] / np.sqrt(np.sum(d["v_proj"].astype(np.float64) ** 2))
    assert np.max(np.abs(bad - ref)) / np.max(np.abs(ref)) > 0.5


def test_qk_norm_real_model_fixture(oracle):
    """q_norm/k_norm: per-head RMS over head_dim times a per-dimension weight shared by all heads.

    The GGUF weights are not in the reference tree; the weight implied by head 0 is applied to
    heads 1..7 through the oracle and must reproduce the fixture."""
    d = np.load(GOLDEN / "layer0_attn.npz")
    q = d["q_proj"].reshape(8, 256).astype(np.float64)
    qn = d["q_norm"].astype(np.float64)
    w0 = qn[0] * np.sqrt(np.mean(q[0] ** 2) + EPS) / q[0]
    wbits = oracle.f32_to_f16_bits(w0)
    got = oracle.fused_per_head_norm_rope(d["q_proj"], wbits, None, 8, 256, EPS, 0, 1e4, 0).reshape(8, 256)
    err = np.max(np.abs(got[1:] - qn[1:])) / np.max(np.abs(qn))
    assert err < 3e-2, err  # bf16 weights and activations
    k = d["k_proj"].astype(np.float64)
    kn = d["k_norm"].ravel().astype(np.float64)
    wk = kn * np.sqrt(np.mean(k ** 2) + EPS) / k
    gotk = oracle.fused_per_head_norm_rope(d["k_proj"], oracle.f32_to_f16_bits(wk), None, 1, 256, EPS, 0, 1e4, 0)
    assert np.max(np.abs(gotk - kn)) / np.max(np.abs(kn)) < 3e-2


# ---- RoPE ---------------------------------------------------------------------------

def _f32_angles(pos, theta, hd, divisor):
    """The WGSL's f32 angle: f32(pos) * (1/pow(theta, f32(2i)/f32(hd)) [/ div_i])."""
    i = np.arange(hd // 2)
    e = (np.float32(2) * i.astype(np.float32)) / np.float32(hd)
    p = np.array([np.float32(np.power(np.float64(np.float32(theta)), np.float64(x))) for x in e], np.float32)
    f = np.float32(1.0) / p
    if divisor:
        f = f / ROPE_FREQS[: hd // 2].view(np.float16).astype(np.float32)
    return np.float32(pos) * f


@pytest.mark.parametrize("pos,theta,div", [(0, 1e4, 0), (14, 1e4, 0), (512, 1e4, 0), (8192, 1e6, 1),
                                           (131071, 1e6, 1), (40000, 1e4, 0)])
def test_norm_rope_closed_form(oracle, pos, theta, div):
    nh, hd = 8, 256
    x = synth.normal(pos + 3, nh * hd)
    wbits = oracle.f32_to_f16_bits(1.0 + 0.1 * synth.normal(9, hd))
    w = oracle.f16_bits_to_f32(wbits)
    got = oracle.fused_per_head_norm_rope(x, wbits, ROPE_FREQS, nh, hd, EPS, pos, theta, div)
    normed = cf.rms_norm(x, w, EPS, hd)
    # rotation at the WGSL's own f32 angle: tight
    ang = _f32_angles(pos, theta, hd, div)
    want = cf.rope(normed, pos, theta, hd, angles=ang.astype(np.float64))
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5)
    # the exact-math angle: error grows with position (one f32 ulp of freq moves the angle by ~pos*6e-8)
    exact = cf.rope(normed, pos, theta, hd, divisor=ROPE_FREQS[:128].view(np.float16).astype(np.float64)
                    if div else None)
    assert np.max(np.abs(got - exact)) < 2e-5 + 6e-8 * pos * 4 * 4


def test_rope_matches_hf_rotate_half(oracle):
    """transformers' apply_rotary_pos_emb with cat(freqs, freqs): the rotate-half pairing (i, i+HD/2)."""
    from transformers.models.gemma4.modeling_gemma4 import apply_rotary_pos_emb
    nh, hd, pos, theta = 8, 256, 1234, 1e4
    x = synth.rms_normalize_rows(synth.normal(77, nh * hd).reshape(nh, hd)).ravel()
    got = oracle.fused_per_head_norm_rope(x, ONES(hd), None, nh, hd, 0.0, pos, theta, 0)
    ang = torch.from_numpy(_f32_angles(pos, theta, hd, 0).astype(np.float64))
    emb = torch.cat([ang, ang])[None, :]
    xn = torch.from_numpy(cf.rms_norm(x, None, 0.0, hd).reshape(1, nh, 1, hd))
    hf = apply_rotary_pos_emb(xn, emb.cos()[None], emb.sin()[None], unsqueeze_dim=1)
    np.testing.assert_allclose(got, hf.numpy().ravel(), atol=2e-6)


def test_rope_invariants(oracle):
    nh, hd = 4, 256
    x = synth.rms_normalize_rows(synth.normal(3, nh * hd).reshape(nh, hd)).ravel()
    # position 0: identity
    np.testing.assert_array_equal(oracle.fused_per_head_norm_rope(x, ONES(hd), ROPE_FREQS, nh, hd, 0.0, 0, 1e4, 0),
                                  oracle.fused_per_head_norm_rope(x, ONES(hd), ROPE_FREQS, nh, hd, 0.0, 0, 1e6, 1))
    y = oracle.fused_per_head_norm_rope(x, ONES(hd), ROPE_FREQS, nh, hd, 0.0, 0, 1e4, 0)
    np.testing.assert_allclose(y, cf.rms_norm(x, None, 0.0, hd), atol=1e-6)
    # pair norms preserved
    z = oracle.fused_per_head_norm_rope(x, ONES(hd), ROPE_FREQS, nh, hd, 0.0, 999, 1e4, 0).reshape(nh, hd)
    yr = y.reshape(nh, hd)
    pn = lambda a: a[:, :128] ** 2 + a[:, 128:] ** 2  # noqa: E731
    np.testing.assert_allclose(pn(z), pn(yr), rtol=1e-5, atol=1e-6)
    # global layers with the rope_freqs table: pairs 64..127 are not rotated (1/+Inf = 0)
    g = oracle.fused_per_head_norm_rope(x, ONES(hd), ROPE_FREQS, nh, hd, 0.0, 999, 1e6, 1).reshape(nh, hd)
    np.testing.assert_array_equal(g[:, 64:128], yr[:, 64:128])
    np.testing.assert_array_equal(g[:, 192:], yr[:, 192:])
    assert np.max(np.abs(g[:, :64] - yr[:, :64])) > 0.1


@pytest.mark.parametrize("theta,div,hd", [(1e4, 0, 256), (1e6, 1, 256), (1e6, 0, 512), (1e4, 1, 256)])
def test_rope_inv_freq_table(oracle, theta, div, hd):
    """The angle's position-independent factor, restated in numpy: the same f32 steps."""
    got = oracle.rope_inv_freq(theta, hd, div, ROPE_FREQS if div else None)
    pos = 1
    want = _f32_angles(pos, theta, hd, div)  # f32(1) * freq == freq
    np.testing.assert_array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))
    assert got[0] == (1.0 / ROPE_FREQS[0:1].view(np.float16).astype(np.float32)[0] if div else 1.0)
    # angle = f32(pos) * freq reproduces the norm-rope kernel's rotation exactly
    x = synth.rms_normalize_rows(synth.normal(5, hd).reshape(1, hd)).ravel()
    ang = (np.float32(777) * got).astype(np.float64)
    c, s_ = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    y = cf.rms_norm(x, None, 0.0, hd).astype(np.float32)
    h = hd // 2
    rot = np.concatenate([y[:h] * c - y[h:] * s_, y[:h] * s_ + y[h:] * c])
    np.testing.assert_allclose(oracle.fused_per_head_norm_rope(x, ONES(hd), ROPE_FREQS, 1, hd, 0.0, 777, theta, div),
                               rot, atol=2e-6)


# ---- kv cache store --------------------------------------------------------------

def test_kv_cache_store_rows(oracle):
    nkh, hd, max_seq, pos = 2, 8, 6, 4
    k, v = synth.normal(1, nkh * hd), synth.normal(2, nkh * hd)
    kc0 = np.full(max_seq * nkh * hd, -7.0, np.float32)
    kc, vc = oracle.kv_cache_store(k, v, kc0, kc0, nkh, hd, pos, max_seq)
    kc, vc = kc.reshape(max_seq, nkh * hd), vc.reshape(max_seq, nkh * hd)
    np.testing.assert_array_equal(kc[pos], k)
    np.testing.assert_array_equal(vc[pos], v)
    assert (np.delete(kc, pos, 0) == -7.0).all() and (np.delete(vc, pos, 0) == -7.0).all()


# ---- attention chain --------------------------------------------------------------

def _cache(seed, rows, nkh, hd):
    return synth.rms_normalize_rows(synth.normal(seed, rows * nkh * hd).reshape(rows * nkh, hd)).reshape(rows, nkh, hd)


CHAIN = [(8, 1, 256, 513, 512), (8, 1, 256, 200, 0), (8, 2, 64, 300, 64), (4, 4, 32, 97, 0), (8, 1, 256, 1, 0),
         (8, 1, 256, 512, 512), (8, 1, 256, 1025, 512)]


@pytest.mark.parametrize("nqh,nkh,hd,seq,win", CHAIN)
def test_chain_vs_fp64_sdpa(oracle, nqh, nkh, hd, seq, win):
    kc, vc = _cache(1, seq, nkh, hd), _cache(2, seq, nkh, hd)
    q = synth.rms_normalize_rows(synth.normal(3, nqh * hd).reshape(nqh, hd)).ravel()
    got = oracle.attention_chain(q, kc, vc, nqh, nkh, hd, seq, 1.0, win)
    want = cf.sdpa(q, kc, vc, nqh, nkh, hd, seq, 1.0, win)
    # f32 serial dot products on scores of magnitude ~16^2 carry ~2e-5 of rounding
    np.testing.assert_allclose(got, want, atol=1e-4)


def test_chain_vs_torch_sdpa(oracle):
    """torch's scaled_dot_product_attention (fp64, CPU) with scale=1.0 as a library routine,
    with an explicit sliding-window boolean mask."""
    nqh, nkh, hd, seq, win = 8, 1, 128, 700, 256
    kc, vc = _cache(11, seq, nkh, hd), _cache(12, seq, nkh, hd)
    q = synth.rms_normalize_rows(synth.normal(13, nqh * hd).reshape(nqh, hd)).ravel()
    got = oracle.attention_chain(q, kc, vc, nqh, nkh, hd, seq, 1.0, win).reshape(nqh, hd)
    Q = torch.from_numpy(q.reshape(1, nqh, 1, hd).astype(np.float64))
    K = torch.from_numpy(kc[:, 0, :].astype(np.float64))[None, None].expand(1, nqh, seq, hd)
    V = torch.from_numpy(vc[:, 0, :].astype(np.float64))[None, None].expand(1, nqh, seq, hd)
    mask = torch.zeros(1, 1, 1, seq, dtype=torch.bool)
    mask[..., seq - win:] = True
    ref = torch.nn.functional.scaled_dot_product_attention(Q, K.contiguous(), V.contiguous(), attn_mask=mask,
                                                           scale=1.0)
    np.testing.assert_allclose(got, ref[0, :, 0].numpy(), atol=1e-4)


def test_chain_invariants(oracle):
    nqh, nkh, hd = 8, 1, 64
    # seq = 1: output is the single V row for every head
    kc, vc = _cache(1, 1, nkh, hd), _cache(2, 1, nkh, hd)
    q = synth.normal(3, nqh * hd)
    out = oracle.attention_chain(q, kc, vc, nqh, nkh, hd, 1).reshape(nqh, hd)
    np.testing.assert_array_equal(out, np.broadcast_to(vc[0, 0], (nqh, hd)))
    # all keys equal: mean of V
    seq = 50
    kc = np.broadcast_to(_cache(4, 1, nkh, hd), (seq, nkh, hd)).copy()
    vc = _cache(5, seq, nkh, hd)
    out = oracle.attention_chain(q, kc, vc, nqh, nkh, hd, seq).reshape(nqh, hd)
    np.testing.assert_allclose(out, np.broadcast_to(vc[:, 0].mean(0), (nqh, hd)), atol=1e-6)
    # convex combination: inside the per-dimension hull of V rows
    kc = _cache(6, seq, nkh, hd)
    out = oracle.attention_chain(q, kc, vc, nqh, nkh, hd, seq).reshape(nqh, hd)
    assert (out <= vc[:, 0].max(0) + 1e-6).all() and (out >= vc[:, 0].min(0) - 1e-6).all()
    # identical query heads give identical outputs
    q2 = np.tile(q[:hd], nqh)
    out = oracle.attention_chain(q2, kc, vc, nqh, nkh, hd, seq).reshape(nqh, hd)
    assert (out == out[0]).all()


def test_window_edges(oracle):
    nqh, nkh, hd, W = 8, 1, 64, 16
    for seq in (W - 1, W, W + 1, 3 * W):
        kc, vc = _cache(seq, seq, nkh, hd), _cache(seq + 1, seq, nkh, hd)
        q = synth.rms_normalize_rows(synth.normal(seq + 2, nqh * hd).reshape(nqh, hd)).ravel()
        loc = oracle.attention_chain(q, kc, vc, nqh, nkh, hd, seq, 1.0, W)
        lo = max(0, seq - W)
        # local == global attention over exactly the last W rows
        glob = oracle.attention_chain(q, kc[lo:], vc[lo:], nqh, nkh, hd, seq - lo, 1.0, 0)
        np.testing.assert_allclose(loc, glob, atol=1e-6)
        if seq <= W:
            np.testing.assert_array_equal(loc, oracle.attention_chain(q, kc, vc, nqh, nkh, hd, seq, 1.0, 0))
    # masked scores carry the -1e30 sentinel; the window excludes exactly row 0 at seq = W + 1
    seq = W + 1
    kc = _cache(9, seq, nkh, hd)
    s = oracle.attn_score(synth.normal(1, nqh * hd), kc, nqh, nkh, hd, seq, 1.0, W).reshape(nqh, seq)
    assert (s[:, 0] == np.float32(-1e30)).all() and (s[:, 1:] > -1e29).all()


def test_scores_head_stride_is_seq_len(oracle):
    """scores[head * seq_len + pos] (attn_score.wgsl:22), and kv_head = head * NKH / NQH."""
    nqh, nkh, hd, seq = 4, 2, 8, 5
    kc = _cache(1, seq, nkh, hd)
    q = synth.normal(2, nqh * hd)
    s = oracle.attn_score(q, kc, nqh, nkh, hd, seq, 0.5, 0)
    for h in range(nqh):
        kvh = h * nkh // nqh
        for p in range(seq):
            want = 0.5 * float(np.dot(q[h * hd:(h + 1) * hd].astype(np.float64), kc[p, kvh].astype(np.float64)))
            assert abs(s[h * seq + p] - want) < 1e-5


def test_softmax_rows_sum_to_one(oracle):
    s = (synth.normal(3, 8 * 1000) * 16).astype(np.float32)
    p = oracle.softmax(s, 8, 1000).reshape(8, 1000)
    np.testing.assert_allclose(p.sum(1), 1.0, atol=1e-5)
    e = np.exp(s.reshape(8, 1000).astype(np.float64) - s.reshape(8, 1000).max(1, keepdims=True))
    np.testing.assert_allclose(p, e / e.sum(1, keepdims=True), atol=1e-6)


def test_chain_brute_force_tiny(oracle):
    """head_dim 4, up to 8 rows: pure-Python loops in fp64."""
    import math
    nqh, nkh, hd = 2, 1, 4
    for seq in range(1, 9):
        for win in (0, 3):
            kc, vc = synth.normal(seq, seq * hd).reshape(seq, 1, hd), synth.normal(seq + 50, seq * hd).reshape(seq, 1, hd)
            q = synth.normal(seq + 99, nqh * hd)
            got = oracle.attention_chain(q, kc, vc, nqh, nkh, hd, seq, 1.0, win)
            lo = max(0, seq - win) if win else 0
            for h in range(nqh):
                sc = [sum(float(q[h * hd + d]) * float(kc[p, 0, d]) for d in range(hd)) for p in range(lo, seq)]
                m = max(sc)
                ex = [math.exp(x - m) for x in sc]
                z = sum(ex)
                for d in range(hd):
                    want = sum(ex[i] / z * float(vc[lo + i, 0, d]) for i in range(len(ex)))
                    assert abs(got[h * hd + d] - want) < 1e-5


# ---- argmax / softcap (the top-1 rule) ---------------------------------------------

def test_argmax_tie_rule(oracle):
    x = np.zeros(1000, np.float32)
    x[300] = 5.0
    assert oracle.argmax(x) == 300
    # ties: smallest index modulo 256 wins, not the smallest index
    x = np.zeros(1000, np.float32)
    x[[700, 600]] = 9.0  # 700 % 256 = 188, 600 % 256 = 88
    assert oracle.argmax(x) == 600
    x = np.zeros(1000, np.float32)
    x[[260, 5 + 256 * 3]] = 9.0  # 260 % 256 = 4 < 5
    assert oracle.argmax(x) == 260
    x = np.zeros(1000, np.float32)
    x[[3, 259]] = 9.0  # same residue: each invocation keeps its first maximum
    assert oracle.argmax(x) == 3
    assert oracle.argmax(np.full(10, -2e30, np.float32)) == 0
    rng = np.random.default_rng(1)
    for _ in range(20):
        y = rng.standard_normal(5000).astype(np.float32)
        assert oracle.argmax(y) == int(np.argmax(y))


def test_argmax_tournament_known_answer(oracle):
    """Hand-traced through argmax.wgsl's tree: residues 1 and 4 hold the same maximum. At stride 4
    slot 0 takes residue 4's pair (strictly greater than its own 0); at stride 1 slot 0 (holding 4) meets
    slot 1 (holding residue 1): equal, so slot 0 keeps index 4."""
    x = np.zeros(256, np.float32)
    x[[1, 4]] = 3.0
    assert oracle.argmax(x) == 4
    x[[1, 4]] = 0.0
    x[[6, 9]] = 3.0  # bit-reversed: 6 -> 96, 9 -> 144: 6 wins
    assert oracle.argmax(x) == 6


def test_argmax_closed_form_rule(oracle):
    """The oracle against the loop-free statement of the rule (closed_form.argmax_rule) on inputs with
    many exact ties, NaN and values at or below the -1e30 start."""
    rng = np.random.default_rng(7)
    for trial in range(200):
        n = int(rng.integers(1, 3000))
        x = rng.integers(-3, 4, size=n).astype(np.float32)  # a handful of values: ties everywhere
        if trial % 3 == 0:
            x[rng.integers(0, n, size=max(1, n // 10))] = np.nan
        if trial % 5 == 0:
            x[rng.integers(0, n, size=max(1, n // 3))] = np.float32(-1e30)
        assert oracle.argmax(x) == cf.argmax_rule(x), trial
    assert oracle.argmax(np.array([np.nan, -1e30, -2e30], np.float32)) == 0
    assert cf.argmax_rule(np.array([np.nan, -1e30], np.float32)) == 0


def _f16_bits(a):
    return np.asarray(a, dtype=np.float16).view(np.uint16)


@pytest.mark.parametrize("M,N", [(37, 1536), (5, 300), (64, 2048), (3, 17)])
def test_matmul_quant_closed_form(oracle, M, N):
    rng = np.random.default_rng(M * 1000 + N)
    w = rng.standard_normal((M, N)).astype(np.float16)
    x = rng.standard_normal(N).astype(np.float32)
    got = oracle.matmul_quant(x, _f16_bits(w), M, N)
    want = cf.matvec(w.astype(np.float32), x)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-4 * np.sqrt(N / 256))


def test_matmul_quant_integers_exact(oracle):
    """Small integers: every partial sum is exact, so any order gives the numpy integer product; a dropped
    term, a wrong index or a transposed operand shows up as a difference."""
    rng = np.random.default_rng(3)
    M, N = 50, 1000
    w = rng.integers(-8, 9, size=(M, N))
    x = rng.integers(-8, 9, size=N)
    got = oracle.matmul_quant(x.astype(np.float32), _f16_bits(w.astype(np.float16)), M, N)
    assert np.array_equal(got, (w @ x).astype(np.float32))


def test_matmul_quant_summation_order(oracle):
    """matmul_quant.wgsl's order: invocation 0 adds k = 0 then k = 256 (2^27 - 2^27 = 0 exactly), and the
    tree then adds invocation 128's 1.0: the result is 1. Summing k = 0, 1, 2, ... instead rounds
    2^27 + 1 to 2^27 and gives 0."""
    N = 512
    w = np.zeros((1, N), np.float16)
    w[0, [0, 128, 256]] = 1.0
    x = np.zeros(N, np.float32)
    x[0], x[128], x[256] = 2.0 ** 27, 1.0, -(2.0 ** 27)
    assert oracle.matmul_quant(x, _f16_bits(w), 1, N)[0] == 1.0
    seq = np.float32(0)
    for k in range(N):
        seq = np.float32(seq + np.float32(w[0, k]) * x[k])
    assert seq == 0.0


def _pack_nibbles(nib):
    """[rows][N] values 0..15 -> u32 words, 8 per word, low nibble first (matmul_q4k.wgsl:42-44)."""
    n = np.asarray(nib, dtype=np.uint32).reshape(-1, 8)
    return (n << (4 * np.arange(8, dtype=np.uint32))).sum(axis=1, dtype=np.uint64).astype(np.uint32)


def test_matmul_q8_equals_f16_path_on_exact_weights(oracle):
    """Scales that are powers of two make every dequantized weight int8 * 2^-e exact in f16, so matmul_q8.wgsl
    must equal matmul_quant.wgsl on those f16 weights bit for bit (the per-row order is the same, and matmul_quant
    is pinned by its own tests). Scales differ per 32-block, so a wrong block index breaks the equality."""
    rng = np.random.default_rng(8)
    M, N = 37, 1024
    q = rng.integers(-128, 128, size=(M, N)).astype(np.int8)
    e = rng.integers(0, 6, size=(M, N // 32))
    sc = (2.0 ** -e).astype(np.float16)
    x = rng.standard_normal(N).astype(np.float32)
    got = oracle.matmul_q8(x, q, _f16_bits(sc), M, N)
    w = (q.astype(np.float32) * np.repeat(sc.astype(np.float32), 32, axis=1)).astype(np.float16)
    assert (w.astype(np.float32) == q * np.repeat(sc.astype(np.float32), 32, axis=1)).all()
    want = oracle.matmul_quant(x, _f16_bits(w), M, N)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_matmul_q8_closed_form(oracle):
    rng = np.random.default_rng(9)
    M, N = 64, 2048
    q = rng.integers(-128, 128, size=(M, N)).astype(np.int8)
    sc = (rng.random((M, N // 32)) * 0.02 + 1e-3).astype(np.float16)
    x = rng.standard_normal(N).astype(np.float32)
    got = oracle.matmul_q8(x, q, _f16_bits(sc), M, N)
    w = q.astype(np.float64) * np.repeat(sc.astype(np.float64), 32, axis=1)
    np.testing.assert_allclose(got, w @ x.astype(np.float64), rtol=0, atol=2e-4 * np.sqrt(N / 256))


def test_matmul_q4k_equals_f16_path_on_exact_weights(oracle):
    """Power-of-two scales and small half-integer mins: scale * nibble + min is exact in f16, so matmul_q4k.wgsl
    equals matmul_quant.wgsl on the dequantized weights bit for bit. Scales and mins differ per sub-block and
    super-block, and the nibbles are packed low nibble first: a swapped nibble order, a scale/min mix-up or a
    wrong block index breaks the equality."""
    rng = np.random.default_rng(10)
    M, N = 29, 1536
    nib = rng.integers(0, 16, size=(M, N))
    sb = N // 256
    scales = (2.0 ** -rng.integers(0, 4, size=(M, sb, 8))).astype(np.float16)
    mins = (rng.integers(-8, 9, size=(M, sb, 8)) * 0.5).astype(np.float16)
    meta = np.concatenate([scales, mins], axis=2)  # [M][sb][16]: 8 scales then 8 mins
    x = rng.standard_normal(N).astype(np.float32)
    got = oracle.matmul_q4k(x, _pack_nibbles(nib), _f16_bits(meta), M, N)
    k = np.arange(N)
    s_full = scales.astype(np.float32)[:, k // 256, (k % 256) // 32]
    m_full = mins.astype(np.float32)[:, k // 256, (k % 256) // 32]
    w32 = s_full * nib + m_full
    w = w32.astype(np.float16)
    assert (w.astype(np.float32) == w32).all()
    want = oracle.matmul_quant(x, _f16_bits(w), M, N)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_matmul_q4k_closed_form(oracle):
    rng = np.random.default_rng(11)
    M, N = 40, 2048
    nib = rng.integers(0, 16, size=(M, N))
    sb = N // 256
    meta = np.concatenate([(rng.random((M, sb, 8)) * 0.01).astype(np.float16),
                           (rng.standard_normal((M, sb, 8)) * 0.05).astype(np.float16)], axis=2)
    x = rng.standard_normal(N).astype(np.float32)
    got = oracle.matmul_q4k(x, _pack_nibbles(nib), _f16_bits(meta), M, N)
    k = np.arange(N)
    s_full = meta[:, :, :8].astype(np.float64)[:, k // 256, (k % 256) // 32]
    m_full = meta[:, :, 8:].astype(np.float64)[:, k // 256, (k % 256) // 32]
    np.testing.assert_allclose(got, (s_full * nib + m_full) @ x.astype(np.float64), rtol=0,
                               atol=2e-4 * np.sqrt(N / 256))


def test_softcap_closed_form(oracle):
    x = (synth.normal(4, 4096) * 40).astype(np.float32)
    np.testing.assert_allclose(oracle.logit_softcap(x, 30.0), cf.softcap(x, 30.0), atol=2e-5)
