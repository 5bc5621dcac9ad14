"""GPU parity of attn.linearQKV with the producer-side prep as its epilogue (g4_linear_qkv_prep, one
launch for the dispatches linearQKV -> vNorm -> fusedNormRope(Q) -> fusedNormRope(K) -> kvCacheStore of
src/engine.ts:2045-2091) against the oracle, bit for bit: the raw rows are the oracle's matmulQuant /
matmulQ8 / matmulQ4K; the q / k / v buffers then hold the oracle's fused_per_head_norm_rope (q, k) and
per_head_rms_norm_no_weight (v) of them, and cache row `slot` the f16 rounding of k and v, other rows
untouched. Calls repeat on one workspace (its per-head arrival counters return to zero), across head
dims, head counts and weight formats.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from g4attn import e2b, ops
from helpers import EPS, f16_weight_bits
from oracle import oracle as orc
from test_gpu_linear import q4k_weights, q8_weights, t_f32, t_i8, t_u16, t_u32, weights

pytestmark = pytest.mark.gpu

ROPE = np.array(e2b.rope_freqs_f16_bits(256), dtype=np.uint16)
POISON = 0x5A5A


class Layer:
    def __init__(self, dev, seed, fmt, n, nqh, nkh, hd, store, rows=40):
        self.fmt, self.n, self.nqh, self.nkh, self.hd, self.store, self.rows = fmt, n, nqh, nkh, hd, store, rows
        rng = np.random.default_rng(seed)
        self.x = rng.standard_normal(n, dtype=np.float32)
        self.seg_rows = [nqh * hd] + ([nkh * hd, nkh * hd] if store else [])
        self.w = []  # host copies, per segment
        self.dev_segs = []
        self.outs = [torch.full((r,), float("nan"), device=dev) for r in self.seg_rows]
        for i, r in enumerate(self.seg_rows):
            if fmt == "f16":
                w = weights(seed + 11 * i, r, n)
                self.w.append((w,))
                self.dev_segs.append((t_u16(w, dev), self.outs[i], r))
            elif fmt == "q8":
                q, sc = q8_weights(seed + 11 * i, r, n)
                self.w.append((q, sc))
                self.dev_segs.append((t_i8(q, dev), t_u16(sc, dev), self.outs[i], r))
            else:
                words, meta = q4k_weights(seed + 11 * i, r, n)
                self.w.append((words, meta))
                self.dev_segs.append((t_u32(words, dev), t_u16(meta, dev), self.outs[i], r))
        self.qw, self.kw = f16_weight_bits(seed + 5, hd), f16_weight_bits(seed + 6, hd)
        self.dqw, self.dkw, self.drf = t_u16(self.qw, dev), t_u16(self.kw, dev), t_u16(ROPE, dev)
        self.kc = torch.full((rows * nkh * hd,), POISON, dtype=torch.int16, device=dev)
        self.vc = torch.full_like(self.kc, POISON)
        self.dx = t_f32(self.x, dev)

    def raw(self, i):
        r = self.seg_rows[i]
        if self.fmt == "f16":
            return orc.matmul_quant(self.x, self.w[i][0], r, self.n)
        if self.fmt == "q8":
            return orc.matmul_q8(self.x, self.w[i][0], self.w[i][1], r, self.n)
        return orc.matmul_q4k(self.x, self.w[i][0], self.w[i][1], r, self.n)

    def run_and_check(self, ws, position, slot, theta, div, inv=None):
        ops.linear_qkv_prep(self.dx, self.n, self.fmt, self.dev_segs, self.dqw, self.nqh, self.nkh, self.hd, position,
                            theta, div, ws, k_weight=self.dkw, rope_freqs=self.drf, rope_inv_freq=inv,
                            k_cache=self.kc if self.store else None, v_cache=self.vc if self.store else None,
                            slot=slot, max_seq_len=self.rows)
        torch.cuda.synchronize()
        hd = self.hd
        q = orc.fused_per_head_norm_rope(self.raw(0), self.qw, ROPE, self.nqh, hd, EPS, position, theta, div)
        np.testing.assert_array_equal(self.outs[0].cpu().numpy().view(np.uint32), q.view(np.uint32), err_msg="q")
        kc = self.kc.cpu().numpy().view(np.uint16).reshape(self.rows, -1)
        vc = self.vc.cpu().numpy().view(np.uint16).reshape(self.rows, -1)
        others = np.arange(self.rows) != slot
        if self.store:
            k = orc.fused_per_head_norm_rope(self.raw(1), self.kw, ROPE, self.nkh, hd, EPS, position, theta, div)
            v = orc.per_head_rms_norm_no_weight(self.raw(2), self.nkh, hd, EPS)
            np.testing.assert_array_equal(self.outs[1].cpu().numpy().view(np.uint32), k.view(np.uint32), err_msg="k")
            np.testing.assert_array_equal(self.outs[2].cpu().numpy().view(np.uint32), v.view(np.uint32), err_msg="v")
            np.testing.assert_array_equal(kc[slot], orc.f32_to_f16_bits(k), err_msg="stored k row")
            np.testing.assert_array_equal(vc[slot], orc.f32_to_f16_bits(v), err_msg="stored v row")
            kc, vc = kc[others], vc[others]
        assert (kc == POISON).all() and (vc == POISON).all(), "rows other than the slot written"


CASES = [  # fmt, n, nqh, nkh, hd, store, position, theta, div, inv table
    ("f16", 1536, 8, 1, 256, True, 513, 1e4, 0, False),      # E2B local producer
    ("f16", 1536, 8, 1, 512, True, 8192, 1e6, 1, True),      # E2B global producer (head_dim 512)
    ("f16", 1536, 8, 1, 256, False, 7, 1e4, 0, False),       # KV consumer: q alone
    ("q8", 1536, 8, 1, 256, True, 131071, 1e6, 1, True),
    ("q4k", 2048, 8, 2, 256, True, 4096, 1e6, 1, False),     # two kv heads
    ("q4k", 1536, 8, 1, 512, True, 0, 1e6, 1, True),
    ("f16", 4096, 16, 2, 256, True, 77, 1e4, 0, True),
    ("q8", 1024, 4, 4, 512, False, 300, 1e4, 0, False),
]


@pytest.mark.parametrize("fmt,n,nqh,nkh,hd,store,pos,theta,div,inv", CASES)
def test_linear_qkv_prep_bits(dev, fmt, n, nqh, nkh, hd, store, pos, theta, div, inv):
    announce(f"linearQkvPrep {fmt} n={n} nqh={nqh} nkh={nkh} hd={hd} store={store} pos={pos}")
    L = Layer(dev, 1000 + n + hd + nqh, fmt, n, nqh, nkh, hd, store)
    ws = torch.zeros(ops.qkv_prep_workspace_bytes(nqh, nkh), dtype=torch.uint8, device=dev)
    table = ops.rope_inv_freq(theta, hd, div, L.drf) if inv else None
    L.run_and_check(ws, pos, 17, theta, div, table)
    assert (ws == 0).all(), "arrival counters not returned to zero"


def test_linear_qkv_prep_workspace_reuse(dev):
    """Twelve calls in a row on one workspace: head dims, head counts, formats and layer kinds alternate,
    every call bit-exact (the counters start each call at zero)."""
    announce("linearQkvPrep: one workspace, 12 calls")
    ws = torch.zeros(ops.qkv_prep_workspace_bytes(16, 4), dtype=torch.uint8, device=dev)
    for i in range(12):
        fmt, n, nqh, nkh, hd, store, pos, theta, div, _ = CASES[i % len(CASES)]
        L = Layer(dev, 77 + i, fmt, n, nqh, nkh, hd, store)
        L.run_and_check(ws, pos + i, i % 40, theta, div)
    assert (ws == 0).all()


def test_linear_qkv_prep_rejects(dev):
    from g4attn.abi import G4Error
    L = Layer(dev, 5, "f16", 1536, 8, 1, 256, True)
    ws = torch.zeros(ops.qkv_prep_workspace_bytes(8, 1), dtype=torch.uint8, device=dev)
    with pytest.raises(G4Error):  # slot past the cache
        ops.linear_qkv_prep(L.dx, 1536, "f16", L.dev_segs, L.dqw, 8, 1, 256, 0, 1e4, 0, ws, k_weight=L.dkw,
                            k_cache=L.kc, v_cache=L.vc, slot=40, max_seq_len=40)
    with pytest.raises(G4Error):  # q alone on a producer
        ops.linear_qkv_prep(L.dx, 1536, "f16", L.dev_segs[:1], L.dqw, 8, 1, 256, 0, 1e4, 0, ws, k_weight=L.dkw,
                            k_cache=L.kc, v_cache=L.vc, slot=0, max_seq_len=40)
    with pytest.raises(G4Error):  # head_dim 128
        ops.linear_qkv_prep(L.dx, 1536, "f16", L.dev_segs[:1], L.dqw, 8, 1, 128, 0, 1e4, 0, ws)


@pytest.mark.parametrize("hd,window,theta,div,seq", [(256, 512, 1e4, 0, 700), (512, 0, 1e6, 1, 3000)])
def test_prep_then_step_equals_raw_step(dev, hd, window, theta, div, seq):
    """A producer layer two ways: (a) attn.linearQKV (g4_linear_f16) then the one-launch step on the raw
    projections (norms, RoPE, KV store inside); (b) g4_linear_qkv_prep (projection, norms, RoPE, KV store)
    then the step with q_ready and the current row read from the cache. attnOut and the stored rows are
    bit-identical, and attnOut matches the oracle's chain within 2e-3."""
    announce(f"linearQkvPrep -> attnStep(q_ready) vs linear -> attnStep, hd={hd} seq={seq}")
    from helpers import cache_f16_torch, max_abs
    n, nqh, nkh = 1536, 8, 1
    pos = seq - 1
    L = Layer(dev, 4000 + hd, "f16", n, nqh, nkh, hd, True, rows=seq)
    prior = [cache_f16_torch(4100 + hd + i, seq - 1, nkh, hd, dev).view(torch.int16).reshape(-1) for i in (0, 1)]
    caches = {}
    for way in ("raw", "ready"):
        kc = torch.zeros(seq * nkh * hd, dtype=torch.int16, device=dev)
        vc = torch.zeros_like(kc)
        kc[: (seq - 1) * hd] = prior[0]
        vc[: (seq - 1) * hd] = prior[1]
        caches[way] = (kc, vc)
    outs = {w: torch.full((nqh * hd,), float("nan"), device=dev) for w in caches}
    inv_host = ops.rope_inv_freq_host(theta, hd, div, ROPE)
    # (a) projection, then the step on raw q/k/v
    ops.linear_f16(L.dx, n, [(s[0], s[1], s[2]) for s in L.dev_segs])
    kc, vc = caches["raw"]
    e = dict(q=L.outs[0], k=L.outs[1], v=L.outs[2], q_weight=L.dqw, k_weight=L.dkw, rope_freqs=L.drf,
             rope_inv_freq_host=inv_host, k_cache=kc, v_cache=vc, out=outs["raw"], seq_len=seq, position=pos,
             sliding_window=window, store_kv=True, theta=theta, apply_divisor=div)
    ws = torch.empty(ops.step_workspace_bytes(1, nqh, nkh, hd), dtype=torch.uint8, device=dev)
    ops.attn_step(ops.make_step_entries([e], nqh, nkh, hd), nqh, nkh, hd, ws)
    torch.cuda.synchronize()
    raw_q = L.outs[0].cpu().numpy().copy()
    # (b) the fused projection + prep, then the step with q_ready (the row is in the cache)
    kc, vc = caches["ready"]
    pws = torch.zeros(ops.qkv_prep_workspace_bytes(nqh, nkh), dtype=torch.uint8, device=dev)
    ops.linear_qkv_prep(L.dx, n, "f16", L.dev_segs, L.dqw, nqh, nkh, hd, pos, theta, div, pws, k_weight=L.dkw,
                        rope_freqs=L.drf, k_cache=kc, v_cache=vc, slot=pos, max_seq_len=seq)
    e2 = dict(e, q=L.outs[0], k=None, v=None, k_weight=None, k_cache=kc, v_cache=vc, out=outs["ready"],
              store_kv=False, q_ready=True)
    ops.attn_step(ops.make_step_entries([e2], nqh, nkh, hd), nqh, nkh, hd, ws)
    torch.cuda.synchronize()
    a, b = outs["raw"].cpu().numpy(), outs["ready"].cpu().numpy()
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32), err_msg="attnOut")
    for x, y in zip(caches["raw"], caches["ready"]):
        np.testing.assert_array_equal(x.cpu().numpy(), y.cpu().numpy(), err_msg="caches")
    # the oracle: prep of the raw projections, then the chain over the cache
    q_ = orc.fused_per_head_norm_rope(raw_q, L.qw, ROPE, nqh, hd, EPS, pos, theta, div)
    kb = caches["raw"][0].cpu().numpy().view(np.uint16).reshape(seq, hd)
    vb = caches["raw"][1].cpu().numpy().view(np.uint16).reshape(seq, hd)
    lo = seq - window if window and seq > window else 0
    want = orc.attention_chain(q_, orc.f16_bits_to_f32(kb[lo:]).reshape(-1), orc.f16_bits_to_f32(vb[lo:]).reshape(-1),
                               nqh, nkh, hd, seq - lo, 1.0, 0)
    assert max_abs(a, want) <= 2e-3


@pytest.mark.parametrize("hd,window,theta,div,seq0", [(256, 512, 1e4, 0, 500), (512, 0, 1e6, 1, 990)])
def test_fused_layer_tokens_with_advanced_plan(dev, hd, window, theta, div, seq0):
    """The fully fused engine order over consecutive tokens: per token a new hidden state, g4_linear_qkv_prep
    (projection, norms, RoPE, the K/V row stored at the token's slot), then the attention of a q_ready plan
    prepared at the first token and advanced on the host every token after (g4_attn_step_advance), across the
    window edge (local layer) and a 32-row tile boundary. Each token: q, k, v and the stored row bit-identical
    to the oracle's matmulQuant followed by the reference prep, attnOut within 2e-3 of the oracle's chain over
    the cache as that token leaves it."""
    from helpers import cache_f16_torch, max_abs
    n, nqh, nkh, T = 1536, 8, 1, 40
    announce(f"linearQkvPrep -> attnStep(q_ready, advanced) over {T} tokens, hd={hd} seq0={seq0}")
    rows = seq0 + T
    L = Layer(dev, 5000 + hd, "f16", n, nqh, nkh, hd, True, rows=rows)
    L.kc.copy_(torch.zeros_like(L.kc))
    L.vc.copy_(torch.zeros_like(L.vc))
    L.kc[: (seq0 - 1) * hd] = cache_f16_torch(5100 + hd, seq0 - 1, nkh, hd, dev).view(torch.int16).reshape(-1)
    L.vc[: (seq0 - 1) * hd] = cache_f16_torch(5200 + hd, seq0 - 1, nkh, hd, dev).view(torch.int16).reshape(-1)
    out = torch.full((nqh * hd,), float("nan"), device=dev)
    pws = torch.zeros(ops.qkv_prep_workspace_bytes(nqh, nkh), dtype=torch.uint8, device=dev)
    sws = torch.empty(ops.step_workspace_bytes(1, nqh, nkh, hd), dtype=torch.uint8, device=dev)
    inv_dev = ops.rope_inv_freq(theta, hd, div, L.drf)
    inv_host = ops.rope_inv_freq_host(theta, hd, div, ROPE)
    plan = None
    rng = np.random.default_rng(5300 + hd)
    for t in range(T):
        seq = seq0 + t
        pos = seq - 1
        L.x = rng.standard_normal(n, dtype=np.float32)
        L.dx.copy_(torch.from_numpy(L.x))
        ops.linear_qkv_prep(L.dx, n, "f16", L.dev_segs, L.dqw, nqh, nkh, hd, pos, theta, div, pws, k_weight=L.dkw,
                            rope_freqs=L.drf, rope_inv_freq=inv_dev, k_cache=L.kc, v_cache=L.vc, slot=pos,
                            max_seq_len=rows)
        if plan is None:
            e = dict(q=L.outs[0], k=None, v=None, q_weight=L.dqw, k_weight=None, rope_freqs=L.drf,
                     rope_inv_freq_host=inv_host, k_cache=L.kc, v_cache=L.vc, out=out, seq_len=seq, position=pos,
                     sliding_window=window, store_kv=False, theta=theta, apply_divisor=div, q_ready=True)
            plan = ops.attn_step_prepare(ops.make_step_entries([e], nqh, nkh, hd), nqh, nkh, hd, sws)
        else:
            ops.attn_step_advance(plan, 1)
        ops.attn_step_run(plan)
        torch.cuda.synchronize()
        q = orc.fused_per_head_norm_rope(L.raw(0), L.qw, ROPE, nqh, hd, EPS, pos, theta, div)
        k = orc.fused_per_head_norm_rope(L.raw(1), L.kw, ROPE, nkh, hd, EPS, pos, theta, div)
        v = orc.per_head_rms_norm_no_weight(L.raw(2), nkh, hd, EPS)
        np.testing.assert_array_equal(L.outs[0].cpu().numpy().view(np.uint32), q.view(np.uint32),
                                      err_msg=f"token {t} q")
        kc = L.kc.cpu().numpy().view(np.uint16).reshape(rows, -1)
        vc = L.vc.cpu().numpy().view(np.uint16).reshape(rows, -1)
        np.testing.assert_array_equal(kc[pos], orc.f32_to_f16_bits(k), err_msg=f"token {t} stored k")
        np.testing.assert_array_equal(vc[pos], orc.f32_to_f16_bits(v), err_msg=f"token {t} stored v")
        lo = seq - window if window and seq > window else 0
        want = orc.attention_chain(q, orc.f16_bits_to_f32(kc[lo:seq]).reshape(-1),
                                   orc.f16_bits_to_f32(vc[lo:seq]).reshape(-1), nqh, nkh, hd, seq - lo, 1.0, 0)
        err = max_abs(out.cpu().numpy(), want)
        assert err <= 2e-3, f"token {t}: attnOut max-abs {err}"
