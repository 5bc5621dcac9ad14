"""GPU parity of the chunked prompt prep (g4_attn_prompt_prep) against the oracle, bit for bit.

The engine preps a prompt one token at a time: vNorm -> fusedNormRope(Q) -> fusedNormRope(K) ->
kvCacheStore at each position (src/engine.ts:2460-2479 -> 2056-2091). The chunked prep does every
token of a chunk in one launch. For each token t at position start + t: q_out[t] must equal the f16
rounding of the oracle's fused_per_head_norm_rope(q_t) bit for bit, and on producer layers the cache
rows start + t must equal the f16 rounding of the oracle's normed and rotated k_t and weightless-normed
v_t; rows outside the chunk stay untouched. Then the prepped chunk through g4_attn_prefill is checked
against the oracle's decode chain on the same f16 query (max-abs 2e-3).

With a V^T cache (g4_attn_prompt_prep_vt) the stored V rows also go to their 32-row V^T blocks: element
(row r, d) of kv head h at [h][r / 32][d][r % 32], bit for bit the stored row, the rest of the chunk's last
block 0, every other element untouched; a prompt prepped and prefilled chunk by chunk through its V^T
cache (no transposition in the prefill) is checked against the oracle's decode chain.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from g4attn import e2b, ops, synth
from helpers import EPS, f16_weight_bits, max_abs
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

ROPE = np.array(e2b.rope_freqs_f16_bits(256), dtype=np.uint16)
POISON = 0x5A5A


def t16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16).reshape(-1)).to(dev)


class Chunk:
    def __init__(self, dev, seed, start, T, hd, theta, div, nqh=8, nkh=1, store=True, vt=False):
        self.start, self.T, self.hd, self.theta, self.div, self.nqh, self.nkh = start, T, hd, theta, div, nqh, nkh
        self.q = synth.normal(seed, T * nqh * hd) * 2.0
        self.k = synth.normal(seed + 1, T * nkh * hd) * 2.0
        self.v = synth.normal(seed + 2, T * nkh * hd) * 2.0
        self.qw, self.kw = f16_weight_bits(seed + 3, hd), f16_weight_bits(seed + 4, hd)
        self.rows = start + T + 3
        self.dq, self.dk, self.dv = (torch.from_numpy(x.copy()).to(dev) for x in (self.q, self.k, self.v))
        self.q_out = torch.full((T * nqh * hd,), POISON, dtype=torch.int16, device=dev)
        self.kc = torch.full((self.rows * nkh * hd,), POISON, dtype=torch.int16, device=dev)
        self.vc = torch.full_like(self.kc, POISON)
        self.store = store
        self.vt = torch.full((ops.vt_cache_elems(self.rows, nkh, hd),), POISON, dtype=torch.int16,
                             device=dev) if vt else None
        self.dqw, self.dkw, self.drf = t16(self.qw, dev), t16(self.kw, dev), t16(ROPE, dev)

    def kwargs(self, inv_table=False):
        """attn_prompt_prep's arguments for this chunk. inv_table: pass the layer's inverse-frequency table from
        g4_rope_inv_freq instead of letting each workgroup evaluate it."""
        kw = dict(k=self.dk, v=self.dv, k_weight=self.dkw, k_cache=self.kc, v_cache=self.vc,
                  max_seq_len=self.rows, vt_cache=self.vt) if self.store else {}
        inv = ops.rope_inv_freq(self.theta, self.hd, self.div, self.drf) if inv_table else None
        return dict(q=self.dq, q_weight=self.dqw, q_out=self.q_out, n_tokens=self.T, start=self.start,
                    num_q_heads=self.nqh, num_kv_heads=self.nkh, head_dim=self.hd, theta=self.theta,
                    apply_divisor=self.div, rope_freqs=self.drf, eps=EPS, rope_inv_freq=inv, **kw)

    def run(self, inv_table=False):
        ops.attn_prompt_prep(**self.kwargs(inv_table))
        torch.cuda.synchronize()

    def expected(self):
        hd, nqh, nkh = self.hd, self.nqh, self.nkh
        qo = np.empty((self.T, nqh * hd), np.uint16)
        ko = np.empty((self.T, nkh * hd), np.uint16)
        vo = np.empty((self.T, nkh * hd), np.uint16)
        for t in range(self.T):
            pos = self.start + t
            qt = self.q[t * nqh * hd:(t + 1) * nqh * hd]
            qo[t] = orc.f32_to_f16_bits(orc.fused_per_head_norm_rope(qt, self.qw, ROPE, nqh, hd, EPS, pos,
                                                                     self.theta, self.div))
            kt = self.k[t * nkh * hd:(t + 1) * nkh * hd]
            vt = self.v[t * nkh * hd:(t + 1) * nkh * hd]
            ko[t] = orc.f32_to_f16_bits(orc.fused_per_head_norm_rope(kt, self.kw, ROPE, nkh, hd, EPS, pos,
                                                                     self.theta, self.div))
            vo[t] = orc.f32_to_f16_bits(orc.per_head_rms_norm_no_weight(vt, nkh, hd, EPS))
        return qo, ko, vo

    def check(self):
        qo, ko, vo = self.expected()
        got_q = self.q_out.cpu().numpy().view(np.uint16).reshape(self.T, -1)
        np.testing.assert_array_equal(got_q, qo, err_msg="q_out")
        kc = self.kc.cpu().numpy().view(np.uint16).reshape(self.rows, -1)
        vc = self.vc.cpu().numpy().view(np.uint16).reshape(self.rows, -1)
        s, e = self.start, self.start + self.T
        if self.store:
            np.testing.assert_array_equal(kc[s:e], ko, err_msg="k rows")
            np.testing.assert_array_equal(vc[s:e], vo, err_msg="v rows")
        else:
            assert (kc[s:e] == POISON).all() and (vc[s:e] == POISON).all(), "consumer layer stored rows"
        for c, name in ((kc, "k"), (vc, "v")):
            assert (c[:s] == POISON).all() and (c[e:] == POISON).all(), f"{name} rows outside the chunk written"
        if self.vt is not None:  # [kv head][block][d][32]
            nb = (self.rows + 31) // 32
            vt = self.vt.cpu().numpy().view(np.uint16).reshape(self.nkh, nb, self.hd, 32)
            want = np.full_like(vt, POISON)
            vrows = vo.reshape(self.T, self.nkh, self.hd)
            for t in range(self.T):
                r = s + t
                want[:, r // 32, :, r % 32] = vrows[t]
            for r in range(e, (e + 31) // 32 * 32):  # the rest of the last block
                want[:, r // 32, :, r % 32] = 0
            np.testing.assert_array_equal(vt, want, err_msg="V^T blocks")


@pytest.mark.parametrize("start,T,hd,theta,div,inv_table,vt", [
    (0, 512, 256, 1e4, 0, False, False),            # local layer, the first chunk
    (131071 - 511, 512, 256, 1e6, 1, False, False),  # global layer, positions up to 131071
    (4096, 512, 512, 1e6, 1, False, False),         # E2B global layer (head_dim 512)
    (77, 5, 256, 1e4, 0, False, False),             # a short ragged chunk
    (60000, 512, 256, 1e4, 0, True, False),         # the inverse frequencies from the caller's table
    (131071 - 511, 512, 256, 1e6, 1, True, False),
    (4096, 512, 512, 1e6, 1, True, False),
    (0, 512, 256, 1e4, 0, True, True),              # V^T blocks: aligned chunk
    (77, 5, 256, 1e4, 0, True, True),               # inside one block
    (45, 70, 256, 1e6, 1, True, True),              # unaligned start and end, three blocks
    (4096 + 19, 301, 512, 1e6, 1, True, True),      # head_dim 512
    (131071 - 300, 300, 256, 1e6, 1, True, True),   # ending at position 131070
])
def test_prompt_prep_bit_exact(dev, start, T, hd, theta, div, inv_table, vt):
    announce(f"attnPromptPrep start={start} T={T} hd={hd} theta={theta} table={inv_table} vt={vt}")
    c = Chunk(dev, 500 + start + hd, start, T, hd, theta, div, vt=vt)
    c.run(inv_table)
    c.check()


@pytest.mark.parametrize("hd", [256, 512])
def test_prompt_prep_many_in_one_launch(dev, hd):
    """g4_attn_prompt_prep_many: chunks of different starts and lengths, producers with and without V^T blocks,
    a consumer, local and global layers and a 4:1 group over two kv heads, in one launch; every chunk bit for
    bit as its own call gives it (the oracle's bits)."""
    announce(f"attnPromptPrepMany hd={hd}")
    chunks = [Chunk(dev, 800 + hd, 0, 512, hd, 1e4, 0, vt=True),
              Chunk(dev, 801 + hd, 4096 + 19, 301, hd, 1e6, 1, vt=True),
              Chunk(dev, 802 + hd, 77, 5, hd, 1e4, 0),
              Chunk(dev, 803 + hd, 300, 64, hd, 1e4, 0, store=False),
              Chunk(dev, 804 + hd, 33, 90, hd, 1e6, 1, nqh=8, nkh=2, vt=True),
              Chunk(dev, 805 + hd, 131071 - 300, 300, hd, 1e6, 1)]
    ops.attn_prompt_prep_many([c.kwargs(inv_table=(i % 2 == 0)) for i, c in enumerate(chunks)])
    torch.cuda.synchronize()
    for c in chunks:
        c.check()


def test_prompt_prep_many_refuses(dev):
    """Mixed head_dims and more than eight entries are refused before anything is enqueued."""
    a, b = Chunk(dev, 900, 0, 8, 256, 1e4, 0), Chunk(dev, 901, 0, 8, 512, 1e4, 0)
    with pytest.raises(RuntimeError, match="head_dim"):
        ops.attn_prompt_prep_many([a.kwargs(), b.kwargs()])
    with pytest.raises(RuntimeError, match="max 8"):
        ops.attn_prompt_prep_many([a.kwargs()] * 9)


def test_prompt_prep_consumer_and_gqa(dev):
    """A KV-consumer layer (q only) and a 4:1 group with two kv heads."""
    announce("attnPromptPrep consumer layer; nqh=8 nkh=2")
    c = Chunk(dev, 71, 300, 64, 256, 1e4, 0, store=False)
    c.run()
    c.check()
    g = Chunk(dev, 72, 0, 40, 256, 1e6, 1, nqh=8, nkh=2)
    g.run()
    g.check()
    g = Chunk(dev, 74, 33, 90, 256, 1e6, 1, nqh=8, nkh=2, vt=True)  # two kv heads' V^T blocks
    g.run()
    g.check()


def test_prompt_prep_rejects(dev):
    from g4attn.abi import G4Error
    c = Chunk(dev, 73, 10, 8, 256, 1e4, 0)
    with pytest.raises(G4Error):  # rows past the cache
        ops.attn_prompt_prep(c.dq, c.dqw, c.q_out, c.T, c.rows, 8, 1, 256, 1e4, 0, k=c.dk, v=c.dv, k_weight=c.dkw,
                             k_cache=c.kc, v_cache=c.vc, max_seq_len=c.rows)
    with pytest.raises(G4Error):  # head_dim 128
        ops.attn_prompt_prep(c.dq, c.dqw, c.q_out, 1, 0, 8, 1, 128, 1e4, 0)


def test_prompt_prep_then_prefill(dev):
    """Two 256-token chunks of a global layer: each chunk prepped (q, k, v norm/RoPE, K/V stored) then run
    through the prefill; tokens checked against the oracle's per-token decode chain on the stored rows."""
    announce("attnPromptPrep + attnPrefill, two chunks")
    T, hd, theta, div = 256, 256, 1e6, 1
    rows = 2 * T
    qw, kw = f16_weight_bits(81, hd), f16_weight_bits(82, hd)
    kc = torch.zeros(rows * hd, dtype=torch.int16, device=dev)
    vc = torch.zeros_like(kc)
    out = torch.full((rows * 8 * hd,), float("nan"), dtype=torch.float32, device=dev)
    qbits = torch.empty(rows * 8 * hd, dtype=torch.int16, device=dev)
    dqw, dkw, drf = t16(qw, dev), t16(kw, dev), t16(ROPE, dev)
    q = synth.normal(83, rows * 8 * hd)
    k = synth.normal(84, rows * hd)
    v = synth.normal(85, rows * hd)
    for c in range(2):
        s = c * T
        dq = torch.from_numpy(q[s * 8 * hd:(s + T) * 8 * hd].copy()).to(dev)
        dk = torch.from_numpy(k[s * hd:(s + T) * hd].copy()).to(dev)
        dv = torch.from_numpy(v[s * hd:(s + T) * hd].copy()).to(dev)
        ops.attn_prompt_prep(dq, dqw, qbits[s * 8 * hd:], T, s, 8, 1, hd, theta, div, rope_freqs=drf, k=dk, v=dv,
                             k_weight=dkw, k_cache=kc, v_cache=vc, max_seq_len=rows, eps=EPS)
        e = dict(q=qbits[s * 8 * hd:], k_cache=kc, v_cache=vc, out=out[s * 8 * hd:], n_tokens=T, start=s,
                 sliding_window=0, scale=1.0)
        arr = ops.make_prefill_entries([e], 8, 1, hd)
        ws = torch.empty(max(ops.prefill_workspace_bytes(arr, 8, 1, hd), 1), dtype=torch.uint8, device=dev)
        ops.attn_prefill(arr, 8, 1, hd, ws)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(rows, -1)
    kf = orc.f16_bits_to_f32(kc.cpu().numpy().view(np.uint16)).reshape(rows, hd)
    vf = orc.f16_bits_to_f32(vc.cpu().numpy().view(np.uint16)).reshape(rows, hd)
    worst = 0.0
    for t in list(range(0, rows, 7)) + [rows - 1]:
        qt = orc.fused_per_head_norm_rope(q[t * 8 * hd:(t + 1) * 8 * hd], qw, ROPE, 8, hd, EPS, t, theta, div)
        qt = orc.f16_bits_to_f32(orc.f32_to_f16_bits(qt))  # the prefill's query operand is f16
        want = orc.attention_chain(qt, kf[:t + 1].reshape(-1), vf[:t + 1].reshape(-1), 8, 1, hd, t + 1, 1.0, 0)
        err = max_abs(got[t], want)
        assert err <= 2e-3, f"token {t}: max-abs {err}"
        worst = max(worst, err)
    print(f"prep + prefill: worst err {worst:.2e}")


@pytest.mark.parametrize("hd,window", [(256, 0), (256, 96), (512, 0)])
def test_prompt_chunks_through_vt_cache(dev, hd, window):
    """A 700-token prompt as chunks of 200, 150, 37 and 313 tokens: each chunk prepped with its V rows
    also written to the V^T cache, then prefilled reading V from that cache (its attended rows come from
    every earlier chunk's prep); every 5th token against the oracle's decode chain."""
    announce(f"attnPromptPrepVt + attnPrefill through the V^T cache, hd={hd} window={window}")
    sizes = [200, 150, 37, 313]
    rows, nqh, theta, div = sum(sizes), 8, (1e4 if window else 1e6), (0 if window else 1)
    qw, kw = f16_weight_bits(91, hd), f16_weight_bits(92, hd)
    kc = torch.zeros(rows * hd, dtype=torch.int16, device=dev)
    vc = torch.zeros_like(kc)
    vt = torch.full((ops.vt_cache_elems(rows, 1, hd),), POISON, dtype=torch.int16, device=dev)
    out = torch.full((rows * nqh * hd,), float("nan"), dtype=torch.float32, device=dev)
    qbits = torch.empty(rows * nqh * hd, dtype=torch.int16, device=dev)
    dqw, dkw, drf = t16(qw, dev), t16(kw, dev), t16(ROPE, dev)
    q = synth.normal(93, rows * nqh * hd)
    k = synth.normal(94, rows * hd)
    v = synth.normal(95, rows * hd)
    s = 0
    for T in sizes:
        dq = torch.from_numpy(q[s * nqh * hd:(s + T) * nqh * hd].copy()).to(dev)
        dk = torch.from_numpy(k[s * hd:(s + T) * hd].copy()).to(dev)
        dv = torch.from_numpy(v[s * hd:(s + T) * hd].copy()).to(dev)
        ops.attn_prompt_prep(dq, dqw, qbits[s * nqh * hd:], T, s, nqh, 1, hd, theta, div, rope_freqs=drf, k=dk, v=dv,
                             k_weight=dkw, k_cache=kc, v_cache=vc, max_seq_len=rows, eps=EPS, vt_cache=vt)
        e = dict(q=qbits[s * nqh * hd:], k_cache=kc, v_cache=vc, out=out[s * nqh * hd:], n_tokens=T, start=s,
                 sliding_window=window, scale=1.0, vt_cache=vt, vt_rows=rows)
        arr = ops.make_prefill_entries([e], nqh, 1, hd)
        ws = torch.empty(max(ops.prefill_workspace_bytes(arr, nqh, 1, hd), 1), dtype=torch.uint8, device=dev)
        ops.attn_prefill(arr, nqh, 1, hd, ws)
        torch.cuda.synchronize()
        s += T
    got = out.cpu().numpy().reshape(rows, -1)
    kf = orc.f16_bits_to_f32(kc.cpu().numpy().view(np.uint16)).reshape(rows, hd)
    vf = orc.f16_bits_to_f32(vc.cpu().numpy().view(np.uint16)).reshape(rows, hd)
    worst = 0.0
    for t in list(range(0, rows, 5)) + [rows - 1]:
        qt = orc.fused_per_head_norm_rope(q[t * nqh * hd:(t + 1) * nqh * hd], qw, ROPE, nqh, hd, EPS, t, theta, div)
        qt = orc.f16_bits_to_f32(orc.f32_to_f16_bits(qt))  # the prefill's query operand is f16
        lo = t + 1 - window if window and t + 1 > window else 0
        want = orc.attention_chain(qt, kf[lo:t + 1].reshape(-1), vf[lo:t + 1].reshape(-1), nqh, 1, hd, t + 1 - lo,
                                   1.0, 0)
        err = max_abs(got[t], want)
        assert np.isfinite(got[t]).all() and err <= 2e-3, f"token {t}: max-abs {err}"
        worst = max(worst, err)
    print(f"chunks through the V^T cache: worst err {worst:.2e}")
