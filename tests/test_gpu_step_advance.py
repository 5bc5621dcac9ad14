"""GPU parity of g4_attn_step_advance: a step plan prepared once and then advanced token by token
(the engine patches the position, slot and seq_len uniforms every token, src/engine.ts:1967-1987)
against a fresh prepare at every token, and against the oracle.

Bit-exact bar: while the prepared partition is also the one a fresh prepare picks (a windowed layer
past its window; a full layer while its rows stay within the prepared number of 32-row tiles), the
advanced step and the freshly prepared one run the same parts, so attnOut and the stored K/V rows must
be bit-identical. The advanced plan evaluates the RoPE factors in the kernel (the uploaded inverse
frequencies, cos and sin in f64 rounded to f32) while the fresh prepare evaluates them on the host, so
this pins the kernel's evaluation against the host's (the C library's) at every position run, up to
131071. Across tile boundaries and while a window fills up the partitions differ; there attnOut is
checked against the oracle's reference chain within 2e-3 and every stored row bit for bit.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from g4attn import abi, e2b, ops, synth
from helpers import EPS, cache_f16_torch, f16_weight_bits, max_abs
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL = 2e-3
NQH, NKH, HD = 8, 1, 256
ROPE = np.array(e2b.rope_freqs_f16_bits(256), dtype=np.uint16)


def t16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)


class Stream:
    """One entry over a run of tokens: cache capacity for every token, raw q/k/v buffers rewritten
    per token, and the entry dict at the token the run starts with."""

    def __init__(self, dev, seed, seq0, tokens, window, theta, divisor, host_table, hd=HD):
        self.seed, self.seq0, self.window, self.theta, self.divisor, self.hd = seed, seq0, window, theta, divisor, hd
        rows = seq0 + tokens
        kc = torch.zeros((rows, NKH * hd), dtype=torch.int16, device=dev)
        vc = torch.zeros_like(kc)
        if seq0 > 1:  # rows before the first token's own
            kc[: seq0 - 1] = cache_f16_torch(seed + 5, seq0 - 1, NKH, hd, dev).view(torch.int16).view(seq0 - 1, -1)
            vc[: seq0 - 1] = cache_f16_torch(seed + 6, seq0 - 1, NKH, hd, dev).view(torch.int16).view(seq0 - 1, -1)
        self.kc, self.vc = kc, vc
        self.qw, self.kw = f16_weight_bits(seed + 3, hd), f16_weight_bits(seed + 4, hd)
        self.dqw, self.dkw, self.drf = t16(self.qw, dev), t16(self.kw, dev), t16(ROPE, dev)
        self.inv = ops.rope_inv_freq_host(theta, hd, divisor, ROPE) if host_table else None
        self.d = {n: torch.empty(m * hd, device=dev) for n, m in (("q", NQH), ("k", NKH), ("v", NKH))}
        self.out = torch.full((NQH * hd,), float("nan"), device=dev)

    def raw(self, t):
        """The token's raw projections (seeded per token)."""
        return {n: synth.normal(self.seed + 1000 * (t + 1) + i, m * self.hd) * 2.0
                for i, (n, m) in enumerate((("q", NQH), ("k", NKH), ("v", NKH)))}

    def load_raw(self, t):
        r = self.raw(t)
        for n, x in r.items():
            self.d[n].copy_(torch.from_numpy(x))
        return r

    def entry(self, t, out=None, kc=None, vc=None):
        seq = self.seq0 + t
        return dict(q=self.d["q"], k=self.d["k"], v=self.d["v"], q_weight=self.dqw, k_weight=self.dkw,
                    rope_freqs=self.drf, rope_inv_freq_host=self.inv, k_cache=self.kc if kc is None else kc,
                    v_cache=self.vc if vc is None else vc, out=self.out if out is None else out, seq_len=seq,
                    position=seq - 1, sliding_window=self.window, store_kv=True, theta=self.theta,
                    apply_divisor=self.divisor)

    def expected(self, t, r):
        """The oracle's chain at token t over the cache as the GPU holds it (earlier tokens' rows were
        stored by earlier steps) with the current row RNE of the oracle's k/v."""
        seq, pos, hd = self.seq0 + t, self.seq0 + t - 1, self.hd
        v_ = orc.per_head_rms_norm_no_weight(r["v"], NKH, hd, EPS)
        k_ = orc.fused_per_head_norm_rope(r["k"], self.kw, ROPE, NKH, hd, EPS, pos, self.theta, self.divisor)
        q_ = orc.fused_per_head_norm_rope(r["q"], self.qw, ROPE, NQH, hd, EPS, pos, self.theta, self.divisor)
        lo = seq - self.window if self.window and seq > self.window else 0
        kb = self.kc[lo:seq].cpu().numpy().view(np.uint16).copy()
        vb = self.vc[lo:seq].cpu().numpy().view(np.uint16).copy()
        kbits, vbits = orc.f32_to_f16_bits(k_), orc.f32_to_f16_bits(v_)
        kb[-1], vb[-1] = kbits, vbits
        out = orc.attention_chain(q_, orc.f16_bits_to_f32(kb).reshape(-1), orc.f16_bits_to_f32(vb).reshape(-1),
                                  NQH, NKH, hd, seq - lo, 1.0, 0)
        return out, kbits, vbits


def prepare(dev, entries, hd=HD):
    arr = ops.make_step_entries(entries, NQH, NKH, hd)
    ws = torch.empty(ops.step_workspace_bytes(len(entries), NQH, NKH, hd), dtype=torch.uint8, device=dev)
    return ops.attn_step_prepare(arr, NQH, NKH, hd, ws), ws


# (seed, first seq_len, window, theta, divisor, host RoPE table). Full layers start one row past a
# multiple of 32, so 31 tokens stay inside the prepared tiles; the windowed ones are past their window.
SAME_PARTS = [(11, 4097, 0, 1e6, 1, True), (12, 2049, 512, 1e4, 0, True), (13, 1025, 0, 1e6, 1, False),
              (14, 120001, 512, 1e4, 0, True), (15, 131041, 0, 1e6, 1, True), (16, 65, 0, 1e4, 0, True)]


def test_advance_bit_identical_to_fresh_prepare(dev):
    """31 tokens: one plan advanced every token against a fresh prepare every token (own caches)."""
    announce("attnStep advance: 31 tokens against a fresh prepare per token")
    T = 31
    streams = [Stream(dev, *p[:1], p[1], T, *p[2:]) for p in SAME_PARTS]
    fresh_k = [s.kc.clone() for s in streams]
    fresh_v = [s.vc.clone() for s in streams]
    fresh_out = [torch.full_like(s.out, float("nan")) for s in streams]
    plan, ws = None, None
    for t in range(T):
        for s in streams:
            s.load_raw(t)
        if t == 0:
            plan, ws = prepare(dev, [s.entry(0) for s in streams])
        else:
            ops.attn_step_advance(plan, 1)
        ops.attn_step_run(plan)
        fplan, fws = prepare(dev, [s.entry(t, fresh_out[i], fresh_k[i], fresh_v[i]) for i, s in enumerate(streams)])
        ops.attn_step_run(fplan)
        torch.cuda.synchronize()
        for i, s in enumerate(streams):
            row = s.seq0 + t - 1
            a, b = s.out.cpu().numpy(), fresh_out[i].cpu().numpy()
            assert np.isfinite(a).all(), (t, i)
            np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32), err_msg=f"token {t} entry {i} attnOut")
            np.testing.assert_array_equal(s.kc[row].cpu().numpy(), fresh_k[i][row].cpu().numpy(),
                                          err_msg=f"token {t} entry {i} K row")
            np.testing.assert_array_equal(s.vc[row].cpu().numpy(), fresh_v[i][row].cpu().numpy(),
                                          err_msg=f"token {t} entry {i} V row")
        del fws


def test_advance_pair_bit_identical_to_fresh_prepare(dev):
    """A token of two head_dims run as one pair launch (g4_attn_step_run_pair): both plans advanced every
    token give the bits of both plans prepared fresh every token, run as a pair too (12 tokens)."""
    announce("attnStep advance: head_dim 256 and 512 plans as one pair launch, against fresh prepares")
    T = 12
    groups = {hd: [Stream(dev, 300 + 10 * i + hd, seq0, T, w, th, dv, tab, hd=hd)
                   for i, (_, seq0, w, th, dv, tab) in enumerate(SAME_PARTS)] for hd in (256, 512)}
    fresh = {hd: [(s.kc.clone(), s.vc.clone(), torch.full_like(s.out, float("nan"))) for s in ss]
             for hd, ss in groups.items()}
    plans = {}
    for t in range(T):
        for ss in groups.values():
            for s in ss:
                s.load_raw(t)
        for hd, ss in groups.items():
            if t == 0:
                plans[hd] = prepare(dev, [s.entry(0) for s in ss], hd)
            else:
                ops.attn_step_advance(plans[hd][0], 1)
        ops.attn_step_run_pair(plans[512][0], plans[256][0])
        fp = {hd: prepare(dev, [s.entry(t, o, k, v) for s, (k, v, o) in zip(ss, fresh[hd])], hd)
              for hd, ss in groups.items()}
        ops.attn_step_run_pair(fp[256][0], fp[512][0])
        torch.cuda.synchronize()
        for hd, ss in groups.items():
            for i, s in enumerate(ss):
                k, v, o = fresh[hd][i]
                row = s.seq0 + t - 1
                a_, b_ = s.out.cpu().numpy(), o.cpu().numpy()
                assert np.isfinite(a_).all(), (t, hd, i)
                np.testing.assert_array_equal(a_.view(np.uint32), b_.view(np.uint32), err_msg=f"t {t} hd {hd} {i}")
                np.testing.assert_array_equal(s.kc[row].cpu().numpy(), k[row].cpu().numpy(), err_msg=f"K {t} {hd} {i}")
                np.testing.assert_array_equal(s.vc[row].cpu().numpy(), v[row].cpu().numpy(), err_msg=f"V {t} {hd} {i}")
        del fp


# (seed, first seq_len, window, theta, divisor, host table): tile boundaries crossed, windows filling up
CROSSING = [(21, 60, 0, 1e6, 1, True), (22, 40, 64, 1e4, 0, True), (23, 500, 512, 1e4, 0, True),
            (24, 1, 0, 1e4, 0, False), (25, 200, 96, 1e6, 1, True)]


def test_advance_across_tiles_and_windows(dev):
    """150 tokens from one prepare: every token's attnOut against the oracle, every stored row bit for bit."""
    announce("attnStep advance: 150 tokens across tile boundaries and window fills, against the oracle")
    T = 150
    streams = [Stream(dev, p[0], p[1], T, *p[2:]) for p in CROSSING]
    plan = ws = None
    worst = 0.0
    for t in range(T):
        raws = [s.load_raw(t) for s in streams]
        if t == 0:
            plan, ws = prepare(dev, [s.entry(0) for s in streams])
        else:
            ops.attn_step_advance(plan, 1)
        ops.attn_step_run(plan)
        torch.cuda.synchronize()
        for i, (s, r) in enumerate(zip(streams, raws)):
            want, kbits, vbits = s.expected(t, r)
            got = s.out.cpu().numpy()
            assert np.isfinite(got).all(), (t, i)
            err = max_abs(got, want)
            worst = max(worst, err)
            assert err <= TOL, f"token {t} entry {i}: max-abs {err}"
            row = s.seq0 + t - 1
            np.testing.assert_array_equal(s.kc[row].cpu().numpy().view(np.uint16), kbits, err_msg=f"token {t} K")
            np.testing.assert_array_equal(s.vc[row].cpu().numpy().view(np.uint16), vbits, err_msg=f"token {t} V")
    print(f"worst max-abs over {T} tokens: {worst:.2e}")


def test_advance_layers_and_merge_paths(dev):
    """Plans of g4_attn_step_prepare_layers advanced per token, run in layer order with the merge launch
    and with the merge folded into o_proj: a KV producer (local), its consumer (k/v NULL, reading the
    producer's stored row) and a global layer split into many parts."""
    announce("attnStep advance: prepare_layers plans, 40 tokens, merge launch and o_proj forms")
    T = 40
    prod = Stream(dev, 31, 700, T, 512, 1e4, 0, True)
    glob = Stream(dev, 33, 9000, T, 0, 1e6, 1, True)
    cons_q = torch.empty(NQH * HD, device=dev)
    cons_out = torch.full((NQH * HD,), float("nan"), device=dev)
    cons_qw = f16_weight_bits(35, HD)
    hidden = 1536
    g = torch.Generator(device=dev)
    g.manual_seed(77)
    wo = (torch.randn(hidden, NQH * HD, generator=g, device=dev) * 0.02).half().view(torch.int16)
    y = torch.empty(hidden, device=dev)
    plans = ws = None
    for t in range(T):
        rp, rg = prod.load_raw(t), glob.load_raw(t)
        cq = synth.normal(36 + 1000 * t, NQH * HD) * 2.0
        cons_q.copy_(torch.from_numpy(cq))
        ce = prod.entry(t, out=cons_out)
        ce.update(q=cons_q, q_weight=t16(cons_qw, dev), k=None, v=None, k_weight=None, store_kv=False)
        if t == 0:
            ents = [prod.entry(0), ce, glob.entry(0)]
            arr = ops.make_step_entries(ents, NQH, NKH, HD)
            ws = torch.empty(ops.step_layers_workspace_bytes(3, NQH, NKH, HD), dtype=torch.uint8, device=dev)
            plans = ops.attn_step_prepare_layers(arr, NQH, NKH, HD, ws)
        else:
            for p in plans:
                ops.attn_step_advance(p, 1)
        for i, p in enumerate(plans):  # engine order: the producer stores its row before the consumer reads it
            ops.attn_step_run_attention(p)
            if i == 2 and t % 2:
                ops.attn_step_run_out(p, NQH * HD, [(wo, y, hidden)])
            else:
                ops.attn_step_run_merge(p)
        torch.cuda.synchronize()
        want_p, kbits, vbits = prod.expected(t, rp)
        want_g, gk, gv = glob.expected(t, rg)
        # the consumer: its own q over the producer's rows (the current row is the producer's stored one)
        seq, pos = prod.seq0 + t, prod.seq0 + t - 1
        q_ = orc.fused_per_head_norm_rope(cq, cons_qw, ROPE, NQH, HD, EPS, pos, 1e4, 0)
        lo = seq - 512 if seq > 512 else 0
        kb = orc.f16_bits_to_f32(prod.kc[lo:seq].cpu().numpy().view(np.uint16)).reshape(-1)
        vb = orc.f16_bits_to_f32(prod.vc[lo:seq].cpu().numpy().view(np.uint16)).reshape(-1)
        want_c = orc.attention_chain(q_, kb, vb, NQH, NKH, HD, seq - lo, 1.0, 0)
        for name, got, want in (("producer", prod.out, want_p), ("consumer", cons_out, want_c),
                                ("global", glob.out, want_g)):
            err = max_abs(got.cpu().numpy(), want)
            assert err <= TOL, f"token {t} {name}: max-abs {err}"
        np.testing.assert_array_equal(prod.kc[pos].cpu().numpy().view(np.uint16), kbits)
        np.testing.assert_array_equal(glob.vc[glob.seq0 + t - 1].cpu().numpy().view(np.uint16), gv)
        if t % 2:  # o_proj with the merge folded in: rows over the merged attnOut
            want_y = orc.matmul_quant(glob.out.cpu().numpy(), wo.cpu().numpy().view(np.uint16), hidden, NQH * HD)
            np.testing.assert_array_equal(y.cpu().numpy(), want_y, err_msg=f"token {t} o_proj")


def test_advance_limits(dev):
    announce("attnStep advance: limits")
    s = Stream(dev, 41, 100, 1, 0, 1e4, 0, True)
    plan, ws = prepare(dev, [s.entry(0)])
    ops.attn_step_advance(plan, 4000)
    ops.attn_step_advance(plan, 96)  # 4096 in all
    with pytest.raises(abi.G4Error) as ei:
        ops.attn_step_advance(plan, 1)
    assert ei.value.status == abi.G4_ERANGE and "prepare again" in str(ei.value)
    with pytest.raises(abi.G4Error):
        ops.attn_step_advance(ops.DecodePlan(), 1)  # never prepared
