"""GPU parity of the one-launch decode step (prep + split-K attention + merge in
one kernel) against the oracle's reference sequence:
vNorm -> fusedNormRope(Q) -> fusedNormRope(K) -> kvCacheStore -> attnScore ->
softmax -> attnOutput (src/engine.ts:2056-2094).

Bars: the stored f16 cache row is bit-identical to RNE of the oracle's k/v;
attnOut within max-abs 2e-3 (f16 KV, f32 accumulate). Rows the step must not
read (the current row before it is stored, rows outside a local window) are
poisoned with NaN, so reading one shows up as a non-finite output.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from g4attn import e2b, ops, synth
from helpers import EPS, cache_f16_torch, f16_weight_bits, max_abs
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL = 2e-3
NQH, NKH, HD = 8, 1, 256
ROPE = np.array(e2b.rope_freqs_f16_bits(256), dtype=np.uint16)
NAN16 = 0x7E00


def t16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)


class Layer:
    """One entry: raw projections, weights, a cache holding rows 0..seq-2, and the oracle's expectation."""

    def __init__(self, dev, seed, seq, window=0, theta=1e4, divisor=0, nqh=NQH, nkh=NKH, cache=None, hd=HD):
        self.seq, self.window, self.theta, self.divisor, self.hd = seq, window, theta, divisor, hd
        self.pos = seq - 1
        rng_scale = 2.0
        self.q = synth.normal(seed, nqh * hd) * rng_scale
        self.k = synth.normal(seed + 1, nkh * hd) * rng_scale
        self.v = synth.normal(seed + 2, nkh * hd) * rng_scale
        self.qw, self.kw = f16_weight_bits(seed + 3, hd), f16_weight_bits(seed + 4, hd)
        if cache is None:
            kc = cache_f16_torch(seed + 5, seq, nkh, hd, dev).view(torch.int16).reshape(seq, nkh * hd)
            vc = cache_f16_torch(seed + 6, seq, nkh, hd, dev).view(torch.int16).reshape(seq, nkh * hd)
            kc[self.pos] = NAN16
            vc[self.pos] = NAN16
            if window and seq > window:  # rows outside the window are never read
                kc[: seq - window] = NAN16
                vc[: seq - window] = NAN16
            self.kc, self.vc = kc.contiguous(), vc.contiguous()
        else:
            self.kc, self.vc = cache
        self.out = torch.full((nqh * hd,), float("nan"), device=dev)
        self.d = {n: torch.from_numpy(x.copy()).to(dev) for n, x in (("q", self.q), ("k", self.k), ("v", self.v))}
        self.dqw, self.dkw, self.drf = t16(self.qw, dev), t16(self.kw, dev), t16(ROPE, dev)
        self.nqh, self.nkh = nqh, nkh

    def entry(self, store=True, raw_kv=None, inv_freq=False):
        k, v = (self.d["k"], self.d["v"]) if raw_kv is None else raw_kv
        e = dict(q=self.d["q"], k=k, v=v, q_weight=self.dqw, k_weight=self.dkw, rope_freqs=self.drf,
                 k_cache=self.kc, v_cache=self.vc, out=self.out, seq_len=self.seq, position=self.pos,
                 sliding_window=self.window, store_kv=store, theta=self.theta, apply_divisor=self.divisor)
        if inv_freq:
            e["rope_inv_freq_host"] = ops.rope_inv_freq_host(self.theta, self.hd, self.divisor, ROPE)
        return e

    def expected(self, kv_from=None):
        """Oracle: prep then the reference chain over f32-widened caches (current row = RNE(k'), RNE(v'))."""
        src = kv_from or self
        hd = self.hd
        v_ = orc.per_head_rms_norm_no_weight(src.v, self.nkh, hd, EPS)
        k_ = orc.fused_per_head_norm_rope(src.k, src.kw, ROPE, self.nkh, hd, EPS, src.pos, src.theta, src.divisor)
        q_ = orc.fused_per_head_norm_rope(self.q, self.qw, ROPE, self.nqh, hd, EPS, self.pos, self.theta, self.divisor)
        kb = self.kc.cpu().numpy().view(np.uint16).copy()
        vb = self.vc.cpu().numpy().view(np.uint16).copy()
        kb[self.pos] = orc.f32_to_f16_bits(k_)
        vb[self.pos] = orc.f32_to_f16_bits(v_)
        lo = self.seq - self.window if self.window and self.seq > self.window else 0
        kf = orc.f16_bits_to_f32(kb[lo:]).reshape(-1)
        vf = orc.f16_bits_to_f32(vb[lo:]).reshape(-1)
        out = orc.attention_chain(q_, kf, vf, self.nqh, self.nkh, hd, self.seq - lo, 1.0, 0)
        return out, kb[self.pos], vb[self.pos]


def run_step(dev, entries, nqh=NQH, nkh=NKH, plan_runs=1, hd=HD):
    arr = ops.make_step_entries(entries, nqh, nkh, hd)
    ws = torch.empty(ops.step_workspace_bytes(len(entries), nqh, nkh, hd), dtype=torch.uint8, device=dev)
    plan = ops.attn_step_prepare(arr, nqh, nkh, hd, ws)
    for _ in range(plan_runs):
        ops.attn_step_run(plan)
    torch.cuda.synchronize()
    return plan, ws


def check(layer, want, kbits, vbits, label):
    got = layer.out.cpu().numpy()
    assert np.isfinite(got).all(), f"{label}: non-finite output (a poisoned row was read)"
    err = max_abs(got, want)
    assert err <= TOL, f"{label}: max-abs {err}"
    np.testing.assert_array_equal(layer.kc[layer.pos].cpu().numpy().view(np.uint16), kbits, err_msg=label)
    np.testing.assert_array_equal(layer.vc[layer.pos].cpu().numpy().view(np.uint16), vbits, err_msg=label)
    return err


SINGLE = [  # (seq, window, theta, divisor)
    (513, 512, 1e4, 0), (1, 0, 1e4, 0), (2, 0, 1e6, 1), (33, 0, 1e6, 1), (64, 512, 1e4, 0), (1000, 512, 1e4, 0),
    (8193, 0, 1e6, 1), (8193, 512, 1e4, 0), (32769, 0, 1e6, 1),
]


@pytest.mark.parametrize("seq,win,theta,div", SINGLE)
def test_step_single_entry(dev, seq, win, theta, div):
    announce(f"attnStep single seq={seq} win={win}")
    L = Layer(dev, 100 + seq, seq, win, theta, div)
    run_step(dev, [L.entry()])
    want, kb, vb = L.expected()
    err = check(L, want, kb, vb, f"seq={seq}")
    print(f"seq={seq} win={win} err={err:.2e}")


@pytest.mark.parametrize("seq,win,theta,div", [(513, 512, 1e4, 0), (8193, 0, 1e6, 1), (40000, 0, 1e6, 1)])
def test_step_rope_table_same_bits(dev, seq, win, theta, div):
    """Entries carrying the host inverse-frequency table (RoPE factors evaluated in prepare) give the same
    bits as entries without (factors evaluated in the kernel)."""
    announce(f"attnStep with a host RoPE table seq={seq} win={win}")
    L = Layer(dev, 400 + seq, seq, win, theta, div)
    want, kb, vb = L.expected()
    run_step(dev, [L.entry(inv_freq=True)])
    check(L, want, kb, vb, "table")
    with_table = L.out.cpu().numpy().copy()
    L.out.fill_(float("nan"))
    run_step(dev, [L.entry()])
    np.testing.assert_array_equal(L.out.cpu().numpy().view(np.uint32), with_table.view(np.uint32))


@pytest.mark.parametrize("seq", [2049, 8193, 32769, 131072])
def test_step_e2b_stack(dev, seq):
    """35 layers (7 global theta 1e6 with the rope_freqs divisor, 28 local W=512 theta 1e4) in one launch.
    Up to 8193 the step is small (one 8-wave workgroup per CU); at 32769 it takes two 4-wave workgroups
    per CU; at 131072 (bench.py's stack128k shape) each workgroup takes ~57 tiles."""
    announce(f"attnStep 35-layer stack seq={seq}")
    cfg = e2b.AttnConfig(num_layers=35)
    layers = [Layer(dev, 1000 * il + seq, seq, e2b.sliding_window(il, cfg), e2b.rope_theta(il, cfg),
                    e2b.apply_divisor(il, cfg)) for il in range(35)]
    run_step(dev, [L.entry(inv_freq=il % 2 == 0) for il, L in enumerate(layers)])
    worst = 0.0
    for il, L in enumerate(layers):
        want, kb, vb = L.expected()
        worst = max(worst, check(L, want, kb, vb, f"layer {il}"))
    print(f"stack seq={seq} worst err={worst:.2e}")


def test_step_long_entry_two_workgroups_per_cu(dev):
    """One entry of 140001 rows: more than 16 tiles per workgroup at one per CU, so the step takes two
    4-wave workgroups per CU."""
    announce("attnStep single seq=140001")
    L = Layer(dev, 77, 140001, 0, 1e6, 1)
    run_step(dev, [L.entry(inv_freq=True)])
    want, kb, vb = L.expected()
    check(L, want, kb, vb, "seq=140001")


def test_step_ragged_batch(dev):
    lens = [1, 2, 31, 32, 33, 100, 511, 512, 513] + [int(x) for x in synth.ragged_lengths(77, 7, 1000, 9000)]
    announce(f"attnStep ragged batch {lens}")
    layers = [Layer(dev, 50 + i, L, 0, 1e6, 1) for i, L in enumerate(lens)]
    run_step(dev, [L.entry() for L in layers])
    for i, L in enumerate(layers):
        want, kb, vb = L.expected()
        check(L, want, kb, vb, f"seq {i} len {lens[i]}")


def test_step_kv_consumer_layer(dev):
    """A KV-consumer layer reads its producer's cache and current row in the same launch, without storing."""
    announce("attnStep producer + consumer sharing a cache")
    prod = Layer(dev, 7, 3000, 0, 1e6, 1)
    cons = Layer(dev, 8, 3000, 0, 1e6, 1, cache=(prod.kc, prod.vc))
    run_step(dev, [prod.entry(), cons.entry(store=False, raw_kv=(prod.d["k"], prod.d["v"]))])
    want_p, kb, vb = prod.expected()
    check(prod, want_p, kb, vb, "producer")
    want_c, _, _ = cons.expected(kv_from=prod)
    got = cons.out.cpu().numpy()
    assert np.isfinite(got).all() and max_abs(got, want_c) <= TOL


@pytest.mark.parametrize("seq,win,theta,div,hd", [(3000, 0, 1e6, 1, 256), (1, 0, 1e4, 0, 256), (700, 512, 1e4, 0, 256),
                                                 (40000, 0, 1e6, 1, 256), (5000, 0, 1e6, 1, 512)])
def test_step_kv_consumer_after_producer(dev, seq, win, theta, div, hd):
    """The engine's layer-by-layer order: the producer's step stores the current row, then the consumer's
    step (a launch of its own, k, v and k_weight NULL) reads that row from the cache like the others."""
    announce(f"attnStep consumer after producer seq={seq} win={win} hd={hd}")
    prod = Layer(dev, 17 + seq, seq, win, theta, div, hd=hd)
    cons = Layer(dev, 18 + seq, seq, win, theta, div, cache=(prod.kc, prod.vc), hd=hd)
    run_step(dev, [prod.entry()], hd=hd)
    want_p, kb, vb = prod.expected()
    check(prod, want_p, kb, vb, "producer")
    e = cons.entry(store=False)
    e["k"] = e["v"] = e["k_weight"] = None
    run_step(dev, [e], hd=hd)
    want_c, _, _ = cons.expected(kv_from=prod)
    got = cons.out.cpu().numpy()
    err = max_abs(got, want_c)
    assert np.isfinite(got).all() and err <= TOL, err
    np.testing.assert_array_equal(prod.kc[prod.pos].cpu().numpy().view(np.uint16), kb)  # not stored again
    print(f"consumer after producer seq={seq} hd={hd}: err={err:.2e}")


def test_step_replay_is_deterministic(dev):
    """A prepared plan replays (merge counters reset themselves) and gives identical bits each time."""
    announce("attnStep replay")
    layers = [Layer(dev, 300 + i, s, w, 1e4, 0) for i, (s, w) in enumerate([(20000, 0), (700, 512), (5, 0)])]
    arr = ops.make_step_entries([L.entry() for L in layers], NQH, NKH, HD)
    ws = torch.empty(ops.step_workspace_bytes(3, NQH, NKH, HD), dtype=torch.uint8, device=dev)
    plan = ops.attn_step_prepare(arr, NQH, NKH, HD, ws)
    outs = []
    for _ in range(3):
        for L in layers:
            L.out.fill_(float("nan"))
        ops.attn_step_run(plan)
        torch.cuda.synchronize()
        outs.append(np.concatenate([L.out.cpu().numpy() for L in layers]).view(np.uint32))
    np.testing.assert_array_equal(outs[0], outs[1])
    np.testing.assert_array_equal(outs[0], outs[2])
    for L in layers:
        want, kb, vb = L.expected()
        check(L, want, kb, vb, "replay")


def test_step_stack_replays_bitwise(dev):
    """The 35-layer stack replayed many times: every replay gives the same bits (split records and
    the fixed-order merge), within tolerance of the oracle."""
    announce("attnStep stack replays")
    cfg = e2b.AttnConfig(num_layers=35)
    layers = [Layer(dev, 500 + il, 4097, e2b.sliding_window(il, cfg), e2b.rope_theta(il, cfg),
                    e2b.apply_divisor(il, cfg)) for il in range(35)]
    arr = ops.make_step_entries([L.entry() for L in layers], NQH, NKH, HD)
    ws = torch.empty(ops.step_workspace_bytes(35, NQH, NKH, HD), dtype=torch.uint8, device=dev)
    plan = ops.attn_step_prepare(arr, NQH, NKH, HD, ws)
    first = None
    for rep in range(12):
        for L in layers:
            L.out.fill_(float("nan"))
        ops.attn_step_run(plan)
        torch.cuda.synchronize()
        got = np.concatenate([L.out.cpu().numpy() for L in layers]).view(np.uint32)
        if first is None:
            first = got.copy()
        np.testing.assert_array_equal(got, first, err_msg=f"replay {rep}")
    for L in layers[:6]:
        want, kb, vb = L.expected()
        check(L, want, kb, vb, "stack replay")


def test_step_gqa_two_kv_heads(dev):
    announce("attnStep nqh=16 nkh=2")
    L = Layer(dev, 9, 1500, 0, 1e6, 1, nqh=16, nkh=2)
    run_step(dev, [L.entry()], nqh=16, nkh=2)
    want, kb, vb = L.expected()
    check(L, want, kb, vb, "gqa")


@pytest.mark.parametrize("seq", [100, 250])
def test_step_group4_few_parts(dev, seq):
    """Four query heads per kv head and a few parts per entry: the merge takes its one-workgroup-per-entry
    form (all heads of an entry, 4 columns per thread)."""
    announce(f"attnStep nqh=8 nkh=2 seq={seq}")
    L = Layer(dev, 31 + seq, seq, 0, 1e6, 1, nqh=8, nkh=2)
    run_step(dev, [L.entry()], nqh=8, nkh=2)
    want, kb, vb = L.expected()
    check(L, want, kb, vb, f"group 4 seq={seq}")


HD512 = [  # (seq, window, theta, divisor): E2B global layers have head_dim 512
    (1, 0, 1e6, 1), (33, 0, 1e6, 1), (513, 0, 1e6, 1), (8193, 0, 1e6, 1), (40000, 0, 1e6, 1), (1000, 512, 1e4, 0),
]


@pytest.mark.parametrize("seq,win,theta,div", HD512)
def test_step_head_dim_512(dev, seq, win, theta, div):
    """head_dim 512 (one 4-wave workgroup per CU): the stored rows bit-identical, attnOut within 2e-3, with and
    without the host RoPE table (same bits)."""
    announce(f"attnStep hd=512 seq={seq} win={win}")
    L = Layer(dev, 600 + seq, seq, win, theta, div, hd=512)
    want, kb, vb = L.expected()
    run_step(dev, [L.entry(inv_freq=True)], hd=512)
    err = check(L, want, kb, vb, f"hd512 seq={seq}")
    with_table = L.out.cpu().numpy().copy()
    L.out.fill_(float("nan"))
    run_step(dev, [L.entry()], hd=512)
    np.testing.assert_array_equal(L.out.cpu().numpy().view(np.uint32), with_table.view(np.uint32))
    print(f"hd512 seq={seq} err={err:.2e}")


def test_step_head_dim_512_layers_and_group4(dev):
    """The seven E2B global layers at 8193 rows in one launch, and a 4:1 group at head_dim 512."""
    announce("attnStep hd=512 7 global layers; nqh=8 nkh=2")
    layers = [Layer(dev, 700 + i, 8193, 0, 1e6, 1, hd=512) for i in range(7)]
    run_step(dev, [L.entry(inv_freq=True) for L in layers], hd=512)
    for i, L in enumerate(layers):
        want, kb, vb = L.expected()
        check(L, want, kb, vb, f"global layer {i}")
    L = Layer(dev, 800, 3000, 0, 1e6, 1, nqh=8, nkh=2, hd=512)
    run_step(dev, [L.entry()], nqh=8, nkh=2, hd=512)
    want, kb, vb = L.expected()
    check(L, want, kb, vb, "hd512 group 4")


@pytest.mark.timeout(900)
def test_step_ragged64_bench_set(dev):
    """The 64 ragged sequences bench.py times (lengths U[1024, 32768] from the same seed; global layers,
    theta 1e6 with the divisor table, host RoPE tables), all in one plan; every sequence checked."""
    from g4attn import workloads

    lens = workloads.ragged64_lengths()
    announce(f"attnStep ragged64 bench set: {len(lens)} sequences, {sum(lens)} rows")
    layers = [Layer(dev, 9000 + i, L, 0, 1e6, 1) for i, L in enumerate(lens)]
    run_step(dev, [L.entry(inv_freq=True) for L in layers])
    worst = 0.0
    for i, L in enumerate(layers):
        want, kb, vb = L.expected()
        worst = max(worst, check(L, want, kb, vb, f"seq {i} len {lens[i]}"))
        if i % 16 == 15:
            print(f"ragged64: {i + 1} sequences checked, worst err {worst:.2e}", flush=True)


@pytest.mark.parametrize("seq,win", [(33, 0), (300, 0), (513, 512), (1000, 512), (1500, 0), (2049, 0), (4000, 0)])
def test_step_single_entry_replays(dev, seq, win):
    """A small single-entry step (the engine's layer-by-layer order), cut into a few parts and merged.
    Replayed three times: every replay gives the same bits."""
    announce(f"attnStep few parts seq={seq} win={win}")
    L = Layer(dev, 1300 + seq, seq, win, 1e4 if win else 1e6, 0 if win else 1)
    want, kb, vb = L.expected()
    plan, ws = run_step(dev, [L.entry(inv_freq=True)])
    check(L, want, kb, vb, f"seq={seq}")
    first = L.out.cpu().numpy().copy()
    for rep in range(3):
        L.out.fill_(float("nan"))
        ops.attn_step_run(plan)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(L.out.cpu().numpy().view(np.uint32), first.view(np.uint32),
                                      err_msg=f"replay {rep}")


def test_step_mixed_part_counts(dev):
    """Entries of few parts, of many parts and whole entries in one step, run twice on one plan."""
    announce("attnStep mixed part counts")
    specs = [(8193, 0), (513, 512), (40, 0), (2000, 0), (700, 512), (20000, 0), (3, 0), (1025, 0)]
    layers = [Layer(dev, 1400 + i, s, w, 1e4 if w else 1e6, 0 if w else 1) for i, (s, w) in enumerate(specs)]
    wants = [L.expected() for L in layers]
    plan, ws = run_step(dev, [L.entry(inv_freq=i % 2 == 0) for i, L in enumerate(layers)], plan_runs=2)
    for i, (L, (want, kb, vb)) in enumerate(zip(layers, wants)):
        check(L, want, kb, vb, f"entry {i}")
