"""GPU parity of the MFMA causal prefill (g4_attn_prefill) against the oracle.

The reference has no prefill kernel; it runs one decode step per prompt token
(src/engine.ts:2469-2475). So token t of an entry (position start + t) is
checked against the oracle's attnScore -> softmax -> attnOutput chain at
seq_len = start + t + 1, with the local-layer window, on the same f16 cache
rows and the f16 query widened to f32. Bar: max-abs 2e-3 (P is rounded to f16
for the output MFMA). Parts of long key ranges go through the log-sum-exp
merge (a call's parts are sized from its total work: these small calls cut
key ranges into parts of 256 keys). head_dim 512 (E2B global layers) runs the
pipelined form with each half of the output in its own workgroup.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from g4attn import ops, synth
from helpers import cache_f16, max_abs
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

HD = 256
TOL = 2e-3


class Chunk:
    def __init__(self, dev, seed, start, T, window, nqh=8, nkh=1, hd=HD):
        self.start, self.T, self.window, self.nqh, self.nkh, self.hd = start, T, window, nqh, nkh, hd
        rows = start + T
        self.kc = cache_f16(seed, rows, nkh, hd)
        self.vc = cache_f16(seed + 1, rows, nkh, hd)
        q = synth.rms_normalize_rows(synth.normal(seed + 2, T * nqh * hd).reshape(T * nqh, hd))
        self.qb = orc.f32_to_f16_bits(q).reshape(T, nqh * hd)
        t16 = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16).reshape(-1)).to(dev)  # noqa: E731
        self.dq, self.dk, self.dv = t16(self.qb), t16(self.kc), t16(self.vc)
        self.out = torch.full((T * nqh * hd,), float("nan"), dtype=torch.float32, device=dev)

    def entry(self):
        return dict(q=self.dq, k_cache=self.dk, v_cache=self.dv, out=self.out, n_tokens=self.T, start=self.start,
                    sliding_window=self.window, scale=1.0)

    def expected(self):
        rows = self.start + self.T
        kf = orc.f16_bits_to_f32(self.kc).reshape(rows, -1)
        vf = orc.f16_bits_to_f32(self.vc).reshape(rows, -1)
        qf = orc.f16_bits_to_f32(self.qb).reshape(self.T, -1)
        want = np.empty((self.T, self.nqh * self.hd), np.float32)
        for t in range(self.T):
            seq = self.start + t + 1
            want[t] = orc.attention_chain(qf[t], kf[:seq].reshape(-1), vf[:seq].reshape(-1), self.nqh, self.nkh,
                                          self.hd, seq, 1.0, self.window)
        return want.reshape(-1)


def run(dev, chunks, nqh=8, nkh=1, hd=HD):
    arr = ops.make_prefill_entries([c.entry() for c in chunks], nqh, nkh, hd)
    ws = torch.empty(max(ops.prefill_workspace_bytes(arr, nqh, nkh, hd), 1), dtype=torch.uint8, device=dev)
    plan = ops.attn_prefill_prepare(arr, nqh, nkh, hd, ws)
    ops.attn_prefill_run(plan)
    torch.cuda.synchronize()
    return plan, ws


def check(c, label):
    got = c.out.cpu().numpy()
    assert np.isfinite(got).all(), f"{label}: non-finite output"
    err = max_abs(got, c.expected())
    assert err <= TOL, f"{label}: max-abs {err}"
    return err


CASES = [  # (start, T, window)
    (0, 40, 0), (0, 100, 32), (600, 70, 512), (2900, 24, 0), (5, 1, 0), (0, 16, 512), (1000, 33, 512),
    (20000, 8, 0),  # more than 8 parts: the merge takes its many-record form
    (0, 512, 0),  # a full chunk: masked, interior (two per pass) and diagonal tiles
    (3000, 200, 0),  # long ranges split into parts, odd and even tile counts
    (300, 64, 16), (50, 40, 7),  # windows narrower than a 32-key tile: both bounds inside one tile
]


@pytest.mark.parametrize("start,T,window", CASES)
def test_prefill_chunk(dev, start, T, window):
    announce(f"attnPrefill start={start} T={T} window={window}")
    c = Chunk(dev, 31 + start + T, start, T, window)
    run(dev, [c])
    print(f"start={start} T={T} W={window} err={check(c, 'chunk'):.2e}")


def test_prefill_many_chunks_one_launch(dev):
    """A global and a local layer, each as two consecutive chunks, in one launch."""
    announce("attnPrefill 4 entries in one launch")
    chunks = [Chunk(dev, 7, 0, 64, 0), Chunk(dev, 8, 64, 64, 0), Chunk(dev, 9, 0, 64, 48), Chunk(dev, 10, 64, 64, 48)]
    run(dev, chunks)
    for i, c in enumerate(chunks):
        check(c, f"entry {i}")


def test_prefill_gqa_two_kv_heads(dev):
    announce("attnPrefill nqh=4 nkh=2")
    c = Chunk(dev, 12, 10, 33, 0, nqh=4, nkh=2)
    run(dev, [c], nqh=4, nkh=2)
    check(c, "gqa")


@pytest.mark.parametrize("nqh,nkh", [(2, 2), (4, 2), (8, 8)])
def test_prefill_fully_masked_part_small_groups(dev, nqh, nkh):
    """Query groups of 1 and 2 heads take the general merge. start=200, T=60 cuts the keys into
    [0, 256) and [256, 260): for positions 200..255 every key of the second part is masked, so
    that part's record is (m=-inf, l=0, o=0) and must weigh nothing in the merge."""
    announce(f"attnPrefill fully masked part nqh={nqh} nkh={nkh}")
    c = Chunk(dev, 70 + nqh + nkh, 200, 60, 0, nqh=nqh, nkh=nkh)
    plan, _ = run(dev, [c], nqh=nqh, nkh=nkh)
    check(c, f"masked part G={nqh // nkh}")


def test_prefill_replay_identical(dev):
    announce("attnPrefill replay")
    c = Chunk(dev, 13, 2000, 40, 0)
    plan, ws = run(dev, [c])
    first = c.out.cpu().numpy().copy()
    c.out.fill_(float("nan"))
    ops.attn_prefill_run(plan)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(c.out.cpu().numpy().view(np.uint32), first.view(np.uint32))
    check(c, "replay")


def test_prefill_rejects_bad_shapes(dev):
    c = Chunk(dev, 14, 0, 4, 0)
    arr = ops.make_prefill_entries([c.entry()], 8, 1, HD)
    from g4attn.abi import G4Error
    with pytest.raises(G4Error):
        ops.prefill_workspace_bytes(arr, 8, 1, 128)
    with pytest.raises(G4Error):
        ops.prefill_workspace_bytes(arr, 24, 1, HD)


@pytest.mark.parametrize("start,T,window,nkh", [(0, 40, 0, 1), (2900, 24, 0, 1), (600, 70, 512, 1), (20000, 8, 0, 1),
                                                (100, 33, 0, 2)])
def test_prefill_head_dim_512(dev, start, T, window, nkh):
    """head_dim 512: full-width scores in both output halves; parts merged at 512."""
    announce(f"attnPrefill hd=512 start={start} T={T} window={window} nkh={nkh}")
    nqh = 8
    c = Chunk(dev, 51 + start + T, start, T, window, nqh=nqh, nkh=nkh, hd=512)
    run(dev, [c], nqh=nqh, nkh=nkh, hd=512)
    print(f"hd=512 start={start} T={T} W={window} err={check(c, 'hd512'):.2e}")


def test_prefill_head_dim_512_with_256_in_one_process(dev):
    """A local (256) and a global (512) layer's chunks, as E2B's prefill issues them: two calls."""
    announce("attnPrefill hd 256 + 512")
    a = Chunk(dev, 61, 0, 48, 32)
    b = Chunk(dev, 62, 0, 48, 0, hd=512)
    run(dev, [a])
    run(dev, [b], hd=512)
    check(a, "hd256")
    check(b, "hd512")


@pytest.mark.timeout(900)
@pytest.mark.parametrize("vt", [True, False])
def test_prefill4k_bench_plan(dev, vt):
    """The exact launch bench.py times for the 4096-token prompt (workloads.prefill4k: a global and a
    512-window local layer, eight 512-token chunks each, 16 entries in one launch; key parts sized from
    the whole call's work, longest items first, the merge's few-record form), with V read from the V^T
    caches the prompt prep wrote (the benchmark's form) and transposed by the prefill itself. Checked
    against the oracle's decode chain: every token of each layer's first and last chunk, every 8th token
    elsewhere. Local layers are checked over their window's rows (the masked rows weigh exactly 0)."""
    from g4attn import workloads

    announce(f"attnPrefill prefill4k bench plan (16 entries, one launch), V^T caches {vt}")
    layers, entries, _ = workloads.prefill4k(dev, 8, 1, HD, vt=vt)
    arr = ops.make_prefill_entries(entries, 8, 1, HD)
    ws = torch.empty(ops.prefill_workspace_bytes(arr, 8, 1, HD), dtype=torch.uint8, device=dev)
    for _, _, _, out, _ in layers:
        out.fill_(float("nan"))
    plan = ops.attn_prefill_prepare(arr, 8, 1, HD, ws)
    ops.attn_prefill_run(plan)
    torch.cuda.synchronize()
    T, C = workloads.PREFILL_T, workloads.PREFILL_CHUNK
    tokens = sorted(set(range(C)) | set(range(T - C, T)) | set(range(C, T - C, 8)))
    worst = 0.0
    for q, kc, vc, out, w in layers:
        got = out.cpu().numpy().reshape(T, 8 * HD)
        assert np.isfinite(got).all(), f"window {w}: non-finite output"
        qf = orc.f16_bits_to_f32(q.cpu().numpy().view(np.uint16)).reshape(T, 8 * HD)
        kf = orc.f16_bits_to_f32(kc.cpu().numpy().view(np.uint16)).reshape(T, HD)
        vf = orc.f16_bits_to_f32(vc.cpu().numpy().view(np.uint16)).reshape(T, HD)
        for t in tokens:
            lo = t + 1 - w if w and t + 1 > w else 0
            want = orc.attention_chain(qf[t], kf[lo:t + 1].reshape(-1), vf[lo:t + 1].reshape(-1), 8, 1, HD,
                                       t + 1 - lo, 1.0, 0)
            err = max_abs(got[t], want)
            assert err <= TOL, f"window {w} token {t}: max-abs {err}"
            worst = max(worst, err)
        print(f"prefill4k window={w}: {len(tokens)} tokens checked, worst err {worst:.2e}", flush=True)


@pytest.mark.timeout(900)
def test_prefill4k512_plan(dev):
    """The head_dim 512 launch g4bench --workload prefill4k512 times: the global layer of the 4096-token
    prompt alone (eight 512-token chunks, one launch), V from the V^T cache the prompt prep wrote. Its
    256 work items (query tiles of 16 to 4096 keys, none split) fill the 128 workgroup lists of a
    head_dim-512 launch (two workgroups per item) two each, so the lists' item loop and the rows passed
    through LDS between items run at 512. Checked against the oracle's decode chain at the first 64
    tokens, every 16th token, and the last 128 tokens."""
    from g4attn import workloads

    H5 = 512
    announce("attnPrefill prefill4k global layer at head_dim 512 (8 entries, one launch)")
    layers, entries, _ = workloads.prefill4k(dev, 8, 1, H5, windows=(0,))
    arr = ops.make_prefill_entries(entries, 8, 1, H5)
    ws = torch.empty(ops.prefill_workspace_bytes(arr, 8, 1, H5), dtype=torch.uint8, device=dev)
    for _, _, _, out, _ in layers:
        out.fill_(float("nan"))
    plan = ops.attn_prefill_prepare(arr, 8, 1, H5, ws)
    ops.attn_prefill_run(plan)
    torch.cuda.synchronize()
    T = workloads.PREFILL_T
    tokens = sorted(set(range(64)) | set(range(T - 128, T)) | set(range(64, T - 128, 16)))
    q, kc, vc, out, w = layers[0]
    got = out.cpu().numpy().reshape(T, 8 * H5)
    assert np.isfinite(got).all(), "non-finite output"
    qf = orc.f16_bits_to_f32(q.cpu().numpy().view(np.uint16)).reshape(T, 8 * H5)
    kf = orc.f16_bits_to_f32(kc.cpu().numpy().view(np.uint16)).reshape(T, H5)
    vf = orc.f16_bits_to_f32(vc.cpu().numpy().view(np.uint16)).reshape(T, H5)
    worst = 0.0
    for t in tokens:
        want = orc.attention_chain(qf[t], kf[:t + 1].reshape(-1), vf[:t + 1].reshape(-1), 8, 1, H5, t + 1, 1.0, 0)
        err = max_abs(got[t], want)
        assert err <= TOL, f"token {t}: max-abs {err}"
        worst = max(worst, err)
    print(f"prefill4k hd=512: {len(tokens)} tokens checked, worst err {worst:.2e}", flush=True)
