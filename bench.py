#!/usr/bin/env python3
"""Decode-attention benchmark on one MI355X: µs/token and HBM GB/s (% of roofline).

    python bench.py [--steps K] [--warmup W] [--workload NAME]

A step is one token's attention over the workload on synthetic, seeded,
inputs resident in HBM:
  stack32k  35-layer Gemma-4-E2B-shaped stack, batch 1, position 32768 (7 global
            layers full causal, RoPE theta 1e6; 28 local layers with a 512-row
            window, theta 1e4), 35 separate f16 KV caches, 8 query heads / 1 KV
            head, head_dim 256: the shape the decode target is set on.  [default]
            The default run also measures stack8k and reports it under
            "stack8k" in the same line.
  stack8k   the same stack at position 8192 (stack4k: 4096, stack128k: 131071; the
            ends of the metric's 4K-128K context range).
  e2b8k     the real Gemma-4-E2B stack at position 8192: head_dim 512 on the
  e2b32k    7 global layers, layers 15..34 reading layer 13's (local) or 14's
            (global) cache (KV sharing, src/config/gemma4-e2b.ts:159-178); one
            launch per head_dim; e2b32k at position 32768.
  long128k  one global layer attending 131072 rows.
  ragged64  64 independent sequences, lengths uniform in [1024, 32768].
  layer512  one local layer at position 512 (launch-bound).
  prefill4k causal prefill of a 4096-token prompt on MFMA: one global and one
            512-window local layer, as 512-token chunks (16 entries in one
            launch); f16 Q/K/V (unit-RMS rows). Reported in TFLOP/s
            (algorithmic 4*HD*NQH per attended key per token) against the
            2.5 PFLOP/s dense f16 MFMA peak.
  lmhead    the sampling head after the last layer (src/engine.ts:2223-2255)
            at Gemma-4-E2B's shape: lm head over the f16 tied embedding
            [262144][1536], logit softcap 30, greedy argmax, as one streaming
            pass plus a one-workgroup pick. Reported in GB/s of algorithmic
            bytes (weight + hidden + logits written).

A decode step is one launch of the fused attention step over every entry of a
head_dim (per entry: q/k RMSNorm + RoPE, weightless v-norm, f16 store of the
new K/V row, split-K flash-decoding attention over the attended rows), plus
the log-sum-exp merge launch when the plan has split entries. Several
distinct cache sets are rotated so the bytes read each cycle exceed twice
MI355X's 256 MB Infinity Cache and come from HBM. `value` is algorithmic bytes
per step (K/V rows attended, f16, read once for all query heads; q read;
attnOut written) over wall time per step. `roofline` is the dominant kernel
(k_attn_step), timed with HIP events on its stream; its `traffic` comes from
the committed rocprofv3 counter summary of the same workload. `decode_loop`
advances the position every step inside the timed region: the prepared plan
moves on the host (g4_attn_step_advance; the kernel evaluates the new
position's RoPE factors) and is prepared again every 32 tokens; its
`prepare_every_token` figure re-prepares every entry every token instead (host
partition, RoPE factors, table uploads). `cpu_baseline` runs the
oracle (the WGSL-semantics C restatement of the reference's six kernels, f32
caches, full-length score/softmax/output on every layer as the WGSL does) on
the host.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "gemma4-webgpu_amd"))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20
NQH, NKH, HD = 8, 1, 256
EPS = 1e-6
BASE_SEED = 20261201
DEFAULT_WORKLOAD = "stack32k"
REPLAN_TOKENS = 32  # decode loop: a plan advances on the host and is prepared again every this many tokens
PREFILL_KERNEL = "k_prefill_pp"  # the prefill kernel at head_dim 256


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---- workload description -----------------------------------------------------

def workload_spec(name: str) -> dict:
    """Layers (entries) of one step: window, theta, divisor, seq (rows incl. the current one), pos,
    hd (head_dim) and producer (the entry whose cache it reads; itself for a KV producer)."""
    from g4attn import e2b

    def layer(**kw):
        d = dict(hd=HD, producer=None)
        d.update(kw)
        return d

    stacks = {"stack4k": (4096, 8), "stack8k": (8192, 1), "stack32k": (32768, 5), "stack128k": (131071, 9)}
    if name in stacks:
        pos, seed_off = stacks[name]
        cfg = e2b.AttnConfig(num_layers=35)
        layers = [layer(window=e2b.sliding_window(il, cfg), theta=e2b.rope_theta(il, cfg),
                        divisor=e2b.apply_divisor(il, cfg), seq=pos + 1, pos=pos) for il in range(35)]
        return dict(name=name, layers=layers, seed=BASE_SEED + seed_off,
                    desc=f"35-layer Gemma-4-E2B attention stack, bs1, position {pos} (7 global + 28 local W=512), "
                         "head_dim 256, 35 separate caches")
    if name in ("e2b8k", "e2b32k"):
        pos = 8192 if name == "e2b8k" else 32768
        cfg = e2b.AttnConfig(num_layers=35)
        pmap = e2b.compute_kv_producer_map(cfg)
        layers = [layer(window=e2b.sliding_window(il, cfg), theta=e2b.rope_theta(il, cfg),
                        divisor=e2b.apply_divisor(il, cfg), seq=pos + 1, pos=pos, hd=e2b.head_dim(il, cfg),
                        producer=None if pmap[il] == il else pmap[il]) for il in range(35)]
        return dict(name=name, layers=layers, seed=BASE_SEED + (6 if name == "e2b8k" else 7),
                    desc=f"Gemma-4-E2B attention stack, bs1, position {pos}: head_dim 512 on the 7 global layers, "
                         "layers 15..34 reading layer 13's / 14's cache, one plan per head_dim, both run as one attention "
                         "launch and one merge launch")
    if name == "long128k":
        pos = 131071
        return dict(name=name, layers=[layer(window=0, theta=1e6, divisor=1, seq=pos + 1, pos=pos)],
                    seed=BASE_SEED + 4, desc="1 global layer, 131072 attended rows, bs1")
    if name == "layer512":
        return dict(name=name, layers=[layer(window=512, theta=1e4, divisor=0, seq=513, pos=512)],
                    seed=BASE_SEED + 0, desc="1 local layer (W=512), position 512, bs1")
    if name == "ragged64":
        from g4attn import workloads

        lens = workloads.ragged64_lengths()
        layers = [layer(window=0, theta=1e6, divisor=1, seq=L, pos=L - 1) for L in lens]
        return dict(name=name, layers=layers, seed=BASE_SEED + 2,
                    desc="64 sequences, ragged lengths U[1024, 32768], global attention")
    raise SystemExit(f"unknown workload {name}")


def attended(seq: int, window: int) -> int:
    return min(seq, window) if window else seq


def layer_bytes(L: dict) -> int:
    """Algorithmic HBM bytes of one entry: attended K and V rows (f16) once for all query heads,
    q read (f32) and attnOut written (f32). A KV-consumer layer reads its producer's rows again."""
    return 2 * attended(L["seq"], L["window"]) * NKH * L["hd"] * 2 + NQH * L["hd"] * 4 * 2


def step_bytes(spec: dict) -> int:
    return sum(layer_bytes(L) for L in spec["layers"])


# ---- GPU side -----------------------------------------------------------------

class CacheSet:
    """One complete set of per-entry buffers (caches, raw q/k/v projections, outputs) and the
    prepared one-launch steps over the entries (one per head_dim)."""

    def __init__(self, spec, set_idx, dev, torch, ops, synth, e2b, extra_rows=0, pair=True):
        import numpy as np

        seed0 = spec["seed"] + 7919 * set_idx
        rf_bits = np.array(e2b.rope_freqs_f16_bits(256), dtype=np.uint16)
        rf = torch.from_numpy(rf_bits.view(np.int16)).to(dev)
        ones = {hd: torch.full((hd,), 0x3C00, dtype=torch.int16, device=dev) for hd in (256, 512)}  # f16 1.0
        self.inv_freq = {}  # one RoPE inverse-frequency table per (theta, divisor, head_dim), as a model holds them
        self.items = []
        for il, L in enumerate(spec["layers"]):
            hd = L["hd"]
            key = (L["theta"], L["divisor"], hd)
            if key not in self.inv_freq:
                self.inv_freq[key] = ops.rope_inv_freq_host(L["theta"], hd, L["divisor"], rf_bits)
            it = dict(q=synth.normal_torch(seed0 + 1000 * il + 2, NQH * hd, dev), q_weight=ones[hd],
                      rope_freqs=rf, rope_inv_freq_host=self.inv_freq[key],
                      out=torch.zeros(NQH * hd, dtype=torch.float32, device=dev), seq_len=L["seq"],
                      position=L["pos"], sliding_window=L["window"], theta=L["theta"], apply_divisor=L["divisor"],
                      scale=1.0, eps=EPS)
            if L["producer"] is None:
                rows = L["seq"] + extra_rows
                kc = torch.empty(rows * NKH * hd, dtype=torch.float16, device=dev)
                vc = torch.empty_like(kc)
                n_att = attended(L["seq"], L["window"])
                lo = L["seq"] - n_att
                for cache, off in ((kc, 0), (vc, 1)):  # rows the step reads: N(0,1), then RMS-normalised per head
                    x = synth.normal_torch(seed0 + 1000 * il + off, n_att * NKH * hd, dev).view(-1, hd)
                    ms = (x.double() ** 2).mean(dim=1, keepdim=True)
                    y = (x.double() / torch.sqrt(ms + EPS)).to(torch.float16)
                    cache.view(rows, -1)[lo:lo + n_att].copy_(y.view(n_att, -1))
                it.update(k=synth.normal_torch(seed0 + 1000 * il + 3, NKH * hd, dev),
                          v=synth.normal_torch(seed0 + 1000 * il + 4, NKH * hd, dev), k_weight=ones[hd],
                          k_cache=kc.view(torch.int16), v_cache=vc.view(torch.int16), store_kv=True)
            else:  # a consumer in its producer's launch: the producer's raw k/v and k_norm, no store
                p = self.items[L["producer"]]
                it.update(k=p["k"], v=p["v"], k_weight=p["k_weight"], k_cache=p["k_cache"], v_cache=p["v_cache"],
                          store_kv=False)
            it["hd"] = hd
            self.items.append(it)
        self.groups = []  # (head_dim, entry indexes, ctypes entries, workspace, plan)
        for hd in sorted({it["hd"] for it in self.items}):
            idx = [i for i, it in enumerate(self.items) if it["hd"] == hd]
            arr = ops.make_step_entries([self.items[i] for i in idx], NQH, NKH, hd)
            ws = torch.empty(ops.step_workspace_bytes(len(idx), NQH, NKH, hd), dtype=torch.uint8, device=dev)
            # [head_dim, entry indexes, ctypes entries, workspace, plan, tokens advanced since its prepare]
            self.groups.append([hd, idx, arr, ws, ops.attn_step_prepare(arr, NQH, NKH, hd, ws), 0])
        # Two head_dims (E2B): both attention passes in one launch (g4_attn_step_run_pair), then each merge.
        self.paired = pair and [g[0] for g in self.groups] == [256, 512]
        self.launches = 1 if self.paired else len(self.groups)
        self.layer_plans = None

    def run(self, ops, ev=None):
        if self.paired:
            p256, p512 = self.groups[0][4], self.groups[1][4]
            if ev is None:
                ops.attn_step_run_pair(p512, p256)
            else:
                ops.attn_step_run_attention_pair_timed(p512, p256, ev[0][0], ev[0][1])
                ops.attn_step_run_merge(p512)
                ops.attn_step_run_merge(p256)
            return
        for gi, (hd, idx, arr, ws, plan, _) in enumerate(self.groups):
            if ev is None:
                ops.attn_step_run(plan)
            else:
                ops.attn_step_run_attention_timed(plan, ev[gi][0], ev[gi][1])
                ops.attn_step_run_merge(plan)

    def advance(self, ops, replan_every):
        """The next token: every entry one row longer (the engine rewrites the position, slot and seq_len
        uniforms every token, src/engine.ts:1967-1987). The prepared plan advances on the host alone
        (g4_attn_step_advance: nothing is enqueued) and is prepared again every `replan_every` tokens
        (1: a full prepare every token: partition, RoPE factors, table upload)."""
        for g in self.groups:
            hd, idx, arr, ws, plan, since = g
            for f in self._fields(arr):  # seq_len and position of every entry, one vectorised bump each
                f += 1
            if since + 1 < replan_every:
                ops.attn_step_advance(plan, 1)
                g[5] = since + 1
            else:
                g[4] = ops.attn_step_prepare(arr, NQH, NKH, hd, ws)
                g[5] = 0

    @staticmethod
    def _fields(arr):
        """numpy views of the seq_len and position fields of a ctypes StepEntry array (writes go to it)."""
        import numpy as np

        from g4attn.abi import StepEntry

        u32 = np.frombuffer(arr, dtype=np.uint32)
        stride = C.sizeof(StepEntry) // 4
        return [u32[StepEntry.seq_len.offset // 4::stride], u32[StepEntry.position.offset // 4::stride]]

    def prepare_per_entry(self, torch, ops, dev):
        """One single-entry plan per entry: the engine's issue order (layer after layer)."""
        self.layer_plans = []
        for it in self.items:
            hd = it["hd"]
            w = torch.empty(ops.step_workspace_bytes(1, NQH, NKH, hd), dtype=torch.uint8, device=dev)
            e = dict(it)
            if not it["store_kv"]:  # engine order: the producer's step already stored the row
                e["k"] = e["v"] = e["k_weight"] = None
            self.layer_plans.append((w, ops.attn_step_prepare(ops.make_step_entries([e], NQH, NKH, hd), NQH, NKH,
                                                              hd, w)))

    def step_sequential(self, ops):
        for _, p in self.layer_plans:
            ops.attn_step_run(p)

    def prepare_chain(self, torch, dev, hidden=1536):
        """The projections either side of every layer's attention (random f16 weights of E2B's shapes):
        attn.linearQKV into the entry's raw q/k/v (q alone for a consumer, whose k/v come from its
        producer) and attn.linearOut from attnOut (src/engine.ts:2045-2052, 2096)."""
        import numpy as np

        from g4attn import e2b, ops
        self.hidden = hidden
        self.x = torch.randn(hidden, device=dev)
        self.chain = []
        for it, (_, plan) in zip(self.items, self.layer_plans):
            hd = it["hd"]
            n = NQH * hd
            segs = [(NQH * hd, it["q"])]
            if it["store_kv"]:
                segs += [(NKH * hd, it["k"]), (NKH * hd, it["v"])]
            qkv = [((torch.randn(rows, hidden, device=dev) * 0.02).half().view(torch.int16), out, rows)
                   for rows, out in segs]
            wo = (torch.randn(hidden, n, device=dev) * 0.02).half().view(torch.int16)
            self.chain.append((plan, qkv, n, wo, it["out"], torch.empty(hidden, device=dev)))
        # The fused variant: attn.linearQKV with the prep as its epilogue (g4_linear_qkv_prep: projection,
        # norms, RoPE, K/V row stored), then steps whose q is ready and whose current row is in the cache.
        rf = torch.from_numpy(np.array(e2b.rope_freqs_f16_bits(256), np.uint16).view(np.int16)).to(dev)
        self.rf_dev, self.inv_dev, self.ready = rf, {}, []
        self.prep_ws = torch.zeros(ops.qkv_prep_workspace_bytes(NQH, NKH), dtype=torch.uint8, device=dev)
        for it in self.items:
            hd = it["hd"]
            key = (it["theta"], it["apply_divisor"], hd)
            if key not in self.inv_dev:
                self.inv_dev[key] = ops.rope_inv_freq(it["theta"], hd, it["apply_divisor"], rf)
            w = torch.empty(ops.step_workspace_bytes(1, NQH, NKH, hd), dtype=torch.uint8, device=dev)
            e = dict(it, k=None, v=None, k_weight=None, store_kv=False, q_ready=True)
            self.ready.append((w, ops.attn_step_prepare(ops.make_step_entries([e], NQH, NKH, hd), NQH, NKH, hd, w)))

    def step_chain_prep(self, ops):
        """One token in the engine's order with the fused projection: per layer, g4_linear_qkv_prep (q/k/v
        projection with norms, RoPE and the K/V store as its epilogue), the attention pass on the ready q,
        and o_proj with the merge folded in (three launches)."""
        for (plan, qkv, n, wo, attn_out, y), (_, ready), it in zip(self.chain, self.ready, self.items):
            hd = it["hd"]
            store = it["store_kv"]
            rows = it["k_cache"].numel() // (NKH * hd)
            ops.linear_qkv_prep(self.x, self.hidden, "f16", qkv, it["q_weight"], NQH, NKH, hd, it["position"],
                                it["theta"], it["apply_divisor"], self.prep_ws, k_weight=it["k_weight"],
                                rope_freqs=self.rf_dev, rope_inv_freq=self.inv_dev[(it["theta"], it["apply_divisor"],
                                                                                     hd)],
                                k_cache=it["k_cache"] if store else None, v_cache=it["v_cache"] if store else None,
                                slot=it["seq_len"] - 1, max_seq_len=rows)
            ops.attn_step_run_attention(ready)
            ops.attn_step_run_out(ready, n, [(wo, y, self.hidden)])

    def step_chain(self, ops, fused):
        """One token in the engine's order: per layer, q/k/v projection, attention pass, then the merge
        launch and o_proj (four launches) or o_proj with the merge folded in (three launches)."""
        for plan, qkv, n, wo, attn_out, y in self.chain:
            ops.linear_f16(self.x, self.hidden, qkv)
            ops.attn_step_run_attention(plan)
            if fused:
                ops.attn_step_run_out(plan, n, [(wo, y, self.hidden)])
            else:
                ops.attn_step_run_merge(plan)
                ops.linear_f16(attn_out, n, [(wo, y, self.hidden)])


def run_gpu(spec, args, decode_loop=False):
    import torch

    from g4attn import abi, e2b, ops, synth

    abi.load()
    abi.call("g4_set_device", 0)
    dev = torch.device("cuda:0")
    per_step = step_bytes(spec)
    sets = args.sets or max(1, math.ceil(2 * MALL_BYTES / max(per_step, 1)) + 1)
    if per_step < 4 << 20:
        sets = 1  # tiny workloads are launch-bound; rotating sets changes nothing
    loop_tokens = 2 * (args.warmup + args.steps) if decode_loop else 0  # two loops append rows
    log(f"workload {spec['name']}: {len(spec['layers'])} entries, {per_step / 1e6:.1f} MB/step, {sets} cache sets")
    t0 = time.time()
    csets = [CacheSet(spec, s, dev, torch, ops, synth, e2b, extra_rows=loop_tokens, pair=args.pair)
             for s in range(sets)]
    torch.cuda.synchronize()
    log(f"inputs ready in {time.time() - t0:.1f}s")

    stream = torch.cuda.current_stream()
    n_groups = csets[0].launches

    def step(i, ev=None):
        csets[i % sets].run(ops, ev)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    log(f"warmup {args.warmup} steps done")

    # Timed region: exactly `steps` steps, synchronised on both sides.
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for i in range(args.steps):
        step(args.warmup + i)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    log(f"timed {args.steps} steps: {wall / args.steps * 1e6:.2f} us/step")

    # The attention kernels alone: HIP events on their stream that take each kernel's own start and
    # end timestamps (hipExtLaunchKernelGGL), the figure rocprofv3 reports for the same kernel.
    evs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n_groups)]
           for _ in range(args.steps)]
    for per in evs:  # create the HIP events
        for a_, b_ in per:
            a_.record(stream)
            b_.record(stream)
    torch.cuda.synchronize()
    for i in range(args.steps):
        step(args.warmup + i, evs[i])
    torch.cuda.synchronize()
    att_ms = sorted(sum(a.elapsed_time(b) for a, b in per) for per in evs)
    att_avg = sum(att_ms) / len(att_ms)
    log(f"k_attn_step: avg {att_avg * 1e3:.2f} us, median {att_ms[len(att_ms) // 2] * 1e3:.2f} us (events, "
        f"{n_groups} launch(es) per step)")
    result = dict(wall_s=wall, steps=args.steps, attn_avg_ms=att_avg, attn_median_ms=att_ms[len(att_ms) // 2],
                  sets=sets, bytes=per_step, launches=n_groups,
                  kernel="k_attn_step_pair" if csets[0].paired else "k_attn_step")

    if decode_loop:
        # Position-advancing decode loops, all inside the timed region: every token every entry is one
        # row further. "advance": the plan advances on the host (g4_attn_step_advance) and is prepared
        # again every REPLAN_TOKENS tokens; "prepare every token": host partition, RoPE factors and
        # pinned-ring table upload per token.
        for key, every in (("loop", REPLAN_TOKENS), ("loop_each", 1)):
            for i in range(args.warmup):
                cs = csets[i % sets]
                cs.advance(ops, every)
                cs.run(ops)
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            host = 0.0
            for i in range(args.steps):
                cs = csets[(args.warmup + i) % sets]
                h0 = time.perf_counter()
                cs.advance(ops, every)
                host += time.perf_counter() - h0
                cs.run(ops)
            torch.cuda.synchronize()
            result[f"{key}_us"] = (time.perf_counter() - t2) / args.steps * 1e6
            result[f"{key}_prepare_us"] = host / args.steps * 1e6
            log(f"decode loop ({'advance, prepare every %d tokens' % every if every > 1 else 'prepare every token'}):"
                f" {result[f'{key}_us']:.2f} us/token, host {result[f'{key}_prepare_us']:.2f} us/token")

    # The engine's issue order: one single-entry step (attention + merge) per layer, replayed as a HIP graph;
    # then the same with each layer's projections around it. Each replay is queued behind a short spin kernel,
    # so the host has submitted the whole graph before the GPU reaches it, and events on the stream time the
    # GPU's execution alone (a graph's host-side submission grows with its nodes and, for one layer, takes
    # longer than the GPU work it submits).
    def graph_us(fn):
        fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        torch.cuda.synchronize()
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize()
        times = []
        for _ in range(max(10, args.steps // 2)):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda._sleep(2_000_000)
            e0.record(stream)
            g.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) * 1e3)
        times.sort()
        return times[len(times) // 2]

    if args.sequential:
        cs = csets[0]
        cs.prepare_per_entry(torch, ops, dev)
        torch.cuda.synchronize()
        if len(spec["layers"]) > 1:
            result["sequential_us"] = graph_us(lambda: cs.step_sequential(ops))
            log(f"layer-sequential (graph replay, GPU time, one cache set): {result['sequential_us']:.1f} us/step")
        cs.prepare_chain(torch, dev)
        result["chain_us"] = graph_us(lambda: cs.step_chain(ops, fused=False))
        result["chain_fused_us"] = graph_us(lambda: cs.step_chain(ops, fused=True))
        result["chain_prep_us"] = graph_us(lambda: cs.step_chain_prep(ops))
        log(f"layer chain with projections (graph replay, GPU time): {result['chain_us']:.1f} us/token with the merge "
            f"launch, {result['chain_fused_us']:.1f} us/token with the merge folded into o_proj, "
            f"{result['chain_prep_us']:.1f} us/token with the prep folded into the q/k/v projection as well")
    del csets
    torch.cuda.empty_cache()
    return result


def measure_read_ceiling(torch, ops, gib: int = 2, reps: int = 10) -> float:
    """GB/s of a plain nontemporal streaming read over `gib` GiB (g4_read_ceiling), timed with events on
    the kernel's own start and end, best of `reps`: the measured ceiling next to the spec-sheet peak."""
    dev = torch.device("cuda:0")
    buf = torch.randint(0, 256, (gib << 30,), dtype=torch.uint8, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    for _ in range(3):
        ops.read_ceiling(buf, sink)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    stream = torch.cuda.current_stream()
    for a_, b_ in evs:
        a_.record(stream)
        b_.record(stream)
    torch.cuda.synchronize()
    for a_, b_ in evs:
        ops.read_ceiling(buf, sink, a_, b_)
    torch.cuda.synchronize()
    ms = min(a_.elapsed_time(b_) for a_, b_ in evs)  # a ceiling: the best of the runs
    del buf
    return (gib << 30) / (ms * 1e-3) / 1e9


_CEILING = None


def ceiling_fields(achieved_gbs: float) -> dict:
    """The measured read-stream ceiling of this GPU and the kernel's fraction of it (next to `frac`, which
    is against the spec sheet's 8 TB/s)."""
    global _CEILING
    import torch

    from g4attn import ops

    if _CEILING is None:
        _CEILING = measure_read_ceiling(torch, ops)
        log(f"read-stream ceiling {_CEILING:.1f} GB/s")
    c = _CEILING
    return {"measured_ceiling": round(c, 1), "frac_of_measured_ceiling": round(achieved_gbs / c, 4),
            "ceiling_source": "g4_read_ceiling: 2 GiB nontemporal 16-byte streaming read, best of 10"}


def read_traffic(workload: str):
    """HBM bytes per k_attn_step launch from the committed counter summary of this workload
    (FETCH_SIZE and WRITE_SIZE passes of rocprofv3 --pmc, scaled by a copy kernel's reading)."""
    return read_traffic_file(ROOT / "profiles" / f"k_attn_step_{workload}_traffic.txt")


def read_traffic_file(f: Path):
    """HBM bytes of the kernel per step: the summary's per-step figure for steps of several launches
    (one per head_dim group), else its per-launch figure."""
    if not f.exists():
        return None
    vals = {}
    for line in f.read_text().splitlines():
        k, _, v = line.partition(":")
        if k in ("hbm_bytes_per_launch", "hbm_bytes_per_step"):
            vals[k] = int(float(v))
    return vals.get("hbm_bytes_per_step", vals.get("hbm_bytes_per_launch"))


# ---- CPU baseline (oracle on the host) --------------------------------------------

def run_cpu_baseline(spec, seconds: float):
    import numpy as np

    from g4attn import e2b, synth
    from oracle import oracle as orc

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
    orc.set_threads(threads)
    rf = np.array(e2b.rope_freqs_f16_bits(256), dtype=np.uint16)
    layers = spec["layers"]
    # The reference's per-layer buffers: f32 caches of seq rows each (the WGSL scores and masks the rows
    # outside a local window, so they are read too); consumer layers read their producer's. Timing only:
    # filled from numpy's generator.
    rng = np.random.default_rng(spec["seed"])
    caches = {}
    for il, L in enumerate(layers):
        if L["producer"] is None:
            rows = L["seq"]
            caches[il] = (rng.standard_normal((rows, L["hd"]), dtype=np.float32),
                          rng.standard_normal((rows, L["hd"]), dtype=np.float32))
    log(f"cpu baseline: {threads} threads, {len(caches)} f32 cache pairs built")
    q0 = [synth.normal(spec["seed"] + 97 * il, NQH * L["hd"]) for il, L in enumerate(layers)]
    kv0 = [(synth.normal(spec["seed"] + 97 * il + 1, L["hd"]), synth.normal(spec["seed"] + 97 * il + 2, L["hd"]))
           for il, L in enumerate(layers)]

    def one_token():
        for il, L in enumerate(layers):
            hd = L["hd"]
            ones = np.full(hd, 0x3C00, dtype=np.uint16)
            own = L["producer"] is None
            kc, vc = caches[il if own else L["producer"]]
            q = orc.fused_per_head_norm_rope(q0[il], ones, rf, NQH, hd, EPS, L["pos"], L["theta"], L["divisor"])
            if own:
                v = orc.per_head_rms_norm_no_weight(kv0[il][1], NKH, hd, EPS)
                k = orc.fused_per_head_norm_rope(kv0[il][0], ones, rf, NKH, hd, EPS, L["pos"], L["theta"],
                                                 L["divisor"])
                kc[L["pos"]] = k  # kvCacheStore (f32 caches)
                vc[L["pos"]] = v
            orc.attention_chain(q, kc, vc, NQH, NKH, hd, L["seq"], 1.0, L["window"])

    n = 0
    t0 = time.perf_counter()
    while True:
        one_token()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 1000:
            break
    per_token = el / n
    return dict(per_token_s=per_token, tokens=n, threads=threads)


# ---- prefill (MFMA) ------------------------------------------------------------------

MFMA_F16_PEAK_TFLOPS = 2500.0


def run_prefill_gpu(args):
    import torch

    from g4attn import abi, ops, workloads

    abi.load()
    abi.call("g4_set_device", 0)
    dev = torch.device("cuda:0")
    _, entries, prep = workloads.prefill4k(dev, NQH, NKH, HD)
    arr = ops.make_prefill_entries(entries, NQH, NKH, HD)
    ws = torch.empty(ops.prefill_workspace_bytes(arr, NQH, NKH, HD), dtype=torch.uint8, device=dev)
    plan = ops.attn_prefill_prepare(arr, NQH, NKH, HD, ws)

    def step():  # the prompt's prep (both layers, every token) then the one prefill launch
        prep()
        ops.attn_prefill_run(plan)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # the prep alone
    for _ in range(3):
        prep()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        prep()
    torch.cuda.synchronize()
    prep_us = (time.perf_counter() - t1) / args.steps * 1e6
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    stream = torch.cuda.current_stream()
    for a_, b_ in evs:
        a_.record(stream)
        b_.record(stream)
    torch.cuda.synchronize()
    for a_, b_ in evs:
        ops.attn_prefill_run_timed(plan, a_, b_)
    torch.cuda.synchronize()
    k_ms = sum(a_.elapsed_time(b_) for a_, b_ in evs) / len(evs)
    log(f"prefill4k: {wall / args.steps * 1e6:.1f} us/step (prep {prep_us:.1f} us), {PREFILL_KERNEL} avg "
        f"{k_ms * 1e3:.1f} us")
    return dict(wall_s=wall, steps=args.steps, kernel_ms=k_ms, entries=len(entries), prep_us=prep_us)


def run_prefill_cpu(seconds: float):
    """The reference computes a prompt as one decode step per token: the oracle's chain at sampled
    positions (every 256th token of each layer), timed and scaled by the attended keys."""
    import numpy as np

    from g4attn.workloads import PREFILL_T, PREFILL_WINDOWS
    from oracle import oracle as orc

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
    orc.set_threads(threads)
    rng = np.random.default_rng(BASE_SEED)
    kc = rng.standard_normal((PREFILL_T, HD), dtype=np.float32)
    vc = rng.standard_normal((PREFILL_T, HD), dtype=np.float32)
    q = rng.standard_normal(NQH * HD, dtype=np.float32)
    done_flops, el, n = 0.0, 0.0, 0
    t0 = time.perf_counter()
    while el < seconds and n < 100000:  # the sampled positions, repeated until the time budget is used
        for w in PREFILL_WINDOWS:
            for t in range(PREFILL_T - 1, -1, -256):
                seq = t + 1
                orc.attention_chain(q, kc[:seq].reshape(-1), vc[:seq].reshape(-1), NQH, NKH, HD, seq, 1.0, w)
                done_flops += 4.0 * HD * NQH * (min(seq, w) if w else seq)
                n += 1
        el = time.perf_counter() - t0
    return dict(tflops=done_flops / el / 1e12, tokens=n, threads=threads, seconds=el)


def main_prefill(args):
    from g4attn import workloads

    r = run_prefill_gpu(args)
    flops = workloads.prefill_flops(NQH, HD)
    ms_per_step = r["wall_s"] / r["steps"] * 1e3
    value = flops / (ms_per_step * 1e-3) / 1e12
    achieved = flops / (r["kernel_ms"] * 1e-3) / 1e12
    line = {
        "metric": "prefill-attention TFLOP/s (% MFMA roofline), E2B-shaped, 4096-token prompt",
        "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16 Q/K/V/P, f32 accumulate", "data": "synthetic (seeded splitmix64 N(0,1), unit-RMS rows)",
        "config": {"workload": "prefill4k", "description": "causal prefill of a 4096-token prompt, 1 global + 1 "
                   "local (W=512) layer: per step the chunked prompt prep of every token (q/k RMSNorm + RoPE, v-norm, "
                   "f16 K/V store; one launch per layer) then one prefill launch over 512-token chunks (16 entries)",
                   "num_q_heads": NQH, "num_kv_heads": NKH, "head_dim": HD, "flops_per_step": flops,
                   "prep_us_per_step": round(r["prep_us"], 2)},
        "roofline": {"bound": "mfma", "kernel": PREFILL_KERNEL, "achieved": round(achieved, 2),
                     "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4),
                     "traffic": None, "avg_us": round(r["kernel_ms"] * 1e3, 2)},
    }
    if not args.no_cpu_baseline:
        c = run_prefill_cpu(args.cpu_seconds)
        line["cpu_baseline"] = {"value": round(c["tflops"], 5), "unit": "TFLOP/s", "cores": c["threads"],
                                "kind": "port", "sample": f"{c['tokens']} per-token decode chains of the oracle at "
                                f"every 256th position of both layers ({c['seconds']:.1f} s), scaled by attended keys"}
    print(json.dumps(line), flush=True)


# ---- sampling head (lm head GEMV + softcap + argmax) ------------------------------------

LM_VOCAB, LM_HIDDEN, LM_CAP = 262144, 1536, 30.0


def lm_bytes() -> int:
    return LM_VOCAB * LM_HIDDEN * 2 + LM_HIDDEN * 4 + LM_VOCAB * 4


def main_lmhead(args):
    import numpy as np
    import torch

    from g4attn import abi, ops

    abi.load()
    abi.call("g4_set_device", 0)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(BASE_SEED + 60)
    w = (torch.randn(LM_VOCAB * LM_HIDDEN, generator=g, device=dev) * 0.05).to(torch.float16).view(torch.int16)
    x = torch.randn(LM_HIDDEN, generator=g, device=dev)
    logits = torch.empty(LM_VOCAB, device=dev)
    res = torch.zeros(1, dtype=torch.int32, device=dev)
    ws = torch.empty(ops.lm_head_workspace_bytes(LM_VOCAB, LM_HIDDEN, LM_CAP), dtype=torch.uint8, device=dev)

    def step():
        ops.lm_head_argmax(x, w, logits, res, ws, LM_VOCAB, LM_HIDDEN, LM_CAP)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    stream = torch.cuda.current_stream()
    for a_, b_ in evs:
        a_.record(stream)
        b_.record(stream)
    torch.cuda.synchronize()
    for a_, b_ in evs:
        ops.lm_head_argmax_timed(x, w, logits, res, ws, LM_VOCAB, LM_HIDDEN, LM_CAP, a_, b_)
    torch.cuda.synchronize()
    k_ms = sum(a_.elapsed_time(b_) for a_, b_ in evs) / len(evs)
    nbytes = lm_bytes()
    ms_per_step = wall / args.steps * 1e3
    achieved = nbytes / (k_ms * 1e-3) / 1e9
    traffic = read_traffic_file(ROOT / "profiles" / "k_lm_head_lmhead_traffic.txt")
    log(f"lmhead: {ms_per_step * 1e3:.1f} us/step, k_lm_head avg {k_ms * 1e3:.1f} us, top-1 {int(res.item())}")
    line = {
        "metric": "sampling-head GB/s (% HBM roofline): lm head GEMV + softcap + argmax, E2B-shaped, bs1",
        "value": round(nbytes / (ms_per_step * 1e-3) / 1e9, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "us_per_token": round(ms_per_step * 1e3, 2),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16 weight, f32 accumulate",
        "data": "synthetic (torch seeded normal weights and hidden state), resident in HBM",
        "config": {"workload": f"lm head {LM_VOCAB} x {LM_HIDDEN} (f16 tied embedding), softcap {LM_CAP}, argmax",
                   "bytes_per_step": nbytes},
        "roofline": {"bound": "hbm", "kernel": "k_lm_head", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "avg_us": round(k_ms * 1e3, 2),
                     "traffic_source": "profiles/k_lm_head_lmhead_traffic.txt" if traffic else None},
    }
    line["roofline"].update(ceiling_fields(achieved))
    if not args.no_cpu_baseline:
        from oracle import oracle as orc

        threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
        orc.set_threads(threads)
        rows = 32768
        wb = w[: rows * LM_HIDDEN].cpu().numpy().view(np.uint16)
        xh = x.cpu().numpy()
        n, t0 = 0, time.perf_counter()
        while True:  # matmulQuant + logitSoftcap + argmax over a sample of rows, scaled to the vocabulary
            lg = orc.matmul_quant(xh, wb, rows, LM_HIDDEN)
            orc.argmax(orc.logit_softcap(lg, LM_CAP))
            n += 1
            el = time.perf_counter() - t0
            if el >= args.cpu_seconds or n >= 10000:
                break
        per_token = el / n * (LM_VOCAB / rows)
        line["cpu_baseline"] = {"value": round(nbytes / per_token / 1e9, 3), "unit": "GB/s", "cores": threads,
                                "kind": "port", "us_per_token": round(per_token * 1e6, 1),
                                "sample": f"{n} passes of the oracle's matmulQuant + logitSoftcap + argmax over "
                                          f"{rows} of the {LM_VOCAB} rows ({el:.1f} s), scaled to the full vocabulary"}
    print(json.dumps(line), flush=True)


def decode_line(name, args, decode_loop):
    spec = workload_spec(name)
    r = run_gpu(spec, args, decode_loop=decode_loop)
    ms_per_step = r["wall_s"] / r["steps"] * 1e3
    value = r["bytes"] / (ms_per_step * 1e-3) / 1e9
    achieved = r["bytes"] / (r["attn_avg_ms"] * 1e-3) / 1e9
    traffic = read_traffic(name)
    line = {
        "metric": "decode-attention us/token & HBM GB/s (% roofline), E2B-shaped, bs1",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "us_per_token": round(ms_per_step * 1e3, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 KV, f32 accumulate",
        "data": "synthetic (seeded splitmix64 N(0,1), unit-RMS rows), resident in HBM",
        "config": {"workload": name, "description": spec["desc"], "batch": 1, "num_q_heads": NQH,
                   "num_kv_heads": NKH, "head_dims": sorted({L["hd"] for L in spec["layers"]}),
                   "bytes_per_step": r["bytes"], "cache_sets_rotated": r["sets"],
                   "issue": "per head_dim, all entries of the step in one attention launch (q/k RMSNorm+RoPE, "
                            "v-norm, KV store, split-K attention) plus the log-sum-exp merge launch when the plan "
                            "has split entries; two head_dims: both plans' attention passes in one launch and "
                            "their merges in one"},
        "roofline": {"bound": "hbm", "kernel": r["kernel"], "launches_per_step": r["launches"],
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "avg_us": round(r["attn_avg_ms"] * 1e3, 2),
                     "traffic_source": f"profiles/k_attn_step_{name}_traffic.txt" if traffic else None},
    }
    line["roofline"].update(ceiling_fields(achieved))
    if "loop_us" in r:
        line["decode_loop"] = {"us_per_token": round(r["loop_us"], 2),
                               "prepare_us_per_token": round(r["loop_prepare_us"], 2),
                               "GBps": round(r["bytes"] / (r["loop_us"] * 1e-6) / 1e9, 1),
                               "vs_replay": round(r["loop_us"] / (ms_per_step * 1e3), 4),
                               "what": f"position advanced every token inside the timed region: the prepared plan "
                                       f"advanced on the host (g4_attn_step_advance, RoPE factors of the new position "
                                       f"evaluated in the kernel) and prepared again every {REPLAN_TOKENS} tokens; "
                                       "prepare_us_per_token is the host time per token (Python included)",
                               "prepare_every_token": {
                                   "us_per_token": round(r["loop_each_us"], 2),
                                   "prepare_us_per_token": round(r["loop_each_prepare_us"], 2),
                                   "what": "every entry prepared again every token (host partition, RoPE factors, "
                                           "pinned-ring table upload) and run"}}
    if "sequential_us" in r:
        line["layer_sequential_us_per_token"] = round(r["sequential_us"], 2)
    if "chain_us" in r:
        line["layer_chain"] = {
            "merge_launch_us_per_token": round(r["chain_us"], 2),
            "merge_in_o_proj_us_per_token": round(r["chain_fused_us"], 2),
            "prep_in_qkv_us_per_token": round(r["chain_prep_us"], 2),
            "what": "per token, every layer in the engine's order: q/k/v projection, attention pass, then the merge "
                    "launch and o_proj, or o_proj with the merge folded in (g4_attn_step_run_out), or with the "
                    "norms, RoPE and K/V store folded into the q/k/v projection (g4_linear_qkv_prep) and the merge "
                    "into o_proj; f16 weights of "
                    "E2B's shapes (hidden 1536); a HIP graph queued ahead of the GPU, median GPU time of a replay"}
    if not args.no_cpu_baseline:
        cpu = run_cpu_baseline(spec, args.cpu_seconds)
        cpu_gbs = r["bytes"] / cpu["per_token_s"] / 1e9
        line["cpu_baseline"] = {"value": round(cpu_gbs, 3), "unit": "GB/s", "cores": cpu["threads"], "kind": "port",
                                "us_per_token": round(cpu["per_token_s"] * 1e6, 1),
                                "sample": f"{cpu['tokens']} tokens of the same workload through the oracle's "
                                          "restatement of the six reference WGSL kernels (f32 caches, full-length "
                                          "scores on every layer); no WebGPU CPU adapter on the host"}
    return line


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default=DEFAULT_WORKLOAD,
                    choices=["stack32k", "stack8k", "stack4k", "stack128k", "e2b8k", "e2b32k", "long128k", "ragged64",
                             "layer512", "prefill4k", "lmhead"])
    ap.add_argument("--sets", type=int, default=0, help="cache sets to rotate (0 = enough to exceed 2x MALL)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--sequential", action=argparse.BooleanOptionalAction, default=True,
                    help="also time the layer-after-layer issue order (HIP graph)")
    ap.add_argument("--decode-loop", action=argparse.BooleanOptionalAction, default=True,
                    help="also time a position-advancing decode loop (prepare + run per token)")
    ap.add_argument("--pair", action=argparse.BooleanOptionalAction, default=True,
                    help="run a two-head_dim token's attention passes as one launch (E2B workloads)")
    ap.add_argument("--also", default=None,
                    help="a second decode workload reported nested in the same line (default: stack8k when the "
                         "workload is the default)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported (the attention path "
              "would shard by sequence or by KV range across GPUs, which is not built here)", file=sys.stderr)
        sys.exit(2)

    if args.workload == "prefill4k":
        main_prefill(args)
        return
    if args.workload == "lmhead":
        main_lmhead(args)
        return
    line = decode_line(args.workload, args, args.decode_loop)
    also = args.also if args.also is not None else ("stack8k" if args.workload == DEFAULT_WORKLOAD else "")
    if also:
        sub = decode_line(also, args, args.decode_loop)
        keep = ("value", "unit", "ms_per_step", "us_per_token", "config", "roofline", "decode_loop",
                "layer_sequential_us_per_token", "layer_chain", "cpu_baseline")
        line[also] = {k: sub[k] for k in keep if k in sub}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
