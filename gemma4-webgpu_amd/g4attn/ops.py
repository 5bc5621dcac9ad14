"""Tensor-level entry points over the C ABI (torch tensors on the HIP device).

Names follow the reference's kernel registry (src/shaders.ts:43-74):
fusedPerHeadNormRope, perHeadRmsNormNoWeight, kvCacheStore, attnScore,
softmax, attnOutput; plus the fused attn_prep / attn_decode /
attn_decode_many. Every wrapper checks device, dtype, contiguity and buffer
sizes on the host before anything is enqueued, so a shape mismatch raises
instead of reaching a kernel. torch is used for device memory and the
current stream only; all arithmetic runs in libg4attn.so.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import abi
from .abi import (G4_WEIGHT_Q4K, G4_WEIGHT_Q8, AttnOutputParams, AttnScoreParams, DecodeEntry, DecodePlan, KvStoreParams,
                  LinearQSeg, LinearSeg, LmHeadParams,
                  MatmulParams, NormParams, NormRopeParams, PrepLayer, PrepParams, SoftcapParams, SoftmaxParams,
                  StepEntry, PromptPrepParams)

F16_TYPES = (torch.float16, torch.int16, torch.uint16)


def _stream(stream=None) -> int:
    if stream is None:
        stream = torch.cuda.current_stream()
    return int(stream.cuda_stream) if hasattr(stream, "cuda_stream") else int(stream)


def _dev(t: torch.Tensor, name: str, dtypes, min_numel: int) -> int:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: must be on the GPU, got {t.device}")
    if t.dtype not in (dtypes if isinstance(dtypes, tuple) else (dtypes,)):
        raise TypeError(f"{name}: dtype {t.dtype} not in {dtypes}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    if t.numel() < min_numel:
        raise ValueError(f"{name}: {t.numel()} elements < {min_numel} required")
    return t.data_ptr()


def _f16(t, name, n):
    return _dev(t, name, F16_TYPES, n)


def _f32(t, name, n):
    return _dev(t, name, torch.float32, n)


# ---- the six reference kernels ---------------------------------------------

def fused_per_head_norm_rope(data, weight, rope_freqs, num_heads, head_dim, eps, position, theta,
                             apply_divisor, stream=None):
    p = NormRopeParams(num_heads, head_dim, eps, position, theta, apply_divisor)
    rf = _f16(rope_freqs, "rope_freqs", head_dim // 2) if apply_divisor else (
        rope_freqs.data_ptr() if rope_freqs is not None else None)
    abi.call("g4_fused_per_head_norm_rope", _f32(data, "data", num_heads * head_dim),
             _f16(weight, "weight", head_dim), rf, p, _stream(stream))


def per_head_rms_norm_no_weight(data, num_heads, head_dim, eps, stream=None):
    p = NormParams(num_heads, head_dim, eps, 0)
    abi.call("g4_per_head_rms_norm_no_weight", _f32(data, "data", num_heads * head_dim), p, _stream(stream))


def kv_cache_store(k_in, v_in, k_cache, v_cache, num_kv_heads, head_dim, position, max_seq_len, stream=None):
    n = num_kv_heads * head_dim
    p = KvStoreParams(num_kv_heads, head_dim, position, max_seq_len)
    need = (position + 1) * n
    abi.call("g4_kv_cache_store", _f32(k_in, "k_in", n), _f32(v_in, "v_in", n), _f16(k_cache, "k_cache", need),
             _f16(v_cache, "v_cache", need), p, _stream(stream))


def attn_score(q, k_cache, scores, num_q_heads, num_kv_heads, head_dim, seq_len, scale, sliding_window,
               stream=None):
    p = AttnScoreParams(num_q_heads, num_kv_heads, head_dim, seq_len, scale, sliding_window)
    abi.call("g4_attn_score", _f32(q, "q", num_q_heads * head_dim),
             _f16(k_cache, "k_cache", seq_len * num_kv_heads * head_dim),
             _f32(scores, "scores", num_q_heads * seq_len), p, _stream(stream))


def softmax(scores, num_heads, seq_len, stream=None):
    abi.call("g4_softmax", _f32(scores, "scores", num_heads * seq_len), SoftmaxParams(num_heads, seq_len),
             _stream(stream))


def attn_output(probs, v_cache, out, num_q_heads, num_kv_heads, head_dim, seq_len, stream=None):
    p = AttnOutputParams(num_q_heads, num_kv_heads, head_dim, seq_len)
    abi.call("g4_attn_output", _f32(probs, "probs", num_q_heads * seq_len),
             _f16(v_cache, "v_cache", seq_len * num_kv_heads * head_dim),
             _f32(out, "out", num_q_heads * head_dim), p, _stream(stream))


# ---- fused paths ------------------------------------------------------------

def attn_prep(q, k, v, q_weight, k_weight, rope_freqs, k_cache, v_cache, num_q_heads, num_kv_heads, head_dim,
              eps, position, theta, apply_divisor, slot, max_seq_len, store_kv=True, stream=None):
    p = PrepParams(num_q_heads, num_kv_heads, head_dim, eps, position, theta, apply_divisor, slot, max_seq_len,
                   1 if store_kv else 0)
    rf = _f16(rope_freqs, "rope_freqs", head_dim // 2) if apply_divisor else None
    nkv = num_kv_heads * head_dim
    if store_kv:
        args = (_f32(k, "k", nkv), _f32(v, "v", nkv), _f16(k_weight, "k_weight", head_dim), rf,
                _f16(k_cache, "k_cache", (slot + 1) * nkv), _f16(v_cache, "v_cache", (slot + 1) * nkv))
        if k_cache.numel() < max_seq_len * nkv or v_cache.numel() < max_seq_len * nkv:
            raise ValueError("attn_prep: caches smaller than max_seq_len rows")
    else:
        args = (None, None, None, rf, None, None)
    k_ptr, v_ptr, kw_ptr, rf_ptr, kc_ptr, vc_ptr = args
    abi.call("g4_attn_prep", _f32(q, "q", num_q_heads * head_dim), k_ptr, v_ptr,
             _f16(q_weight, "q_weight", head_dim), kw_ptr, rf_ptr, kc_ptr, vc_ptr, p, _stream(stream))


def make_prep_table(layers, num_q_heads, num_kv_heads, device):
    """Validate per-layer prep bindings on the host and upload them as a device table.

    layers: iterable of dicts with q, k, v, q_weight, k_weight, rope_freqs (or None), k_cache, v_cache
    (tensors; k/v/k_weight/caches may be None when store_kv is False), head_dim, theta, apply_divisor,
    store_kv, max_seq_len. Returns a uint8 device tensor holding the g4_prep_layer array.
    """
    layers = list(layers)
    arr = (PrepLayer * len(layers))()
    for i, L in enumerate(layers):
        hd = int(L["head_dim"])
        if hd <= 0 or hd % 2:
            raise ValueError(f"layer {i}: head_dim {hd}")
        store = bool(L["store_kv"])
        nkv = num_kv_heads * hd
        rf = L.get("rope_freqs")
        if L["apply_divisor"] and rf is None:
            raise ValueError(f"layer {i}: apply_divisor needs rope_freqs")
        arr[i] = PrepLayer(
            _f32(L["q"], f"layer {i} q", num_q_heads * hd),
            _f32(L["k"], f"layer {i} k", nkv) if store else None,
            _f32(L["v"], f"layer {i} v", nkv) if store else None,
            _f16(L["q_weight"], f"layer {i} q_weight", hd),
            _f16(L["k_weight"], f"layer {i} k_weight", hd) if store else None,
            _f16(rf, f"layer {i} rope_freqs", hd // 2) if rf is not None else None,
            _f16(L["k_cache"], f"layer {i} k_cache", L["max_seq_len"] * nkv) if store else None,
            _f16(L["v_cache"], f"layer {i} v_cache", L["max_seq_len"] * nkv) if store else None,
            hd, float(L["theta"]), int(L["apply_divisor"]), 1 if store else 0, int(L["max_seq_len"]),
        )
    host = torch.frombuffer(bytearray(bytes(arr)), dtype=torch.uint8)
    return host.to(device)


def attn_prep_many(table, n_layers, num_q_heads, num_kv_heads, eps, position, slot, stream=None):
    abi.call("g4_attn_prep_many", _dev(table, "table", torch.uint8, n_layers * C.sizeof(PrepLayer)), n_layers,
             num_q_heads, num_kv_heads, eps, position, slot, _stream(stream))


def decode_workspace_bytes(num_q_heads, num_kv_heads, head_dim, max_seq_len) -> int:
    n = C.c_size_t(0)
    abi.call("g4_attn_decode_workspace_size", num_q_heads, num_kv_heads, head_dim, max_seq_len, C.byref(n))
    return n.value


def attn_decode(q, k_cache, v_cache, out, workspace, num_q_heads, num_kv_heads, head_dim, seq_len, scale=1.0,
                sliding_window=0, stream=None):
    p = AttnScoreParams(num_q_heads, num_kv_heads, head_dim, seq_len, scale, sliding_window)
    rows = seq_len * num_kv_heads * head_dim
    ws_ptr, ws_bytes = (None, 0) if workspace is None else (_dev(workspace, "workspace", torch.uint8, 0),
                                                             workspace.numel())
    abi.call("g4_attn_decode", _f32(q, "q", num_q_heads * head_dim), _f16(k_cache, "k_cache", rows),
             _f16(v_cache, "v_cache", rows), _f32(out, "out", num_q_heads * head_dim), p, ws_ptr, ws_bytes,
             _stream(stream))


def attn_decode_noalloc(q, k_cache, v_cache, out, num_q_heads, num_kv_heads, head_dim, seq_len, scale=1.0,
                        sliding_window=0, stream=None):
    """attn_decode without a workspace: the split partials use the library's fixed scratch array."""
    p = AttnScoreParams(num_q_heads, num_kv_heads, head_dim, seq_len, scale, sliding_window)
    rows = seq_len * num_kv_heads * head_dim
    abi.call("g4_attn_decode_noalloc", _f32(q, "q", num_q_heads * head_dim), _f16(k_cache, "k_cache", rows),
             _f16(v_cache, "v_cache", rows), _f32(out, "out", num_q_heads * head_dim), p, _stream(stream))


def decode_many_workspace_bytes(n_entries, num_q_heads, num_kv_heads, head_dim, total_rows) -> int:
    n = C.c_size_t(0)
    abi.call("g4_attn_decode_many_workspace_size", n_entries, num_q_heads, num_kv_heads, head_dim, total_rows,
             C.byref(n))
    return n.value


def make_entries(items, num_q_heads, num_kv_heads, head_dim):
    """items: iterable of (q, k_cache, v_cache, out, seq_len, sliding_window, scale)."""
    items = list(items)
    arr = (DecodeEntry * len(items))()
    for i, (q, kc, vc, out, seq_len, window, scale) in enumerate(items):
        rows = seq_len * num_kv_heads * head_dim
        arr[i] = DecodeEntry(_f32(q, f"entry {i} q", num_q_heads * head_dim), _f16(kc, f"entry {i} k", rows),
                             _f16(vc, f"entry {i} v", rows), _f32(out, f"entry {i} out", num_q_heads * head_dim),
                             seq_len, window, scale, 0)
    return arr


def attn_decode_many_prepare(entries, num_q_heads, num_kv_heads, head_dim, workspace, stream=None) -> DecodePlan:
    plan = DecodePlan()
    abi.call("g4_attn_decode_many_prepare", entries, len(entries), num_q_heads, num_kv_heads, head_dim,
             _dev(workspace, "workspace", torch.uint8, 0), workspace.numel(), C.byref(plan), _stream(stream))
    return plan


def attn_decode_many_run(plan: DecodePlan, stream=None):
    abi.call("g4_attn_decode_many_run", C.byref(plan), _stream(stream))


def attn_decode_many_run_split(plan: DecodePlan, stream=None):
    abi.call("g4_attn_decode_many_run_split", C.byref(plan), _stream(stream))


def attn_decode_many_run_merge(plan: DecodePlan, stream=None):
    abi.call("g4_attn_decode_many_run_merge", C.byref(plan), _stream(stream))


def attn_decode_many(entries, num_q_heads, num_kv_heads, head_dim, workspace, stream=None):
    abi.call("g4_attn_decode_many", entries, len(entries), num_q_heads, num_kv_heads, head_dim,
             _dev(workspace, "workspace", torch.uint8, 0), workspace.numel(), _stream(stream))


# ---- one-launch decode step --------------------------------------------------

def step_workspace_bytes(n_entries, num_q_heads, num_kv_heads, head_dim) -> int:
    n = C.c_size_t(0)
    abi.call("g4_attn_step_workspace_size", n_entries, num_q_heads, num_kv_heads, head_dim, C.byref(n))
    return n.value


def rope_inv_freq(theta, head_dim, apply_divisor, rope_freqs=None, stream=None) -> torch.Tensor:
    """The [head_dim/2] f32 RoPE inverse-frequency table of one (theta, divisor) configuration."""
    if apply_divisor and rope_freqs is None:
        raise ValueError("apply_divisor needs rope_freqs")
    dev = rope_freqs.device if rope_freqs is not None else torch.device("cuda", torch.cuda.current_device())
    out = torch.empty(head_dim // 2, dtype=torch.float32, device=dev)
    rf = _f16(rope_freqs, "rope_freqs", head_dim // 2) if rope_freqs is not None else None
    abi.call("g4_rope_inv_freq", float(theta), head_dim, 1 if apply_divisor else 0, rf, _f32(out, "out", head_dim // 2),
             _stream(stream))
    return out


def rope_inv_freq_host(theta, head_dim, apply_divisor, rope_freqs_bits=None):
    """The [head_dim/2] RoPE inverse-frequency table computed on the host (numpy float32), for
    step entries' rope_inv_freq_host; rope_freqs_bits: host f16 bits of the divisor table."""
    import numpy as np

    if apply_divisor and rope_freqs_bits is None:
        raise ValueError("apply_divisor needs rope_freqs_bits")
    out = np.empty(head_dim // 2, dtype=np.float32)
    rf = None
    if rope_freqs_bits is not None:
        rf = np.ascontiguousarray(rope_freqs_bits, dtype=np.uint16)
        if rf.size < head_dim // 2:
            raise ValueError("rope_freqs_bits: too short")
    abi.call("g4_rope_inv_freq_host", float(theta), head_dim, 1 if apply_divisor else 0,
             rf.ctypes.data if rf is not None else None, out.ctypes.data)
    return out


def _host_f32(a, name, n):
    import numpy as np

    if not isinstance(a, np.ndarray) or a.dtype != np.float32 or not a.flags.c_contiguous or a.size < n:
        raise TypeError(f"{name}: expected a contiguous host float32 array of at least {n} values")
    return a.ctypes.data


def make_step_entries(items, num_q_heads, num_kv_heads, head_dim):
    """items: iterable of dicts with q, k, v (raw f32 projections), q_weight, k_weight (f16), rope_freqs (f16 or
    None), rope_inv_freq_host (optional host f32 numpy table from rope_inv_freq_host(); kept alive by the caller
    until prepare returns), k_cache, v_cache (f16, at least seq_len rows),
    out (f32), seq_len, position, sliding_window, store_kv, theta, apply_divisor, scale, eps, and q_ready (q
    already holds the post-norm, post-RoPE query, as linear_qkv_prep leaves it).
    k, v and k_weight None (with store_kv False): the current row is already in the cache (a KV-consumer
    layer stepped after its producer)."""
    items = list(items)
    arr = (StepEntry * len(items))()
    for i, it in enumerate(items):
        L = int(it["seq_len"])
        nkv = num_kv_heads * head_dim
        rf = it.get("rope_freqs")
        if it["apply_divisor"] and rf is None:
            raise ValueError(f"entry {i}: apply_divisor needs rope_freqs")
        def opt(t, conv, name, n):
            return None if t is None else conv(t, name, n)

        arr[i] = StepEntry(
            _f32(it["q"], f"entry {i} q", num_q_heads * head_dim), opt(it.get("k"), _f32, f"entry {i} k", nkv),
            opt(it.get("v"), _f32, f"entry {i} v", nkv), _f16(it["q_weight"], f"entry {i} q_weight", head_dim),
            opt(it.get("k_weight"), _f16, f"entry {i} k_weight", head_dim),
            _f16(rf, f"entry {i} rope_freqs", head_dim // 2) if rf is not None else None,
            _host_f32(it["rope_inv_freq_host"], f"entry {i} rope_inv_freq_host", head_dim // 2)
            if it.get("rope_inv_freq_host") is not None else None,
            _f16(it["k_cache"], f"entry {i} k_cache", L * nkv), _f16(it["v_cache"], f"entry {i} v_cache", L * nkv),
            _f32(it["out"], f"entry {i} out", num_q_heads * head_dim), L, int(it["position"]),
            int(it.get("sliding_window", 0)), 1 if it.get("store_kv", True) else 0, float(it["theta"]),
            int(it["apply_divisor"]), float(it.get("scale", 1.0)), float(it.get("eps", 1e-6)),
            1 if it.get("q_ready") else 0)
    return arr


def attn_step_prepare(entries, num_q_heads, num_kv_heads, head_dim, workspace, stream=None) -> DecodePlan:
    plan = DecodePlan()
    abi.call("g4_attn_step_prepare", entries, len(entries), num_q_heads, num_kv_heads, head_dim,
             _dev(workspace, "workspace", torch.uint8, 0), workspace.numel(), C.byref(plan), _stream(stream))
    return plan


def step_layers_workspace_bytes(n_layers, num_q_heads, num_kv_heads, head_dim, entries_per_layer=1) -> int:
    n = C.c_size_t(0)
    abi.call("g4_attn_step_layers_workspace_size", n_layers, entries_per_layer, num_q_heads, num_kv_heads, head_dim,
             C.byref(n))
    return n.value


def attn_step_prepare_layers(entries, num_q_heads, num_kv_heads, head_dim, workspace, entries_per_layer=1,
                             stream=None) -> list:
    """One token's layers prepared together (one upload): layer i is entries[i * entries_per_layer ..
    (i + 1) * entries_per_layer); a plan per layer, each run on its own in layer order with
    attn_step_run_attention then attn_step_run_merge or attn_step_run_out."""
    if entries_per_layer < 1 or len(entries) % entries_per_layer:
        raise ValueError(f"{len(entries)} entries are not whole layers of {entries_per_layer}")
    n_layers = len(entries) // entries_per_layer
    plans = (DecodePlan * n_layers)()
    abi.call("g4_attn_step_prepare_layers", entries, n_layers, entries_per_layer, num_q_heads, num_kv_heads, head_dim,
             _dev(workspace, "workspace", torch.uint8, 0), workspace.numel(), plans, _stream(stream))
    return list(plans)


def attn_step_advance(plan: DecodePlan, tokens: int = 1):
    """The next token(s) of a prepared plan without a new prepare: host-only (nothing is enqueued);
    every entry's seq_len and position grow by `tokens` (g4_attn_step_advance). Raises G4Error with
    status G4_ERANGE past 4096 tokens since the prepare."""
    abi.call("g4_attn_step_advance", C.byref(plan), tokens)


def attn_step_run(plan: DecodePlan, stream=None):
    abi.call("g4_attn_step_run", C.byref(plan), _stream(stream))


def attn_step_run_attention(plan: DecodePlan, stream=None):
    abi.call("g4_attn_step_run_attention", C.byref(plan), _stream(stream))


def attn_step_run_merge(plan: DecodePlan, stream=None):
    abi.call("g4_attn_step_run_merge", C.byref(plan), _stream(stream))


def attn_step_run_pair(plan_1: DecodePlan, plan_2: DecodePlan, stream=None):
    """A token's head_dim-512 and head_dim-256 plans (either order): both attention passes in one launch, then
    each plan's merge."""
    abi.call("g4_attn_step_run_pair", C.byref(plan_1), C.byref(plan_2), _stream(stream))


def attn_step_run_attention_pair(plan_1: DecodePlan, plan_2: DecodePlan, stream=None):
    abi.call("g4_attn_step_run_attention_pair", C.byref(plan_1), C.byref(plan_2), _stream(stream))


def attn_step_run_attention_pair_timed(plan_1: DecodePlan, plan_2: DecodePlan, start, stop, stream=None):
    """attn_step_run_attention_pair with torch.cuda.Events (timing enabled) around the one launch."""
    for e, name in ((start, "start"), (stop, "stop")):
        if not getattr(e, "cuda_event", 0):
            raise ValueError(f"{name} event has no HIP event yet (record it once first)")
    abi.call("g4_attn_step_run_attention_pair_timed", C.byref(plan_1), C.byref(plan_2), _stream(stream),
             C.c_void_p(start.cuda_event), C.c_void_p(stop.cuda_event))


def attn_step_run_out(plan: DecodePlan, n, segments, stream=None):
    """attn.linearOut after g4_attn_step_run_attention, with the step's merge folded in: one
    (weight f16 [rows][n], out f32 [rows], rows) segment per entry of the plan, n = num_q_heads * head_dim.
    Writes every entry's attnOut as g4_attn_step_run_merge does and out = weight @ attnOut."""
    segs = (LinearSeg * len(segments))()
    for i, (w, out, rows) in enumerate(segments):
        segs[i] = LinearSeg(_f16(w, f"segment {i} weight", rows * n), _f32(out, f"segment {i} out", rows), rows)
    abi.call("g4_attn_step_run_out", C.byref(plan), segs, len(segments), _stream(stream))


def attn_step_run_attention_timed(plan: DecodePlan, start, stop, stream=None):
    """The attention launch with torch.cuda.Events (timing enabled) that take the kernel's own
    start and end timestamps. The events must exist: record each once before the first use."""
    for e, name in ((start, "start"), (stop, "stop")):
        if not getattr(e, "cuda_event", 0):
            raise ValueError(f"{name} event has no HIP event yet (record it once first)")
    abi.call("g4_attn_step_run_attention_timed", C.byref(plan), _stream(stream), C.c_void_p(start.cuda_event),
             C.c_void_p(stop.cuda_event))


def read_ceiling(buf, sink, start=None, stop=None, stream=None):
    """The device's read-stream ceiling: streams buf (a contiguous GPU tensor) with the decode kernels'
    nontemporal 16-byte loads; with events (timing enabled, recorded once before), they take the kernel's
    own start and end."""
    ev = [C.c_void_p(e.cuda_event) if e is not None else None for e in (start, stop)]
    abi.call("g4_read_ceiling", _dev(buf, "buf", buf.dtype, 1), buf.numel() * buf.element_size(),
             _dev(sink, "sink", (torch.int32, torch.uint32), 1), _stream(stream), ev[0], ev[1])


class QuerySet:
    """Timestamp queries for labelled passes (g4_query_set_*; the engine's GPUQuerySet, src/engine.ts:
    3089-3110, 3208-3227, 3253-3288). begin_pass(slot) .. end_pass(): the library kernels launched from
    this thread in between carry the pair (slot, slot+1) on their own dispatches; write(slot) records a
    marker in stream order instead. resolve(first, n_pairs) waits and returns each pair's ns (float64,
    NaN for a pair not written since its last resolve)."""

    def __init__(self, count: int):
        h = C.c_void_p(0)
        abi.call("g4_query_set_create", count, C.byref(h))
        self.handle, self.count = h, count

    def begin_pass(self, slot: int):
        abi.call("g4_query_begin_pass", self.handle, slot)

    @staticmethod
    def end_pass():
        abi.call("g4_query_end_pass")

    def write(self, slot: int, stream=None):
        abi.call("g4_query_write", self.handle, slot, _stream(stream))

    def resolve(self, first: int, n_pairs: int):
        import numpy as np
        out = np.zeros(max(n_pairs, 1), np.float64)
        abi.call("g4_query_resolve", self.handle, first, n_pairs, out.ctypes.data_as(C.POINTER(C.c_double)))
        return out[:n_pairs]

    def close(self):
        if self.handle:
            abi.call("g4_query_set_destroy", self.handle)
            self.handle = None


def attn_step(entries, num_q_heads, num_kv_heads, head_dim, workspace, stream=None):
    abi.call("g4_attn_step", entries, len(entries), num_q_heads, num_kv_heads, head_dim,
             _dev(workspace, "workspace", torch.uint8, 0), workspace.numel(), _stream(stream))


# ---- chunked prompt prep ----------------------------------------------------------

def vt_cache_elems(max_seq_len, num_kv_heads, head_dim) -> int:
    """f16 elements of a V^T block cache for max_seq_len rows ([kv head][ceil(rows / 32)][HD][32])."""
    return (max_seq_len + 31) // 32 * 32 * num_kv_heads * head_dim


def _prompt_prep_args(q, q_weight, q_out, n_tokens, start, num_q_heads, num_kv_heads, head_dim, theta, apply_divisor,
                      rope_freqs=None, k=None, v=None, k_weight=None, k_cache=None, v_cache=None, max_seq_len=0,
                      eps=1e-6, rope_inv_freq=None, vt_cache=None):
    """The checked device pointers and params of one chunk's prompt prep (attn_prompt_prep's arguments)."""
    store = k is not None
    nq = n_tokens * num_q_heads * head_dim
    nk = n_tokens * num_kv_heads * head_dim
    p = PromptPrepParams(num_q_heads, num_kv_heads, head_dim, n_tokens, start, eps, theta, 1 if apply_divisor else 0,
                         1 if store else 0, max_seq_len)
    rows = max_seq_len * num_kv_heads * head_dim
    args = [_f32(q, "q", nq), _f32(k, "k", nk) if store else None,
            _f32(v, "v", nk) if store else None, _f16(q_weight, "q_weight", head_dim),
            _f16(k_weight, "k_weight", head_dim) if store else None,
            _f16(rope_freqs, "rope_freqs", head_dim // 2) if rope_freqs is not None else None,
            _f32(rope_inv_freq, "rope_inv_freq", head_dim // 2) if rope_inv_freq is not None else None,
            _f16(q_out, "q_out", nq), _f16(k_cache, "k_cache", rows) if store else None,
            _f16(v_cache, "v_cache", rows) if store else None]
    vt = _f16(vt_cache, "vt_cache", vt_cache_elems(max_seq_len, num_kv_heads, head_dim)) \
        if vt_cache is not None else None
    return args, vt, p


def attn_prompt_prep_many(chunks, stream=None):
    """Several chunks' prompt preps (dicts of attn_prompt_prep's keyword arguments, one head_dim) in one launch
    (g4_attn_prompt_prep_many), each giving the bits of its own attn_prompt_prep call."""
    from .abi import PromptPrepEntry

    chunks = list(chunks)
    arr = (PromptPrepEntry * len(chunks))()
    for i, kw in enumerate(chunks):
        args, vt, p = _prompt_prep_args(**kw)
        arr[i] = PromptPrepEntry(*args, vt, p)
    abi.call("g4_attn_prompt_prep_many", arr, len(chunks), _stream(stream))


def attn_prompt_prep(q, q_weight, q_out, n_tokens, start, num_q_heads, num_kv_heads, head_dim, theta, apply_divisor,
                     rope_freqs=None, k=None, v=None, k_weight=None, k_cache=None, v_cache=None, max_seq_len=0,
                     eps=1e-6, rope_inv_freq=None, vt_cache=None, stream=None):
    """q/k/v/norm+RoPE/store of n_tokens prompt tokens at positions start.. in one launch. q: f32
    [n_tokens][NQH][HD]; q_out: f16 [n_tokens][NQH][HD]; with k (and v, k_weight, caches of max_seq_len rows)
    the layer is a KV producer and rows start .. start + n_tokens - 1 are stored. rope_inv_freq: optional
    device table from rope_inv_freq() for this layer's theta/divisor (else each workgroup evaluates it).
    vt_cache (KV producers): the V rows also go there as V^T blocks (g4_attn_prompt_prep_vt), of
    vt_cache_elems(max_seq_len, ...) f16 elements."""
    args, vt, p = _prompt_prep_args(q, q_weight, q_out, n_tokens, start, num_q_heads, num_kv_heads, head_dim, theta,
                                    apply_divisor, rope_freqs, k, v, k_weight, k_cache, v_cache, max_seq_len, eps,
                                    rope_inv_freq, vt_cache)
    if vt is None:
        abi.call("g4_attn_prompt_prep", *args, p, _stream(stream))
    else:
        abi.call("g4_attn_prompt_prep_vt", *args, vt, p, _stream(stream))


# ---- causal prefill ------------------------------------------------------------

def make_prefill_entries(items, num_q_heads, num_kv_heads, head_dim):
    """items: dicts with q (f16 [n_tokens][NQH][HD]), k_cache, v_cache (f16, at least start + n_tokens rows),
    out (f32 [n_tokens][NQH][HD]), n_tokens, start, sliding_window, scale; optionally vt_cache (the V^T
    blocks the prompt prep wrote) with vt_rows (the max_seq_len it was sized for)."""
    from .abi import PrefillEntry

    items = list(items)
    arr = (PrefillEntry * len(items))()
    for i, it in enumerate(items):
        T, s0 = int(it["n_tokens"]), int(it["start"])
        kv = (s0 + T) * num_kv_heads * head_dim
        vt, vt_rows = it.get("vt_cache"), int(it.get("vt_rows", 0))
        arr[i] = PrefillEntry(_f16(it["q"], f"entry {i} q", T * num_q_heads * head_dim),
                              _f16(it["k_cache"], f"entry {i} k_cache", kv), _f16(it["v_cache"], f"entry {i} v_cache", kv),
                              _f32(it["out"], f"entry {i} out", T * num_q_heads * head_dim), T, s0,
                              int(it.get("sliding_window", 0)), float(it.get("scale", 1.0)),
                              _f16(vt, f"entry {i} vt_cache", vt_cache_elems(vt_rows, num_kv_heads, head_dim))
                              if vt is not None else None, vt_rows)
    return arr


def prefill_workspace_bytes(entries, num_q_heads, num_kv_heads, head_dim) -> int:
    n = C.c_size_t()
    abi.call("g4_attn_prefill_workspace_size", entries, len(entries), num_q_heads, num_kv_heads, head_dim,
             C.byref(n))
    return n.value


def attn_prefill_prepare(entries, num_q_heads, num_kv_heads, head_dim, workspace, stream=None) -> DecodePlan:
    plan = DecodePlan()
    abi.call("g4_attn_prefill_prepare", entries, len(entries), num_q_heads, num_kv_heads, head_dim,
             _dev(workspace, "workspace", torch.uint8, 0), workspace.numel(), C.byref(plan), _stream(stream))
    return plan


def attn_prefill_run(plan: DecodePlan, stream=None):
    abi.call("g4_attn_prefill_run", C.byref(plan), _stream(stream))


def attn_prefill_run_timed(plan: DecodePlan, start, stop, stream=None):
    for e, name in ((start, "start"), (stop, "stop")):
        if not getattr(e, "cuda_event", 0):
            raise ValueError(f"{name} event has no HIP event yet (record it once first)")
    abi.call("g4_attn_prefill_run_timed", C.byref(plan), _stream(stream), C.c_void_p(start.cuda_event),
             C.c_void_p(stop.cuda_event))


def attn_prefill(entries, num_q_heads, num_kv_heads, head_dim, workspace, stream=None):
    abi.call("g4_attn_prefill", entries, len(entries), num_q_heads, num_kv_heads, head_dim,
             _dev(workspace, "workspace", torch.uint8, 0), workspace.numel(), _stream(stream))


# ---- lm head -> logit softcap -> argmax ------------------------------------------

def matmul_quant_f16(x, weight, out, M, N, stream=None):
    """SHADERS.matmulQuant: out[m] = sum_k f16 weight[m][k] * x[k] (matmul_quant.wgsl order)."""
    abi.call("g4_matmul_quant_f16", _f32(x, "input", N), _f16(weight, "weight", M * N), _f32(out, "output", M),
             MatmulParams(M, N), _stream(stream))


def linear_f16(x, n, segments, stream=None):
    """attn.linearQKV / attn.linearOut: for each (weight f16 [rows][n], out f32 [rows], rows) segment,
    out = weight @ x with matmul_quant.wgsl's summation order; up to four segments in one launch."""
    segs = (LinearSeg * len(segments))()
    for i, (w, out, rows) in enumerate(segments):
        segs[i] = LinearSeg(_f16(w, f"segment {i} weight", rows * n), _f32(out, f"segment {i} out", rows), rows)
    abi.call("g4_linear_f16", _f32(x, "input", n), n, segs, len(segments), _stream(stream))


I8_TYPES = (torch.int8, torch.uint8)
U32_TYPES = (torch.int32, torch.uint32)


def matmul_q8(x, qweight, qscale, out, M, N, stream=None):
    """SHADERS.matmulQ8: out[m] = sum_k (int8 qweight[m][k] * f16 qscale[m][k / 32]) * x[k]."""
    abi.call("g4_matmul_q8", _f32(x, "input", N), _dev(qweight, "qweight", I8_TYPES, M * N),
             _f16(qscale, "qscale", M * (N // 32)), _f32(out, "output", M), MatmulParams(M, N), _stream(stream))


def matmul_q4k(x, qweight, qmeta, out, M, N, stream=None):
    """SHADERS.matmulQ4K: 4-bit weights packed 8 per u32 (low nibble first), f16 meta [M][N/256][16]."""
    abi.call("g4_matmul_q4k", _f32(x, "input", N), _dev(qweight, "qweight", U32_TYPES, M * N // 8),
             _f16(qmeta, "qmeta", M * (N // 256) * 16), _f32(out, "output", M), MatmulParams(M, N), _stream(stream))


def linear_quant(x, n, fmt, segments, stream=None):
    """The projections with quantized weights: fmt "q8" (segments of (int8 weight [rows][n], f16 scales
    [rows][n/32], out, rows)) or "q4k" (u32 weight [rows][n/8], f16 meta [rows][n/256][16], out, rows)."""
    q8 = fmt == "q8"
    segs = (LinearQSeg * len(segments))()
    for i, (w, meta, out, rows) in enumerate(segments):
        wp = _dev(w, f"segment {i} weight", I8_TYPES, rows * n) if q8 else \
            _dev(w, f"segment {i} weight", U32_TYPES, rows * n // 8)
        mp = _f16(meta, f"segment {i} meta", rows * (n // 32 if q8 else n // 16))
        segs[i] = LinearQSeg(wp, mp, _f32(out, f"segment {i} out", rows), rows)
    abi.call("g4_linear_quant", _f32(x, "input", n), n, G4_WEIGHT_Q8 if q8 else G4_WEIGHT_Q4K, segs, len(segments),
             _stream(stream))


def qkv_prep_workspace_bytes(num_q_heads, num_kv_heads) -> int:
    n = C.c_size_t(0)
    abi.call("g4_linear_qkv_prep_workspace_size", num_q_heads, num_kv_heads, C.byref(n))
    return n.value


def linear_qkv_prep(x, n, fmt, segments, q_weight, num_q_heads, num_kv_heads, head_dim, position, theta,
                    apply_divisor, workspace, k_weight=None, rope_freqs=None, rope_inv_freq=None, k_cache=None,
                    v_cache=None, slot=0, max_seq_len=0, eps=1e-6, stream=None):
    """attn.linearQKV with the producer-side prep as its epilogue (g4_linear_qkv_prep). fmt "f16"
    (segments of (weight f16 [rows][n], out, rows)), "q8" or "q4k" (as linear_quant); segments q, k, v
    on a KV producer (k_weight, caches of max_seq_len rows and slot given), q alone otherwise. The
    workspace (qkv_prep_workspace_bytes) must be zero before the first call."""
    from .abi import QkvPrepParams

    fmt_code = {"f16": abi.G4_WEIGHT_F16, "q8": G4_WEIGHT_Q8, "q4k": G4_WEIGHT_Q4K}[fmt]
    segs = (LinearQSeg * len(segments))()
    for i, sg in enumerate(segments):
        if fmt == "f16":
            w, out, rows = sg
            wp, mp = _f16(w, f"segment {i} weight", rows * n), None
        else:
            w, meta, out, rows = sg
            wp = _dev(w, f"segment {i} weight", I8_TYPES, rows * n) if fmt == "q8" else \
                _dev(w, f"segment {i} weight", U32_TYPES, rows * n // 8)
            mp = _f16(meta, f"segment {i} meta", rows * (n // 32 if fmt == "q8" else n // 16))
        segs[i] = LinearQSeg(wp, mp, _f32(out, f"segment {i} out", rows), rows)
    store = k_cache is not None
    p = QkvPrepParams(num_q_heads, num_kv_heads, head_dim, position, slot, max_seq_len, eps, theta,
                      1 if apply_divisor else 0, 1 if store else 0)
    rows = max_seq_len * num_kv_heads * head_dim
    abi.call("g4_linear_qkv_prep", _f32(x, "input", n), n, fmt_code, segs, len(segments),
             _f16(q_weight, "q_weight", head_dim), _f16(k_weight, "k_weight", head_dim) if store else None,
             _f16(rope_freqs, "rope_freqs", head_dim // 2) if rope_freqs is not None else None,
             _f32(rope_inv_freq, "rope_inv_freq", head_dim // 2) if rope_inv_freq is not None else None,
             _f16(k_cache, "k_cache", rows) if store else None, _f16(v_cache, "v_cache", rows) if store else None,
             p, _dev(workspace, "workspace", torch.uint8, 0), _stream(stream))


def logit_softcap(logits, size, cap, stream=None):
    abi.call("g4_logit_softcap", _f32(logits, "logits", size), SoftcapParams(size, cap), _stream(stream))


def argmax(logits, result, size, stream=None):
    """SHADERS.argmax: result[0] = top-1 index under argmax.wgsl's rule."""
    abi.call("g4_argmax", _f32(logits, "logits", size), _dev(result, "result", (torch.int32, torch.uint32), 1),
             size, _stream(stream))


def lm_head_workspace_bytes(vocab, hidden, cap) -> int:
    n = C.c_size_t(0)
    abi.call("g4_lm_head_workspace_size", LmHeadParams(vocab, hidden, cap), C.byref(n))
    return int(n.value)


def _lm_head_args(hidden, weight, logits, result, workspace, vocab, hidden_size, cap):
    return (_f32(hidden, "hidden", hidden_size), _f16(weight, "weight", vocab * hidden_size),
            _f32(logits, "logits", vocab) if logits is not None else None,
            _dev(result, "result", (torch.int32, torch.uint32), 1), _dev(workspace, "workspace", torch.uint8, 0),
            workspace.numel(), LmHeadParams(vocab, hidden_size, cap))


def lm_head_argmax(hidden, weight, logits, result, workspace, vocab, hidden_size, cap, stream=None):
    """lmHead -> logitSoftcap -> argmax in one streaming pass (+ a one-workgroup pick): result[0] = top-1
    index; logits (optional) = the softcapped logits, bit-identical to the three-kernel chain."""
    abi.call("g4_lm_head_argmax", *_lm_head_args(hidden, weight, logits, result, workspace, vocab, hidden_size, cap),
             _stream(stream))


def lm_head_argmax_timed(hidden, weight, logits, result, workspace, vocab, hidden_size, cap, start, stop,
                         stream=None):
    """lm_head_argmax with torch.cuda.Events (timing enabled) around the streaming kernel; the events
    must exist (record each once before the first use)."""
    for e, name in ((start, "start"), (stop, "stop")):
        if not getattr(e, "cuda_event", 0):
            raise ValueError(f"{name} event has no HIP event yet (record it once first)")
    abi.call("g4_lm_head_argmax_timed", *_lm_head_args(hidden, weight, logits, result, workspace, vocab,
                                                      hidden_size, cap),
             _stream(stream), C.c_void_p(start.cuda_event), C.c_void_p(stop.cuda_event))
