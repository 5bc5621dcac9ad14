"""Oracle — TEST INFRASTRUCTURE ONLY (imported by tests/, __graft_entry__.smoke()
and bench.py's CPU-baseline leg; never by the product library).

numpy bindings of oracle/wgsl_ref.c, the WGSL-semantics C restatement of
gemma4-webgpu's six attention shaders (shaders/fused_per_head_norm_rope.wgsl,
per_head_rms_norm_no_weight.wgsl, kv_cache_store.wgsl, attn_score.wgsl,
softmax.wgsl, attn_output.wgsl; dispatch grids from src/engine.ts:2060-2094).

Every function takes and returns numpy arrays; in-place WGSL kernels return
the updated copy. Caches passed to the WGSL functions are f32 (as the WGSL
binds them); `f16_bits_to_f32` widens the build's f16 cache format exactly.

How each function is pinned (tests/test_oracle.py):
  f32_to_f16 / f16_to_f32     numpy float16 casts (IEEE RNE), exhaustive over all 65536 bit patterns
  fused_per_head_norm_rope    fp64 closed form (closed_form.norm_rope64), HF-style rotate-half RoPE from
                              the installed transformers, invariants (pos 0 identity, pair norms, divisor
                              table), real-model layer-0 q/k norm vectors (public/ref/layer_0_detail.npz)
  per_head_rms_norm_no_weight fp64 closed form, layer-0 v_norm fixture, scale invariance
  kv_cache_store              exact copy into row `position`; other rows untouched
  attn_score/softmax/output   fp64 SDPA closed form and torch SDPA (fp64, CPU), invariants (seq=1, equal
                              keys, convex hull, window edges, local == global for seq <= W), brute force
                              at head_dim 4
  argmax / logit_softcap      brute force of the stated tie rule; tanh closed form
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libwgsl_ref.so"
WG = 256


class NormRopeP(C.Structure):
    _fields_ = [("num_heads", C.c_uint32), ("head_dim", C.c_uint32), ("eps", C.c_float),
                ("position", C.c_uint32), ("theta", C.c_float), ("apply_divisor", C.c_uint32)]


class NormP(C.Structure):
    _fields_ = [("num_heads", C.c_uint32), ("head_dim", C.c_uint32), ("eps", C.c_float), ("pad", C.c_uint32)]


class KvStoreP(C.Structure):
    _fields_ = [("num_kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("position", C.c_uint32),
                ("max_seq_len", C.c_uint32)]


class AttnScoreP(C.Structure):
    _fields_ = [("num_q_heads", C.c_uint32), ("num_kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("seq_len", C.c_uint32), ("scale", C.c_float), ("sliding_window", C.c_uint32)]


class SoftmaxP(C.Structure):
    _fields_ = [("num_heads", C.c_uint32), ("seq_len", C.c_uint32)]


class AttnOutputP(C.Structure):
    _fields_ = [("num_q_heads", C.c_uint32), ("num_kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("seq_len", C.c_uint32)]


_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = C.CDLL(str(LIB_PATH))
        _lib.wr_f16_to_f32.restype = C.c_float
        _lib.wr_f16_to_f32.argtypes = [C.c_uint16]
        _lib.wr_f32_to_f16.restype = C.c_uint16
        _lib.wr_f32_to_f16.argtypes = [C.c_float]
        _lib.wr_argmax.restype = C.c_uint32
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).copy()


def _u16(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint16)


def set_threads(n: int) -> None:
    lib().wr_set_num_threads(C.c_int(n))


def max_threads() -> int:
    return int(lib().wr_get_max_threads())


# ---- conversions -------------------------------------------------------------

def f32_to_f16_bits(x) -> np.ndarray:
    x = _f32(x).ravel()
    out = np.empty(x.size, dtype=np.uint16)
    lib().wr_f32_to_f16_array(_p(x), _p(out), C.c_uint64(x.size))
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    h = _u16(h).ravel()
    out = np.empty(h.size, dtype=np.float32)
    lib().wr_f16_to_f32_array(_p(h), _p(out), C.c_uint64(h.size))
    return out


# ---- the six WGSL kernels ----------------------------------------------------

def rope_inv_freq(theta, head_dim, apply_divisor, rope_freqs_bits=None) -> np.ndarray:
    """fused_per_head_norm_rope.wgsl:50-54 for i < head_dim/2: the angle's position-independent factor."""
    rf = _u16(rope_freqs_bits if rope_freqs_bits is not None else np.zeros(max(head_dim // 2, 1), np.uint16))
    out = np.empty(head_dim // 2, dtype=np.float32)
    lib().wr_rope_inv_freq(C.c_float(theta), C.c_uint32(head_dim), C.c_uint32(apply_divisor), _p(rf), _p(out))
    return out


def fused_per_head_norm_rope(data, weight_bits, rope_freqs_bits, num_heads, head_dim, eps, position, theta,
                             apply_divisor, num_workgroups=None):
    d = _f32(data)
    w = _u16(weight_bits)
    rf = _u16(rope_freqs_bits if rope_freqs_bits is not None else np.zeros(max(head_dim // 2, 1), np.uint16))
    p = NormRopeP(num_heads, head_dim, eps, position, theta, apply_divisor)
    lib().wr_fused_per_head_norm_rope(_p(d), _p(w), C.byref(p), _p(rf),
                                      C.c_uint32(num_heads if num_workgroups is None else num_workgroups))
    return d


def per_head_rms_norm_no_weight(data, num_heads, head_dim, eps, num_workgroups=None):
    d = _f32(data)
    p = NormP(num_heads, head_dim, eps, 0)
    lib().wr_per_head_rms_norm_no_weight(_p(d), C.byref(p),
                                         C.c_uint32(num_heads if num_workgroups is None else num_workgroups))
    return d


def kv_cache_store(k_in, v_in, k_cache, v_cache, num_kv_heads, head_dim, position, max_seq_len):
    """f32 caches, as kv_cache_store.wgsl binds them. Returns updated copies."""
    k, v = _f32(k_in), _f32(v_in)
    kc, vc = _f32(k_cache), _f32(v_cache)
    p = KvStoreP(num_kv_heads, head_dim, position, max_seq_len)
    nwg = (num_kv_heads * head_dim + WG - 1) // WG
    lib().wr_kv_cache_store(_p(k), _p(v), _p(kc), _p(vc), C.byref(p), C.c_uint32(nwg))
    return kc, vc


def attn_score(q, k_cache, num_q_heads, num_kv_heads, head_dim, seq_len, scale, sliding_window):
    q, kc = _f32(q), np.ascontiguousarray(k_cache, dtype=np.float32)
    scores = np.zeros(num_q_heads * seq_len, dtype=np.float32)
    p = AttnScoreP(num_q_heads, num_kv_heads, head_dim, seq_len, scale, sliding_window)
    nwg = (num_q_heads * seq_len + WG - 1) // WG
    lib().wr_attn_score(_p(q), _p(kc), _p(scores), C.byref(p), C.c_uint32(nwg))
    return scores


def softmax(scores, num_heads, seq_len):
    s = _f32(scores)
    p = SoftmaxP(num_heads, seq_len)
    lib().wr_softmax(_p(s), C.byref(p), C.c_uint32(num_heads))
    return s


def attn_output(probs, v_cache, num_q_heads, num_kv_heads, head_dim, seq_len):
    pr, vc = _f32(probs), np.ascontiguousarray(v_cache, dtype=np.float32)
    out = np.zeros(num_q_heads * head_dim, dtype=np.float32)
    p = AttnOutputP(num_q_heads, num_kv_heads, head_dim, seq_len)
    nwg = (num_q_heads * head_dim + WG - 1) // WG
    lib().wr_attn_output(_p(pr), _p(vc), _p(out), C.byref(p), C.c_uint32(nwg))
    return out


def attention_chain(q, k_cache, v_cache, num_q_heads, num_kv_heads, head_dim, seq_len, scale=1.0,
                    sliding_window=0):
    """attnScore -> softmax -> attnOutput on f32 caches; returns attnOut [NQH*HD]."""
    s = attn_score(q, k_cache, num_q_heads, num_kv_heads, head_dim, seq_len, scale, sliding_window)
    pr = softmax(s, num_q_heads, seq_len)
    return attn_output(pr, v_cache, num_q_heads, num_kv_heads, head_dim, seq_len)


def matmul_quant(x, weight_bits, M, N):
    """matmul_quant.wgsl over f16 weight bits [M][N] and f32 input [N]; returns f32 [M]."""
    x = _f32(x)
    w = _u16(weight_bits)
    assert x.size >= N and w.size >= M * N
    out = np.empty(M, dtype=np.float32)
    lib().wr_matmul_quant(_p(x), _p(w), _p(out), C.c_uint32(M), C.c_uint32(N))
    return out


def matmul_q8(x, qweight, qscale_bits, M, N):
    """matmul_q8.wgsl: int8 weights [M][N] (numpy int8 or their bytes), f16 scale bits [M][N/32], f32 input [N]."""
    assert N % 32 == 0
    x = _f32(x)
    q = np.ascontiguousarray(qweight).view(np.int8).ravel()
    s = _u16(qscale_bits).ravel()
    assert x.size >= N and q.size >= M * N and s.size >= M * (N // 32)
    out = np.empty(M, dtype=np.float32)
    lib().wr_matmul_q8(_p(x), _p(q), _p(s), _p(out), C.c_uint32(M), C.c_uint32(N))
    return out


def matmul_q4k(x, qweight_words, qmeta_bits, M, N):
    """matmul_q4k.wgsl: 4-bit weights packed 8 per u32 [M*N/8], f16 meta [M][N/256][16] (8 scales, 8 mins)."""
    assert N % 256 == 0
    x = _f32(x)
    q = np.ascontiguousarray(qweight_words, dtype=np.uint32).ravel()
    s = _u16(qmeta_bits).ravel()
    assert x.size >= N and q.size >= M * N // 8 and s.size >= M * (N // 256) * 16
    out = np.empty(M, dtype=np.float32)
    lib().wr_matmul_q4k(_p(x), _p(q), _p(s), _p(out), C.c_uint32(M), C.c_uint32(N))
    return out


def logit_softcap(logits, cap):
    x = _f32(logits)
    lib().wr_logit_softcap(_p(x), C.c_uint32(x.size), C.c_float(cap))
    return x


def argmax(logits) -> int:
    x = _f32(logits)
    return int(lib().wr_argmax(_p(x), C.c_uint32(x.size)))
