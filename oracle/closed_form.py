"""fp64 closed forms — TEST INFRASTRUCTURE ONLY.

Independent textbook statements of the attention-path math, used to pin the
oracle (oracle/wgsl_ref.c). They share no code with it: plain numpy in
float64.

  rms_norm:  y = x * w / sqrt(mean(x^2) + eps), per head (HF Gemma RMSNorm;
             with_scale=False gives w = 1)
  rope:      rotate-half pairs (i, i + HD/2), inv_freq_i = theta^(-2i/HD),
             optionally divided by a per-pair divisor; angle = pos * inv_freq
  sdpa:      softmax(scale * q K^T over the attended rows) V, GQA kv_head =
             h * NKH / NQH, local window = the last W rows
"""
from __future__ import annotations

import numpy as np


def rms_norm(x, w=None, eps=1e-6, head_dim=None):
    x = np.asarray(x, dtype=np.float64)
    hd = head_dim or x.shape[-1]
    xs = x.reshape(-1, hd)
    r = np.sqrt(np.mean(xs * xs, axis=1, keepdims=True) + eps)
    y = xs / r
    if w is not None:
        y = y * np.asarray(w, dtype=np.float64)[None, :]
    return y.reshape(x.shape)


def rope_angles(position, theta, head_dim, divisor=None):
    i = np.arange(head_dim // 2, dtype=np.float64)
    inv = theta ** (-2.0 * i / head_dim)
    if divisor is not None:
        inv = inv / np.asarray(divisor, dtype=np.float64)[: head_dim // 2]
    return position * inv


def rope(x, position, theta, head_dim, divisor=None, angles=None):
    x = np.asarray(x, dtype=np.float64).reshape(-1, head_dim)
    a = rope_angles(position, theta, head_dim, divisor) if angles is None else np.asarray(angles, np.float64)
    c, s = np.cos(a), np.sin(a)
    h = head_dim // 2
    x0, x1 = x[:, :h], x[:, h:]
    return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=1).ravel()


def attended_rows(seq_len, window):
    start = max(0, seq_len - window) if window else 0
    return start, seq_len


def sdpa(q, k_cache, v_cache, num_q_heads, num_kv_heads, head_dim, seq_len, scale=1.0, window=0):
    """q [NQH*HD]; caches [rows, NKH, HD] (any float dtype); returns [NQH*HD] float64."""
    q = np.asarray(q, dtype=np.float64).reshape(num_q_heads, head_dim)
    K = np.asarray(k_cache, dtype=np.float64).reshape(-1, num_kv_heads, head_dim)
    V = np.asarray(v_cache, dtype=np.float64).reshape(-1, num_kv_heads, head_dim)
    b, e = attended_rows(seq_len, window)
    out = np.empty((num_q_heads, head_dim))
    for h in range(num_q_heads):
        kvh = h * num_kv_heads // num_q_heads
        s = scale * (K[b:e, kvh, :] @ q[h])
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ V[b:e, kvh, :]
    return out.ravel()


def softcap(x, cap):
    return np.tanh(np.clip(np.asarray(x, np.float64) / cap, -15.0, 15.0)) * cap


def matvec(weight_f32, x):
    """Textbook f64 matrix-vector product."""
    return np.asarray(weight_f32, dtype=np.float64) @ np.asarray(x, dtype=np.float64)


def bitrev8(r):
    r = int(r)
    return int(f"{r:08b}"[::-1], 2)


def argmax_rule(x):
    """Top-1 index under argmax.wgsl's rule, stated without its loops: the
    maximum M over values above -1e30 (NaN excluded); among indices i with
    x[i] == M the one with the smallest (bit-reversed 8-bit i mod 256, i); 0
    when no value is above -1e30."""
    x = np.asarray(x, dtype=np.float32)
    ok = (x > np.float32(-1e30)) & ~np.isnan(x)
    if not ok.any():
        return 0
    m = x[ok].max()
    cand = np.nonzero(ok & (x == m))[0]
    return int(min(cand, key=lambda i: (bitrev8(i % 256), i)))
