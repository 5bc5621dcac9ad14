"""Seeded synthetic inputs: splitmix64 -> Box-Muller N(0,1), f32.

The same stream is produced by the numpy path (host) and the torch path
(device-side generation for large caches); `normal(seed, n)` element i is
identical in both. Seeds follow `20261201 + config index`.

splitmix64 (Steele, Lea, Flood 2014, "Fast splittable pseudorandom number
generators"): state_i = seed + i * 0x9E3779B97F4A7C15 (i >= 1), mixed by
xor-shift-multiply with the published constants. Uniforms take the top 53
bits. Box-Muller pairs (u1, u2) -> sqrt(-2 ln u1) * (cos 2 pi u2, sin 2 pi u2),
with u1 in (0, 1].
"""
from __future__ import annotations

import numpy as np

GAMMA = 0x9E3779B97F4A7C15
M1 = 0xBF58476D1CE4E5B9
M2 = 0x94D049BB133111EB
BASE_SEED = 20261201


def _mix_np(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * np.uint64(M1)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(M2)
    return z ^ (z >> np.uint64(31))


def splitmix64(seed: int, n: int, start: int = 0) -> np.ndarray:
    idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed % (1 << 64)) + idx * np.uint64(GAMMA)
        return _mix_np(z)


def normal(seed: int, n: int) -> np.ndarray:
    """n standard normals (float32) from stream `seed`."""
    m = (n + 1) // 2
    u = splitmix64(seed, 2 * m)
    u1 = ((u[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0**-53
    u2 = (u[1::2] >> np.uint64(11)).astype(np.float64) * 2.0**-53
    r = np.sqrt(-2.0 * np.log(u1))
    th = 2.0 * np.pi * u2
    out = np.empty(2 * m, dtype=np.float64)
    out[0::2] = r * np.cos(th)
    out[1::2] = r * np.sin(th)
    return out[:n].astype(np.float32)


def uniform_u64(seed: int, n: int) -> np.ndarray:
    return splitmix64(seed, n)


def normal_torch(seed: int, n: int, device, chunk: int = 1 << 26):
    """Same stream as `normal`, generated with torch int64 arithmetic on `device`."""
    import torch

    def to_i64(x: int) -> int:
        x %= 1 << 64
        return x - (1 << 64) if x >= 1 << 63 else x

    def lsr(z, k):  # logical shift right on int64 bit patterns
        return (z >> k) & ((1 << (64 - k)) - 1)

    m = (n + 1) // 2
    out = torch.empty(2 * m, dtype=torch.float32, device=device)
    seed_i, gamma_i, m1, m2 = to_i64(seed), to_i64(GAMMA), to_i64(M1), to_i64(M2)
    for p0 in range(0, m, chunk):
        p1 = min(m, p0 + chunk)
        pairs = torch.arange(p0, p1, dtype=torch.int64, device=device)
        res = []
        for off in (1, 2):  # element indices 2p+1 (u1) and 2p+2 (u2), 1-based
            z = (2 * pairs + off) * gamma_i + seed_i
            z = (z ^ lsr(z, 30)) * m1
            z = (z ^ lsr(z, 27)) * m2
            z = z ^ lsr(z, 31)
            res.append(lsr(z, 11).to(torch.float64))
        u1 = (res[0] + 1.0) * 2.0**-53
        u2 = res[1] * 2.0**-53
        r = torch.sqrt(-2.0 * torch.log(u1))
        th = 2.0 * torch.pi * u2
        out[2 * p0:2 * p1:2] = (r * torch.cos(th)).to(torch.float32)
        out[2 * p0 + 1:2 * p1:2] = (r * torch.sin(th)).to(torch.float32)
    return out[:n]


def rms_normalize_rows(x: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """Row-wise x / sqrt(mean(x^2) + eps) in f32 (unit-RMS cache rows)."""
    x = np.asarray(x, dtype=np.float32)
    ms = np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True)
    return (x / np.sqrt(ms + eps)).astype(np.float32)


def ragged_lengths(seed: int, batch: int, lo: int, hi: int) -> np.ndarray:
    """Lengths uniform in [lo, hi] inclusive: lo + floor(u * (hi - lo + 1)), u from the top 53 bits."""
    u = (splitmix64(seed, batch) >> np.uint64(11)).astype(np.float64) * 2.0**-53
    return (lo + np.floor(u * (hi - lo + 1))).astype(np.int64)
