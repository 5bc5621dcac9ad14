"""Input builders shared by the tests (seeded, same stream on host and device)."""
from __future__ import annotations

import numpy as np

from g4attn import synth
from oracle import oracle as orc

EPS = 1e-6


def f16_weight_bits(seed: int, n: int, spread: float = 0.1) -> np.ndarray:
    """A q/k_norm weight near 1, f16 bits (the reference binds norm weights as f16)."""
    w = 1.0 + spread * synth.normal(seed, n)
    return orc.f32_to_f16_bits(w)


def unit_rms_rows_f16(seed: int, rows: int, width: int) -> np.ndarray:
    """rows x width N(0,1), each row RMS-normalised, as f16 bits."""
    x = synth.normal(seed, rows * width).reshape(rows, width)
    return orc.f32_to_f16_bits(synth.rms_normalize_rows(x, EPS)).reshape(rows, width)


def cache_f16(seed: int, rows: int, nkh: int, hd: int) -> np.ndarray:
    """[rows, nkh, hd] unit-RMS per head, f16 bits."""
    return unit_rms_rows_f16(seed, rows * nkh, hd).reshape(rows, nkh, hd)


def cache_f16_torch(seed: int, rows: int, nkh: int, hd: int, device):
    """Device-side version of cache_f16 for large caches: the same normal stream; the
    row normalisation may differ from the host version in the last bit of a few rows."""
    import torch

    x = synth.normal_torch(seed, rows * nkh * hd, device).view(rows * nkh, hd)
    ms = (x.double() ** 2).mean(dim=1, keepdim=True)
    y = (x.double() / torch.sqrt(ms + EPS)).float().to(torch.float16)
    return y.view(rows, nkh, hd)


def unit_q(seed: int, nqh: int, hd: int) -> np.ndarray:
    """Post-norm query stand-in: unit RMS per head, f32."""
    return synth.rms_normalize_rows(synth.normal(seed, nqh * hd).reshape(nqh, hd), EPS).ravel()


def max_abs(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))
