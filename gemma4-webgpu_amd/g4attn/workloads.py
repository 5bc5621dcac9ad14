"""Workload builders shared by bench.py and the full-size parity tests, so that a test
checks exactly the plan the benchmark times.

prefill4k   causal prefill of a 4096-token prompt: one global layer and one 512-window
            local layer, each as eight 512-token chunks, 16 entries in one launch; f16
            Q/K/V drawn N(0,1) then RMS-normalised per row (q stands for the post norm +
            RoPE query).
ragged64    64 sequences, lengths uniform in [1024, 32768] (seeded).
"""
from __future__ import annotations

from . import synth

BASE_SEED = 20261201
EPS = 1e-6

PREFILL_T, PREFILL_CHUNK, PREFILL_WINDOWS = 4096, 512, (0, 512)


def ragged64_lengths():
    return [int(x) for x in synth.ragged_lengths(BASE_SEED + 2, 64, 1024, 32768)]


def unit_rows_f16(seed: int, rows: int, width: int, dev):
    """rows x width N(0,1) from stream `seed`, each row RMS-normalised, as f16 on `dev` (flat)."""
    import torch

    x = synth.normal_torch(seed, rows * width, dev).view(rows, width).double()
    return (x / torch.sqrt((x ** 2).mean(dim=1, keepdim=True) + EPS)).to(torch.float16).view(-1)


def prefill4k(dev, nqh=8, nkh=1, hd=256, T=PREFILL_T, chunk=PREFILL_CHUNK, windows=PREFILL_WINDOWS):
    """Per layer (q, k_cache, v_cache, out, window) device tensors, and the prefill entries: every
    chunk of every layer, in layer order then chunk order."""
    import torch

    layers, entries = [], []
    for li, w in enumerate(windows):
        q = unit_rows_f16(BASE_SEED + 30 + li, T * nqh, hd, dev).view(torch.int16)
        kc = unit_rows_f16(BASE_SEED + 40 + li, T * nkh, hd, dev).view(torch.int16)
        vc = unit_rows_f16(BASE_SEED + 50 + li, T * nkh, hd, dev).view(torch.int16)
        out = torch.empty(T * nqh * hd, dtype=torch.float32, device=dev)
        layers.append((q, kc, vc, out, w))
        for c0 in range(0, T, chunk):
            entries.append(dict(q=q[c0 * nqh * hd:], k_cache=kc, v_cache=vc, out=out[c0 * nqh * hd:],
                                n_tokens=min(chunk, T - c0), start=c0, sliding_window=w, scale=1.0))
    return layers, entries


def prefill_flops(nqh=8, hd=256, T=PREFILL_T, windows=PREFILL_WINDOWS) -> float:
    """Algorithmic flops: 4 * hd * nqh per attended (token, key) pair."""
    f = 0.0
    for w in windows:
        for i in range(T):
            f += 4.0 * hd * nqh * (min(i + 1, w) if w else i + 1)
    return f
