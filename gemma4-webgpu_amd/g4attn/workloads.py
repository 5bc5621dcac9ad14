"""Workload builders shared by bench.py and the full-size parity tests, so that a test
checks exactly the plan the benchmark times.

prefill4k   causal prefill of a 4096-token prompt: one global layer and one 512-window
            local layer, each as eight 512-token chunks, 16 entries in one launch; the
            f16 query and K/V rows come from raw N(0,1) projections through the
            chunked prompt prep (q/k RMSNorm + RoPE, v-norm, K/V store, and the V rows
            as V^T blocks beside the cache, which the prefill reads V from).
ragged64    64 sequences, lengths uniform in [1024, 32768] (seeded).
"""
from __future__ import annotations

from . import synth

BASE_SEED = 20261201
EPS = 1e-6

PREFILL_T, PREFILL_CHUNK, PREFILL_WINDOWS = 4096, 512, (0, 512)


def ragged64_lengths():
    return [int(x) for x in synth.ragged_lengths(BASE_SEED + 2, 64, 1024, 32768)]


def prefill4k(dev, nqh=8, nkh=1, hd=256, T=PREFILL_T, chunk=PREFILL_CHUNK, windows=PREFILL_WINDOWS, vt=True):
    """A prompt's attention for one global and one local layer, from raw projections.

    Per layer: raw f32 q/k/v projections N(0,1) (one row of each head per token), norm weights 1.0 and
    the engine's rope_freqs table; the chunked prompt prep (q/k RMSNorm + RoPE at every position, v
    weightless norm, f16 K/V rows stored) fills the f16 query and the caches. Returns the per-layer
    device tensors (q f16, k_cache, v_cache, out, window), the prefill entries (every chunk of every
    layer, layer order then chunk order) and `prep()`, which re-runs the two layers' preps (one launch).
    vt: the prep also writes V^T blocks beside each cache and the entries read V from them (False: the
    prefill transposes the attended rows itself at every call)."""
    import numpy as np
    import torch

    from . import e2b, ops

    rf_bits = np.array(e2b.rope_freqs_f16_bits(256), dtype=np.uint16)
    rf = torch.from_numpy(rf_bits.view(np.int16)).to(dev)
    ones = torch.full((hd,), 0x3C00, dtype=torch.int16, device=dev)
    layers, entries, preps = [], [], []
    for li, w in enumerate(windows):
        qr = synth.normal_torch(BASE_SEED + 30 + li, T * nqh * hd, dev)
        kr = synth.normal_torch(BASE_SEED + 40 + li, T * nkh * hd, dev)
        vr = synth.normal_torch(BASE_SEED + 50 + li, T * nkh * hd, dev)
        q = torch.empty(T * nqh * hd, dtype=torch.int16, device=dev)
        kc = torch.empty(T * nkh * hd, dtype=torch.int16, device=dev)
        vc = torch.empty_like(kc)
        vtc = torch.empty(ops.vt_cache_elems(T, nkh, hd), dtype=torch.int16, device=dev) if vt else None
        out = torch.empty(T * nqh * hd, dtype=torch.float32, device=dev)
        theta, div = (1e4, 0) if w else (1e6, 1)
        inv = ops.rope_inv_freq(theta, hd, div, rf)  # the layer's inverse frequencies, once (as at load)
        preps.append(dict(q=qr, q_weight=ones, q_out=q, n_tokens=T, start=0, num_q_heads=nqh, num_kv_heads=nkh,
                          head_dim=hd, theta=theta, apply_divisor=div, rope_freqs=rf, k=kr, v=vr, k_weight=ones,
                          k_cache=kc, v_cache=vc, max_seq_len=T, eps=EPS, rope_inv_freq=inv, vt_cache=vtc))
        layers.append((q, kc, vc, out, w))
        for c0 in range(0, T, chunk):
            entries.append(dict(q=q[c0 * nqh * hd:], k_cache=kc, v_cache=vc, out=out[c0 * nqh * hd:],
                                n_tokens=min(chunk, T - c0), start=c0, sliding_window=w, scale=1.0,
                                vt_cache=vtc, vt_rows=T))

    def prep():  # both layers' chunks in one launch
        ops.attn_prompt_prep_many(preps)

    prep()
    return layers, entries, prep


def prefill_flops(nqh=8, hd=256, T=PREFILL_T, windows=PREFILL_WINDOWS) -> float:
    """Algorithmic flops: 4 * hd * nqh per attended (token, key) pair."""
    f = 0.0
    for w in windows:
        for i in range(T):
            f += 4.0 * hd * nqh * (min(i + 1, w) if w else i + 1)
    return f
