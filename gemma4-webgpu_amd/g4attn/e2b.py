"""Gemma-4-E2B attention shape parameters.

Restates the attention fields of the reference's E2B config and its helpers:
src/config/gemma4-e2b.ts:16-63 (defaults), :151-178 (KV producer map) and
src/types.ts:139-162 (isSwaLayer / getRopeTheta / getHeadDim /
isKvProducerLayer). `head_dim_global` is 512 in the real model; the benchmark
workloads use 256 on every layer.
"""
from __future__ import annotations

from dataclasses import dataclass, field

GLOBAL_LAYERS = (4, 9, 14, 19, 24, 29, 34)


@dataclass
class AttnConfig:
    num_layers: int = 35
    num_q_heads: int = 8
    num_kv_heads: int = 1
    head_dim_local: int = 256
    head_dim_global: int = 512
    rms_norm_eps: float = 1e-6
    rope_theta_global: float = 1_000_000.0
    rope_theta_swa: float = 10_000.0
    sliding_window: int = 512
    num_unshared_layers: int = 15
    context_length: int = 2048
    attention_is_sliding: list = field(default_factory=list)
    kv_producer_for_layer: list = field(default_factory=list)

    def __post_init__(self):
        if not self.attention_is_sliding:
            self.attention_is_sliding = [i not in GLOBAL_LAYERS for i in range(self.num_layers)]
        if not self.kv_producer_for_layer:
            self.kv_producer_for_layer = compute_kv_producer_map(self)


def compute_kv_producer_map(c: AttnConfig) -> list:
    """Consumer layers share the cache of the last unshared layer of the same type
    (src/config/gemma4-e2b.ts:159-178)."""
    last_local = last_global = -1
    for i in range(c.num_unshared_layers):
        if c.attention_is_sliding[i]:
            last_local = i
        else:
            last_global = i
    out = []
    for i in range(c.num_layers):
        if i < c.num_unshared_layers:
            out.append(i)
        else:
            out.append(last_local if c.attention_is_sliding[i] else last_global)
    return out


def is_swa_layer(il: int, c: AttnConfig) -> bool:
    return bool(c.attention_is_sliding[il])


def rope_theta(il: int, c: AttnConfig) -> float:
    return c.rope_theta_swa if is_swa_layer(il, c) else c.rope_theta_global


def head_dim(il: int, c: AttnConfig) -> int:
    return c.head_dim_local if is_swa_layer(il, c) else c.head_dim_global


def is_kv_producer(il: int, c: AttnConfig) -> bool:
    return c.kv_producer_for_layer[il] == il


def sliding_window(il: int, c: AttnConfig) -> int:
    """attnScore Params.sliding_window: W on local layers, 0 on global (src/engine.ts:554)."""
    return c.sliding_window if is_swa_layer(il, c) else 0


def apply_divisor(il: int, c: AttnConfig) -> int:
    """fusedNormRope Params.apply_divisor: 1 on global layers (src/engine.ts:571-576)."""
    return 0 if is_swa_layer(il, c) else 1


def rope_freqs_f16_bits(n: int = 256) -> list:
    """The rope_freqs table as the engine binds it: 1.0 for entries 0..63, 1e30 saturated
    to f16 +Inf for 64..255 (fused_per_head_norm_rope.wgsl:4-11)."""
    return [0x3C00 if i < 64 else 0x7C00 for i in range(n)]
