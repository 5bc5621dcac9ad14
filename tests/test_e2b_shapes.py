"""Gemma-4-E2B attention-shape helpers (g4attn/e2b.py) pinned on the CPU.

g4attn/e2b.py restates src/config/gemma4-e2b.ts:16-63 (layer classes, head dims, thetas,
window) and :159-178 (computeKvProducerMap), and src/types.ts:139-162 (isSwaLayer,
getRopeTheta, getHeadDim, isKvProducerLayer). Two independent pins:

* a known answer written out from the reference file: global layers {4, 9, ..., 34};
  layers 0..14 produce their own K/V; consumers 15..34 read layer 14's cache (global) or
  layer 13's (local);
* transformers' Gemma-4 text attention (a library routine, not derived from the reference):
  for a 35-layer config with 20 KV-shared layers and the reference's layer classes it marks
  which layers share and which layer stores the shared K/V of each class, and gives head_dim,
  window, scale and the RoPE parameters per layer class.
"""
import numpy as np
import pytest

from g4attn import e2b

REF_GLOBAL = (4, 9, 14, 19, 24, 29, 34)  # src/config/gemma4-e2b.ts:21


def test_layer_classes_known_answer():
    c = e2b.AttnConfig()
    assert c.num_layers == 35 and c.num_unshared_layers == 15
    assert [il for il in range(35) if not e2b.is_swa_layer(il, c)] == list(REF_GLOBAL)
    for il in range(35):
        g = il in REF_GLOBAL
        assert e2b.head_dim(il, c) == (512 if g else 256)
        assert e2b.rope_theta(il, c) == (1e6 if g else 1e4)
        assert e2b.sliding_window(il, c) == (0 if g else 512)
        assert e2b.apply_divisor(il, c) == (1 if g else 0)


def test_producer_map_known_answer():
    c = e2b.AttnConfig()
    want = list(range(15)) + [14 if il in REF_GLOBAL else 13 for il in range(15, 35)]
    assert e2b.compute_kv_producer_map(c) == want
    assert c.kv_producer_for_layer == want
    assert [il for il in range(35) if e2b.is_kv_producer(il, c)] == list(range(15))


def test_producer_map_other_splits():
    """The rule for other unshared counts: the last unshared layer of the same class."""
    c = e2b.AttnConfig(num_unshared_layers=10)
    m = e2b.compute_kv_producer_map(c)
    assert m[:10] == list(range(10))
    assert all(m[il] == (9 if il in REF_GLOBAL else 8) for il in range(10, 35))
    c = e2b.AttnConfig(num_unshared_layers=35)
    assert e2b.compute_kv_producer_map(c) == list(range(35))


def _hf_layers(num_layers=35, shared=20):
    from transformers.models.gemma4.configuration_gemma4 import Gemma4TextConfig
    from transformers.models.gemma4.modeling_gemma4 import Gemma4TextAttention

    types = ["full_attention" if il in REF_GLOBAL else "sliding_attention" for il in range(num_layers)]
    cfg = Gemma4TextConfig(num_hidden_layers=num_layers, num_kv_shared_layers=shared, layer_types=types,
                           hidden_size=16, num_attention_heads=8, num_key_value_heads=1, intermediate_size=32,
                           vocab_size=64, vocab_size_per_layer_input=64)
    return cfg, [Gemma4TextAttention(cfg, il) for il in range(num_layers)]


@pytest.mark.parametrize("shared", [20, 25])
def test_producer_map_matches_transformers(shared):
    cfg, att = _hf_layers(shared=shared)
    stores = {a.layer_type: il for il, a in enumerate(att) if a.store_full_length_kv}
    hf_map = [stores[a.layer_type] if a.is_kv_shared_layer else il for il, a in enumerate(att)]
    c = e2b.AttnConfig(num_unshared_layers=35 - shared)
    assert e2b.compute_kv_producer_map(c) == hf_map


def test_per_layer_shapes_match_transformers():
    cfg, att = _hf_layers()
    c = e2b.AttnConfig()
    for il, a in enumerate(att):
        assert a.head_dim == e2b.head_dim(il, c)
        assert (a.sliding_window or 0) == e2b.sliding_window(il, c)
        assert a.scaling == 1.0
        rp = cfg.rope_parameters[a.layer_type]
        assert rp["rope_theta"] == e2b.rope_theta(il, c)
        assert (rp["rope_type"] == "proportional") == bool(e2b.apply_divisor(il, c))


def test_global_rope_table_matches_proportional_rope(oracle):
    """The engine's rope_freqs divisor table on a head_dim-512 global layer gives transformers'
    proportional RoPE (partial_rotary_factor 0.25): 64 rotated pairs at theta^(-2i/512), the
    other 192 pairs unrotated (inverse frequency 0)."""
    import torch

    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS

    cfg, _ = _hf_layers()
    inv_hf, _ = ROPE_INIT_FUNCTIONS["proportional"](cfg, torch.device("cpu"), layer_type="full_attention")
    inv_hf = inv_hf.numpy().astype(np.float64)
    rf = np.array(e2b.rope_freqs_f16_bits(256), np.uint16)
    got = oracle.rope_inv_freq(1e6, 512, 1, rf).astype(np.float64)
    assert got.shape == inv_hf.shape == (256,)
    np.testing.assert_array_equal(got[64:], 0.0)
    np.testing.assert_array_equal(inv_hf[64:], 0.0)
    np.testing.assert_allclose(got[:64], inv_hf[:64], rtol=3e-7)
