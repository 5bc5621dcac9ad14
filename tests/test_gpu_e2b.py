"""One decode token of the real Gemma-4-E2B attention stack through the one-launch step, checked
against the oracle: 35 layers with head_dim 256 on local layers and 512 on the seven global ones,
KV sharing by the reference's producer map (src/config/gemma4-e2b.ts:159-178; layers 0..14 own
caches, consumers 15..34 read layer 13's cache (local) or layer 14's (global),
src/engine.ts:1518-1522), two launches per token (one per head_dim). A consumer in its producer's
launch recomputes the current row from the producer's raw k/v and k_norm weight (it has no K/V
projection of its own) and does not store it.

Bars: every producer's stored f16 row bit-identical to RNE of the oracle's k/v; every layer's
attnOut within max-abs 2e-3 of the oracle's chain on the same cache bits.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from g4attn import e2b
from helpers import max_abs
from g4attn import ops
from test_gpu_step import NKH, NQH, TOL, Layer, check, run_step

pytestmark = pytest.mark.gpu


def build_stack(dev, seq, seed0):
    cfg = e2b.AttnConfig(num_layers=35)
    pmap = e2b.compute_kv_producer_map(cfg)
    layers = []
    for il in range(35):
        hd = e2b.head_dim(il, cfg)
        args = (dev, seed0 + 1000 * il, seq, e2b.sliding_window(il, cfg), e2b.rope_theta(il, cfg),
                e2b.apply_divisor(il, cfg))
        if pmap[il] == il:
            layers.append(Layer(*args, hd=hd))
        else:
            p = layers[pmap[il]]
            layers.append(Layer(*args, hd=hd, cache=(p.kc, p.vc)))
    return cfg, pmap, layers


def entries_for(layers, pmap, hd, cfg):
    out = []
    for il, L in enumerate(layers):
        if e2b.head_dim(il, cfg) != hd:
            continue
        if pmap[il] == il:
            out.append(L.entry(inv_freq=True))
        else:
            p = layers[pmap[il]]
            e = L.entry(store=False, raw_kv=(p.d["k"], p.d["v"]), inv_freq=True)
            e["k_weight"] = p.dkw  # the producer's k_norm: the row is the producer's
            out.append(e)
    return out


@pytest.mark.timeout(900)
@pytest.mark.parametrize("seq", [2049, 8193, 32769])
def test_e2b_token_two_launches(dev, seq):
    announce(f"E2B stack one token seq={seq}: hd256 launch + hd512 launch")
    cfg, pmap, layers = build_stack(dev, seq, 40000 + seq)
    for hd in (256, 512):
        run_step(dev, entries_for(layers, pmap, hd, cfg), hd=hd)
    worst = 0.0
    for il, L in enumerate(layers):
        if pmap[il] == il:
            want, kb, vb = L.expected()
            worst = max(worst, check(L, want, kb, vb, f"producer layer {il}"))
        else:
            want, _, _ = L.expected(kv_from=layers[pmap[il]])
            got = L.out.cpu().numpy()
            assert np.isfinite(got).all(), f"consumer layer {il}: non-finite output"
            err = max_abs(got, want)
            assert err <= TOL, f"consumer layer {il}: max-abs {err}"
            worst = max(worst, err)
    print(f"E2B stack seq={seq}: 35 layers checked, worst err {worst:.2e}", flush=True)


@pytest.mark.timeout(900)
@pytest.mark.parametrize("seq", [2049, 32769])
def test_e2b_token_one_pair_launch(dev, seq):
    """The same token with both head_dims' attention passes in one launch and both merges in one
    (g4_attn_step_run_pair): every layer against the oracle as above, three replays with the same bits, and
    the same bits through the two plans' own merge launches."""
    announce(f"E2B stack one token seq={seq}: both head_dims in one launch")
    cfg, pmap, layers = build_stack(dev, seq, 41000 + seq)
    plans = {}
    for hd in (256, 512):
        ents = entries_for(layers, pmap, hd, cfg)
        arr = ops.make_step_entries(ents, NQH, NKH, hd)
        ws = torch.empty(ops.step_workspace_bytes(len(ents), NQH, NKH, hd), dtype=torch.uint8, device=dev)
        plans[hd] = (arr, ws, ops.attn_step_prepare(arr, NQH, NKH, hd, ws))
    outs = []
    for rep in range(3):
        for L in layers:
            L.out.fill_(float("nan"))
        ops.attn_step_run_pair(plans[512][2], plans[256][2])
        torch.cuda.synchronize()
        outs.append(np.concatenate([L.out.cpu().numpy() for L in layers]).view(np.uint32))
    np.testing.assert_array_equal(outs[0], outs[1])
    np.testing.assert_array_equal(outs[0], outs[2])
    # the one merge launch gives the bits of the two plans' own merges
    for L in layers:
        L.out.fill_(float("nan"))
    ops.attn_step_run_attention_pair(plans[512][2], plans[256][2])
    ops.attn_step_run_merge(plans[512][2])
    ops.attn_step_run_merge(plans[256][2])
    torch.cuda.synchronize()
    np.testing.assert_array_equal(np.concatenate([L.out.cpu().numpy() for L in layers]).view(np.uint32), outs[0])
    worst = 0.0
    for il, L in enumerate(layers):
        if pmap[il] == il:
            want, kb, vb = L.expected()
            worst = max(worst, check(L, want, kb, vb, f"producer layer {il}"))
        else:
            want, _, _ = L.expected(kv_from=layers[pmap[il]])
            got = L.out.cpu().numpy()
            assert np.isfinite(got).all(), f"consumer layer {il}: non-finite output"
            err = max_abs(got, want)
            assert err <= TOL, f"consumer layer {il}: max-abs {err}"
            worst = max(worst, err)
    print(f"E2B stack seq={seq} (one launch): 35 layers checked, worst err {worst:.2e}", flush=True)


def test_e2b_step_pair_refuses_bad_plans(dev):
    """Two plans of one head_dim, or one plan twice, are refused before anything is enqueued."""
    cfg, pmap, layers = build_stack(dev, 600, 42000)
    ents = entries_for(layers, pmap, 256, cfg)
    arr = ops.make_step_entries(ents, NQH, NKH, 256)
    ws = torch.empty(ops.step_workspace_bytes(len(ents), NQH, NKH, 256), dtype=torch.uint8, device=dev)
    p256 = ops.attn_step_prepare(arr, NQH, NKH, 256, ws)
    with pytest.raises(RuntimeError, match="head_dim 512 and one of 256"):
        ops.attn_step_run_pair(p256, p256)


def test_e2b_token_engine_order(dev):
    """The engine's layer order: one step per layer; consumers (k, v, k_weight NULL) read the row their
    producer's step stored."""
    seq = 4097
    announce(f"E2B stack engine order seq={seq}: 35 launches")
    cfg, pmap, layers = build_stack(dev, seq, 90000)
    for il, L in enumerate(layers):
        hd = e2b.head_dim(il, cfg)
        if pmap[il] == il:
            run_step(dev, [L.entry(inv_freq=True)], hd=hd)
        else:
            e = L.entry(store=False, inv_freq=True)
            e["k"] = e["v"] = e["k_weight"] = None
            run_step(dev, [e], hd=hd)
    for il, L in enumerate(layers):
        if pmap[il] == il:
            want, kb, vb = L.expected()
            check(L, want, kb, vb, f"producer layer {il}")
        else:
            want, _, _ = L.expected(kv_from=layers[pmap[il]])
            got = L.out.cpu().numpy()
            assert np.isfinite(got).all() and max_abs(got, want) <= TOL, f"consumer layer {il}"
