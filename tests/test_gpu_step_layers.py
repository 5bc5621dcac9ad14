"""GPU parity of one token's layers prepared together (g4_attn_step_prepare_layers): a plan per layer
from one prepare and one table upload, each run on its own in layer order, as the engine runs a token
(src/engine.ts:2029-2156, every layer's uniforms patched once per token at :1967-1987).

Bars: every layer's attnOut, stored K/V rows and o_proj rows are bit-identical to the same layer
prepared alone (g4_attn_step_prepare with one entry, the form test_gpu_step and test_gpu_step_out pin
to the oracle), through both run forms (attention + merge launch, attention + o_proj with the merge
folded in) and on a second run of the same plans; attnOut is within max-abs 2e-3 of the oracle's
reference chain. Layers at one position with the same host RoPE table share one set of factors (the
planner's CPU check covers the sharing itself); KV-consumer layers read the row their producer's run
stored earlier in the same token.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from g4attn import abi, ops
from test_gpu_linear import t_u16, weights
from test_gpu_step import ROPE, TOL, Layer

pytestmark = pytest.mark.gpu

H = 1536  # E2B hidden size: o_proj rows


def bits(t):
    return t.cpu().numpy().view(np.uint32)


def host_tables(hd):
    """One host RoPE table per (theta, divisor) kind, shared by the layers of that kind."""
    return {(1e4, 0): ops.rope_inv_freq_host(1e4, hd, 0, ROPE), (1e6, 1): ops.rope_inv_freq_host(1e6, hd, 1, ROPE)}


def build(dev, specs, hd, seed):
    """specs: (seq, window, theta, divisor, producer index or None, host table). Consumers share their
    producer's cache and step after it with k/v/k_weight NULL."""
    layers, entries = [], []
    tabs = host_tables(hd)
    for i, (seq, win, theta, div, prod, host) in enumerate(specs):
        cache = None if prod is None else (layers[prod].kc, layers[prod].vc)
        L = Layer(dev, seed + 13 * i, seq, win, theta, div, cache=cache, hd=hd)
        e = L.entry(store=prod is None)
        if prod is not None:
            e["k"] = e["v"] = e["k_weight"] = None
        if host:
            e["rope_inv_freq_host"] = tabs[(theta, div)]
        layers.append(L)
        entries.append(e)
    return layers, entries, tabs


def run_alone(dev, layers, entries, hd, wo, rows):
    """Reference: each layer prepared alone, in layer order (attention, merge; then o_proj)."""
    outs, ys, krows, vrows = [], [], [], []
    for L, e, w in zip(layers, entries, wo):
        arr = ops.make_step_entries([e], 8, 1, hd)
        ws = torch.empty(ops.step_workspace_bytes(1, 8, 1, hd), dtype=torch.uint8, device=dev)
        plan = ops.attn_step_prepare(arr, 8, 1, hd, ws)
        ops.attn_step_run_attention(plan)
        ops.attn_step_run_merge(plan)
        y = torch.empty(rows, device=dev)
        ops.linear_f16(L.out, 8 * hd, [(w, y, rows)])
        torch.cuda.synchronize()
        outs.append(L.out.clone())
        ys.append(y)
        krows.append(L.kc[L.pos].clone())
        vrows.append(L.vc[L.pos].clone())
    return outs, ys, krows, vrows


CASES = [  # (label, hd, [(seq, window, theta, divisor, producer, host table)])
    ("E2B-like order, head_dim 256", 256,
     [(513, 512, 1e4, 0, None, True), (513, 512, 1e4, 0, None, True), (1200, 0, 1e6, 1, None, True),
      (513, 512, 1e4, 0, None, False), (513, 512, 1e4, 0, 1, True), (1200, 0, 1e6, 1, 2, True),
      (40, 0, 1e4, 0, None, True), (9000, 0, 1e6, 1, None, True)]),
    ("global layers, head_dim 512", 512,
     [(2100, 0, 1e6, 1, None, True), (2100, 0, 1e6, 1, 0, True), (300, 0, 1e6, 1, None, False),
      (2100, 0, 1e6, 1, None, True)]),
]


@pytest.mark.parametrize("label,hd,specs", CASES, ids=[c[0] for c in CASES])
def test_layers_match_layers_prepared_alone(dev, label, hd, specs):
    announce(f"attnStepLayers {label}")
    layers, entries, tabs = build(dev, specs, hd, 5100 + hd)
    n = 8 * hd
    rows = H
    wo = [t_u16(weights(700 + i, rows, n, 0.02), dev) for i in range(len(layers))]
    outs, ys, krows, vrows = run_alone(dev, layers, entries, hd, wo, rows)
    arr = ops.make_step_entries(entries, 8, 1, hd)
    ws = torch.empty(ops.step_layers_workspace_bytes(len(entries), 8, 1, hd), dtype=torch.uint8, device=dev)
    plans = ops.attn_step_prepare_layers(arr, 8, 1, hd, ws)
    for rep in range(2):
        fused = rep == 0
        for L in layers:
            L.out.fill_(float("nan"))
            L.kc[L.pos] = 0
            L.vc[L.pos] = 0
        y = [torch.full((rows,), float("nan"), device=dev) for _ in layers]
        for i, plan in enumerate(plans):  # layer order: a consumer runs after its producer stored the row
            ops.attn_step_run_attention(plan)
            if fused:
                ops.attn_step_run_out(plan, n, [(wo[i], y[i], rows)])
            else:
                ops.attn_step_run_merge(plan)
                ops.linear_f16(layers[i].out, n, [(wo[i], y[i], rows)])
        torch.cuda.synchronize()
        for i, L in enumerate(layers):
            tag = f"layer {i} ({'o_proj with merge' if fused else 'merge launch'})"
            np.testing.assert_array_equal(bits(L.out), bits(outs[i]), err_msg=f"attnOut {tag}")
            np.testing.assert_array_equal(bits(y[i]), bits(ys[i]), err_msg=f"o_proj {tag}")
            np.testing.assert_array_equal(L.kc[L.pos].cpu().numpy(), krows[i].cpu().numpy(), err_msg=f"K row {tag}")
            np.testing.assert_array_equal(L.vc[L.pos].cpu().numpy(), vrows[i].cpu().numpy(), err_msg=f"V row {tag}")
    for i, (L, s) in enumerate(zip(layers, specs)):
        want, kb, vb = L.expected(kv_from=None if s[4] is None else layers[s[4]])
        got = outs[i].cpu().numpy()
        err = float(np.abs(got - want).max())
        assert err <= TOL, f"layer {i}: attnOut max-abs {err} vs the oracle"
        if s[4] is None:
            np.testing.assert_array_equal(L.kc[L.pos].cpu().numpy().view(np.uint16), kb, err_msg=f"layer {i} K")
            np.testing.assert_array_equal(L.vc[L.pos].cpu().numpy().view(np.uint16), vb, err_msg=f"layer {i} V")
    del tabs


def test_layers_workspace_and_errors(dev):
    announce("attnStepLayers argument errors")
    layers, entries, tabs = build(dev, [(513, 512, 1e4, 0, None, True), (100, 0, 1e6, 1, None, True)], 256, 77)
    arr = ops.make_step_entries(entries, 8, 1, 256)
    need = ops.step_layers_workspace_bytes(2, 8, 1, 256)
    assert need == 2 * ops.step_workspace_bytes(1, 8, 1, 256)
    small = torch.empty(need - 256, dtype=torch.uint8, device=dev)
    with pytest.raises(RuntimeError, match="attnStepLayers: workspace"):
        ops.attn_step_prepare_layers(arr, 8, 1, 256, small)
    bad = ops.make_step_entries(entries, 8, 1, 256)
    bad[1].seq_len = 0
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    plans = (abi.DecodePlan * 2)()
    with pytest.raises(RuntimeError, match="layer 1: attnStep: entry 0 seq_len 0"):
        abi.call("g4_attn_step_prepare_layers", bad, 2, 1, 8, 1, 256, ws.data_ptr(), ws.numel(), plans, None)
    for i in range(2):  # no plan of a failed call runs: layer 0's tables were never uploaded
        with pytest.raises(RuntimeError, match="not prepared"):
            ops.attn_step_run_attention(plans[i])
    torch.cuda.synchronize()
    del tabs


def test_batched_layers_match_batches_prepared_alone(dev):
    """Three layers of a batched decode (three sequences of different lengths per layer, as the TS host's
    scheduler steps them), prepared together with entries_per_layer 3: every layer's attnOut and stored rows
    bit-identical to that layer's three entries prepared alone, and within max-abs 2e-3 of the oracle."""
    announce("attnStepLayers 3 layers x 3 sequences")
    lens = [(700, 300, 2500), (700, 300, 2500), (700, 300, 2500)]
    kinds = [(512, 1e4, 0), (0, 1e6, 1), (512, 1e4, 0)]
    tabs = host_tables(256)
    layers, entries = [], []
    for li, ((win, theta, div), seqs) in enumerate(zip(kinds, lens)):
        for si, seq in enumerate(seqs):
            L = Layer(dev, 8300 + 37 * li + si, seq, win, theta, div)
            e = L.entry()
            e["rope_inv_freq_host"] = tabs[(theta, div)]
            layers.append(L)
            entries.append(e)
    ref = []
    for li in range(3):  # each layer's batch prepared alone
        arr = ops.make_step_entries(entries[3 * li:3 * li + 3], 8, 1, 256)
        ws1 = torch.empty(ops.step_workspace_bytes(3, 8, 1, 256), dtype=torch.uint8, device=dev)
        ops.attn_step_run(ops.attn_step_prepare(arr, 8, 1, 256, ws1))
        torch.cuda.synchronize()
        ref += [bits(L.out) for L in layers[3 * li:3 * li + 3]]
    arr = ops.make_step_entries(entries, 8, 1, 256)
    ws = torch.empty(ops.step_layers_workspace_bytes(3, 8, 1, 256, entries_per_layer=3), dtype=torch.uint8,
                     device=dev)
    plans = ops.attn_step_prepare_layers(arr, 8, 1, 256, ws, entries_per_layer=3)
    assert len(plans) == 3
    for L in layers:
        L.out.fill_(float("nan"))
    for plan in plans:
        ops.attn_step_run(plan)
    torch.cuda.synchronize()
    for i, L in enumerate(layers):
        np.testing.assert_array_equal(bits(L.out), ref[i], err_msg=f"entry {i}")
        want, kb, vb = L.expected()
        assert float(np.abs(L.out.cpu().numpy() - want).max()) <= TOL, f"entry {i} vs the oracle"
        np.testing.assert_array_equal(L.kc[L.pos].cpu().numpy().view(np.uint16), kb, err_msg=f"entry {i} K")
    del tabs


def test_e2b_order_two_head_dim_groups(dev):
    """A token in E2B's layer order with both head_dim groups: the local layers (head_dim 256) prepared
    together and the global layers (head_dim 512) prepared together, each group in its own workspace,
    then every layer run in layer order; every attnOut and o_proj row bit-identical to the layer
    prepared alone."""
    announce("attnStepLayers E2B order, head_dim 256 and 512 groups")
    specs = [(700, 512, 1e4, 0, 256), (700, 512, 1e4, 0, 256), (2100, 0, 1e6, 1, 512), (700, 512, 1e4, 0, 256),
             (700, 512, 1e4, 0, 256), (2100, 0, 1e6, 1, 512), (700, 512, 1e4, 0, 256)]
    tabs = {256: host_tables(256), 512: host_tables(512)}
    layers, entries = [], []
    for i, (seq, win, theta, div, hd) in enumerate(specs):
        L = Layer(dev, 9700 + 29 * i, seq, win, theta, div, hd=hd)
        e = L.entry()
        e["rope_inv_freq_host"] = tabs[hd][(theta, div)]
        layers.append(L)
        entries.append(e)
    rows = H
    wo = [t_u16(weights(800 + i, rows, 8 * s[4], 0.02), dev) for i, s in enumerate(specs)]
    ref_out, ref_y = [], []
    for L, e, w, s in zip(layers, entries, wo, specs):  # each layer prepared alone, in layer order
        hd = s[4]
        ws1 = torch.empty(ops.step_workspace_bytes(1, 8, 1, hd), dtype=torch.uint8, device=dev)
        plan = ops.attn_step_prepare(ops.make_step_entries([e], 8, 1, hd), 8, 1, hd, ws1)
        ops.attn_step_run_attention(plan)
        y = torch.empty(rows, device=dev)
        ops.attn_step_run_out(plan, 8 * hd, [(w, y, rows)])
        torch.cuda.synchronize()
        ref_out.append(bits(L.out))
        ref_y.append(bits(y))
    plans = [None] * len(specs)
    keep = []
    for hd in (256, 512):  # one prepare per head_dim group
        idx = [i for i, s in enumerate(specs) if s[4] == hd]
        arr = ops.make_step_entries([entries[i] for i in idx], 8, 1, hd)
        ws = torch.empty(ops.step_layers_workspace_bytes(len(idx), 8, 1, hd), dtype=torch.uint8, device=dev)
        keep.append(ws)
        for i, p in zip(idx, ops.attn_step_prepare_layers(arr, 8, 1, hd, ws)):
            plans[i] = p
    for L in layers:
        L.out.fill_(float("nan"))
    ys = [torch.full((rows,), float("nan"), device=dev) for _ in specs]
    for i, s in enumerate(specs):  # layer order across the groups
        ops.attn_step_run_attention(plans[i])
        ops.attn_step_run_out(plans[i], 8 * s[4], [(wo[i], ys[i], rows)])
    torch.cuda.synchronize()
    for i, L in enumerate(layers):
        np.testing.assert_array_equal(bits(L.out), ref_out[i], err_msg=f"attnOut layer {i}")
        np.testing.assert_array_equal(bits(ys[i]), ref_y[i], err_msg=f"o_proj layer {i}")
    del tabs, keep
