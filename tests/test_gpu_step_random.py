"""GPU parity of the one-launch step over seeded random steps: the number of entries, their lengths
(1 .. 20000 rows), sliding windows (none, narrower than a tile, the E2B 512, arbitrary), head_dim 256
or 512, 8 or 4 query heads per kv head with one or two kv heads, RoPE factors from a host table or
from the kernel, and KV-consumer entries (of their producer's layer type) that read its cache after it stored the row.

Bars: every entry's attnOut within max-abs 2e-3 of the oracle's reference chain, and every stored K/V
row bit-identical to the oracle's norm (+ RoPE) rounded to f16; each case is run through prepare and
run twice (the second run on the same plan must give the same bits).
"""
import numpy as np
import pytest
import torch

from conftest import announce
from g4attn import ops
from test_gpu_step import TOL, Layer

pytestmark = pytest.mark.gpu


def draw_case(rng):
    hd = int(rng.choice([256, 256, 512]))
    nkh = int(rng.choice([1, 1, 2]))
    group = int(rng.choice([8, 4]))
    n = int(rng.integers(1, 9))
    specs = []
    for i in range(n):
        r = rng.random()
        seq = int(rng.integers(1, 40)) if r < 0.2 else int(rng.integers(40, 3000)) if r < 0.7 else \
            int(rng.integers(3000, 20001))
        w = int(rng.choice([0, 0, 512, int(rng.integers(1, 33)), int(rng.integers(33, 2000))]))
        glob = w == 0
        consumer = i > 0 and rng.random() < 0.2  # reads entry i-1's cache after it stored the row
        if consumer:  # a consumer is of its producer's layer type (its window, theta, divisor), as in E2B
            p = specs[i - 1]
            w, glob = p["window"], p["window"] == 0
        specs.append(dict(seq=seq, window=w, theta=1e6 if glob else 1e4, div=1 if glob else 0,
                          host=bool(rng.random() < 0.5), consumer=consumer))
    return hd, nkh, group, specs


@pytest.mark.parametrize("seed", range(12))
def test_random_steps_match_the_oracle(dev, seed):
    rng = np.random.default_rng(7000 + seed)
    hd, nkh, group, specs = draw_case(rng)
    nqh = nkh * group
    announce(f"attnStep random case {seed}: hd={hd} nkh={nkh} group={group} "
             f"{[(s['seq'], s['window'], s['consumer']) for s in specs]}")
    layers, entries, runs, root = [], [], [], []
    for i, s in enumerate(specs):
        root.append(root[i - 1] if s["consumer"] else i)  # the layer that stored the shared cache's row
        if s["consumer"]:  # same cache, length and position as its producer
            P = layers[i - 1]
            L = Layer(dev, 600 + 17 * i + seed, P.seq, s["window"], s["theta"], s["div"], nqh=nqh, nkh=nkh,
                      cache=(P.kc, P.vc), hd=hd)
        else:
            L = Layer(dev, 600 + 17 * i + seed, s["seq"], s["window"], s["theta"], s["div"], nqh=nqh, nkh=nkh,
                      hd=hd)
        e = L.entry(store=not s["consumer"], inv_freq=s["host"])
        if s["consumer"]:
            e["k"] = e["v"] = e["k_weight"] = None
        layers.append(L)
        entries.append(e)
    # producers before their consumers: a consumer's step runs after its producer stored the row
    groups, cur = [], []
    for i, s in enumerate(specs):
        if s["consumer"]:
            groups.append(cur)
            cur = []
        cur.append(i)
    groups.append(cur)
    for rep in range(2):
        for g in groups:
            if not g:
                continue
            arr = ops.make_step_entries([entries[i] for i in g], nqh, nkh, hd)
            ws = torch.empty(ops.step_workspace_bytes(len(g), nqh, nkh, hd), dtype=torch.uint8, device=dev)
            plan = ops.attn_step_prepare(arr, nqh, nkh, hd, ws)
            ops.attn_step_run(plan)
            torch.cuda.synchronize()
        runs.append([L.out.cpu().numpy().copy() for L in layers])
    for i, (L, s) in enumerate(zip(layers, specs)):
        np.testing.assert_array_equal(runs[0][i].view(np.uint32), runs[1][i].view(np.uint32),
                                      err_msg=f"entry {i}: second run differs")
        want, kb, vb = L.expected(kv_from=layers[root[i]] if s["consumer"] else None)
        got = runs[1][i]
        assert np.isfinite(got).all(), f"entry {i}: non-finite attnOut"
        err = float(np.abs(got - want).max())
        assert err <= TOL, f"entry {i} {s}: attnOut max-abs {err}"
        if not s["consumer"]:
            np.testing.assert_array_equal(L.kc[L.pos].cpu().numpy().view(np.uint16), kb, err_msg=f"entry {i} K")
            np.testing.assert_array_equal(L.vc[L.pos].cpu().numpy().view(np.uint16), vb, err_msg=f"entry {i} V")
