"""GPU parity of the two-head_dim launch (g4_attn_step_run_pair) over seeded random pairs of plans: a
head_dim-512 plan and a head_dim-256 plan, each with its own number of kv heads (1 or 2), query heads per
kv head (8 or 4), entries (1-6) and their lengths (1 .. 16000 rows) and sliding windows. The partitions
then range over single-part entries, the 8-wave form of a small head_dim-256 step, and long entries in
many parts, so the merge runs as one pair launch or falls back to the two plans' own merges.

Bars: every entry's attnOut within max-abs 2e-3 of the oracle's reference chain, every stored K/V row
bit-identical to the oracle's norm (+ RoPE) rounded to f16, and a second run of the pair gives the same
bits. The pair is given the plans in either order.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from g4attn import ops
from test_gpu_step import TOL, Layer

pytestmark = pytest.mark.gpu


def draw_group(rng, hd, large=False):
    """large: 6-8 entries of 24000-40000 rows with no window or a wide one (at least 144000 attended rows,
    above the 131072 up to which a head_dim-256 step is cut for one 8-wave workgroup per CU), so the
    head_dim-256 plan takes its 4-wave form."""
    nkh = int(rng.choice([1, 1, 2]))
    group = int(rng.choice([8, 4]))
    specs = []
    for _ in range(int(rng.integers(6, 9)) if large else int(rng.integers(1, 7))):
        r = rng.random()
        if large:
            seq = int(rng.integers(24000, 40001))
            w = int(rng.choice([0, 0, int(rng.integers(24000, 40001))]))
        else:
            seq = int(rng.integers(1, 40)) if r < 0.25 else int(rng.integers(40, 3000)) if r < 0.7 else \
                int(rng.integers(3000, 16001))
            w = int(rng.choice([0, 0, 512, int(rng.integers(1, 33)), int(rng.integers(33, 2000))]))
        glob = w == 0
        specs.append(dict(seq=seq, window=w, theta=1e6 if glob else 1e4, div=1 if glob else 0,
                          host=bool(rng.random() < 0.5)))
    return dict(hd=hd, nkh=nkh, group=group, specs=specs)


@pytest.mark.parametrize("seed", range(13))
def test_random_pairs_match_the_oracle(dev, seed):
    """Seeds 10-12 draw a large head_dim-256 plan (its 4-wave form); the others draw small ones."""
    rng = np.random.default_rng(9100 + seed)
    groups = [draw_group(rng, 512), draw_group(rng, 256, large=seed >= 10)]
    swap = bool(seed % 2)
    announce(f"attnStep pair random case {seed}: swap={swap} " + " | ".join(
        f"hd={g['hd']} nkh={g['nkh']} group={g['group']} {[(s['seq'], s['window']) for s in g['specs']]}"
        for g in groups))
    plans = []
    for gi, g in enumerate(groups):
        nqh = g["nkh"] * g["group"]
        g["layers"] = [Layer(dev, 900 + 31 * gi + 7 * i + seed, s["seq"], s["window"], s["theta"], s["div"], nqh=nqh,
                             nkh=g["nkh"], hd=g["hd"]) for i, s in enumerate(g["specs"])]
        entries = [L.entry(inv_freq=s["host"]) for L, s in zip(g["layers"], g["specs"])]
        arr = ops.make_step_entries(entries, nqh, g["nkh"], g["hd"])
        ws = torch.empty(ops.step_workspace_bytes(len(entries), nqh, g["nkh"], g["hd"]), dtype=torch.uint8,
                         device=dev)
        plans.append((arr, ws, ops.attn_step_prepare(arr, nqh, g["nkh"], g["hd"], ws)))
    first, second = (plans[1][2], plans[0][2]) if swap else (plans[0][2], plans[1][2])
    runs = []
    for _ in range(2):
        ops.attn_step_run_pair(first, second)
        torch.cuda.synchronize()
        runs.append([[L.out.cpu().numpy().copy() for L in g["layers"]] for g in groups])
    for gi, g in enumerate(groups):
        for i, (L, s) in enumerate(zip(g["layers"], g["specs"])):
            tag = f"head_dim {g['hd']} entry {i} {s}"
            np.testing.assert_array_equal(runs[0][gi][i].view(np.uint32), runs[1][gi][i].view(np.uint32),
                                          err_msg=f"{tag}: second run differs")
            want, kb, vb = L.expected()
            got = runs[1][gi][i]
            assert np.isfinite(got).all(), f"{tag}: non-finite attnOut"
            err = float(np.abs(got - want).max())
            assert err <= TOL, f"{tag}: attnOut max-abs {err}"
            np.testing.assert_array_equal(L.kc[L.pos].cpu().numpy().view(np.uint16), kb, err_msg=f"{tag} K")
            np.testing.assert_array_equal(L.vc[L.pos].cpu().numpy().view(np.uint16), vb, err_msg=f"{tag} V")
