"""GPU parity of the chunked prompt prep over seeded random launches, bit for bit against the oracle.

Each case draws a head_dim (256 or 512), a kv-head count and group (num_q_heads = kv heads x group), a
layer class (local: theta 1e4; global: theta 1e6 with the rope_freqs divisor), a chunk start anywhere up to
position 131071, a chunk length (short ragged chunks and full 512-token ones), a producer or a consumer
layer, a V^T cache on producers and the caller's inverse-frequency table or none. The bars are those of
test_gpu_prompt_prep: q_out, the stored K and V rows and the V^T blocks equal the f16 rounding of the
oracle's fused_per_head_norm_rope / per_head_rms_norm_no_weight bit for bit, and nothing outside the chunk
(or, on a consumer layer, nothing at all) is written in the caches.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from g4attn import ops
from test_gpu_prompt_prep import Chunk

pytestmark = pytest.mark.gpu

CASES = 12


def draw(seed, hd=None):
    r = np.random.default_rng(seed)
    hd = int(r.choice([256, 512])) if hd is None else hd
    nkh = int(r.choice([1, 1, 2, 4]))
    group = int(r.choice([1, 2, 4, 8]))
    glob = bool(r.integers(2))
    theta, div = (1e6, 1) if glob else (1e4, 0)
    T = int(r.choice([1, 2, 3, 31, 33, 64, 97, 512])) if r.integers(2) else int(r.integers(1, 600))
    start = int(r.integers(0, 131072 - T))
    store = bool(r.integers(4))  # mostly producers
    vt = store and bool(r.integers(2))
    inv_table = bool(r.integers(2))
    return dict(hd=hd, nkh=nkh, nqh=nkh * group, theta=theta, div=div, T=T, start=start, store=store, vt=vt,
                inv_table=inv_table)


@pytest.mark.parametrize("case", range(CASES))
def test_random_prompt_prep_launches_match_the_oracle(dev, case):
    p = draw(7100 + case)
    announce(f"attnPromptPrep random case {case}: {p}")
    c = Chunk(dev, 9000 + 17 * case, p["start"], p["T"], p["hd"], p["theta"], p["div"], nqh=p["nqh"], nkh=p["nkh"],
              store=p["store"], vt=p["vt"])
    c.run(p["inv_table"])
    c.check()


@pytest.mark.parametrize("case", range(6))
def test_random_prompt_prep_many_launches_match_the_oracle(dev, case):
    """g4_attn_prompt_prep_many over 1-8 chunks of one head_dim, each drawn as above (its own kv heads,
    group, layer class, start, length, producer or consumer, V^T cache and inverse-frequency table): every
    chunk to the same bars, in one launch."""
    hd = 512 if case % 3 == 2 else 256
    n = int(np.random.default_rng(7300 + case).integers(1, 9))
    ps = [draw(7400 + 11 * case + i, hd) for i in range(n)]
    announce(f"attnPromptPrepMany random case {case}: hd={hd} "
             f"{[(p['start'], p['T'], p['nkh'], p['nqh'], p['store'], p['vt']) for p in ps]}")
    chunks = [Chunk(dev, 9500 + 17 * case + 3 * i, p["start"], p["T"], hd, p["theta"], p["div"], nqh=p["nqh"],
                    nkh=p["nkh"], store=p["store"], vt=p["vt"]) for i, p in enumerate(ps)]
    ops.attn_prompt_prep_many([c.kwargs(p["inv_table"]) for c, p in zip(chunks, ps)])
    torch.cuda.synchronize()
    for i, c in enumerate(chunks):
        announce(f"  chunk {i}")
        c.check()
