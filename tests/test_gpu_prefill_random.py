"""GPU parity of the MFMA causal prefill over seeded random launches: 1 to 4 chunk entries in one
launch, chunk starts from 0 to 6000 and lengths from 1 to 160 tokens, windows (none, the E2B 512,
narrower than a tile, arbitrary), head_dim 256 or 512 (every third seed), and query-to-kv-head groups
of 8, 4, 2 and 1 with one or two kv heads. The reference has no prefill kernel; it runs one decode step
per prompt token (src/engine.ts:2469-2475), so every token of every entry is checked against the
oracle's attnScore -> softmax -> attnOutput chain at its own seq_len, within max-abs 2e-3. Preparing
and running the same launch again must give the same bits."""
import numpy as np
import pytest

from conftest import announce
from test_gpu_prefill import Chunk, check, run

pytestmark = pytest.mark.gpu

SHAPES = [(8, 1), (8, 1), (4, 1), (8, 2), (4, 2), (2, 2)]  # (query heads, kv heads)


def draw_case(rng, hd):
    nqh, nkh = SHAPES[int(rng.integers(len(SHAPES)))]
    specs = []
    for _ in range(int(rng.integers(1, 5))):
        r = rng.random()
        start = 0 if r < 0.25 else int(rng.integers(1, 600)) if r < 0.6 else int(rng.integers(600, 6001))
        T = int(rng.choice([1, int(rng.integers(2, 33)), int(rng.integers(33, 161))]))
        w = int(rng.choice([0, 0, 512, int(rng.integers(1, 33)), int(rng.integers(33, 1500))]))
        specs.append((start, T, w))
    return nqh, nkh, specs


@pytest.mark.parametrize("seed", range(12))
def test_random_prefill_launches_match_the_oracle(dev, seed):
    rng = np.random.default_rng(9100 + seed)
    hd = 512 if seed % 3 == 2 else 256
    nqh, nkh, specs = draw_case(rng, hd)
    announce(f"attnPrefill random case {seed}: hd={hd} nqh={nqh} nkh={nkh} (start, T, window) {specs}")
    chunks = [Chunk(dev, 5000 + 13 * i + 101 * seed, s, T, w, nqh=nqh, nkh=nkh, hd=hd)
              for i, (s, T, w) in enumerate(specs)]
    run(dev, chunks, nqh=nqh, nkh=nkh, hd=hd)
    first = [c.out.cpu().numpy().copy() for c in chunks]
    run(dev, chunks, nqh=nqh, nkh=nkh, hd=hd)
    for i, c in enumerate(chunks):
        np.testing.assert_array_equal(first[i].view(np.uint32), c.out.cpu().numpy().view(np.uint32),
                                      err_msg=f"entry {i}: second run differs")
        err = check(c, f"entry {i} {specs[i]}")
        print(f"entry {i} {specs[i]}: max-abs {err:.2e}")
