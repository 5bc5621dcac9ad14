"""GPU parity of the fused projections over seeded random launches, bit for bit against the oracle.

Each case draws an input length N (a multiple of 256 in [1024, 4096]), a weight format (f16, q8 or q4k),
one to four weight matrices of 1-5000 rows read in one launch, and an input scale; every output row must
equal the oracle's matmul_quant.wgsl / matmul_q8.wgsl / matmul_q4k.wgsl restatement bit for bit, as in
test_gpu_linear.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import oracle as orc
from g4attn import ops
from test_gpu_linear import q4k_weights, q8_weights, t_f32, t_i8, t_u16, t_u32, weights

pytestmark = pytest.mark.gpu

CASES = 12


def draw(seed):
    r = np.random.default_rng(seed)
    N = 256 * int(r.integers(4, 17))
    fmt = str(r.choice(["f16", "q8", "q4k"]))
    n_seg = int(r.integers(1, 5))
    rows = [int(r.choice([1, 2, 7, 256, 1536])) if r.integers(2) else int(r.integers(1, 5001)) for _ in range(n_seg)]
    scale = float(r.choice([1e-3, 1.0, 30.0]))
    return N, fmt, rows, scale


@pytest.mark.parametrize("case", range(CASES))
def test_random_linear_launches_match_the_oracle(dev, case):
    N, fmt, rows, scale = draw(8200 + case)
    announce(f"linear random case {case}: N={N} fmt={fmt} rows={rows} scale={scale}")
    x = (np.random.default_rng(8300 + case).standard_normal(N, dtype=np.float32) * scale).astype(np.float32)
    outs = [torch.full((r,), float("nan"), device=dev) for r in rows]
    segs, wants = [], []
    for i, (r, o) in enumerate(zip(rows, outs)):
        seed = 8400 + 37 * case + i
        if fmt == "f16":
            w = weights(seed, r, N)
            segs.append((t_u16(w, dev), o, r))
            wants.append(orc.matmul_quant(x, w, r, N))
        elif fmt == "q8":
            q, sc = q8_weights(seed, r, N)
            segs.append((t_i8(q, dev), t_u16(sc, dev), o, r))
            wants.append(orc.matmul_q8(x, q, sc, r, N))
        else:
            w, meta = q4k_weights(seed, r, N)
            segs.append((t_u32(w, dev), t_u16(meta, dev), o, r))
            wants.append(orc.matmul_q4k(x, w, meta, r, N))
    if fmt == "f16":
        ops.linear_f16(t_f32(x, dev), N, segs)
    else:
        ops.linear_quant(t_f32(x, dev), N, fmt, segs)
    torch.cuda.synchronize()
    for i, (o, want) in enumerate(zip(outs, wants)):
        np.testing.assert_array_equal(o.cpu().numpy().view(np.uint32), want.view(np.uint32), err_msg=f"segment {i}")
