"""The one-launch step's host planner (gemma4-webgpu_amd/csrc/step_plan.h) on the CPU, under
AddressSanitizer and UndefinedBehaviorSanitizer: tests/step_plan_check.cpp plans the benchmark's workloads
(the 35-layer stacks at 8K and 32K, the E2B head_dim-512 group, the 64 ragged sequences, one 128K layer,
one local layer) and random ragged sets, and checks every plan: each entry's attended rows covered once
and in order by its workgroups, partial-record slots unique and inside the workspace, the merge table
listing exactly the split entries, RoPE-factor pointers inside the uploaded factors with the C library's
values, and the packed tables inside the workspace's tables region. Every scenario is also planned layer by
layer as g4_attn_step_prepare_layers does (one packed upload, RoPE sets shared between layers at one
position), with one entry per layer and, for an even count, two: each layer's plan must equal the plan
of its entries alone apart from the RoPE pointers.
"""
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from g4attn import e2b, workloads

ROOT = Path(__file__).resolve().parent.parent
SRC = ROOT / "tests" / "step_plan_check.cpp"
GXX = shutil.which("g++")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if GXX is None:
        pytest.skip("g++ is not installed")
    exe = tmp_path_factory.mktemp("plan") / "step_plan_check"
    subprocess.run([GXX, "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    f"-I{ROOT / 'include'}", str(SRC), "-o", str(exe)], check=True)
    return exe


def stack(pos, hd_global=256, shared=False):
    cfg = e2b.AttnConfig(num_layers=35)
    out = []
    for il in range(35):
        out.append((pos + 1, e2b.sliding_window(il, cfg)))
    return out


def line(nqh, nkh, hd, cus, ents):
    return f"{nqh} {nkh} {hd} {cus} " + " ".join(f"{s}:{w}" + (":c" if c else "") for s, w, c in ents)


def scenarios():
    rng = np.random.default_rng(7)
    L = []
    for pos in (8192, 32768, 4096, 512):
        L.append(line(8, 1, 256, 256, [(s, w, False) for s, w in stack(pos)]))
    cfg = e2b.AttnConfig(num_layers=35)
    pmap = e2b.compute_kv_producer_map(cfg)
    for pos in (8192, 32768):  # the E2B head_dim-512 group (globals; consumers read the cached row)
        L.append(line(8, 1, 512, 256, [(pos + 1, 0, pmap[il] != il) for il in range(35) if il in e2b.GLOBAL_LAYERS]))
    L.append(line(8, 1, 256, 256, [(s, 0, False) for s in workloads.ragged64_lengths()]))
    L.append(line(8, 1, 256, 256, [(131072, 0, False)]))
    L.append(line(8, 1, 256, 256, [(513, 512, False)]))
    L.append(line(8, 1, 256, 256, [(1, 0, False), (2, 0, True), (33, 512, False)]))
    L.append(line(16, 2, 256, 256, [(1500, 0, False), (700, 512, False)]))
    for cus in (256, 304, 80):
        for _ in range(10):
            n = int(rng.integers(1, 80))
            ents = [(int(rng.integers(1, 70000)), int(rng.choice([0, 512, 4096])), bool(rng.integers(0, 4) == 0))
                    for _ in range(n)]
            L.append(line(8, 1, int(rng.choice([256, 512])), cus, ents))
    return L


def test_step_plans_hold_their_invariants(checker):
    scen = scenarios()
    r = subprocess.run([str(checker)], input="\n".join(scen) + "\n", capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    oks = [l for l in r.stdout.splitlines() if l.startswith("ok")]
    assert len(oks) == len(scen), r.stdout[-2000:]
    # ragged64 fills the GPU in one wave of two 4-wave workgroups per CU; every sequence split at most this much
    wgs, merges = map(int, oks[6].split()[1:])
    assert wgs <= 512 and merges <= 64


def test_step_plan_rejects_bad_entries(checker):
    # a zero-length entry fails the plan with a message, not a crash
    r = subprocess.run([str(checker)], input="8 1 256 256 0:0\n", capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "seq_len 0" in r.stdout


def test_rope_factors_match_the_c_library(checker):
    """The planner's RoPE factors (Cody-Waite reduction and Taylor polynomials in f64, with the C library
    taken near f32 rounding boundaries) equal (float)cos/sin((double)angle) of the C library at every
    position 0..131071, at head_dim 256 and 512 and theta 1e4 and 1e6, and at angles past 2^20."""
    r = subprocess.run([str(checker), "rope", "1"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert r.stdout.startswith("ok rope "), r.stdout
    assert int(r.stdout.split()[2]) > 100_000_000
