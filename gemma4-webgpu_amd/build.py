"""Build recipe for the gfx950 attention library and its N-API addon.

    python gemma4-webgpu_amd/build.py            # library (+ addon when Node headers exist)

Outputs (in-tree, so they travel with the source tree to a GPU host):
    gemma4-webgpu_amd/lib/libg4attn.so   C ABI declared in include/g4attn.h
    gemma4-webgpu_amd/lib/g4attn.node    Node N-API addon over the same ABI
    gemma4-webgpu_amd/lib/g4bench        C++ decode benchmark driver over the same ABI

Every HIP source is compiled for gfx950 only, with packed-FP32 instruction
selection disabled (-packed-fp32-ops).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
OBJ = PKG / "_build"
INCLUDE = ROOT / "include"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]
NODE_INCLUDE = Path("/usr/include/node")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


# Per-file code generation options. prefill.hip: MFMA accumulators in VGPRs (the
# pipelined prefill rescales them with plain VALU; its q operand is kept in AGPRs),
# and IEEE mode off with NaN-free math, so that max over scores is one v_max each
# instead of canonicalize + max (scores are finite or -inf; no NaN is produced).
# step.hip, decode.hip: kernel arguments (scalars and pointers) preloaded into
# SGPRs at wave start, so a workgroup's first scalar load is its work item.
FILE_FLAGS = {"prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-mno-amdgpu-ieee", "-fno-honor-nans"],
              "step.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
              "decode.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"]}


def _compile(src: Path) -> Path:
    obj = OBJ / (src.name + ".o")
    lang = [] if src.suffix == ".hip" else ["-x", "hip"]
    _run([HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(src.name, []), *lang, "-c", str(src), "-o", str(obj)])
    return obj


def build_library(jobs: int | None = None) -> Path:
    OBJ.mkdir(exist_ok=True)
    LIB.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, sources))
    out = LIB / "libg4attn.so"
    tmp = LIB / "libg4attn.so.tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, out)
    return out


def build_bench() -> Path:
    """g4bench: C++ driver of the decode path over the C ABI (no Python in the process)."""
    src = PKG / "bench" / "g4bench.hip"
    out = LIB / "g4bench"
    tmp = LIB / "g4bench.tmp"
    _run([HIPCC, *HIP_FLAGS, str(src), "-o", str(tmp), f"-L{LIB}", "-lg4attn", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, out)
    return out


def build_addon() -> Path | None:
    """Node N-API addon: a thin C++ shim that links libg4attn.so (no HIP code)."""
    src = PKG / "addon" / "g4attn_napi.cc"
    if not src.exists() or not (NODE_INCLUDE / "node_api.h").exists():
        return None
    out = LIB / "g4attn.node"
    tmp = LIB / "g4attn.node.tmp"
    cxx = shutil.which("g++") or "g++"
    _run([cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", f"-I{NODE_INCLUDE}", f"-I{INCLUDE}",
          "-DNAPI_VERSION=8", str(src), "-o", str(tmp), f"-L{LIB}", "-lg4attn", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, out)
    return out


def main() -> None:
    lib = build_library()
    print(f"built {lib}")
    print(f"built {build_bench()}")
    addon = build_addon()
    if addon:
        print(f"built {addon}")


if __name__ == "__main__":
    main()
