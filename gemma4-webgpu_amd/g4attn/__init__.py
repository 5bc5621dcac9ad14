"""Python host binding of the gfx950 Gemma-4 attention library (libg4attn.so).

`abi` declares the C ABI of include/g4attn.h; `ops` wraps it for torch
device tensors; `synth` makes the seeded synthetic inputs; `e2b` holds the
Gemma-4-E2B attention shape helpers.
"""
from . import abi, e2b, synth  # noqa: F401

__all__ = ["abi", "e2b", "synth"]
