"""Writes tests/golden/layer0_attn.npz from the reference's committed fixture.

Source: public/ref/layer_0_detail.npz of gemma4-webgpu (HF transformers bf16
forward-hook dump of Gemma-4-E2B layer 0 at position 14 of the canonical
15-token prompt; see reference/pytorch/README.md there). Only the attention
entries on this path are kept, as data: the q/k/v projections and their
per-head norms.

    python tests/golden/make_golden.py /root/reference/public/ref/layer_0_detail.npz
"""
import sys
from pathlib import Path

import numpy as np

KEYS = {
    "q_proj": "L0_self_attn.q_proj_output",
    "q_norm": "L0_self_attn.q_norm_output",
    "k_proj": "L0_self_attn.k_proj_output",
    "k_norm": "L0_self_attn.k_norm_output",
    "v_proj": "L0_self_attn.v_proj_output",
    "v_norm": "L0_self_attn.v_norm_output",
    "o_proj_input": "L0_self_attn_o_proj_input",
    "position": "position",
    "tokens": "tokens",
}


def main(src: str) -> None:
    d = np.load(src, allow_pickle=False)
    out = {k: np.asarray(d[v]) for k, v in KEYS.items()}
    dst = Path(__file__).resolve().parent / "layer0_attn.npz"
    np.savez_compressed(dst, **out)
    print(f"wrote {dst}: " + ", ".join(f"{k}{tuple(v.shape)}" for k, v in out.items()))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/public/ref/layer_0_detail.npz")
