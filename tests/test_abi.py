"""The C ABI boundary on the CPU: the library loads, exports every entry point
include/g4attn.h declares, its POD structs have the C compiler's layout and
the reference's uniform field offsets, and argument errors are rejected on
the host (no GPU needed) with a message from g4_last_error().
"""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from g4attn import abi

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "g4attn.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(g4_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = abi.load()
    names = declared_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and every declared function has a ctypes signature in the Python binding
    bound = set(abi.SIGNATURES) | set(abi.STRING_FUNCS)
    assert set(names) <= bound, set(names) - bound


def test_version_string():
    assert abi.load().g4_version().decode().startswith("g4attn")


STRUCTS = {
    "g4_norm_rope_params": abi.NormRopeParams,
    "g4_norm_params": abi.NormParams,
    "g4_kv_store_params": abi.KvStoreParams,
    "g4_attn_score_params": abi.AttnScoreParams,
    "g4_softmax_params": abi.SoftmaxParams,
    "g4_attn_output_params": abi.AttnOutputParams,
    "g4_prep_params": abi.PrepParams,
    "g4_prep_layer": abi.PrepLayer,
    "g4_decode_entry": abi.DecodeEntry,
    "g4_decode_plan": abi.DecodePlan,
    "g4_step_entry": abi.StepEntry,
    "g4_prefill_entry": abi.PrefillEntry,
    "g4_matmul_params": abi.MatmulParams,
    "g4_softcap_params": abi.SoftcapParams,
    "g4_lm_head_params": abi.LmHeadParams,
    "g4_linear_seg": abi.LinearSeg,
    "g4_linear_qseg": abi.LinearQSeg,
}


def test_struct_layouts_match_c(tmp_path):
    """sizeof/offsetof from gcc on include/g4attn.h equal the ctypes mirrors."""
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void) {"]
    for cname, py in STRUCTS.items():
        lines.append(f'printf("{cname} __sizeof__ %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {}
    for line in filter(None, out):
        cname, field, val = line.split()
        got[(cname, field)] = int(val)
    for cname, py in STRUCTS.items():
        assert got[(cname, "__sizeof__")] == C.sizeof(py), cname
        for fname, _ in py._fields_:
            assert got[(cname, fname)] == getattr(py, fname).offset, (cname, fname)


def test_params_match_reference_uniform_offsets():
    """Per-token fields sit where encodeTransformerPass writes them (src/engine.ts:1977-1987):
    position at byte 12 of fusedNormRope, slot at 8 of kvCacheStore, seq_len at 12 of
    attnScore/attnOutput and at 4 of softmax."""
    assert abi.NormRopeParams.position.offset == 12
    assert abi.KvStoreParams.position.offset == 8
    assert abi.AttnScoreParams.seq_len.offset == 12
    assert abi.AttnOutputParams.seq_len.offset == 12
    assert abi.SoftmaxParams.seq_len.offset == 4
    assert abi.AttnScoreParams.scale.offset == 16 and abi.AttnScoreParams.sliding_window.offset == 20
    assert abi.NormRopeParams.theta.offset == 16 and abi.NormRopeParams.apply_divisor.offset == 20


def _err(status_fn):
    lib = abi.load()
    st = status_fn(lib)
    return st, lib.g4_last_error().decode()


def test_argument_errors_rejected_on_host():
    p = abi.AttnScoreParams(8, 1, 128, 10, 1.0, 0)
    st, msg = _err(lambda L: L.g4_attn_decode(None, None, None, None, p, None, 0, None))
    assert st == abi.G4_EINVAL and "head_dim" in msg
    p = abi.AttnScoreParams(8, 1, 256, 10, 1.0, 0)
    st, msg = _err(lambda L: L.g4_attn_decode(None, None, None, None, p, None, 0, None))
    assert st == abi.G4_EINVAL and "NULL" in msg
    p = abi.AttnScoreParams(16, 1, 256, 10, 1.0, 0)
    st, msg = _err(lambda L: L.g4_attn_decode(1, 1, 1, 1, p, None, 0, None))
    assert st == abi.G4_EINVAL and "per kv head" in msg
    p = abi.AttnScoreParams(8, 3, 256, 10, 1.0, 0)
    st, msg = _err(lambda L: L.g4_attn_score(1, 1, 1, p, None))
    assert st == abi.G4_EINVAL and "multiple" in msg
    st, msg = _err(lambda L: L.g4_kv_cache_store(1, 1, 1, 1, abi.KvStoreParams(1, 256, 9, 9), None))
    assert st == abi.G4_EINVAL and "max_seq_len" in msg
    st, msg = _err(lambda L: L.g4_fused_per_head_norm_rope(1, 1, None, abi.NormRopeParams(8, 256, 1e-6, 0, 1e4, 1),
                                                            None))
    assert st == abi.G4_EINVAL and "rope_freqs" in msg
    st, msg = _err(lambda L: L.g4_attn_decode_many_run(C.byref(abi.DecodePlan()), None))
    assert st == abi.G4_EINVAL and "not prepared" in msg
    st, msg = _err(lambda L: L.g4_attn_step_run_out(C.byref(abi.DecodePlan()), None, 1, None))
    assert st == abi.G4_EINVAL and "not prepared" in msg


def test_lm_head_argument_errors_rejected_on_host():
    n = C.c_size_t(0)
    lib = abi.load()
    assert lib.g4_lm_head_workspace_size(abi.LmHeadParams(262144, 1536, 30.0), C.byref(n)) == abi.G4_OK
    assert 0 < n.value <= 2048 * 8
    st, msg = _err(lambda L: L.g4_lm_head_workspace_size(abi.LmHeadParams(1000, 300, 30.0), C.byref(n)))
    assert st == abi.G4_EINVAL and "hidden 300" in msg
    st, msg = _err(lambda L: L.g4_lm_head_workspace_size(abi.LmHeadParams(0, 1536, 30.0), C.byref(n)))
    assert st == abi.G4_EINVAL and "vocab 0" in msg
    p = abi.LmHeadParams(1000, 1536, 30.0)
    st, msg = _err(lambda L: L.g4_lm_head_argmax(None, 16, None, 16, 16, 4096, p, None))
    assert st == abi.G4_EINVAL and "NULL" in msg
    st, msg = _err(lambda L: L.g4_lm_head_argmax(8, 16, None, 16, 16, 4096, p, None))
    assert st == abi.G4_EINVAL and "aligned" in msg
    st, msg = _err(lambda L: L.g4_lm_head_argmax(16, 16, None, 16, 16, 8, p, None))
    assert st == abi.G4_ENOSPC and "workspace" in msg
    st, msg = _err(lambda L: L.g4_lm_head_argmax(16, 16, None, 16, 16, 4096, abi.LmHeadParams(1000, 1536, -1.0), None))
    assert st == abi.G4_EINVAL and "softcap" in msg
    n = C.c_size_t(0)
    st, _ = _err(lambda L: L.g4_attn_decode_workspace_size(8, 1, 256, 131072, C.byref(n)))
    assert st == abi.G4_OK and n.value > 131072 // 128 * 8 * 256 * 4


def test_python_wrappers_check_before_launch():
    """The tensor wrappers refuse CPU tensors and short buffers before calling the library."""
    torch = pytest.importorskip("torch")
    from g4attn import ops

    q = torch.zeros(8 * 256)
    with pytest.raises(ValueError, match="GPU"):
        ops.attn_decode(q, q, q, q, None, 8, 1, 256, 1)


def test_no_cpu_fallback_in_product_code():
    """The product package neither imports the oracle nor computes attention in Python."""
    pkg = ROOT / "gemma4-webgpu_amd"
    for f in list(pkg.rglob("*.py")) + list(pkg.rglob("*.js")) + list(pkg.rglob("*.cc")):
        text = f.read_text()
        assert "oracle" not in text.replace("oracle's", "").lower() or f.name == "build.py", f


def test_misaligned_out_rejected_on_host():
    """Outputs are written as 16-byte vectors: a misaligned out is refused before any launch."""
    lib = abi.load()
    n = C.c_size_t(0)
    assert lib.g4_attn_step_workspace_size(1, 8, 1, 256, C.byref(n)) == abi.G4_OK
    e = abi.StepEntry()
    e.q = e.k = e.v = e.q_weight = e.k_weight = e.k_cache = e.v_cache = 256
    e.out = 260
    e.seq_len, e.position, e.theta, e.scale, e.eps = 10, 9, 1e4, 1.0, 1e-6
    plan = abi.DecodePlan()
    st, msg = _err(lambda L: L.g4_attn_step_prepare(C.byref(e), 1, 8, 1, 256, 256, n.value, C.byref(plan), None))
    assert st == abi.G4_EINVAL and "16-byte aligned" in msg


def test_step_cached_row_entries_checked_on_host():
    """A consumer entry whose producer already stored the current row passes k, v and k_weight all NULL
    (and store_kv 0); a partial set, or store_kv without the raw k and v, is refused before any launch."""
    lib = abi.load()
    n = C.c_size_t(0)
    assert lib.g4_attn_step_workspace_size(1, 8, 1, 256, C.byref(n)) == abi.G4_OK
    plan = abi.DecodePlan()
    for k, v, kw, store, want in [(256, None, 256, 0, "all set or all NULL"), (None, None, 256, 0, "all set or all NULL"),
                                  (None, None, None, 1, "store_kv needs the raw k and v")]:
        e = abi.StepEntry()
        e.q = e.q_weight = e.k_cache = e.v_cache = e.out = 256
        e.k, e.v, e.k_weight, e.store_kv = k, v, kw, store
        e.seq_len, e.position, e.theta, e.scale, e.eps = 10, 9, 1e4, 1.0, 1e-6
        st, msg = _err(lambda L: L.g4_attn_step_prepare(C.byref(e), 1, 8, 1, 256, 256, n.value, C.byref(plan), None))
        assert st == abi.G4_EINVAL and want in msg, (k, v, kw, store, msg)


def test_layers_prepare_and_prompt_prep_checked_on_host():
    """g4_attn_step_prepare_layers and g4_attn_prompt_prep refuse bad arguments before any upload or launch:
    layer and entry counts, a bad entry in a later layer (reported with the layer, and no plan of the call
    left usable), a divisor with neither rope_freqs nor the inverse-frequency table."""
    lib = abi.load()
    n = C.c_size_t(0)
    st, msg = _err(lambda L: L.g4_attn_step_layers_workspace_size(0, 1, 8, 1, 256, C.byref(n)))
    assert st == abi.G4_EINVAL and "layers" in msg
    st, msg = _err(lambda L: L.g4_attn_step_layers_workspace_size(3, 0, 8, 1, 256, C.byref(n)))
    assert st == abi.G4_EINVAL and "entries per layer" in msg
    assert lib.g4_attn_step_layers_workspace_size(2, 3, 8, 1, 256, C.byref(n)) == abi.G4_OK
    one = C.c_size_t(0)
    assert lib.g4_attn_step_workspace_size(3, 8, 1, 256, C.byref(one)) == abi.G4_OK
    assert n.value == 2 * one.value
    ents = (abi.StepEntry * 2)()
    for i, e in enumerate(ents):
        e.q = e.k = e.v = e.q_weight = e.k_weight = e.k_cache = e.v_cache = 256
        e.out = 260 if i == 1 else 256  # layer 1's attnOut misaligned
        e.store_kv, e.seq_len, e.position, e.theta, e.scale, e.eps = 1, 10, 9, 1e4, 1.0, 1e-6
    plans = (abi.DecodePlan * 2)()
    assert lib.g4_attn_step_layers_workspace_size(2, 1, 8, 1, 256, C.byref(n)) == abi.G4_OK
    st, msg = _err(lambda L: L.g4_attn_step_prepare_layers(ents, 2, 1, 8, 1, 256, 256, n.value, plans, None))
    assert st == abi.G4_EINVAL and "layer 1" in msg and "16-byte aligned" in msg
    for p in plans:
        st, msg = _err(lambda L: L.g4_attn_step_run_attention(C.byref(p), None))
        assert st == abi.G4_EINVAL and "not prepared" in msg
    pp = abi.PromptPrepParams(8, 1, 128, 4, 0, 1e-6, 1e4, 0, 0, 0)
    st, msg = _err(lambda L: L.g4_attn_prompt_prep(1, None, None, 1, None, None, None, 1, None, None, pp, None))
    assert st == abi.G4_EINVAL and "head_dim 128" in msg
    pp = abi.PromptPrepParams(8, 1, 256, 4, 0, 1e-6, 1e6, 1, 0, 0)
    st, msg = _err(lambda L: L.g4_attn_prompt_prep(1, None, None, 1, None, None, None, 1, None, None, pp, None))
    assert st == abi.G4_EINVAL and "rope_freqs" in msg


def test_query_set_arguments_checked_on_host():
    """The timestamp query set refuses a slot count of 0 or above 65536, NULL handles and NULL outputs,
    and an end_pass with no pass open, before any HIP call."""
    q = C.c_void_p(0)
    for count in (0, 65537):
        st, msg = _err(lambda L: L.g4_query_set_create(count, C.byref(q)))
        assert st == abi.G4_EINVAL and "count" in msg and q.value is None
    st, msg = _err(lambda L: L.g4_query_set_create(4, None))
    assert st == abi.G4_EINVAL and "NULL" in msg
    st, msg = _err(lambda L: L.g4_query_write(None, 0, None))
    assert st == abi.G4_EINVAL and "NULL" in msg
    st, msg = _err(lambda L: L.g4_query_begin_pass(None, 0))
    assert st == abi.G4_EINVAL and "NULL" in msg
    st, msg = _err(lambda L: L.g4_query_end_pass())
    assert st == abi.G4_EINVAL and "no pass open" in msg
    ns = (C.c_double * 4)()
    st, msg = _err(lambda L: L.g4_query_resolve(None, 0, 2, ns))
    assert st == abi.G4_EINVAL and "NULL" in msg
    st, msg = _err(lambda L: L.g4_query_set_destroy(None))
    assert st == abi.G4_EINVAL and "NULL" in msg
