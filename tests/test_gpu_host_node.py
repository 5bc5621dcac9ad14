"""One attention layer through the TypeScript host (node host/run.js layer): the engine's six
dispatches in order, with uniforms built and patched as src/engine.ts does, and the fused attnStep,
both over the N-API addon. Checked against the oracle: the six-kernel path bit-identical (those
kernels evaluate the reference's expressions), attnStep within max-abs 2e-3, and the stored f16
K/V rows bit-identical on both paths. The sampling head likewise (node host/run.js head): the
engine's lmHead, logitSoftcap and sample.argmax dispatches and the fused lmHeadArgmax, logits
bit-identical and top-1 equal to the oracle's. And attnPrefill (node host/run.js prefill): two
chunks in one call, each token within max-abs 2e-3 of the oracle's decode chain at its position.
The projections (node host/run.js linear): one matmulQuant dispatch per matrix and one linear call,
both bit-identical to the oracle's matmulQuant. The layer case also runs the step as its attention
pass plus attnStepOut (attn.linearOut with the merge folded in): attnOut bit-identical to attnStep's,
and the projected rows bit-identical to linear() over it and to the oracle's matmulQuant.
"""
import json
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from conftest import announce
from g4attn import e2b, synth
from helpers import EPS, cache_f16, f16_weight_bits, max_abs
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
RUN = ROOT / "gemma4-webgpu_amd" / "host" / "run.js"
NODE = shutil.which("node")
NQH, NKH, HD = 8, 1, 256
ROPE = np.array(e2b.rope_freqs_f16_bits(256), dtype=np.uint16)
O_ROWS = 96  # o_proj rows of the layer case


def write_case(d: Path, seed, seq, window, theta, div, hd=HD):
    pos = seq - 1
    arrs = {
        "q": synth.normal(seed, NQH * hd) * 2.0, "k": synth.normal(seed + 1, NKH * hd) * 2.0,
        "v": synth.normal(seed + 2, NKH * hd) * 2.0, "qw": f16_weight_bits(seed + 3, hd),
        "kw": f16_weight_bits(seed + 4, hd), "rf": ROPE,
        "kc": cache_f16(seed + 5, seq, NKH, hd).reshape(-1), "vc": cache_f16(seed + 6, seq, NKH, hd).reshape(-1),
        "wo": (np.random.default_rng(seed + 7).standard_normal((O_ROWS, NQH * hd), dtype=np.float32) * 0.02)
        .astype(np.float16).view(np.uint16).reshape(-1),
    }
    blob, index = bytearray(), {}
    for name, a in arrs.items():
        b = np.ascontiguousarray(a).tobytes()
        index[name] = [len(blob), len(b)]
        blob += b
    (d / "case.bin").write_bytes(bytes(blob))
    (d / "case.json").write_text(json.dumps(dict(nqh=NQH, nkh=NKH, hd=hd, seq=seq, pos=pos, window=window,
                                                 theta=theta, div=div, eps=EPS, oRows=O_ROWS, arrays=index)))
    return arrs, pos


def expected(arrs, seq, pos, window, theta, div, hd=HD):
    v_ = orc.per_head_rms_norm_no_weight(arrs["v"], NKH, hd, EPS)
    k_ = orc.fused_per_head_norm_rope(arrs["k"], arrs["kw"], ROPE, NKH, hd, EPS, pos, theta, div)
    q_ = orc.fused_per_head_norm_rope(arrs["q"], arrs["qw"], ROPE, NQH, hd, EPS, pos, theta, div)
    kb = arrs["kc"].reshape(seq, NKH * hd).copy()
    vb = arrs["vc"].reshape(seq, NKH * hd).copy()
    kb[pos] = orc.f32_to_f16_bits(k_)
    vb[pos] = orc.f32_to_f16_bits(v_)
    out = orc.attention_chain(q_, orc.f16_bits_to_f32(kb).reshape(-1), orc.f16_bits_to_f32(vb).reshape(-1),
                              NQH, NKH, hd, seq, 1.0, window)
    return out, kb[pos], vb[pos]


@pytest.mark.skipif(NODE is None, reason="node is not installed")
@pytest.mark.parametrize("seq,window,theta,div,hd", [(513, 512, 1e4, 0, 256), (2049, 0, 1e6, 1, 256),
                                                     (7, 0, 1e4, 0, 256), (2049, 0, 1e6, 1, 512)])
def test_layer_through_ts_host(tmp_path, seq, window, theta, div, hd):
    announce(f"TS host layer seq={seq} window={window} hd={hd}")
    arrs, pos = write_case(tmp_path, 77 + seq, seq, window, theta, div, hd)
    r = subprocess.run([NODE, str(RUN), "layer", str(tmp_path)], cwd=ROOT, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    raw = (tmp_path / "out.bin").read_bytes()
    o = NQH * hd * 4
    row = NKH * hd * 2
    yb = O_ROWS * 4
    out_ref = np.frombuffer(raw[:o], np.float32)
    out_step = np.frombuffer(raw[o:2 * o], np.float32)
    out_split = np.frombuffer(raw[2 * o:3 * o], np.float32)
    y_linear = np.frombuffer(raw[3 * o:3 * o + yb], np.float32)
    y_out = np.frombuffer(raw[3 * o + yb:3 * o + 2 * yb], np.float32)
    base = 3 * o + 2 * yb
    rows = [np.frombuffer(raw[base + i * row:base + (i + 1) * row], np.uint16) for i in range(4)]
    want, kbits, vbits = expected(arrs, seq, pos, window, theta, div, hd)
    np.testing.assert_array_equal(out_ref.view(np.uint32), want.view(np.uint32))
    assert np.isfinite(out_step).all() and max_abs(out_step, want) <= 2e-3
    for got, exp in zip(rows, (kbits, vbits, kbits, vbits)):
        np.testing.assert_array_equal(got, exp)
    # attention pass + attnStepOut: attnOut as attnStep writes it, rows as linear() and matmulQuant give them
    np.testing.assert_array_equal(out_split.view(np.uint32), out_step.view(np.uint32))
    np.testing.assert_array_equal(y_out.view(np.uint32), y_linear.view(np.uint32))
    np.testing.assert_array_equal(y_out.view(np.uint32),
                                  orc.matmul_quant(out_step, arrs["wo"], O_ROWS, NQH * hd).view(np.uint32))
    # two layers prepared together (attnStepPrepareLayers): each layer's attnOut, rows and projection as the
    # one-layer step gives them
    b4 = base + 4 * row
    for i in range(2):
        got = np.frombuffer(raw[b4 + i * o:b4 + (i + 1) * o], np.float32)
        np.testing.assert_array_equal(got.view(np.uint32), out_step.view(np.uint32), err_msg=f"layer {i}")
    y4 = np.frombuffer(raw[b4 + 2 * o:b4 + 2 * o + yb], np.float32)
    np.testing.assert_array_equal(y4.view(np.uint32), y_linear.view(np.uint32))
    rows4 = [np.frombuffer(raw[b4 + 2 * o + yb + i * row:b4 + 2 * o + yb + (i + 1) * row], np.uint16)
             for i in range(4)]
    for got, exp in zip(rows4, (kbits, vbits, kbits, vbits)):
        np.testing.assert_array_equal(got, exp)


@pytest.mark.skipif(NODE is None, reason="node is not installed")
@pytest.mark.parametrize("vocab,hidden,cap", [(5000, 1536, 30.0), (777, 2048, 0.0)])
def test_sampling_head_through_ts_host(tmp_path, vocab, hidden, cap):
    announce(f"TS host sampling head vocab={vocab} hidden={hidden} cap={cap}")
    rng = np.random.default_rng(vocab)
    x = rng.standard_normal(hidden, dtype=np.float32)
    w = (rng.standard_normal((vocab, hidden), dtype=np.float32) * 0.05).astype(np.float16).view(np.uint16)
    w[[10, 266]] = (np.sign(x) * 0.2).astype(np.float16).view(np.uint16)  # a tie at the top
    blob = x.tobytes() + w.tobytes()
    (tmp_path / "case.bin").write_bytes(blob)
    (tmp_path / "case.json").write_text(json.dumps(dict(vocab=vocab, hidden=hidden, cap=cap, arrays=dict(
        x=[0, x.nbytes], w=[x.nbytes, w.nbytes]))))
    r = subprocess.run([NODE, str(RUN), "head", str(tmp_path)], cwd=ROOT, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    raw = (tmp_path / "out.bin").read_bytes()
    n = vocab * 4
    want = orc.matmul_quant(x, w, vocab, hidden)
    if cap > 0:
        want = orc.logit_softcap(want, cap)
    top = orc.argmax(want)
    assert top in (10, 266)
    for i in range(2):
        np.testing.assert_array_equal(np.frombuffer(raw[i * n:(i + 1) * n], np.uint32), want.view(np.uint32))
    res = np.frombuffer(raw[2 * n:2 * n + 8], np.uint32)
    assert res[0] == top and res[1] == top


@pytest.mark.skipif(NODE is None, reason="node is not installed")
def test_prefill_through_ts_host(tmp_path):
    announce("TS host attnPrefill: 2 chunks")
    chunks, blob, spec = [], bytearray(), []
    for i, (start, T, window) in enumerate(((0, 37, 0), (600, 20, 512))):
        rows = start + T
        kc, vc = cache_f16(70 + i, rows, NKH, HD), cache_f16(80 + i, rows, NKH, HD)
        q = synth.rms_normalize_rows(synth.normal(90 + i, T * NQH * HD).reshape(T * NQH, HD))
        qb = orc.f32_to_f16_bits(q).reshape(T, NQH * HD)
        idx = {}
        for name, a in (("q", qb), ("kc", kc), ("vc", vc)):
            b = np.ascontiguousarray(a).tobytes()
            idx[name] = [len(blob), len(b)]
            blob += b
        spec.append(dict(start=start, nTokens=T, window=window, **idx))
        chunks.append((start, T, window, qb, kc, vc))
    (tmp_path / "case.bin").write_bytes(bytes(blob))
    (tmp_path / "case.json").write_text(json.dumps(dict(nqh=NQH, nkh=NKH, hd=HD, chunks=spec)))
    r = subprocess.run([NODE, str(RUN), "prefill", str(tmp_path)], cwd=ROOT, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    got = np.frombuffer((tmp_path / "out.bin").read_bytes(), np.float32)
    off = 0
    for start, T, window, qb, kc, vc in chunks:
        rows = start + T
        kf = orc.f16_bits_to_f32(kc).reshape(rows, -1)
        vf = orc.f16_bits_to_f32(vc).reshape(rows, -1)
        qf = orc.f16_bits_to_f32(qb).reshape(T, -1)
        for t in range(T):
            seq = start + t + 1
            want = orc.attention_chain(qf[t], kf[:seq].reshape(-1), vf[:seq].reshape(-1), NQH, NKH, HD, seq, 1.0,
                                       window)
            g = got[off + t * NQH * HD: off + (t + 1) * NQH * HD]
            assert np.isfinite(g).all() and max_abs(g, want) <= 2e-3, (start, t)
        off += T * NQH * HD


@pytest.mark.skipif(NODE is None, reason="node is not installed")
@pytest.mark.parametrize("n,rows", [(1536, [2048, 256, 256]), (4096, [1536]), (2048, [7, 300, 1, 33])])
def test_linear_through_ts_host(tmp_path, n, rows):
    announce(f"TS host linear n={n} rows={rows}")
    rng = np.random.default_rng(n + len(rows))
    x = rng.standard_normal(n, dtype=np.float32)
    ws = [(rng.standard_normal((r, n), dtype=np.float32) * 0.05).astype(np.float16).view(np.uint16) for r in rows]
    arrays, blob = dict(x=[0, x.nbytes]), [x.tobytes()]
    off = x.nbytes
    for i, w in enumerate(ws):
        arrays[f"w{i}"] = [off, w.nbytes]
        blob.append(w.tobytes())
        off += w.nbytes
    (tmp_path / "case.bin").write_bytes(b"".join(blob))
    (tmp_path / "case.json").write_text(json.dumps(dict(n=n, rows=rows, arrays=arrays)))
    r = subprocess.run([NODE, str(RUN), "linear", str(tmp_path)], cwd=ROOT, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    got = np.frombuffer((tmp_path / "out.bin").read_bytes(), np.uint32)
    want = np.concatenate([orc.matmul_quant(x, w, rr, n) for w, rr in zip(ws, rows)]).view(np.uint32)
    total = sum(rows)
    np.testing.assert_array_equal(got[:total], want)
    np.testing.assert_array_equal(got[total:], want)


@pytest.mark.skipif(NODE is None, reason="node is not installed")
def test_continuous_batching_through_ts_host(tmp_path):
    """DecodeScheduler (host/scheduler.ts): sequences are submitted, admitted into three cache slots
    (FIFO, lowest free slot), released and replaced over eight token steps; steps 0 and 4 run layer by
    layer, the rest prepare at beginToken (steps 1, 2 and 5) or, where the batch is the previous token's
    (steps 3, 6 and 7), advance its plans on the host (attnStepAdvance). Each step runs every layer
    as one attnStep over the active sequences: a local head_dim-256 producer (window 40), a global
    head_dim-512 producer, and a local consumer of layer 0 that projects only q and reads the row its
    producer stored earlier in the same token. Every attnOut is checked against the oracle's decode
    chain over the cache the oracle keeps for each sequence, within max-abs 2e-3. The loop runs with the
    per-pass profiler on (a forward per token step): the report must hold one attn.decodeFused sample
    per attnStep launch, so timing changes no result."""
    announce("TS host continuous batching")
    layers = [dict(slidingWindow=40, theta=1e4, applyDivisor=0, kvSource=0, headDim=256),
              dict(slidingWindow=0, theta=1e6, applyDivisor=1, kvSource=1, headDim=512),
              dict(slidingWindow=40, theta=1e4, applyDivisor=0, kvSource=0, headDim=256)]
    max_batch, max_seq = 3, 300
    steps = [dict(release=[], submit=[["A", 100], ["B", 37], ["C", 250], ["D", 5]], admitted=["A", "B", "C"]),
             dict(release=["B"], submit=[], admitted=["D"]),
             dict(release=["A"], submit=[["E", 0]], admitted=["E"]),
             dict(release=[], submit=[], admitted=[]),
             dict(release=["D"], submit=[["F", 60]], admitted=["F"]),
             dict(release=[], submit=[], admitted=[]),
             dict(release=[], submit=[], admitted=[]),
             dict(release=[], submit=[], admitted=[])]
    arrays, blob = {}, bytearray()

    def put(name, a):
        b = np.ascontiguousarray(a).tobytes()
        arrays[name] = [len(blob), len(b)]
        blob.extend(b)

    put("rf", ROPE)
    qw = [f16_weight_bits(900 + l, L["headDim"]) for l, L in enumerate(layers)]
    kw = [f16_weight_bits(950 + l, L["headDim"]) for l, L in enumerate(layers)]
    for l in range(len(layers)):
        put(f"qw{l}", qw[l])
        put(f"kw{l}", kw[l])
    producers = [l for l, L in enumerate(layers) if L["kvSource"] == l]
    cache, length, active, waiting, expected = {}, {}, [], [], []
    seed = 1000
    for si, st in enumerate(steps):
        for sid in st["release"]:
            active.remove(sid)
        waiting += st["submit"]
        admitted = []
        while waiting and len(active) < max_batch:
            sid, n = waiting.pop(0)
            active.append(sid)
            admitted.append(sid)
            length[sid] = n
            for p in producers:
                hd = layers[p]["headDim"]
                kc = np.zeros((max_seq, NKH * hd), np.uint16)
                vc = np.zeros((max_seq, NKH * hd), np.uint16)
                if n:
                    kc[:n] = cache_f16(seed, n, NKH, hd).reshape(n, -1)
                    vc[:n] = cache_f16(seed + 1, n, NKH, hd).reshape(n, -1)
                seed += 2
                cache[(sid, p)] = [kc, vc]
                put(f"kc:{sid}:{p}", kc[:n])
                put(f"vc:{sid}:{p}", vc[:n])
        assert admitted == st["admitted"]
        for l, L in enumerate(layers):
            hd, src = L["headDim"], L["kvSource"]
            for sid in active:
                pos = length[sid]
                q = synth.normal(seed, NQH * hd) * 2.0
                k = synth.normal(seed + 1, NKH * hd) * 2.0
                v = synth.normal(seed + 2, NKH * hd) * 2.0
                seed += 3
                put(f"q:{si}:{sid}:{l}", q)
                if src == l:
                    put(f"k:{si}:{sid}:{l}", k)
                    put(f"v:{si}:{sid}:{l}", v)
                    k_ = orc.fused_per_head_norm_rope(k, kw[l], ROPE, NKH, hd, EPS, pos, L["theta"], L["applyDivisor"])
                    v_ = orc.per_head_rms_norm_no_weight(v, NKH, hd, EPS)
                    cache[(sid, l)][0][pos] = orc.f32_to_f16_bits(k_)
                    cache[(sid, l)][1][pos] = orc.f32_to_f16_bits(v_)
                q_ = orc.fused_per_head_norm_rope(q, qw[l], ROPE, NQH, hd, EPS, pos, L["theta"], L["applyDivisor"])
                kc, vc = cache[(sid, src)]
                seq = pos + 1
                out = orc.attention_chain(q_, orc.f16_bits_to_f32(kc[:seq]).reshape(-1),
                                          orc.f16_bits_to_f32(vc[:seq]).reshape(-1), NQH, NKH, hd, seq, 1.0,
                                          L["slidingWindow"])
                expected.append((si, l, sid, out))
        for sid in active:
            length[sid] += 1
    (tmp_path / "case.bin").write_bytes(bytes(blob))
    (tmp_path / "case.json").write_text(json.dumps(dict(nqh=NQH, nkh=NKH, hd=256, maxBatch=max_batch,
                                                        maxSeqLen=max_seq, eps=EPS, layers=layers, steps=steps,
                                                        arrays=arrays)))
    r = subprocess.run([NODE, str(RUN), "batch", str(tmp_path)], cwd=ROOT, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    got = np.frombuffer((tmp_path / "out.bin").read_bytes(), np.float32)
    off, worst = 0, 0.0
    for si, l, sid, want in expected:
        g = got[off:off + want.size]
        off += want.size
        err = max_abs(g, want)
        worst = max(worst, err)
        assert np.isfinite(g).all() and err <= 2e-3, (si, l, sid, err)
    assert off == got.size
    assert "beginToken: 3 prepared, 3 advanced" in r.stdout, r.stdout
    print(f"continuous batching: {len(expected)} outputs, worst max-abs {worst:.2e}")


@pytest.mark.skipif(NODE is None, reason="node is not installed")
def test_promise_readback_through_ts_host(tmp_path):
    """readBufferAsync (mapAsync's shape): the copy is ordered where it was issued, so the values read
    before a later clearBuffer are the soft-capped ones (bit-identical to the oracle), and those read
    after it are zeros; a read past the end rejects."""
    announce("TS host promise readback")
    x = np.random.default_rng(4).standard_normal(300000, dtype=np.float32) * 400.0
    (tmp_path / "case.bin").write_bytes(x.tobytes())
    r = subprocess.run([NODE, str(RUN), "readback", str(tmp_path)], cwd=ROOT, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    assert '"ok":true' in r.stdout
    got = np.frombuffer((tmp_path / "out.bin").read_bytes(), np.uint32)
    np.testing.assert_array_equal(got[:x.size], orc.logit_softcap(x, 30.0).view(np.uint32))
    assert not got[x.size:].any()


@pytest.mark.skipif(NODE is None, reason="node is not installed")
@pytest.mark.parametrize("fmt", ["q8", "q4k"])
def test_quantized_linear_through_ts_host(tmp_path, fmt):
    """The engine's matmulQ8 / matmulQ4K dispatches (one per matrix) and one linearQuant call, both
    bit-identical to the oracle."""
    announce(f"TS host linear {fmt}")
    n, rows = 1536, [2048, 256, 256]
    rng = np.random.default_rng(41)
    x = rng.standard_normal(n, dtype=np.float32)
    arrays, blob, wants = dict(x=[0, x.nbytes]), [x.tobytes()], []
    off = x.nbytes
    for i, r in enumerate(rows):
        if fmt == "q8":
            w = rng.integers(-128, 128, size=(r, n)).astype(np.int8)
            m = (rng.random((r, n // 32)) * 0.002 + 1e-4).astype(np.float16).view(np.uint16)
            wants.append(orc.matmul_q8(x, w, m, r, n))
        else:
            nib = rng.integers(0, 16, size=(r * n // 8, 8)).astype(np.uint32)
            w = (nib << (4 * np.arange(8, dtype=np.uint32))).sum(axis=1, dtype=np.uint64).astype(np.uint32)
            m = np.concatenate([(rng.random((r, n // 256, 8)) * 0.01).astype(np.float16),
                                (rng.standard_normal((r, n // 256, 8)) * 0.05).astype(np.float16)], axis=2).view(np.uint16)
            wants.append(orc.matmul_q4k(x, w, m, r, n))
        for name, a in ((f"w{i}", w), (f"m{i}", m)):
            b = np.ascontiguousarray(a).tobytes()
            arrays[name] = [off, len(b)]
            blob.append(b)
            off += len(b)
    (tmp_path / "case.bin").write_bytes(b"".join(blob))
    (tmp_path / "case.json").write_text(json.dumps(dict(n=n, rows=rows, format=fmt, arrays=arrays)))
    r = subprocess.run([NODE, str(RUN), "linear", str(tmp_path)], cwd=ROOT, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    got = np.frombuffer((tmp_path / "out.bin").read_bytes(), np.uint32)
    want = np.concatenate(wants).view(np.uint32)
    total = sum(rows)
    np.testing.assert_array_equal(got[:total], want)
    np.testing.assert_array_equal(got[total:], want)


@pytest.mark.skipif(NODE is None, reason="node is not installed")
@pytest.mark.parametrize("start,T,hd,theta,div,vt", [(0, 64, 256, 1e4, 0, False), (5000, 33, 512, 1e6, 1, False),
                                                     (1000, 77, 256, 1e6, 1, True)])
def test_prompt_prep_through_ts_host(tmp_path, start, T, hd, theta, div, vt):
    """HipAttention.attnPromptPrep over the addon: q_out and the stored K/V rows bit-identical to the oracle's
    per-token fused_per_head_norm_rope / per_head_rms_norm_no_weight rounded to f16; other rows untouched.
    With a vtCache: the V^T blocks hold the stored V rows (the rest of the last block 0), and attnPrefill
    of the chunk reading V from them matches the oracle's decode chain within 2e-3."""
    announce(f"TS host attnPromptPrep start={start} T={T} hd={hd} vt={vt}")
    seed = 300 + start + T
    rows = start + T + 2
    arrs = {"q": synth.normal(seed, T * NQH * hd), "k": synth.normal(seed + 1, T * NKH * hd),
            "v": synth.normal(seed + 2, T * NKH * hd), "qw": f16_weight_bits(seed + 3, hd),
            "kw": f16_weight_bits(seed + 4, hd), "rf": ROPE}
    blob, index = bytearray(), {}
    for name, a in arrs.items():
        b = np.ascontiguousarray(a).tobytes()
        index[name] = [len(blob), len(b)]
        blob += b
    (tmp_path / "case.bin").write_bytes(bytes(blob))
    (tmp_path / "case.json").write_text(json.dumps(dict(nqh=NQH, nkh=NKH, hd=hd, start=start, nTokens=T,
                                                        theta=theta, div=div, rows=rows, vt=vt, arrays=index)))
    r = subprocess.run([NODE, str(RUN), "promptprep", str(tmp_path)], cwd=ROOT, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    raw_bytes = (tmp_path / "out.bin").read_bytes()
    raw = np.frombuffer(raw_bytes, np.uint16)
    nq = T * NQH * hd
    nc = rows * NKH * hd
    q_out = raw[:nq].reshape(T, NQH * hd)
    kc = raw[nq:nq + nc].reshape(rows, NKH * hd)
    vc = raw[nq + nc:nq + 2 * nc].reshape(rows, NKH * hd)
    if vt:
        nb = (rows + 31) // 32
        vtb = raw[nq + 2 * nc:nq + 2 * nc + nb * 32 * hd].reshape(nb, hd, 32)
        want_vt = np.zeros((nb, hd, 32), np.uint16)  # allocated zeroed; the prep writes the chunk's rows
        for r_ in range(start, start + T):
            want_vt[r_ // 32, :, r_ % 32] = vc[r_]
        np.testing.assert_array_equal(vtb, want_vt, err_msg="V^T blocks")
        out = np.frombuffer(raw_bytes[2 * (nq + 2 * nc + nb * 32 * hd):], np.float32).reshape(T, NQH * hd)
        kf = orc.f16_bits_to_f32(kc).reshape(rows, hd)
        vf = orc.f16_bits_to_f32(vc).reshape(rows, hd)
        for t in range(0, T, 4):
            pos = start + t
            qf = orc.f16_bits_to_f32(q_out[t])
            want = orc.attention_chain(qf, kf[:pos + 1].reshape(-1), vf[:pos + 1].reshape(-1), NQH, NKH, hd, pos + 1,
                                       1.0, 0)
            assert max_abs(out[t], want) <= 2e-3, t
    for t in range(T):
        pos = start + t
        q_ = orc.fused_per_head_norm_rope(arrs["q"][t * NQH * hd:(t + 1) * NQH * hd], arrs["qw"], ROPE, NQH, hd, EPS,
                                          pos, theta, div)
        k_ = orc.fused_per_head_norm_rope(arrs["k"][t * NKH * hd:(t + 1) * NKH * hd], arrs["kw"], ROPE, NKH, hd, EPS,
                                          pos, theta, div)
        v_ = orc.per_head_rms_norm_no_weight(arrs["v"][t * NKH * hd:(t + 1) * NKH * hd], NKH, hd, EPS)
        np.testing.assert_array_equal(q_out[t], orc.f32_to_f16_bits(q_), err_msg=f"q token {t}")
        np.testing.assert_array_equal(kc[pos], orc.f32_to_f16_bits(k_), err_msg=f"k token {t}")
        np.testing.assert_array_equal(vc[pos], orc.f32_to_f16_bits(v_), err_msg=f"v token {t}")
    assert (kc[:start] == 0).all() and (kc[start + T:] == 0).all() and (vc[:start] == 0).all()


@pytest.mark.skipif(NODE is None, reason="node is not installed")
def test_profiler_through_ts_host(tmp_path):
    """Per-pass GPU timing in the TS host (enableProfile / collectProfileSamples / getProfileReport,
    src/engine.ts:3085-3288): labels and sample counts per forward, each pass's p50 at least its bytes at
    the 8 TB/s HBM peak, a forward enqueued while the previous one resolves, the overflow flag, and no
    timing while profiling is off (the checks run in host/selftest.ts)."""
    announce("TS host per-pass profiler")
    r = subprocess.run([NODE, str(RUN), "profile", str(tmp_path)], cwd=ROOT, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    assert '"ok":true' in r.stdout
    print(r.stdout.strip())


@pytest.mark.skipif(NODE is None, reason="node is not installed")
def test_linear_qkv_prep_through_ts_host(tmp_path):
    """HipAttention.linearQkvPrep over the addon (the q/k/v projection with the norms, RoPE and K/V store as
    its epilogue), then attnStep on the ready q with the row read from the cache: q, k, v and the stored row
    bit-identical to the oracle's matmulQuant followed by the reference prep kernels; attnOut within 2e-3."""
    announce("TS host linearQkvPrep -> attnStep(qReady)")
    n, hd, theta, div, seq = 1536, 256, 1e6, 1, 300
    pos = seq - 1
    rng = np.random.default_rng(61)
    x = rng.standard_normal(n, dtype=np.float32)
    w = [(rng.standard_normal((r, n), dtype=np.float32) * 0.05).astype(np.float16).view(np.uint16)
         for r in (NQH * hd, NKH * hd, NKH * hd)]
    qw, kw = f16_weight_bits(62, hd), f16_weight_bits(63, hd)
    kc = np.zeros((seq, NKH * hd), np.uint16)
    vc = np.zeros((seq, NKH * hd), np.uint16)
    kc[:pos] = cache_f16(64, pos, NKH, hd).reshape(pos, -1)
    vc[:pos] = cache_f16(65, pos, NKH, hd).reshape(pos, -1)
    arrs = {"x": x, "w0": w[0], "w1": w[1], "w2": w[2], "qw": qw, "kw": kw, "rf": ROPE, "kc": kc, "vc": vc}
    blob, index = bytearray(), {}
    for name, a in arrs.items():
        b = np.ascontiguousarray(a).tobytes()
        index[name] = [len(blob), len(b)]
        blob += b
    (tmp_path / "case.bin").write_bytes(bytes(blob))
    (tmp_path / "case.json").write_text(json.dumps(dict(n=n, nqh=NQH, nkh=NKH, hd=hd, position=pos, slot=pos, rows=seq,
                                                        theta=theta, div=div, seq=seq, arrays=index)))
    r = subprocess.run([NODE, str(RUN), "qkvprep", str(tmp_path)], cwd=ROOT, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    raw = (tmp_path / "out.bin").read_bytes()
    sizes = [NQH * hd * 4, NKH * hd * 4, NKH * hd * 4, seq * NKH * hd * 2, seq * NKH * hd * 2, NQH * hd * 4]
    parts, off = [], 0
    for sz in sizes:
        parts.append(raw[off:off + sz])
        off += sz
    q, k, v = (np.frombuffer(p_, np.float32) for p_ in parts[:3])
    gkc, gvc = (np.frombuffer(p_, np.uint16).reshape(seq, -1) for p_ in parts[3:5])
    out = np.frombuffer(parts[5], np.float32)
    want_q = orc.fused_per_head_norm_rope(orc.matmul_quant(x, w[0], NQH * hd, n), qw, ROPE, NQH, hd, EPS, pos,
                                          theta, div)
    want_k = orc.fused_per_head_norm_rope(orc.matmul_quant(x, w[1], NKH * hd, n), kw, ROPE, NKH, hd, EPS, pos,
                                          theta, div)
    want_v = orc.per_head_rms_norm_no_weight(orc.matmul_quant(x, w[2], NKH * hd, n), NKH, hd, EPS)
    np.testing.assert_array_equal(q.view(np.uint32), want_q.view(np.uint32))
    np.testing.assert_array_equal(k.view(np.uint32), want_k.view(np.uint32))
    np.testing.assert_array_equal(v.view(np.uint32), want_v.view(np.uint32))
    np.testing.assert_array_equal(gkc[pos], orc.f32_to_f16_bits(want_k))
    np.testing.assert_array_equal(gvc[pos], orc.f32_to_f16_bits(want_v))
    np.testing.assert_array_equal(gkc[:pos], kc[:pos])
    want = orc.attention_chain(want_q, orc.f16_bits_to_f32(gkc).reshape(-1), orc.f16_bits_to_f32(gvc).reshape(-1),
                               NQH, NKH, hd, seq, 1.0, 0)
    assert max_abs(out, want) <= 2e-3


@pytest.mark.skipif(NODE is None, reason="node is not installed")
def test_capture_points_through_ts_host(tmp_path):
    """HipAttention.captureAttention (captureHidden's per-layer stop points, src/engine.ts:2053-2095,
    2749-2815) on the fused kernels: for a KV-producer layer preRopeQ/K/V are the oracle's matmulQuant rows,
    postRopeQ/K its fused_per_head_norm_rope over them (bit-identical), attnOut within 2e-3 of its chain; a
    consumer layer's postRopeQ and attnOut over the producer's caches likewise, its postRopeK refused."""
    announce("TS host captureAttention")
    n, hd, theta, div, seq = 1536, 256, 1e4, 0, 700
    pos = seq - 1
    rng = np.random.default_rng(71)
    x = rng.standard_normal(n, dtype=np.float32)
    w = [(rng.standard_normal((r, n), dtype=np.float32) * 0.05).astype(np.float16).view(np.uint16)
         for r in (NQH * hd, NKH * hd, NKH * hd)]
    cw = (rng.standard_normal((NQH * hd, n), dtype=np.float32) * 0.05).astype(np.float16).view(np.uint16)
    qw, kw, cqw = f16_weight_bits(72, hd), f16_weight_bits(73, hd), f16_weight_bits(74, hd)
    kc = np.zeros((seq, NKH * hd), np.uint16)
    vc = np.zeros((seq, NKH * hd), np.uint16)
    kc[:pos] = cache_f16(75, pos, NKH, hd).reshape(pos, -1)
    vc[:pos] = cache_f16(76, pos, NKH, hd).reshape(pos, -1)
    arrs = {"x": x, "w0": w[0], "w1": w[1], "w2": w[2], "cw0": cw, "qw": qw, "kw": kw, "cqw": cqw, "rf": ROPE,
            "kc": kc, "vc": vc}
    blob, index = bytearray(), {}
    for name, a in arrs.items():
        b = np.ascontiguousarray(a).tobytes()
        index[name] = [len(blob), len(b)]
        blob += b
    (tmp_path / "case.bin").write_bytes(bytes(blob))
    (tmp_path / "case.json").write_text(json.dumps(dict(n=n, nqh=NQH, nkh=NKH, hd=hd, position=pos, slot=pos, rows=seq,
                                                        theta=theta, div=div, seq=seq, arrays=index)))
    r = subprocess.run([NODE, str(RUN), "capture", str(tmp_path)], cwd=ROOT, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    assert '"ok":true' in r.stdout
    raw = (tmp_path / "out.bin").read_bytes()
    qn, kn = NQH * hd, NKH * hd
    sizes = [qn * 4, kn * 4, kn * 4, qn * 4, kn * 4, qn * 4, qn * 4, qn * 4, seq * kn * 2, seq * kn * 2]
    parts, off = [], 0
    for sz in sizes:
        parts.append(raw[off:off + sz])
        off += sz
    f = [np.frombuffer(p_, np.float32) for p_ in parts[:8]]
    gkc, gvc = (np.frombuffer(p_, np.uint16).reshape(seq, -1) for p_ in parts[8:])
    pre = [orc.matmul_quant(x, w[i], rr, n) for i, rr in enumerate((qn, kn, kn))]
    for i, name in enumerate(("preRopeQ", "preRopeK", "preRopeV")):
        np.testing.assert_array_equal(f[i].view(np.uint32), pre[i].view(np.uint32), err_msg=name)
    want_q = orc.fused_per_head_norm_rope(pre[0], qw, ROPE, NQH, hd, EPS, pos, theta, div)
    want_k = orc.fused_per_head_norm_rope(pre[1], kw, ROPE, NKH, hd, EPS, pos, theta, div)
    want_v = orc.per_head_rms_norm_no_weight(pre[2], NKH, hd, EPS)
    np.testing.assert_array_equal(f[3].view(np.uint32), want_q.view(np.uint32), err_msg="postRopeQ")
    np.testing.assert_array_equal(f[4].view(np.uint32), want_k.view(np.uint32), err_msg="postRopeK")
    np.testing.assert_array_equal(gkc[pos], orc.f32_to_f16_bits(want_k))
    np.testing.assert_array_equal(gvc[pos], orc.f32_to_f16_bits(want_v))
    kb, vb = orc.f16_bits_to_f32(gkc).reshape(-1), orc.f16_bits_to_f32(gvc).reshape(-1)
    assert max_abs(f[5], orc.attention_chain(want_q, kb, vb, NQH, NKH, hd, seq, 1.0, 0)) <= 2e-3
    cq = orc.fused_per_head_norm_rope(orc.matmul_quant(x, cw, qn, n), cqw, ROPE, NQH, hd, EPS, pos, theta, div)
    np.testing.assert_array_equal(f[6].view(np.uint32), cq.view(np.uint32), err_msg="consumer postRopeQ")
    assert max_abs(f[7], orc.attention_chain(cq, kb, vb, NQH, NKH, hd, seq, 1.0, 0)) <= 2e-3
    print(r.stdout.strip())
