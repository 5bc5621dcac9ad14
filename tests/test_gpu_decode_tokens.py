"""GPU parity of consecutive decode tokens through the per-token prepare, as a decode loop issues them:
each token is prepared at the next position (seq_len and position one further, src/engine.ts:1967-1987)
and run, its K/V rows are stored by the step, and the tokens after it attend them. Two forms: the stack
(one g4_attn_step_prepare over every layer per token, then the step) and the engine's layer order (one
g4_attn_step_prepare_layers per token, then each layer's plan in turn).

Bars, per token and layer: the stored K and V rows bit-identical to the oracle's norm (+ RoPE) of the
token's raw k and v rounded to f16, and attnOut within max-abs 2e-3 of the oracle's reference chain over
the cache as it stands (the earlier rows as generated, the tokens' rows as the oracle computes them).
Windows of 40 and 512 rows on the local layers, so that a local layer's window slides past the rows
the earlier tokens stored.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from g4attn import e2b, ops, synth
from helpers import EPS, cache_f16_torch, f16_weight_bits
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

NQH, NKH, HD = 8, 1, 256
TOL = 2e-3
ROPE = np.array(e2b.rope_freqs_f16_bits(256), dtype=np.uint16)
T = 4  # tokens


def t16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)


class Layer:
    """A layer's cache (rows 0 .. s0-2 generated, room for T more), weights and per-token raw projections."""

    def __init__(self, dev, seed, s0, window, theta, div, tabs):
        self.s0, self.window, self.theta, self.div = s0, window, theta, div
        self.seed = seed
        rows = s0 - 1 + T
        self.kc = cache_f16_torch(seed + 5, rows, NKH, HD, dev).view(torch.int16).reshape(rows, NKH * HD).contiguous()
        self.vc = cache_f16_torch(seed + 6, rows, NKH, HD, dev).view(torch.int16).reshape(rows, NKH * HD).contiguous()
        self.kb = self.kc.cpu().numpy().view(np.uint16).copy()  # the oracle's copy of the cache
        self.vb = self.vc.cpu().numpy().view(np.uint16).copy()
        self.qw, self.kw = f16_weight_bits(seed + 3, HD), f16_weight_bits(seed + 4, HD)
        self.dqw, self.dkw, self.drf = t16(self.qw, dev), t16(self.kw, dev), t16(ROPE, dev)
        self.dq = torch.empty(NQH * HD, device=dev)
        self.dk = torch.empty(NKH * HD, device=dev)
        self.dv = torch.empty(NKH * HD, device=dev)
        self.out = torch.empty(NQH * HD, device=dev)
        self.inv = tabs.get((theta, div))

    def token(self, t):
        """The raw projections of token t (written to the device buffers) and its entry."""
        self.q = synth.normal(self.seed + 100 * t + 10, NQH * HD) * 2.0
        self.k = synth.normal(self.seed + 100 * t + 11, NKH * HD) * 2.0
        self.v = synth.normal(self.seed + 100 * t + 12, NKH * HD) * 2.0
        for d, h in ((self.dq, self.q), (self.dk, self.k), (self.dv, self.v)):
            d.copy_(torch.from_numpy(h))
        self.out.fill_(float("nan"))
        seq = self.s0 + t
        e = dict(q=self.dq, k=self.dk, v=self.dv, q_weight=self.dqw, k_weight=self.dkw, rope_freqs=self.drf,
                 k_cache=self.kc, v_cache=self.vc, out=self.out, seq_len=seq, position=seq - 1,
                 sliding_window=self.window, store_kv=True, theta=self.theta, apply_divisor=self.div)
        if self.inv is not None:
            e["rope_inv_freq_host"] = self.inv
        return e

    def check(self, t, label):
        seq = self.s0 + t
        pos = seq - 1
        k_ = orc.fused_per_head_norm_rope(self.k, self.kw, ROPE, NKH, HD, EPS, pos, self.theta, self.div)
        v_ = orc.per_head_rms_norm_no_weight(self.v, NKH, HD, EPS)
        q_ = orc.fused_per_head_norm_rope(self.q, self.qw, ROPE, NQH, HD, EPS, pos, self.theta, self.div)
        self.kb[pos] = orc.f32_to_f16_bits(k_)
        self.vb[pos] = orc.f32_to_f16_bits(v_)
        np.testing.assert_array_equal(self.kc[pos].cpu().numpy().view(np.uint16), self.kb[pos], err_msg=f"{label} K")
        np.testing.assert_array_equal(self.vc[pos].cpu().numpy().view(np.uint16), self.vb[pos], err_msg=f"{label} V")
        lo = seq - self.window if self.window and seq > self.window else 0
        kf = orc.f16_bits_to_f32(self.kb[lo:seq]).reshape(-1)
        vf = orc.f16_bits_to_f32(self.vb[lo:seq]).reshape(-1)
        want = orc.attention_chain(q_, kf, vf, NQH, NKH, HD, seq - lo, 1.0, 0)
        got = self.out.cpu().numpy()
        assert np.isfinite(got).all(), f"{label}: non-finite attnOut"
        err = float(np.abs(got - want).max())
        assert err <= TOL, f"{label}: attnOut max-abs {err}"


SPECS = [(38, 40, 1e4, 0), (600, 0, 1e6, 1), (520, 512, 1e4, 0), (3000, 0, 1e6, 1), (300, 40, 1e4, 0)]


@pytest.mark.parametrize("form", ["stack", "layers"])
def test_tokens_in_a_row(dev, form):
    announce(f"decode {T} tokens in a row, {form} prepare")
    tabs = {(1e4, 0): ops.rope_inv_freq_host(1e4, HD, 0, ROPE), (1e6, 1): ops.rope_inv_freq_host(1e6, HD, 1, ROPE)}
    layers = [Layer(dev, 2300 + 41 * i, s0, w, th, dv, tabs if i % 2 == 0 else {}) for i, (s0, w, th, dv)
              in enumerate(SPECS)]
    n = len(layers)
    ws = torch.empty(ops.step_workspace_bytes(n, NQH, NKH, HD) if form == "stack"
                     else ops.step_layers_workspace_bytes(n, NQH, NKH, HD), dtype=torch.uint8, device=dev)
    for t in range(T):
        arr = ops.make_step_entries([L.token(t) for L in layers], NQH, NKH, HD)
        if form == "stack":
            ops.attn_step_run(ops.attn_step_prepare(arr, NQH, NKH, HD, ws))
        else:
            for plan in ops.attn_step_prepare_layers(arr, NQH, NKH, HD, ws):
                ops.attn_step_run(plan)
        torch.cuda.synchronize()
        for i, L in enumerate(layers):
            L.check(t, f"token {t} layer {i}")
    del tabs
