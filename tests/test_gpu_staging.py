"""GPU test of the table uploads behind the prepares: pinned staging slots read by a copy kernel on the
stream, each slot reused only once the copy that read it has completed, the ring growing while copies
are still queued (include/g4attn.h, conventions).

150 prepares are queued behind a long kernel (no slot can be reused, the ring grows), then 150 more with
short kernels between them (some slots complete and are reused while others are still queued). Every
prepare has its own workspace and output; each plan's attnOut must be bit-identical to its layer's
output from a prepare and run with the stream idle.
"""
import numpy as np
import pytest
import torch

from conftest import announce
from g4attn import ops
from test_gpu_step import Layer

pytestmark = pytest.mark.gpu

SPECS = [(40, 0, 1e4, 0), (513, 512, 1e4, 0), (700, 0, 1e6, 1), (1500, 512, 1e4, 0), (2100, 0, 1e6, 1)]
N = 150


def bits(t):
    return t.cpu().numpy().view(np.uint32)


def prepare_run(dev, L, ws, out):
    e = L.entry(inv_freq=True)
    e["out"] = out
    arr = ops.make_step_entries([e], 8, 1, 256)
    plan = ops.attn_step_prepare(arr, 8, 1, 256, ws)
    ops.attn_step_run(plan)
    return e  # keeps the host RoPE table alive until the caller drops it


def test_prepares_in_flight_reuse_no_slot_early(dev):
    announce(f"staging ring: {N} prepares behind a busy stream, {N} interleaved")
    layers = [Layer(dev, 6600 + 11 * i, *s) for i, s in enumerate(SPECS)]
    wsb = ops.step_workspace_bytes(1, 8, 1, 256)
    ref = []
    for L in layers:
        out = torch.full((8 * 256,), float("nan"), device=dev)
        prepare_run(dev, L, torch.empty(wsb, dtype=torch.uint8, device=dev), out)
        torch.cuda.synchronize()
        ref.append(bits(out))
    wss = [torch.empty(wsb, dtype=torch.uint8, device=dev) for _ in range(N)]
    for phase in range(2):
        outs = [torch.full((8 * 256,), float("nan"), device=dev) for _ in range(N)]
        keep = []
        if phase == 0:
            torch.cuda._sleep(50_000_000)  # every copy below queues behind this kernel
        for i in range(N):
            if phase == 1 and i % 10 == 0:
                torch.cuda._sleep(200_000)
            keep.append(prepare_run(dev, layers[i % len(layers)], wss[i], outs[i]))
        torch.cuda.synchronize()
        for i in range(N):
            np.testing.assert_array_equal(bits(outs[i]), ref[i % len(layers)],
                                          err_msg=f"phase {phase} prepare {i} (layer {i % len(layers)})")
        del keep


def test_rings_of_ended_threads_are_reused(dev):
    """Worker threads queue prepares behind a busy stream and end while their copies are still queued;
    their slots go to the process-wide pool, and later prepares (new threads and this one) take them
    only once those copies have completed: every plan's attnOut stays bit-identical."""
    import threading

    announce("staging ring: threads that end with copies in flight, their slots reused")
    layers = [Layer(dev, 6700 + 13 * i, *s) for i, s in enumerate(SPECS)]
    wsb = ops.step_workspace_bytes(1, 8, 1, 256)
    ref = []
    for L in layers:
        out = torch.full((8 * 256,), float("nan"), device=dev)
        prepare_run(dev, L, torch.empty(wsb, dtype=torch.uint8, device=dev), out)
        torch.cuda.synchronize()
        ref.append(bits(out))
    M = 40
    for rnd in range(3):
        wss = [torch.empty(wsb, dtype=torch.uint8, device=dev) for _ in range(2 * M)]
        outs = [torch.full((8 * 256,), float("nan"), device=dev) for _ in range(2 * M)]
        keep, errors = [], []
        torch.cuda._sleep(20_000_000)  # the workers' copies queue behind this kernel

        def work(lo, hi):
            try:
                for i in range(lo, hi):
                    keep.append(prepare_run(dev, layers[i % len(layers)], wss[i], outs[i]))
            except Exception as e:  # reported by the main thread
                errors.append(e)

        threads = [threading.Thread(target=work, args=(k * M // 2, (k + 1) * M // 2)) for k in range(2)]
        for t in threads:
            t.start()
        for t in threads:
            t.join()  # ended, its ring handed to the pool while copies may still be queued
        for i in range(M, 2 * M):  # this thread's prepares may take the ended rings' slots
            keep.append(prepare_run(dev, layers[i % len(layers)], wss[i], outs[i]))
        torch.cuda.synchronize()
        assert not errors, errors
        for i in range(2 * M):
            np.testing.assert_array_equal(bits(outs[i]), ref[i % len(layers)],
                                          err_msg=f"round {rnd} prepare {i} (layer {i % len(layers)})")
        del keep
