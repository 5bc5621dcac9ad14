"""GPU checks of the timestamp query set (g4_query_set_*; the engine's per-pass timestamp queries,
src/engine.ts:3208-3227, 3253-3288) through the C ABI.

A pass (begin_pass .. end_pass) around one 256 MiB streaming read takes the kernel's own start and end:
at least the time 256 MiB takes at the 8 TB/s HBM peak, and inside the spread of the same read timed with
events on its own dispatch (several launches, queued under the same conditions as the passes: one such
read varies by ~25% from launch to launch on one box, 39-50 us). A pass around two reads spans both
(first kernel's start to the last one's end: between 1.5x and 2.6x of one read). A pass that launched
nothing resolves to NaN. A marker pair (write) spans the work between the markers.
Slots are written again after a resolve, and misuse is refused (a second open pass, a resolve of an
open pass's set, pairs outside the set)."""
import ctypes as C
import math

import pytest
import torch

from conftest import announce
from g4attn import abi, ops

pytestmark = pytest.mark.gpu

MIB = 1 << 20


def test_pass_pairs_time_their_kernels(dev):
    announce("timestamp queries: passes around 256 MiB reads")
    buf = torch.randint(0, 256, (256 * MIB,), dtype=torch.uint8, device=dev)
    busy = torch.empty(1024 * MIB, dtype=torch.uint8, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(4)]
    for a_, b_ in evs:
        a_.record()
        b_.record()
    for _ in range(3):
        ops.read_ceiling(buf, sink)
    torch.cuda.synchronize()
    floor_ns = 256 * MIB / 8e12 * 1e9  # 256 MiB at 8 TB/s
    q = ops.QuerySet(8)
    lib = abi.load()
    try:
        for rep in range(2):  # the second round writes the resolved slots again
            ops.read_ceiling(busy, sink)  # the GPU is busy while the rest is enqueued behind it
            for a_, b_ in evs:  # the kernel's own time, for comparison: the same read, queued the same way
                ops.read_ceiling(buf, sink, a_, b_)
            q.begin_pass(0)
            ops.read_ceiling(buf, sink)
            q.end_pass()
            q.begin_pass(2)
            ops.read_ceiling(buf, sink)
            ops.read_ceiling(buf, sink)
            q.end_pass()
            q.begin_pass(4)  # launches nothing
            q.end_pass()
            q.write(6)
            ops.read_ceiling(buf, sink)
            q.write(7)
            ns = q.resolve(0, 4)
            kernel_ns = sorted(a_.elapsed_time(b_) * 1e6 for a_, b_ in evs)
            lo, hi = kernel_ns[0], kernel_ns[-1]
            print(f"round {rep}: passes {[round(x) if not math.isnan(x) else x for x in ns]} ns, "
                  f"kernel {[round(x) for x in kernel_ns]} ns")
            one, two, empty, marked = ns
            assert one >= floor_ns and 0.75 * lo <= one <= 1.3 * hi, (one, kernel_ns)
            assert two >= 2 * floor_ns and 1.5 * lo <= two <= 2.6 * hi, (two, kernel_ns)
            assert math.isnan(empty), empty
            assert marked >= floor_ns and marked >= 0.75 * lo, (marked, kernel_ns)
        q.begin_pass(0)
        st = lib.g4_query_begin_pass(q.handle, 2)
        assert st == abi.G4_EINVAL and "already open" in lib.g4_last_error().decode()
        out = (C.c_double * 4)()
        st = lib.g4_query_resolve(q.handle, 0, 1, out)
        assert st == abi.G4_EINVAL and "still open" in lib.g4_last_error().decode()
        q.end_pass()
        st = lib.g4_query_resolve(q.handle, 6, 2, out)
        assert st == abi.G4_EINVAL and "outside" in lib.g4_last_error().decode()
        st = lib.g4_query_begin_pass(q.handle, 7)
        assert st == abi.G4_EINVAL and "outside" in lib.g4_last_error().decode()
        st = lib.g4_query_write(q.handle, 8, None)
        assert st == abi.G4_EINVAL and "outside" in lib.g4_last_error().decode()
    finally:
        q.close()


def test_open_pass_seen_from_other_threads(dev):
    """A pass opened on one thread is seen by calls from another: a resolve of its slots, a second pass
    on the set and the set's destroy are refused there, while a resolve of other slots goes on."""
    import threading

    announce("timestamp queries: a pass open on another thread")
    q = ops.QuerySet(8)
    lib = abi.load()
    opened, release, done = threading.Event(), threading.Event(), threading.Event()
    errors = []

    def holder():
        try:
            q.begin_pass(2)
            opened.set()
            release.wait(30)
            q.end_pass()
        except Exception as e:  # reported by the main thread
            errors.append(e)
        finally:
            opened.set()
            done.set()

    t = threading.Thread(target=holder)
    t.start()
    try:
        assert opened.wait(30) and not errors, errors
        out = (C.c_double * 4)()
        st = lib.g4_query_resolve(q.handle, 2, 1, out)
        assert st == abi.G4_EINVAL and "still open" in lib.g4_last_error().decode()
        st = lib.g4_query_resolve(q.handle, 0, 2, out)  # slots 0..3 meet the pass's 2, 3
        assert st == abi.G4_EINVAL and "still open" in lib.g4_last_error().decode()
        assert math.isnan(q.resolve(4, 2)[0])  # other slots: nothing written, NaN
        st = lib.g4_query_begin_pass(q.handle, 6)
        assert st == abi.G4_EINVAL and "another thread" in lib.g4_last_error().decode()
        st = lib.g4_query_set_destroy(q.handle)
        assert st == abi.G4_EINVAL and "another thread" in lib.g4_last_error().decode()
    finally:
        release.set()
        done.wait(30)
        t.join(30)
    assert not errors, errors
    assert math.isnan(q.resolve(2, 1)[0])  # closed, and it launched nothing
    q.begin_pass(6)  # free again
    q.end_pass()
    q.close()
