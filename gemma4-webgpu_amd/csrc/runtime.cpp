// Device, stream and buffer entry points of the C ABI, and the per-thread
// error slot behind g4_last_error(). These replace the WebGPU device, queue
// and buffer calls the reference engine makes (src/engine.ts:350-353,
// 402-437, 1347-1426); buffers stay owned by the caller.
#include <math.h>
#include <stdarg.h>
#include <string.h>

#include <map>
#include <mutex>
#include <vector>

#include "common.h"

namespace g4 {

static thread_local char t_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_err, sizeof t_err, fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(G4_EHIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

namespace {

struct StageSlot {
    void* buf = nullptr;
    size_t cap = 0;
    hipEvent_t done = nullptr;  // recorded after the copy that last read buf
};

// The calling thread's ring. Slots and their pinned buffers live until the
// thread ends (they are not returned to the runtime, which may already be torn
// down when thread-local storage is destroyed at process exit). A slot that
// outgrows its buffer takes a new one of at least twice the size; the old
// buffer, which kernels have read, is kept rather than freed.
struct StageRing {
    std::vector<StageSlot> slots;
    std::vector<void*> retired;
    size_t next = 0;
};

StageRing& ring() {
    static thread_local StageRing* r = new StageRing();
    return *r;
}

// The upload itself: the GPU reads the pinned slot (mapped into its address
// space) and writes the table, 16 bytes per lane, with the last bytes one per
// lane. A kernel on the caller's stream follows the previous kernel directly;
// a copy-engine transfer would be ordered against the stream's kernels through
// signals between the engines, measured at about 20 us per upload of a 35-layer
// step table (a 6.6 us transfer plus the hand-offs either side of it).
__global__ __launch_bounds__(256) void k_stage_copy(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                    uint32_t n16, uint32_t tail) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n16) dst[i] = src[i];
    if (i < tail)
        reinterpret_cast<uint8_t*>(dst + n16)[i] = reinterpret_cast<const uint8_t*>(src + n16)[i];
}

}  // namespace

int stage_upload(void* dst, const void* src, size_t bytes, hipStream_t st) {
    if (bytes == 0) return G4_OK;
    StageRing& R = ring();
    // A free slot: never used, or its last copy has completed (hipEventQuery
    // does not wait). Slots are tried from the oldest use on.
    StageSlot* s = nullptr;
    const size_t n = R.slots.size();
    for (size_t i = 0; i < n && !s; i++) {
        StageSlot& c = R.slots[(R.next + i) % n];
        const hipError_t q = hipEventQuery(c.done);
        if (q == hipSuccess) {
            s = &c;
            R.next = (R.next + i + 1) % n;
        } else if (q != hipErrorNotReady) {
            return hip_fail(q, "stage_upload: hipEventQuery");
        }
    }
    if (!s && n < (size_t)kStageMaxSlots) {
        StageSlot fresh;
        // The host only learns from the event that the copy has read the slot: no timing, and no
        // system-scope release (an L2 write-back) behind the copy.
        G4_CHECK_HIP(hipEventCreateWithFlags(&fresh.done, hipEventDisableTiming | hipEventDisableSystemFence));
        R.slots.insert(R.slots.begin() + R.next, fresh);  // the newest use sits just before `next`
        s = &R.slots[R.next];
        R.next = (R.next + 1) % R.slots.size();
    }
    if (!s) {  // kStageMaxSlots copies in flight: wait for the oldest
        s = &R.slots[R.next];
        R.next = (R.next + 1) % n;
        G4_CHECK_HIP(hipEventSynchronize(s->done));
    }
    if (s->cap < bytes) {
        // Coherent: the copy kernel's loads reach host memory, not lines the GPU cached from an
        // earlier use of the slot.
        size_t cap = bytes < 4096 ? 4096 : bytes;
        if (cap < 2 * s->cap) cap = 2 * s->cap;
        void* buf = nullptr;
        G4_CHECK_HIP(hipHostMalloc(&buf, cap, hipHostMallocCoherent));
        if (s->buf) R.retired.push_back(s->buf);
        s->buf = buf;
        s->cap = cap;
    }
    memcpy(s->buf, src, bytes);
    if (reinterpret_cast<uintptr_t>(dst) & 15 || bytes / 16 > 0xffffffffull) {
        G4_CHECK_HIP(hipMemcpyAsync(dst, s->buf, bytes, hipMemcpyHostToDevice, st));
    } else {
        const uint32_t n16 = (uint32_t)(bytes / 16), tail = (uint32_t)(bytes % 16);
        const uint32_t lanes = n16 > tail ? n16 : tail;
        hipLaunchKernelGGL(k_stage_copy, dim3((lanes + 255) / 256), dim3(256), 0, st,
                           static_cast<const u32x4*>(s->buf), static_cast<u32x4*>(dst), n16, tail);
        G4_CHECK_LAUNCH("stage_upload");
    }
    G4_CHECK_HIP(hipEventRecord(s->done, st));
    return G4_OK;
}

int stage_slots() { return (int)ring().slots.size(); }

unsigned device_cus() {
    static std::mutex mu;
    static std::map<int, unsigned> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = -1;
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(dev);
    if (it != cache.end()) return it->second;
    int cus = 0;
    if (dev < 0 || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
        cus = 256;  // MI355X
    cache.emplace(dev, (unsigned)cus);
    return (unsigned)cus;
}

}  // namespace g4

using namespace g4;

extern "C" {

const char* g4_last_error(void) { return t_err; }

const char* g4_version(void) { return "g4attn 0.1 gfx950"; }

int g4_device_count(int* count) {
    if (!count) return fail(G4_EINVAL, "g4_device_count: count is NULL");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) n = 0;
    *count = n;
    return G4_OK;
}

int g4_set_device(int device) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(G4_ENODEV, "g4_set_device: no HIP device");
    if (device < 0 || device >= n) return fail(G4_EINVAL, "g4_set_device: device %d out of range [0,%d)", device, n);
    hipDeviceProp_t prop;
    G4_CHECK_HIP(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(G4_ENODEV, "g4_set_device: device %d is %s, this library is built for gfx950", device,
                    prop.gcnArchName);
    G4_CHECK_HIP(hipSetDevice(device));
    return G4_OK;
}

int g4_stream_create(void** stream) {
    if (!stream) return fail(G4_EINVAL, "g4_stream_create: stream is NULL");
    hipStream_t s;
    G4_CHECK_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return G4_OK;
}

int g4_stream_destroy(void* stream) {
    if (!stream) return G4_OK;
    G4_CHECK_HIP(hipStreamDestroy(as_stream(stream)));
    return G4_OK;
}

int g4_stream_synchronize(void* stream) {
    G4_CHECK_HIP(hipStreamSynchronize(as_stream(stream)));
    return G4_OK;
}

int g4_malloc(void** dev_ptr, size_t bytes) {
    if (!dev_ptr) return fail(G4_EINVAL, "g4_malloc: dev_ptr is NULL");
    if (bytes == 0) return fail(G4_EINVAL, "g4_malloc: zero bytes");
    G4_CHECK_HIP(hipMalloc(dev_ptr, bytes));
    return G4_OK;
}

int g4_free(void* dev_ptr) {
    if (!dev_ptr) return G4_OK;
    G4_CHECK_HIP(hipFree(dev_ptr));
    return G4_OK;
}

int g4_upload(void* dev_dst, size_t offset, const void* host_src, size_t bytes, void* stream) {
    if (!dev_dst || (!host_src && bytes)) return fail(G4_EINVAL, "g4_upload: NULL pointer");
    if (bytes == 0) return G4_OK;
    G4_CHECK_HIP(hipMemcpyAsync(static_cast<char*>(dev_dst) + offset, host_src, bytes, hipMemcpyHostToDevice,
                                as_stream(stream)));
    return G4_OK;
}

int g4_download(void* host_dst, const void* dev_src, size_t offset, size_t bytes, void* stream) {
    if (!host_dst || (!dev_src && bytes)) return fail(G4_EINVAL, "g4_download: NULL pointer");
    if (bytes == 0) return G4_OK;
    G4_CHECK_HIP(hipMemcpyAsync(host_dst, static_cast<const char*>(dev_src) + offset, bytes, hipMemcpyDeviceToHost,
                                as_stream(stream)));
    G4_CHECK_HIP(hipStreamSynchronize(as_stream(stream)));
    return G4_OK;
}

// Readback in two halves (the engine's copyBufferToBuffer into a staging
// buffer, then mapAsync, src/engine.ts:2309): `begin` enqueues the copy into
// pinned staging memory on the stream, so it is ordered with the work already
// enqueued there, and records an event; `finish` (from any thread) waits for
// the event, copies the bytes out and frees the staging memory.
struct g4_readback {
    void* staging;
    size_t bytes;
    hipEvent_t done;
};

int g4_readback_begin(const void* dev_src, size_t offset, size_t bytes, void* stream, g4_readback** handle) {
    if (!handle) return fail(G4_EINVAL, "g4_readback_begin: handle is NULL");
    *handle = nullptr;
    if (!dev_src || bytes == 0) return fail(G4_EINVAL, "g4_readback_begin: NULL source or zero bytes");
    g4_readback* r = new g4_readback{nullptr, bytes, nullptr};
    hipError_t e = hipHostMalloc(&r->staging, bytes, hipHostMallocDefault);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&r->done, hipEventDisableTiming);
    if (e == hipSuccess)
        e = hipMemcpyAsync(r->staging, static_cast<const char*>(dev_src) + offset, bytes, hipMemcpyDeviceToHost,
                           as_stream(stream));
    if (e == hipSuccess) e = hipEventRecord(r->done, as_stream(stream));
    if (e != hipSuccess) {
        if (r->done) (void)hipEventDestroy(r->done);
        if (r->staging) (void)hipHostFree(r->staging);
        delete r;
        return hip_fail(e, "g4_readback_begin");
    }
    *handle = r;
    return G4_OK;
}

int g4_readback_finish(g4_readback* handle, void* host_dst) {
    if (!handle) return fail(G4_EINVAL, "g4_readback_finish: handle is NULL");
    hipError_t e = hipEventSynchronize(handle->done);
    if (e == hipSuccess && host_dst) memcpy(host_dst, handle->staging, handle->bytes);
    (void)hipEventDestroy(handle->done);
    (void)hipHostFree(handle->staging);
    delete handle;
    if (e != hipSuccess) return hip_fail(e, "g4_readback_finish");
    return G4_OK;
}

}  // extern "C"

// Timestamp queries (the engine's GPUQuerySet, src/engine.ts:3089-3110,
// 3208-3227, 3253-3288): one timing event per slot, and a flag per slot that
// says it was written since the last resolve. A slot is written either by a
// marker on the stream (g4_query_write: the GPU's timestamp once the work
// before it has finished; the marker costs a few microseconds of GPU time) or
// by the kernels of an open pass (g4_query_begin_pass: the timestamps are the
// kernels' own start and end, with nothing launched between them). Markers
// release to agent scope only (no system-scope cache write-back: a timestamp
// orders nothing for the host). The events live as long as the set.
struct g4_query_set {
    std::vector<hipEvent_t> ev;
    std::vector<uint8_t> written;
};

namespace {

struct OpenPass {
    g4_query_set* set = nullptr;  // null: no pass open on this thread
    uint32_t slot = 0;
    bool started = false;
};

thread_local OpenPass t_pass;

}  // namespace

bool g4::pass_events(hipEvent_t* start, hipEvent_t* stop) {
    OpenPass& p = t_pass;
    if (!p.set) return false;
    *start = p.started ? nullptr : p.set->ev[p.slot];
    *stop = p.set->ev[p.slot + 1];
    p.set->written[p.slot] = p.set->written[p.slot + 1] = 1;
    p.started = true;
    return true;
}

extern "C" {

static const uint32_t kMaxQuerySlots = 65536;

int g4_query_set_create(uint32_t count, g4_query_set** out) {
    if (!out) return fail(G4_EINVAL, "g4_query_set_create: out is NULL");
    *out = nullptr;
    if (count == 0 || count > kMaxQuerySlots)
        return fail(G4_EINVAL, "g4_query_set_create: count %u outside 1 .. %u", count, kMaxQuerySlots);
    g4_query_set* q = new g4_query_set;
    q->ev.assign(count, nullptr);
    q->written.assign(count, 0);
    for (uint32_t i = 0; i < count; ++i) {
        const hipError_t e = hipEventCreateWithFlags(&q->ev[i], hipEventDisableSystemFence);
        if (e != hipSuccess) {
            for (uint32_t j = 0; j < i; ++j) (void)hipEventDestroy(q->ev[j]);
            delete q;
            return hip_fail(e, "g4_query_set_create: hipEventCreate");
        }
    }
    *out = q;
    return G4_OK;
}

int g4_query_write(g4_query_set* set, uint32_t slot, void* stream) {
    if (!set) return fail(G4_EINVAL, "g4_query_write: set is NULL");
    if (slot >= set->ev.size())
        return fail(G4_EINVAL, "g4_query_write: slot %u outside a set of %zu", slot, set->ev.size());
    G4_CHECK_HIP(hipEventRecord(set->ev[slot], as_stream(stream)));
    set->written[slot] = 1;
    return G4_OK;
}

int g4_query_begin_pass(g4_query_set* set, uint32_t slot) {
    if (!set) return fail(G4_EINVAL, "g4_query_begin_pass: set is NULL");
    if ((uint64_t)slot + 2 > set->ev.size())
        return fail(G4_EINVAL, "g4_query_begin_pass: slots %u, %u outside a set of %zu", slot, slot + 1,
                    set->ev.size());
    if (t_pass.set) return fail(G4_EINVAL, "g4_query_begin_pass: a pass is already open on this thread");
    t_pass.set = set;
    t_pass.slot = slot;
    t_pass.started = false;
    return G4_OK;
}

int g4_query_end_pass(void) {
    if (!t_pass.set) return fail(G4_EINVAL, "g4_query_end_pass: no pass open on this thread");
    t_pass = OpenPass();
    return G4_OK;
}

int g4_query_resolve(g4_query_set* set, uint32_t first, uint32_t n_pairs, double* ns_out) {
    if (!set) return fail(G4_EINVAL, "g4_query_resolve: set is NULL");
    if (n_pairs == 0 || !ns_out) return fail(G4_EINVAL, "g4_query_resolve: n_pairs == 0 or ns_out is NULL");
    if ((uint64_t)first + 2ull * n_pairs > set->ev.size())
        return fail(G4_EINVAL, "g4_query_resolve: %u pairs from slot %u outside a set of %zu", n_pairs, first,
                    set->ev.size());
    if (t_pass.set == set) return fail(G4_EINVAL, "g4_query_resolve: a pass of this set is still open");
    for (uint32_t i = 0; i < n_pairs; ++i) {
        const uint32_t b = first + 2 * i, e = b + 1;
        ns_out[i] = NAN;
        if (!set->written[b] || !set->written[e]) continue;
        G4_CHECK_HIP(hipEventSynchronize(set->ev[e]));
        float ms = 0.f;
        G4_CHECK_HIP(hipEventElapsedTime(&ms, set->ev[b], set->ev[e]));
        ns_out[i] = (double)ms * 1e6;
    }
    for (uint32_t i = 0; i < 2 * n_pairs; ++i) set->written[first + i] = 0;
    return G4_OK;
}

int g4_query_set_destroy(g4_query_set* set) {
    if (!set) return fail(G4_EINVAL, "g4_query_set_destroy: set is NULL");
    if (t_pass.set == set) t_pass = OpenPass();
    hipError_t first_err = hipSuccess;
    for (hipEvent_t e : set->ev) {
        const hipError_t r = hipEventDestroy(e);
        if (r != hipSuccess && first_err == hipSuccess) first_err = r;
    }
    delete set;
    if (first_err != hipSuccess) return hip_fail(first_err, "g4_query_set_destroy");
    return G4_OK;
}

}  // extern "C"
