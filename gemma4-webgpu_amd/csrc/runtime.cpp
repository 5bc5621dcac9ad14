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
    hipEvent_t done = nullptr;  // recorded after the copy that last read buf (nullptr: no copy pending)
};

// Whether a slot's last copy has completed (hipEventQuery does not wait).
int slot_free(const StageSlot& s, bool* is_free) {
    *is_free = true;
    if (!s.done) return G4_OK;
    const hipError_t q = hipEventQuery(s.done);
    if (q == hipErrorNotReady) *is_free = false;
    else if (q != hipSuccess) return hip_fail(q, "stage_upload: hipEventQuery");
    return G4_OK;
}

// Process-wide spares: the buffers a slot outgrew (their copies had
// completed) and the slots of rings whose thread has ended, for any thread's
// ring to take. Past kStagePoolBytes the smallest free spares are returned to
// the runtime. Never destroyed, so rings ending at process exit can still
// hand their slots over (they make no HIP call then: the runtime may already
// be torn down).
constexpr size_t kStagePoolBytes = 64ull << 20;
struct StagePool {
    std::mutex mu;
    std::vector<StageSlot> spare;
    size_t bytes = 0;
};

StagePool& pool() {
    static StagePool* p = new StagePool();
    return *p;
}

// The calling thread's ring. A slot that outgrows its buffer takes a spare
// or a new one of at least twice the size and gives the old one to the pool.
// Past kStageRingBytes of pinned memory the ring stops growing and waits for
// its oldest copy instead, so a thread that queues far ahead of the GPU holds
// a bounded amount.
constexpr size_t kStageRingBytes = 64ull << 20;
struct StageRing {
    std::vector<StageSlot> slots;
    size_t next = 0;
    size_t bytes = 0;  // pinned bytes held by the slots
    ~StageRing() {
        StagePool& p = pool();
        std::lock_guard<std::mutex> lock(p.mu);
        for (const StageSlot& s : slots) {
            p.spare.push_back(s);
            p.bytes += s.cap;
        }
    }
};

StageRing& ring() {
    static thread_local StageRing r;
    return r;
}

// A spare slot whose copy has completed and whose buffer holds `bytes` (any
// size when bytes is 0), removed from the pool; false when there is none.
int take_spare(size_t bytes, StageSlot* out, bool* found) {
    *found = false;
    StagePool& p = pool();
    std::lock_guard<std::mutex> lock(p.mu);
    size_t best = p.spare.size();
    for (size_t i = 0; i < p.spare.size(); i++) {
        const StageSlot& c = p.spare[i];
        if (c.cap < bytes || (best < p.spare.size() && c.cap >= p.spare[best].cap)) continue;
        bool fr = false;
        if (int rc = slot_free(c, &fr)) return rc;
        if (fr) best = i;
    }
    if (best == p.spare.size()) return G4_OK;
    *out = p.spare[best];
    p.spare.erase(p.spare.begin() + best);
    p.bytes -= out->cap;
    *found = true;
    return G4_OK;
}

// A buffer whose copies have completed goes to the pool; the pool then
// returns its smallest free buffers to the runtime while it holds more than
// kStagePoolBytes.
int give_spare(void* buf, size_t cap) {
    StagePool& p = pool();
    std::lock_guard<std::mutex> lock(p.mu);
    p.spare.push_back(StageSlot{buf, cap, nullptr});
    p.bytes += cap;
    while (p.bytes > kStagePoolBytes) {
        size_t pick = p.spare.size();
        for (size_t i = 0; i < p.spare.size(); i++) {
            bool fr = false;
            if (int rc = slot_free(p.spare[i], &fr)) return rc;
            if (fr && (pick == p.spare.size() || p.spare[i].cap < p.spare[pick].cap)) pick = i;
        }
        if (pick == p.spare.size()) break;  // every spare is still read by a queued copy
        StageSlot v = p.spare[pick];
        p.spare.erase(p.spare.begin() + pick);
        p.bytes -= v.cap;
        if (v.done) G4_CHECK_HIP(hipEventDestroy(v.done));
        G4_CHECK_HIP(hipHostFree(v.buf));
    }
    return G4_OK;
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
    // A free slot: its last copy has completed. Slots are tried from the oldest use on.
    StageSlot* s = nullptr;
    const size_t n = R.slots.size();
    for (size_t i = 0; i < n && !s; i++) {
        StageSlot& c = R.slots[(R.next + i) % n];
        bool fr = false;
        if (int rc = slot_free(c, &fr)) return rc;
        if (fr) {
            s = &c;
            R.next = (R.next + i + 1) % n;
        }
    }
    if (!s && n < (size_t)kStageMaxSlots && R.bytes < kStageRingBytes) {
        StageSlot fresh;
        bool found = false;
        if (int rc = take_spare(0, &fresh, &found)) return rc;
        if (found) R.bytes += fresh.cap;
        if (!fresh.done) {
            // The host only learns from the event that the copy has read the slot: no timing, and no
            // system-scope release (an L2 write-back) behind the copy.
            G4_CHECK_HIP(hipEventCreateWithFlags(&fresh.done, hipEventDisableTiming | hipEventDisableSystemFence));
        }
        R.slots.insert(R.slots.begin() + R.next, fresh);  // the newest use sits just before `next`
        s = &R.slots[R.next];
        R.next = (R.next + 1) % R.slots.size();
    }
    if (!s) {  // every slot in flight and the ring at its limit: wait for the oldest
        s = &R.slots[R.next];
        R.next = (R.next + 1) % n;
        G4_CHECK_HIP(hipEventSynchronize(s->done));
    }
    if (s->cap < bytes) {
        // A spare that holds the table, or a new buffer. Coherent: the copy kernel's loads reach
        // host memory, not lines the GPU cached from an earlier use of the buffer.
        StageSlot sp;
        bool found = false;
        if (int rc = take_spare(bytes, &sp, &found)) return rc;
        void* buf = sp.buf;
        size_t cap = sp.cap;
        if (found) {
            if (sp.done) G4_CHECK_HIP(hipEventDestroy(sp.done));  // completed: the slot's own event stays
        } else {
            cap = bytes < 4096 ? 4096 : bytes;
            if (cap < 2 * s->cap) cap = 2 * s->cap;
            G4_CHECK_HIP(hipHostMalloc(&buf, cap, hipHostMallocCoherent));
        }
        void* old = s->buf;
        const size_t old_cap = s->cap;
        s->buf = buf;
        s->cap = cap;
        R.bytes += cap - old_cap;
        if (old)  // its last copy has completed (the slot was free)
            if (int rc = give_spare(old, old_cap)) return rc;
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
//
// The set itself records its open pass (at most one, on the thread that
// opened it) and the slot ranges being resolved, under its mutex, so that
// calls from different threads see each other: a resolve refuses slots of
// the open pass, and a pass or marker refuses slots being resolved.
struct g4_query_set {
    std::vector<hipEvent_t> ev;
    std::vector<uint8_t> written;
    std::mutex mu;
    int64_t open_slot = -1;                                 // first slot of the open pass, or -1
    std::vector<std::pair<uint32_t, uint32_t>> resolving;  // [first, end) ranges being resolved
    bool busy(uint32_t b, uint32_t e) const {              // [b, e) meets a range being resolved
        for (const auto& r : resolving)
            if (b < r.second && r.first < e) return true;
        return false;
    }
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
    {
        std::lock_guard<std::mutex> lock(p.set->mu);
        p.set->written[p.slot] = p.set->written[p.slot + 1] = 1;
    }
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
    std::lock_guard<std::mutex> lock(set->mu);
    if (set->busy(slot, slot + 1)) return fail(G4_EINVAL, "g4_query_write: slot %u is being resolved", slot);
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
    {
        std::lock_guard<std::mutex> lock(set->mu);
        if (set->open_slot >= 0) return fail(G4_EINVAL, "g4_query_begin_pass: a pass of this set is open on another thread");
        if (set->busy(slot, slot + 2))
            return fail(G4_EINVAL, "g4_query_begin_pass: slots %u, %u are being resolved", slot, slot + 1);
        set->open_slot = slot;
    }
    t_pass.set = set;
    t_pass.slot = slot;
    t_pass.started = false;
    return G4_OK;
}

int g4_query_end_pass(void) {
    if (!t_pass.set) return fail(G4_EINVAL, "g4_query_end_pass: no pass open on this thread");
    {
        std::lock_guard<std::mutex> lock(t_pass.set->mu);
        t_pass.set->open_slot = -1;
    }
    t_pass = OpenPass();
    return G4_OK;
}

int g4_query_resolve(g4_query_set* set, uint32_t first, uint32_t n_pairs, double* ns_out) {
    if (!set) return fail(G4_EINVAL, "g4_query_resolve: set is NULL");
    if (n_pairs == 0 || !ns_out) return fail(G4_EINVAL, "g4_query_resolve: n_pairs == 0 or ns_out is NULL");
    if ((uint64_t)first + 2ull * n_pairs > set->ev.size())
        return fail(G4_EINVAL, "g4_query_resolve: %u pairs from slot %u outside a set of %zu", n_pairs, first,
                    set->ev.size());
    const uint32_t end = first + 2 * n_pairs;
    std::vector<uint8_t> w;
    {
        std::lock_guard<std::mutex> lock(set->mu);
        if (set->open_slot >= 0 && (uint64_t)set->open_slot < end && first < (uint64_t)set->open_slot + 2)
            return fail(G4_EINVAL, "g4_query_resolve: a pass of this set on slots %lld, %lld is still open",
                        (long long)set->open_slot, (long long)set->open_slot + 1);
        if (set->busy(first, end)) return fail(G4_EINVAL, "g4_query_resolve: slots already being resolved");
        set->resolving.emplace_back(first, end);
        w.assign(set->written.begin() + first, set->written.begin() + end);
    }
    hipError_t err = hipSuccess;
    for (uint32_t i = 0; i < n_pairs; ++i) {  // outside the lock: passes on other slots go on meanwhile
        const uint32_t b = 2 * i, e = b + 1;
        ns_out[i] = NAN;
        if (!w[b] || !w[e] || err != hipSuccess) continue;
        float ms = 0.f;
        if ((err = hipEventSynchronize(set->ev[first + e])) != hipSuccess ||
            (err = hipEventElapsedTime(&ms, set->ev[first + b], set->ev[first + e])) != hipSuccess)
            continue;
        ns_out[i] = (double)ms * 1e6;
    }
    {
        std::lock_guard<std::mutex> lock(set->mu);
        for (uint32_t i = first; i < end; ++i) set->written[i] = 0;
        for (size_t r = 0; r < set->resolving.size(); ++r)
            if (set->resolving[r].first == first && set->resolving[r].second == end) {
                set->resolving.erase(set->resolving.begin() + r);
                break;
            }
    }
    if (err != hipSuccess) return hip_fail(err, "g4_query_resolve");
    return G4_OK;
}

int g4_query_set_destroy(g4_query_set* set) {
    if (!set) return fail(G4_EINVAL, "g4_query_set_destroy: set is NULL");
    {
        std::lock_guard<std::mutex> lock(set->mu);
        if (set->open_slot >= 0 && t_pass.set != set)
            return fail(G4_EINVAL, "g4_query_set_destroy: a pass of this set is open on another thread");
        if (!set->resolving.empty()) return fail(G4_EINVAL, "g4_query_set_destroy: slots of this set are being resolved");
    }
    if (t_pass.set == set) t_pass = OpenPass();  // this thread's own pass: closed with the set
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
