// Shared helpers for the gfx950 attention library: status handling, f16
// vector types, lane helpers. Every kernel in this library is written for
// CDNA4 wave64; nothing here is portable to other targets by design.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/g4attn.h"
#include "tables.h"

namespace g4 {

// ---- status ----------------------------------------------------------------

// Records `msg` as this thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t e, const char* what);

#define G4_CHECK_HIP(expr)                                 \
    do {                                                   \
        hipError_t e_ = (expr);                            \
        if (e_ != hipSuccess) return ::g4::hip_fail(e_, #expr); \
    } while (0)

// After a kernel launch: reports launch-configuration errors synchronously.
#define G4_CHECK_LAUNCH(name)                              \
    do {                                                   \
        hipError_t e_ = hipGetLastError();                 \
        if (e_ != hipSuccess) return ::g4::hip_fail(e_, name); \
    } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Per-pass timing: while the calling thread has a pass open
// (g4_query_begin_pass), every kernel the library launches takes the pass's
// events on its own dispatch (the first kernel the begin event, at its start;
// each kernel the end event, at its end, so the last one's end stands), so no
// marker packet sits between kernels. pass_events returns false when no pass
// is open.
bool pass_events(hipEvent_t* start, hipEvent_t* stop);

#define G4_LAUNCH(K, GRID, BLOCK, SHM, ST, ...)                                         \
    do {                                                                                \
        hipEvent_t g4_ps_ = nullptr, g4_pe_ = nullptr;                                  \
        if (::g4::pass_events(&g4_ps_, &g4_pe_))                                        \
            hipExtLaunchKernelGGL(K, GRID, BLOCK, SHM, ST, g4_ps_, g4_pe_, 0, __VA_ARGS__); \
        else                                                                            \
            hipLaunchKernelGGL(K, GRID, BLOCK, SHM, ST, __VA_ARGS__);                   \
    } while (0)

// Host -> device upload of a prepared table, ordered on `st`, through pinned
// staging memory from a per-thread ring of slots, copied by a kernel on `st`
// (16-byte aligned dst; otherwise by the copy engine). A slot is reused only once
// the copy that last read it has completed; when every slot is still in flight
// the ring grows (up to kStageMaxSlots slots and 64 MiB of pinned memory, past
// which the oldest slot is waited for), so enqueueing rarely waits on the GPU.
// Buffers a slot outgrew, and the rings of threads that have ended, go to a
// process-wide pool that every thread's ring takes from first.
constexpr int kStageMaxSlots = 4096;
int stage_upload(void* dst, const void* src, size_t bytes, hipStream_t st);
// Slots currently held by the calling thread's ring (for tests).
int stage_slots();

// Compute units of the current device (queried once per device).
unsigned device_cus();

// ---- types -----------------------------------------------------------------

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Loads and stores through the global address space (global_load/store with
// an SGPR base), for pointers the compiler cannot prove global by itself.
template <typename T>
__device__ __forceinline__ T ldg(const void* p) {
    typedef const __attribute__((address_space(1))) T* gp;
    return *(gp)(p);
}
template <typename T>
__device__ __forceinline__ void stg(void* p, T v) {
    typedef __attribute__((address_space(1))) T* gp;
    *(gp)(p) = v;
}

__device__ __forceinline__ float h2f(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(f16, h));
}
__device__ __forceinline__ uint16_t f2h(float f) {  // round to nearest even
    return __builtin_bit_cast(uint16_t, static_cast<f16>(f));
}

}  // namespace g4
