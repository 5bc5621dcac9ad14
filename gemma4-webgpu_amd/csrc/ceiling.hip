// Read-stream ceiling of the device: the bandwidth a plain streaming read
// reaches on this GPU, measured next to each roofline so that a kernel's
// achieved bandwidth can be stated against the spec sheet and against what
// the memory system actually delivers. Every lane reads 16-byte words with
// nontemporal loads (the decode kernels' load form), grid-stride, and folds
// them into one word per lane that is stored only when it matches a value
// no input produces, so the loads cannot be dropped and nothing is written.
#include <hip/hip_ext.h>

#include "common.h"

namespace g4 {

__global__ __launch_bounds__(256) void k_read_ceiling(const u32x4* __restrict__ src, uint64_t n, uint32_t* sink) {
    typedef const __attribute__((address_space(1))) u32x4* gp;
    u32x4 acc = {0u, 0u, 0u, 0u};
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    constexpr int U = 8;  // loads in flight per lane
    for (; i + (U - 1) * stride < n; i += U * stride) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = __builtin_nontemporal_load((gp)(src + i + u * stride));
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u];
    }
    for (; i < n; i += stride) acc ^= __builtin_nontemporal_load((gp)(src + i));
    const uint32_t r = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    if (r == 0x9E3779B9u && threadIdx.x == 0) stg<uint32_t>(sink, r);
}

}  // namespace g4

using namespace g4;

extern "C" {

int g4_read_ceiling(const void* buf, size_t bytes, uint32_t* sink, void* stream, void* start_event, void* stop_event) {
    if (!buf || !sink) return fail(G4_EINVAL, "readCeiling: NULL pointer");
    if (bytes < 16 || (reinterpret_cast<uintptr_t>(buf) & 15))
        return fail(G4_EINVAL, "readCeiling: buffer must be 16-byte aligned and at least 16 bytes");
    // 32 workgroups of 4 waves per CU, 8 loads in flight per lane: the best of a sweep over
    // 4 .. 64 workgroups per CU and 4 .. 16 loads per lane (6.5 TB/s on a 2 GiB buffer).
    const dim3 grid(256 * 32), block(256);
    hipStream_t st = as_stream(stream);
    const u32x4* src = static_cast<const u32x4*>(buf);
    if (start_event || stop_event)
        hipExtLaunchKernelGGL(k_read_ceiling, grid, block, 0, st, static_cast<hipEvent_t>(start_event),
                              static_cast<hipEvent_t>(stop_event), 0, src, (uint64_t)(bytes / 16), sink);
    else
        G4_LAUNCH(k_read_ceiling, grid, block, 0, st, src, (uint64_t)(bytes / 16), sink);
    G4_CHECK_LAUNCH("readCeiling");
    return G4_OK;
}

}  // extern "C"
