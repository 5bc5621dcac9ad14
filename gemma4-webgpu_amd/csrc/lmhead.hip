// Greedy sampling head of a decode step: lmHead -> logitSoftcap -> argmax
// (src/engine.ts:2223-2255).
//
// Reference-shaped kernels (bit-identical to the WGSL, one per pass):
//   matmulQuant   shaders/matmul_quant.wgsl:20-52   one workgroup per row
//   matmulQ8      shaders/matmul_q8.wgsl:31-64      one workgroup per row (int8, f16 block scales)
//   matmulQ4K     shaders/matmul_q4k.wgsl:30-72     one workgroup per row (4-bit, f16 scale/min)
//   logitSoftcap  shaders/logit_softcap.wgsl:9-16
//   argmax        shaders/argmax.wgsl:7-34          one workgroup
//
// The fused path (k_lm_head + k_lm_head_pick) streams the f16 weight once
// over the whole chip. Each logit keeps matmul_quant.wgsl's summation order
// (gemv_core.h: one row per half-wave), bit-identical to the shader's.
//
// The top-1 follows argmax.wgsl: per index residue mod 256 the first strict
// maximum, then the 128 -> 1 tree, which keeps its own pair on ties. Among
// residues holding the maximum the tree's last level prefers residue bit 0
// clear, the level before bit 1, and so on, so the winner is the maximum
// holder with the smallest (bit-reversed 8-bit residue, index). That order is
// a total order on candidates, so each workgroup keeps its best candidate as
// one 64-bit key (value in the high half, order-preserving; the inverted
// tie key in the low half) and a one-workgroup pick kernel takes the largest.
// Values not above the shader's -1e30 start and NaN never become candidates;
// with none, the result is index 0, as in the shader.
#include <hip/hip_ext.h>

#include "gemv_core.h"

namespace g4 {

// ---- reference-shaped kernels ------------------------------------------------

__device__ __forceinline__ float softcap_val(float v, float cap) {  // logit_softcap.wgsl:13-15
    const float x = v / cap;
    const float c = x < -15.0f ? -15.0f : (x > 15.0f ? 15.0f : x);
    return (float)tanh((double)c) * cap;
}

__global__ __launch_bounds__(kWG) void k_matmul_quant_f16(const float* __restrict__ input,
                                                          const uint16_t* __restrict__ weight,
                                                          float* __restrict__ output, g4_matmul_params p) {
    __shared__ float partials[kWG];
    const unsigned m = blockIdx.y * gridDim.x + blockIdx.x;  // matmul_quant.wgsl:25
    if (m >= p.M) return;
    const unsigned tid = threadIdx.x;
    const uint16_t* row = weight + (uint64_t)m * p.N;
    float acc = 0.0f;
    for (unsigned k = tid; k < p.N; k += kWG) acc = acc + h2f(row[k]) * input[k];
    partials[tid] = acc;
    __syncthreads();
    const float r = wg_tree_sum(partials, tid);
    if (tid == 0) output[m] = r;
}

__global__ __launch_bounds__(kWG) void k_matmul_q8(const float* __restrict__ input, const int8_t* __restrict__ qweight,
                                                   const uint16_t* __restrict__ qscale, float* __restrict__ output,
                                                   g4_matmul_params p) {
    __shared__ float partials[kWG];
    const unsigned m = blockIdx.y * gridDim.x + blockIdx.x;
    if (m >= p.M) return;
    const unsigned tid = threadIdx.x;
    const int8_t* row = qweight + (uint64_t)m * p.N;
    const uint16_t* sc = qscale + (uint64_t)m * (p.N / 32);
    float acc = 0.0f;
    for (unsigned k = tid; k < p.N; k += kWG) {
        const float w = (float)row[k] * h2f(sc[k >> 5]);
        acc = acc + w * input[k];
    }
    partials[tid] = acc;
    __syncthreads();
    const float r = wg_tree_sum(partials, tid);
    if (tid == 0) output[m] = r;
}

__global__ __launch_bounds__(kWG) void k_matmul_q4k(const float* __restrict__ input, const uint32_t* __restrict__ qweight,
                                                    const uint16_t* __restrict__ qmeta, float* __restrict__ output,
                                                    g4_matmul_params p) {
    __shared__ float partials[kWG];
    const unsigned m = blockIdx.y * gridDim.x + blockIdx.x;
    if (m >= p.M) return;
    const unsigned tid = threadIdx.x;
    const uint64_t qbase = (uint64_t)m * p.N;
    const uint16_t* meta = qmeta + (uint64_t)m * (p.N / 256) * 16;
    float acc = 0.0f;
    for (unsigned k = tid; k < p.N; k += kWG) {
        const uint64_t fi = qbase + k;
        const unsigned nib = (qweight[fi >> 3] >> ((fi & 7) * 4)) & 15u;
        const uint16_t* mb = meta + (k >> 8) * 16;
        const unsigned sub = (k & 255u) >> 5;
        const float t = h2f(mb[sub]) * (float)nib;
        const float w = t + h2f(mb[8 + sub]);
        acc = acc + w * input[k];
    }
    partials[tid] = acc;
    __syncthreads();
    const float r = wg_tree_sum(partials, tid);
    if (tid == 0) output[m] = r;
}

__global__ __launch_bounds__(kWG) void k_logit_softcap(float* __restrict__ logits, g4_softcap_params p) {
    const unsigned i = blockIdx.x * kWG + threadIdx.x;
    if (i >= p.size) return;
    logits[i] = softcap_val(logits[i], p.cap);
}

__global__ __launch_bounds__(kWG) void k_argmax(const float* __restrict__ logits, uint32_t* __restrict__ result,
                                               uint32_t size) {
    __shared__ float smax[kWG];
    __shared__ uint32_t sidx[kWG];
    const unsigned tid = threadIdx.x;
    float local_max = -1e30f;
    uint32_t local_idx = 0;
    for (unsigned i = tid; i < size; i += kWG) {
        const float v = logits[i];
        if (v > local_max) {
            local_max = v;
            local_idx = i;
        }
    }
    smax[tid] = local_max;
    sidx[tid] = local_idx;
    __syncthreads();
    for (unsigned stride = 128; stride > 0; stride >>= 1) {
        if (tid < stride && smax[tid + stride] > smax[tid]) {
            smax[tid] = smax[tid + stride];
            sidx[tid] = sidx[tid + stride];
        }
        __syncthreads();
    }
    if (tid == 0) result[0] = sidx[0];
}

// ---- fused lm head ------------------------------------------------------------

constexpr unsigned kLmWaves = 4;       // waves per workgroup
constexpr unsigned kLmBlockRows = 64;  // rows per wave block: one logit per lane
constexpr unsigned kLmMaxWgs = 2048;   // bound of the candidate workspace
constexpr int kLmMinJ = 4, kLmMaxJ = 10;  // hidden 1024 .. 2560

__device__ __forceinline__ unsigned bitrev8(unsigned r) { return __builtin_bitreverse32(r) >> 24; }

// Candidate key of row `row` with final logit v (larger wins; 0 = none).
__device__ __forceinline__ uint64_t lm_candidate(float v, unsigned row) {
    if (!(v > -1e30f)) return 0;                             // NaN or not above the shader's start
    const uint32_t bits = __float_as_uint(v == 0.0f ? 0.0f : v);  // -0 and +0 compare equal
    const uint32_t ord = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
    const uint32_t key = (bitrev8(row & 255u) << 24) | (row >> 8);
    return ((uint64_t)ord << 32) | (uint64_t)(0xFFFFFFFFu - key);
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
    const unsigned lo = __shfl_xor((unsigned)v, m), hi = __shfl_xor((unsigned)(v >> 32), m);
    return ((uint64_t)hi << 32) | lo;
}

template <int NJ>
__global__ __launch_bounds__(kLmWaves * 64) void k_lm_head(const float* __restrict__ x,
                                                           const uint16_t* __restrict__ weight,
                                                           float* __restrict__ logits, uint64_t* __restrict__ best_out,
                                                           unsigned vocab, float cap) {
    constexpr unsigned N = NJ * 256;
    const unsigned lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const unsigned lq = lane & 31, half = lane >> 5;

    float xr[NJ][8];  // x[256 j + 8 lq + e]
    gemv_load_x<NJ>(x, lq, xr);

    uint64_t best = 0;
    const unsigned nblocks = (vocab + kLmBlockRows - 1) / kLmBlockRows;
    const unsigned n_waves = gridDim.x * kLmWaves;
    for (unsigned blk = blockIdx.x * kLmWaves + wave; blk < nblocks; blk += n_waves) {
        float val = 0.0f;
        for (unsigned pr = 0; pr < kLmBlockRows / 2; pr++) {
            const unsigned row = min(blk * kLmBlockRows + 2 * pr + half, vocab - 1);  // clamped: tail rows discarded
            const float dot = gemv_row_dot<NJ>(weight + (uint64_t)row * N, xr, lq);
            if (lq == pr) val = dot;  // lane lq of half h keeps row 2 lq + h of the block
        }
        const unsigned row = blk * kLmBlockRows + 2 * lq + half;
        const float v = cap > 0.0f ? softcap_val(val, cap) : val;
        if (row < vocab) {
            if (logits) logits[row] = v;
            best = max_u64(best, lm_candidate(v, row));
        }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) best = max_u64(best, shfl_xor_u64(best, m));
    __shared__ uint64_t wbest[kLmWaves];
    if (lane == 0) wbest[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = wbest[0];
        for (unsigned w = 1; w < kLmWaves; w++) b = max_u64(b, wbest[w]);
        best_out[blockIdx.x] = b;
    }
}

__global__ __launch_bounds__(256) void k_lm_head_pick(const uint64_t* __restrict__ best, unsigned n,
                                                      uint32_t* __restrict__ result) {
    __shared__ uint64_t wbest[4];
    uint64_t b = 0;
    for (unsigned i = threadIdx.x; i < n; i += 256) b = max_u64(b, best[i]);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) b = max_u64(b, shfl_xor_u64(b, m));
    if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = b;
    __syncthreads();
    if (threadIdx.x == 0) {
        b = max_u64(max_u64(wbest[0], wbest[1]), max_u64(wbest[2], wbest[3]));
        uint32_t idx = 0;
        if (b) {
            const uint32_t key = 0xFFFFFFFFu - (uint32_t)b;
            idx = ((key & 0xFFFFFFu) << 8) | bitrev8(key >> 24);
        }
        result[0] = idx;
    }
}

// Workgroups resident at once for k_lm_head<NJ> on the current device (one
// round: every workgroup starts immediately), cached per width.
template <int NJ>
unsigned lm_head_resident() {
    static unsigned cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (!cached[dev]) {
        int per_cu = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_lm_head<NJ>, kLmWaves * 64, 0) != hipSuccess ||
            per_cu < 1)
            per_cu = 1;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
        const unsigned n = (unsigned)per_cu * (unsigned)cus;
        cached[dev] = n < kLmMaxWgs ? n : kLmMaxWgs;
    }
    return cached[dev];
}

template <int NJ>
void launch_lm_head(unsigned& wgs, hipStream_t st, hipEvent_t start, hipEvent_t stop, const float* x,
                    const uint16_t* w, float* logits, uint64_t* best, unsigned vocab, float cap) {
    const unsigned res = lm_head_resident<NJ>();
    if (wgs > res) wgs = res;
    if (start || stop)
        hipExtLaunchKernelGGL(k_lm_head<NJ>, dim3(wgs), dim3(kLmWaves * 64), 0, st, start, stop, 0, x, w, logits, best,
                              vocab, cap);
    else
        G4_LAUNCH(k_lm_head<NJ>, dim3(wgs), dim3(kLmWaves * 64), 0, st, x, w, logits, best, vocab, cap);
}

}  // namespace g4

using namespace g4;

namespace {

int lm_head_check(const g4_lm_head_params& p) {
    if (p.vocab == 0) return fail(G4_EINVAL, "lmHead: vocab 0");
    if (p.hidden % 256 || p.hidden / 256 < (uint32_t)kLmMinJ || p.hidden / 256 > (uint32_t)kLmMaxJ)
        return fail(G4_EINVAL, "lmHead: hidden %u unsupported (a multiple of 256 in [%d, %d])", p.hidden,
                    kLmMinJ * 256, kLmMaxJ * 256);
    if (!(p.cap >= 0.0f)) return fail(G4_EINVAL, "lmHead: softcap %g", (double)p.cap);
    return G4_OK;
}

// Workgroups wanted: one wave block each, at most the workspace bound (the
// launch lowers it further to what is resident at once).
unsigned lm_head_wgs(uint32_t vocab) {
    const uint64_t blocks = ((uint64_t)vocab + kLmBlockRows - 1) / kLmBlockRows;
    const uint64_t wgs = (blocks + kLmWaves - 1) / kLmWaves;
    return (unsigned)(wgs < kLmMaxWgs ? wgs : kLmMaxWgs);
}

int lm_head_run(const float* hidden, const uint16_t* weight, float* logits, uint32_t* result, void* workspace,
                size_t workspace_bytes, g4_lm_head_params p, void* stream, hipEvent_t start, hipEvent_t stop) {
    int rc = lm_head_check(p);
    if (rc) return rc;
    if (!hidden || !weight || !result || !workspace) return fail(G4_EINVAL, "lmHead: NULL pointer");
    if ((reinterpret_cast<uintptr_t>(hidden) | reinterpret_cast<uintptr_t>(weight)) & 15)
        return fail(G4_EINVAL, "lmHead: hidden and weight must be 16-byte aligned");
    unsigned wgs = lm_head_wgs(p.vocab);
    if (workspace_bytes < (size_t)wgs * sizeof(uint64_t))
        return fail(G4_ENOSPC, "lmHead: workspace %zu bytes < %zu needed", workspace_bytes,
                    (size_t)wgs * sizeof(uint64_t));
    hipStream_t st = as_stream(stream);
    uint64_t* best = static_cast<uint64_t*>(workspace);
    switch (p.hidden / 256) {
        case 4: launch_lm_head<4>(wgs, st, start, stop, hidden, weight, logits, best, p.vocab, p.cap); break;
        case 5: launch_lm_head<5>(wgs, st, start, stop, hidden, weight, logits, best, p.vocab, p.cap); break;
        case 6: launch_lm_head<6>(wgs, st, start, stop, hidden, weight, logits, best, p.vocab, p.cap); break;
        case 7: launch_lm_head<7>(wgs, st, start, stop, hidden, weight, logits, best, p.vocab, p.cap); break;
        case 8: launch_lm_head<8>(wgs, st, start, stop, hidden, weight, logits, best, p.vocab, p.cap); break;
        case 9: launch_lm_head<9>(wgs, st, start, stop, hidden, weight, logits, best, p.vocab, p.cap); break;
        default: launch_lm_head<10>(wgs, st, start, stop, hidden, weight, logits, best, p.vocab, p.cap); break;
    }
    G4_CHECK_LAUNCH("lmHead");
    G4_LAUNCH(k_lm_head_pick, dim3(1), dim3(256), 0, st, best, wgs, result);
    G4_CHECK_LAUNCH("lmHead pick");
    return G4_OK;
}

}  // namespace

extern "C" {

// dispatchMatmul (src/engine.ts:370-377): M workgroups, or a sqrt-shaped 2D grid above 65535.
static dim3 matmul_grid(uint32_t M) {
    unsigned gx = M, gy = 1;
    if (M > 65535u) {
        gx = (unsigned)ceil(sqrt((double)M));
        if (gx > 65535u) gx = 65535u;
        gy = (M + gx - 1) / gx;
    }
    return dim3(gx, gy);
}

int g4_matmul_quant_f16(const float* input, const uint16_t* weight, float* output, g4_matmul_params p, void* stream) {
    if (!input || !weight || !output) return fail(G4_EINVAL, "matmulQuant: NULL pointer");
    if (p.M == 0) return G4_OK;
    G4_LAUNCH(k_matmul_quant_f16, matmul_grid(p.M), dim3(kWG), 0, as_stream(stream), input, weight, output, p);
    G4_CHECK_LAUNCH("matmulQuant");
    return G4_OK;
}

int g4_matmul_q8(const float* input, const int8_t* qweight, const uint16_t* qscale, float* output, g4_matmul_params p,
                 void* stream) {
    if (!input || !qweight || !qscale || !output) return fail(G4_EINVAL, "matmulQ8: NULL pointer");
    if (p.N % 32) return fail(G4_EINVAL, "matmulQ8: N %u is not a multiple of 32", p.N);
    if (p.M == 0) return G4_OK;
    G4_LAUNCH(k_matmul_q8, matmul_grid(p.M), dim3(kWG), 0, as_stream(stream), input, qweight, qscale, output,
                       p);
    G4_CHECK_LAUNCH("matmulQ8");
    return G4_OK;
}

int g4_matmul_q4k(const float* input, const uint32_t* qweight, const uint16_t* qmeta, float* output,
                  g4_matmul_params p, void* stream) {
    if (!input || !qweight || !qmeta || !output) return fail(G4_EINVAL, "matmulQ4K: NULL pointer");
    if (p.N % 256) return fail(G4_EINVAL, "matmulQ4K: N %u is not a multiple of 256", p.N);
    if (p.M == 0) return G4_OK;
    G4_LAUNCH(k_matmul_q4k, matmul_grid(p.M), dim3(kWG), 0, as_stream(stream), input, qweight, qmeta, output,
                       p);
    G4_CHECK_LAUNCH("matmulQ4K");
    return G4_OK;
}

int g4_logit_softcap(float* logits, g4_softcap_params p, void* stream) {
    if (!logits) return fail(G4_EINVAL, "logitSoftcap: NULL logits");
    if (p.size == 0) return G4_OK;
    G4_LAUNCH(k_logit_softcap, dim3((p.size + kWG - 1) / kWG), dim3(kWG), 0, as_stream(stream), logits, p);
    G4_CHECK_LAUNCH("logitSoftcap");
    return G4_OK;
}

int g4_argmax(const float* logits, uint32_t* result, uint32_t size, void* stream) {
    if (!logits || !result) return fail(G4_EINVAL, "argmax: NULL pointer");
    G4_LAUNCH(k_argmax, dim3(1), dim3(kWG), 0, as_stream(stream), logits, result, size);
    G4_CHECK_LAUNCH("argmax");
    return G4_OK;
}

int g4_lm_head_workspace_size(g4_lm_head_params p, size_t* bytes) {
    if (!bytes) return fail(G4_EINVAL, "g4_lm_head_workspace_size: bytes is NULL");
    int rc = lm_head_check(p);
    if (rc) return rc;
    *bytes = (size_t)lm_head_wgs(p.vocab) * sizeof(uint64_t);
    return G4_OK;
}

int g4_lm_head_argmax(const float* hidden, const uint16_t* weight, float* logits, uint32_t* result, void* workspace,
                      size_t workspace_bytes, g4_lm_head_params p, void* stream) {
    return lm_head_run(hidden, weight, logits, result, workspace, workspace_bytes, p, stream, nullptr, nullptr);
}

int g4_lm_head_argmax_timed(const float* hidden, const uint16_t* weight, float* logits, uint32_t* result,
                            void* workspace, size_t workspace_bytes, g4_lm_head_params p, void* stream,
                            void* start_event, void* stop_event) {
    if (!start_event || !stop_event) return fail(G4_EINVAL, "lmHead: timing events are NULL");
    return lm_head_run(hidden, weight, logits, result, workspace, workspace_bytes, p, stream,
                       static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event));
}

}  // extern "C"
