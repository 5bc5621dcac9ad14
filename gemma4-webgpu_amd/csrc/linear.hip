// The engine's f16 projections either side of the attention block:
// attn.linearQKV (q, k, v from the normed hidden state, src/engine.ts:
// 2045-2051) and attn.linearOut (src/engine.ts:2096), both matmulQuant /
// matmulQuantMR4 with f16 weights. One launch covers up to kLinearMaxSegs
// weight matrices that read the same input (q, k and v in one pass), each
// row bit-identical to matmul_quant.wgsl (gemv_core.h).
//
// A wave takes `rows_per_wave` consecutive rows of the concatenated segments
// (two rows at a time, one per half-wave), chosen on the host so that the
// rows spread over every resident wave: the projections are a few thousand
// rows, a latency-bound size where the grid, not the bytes, sets the time.
#include <hip/hip_ext.h>

#include "gemv_core.h"

namespace g4 {

constexpr int kLinearMaxSegs = 4;
constexpr int kLinearMinJ = 4, kLinearMaxJ = 16;  // input length 1024 .. 4096

struct LinearSegDev {
    const uint16_t* w;  // f16 [rows][N]
    float* y;           // f32 [rows]
    uint32_t rows;
    uint32_t first;     // first row of the segment in the concatenation
};

struct LinearArgs {
    const float* x;
    LinearSegDev seg[kLinearMaxSegs];
    uint32_t n_segs;
    uint32_t total_rows;
    uint32_t rows_per_wave;  // even
};

template <int NJ>
__global__ __launch_bounds__(256) void k_linear(LinearArgs a) {
    constexpr unsigned N = NJ * 256;
    const unsigned lane = threadIdx.x & 63;
    const unsigned lq = lane & 31, half = lane >> 5;
    float xr[NJ][8];
    gemv_load_x<NJ>(a.x, lq, xr);
    const unsigned gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    const unsigned r0 = gw * a.rows_per_wave;
    const unsigned r1 = min(r0 + a.rows_per_wave, a.total_rows);
    for (unsigned r = r0; r < r1; r += 2) {
        const unsigned row = r + half;
        const bool valid = row < r1;
        const unsigned gr = valid ? row : r1 - 1;  // clamped: the duplicate's value is discarded
        int s = 0;
#pragma unroll
        for (int i = 1; i < kLinearMaxSegs; i++)
            if (i < (int)a.n_segs && gr >= a.seg[i].first) s = i;
        const LinearSegDev& sg = a.seg[s];
        const unsigned lr = gr - sg.first;
        const float v = gemv_row_dot<NJ>(sg.w + (uint64_t)lr * N, xr, lq);
        if (valid && lq == 0) sg.y[lr] = v;
    }
}

template <int NJ>
unsigned linear_resident_waves() {
    static unsigned cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (!cached[dev]) {
        int per_cu = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_linear<NJ>, 256, 0) != hipSuccess || per_cu < 1)
            per_cu = 1;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
        cached[dev] = (unsigned)per_cu * (unsigned)cus * 4;
    }
    return cached[dev];
}

template <int NJ>
int launch_linear(LinearArgs& a, hipStream_t st) {
    const unsigned waves = linear_resident_waves<NJ>();
    unsigned rpw = 2 * ((a.total_rows + 2 * waves - 1) / (2 * waves));
    if (rpw < 2) rpw = 2;
    a.rows_per_wave = rpw;
    const unsigned n_waves = (a.total_rows + rpw - 1) / rpw;
    hipLaunchKernelGGL(k_linear<NJ>, dim3((n_waves + 3) / 4), dim3(256), 0, st, a);
    G4_CHECK_LAUNCH("linear");
    return G4_OK;
}

}  // namespace g4

using namespace g4;

extern "C" {

int g4_linear_f16(const float* input, uint32_t n, const g4_linear_seg* segs, uint32_t n_segs, void* stream) {
    if (!input || !segs) return fail(G4_EINVAL, "linear: NULL pointer");
    if (n_segs == 0 || n_segs > (uint32_t)kLinearMaxSegs)
        return fail(G4_EINVAL, "linear: %u weight segments (1..%d)", n_segs, kLinearMaxSegs);
    if (n % 256 || n / 256 < (uint32_t)kLinearMinJ || n / 256 > (uint32_t)kLinearMaxJ)
        return fail(G4_EINVAL, "linear: input length %u unsupported (a multiple of 256 in [%d, %d])", n,
                    kLinearMinJ * 256, kLinearMaxJ * 256);
    if (reinterpret_cast<uintptr_t>(input) & 15) return fail(G4_EINVAL, "linear: input must be 16-byte aligned");
    LinearArgs a = {};
    a.x = input;
    a.n_segs = n_segs;
    uint64_t total = 0;
    for (uint32_t i = 0; i < n_segs; i++) {
        const g4_linear_seg& sg = segs[i];
        if (!sg.weight || !sg.out) return fail(G4_EINVAL, "linear: segment %u has a NULL pointer", i);
        if (reinterpret_cast<uintptr_t>(sg.weight) & 15)
            return fail(G4_EINVAL, "linear: segment %u weight must be 16-byte aligned", i);
        if (sg.rows == 0) return fail(G4_EINVAL, "linear: segment %u has no rows", i);
        a.seg[i] = LinearSegDev{sg.weight, sg.out, sg.rows, (uint32_t)total};
        total += sg.rows;
    }
    if (total > 0x7fffffffull) return fail(G4_EINVAL, "linear: %llu rows", (unsigned long long)total);
    a.total_rows = (uint32_t)total;
    hipStream_t st = as_stream(stream);
    switch (n / 256) {
        case 4: return launch_linear<4>(a, st);
        case 5: return launch_linear<5>(a, st);
        case 6: return launch_linear<6>(a, st);
        case 7: return launch_linear<7>(a, st);
        case 8: return launch_linear<8>(a, st);
        case 9: return launch_linear<9>(a, st);
        case 10: return launch_linear<10>(a, st);
        case 11: return launch_linear<11>(a, st);
        case 12: return launch_linear<12>(a, st);
        case 13: return launch_linear<13>(a, st);
        case 14: return launch_linear<14>(a, st);
        case 15: return launch_linear<15>(a, st);
        default: return launch_linear<16>(a, st);
    }
}

}  // extern "C"
