// The engine's projections either side of the attention block, for f16 and
// for its in-shader quantized weights (q8, q4k):
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

enum LinearFormat { kF16 = 0, kQ8 = G4_WEIGHT_Q8, kQ4K = G4_WEIGHT_Q4K };

struct LinearSegDev {
    const void* w;         // f16 [rows][N], int8 [rows][N] or u32 [rows][N/8]
    const uint16_t* meta;  // q8: f16 scales [rows][N/32]; q4k: f16 [rows][N/256][16]
    float* y;              // f32 [rows]
    uint32_t rows;
    uint32_t first;        // first row of the segment in the concatenation
};

struct LinearArgs {
    const float* x;
    LinearSegDev seg[kLinearMaxSegs];
    uint32_t n_segs;
    uint32_t total_rows;
    uint32_t rows_per_wave;  // even
};

template <int FMT, int NJ>
__device__ __forceinline__ float linear_row(const LinearSegDev& sg, unsigned lr, const float (&xr)[NJ][8], unsigned lq) {
    constexpr unsigned N = NJ * 256;
    if constexpr (FMT == kQ8)
        return gemv_row_dot_q8<NJ, false>(static_cast<const int8_t*>(sg.w) + (uint64_t)lr * N,
                                          sg.meta + (uint64_t)lr * (N / 32), xr, lq);
    else if constexpr (FMT == kQ4K)
        return gemv_row_dot_q4k<NJ, false>(static_cast<const uint32_t*>(sg.w) + (uint64_t)lr * (N / 8),
                                           sg.meta + (uint64_t)lr * (N / 16), xr, lq);
    else
        return gemv_row_dot<NJ, false>(static_cast<const uint16_t*>(sg.w) + (uint64_t)lr * N, xr, lq);
}

template <int FMT, int NJ>
__global__ __launch_bounds__(256) void k_linear(LinearArgs a) {
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
        const float v = linear_row<FMT, NJ>(sg, lr, xr, lq);  // the row's value in lane 0 of the half
        if (valid && lq == 0) sg.y[lr] = v;
    }
}

template <int FMT, int NJ>
unsigned linear_resident_waves() {
    static unsigned cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (!cached[dev]) {
        int per_cu = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_linear<FMT, NJ>, 256, 0) != hipSuccess || per_cu < 1)
            per_cu = 1;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
        cached[dev] = (unsigned)per_cu * (unsigned)cus * 4;
    }
    return cached[dev];
}

template <int FMT, int NJ>
int launch_linear(LinearArgs& a, hipStream_t st) {
    const unsigned waves = linear_resident_waves<FMT, NJ>();
    unsigned rpw = 2 * ((a.total_rows + 2 * waves - 1) / (2 * waves));
    if (rpw < 2) rpw = 2;
    a.rows_per_wave = rpw;
    const unsigned n_waves = (a.total_rows + rpw - 1) / rpw;
    G4_LAUNCH((k_linear<FMT, NJ>), dim3((n_waves + 3) / 4), dim3(256), 0, st, a);
    G4_CHECK_LAUNCH("linear");
    return G4_OK;
}

template <int FMT>
int launch_linear_n(LinearArgs& a, uint32_t n, hipStream_t st) {
    switch (n / 256) {
        case 4: return launch_linear<FMT, 4>(a, st);
        case 5: return launch_linear<FMT, 5>(a, st);
        case 6: return launch_linear<FMT, 6>(a, st);
        case 7: return launch_linear<FMT, 7>(a, st);
        case 8: return launch_linear<FMT, 8>(a, st);
        case 9: return launch_linear<FMT, 9>(a, st);
        case 10: return launch_linear<FMT, 10>(a, st);
        case 11: return launch_linear<FMT, 11>(a, st);
        case 12: return launch_linear<FMT, 12>(a, st);
        case 13: return launch_linear<FMT, 13>(a, st);
        case 14: return launch_linear<FMT, 14>(a, st);
        case 15: return launch_linear<FMT, 15>(a, st);
        default: return launch_linear<FMT, 16>(a, st);
    }
}

// Checks shared by both entry points; fills the segment table.
int linear_args(const char* who, const float* input, uint32_t n, uint32_t n_segs, LinearArgs* a) {
    if (!input) return fail(G4_EINVAL, "%s: NULL input", who);
    if (n_segs == 0 || n_segs > (uint32_t)kLinearMaxSegs)
        return fail(G4_EINVAL, "%s: %u weight segments (1..%d)", who, n_segs, kLinearMaxSegs);
    if (n % 256 || n / 256 < (uint32_t)kLinearMinJ || n / 256 > (uint32_t)kLinearMaxJ)
        return fail(G4_EINVAL, "%s: input length %u unsupported (a multiple of 256 in [%d, %d])", who, n,
                    kLinearMinJ * 256, kLinearMaxJ * 256);
    if (reinterpret_cast<uintptr_t>(input) & 15) return fail(G4_EINVAL, "%s: input must be 16-byte aligned", who);
    *a = LinearArgs{};
    a->x = input;
    a->n_segs = n_segs;
    return G4_OK;
}

int add_segment(const char* who, LinearArgs* a, uint32_t i, const void* w, const uint16_t* meta, bool need_meta,
                float* out, uint32_t rows, uint64_t* total) {
    if (!w || !out || (need_meta && !meta)) return fail(G4_EINVAL, "%s: segment %u has a NULL pointer", who, i);
    if (reinterpret_cast<uintptr_t>(w) & 15) return fail(G4_EINVAL, "%s: segment %u weight must be 16-byte aligned", who, i);
    if (rows == 0) return fail(G4_EINVAL, "%s: segment %u has no rows", who, i);
    a->seg[i] = LinearSegDev{w, meta, out, rows, (uint32_t)*total};
    *total += rows;
    if (*total > 0x7fffffffull) return fail(G4_EINVAL, "%s: %llu rows", who, (unsigned long long)*total);
    a->total_rows = (uint32_t)*total;
    return G4_OK;
}

}  // namespace g4

using namespace g4;

extern "C" {

int g4_linear_f16(const float* input, uint32_t n, const g4_linear_seg* segs, uint32_t n_segs, void* stream) {
    LinearArgs a;
    int rc = linear_args("linear", input, n, n_segs, &a);
    if (rc) return rc;
    if (!segs) return fail(G4_EINVAL, "linear: NULL pointer");
    uint64_t total = 0;
    for (uint32_t i = 0; i < n_segs; i++)
        if ((rc = add_segment("linear", &a, i, segs[i].weight, nullptr, false, segs[i].out, segs[i].rows, &total)))
            return rc;
    return launch_linear_n<kF16>(a, n, as_stream(stream));
}

int g4_linear_quant(const float* input, uint32_t n, uint32_t format, const g4_linear_qseg* segs, uint32_t n_segs,
                    void* stream) {
    if (format != G4_WEIGHT_Q8 && format != G4_WEIGHT_Q4K)
        return fail(G4_EINVAL, "linearQuant: weight format %u (G4_WEIGHT_Q8 or G4_WEIGHT_Q4K)", format);
    LinearArgs a;
    int rc = linear_args("linearQuant", input, n, n_segs, &a);
    if (rc) return rc;
    if (!segs) return fail(G4_EINVAL, "linearQuant: NULL pointer");
    uint64_t total = 0;
    for (uint32_t i = 0; i < n_segs; i++)
        if ((rc = add_segment("linearQuant", &a, i, segs[i].weight, segs[i].meta, true, segs[i].out, segs[i].rows,
                              &total)))
            return rc;
    return format == G4_WEIGHT_Q8 ? launch_linear_n<kQ8>(a, n, as_stream(stream))
                                  : launch_linear_n<kQ4K>(a, n, as_stream(stream));
}

}  // extern "C"
