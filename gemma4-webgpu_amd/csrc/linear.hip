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
#include "ref_math.h"

namespace g4 {

constexpr int kLinearMaxSegs = 4;
constexpr int kLinearMinJ = 4, kLinearMaxJ = 16;  // input length 1024 .. 4096

enum LinearFormat { kF16 = G4_WEIGHT_F16, kQ8 = G4_WEIGHT_Q8, kQ4K = G4_WEIGHT_Q4K };

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

// attn.linearQKV with the producer-side prep of the attention block as its
// epilogue (src/engine.ts:2045-2091: linearQKV, then perHeadRmsNormNoWeight
// on v, fusedPerHeadNormRope on q and k, kvCacheStore), in one launch. The
// rows are k_linear's (bit-identical to matmul_quant / matmul_q8 /
// matmul_q4k) and land in the segments' outputs as the reference's raw
// projections do. A workgroup's four waves take 8 consecutive rows of one
// head (a pair each) and store them with agent-scope relaxed stores, which
// write through to the device's coherence point; once they are complete (an
// explicit wait, then the barrier), one thread adds 8 to the head's arrival
// counter, and the workgroup that brings it to head_dim runs the head's
// epilogue in one wave: its raw values read with agent-scope loads, the
// reference's RMSNorm (+ RoPE for q and k) written back in place, and the f16
// store of k and v at row `slot` (wave_norm_rope: bit-identical to the
// reference kernels). That wave sets the counter back to 0 for the next call.
// (With an agent-scope release fence per wave instead, every wave wrote back
// its XCD's L2: 26 us per E2B layer against 7.8 us for projection + prep
// launches.)
constexpr unsigned kPrepRowsPerWg = 8;  // 4 waves x a row pair; divides head_dim

struct QkvPrepDev {
    const uint16_t* q_weight;
    const uint16_t* k_weight;
    const uint16_t* rope_freqs;
    const float* rope_inv;  // device [head_dim / 2] inverse frequencies, or nullptr (evaluated here)
    uint16_t* k_cache;
    uint16_t* v_cache;
    uint32_t* counters;     // per head: q heads, then k heads, then v heads
    uint32_t num_q_heads, num_kv_heads, head_dim;
    uint32_t position, slot;
    float eps, theta;
    uint32_t apply_divisor, store_kv;
};

// One head's epilogue by one wave: segment s (0 q, 1 k, 2 v), head `head` of
// the segment, whose raw values sit at y.
template <int HD>
__device__ __forceinline__ void qkv_head_epilogue(const QkvPrepDev& e, unsigned s, unsigned head, float* y,
                                                  unsigned lane) {
    constexpr int J = HD / 64, PJ = J / 2;
    const bool rope = s != 2;  // v: the weightless norm only
    const uint16_t* w = s == 0 ? e.q_weight : e.k_weight;
    float x[J];
    uint32_t wb[J];
#pragma unroll
    for (int j = 0; j < J; j++) {
        x[j] = __hip_atomic_load(y + lane + 64 * j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        wb[j] = rope ? w[lane + 64 * j] : 0u;
    }
    RopeLane<PJ> rl;
    if (rope) {  // uniform: this lane's pairs, cos and sin of the f32 angle in f64 (fused_per_head_norm_rope.wgsl:55)
#pragma unroll
        for (int p = 0; p < PJ; p++) {
            const unsigned i = lane + 64 * p;
            const float inv = e.rope_inv ? e.rope_inv[i]
                                         : rope_inv_freq(i, HD, e.theta, e.apply_divisor,
                                                         e.apply_divisor ? h2f(e.rope_freqs[i]) : 1.0f);
            f64_cos_sin((float)e.position * inv, rl.c[p], rl.s[p]);
        }
    }
    wave_norm_rope<J>(x, wb, rope, rope, rl, e.eps);
#pragma unroll
    for (int j = 0; j < J; j++) y[lane + 64 * j] = x[j];
    if (s != 0 && e.store_kv) {
        uint16_t* dst = (s == 1 ? e.k_cache : e.v_cache) + ((uint64_t)e.slot * e.num_kv_heads + head) * HD;
#pragma unroll
        for (int j = 0; j < J; j++) dst[lane + 64 * j] = f2h(x[j]);
    }
}

template <int FMT, int NJ>
__global__ __launch_bounds__(256) void k_linear_prep(LinearArgs a, QkvPrepDev e) {
    __shared__ unsigned last;
    const unsigned lane = threadIdx.x & 63;
    const unsigned lq = lane & 31, half = lane >> 5;
    const unsigned wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    float xr[NJ][8];
    gemv_load_x<NJ>(a.x, lq, xr);
    const unsigned r0 = blockIdx.x * kPrepRowsPerWg;  // the workgroup's rows, all in one head
    int s = 0;
#pragma unroll
    for (int i = 1; i < kLinearMaxSegs; i++)
        if (i < (int)a.n_segs && r0 >= a.seg[i].first) s = i;
    const LinearSegDev& sg = a.seg[s];
    const unsigned HD = e.head_dim;
    const unsigned head = (r0 - sg.first) / HD;
    const unsigned lr = r0 - sg.first + 2 * wave + half;
    const float v = linear_row<FMT, NJ>(sg, lr, xr, lq);  // the row's value in lane 0 of the half
    if (lq == 0) __hip_atomic_store(sg.y + lr, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // the stores have reached the coherence point
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned cid = s == 0 ? head : e.num_q_heads + (unsigned)(s - 1) * e.num_kv_heads + head;
        const unsigned old =
            __hip_atomic_fetch_add(&e.counters[cid], kPrepRowsPerWg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = old + kPrepRowsPerWg == HD ? cid + 1 : 0u;
    }
    __syncthreads();
    const unsigned done = last;
    if (done && wave == 0) {  // uniform: every row of the head has arrived
        float* y = sg.y + (uint64_t)head * HD;
        if (HD == 512)
            qkv_head_epilogue<512>(e, (unsigned)s, head, y, lane);
        else
            qkv_head_epilogue<256>(e, (unsigned)s, head, y, lane);
        if (lane == 0) __hip_atomic_store(&e.counters[done - 1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int FMT, int NJ>
int launch_linear_prep(LinearArgs& a, const QkvPrepDev& e, hipStream_t st) {
    a.rows_per_wave = 2;
    G4_LAUNCH((k_linear_prep<FMT, NJ>), dim3(a.total_rows / kPrepRowsPerWg), dim3(256), 0, st, a, e);
    G4_CHECK_LAUNCH("linearQkvPrep");
    return G4_OK;
}

template <int FMT>
int launch_linear_prep_n(LinearArgs& a, const QkvPrepDev& e, uint32_t n, hipStream_t st) {
    switch (n / 256) {
        case 4: return launch_linear_prep<FMT, 4>(a, e, st);
        case 5: return launch_linear_prep<FMT, 5>(a, e, st);
        case 6: return launch_linear_prep<FMT, 6>(a, e, st);
        case 7: return launch_linear_prep<FMT, 7>(a, e, st);
        case 8: return launch_linear_prep<FMT, 8>(a, e, st);
        case 9: return launch_linear_prep<FMT, 9>(a, e, st);
        case 10: return launch_linear_prep<FMT, 10>(a, e, st);
        case 11: return launch_linear_prep<FMT, 11>(a, e, st);
        case 12: return launch_linear_prep<FMT, 12>(a, e, st);
        case 13: return launch_linear_prep<FMT, 13>(a, e, st);
        case 14: return launch_linear_prep<FMT, 14>(a, e, st);
        case 15: return launch_linear_prep<FMT, 15>(a, e, st);
        default: return launch_linear_prep<FMT, 16>(a, e, st);
    }
}

}  // namespace g4

using namespace g4;

extern "C" {

int g4_linear_qkv_prep_workspace_size(uint32_t num_q_heads, uint32_t num_kv_heads, size_t* bytes) {
    if (!bytes) return fail(G4_EINVAL, "linearQkvPrep: bytes is NULL");
    if (num_q_heads == 0 || num_kv_heads == 0 || num_q_heads > 4096 || num_kv_heads > 4096)
        return fail(G4_EINVAL, "linearQkvPrep: %u query heads, %u kv heads", num_q_heads, num_kv_heads);
    *bytes = ((num_q_heads + 2ull * num_kv_heads) * 4 + 255) & ~255ull;
    return G4_OK;
}

int g4_linear_qkv_prep(const float* input, uint32_t n, uint32_t format, const g4_linear_qseg* segs, uint32_t n_segs,
                       const uint16_t* q_weight, const uint16_t* k_weight, const uint16_t* rope_freqs,
                       const float* rope_inv_freq, uint16_t* k_cache, uint16_t* v_cache, g4_qkv_prep_params p,
                       void* workspace, void* stream) {
    const char* who = "linearQkvPrep";
    if (format != G4_WEIGHT_F16 && format != G4_WEIGHT_Q8 && format != G4_WEIGHT_Q4K)
        return fail(G4_EINVAL, "%s: weight format %u", who, format);
    size_t ws_need = 0;
    int rc = g4_linear_qkv_prep_workspace_size(p.num_q_heads, p.num_kv_heads, &ws_need);
    if (rc) return rc;
    if (p.head_dim != 256 && p.head_dim != 512) return fail(G4_EINVAL, "%s: head_dim %u (256 or 512)", who, p.head_dim);
    if (!segs || !q_weight || !workspace) return fail(G4_EINVAL, "%s: NULL segments, q_weight or workspace", who);
    if (reinterpret_cast<uintptr_t>(workspace) & 3) return fail(G4_EINVAL, "%s: workspace must be 4-byte aligned", who);
    if (n_segs != (p.store_kv ? 3u : 1u))
        return fail(G4_EINVAL, "%s: %u segments (q, k, v on a KV producer; q alone otherwise)", who, n_segs);
    if (segs[0].rows != p.num_q_heads * p.head_dim)
        return fail(G4_EINVAL, "%s: q segment has %u rows, not %u", who, segs[0].rows, p.num_q_heads * p.head_dim);
    for (uint32_t i = 1; i < n_segs; i++)
        if (segs[i].rows != p.num_kv_heads * p.head_dim)
            return fail(G4_EINVAL, "%s: segment %u has %u rows, not %u", who, i, segs[i].rows,
                        p.num_kv_heads * p.head_dim);
    if (p.store_kv) {
        if (!k_weight || !k_cache || !v_cache) return fail(G4_EINVAL, "%s: a KV producer needs k_weight and caches", who);
        if (p.slot >= p.max_seq_len) return fail(G4_EINVAL, "%s: slot %u >= max_seq_len %u", who, p.slot, p.max_seq_len);
    }
    if (p.apply_divisor && !rope_freqs && !rope_inv_freq)
        return fail(G4_EINVAL, "%s: apply_divisor needs rope_freqs (or the inverse-frequency table)", who);
    LinearArgs a;
    if ((rc = linear_args(who, input, n, n_segs, &a))) return rc;
    uint64_t total = 0;
    for (uint32_t i = 0; i < n_segs; i++)
        if ((rc = add_segment(who, &a, i, segs[i].weight, segs[i].meta, format != G4_WEIGHT_F16, segs[i].out,
                              segs[i].rows, &total)))
            return rc;
    QkvPrepDev e{q_weight, k_weight, rope_freqs, rope_inv_freq, k_cache, v_cache, static_cast<uint32_t*>(workspace),
                 p.num_q_heads, p.num_kv_heads, p.head_dim, p.position, p.slot, p.eps, p.theta,
                 p.apply_divisor ? 1u : 0u, p.store_kv ? 1u : 0u};
    hipStream_t st = as_stream(stream);
    if (format == G4_WEIGHT_Q8) return launch_linear_prep_n<kQ8>(a, e, n, st);
    if (format == G4_WEIGHT_Q4K) return launch_linear_prep_n<kQ4K>(a, e, n, st);
    return launch_linear_prep_n<kF16>(a, e, n, st);
}

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
