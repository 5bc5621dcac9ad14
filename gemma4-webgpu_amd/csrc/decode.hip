// Fused decode attention for gfx950: attnScore -> softmax -> attnOutput of
// gemma4-webgpu (shaders/attn_score.wgsl:15-40, softmax.wgsl:7-46,
// attn_output.wgsl:7-23, dispatched at src/engine.ts:2092-2094) as one
// flash-decoding pass over the attended K/V rows.
//
// Work decomposition
//   One workgroup (4 waves) per (split, kv head). A split is a contiguous run
//   of `chunk` cache rows of one problem ("entry": a layer of a token's stack,
//   or a sequence of a ragged batch). Each wave walks 32-row tiles of the
//   split, keeps an online softmax state, and the 4 waves are combined through
//   LDS. A problem with one split writes its output directly; otherwise the
//   split writes (m, l, o) partials and k_decode_merge combines them with a
//   fixed-order log-sum-exp. All G <= 8 query heads of a kv head are served
//   by one read of each K/V row (GQA: the reference re-reads K and V once per
//   query head).
//
// MFMA mapping (v_mfma_f32_16x16x32_f16; lane = 16*g + n)
//   Scores  S^T[16 keys x 16 cols] = K[16 keys x 32 d] * Qc^T[32 d x 16 cols].
//           Columns 0..7 hold the f16 "hi" part of q*scale*log2(e) for query
//           heads 0..7, columns 8..15 the f16 "lo" residual, so hi+lo carries
//           ~22 mantissa bits and scores keep f32-level accuracy. Lane (n, g)
//           supplies K[key n][d in 32c + 8g .. +8]: one 16-byte load.
//   Output  O^T[16 d x 16 cols] += V^T[16 d x 32 keys] * P^T[32 keys x 16 cols],
//           P split into hi/lo columns the same way. Lane (n, g) loads 8 full
//           16-byte pieces of V rows (lanes n = 0..15 of a row read 256
//           contiguous bytes) and transposes the 8x8 f16 block in registers
//           with v_perm_b32, so no LDS staging is needed for K or V.
//   The hi and lo columns are added with one DPP row rotation by 8.
//
// Masking: rows outside [key_begin, key_end) get score -inf (probability 0,
// as exp(-1e30 - max) == 0 in the reference) and their loads are clamped to
// the last valid row, so nothing outside the attended rows is read.
#include <stdlib.h>
#include <string.h>

#include "common.h"

namespace g4 {

constexpr int kDecodeWaves = 4;
constexpr int kDecodeThreads = 64 * kDecodeWaves;
constexpr int kTileKeys = 32;
constexpr int kMaxGroup = 8;  // query heads per kv head served by one MFMA column block

struct DecodeEntryDev {
    const float* q;       // [num_kv_heads][group][HD]
    const uint16_t* k;    // [rows][num_kv_heads][HD]
    const uint16_t* v;
    float* out;           // [num_kv_heads][group][HD]
    uint32_t key_begin;   // first attended row
    uint32_t key_end;     // one past the last attended row
    uint32_t split_base;  // first split index of this entry
    uint32_t n_splits;
    float qscale;         // attention scale * log2(e)
    uint32_t pad;
};

struct DecodeArgs {
    const DecodeEntryDev* table;  // device table, or nullptr to use `one`
    DecodeEntryDev one;
    uint32_t n_entries;
    uint32_t num_kv_heads;
    uint32_t group;
    uint32_t chunk;       // rows per split, multiple of kTileKeys
    float* part_o;        // [split][kv_head][group][HD]
    float* part_ml;       // [split][kv_head][group][2]
};

__device__ __forceinline__ float dpp_ror8_add(float x) {
    int y = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x128, 0xf, 0xf, false);  // row_ror:8
    return x + __builtin_bit_cast(float, y);
}

__device__ __forceinline__ uint32_t perm_lo(uint32_t a, uint32_t b) {  // (a.lo16, b.lo16)
    return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t perm_hi(uint32_t a, uint32_t b) {  // (a.hi16, b.hi16)
    return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

__device__ __forceinline__ DecodeEntryDev find_entry(const DecodeArgs& a, unsigned split) {
    if (!a.table) return a.one;
    unsigned lo = 0, hi = a.n_entries;  // last entry with split_base <= split
    while (hi - lo > 1) {
        unsigned mid = (lo + hi) >> 1;
        if (a.table[mid].split_base <= split) lo = mid;
        else hi = mid;
    }
    return a.table[lo];
}

template <int HD>
__global__ __launch_bounds__(kDecodeThreads) void k_decode_split(DecodeArgs a) {
    constexpr int NC = HD / 32;   // K chunks of 32 d per score MFMA chain
    constexpr int NB = HD / 128;  // V blocks of 16 lanes x 8 d
    constexpr int NO = NB * 8;    // output MFMA tiles of 16 d

    __shared__ float lds_o[kDecodeWaves][NO * 4][32];
    __shared__ float lds_m[kDecodeWaves][kMaxGroup];
    __shared__ float lds_l[kDecodeWaves][kMaxGroup];

    const unsigned split = blockIdx.x;
    const unsigned kvh = blockIdx.y;
    const DecodeEntryDev ent = find_entry(a, split);
    const float* __restrict__ qp = ent.q;
    const uint16_t* __restrict__ kp = ent.k;
    const uint16_t* __restrict__ vp = ent.v;
    float* __restrict__ outp = ent.out;
    const unsigned key_end = ent.key_end;
    const unsigned n_splits = ent.n_splits;
    const float qscale = ent.qscale;
    const unsigned s_local = split - ent.split_base;
    const unsigned k0 = ent.key_begin + s_local * a.chunk;
    const unsigned k1 = min(key_end, k0 + a.chunk);
    const unsigned G = a.group;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n = lane & 15;
    const int g = lane >> 4;
    const int head = n & 7;
    const bool lo_col = n >= 8;
    const uint64_t row_stride = (uint64_t)a.num_kv_heads * HD;  // f16 elements per cache row
    const uint16_t* K = kp + (uint64_t)kvh * HD;
    const uint16_t* V = vp + (uint64_t)kvh * HD;

    // Query operand: q * scale * log2(e), split into f16 hi + lo columns.
    f16x8 qop[NC];
    {
        const float* qh = qp + ((uint64_t)kvh * G + head) * HD;
        const bool live = (unsigned)head < G;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            f16x8 v;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float x = live ? qh[c * 32 + g * 8 + i] * qscale : 0.0f;
                f16 hi = (f16)x;
                v[i] = lo_col ? (f16)(x - (float)hi) : hi;
            }
            qop[c] = v;
        }
    }

    float m_run = -INFINITY;
    float l_run = 0.0f;
    f32x4 acc[NO];
#pragma unroll
    for (int i = 0; i < NO; i++) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    const unsigned nkeys = k1 - k0;
    const unsigned last = k1 - 1;
    for (unsigned t0 = (unsigned)wave * kTileKeys; t0 < nkeys; t0 += kDecodeWaves * kTileKeys) {
        const unsigned kt0 = k0 + t0;
        // ---- loads: K in score-operand layout, V as 16-byte row pieces ----
        f16x8 kreg[2][NC];
#pragma unroll
        for (int h2 = 0; h2 < 2; h2++) {
            const unsigned key = min(kt0 + h2 * 16 + n, last);
            const uint16_t* row = K + key * row_stride + g * 8;
#pragma unroll
            for (int c = 0; c < NC; c++) kreg[h2][c] = *reinterpret_cast<const f16x8*>(row + c * 32);
        }
        u32x4 vreg[NB][8];
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const unsigned key = min(kt0 + (t < 4 ? g * 4 + t : 16 + g * 4 + (t - 4)), last);
            const uint16_t* row = V + key * row_stride;
#pragma unroll
            for (int b = 0; b < NB; b++) vreg[b][t] = *reinterpret_cast<const u32x4*>(row + (n + 16 * b) * 8);
        }

        // ---- scores (log2 units) ----
        f32x4 s[2];
#pragma unroll
        for (int h2 = 0; h2 < 2; h2++) {
            s[h2] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NC; c++) s[h2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kreg[h2][c], qop[c], s[h2], 0, 0, 0);
        }
        float sv[8];
        float tmax = -INFINITY;
#pragma unroll
        for (int h2 = 0; h2 < 2; h2++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float x = dpp_ror8_add(s[h2][j]);
                const unsigned key = kt0 + h2 * 16 + g * 4 + j;
                x = key < k1 ? x : -INFINITY;
                sv[h2 * 4 + j] = x;
                tmax = fmaxf(tmax, x);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float m_new = fmaxf(m_run, tmax);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        f16x8 pop;
        float psum = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            float p = __builtin_amdgcn_exp2f(sv[t] - m_new);
            psum += p;
            f16 hi = (f16)p;
            pop[t] = lo_col ? (f16)(p - (float)hi) : hi;
        }
        l_run = l_run * alpha + psum;
#pragma unroll
        for (int i = 0; i < NO; i++) acc[i] *= alpha;

        // ---- output: transpose each 8x8 f16 block of V, then MFMA ----
#pragma unroll
        for (int b = 0; b < NB; b++) {
#pragma unroll
            for (int e2 = 0; e2 < 4; e2++) {  // d pair (2*e2, 2*e2+1) lives in word e2 of every row piece
                u32x4 lo, hi;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    lo[q] = perm_lo(vreg[b][2 * q][e2], vreg[b][2 * q + 1][e2]);
                    hi[q] = perm_hi(vreg[b][2 * q][e2], vreg[b][2 * q + 1][e2]);
                }
                acc[b * 8 + 2 * e2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, lo), pop,
                                                                             acc[b * 8 + 2 * e2], 0, 0, 0);
                acc[b * 8 + 2 * e2 + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, hi), pop,
                                                                                 acc[b * 8 + 2 * e2 + 1], 0, 0, 0);
            }
        }
    }

    // ---- per-wave totals: l over the 4 lane groups, hi+lo columns of o ----
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
#pragma unroll
    for (int i = 0; i < NO; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = dpp_ror8_add(acc[i][j]);
    if (n < 8) {
#pragma unroll
        for (int i = 0; i < NO; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) lds_o[wave][i * 4 + j][g * 8 + n] = acc[i][j];
        if (g == 0) {
            lds_m[wave][n] = m_run;
            lds_l[wave][n] = l_run;
        }
    }
    __syncthreads();

    // ---- combine the 4 waves; write final output or the split partial ----
    const int t = threadIdx.x;
    const int lane32 = t & 31;
    const int h = lane32 & 7;
    const int gg = lane32 >> 3;
    if ((unsigned)h >= G) return;
    float mw[kDecodeWaves], M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; w++) {
        mw[w] = lds_m[w][h];
        M = fmaxf(M, mw[w]);
    }
    float L = 0.0f, sc[kDecodeWaves];
#pragma unroll
    for (int w = 0; w < kDecodeWaves; w++) {
        sc[w] = __builtin_amdgcn_exp2f(mw[w] - M);
        L += lds_l[w][h] * sc[w];
    }
    const bool final_out = n_splits == 1;
    const float inv_l = 1.0f / L;
    float* dst;
    if (final_out) {
        dst = outp + ((uint64_t)kvh * G + h) * HD;
    } else {
        const uint64_t pidx = ((uint64_t)split * a.num_kv_heads + kvh) * G + h;
        dst = a.part_o + pidx * HD;
        if (t < 32 && gg == 0) {
            a.part_ml[pidx * 2 + 0] = M;
            a.part_ml[pidx * 2 + 1] = L;
        }
    }
    constexpr int kSlots = NO * 4;
#pragma unroll
    for (int sl = t >> 5; sl < kSlots; sl += kDecodeThreads / 32) {
        float o = 0.0f;
#pragma unroll
        for (int w = 0; w < kDecodeWaves; w++) o += lds_o[w][sl][lane32] * sc[w];
        const int i = sl >> 2, j = sl & 3;       // MFMA tile i = b*8 + e, row j
        const int b = i >> 3, e = i & 7;
        const int d = ((gg * 4 + j) + 16 * b) * 8 + e;
        dst[d] = final_out ? o * inv_l : o;
    }
}

// Fixed-order log-sum-exp merge of the split partials of one entry.
template <int HD>
__global__ __launch_bounds__(256) void k_decode_merge(DecodeArgs a) {
    const DecodeEntryDev ent = a.table ? a.table[blockIdx.x] : a.one;
    const unsigned ns = ent.n_splits;
    if (ns <= 1) return;
    const unsigned kvh = blockIdx.y;
    const unsigned idx = blockIdx.z * 256 + threadIdx.x;
    const unsigned G = a.group;
    if (idx >= G * HD) return;
    const unsigned h = idx / HD, d = idx % HD;
    const uint64_t stride = (uint64_t)a.num_kv_heads * G;  // partial records per split
    const uint64_t base = ((uint64_t)ent.split_base * a.num_kv_heads + kvh) * G + h;
    float M = -INFINITY;
    for (unsigned s = 0; s < ns; s++) M = fmaxf(M, a.part_ml[(base + s * stride) * 2]);
    float L = 0.0f, O = 0.0f;
    for (unsigned s = 0; s < ns; s++) {
        const uint64_t r = base + s * stride;
        const float sc = __builtin_amdgcn_exp2f(a.part_ml[r * 2] - M);
        L += a.part_ml[r * 2 + 1] * sc;
        O += a.part_o[r * HD + d] * sc;
    }
    ent.out[((uint64_t)kvh * G + h) * HD + d] = O / L;
}

}  // namespace g4

using namespace g4;

namespace {

constexpr unsigned kMinChunk = 128;
constexpr unsigned kCUs = 256;

inline unsigned round_up(unsigned x, unsigned m) { return (x + m - 1) / m * m; }

// Rows per split: enough splits to put about two workgroups on every CU, but
// never fewer than kMinChunk rows, so partial traffic stays small.
unsigned pick_chunk(uint64_t total_rows, unsigned num_kv_heads) {
    static int env = -1;
    if (env < 0) {
        const char* s = getenv("G4_DECODE_CHUNK");
        env = s ? atoi(s) : 0;
    }
    if (env > 0) return round_up((unsigned)env, kTileKeys);
    const uint64_t target = (uint64_t)2 * kCUs / (num_kv_heads ? num_kv_heads : 1);
    uint64_t c = (total_rows + target - 1) / (target ? target : 1);
    unsigned chunk = round_up((unsigned)(c < kMinChunk ? kMinChunk : c), kTileKeys);
    return chunk;
}

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int check_shape(const char* who, uint32_t nqh, uint32_t nkh, uint32_t hd) {
    if (nkh == 0 || nqh == 0 || nqh % nkh)
        return fail(G4_EINVAL, "%s: num_q_heads %u not a positive multiple of num_kv_heads %u", who, nqh, nkh);
    if (nqh / nkh > (uint32_t)kMaxGroup)
        return fail(G4_EINVAL, "%s: %u query heads per kv head (max %d)", who, nqh / nkh, kMaxGroup);
    if (hd != 256) return fail(G4_EINVAL, "%s: head_dim %u unsupported (256)", who, hd);
    return G4_OK;
}

size_t partial_bytes(uint64_t splits, uint32_t nkh, uint32_t group, uint32_t hd) {
    return align256(splits * nkh * group * 2 * sizeof(float)) + align256(splits * nkh * group * hd * sizeof(float));
}

void attended_range(uint32_t seq_len, uint32_t window, uint32_t* begin, uint32_t* end) {
    // attn_score.wgsl:23-30: rows [seq_len - W, seq_len) on local layers.
    *end = seq_len;
    *begin = (window != 0 && seq_len > window) ? seq_len - window : 0;
}

int launch_split(const DecodeArgs& a, unsigned total_splits, hipStream_t st) {
    hipLaunchKernelGGL(k_decode_split<256>, dim3(total_splits, a.num_kv_heads), dim3(kDecodeThreads), 0, st, a);
    G4_CHECK_LAUNCH("attnDecode split");
    return G4_OK;
}

int launch_merge(const DecodeArgs& a, unsigned merge_entries, hipStream_t st) {
    if (!merge_entries) return G4_OK;
    const unsigned zb = (a.group * 256 + 255) / 256;
    hipLaunchKernelGGL(k_decode_merge<256>, dim3(merge_entries, a.num_kv_heads, zb), dim3(256), 0, st, a);
    G4_CHECK_LAUNCH("attnDecode merge");
    return G4_OK;
}

int launch(const DecodeArgs& a, unsigned total_splits, unsigned merge_entries, hipStream_t st) {
    int rc = launch_split(a, total_splits, st);
    if (rc) return rc;
    return launch_merge(a, merge_entries, st);
}

}  // namespace

extern "C" {

int g4_attn_decode_workspace_size(uint32_t num_q_heads, uint32_t num_kv_heads, uint32_t head_dim,
                                  uint32_t max_seq_len, size_t* bytes) {
    if (!bytes) return fail(G4_EINVAL, "g4_attn_decode_workspace_size: bytes is NULL");
    int rc = check_shape("g4_attn_decode_workspace_size", num_q_heads, num_kv_heads, head_dim);
    if (rc) return rc;
    const uint64_t splits = (max_seq_len + kMinChunk - 1) / kMinChunk;
    *bytes = partial_bytes(splits, num_kv_heads, num_q_heads / num_kv_heads, head_dim);
    return G4_OK;
}

int g4_attn_decode(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out,
                   g4_attn_score_params p, void* workspace, size_t workspace_bytes, void* stream) {
    int rc = check_shape("attnDecode", p.num_q_heads, p.num_kv_heads, p.head_dim);
    if (rc) return rc;
    if (!q || !k_cache || !v_cache || !out) return fail(G4_EINVAL, "attnDecode: NULL pointer");
    if (p.seq_len == 0) return fail(G4_EINVAL, "attnDecode: seq_len 0");
    uint32_t kb, ke;
    attended_range(p.seq_len, p.sliding_window, &kb, &ke);
    const unsigned chunk = pick_chunk(ke - kb, p.num_kv_heads);
    const unsigned ns = (ke - kb + chunk - 1) / chunk;
    const uint32_t group = p.num_q_heads / p.num_kv_heads;
    DecodeArgs a = {};
    a.table = nullptr;
    a.one = DecodeEntryDev{q, k_cache, v_cache, out, kb, ke, 0, ns, p.scale * kLog2e, 0};
    a.n_entries = 1;
    a.num_kv_heads = p.num_kv_heads;
    a.group = group;
    a.chunk = chunk;
    if (ns > 1) {
        const size_t need = partial_bytes(ns, p.num_kv_heads, group, p.head_dim);
        if (!workspace || workspace_bytes < need)
            return fail(G4_ENOSPC, "attnDecode: workspace %zu bytes < %zu needed", workspace_bytes, need);
        a.part_ml = static_cast<float*>(workspace);
        a.part_o = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                            align256((size_t)ns * p.num_kv_heads * group * 2 * sizeof(float)));
    }
    return launch(a, ns, ns > 1 ? 1 : 0, as_stream(stream));
}

int g4_attn_decode_many_workspace_size(uint32_t n_entries, uint32_t num_q_heads, uint32_t num_kv_heads,
                                       uint32_t head_dim, uint64_t total_rows, size_t* bytes) {
    if (!bytes) return fail(G4_EINVAL, "g4_attn_decode_many_workspace_size: bytes is NULL");
    int rc = check_shape("g4_attn_decode_many_workspace_size", num_q_heads, num_kv_heads, head_dim);
    if (rc) return rc;
    const uint64_t splits = (total_rows + kMinChunk - 1) / kMinChunk + n_entries;
    *bytes = align256((size_t)n_entries * sizeof(DecodeEntryDev)) +
             partial_bytes(splits, num_kv_heads, num_q_heads / num_kv_heads, head_dim);
    return G4_OK;
}

struct PlanRep {
    const DecodeEntryDev* table;
    float* part_ml;
    float* part_o;
    uint32_t n_entries;
    uint32_t num_kv_heads;
    uint32_t group;
    uint32_t chunk;
    uint32_t total_splits;
    uint32_t head_dim;
    uint32_t magic;
};
static_assert(sizeof(PlanRep) <= sizeof(g4_decode_plan), "plan size");
constexpr uint32_t kPlanMagic = 0x67345041u;

int g4_attn_decode_many_prepare(const g4_decode_entry* entries, uint32_t n_entries, uint32_t num_q_heads,
                                uint32_t num_kv_heads, uint32_t head_dim, void* workspace, size_t workspace_bytes,
                                g4_decode_plan* plan, void* stream) {
    int rc = check_shape("attnDecodeMany", num_q_heads, num_kv_heads, head_dim);
    if (rc) return rc;
    if (!plan) return fail(G4_EINVAL, "attnDecodeMany: plan is NULL");
    if (!entries || n_entries == 0) return fail(G4_EINVAL, "attnDecodeMany: no entries");
    if (n_entries > 65535) return fail(G4_EINVAL, "attnDecodeMany: %u entries (max 65535)", n_entries);
    uint64_t total_rows = 0;
    for (uint32_t i = 0; i < n_entries; i++) {
        const g4_decode_entry& e = entries[i];
        if (!e.q || !e.k_cache || !e.v_cache || !e.out) return fail(G4_EINVAL, "attnDecodeMany: entry %u has NULL", i);
        if (e.seq_len == 0) return fail(G4_EINVAL, "attnDecodeMany: entry %u seq_len 0", i);
        uint32_t kb, ke;
        attended_range(e.seq_len, e.sliding_window, &kb, &ke);
        total_rows += ke - kb;
    }
    const unsigned chunk = pick_chunk(total_rows, num_kv_heads);
    const uint32_t group = num_q_heads / num_kv_heads;
    // Pinned staging for the table, reused once the previous upload has completed.
    static thread_local DecodeEntryDev* staging = nullptr;
    static thread_local uint32_t staging_cap = 0;
    static thread_local hipEvent_t staged = nullptr;
    if (!staged) G4_CHECK_HIP(hipEventCreateWithFlags(&staged, hipEventDisableTiming));
    G4_CHECK_HIP(hipEventSynchronize(staged));
    if (staging_cap < n_entries) {
        if (staging) G4_CHECK_HIP(hipHostFree(staging));
        staging = nullptr;
        staging_cap = 0;
        G4_CHECK_HIP(hipHostMalloc((void**)&staging, (size_t)n_entries * sizeof(DecodeEntryDev), hipHostMallocDefault));
        staging_cap = n_entries;
    }
    uint64_t total_splits = 0;
    for (uint32_t i = 0; i < n_entries; i++) {
        const g4_decode_entry& e = entries[i];
        uint32_t kb, ke;
        attended_range(e.seq_len, e.sliding_window, &kb, &ke);
        const unsigned ns = (ke - kb + chunk - 1) / chunk;
        staging[i] = DecodeEntryDev{e.q, e.k_cache, e.v_cache, e.out, kb, ke, (uint32_t)total_splits, ns,
                                    e.scale * kLog2e, 0};
        total_splits += ns;
    }
    if (total_splits > 0x7fffffffu) return fail(G4_EINVAL, "attnDecodeMany: too many splits");
    const size_t table_bytes = align256((size_t)n_entries * sizeof(DecodeEntryDev));
    const size_t need = table_bytes + partial_bytes(total_splits, num_kv_heads, group, head_dim);
    if (!workspace || workspace_bytes < need)
        return fail(G4_ENOSPC, "attnDecodeMany: workspace %zu bytes < %zu needed", workspace_bytes, need);
    hipStream_t st = as_stream(stream);
    G4_CHECK_HIP(hipMemcpyAsync(workspace, staging, (size_t)n_entries * sizeof(DecodeEntryDev), hipMemcpyHostToDevice, st));
    G4_CHECK_HIP(hipEventRecord(staged, st));
    PlanRep r = {};
    r.table = static_cast<const DecodeEntryDev*>(workspace);
    char* ws = static_cast<char*>(workspace) + table_bytes;
    r.part_ml = reinterpret_cast<float*>(ws);
    r.part_o = reinterpret_cast<float*>(ws + align256((size_t)total_splits * num_kv_heads * group * 2 * sizeof(float)));
    r.n_entries = n_entries;
    r.num_kv_heads = num_kv_heads;
    r.group = group;
    r.chunk = chunk;
    r.total_splits = (uint32_t)total_splits;
    r.head_dim = head_dim;
    r.magic = kPlanMagic;
    memset(plan, 0, sizeof *plan);
    memcpy(plan, &r, sizeof r);
    return G4_OK;
}

static int plan_args(const g4_decode_plan* plan, PlanRep* r, DecodeArgs* a) {
    if (!plan) return fail(G4_EINVAL, "attnDecodeMany: plan is NULL");
    memcpy(r, plan, sizeof *r);
    if (r->magic != kPlanMagic) return fail(G4_EINVAL, "attnDecodeMany: plan was not prepared");
    *a = DecodeArgs{};
    a->table = r->table;
    a->n_entries = r->n_entries;
    a->num_kv_heads = r->num_kv_heads;
    a->group = r->group;
    a->chunk = r->chunk;
    a->part_ml = r->part_ml;
    a->part_o = r->part_o;
    return G4_OK;
}

int g4_attn_decode_many_run(const g4_decode_plan* plan, void* stream) {
    PlanRep r;
    DecodeArgs a;
    int rc = plan_args(plan, &r, &a);
    if (rc) return rc;
    return launch(a, r.total_splits, r.n_entries, as_stream(stream));
}

int g4_attn_decode_many_run_split(const g4_decode_plan* plan, void* stream) {
    PlanRep r;
    DecodeArgs a;
    int rc = plan_args(plan, &r, &a);
    if (rc) return rc;
    return launch_split(a, r.total_splits, as_stream(stream));
}

int g4_attn_decode_many_run_merge(const g4_decode_plan* plan, void* stream) {
    PlanRep r;
    DecodeArgs a;
    int rc = plan_args(plan, &r, &a);
    if (rc) return rc;
    return launch_merge(a, r.n_entries, as_stream(stream));
}

int g4_attn_decode_many(const g4_decode_entry* entries, uint32_t n_entries, uint32_t num_q_heads,
                        uint32_t num_kv_heads, uint32_t head_dim, void* workspace, size_t workspace_bytes,
                        void* stream) {
    g4_decode_plan plan;
    int rc = g4_attn_decode_many_prepare(entries, n_entries, num_q_heads, num_kv_heads, head_dim, workspace,
                                         workspace_bytes, &plan, stream);
    if (rc) return rc;
    return g4_attn_decode_many_run(&plan, stream);
}

}  // extern "C"
