// Fused decode attention for gfx950: attnScore -> softmax -> attnOutput of
// gemma4-webgpu (shaders/attn_score.wgsl:15-40, softmax.wgsl:7-46,
// attn_output.wgsl:7-23, dispatched at src/engine.ts:2092-2094) as one
// flash-decoding pass over the attended K/V rows, reading rows already in
// the cache (the prep or kvCacheStore has stored the current row).
//
// Work decomposition: one workgroup (4 waves) per (split, kv head). A split is
// a contiguous run of `chunk` cache rows of one problem ("entry": a layer of a
// token's stack, or a sequence of a ragged batch). Each wave walks 32-row
// tiles of the split with an online softmax (decode_core.h), the 4 waves are
// combined through LDS, and a problem with one split writes its output
// directly; otherwise the split writes (m, l, o) partials and k_decode_merge
// combines them with a fixed-order log-sum-exp. All G <= 8 query heads of a kv
// head are served by one read of each K/V row (the reference re-reads K and V
// once per query head).
#include <stdlib.h>
#include <string.h>

#include <map>
#include <mutex>
#include <vector>

#include "decode_core.h"
#include "gemv_core.h"

namespace g4 {

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
__global__ __launch_bounds__(kDecodeThreads, HD == 256 ? 2 : 1) void k_decode_split(DecodeArgs a) {
    using D = DecodeDims<HD>;
    __shared__ DecodeSmem<HD> sm;

    const unsigned split = blockIdx.x;
    const unsigned kvh = blockIdx.y;
    const DecodeEntryDev ent = find_entry(a, split);
    const unsigned s_local = split - ent.split_base;
    const unsigned k0 = ent.key_begin + s_local * a.chunk;
    const unsigned k1 = min(ent.key_end, k0 + a.chunk);
    const unsigned G = a.group;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n = lane & 15;
    const int g = lane >> 4;
    const int head = n & 7;
    const bool lo_col = n >= 8;
    const uint64_t row_stride = (uint64_t)a.num_kv_heads * HD;  // f16 elements per cache row
    // Byte offsets from the wave-uniform cache base stay 32-bit (caches are
    // limited to 4 GiB on the host), so loads use an SGPR base + VGPR offset.
    const char* Kb = reinterpret_cast<const char*>(ent.k + (uint64_t)kvh * HD);
    const char* Vb = reinterpret_cast<const char*>(ent.v + (uint64_t)kvh * HD);
    const uint32_t row_bytes = (uint32_t)row_stride * 2u;
    const unsigned last = k1 - 1;
    const unsigned nkeys = k1 - k0;
    constexpr unsigned kStride = kDecodeWaves * kTileKeys;

    // Issue the first tile before the query is read, so both latencies overlap.
    unsigned t0 = (unsigned)wave * kTileKeys;
    f16x8 kreg[2][D::NC];
    u32x4 vreg[D::NB][8];
    if (t0 < nkeys) {
        load_k_tile<HD>(Kb, row_bytes, last, n, g, k0 + t0, kreg);
        load_v_tile<HD>(Vb, row_bytes, last, n, g, k0 + t0, vreg);
    }

    // Query operand: q * scale * log2(e) as hi/lo f16 columns, built once per
    // workgroup into LDS (all waves share it).
    {
        const bool live = (unsigned)head < G;
        const float* qh = ent.q + ((uint64_t)kvh * G + (live ? head : 0)) * HD + g * 8;
        const float qs = live ? ent.qscale : 0.0f;
#pragma unroll
        for (int cc = 0; cc < D::NC / kDecodeWaves; cc++) {
            const int c = wave * (D::NC / kDecodeWaves) + cc;
            const f32x4 a4 = ldg<f32x4>(qh + c * 32);
            const f32x4 b4 = ldg<f32x4>(qh + c * 32 + 4);
            float x[8];
#pragma unroll
            for (int i = 0; i < 8; i++) x[i] = (i < 4 ? a4[i] : b4[i - 4]) * qs;
            store_q_chunk<HD>(sm, c, lane, x, lo_col);
        }
    }
    __syncthreads();

    float m_run = -INFINITY, l_run = 0.0f;
    f32x4 acc[D::NO];
#pragma unroll
    for (int i = 0; i < D::NO; i++) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (t0 < nkeys) {  // the first tile was requested above; the loop requests its own
        tile_step<HD>(sm, lane, g, lo_col, k0 + t0, k1, kreg, vreg, m_run, l_run, acc);
        for (t0 += kStride; t0 < nkeys; t0 += kStride) {
            load_k_tile<HD>(Kb, row_bytes, last, n, g, k0 + t0, kreg);
            load_v_tile<HD>(Vb, row_bytes, last, n, g, k0 + t0, vreg);
            tile_step<HD>(sm, lane, g, lo_col, k0 + t0, k1, kreg, vreg, m_run, l_run, acc);
        }
    }
    wave_publish<HD>(sm, wave, n, g, m_run, l_run, acc);
    __syncthreads();
    const uint64_t pidx = ((uint64_t)split * a.num_kv_heads + kvh) * G;
    wg_combine_write<HD>(sm, G, ent.n_splits == 1, ent.out + (uint64_t)kvh * G * HD, a.part_o + pidx * HD,
                         a.part_ml + pidx * 2);
}

// Fixed-order log-sum-exp merge of the split partials: one workgroup per
// (entry, kv head x query head, column chunk). The dc = HD / n_chunks columns
// of a chunk are read as float4 by R = dc / 4 threads per record; the
// P = 256 / R thread groups take records s = grp, grp + P, ... (a fixed
// assignment). Each thread requests a batch of its records' (m, l) and
// columns at once and folds them into a running (m, l, o) in record order;
// the groups' results are then rescaled to the common max and added in group
// order, so the result does not depend on scheduling. A merge of up to
// kMergeBatch * P records waits on memory once; long merges use more chunks
// (P = 4 * chunks), spreading their records over more CUs.
constexpr int kMergeThreads = 256;
constexpr int kMergeBatch = 8;
constexpr int kMaxMergeSplits = 8192;
constexpr unsigned kMaxMergeChunks = 16;

// The merge kernels take scalars and pointers (preloaded into SGPRs at wave
// start; decode.hip is compiled with kernarg preloading): the entry is then
// one batch of scalar loads from the table, or the single entry's fields
// passed by value when there is no table.

__device__ __forceinline__ DecodeEntryDev merge_entry(const DecodeEntryDev* table, float* one_out,
                                                      uint32_t one_split_base, uint32_t one_splits, unsigned bx) {
    if (table) return table[bx];
    DecodeEntryDev e{};
    e.out = one_out;
    e.split_base = one_split_base;
    e.n_splits = one_splits;
    return e;
}

// One workgroup (entry bx, query head by of its kv head, column chunk bz) of k_decode_merge.
template <int HD>
__device__ __forceinline__ void merge_body(const DecodeEntryDev* __restrict__ table, float* one_out,
                                           uint32_t one_split_base, uint32_t one_splits, float* part_ml,
                                           float* part_o, uint32_t num_kv_heads, uint32_t group, uint32_t n_chunks,
                                           unsigned bx, unsigned by, unsigned bz) {
    __shared__ f32x4 part[kMergeThreads];
    __shared__ float gm[kMergeThreads], gl[kMergeThreads];  // per group: running max, rescaled l
    const DecodeEntryDev ent = merge_entry(table, one_out, one_split_base, one_splits, bx);
    DecodeArgs a{};
    a.num_kv_heads = num_kv_heads;
    a.group = group;
    a.part_ml = part_ml;
    a.part_o = part_o;
    const unsigned ns = ent.n_splits;
    if (ns <= 1) return;
    const unsigned G = a.group;
    const unsigned kvh = by / G, h = by % G;
    const unsigned t = threadIdx.x;
    const unsigned dc = HD / n_chunks, R = dc / 4, P = kMergeThreads / R;
    const unsigned grp = t / R, q = t % R;
    const unsigned d = bz * dc + q * 4;
    const uint64_t rec_stride = (uint64_t)a.num_kv_heads * G;  // partial records per split
    const uint64_t rec0 = ((uint64_t)ent.split_base * a.num_kv_heads + kvh) * G + h;
    const float* o = a.part_o + rec0 * HD + d;
    const float* ml = a.part_ml + rec0 * 2;
    const uint64_t o_stride = rec_stride * HD;

    float m_run = -INFINITY, l_run = 0.0f;
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    for (unsigned s0 = grp; s0 < ns; s0 += kMergeBatch * P) {
        f32x4 v[kMergeBatch];
        f32x2 w[kMergeBatch];
#pragma unroll
        for (int u = 0; u < kMergeBatch; u++) {  // every request of the batch before any use
            const unsigned s = s0 + u * P;
            const bool live = s < ns;
            v[u] = live ? ldg<f32x4>(o + s * o_stride) : f32x4{0.f, 0.f, 0.f, 0.f};
            w[u] = live ? ldg<f32x2>(ml + s * rec_stride * 2) : f32x2{-INFINITY, 0.f};
        }
        float mb = m_run;
#pragma unroll
        for (int u = 0; u < kMergeBatch; u++) mb = fmaxf(mb, w[u][0]);
        const float c = mb == m_run ? 1.0f : __builtin_amdgcn_exp2f(m_run - mb);  // also 1 while both are -inf
        acc *= c;
        l_run *= c;
#pragma unroll
        for (int u = 0; u < kMergeBatch; u++) {
            if (s0 + u * P < ns) {
                // A record whose keys were all masked (a prefill part past a token's
                // position: m = -inf, l = 0, o = 0) weighs 0; exp2(-inf - -inf) would be NaN
                // while every record of this group so far is of that kind.
                const float f = w[u][0] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(w[u][0] - mb);
                acc += v[u] * f;
                l_run += w[u][1] * f;
            }
        }
        m_run = mb;
    }
    if (q == 0) gm[grp] = m_run;
    __syncthreads();
    float M = gm[0];
    for (unsigned g2 = 1; g2 < P; g2++) M = fmaxf(M, gm[g2]);
    const float sc = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - M);  // a group without records
    part[t] = acc * sc;
    if (q == 0) gl[grp] = l_run * sc;
    __syncthreads();
    if (grp == 0) {
        f32x4 sum = part[q];
        float L = gl[0];
        for (unsigned g2 = 1; g2 < P; g2++) {
            sum += part[g2 * R + q];
            L += gl[g2];
        }
        stg<f32x4>(ent.out + ((uint64_t)kvh * G + h) * HD + d, sum / L);
    }
}

template <int HD>
__global__ __launch_bounds__(kMergeThreads) void k_decode_merge(const DecodeEntryDev* __restrict__ table, float* one_out,
                                                                uint32_t one_split_base, uint32_t one_splits,
                                                                float* part_ml, float* part_o, uint32_t num_kv_heads,
                                                                uint32_t group, uint32_t n_chunks) {
    merge_body<HD>(table, one_out, one_split_base, one_splits, part_ml, part_o, num_kv_heads, group, n_chunks,
                   blockIdx.x, blockIdx.y, blockIdx.z);
}

// The same merge for entries of at most kSmallMergeSplits records: one
// workgroup per (entry, kv head) covers all G query heads (256 / G threads per
// head, COLS = G * HD / 256 columns per thread), so a merge of many entries
// with few records (prefill tokens whose keys were cut into parts) needs G x
// fewer workgroups. Every record's (m, l) and columns are requested at once
// (indexes clamped to the last record; the extra ones weigh 0), then combined
// in record order.
constexpr unsigned kSmallMergeSplits = 8;

// One query head's columns [d, d + COLS) of the first `ns` records from rec0
// (record s at rec0 + s * rec_stride), for NS slots: every (m, l) and column is
// requested at once, indexes clamped to the last record (the extra slots
// weigh 0 in merge_small_fold).
template <int HD, int COLS, int NS>
__device__ __forceinline__ void merge_small_load(const float* part_ml, const float* part_o, uint64_t rec0,
                                                 uint64_t rec_stride, unsigned ns, unsigned d,
                                                 f32x4 (&v)[NS][COLS / 4], f32x2 (&w)[NS]) {
#pragma unroll
    for (unsigned s = 0; s < (unsigned)NS; s++) {
        const uint64_t rec = rec0 + (uint64_t)min(s, ns - 1) * rec_stride;
        w[s] = ldg<f32x2>(part_ml + rec * 2);
#pragma unroll
        for (int c = 0; c < COLS / 4; c++) v[s][c] = ldg<f32x4>(part_o + rec * HD + d + 4 * c);
    }
}

// The merged columns: common max M, then the rescaled l and o summed in record
// order, o / l.
template <int COLS, int NS>
__device__ __forceinline__ void merge_small_fold(const f32x4 (&v)[NS][COLS / 4], const f32x2 (&w)[NS], unsigned ns,
                                                 f32x4 (&res)[COLS / 4]) {
    float M = w[0][0];
#pragma unroll
    for (unsigned s = 1; s < (unsigned)NS; s++)
        if (s < ns) M = fmaxf(M, w[s][0]);
    float L = 0.0f;
    f32x4 acc[COLS / 4];
#pragma unroll
    for (int c = 0; c < COLS / 4; c++) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (unsigned s = 0; s < (unsigned)NS; s++) {  // M is finite: every token attends at least its own key
        const float f = s < ns && w[s][0] != -INFINITY ? __builtin_amdgcn_exp2f(w[s][0] - M) : 0.0f;
        L += w[s][1] * f;
#pragma unroll
        for (int c = 0; c < COLS / 4; c++) acc[c] += v[s][c] * f;
    }
#pragma unroll
    for (int c = 0; c < COLS / 4; c++) res[c] = acc[c] / L;
}

// NS: the launch's largest split count rounded up to 2, 4 or 8 (records past an entry's own count
// are not loaded).
template <int HD, int COLS, int NS>
__device__ __forceinline__ void merge_small_body(const DecodeEntryDev* __restrict__ table, float* one_out,
                                                 uint32_t one_split_base, uint32_t one_splits, float* part_ml,
                                                 float* part_o, uint32_t num_kv_heads, uint32_t group, unsigned bx,
                                                 unsigned by) {
    constexpr unsigned TPH = HD / COLS;  // threads per query head
    const DecodeEntryDev ent = merge_entry(table, one_out, one_split_base, one_splits, bx);
    const unsigned ns = ent.n_splits;
    if (ns <= 1) return;
    const unsigned G = group, kvh = by;
    const unsigned h = threadIdx.x / TPH, d = (threadIdx.x % TPH) * COLS;
    if (h >= G) return;
    const uint64_t rec_stride = (uint64_t)num_kv_heads * G;  // partial records per split
    const uint64_t rec0 = ((uint64_t)ent.split_base * num_kv_heads + kvh) * G + h;
    f32x4 v[NS][COLS / 4];
    f32x2 w[NS];
    merge_small_load<HD, COLS, NS>(part_ml, part_o, rec0, rec_stride, ns, d, v, w);
    f32x4 res[COLS / 4];
    merge_small_fold<COLS, NS>(v, w, ns, res);
    float* out = ent.out + ((uint64_t)kvh * G + h) * HD + d;
#pragma unroll
    for (int c = 0; c < COLS / 4; c++) stg<f32x4>(out + 4 * c, res[c]);
}

template <int HD, int COLS, int NS>
__global__ __launch_bounds__(kMergeThreads) void k_decode_merge_small(const DecodeEntryDev* __restrict__ table,
                                                                      float* one_out, uint32_t one_split_base,
                                                                      uint32_t one_splits, float* part_ml,
                                                                      float* part_o, uint32_t num_kv_heads,
                                                                      uint32_t group) {
    merge_small_body<HD, COLS, NS>(table, one_out, one_split_base, one_splits, part_ml, part_o, num_kv_heads, group,
                                   blockIdx.x, blockIdx.y);
}

// The merges of two step plans of one token in one launch (E2B's head_dim-512
// plan with many parts per entry, then its head_dim-256 plan with at most
// kSmallMergeSplits): workgroups 0 .. n_a - 1 are k_decode_merge<512>'s
// (entry, query head, chunk), the rest k_decode_merge_small<256, COLS, NS>'s
// (entry, kv head); the same arithmetic, so the same bits as the two launches.
template <int COLS, int NS>
__global__ __launch_bounds__(kMergeThreads) void k_decode_merge_pair(
    const DecodeEntryDev* __restrict__ table_a, float* ml_a, float* o_a, uint32_t nkh_a, uint32_t group_a,
    uint32_t ents_a, uint32_t chunks_a, const DecodeEntryDev* __restrict__ table_b, float* ml_b, float* o_b,
    uint32_t nkh_b, uint32_t group_b, uint32_t ents_b) {
    const unsigned heads_a = nkh_a * group_a, n_a = ents_a * heads_a * chunks_a;
    unsigned x = blockIdx.x;
    if (x < n_a) {  // uniform
        const unsigned e = x % ents_a;
        x /= ents_a;
        merge_body<512>(table_a, nullptr, 0, 0, ml_a, o_a, nkh_a, group_a, chunks_a, e, x % heads_a, x / heads_a);
    } else {
        x -= n_a;
        merge_small_body<256, COLS, NS>(table_b, nullptr, 0, 0, ml_b, o_b, nkh_b, group_b, x % ents_b, x / ents_b);
    }
}

#define MERGE_KARGS                                                                                               \
    a.table, a.one.out, a.one.split_base, a.one.n_splits, a.part_ml, a.part_o, a.num_kv_heads, a.group

template <int HD>
int launch_decode_merge_hd(const DecodeArgs& a, unsigned n_entries, unsigned max_splits, hipStream_t st) {
    if (max_splits <= kSmallMergeSplits && (a.group == 8 || a.group == 4)) {
        const dim3 grid(n_entries, a.num_kv_heads);
        const dim3 block(kMergeThreads);
        if (a.group == 8) {
            constexpr int C = HD * 8 / 256;
            if (max_splits <= 2)
                G4_LAUNCH((k_decode_merge_small<HD, C, 2>), grid, block, 0, st, MERGE_KARGS);
            else if (max_splits <= 4)
                G4_LAUNCH((k_decode_merge_small<HD, C, 4>), grid, block, 0, st, MERGE_KARGS);
            else
                G4_LAUNCH((k_decode_merge_small<HD, C, 8>), grid, block, 0, st, MERGE_KARGS);
        } else {
            constexpr int C = HD * 4 / 256;
            if (max_splits <= 2)
                G4_LAUNCH((k_decode_merge_small<HD, C, 2>), grid, block, 0, st, MERGE_KARGS);
            else if (max_splits <= 4)
                G4_LAUNCH((k_decode_merge_small<HD, C, 4>), grid, block, 0, st, MERGE_KARGS);
            else
                G4_LAUNCH((k_decode_merge_small<HD, C, 8>), grid, block, 0, st, MERGE_KARGS);
        }
        G4_CHECK_LAUNCH("attnDecode merge");
        return G4_OK;
    }
    if (max_splits > (unsigned)kMaxMergeSplits)
        return fail(G4_EINVAL, "attnDecode merge: %u splits (max %d)", max_splits, kMaxMergeSplits);
    // one round trip covers kMergeBatch * P = kMergeBatch * 4 * kMergeThreads / HD records per chunk
    constexpr unsigned kRecsPerChunk = kMergeBatch * 4 * kMergeThreads / HD;
    unsigned chunks = 1;
    while (chunks < kMaxMergeChunks && max_splits > kRecsPerChunk * chunks) chunks *= 2;
    G4_LAUNCH(k_decode_merge<HD>, dim3(n_entries, a.num_kv_heads * a.group, chunks), dim3(kMergeThreads), 0,
                       st, MERGE_KARGS, chunks);
    G4_CHECK_LAUNCH("attnDecode merge");
    return G4_OK;
}

#undef MERGE_KARGS

int launch_decode_merge_pair(const DecodeArgs& a, unsigned n_a, unsigned max_a, const DecodeArgs& b, unsigned n_b,
                             unsigned max_b, hipStream_t st) {
    if (!n_a || max_a <= kSmallMergeSplits || max_a > (unsigned)kMaxMergeSplits) return 1;
    if (!n_b || max_b <= 1 || max_b > kSmallMergeSplits || (b.group != 8 && b.group != 4)) return 1;
    constexpr unsigned kRecsPerChunk = kMergeBatch * 4 * kMergeThreads / 512;  // as launch_decode_merge_hd<512>
    unsigned chunks = 1;
    while (chunks < kMaxMergeChunks && max_a > kRecsPerChunk * chunks) chunks *= 2;
    const uint64_t wgs = (uint64_t)n_a * a.num_kv_heads * a.group * chunks + (uint64_t)n_b * b.num_kv_heads;
    if (wgs > 0x7fffffffu) return 1;
    const dim3 grid((uint32_t)wgs), block(kMergeThreads);
#define PAIR_KARGS a.table, a.part_ml, a.part_o, a.num_kv_heads, a.group, n_a, chunks, b.table, b.part_ml, b.part_o, \
                   b.num_kv_heads, b.group, n_b
    if (b.group == 8) {
        if (max_b <= 2)
            G4_LAUNCH((k_decode_merge_pair<8, 2>), grid, block, 0, st, PAIR_KARGS);
        else if (max_b <= 4)
            G4_LAUNCH((k_decode_merge_pair<8, 4>), grid, block, 0, st, PAIR_KARGS);
        else
            G4_LAUNCH((k_decode_merge_pair<8, 8>), grid, block, 0, st, PAIR_KARGS);
    } else {
        if (max_b <= 2)
            G4_LAUNCH((k_decode_merge_pair<4, 2>), grid, block, 0, st, PAIR_KARGS);
        else if (max_b <= 4)
            G4_LAUNCH((k_decode_merge_pair<4, 4>), grid, block, 0, st, PAIR_KARGS);
        else
            G4_LAUNCH((k_decode_merge_pair<4, 8>), grid, block, 0, st, PAIR_KARGS);
    }
#undef PAIR_KARGS
    G4_CHECK_LAUNCH("attnStepPair merge");
    return G4_OK;
}

int launch_decode_merge(const DecodeArgs& a, unsigned n_entries, unsigned max_splits, hipStream_t st,
                        unsigned head_dim) {
    if (!n_entries || max_splits <= 1) return G4_OK;
    if (head_dim == 512) return launch_decode_merge_hd<512>(a, n_entries, max_splits, st);
    return launch_decode_merge_hd<256>(a, n_entries, max_splits, st);
}

// attn.linearOut after a decode step (src/engine.ts:2096, the projection that
// follows the attention block), with the step's log-sum-exp merge folded in, so
// that a layer's attention output needs no launch of its own. Workgroup (x, e)
// serves entry e: when the entry was cut into parts it merges their records
// (merge_small_load / merge_small_fold: the arithmetic and record order of
// k_decode_merge_small, so the values are bit-identical to the merge launch's),
// keeps the merged attnOut in LDS, and workgroups with x == 0 also write it to
// the entry's attnOut; otherwise it reads attnOut. Its four waves then take
// rows_per_wave rows each of seg[e]'s weight, two at a time, with k_linear's
// row arithmetic (gemv_core.h), so each row is bit-identical to g4_linear_f16
// over the merged attnOut. The first row pair's weights are requested after
// the records and before the merge arithmetic, so they arrive under it.
// NS > 1: the merged form (one kv head; COLS = group * HD / 256 columns per
// thread, NJ = COLS); NS = 1: every entry's attnOut is final.
template <int HD, int COLS, int NS, int NJ>
__global__ __launch_bounds__(256) void k_step_out(StepOutArgs a) {
    constexpr unsigned N = NJ * 256;
    __shared__ float xs[NS > 1 ? N : 4];
    const unsigned e = blockIdx.y;
    const DecodeEntryDev ent = a.ents[e];
    const OutSegDev sg = a.seg[e];
    const unsigned t = threadIdx.x, lane = t & 63, lq = lane & 31, half = lane >> 5;
    const unsigned gw = blockIdx.x * 4 + (t >> 6);
    const unsigned rows = sg.rows;
    const unsigned r0 = gw * a.rows_per_wave;
    const unsigned r1 = min(r0 + a.rows_per_wave, rows);
    float xr[NJ][8];
    f16x8 wv[NJ];
    const uint16_t* w0 = sg.w + (uint64_t)min(r0 + half, rows - 1) * N;  // clamped: a valid address
    bool merged = false;
    if constexpr (NS > 1) {
        if (a.merge && ent.n_splits > 1) {  // uniform: the entry's fields are scalars
            merged = true;
            constexpr unsigned TPH = HD / COLS;  // threads per query head (TPH * group = 256)
            const unsigned h = t / TPH, d = (t % TPH) * COLS;
            const unsigned ns = ent.n_splits;
            f32x4 v[NS][COLS / 4];
            f32x2 w[NS];
            merge_small_load<HD, COLS, NS>(a.part_ml, a.part_o, (uint64_t)ent.split_base * a.group + h, a.group,
                                           ns, d, v, w);
            gemv_row_load<NJ>(w0, lq, wv);
            f32x4 res[COLS / 4];
            merge_small_fold<COLS, NS>(v, w, ns, res);
            float* xo = xs + h * HD + d;
#pragma unroll
            for (int c = 0; c < COLS / 4; c++) *reinterpret_cast<f32x4*>(xo + 4 * c) = res[c];
            if (blockIdx.x == 0) {
#pragma unroll
                for (int c = 0; c < COLS / 4; c++) stg<f32x4>(ent.out + h * HD + d + 4 * c, res[c]);
            }
            __syncthreads();
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const f32x4 p = *reinterpret_cast<const f32x4*>(xs + 256 * j + 8 * lq);
                const f32x4 q = *reinterpret_cast<const f32x4*>(xs + 256 * j + 8 * lq + 4);
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    xr[j][u] = p[u];
                    xr[j][u + 4] = q[u];
                }
            }
        }
    }
    if (!merged) {
        gemv_load_x<NJ>(ent.out, lq, xr);
        gemv_row_load<NJ>(w0, lq, wv);
    }
    for (unsigned r = r0; r < r1; r += 2) {
        const unsigned row = r + half;
        const bool valid = row < r1;
        if (r != r0) gemv_row_load<NJ>(sg.w + (uint64_t)(valid ? row : r1 - 1) * N, lq, wv);
        const float y = gemv_row_fold<NJ, false>(wv, xr);  // the row's value in lane 0 of the half
        if (valid && lq == 0) sg.y[row] = y;
    }
}

bool step_out_merges(unsigned max_parts, unsigned group, unsigned num_kv_heads) {
    return max_parts > 1 && max_parts <= kSmallMergeSplits && (group == 4 || group == 8) && num_kv_heads == 1;
}

namespace {

// Waves of a 256-thread kernel resident on the device at once.
unsigned resident_waves_of(const void* kernel) {
    static std::mutex mu;
    static std::map<std::pair<int, const void*>, unsigned> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find({dev, kernel});
    if (it != cache.end()) return it->second;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 256, 0) != hipSuccess || per_cu < 1) per_cu = 1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
    const unsigned w = (unsigned)per_cu * (unsigned)cus * 4;
    cache.emplace(std::make_pair(dev, kernel), w);
    return w;
}

// Rows per wave spread every entry's rows over the resident waves (at least
// one row pair per wave); grid x covers the longest entry.
template <int HD, int COLS, int NS, int NJ>
int run_step_out(StepOutArgs& a, unsigned n_entries, hipStream_t st) {
    const auto kernel = k_step_out<HD, COLS, NS, NJ>;
    uint64_t total = 0;
    unsigned max_rows = 0;
    for (unsigned i = 0; i < n_entries; i++) {
        total += a.seg[i].rows;
        max_rows = max(max_rows, a.seg[i].rows);
    }
    const uint64_t waves = resident_waves_of(reinterpret_cast<const void*>(kernel));
    uint64_t rpw = 2 * ((total + 2 * waves - 1) / (2 * waves));
    if (rpw < 2) rpw = 2;
    a.rows_per_wave = (uint32_t)rpw;
    const uint64_t wave_count = (max_rows + rpw - 1) / rpw;
    G4_LAUNCH(kernel, dim3((unsigned)((wave_count + 3) / 4), n_entries), dim3(256), 0, st, a);
    G4_CHECK_LAUNCH("attnStepOut");
    return G4_OK;
}

template <int HD, int COLS>
int run_step_out_merged(StepOutArgs& a, unsigned n_entries, unsigned max_parts, hipStream_t st) {
    if (max_parts <= 2) return run_step_out<HD, COLS, 2, COLS>(a, n_entries, st);
    if (max_parts <= 4) return run_step_out<HD, COLS, 4, COLS>(a, n_entries, st);
    return run_step_out<HD, COLS, 8, COLS>(a, n_entries, st);
}

}  // namespace

int launch_step_out(StepOutArgs& a, unsigned n_entries, unsigned max_parts, unsigned head_dim, unsigned n,
                    hipStream_t st) {
    if (a.merge) {
        if (!step_out_merges(max_parts, a.group, a.num_kv_heads) || n != a.group * head_dim)
            return fail(G4_EINVAL, "attnStepOut: internal: merge of %u parts, group %u, %u kv heads", max_parts,
                        a.group, a.num_kv_heads);
        if (head_dim == 512)
            return a.group == 8 ? run_step_out_merged<512, 16>(a, n_entries, max_parts, st)
                                : run_step_out_merged<512, 8>(a, n_entries, max_parts, st);
        return a.group == 8 ? run_step_out_merged<256, 8>(a, n_entries, max_parts, st)
                            : run_step_out_merged<256, 4>(a, n_entries, max_parts, st);
    }
    switch (n / 256) {
        case 4: return run_step_out<256, 4, 1, 4>(a, n_entries, st);
        case 5: return run_step_out<256, 4, 1, 5>(a, n_entries, st);
        case 6: return run_step_out<256, 4, 1, 6>(a, n_entries, st);
        case 7: return run_step_out<256, 4, 1, 7>(a, n_entries, st);
        case 8: return run_step_out<256, 4, 1, 8>(a, n_entries, st);
        case 9: return run_step_out<256, 4, 1, 9>(a, n_entries, st);
        case 10: return run_step_out<256, 4, 1, 10>(a, n_entries, st);
        case 11: return run_step_out<256, 4, 1, 11>(a, n_entries, st);
        case 12: return run_step_out<256, 4, 1, 12>(a, n_entries, st);
        case 13: return run_step_out<256, 4, 1, 13>(a, n_entries, st);
        case 14: return run_step_out<256, 4, 1, 14>(a, n_entries, st);
        case 15: return run_step_out<256, 4, 1, 15>(a, n_entries, st);
        case 16: return run_step_out<256, 4, 1, 16>(a, n_entries, st);
        default: return fail(G4_EINVAL, "attnStepOut: input length %u unsupported", n);
    }
}

}  // namespace g4

using namespace g4;

// ---- scratch of the allocation-free decode (g4_attn_decode_noalloc) ----------
// Split partials of one decode call in a fixed device array instead of a
// caller's workspace: records (m, l) and o for up to kNoAllocSplits splits of
// up to kNoAllocHeads query heads at head_dim up to 512. Each GPU the library
// runs on holds its own copy until the process ends.
constexpr unsigned kNoAllocSplits = 512;
constexpr unsigned kNoAllocHeads = 8;
constexpr size_t kNoAllocMlBytes = (size_t)kNoAllocSplits * kNoAllocHeads * 2 * sizeof(float);  // 32 KiB
constexpr size_t kNoAllocBytes = kNoAllocMlBytes + (size_t)kNoAllocSplits * kNoAllocHeads * 512 * sizeof(float);
static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

namespace {

// The device address of `scratch` on the current device, looked up once per
// device with that device current (the host-side name is not a device address).
int noalloc_scratch(char** out) {
    static std::mutex mu;
    static std::map<int, char*> addr;
    int dev = 0;
    G4_CHECK_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(mu);
    auto it = addr.find(dev);
    if (it == addr.end()) {
        void* p = nullptr;
        G4_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail(G4_EHIP, "attnDecodeNoAlloc: no device address for the scratch array");
        it = addr.emplace(dev, static_cast<char*>(p)).first;
    }
    *out = it->second;
    return G4_OK;
}

}  // namespace

namespace {

constexpr unsigned kMinChunk = 128;

inline unsigned round_up(unsigned x, unsigned m) { return (x + m - 1) / m * m; }


// Rows per split: about two workgroups per CU over the whole launch (one at
// head_dim 512: its accumulators take twice the registers), never fewer than
// kMinChunk rows (so the partials stay small next to the rows read), and never
// more than kMaxMergeSplits splits for the longest entry.
unsigned pick_chunk(uint64_t total_rows, uint64_t max_entry_rows, unsigned num_kv_heads, unsigned head_dim) {
    const uint64_t wgs_per_cu = head_dim == 512 ? 1 : 2;
    const uint64_t target = wgs_per_cu * device_cus() / (num_kv_heads ? num_kv_heads : 1);
    const uint64_t c = (total_rows + target - 1) / (target ? target : 1);
    unsigned chunk = round_up((unsigned)(c < kMinChunk ? kMinChunk : c), kTileKeys);
    const uint64_t floor_rows = (max_entry_rows + kMaxMergeSplits - 1) / kMaxMergeSplits;
    if (chunk < floor_rows) chunk = round_up((unsigned)floor_rows, kTileKeys);
    return chunk;
}

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int check_shape(const char* who, uint32_t nqh, uint32_t nkh, uint32_t hd) {
    if (nkh == 0 || nqh == 0 || nqh % nkh)
        return fail(G4_EINVAL, "%s: num_q_heads %u not a positive multiple of num_kv_heads %u", who, nqh, nkh);
    if (nqh / nkh > (uint32_t)kMaxGroup)
        return fail(G4_EINVAL, "%s: %u query heads per kv head (max %d)", who, nqh / nkh, kMaxGroup);
    if (hd != 256 && hd != 512) return fail(G4_EINVAL, "%s: head_dim %u unsupported (256 or 512)", who, hd);
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

int launch_split(const DecodeArgs& a, unsigned total_splits, unsigned head_dim, hipStream_t st) {
    if (head_dim == 512)
        G4_LAUNCH(k_decode_split<512>, dim3(total_splits, a.num_kv_heads), dim3(kDecodeThreads), 0, st, a);
    else
        G4_LAUNCH(k_decode_split<256>, dim3(total_splits, a.num_kv_heads), dim3(kDecodeThreads), 0, st, a);
    G4_CHECK_LAUNCH("attnDecode split");
    return G4_OK;
}

int launch(const DecodeArgs& a, unsigned total_splits, unsigned merge_entries, unsigned max_splits, unsigned head_dim,
           hipStream_t st) {
    int rc = launch_split(a, total_splits, head_dim, st);
    if (rc) return rc;
    return launch_decode_merge(a, merge_entries, max_splits, st, head_dim);
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
    if (reinterpret_cast<uintptr_t>(out) & 15) return fail(G4_EINVAL, "attnDecode: out must be 16-byte aligned");
    if (p.seq_len == 0) return fail(G4_EINVAL, "attnDecode: seq_len 0");
    uint32_t kb, ke;
    attended_range(p.seq_len, p.sliding_window, &kb, &ke);
    const unsigned chunk = pick_chunk(ke - kb, ke - kb, p.num_kv_heads, p.head_dim);
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
    return launch(a, ns, 1, ns, p.head_dim, as_stream(stream));
}

int g4_attn_decode_noalloc(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, float* out,
                           g4_attn_score_params p, void* stream) {
    int rc = check_shape("attnDecodeNoAlloc", p.num_q_heads, p.num_kv_heads, p.head_dim);
    if (rc) return rc;
    if (p.num_q_heads > kNoAllocHeads)
        return fail(G4_EINVAL, "attnDecodeNoAlloc: %u query heads (the scratch array holds at most %u)", p.num_q_heads,
                    kNoAllocHeads);
    if (!q || !k_cache || !v_cache || !out) return fail(G4_EINVAL, "attnDecodeNoAlloc: NULL pointer");
    if (reinterpret_cast<uintptr_t>(out) & 15) return fail(G4_EINVAL, "attnDecodeNoAlloc: out must be 16-byte aligned");
    if (p.seq_len == 0) return fail(G4_EINVAL, "attnDecodeNoAlloc: seq_len 0");
    uint32_t kb, ke;
    attended_range(p.seq_len, p.sliding_window, &kb, &ke);
    // g4_attn_decode's split size, raised where needed so that the splits fit the scratch array.
    unsigned chunk = pick_chunk(ke - kb, ke - kb, p.num_kv_heads, p.head_dim);
    const unsigned min_chunk = round_up((ke - kb + kNoAllocSplits - 1) / kNoAllocSplits, kTileKeys);
    if (chunk < min_chunk) chunk = min_chunk;
    const unsigned ns = (ke - kb + chunk - 1) / chunk;
    const uint32_t group = p.num_q_heads / p.num_kv_heads;
    if ((size_t)ns * p.num_q_heads > (size_t)kNoAllocSplits * kNoAllocHeads)
        return fail(G4_EINVAL, "attnDecodeNoAlloc: %u splits of %u heads exceed the scratch array", ns, p.num_q_heads);
    DecodeArgs a = {};
    a.table = nullptr;
    a.one = DecodeEntryDev{q, k_cache, v_cache, out, kb, ke, 0, ns, p.scale * kLog2e, 0};
    a.n_entries = 1;
    a.num_kv_heads = p.num_kv_heads;
    a.group = group;
    a.chunk = chunk;
    if (ns > 1) {
        char* base = nullptr;
        rc = noalloc_scratch(&base);
        if (rc) return rc;
        a.part_ml = reinterpret_cast<float*>(base);
        a.part_o = reinterpret_cast<float*>(base + kNoAllocMlBytes);
    }
    return launch(a, ns, 1, ns, p.head_dim, as_stream(stream));
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
    uint32_t max_splits;
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
    uint64_t total_rows = 0, max_rows = 0;
    for (uint32_t i = 0; i < n_entries; i++) {
        const g4_decode_entry& e = entries[i];
        if (!e.q || !e.k_cache || !e.v_cache || !e.out) return fail(G4_EINVAL, "attnDecodeMany: entry %u has NULL", i);
        if (reinterpret_cast<uintptr_t>(e.out) & 15)
            return fail(G4_EINVAL, "attnDecodeMany: entry %u out must be 16-byte aligned", i);
        if (e.seq_len == 0) return fail(G4_EINVAL, "attnDecodeMany: entry %u seq_len 0", i);
        uint32_t kb, ke;
        attended_range(e.seq_len, e.sliding_window, &kb, &ke);
        total_rows += ke - kb;
        if (ke - kb > max_rows) max_rows = ke - kb;
    }
    const unsigned chunk = pick_chunk(total_rows, max_rows, num_kv_heads, head_dim);
    const uint32_t group = num_q_heads / num_kv_heads;
    std::vector<DecodeEntryDev> staging(n_entries);
    uint64_t total_splits = 0;
    uint32_t max_splits = 0;
    for (uint32_t i = 0; i < n_entries; i++) {
        const g4_decode_entry& e = entries[i];
        uint32_t kb, ke;
        attended_range(e.seq_len, e.sliding_window, &kb, &ke);
        const unsigned ns = (ke - kb + chunk - 1) / chunk;
        staging[i] = DecodeEntryDev{e.q, e.k_cache, e.v_cache, e.out, kb, ke, (uint32_t)total_splits, ns,
                                    e.scale * kLog2e, 0};
        total_splits += ns;
        if (ns > max_splits) max_splits = ns;
    }
    if (total_splits > 0x7fffffffu) return fail(G4_EINVAL, "attnDecodeMany: too many splits");
    const size_t table_bytes = align256((size_t)n_entries * sizeof(DecodeEntryDev));
    const size_t need = table_bytes + partial_bytes(total_splits, num_kv_heads, group, head_dim);
    if (!workspace || workspace_bytes < need)
        return fail(G4_ENOSPC, "attnDecodeMany: workspace %zu bytes < %zu needed", workspace_bytes, need);
    hipStream_t st = as_stream(stream);
    rc = stage_upload(workspace, staging.data(), (size_t)n_entries * sizeof(DecodeEntryDev), st);
    if (rc) return rc;
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
    r.max_splits = max_splits;
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
    return launch(a, r.total_splits, r.n_entries, r.max_splits, r.head_dim, as_stream(stream));
}

int g4_attn_decode_many_run_split(const g4_decode_plan* plan, void* stream) {
    PlanRep r;
    DecodeArgs a;
    int rc = plan_args(plan, &r, &a);
    if (rc) return rc;
    return launch_split(a, r.total_splits, r.head_dim, as_stream(stream));
}

int g4_attn_decode_many_run_merge(const g4_decode_plan* plan, void* stream) {
    PlanRep r;
    DecodeArgs a;
    int rc = plan_args(plan, &r, &a);
    if (rc) return rc;
    return launch_decode_merge(a, r.n_entries, r.max_splits, as_stream(stream), r.head_dim);
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
