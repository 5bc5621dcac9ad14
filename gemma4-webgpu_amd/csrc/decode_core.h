// Building blocks of the gfx950 flash-decoding kernels (decode.hip, step.hip):
// the per-wave tile loop on MFMA and the per-workgroup combine of the four
// waves' online-softmax states. Shared so that the unfused decode and the
// fused one-launch step compute bit-identical attention.
//
// MFMA mapping (v_mfma_f32_16x16x32_f16; lane = 16*g + n)
//   Scores  S^T[16 rows x 16 cols] = K[16 rows x 32 d] * Qc^T[32 d x 16 cols].
//           Columns 0..7 hold the f16 "hi" part of q*scale*log2(e) for query
//           heads 0..7, columns 8..15 the f16 "lo" residual, so hi+lo carries
//           ~22 mantissa bits and scores keep f32-level accuracy. Lane (n, g)
//           supplies K[row n][d in 32c + 8g .. +8]: one 16-byte load.
//   Output  O^T[16 d x 16 cols] += V^T[16 d x 32 rows] * P^T[32 rows x 16 cols],
//           P split into hi/lo columns the same way. Lane (n, g) loads 8
//           16-byte pieces of V rows (lanes n = 0..15 of a row read 256
//           contiguous bytes) and transposes the 8x8 f16 block in registers
//           with v_perm_b32, so K and V go from HBM straight to registers.
//   The hi and lo columns are added with one DPP row rotation by 8.
// K and V rows are read once per token and never reused, so they are loaded
// non-temporally (streaming loads measured ~10% faster than cached ones).
#pragma once

#include "common.h"

namespace g4 {

constexpr int kDecodeWaves = 4;
constexpr int kDecodeThreads = 64 * kDecodeWaves;

template <typename T>
__device__ __forceinline__ T ldg_stream(const void* p) {
    typedef const __attribute__((address_space(1))) T* gp;
    return __builtin_nontemporal_load((gp)(p));
}

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

// One LDS-DMA instruction: lane j copies 16 bytes from its global address to
// LDS byte address lds + 16 j (lds wave-uniform). M0 carries the LDS base and
// is restored afterwards. Completion is counted by vmcnt, which the compiler
// does not track for this statement: the pipeline waits for it explicitly.
__device__ __forceinline__ void lds_dma16(const void* gaddr, uint32_t lds) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(gaddr), "s"(lds)
                 : "memory");
}

// The same with a wave-uniform 64-bit base in SGPRs and a per-lane 32-bit
// offset (the instruction's saddr form: no per-lane address arithmetic).
__device__ __forceinline__ void lds_dma16_s(uint32_t voff, const void* sbase, uint32_t lds) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\tglobal_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(voff), "s"(sbase), "s"(lds)
                 : "memory");
}

__device__ __forceinline__ const char* uniform_ptr(const char* p) {
    const uint64_t x = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x), hi = __builtin_amdgcn_readfirstlane((uint32_t)(x >> 32));
    return reinterpret_cast<const char*>(((uint64_t)hi << 32) | lo);
}


// Butterfly steps between lanes l and l ^ 16 / l ^ 32 without an LDS round trip:
// v_permlane16_swap / v_permlane32_swap exchange 16-lane rows / 32-lane halves,
// so the two results hold a lane's own value and its partner's (in either
// order: max and + commute, so every lane gets the same bits as x op partner).
__device__ __forceinline__ float max_xor16(float x) {
    const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}
__device__ __forceinline__ float add_xor16(float x) {
    const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}
__device__ __forceinline__ float add_xor32(float x) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

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

// Launches the fixed-order log-sum-exp merge of split partials (decode.hip)
// for entries 0..n_entries-1 of a.table (or a.one); entries with one split are
// skipped. max_splits: the largest n_splits among them.
// head_dim: 256 or 512.
int launch_decode_merge(const DecodeArgs& a, unsigned n_entries, unsigned max_splits, hipStream_t st,
                        unsigned head_dim = 256);
// The merges of a token's head_dim-512 step plan (a: more than 8 parts per
// entry) and head_dim-256 plan (b: at most 8, group 4 or 8) in one launch, with
// the bits of the two separate merges. Returns 1, launching nothing, when the
// plans are not of those kinds.
int launch_decode_merge_pair(const DecodeArgs& a, unsigned n_a, unsigned max_a, const DecodeArgs& b, unsigned n_b,
                             unsigned max_b, hipStream_t st);

// attn.linearOut over the entries of a decode step, with the step's merge
// folded in (decode.hip): workgroup (x, e) merges entry e's partial records
// (or reads its attnOut when the entry had one part, or when `merge` is 0),
// and workgroups x == 0 write the merged attnOut; then its waves take rows
// of seg[e]'s f16 weight like k_linear (linear.hip), each row bit-identical to
// g4_linear_f16 over the merged attnOut.
constexpr int kOutMaxSegs = 64;
struct OutSegDev {
    const uint16_t* w;  // f16 [rows][n]
    float* y;           // f32 [rows]
    uint32_t rows;
    uint32_t pad;
};
struct StepOutArgs {
    const DecodeEntryDev* ents;  // per entry: out (attnOut), split_base, n_splits
    const float* part_ml;
    const float* part_o;
    uint32_t num_kv_heads;
    uint32_t group;
    uint32_t rows_per_wave;  // even
    uint32_t merge;          // 1: entries with more than one part are merged here; 0: attnOut is final
    OutSegDev seg[kOutMaxSegs];
};
// n = num_kv_heads * group * head_dim (a multiple of 256 in [1024, 4096]);
// max_parts: the largest part count of an entry. Merges here when max_parts
// <= 8, group is 4 or 8 and num_kv_heads is 1 (otherwise the caller runs the
// merge launch first and passes merge = 0).
bool step_out_merges(unsigned max_parts, unsigned group, unsigned num_kv_heads);
int launch_step_out(StepOutArgs& a, unsigned n_entries, unsigned max_parts, unsigned head_dim, unsigned n,
                    hipStream_t st);

template <int HD>
struct DecodeDims {
    static constexpr int NC = HD / 32;   // K chunks of 32 d per score MFMA chain
    static constexpr int NB = HD / 128;  // V blocks of 16 lanes x 8 d
    static constexpr int NO = NB * 8;    // output MFMA tiles of 16 d
};

// Workgroup memory of one decode workgroup.
template <int HD, int W = kDecodeWaves>
struct DecodeSmem {
    f16x8 q[DecodeDims<HD>::NC][64];          // score B operand, lane-major
    float o[W][DecodeDims<HD>::NO * 4][32];   // per-wave outputs for the combine
    float m[W][kMaxGroup];
    float l[W][kMaxGroup];
};

// Writes 8 consecutive q values (already times scale*log2(e)) of one column as
// the lane's chunk c of the score operand: hi part in columns 0..7, lo in 8..15.
template <int HD, int W>
__device__ __forceinline__ void store_q_chunk(DecodeSmem<HD, W>& sm, int c, int lane, const float (&x)[8], bool lo_col) {
    f16x8 v;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const f16 hi = (f16)x[i];
        v[i] = lo_col ? (f16)(x[i] - (float)hi) : hi;
    }
    sm.q[c][lane] = v;
}

// Tile loads. K in score-operand layout: lane (n, g) holds K[row n][32c + 8g .. +8].
// Offsets are 32-bit bytes from the wave-uniform cache base of the kv head
// (caches are limited to 4 GiB on the host), so loads use an SGPR base and a
// VGPR offset. Rows beyond `last` are clamped to it.
template <int HD>
__device__ __forceinline__ void load_k_tile(const char* Kb, uint32_t row_bytes, unsigned last, int n, int g, unsigned kt0,
                                            f16x8 (&kr)[2][DecodeDims<HD>::NC]) {
#pragma unroll
    for (int h2 = 0; h2 < 2; h2++) {
        const uint32_t off = min(kt0 + h2 * 16 + n, last) * row_bytes + (uint32_t)g * 16u;
#pragma unroll
        for (int c = 0; c < DecodeDims<HD>::NC; c++) kr[h2][c] = ldg_stream<f16x8>(Kb + (off + c * 64u));
    }
}

// V as 16-byte row pieces: lane (n, g) holds V[row(g, t)][8(n + 16b) .. +8],
// row(g, t) = 4g + t for t < 4, 16 + 4g + (t - 4) otherwise.
__device__ __forceinline__ unsigned v_row(int g, int t) { return t < 4 ? g * 4 + t : 16 + g * 4 + (t - 4); }

template <int HD>
__device__ __forceinline__ void load_v_tile(const char* Vb, uint32_t row_bytes, unsigned last, int n, int g, unsigned kt0,
                                            u32x4 (&vr)[DecodeDims<HD>::NB][8]) {
#pragma unroll
    for (int t = 0; t < 8; t++) {
        const uint32_t off = min(kt0 + v_row(g, t), last) * row_bytes + (uint32_t)n * 16u;
#pragma unroll
        for (int b = 0; b < DecodeDims<HD>::NB; b++) vr[b][t] = ldg_stream<u32x4>(Vb + (off + b * 256u));
    }
}

// Replaces the pieces of row `row` (where loaded, including clamped loads) with
// the given f16 row held in LDS: the current token's row, not yet in the cache.
template <int HD>
__device__ __forceinline__ void override_row(unsigned last, int n, int g, unsigned kt0, unsigned row,
                                             const f16x8* knew, const f16x8* vnew,
                                             f16x8 (&kr)[2][DecodeDims<HD>::NC], u32x4 (&vr)[DecodeDims<HD>::NB][8]) {
#pragma unroll
    for (int h2 = 0; h2 < 2; h2++)
        if (min(kt0 + h2 * 16 + n, last) == row) {
#pragma unroll
            for (int c = 0; c < DecodeDims<HD>::NC; c++) kr[h2][c] = knew[c * 4 + g];
        }
#pragma unroll
    for (int t = 0; t < 8; t++)
        if (min(kt0 + v_row(g, t), last) == row) {
#pragma unroll
            for (int b = 0; b < DecodeDims<HD>::NB; b++) vr[b][t] = __builtin_bit_cast(u32x4, vnew[n + 16 * b]);
        }
}

// The score half of a tile: S^T of the tile's 32 rows for the 16 operand
// columns (two 16-row halves), from K in registers and q in LDS. After this
// the K registers are free (the next tile's K can be requested into them).
template <int HD, int W>
__device__ __forceinline__ void tile_scores(const DecodeSmem<HD, W>& sm, int lane,
                                            const f16x8 (&kreg)[2][DecodeDims<HD>::NC], f32x4 (&s)[2]) {
    constexpr int NC = DecodeDims<HD>::NC;
#pragma unroll
    for (int h2 = 0; h2 < 2; h2++) {
        s[h2] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NC; c++) s[h2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kreg[h2][c], sm.q[c][lane], s[h2], 0, 0, 0);
    }
}

// The rest of a tile: online softmax of the scores into a wave's state
// (running max m (log2 units) and sum l of its column) and the O^T
// accumulators, from V in registers. Rows at or beyond `k1` are masked
// (probability 0, as exp(-1e30 - max) == 0 in the reference); their loads
// were clamped in range. (The state is passed as separate references: wrapped
// in a struct it is not kept in registers and spills.)
template <int HD>
__device__ __forceinline__ void tile_update(const f32x4 (&s)[2], int g, bool lo_col, unsigned kt0, unsigned k1,
                                            const u32x4 (&vreg)[DecodeDims<HD>::NB][8], float& m_run, float& l_run,
                                            f32x4 (&acc)[DecodeDims<HD>::NO]) {
    constexpr int NB = DecodeDims<HD>::NB, NO = DecodeDims<HD>::NO;
    float sv[8];
    float tmax = -INFINITY;
#pragma unroll
    for (int h2 = 0; h2 < 2; h2++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float x = dpp_ror8_add(s[h2][j]);
            const unsigned row = kt0 + h2 * 16 + g * 4 + j;
            x = row < k1 ? x : -INFINITY;
            sv[h2 * 4 + j] = x;
            tmax = fmaxf(tmax, x);
        }
    tmax = max_xor16(tmax);  // max over the four lane groups of a column
    tmax = max_xor32(tmax);
    const float m_new = fmaxf(m_run, tmax);
    if (__any(m_new > m_run)) {  // rescale only when some column's running max moved
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int i = 0; i < NO; i++) acc[i] *= alpha;
    }
    m_run = m_new;
    f16x8 pop;
    float psum = 0.0f;
#pragma unroll
    for (int t = 0; t < 8; t++) {
        const float p = __builtin_amdgcn_exp2f(sv[t] - m_new);
        psum += p;
        const f16 hi = (f16)p;
        pop[t] = lo_col ? (f16)(p - (float)hi) : hi;
    }
    l_run += psum;
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
            acc[b * 8 + 2 * e2] =
                __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, lo), pop, acc[b * 8 + 2 * e2], 0, 0, 0);
            acc[b * 8 + 2 * e2 + 1] =
                __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, hi), pop, acc[b * 8 + 2 * e2 + 1], 0, 0, 0);
        }
    }
}

// Consumes one 32-row tile (already in registers) into a wave's online-softmax state.
template <int HD, int W>
__device__ __forceinline__ void tile_step(const DecodeSmem<HD, W>& sm, int lane, int g, bool lo_col, unsigned kt0,
                                          unsigned k1, const f16x8 (&kreg)[2][DecodeDims<HD>::NC],
                                          const u32x4 (&vreg)[DecodeDims<HD>::NB][8], float& m_run, float& l_run,
                                          f32x4 (&acc)[DecodeDims<HD>::NO]) {
    f32x4 s[2];
    tile_scores<HD>(sm, lane, kreg, s);
    tile_update<HD>(s, g, lo_col, kt0, k1, vreg, m_run, l_run, acc);
}

// Publishes a wave's final state to workgroup memory (sums over the 4 lane
// groups, hi + lo columns added).
template <int HD, int W>
__device__ __forceinline__ void wave_publish(DecodeSmem<HD, W>& sm, int wave, int n, int g, float m_run, float l_run,
                                             f32x4 (&acc)[DecodeDims<HD>::NO]) {
    constexpr int NO = DecodeDims<HD>::NO;
    float l = l_run;
    l = add_xor16(l);
    l = add_xor32(l);
#pragma unroll
    for (int i = 0; i < NO; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = dpp_ror8_add(acc[i][j]);
    if (n < 8) {
#pragma unroll
        for (int i = 0; i < NO; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) sm.o[wave][i * 4 + j][g * 8 + n] = acc[i][j];
        if (g == 0) {
            sm.m[wave][n] = m_run;
            sm.l[wave][n] = l;
        }
    }
}

// Combines the W waves (after a barrier) and writes either the normalised
// output out[h][d] (final) or the unnormalised partial o[h][d] with (m, l)
// per head, for the G heads of one kv head. Thread t (0..64W-1 within the
// waves that published) takes lane32 = t & 31 (head t & 7, lane group
// (t >> 3) & 3). The output columns of a head come in ROWS = 4 * NB runs of 8
// (d = ((gg*4 + j) + 16*b)*8 + e, run (b, j), e = 0..7, read from slot
// (b*8 + e)*4 + j of the published tiles); k = t >> 5 takes runs k, k + 2W, ...
// whole, or, with fewer runs than 2W, a part of run k / (2W / ROWS). Its
// stores are 16-byte vectors.
// `extra_m` (optional, per head, log2 units) with `extra_v` (one f16 row shared
// by the heads) adds a further state holding a single row of weight 1: the
// current token's row when it was not part of the tile loop.
template <int HD, int W>
__device__ __forceinline__ void wg_combine_write(const DecodeSmem<HD, W>& sm, unsigned G, bool final_out, float* out,
                                                 float* part_o, float* part_ml, const float* extra_m = nullptr,
                                                 const f16* extra_v = nullptr, int t = threadIdx.x) {
    constexpr int NB = DecodeDims<HD>::NB;
    constexpr int ROWS = 4 * NB;                        // runs of 8 columns per head and lane group
    constexpr int EPB = ROWS >= 2 * W ? 1 : 2 * W / ROWS;  // threads per run
    constexpr int E = 8 / EPB;                          // consecutive columns per thread and run
    const int lane32 = t & 31;
    const int h = lane32 & 7;
    const int gg = lane32 >> 3;
    if ((unsigned)h >= G) return;
    float mw[W], M = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; w++) {
        mw[w] = sm.m[w][h];
        M = fmaxf(M, mw[w]);
    }
    const float me = extra_m ? extra_m[h] : -INFINITY;
    M = fmaxf(M, me);
    float L = 0.0f, sc[W];
#pragma unroll
    for (int w = 0; w < W; w++) {
        sc[w] = __builtin_amdgcn_exp2f(mw[w] - M);
        L += sm.l[w][h] * sc[w];
    }
    const float se = extra_m ? __builtin_amdgcn_exp2f(me - M) : 0.0f;
    L += se;
    const float inv_l = 1.0f / L;  // L includes the extra state
    float* dst = final_out ? out + (uint64_t)h * HD : part_o + (uint64_t)h * HD;
    if (!final_out && t < 32 && gg == 0) stg<f32x2>(part_ml + h * 2, f32x2{M, L});
    const int k = t >> 5;  // 0 .. 2W-1
#pragma unroll
    for (int r0 = 0; r0 < (ROWS >= 2 * W ? ROWS : 2 * W); r0 += 2 * W) {
        const int r = (r0 + k) / EPB;  // run (b, j)
        const int e0 = ((r0 + k) % EPB) * E, j = r & 3, b = r >> 2;
        const int d0 = ((gg * 4 + j) + 16 * b) * 8 + e0;  // the E columns d0 .. d0 + E - 1
        float o[E];
#pragma unroll
        for (int e = 0; e < E; e++) {
            const int sl = (b * 8 + e0 + e) * 4 + j;
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < W; w++) v += sm.o[w][sl][lane32] * sc[w];
            if (extra_m) v += (float)extra_v[d0 + e] * se;
            o[e] = final_out ? v * inv_l : v;
        }
#pragma unroll
        for (int e = 0; e < E; e += 4) stg<f32x4>(dst + d0 + e, f32x4{o[e], o[e + 1], o[e + 2], o[e + 3]});
    }
}

}  // namespace g4
