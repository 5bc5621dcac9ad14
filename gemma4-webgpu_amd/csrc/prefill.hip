// Causal prefill attention for gfx950 on MFMA (v_mfma_f32_32x32x16_f16).
//
// The reference has no prefill kernel: it runs a prompt as one decode step per
// token (src/engine.ts:2469-2475), each the attnScore -> softmax -> attnOutput
// chain of shaders/attn_score.wgsl, softmax.wgsl, attn_output.wgsl. Here token
// t of a chunk (absolute position p = start + t) attends cache rows
// [lo(p), p], lo(p) = p + 1 - W on sliding-window layers (0 when p + 1 <= W or
// W = 0), exactly the rows the decode step at position p reads; the output
// row equals that decode step's attnOut within f32/f16 rounding.
//
// Query rows: one kv head's G query heads of every token ("q-rows"
// rho = token * G + head). A workgroup takes a tile of 128 q-rows (128/G
// tokens) and a contiguous part of its key range, in groups of 32 q-rows whose
// query is held as the B operand of the score MFMA for the whole pass.
//
// Per 32-key tile (K rows and V^T blocks shared through LDS rings):
//   S^T[32 keys x 32 q-rows] = K[keys x 16 d] * Q^T[16 d x q-rows], 16 MFMAs over HD = 256.
//     The MFMA's A row m holds key pi(m) = m with bits 2 and 3 swapped, so the
//     result register r of lane l holds key 16*(r/8) + 8*(l/32) + r%8 of q-row
//     l%32: registers 8s..8s+7 are already the B operand (keys 16s + 8*(l/32)
//     .. +8) of the output MFMA for key step s.
//   online softmax per q-row in log2 units (the two half-waves hold 16 keys each)
//   O^T[32 d x 32 q-rows] += V^T[32 d x 16 keys] * P^T[16 keys x q-rows], 8 d blocks x 2 key steps.
//     V is read as 32-key V^T blocks [HD][32]: kept beside the cache by the
//     prompt prep, or transposed once per call (k_vt_blocks).
// P is rounded to f16 for the output MFMA (relative error <= 2^-11 per
// probability); scores and sums stay f32.
//
// A part that covers a tile's whole key range writes attnOut rows directly;
// otherwise it writes a partial record (m, l, unnormalised o) per q-row and
// the fixed-order log-sum-exp merge of decode.hip combines the parts.
//
// Work items (a tile's part) are spread on the host over one list per CU,
// longest first to the least loaded list, and each workgroup runs its list's
// items in a loop: a workgroup's end waits for its result stores, which cost
// ~5 us per item when every item was a workgroup of its own (prefill4k: 100 us
// with the stores skipped against 116), while in the loop they drain under the
// next item's first tiles.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_ext.h>

#include <algorithm>
#include <queue>
#include <vector>

#include "decode_core.h"

namespace g4 {

typedef float f32x16 __attribute__((ext_vector_type(16)));

// Work-item and workgroup ids straight from the builtins: this file is compiled
// with IEEE mode off, and the device library's id functions behind threadIdx
// and blockIdx (built with it on) are then called rather than inlined.
__device__ __forceinline__ unsigned tid_x() { return __builtin_amdgcn_workitem_id_x(); }
__device__ __forceinline__ unsigned wg_x() { return __builtin_amdgcn_workgroup_id_x(); }
__device__ __forceinline__ unsigned wg_y() { return __builtin_amdgcn_workgroup_id_y(); }
__device__ __forceinline__ unsigned wg_z() { return __builtin_amdgcn_workgroup_id_z(); }

constexpr int kPfWaves = 4;
constexpr int kPfThreads = 64 * kPfWaves;
constexpr int kPfRows = 32 * kPfWaves;   // q-rows per tile
constexpr int kPfKeys = 32;              // keys per tile
constexpr float kPfLazy = 15.0f;         // lazy-rescale threshold (log2 units): probabilities <= 2^15 (f16 max 65504)

struct PrefillEntryDev {
    const uint16_t* q;    // f16 [n_tokens][num_q_heads][HD]
    const uint16_t* k;    // f16 [rows][num_kv_heads][HD]
    float* out;           // f32 [n_tokens][num_q_heads][HD]
    uint32_t n_tokens;
    uint32_t start;       // position of token 0
    uint32_t window;      // 0 = full
    float qscale;         // scale * log2(e)
    const uint16_t* vt;   // V^T in 32-key blocks [kv head][block][HD][32]
    uint32_t vt_blocks;   // blocks per kv head
    uint32_t pad;
};

// One workgroup: tile `tile` of entry `entry`, keys [key_begin, key_end).
struct PrefillWorkDev {
    uint32_t entry;
    uint32_t tile;
    uint32_t key_begin;
    uint32_t key_end;
    uint32_t part;        // index among the tile's parts
    uint32_t n_parts;
    uint32_t split_base;  // record slot of (first token of the tile, part 0); token t, part s -> base + t * n_parts + s
    uint32_t pad;
};

// The kernels' scalars and record pointers. The plan's tables (entries, work
// items, lists: list l is work[lists[l] .. lists[l + 1])) come as kernel
// arguments of their own, declared __restrict__: nothing the kernel stores
// aliases them, so their loads stay scalar loads after an item's stores (a
// vector load's wait would also wait for those stores).
struct PrefillArgs {
    uint32_t num_q_heads;
    uint32_t num_kv_heads;
    uint32_t group;
    uint32_t pad;
    float* part_ml;  // [slot][num_kv_heads][group][2]
    float* part_o;   // [slot][num_kv_heads][group][HD]
};

__device__ __forceinline__ unsigned key_of_row(unsigned m) {  // swap bits 2 and 3
    return (m & ~12u) | ((m & 4u) << 1) | ((m & 8u) >> 1);
}

// ---- tiles: LDS-DMA of K rows and V^T blocks -------------------------------
//
// K rows and V^T blocks go from global memory straight into LDS
// (global_load_lds_dwordx4, no register staging), one barrier per tile; a V^T
// tile is one contiguous read. The 16-byte chunks of both LDS tiles are
// XOR-swizzled so that the MFMA operand reads hit distinct banks in every
// group of sixteen lanes (a 128-bit LDS read is served 256 bytes at a time on
// gfx950; sixteen lanes, each a different row, per LDS cycle).

template <int HD>
constexpr unsigned kPfKTileBytes = kPfKeys * HD * 2;  // one K tile; also one V^T block in global memory
constexpr unsigned kPfVtTileBytes = kPfKeys * 256 * 2;  // the V^T rows of one 256-wide output half

__device__ __forceinline__ unsigned swz_k(unsigned r) { return r & 15u; }
__device__ __forceinline__ unsigned swz_v(unsigned d) { return (d >> 2) & 3u; }

// This wave's share of a tile: HD/64 DMA instructions of K (1 KiB each: 2
// rows at head_dim 256, 1 at 512; rows past the range's last clamp to it) and
// 4 of V^T (16 rows of 64 B each). dma_k_lane gives the lane's K row and
// source chunk, dma_v_offsets its byte offsets inside a V^T half block.
template <int HD>
__device__ __forceinline__ void dma_k_lane(int wave, int lane, int i, unsigned* r, unsigned* c) {
    constexpr unsigned CPR = HD / 8, RPI = 64 / CPR;  // 16-byte chunks per K row, rows per instruction
    const unsigned inst = (HD / 64u) * wave + i;
    *r = RPI * inst + (unsigned)lane / CPR;
    *c = ((unsigned)lane % CPR) ^ swz_k(*r);
}

struct DmaVOffsets {
    uint32_t v[4];
};

__device__ __forceinline__ DmaVOffsets dma_v_offsets(int wave, int lane) {
    DmaVOffsets o;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const unsigned d = 16u * (4u * wave + i) + (unsigned)(lane >> 2);
        o.v[i] = d * 64u + ((((unsigned)lane & 3u) ^ swz_v(d)) << 4);
    }
    return o;
}

// ---- two waves per SIMD: score waves and output waves (head_dim 256) -------
//
// Each group of 32 q-rows is served by two waves that share a SIMD:
// waves 0..3 ("score waves") compute the scores and the online softmax of
// their 32 q-rows, waves 4..7 ("output waves") accumulate O^T of the same rows
// over the full head dimension and issue the tile DMAs. Wave w and w + 4 are
// placed on one SIMD, so the softmax VALU of one wave runs while the other
// wave's MFMAs hold the matrix core, and no MFMA is issued twice. The
// probabilities (f16, already in the output MFMA's B-operand layout) and each
// row's rescale factor pass through LDS lane to lane (lane l of both waves
// holds q-row l % 32), two slots per pair.
//
// Phases, one barrier each. Phase it (1 <= it <= n - 2): the score wave
// computes the scores of tile it + 1 and the probabilities of tile it (slot
// it % 2); the output wave rescales by alpha(it - 1), adds tile it - 1's
// output and issues tile it + 1 + D. Prologue: scores of tiles 0 and 1 and
// the probabilities of tile 0. Epilogue: probabilities of tile n - 1 with the
// output of tile n - 2, then the output of tile n - 1, then (m, l) to LDS for
// the output waves' stores. Both roles pass the same number of barriers.
constexpr int kPpStages = 4;  // K and V^T stages (a power of two: a tile's stage is t & 3)
struct PrefillPpSmem {
    unsigned char k[kPpStages][kPfKTileBytes<256>];  // key row r: chunk c (8 d) at r*512 + ((c ^ swz_k(r)) * 16)
    unsigned char vt[kPpStages][kPfVtTileBytes];     // d row: chunk c (8 keys) at d*64 + ((c ^ swz_v(d)) * 16)
    f16x8 p[4][2][2][64];  // [pair][slot][operand register][lane]
    float alpha[4][2][64];
    float ml[4][2][64];    // [pair][m, l][lane]
};

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Waits until at most N DMA instructions of this wave are in flight and its
// LDS reads have returned, then joins the workgroup's barrier.
template <int N>
__device__ __forceinline__ void vm_wait_barrier() {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// An output wave's 32 q-rows of 256 f32 columns to global memory, 512
// contiguous bytes per row and store instruction. Accumulator block b of lane
// (col, half) holds columns 32 b + 8 g + 4 half + 0..3 of q-row col in
// acc[b][4 g .. 4 g + 3]; stored in that layout, an instruction writes 32-byte
// pieces of 32 rows, and issuing an item's stores took ~7 us under the other
// CUs' tile traffic (~5 us this way). The columns go through 16 KiB of LDS in
// two rounds of 128 (blocks 4k .. 4k + 3, whose registers are then free; row
// r's 16-byte chunk C at r * 512 + 16 (C ^ (r % 16)): sixteen rows per sixteen
// lanes when written, sixteen chunks of one row when read, distinct banks both
// ways); each store instruction then writes rows r (lanes 0-31) and r + 16
// (lanes 32-63). Rows r < n_live go to row_ptr(r); `scale` multiplies every
// value.
template <typename RowPtr>
__device__ __forceinline__ void store_rows(const f32x16 (&acc)[8], float scale, unsigned char* lds, int lane,
                                           unsigned n_live, RowPtr row_ptr) {
    const unsigned col = (unsigned)lane & 31u, half = (unsigned)lane >> 5;
#pragma unroll
    for (int k = 0; k < 2; k++) {
#pragma unroll
        for (int b = 0; b < 4; b++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const f32x16& x = acc[4 * k + b];
                const unsigned c = 8u * b + 2u * g + half;
                *reinterpret_cast<f32x4*>(lds + col * 512u + ((c ^ (col & 15u)) << 4)) =
                    f32x4{x[4 * g] * scale, x[4 * g + 1] * scale, x[4 * g + 2] * scale, x[4 * g + 3] * scale};
            }
#pragma unroll 1
        for (unsigned r0 = 0; r0 < 16; r0 += 4) {  // four row pairs at a time (bounds the registers in flight)
            f32x4 v[4];
#pragma unroll
            for (unsigned r = r0; r < r0 + 4; r++)
                v[r - r0] = *reinterpret_cast<const f32x4*>(lds + (r + 16 * half) * 512u + ((col ^ r) << 4));
#pragma unroll
            for (unsigned r = r0; r < r0 + 4; r++)
                if (r + 16 * half < n_live) stg<f32x4>(row_ptr(r + 16 * half) + 128 * k + 4 * col, v[r - r0]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// lds_dma16_s for a kernel in which the compiler itself never uses M0 (checked
// in the assembly of k_prefill_pp: its only M0 writes are these): M0 is set
// and left, two scalar instructions fewer per DMA than saving and restoring it.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // M0 is a reserved register: clobbering it is what is meant
__device__ __forceinline__ void lds_dma16_m0(uint32_t voff, const void* sbase, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop

// One work item: the body of k_prefill_pp's loop.
__device__ __forceinline__ void prefill_pp_item(const PrefillArgs& a, const PrefillEntryDev* __restrict__ table,
                                                const PrefillWorkDev wk, PrefillPpSmem& sm) {
    constexpr int HD = 256;
    constexpr unsigned SM = kPpStages - 1;                       // stage of tile t: t & SM
    constexpr int NQ = HD / 16, KPER = HD / 64, PER = KPER + 4;  // score steps; K and all DMAs per tile and score wave
    constexpr int R = 3;                                         // LDS operand reads ahead of their MFMA
    const PrefillEntryDev& ent = table[wk.entry];
    const unsigned kvh = wg_y();
    const unsigned G = a.group, NQH = a.num_q_heads, NKH = a.num_kv_heads;
    const int lane = tid_x() & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid_x() >> 6);
    const int pair = wave & 3;
    const int half = lane >> 5;
    const int col = lane & 31;

    const unsigned rho = (unsigned)wk.tile * kPfRows + (unsigned)pair * 32u + (unsigned)col;
    const unsigned tok = rho / G, head = rho % G;
    const bool row_live = tok < ent.n_tokens;
    const unsigned tok_c = row_live ? tok : ent.n_tokens - 1;
    const unsigned kb = wk.key_begin, ke = wk.key_end, last = ke - 1;  // kb is 32-aligned
    const int n_tiles = (int)((ke - kb + kPfKeys - 1) / kPfKeys);

    const uint32_t row_bytes = NKH * HD * 2u;
    const char* Kb = reinterpret_cast<const char*>(ent.k + (uint64_t)kvh * HD);
    const char* VTb = reinterpret_cast<const char*>(ent.vt + (uint64_t)kvh * ent.vt_blocks * (HD * 32));
    const DmaVOffsets dof = dma_v_offsets(pair, lane);
    // One DMA request: the K rows of tile tk and the V^T block of tile tv (tiles past the range
    // reload its last tile into stages nobody reads).
    struct DmaTiles {
        const char* k;
        const char* v;
        uint32_t kclamp;
        uint32_t lds_k, lds_v;
    };
    uint32_t krow_off[KPER], kchunk_off[KPER];
#pragma unroll
    for (int k = 0; k < KPER; k++) {
        unsigned r, c;
        dma_k_lane<HD>(pair, lane, k, &r, &c);
        krow_off[k] = r * row_bytes;
        kchunk_off[k] = c * 16u;
    }
    auto dma_tiles = [&](unsigned tk, unsigned tv) __attribute__((always_inline)) {
        tk = __builtin_amdgcn_readfirstlane(tk);
        tv = __builtin_amdgcn_readfirstlane(tv);
        const unsigned nl = (unsigned)n_tiles - 1;
        const unsigned k0 = kb + min(tk, nl) * kPfKeys, v0 = kb + min(tv, nl) * kPfKeys;
        DmaTiles d;
        d.k = uniform_ptr(Kb + (uint64_t)k0 * row_bytes);
        d.v = uniform_ptr(VTb + (uint64_t)(v0 >> 5) * kPfKTileBytes<HD>);
        d.kclamp = __builtin_amdgcn_readfirstlane((last - k0) * row_bytes);
        d.lds_k = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sm.k[tk & SM][KPER * pair * 1024u]);
        d.lds_v = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sm.vt[tv & SM][4u * pair * 1024u]);
        return d;
    };
    auto dma_part = [&](int k, const DmaTiles& d) __attribute__((always_inline)) {
        if (k < KPER)
            lds_dma16_m0(min(krow_off[k], d.kclamp) + kchunk_off[k], d.k, d.lds_k + 1024u * k);
        else
            lds_dma16_m0(dof.v[k - KPER], d.v, d.lds_v + 1024u * (k - KPER));
    };

    if (wave < 4) {
        // ---------------- score wave ----------------
        // Each score wave also issues its quarter of every tile's DMAs (the output waves carry the
        // longer part of each phase). Phase j >= 2 requests K(j + 1) and V^T(j - 1), each two phases
        // ahead of its first reader (the score MFMAs of phase j + 2, the output MFMAs of phase
        // j + 2); the prologue requests K(0..2) and V^T(0) after q, so that the first barrier waits
        // for q and K(0) only.
        const unsigned pos = ent.start + tok_c;
        const unsigned lo = (ent.window != 0 && pos + 1 > ent.window) ? pos + 1 - ent.window : 0u;
        const unsigned hi = row_live ? pos : 0u;
        const bool dead = !row_live;
        const float qs = ent.qscale;
        // The score MFMA's B operand. The kernel uses no AGPRs: a kernel that does gets half of its
        // 256 registers (two waves per SIMD) as AGPRs, and the output wave's 128 accumulators plus
        // its operands need more than the other half.
        f16x8 qop[NQ];
        {
            const uint16_t* qr = ent.q + ((uint64_t)tok_c * NQH + kvh * G + head) * HD + 8 * half;
#pragma unroll
            for (int s = 0; s < NQ; s++) qop[s] = ldg<f16x8>(qr + 16 * s);
        }
        {
            const DmaTiles d0 = dma_tiles(0, 0), d1 = dma_tiles(1, 0), d2 = dma_tiles(2, 0);
#pragma unroll
            for (int k = 0; k < KPER; k++) dma_part(k, d0);
#pragma unroll
            for (int k = 0; k < KPER; k++) dma_part(k, d1);
#pragma unroll
            for (int k = 0; k < KPER; k++) dma_part(k, d2);
#pragma unroll
            for (int k = KPER; k < PER; k++) dma_part(k, d0);  // V^T(0)
        }
        float m_run = -INFINITY, l_run = 0.0f;
        const unsigned krow = key_of_row((unsigned)col);
        const unsigned kx = swz_k(krow);
        unsigned koff[8];  // chunk 2s + half of the key row lies at koff[s % 8] + 256 (s / 8)
#pragma unroll
        for (int b = 0; b < 8; b++) koff[b] = krow * (2u * HD) + ((((unsigned)(2 * b + half)) ^ kx) << 4);
        const unsigned span = dead ? 0u : hi - lo + 1u;

        auto scores = [&](int stage) __attribute__((always_inline)) {
            const unsigned char* kbuf = sm.k[stage];
            f32x16 sc = f32x16{};
#pragma unroll
            for (int s = 0; s < NQ; s++) {
                const f16x8 k0 = *reinterpret_cast<const f16x8*>(kbuf + koff[s & 7] + 256u * (s >> 3));
                sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(k0, qop[s], sc, 0, 0, 0);
            }
            return sc;
        };
        // Probabilities of one tile's raw scores (register r: key kt0 + 16 (r / 8) + 8 half + r % 8),
        // with the lazy update of the row's reference max (alpha: the accumulators' rescale factor, 1
        // when the reference did not move).
        auto softmax = [&](f32x16 sc, unsigned kt0, f16x8 (&pop)[2], float& alpha) __attribute__((always_inline)) {
            const unsigned rel = kt0 + 8u * (unsigned)half - lo;
#pragma unroll
            for (int r = 0; r < 16; r++)
                sc[r] = rel + (unsigned)(16 * (r >> 3) + (r & 7)) < span ? sc[r] : -INFINITY;
            float smax = sc[0];
#pragma unroll
            for (int r = 1; r < 16; r++) smax = fmaxf(smax, sc[r]);
            float tmax = smax * qs;  // the scale is positive
            {
                const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(tmax), __float_as_uint(tmax), false, false);
                tmax = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));  // max over both halves of the row
            }
            const bool move = tmax > m_run + kPfLazy;
            const float m_new = move ? tmax : m_run;
            alpha = move ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;  // 0 from -inf (acc, l are 0)
            l_run *= alpha;
            m_run = m_new;
            const float nmu = m_run == -INFINITY ? 0.0f : -m_run;
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const f16x2 h = f16x2{(f16)__builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], qs, nmu)),
                                      (f16)__builtin_amdgcn_exp2f(__builtin_fmaf(sc[r + 1], qs, nmu))};
                pop[r >> 3][r & 7] = h[0];
                pop[r >> 3][(r + 1) & 7] = h[1];
                l_run = __builtin_amdgcn_fdot2(h, f16x2{(f16)1.0f, (f16)1.0f}, l_run, false);
            }
        };
        // One phase: the NQ score MFMAs of the next tile with this tile's softmax cut into 26 slots
        // spread over them (0-7: masking and running max of two scores; 8-9: the row's reference max
        // and alpha; 10-25: one exponential each, every second one packing the f16 pair and adding it
        // to the row sum), sched_barrier(0) keeping that order. `mask` is false for tiles inside the
        // window of every row of the wave.
        auto steady = [&](bool mask, unsigned ks, unsigned kt0, const DmaTiles& tdma, f32x16& sc, f16x8 (&pout)[2],
                          f32x16& nxt, float& alpha) __attribute__((always_inline)) {
            const unsigned char* kbuf = sm.k[ks];
            f16x8 kr[NQ];
            auto kread = [&](int s) __attribute__((always_inline)) {
                kr[s] = *reinterpret_cast<const f16x8*>(kbuf + koff[s & 7] + 256u * (s >> 3));
            };
#pragma unroll
            for (int i = 0; i < R; i++) kread(i);
            const unsigned rel = kt0 + 8u * (unsigned)half - lo;
            float mx = -INFINITY, tmax = 0.0f, nmu = 0.0f;
            float p[16];
            auto slot = [&](int q) __attribute__((always_inline)) {
                if (q < 8) {
                    const int r = 2 * q;
                    if (mask) {
                        sc[r] = rel + (unsigned)(16 * (r >> 3) + (r & 7)) < span ? sc[r] : -INFINITY;
                        sc[r + 1] = rel + (unsigned)(16 * ((r + 1) >> 3) + ((r + 1) & 7)) < span ? sc[r + 1] : -INFINITY;
                    }
                    mx = fmaxf(mx, fmaxf(sc[r], sc[r + 1]));
                } else if (q == 8) {
                    tmax = mx * qs;
                    const auto sw =
                        __builtin_amdgcn_permlane32_swap(__float_as_uint(tmax), __float_as_uint(tmax), false, false);
                    tmax = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
                } else if (q == 9) {
                    const bool move = tmax > m_run + kPfLazy;
                    const float m_new = move ? tmax : m_run;
                    alpha = move ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
                    l_run *= alpha;
                    m_run = m_new;
                    nmu = m_run == -INFINITY ? 0.0f : -m_run;
                } else if (q < 26) {
                    const int r = q - 10;
                    p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], qs, nmu));
                    if (r & 1) {
                        const f16x2 h = f16x2{(f16)p[r - 1], (f16)p[r]};
                        pout[r >> 3][(r - 1) & 7] = h[0];
                        pout[r >> 3][r & 7] = h[1];
                        l_run = __builtin_amdgcn_fdot2(h, f16x2{(f16)1.0f, (f16)1.0f}, l_run, false);
                    }
                }
            };
            nxt = f32x16{};
            int q = 0;
#pragma unroll
            for (int j = 0; j < NQ; j++) {
                nxt = __builtin_amdgcn_mfma_f32_32x32x16_f16(kr[j], qop[j], nxt, 0, 0, 0);
                if (j + R < NQ) kread(j + R);
                if (j % 2 == 0 && j / 2 < PER) dma_part(j / 2, tdma);  // one instruction per two steps
#pragma unroll
                for (; q < 26 * (j + 1) / NQ; q++) slot(q);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        auto put = [&](int it, const f16x8 (&pp)[2], float alpha) __attribute__((always_inline)) {
            sm.p[pair][it & 1][0][lane] = pp[0];
            sm.p[pair][it & 1][1][lane] = pp[1];
            sm.alpha[pair][it & 1][lane] = alpha;
        };
        int t_in0, t_in1;  // tiles [t_in0, t_in1) lie inside every row's window of this wave
        {
            int a0 = dead ? 0x7fffffff : (lo > kb ? (int)((lo - kb + kPfKeys - 1) / kPfKeys) : 0);
            int a1 = dead || hi + 1 < kb ? 0 : (int)((hi + 1 - kb) / kPfKeys);
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) {
                a0 = max(a0, __shfl_xor(a0, m));
                a1 = min(a1, __shfl_xor(a1, m));
            }
            t_in0 = __builtin_amdgcn_readfirstlane(a0);
            t_in1 = __builtin_amdgcn_readfirstlane(a1);
        }
        f16x8 pa[2], pb[2];
        f32x16 sa, sb;
        float alpha;
        // Phase it + 2: K(it + 1) and V^T(it - 1) are in LDS; the phase requests K(it + 3) (into the
        // stage of K(it - 1)) and V^T(it + 1) (into the stage of V^T(it - 3)), scores tile it + 1 and
        // turns tile it into probabilities.
        auto step = [&](bool mask, int it, f32x16& sc, f16x8 (&pout)[2], f32x16& nxt) __attribute__((always_inline)) {
            const unsigned ut = (unsigned)__builtin_amdgcn_readfirstlane(it);
            vm_wait_barrier<PER>();
            float al;
            const DmaTiles d = dma_tiles(ut + 3, ut + 1);
            steady(mask, (ut + 1) & SM, kb + ut * kPfKeys, d, sc, pout, nxt, al);
            put(it, pout, al);
        };
        vm_wait_barrier<3 * KPER>();  // barrier 1: q and K(0) are in; K(1), K(2), V^T(0) may be in flight
        sa = scores(0);
        if (n_tiles == 1) {
            softmax(sa, kb, pa, alpha);
            put(0, pa, alpha);
        } else {
            vm_wait_barrier<PER>();  // barrier 2: K(1) is in LDS; every wave is past scores(0)
            {
                const DmaTiles d = dma_tiles(3, 1);
#pragma unroll
                for (int k = 0; k < PER; k++) dma_part(k, d);
            }
            sb = scores(1);
            softmax(sa, kb, pa, alpha);
            put(0, pa, alpha);
            int it = 1;
            for (; it + 1 < n_tiles && it < t_in0; it++) {
                step(true, it, sb, pb, sa);
                sb = sa;
            }
            for (; it + 2 < n_tiles && it + 1 < t_in1; it += 2) {
                step(false, it, sb, pb, sa);      // scores of tile it + 1 into sa
                step(false, it + 1, sa, pa, sb);  // scores of tile it + 2 into sb
            }
            for (; it + 1 < n_tiles; it++) {
                step(true, it, sb, pb, sa);
                sb = sa;
            }
            vm_wait_barrier<PER>();  // barrier n + 1: V^T(n - 2) is in LDS
            softmax(sb, kb + (unsigned)it * kPfKeys, pb, alpha);
            put(it, pb, alpha);
        }
        // barrier n + 2 (2 when n = 1): V^T(n - 1) is in LDS, and no DMA of this wave is in flight
        // (none may outlive the workgroup); the output waves add the last tile
        vm_wait_barrier<0>();
        sm.ml[pair][0][lane] = m_run;
        sm.ml[pair][1][lane] = l_run + __shfl_xor(l_run, 32);
        lds_barrier();
        return;
    }

    // ---------------- output wave ----------------
    f32x16 acc[8];
#pragma unroll
    for (int b = 0; b < 8; b++) acc[b] = f32x16{};
    const unsigned vx = swz_v((unsigned)col);
    unsigned voff[2];
#pragma unroll
    for (int s = 0; s < 2; s++) voff[s] = (unsigned)col * 64u + ((((unsigned)(2 * s + half)) ^ vx) << 4);
    // Tile it's output: its probabilities and alpha from the score wave's slot, the rescale when a
    // row's reference max moved, then the 16 MFMAs with the V^T operands read R ahead.
    auto output = [&](int it) __attribute__((always_inline)) {
        it = __builtin_amdgcn_readfirstlane(it);
        const unsigned char* vbuf = sm.vt[(unsigned)it & SM];
        f16x8 vr[16];
        auto vread = [&](int o) __attribute__((always_inline)) {
            vr[o] = *reinterpret_cast<const f16x8*>(vbuf + voff[o & 1] + 2048u * (o >> 1));
        };
#pragma unroll
        for (int i = 0; i < R; i++) vread(i);
        const f16x8 pin[2] = {sm.p[pair][it & 1][0][lane], sm.p[pair][it & 1][1][lane]};
        const float al = sm.alpha[pair][it & 1][lane];
        if (__any(al != 1.0f)) {
#pragma unroll
            for (int b = 0; b < 8; b++) acc[b] *= al;
        }
#pragma unroll
        for (int o = 0; o < 16; o++) {
            acc[o >> 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vr[o], pin[o & 1], acc[o >> 1], 0, 0, 0);
            if (o + R < 16) vread(o + R);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    lds_barrier();  // tile 0 is in LDS
    if (n_tiles == 1) {
        lds_barrier();
        output(0);
    } else {
        lds_barrier();  // tile 1 is in LDS
        int it = 1;
        for (; it + 1 < n_tiles; it++) {
            lds_barrier();  // tile it + 1 is in LDS
            output(it - 1);
        }
        lds_barrier();
        output(it - 1);
        lds_barrier();
        output(it);
    }
    // (m, l) of every row are in LDS, and every read of this item's tiles is done. Until the next
    // item's barrier 2, its DMAs write only K stages 0-2 and V^T stage 0: the output waves pass
    // their rows through K stage 3 and V^T stages 1-3.
    lds_barrier();
    const float m_fin = sm.ml[pair][0][lane];
    const float L = sm.ml[pair][1][lane];
    const unsigned rho0 = (unsigned)wk.tile * kPfRows + (unsigned)pair * 32u;  // the wave's first q-row
    const int live = (int)(ent.n_tokens * G) - (int)rho0;
    const unsigned n_live = live <= 0 ? 0u : live >= 32 ? 32u : (unsigned)live;
    const unsigned gs = (unsigned)__builtin_ctz(G);  // G divides 32: row r is head r % G of token tok0 + r / G
    const unsigned tok0 = rho0 >> gs;
    unsigned char* lds = pair == 0 ? sm.k[kPpStages - 1] : sm.vt[pair];
    if (wk.n_parts == 1) {
        float* out = ent.out + (uint64_t)kvh * G * HD;
        store_rows(acc, 1.0f / L, lds, lane, n_live, [&](unsigned r) __attribute__((always_inline)) {
            return out + ((uint64_t)(tok0 + (r >> gs)) * NQH + (r & (G - 1))) * HD;
        });
        return;
    }
    const unsigned tile_tok0 = (unsigned)wk.tile * kPfRows / G;
    const uint64_t slot0 = (uint64_t)wk.split_base + (uint64_t)(tok0 - tile_tok0) * wk.n_parts + wk.part;
    store_rows(acc, 1.0f, lds, lane, n_live, [&](unsigned r) __attribute__((always_inline)) {
        return a.part_o + (((slot0 + (uint64_t)(r >> gs) * wk.n_parts) * NKH + kvh) * G + (r & (G - 1))) * HD;
    });
    if (row_live && half == 0) {
        const uint64_t slot = (uint64_t)wk.split_base + (uint64_t)(tok - tile_tok0) * wk.n_parts + wk.part;
        stg<f32x2>(a.part_ml + ((slot * NKH + kvh) * G + head) * 2, f32x2{m_fin, L});
    }
}

// A workgroup runs the work items of its list (lists[l] .. lists[l + 1] of the
// work array, built on the host longest first to the least loaded list) one
// after the other: the output waves' stores of an item drain while the score
// waves load the next item's q and first tiles, and no workgroup is launched
// per item. Grid: the lists x kv heads.
__global__ __launch_bounds__(512, 1) void k_prefill_pp(PrefillArgs a, const PrefillEntryDev* __restrict__ table,
                                                      const PrefillWorkDev* __restrict__ work,
                                                      const uint32_t* __restrict__ lists) {
    __shared__ PrefillPpSmem sm;
    const unsigned l = wg_x();
    const unsigned i1 = lists[l + 1];
    for (unsigned i = lists[l]; i < i1; i++)  // i is uniform; the item's early exits hide that
        prefill_pp_item(a, table, work[__builtin_amdgcn_readfirstlane(i)], sm);
}

// ---- head_dim 512: shared scores, six waves -----------------------------------
//
// The head_dim 512 form of k_prefill_pp. A workgroup takes one 64-row half of a
// work item's 128 q-rows (grid z). Waves 2 and 3 ("score waves") compute the
// scores and softmax of 32 rows each at the full width (q in 128 registers,
// 32 score MFMAs per tile); waves 0, 1, 4 and 5 ("output waves") accumulate
// one 256-wide half of the output of one score wave's rows (wave w: rows of
// score wave 2 + (w & 1), half w >> 2; 16 MFMAs per tile). Waves are placed on
// the SIMDs round robin, so each score wave has a SIMD to itself and the two
// SIMDs left hold two output waves each: 32 MFMAs per SIMD and tile, and no
// MFMA is issued twice (the one-wave form computes the full scores in both
// halves' workgroups, 1.5x the algorithmic MFMA work).
//
// LDS: two K stages and two V^T stages of 32 KiB (a full 512-wide block), the
// probabilities and rescale factors of the two score waves. Each role DMAs
// what it reads, one phase ahead: the score waves tile t + 1's K rows while
// they score tile t (into the stage of tile t - 1), the output waves tile t's
// V^T block while they add tile t - 1 (into the stage of tile t - 2). So every
// barrier waits for all of the wave's DMAs (only the previous phase's are in
// flight). Phases as in k_prefill_pp; both roles pass n + 3 barriers for n
// tiles (3 for one tile).
struct PrefillPp512Smem {
    unsigned char k[2][kPfKeys * 512 * 2];  // key row r: chunk c (8 d) at r*1024 + ((c ^ swz_k(r)) * 16)
    unsigned char vt[2][512 * kPfKeys * 2];  // d row: chunk c (8 keys) at d*64 + ((c ^ swz_v(d)) * 16)
    f16x8 p[2][2][2][64];                    // [score wave][slot][operand register][lane]
    float alpha[2][2][64];
    float ml[2][2][64];                      // [score wave][m, l][lane]
};

__device__ __forceinline__ void vm_barrier() {
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// One work item's row half zh: the body of k_prefill_pp512's loop.
__device__ __forceinline__ void prefill_pp512_item(const PrefillArgs& a, const PrefillEntryDev* __restrict__ table,
                                                   const PrefillWorkDev wk, unsigned zh, PrefillPp512Smem& sm) {
    constexpr int HD = 512;
    constexpr int NQ = HD / 16;  // score steps
    constexpr int R = 3;         // LDS operand reads ahead of their MFMA
    const PrefillEntryDev& ent = table[wk.entry];
    const unsigned kvh = wg_y();
    const unsigned G = a.group, NQH = a.num_q_heads, NKH = a.num_kv_heads;
    const int lane = tid_x() & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid_x() >> 6);
    const bool scorer = wave == 2 || wave == 3;
    const int sw = scorer ? wave - 2 : (wave & 1);  // the score wave whose rows this wave holds
    const int half = lane >> 5;
    const int col = lane & 31;

    const unsigned rho = (unsigned)wk.tile * kPfRows + 64u * zh + (unsigned)sw * 32u + (unsigned)col;
    const unsigned tok = rho / G, head = rho % G;
    const bool row_live = tok < ent.n_tokens;
    const unsigned tok_c = row_live ? tok : ent.n_tokens - 1;
    const unsigned kb = wk.key_begin, ke = wk.key_end, last = ke - 1;  // kb is 32-aligned
    const int n_tiles = (int)((ke - kb + kPfKeys - 1) / kPfKeys);
    const uint32_t row_bytes = NKH * HD * 2u;

    if (scorer) {
        // ---------------- score wave ----------------
        const char* Kb = reinterpret_cast<const char*>(ent.k + (uint64_t)kvh * HD);
        // Rows 16 sw .. 16 sw + 15 of tile t's K into stage t & 1 (rows past the range clamp to its last).
        auto kdma = [&](int t) __attribute__((always_inline)) {
            t = __builtin_amdgcn_readfirstlane(t);
            const unsigned t0 = kb + (unsigned)t * kPfKeys;
            const char* src = uniform_ptr(Kb + (uint64_t)t0 * row_bytes);
            const uint32_t kclamp = __builtin_amdgcn_readfirstlane((last - t0) * row_bytes);
            const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sm.k[t & 1][0]);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const unsigned r = 16u * sw + (unsigned)i;  // swz_k(r) = i
                lds_dma16_s(min(r * row_bytes, kclamp) + ((((unsigned)lane) ^ (unsigned)i) << 4), src, lds + r * 1024u);
            }
        };
        kdma(0);
        const unsigned pos = ent.start + tok_c;
        const unsigned lo = (ent.window != 0 && pos + 1 > ent.window) ? pos + 1 - ent.window : 0u;
        const unsigned hi = row_live ? pos : 0u;
        const bool dead = !row_live;
        const float qs = ent.qscale;
        f16x8 qop[NQ];  // the score MFMA's B operand (the kernel uses no AGPRs)
        {
            const uint16_t* qr = ent.q + ((uint64_t)tok_c * NQH + kvh * G + head) * HD + 8 * half;
#pragma unroll
            for (int s = 0; s < NQ; s++) qop[s] = ldg<f16x8>(qr + 16 * s);
        }
        float m_run = -INFINITY, l_run = 0.0f;
        const unsigned krow = key_of_row((unsigned)col);
        const unsigned kx = swz_k(krow);
        unsigned koff[8];  // chunk 2s + half of the key row lies at koff[s % 8] + 256 (s / 8)
#pragma unroll
        for (int b = 0; b < 8; b++) koff[b] = krow * (2u * HD) + ((((unsigned)(2 * b + half)) ^ kx) << 4);
        const unsigned span = dead ? 0u : hi - lo + 1u;

        auto scores = [&](int stage) __attribute__((always_inline)) {
            const unsigned char* kbuf = sm.k[stage];
            f32x16 sc = f32x16{};
#pragma unroll
            for (int s = 0; s < NQ; s++) {
                const f16x8 k0 = *reinterpret_cast<const f16x8*>(kbuf + koff[s & 7] + 256u * (s >> 3));
                sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(k0, qop[s], sc, 0, 0, 0);
            }
            return sc;
        };
        auto softmax = [&](f32x16 sc, unsigned kt0, f16x8 (&pop)[2], float& alpha) __attribute__((always_inline)) {
            const unsigned rel = kt0 + 8u * (unsigned)half - lo;
#pragma unroll
            for (int r = 0; r < 16; r++)
                sc[r] = rel + (unsigned)(16 * (r >> 3) + (r & 7)) < span ? sc[r] : -INFINITY;
            float smax = sc[0];
#pragma unroll
            for (int r = 1; r < 16; r++) smax = fmaxf(smax, sc[r]);
            float tmax = smax * qs;  // the scale is positive
            {
                const auto swp = __builtin_amdgcn_permlane32_swap(__float_as_uint(tmax), __float_as_uint(tmax), false, false);
                tmax = fmaxf(__uint_as_float(swp[0]), __uint_as_float(swp[1]));  // max over both halves of the row
            }
            const bool move = tmax > m_run + kPfLazy;
            const float m_new = move ? tmax : m_run;
            alpha = move ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;  // 0 from -inf (acc, l are 0)
            l_run *= alpha;
            m_run = m_new;
            const float nmu = m_run == -INFINITY ? 0.0f : -m_run;
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const f16x2 h = f16x2{(f16)__builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], qs, nmu)),
                                      (f16)__builtin_amdgcn_exp2f(__builtin_fmaf(sc[r + 1], qs, nmu))};
                pop[r >> 3][r & 7] = h[0];
                pop[r >> 3][(r + 1) & 7] = h[1];
                l_run = __builtin_amdgcn_fdot2(h, f16x2{(f16)1.0f, (f16)1.0f}, l_run, false);
            }
        };
        // One phase: the NQ score MFMAs of the next tile with this tile's softmax cut into 26 slots
        // spread over them (as in k_prefill_pp).
        auto steady = [&](bool mask, int ks, unsigned kt0, f32x16& sc, f16x8 (&pout)[2], f32x16& nxt,
                          float& alpha) __attribute__((always_inline)) {
            const unsigned char* kbuf = sm.k[ks];
            f16x8 kr[NQ];
            auto kread = [&](int s) __attribute__((always_inline)) {
                kr[s] = *reinterpret_cast<const f16x8*>(kbuf + koff[s & 7] + 256u * (s >> 3));
            };
#pragma unroll
            for (int i = 0; i < R; i++) kread(i);
            const unsigned rel = kt0 + 8u * (unsigned)half - lo;
            float mx = -INFINITY, tmax = 0.0f, nmu = 0.0f;
            float p[16];
            auto slot = [&](int q) __attribute__((always_inline)) {
                if (q < 8) {
                    const int r = 2 * q;
                    if (mask) {
                        sc[r] = rel + (unsigned)(16 * (r >> 3) + (r & 7)) < span ? sc[r] : -INFINITY;
                        sc[r + 1] = rel + (unsigned)(16 * ((r + 1) >> 3) + ((r + 1) & 7)) < span ? sc[r + 1] : -INFINITY;
                    }
                    mx = fmaxf(mx, fmaxf(sc[r], sc[r + 1]));
                } else if (q == 8) {
                    tmax = mx * qs;
                    const auto swp =
                        __builtin_amdgcn_permlane32_swap(__float_as_uint(tmax), __float_as_uint(tmax), false, false);
                    tmax = fmaxf(__uint_as_float(swp[0]), __uint_as_float(swp[1]));
                } else if (q == 9) {
                    const bool move = tmax > m_run + kPfLazy;
                    const float m_new = move ? tmax : m_run;
                    alpha = move ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
                    l_run *= alpha;
                    m_run = m_new;
                    nmu = m_run == -INFINITY ? 0.0f : -m_run;
                } else if (q < 26) {
                    const int r = q - 10;
                    p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], qs, nmu));
                    if (r & 1) {
                        const f16x2 h = f16x2{(f16)p[r - 1], (f16)p[r]};
                        pout[r >> 3][(r - 1) & 7] = h[0];
                        pout[r >> 3][r & 7] = h[1];
                        l_run = __builtin_amdgcn_fdot2(h, f16x2{(f16)1.0f, (f16)1.0f}, l_run, false);
                    }
                }
            };
            nxt = f32x16{};
            int q = 0;
#pragma unroll
            for (int j = 0; j < NQ; j++) {
                nxt = __builtin_amdgcn_mfma_f32_32x32x16_f16(kr[j], qop[j], nxt, 0, 0, 0);
                if (j + R < NQ) kread(j + R);
#pragma unroll
                for (; q < 26 * (j + 1) / NQ; q++) slot(q);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        auto put = [&](int it, const f16x8 (&pp)[2], float alpha) __attribute__((always_inline)) {
            sm.p[sw][it & 1][0][lane] = pp[0];
            sm.p[sw][it & 1][1][lane] = pp[1];
            sm.alpha[sw][it & 1][lane] = alpha;
        };
        int t_in0, t_in1;  // tiles [t_in0, t_in1) lie inside every row's window of this wave
        {
            int a0 = dead ? 0x7fffffff : (lo > kb ? (int)((lo - kb + kPfKeys - 1) / kPfKeys) : 0);
            int a1 = dead || hi + 1 < kb ? 0 : (int)((hi + 1 - kb) / kPfKeys);
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) {
                a0 = max(a0, __shfl_xor(a0, m));
                a1 = min(a1, __shfl_xor(a1, m));
            }
            t_in0 = __builtin_amdgcn_readfirstlane(a0);
            t_in1 = __builtin_amdgcn_readfirstlane(a1);
        }
        f16x8 pa[2], pb[2];
        f32x16 sa, sb;
        float alpha;
        auto step = [&](bool mask, int it, f32x16& sc, f16x8 (&pout)[2], f32x16& nxt) __attribute__((always_inline)) {
            it = __builtin_amdgcn_readfirstlane(it);
            vm_barrier();  // tile it + 1's K is in LDS
            if (it + 2 < n_tiles) kdma(it + 2);  // into the stage of tile it, scored in the previous phase
            float al;
            steady(mask, (it + 1) & 1, kb + (unsigned)it * kPfKeys, sc, pout, nxt, al);
            put(it, pout, al);
        };
        vm_barrier();  // tile 0's K is in LDS
        if (n_tiles > 1) kdma(1);
        sa = scores(0);
        if (n_tiles == 1) {
            softmax(sa, kb, pa, alpha);
            put(0, pa, alpha);
        } else {
            vm_barrier();  // tile 1's K is in LDS
            if (n_tiles > 2) kdma(2);
            sb = scores(1);
            softmax(sa, kb, pa, alpha);
            put(0, pa, alpha);
            int it = 1;
            for (; it + 1 < n_tiles && it < t_in0; it++) {
                step(true, it, sb, pb, sa);
                sb = sa;
            }
            for (; it + 2 < n_tiles && it + 1 < t_in1; it += 2) {
                step(false, it, sb, pb, sa);
                step(false, it + 1, sa, pa, sb);
            }
            for (; it + 1 < n_tiles; it++) {
                step(true, it, sb, pb, sa);
                sb = sa;
            }
            lds_barrier();
            softmax(sb, kb + (unsigned)it * kPfKeys, pb, alpha);
            put(it, pb, alpha);
        }
        lds_barrier();  // the output waves add the last tile
        sm.ml[sw][0][lane] = m_run;
        sm.ml[sw][1][lane] = l_run + __shfl_xor(l_run, 32);
        lds_barrier();
        return;
    }

    // ---------------- output wave ----------------
    const int dh = wave >> 2;  // output half of the head dimension
    const char* VTb = reinterpret_cast<const char*>(ent.vt + (uint64_t)kvh * ent.vt_blocks * (HD * 32));
    // This wave's quarter of tile t's V^T block (d rows 256 dh + 128 (wave & 1) + 0..127) into stage t & 1.
    const unsigned d0 = 256u * dh + 128u * (unsigned)(wave & 1);
    uint32_t voffs[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const unsigned d = d0 + 16u * i + ((unsigned)lane >> 2);
        voffs[i] = d * 64u + ((((unsigned)lane & 3u) ^ swz_v(d)) << 4);
    }
    auto vdma = [&](int t) __attribute__((always_inline)) {
        t = __builtin_amdgcn_readfirstlane(t);
        const unsigned t0 = kb + (unsigned)t * kPfKeys;
        const char* src = uniform_ptr(VTb + (uint64_t)(t0 >> 5) * kPfKTileBytes<HD>);
        const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sm.vt[t & 1][d0 * 64u]);
#pragma unroll
        for (int i = 0; i < 8; i++) lds_dma16_s(voffs[i], src, lds + 1024u * i);
    };
    f32x16 acc[8];
#pragma unroll
    for (int b = 0; b < 8; b++) acc[b] = f32x16{};
    const unsigned vx = swz_v((unsigned)col);
    unsigned voff[2];
#pragma unroll
    for (int s = 0; s < 2; s++) voff[s] = (unsigned)col * 64u + ((((unsigned)(2 * s + half)) ^ vx) << 4);
    // Tile it's output for this half: probabilities and alpha from the score wave's slot, the
    // rescale when a row's reference max moved, the 16 MFMAs with the V^T operands read R ahead.
    auto output = [&](int it) __attribute__((always_inline)) {
        it = __builtin_amdgcn_readfirstlane(it);
        const unsigned char* vbuf = sm.vt[it & 1] + 256u * 64u * dh;
        f16x8 vr[16];
        auto vread = [&](int o) __attribute__((always_inline)) {
            vr[o] = *reinterpret_cast<const f16x8*>(vbuf + voff[o & 1] + 2048u * (o >> 1));
        };
#pragma unroll
        for (int i = 0; i < R; i++) vread(i);
        const f16x8 pin[2] = {sm.p[sw][it & 1][0][lane], sm.p[sw][it & 1][1][lane]};
        const float al = sm.alpha[sw][it & 1][lane];
        if (__any(al != 1.0f)) {
#pragma unroll
            for (int b = 0; b < 8; b++) acc[b] *= al;
        }
#pragma unroll
        for (int o = 0; o < 16; o++) {
            acc[o >> 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vr[o], pin[o & 1], acc[o >> 1], 0, 0, 0);
            if (o + R < 16) vread(o + R);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    vm_barrier();  // (tile 0's K)
    vdma(0);
    if (n_tiles == 1) {
        vm_barrier();  // tile 0's V^T is in LDS
        output(0);
    } else {
        vm_barrier();  // (tile 1's K)
        int it = 1;
        for (; it + 1 < n_tiles; it++) {
            vm_barrier();  // tile it - 1's V^T is in LDS
            vdma(it);      // into the stage of tile it - 2, added in the previous phase
            output(it - 1);
        }
        vm_barrier();
        vdma(it);  // the last tile's V^T (it = n - 1)
        output(it - 1);
        vm_barrier();
        output(it);
    }
    // (m, l) of every row are in LDS, and every read of this item's tiles is done. Until the next
    // item's barrier 1, its DMAs write only K stage 0: the output waves pass their rows through
    // K stage 1 (half 0) and V^T stage 1 (half 1), 16 KiB per wave.
    lds_barrier();
    const float m_fin = sm.ml[sw][0][lane];
    const float L = sm.ml[sw][1][lane];
    const unsigned rho0 = (unsigned)wk.tile * kPfRows + 64u * zh + (unsigned)sw * 32u;  // the wave's first q-row
    const int live = (int)(ent.n_tokens * G) - (int)rho0;
    const unsigned n_live = live <= 0 ? 0u : live >= 32 ? 32u : (unsigned)live;
    const unsigned gs = (unsigned)__builtin_ctz(G);  // G divides 32: row r is head r % G of token tok0 + r / G
    const unsigned tok0 = rho0 >> gs;
    unsigned char* lds = (dh == 0 ? sm.k[1] : sm.vt[1]) + 16384u * (unsigned)sw;
    if (wk.n_parts == 1) {
        float* out = ent.out + (uint64_t)kvh * G * HD + 256u * dh;
        store_rows(acc, 1.0f / L, lds, lane, n_live, [&](unsigned r) __attribute__((always_inline)) {
            return out + ((uint64_t)(tok0 + (r >> gs)) * NQH + (r & (G - 1))) * HD;
        });
        return;
    }
    const unsigned tile_tok0 = (unsigned)wk.tile * kPfRows / G;
    const uint64_t slot0 = (uint64_t)wk.split_base + (uint64_t)(tok0 - tile_tok0) * wk.n_parts + wk.part;
    store_rows(acc, 1.0f, lds, lane, n_live, [&](unsigned r) __attribute__((always_inline)) {
        return a.part_o + (((slot0 + (uint64_t)(r >> gs) * wk.n_parts) * NKH + kvh) * G + (r & (G - 1))) * HD +
               256u * dh;
    });
    if (row_live && half == 0 && dh == 0) {
        const uint64_t slot = (uint64_t)wk.split_base + (uint64_t)(tok - tile_tok0) * wk.n_parts + wk.part;
        stg<f32x2>(a.part_ml + ((slot * NKH + kvh) * G + head) * 2, f32x2{m_fin, L});
    }
}

// A workgroup runs the work items of its list (lists[l] .. lists[l + 1] of the
// work array, built on the host longest first to the least loaded list) one
// after the other, so that an item's result stores drain while the next item's
// q and first tiles load, and no workgroup is launched per item. Grid: the
// lists x kv heads x the two row halves.
__global__ __launch_bounds__(384, 1) void k_prefill_pp512(PrefillArgs a, const PrefillEntryDev* __restrict__ table,
                                                         const PrefillWorkDev* __restrict__ work,
                                                         const uint32_t* __restrict__ lists) {
    __shared__ PrefillPp512Smem sm;
    const unsigned l = wg_x(), zh = wg_z();
    const unsigned i1 = lists[l + 1];
    for (unsigned i = lists[l]; i < i1; i++)  // i is uniform; the item's early exits hide that
        prefill_pp512_item(a, table, work[__builtin_amdgcn_readfirstlane(i)], zh, sm);
}

// V of one cache in 32-key blocks [kv head][block][HD][32] (f16): block j holds
// rows 32 j .. 32 j + 31 (rows past the cache's end repeat its last row).
struct VtCacheDev {
    const uint16_t* v;   // f16 [rows][num_kv_heads][HD]
    uint16_t* vt;
    uint32_t rows;
    uint32_t blocks;
    uint32_t block0;     // first global block index of this cache in the launch
    uint32_t pad;
};

template <int HD>
__global__ __launch_bounds__(256) void k_vt_blocks(const VtCacheDev* caches, uint32_t n_caches, uint32_t nkh) {
    __shared__ __attribute__((aligned(16))) uint16_t tb[kPfKeys][HD + 8];
    unsigned c = 0;
    while (c + 1 < n_caches && wg_x() >= caches[c + 1].block0) c++;
    const VtCacheDev cd = caches[c];
    const unsigned blk = wg_x() - cd.block0;
    const unsigned kvh = wg_y();
#pragma unroll
    for (int i = 0; i < HD / 64; i++) {
        const unsigned piece = tid_x() + 256u * i;  // 32 keys x HD/8 chunks of 8 d
        const unsigned key = piece / (HD / 8), ch = piece % (HD / 8);
        const unsigned row = min(blk * 32u + key, cd.rows - 1);
        const u32x4 x = ldg<u32x4>(cd.v + ((uint64_t)row * nkh + kvh) * HD + ch * 8u);
        *reinterpret_cast<u32x4*>(&tb[key][ch * 8u]) = x;
    }
    __syncthreads();
    uint16_t* dst = cd.vt + ((uint64_t)kvh * cd.blocks + blk) * (HD * 32);
#pragma unroll
    for (int i = 0; i < HD / 64; i++) {
        const unsigned piece = tid_x() + 256u * i;  // HD d x 4 chunks of 8 keys
        const unsigned d = piece >> 2, kc = piece & 3u;
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; e++)
            o[e] = (uint32_t)tb[8 * kc + 2 * e][d] | ((uint32_t)tb[8 * kc + 2 * e + 1][d] << 16);
        stg<u32x4>(dst + d * 32u + kc * 8u, o);
    }
}

}  // namespace g4

using namespace g4;

namespace {

constexpr uint32_t kPrefillMagic = 0x67345046u;

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct PrefillPlanRep {
    char* ws;
    uint32_t n_entries;
    uint32_t n_work;
    uint32_t n_merge;      // merge entries (tokens of split tiles)
    uint32_t max_parts;
    uint16_t num_q_heads;
    uint16_t num_kv_heads;
    uint16_t head_dim;     // 256 or 512
    uint16_t n_lists;      // workgroup lists (at most one per CU)
    uint32_t magic;
    uint32_t off_work, off_merge, off_ml, off_o;  // workspace byte offsets (workspaces stay under 4 GiB)
    uint32_t off_vtc;      // V^T cache table
    uint32_t n_vtc;        // caches to transpose (none when every entry brings its V^T cache)
    uint32_t vt_blocks;    // their 32-key blocks, in total
};
static_assert(sizeof(PrefillPlanRep) <= sizeof(g4_decode_plan), "plan size");

// The key range of tile `tile`: [lo of its first token, position of its last token].
void tile_keys(const g4_prefill_entry& e, uint32_t G, uint32_t tile, uint32_t* kb, uint32_t* ke) {
    const uint32_t t0 = tile * (uint32_t)kPfRows / G;
    const uint32_t t1 = std::min(e.n_tokens, (tile + 1) * (uint32_t)kPfRows / G) - 1;
    const uint32_t p0 = e.start + t0, p1 = e.start + t1;
    *kb = (e.sliding_window != 0 && p0 + 1 > e.sliding_window) ? p0 + 1 - e.sliding_window : 0;
    *ke = p1 + 1;
}

struct Layout {
    size_t table, work, lists, merge, ml, o, vtc, vt, total;
};

// The fixed cost of a work item (its first tiles' latency, the result
// stores), in tiles, when items are spread over the workgroups' lists. A
// later item of a list waits ~5 us for its first tiles and the previous
// item's stores, the first one ~4 us; a tile takes ~1 us. Measured on
// prefill4k: 6 -> 109-110 us, 8 -> 110-113, 10 -> 111-113, 13 -> 112-114.
constexpr uint64_t kPfItemCost = 6;

// The caches whose V the pipelined form transposes: one per distinct v_cache
// of the entries without a V^T cache of their own, long enough for every
// entry on it.
struct VtPlan {
    std::vector<const uint16_t*> v;
    std::vector<uint32_t> rows, blocks, block0;
    std::vector<size_t> off;      // byte offset of each cache's blocks in the V^T region
    std::vector<uint32_t> of;     // entry -> cache
    uint32_t total_blocks = 0;
};

// Work list, merge list and workspace layout for a set of entries.
int build(const g4_prefill_entry* ents, uint32_t n, uint32_t nqh, uint32_t nkh, uint32_t hd,
          std::vector<PrefillEntryDev>* tab, std::vector<PrefillWorkDev>* work, std::vector<uint32_t>* lists,
          std::vector<DecodeEntryDev>* merge, uint32_t* max_parts, Layout* L, VtPlan* vp) {
    const uint32_t G = nqh / nkh;
    *vp = VtPlan{};
    {
        vp->of.assign(n, ~0u);
        for (uint32_t i = 0; i < n; i++) {
            const g4_prefill_entry& e = ents[i];
            if (e.vt_cache) continue;  // read from the entry's own V^T cache
            const uint32_t end = e.start + e.n_tokens;
            uint32_t c = 0;
            while (c < vp->v.size() && vp->v[c] != e.v_cache) c++;
            if (c == vp->v.size()) {
                vp->v.push_back(e.v_cache);
                vp->rows.push_back(end);
            } else if (end > vp->rows[c]) {
                vp->rows[c] = end;
            }
            vp->of[i] = c;
        }
        size_t off = 0;
        for (size_t c = 0; c < vp->v.size(); c++) {
            const uint32_t blocks = (vp->rows[c] + kPfKeys - 1) / kPfKeys;
            vp->blocks.push_back(blocks);
            vp->block0.push_back(vp->total_blocks);
            vp->off.push_back(off);
            vp->total_blocks += blocks;
            off += align256((size_t)nkh * blocks * kPfKeys * hd * 2);
        }
    }
    uint64_t slots = 0;
    *max_parts = 1;
    tab->resize(n);
    struct Item {
        PrefillWorkDev w;
        uint32_t keys;
    };
    std::vector<Item> items;
    uint32_t part_keys = 0;
    {
        // Parts about 1.15x the keys per CU of the whole call (one workgroup per CU): long query
        // tiles split so that the longest item stays near a CU's share, short ones stay whole
        // (every extra part costs a record write and its merge). prefill4k: 3008 keys; measured
        // 168 us against 177 us at 1536 and 183 us at 3840.
        uint64_t w = 0;
        for (uint32_t i = 0; i < n; i++) {
            const g4_prefill_entry& e = ents[i];
            const uint32_t tiles = (uint32_t)(((uint64_t)e.n_tokens * G + kPfRows - 1) / kPfRows);
            for (uint32_t t = 0; t < tiles; t++) {
                uint32_t kb, ke;
                tile_keys(e, G, t, &kb, &ke);
                w += ke - (kb & ~(uint32_t)(kPfKeys - 1));
            }
        }
        const uint64_t share = w * nkh * (hd / 256) * 115 / (100 * (uint64_t)device_cus());  // head_dim 512: two halves
        part_keys = (uint32_t)std::min<uint64_t>(std::max<uint64_t>(share, 256), 1u << 30);
        part_keys = (part_keys + kPfKeys - 1) / kPfKeys * kPfKeys;
    }
    for (uint32_t i = 0; i < n; i++) {
        const g4_prefill_entry& e = ents[i];
        const uint32_t vt_blocks = e.vt_cache ? (e.vt_rows + kPfKeys - 1) / kPfKeys : vp->blocks[vp->of[i]];
        (*tab)[i] = PrefillEntryDev{e.q, e.k_cache, e.out, e.n_tokens, e.start, e.sliding_window,
                                    e.scale * kLog2e, e.vt_cache, vt_blocks, 0u};
        const uint32_t tiles = (uint32_t)(((uint64_t)e.n_tokens * G + kPfRows - 1) / kPfRows);
        for (uint32_t t = 0; t < tiles; t++) {
            uint32_t kb, ke;
            tile_keys(e, G, t, &kb, &ke);
            kb &= ~(uint32_t)(kPfKeys - 1);  // tiles are 32-aligned
            const uint32_t nk = ke - kb;
            const uint32_t parts = (nk + part_keys - 1) / part_keys;
            const uint32_t tok0 = t * (uint32_t)kPfRows / G;
            const uint32_t ntok = std::min(e.n_tokens, (t + 1) * (uint32_t)kPfRows / G) - tok0;
            const uint32_t base = parts > 1 ? (uint32_t)slots : 0u;
            for (uint32_t p = 0; p < parts; p++) {
                const uint32_t b0 = kb + p * part_keys, b1 = std::min(ke, b0 + part_keys);
                items.push_back(Item{PrefillWorkDev{i, t, b0, b1, p, parts, base, 0}, b1 - b0});
            }
            if (parts > 1) {
                for (uint32_t tk = 0; tk < ntok; tk++)
                    merge->push_back(DecodeEntryDev{nullptr, nullptr, nullptr,
                                                    e.out + (uint64_t)(tok0 + tk) * nqh * hd, 0, 0,
                                                    base + tk * parts, parts, 0.0f, 0});
                slots += (uint64_t)ntok * parts;
                *max_parts = std::max(*max_parts, parts);
            }
        }
    }
    // One list per workgroup running at once (one per CU; an item takes num_kv_heads workgroups,
    // twice that at head_dim 512): the items, longest first, each to the least loaded list (its
    // tiles plus the fixed cost of an item). A list's items lie together in the work array.
    std::stable_sort(items.begin(), items.end(), [](const Item& x, const Item& y) { return x.keys > y.keys; });
    const uint32_t wgs_per_item = nkh * (hd / 256);
    const uint32_t n_lists = (uint32_t)std::min<uint64_t>(std::max(1u, (uint32_t)device_cus() / wgs_per_item),
                                                          std::max<size_t>(items.size(), 1));
    std::vector<std::vector<uint32_t>> member(n_lists);
    {
        using Load = std::pair<uint64_t, uint32_t>;  // (load, list): the smallest load first, then the lowest list
        std::priority_queue<Load, std::vector<Load>, std::greater<Load>> heap;
        for (uint32_t l = 0; l < n_lists; l++) heap.push({0, l});
        for (uint32_t i = 0; i < items.size(); i++) {
            const Load top = heap.top();
            heap.pop();
            member[top.second].push_back(i);
            heap.push({top.first + (items[i].keys + kPfKeys - 1) / kPfKeys + kPfItemCost, top.second});
        }
    }
    work->clear();
    lists->assign(1, 0u);
    for (const auto& m : member) {
        for (uint32_t i : m) work->push_back(items[i].w);
        lists->push_back((uint32_t)work->size());
    }
    if (work->size() > 0x7fffffffu || slots > 0x7fffffffu) return fail(G4_EINVAL, "attnPrefill: too much work");
    size_t off = 0;
    L->table = off;
    off += align256(n * sizeof(PrefillEntryDev));
    L->work = off;
    off += align256(work->size() * sizeof(PrefillWorkDev));
    L->lists = off;
    off += align256(lists->size() * sizeof(uint32_t));
    L->merge = off;
    off += align256(merge->size() * sizeof(DecodeEntryDev));
    L->vtc = off;  // the four tables are contiguous: prepare uploads them in one copy
    off += align256(vp->v.size() * sizeof(VtCacheDev));
    L->ml = off;
    off += align256(slots * nkh * G * 2 * sizeof(float));
    L->o = off;
    off += align256(slots * nkh * G * hd * sizeof(float));
    L->vt = off;
    for (size_t c = 0; c < vp->v.size(); c++) off += align256((size_t)nkh * vp->blocks[c] * kPfKeys * hd * 2);
    L->total = off;
    return G4_OK;
}

int check(const g4_prefill_entry* ents, uint32_t n, uint32_t nqh, uint32_t nkh, uint32_t hd) {
    if (!ents || n == 0) return fail(G4_EINVAL, "attnPrefill: no entries");
    if (hd != 256 && hd != 512) return fail(G4_EINVAL, "attnPrefill: head_dim %u unsupported (256 or 512)", hd);
    if (nkh == 0 || nqh % nkh || nqh / nkh > (uint32_t)kMaxGroup || 32 % (nqh / nkh))
        return fail(G4_EINVAL, "attnPrefill: %u query heads over %u kv heads unsupported", nqh, nkh);
    for (uint32_t i = 0; i < n; i++) {
        const g4_prefill_entry& e = ents[i];
        if (!e.q || !e.k_cache || !e.v_cache || !e.out) return fail(G4_EINVAL, "attnPrefill: entry %u has NULL", i);
        if (reinterpret_cast<uintptr_t>(e.out) & 15)
            return fail(G4_EINVAL, "attnPrefill: entry %u out must be 16-byte aligned", i);
        if (e.n_tokens == 0) return fail(G4_EINVAL, "attnPrefill: entry %u has no tokens", i);
        if ((uint64_t)e.start + e.n_tokens > 0xffffffffull) return fail(G4_EINVAL, "attnPrefill: entry %u range", i);
        if (e.vt_cache && (uint64_t)e.start + e.n_tokens > e.vt_rows)
            return fail(G4_EINVAL, "attnPrefill: entry %u attends rows up to %u past its V^T cache's %u rows", i,
                        e.start + e.n_tokens - 1, e.vt_rows);
    }
    return G4_OK;
}

}  // namespace

extern "C" {

int g4_attn_prefill_workspace_size(const g4_prefill_entry* entries, uint32_t n_entries, uint32_t num_q_heads,
                                   uint32_t num_kv_heads, uint32_t head_dim, size_t* bytes) {
    if (!bytes) return fail(G4_EINVAL, "g4_attn_prefill_workspace_size: bytes is NULL");
    int rc = check(entries, n_entries, num_q_heads, num_kv_heads, head_dim);
    if (rc) return rc;
    std::vector<PrefillEntryDev> tab;
    std::vector<PrefillWorkDev> work;
    std::vector<uint32_t> lists;
    std::vector<DecodeEntryDev> merge;
    uint32_t mp;
    Layout L;
    VtPlan vp;
    rc = build(entries, n_entries, num_q_heads, num_kv_heads, head_dim, &tab, &work, &lists, &merge, &mp, &L, &vp);
    if (rc) return rc;
    *bytes = L.total;
    return G4_OK;
}

int g4_attn_prefill_prepare(const g4_prefill_entry* entries, uint32_t n_entries, uint32_t num_q_heads,
                            uint32_t num_kv_heads, uint32_t head_dim, void* workspace, size_t workspace_bytes,
                            g4_decode_plan* plan, void* stream) {
    int rc = check(entries, n_entries, num_q_heads, num_kv_heads, head_dim);
    if (rc) return rc;
    if (!plan) return fail(G4_EINVAL, "attnPrefill: plan is NULL");
    std::vector<PrefillEntryDev> tab;
    std::vector<PrefillWorkDev> work;
    std::vector<uint32_t> lists;
    std::vector<DecodeEntryDev> merge;
    uint32_t max_parts;
    Layout L;
    VtPlan vp;
    rc = build(entries, n_entries, num_q_heads, num_kv_heads, head_dim, &tab, &work, &lists, &merge, &max_parts, &L, &vp);
    if (rc) return rc;
    if (max_parts > 8192) return fail(G4_EINVAL, "attnPrefill: %u key parts per tile (max 8192)", max_parts);
    if (!workspace || workspace_bytes < L.total)
        return fail(G4_ENOSPC, "attnPrefill: workspace %zu bytes < %zu needed", workspace_bytes, L.total);
    if (L.vt >= (1ull << 32)) return fail(G4_EINVAL, "attnPrefill: workspace layout exceeds 4 GiB");
    hipStream_t st = as_stream(stream);
    char* ws = static_cast<char*>(workspace);
    std::vector<VtCacheDev> vtc(vp.v.size());
    for (size_t c = 0; c < vp.v.size(); c++)
        vtc[c] = VtCacheDev{vp.v[c], reinterpret_cast<uint16_t*>(ws + L.vt + vp.off[c]), vp.rows[c], vp.blocks[c],
                            vp.block0[c], 0u};
    for (uint32_t i = 0; i < n_entries; i++)
        if (!entries[i].vt_cache) tab[i].vt = vtc[vp.of[i]].vt;
    std::vector<char> blob(L.vtc - L.table + vtc.size() * sizeof(VtCacheDev));
    memcpy(blob.data(), tab.data(), tab.size() * sizeof(PrefillEntryDev));
    memcpy(blob.data() + (L.work - L.table), work.data(), work.size() * sizeof(PrefillWorkDev));
    memcpy(blob.data() + (L.lists - L.table), lists.data(), lists.size() * sizeof(uint32_t));
    if (!merge.empty()) memcpy(blob.data() + (L.merge - L.table), merge.data(), merge.size() * sizeof(DecodeEntryDev));
    if (!vtc.empty()) memcpy(blob.data() + (L.vtc - L.table), vtc.data(), vtc.size() * sizeof(VtCacheDev));
    rc = stage_upload(ws + L.table, blob.data(), blob.size(), st);  // the four tables in one copy
    if (rc) return rc;
    PrefillPlanRep r = {};
    r.ws = ws;
    r.n_entries = n_entries;
    r.n_work = (uint32_t)work.size();
    r.n_merge = (uint32_t)merge.size();
    r.max_parts = max_parts;
    r.num_q_heads = (uint16_t)num_q_heads;  // at most 8 per kv head (checked); kv heads below 2^16
    r.num_kv_heads = (uint16_t)num_kv_heads;
    r.head_dim = (uint16_t)head_dim;
    r.magic = kPrefillMagic;
    r.off_work = (uint32_t)L.work;
    r.n_lists = (uint16_t)(lists.size() - 1);
    r.off_merge = (uint32_t)L.merge;
    r.off_ml = (uint32_t)L.ml;
    r.off_o = (uint32_t)L.o;
    r.off_vtc = (uint32_t)L.vtc;
    r.n_vtc = (uint32_t)vp.v.size();
    r.vt_blocks = vp.total_blocks;
    memset(plan, 0, sizeof *plan);
    memcpy(plan, &r, sizeof r);
    return G4_OK;
}

static int prefill_run(const g4_decode_plan* plan, void* stream, hipEvent_t start_ev, hipEvent_t stop_ev) {
    if (!plan) return fail(G4_EINVAL, "attnPrefill: plan is NULL");
    PrefillPlanRep r;
    memcpy(&r, plan, sizeof r);
    if (r.magic != kPrefillMagic) return fail(G4_EINVAL, "attnPrefill: plan was not prepared by g4_attn_prefill_prepare");
    PrefillArgs a = {};
    const PrefillEntryDev* table = reinterpret_cast<const PrefillEntryDev*>(r.ws);
    const PrefillWorkDev* work = reinterpret_cast<const PrefillWorkDev*>(r.ws + r.off_work);
    const uint32_t* lists =
        reinterpret_cast<const uint32_t*>(r.ws + r.off_work + align256((size_t)r.n_work * sizeof(PrefillWorkDev)));
    a.num_q_heads = r.num_q_heads;
    a.num_kv_heads = r.num_kv_heads;
    a.group = r.num_q_heads / r.num_kv_heads;
    a.part_ml = reinterpret_cast<float*>(r.ws + r.off_ml);
    a.part_o = reinterpret_cast<float*>(r.ws + r.off_o);
    hipStream_t st = as_stream(stream);
    const bool hd512 = r.head_dim == 512;
    if (r.n_vtc) {  // V^T blocks of the caches without their own
        const VtCacheDev* vtc = reinterpret_cast<const VtCacheDev*>(r.ws + r.off_vtc);
        const dim3 vgrid(r.vt_blocks, r.num_kv_heads);
        if (hd512)
            G4_LAUNCH(k_vt_blocks<512>, vgrid, dim3(256), 0, st, vtc, r.n_vtc, (uint32_t)r.num_kv_heads);
        else
            G4_LAUNCH(k_vt_blocks<256>, vgrid, dim3(256), 0, st, vtc, r.n_vtc, (uint32_t)r.num_kv_heads);
        G4_CHECK_LAUNCH("attnPrefill (V^T blocks)");
    }
    const dim3 grid(r.n_lists, r.num_kv_heads, r.head_dim / 256);
    if (hd512) {  // grid z: the row half of each work item's query tile
        if (start_ev || stop_ev)
            hipExtLaunchKernelGGL(k_prefill_pp512, grid, dim3(6 * 64), 0, st, start_ev, stop_ev, 0, a, table, work,
                                  lists);
        else
            G4_LAUNCH(k_prefill_pp512, grid, dim3(6 * 64), 0, st, a, table, work, lists);
    } else if (start_ev || stop_ev) {
        hipExtLaunchKernelGGL(k_prefill_pp, grid, dim3(2 * kPfThreads), 0, st, start_ev, stop_ev, 0, a, table, work,
                              lists);
    } else {
        G4_LAUNCH(k_prefill_pp, grid, dim3(2 * kPfThreads), 0, st, a, table, work, lists);
    }
    G4_CHECK_LAUNCH("attnPrefill");
    if (!r.n_merge) return G4_OK;
    DecodeArgs m = {};
    m.table = reinterpret_cast<const DecodeEntryDev*>(r.ws + r.off_merge);
    m.n_entries = r.n_merge;
    m.num_kv_heads = r.num_kv_heads;
    m.group = a.group;
    m.part_ml = a.part_ml;
    m.part_o = a.part_o;
    return launch_decode_merge(m, r.n_merge, r.max_parts, st, r.head_dim);
}

int g4_attn_prefill_run(const g4_decode_plan* plan, void* stream) { return prefill_run(plan, stream, nullptr, nullptr); }

int g4_attn_prefill_run_timed(const g4_decode_plan* plan, void* stream, void* start_event, void* stop_event) {
    if (!start_event || !stop_event) return fail(G4_EINVAL, "attnPrefill: timing events are NULL");
    return prefill_run(plan, stream, static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event));
}

int g4_attn_prefill(const g4_prefill_entry* entries, uint32_t n_entries, uint32_t num_q_heads, uint32_t num_kv_heads,
                    uint32_t head_dim, void* workspace, size_t workspace_bytes, void* stream) {
    g4_decode_plan plan;
    int rc = g4_attn_prefill_prepare(entries, n_entries, num_q_heads, num_kv_heads, head_dim, workspace,
                                     workspace_bytes, &plan, stream);
    if (rc) return rc;
    return g4_attn_prefill_run(&plan, stream);
}

}  // extern "C"
