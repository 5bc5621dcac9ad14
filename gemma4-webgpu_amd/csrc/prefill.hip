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
// tokens) and a contiguous part of its key range; each of its 4 waves owns 32
// q-rows, held as the B operand of the score MFMA for the whole pass.
//
// Per 32-key tile (shared by the 4 waves through LDS, double-buffered):
//   S^T[32 keys x 32 q-rows] = K[keys x 16 d] * Q^T[16 d x q-rows], 16 MFMAs over HD = 256.
//     The MFMA's A row m holds key pi(m) = m with bits 2 and 3 swapped, so the
//     result register r of lane l holds key 16*(r/8) + 8*(l/32) + r%8 of q-row
//     l%32: registers 8s..8s+7 are already the B operand (keys 16s + 8*(l/32)
//     .. +8) of the output MFMA for key step s.
//   online softmax per q-row in log2 units (the two half-waves hold 16 keys each)
//   O^T[32 d x 32 q-rows] += V^T[32 d x 16 keys] * P^T[16 keys x q-rows], 8 d blocks x 2 key steps.
//     V is stored transposed in LDS ([d][key]); 8x8 f16 blocks are transposed
//     in registers (v_perm_b32) between the global load and the LDS store.
// P is rounded to f16 for the output MFMA (relative error <= 2^-11 per
// probability); scores and sums stay f32.
//
// A part that covers a tile's whole key range writes attnOut rows directly;
// otherwise it writes a partial record (m, l, unnormalised o) per q-row and
// the fixed-order log-sum-exp merge of decode.hip combines the parts.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_ext.h>

#include <algorithm>
#include <vector>

#include "decode_core.h"

namespace g4 {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kPfHD = 256;
constexpr int kPfWaves = 4;
constexpr int kPfThreads = 64 * kPfWaves;
constexpr int kPfRows = 32 * kPfWaves;   // q-rows per tile
constexpr int kPfKeys = 32;              // keys per tile
constexpr int kKRowBytes = kPfHD * 2 + 16;       // padded K row in LDS
constexpr int kVtRowBytes = kPfKeys * 2 + 16;    // padded V^T row (one d) in LDS

struct PrefillEntryDev {
    const uint16_t* q;    // f16 [n_tokens][num_q_heads][HD]
    const uint16_t* k;    // f16 [rows][num_kv_heads][HD]
    const uint16_t* v;
    float* out;           // f32 [n_tokens][num_q_heads][HD]
    uint32_t n_tokens;
    uint32_t start;       // position of token 0
    uint32_t window;      // 0 = full
    float qscale;         // scale * log2(e)
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

struct PrefillArgs {
    const PrefillEntryDev* table;
    const PrefillWorkDev* work;
    uint32_t num_q_heads;
    uint32_t num_kv_heads;
    uint32_t group;
    uint32_t pad;
    float* part_ml;  // [slot][num_kv_heads][group][2]
    float* part_o;   // [slot][num_kv_heads][group][HD]
};

struct PrefillSmem {
    unsigned char k[2][kPfKeys * kKRowBytes];
    unsigned char vt[2][kPfHD * kVtRowBytes];
};

__device__ __forceinline__ unsigned key_of_row(unsigned m) {  // swap bits 2 and 3
    return (m & ~12u) | ((m & 4u) << 1) | ((m & 8u) >> 1);
}

// Global -> LDS for one 32-key tile starting at row kt0 (rows past `last` clamp to it).
// Threads 0..127 move V as 8x8 blocks (8 keys x 8 d), transposed on the way;
// threads 128..255 copy K rows (8 pieces of 16 bytes each).
struct TileRegs {
    u32x4 x[8];
};

__device__ __forceinline__ void tile_load(const char* Kb, const char* Vb, uint32_t row_bytes, unsigned kt0,
                                          unsigned last, TileRegs& r) {
    const int t = threadIdx.x;
    if (t < 128) {
        const int kg = t >> 5, dg = t & 31;  // keys 8kg..8kg+8, d 8dg..8dg+8
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const unsigned row = min(kt0 + 8u * kg + i, last);
            r.x[i] = ldg<u32x4>(Vb + ((uint64_t)row * row_bytes + dg * 16u));
        }
    } else {
        const int u = t - 128;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int piece = u + 128 * i;  // 32 keys x 32 pieces of 16 bytes
            const unsigned row = min(kt0 + (unsigned)(piece >> 5), last);
            r.x[i] = ldg<u32x4>(Kb + ((uint64_t)row * row_bytes + (piece & 31) * 16u));
        }
    }
}

__device__ __forceinline__ void tile_store(PrefillSmem& sm, int buf, const TileRegs& r) {
    const int t = threadIdx.x;
    if (t < 128) {
        const int kg = t >> 5, dg = t & 31;
        // out[c] = the 8 keys at d = 8dg + c: word w holds keys (2w, 2w + 1), d-half c%2 of word c/2
#pragma unroll
        for (int c = 0; c < 8; c++) {
            u32x4 o;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const uint32_t a = r.x[2 * w][c >> 1], b = r.x[2 * w + 1][c >> 1];
                o[w] = (c & 1) ? perm_hi(a, b) : perm_lo(a, b);
            }
            *reinterpret_cast<u32x4*>(&sm.vt[buf][(8 * dg + c) * kVtRowBytes + kg * 16]) = o;
        }
    } else {
        const int u = t - 128;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int piece = u + 128 * i;
            *reinterpret_cast<u32x4*>(&sm.k[buf][(piece >> 5) * kKRowBytes + (piece & 31) * 16]) = r.x[i];
        }
    }
}

__global__ __launch_bounds__(kPfThreads, 1) void k_prefill(PrefillArgs a) {
    __shared__ PrefillSmem sm;
    const PrefillWorkDev wk = a.work[blockIdx.x];
    const PrefillEntryDev& ent = a.table[wk.entry];
    const unsigned kvh = blockIdx.y;
    const unsigned G = a.group, NQH = a.num_q_heads, NKH = a.num_kv_heads;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int half = lane >> 5;    // which 8 of each 16 keys / d elements this lane supplies
    const int col = lane & 31;     // this lane's q-row within the wave

    // This lane's q-row: token and head, its absolute position and key window.
    const unsigned rho = (unsigned)wk.tile * kPfRows + (unsigned)wave * 32u + (unsigned)col;
    const unsigned tok = rho / G, head = rho % G;
    const bool row_live = tok < ent.n_tokens;
    const unsigned tok_c = row_live ? tok : ent.n_tokens - 1;
    const unsigned pos = ent.start + tok_c;
    const unsigned lo = (ent.window != 0 && pos + 1 > ent.window) ? pos + 1 - ent.window : 0u;
    const unsigned hi = row_live ? pos : 0u;  // rows outside [lo, hi] are masked; dead rows see none
    const bool dead = !row_live;

    // Q^T operand: 16 key-steps of 8 f16 (d = 16s + 8*half .. +8), loaded once.
    f16x8 qop[16];
    {
        const uint16_t* qr = ent.q + ((uint64_t)tok_c * NQH + kvh * G + head) * kPfHD + 8 * half;
#pragma unroll
        for (int s = 0; s < 16; s++) qop[s] = ldg<f16x8>(qr + 16 * s);
    }

    const uint32_t row_bytes = NKH * kPfHD * 2u;
    const char* Kb = reinterpret_cast<const char*>(ent.k + (uint64_t)kvh * kPfHD);
    const char* Vb = reinterpret_cast<const char*>(ent.v + (uint64_t)kvh * kPfHD);
    const unsigned kb = wk.key_begin, ke = wk.key_end, last = ke - 1;
    const unsigned n_tiles = (ke - kb + kPfKeys - 1) / kPfKeys;
    const float qs = ent.qscale;

    TileRegs stage;
    tile_load(Kb, Vb, row_bytes, kb, last, stage);
    tile_store(sm, 0, stage);
    __syncthreads();

    float m_run = -INFINITY, l_run = 0.0f;
    f32x16 acc[8];
#pragma unroll
    for (int b = 0; b < 8; b++) acc[b] = f32x16{};
    const unsigned krow = key_of_row((unsigned)col);  // K row this lane supplies to the score MFMA

    for (unsigned it = 0; it < n_tiles; it++) {
        const int buf = it & 1;
        const unsigned kt0 = kb + it * kPfKeys;
        if (it + 1 < n_tiles) tile_load(Kb, Vb, row_bytes, kt0 + kPfKeys, last, stage);

        // scores: two accumulators over alternating d steps for MFMA overlap
        f32x16 s0 = f32x16{}, s1 = f32x16{};
        const unsigned char* kr = &sm.k[buf][krow * kKRowBytes + 16 * half];
#pragma unroll
        for (int s = 0; s < 16; s += 2) {
            const f16x8 k0 = *reinterpret_cast<const f16x8*>(kr + 32 * s);
            const f16x8 k1 = *reinterpret_cast<const f16x8*>(kr + 32 * (s + 1));
            s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(k0, qop[s], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(k1, qop[s + 1], s1, 0, 0, 0);
        }
        // mask, tile max (the two half-waves hold the row's other 16 keys)
        float x[16];
        float tmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const unsigned key = kt0 + 16u * (r >> 3) + 8u * half + (r & 7);
            const bool ok = !dead && key < ke && key >= lo && key <= hi;
            x[r] = ok ? (s0[r] + s1[r]) * qs : -INFINITY;
            tmax = fmaxf(tmax, x[r]);
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float m_new = fmaxf(m_run, tmax);
        if (__any(m_new > m_run)) {
            const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int b = 0; b < 8; b++) acc[b] *= alpha;
        }
        m_run = m_new;
        const float mu = m_new == -INFINITY ? 0.0f : m_new;
        f16x8 pop[2];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const float p = __builtin_amdgcn_exp2f(x[r] - mu);
            l_run += p;
            pop[r >> 3][r & 7] = (f16)p;
        }
        // O^T += V^T P^T
        const unsigned char* vr = &sm.vt[buf][col * kVtRowBytes + 16 * half];
#pragma unroll
        for (int b = 0; b < 8; b++) {
#pragma unroll
            for (int s = 0; s < 2; s++) {
                const f16x8 vop = *reinterpret_cast<const f16x8*>(vr + (32 * b) * kVtRowBytes + 32 * s);
                acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vop, pop[s], acc[b], 0, 0, 0);
            }
        }
        if (it + 1 < n_tiles) tile_store(sm, buf ^ 1, stage);
        __syncthreads();
    }

    // Row sums: this lane's 16 keys plus the other half-wave's.
    const float L = l_run + __shfl_xor(l_run, 32);
    if (dead) return;
    // Lane holds O^T rows d = 32b + 8*(r/4) + 4*half + r%4 of its q-row: 4 consecutive d per group.
    const uint64_t qrow = (uint64_t)tok * NQH + kvh * G + head;
    if (wk.n_parts == 1) {
        float* dst = ent.out + qrow * kPfHD + 4 * half;
        const float inv = 1.0f / L;
#pragma unroll
        for (int b = 0; b < 8; b++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                stg<f32x4>(dst + 32 * b + 8 * g, f32x4{acc[b][4 * g] * inv, acc[b][4 * g + 1] * inv,
                                                      acc[b][4 * g + 2] * inv, acc[b][4 * g + 3] * inv});
        return;
    }
    const unsigned tile_tok0 = (unsigned)wk.tile * kPfRows / G;
    const uint64_t slot = (uint64_t)wk.split_base + (uint64_t)(tok - tile_tok0) * wk.n_parts + wk.part;
    const uint64_t rec = (slot * NKH + kvh) * G + head;
    float* po = a.part_o + rec * kPfHD + 4 * half;
#pragma unroll
    for (int b = 0; b < 8; b++)
#pragma unroll
        for (int g = 0; g < 4; g++)
            stg<f32x4>(po + 32 * b + 8 * g, f32x4{acc[b][4 * g], acc[b][4 * g + 1], acc[b][4 * g + 2], acc[b][4 * g + 3]});
    if (half == 0) stg<f32x2>(a.part_ml + rec * 2, f32x2{m_run, L});
}

}  // namespace g4

using namespace g4;

namespace {

constexpr uint32_t kPrefillMagic = 0x67345046u;

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int pf_env(const char* name, int dflt) {
    const char* s = getenv(name);
    return s && *s ? atoi(s) : dflt;
}

struct PrefillPlanRep {
    char* ws;
    uint32_t n_entries;
    uint32_t n_work;
    uint32_t n_merge;      // merge entries (tokens of split tiles)
    uint32_t max_parts;
    uint32_t num_q_heads;
    uint32_t num_kv_heads;
    uint32_t magic;
    uint32_t off_work, off_merge, off_ml, off_o;  // workspace byte offsets (workspaces stay under 4 GiB)
};
static_assert(sizeof(PrefillPlanRep) <= sizeof(g4_decode_plan), "plan size");

struct Staging {
    void* buf = nullptr;
    size_t cap = 0;
    hipEvent_t done = nullptr;
};

int stage_upload(Staging& sg, void* dst, const void* src, size_t bytes, hipStream_t st) {
    if (!bytes) return G4_OK;
    if (!sg.done) G4_CHECK_HIP(hipEventCreateWithFlags(&sg.done, hipEventDisableTiming));
    G4_CHECK_HIP(hipEventSynchronize(sg.done));
    if (sg.cap < bytes) {
        if (sg.buf) G4_CHECK_HIP(hipHostFree(sg.buf));
        sg.buf = nullptr;
        sg.cap = 0;
        G4_CHECK_HIP(hipHostMalloc(&sg.buf, bytes, hipHostMallocDefault));
        sg.cap = bytes;
    }
    memcpy(sg.buf, src, bytes);
    G4_CHECK_HIP(hipMemcpyAsync(dst, sg.buf, bytes, hipMemcpyHostToDevice, st));
    G4_CHECK_HIP(hipEventRecord(sg.done, st));
    return G4_OK;
}

// The key range of tile `tile`: [lo of its first token, position of its last token].
void tile_keys(const g4_prefill_entry& e, uint32_t G, uint32_t tile, uint32_t* kb, uint32_t* ke) {
    const uint32_t t0 = tile * (uint32_t)kPfRows / G;
    const uint32_t t1 = std::min(e.n_tokens, (tile + 1) * (uint32_t)kPfRows / G) - 1;
    const uint32_t p0 = e.start + t0, p1 = e.start + t1;
    *kb = (e.sliding_window != 0 && p0 + 1 > e.sliding_window) ? p0 + 1 - e.sliding_window : 0;
    *ke = p1 + 1;
}

struct Layout {
    size_t table, work, merge, ml, o, total;
};

// Work list, merge list and workspace layout for a set of entries.
int build(const g4_prefill_entry* ents, uint32_t n, uint32_t nqh, uint32_t nkh, uint32_t part_keys,
          std::vector<PrefillEntryDev>* tab, std::vector<PrefillWorkDev>* work, std::vector<DecodeEntryDev>* merge,
          uint32_t* max_parts, Layout* L) {
    const uint32_t G = nqh / nkh;
    uint64_t slots = 0;
    *max_parts = 1;
    tab->resize(n);
    struct Item {
        PrefillWorkDev w;
        uint32_t keys;
    };
    std::vector<Item> items;
    for (uint32_t i = 0; i < n; i++) {
        const g4_prefill_entry& e = ents[i];
        (*tab)[i] = PrefillEntryDev{e.q, e.k_cache, e.v_cache, e.out, e.n_tokens, e.start, e.sliding_window,
                                    e.scale * kLog2e};
        const uint32_t tiles = (uint32_t)(((uint64_t)e.n_tokens * G + kPfRows - 1) / kPfRows);
        for (uint32_t t = 0; t < tiles; t++) {
            uint32_t kb, ke;
            tile_keys(e, G, t, &kb, &ke);
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
                                                    e.out + (uint64_t)(tok0 + tk) * nqh * kPfHD, 0, 0,
                                                    base + tk * parts, parts, 0.0f, 0});
                slots += (uint64_t)ntok * parts;
                *max_parts = std::max(*max_parts, parts);
            }
        }
    }
    // Longest items first: the dispatcher starts workgroups in index order.
    std::stable_sort(items.begin(), items.end(), [](const Item& x, const Item& y) { return x.keys > y.keys; });
    work->clear();
    for (auto& it : items) work->push_back(it.w);
    if (work->size() > 0x7fffffffu || slots > 0x7fffffffu) return fail(G4_EINVAL, "attnPrefill: too much work");
    size_t off = 0;
    L->table = off;
    off += align256(n * sizeof(PrefillEntryDev));
    L->work = off;
    off += align256(work->size() * sizeof(PrefillWorkDev));
    L->merge = off;
    off += align256(merge->size() * sizeof(DecodeEntryDev));
    L->ml = off;
    off += align256(slots * nkh * G * 2 * sizeof(float));
    L->o = off;
    off += align256(slots * nkh * G * kPfHD * sizeof(float));
    L->total = off;
    return G4_OK;
}

int check(const g4_prefill_entry* ents, uint32_t n, uint32_t nqh, uint32_t nkh, uint32_t hd) {
    if (!ents || n == 0) return fail(G4_EINVAL, "attnPrefill: no entries");
    if (hd != (uint32_t)kPfHD) return fail(G4_EINVAL, "attnPrefill: head_dim %u unsupported (256)", hd);
    if (nkh == 0 || nqh % nkh || nqh / nkh > (uint32_t)kMaxGroup || 32 % (nqh / nkh))
        return fail(G4_EINVAL, "attnPrefill: %u query heads over %u kv heads unsupported", nqh, nkh);
    for (uint32_t i = 0; i < n; i++) {
        const g4_prefill_entry& e = ents[i];
        if (!e.q || !e.k_cache || !e.v_cache || !e.out) return fail(G4_EINVAL, "attnPrefill: entry %u has NULL", i);
        if (reinterpret_cast<uintptr_t>(e.out) & 15)
            return fail(G4_EINVAL, "attnPrefill: entry %u out must be 16-byte aligned", i);
        if (e.n_tokens == 0) return fail(G4_EINVAL, "attnPrefill: entry %u has no tokens", i);
        if ((uint64_t)e.start + e.n_tokens > 0xffffffffull) return fail(G4_EINVAL, "attnPrefill: entry %u range", i);
    }
    return G4_OK;
}

uint32_t part_keys_default() {
    static const int env = pf_env("G4_PREFILL_PART_KEYS", 0);
    return env > 0 ? (uint32_t)((env + kPfKeys - 1) / kPfKeys * kPfKeys) : 1536u;  // measured best of 512..4096
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
    std::vector<DecodeEntryDev> merge;
    uint32_t mp;
    Layout L;
    rc = build(entries, n_entries, num_q_heads, num_kv_heads, part_keys_default(), &tab, &work, &merge, &mp, &L);
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
    std::vector<DecodeEntryDev> merge;
    uint32_t max_parts;
    Layout L;
    rc = build(entries, n_entries, num_q_heads, num_kv_heads, part_keys_default(), &tab, &work, &merge, &max_parts,
               &L);
    if (rc) return rc;
    if (max_parts > 8192) return fail(G4_EINVAL, "attnPrefill: %u key parts per tile (max 8192)", max_parts);
    if (!workspace || workspace_bytes < L.total)
        return fail(G4_ENOSPC, "attnPrefill: workspace %zu bytes < %zu needed", workspace_bytes, L.total);
    if (L.o >= (1ull << 32)) return fail(G4_EINVAL, "attnPrefill: workspace layout exceeds 4 GiB");
    hipStream_t st = as_stream(stream);
    char* ws = static_cast<char*>(workspace);
    static thread_local Staging s_tab, s_work, s_merge;
    rc = stage_upload(s_tab, ws + L.table, tab.data(), tab.size() * sizeof(PrefillEntryDev), st);
    if (rc) return rc;
    rc = stage_upload(s_work, ws + L.work, work.data(), work.size() * sizeof(PrefillWorkDev), st);
    if (rc) return rc;
    rc = stage_upload(s_merge, ws + L.merge, merge.data(), merge.size() * sizeof(DecodeEntryDev), st);
    if (rc) return rc;
    PrefillPlanRep r = {};
    r.ws = ws;
    r.n_entries = n_entries;
    r.n_work = (uint32_t)work.size();
    r.n_merge = (uint32_t)merge.size();
    r.max_parts = max_parts;
    r.num_q_heads = num_q_heads;
    r.num_kv_heads = num_kv_heads;
    r.magic = kPrefillMagic;
    r.off_work = (uint32_t)L.work;
    r.off_merge = (uint32_t)L.merge;
    r.off_ml = (uint32_t)L.ml;
    r.off_o = (uint32_t)L.o;
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
    a.table = reinterpret_cast<const PrefillEntryDev*>(r.ws);
    a.work = reinterpret_cast<const PrefillWorkDev*>(r.ws + r.off_work);
    a.num_q_heads = r.num_q_heads;
    a.num_kv_heads = r.num_kv_heads;
    a.group = r.num_q_heads / r.num_kv_heads;
    a.part_ml = reinterpret_cast<float*>(r.ws + r.off_ml);
    a.part_o = reinterpret_cast<float*>(r.ws + r.off_o);
    hipStream_t st = as_stream(stream);
    if (start_ev || stop_ev)
        hipExtLaunchKernelGGL(k_prefill, dim3(r.n_work, r.num_kv_heads), dim3(kPfThreads), 0, st, start_ev, stop_ev, 0,
                              a);
    else
        hipLaunchKernelGGL(k_prefill, dim3(r.n_work, r.num_kv_heads), dim3(kPfThreads), 0, st, a);
    G4_CHECK_LAUNCH("attnPrefill");
    if (!r.n_merge) return G4_OK;
    DecodeArgs m = {};
    m.table = reinterpret_cast<const DecodeEntryDev*>(r.ws + r.off_merge);
    m.n_entries = r.n_merge;
    m.num_kv_heads = r.num_kv_heads;
    m.group = a.group;
    m.part_ml = a.part_ml;
    m.part_o = a.part_o;
    return launch_decode_merge(m, r.n_merge, r.max_parts, st);
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
