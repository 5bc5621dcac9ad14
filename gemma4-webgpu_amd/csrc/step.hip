// One-launch decode step for gfx950: the whole attention block of one token
// for a set of layers or sequences ("entries"), in a single kernel:
//
//   vNorm + fusedNormRope(Q, K) + kvCacheStore + attnScore -> softmax ->
//   attnOutput
//
// i.e. the dispatch sequence of src/engine.ts:2056-2094 (shaders
// per_head_rms_norm_no_weight.wgsl, fused_per_head_norm_rope.wgsl,
// kv_cache_store.wgsl, attn_score.wgsl, softmax.wgsl, attn_output.wgsl),
// with flash-decoding split-K; entries split over several workgroups are
// merged by a second launch (the log-sum-exp merge of decode.hip), or inside
// the output projection's launch (k_step_out).
//
// Work split: the host cuts every entry's attended rows into 32-row tiles and
// gives each entry a number of workgroups proportional to its tiles (at least
// one), choosing the tiles per workgroup so that all workgroups fit the GPU at
// once; workgroup w then reads its entry and row range from a per-workgroup
// table. No workgroup spans two entries.
//
// Every workgroup computes its entry's post-norm, post-RoPE query itself (from
// the raw projection; one wave per head, evaluating exactly the reference's
// expressions and reduction tree, so the values are bit-identical to the prep
// kernel's) while its first tile is in flight: the small operands are
// requested before the tile (vector-memory results return in issue order, so
// anything requested after the tile would wait for it), then the RoPE factors
// (f64 transcendentals, one pair per lane, shared through LDS) and the norms
// run under the tile's latency. The workgroup whose range holds the entry's last row (the current token's row)
// also computes that row's k (norm + RoPE) and v (weightless norm), uses them
// for that row instead of the cache, and stores them as f16 when the entry
// owns the cache (KV-producer layers).
//
// Merge: a workgroup covering a whole entry writes attnOut directly; otherwise
// it writes a partial record (m, l, unnormalised o per head) and the fixed-order
// log-sum-exp merge kernel of decode.hip combines an entry's records in a
// second launch. (Merging inside this launch needs a device-scope release per
// workgroup; on gfx950 that is an L2 write-back plus invalidate, measured far
// costlier than the second launch.)
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_ext.h>

#include <algorithm>
#include <type_traits>
#include <utility>
#include <vector>

#include "decode_core.h"
#include "ref_math.h"
#include "step_plan.h"

namespace g4 {

struct StepArgs {
    const StepWorkDev* work;
    uint32_t num_kv_heads;
    uint32_t group;
    float* part_ml;  // partial records [part * NKH + kvh][group][2]
    float* part_o;   //                  [part * NKH + kvh][group][HD]
};

template <int W, int HD>
struct StepSmem {
    DecodeSmem<HD, W> dec;
    float qf[kMaxGroup][HD];  // post-prep q * qscale
    f16x8 knew[HD / 8];       // current row's k and v, f16 (as stored)
    f16x8 vnew[HD / 8];
    float rope_c[HD / 2];     // RoPE factors of the HD/2 pairs, when evaluated in the kernel
    float rope_s[HD / 2];
    float mnew[kMaxGroup];    // current row's scores (log2 units)
};

// W waves per workgroup. head_dim 256: two waves per SIMD (two 4-wave
// workgroups or one 8-wave workgroup per CU), enough rows in flight to cover
// the HBM latency with one 32-row tile per wave. head_dim 512: one 4-wave
// workgroup per CU at one wave per SIMD (a 32-row tile is 64 KB of K and V,
// the accumulators take 128 registers more).
//
// The arguments are scalars and pointers (not one struct) so that they are
// preloaded into SGPRs at wave start (the file is compiled with kernarg
// preloading), and the work item is copied by value: its fields arrive in one
// batch of scalar loads. Reading fields where used, or selecting a field's
// address by a value loaded before, chains dependent scalar loads (measured:
// six round trips, ~4.6 us before a workgroup's first vector load).
//
// `adv`: tokens the plan has been advanced since it was prepared (0 for a plan
// as prepared). Every entry then ends adv rows later at position + adv, its
// parts move with its first attended row (step_part_rows), and the RoPE
// factors are evaluated here from the inverse frequencies of the entry's set,
// in f64 rounded to f32 as the host evaluates the prepared position's.
template <int W, int HD>
__device__ __forceinline__ void attn_step_body(const StepWorkDev* __restrict__ work, float* part_ml, float* part_o,
                                               uint32_t num_kv_heads, uint32_t group, uint32_t adv, unsigned wg,
                                               unsigned kvh, StepSmem<W, HD>& sm) {
    const StepArgs a{work, num_kv_heads, group, part_ml, part_o};
    using D = DecodeDims<HD>;
    constexpr int J = HD / 64;                          // elements of a head per lane
    constexpr int PJ = J / 2;                           // RoPE pairs per lane
    constexpr int kQPerWave = (kMaxGroup + W - 1) / W;  // query heads per wave
    const unsigned NKH = a.num_kv_heads;
    const unsigned G = a.group;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: branches on it stay scalar
    const int n = lane & 15;
    const int g = lane >> 4;
    const bool lo_col = n >= 8;

    const StepWorkDev wk = work[wg];
    const StepEntryDev& ent = wk.ent;
    const unsigned key_end = ent.key_end + adv;
    const unsigned position = ent.position + adv;
    const StepRows rows = step_part_rows(wk.row_begin, wk.row_end, ent.key_end, ent.window, adv);
    const unsigned k0 = rows.begin;
    // This workgroup holds the current token's row, and computes it (unless it is already cached).
    const bool has_new = rows.end == key_end && !(ent.flags & kRowCached);
    const unsigned new_row = key_end - 1;
    const unsigned k1t = has_new ? new_row : rows.end;  // rows read from the cache: [k0, k1t)
    const unsigned nkeys = k1t - k0;
    const unsigned last = nkeys ? k1t - 1 : k0;  // loads are clamped to it (k0 < key_end: in the cache)

    constexpr unsigned kStride = W * kTileKeys;
    unsigned t0 = (unsigned)wave * kTileKeys;
    float m_run = -INFINITY, l_run = 0.0f;
    f32x4 acc[D::NO];
#pragma unroll
    for (int i = 0; i < D::NO; i++) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    // The prologue and the tiles, as two straight-line copies: waves with a
    // first tile and waves without one (short parts: a one-tile part leaves
    // seven of eight waves without rows). Within one copy every load is
    // unconditional (clamped to valid addresses where the value is not needed):
    // with loads under branches the compiler cannot count the younger loads on
    // every path, and its wait for a small operand would also wait for the
    // tile. A wave without rows issues no tile loads at all: a CU's load path
    // takes the same time for a clamped load as for a real one (~0.2 us per
    // wave and tile at head_dim 256), which would delay the one real tile.
    // Both copies meet the same barriers in the same order.
    auto body = [&](auto tile_tag) {
        constexpr bool kTile = decltype(tile_tag)::value;
        // ---- small operands first, then the first tile ----
        // f16 values stay unconverted until used. RoPE factors of this lane's
        // pairs from the host-evaluated set (a plan as prepared); otherwise the
        // pair's inverse frequency from the set, or the divisor to evaluate it
        // with. Absent tables are replaced by valid dummy addresses (the values
        // are not used).
        const float* rcs = ent.rope_cs;
        const bool host_cs = rcs && adv == 0;  // uniform
        const float* rsrc = host_cs ? rcs : ent.q;
        RopeLane<PJ> rl;
#pragma unroll
        for (int p = 0; p < PJ; p++) {
            rl.c[p] = ldg<float>(rsrc + lane + 64 * p);
            rl.s[p] = ldg<float>(rsrc + HD / 2 + lane + 64 * p);
        }
        const unsigned pair = threadIdx.x % (HD / 2);  // pair evaluated by this thread otherwise
        const bool apply_divisor = ent.flags & kApplyDivisor;
        const uint32_t fbits = ldg<uint16_t>((apply_divisor ? ent.rope_freqs : ent.q_weight) + pair);
        float inv_l[PJ];  // this lane's pairs' inverse frequencies from the set (advanced plans)
#pragma unroll
        for (int p = 0; p < PJ; p++) inv_l[p] = ldg<float>((rcs ? rcs + HD : ent.q) + lane + 64 * p);
        float xq[kQPerWave][J];
#pragma unroll
        for (int r = 0; r < kQPerWave; r++) {
            const unsigned hq = min((unsigned)wave + W * r, G - 1);
            const float* src = ent.q + ((uint64_t)kvh * G + hq) * HD;
#pragma unroll
            for (int j = 0; j < J; j++) xq[r][j] = ldg<float>(src + lane + 64 * j);
        }
        uint32_t wq[J], wn[J];
#pragma unroll
        for (int j = 0; j < J; j++) wq[j] = ldg<uint16_t>(ent.q_weight + lane + 64 * j);
        const bool do_new = has_new && wave < 2;  // wave 0: k, wave 1: v
        float xn[J];
        {
            const float* src = (wave == 1 ? ent.v : ent.k) + (uint64_t)kvh * HD;
#pragma unroll
            for (int j = 0; j < J; j++) xn[j] = ldg<float>(src + lane + 64 * j);
#pragma unroll
            for (int j = 0; j < J; j++) wn[j] = ldg<uint16_t>(ent.k_weight + lane + 64 * j);
        }
        const uint32_t row_bytes = NKH * HD * 2u;
        const char* Kb = reinterpret_cast<const char*>(ent.k_cache + (uint64_t)kvh * HD);
        const char* Vb = reinterpret_cast<const char*>(ent.v_cache + (uint64_t)kvh * HD);
        f16x8 kreg[2][D::NC];
        u32x4 vreg[D::NB][8];
        if constexpr (kTile) {
            load_k_tile<HD>(Kb, row_bytes, last, n, g, k0 + t0, kreg);
            load_v_tile<HD>(Vb, row_bytes, last, n, g, k0 + t0, vreg);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep every request above ahead of the arithmetic below

        // ---- q heads straight into the score operand; the current row's k and v ----
        if (rcs && !host_cs) {  // uniform: each lane evaluates its own pairs at the advanced position,
            // cos and sin of the f32 angle in f64 rounded to f32, as the host evaluates a prepared one
#pragma unroll
            for (int p = 0; p < PJ; p++) f64_cos_sin((float)position * inv_l[p], rl.c[p], rl.s[p]);
        } else if (!rcs) {  // uniform: one pair per thread, the reference's expressions with f64
            // transcendentals; division by 1 is exact, so the load above stays unconditional
            const float freq = rope_inv_freq(pair, HD, ent.theta, 1u, apply_divisor ? h2f((uint16_t)fbits) : 1.0f);
            const float ang = (float)position * freq;
            float c, sn;
            f64_cos_sin(ang, c, sn);
            if (threadIdx.x < HD / 2) {
                sm.rope_c[pair] = c;
                sm.rope_s[pair] = sn;
            }
            __syncthreads();
#pragma unroll
            for (int p = 0; p < PJ; p++) {
                rl.c[p] = sm.rope_c[lane + 64 * p];
                rl.s[p] = sm.rope_s[lane + 64 * p];
            }
        }

        const float qscale = ent.qscale, eps = ent.eps;
        const bool q_ready = ent.flags & kQReady;  // uniform: q is the post-norm, post-RoPE query already
        f16* qop = reinterpret_cast<f16*>(sm.dec.q);  // [chunk c][operand lane 16*g + column][8]
#pragma unroll
        for (int r = 0; r < kQPerWave; r++) {
            const unsigned hq = (unsigned)wave + W * r;
            const bool live = hq < G;  // columns of absent heads are zero
            if (live && !q_ready) wave_norm_rope<J>(xq[r], wq, true, true, rl, eps);
#pragma unroll
            for (int j = 0; j < J; j++) {
                const unsigned d = (unsigned)lane + 64u * j;
                const float x = live ? xq[r][j] * qscale : 0.0f;
                if (live) sm.qf[hq][d] = x;
                const f16 hi = (f16)x;  // hi in column hq, the f16 residual in column hq + 8
                const unsigned base = ((d >> 5) * 64u + 16u * ((d >> 3) & 3u) + hq) * 8u + (d & 7u);
                qop[base] = hi;
                qop[base + 64] = (f16)(x - (float)hi);
            }
        }
        if (do_new) {
            const bool is_k = wave == 0;
            wave_norm_rope<J>(xn, wn, is_k, is_k, rl, eps);
            uint16_t* row = reinterpret_cast<uint16_t*>(is_k ? sm.knew : sm.vnew);
#pragma unroll
            for (int j = 0; j < J; j++) row[lane + 64 * j] = f2h(xn[j]);
            if (ent.flags & kStoreKv) {
                uint16_t* dst = (is_k ? ent.k_cache : ent.v_cache) + ((uint64_t)new_row * NKH + kvh) * HD;
#pragma unroll
                for (int j = 0; j < J; j++) stg<uint16_t>(dst + lane + 64 * j, f2h(xn[j]));
            }
        }
        __syncthreads();

        // The current row's scores (read by the combine, after later barriers).
        if (has_new) {
            const f16* kn = reinterpret_cast<const f16*>(sm.knew);
            for (unsigned h = (unsigned)wave; h < G; h += W) {
                float p = 0.0f;
#pragma unroll
                for (int j = 0; j < J; j++) p += sm.qf[h][lane + 64 * j] * (float)kn[lane + 64 * j];
                p = wave_tree_sum(p);  // the same operand pairs at lane 0 as a 32 .. 1 butterfly
                if (lane == 0) sm.mnew[h] = p;
            }
        }

        // ---- tiles ----
        if constexpr (kTile) {  // the first tile was requested above; the loop requests its own
            tile_step<HD>(sm.dec, lane, g, lo_col, k0 + t0, k1t, kreg, vreg, m_run, l_run, acc);
            for (t0 += kStride; t0 < nkeys; t0 += kStride) {
                load_k_tile<HD>(Kb, row_bytes, last, n, g, k0 + t0, kreg);
                load_v_tile<HD>(Vb, row_bytes, last, n, g, k0 + t0, vreg);
                tile_step<HD>(sm.dec, lane, g, lo_col, k0 + t0, k1t, kreg, vreg, m_run, l_run, acc);
            }
        }
    };
    if (t0 < nkeys)  // uniform: wave and nkeys are scalars
        body(std::true_type{});
    else
        body(std::false_type{});
    wave_publish<HD>(sm.dec, wave, n, g, m_run, l_run, acc);
    __syncthreads();

    const float* em = has_new ? sm.mnew : nullptr;
    const f16* ev = reinterpret_cast<const f16*>(sm.vnew);
    if (ent.n_parts == 1) {
        wg_combine_write<HD>(sm.dec, G, true, ent.out + (uint64_t)kvh * G * HD, nullptr, nullptr, em, ev);
        return;
    }
    const uint64_t rec = ((uint64_t)wk.part * NKH + kvh) * G;
    wg_combine_write<HD>(sm.dec, G, false, nullptr, a.part_o + rec * HD, a.part_ml + rec * 2, em, ev);
}

template <int W, int HD>
__global__ __launch_bounds__(64 * W, HD == 256 ? 8 / W : 1) void k_attn_step(
    const StepWorkDev* __restrict__ work, float* part_ml, float* part_o, uint32_t num_kv_heads, uint32_t group,
    uint32_t adv) {
    __shared__ StepSmem<W, HD> sm;
    attn_step_body<W, HD>(work, part_ml, part_o, num_kv_heads, group, adv, blockIdx.x, blockIdx.y, sm);
}

// Two plans of one token in one launch (E2B's two head_dim groups): the
// head_dim-512 plan's workgroups first, one per CU, then the head_dim-256
// plan's, in 4-wave workgroups of the same size, which take the CUs the first
// ones leave as they finish. Grid: (wgs_a + wgs_b) x the larger kv-head count.
union StepPairSmem {
    StepSmem<4, 512> a;
    StepSmem<4, 256> b;
};

__global__ __launch_bounds__(256, 1) void k_attn_step_pair(
    const StepWorkDev* __restrict__ work_a, float* ml_a, float* o_a, uint32_t nkh_a, uint32_t group_a, uint32_t adv_a,
    uint32_t wgs_a, const StepWorkDev* __restrict__ work_b, float* ml_b, float* o_b, uint32_t nkh_b, uint32_t group_b,
    uint32_t adv_b) {
    __shared__ StepPairSmem sm;
    const unsigned x = blockIdx.x, y = blockIdx.y;
    if (x < wgs_a) {  // uniform
        if (y < nkh_a) attn_step_body<4, 512>(work_a, ml_a, o_a, nkh_a, group_a, adv_a, x, y, sm.a);
    } else if (y < nkh_b) {
        attn_step_body<4, 256>(work_b, ml_b, o_b, nkh_b, group_b, adv_b, x - wgs_a, y, sm.b);
    }
}

}  // namespace g4

using namespace g4;

namespace {

constexpr uint32_t kStepMagic = 0x67345354u;

struct StepPlanRep {
    char* tables;   // the plan's tables region (work items | merge table | entry table | RoPE factors)
    char* part_ml;  // its partial records: (m, l) pairs, then the o rows at step_part_o_offset()
    uint16_t n_entries;     // <= 65535 (checked by the planner)
    uint16_t num_kv_heads;  // <= 65535
    uint16_t n_wgs;         // <= max(n_entries, kStepMaxWgs)
    uint16_t n_merge;       // entries spanning more than one workgroup (listed in the merge table)
    uint16_t max_parts;     // <= kStepMaxWgs
    uint8_t group;          // <= kMaxGroup
    uint8_t waves;          // waves per workgroup of the attention kernel (4 or 8)
    uint32_t head_dim;      // 256 or 512
    uint32_t magic;
    uint32_t off_merge;  // byte offsets of the merge table, the entry table and the RoPE factors in the tables region
    uint32_t off_rope;
    uint32_t off_ents;
    uint32_t adv;        // tokens advanced since the prepare (g4_attn_step_advance)
    uint32_t max_rows;   // the largest seq_len of the prepared entries
    uint32_t max_pos;    // the largest position of the prepared entries
};
static_assert(sizeof(StepPlanRep) <= sizeof(g4_decode_plan), "plan size");
static_assert(kStepMaxWgs <= 65535 && kMaxGroup <= 255, "plan field widths");

// A plan advances at most this many tokens between prepares: beyond it, the
// part holding the last row of a full-attention entry would carry a growing
// share of the rows (32 tokens add one 32-row tile to it).
constexpr uint32_t kStepMaxAdvance = 4096;

}  // namespace

extern "C" {

int g4_attn_step_workspace_size(uint32_t n_entries, uint32_t num_q_heads, uint32_t num_kv_heads, uint32_t head_dim,
                                size_t* bytes) {
    if (!bytes) return fail(G4_EINVAL, "g4_attn_step_workspace_size: bytes is NULL");
    if (head_dim != 256 && head_dim != 512)
        return fail(G4_EINVAL, "attnStep: head_dim %u unsupported (256 or 512)", head_dim);
    if (num_kv_heads == 0 || num_q_heads % num_kv_heads || num_q_heads / num_kv_heads > (uint32_t)kMaxGroup)
        return fail(G4_EINVAL, "attnStep: %u query heads over %u kv heads unsupported", num_q_heads, num_kv_heads);
    if (num_kv_heads > 65535) return fail(G4_EINVAL, "attnStep: %u kv heads (max 65535)", num_kv_heads);
    *bytes = step_layout(n_entries, num_kv_heads, num_q_heads / num_kv_heads, head_dim).total;
    return G4_OK;
}

static void write_plan(g4_decode_plan* plan, char* tables, char* part_ml, const g4_step_entry* entries,
                       uint32_t n_entries, uint32_t num_kv_heads, uint32_t G, uint32_t head_dim,
                       const StepPlanHost& ph) {
    StepPlanRep r = {};
    r.tables = tables;
    r.part_ml = part_ml;
    r.n_entries = (uint16_t)n_entries;
    r.num_kv_heads = (uint16_t)num_kv_heads;
    r.n_wgs = (uint16_t)ph.n_wgs;
    r.n_merge = (uint16_t)ph.n_merge;
    r.max_parts = (uint16_t)ph.max_parts;
    r.group = (uint8_t)G;
    r.waves = (uint8_t)ph.waves;
    r.head_dim = head_dim;
    r.magic = kStepMagic;
    r.off_merge = (uint32_t)ph.off_merge;
    r.off_rope = (uint32_t)ph.off_rope;
    r.off_ents = (uint32_t)ph.off_ents;
    for (uint32_t i = 0; i < n_entries; i++) {
        r.max_rows = std::max(r.max_rows, entries[i].seq_len);
        r.max_pos = std::max(r.max_pos, entries[i].position);
    }
    memset(plan, 0, sizeof *plan);
    memcpy(plan, &r, sizeof r);
}

int g4_attn_step_prepare(const g4_step_entry* entries, uint32_t n_entries, uint32_t num_q_heads,
                         uint32_t num_kv_heads, uint32_t head_dim, void* workspace, size_t workspace_bytes,
                         g4_decode_plan* plan, void* stream) {
    size_t need = 0;
    int rc = g4_attn_step_workspace_size(n_entries, num_q_heads, num_kv_heads, head_dim, &need);
    if (rc) return rc;
    if (!plan) return fail(G4_EINVAL, "attnStep: plan is NULL");
    if (!workspace || workspace_bytes < need)
        return fail(G4_ENOSPC, "attnStep: workspace %zu bytes < %zu needed", workspace_bytes, need);
    const uint32_t G = num_q_heads / num_kv_heads;
    const StepLayout L = step_layout(n_entries, num_kv_heads, G, head_dim);
    char* ws = static_cast<char*>(workspace);
    static thread_local StepPlanHost ph;  // the planner's storage, kept between the thread's prepares
    char err[256];
    rc = plan_step(entries, n_entries, num_q_heads, num_kv_heads, head_dim, device_cus(), StepTuning{},
                   ws + L.tables, &ph, err, sizeof err);
    if (rc) return fail(rc, "%s", err);
    rc = stage_upload(ws + L.tables, ph.blob.data(), ph.blob.size(), as_stream(stream));  // the tables in one copy
    if (rc) return rc;
    write_plan(plan, ws + L.tables, ws + L.part_ml, entries, n_entries, num_kv_heads, G, head_dim, ph);
    return G4_OK;
}

// Layers workspace: every layer's tables region (as a step of entries_per_layer
// entries), packed from the start, then every layer's partial records.
int g4_attn_step_layers_workspace_size(uint32_t n_layers, uint32_t entries_per_layer, uint32_t num_q_heads,
                                       uint32_t num_kv_heads, uint32_t head_dim, size_t* bytes) {
    size_t one = 0;
    int rc = g4_attn_step_workspace_size(entries_per_layer, num_q_heads, num_kv_heads, head_dim, &one);
    if (rc) return rc;
    if (n_layers == 0 || n_layers > 65535) return fail(G4_EINVAL, "attnStepLayers: %u layers (1..65535)", n_layers);
    if (entries_per_layer == 0 || entries_per_layer > 65535)
        return fail(G4_EINVAL, "attnStepLayers: %u entries per layer (1..65535)", entries_per_layer);
    *bytes = (size_t)n_layers * one;
    return G4_OK;
}

int g4_attn_step_prepare_layers(const g4_step_entry* entries, uint32_t n_layers, uint32_t entries_per_layer,
                                uint32_t num_q_heads, uint32_t num_kv_heads, uint32_t head_dim, void* workspace,
                                size_t workspace_bytes, g4_decode_plan* plans, void* stream) {
    size_t need = 0;
    int rc = g4_attn_step_layers_workspace_size(n_layers, entries_per_layer, num_q_heads, num_kv_heads, head_dim,
                                                &need);
    if (rc) return rc;
    if (!entries || !plans) return fail(G4_EINVAL, "attnStepLayers: NULL pointer");
    if (!workspace || workspace_bytes < need)
        return fail(G4_ENOSPC, "attnStepLayers: workspace %zu bytes < %zu needed", workspace_bytes, need);
    for (uint32_t i = 0; i < n_layers; i++) memset(&plans[i], 0, sizeof plans[i]);
    const uint32_t G = num_q_heads / num_kv_heads, E = entries_per_layer;
    const StepLayout L1 = step_layout(E, num_kv_heads, G, head_dim);
    const size_t tables_one = L1.part_ml, records_one = L1.total - L1.part_ml;
    char* ws = static_cast<char*>(workspace);
    char* const records = ws + (size_t)n_layers * tables_one;
    static thread_local StepPlanHost ph;
    static thread_local StepRopeShare share;  // RoPE factor sets placed by earlier layers of this upload
    static thread_local std::vector<char> blob;
    share.clear();
    blob.clear();
    char err[256];
    for (uint32_t i = 0; i < n_layers; i++) {
        char* const tables = ws + blob.size();
        rc = plan_step(entries + (size_t)i * E, E, num_q_heads, num_kv_heads, head_dim, device_cus(), StepTuning{},
                       tables, &ph, err, sizeof err, &share);
        if (rc) {  // no plan of this call is usable: their tables were never uploaded
            for (uint32_t j = 0; j < i; j++) memset(&plans[j], 0, sizeof plans[j]);
            return fail(rc, "attnStepLayers: layer %u: %s", i, err);
        }
        // packed tables never outgrow one layer's share of the region (each fits a step of E entries)
        const size_t at = blob.size(), bytes = align256(ph.blob.size());
        blob.resize(at + bytes);
        memcpy(blob.data() + at, ph.blob.data(), ph.blob.size());
        memset(blob.data() + at + ph.blob.size(), 0, bytes - ph.blob.size());
        write_plan(&plans[i], tables, records + (size_t)i * records_one, entries + (size_t)i * E, E, num_kv_heads, G,
                   head_dim, ph);
    }
    rc = stage_upload(ws, blob.data(), blob.size(), as_stream(stream));  // every layer's tables in one copy
    if (rc) {
        for (uint32_t i = 0; i < n_layers; i++) memset(&plans[i], 0, sizeof plans[i]);
        return rc;
    }
    return G4_OK;
}

static int step_plan(const g4_decode_plan* plan, StepPlanRep* r) {
    if (!plan) return fail(G4_EINVAL, "attnStep: plan is NULL");
    memcpy(r, plan, sizeof *r);
    if (r->magic != kStepMagic)
        return fail(G4_EINVAL, "attnStep: plan was not prepared by g4_attn_step_prepare or g4_attn_step_prepare_layers");
    return G4_OK;
}

static int launch_attention(const g4_decode_plan* plan, void* stream, hipEvent_t start, hipEvent_t stop) {
    StepPlanRep r;
    int rc = step_plan(plan, &r);
    if (rc) return rc;
    StepArgs a = {};
    a.work = reinterpret_cast<const StepWorkDev*>(r.tables);
    a.num_kv_heads = r.num_kv_heads;
    a.group = r.group;
    a.part_ml = reinterpret_cast<float*>(r.part_ml);
    a.part_o = reinterpret_cast<float*>(r.part_ml + step_part_o_offset(r.num_kv_heads, r.group));
    const dim3 grid(r.n_wgs, r.num_kv_heads);
    hipStream_t st = as_stream(stream);
    const uint32_t adv = r.adv;
    if (r.head_dim == 512) {
        if (start || stop)
            hipExtLaunchKernelGGL((k_attn_step<4, 512>), grid, dim3(256), 0, st, start, stop, 0, a.work, a.part_ml,
                                  a.part_o, a.num_kv_heads, a.group, adv);
        else
            G4_LAUNCH((k_attn_step<4, 512>), grid, dim3(256), 0, st, a.work, a.part_ml, a.part_o, a.num_kv_heads,
                      a.group, adv);
    } else if (r.waves == 8) {
        if (start || stop)
            hipExtLaunchKernelGGL((k_attn_step<8, 256>), grid, dim3(512), 0, st, start, stop, 0, a.work, a.part_ml,
                                  a.part_o, a.num_kv_heads, a.group, adv);
        else
            G4_LAUNCH((k_attn_step<8, 256>), grid, dim3(512), 0, st, a.work, a.part_ml, a.part_o, a.num_kv_heads,
                      a.group, adv);
    } else {
        if (start || stop)
            hipExtLaunchKernelGGL((k_attn_step<4, 256>), grid, dim3(256), 0, st, start, stop, 0, a.work, a.part_ml,
                                  a.part_o, a.num_kv_heads, a.group, adv);
        else
            G4_LAUNCH((k_attn_step<4, 256>), grid, dim3(256), 0, st, a.work, a.part_ml, a.part_o, a.num_kv_heads,
                      a.group, adv);
    }
    G4_CHECK_LAUNCH("attnStep");
    return G4_OK;
}

// The head_dim-512 and head_dim-256 plans of one token as one launch (k_attn_step_pair).
static int launch_attention_pair(const g4_decode_plan* plan_1, const g4_decode_plan* plan_2, void* stream,
                                 hipEvent_t start, hipEvent_t stop) {
    StepPlanRep r1, r2;
    int rc = step_plan(plan_1, &r1);
    if (rc) return rc;
    rc = step_plan(plan_2, &r2);
    if (rc) return rc;
    const StepPlanRep& a = r1.head_dim == 512 ? r1 : r2;
    const StepPlanRep& b = r1.head_dim == 512 ? r2 : r1;
    if (a.head_dim != 512 || b.head_dim != 256)
        return fail(G4_EINVAL, "attnStepPair: needs one plan of head_dim 512 and one of 256 (got %u and %u)",
                    r1.head_dim, r2.head_dim);
    if (a.tables == b.tables) return fail(G4_EINVAL, "attnStepPair: the two plans share their tables");
    auto ml = [](const StepPlanRep& r) { return reinterpret_cast<float*>(r.part_ml); };
    auto po = [](const StepPlanRep& r) {
        return reinterpret_cast<float*>(r.part_ml + step_part_o_offset(r.num_kv_heads, r.group));
    };
    const dim3 grid((uint32_t)a.n_wgs + b.n_wgs, std::max(a.num_kv_heads, b.num_kv_heads));
    const StepWorkDev* wa = reinterpret_cast<const StepWorkDev*>(a.tables);
    const StepWorkDev* wb = reinterpret_cast<const StepWorkDev*>(b.tables);
    hipStream_t st = as_stream(stream);
    if (start || stop)
        hipExtLaunchKernelGGL(k_attn_step_pair, grid, dim3(256), 0, st, start, stop, 0, wa, ml(a), po(a),
                              (uint32_t)a.num_kv_heads, (uint32_t)a.group, a.adv, (uint32_t)a.n_wgs, wb, ml(b), po(b),
                              (uint32_t)b.num_kv_heads, (uint32_t)b.group, b.adv);
    else
        G4_LAUNCH(k_attn_step_pair, grid, dim3(256), 0, st, wa, ml(a), po(a), (uint32_t)a.num_kv_heads,
                  (uint32_t)a.group, a.adv, (uint32_t)a.n_wgs, wb, ml(b), po(b), (uint32_t)b.num_kv_heads,
                  (uint32_t)b.group, b.adv);
    G4_CHECK_LAUNCH("attnStepPair");
    return G4_OK;
}

int g4_attn_step_run_attention_pair(const g4_decode_plan* plan_1, const g4_decode_plan* plan_2, void* stream) {
    return launch_attention_pair(plan_1, plan_2, stream, nullptr, nullptr);
}

int g4_attn_step_run_attention_pair_timed(const g4_decode_plan* plan_1, const g4_decode_plan* plan_2, void* stream,
                                          void* start_event, void* stop_event) {
    if (!start_event || !stop_event) return fail(G4_EINVAL, "attnStepPair: timing events are NULL");
    return launch_attention_pair(plan_1, plan_2, stream, static_cast<hipEvent_t>(start_event),
                                 static_cast<hipEvent_t>(stop_event));
}

static DecodeArgs merge_args(const StepPlanRep& r) {
    DecodeArgs m = {};
    m.table = reinterpret_cast<const DecodeEntryDev*>(r.tables + r.off_merge);
    m.n_entries = r.n_merge;
    m.num_kv_heads = r.num_kv_heads;
    m.group = r.group;
    m.part_ml = reinterpret_cast<float*>(r.part_ml);
    m.part_o = reinterpret_cast<float*>(r.part_ml + step_part_o_offset(r.num_kv_heads, r.group));
    return m;
}

int g4_attn_step_run_pair(const g4_decode_plan* plan_1, const g4_decode_plan* plan_2, void* stream) {
    int rc = launch_attention_pair(plan_1, plan_2, stream, nullptr, nullptr);
    if (rc) return rc;
    // Both merges in one launch when the plans' merges are of the two kinds it takes (checked above:
    // one plan per head_dim); otherwise one after the other.
    StepPlanRep r1, r2;
    memcpy(&r1, plan_1, sizeof r1);
    memcpy(&r2, plan_2, sizeof r2);
    const StepPlanRep& a = r1.head_dim == 512 ? r1 : r2;
    const StepPlanRep& b = r1.head_dim == 512 ? r2 : r1;
    rc = launch_decode_merge_pair(merge_args(a), a.n_merge, a.max_parts, merge_args(b), b.n_merge, b.max_parts,
                                  as_stream(stream));
    if (rc <= 0) return rc;
    rc = g4_attn_step_run_merge(plan_1, stream);
    if (rc) return rc;
    return g4_attn_step_run_merge(plan_2, stream);
}

int g4_attn_step_advance(g4_decode_plan* plan, uint32_t tokens) {
    StepPlanRep r;
    int rc = step_plan(plan, &r);
    if (rc) return rc;
    const uint64_t adv = (uint64_t)r.adv + tokens;
    if (adv > kStepMaxAdvance)
        return fail(G4_ERANGE, "attnStepAdvance: %llu tokens since the prepare (max %u): prepare again",
                    (unsigned long long)adv, kStepMaxAdvance);
    const uint64_t row_bytes = (uint64_t)r.num_kv_heads * r.head_dim * 2;
    if ((r.max_rows + adv) * row_bytes > 0xffffffffull)
        return fail(G4_EINVAL, "attnStepAdvance: a cache would exceed 4 GiB at %llu rows",
                    (unsigned long long)(r.max_rows + adv));
    if (r.max_pos + adv > 0xffffffffull)
        return fail(G4_EINVAL, "attnStepAdvance: position %llu out of range", (unsigned long long)(r.max_pos + adv));
    r.adv = (uint32_t)adv;
    memcpy(plan, &r, sizeof r);
    return G4_OK;
}

int g4_attn_step_run_attention(const g4_decode_plan* plan, void* stream) {
    return launch_attention(plan, stream, nullptr, nullptr);
}

int g4_attn_step_run_attention_timed(const g4_decode_plan* plan, void* stream, void* start_event, void* stop_event) {
    if (!start_event || !stop_event) return fail(G4_EINVAL, "attnStep: timing events are NULL");
    return launch_attention(plan, stream, static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event));
}

int g4_attn_step_run_merge(const g4_decode_plan* plan, void* stream) {
    StepPlanRep r;
    int rc = step_plan(plan, &r);
    if (rc) return rc;
    if (!r.n_merge) return G4_OK;
    DecodeArgs m = {};
    m.table = reinterpret_cast<const DecodeEntryDev*>(r.tables + r.off_merge);
    m.n_entries = r.n_merge;
    m.num_kv_heads = r.num_kv_heads;
    m.group = r.group;
    m.part_ml = reinterpret_cast<float*>(r.part_ml);
    m.part_o = reinterpret_cast<float*>(r.part_ml + step_part_o_offset(r.num_kv_heads, r.group));
    return launch_decode_merge(m, r.n_merge, r.max_parts, as_stream(stream), r.head_dim);
}

int g4_attn_step_run_out(const g4_decode_plan* plan, const g4_linear_seg* o_proj, uint32_t n_segs, void* stream) {
    StepPlanRep r;
    int rc = step_plan(plan, &r);
    if (rc) return rc;
    if (!o_proj) return fail(G4_EINVAL, "attnStepOut: o_proj is NULL");
    if (n_segs != r.n_entries)
        return fail(G4_EINVAL, "attnStepOut: %u weight segments for a step of %u entries", n_segs, r.n_entries);
    if (n_segs > (uint32_t)kOutMaxSegs)
        return fail(G4_EINVAL, "attnStepOut: %u entries (max %d)", n_segs, kOutMaxSegs);
    const uint32_t n = r.num_kv_heads * r.group * r.head_dim;
    if (n % 256 || n / 256 < 4 || n / 256 > 16)
        return fail(G4_EINVAL, "attnStepOut: input length %u unsupported (a multiple of 256 in [1024, 4096])", n);
    StepOutArgs a = {};
    for (uint32_t i = 0; i < n_segs; i++) {
        const g4_linear_seg& sg = o_proj[i];
        if (!sg.weight || !sg.out) return fail(G4_EINVAL, "attnStepOut: segment %u has a NULL pointer", i);
        if (reinterpret_cast<uintptr_t>(sg.weight) & 15)
            return fail(G4_EINVAL, "attnStepOut: segment %u weight must be 16-byte aligned", i);
        if (sg.rows == 0 || sg.rows > 0x7fffffffu) return fail(G4_EINVAL, "attnStepOut: segment %u has %u rows", i, sg.rows);
        a.seg[i] = OutSegDev{sg.weight, sg.out, sg.rows, 0};
    }
    hipStream_t st = as_stream(stream);
    const bool fused = step_out_merges(r.max_parts, r.group, r.num_kv_heads);
    if (!fused && (rc = g4_attn_step_run_merge(plan, stream))) return rc;
    a.ents = reinterpret_cast<const DecodeEntryDev*>(r.tables + r.off_ents);
    a.part_ml = reinterpret_cast<const float*>(r.part_ml);
    a.part_o = reinterpret_cast<const float*>(r.part_ml + step_part_o_offset(r.num_kv_heads, r.group));
    a.num_kv_heads = r.num_kv_heads;
    a.group = r.group;
    a.merge = fused ? 1u : 0u;
    return launch_step_out(a, r.n_entries, r.max_parts, r.head_dim, n, st);
}

int g4_attn_step_run(const g4_decode_plan* plan, void* stream) {
    int rc = g4_attn_step_run_attention(plan, stream);
    if (rc) return rc;
    return g4_attn_step_run_merge(plan, stream);
}

int g4_attn_step(const g4_step_entry* entries, uint32_t n_entries, uint32_t num_q_heads, uint32_t num_kv_heads,
                 uint32_t head_dim, void* workspace, size_t workspace_bytes, void* stream) {
    g4_decode_plan plan;
    int rc = g4_attn_step_prepare(entries, n_entries, num_q_heads, num_kv_heads, head_dim, workspace,
                                  workspace_bytes, &plan, stream);
    if (rc) return rc;
    return g4_attn_step_run(&plan, stream);
}

}  // extern "C"
