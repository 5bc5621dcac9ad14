// One-launch decode step for gfx950: the whole attention block of one token
// for a set of layers or sequences ("entries"), in a single kernel:
//
//   vNorm + fusedNormRope(Q, K) + kvCacheStore + attnScore -> softmax ->
//   attnOutput
//
// i.e. the dispatch sequence of src/engine.ts:2056-2094 (shaders
// per_head_rms_norm_no_weight.wgsl, fused_per_head_norm_rope.wgsl,
// kv_cache_store.wgsl, attn_score.wgsl, softmax.wgsl, attn_output.wgsl),
// with flash-decoding split-K and the split merge inside the same launch.
//
// Work split: all entries' attended rows form one sequence of 32-row tiles;
// workgroup w takes tiles [w*T/W, (w+1)*T/W), so every workgroup streams the
// same number of rows whatever the mix of long and short entries. A range that
// crosses entries is processed entry by entry ("segments").
//
// Per segment a workgroup computes the entry's post-norm, post-RoPE query
// itself (from the raw projection; one wave per head, evaluating exactly the
// reference's expressions and reduction tree, so the values are bit-identical
// to the prep kernel's), overlapped with the first tile's loads. The
// workgroup whose range holds the entry's last row (the current token's row)
// also computes that row's k (norm + RoPE) and v (weightless norm), uses them
// for that row instead of the cache, and stores them as f16 when the entry
// owns the cache (KV-producer layers).
//
// Merge: a segment covering a whole entry writes attnOut directly; otherwise
// it writes a partial record (m, l, unnormalised o per head) and the fixed-order
// log-sum-exp merge kernel of decode.hip combines an entry's records in a
// second launch. (Merging inside this launch needs a device-scope release per
// workgroup; on gfx950 that is an L2 write-back plus invalidate, measured far
// costlier than the second launch.)
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "decode_core.h"
#include "ref_math.h"

namespace g4 {

struct StepEntryDev {
    const float* q;  // raw projections, [num_kv_heads][group][HD] and [num_kv_heads][HD]
    const float* k;
    const float* v;
    const uint16_t* q_weight;
    const uint16_t* k_weight;
    const uint16_t* rope_freqs;
    uint16_t* k_cache;  // [rows][num_kv_heads][HD]
    uint16_t* v_cache;
    float* out;         // attnOut [num_kv_heads][group][HD]
    uint32_t key_begin; // attended rows [key_begin, key_end); the current row is key_end - 1
    uint32_t key_end;
    uint32_t tile_base; // first global tile
    uint32_t n_tiles;
    uint32_t w_first;   // first workgroup on this entry
    uint32_t n_parts;   // workgroups on this entry
    uint32_t position;  // RoPE position
    uint32_t store_kv;
    float theta;
    uint32_t apply_divisor;
    float qscale;       // attention scale * log2(e)
    float eps;
};

struct StepArgs {
    const StepEntryDev* table;
    uint32_t n_entries;
    uint32_t total_tiles;
    uint32_t n_wgs;
    uint32_t num_kv_heads;
    uint32_t group;
    uint32_t pad;
    float* part_ml;  // partial records [(w + e) * NKH + kvh][group][2]
    float* part_o;   //                  [(w + e) * NKH + kvh][group][HD]
};

constexpr int kStepHD = 256;

// RoPE factors of pairs (l, l + 128) and (l + 64, l + 192) for lane l (head_dim
// 256), exactly the reference expressions (rope_angle in ref_math.h).
struct RopeLane {
    float c0, s0, c1, s1;
};

// Not inlined: inlined into the segment loop, the f64 library code's constants
// are hoisted out of the loop and spill.
__device__ __attribute__((noinline)) RopeLane rope_lane(int lane, float theta, unsigned position,
                                                        unsigned apply_divisor, const uint16_t* rope_freqs) {
    RopeLane r;
    const float a0 = rope_angle((unsigned)lane, kStepHD, theta, position, apply_divisor, rope_freqs);
    const float a1 = rope_angle((unsigned)lane + 64u, kStepHD, theta, position, apply_divisor, rope_freqs);
    r.c0 = (float)cos((double)a0);
    r.s0 = (float)sin((double)a0);
    r.c1 = (float)cos((double)a1);
    r.s1 = (float)sin((double)a1);
    return r;
}

// Per-head RMSNorm (+ RoPE) of one 256-wide head by one wave; lane l holds
// x[l + 64j], j = 0..3, and receives the results in place. The sum of squares
// adds the same pairs in the same order as the reference's workgroup tree
// (strides 128, 64, then 32..1), so every value is bit-identical to
// fused_per_head_norm_rope.wgsl / per_head_rms_norm_no_weight.wgsl.
__device__ __forceinline__ void wave_norm_rope(float (&x)[4], const uint16_t* weight, bool rope, const RopeLane& r,
                                               float eps, int lane) {
#pragma clang fp contract(off)
    float p[4];
#pragma unroll
    for (int j = 0; j < 4; j++) p[j] = x[j] * x[j];
    const float a = p[0] + p[2];  // t = lane      : s[t] + s[t + 128]
    const float b = p[1] + p[3];  // t = lane + 64 : s[t] + s[t + 128]
    float c = a + b;              // stride 64
    for (int stride = 32; stride > 0; stride >>= 1) c = c + __shfl_down(c, stride);
    const float total = __shfl(c, 0);
    const float rms = sqrtf(total / (float)kStepHD + eps);
#pragma unroll
    for (int j = 0; j < 4; j++) x[j] = weight ? x[j] * h2f(weight[lane + 64 * j]) / rms : x[j] / rms;
    if (!rope) return;
    const float x0 = x[0], x1 = x[1], x2 = x[2], x3 = x[3];
    x[0] = x0 * r.c0 - x2 * r.s0;
    x[2] = x0 * r.s0 + x2 * r.c0;
    x[1] = x1 * r.c1 - x3 * r.s1;
    x[3] = x1 * r.s1 + x3 * r.c1;
}

struct StepSmem {
    DecodeSmem<kStepHD> dec;
    float qf[kMaxGroup][kStepHD];  // post-prep q * qscale
    f16x8 knew[kStepHD / 8];       // current row's k and v, f16 (as stored)
    f16x8 vnew[kStepHD / 8];
    float mnew[kMaxGroup];         // current row's scores (log2 units)
};

__host__ __device__ __forceinline__ unsigned wg_of_tile(uint64_t x, uint64_t T, uint64_t W) {  // max w: floor(wT/W) <= x
    return (unsigned)(((x + 1) * W - 1) / T);
}

// One segment: entry e, this workgroup's tiles [t_begin, t_end) of it (global
// tile indices).
__device__ __forceinline__ void attn_segment(const StepArgs a, StepSmem& sm, unsigned w, unsigned kvh,
                                                       unsigned e, unsigned t_begin, unsigned t_end) {
    using D = DecodeDims<kStepHD>;
    constexpr unsigned HD = kStepHD;
    const unsigned NKH = a.num_kv_heads;
    const unsigned G = a.group;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n = lane & 15;
    const int g = lane >> 4;
    const int head = n & 7;
    const bool lo_col = n >= 8;

    const StepEntryDev& ent = a.table[e];  // fields read where used (scalar loads)
    const unsigned tile_base = ent.tile_base;
    const unsigned key_begin = ent.key_begin, key_end = ent.key_end;
    const unsigned k0 = key_begin + (t_begin - tile_base) * kTileKeys;
    const unsigned k1 = min(key_end, key_begin + (t_end - tile_base) * kTileKeys);
    const bool has_new = k1 == key_end;  // this segment holds the current token's row
    const unsigned new_row = key_end - 1;
    const unsigned k1t = has_new ? new_row : k1;  // rows read from the cache: [k0, k1t)

    const RopeLane rl = rope_lane(lane, ent.theta, ent.position, ent.apply_divisor, ent.rope_freqs);

    const uint32_t row_bytes = NKH * HD * 2u;
    const char* Kb = reinterpret_cast<const char*>(ent.k_cache + (uint64_t)kvh * HD);
    const char* Vb = reinterpret_cast<const char*>(ent.v_cache + (uint64_t)kvh * HD);
    const unsigned nkeys = k1t - k0;
    const unsigned last = k1t - 1;  // only used when nkeys > 0
    constexpr unsigned kStride = kDecodeWaves * kTileKeys;

    // First tile in flight while the query is normalised and rotated.
    unsigned t0 = (unsigned)wave * kTileKeys;
    f16x8 kreg[2][D::NC];
    u32x4 vreg[D::NB][8];
    if (t0 < nkeys) {
        load_k_tile<HD>(Kb, row_bytes, last, n, g, k0 + t0, kreg);
        load_v_tile<HD>(Vb, row_bytes, last, n, g, k0 + t0, vreg);
    }

    // ---- prep: q heads (2 per wave), and the current row's k and v ----
    const float qscale = ent.qscale, eps = ent.eps;
    for (unsigned hq = (unsigned)wave; hq < G; hq += kDecodeWaves) {
        const float* src = ent.q + ((uint64_t)kvh * G + hq) * HD;
        float x[4];
#pragma unroll
        for (int j = 0; j < 4; j++) x[j] = ldg<float>(src + lane + 64 * j);
        wave_norm_rope(x, ent.q_weight, true, rl, eps, lane);
#pragma unroll
        for (int j = 0; j < 4; j++) sm.qf[hq][lane + 64 * j] = x[j] * qscale;
    }
    if (has_new && wave < 2) {
        const bool is_k = wave == 0;
        const float* src = (is_k ? ent.k : ent.v) + (uint64_t)kvh * HD;
        float x[4];
#pragma unroll
        for (int j = 0; j < 4; j++) x[j] = ldg<float>(src + lane + 64 * j);
        wave_norm_rope(x, is_k ? ent.k_weight : nullptr, is_k, rl, eps, lane);
        uint16_t* row = reinterpret_cast<uint16_t*>(is_k ? sm.knew : sm.vnew);
#pragma unroll
        for (int j = 0; j < 4; j++) row[lane + 64 * j] = f2h(x[j]);
        if (ent.store_kv) {
            uint16_t* dst = (is_k ? ent.k_cache : ent.v_cache) + ((uint64_t)new_row * NKH + kvh) * HD;
#pragma unroll
            for (int j = 0; j < 4; j++) stg<uint16_t>(dst + lane + 64 * j, f2h(x[j]));
        }
    }
    __syncthreads();
    // Score operand from the prepared query, and the current row's scores.
    {
        const bool live = (unsigned)head < G;
#pragma unroll
        for (int cc = 0; cc < D::NC / kDecodeWaves; cc++) {
            const int c = wave * (D::NC / kDecodeWaves) + cc;
            float x[8];
#pragma unroll
            for (int i = 0; i < 8; i++) x[i] = live ? sm.qf[head][c * 32 + g * 8 + i] : 0.0f;
            store_q_chunk<HD>(sm.dec, c, lane, x, lo_col);
        }
        if (has_new) {
            const f16* kn = reinterpret_cast<const f16*>(sm.knew);
            for (unsigned h = (unsigned)wave; h < G; h += kDecodeWaves) {
                float p = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; j++) p += sm.qf[h][lane + 64 * j] * (float)kn[lane + 64 * j];
                for (int off = 32; off > 0; off >>= 1) p += __shfl_xor(p, off);
                if (lane == 0) sm.mnew[h] = p;
            }
        }
    }
    __syncthreads();

    float m_run = -INFINITY, l_run = 0.0f;
    f32x4 acc[D::NO];
#pragma unroll
    for (int i = 0; i < D::NO; i++) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (t0 < nkeys) {  // the first tile was requested above; the loop requests its own
        tile_step<HD>(sm.dec, lane, g, lo_col, k0 + t0, k1t, kreg, vreg, m_run, l_run, acc);
        for (t0 += kStride; t0 < nkeys; t0 += kStride) {
            load_k_tile<HD>(Kb, row_bytes, last, n, g, k0 + t0, kreg);
            load_v_tile<HD>(Vb, row_bytes, last, n, g, k0 + t0, vreg);
            tile_step<HD>(sm.dec, lane, g, lo_col, k0 + t0, k1t, kreg, vreg, m_run, l_run, acc);
        }
    }
    wave_publish<HD>(sm.dec, wave, n, g, m_run, l_run, acc);
    __syncthreads();

    const float* em = has_new ? sm.mnew : nullptr;
    const f16* ev = reinterpret_cast<const f16*>(sm.vnew);
    float* out = ent.out + (uint64_t)kvh * G * HD;
    const unsigned n_parts = ent.n_parts;
    if (n_parts == 1) {
        wg_combine_write<HD>(sm.dec, G, true, out, nullptr, nullptr, em, ev);
        __syncthreads();
        return;
    }
    // Partial record at slot (w + e) * NKH + kvh: unique, and consecutive over the
    // workgroups of an entry, so the merge reads split_base = w_first + e.
    const uint64_t rec = ((uint64_t)(w + e) * NKH + kvh) * G;
    wg_combine_write<HD>(sm.dec, G, false, nullptr, a.part_o + rec * HD, a.part_ml + rec * 2, em, ev);
    __syncthreads();
}

__global__ __launch_bounds__(kDecodeThreads, 2) void k_attn_step(StepArgs a) {
    __shared__ StepSmem sm;
    const unsigned w = blockIdx.x;
    const unsigned kvh = blockIdx.y;
    const uint64_t T = a.total_tiles, W = a.n_wgs;
    unsigned tb = (unsigned)((uint64_t)w * T / W);
    const unsigned te = (unsigned)((uint64_t)(w + 1) * T / W);
    unsigned e;  // entry holding tile tb: last with tile_base <= tb
    {
        unsigned lo = 0, hi = a.n_entries;
        while (hi - lo > 1) {
            const unsigned mid = (lo + hi) >> 1;
            if (a.table[mid].tile_base <= tb) lo = mid;
            else hi = mid;
        }
        e = lo;
    }
    for (; tb < te; e++) {
        const unsigned seg_end = min(te, a.table[e].tile_base + a.table[e].n_tiles);
        attn_segment(a, sm, w, kvh, e, tb, seg_end);
        tb = seg_end;
    }
}

}  // namespace g4

using namespace g4;

namespace {

constexpr unsigned kStepMaxWgs = 1024;
constexpr uint32_t kStepMagic = 0x67345354u;

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int step_env(const char* name, int dflt) {
    const char* s = getenv(name);
    return s && *s ? atoi(s) : dflt;
}

struct StepPlanRep {
    char* ws;
    uint32_t n_entries;
    uint32_t total_tiles;
    uint32_t n_wgs;
    uint32_t num_kv_heads;
    uint32_t group;
    uint32_t any_split;  // some entry spans more than one workgroup: run the merge
    uint32_t magic;
};
static_assert(sizeof(StepPlanRep) <= sizeof(g4_decode_plan), "plan size");

struct StepLayout {
    size_t table, merge_table, part_ml, part_o, total;
};

StepLayout step_layout(uint64_t n, uint64_t wgs, uint64_t nkh, uint64_t group, uint64_t hd) {
    StepLayout L;
    size_t off = 0;
    L.table = off;
    off += align256(n * sizeof(StepEntryDev));
    L.merge_table = off;
    off += align256(n * sizeof(DecodeEntryDev));
    const uint64_t recs = (wgs + n) * nkh * group;
    L.part_ml = off;
    off += align256(recs * 2 * 4);
    L.part_o = off;
    off += align256(recs * hd * 4);
    L.total = off;
    return L;
}

// Pinned host staging for one table upload, reused once its previous copy completed.
struct Staging {
    void* buf = nullptr;
    size_t cap = 0;
    hipEvent_t done = nullptr;
};

int stage_upload(Staging& sg, void* dst, const void* src, size_t bytes, hipStream_t st) {
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

}  // namespace

extern "C" {

int g4_attn_step_workspace_size(uint32_t n_entries, uint32_t num_q_heads, uint32_t num_kv_heads, uint32_t head_dim,
                                size_t* bytes) {
    if (!bytes) return fail(G4_EINVAL, "g4_attn_step_workspace_size: bytes is NULL");
    if (head_dim != kStepHD) return fail(G4_EINVAL, "attnStep: head_dim %u unsupported (256)", head_dim);
    if (num_kv_heads == 0 || num_q_heads % num_kv_heads || num_q_heads / num_kv_heads > (uint32_t)kMaxGroup)
        return fail(G4_EINVAL, "attnStep: %u query heads over %u kv heads unsupported", num_q_heads, num_kv_heads);
    *bytes = step_layout(n_entries, kStepMaxWgs, num_kv_heads, num_q_heads / num_kv_heads, head_dim).total;
    return G4_OK;
}

int g4_attn_step_prepare(const g4_step_entry* entries, uint32_t n_entries, uint32_t num_q_heads,
                         uint32_t num_kv_heads, uint32_t head_dim, void* workspace, size_t workspace_bytes,
                         g4_decode_plan* plan, void* stream) {
    size_t need_max = 0;
    int rc = g4_attn_step_workspace_size(n_entries, num_q_heads, num_kv_heads, head_dim, &need_max);
    if (rc) return rc;
    if (!plan) return fail(G4_EINVAL, "attnStep: plan is NULL");
    if (!entries || n_entries == 0) return fail(G4_EINVAL, "attnStep: no entries");
    if (n_entries > 65535) return fail(G4_EINVAL, "attnStep: %u entries (max 65535)", n_entries);
    const uint32_t G = num_q_heads / num_kv_heads;
    const uint64_t row_bytes = (uint64_t)num_kv_heads * head_dim * 2;
    std::vector<StepEntryDev> tab(n_entries);
    uint64_t T = 0;
    for (uint32_t i = 0; i < n_entries; i++) {
        const g4_step_entry& s = entries[i];
        if (!s.q || !s.k || !s.v || !s.q_weight || !s.k_weight || !s.k_cache || !s.v_cache || !s.out)
            return fail(G4_EINVAL, "attnStep: entry %u has a NULL pointer", i);
        if (s.apply_divisor && !s.rope_freqs) return fail(G4_EINVAL, "attnStep: entry %u needs rope_freqs", i);
        if (s.seq_len == 0) return fail(G4_EINVAL, "attnStep: entry %u seq_len 0", i);
        if ((uint64_t)s.seq_len * row_bytes > 0xffffffffull)
            return fail(G4_EINVAL, "attnStep: entry %u cache exceeds 4 GiB", i);
        StepEntryDev& d = tab[i];
        d = StepEntryDev{};
        d.q = s.q;
        d.k = s.k;
        d.v = s.v;
        d.q_weight = s.q_weight;
        d.k_weight = s.k_weight;
        d.rope_freqs = s.rope_freqs;
        d.k_cache = s.k_cache;
        d.v_cache = s.v_cache;
        d.out = s.out;
        d.key_end = s.seq_len;
        d.key_begin = (s.sliding_window != 0 && s.seq_len > s.sliding_window) ? s.seq_len - s.sliding_window : 0;
        d.n_tiles = (d.key_end - d.key_begin + kTileKeys - 1) / kTileKeys;
        d.tile_base = (uint32_t)T;
        T += d.n_tiles;
        d.position = s.position;
        d.store_kv = s.store_kv;
        d.theta = s.theta;
        d.apply_divisor = s.apply_divisor;
        d.qscale = s.scale * kLog2e;
        d.eps = s.eps;
    }
    if (T > 0x7fffffffull) return fail(G4_EINVAL, "attnStep: too many rows");
    static const int wgs_per_cu = step_env("G4_STEP_WGS_PER_CU", 2);
    uint64_t W = (uint64_t)(wgs_per_cu > 0 ? wgs_per_cu : 2) * 256 / num_kv_heads;
    if (W > kStepMaxWgs) W = kStepMaxWgs;
    if (W > T) W = T;
    if (W == 0) W = 1;
    std::vector<DecodeEntryDev> merge(n_entries);
    uint32_t any_split = 0;
    for (uint32_t i = 0; i < n_entries; i++) {
        StepEntryDev& d = tab[i];
        const unsigned w0 = wg_of_tile(d.tile_base, T, W);
        const unsigned w1 = wg_of_tile((uint64_t)d.tile_base + d.n_tiles - 1, T, W);
        d.w_first = w0;
        d.n_parts = w1 - w0 + 1;
        any_split |= d.n_parts > 1;
        merge[i] = DecodeEntryDev{nullptr, nullptr, nullptr, d.out, 0, 0, w0 + i, d.n_parts, 0.0f, 0};
    }
    const StepLayout L = step_layout(n_entries, W, num_kv_heads, G, head_dim);
    if (!workspace || workspace_bytes < L.total)
        return fail(G4_ENOSPC, "attnStep: workspace %zu bytes < %zu needed", workspace_bytes, L.total);
    hipStream_t st = as_stream(stream);
    char* ws = static_cast<char*>(workspace);
    static thread_local Staging sg_table, sg_merge;
    rc = stage_upload(sg_table, ws + L.table, tab.data(), (size_t)n_entries * sizeof(StepEntryDev), st);
    if (rc) return rc;
    rc = stage_upload(sg_merge, ws + L.merge_table, merge.data(), (size_t)n_entries * sizeof(DecodeEntryDev), st);
    if (rc) return rc;
    StepPlanRep r = {ws, n_entries, (uint32_t)T, (uint32_t)W, num_kv_heads, G, any_split, kStepMagic};
    memset(plan, 0, sizeof *plan);
    memcpy(plan, &r, sizeof r);
    return G4_OK;
}

int g4_attn_step_run(const g4_decode_plan* plan, void* stream) {
    if (!plan) return fail(G4_EINVAL, "attnStep: plan is NULL");
    StepPlanRep r;
    memcpy(&r, plan, sizeof r);
    if (r.magic != kStepMagic) return fail(G4_EINVAL, "attnStep: plan was not prepared by g4_attn_step_prepare");
    const StepLayout L = step_layout(r.n_entries, r.n_wgs, r.num_kv_heads, r.group, kStepHD);
    StepArgs a = {};
    a.table = reinterpret_cast<const StepEntryDev*>(r.ws + L.table);
    a.n_entries = r.n_entries;
    a.total_tiles = r.total_tiles;
    a.n_wgs = r.n_wgs;
    a.num_kv_heads = r.num_kv_heads;
    a.group = r.group;
    a.part_ml = reinterpret_cast<float*>(r.ws + L.part_ml);
    a.part_o = reinterpret_cast<float*>(r.ws + L.part_o);
    hipStream_t st = as_stream(stream);
    hipLaunchKernelGGL(k_attn_step, dim3(r.n_wgs, r.num_kv_heads), dim3(kDecodeThreads), 0, st, a);
    G4_CHECK_LAUNCH("attnStep");
    if (!r.any_split) return G4_OK;
    DecodeArgs m = {};
    m.table = reinterpret_cast<const DecodeEntryDev*>(r.ws + L.merge_table);
    m.n_entries = r.n_entries;
    m.num_kv_heads = r.num_kv_heads;
    m.group = r.group;
    m.part_o = a.part_o;
    m.part_ml = a.part_ml;
    return launch_decode_merge(m, r.n_entries, st);
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
