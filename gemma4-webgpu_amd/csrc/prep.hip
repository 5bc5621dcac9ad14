// Fused producer-side prep for one layer and one token, in one launch:
// vNorm -> fusedNormRope(Q) -> fusedNormRope(K) -> kvCacheStore, the
// sequence gemma4-webgpu dispatches as four passes (src/engine.ts:2056-2091;
// shaders/per_head_rms_norm_no_weight.wgsl, fused_per_head_norm_rope.wgsl,
// kv_cache_store.wgsl). Workgroup b handles one head: b < NQH a query head,
// then NKH key heads, then NKH value heads. The per-head arithmetic is the
// shared head_norm_rope, so q/k/v and the stored f16 rows are bit-identical
// to the four reference kernels run in order. Launch-bound by nature
// (NQH + 2*NKH workgroups of 256 threads), so fusing the four passes into
// one removes three launches per producer layer.
#include "ref_math.h"

namespace g4 {

__global__ __launch_bounds__(kWG) void k_attn_prep(float* __restrict__ q, float* __restrict__ k, float* __restrict__ v,
                                                   const uint16_t* __restrict__ q_weight,
                                                   const uint16_t* __restrict__ k_weight,
                                                   const uint16_t* __restrict__ rope_freqs,
                                                   uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
                                                   g4_prep_params p) {
    __shared__ float scratch[kNormScratch];
    const unsigned b = blockIdx.x;
    const unsigned hd = p.head_dim;
    if (b < p.num_q_heads) {
        head_norm_rope(q + b * hd, q_weight, true, rope_freqs, hd, p.eps, p.position, p.theta, p.apply_divisor,
                       scratch);
        return;
    }
    const unsigned r = b - p.num_q_heads;
    const bool is_k = r < p.num_kv_heads;
    const unsigned h = is_k ? r : r - p.num_kv_heads;
    float* x = (is_k ? k : v) + h * hd;
    uint16_t* dst = (is_k ? k_cache : v_cache) + ((uint64_t)p.slot * p.num_kv_heads + h) * hd;
    if (is_k) {
        head_norm_rope(x, k_weight, true, rope_freqs, hd, p.eps, p.position, p.theta, p.apply_divisor, scratch, dst);
    } else {
        head_norm_rope(x, nullptr, false, nullptr, hd, p.eps, 0, 0.0f, 0, scratch, dst);
    }
}

// Many layers: blockIdx.y selects the layer's table entry.
__global__ __launch_bounds__(kWG) void k_attn_prep_many(const g4_prep_layer* __restrict__ layers,
                                                        uint32_t num_q_heads, uint32_t num_kv_heads, float eps,
                                                        uint32_t position, uint32_t slot) {
    __shared__ float scratch[kNormScratch];
    const g4_prep_layer L = layers[blockIdx.y];
    const unsigned b = blockIdx.x;
    const unsigned hd = L.head_dim;
    if (b < num_q_heads) {
        head_norm_rope(L.q + b * hd, L.q_weight, true, L.rope_freqs, hd, eps, position, L.theta, L.apply_divisor,
                       scratch);
        return;
    }
    if (!L.store_kv || slot >= L.max_seq_len) return;
    const unsigned r = b - num_q_heads;
    const bool is_k = r < num_kv_heads;
    const unsigned h = is_k ? r : r - num_kv_heads;
    float* x = (is_k ? L.k : L.v) + h * hd;
    uint16_t* dst = (is_k ? L.k_cache : L.v_cache) + ((uint64_t)slot * num_kv_heads + h) * hd;
    if (is_k) {
        head_norm_rope(x, L.k_weight, true, L.rope_freqs, hd, eps, position, L.theta, L.apply_divisor, scratch, dst);
    } else {
        head_norm_rope(x, nullptr, false, nullptr, hd, eps, 0, 0.0f, 0, scratch, dst);
    }
}

// Chunked prompt prep: the producer-side prep of every token of a prompt
// chunk in one launch. The engine runs vNorm -> fusedNormRope(Q, K) ->
// kvCacheStore once per prompt token (src/engine.ts:2460-2479, each token
// through 2056-2091). One workgroup per kPrepTokens consecutive tokens: its
// threads first take the RoPE inverse frequencies (from the caller's table
// when given, else the reference's f32 expression with its f64 pow; they do
// not depend on the position: measured on prefill4k's two layers, the table
// takes the prep from 41 to 37 us), then
// the cos and sin of every pair's f32 angle at each of its tokens' positions
// (in f64, as the reference does) into LDS; then its four waves take the
// tokens' head slots in turn: per token, slots 0 .. NQH-1 are the query heads
// (norm + RoPE, written as f16: the query operand g4_attn_prefill takes), then
// NKH key heads (norm + RoPE, stored as cache row start + t), then NKH value
// heads (weightless norm, stored). The per-head arithmetic is wave_norm_rope
// (the reference's 256 partials and 128 -> 1 tree), so every stored value is
// the f16 rounding of what the reference kernels compute token by token.
constexpr unsigned kPrepTokens = 2;  // measured: 1, 2, 4, 8 tokens -> 43.0, 40.6, 43.3, 52.4 us (prefill4k, both layers)

// Workgroups per 32-row block (kPrepTokens tokens each), and the XCDs whose
// workgroups a launch interleaves (workgroup b runs on XCD b % kXcds).
constexpr unsigned kPrepPerBlock = 32 / kPrepTokens;
constexpr unsigned kPromptPrepMany = 8;  // entries of one g4_attn_prompt_prep_many launch
constexpr unsigned kXcds = 8;

// The chunk's positions [start, start + n) in whole 32-row blocks from
// base = start rounded down to 32: workgroup b takes the kPrepTokens
// positions at base + kPrepTokens * (block * kPrepPerBlock + m) (those inside
// the chunk), where the workgroups of one block share an XCD: x = b % kXcds,
// i = b / kXcds, block = (i / kPrepPerBlock) * kXcds + x, m = i % kPrepPerBlock.
// So the V^T block a workgroup writes into is written by one XCD's workgroups
// only (its lines are assembled in one L2). The grid has
// kXcds * kPrepPerBlock * ceil(blocks / kXcds) workgroups; those past the
// last block exit.
__device__ __forceinline__ unsigned prep_first_pos(unsigned b, unsigned base) {
    const unsigned x = b % kXcds, i = b / kXcds;
    const unsigned block = (i / kPrepPerBlock) * kXcds + x, m = i % kPrepPerBlock;
    return base + (block * kPrepPerBlock + m) * kPrepTokens;
}

// vt_cache (optional): V^T in 32-row blocks [kv head][blocks][HD][32] f16,
// blocks = ceil(max_seq_len / 32): row r of kv head h, element d at
// [h][r / 32][d][r % 32]. The stored V rows go there too, and the rows of the
// chunk's last block past its end are written as 0, so that a prefill reading
// whole blocks multiplies finite values by the zero probabilities of keys it
// does not attend (the next chunk's prep overwrites them).
template <int HD>
__device__ __forceinline__ void prompt_prep_body(const float* __restrict__ q, const float* __restrict__ k,
                                                 const float* __restrict__ v, const uint16_t* __restrict__ q_weight,
                                                 const uint16_t* __restrict__ k_weight,
                                                 const uint16_t* __restrict__ rope_freqs,
                                                 const float* __restrict__ inv_table, uint16_t* __restrict__ q_out,
                                                 uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
                                                 uint16_t* __restrict__ vt_cache, const g4_prompt_prep_params& p,
                                                 unsigned wg) {
    constexpr int J = HD / 64, PJ = J / 2;
    constexpr unsigned NP = HD / 2;  // RoPE pairs
    static_assert(NP <= kWG, "one thread per RoPE pair");
    __shared__ float inv[NP];
    __shared__ float rc[kPrepTokens][NP], rs[kPrepTokens][NP];
    const unsigned base = p.start & ~31u, end = p.start + p.n_tokens;
    const unsigned pos0 = prep_first_pos(wg, base);
    if (pos0 >= end) return;  // uniform: past the chunk's last block (or a block's pair past its end)
    const unsigned lo = max(pos0, p.start);  // this workgroup's positions [lo, hi)
    const unsigned hi = min(pos0 + kPrepTokens, end);
    const unsigned nt = hi > lo ? hi - lo : 0u;
    const unsigned t0 = lo - p.start;  // token index of position lo
    if (vt_cache && p.store_kv && hi == end && (end & 31u)) {  // zeros past the chunk's end in its last block
        const unsigned blocks = (p.max_seq_len + 31) / 32, pad = 32 - (end & 31u);
        for (unsigned i = threadIdx.x; i < p.num_kv_heads * HD * pad; i += kWG) {
            const unsigned r = end + i % pad, hd = i / pad, h = hd / HD, d = hd % HD;
            vt_cache[(((uint64_t)h * blocks + r / 32) * HD + d) * 32 + r % 32] = 0;
        }
    }
    if (nt == 0) return;
    if (threadIdx.x < NP)
        inv[threadIdx.x] = inv_table ? inv_table[threadIdx.x]
                                     : rope_inv_freq(threadIdx.x, HD, p.theta, p.apply_divisor,
                                                     p.apply_divisor ? h2f(rope_freqs[threadIdx.x]) : 1.0f);
    __syncthreads();
    for (unsigned i = threadIdx.x; i < nt * NP; i += kWG) {
        const unsigned tt = i / NP, pr = i % NP;
        const float ang = (float)(lo + tt) * inv[pr];  // rope_angle's expression
        f64_cos_sin(ang, rc[tt][pr], rs[tt][pr]);
    }
    __syncthreads();
    const unsigned lane = threadIdx.x & 63;
    const unsigned wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // slot stepping stays scalar
    const unsigned S = p.num_q_heads + (p.store_kv ? 2 * p.num_kv_heads : 0);
    const unsigned vt_blocks = (p.max_seq_len + 31) / 32;
    uint32_t wq[J], wk[J];  // the norm weights, loaded once per wave
#pragma unroll
    for (int j = 0; j < J; j++) {
        wq[j] = q_weight[lane + 64 * j];
        wk[j] = p.store_kv ? k_weight[lane + 64 * j] : 0u;
    }
    // The wave's slots w = wave, wave + 4, ... of the nt * S (token, head slot) pairs, as (tt, slot)
    // stepped without a division.
    if (S == 0) return;  // (the host refuses it) every step below takes slot down by S
    unsigned tt = 0, slot = wave;
    while (slot >= S && tt < nt) {  // uniform
        slot -= S;
        tt++;
    }
    // Each row is requested one slot ahead, before the previous row's stores: a wait for a load
    // also waits for every older vector memory operation, so a row requested after those stores
    // would wait for them.
    auto row_src = [&](unsigned tt_, unsigned slot_) __attribute__((always_inline)) {
        const unsigned t_ = t0 + tt_;
        const unsigned r_ = slot_ - p.num_q_heads;
        return slot_ < p.num_q_heads ? q + ((uint64_t)t_ * p.num_q_heads + slot_) * HD
                                     : (r_ < p.num_kv_heads ? k + ((uint64_t)t_ * p.num_kv_heads + r_) * HD
                                                            : v + ((uint64_t)t_ * p.num_kv_heads + r_ - p.num_kv_heads) * HD);
    };
    if (tt >= nt) return;
    float x[J];
    {
        const float* src = row_src(tt, slot);
#pragma unroll
        for (int j = 0; j < J; j++) x[j] = src[lane + 64 * j];
    }
    for (;;) {  // uniform per wave
        unsigned tn = tt, sn = slot + kWG / 64;  // the wave's next slot
        while (sn >= S) {  // uniform
            sn -= S;
            tn++;
        }
        const bool more = tn < nt;
        float xn[J];
        {  // unconditional (the last slot re-reads its own row), so the waits below count exactly
            const float* src = more ? row_src(tn, sn) : row_src(tt, slot);
#pragma unroll
            for (int j = 0; j < J; j++) xn[j] = src[lane + 64 * j];
        }
        const unsigned t = t0 + tt, pos = p.start + t;
        const bool is_q = slot < p.num_q_heads;
        const unsigned r = slot - p.num_q_heads;
        const bool is_k = !is_q && r < p.num_kv_heads;
        const bool rope = is_q || is_k;  // v: weightless norm only
        const unsigned h = is_q ? slot : (is_k ? r : r - p.num_kv_heads);
        uint32_t wb[J];
#pragma unroll
        for (int j = 0; j < J; j++) wb[j] = is_q ? wq[j] : wk[j];  // v: not used (weightless)
        RopeLane<PJ> rl;
#pragma unroll
        for (int pp = 0; pp < PJ; pp++) {
            rl.c[pp] = rc[tt][lane + 64 * pp];
            rl.s[pp] = rs[tt][lane + 64 * pp];
        }
        wave_norm_rope<J>(x, wb, rope, rope, rl, p.eps);
        uint16_t* dst = is_q ? q_out + ((uint64_t)t * p.num_q_heads + h) * HD
                             : (is_k ? k_cache : v_cache) + ((uint64_t)pos * p.num_kv_heads + h) * HD;
#pragma unroll
        for (int j = 0; j < J; j++) dst[lane + 64 * j] = f2h(x[j]);
        if (vt_cache && !rope) {  // uniform: the V row into its V^T block too
            uint16_t* vt = vt_cache + ((uint64_t)h * vt_blocks + pos / 32) * (HD * 32) + pos % 32;
#pragma unroll
            for (int j = 0; j < J; j++) vt[(lane + 64 * j) * 32] = f2h(x[j]);
        }
        if (!more) break;
        tt = tn;
        slot = sn;
#pragma unroll
        for (int j = 0; j < J; j++) x[j] = xn[j];
    }
}

template <int HD>
__global__ __launch_bounds__(kWG) void k_prompt_prep(const float* __restrict__ q, const float* __restrict__ k,
                                                     const float* __restrict__ v,
                                                     const uint16_t* __restrict__ q_weight,
                                                     const uint16_t* __restrict__ k_weight,
                                                     const uint16_t* __restrict__ rope_freqs,
                                                     const float* __restrict__ inv_table,
                                                     uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache,
                                                     uint16_t* __restrict__ v_cache, uint16_t* __restrict__ vt_cache,
                                                     g4_prompt_prep_params p) {
    prompt_prep_body<HD>(q, k, v, q_weight, k_weight, rope_freqs, inv_table, q_out, k_cache, v_cache, vt_cache, p,
                         blockIdx.x);
}

// Several chunks' preps in one launch (layers or sequences of one head_dim): entry i takes workgroups
// [first[i], first[i + 1]) of the grid, each a multiple of the XCD count (so a workgroup's XCD is the one
// its index within the entry names). The entries come by value in the kernel arguments.
struct PromptPrepMany {
    g4_prompt_prep_entry e[kPromptPrepMany];
    uint32_t first[kPromptPrepMany + 1];
    uint32_t n;
};

template <int HD>
__global__ __launch_bounds__(kWG) void k_prompt_prep_many(const PromptPrepMany m) {
    const unsigned g = blockIdx.x;
    unsigned i = 0;
    while (i + 1 < m.n && g >= m.first[i + 1]) i++;  // uniform
    const g4_prompt_prep_entry& e = m.e[i];
    prompt_prep_body<HD>(e.q, e.k, e.v, e.q_weight, e.k_weight, e.rope_freqs, e.rope_inv_freq, e.q_out, e.k_cache,
                         e.v_cache, e.vt_cache, e.p, g - m.first[i]);
}

}  // namespace g4

using namespace g4;

extern "C" int g4_attn_prep_many(const g4_prep_layer* layers, uint32_t n_layers, uint32_t num_q_heads,
                                 uint32_t num_kv_heads, float eps, uint32_t position, uint32_t slot,
                                 void* stream) {
    if (!layers) return fail(G4_EINVAL, "attnPrepMany: NULL layer table");
    if (n_layers == 0) return G4_OK;
    if (n_layers > 65535) return fail(G4_EINVAL, "attnPrepMany: %u layers (max 65535)", n_layers);
    const unsigned blocks = num_q_heads + 2 * num_kv_heads;
    if (blocks == 0) return G4_OK;
    G4_LAUNCH(k_attn_prep_many, dim3(blocks, n_layers), dim3(kWG), 0, as_stream(stream), layers,
                       num_q_heads, num_kv_heads, eps, position, slot);
    G4_CHECK_LAUNCH("attnPrepMany");
    return G4_OK;
}

extern "C" int g4_attn_prep(float* q, float* k, float* v, const uint16_t* q_weight, const uint16_t* k_weight,
                            const uint16_t* rope_freqs, uint16_t* k_cache, uint16_t* v_cache, g4_prep_params p,
                            void* stream) {
    if (!q || !q_weight) return fail(G4_EINVAL, "attnPrep: NULL q/q_weight");
    if (p.head_dim == 0 || p.head_dim % 2) return fail(G4_EINVAL, "attnPrep: head_dim %u", p.head_dim);
    if (p.apply_divisor && !rope_freqs) return fail(G4_EINVAL, "attnPrep: apply_divisor needs rope_freqs");
    unsigned blocks = p.num_q_heads;
    if (p.store_kv) {
        if (!k || !v || !k_weight || !k_cache || !v_cache) return fail(G4_EINVAL, "attnPrep: store_kv with NULL k/v");
        if (p.slot >= p.max_seq_len) return fail(G4_EINVAL, "attnPrep: slot %u >= max_seq_len %u", p.slot, p.max_seq_len);
        blocks += 2 * p.num_kv_heads;
    }
    if (blocks == 0) return G4_OK;
    G4_LAUNCH(k_attn_prep, dim3(blocks), dim3(kWG), 0, as_stream(stream), q, k, v, q_weight, k_weight,
                       rope_freqs, k_cache, v_cache, p);
    G4_CHECK_LAUNCH("attnPrep");
    return G4_OK;
}

// Checks one chunk's prep and gives its workgroup count (0: nothing to do).
static int prompt_prep_check(const float* q, const float* k, const float* v, const uint16_t* q_weight,
                             const uint16_t* k_weight, const uint16_t* rope_freqs, const float* rope_inv_freq,
                             uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache, uint16_t* vt_cache,
                             const g4_prompt_prep_params& p, uint32_t* wgs_out) {
    *wgs_out = 0;
    if (p.head_dim != 256 && p.head_dim != 512)
        return fail(G4_EINVAL, "attnPromptPrep: head_dim %u unsupported (256 or 512)", p.head_dim);
    if (p.num_q_heads == 0 || p.num_kv_heads == 0) return fail(G4_EINVAL, "attnPromptPrep: no heads");
    if (!q || !q_weight || !q_out) return fail(G4_EINVAL, "attnPromptPrep: NULL q/q_weight/q_out");
    if (p.apply_divisor && !rope_freqs && !rope_inv_freq)
        return fail(G4_EINVAL, "attnPromptPrep: apply_divisor needs rope_freqs");
    if (p.store_kv) {
        if (!k || !v || !k_weight || !k_cache || !v_cache)
            return fail(G4_EINVAL, "attnPromptPrep: store_kv with NULL k/v/k_weight/caches");
        if ((uint64_t)p.start + p.n_tokens > p.max_seq_len)
            return fail(G4_EINVAL, "attnPromptPrep: rows %u..%u past max_seq_len %u", p.start,
                        p.start + p.n_tokens - 1, p.max_seq_len);
    }
    if (vt_cache && !p.store_kv) return fail(G4_EINVAL, "attnPromptPrep: vt_cache needs store_kv (a KV producer)");
    if ((uint64_t)p.start + p.n_tokens + 31 > 0xffffffffull) return fail(G4_EINVAL, "attnPromptPrep: position range");
    (void)rope_inv_freq;
    if (p.n_tokens == 0) return G4_OK;
    const uint64_t blocks = ((uint64_t)p.start + p.n_tokens - (p.start & ~31u) + 31) / 32;
    const uint64_t wgs = (blocks + kXcds - 1) / kXcds * kXcds * kPrepPerBlock;
    if (wgs > 0x7fffffffu) return fail(G4_EINVAL, "attnPromptPrep: too many tokens");
    *wgs_out = (uint32_t)wgs;
    return G4_OK;
}

static int prompt_prep(const float* q, const float* k, const float* v, const uint16_t* q_weight, const uint16_t* k_weight,
                       const uint16_t* rope_freqs, const float* rope_inv_freq, uint16_t* q_out, uint16_t* k_cache,
                       uint16_t* v_cache, uint16_t* vt_cache, const g4_prompt_prep_params& p, void* stream) {
    uint32_t wgs = 0;
    const int rc = prompt_prep_check(q, k, v, q_weight, k_weight, rope_freqs, rope_inv_freq, q_out, k_cache, v_cache,
                                     vt_cache, p, &wgs);
    if (rc || !wgs) return rc;
    hipStream_t st = as_stream(stream);
    const dim3 grid(wgs);
    if (p.head_dim == 512)
        G4_LAUNCH(k_prompt_prep<512>, grid, dim3(kWG), 0, st, q, k, v, q_weight, k_weight, rope_freqs,
                           rope_inv_freq, q_out, k_cache, v_cache, vt_cache, p);
    else
        G4_LAUNCH(k_prompt_prep<256>, grid, dim3(kWG), 0, st, q, k, v, q_weight, k_weight, rope_freqs,
                           rope_inv_freq, q_out, k_cache, v_cache, vt_cache, p);
    G4_CHECK_LAUNCH("attnPromptPrep");
    return G4_OK;
}

extern "C" int g4_attn_prompt_prep_many(const g4_prompt_prep_entry* entries, uint32_t n_entries, void* stream) {
    if (!entries || n_entries == 0) return fail(G4_EINVAL, "attnPromptPrepMany: no entries");
    if (n_entries > kPromptPrepMany)
        return fail(G4_EINVAL, "attnPromptPrepMany: %u entries (max %u)", n_entries, kPromptPrepMany);
    PromptPrepMany m = {};
    uint64_t total = 0;
    for (uint32_t i = 0; i < n_entries; i++) {
        const g4_prompt_prep_entry& e = entries[i];
        if (e.p.head_dim != entries[0].p.head_dim)
            return fail(G4_EINVAL, "attnPromptPrepMany: entry %u has head_dim %u, entry 0 %u", i, e.p.head_dim,
                        entries[0].p.head_dim);
        uint32_t wgs = 0;
        const int rc = prompt_prep_check(e.q, e.k, e.v, e.q_weight, e.k_weight, e.rope_freqs, e.rope_inv_freq,
                                         e.q_out, e.k_cache, e.v_cache, e.vt_cache, e.p, &wgs);
        if (rc) return rc;
        m.e[i] = e;
        m.first[i] = (uint32_t)total;
        total += wgs;  // a multiple of kXcds
    }
    if (total == 0) return G4_OK;
    if (total > 0x7fffffffu) return fail(G4_EINVAL, "attnPromptPrepMany: too many tokens");
    m.first[n_entries] = (uint32_t)total;
    m.n = n_entries;
    hipStream_t st = as_stream(stream);
    if (entries[0].p.head_dim == 512)
        G4_LAUNCH(k_prompt_prep_many<512>, dim3((uint32_t)total), dim3(kWG), 0, st, m);
    else
        G4_LAUNCH(k_prompt_prep_many<256>, dim3((uint32_t)total), dim3(kWG), 0, st, m);
    G4_CHECK_LAUNCH("attnPromptPrepMany");
    return G4_OK;
}

extern "C" int g4_attn_prompt_prep(const float* q, const float* k, const float* v, const uint16_t* q_weight,
                                   const uint16_t* k_weight, const uint16_t* rope_freqs, const float* rope_inv_freq,
                                   uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache, g4_prompt_prep_params p,
                                   void* stream) {
    return prompt_prep(q, k, v, q_weight, k_weight, rope_freqs, rope_inv_freq, q_out, k_cache, v_cache, nullptr, p,
                       stream);
}

extern "C" int g4_attn_prompt_prep_vt(const float* q, const float* k, const float* v, const uint16_t* q_weight,
                                      const uint16_t* k_weight, const uint16_t* rope_freqs, const float* rope_inv_freq,
                                      uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache, uint16_t* vt_cache,
                                      g4_prompt_prep_params p, void* stream) {
    if (!vt_cache) return fail(G4_EINVAL, "attnPromptPrepVt: vt_cache is NULL");
    return prompt_prep(q, k, v, q_weight, k_weight, rope_freqs, rope_inv_freq, q_out, k_cache, v_cache, vt_cache, p,
                       stream);
}

namespace g4 {

// RoPE inverse frequencies of one (theta, divisor) configuration: the
// position-independent factor of every angle (fused_per_head_norm_rope.wgsl:
// 50-54), evaluated exactly as the reference kernels do.
__global__ __launch_bounds__(kWG) void k_rope_inv_freq(float theta, unsigned head_dim, unsigned apply_divisor,
                                                       const uint16_t* __restrict__ rope_freqs,
                                                       float* __restrict__ inv_freq) {
    const unsigned i = blockIdx.x * kWG + threadIdx.x;
    if (i >= head_dim / 2) return;
    inv_freq[i] = rope_inv_freq(i, head_dim, theta, apply_divisor, apply_divisor ? h2f(rope_freqs[i]) : 1.0f);
}

}  // namespace g4

extern "C" int g4_rope_inv_freq(float theta, uint32_t head_dim, uint32_t apply_divisor, const uint16_t* rope_freqs,
                                float* inv_freq, void* stream) {
    if (!inv_freq) return fail(G4_EINVAL, "ropeInvFreq: NULL output");
    if (head_dim == 0 || head_dim % 2) return fail(G4_EINVAL, "ropeInvFreq: head_dim %u", head_dim);
    if (apply_divisor && !rope_freqs) return fail(G4_EINVAL, "ropeInvFreq: apply_divisor needs rope_freqs");
    const unsigned half = head_dim / 2;
    G4_LAUNCH(k_rope_inv_freq, dim3((half + kWG - 1) / kWG), dim3(kWG), 0, as_stream(stream), theta,
                       head_dim, apply_divisor, rope_freqs, inv_freq);
    G4_CHECK_LAUNCH("ropeInvFreq");
    return G4_OK;
}

// The same table on the host (one configuration, computed once at load): the
// same f32 expression with the host's pow, whose f64 result rounded to f32
// equals the device's.
extern "C" int g4_rope_inv_freq_host(float theta, uint32_t head_dim, uint32_t apply_divisor,
                                     const uint16_t* rope_freqs_host, float* inv_freq_host) {
    if (!inv_freq_host) return fail(G4_EINVAL, "ropeInvFreqHost: NULL output");
    if (head_dim == 0 || head_dim % 2) return fail(G4_EINVAL, "ropeInvFreqHost: head_dim %u", head_dim);
    if (apply_divisor && !rope_freqs_host) return fail(G4_EINVAL, "ropeInvFreqHost: apply_divisor needs rope_freqs");
    for (uint32_t i = 0; i < head_dim / 2; i++) {
        const float e = (float)(i * 2u) / (float)head_dim;
        const float base_freq = 1.0f / (float)pow((double)theta, (double)e);
        inv_freq_host[i] =
            apply_divisor ? base_freq / (float)__builtin_bit_cast(_Float16, rope_freqs_host[i]) : base_freq;
    }
    return G4_OK;
}
