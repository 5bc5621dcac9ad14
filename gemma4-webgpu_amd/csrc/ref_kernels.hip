// The six gemma4-webgpu attention kernels, one HIP kernel each, with the
// reference's semantics, dispatch grids and reduction order:
//
//   fusedPerHeadNormRope    shaders/fused_per_head_norm_rope.wgsl:20-64
//   perHeadRmsNormNoWeight  shaders/per_head_rms_norm_no_weight.wgsl:13-38
//   kvCacheStore            shaders/kv_cache_store.wgsl:8-18     (f16 cache)
//   attnScore               shaders/attn_score.wgsl:15-40        (f16 cache)
//   softmax                 shaders/softmax.wgsl:7-46
//   attnOutput              shaders/attn_output.wgsl:7-23        (f16 cache)
//
// They are the per-kernel drop-in surface (the engine's capture points
// postRopeQ/K and attnOut sit between them, src/engine.ts:2086-2095) and the
// unfused comparison path for the fused kernels. Arithmetic: every f32
// operation rounds separately (no FMA contraction), sqrt and division are
// IEEE correctly rounded, and pow/sin/cos/exp return the f32 nearest to the
// exact value (evaluated in f64), so results are reproducible bit for bit on
// any IEEE machine that evaluates the same expressions.
#include "ref_math.h"

namespace g4 {

__global__ __launch_bounds__(kWG) void k_fused_per_head_norm_rope(float* __restrict__ data,
                                                                  const uint16_t* __restrict__ weight,
                                                                  const uint16_t* __restrict__ rope_freqs,
                                                                  g4_norm_rope_params p) {
    __shared__ float scratch[kNormScratch];
    const unsigned head = blockIdx.x;
    if (head >= p.num_heads) return;
    head_norm_rope(data + head * p.head_dim, weight, true, rope_freqs, p.head_dim, p.eps, p.position, p.theta,
                   p.apply_divisor, scratch);
}

__global__ __launch_bounds__(kWG) void k_per_head_rms_norm_no_weight(float* __restrict__ data, g4_norm_params p) {
    __shared__ float scratch[kNormScratch];
    const unsigned head = blockIdx.x;
    if (head >= p.num_heads) return;
    head_norm_rope(data + head * p.head_dim, nullptr, false, nullptr, p.head_dim, p.eps, 0, 0.0f, 0, scratch);
}

__global__ __launch_bounds__(kWG) void k_kv_cache_store(const float* __restrict__ k_in, const float* __restrict__ v_in,
                                                        uint16_t* __restrict__ k_cache,
                                                        uint16_t* __restrict__ v_cache, g4_kv_store_params p) {
    const unsigned i = blockIdx.x * kWG + threadIdx.x;
    const unsigned total = p.num_kv_heads * p.head_dim;
    if (i >= total) return;
    const unsigned head = i / p.head_dim;
    const unsigned d = i % p.head_dim;
    const uint64_t cache_idx = (uint64_t)p.position * total + head * p.head_dim + d;
    k_cache[cache_idx] = f2h(k_in[i]);
    v_cache[cache_idx] = f2h(v_in[i]);
}

__global__ __launch_bounds__(kWG) void k_attn_score(const float* __restrict__ q, const uint16_t* __restrict__ k_cache,
                                                    float* __restrict__ scores, g4_attn_score_params p) {
    const uint64_t idx = (uint64_t)blockIdx.x * kWG + threadIdx.x;
    const uint64_t total = (uint64_t)p.num_q_heads * p.seq_len;
    if (idx >= total) return;
    const unsigned head = (unsigned)(idx / p.seq_len);
    const unsigned pos = (unsigned)(idx % p.seq_len);
    const uint64_t score_idx = (uint64_t)head * p.seq_len + pos;
    if (p.sliding_window != 0u) {
        const unsigned current_pos = p.seq_len - 1u;
        const unsigned window_start =
            (current_pos + 1u > p.sliding_window) ? current_pos + 1u - p.sliding_window : 0u;
        if (pos < window_start) {
            scores[score_idx] = -1e30f;
            return;
        }
    }
    const unsigned kv_head = head * p.num_kv_heads / p.num_q_heads;
    const unsigned q_offset = head * p.head_dim;
    const unsigned kv_stride = p.num_kv_heads * p.head_dim;
    const uint64_t k_offset = (uint64_t)pos * kv_stride + kv_head * p.head_dim;
    float dot = 0.0f;
    for (unsigned d = 0; d < p.head_dim; d++) dot = dot + q[q_offset + d] * h2f(k_cache[k_offset + d]);
    scores[score_idx] = dot * p.scale;
}

__global__ __launch_bounds__(kWG) void k_softmax(float* __restrict__ scores, g4_softmax_params p) {
    __shared__ float shared_max[kWG];
    __shared__ float shared_sum[kWG];
    const unsigned tid = threadIdx.x;
    const unsigned head = blockIdx.x;
    if (head >= p.num_heads) return;
    const uint64_t base = (uint64_t)head * p.seq_len;
    float local_max = -1e30f;
    for (unsigned i = tid; i < p.seq_len; i += kWG) local_max = wgsl_max(local_max, scores[base + i]);
    shared_max[tid] = local_max;
    __syncthreads();
    const float max_val = wg_tree_max(shared_max, tid);
    float local_sum = 0.0f;
    for (unsigned i = tid; i < p.seq_len; i += kWG) {
        float e = (float)exp((double)(scores[base + i] - max_val));
        scores[base + i] = e;
        local_sum = local_sum + e;
    }
    shared_sum[tid] = local_sum;
    __syncthreads();
    const float sum_val = wg_tree_sum(shared_sum, tid);
    for (unsigned i = tid; i < p.seq_len; i += kWG) scores[base + i] = scores[base + i] / sum_val;
}

__global__ __launch_bounds__(kWG) void k_attn_output(const float* __restrict__ probs,
                                                     const uint16_t* __restrict__ v_cache, float* __restrict__ out,
                                                     g4_attn_output_params p) {
    const unsigned idx = blockIdx.x * kWG + threadIdx.x;
    const unsigned total = p.num_q_heads * p.head_dim;
    if (idx >= total) return;
    const unsigned head = idx / p.head_dim;
    const unsigned d = idx % p.head_dim;
    const unsigned kv_head = head * p.num_kv_heads / p.num_q_heads;
    const unsigned kv_stride = p.num_kv_heads * p.head_dim;
    float sum = 0.0f;
    for (unsigned pos = 0; pos < p.seq_len; pos++) {
        float prob = probs[(uint64_t)head * p.seq_len + pos];
        const uint64_t v_idx = (uint64_t)pos * kv_stride + kv_head * p.head_dim + d;
        sum = sum + prob * h2f(v_cache[v_idx]);
    }
    out[(uint64_t)head * p.head_dim + d] = sum;
}

__global__ __launch_bounds__(kWG) void k_zero(uint32_t* __restrict__ dst, uint64_t words, uint8_t* tail,
                                              unsigned tail_bytes) {
    const uint64_t stride = (uint64_t)gridDim.x * kWG;
    for (uint64_t i = (uint64_t)blockIdx.x * kWG + threadIdx.x; i < words; i += stride) dst[i] = 0u;
    if (blockIdx.x == 0 && threadIdx.x < tail_bytes) tail[threadIdx.x] = 0;
}

}  // namespace g4

using namespace g4;

static inline unsigned ceil_div_u(uint64_t a, uint64_t b) { return (unsigned)((a + b - 1) / b); }

extern "C" {

int g4_fused_per_head_norm_rope(float* data, const uint16_t* weight, const uint16_t* rope_freqs,
                                g4_norm_rope_params p, void* stream) {
    if (!data || !weight) return fail(G4_EINVAL, "fusedPerHeadNormRope: NULL data/weight");
    if (p.apply_divisor && !rope_freqs) return fail(G4_EINVAL, "fusedPerHeadNormRope: apply_divisor needs rope_freqs");
    if (p.head_dim == 0 || p.head_dim % 2) return fail(G4_EINVAL, "fusedPerHeadNormRope: head_dim %u", p.head_dim);
    if (p.num_heads == 0) return G4_OK;
    G4_LAUNCH(k_fused_per_head_norm_rope, dim3(p.num_heads), dim3(kWG), 0, as_stream(stream), data, weight,
                       rope_freqs, p);
    G4_CHECK_LAUNCH("fusedPerHeadNormRope");
    return G4_OK;
}

int g4_per_head_rms_norm_no_weight(float* data, g4_norm_params p, void* stream) {
    if (!data) return fail(G4_EINVAL, "perHeadRmsNormNoWeight: NULL data");
    if (p.head_dim == 0) return fail(G4_EINVAL, "perHeadRmsNormNoWeight: head_dim 0");
    if (p.num_heads == 0) return G4_OK;
    G4_LAUNCH(k_per_head_rms_norm_no_weight, dim3(p.num_heads), dim3(kWG), 0, as_stream(stream), data, p);
    G4_CHECK_LAUNCH("perHeadRmsNormNoWeight");
    return G4_OK;
}

int g4_kv_cache_store(const float* k_in, const float* v_in, uint16_t* k_cache, uint16_t* v_cache,
                      g4_kv_store_params p, void* stream) {
    if (!k_in || !v_in || !k_cache || !v_cache) return fail(G4_EINVAL, "kvCacheStore: NULL pointer");
    if (p.position >= p.max_seq_len)
        return fail(G4_EINVAL, "kvCacheStore: slot %u >= max_seq_len %u", p.position, p.max_seq_len);
    const uint64_t total = (uint64_t)p.num_kv_heads * p.head_dim;
    if (total == 0) return G4_OK;
    G4_LAUNCH(k_kv_cache_store, dim3(ceil_div_u(total, kWG)), dim3(kWG), 0, as_stream(stream), k_in, v_in,
                       k_cache, v_cache, p);
    G4_CHECK_LAUNCH("kvCacheStore");
    return G4_OK;
}

int g4_attn_score(const float* q, const uint16_t* k_cache, float* scores, g4_attn_score_params p, void* stream) {
    if (!q || !k_cache || !scores) return fail(G4_EINVAL, "attnScore: NULL pointer");
    if (p.seq_len == 0) return fail(G4_EINVAL, "attnScore: seq_len 0");
    if (p.num_kv_heads == 0 || p.num_q_heads % p.num_kv_heads)
        return fail(G4_EINVAL, "attnScore: num_q_heads %u not a multiple of num_kv_heads %u", p.num_q_heads,
                    p.num_kv_heads);
    const uint64_t total = (uint64_t)p.num_q_heads * p.seq_len;
    if (total == 0) return G4_OK;
    G4_LAUNCH(k_attn_score, dim3(ceil_div_u(total, kWG)), dim3(kWG), 0, as_stream(stream), q, k_cache,
                       scores, p);
    G4_CHECK_LAUNCH("attnScore");
    return G4_OK;
}

int g4_softmax(float* scores, g4_softmax_params p, void* stream) {
    if (!scores) return fail(G4_EINVAL, "softmax: NULL scores");
    if (p.seq_len == 0) return fail(G4_EINVAL, "softmax: seq_len 0");
    if (p.num_heads == 0) return G4_OK;
    G4_LAUNCH(k_softmax, dim3(p.num_heads), dim3(kWG), 0, as_stream(stream), scores, p);
    G4_CHECK_LAUNCH("softmax");
    return G4_OK;
}

int g4_attn_output(const float* probs, const uint16_t* v_cache, float* out, g4_attn_output_params p, void* stream) {
    if (!probs || !v_cache || !out) return fail(G4_EINVAL, "attnOutput: NULL pointer");
    if (p.num_kv_heads == 0 || p.num_q_heads % p.num_kv_heads)
        return fail(G4_EINVAL, "attnOutput: num_q_heads %u not a multiple of num_kv_heads %u", p.num_q_heads,
                    p.num_kv_heads);
    const uint64_t total = (uint64_t)p.num_q_heads * p.head_dim;
    if (total == 0) return G4_OK;
    G4_LAUNCH(k_attn_output, dim3(ceil_div_u(total, kWG)), dim3(kWG), 0, as_stream(stream), probs, v_cache,
                       out, p);
    G4_CHECK_LAUNCH("attnOutput");
    return G4_OK;
}

int g4_zero(void* dev_dst, size_t bytes, void* stream) {
    if (!dev_dst) return fail(G4_EINVAL, "g4_zero: NULL pointer");
    if (bytes == 0) return G4_OK;
    if (reinterpret_cast<uintptr_t>(dev_dst) % 4) return fail(G4_EINVAL, "g4_zero: pointer not 4-byte aligned");
    const uint64_t words = bytes / 4;
    const unsigned tail = (unsigned)(bytes % 4);
    unsigned blocks = words ? ceil_div_u(words, kWG) : 1;
    if (blocks > 4096) blocks = 4096;
    G4_LAUNCH(k_zero, dim3(blocks), dim3(kWG), 0, as_stream(stream), static_cast<uint32_t*>(dev_dst), words,
                       static_cast<uint8_t*>(dev_dst) + words * 4, tail);
    G4_CHECK_LAUNCH("g4_zero");
    return G4_OK;
}

}  // extern "C"
