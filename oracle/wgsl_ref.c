/*
 * oracle/wgsl_ref.c — TEST INFRASTRUCTURE ONLY.
 *
 * A CPU restatement of gemma4-webgpu's six attention WGSL kernels, used by the
 * test-suite and by bench.py's CPU-baseline leg as the checker. Nothing in the
 * product library links or calls this file.
 *
 * Each function restates one WGSL compute shader of the reference, dispatch
 * for dispatch: the same workgroup grid, the same 256-invocation strided loops,
 * the same 128->1 workgroup-memory reduction trees, the same -1e30 sentinels,
 * the same buffer layouts (slot-major [slot][kv_head][head_dim] caches, scores
 * with a head stride equal to the current seq_len). Workgroups run in parallel
 * with OpenMP; invocations inside a workgroup are simulated phase by phase
 * between the shader's workgroupBarrier() calls.
 *
 * Arithmetic conventions (the WGSL spec leaves some of them to the
 * implementation; the choices here are fixed and stated):
 *   - f32 everywhere the shader uses f32; every + - * / rounds to f32
 *     (built with -ffp-contract=off: no fused multiply-add).
 *   - sqrt: IEEE-754 correctly rounded (sqrtf).
 *   - pow, sin, cos, exp: the f32 value closest to the exact result, computed
 *     as (float)f((double)x). The reference's WebGPU implementation may differ
 *     from these in the last ulp ("parity unpinned" against a specific browser).
 *   - f16 -> f32 widening is exact; f32 -> f16 uses round-to-nearest-even
 *     with overflow to +-Inf (the build's cache format; the WGSL caches are f32).
 *
 * Reference files restated (paths relative to the gemma4-webgpu repository):
 *   shaders/fused_per_head_norm_rope.wgsl:20-64
 *   shaders/per_head_rms_norm_no_weight.wgsl:13-38
 *   shaders/kv_cache_store.wgsl:8-18
 *   shaders/attn_score.wgsl:15-40
 *   shaders/softmax.wgsl:7-46
 *   shaders/attn_output.wgsl:7-23
 *   lm head and sampling: shaders/matmul_quant.wgsl:20-52 (f16 weights),
 *     shaders/logit_softcap.wgsl:9-16, shaders/argmax.wgsl:7-34
 *   dispatch grids: src/engine.ts:2060-2094
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define WG 256u /* @workgroup_size(256) in every reference shader */

/* ---- f16 <-> f32 ------------------------------------------------------- */

float wr_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: renormalise */
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400u) == 0);
            man &= 0x3ffu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t wr_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    }
    if (ax >= 0x477ff000u) { /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax < 0x38800000u) { /* below f16 min normal: subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to 0 */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e; /* 14..24 */
        uint32_t r = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ax + 0xc8000fffu + ((ax >> 13) & 1u); /* rebias and RNE */
    return (uint16_t)(sign | (r >> 13));
}

void wr_f32_to_f16_array(const float* src, uint16_t* dst, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) dst[i] = wr_f32_to_f16(src[i]);
}

void wr_f16_to_f32_array(const uint16_t* src, float* dst, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) dst[i] = wr_f16_to_f32(src[i]);
}

/* WGSL builtins at correctly rounded f32 accuracy. */
static float wgsl_pow(float a, float b) { return (float)pow((double)a, (double)b); }
static float wgsl_sin(float a) { return (float)sin((double)a); }
static float wgsl_cos(float a) { return (float)cos((double)a); }
static float wgsl_exp(float a) { return (float)exp((double)a); }
static float wgsl_max(float a, float b) { return a > b ? a : (b > a ? b : a); }

/* 128 -> 1 workgroup-memory tree, exactly as the shaders' stride loop. */
static float tree_sum(float* s) {
    for (uint32_t stride = 128u; stride > 0u; stride >>= 1u)
        for (uint32_t t = 0; t < stride; t++) s[t] = s[t] + s[t + stride];
    return s[0];
}

static float tree_max(float* s) {
    for (uint32_t stride = 128u; stride > 0u; stride >>= 1u)
        for (uint32_t t = 0; t < stride; t++) s[t] = wgsl_max(s[t], s[t + stride]);
    return s[0];
}

/* ---- Params: the reference uniform layouts (src/engine.ts:526-595) ------ */

typedef struct { uint32_t num_heads, head_dim; float eps; uint32_t position; float theta; uint32_t apply_divisor; } wr_norm_rope_params;
typedef struct { uint32_t num_heads, head_dim; float eps; uint32_t pad; } wr_norm_params;
typedef struct { uint32_t num_kv_heads, head_dim, position, max_seq_len; } wr_kv_store_params;
typedef struct { uint32_t num_q_heads, num_kv_heads, head_dim, seq_len; float scale; uint32_t sliding_window; } wr_attn_score_params;
typedef struct { uint32_t num_heads, seq_len; } wr_softmax_params;
typedef struct { uint32_t num_q_heads, num_kv_heads, head_dim, seq_len; } wr_attn_output_params;

/* ---- shaders/fused_per_head_norm_rope.wgsl:20-64 ----------------------- *
 * Dispatched with num_workgroups = num_heads (engine.ts:2078-2085).        */
/* fused_per_head_norm_rope.wgsl:50-54: the position-independent factor of
 * the angle of pair i. */
static float rope_freq(uint32_t i, uint32_t head_dim, float theta, uint32_t apply_divisor,
                       const uint16_t* rope_freqs) {
    float base_freq = 1.0f / wgsl_pow(theta, (float)(i * 2u) / (float)head_dim);
    float freq = base_freq;
    if (apply_divisor != 0u) freq = base_freq / wr_f16_to_f32(rope_freqs[i]);
    return freq;
}

/* The table of rope_freq over i < head_dim/2 (what g4_rope_inv_freq computes). */
void wr_rope_inv_freq(float theta, uint32_t head_dim, uint32_t apply_divisor, const uint16_t* rope_freqs,
                      float* out) {
    for (uint32_t i = 0; i < head_dim / 2u; i++) out[i] = rope_freq(i, head_dim, theta, apply_divisor, rope_freqs);
}

void wr_fused_per_head_norm_rope(float* data, const uint16_t* weight, const wr_norm_rope_params* p,
                                 const uint16_t* rope_freqs, uint32_t num_workgroups) {
#pragma omp parallel for schedule(static)
    for (int64_t w = 0; w < (int64_t)num_workgroups; w++) {
        uint32_t head = (uint32_t)w;
        if (head >= p->num_heads) continue;
        uint32_t base = head * p->head_dim;
        float shared_sum[WG];
        for (uint32_t tid = 0; tid < WG; tid++) {
            float partial = 0.0f;
            for (uint32_t i = tid; i < p->head_dim; i += WG) {
                float val = data[base + i];
                partial = partial + val * val;
            }
            shared_sum[tid] = partial;
        }
        float rms = sqrtf(tree_sum(shared_sum) / (float)p->head_dim + p->eps);
        for (uint32_t tid = 0; tid < WG; tid++)
            for (uint32_t i = tid; i < p->head_dim; i += WG)
                data[base + i] = data[base + i] * wr_f16_to_f32(weight[i]) / rms;
        uint32_t half_dim = p->head_dim / 2u;
        for (uint32_t tid = 0; tid < WG; tid++) {
            for (uint32_t i = tid; i < half_dim; i += WG) {
                float freq = rope_freq(i, p->head_dim, p->theta, p->apply_divisor, rope_freqs);
                float angle = (float)p->position * freq;
                float cos_a = wgsl_cos(angle);
                float sin_a = wgsl_sin(angle);
                float x0 = data[base + i];
                float x1 = data[base + i + half_dim];
                data[base + i] = x0 * cos_a - x1 * sin_a;
                data[base + i + half_dim] = x0 * sin_a + x1 * cos_a;
            }
        }
    }
}

/* ---- shaders/per_head_rms_norm_no_weight.wgsl:13-38 --------------------- *
 * Dispatched with num_workgroups = NKH (engine.ts:2060-2066).               */
void wr_per_head_rms_norm_no_weight(float* data, const wr_norm_params* p, uint32_t num_workgroups) {
#pragma omp parallel for schedule(static)
    for (int64_t w = 0; w < (int64_t)num_workgroups; w++) {
        uint32_t head = (uint32_t)w;
        if (head >= p->num_heads) continue;
        uint32_t base = head * p->head_dim;
        float shared_sum[WG];
        for (uint32_t tid = 0; tid < WG; tid++) {
            float partial = 0.0f;
            for (uint32_t i = tid; i < p->head_dim; i += WG) {
                float val = data[base + i];
                partial = partial + val * val;
            }
            shared_sum[tid] = partial;
        }
        float rms = sqrtf(tree_sum(shared_sum) / (float)p->head_dim + p->eps);
        for (uint32_t tid = 0; tid < WG; tid++)
            for (uint32_t i = tid; i < p->head_dim; i += WG) data[base + i] = data[base + i] / rms;
    }
}

/* ---- shaders/kv_cache_store.wgsl:8-18 (f32 caches, as the WGSL binds) ---- *
 * Dispatched with ceil(NKH*HD/256) workgroups (engine.ts:2089-2091).         */
void wr_kv_cache_store(const float* k_in, const float* v_in, float* k_cache, float* v_cache,
                       const wr_kv_store_params* p, uint32_t num_workgroups) {
    uint32_t total = p->num_kv_heads * p->head_dim;
    for (uint64_t i = 0; i < (uint64_t)num_workgroups * WG; i++) {
        if (i >= total) continue;
        uint32_t head = (uint32_t)i / p->head_dim;
        uint32_t d = (uint32_t)i % p->head_dim;
        uint64_t cache_idx = (uint64_t)p->position * total + head * p->head_dim + d;
        k_cache[cache_idx] = k_in[i];
        v_cache[cache_idx] = v_in[i];
    }
}

/* The build's cache format: the same store into f16 caches, RNE. */
void wr_kv_cache_store_f16(const float* k_in, const float* v_in, uint16_t* k_cache, uint16_t* v_cache,
                           const wr_kv_store_params* p) {
    uint32_t total = p->num_kv_heads * p->head_dim;
    for (uint32_t i = 0; i < total; i++) {
        uint32_t head = i / p->head_dim;
        uint32_t d = i % p->head_dim;
        uint64_t cache_idx = (uint64_t)p->position * total + head * p->head_dim + d;
        k_cache[cache_idx] = wr_f32_to_f16(k_in[i]);
        v_cache[cache_idx] = wr_f32_to_f16(v_in[i]);
    }
}

/* ---- shaders/attn_score.wgsl:15-40 --------------------------------------- *
 * Dispatched with ceil(NQH*seq_len/256) workgroups (engine.ts:2092).          */
void wr_attn_score(const float* q, const float* k_cache, float* scores, const wr_attn_score_params* p,
                   uint32_t num_workgroups) {
    uint64_t total = (uint64_t)p->num_q_heads * p->seq_len;
    uint64_t n_inv = (uint64_t)num_workgroups * WG;
#pragma omp parallel for schedule(static)
    for (int64_t idx_s = 0; idx_s < (int64_t)n_inv; idx_s++) {
        uint64_t idx = (uint64_t)idx_s;
        if (idx >= total) continue;
        uint32_t head = (uint32_t)(idx / p->seq_len);
        uint32_t pos = (uint32_t)(idx % p->seq_len);
        uint64_t score_idx = (uint64_t)head * p->seq_len + pos;
        if (p->sliding_window != 0u) {
            uint32_t current_pos = p->seq_len - 1u;
            uint32_t window_start = (current_pos + 1u > p->sliding_window) ? current_pos + 1u - p->sliding_window : 0u;
            if (pos < window_start) {
                scores[score_idx] = -1e30f;
                continue;
            }
        }
        uint32_t kv_head = head * p->num_kv_heads / p->num_q_heads;
        uint32_t q_offset = head * p->head_dim;
        uint32_t kv_stride = p->num_kv_heads * p->head_dim;
        uint64_t k_offset = (uint64_t)pos * kv_stride + kv_head * p->head_dim;
        float dot = 0.0f;
        for (uint32_t d = 0; d < p->head_dim; d++) dot = dot + q[q_offset + d] * k_cache[k_offset + d];
        scores[score_idx] = dot * p->scale;
    }
}

/* ---- shaders/softmax.wgsl:7-46 ------------------------------------------- *
 * Dispatched with NQH workgroups (engine.ts:2093).                            */
void wr_softmax(float* scores, const wr_softmax_params* p, uint32_t num_workgroups) {
#pragma omp parallel for schedule(static)
    for (int64_t w = 0; w < (int64_t)num_workgroups; w++) {
        uint32_t head = (uint32_t)w;
        if (head >= p->num_heads) continue;
        uint64_t base = (uint64_t)head * p->seq_len;
        float shared_max[WG], shared_sum[WG];
        for (uint32_t tid = 0; tid < WG; tid++) {
            float local_max = -1e30f;
            for (uint32_t i = tid; i < p->seq_len; i += WG) local_max = wgsl_max(local_max, scores[base + i]);
            shared_max[tid] = local_max;
        }
        float max_val = tree_max(shared_max);
        for (uint32_t tid = 0; tid < WG; tid++) {
            float local_sum = 0.0f;
            for (uint32_t i = tid; i < p->seq_len; i += WG) {
                float e = wgsl_exp(scores[base + i] - max_val);
                scores[base + i] = e;
                local_sum = local_sum + e;
            }
            shared_sum[tid] = local_sum;
        }
        float sum_val = tree_sum(shared_sum);
        for (uint32_t tid = 0; tid < WG; tid++)
            for (uint32_t i = tid; i < p->seq_len; i += WG) scores[base + i] = scores[base + i] / sum_val;
    }
}

/* ---- shaders/attn_output.wgsl:7-23 --------------------------------------- *
 * Dispatched with ceil(NQH*HD/256) workgroups (engine.ts:2094).               */
void wr_attn_output(const float* probs, const float* v_cache, float* output, const wr_attn_output_params* p,
                    uint32_t num_workgroups) {
    uint64_t total = (uint64_t)p->num_q_heads * p->head_dim;
    uint64_t n_inv = (uint64_t)num_workgroups * WG;
#pragma omp parallel for schedule(static)
    for (int64_t idx_s = 0; idx_s < (int64_t)n_inv; idx_s++) {
        uint64_t idx = (uint64_t)idx_s;
        if (idx >= total) continue;
        uint32_t head = (uint32_t)(idx / p->head_dim);
        uint32_t d = (uint32_t)(idx % p->head_dim);
        uint32_t kv_head = head * p->num_kv_heads / p->num_q_heads;
        uint32_t kv_stride = p->num_kv_heads * p->head_dim;
        float sum = 0.0f;
        for (uint32_t pos = 0; pos < p->seq_len; pos++) {
            float prob = probs[(uint64_t)head * p->seq_len + pos];
            uint64_t v_idx = (uint64_t)pos * kv_stride + kv_head * p->head_dim + d;
            sum = sum + prob * v_cache[v_idx];
        }
        output[(uint64_t)head * p->head_dim + d] = sum;
    }
}

/* ---- shaders/matmul_quant.wgsl:20-52 ------------------------------------ *
 * One workgroup per output row m (dispatched by engine.ts dispatchMatmul,
 * a 2D grid above 65535 rows; m = wg.y * ng.x + wg.x covers 0..M-1): the
 * invocation tid sums weight[m, k] * input[k] over k = tid, tid + 256, ...
 * in order (f16 weight widened exactly), then the 128 -> 1 tree.            */
void wr_matmul_quant(const float* input, const uint16_t* weight, float* output, uint32_t M, uint32_t N) {
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < (int64_t)M; m++) {
        float partials[WG];
        const uint16_t* row = weight + (uint64_t)m * N;
        for (uint32_t tid = 0; tid < WG; tid++) {
            float acc = 0.0f;
            for (uint32_t k = tid; k < N; k += WG) acc = acc + wr_f16_to_f32(row[k]) * input[k];
            partials[tid] = acc;
        }
        output[m] = tree_sum(partials);
    }
}

/* ---- shaders/matmul_q8.wgsl:31-64 (and matmul_q8_mr.wgsl:50-79, the same
 * per-row order) -------------------------------------------------------------
 * int8 weights (row-major [M][N], two's complement bytes), one f16 scale per
 * 32-element block of a row ([M][N/32]). Partial t: acc + (q * scale) * x over
 * k = t, t + 256, ..., each operation rounded to f32; then the 128 -> 1 tree. */
void wr_matmul_q8(const float* input, const int8_t* qweight, const uint16_t* qscale, float* output, uint32_t M,
                  uint32_t N) {
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < (int64_t)M; m++) {
        float partials[WG];
        const int8_t* row = qweight + (uint64_t)m * N;
        const uint16_t* sc = qscale + (uint64_t)m * (N / 32);
        for (uint32_t tid = 0; tid < WG; tid++) {
            float acc = 0.0f;
            for (uint32_t k = tid; k < N; k += WG) {
                const float w = (float)row[k] * wr_f16_to_f32(sc[k >> 5]);
                const float prod = w * input[k];
                acc = acc + prod;
            }
            partials[tid] = acc;
        }
        output[m] = tree_sum(partials);
    }
}

/* ---- shaders/matmul_q4k.wgsl:34-58 (and matmul_q4k_mr.wgsl) ---------------
 * 4-bit unsigned weights, 8 per u32 little-endian nibble order over the flat
 * [M][N] array; per row and 256-element super-block, 16 f16 values: the scales
 * of its 8 sub-blocks of 32, then their mins. dequant = scale * nibble + min
 * (two rounded operations), acc + dequant * x; then the tree.                */
void wr_matmul_q4k(const float* input, const uint32_t* qweight, const uint16_t* qmeta, float* output, uint32_t M,
                   uint32_t N) {
    const uint32_t nsblk = N / 256;
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < (int64_t)M; m++) {
        float partials[WG];
        const uint64_t qbase = (uint64_t)m * N;
        const uint64_t mbase_row = (uint64_t)m * nsblk * 16;
        for (uint32_t tid = 0; tid < WG; tid++) {
            float acc = 0.0f;
            for (uint32_t k = tid; k < N; k += WG) {
                const uint64_t fi = qbase + k;
                const uint32_t nib = (qweight[fi >> 3] >> ((fi & 7) * 4)) & 0xfu;
                const uint64_t mb = mbase_row + (uint64_t)(k >> 8) * 16;
                const uint32_t sub = (k & 255u) >> 5;
                const float scale = wr_f16_to_f32(qmeta[mb + sub]);
                const float mn = wr_f16_to_f32(qmeta[mb + 8 + sub]);
                const float t = scale * (float)nib;
                const float dq = t + mn;
                const float prod = dq * input[k];
                acc = acc + prod;
            }
            partials[tid] = acc;
        }
        output[m] = tree_sum(partials);
    }
}

/* ---- shaders/logit_softcap.wgsl:9-16 ------------------------------------ */
void wr_logit_softcap(float* logits, uint32_t size, float cap) {
    for (uint32_t i = 0; i < size; i++) {
        float x = logits[i] / cap;
        float c = x < -15.0f ? -15.0f : (x > 15.0f ? 15.0f : x);
        logits[i] = (float)tanh((double)c) * cap;
    }
}

/* ---- shaders/argmax.wgsl:7-34 (one workgroup) --------------------------- *
 * Per-invocation first strict maximum over i = tid (mod 256) (values not
 * above the -1e30 start and NaN never win; index 0 if nothing does), then the
 * 128 -> 1 tree, in which a slot takes its partner's pair only when strictly
 * greater. Among residues holding the maximum, the tree's last level prefers
 * bit 0 of the residue clear, the level before bit 1, and so on: the winner is
 * the residue with the smallest bit-reversed (8-bit) value, not the smallest
 * residue (residues 1 and 4 tie: 4 wins).                                    */
uint32_t wr_argmax(const float* logits, uint32_t size) {
    float smax[WG];
    uint32_t sidx[WG];
    for (uint32_t tid = 0; tid < WG; tid++) {
        float local_max = -1e30f;
        uint32_t local_idx = 0u;
        for (uint32_t i = tid; i < size; i += WG) {
            float val = logits[i];
            if (val > local_max) {
                local_max = val;
                local_idx = i;
            }
        }
        smax[tid] = local_max;
        sidx[tid] = local_idx;
    }
    for (uint32_t stride = 128u; stride > 0u; stride >>= 1u)
        for (uint32_t t = 0; t < stride; t++)
            if (smax[t + stride] > smax[t]) {
                smax[t] = smax[t + stride];
                sidx[t] = sidx[t + stride];
            }
    return sidx[0];
}

/* ---- Composite: one reference decode step of one layer's attention block,
 * in the order encodeTransformerPass dispatches it (engine.ts:2056-2095):
 * vNorm (producer) -> fusedNormRope Q,K -> kvCacheStore (producer) ->
 * attnScore -> softmax -> attnOutput. Caches are f32 as the WGSL binds them. */
void wr_attention_layer_step(float* q, float* k, float* v, const uint16_t* q_weight, const uint16_t* k_weight,
                             const uint16_t* rope_freqs, float* k_cache, float* v_cache, float* scores,
                             float* out, uint32_t nqh, uint32_t nkh, uint32_t hd, float eps, uint32_t position,
                             float theta, uint32_t apply_divisor, uint32_t sliding_window, float scale,
                             uint32_t max_seq, int producer) {
    uint32_t seq_len = position + 1u;
    if (producer) {
        wr_norm_params vp = {nkh, hd, eps, 0u};
        wr_per_head_rms_norm_no_weight(v, &vp, nkh);
    }
    wr_norm_rope_params qp = {nqh, hd, eps, position, theta, apply_divisor};
    wr_fused_per_head_norm_rope(q, q_weight, &qp, rope_freqs, nqh);
    if (producer) {
        wr_norm_rope_params kp = {nkh, hd, eps, position, theta, apply_divisor};
        wr_fused_per_head_norm_rope(k, k_weight, &kp, rope_freqs, nkh);
        wr_kv_store_params sp = {nkh, hd, position, max_seq};
        wr_kv_cache_store(k, v, k_cache, v_cache, &sp, (nkh * hd + WG - 1u) / WG);
    }
    wr_attn_score_params ap = {nqh, nkh, hd, seq_len, scale, sliding_window};
    wr_attn_score(q, k_cache, scores, &ap, (uint32_t)(((uint64_t)nqh * seq_len + WG - 1u) / WG));
    wr_softmax_params smp = {nqh, seq_len};
    wr_softmax(scores, &smp, nqh);
    wr_attn_output_params op = {nqh, nkh, hd, seq_len};
    wr_attn_output(scores, v_cache, out, &op, (nqh * hd + WG - 1u) / WG);
}

/* Thread count of the OpenMP workgroup loops (the CPU baseline states it). */
#include <omp.h>
void wr_set_num_threads(int n) { omp_set_num_threads(n); }
int wr_get_max_threads(void) { return omp_get_max_threads(); }
