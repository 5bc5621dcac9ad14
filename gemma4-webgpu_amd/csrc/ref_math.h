// Device helpers shared by the reference-semantics kernels and the fused
// prep kernel, so that both evaluate the same expressions in the same order
// and produce identical bits. Every f32 operation in code that includes this
// header rounds separately: FMA contraction is off from here on.
#pragma once

#include "common.h"

#pragma clang fp contract(off)

namespace g4 {

constexpr unsigned kWG = 256;  // @workgroup_size(256) of every reference shader

// The reference's 128 -> 1 workgroup tree (stride loop with barriers).
__device__ __forceinline__ float wg_tree_sum(float* s, unsigned tid) {
    for (unsigned stride = 128; stride > 0; stride >>= 1) {
        if (tid < stride) s[tid] = s[tid] + s[tid + stride];
        __syncthreads();
    }
    return s[0];
}

__device__ __forceinline__ float wgsl_max(float a, float b) { return a > b ? a : (b > a ? b : a); }

__device__ __forceinline__ float wg_tree_max(float* s, unsigned tid) {
    for (unsigned stride = 128; stride > 0; stride >>= 1) {
        if (tid < stride) s[tid] = wgsl_max(s[tid], s[tid + stride]);
        __syncthreads();
    }
    return s[0];
}

// RoPE angle terms of pair i: freq = 1/pow(theta, 2i/HD) (optionally divided
// by rope_freqs[i]), angle = f32(position) * freq.
__device__ __forceinline__ float rope_angle(unsigned i, unsigned head_dim, float theta, unsigned position,
                                            unsigned apply_divisor, const uint16_t* rope_freqs) {
    float e = (float)(i * 2u) / (float)head_dim;
    float base_freq = 1.0f / (float)pow((double)theta, (double)e);
    float freq = base_freq;
    if (apply_divisor != 0u) freq = base_freq / h2f(rope_freqs[i]);
    return (float)position * freq;
}

// Per-head RMSNorm (optionally weighted) + RoPE of one head held in global
// memory, by one 256-thread workgroup; fused_per_head_norm_rope.wgsl:23-63
// when `weight` is non-null and rope is on, per_head_rms_norm_no_weight.wgsl:
// 15-37 when weight is null and rope is off. `shared_sum` is a 256-float
// workgroup buffer.
__device__ __forceinline__ void head_norm_rope(float* __restrict__ data, const uint16_t* __restrict__ weight,
                                               bool rope, const uint16_t* __restrict__ rope_freqs,
                                               unsigned head_dim, float eps, unsigned position, float theta,
                                               unsigned apply_divisor, float* shared_sum) {
    const unsigned tid = threadIdx.x;
    float partial = 0.0f;
    for (unsigned i = tid; i < head_dim; i += kWG) {
        float val = data[i];
        partial = partial + val * val;
    }
    shared_sum[tid] = partial;
    __syncthreads();
    const float rms = sqrtf(wg_tree_sum(shared_sum, tid) / (float)head_dim + eps);
    if (weight) {
        for (unsigned i = tid; i < head_dim; i += kWG) data[i] = data[i] * h2f(weight[i]) / rms;
    } else {
        for (unsigned i = tid; i < head_dim; i += kWG) data[i] = data[i] / rms;
    }
    __syncthreads();
    if (!rope) return;
    const unsigned half_dim = head_dim / 2u;
    for (unsigned i = tid; i < half_dim; i += kWG) {
        float angle = rope_angle(i, head_dim, theta, position, apply_divisor, rope_freqs);
        float cos_a = (float)cos((double)angle);
        float sin_a = (float)sin((double)angle);
        float x0 = data[i];
        float x1 = data[i + half_dim];
        data[i] = x0 * cos_a - x1 * sin_a;
        data[i + half_dim] = x0 * sin_a + x1 * cos_a;
    }
}

}  // namespace g4
