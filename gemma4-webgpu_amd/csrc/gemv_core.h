// Row dot products of an f16 weight matrix with an f32 vector, in
// matmul_quant.wgsl's order (shaders/matmul_quant.wgsl:28-52, and the
// per-row order of matmul_quant_mr4.wgsl): the 256 partial sums
// p[t] = sum_j w[t + 256 j] * x[t + 256 j] (in j order, each product and sum
// rounded, no fused multiply-add), then the 128 -> 1 tree.
//
// A half-wave (32 lanes) owns one row: lane l (0..31 within the half) loads
// 16 bytes (8 columns) of every 256-column block with nontemporal loads, so
// it holds partials t = 8 l .. 8 l + 7 and accumulates them in j order. The
// tree's strides 128..8 pair lanes l and l + 16 .. l + 1 (gemv_tree_sum),
// strides 4, 2, 1 stay in the lane. The row's value, bit-identical to the
// shader's, ends in every lane of the half or in its lane 0 (kAll).
#pragma once

#include "ref_math.h"

namespace g4 {

template <typename T>
__device__ __forceinline__ T ldg_nt(const void* p) {
    typedef const __attribute__((address_space(1))) T* gp;
    return __builtin_nontemporal_load((gp)(p));
}

// x[256 j + 8 lq + e] into registers (lq: lane within the half-wave).
template <int NJ>
__device__ __forceinline__ void gemv_load_x(const float* x, unsigned lq, float (&xr)[NJ][8]) {
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const f32x4 a = ldg<f32x4>(x + 256 * j + 8 * lq), b = ldg<f32x4>(x + 256 * j + 8 * lq + 4);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            xr[j][e] = a[e];
            xr[j][e + 4] = b[e];
        }
    }
}

// The lane's weights of a row (8 columns of every 256-column block); `row`
// points at the row's first element, 16-byte aligned.
template <int NJ>
__device__ __forceinline__ void gemv_row_load(const uint16_t* row, unsigned lq, f16x8 (&wv)[NJ]) {
    const uint16_t* w = row + 8 * lq;
#pragma unroll
    for (int j = 0; j < NJ; j++) wv[j] = ldg_nt<f16x8>(w + 256 * j);
}

// The tree over the half-wave's 256 partials (8 per lane). kAll: every lane of
// the half ends with the value (strides 128 .. 8 as butterflies between lanes
// l and l ^ 16 .. l ^ 1, through LDS shuffles); otherwise only lane 0 of each
// half does, with the same operand pairs: stride 128 swaps 16-lane rows
// (v_permlane16_swap, both lanes of a pair then hold their sum) and strides
// 64 .. 8 shift within rows (DPP row_shl: lane l takes lane l + s), all in
// VALU. Strides 4, 2, 1 stay in the lane.
template <bool kAll>
__device__ __forceinline__ float gemv_tree_sum(float (&acc)[8]) {
#pragma clang fp contract(off)
    if constexpr (kAll) {
#pragma unroll
        for (int m = 16; m >= 1; m >>= 1)  // tree strides 128 .. 8
#pragma unroll
            for (int e = 0; e < 8; e++) acc[e] = acc[e] + __shfl_xor(acc[e], m);
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(acc[e]), __float_as_uint(acc[e]), false, false);
            acc[e] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);  // stride 128
        }
#pragma unroll
        for (int e = 0; e < 8; e++)  // stride 64
            acc[e] = acc[e] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc[e]), 0x108, 0xf, 0xf, false));
#pragma unroll
        for (int e = 0; e < 8; e++)  // stride 32
            acc[e] = acc[e] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc[e]), 0x104, 0xf, 0xf, false));
#pragma unroll
        for (int e = 0; e < 8; e++)  // stride 16
            acc[e] = acc[e] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc[e]), 0x102, 0xf, 0xf, false));
#pragma unroll
        for (int e = 0; e < 8; e++)  // stride 8
            acc[e] = acc[e] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc[e]), 0x101, 0xf, 0xf, false));
    }
#pragma unroll
    for (int e = 0; e < 4; e++) acc[e] = acc[e] + acc[e + 4];  // stride 4
    acc[0] = acc[0] + acc[2];                                    // stride 2
    acc[1] = acc[1] + acc[3];
    return acc[0] + acc[1];                                      // stride 1
}

// The row's value from weights loaded by gemv_row_load (in every lane of the
// half-wave, or in its lane 0 when kAll is false).
template <int NJ, bool kAll = true>
__device__ __forceinline__ float gemv_row_fold(const f16x8 (&wv)[NJ], const float (&xr)[NJ][8]) {
#pragma clang fp contract(off)
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; e++) acc[e] = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] = acc[e] + (float)wv[j][e] * xr[j][e];
    return gemv_tree_sum<kAll>(acc);
}

// The row's value (in every lane of the half-wave, or in its lane 0 when kAll
// is false); `row` points at the row's first element, 16-byte aligned.
template <int NJ, bool kAll = true>
__device__ __forceinline__ float gemv_row_dot(const uint16_t* row, const float (&xr)[NJ][8], unsigned lq) {
    f16x8 wv[NJ];
    gemv_row_load<NJ>(row, lq, wv);
    // Every weight load is issued before the arithmetic: left to itself the compiler spreads the
    // loads of the lane-0 form (which needs fewer registers) over the products, and each then
    // waits a memory round trip (k_linear at input 4096: 11.0 us instead of 6.1).
    if constexpr (!kAll) __builtin_amdgcn_sched_barrier(0);
    return gemv_row_fold<NJ, kAll>(wv, xr);
}

// The same row value for quantized weights, in matmul_q8.wgsl's and
// matmul_q4k.wgsl's per-element order (each operation rounded, no fused
// multiply-add), with the same partials, j order and tree:
//   Q8:  w = f32(int8) * f32(scale[k / 32]);           acc = acc + w * x[k]
//   Q4K: w = f32(scale[sub]) * f32(nibble) + f32(min[sub]); acc = acc + w * x[k]
// Lane l of the half-wave covers k = 256 j + 8 l .. + 7, which lie in one
// 32-element block (Q8 scale 8 j + l / 4; Q4K super-block j, sub-block l / 4).
// qrow: the row's int8 weights (N bytes, 8-byte aligned); srow: its N/32 f16 scales.
template <int NJ, bool kAll = true>
__device__ __forceinline__ float gemv_row_dot_q8(const int8_t* qrow, const uint16_t* srow, const float (&xr)[NJ][8],
                                                 unsigned lq) {
#pragma clang fp contract(off)
    uint64_t qv[NJ];
    uint32_t sv[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        qv[j] = ldg_nt<uint64_t>(qrow + 256 * j + 8 * lq);
        sv[j] = ldg<uint16_t>(srow + 8 * j + (lq >> 2));
    }
    if constexpr (!kAll) __builtin_amdgcn_sched_barrier(0);  // every load before the arithmetic (gemv_row_dot)
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; e++) acc[e] = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const float sc = h2f((uint16_t)sv[j]);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float w = (float)(int8_t)(qv[j] >> (8 * e)) * sc;
            acc[e] = acc[e] + w * xr[j][e];
        }
    }
    return gemv_tree_sum<kAll>(acc);
}

// qrow: the row's nibbles (N / 8 words, 8 per word, low nibble first); mrow: its
// (N / 256) x 16 f16 values (8 scales, then 8 mins, per super-block).
template <int NJ, bool kAll = true>
__device__ __forceinline__ float gemv_row_dot_q4k(const uint32_t* qrow, const uint16_t* mrow, const float (&xr)[NJ][8],
                                                  unsigned lq) {
#pragma clang fp contract(off)
    uint32_t qv[NJ], sv[NJ], mv[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        qv[j] = ldg_nt<uint32_t>(qrow + 32 * j + lq);
        sv[j] = ldg<uint16_t>(mrow + 16 * j + (lq >> 2));
        mv[j] = ldg<uint16_t>(mrow + 16 * j + 8 + (lq >> 2));
    }
    if constexpr (!kAll) __builtin_amdgcn_sched_barrier(0);  // every load before the arithmetic (gemv_row_dot)
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; e++) acc[e] = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const float sc = h2f((uint16_t)sv[j]), mn = h2f((uint16_t)mv[j]);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float t = sc * (float)((qv[j] >> (4 * e)) & 15u);
            const float w = t + mn;
            acc[e] = acc[e] + w * xr[j][e];
        }
    }
    return gemv_tree_sum<kAll>(acc);
}

}  // namespace g4
