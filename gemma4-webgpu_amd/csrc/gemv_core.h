// Row dot products of an f16 weight matrix with an f32 vector, in
// matmul_quant.wgsl's order (shaders/matmul_quant.wgsl:28-52, and the
// per-row order of matmul_quant_mr4.wgsl): the 256 partial sums
// p[t] = sum_j w[t + 256 j] * x[t + 256 j] (in j order, each product and sum
// rounded, no fused multiply-add), then the 128 -> 1 tree.
//
// A half-wave (32 lanes) owns one row: lane l (0..31 within the half) loads
// 16 bytes (8 columns) of every 256-column block with nontemporal loads, so
// it holds partials t = 8 l .. 8 l + 7 and accumulates them in j order. The
// tree's strides 128..8 pair lanes l and l ^ 16 .. l ^ 1 (butterfly: both
// lanes form the same commutative sum), strides 4, 2, 1 stay in the lane.
// Every lane of the half ends with the row's value, bit-identical to the
// shader's.
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

// The row's value (in every lane of the half-wave); `row` points at the
// row's first element, 16-byte aligned.
template <int NJ>
__device__ __forceinline__ float gemv_row_dot(const uint16_t* row, const float (&xr)[NJ][8], unsigned lq) {
#pragma clang fp contract(off)
    const uint16_t* w = row + 8 * lq;
    f16x8 wv[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) wv[j] = ldg_nt<f16x8>(w + 256 * j);
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; e++) acc[e] = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] = acc[e] + (float)wv[j][e] * xr[j][e];
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1)  // tree strides 128 .. 8
#pragma unroll
        for (int e = 0; e < 8; e++) acc[e] = acc[e] + __shfl_xor(acc[e], m);
#pragma unroll
    for (int e = 0; e < 4; e++) acc[e] = acc[e] + acc[e + 4];  // stride 4
    acc[0] = acc[0] + acc[2];                                    // stride 2
    acc[1] = acc[1] + acc[3];
    return acc[0] + acc[1];                                      // stride 1
}

}  // namespace g4
