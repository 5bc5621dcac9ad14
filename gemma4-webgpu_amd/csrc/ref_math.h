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

// RoPE inverse frequency of pair i (fused_per_head_norm_rope.wgsl:50-54):
// 1/pow(theta, 2i/HD) (pow in f64, rounded to f32), optionally divided by
// rope_freqs[i] (given here as its value). Independent of the position.
__device__ __forceinline__ float rope_inv_freq(unsigned i, unsigned head_dim, float theta, unsigned apply_divisor,
                                               float divisor) {
    float e = (float)(i * 2u) / (float)head_dim;
    float base_freq = 1.0f / (float)pow((double)theta, (double)e);
    float freq = base_freq;
    if (apply_divisor != 0u) freq = base_freq / divisor;
    return freq;
}

// f32(cos a) and f32(sin a) of an f32 angle evaluated in f64, as the reference
// expressions are restated (fused_per_head_norm_rope.wgsl:56-57): equal to
// (float)cos((double)a) and (float)sin((double)a). One Cody-Waite reduction
// a = k pi/2 + r (pi/2 in parts of 33, 33 and 53 bits: k P1 and k P2 are exact
// for |k| < 2^20) and Taylor polynomials on |r| <= pi/4 (next terms below
// 2^-62 relative) leave the value d a few f64 ulps from the exact one; the
// device library's cos and sin are within one ulp of it. Where d +- 2^-46 |d|
// rounds to one f32, both round to that f32; a value near an f32 rounding
// boundary, or an angle beyond 2^20 or not finite, takes the device library's
// cos and sin.
__device__ __forceinline__ void f64_cos_sin(float a, float& c, float& s) {
    constexpr double kTwoOverPi = 0x1.45f306dc9c883p-1;
    constexpr double kP1 = 0x1.921fb544p+0, kP2 = 0x1.0b4611a6p-34, kP3 = 0x1.3198a2e037073p-69;
    constexpr double kRound = 0x1.8p52;  // adding and subtracting it rounds to an integer (|x| < 2^51)
    const double x = (double)a;
    const double kr = fma(x, kTwoOverPi, kRound);
    const double k = kr - kRound;
    const unsigned q = (unsigned)__double2loint(kr) & 3u;  // quadrant: a = k pi/2 + r
    const double r = fma(-k, kP3, fma(-k, kP2, fma(-k, kP1, x)));
    const double z = r * r;
    double ps = 1.0 / 355687428096000;  // sin r = r + r z (-1/3! + z (1/5! - ...)), terms to r^17
    ps = fma(z, ps, -1.0 / 1307674368000);
    ps = fma(z, ps, 1.0 / 6227020800);
    ps = fma(z, ps, -1.0 / 39916800);
    ps = fma(z, ps, 1.0 / 362880);
    ps = fma(z, ps, -1.0 / 5040);
    ps = fma(z, ps, 1.0 / 120);
    ps = fma(z, ps, -1.0 / 6);
    const double sr = fma(r * z, ps, r);
    double pc = -1.0 / 6402373705728000;  // cos r = 1 + z (-1/2! + z (1/4! - ...)), terms to r^18
    pc = fma(z, pc, 1.0 / 20922789888000);
    pc = fma(z, pc, -1.0 / 87178291200);
    pc = fma(z, pc, 1.0 / 479001600);
    pc = fma(z, pc, -1.0 / 3628800);
    pc = fma(z, pc, 1.0 / 40320);
    pc = fma(z, pc, -1.0 / 720);
    pc = fma(z, pc, 1.0 / 24);
    pc = fma(z, pc, -0.5);
    const double cr = fma(z, pc, 1.0);
    const double sv = q & 1u ? cr : sr, cv = q & 1u ? sr : cr;
    const double sin_a = q & 2u ? -sv : sv;
    const double cos_a = (q + 1u) & 2u ? -cv : cv;
    const double es = 0x1p-46 * fabs(sin_a), ec = 0x1p-46 * fabs(cos_a);
    const bool ok = fabs(x) <= 0x1p20 && (float)(sin_a - es) == (float)(sin_a + es) &&
                    (float)(cos_a - ec) == (float)(cos_a + ec);
    if (ok) {
        c = (float)cos_a;
        s = (float)sin_a;
    } else {
        c = (float)cos(x);
        s = (float)sin(x);
    }
}

// The angle of pair i at `position` (fused_per_head_norm_rope.wgsl:55).
__device__ __forceinline__ float rope_angle_val(unsigned i, unsigned head_dim, float theta, unsigned position,
                                                unsigned apply_divisor, float divisor) {
    return (float)position * rope_inv_freq(i, head_dim, theta, apply_divisor, divisor);
}

__device__ __forceinline__ float rope_angle(unsigned i, unsigned head_dim, float theta, unsigned position,
                                            unsigned apply_divisor, const uint16_t* rope_freqs) {
    return rope_angle_val(i, head_dim, theta, position, apply_divisor, apply_divisor ? h2f(rope_freqs[i]) : 1.0f);
}

// The reference's 128 -> 1 tree over 256 partials with two LDS steps
// (strides 128, 64) and wave shuffles for strides 32..1: the same operand
// pairs are added, so the total is bit-identical to wg_tree_sum. The total is
// returned to every thread. `s` holds at least 256 floats.
__device__ __forceinline__ float wg_tree_sum_fast(float partial, float* s, unsigned tid) {
    s[tid] = partial;
    __syncthreads();
    if (tid < 128) s[tid] = s[tid] + s[tid + 128];
    __syncthreads();
    if (tid < 64) {
        float x = s[tid] + s[tid + 64];
        for (int stride = 32; stride > 0; stride >>= 1) x = x + __shfl_down(x, stride);
        if (tid == 0) s[256] = x;
    }
    __syncthreads();
    return s[256];
}

// Per-head RMSNorm (optionally weighted) + RoPE of one head held in global
// memory, by one 256-thread workgroup: fused_per_head_norm_rope.wgsl:23-63
// when `weight` is non-null and rope is on, per_head_rms_norm_no_weight.wgsl:
// 15-37 when weight is null and rope is off. When `f16_out` is non-null the
// final values are also stored there as f16 (the KV-cache row). `scratch`
// is a workgroup buffer of at least 257 + head_dim floats.
//
// head_dim <= 512: RoPE factors are computed first (they do not depend on the
// data, so the f64 transcendental latency overlaps the load and reduction),
// and the rotate-half pairs are exchanged through LDS. Larger heads take the
// literal loop form. Both evaluate the same expressions as the WGSL.
__device__ __forceinline__ void head_norm_rope(float* __restrict__ data, const uint16_t* __restrict__ weight,
                                               bool rope, const uint16_t* __restrict__ rope_freqs,
                                               unsigned head_dim, float eps, unsigned position, float theta,
                                               unsigned apply_divisor, float* scratch,
                                               uint16_t* __restrict__ f16_out = nullptr) {
    const unsigned tid = threadIdx.x;
    const unsigned half_dim = head_dim / 2u;
    if (head_dim <= 2 * kWG) {
        float cos_a = 1.0f, sin_a = 0.0f;
        if (rope && tid < half_dim) {
            const float angle = rope_angle(tid, head_dim, theta, position, apply_divisor, rope_freqs);
            cos_a = (float)cos((double)angle);
            sin_a = (float)sin((double)angle);
        }
        float xv[2] = {0.0f, 0.0f};
        float partial = 0.0f;
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const unsigned i = tid + r * kWG;
            if (i < head_dim) {
                xv[r] = data[i];
                partial = partial + xv[r] * xv[r];
            }
        }
        const float rms = sqrtf(wg_tree_sum_fast(partial, scratch, tid) / (float)head_dim + eps);
        float* buf = scratch + 257;
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const unsigned i = tid + r * kWG;
            if (i < head_dim) {
                xv[r] = weight ? xv[r] * h2f(weight[i]) / rms : xv[r] / rms;
                if (rope) {
                    buf[i] = xv[r];
                } else {
                    data[i] = xv[r];
                    if (f16_out) f16_out[i] = f2h(xv[r]);
                }
            }
        }
        if (!rope) return;
        __syncthreads();
        if (tid < half_dim) {
            const float x0 = buf[tid];
            const float x1 = buf[tid + half_dim];
            const float y0 = x0 * cos_a - x1 * sin_a;
            const float y1 = x0 * sin_a + x1 * cos_a;
            data[tid] = y0;
            data[tid + half_dim] = y1;
            if (f16_out) {
                f16_out[tid] = f2h(y0);
                f16_out[tid + half_dim] = f2h(y1);
            }
        }
        return;
    }
    float partial = 0.0f;
    for (unsigned i = tid; i < head_dim; i += kWG) {
        float val = data[i];
        partial = partial + val * val;
    }
    scratch[tid] = partial;
    __syncthreads();
    const float rms = sqrtf(wg_tree_sum(scratch, tid) / (float)head_dim + eps);
    if (weight) {
        for (unsigned i = tid; i < head_dim; i += kWG) data[i] = data[i] * h2f(weight[i]) / rms;
    } else {
        for (unsigned i = tid; i < head_dim; i += kWG) data[i] = data[i] / rms;
    }
    __syncthreads();
    if (rope) {
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
    if (f16_out) {
        __syncthreads();
        for (unsigned i = tid; i < head_dim; i += kWG) f16_out[i] = f2h(data[i]);
    }
}

// Workgroup scratch for head_norm_rope with head_dim <= 512.
constexpr unsigned kNormScratch = 257 + 2 * kWG;

// RoPE factors of pairs (l + 64p, l + 64p + HD/2), p = 0 .. HD/128 - 1, for lane l.
template <int PJ>
struct RopeLane {
    float c[PJ], s[PJ];
};

// The reference's tree over one value per lane, strides 32, 16, 8, 4, 2, 1:
// lane 0 ends with ((v0 + v32) + (v16 + v48)) + ... , the operand pairs of a
// shuffle-down tree, and the total is returned to every lane. Strides 32 and
// 16 swap lane halves and row pairs (v_permlane32_swap / v_permlane16_swap,
// every lane then holds its butterfly sum), strides 8..1 shift within 16-lane
// rows (DPP row_shl: lane l takes lane l + s), so no step goes through LDS.
__device__ __forceinline__ float wave_tree_sum(float c) {
    {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(c), __float_as_uint(c), false, false);
        c = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    {
        const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(c), __float_as_uint(c), false, false);
        c = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    c = c + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(c), 0x108, 0xf, 0xf, false));  // row_shl:8
    c = c + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(c), 0x104, 0xf, 0xf, false));  // row_shl:4
    c = c + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(c), 0x102, 0xf, 0xf, false));  // row_shl:2
    c = c + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(c), 0x101, 0xf, 0xf, false));  // row_shl:1
    return __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(c)));
}

// Per-head RMSNorm (+ RoPE) of one HD-wide head by one wave; lane l holds
// x[l + 64j], j = 0 .. HD/64 - 1 (and the weight's f16 bits at the same
// places), and receives the results in place. The sum of squares adds the
// same terms in the same order as the reference's workgroup: partial t
// (= l + 64q, q = 0..3) sums x[t]^2, x[t + 256]^2, ... in order, then the
// tree with strides 128, 64 (in the lane) and 32..1 (across lanes), so every
// value is bit-identical to fused_per_head_norm_rope.wgsl /
// per_head_rms_norm_no_weight.wgsl.
// a / b, correctly rounded, for many dividends over one divisor b whose
// correctly rounded reciprocal y = 1.0f / b is computed once: q0 = a y is
// within an ulp of a / b, the residual a - q0 b is exact in one FMA, and
// q0 + (a - q0 b) y rounds to the correctly rounded quotient (Markstein's
// theorem; Muller et al., Handbook of Floating-Point Arithmetic, 2nd ed.,
// ch. 4). Tiny, zero or non-finite dividends and divisors of 2^32 or more,
// where an intermediate could leave the normal range, take the IEEE
// division. Checked bit for bit against a / b over 10^9 operand pairs
// (tests/div_check.c).
__device__ __forceinline__ float div_shared(float a, float b, float y) {
    if (!(fabsf(a) >= 0x1p-64f) || !(b < 0x1p32f)) return a / b;
    const float q0 = a * y;
    return __builtin_fmaf(__builtin_fmaf(-q0, b, a), y, q0);
}

template <int J>
__device__ __forceinline__ void wave_norm_rope(float (&x)[J], const uint32_t (&wbits)[J], bool weighted, bool rope,
                                               const RopeLane<J / 2>& r, float eps) {
#pragma clang fp contract(off)
    constexpr int HD = 64 * J, PJ = J / 2;
    float part[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        part[q] = x[q] * x[q];
#pragma unroll
        for (int m = 1; m < J / 4; m++) part[q] = part[q] + x[q + 4 * m] * x[q + 4 * m];
    }
    const float a = part[0] + part[2];  // t = lane      : s[t] + s[t + 128]
    const float b = part[1] + part[3];  // t = lane + 64 : s[t] + s[t + 128]
    const float total = wave_tree_sum(a + b);  // stride 64, then 32 .. 1
    const float rms = sqrtf(total / (float)HD + eps);
    const float inv = 1.0f / rms;  // correctly rounded: the divisor's reciprocal for div_shared
#pragma unroll
    for (int j = 0; j < J; j++) x[j] = div_shared(weighted ? x[j] * h2f((uint16_t)wbits[j]) : x[j], rms, inv);
    if (!rope) return;
#pragma unroll
    for (int p = 0; p < PJ; p++) {
        const float x0 = x[p], x1 = x[p + PJ];
        x[p] = x0 * r.c[p] - x1 * r.s[p];
        x[p + PJ] = x0 * r.s[p] + x1 * r.c[p];
    }
}

}  // namespace g4
