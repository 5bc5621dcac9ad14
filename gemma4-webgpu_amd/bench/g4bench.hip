// g4bench: command-line driver of the decode path over the C ABI, with no
// Python or torch in the process (so it runs cleanly under rocprofv3
// counter collection). Inputs are synthetic: f16 cache rows from a
// counter-based hash (values in [-2, 2), unit-RMS scale), queries likewise.
//
//   g4bench [--workload stack4k|stack8k|stack32k|stack128k|long128k|ragged64|layer512|prefill4k|prefill4k512|
//            lmhead|copy] [--iters N]
//           [--sets S] [--mode M]
//
// Decode workloads: the configurations above; `e2b8k` / `e2b32k` (35 layers at E2B's head dims,
// 512 on global layers: one step per head_dim group); `e2bshared8k` / `e2bshared32k` (the same
// with E2B's cache sharing: layers 15..34 read layer 13's or 14's cache and store nothing);
// `long128k_hd512`. --mode step (default: the one-launch step), graph (the step replayed as a
// captured HIP graph), or, for head_dim 256 only, the unfused prep + split + merge. Token loops,
// where the position advances every iteration and every plan is prepared again inside the timed
// region: --mode loop (one step per head_dim group per token), layers (the engine's layer order:
// one g4_attn_step_prepare_layers per head_dim group per token, then each layer's attention and
// merge launches in turn), layers_each (the same order with one g4_attn_step_prepare per layer), chain
// and chain_each (those two orders with each layer's q/k/v projection and o_proj around its attention).
// advance, layers_adv, chain_adv: loop, layers and chain with each plan advanced on the host every token
// (g4_attn_step_advance) and prepared again every 32 tokens.
//
// `prefill4k` runs the causal MFMA prefill of a 4096-token prompt for one
// global layer and one 512-window local layer, as 512-token chunks (16
// entries in one launch; --mode whole: one entry per layer). `prefill4k512`
// runs the global layer alone at head_dim 512 (E2B's global layers).
//
// `proj256` / `proj512` run the block's projections (q, k, v and o_proj) of a
// local / global E2B layer (--mode fused|chain).
//
// `lmhead` runs the sampling head (lm head GEMV, softcap, argmax) at Gemma 4
// E2B's shape (--mode fused|chain).
//
// `copy` runs a plain 512 MiB device copy kernel instead: the reference for
// scaling FETCH_SIZE / WRITE_SIZE counter readings to bytes.
//
// Each iteration runs, on one stream: the multi-layer prep (when the workload
// has one position for all entries), the split pass and the merge pass of a
// prepared multi-entry decode plan, rotating over S cache sets.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "../../include/g4attn.h"

#define CK(x)                                                                       \
    do {                                                                            \
        int rc_ = (x);                                                              \
        if (rc_) {                                                                  \
            fprintf(stderr, "%s failed: %d %s\n", #x, rc_, g4_last_error());        \
            exit(1);                                                                \
        }                                                                           \
    } while (0)
#define HK(x)                                                                       \
    do {                                                                            \
        hipError_t e_ = (x);                                                        \
        if (e_ != hipSuccess) {                                                     \
            fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));          \
            exit(1);                                                                \
        }                                                                           \
    } while (0)

static const unsigned NQH = 8, NKH = 1, HD = 256;
static const unsigned kHidden = 1536;  // E2B's hidden size: the projections' input length and o_proj rows

__device__ __forceinline__ float hash_unit(uint64_t x) {  // splitmix64 finaliser -> [-2, 2)
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    x ^= x >> 31;
    return (float)((x >> 40) * (1.0 / 16777216.0)) * 4.0f - 2.0f;
}

__global__ void k_fill_f16(_Float16* p, uint64_t n, uint64_t seed) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        p[i] = (_Float16)(hash_unit(seed * 0x100000001B3ull + i) * 0.866f);  // uniform[-2,2) has RMS 1.155
}
__global__ void k_fill_f32(float* p, uint64_t n, uint64_t seed) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        p[i] = hash_unit(seed * 0x100000001B3ull + i) * 0.866f;
}

// Plain copy of n 16-byte words: the counter calibration reference (reads and
// writes exactly n * 16 bytes each).
__global__ void k_copy(uint4* __restrict__ dst, const uint4* __restrict__ src, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

static int run_copy(int iters) {
    const uint64_t bytes = 512ull << 20;
    void *src, *dst;
    CK(g4_malloc(&src, bytes));
    CK(g4_malloc(&dst, bytes));
    hipEvent_t a, b;
    HK(hipEventCreate(&a));
    HK(hipEventCreate(&b));
    hipLaunchKernelGGL(k_copy, dim3(4096), dim3(256), 0, 0, (uint4*)dst, (const uint4*)src, bytes / 16);
    HK(hipDeviceSynchronize());
    HK(hipEventRecord(a, 0));
    for (int i = 0; i < iters; i++)
        hipLaunchKernelGGL(k_copy, dim3(4096), dim3(256), 0, 0, (uint4*)dst, (const uint4*)src, bytes / 16);
    HK(hipEventRecord(b, 0));
    HK(hipEventSynchronize(b));
    float ms = 0;
    HK(hipEventElapsedTime(&ms, a, b));
    printf("copy: %llu bytes read + written per launch, %.1f GB/s (read+write)\n", (unsigned long long)bytes,
           2.0 * bytes * iters / (ms * 1e-3) / 1e9);
    return 0;
}

// Sampling head at Gemma 4 E2B's shape: the f16 tied embedding [262144][1536]
// as the lm head, softcap 30, greedy argmax. mode `fused` (default): the
// streaming lm head + pick; `chain`: matmulQuant, logitSoftcap, argmax as
// the reference dispatches them. Two weight copies are rotated (1.6 GB).
static int run_lmhead(const std::string& mode, int iters) {
    const uint32_t V = 262144, H = 1536;
    const float cap = 30.0f;
    const uint64_t wbytes = (uint64_t)V * H * 2;
    const uint64_t bytes = wbytes + (uint64_t)H * 4 + (uint64_t)V * 4;  // weight + hidden + logits
    printf("workload lmhead: vocab %u hidden %u, %.1f MB/step\n", V, H, bytes / 1e6);
    printf("bytes_per_step: %llu\n", (unsigned long long)bytes);
    hipStream_t st;
    HK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    void *w[2], *x, *logits, *res, *ws;
    size_t ws_bytes = 0;
    g4_lm_head_params p = {V, H, cap};
    CK(g4_lm_head_workspace_size(p, &ws_bytes));
    for (int i = 0; i < 2; i++) {
        CK(g4_malloc(&w[i], wbytes));
        hipLaunchKernelGGL(k_fill_f16, dim3(4096), dim3(256), 0, st, (_Float16*)w[i], wbytes / 2, 77ull + i);
    }
    CK(g4_malloc(&x, H * 4));
    CK(g4_malloc(&logits, V * 4));
    CK(g4_malloc(&res, 4));
    CK(g4_malloc(&ws, ws_bytes));
    hipLaunchKernelGGL(k_fill_f32, dim3(8), dim3(256), 0, st, (float*)x, (uint64_t)H, 5ull);
    HK(hipGetLastError());
    const bool fused = mode != "chain";
    auto step = [&](int i) {
        const uint16_t* wi = (const uint16_t*)w[i & 1];
        if (fused) {
            CK(g4_lm_head_argmax((const float*)x, wi, (float*)logits, (uint32_t*)res, ws, ws_bytes, p, st));
            return;
        }
        CK(g4_matmul_quant_f16((const float*)x, wi, (float*)logits, g4_matmul_params{V, H}, st));
        CK(g4_logit_softcap((float*)logits, g4_softcap_params{V, cap}, st));
        CK(g4_argmax((const float*)logits, (uint32_t*)res, V, st));
    };
    for (int i = 0; i < 3; i++) step(i);
    CK(g4_stream_synchronize(st));
    hipEvent_t a, b;
    HK(hipEventCreate(&a));
    HK(hipEventCreate(&b));
    HK(hipEventRecord(a, st));
    for (int i = 0; i < iters; i++) step(i);
    HK(hipEventRecord(b, st));
    HK(hipEventSynchronize(b));
    float ms = 0;
    HK(hipEventElapsedTime(&ms, a, b));
    const double us = ms * 1e3 / iters;
    step(0);  // the same weight copy in both modes: their top-1 must agree
    uint32_t top = 0;
    CK(g4_download(&top, res, 0, 4, st));
    printf("lmhead [%s]: %.2f us/step, %.1f GB/s algorithmic (%d iterations), top-1 of weight copy 0: %u\n",
           fused ? "fused" : "chain", us, bytes / (us * 1e3), iters, top);
    return 0;
}

// The attention block's projections at Gemma 4 E2B's shapes (hidden 1536):
// attn.linearQKV (q, k, v: 8 + 1 + 1 heads of head_dim hd) and attn.linearOut
// (hidden from 8 heads x hd), for a local (hd 256) or a global (hd 512)
// layer. mode `fused`: g4_linear_f16 (q, k, v in one launch); `chain`: the
// reference's one-workgroup-per-row matmulQuant per matrix. Weight sets are
// rotated so the bytes read per cycle exceed twice the 256 MB MALL.
//   --mode q8 | q4k: the same with the engine's quantized weights (g4_linear_quant), and
//   q8chain | q4kchain: one matmulQ8 / matmulQ4K dispatch per matrix.
static int run_proj(const std::string& wl, const std::string& mode, int iters, int sets_arg) {
    const uint32_t H = 1536, hd = wl == "proj512" ? 512 : 256, NQ = NQH * hd, NK = NKH * hd;
    const int fmt = mode.rfind("q8", 0) == 0 ? 1 : mode.rfind("q4k", 0) == 0 ? 2 : 0;
    const bool qchain = fmt && mode.find("chain") != std::string::npos;
    // bytes per weight element: f16 2; q8 1 + scale 2/32; q4k 1/2 + meta 2*16/256
    const double bpe = fmt == 0 ? 2.0 : fmt == 1 ? 1.0 + 2.0 / 32 : 0.5 + 32.0 / 256;
    const uint64_t welems = (uint64_t)(NQ + 2 * NK) * H + (uint64_t)H * NQ;
    const uint64_t wbytes = (uint64_t)(welems * bpe);
    const uint64_t bytes = wbytes + (H + NQ) * 4 + (uint64_t)(NQ + 2 * NK + H) * 4;
    // --sets N: N weight sets instead (1: the same weights every iteration, served from the MALL)
    const int sets = sets_arg > 0 ? sets_arg : (int)((512ull << 20) / wbytes) + 1;
    printf("workload %s: head_dim %u, %.2f MB of weights per layer, %d weight sets\n", wl.c_str(), hd, wbytes / 1e6,
           sets);
    printf("bytes_per_step: %llu\n", (unsigned long long)bytes);
    hipStream_t st;
    HK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    void *x, *q, *k, *v, *attn, *y;
    CK(g4_malloc(&x, H * 4));
    CK(g4_malloc(&q, NQ * 4));
    CK(g4_malloc(&k, NK * 4));
    CK(g4_malloc(&v, NK * 4));
    CK(g4_malloc(&attn, NQ * 4));
    CK(g4_malloc(&y, H * 4));
    hipLaunchKernelGGL(k_fill_f32, dim3(8), dim3(256), 0, st, (float*)x, (uint64_t)H, 3ull);
    hipLaunchKernelGGL(k_fill_f32, dim3(8), dim3(256), 0, st, (float*)attn, (uint64_t)NQ, 4ull);
    std::vector<void*> wq(sets), wk(sets), wv(sets), wo(sets), mq(sets), mk(sets), mv(sets), mo(sets);
    // Weights are filled as f16 noise over the bytes they occupy (the quantized forms read them as int8 /
    // nibbles, and their scale tables likewise as f16 noise): the timing does not depend on the values.
    auto alloc_fill = [&](void** p, uint64_t elems, unsigned long long seed) {
        const uint64_t bytes = fmt == 0 ? elems * 2 : fmt == 1 ? elems : elems / 2;
        CK(g4_malloc(p, bytes));
        hipLaunchKernelGGL(k_fill_f16, dim3(1024), dim3(256), 0, st, (_Float16*)*p, bytes / 2, seed);
    };
    auto alloc_meta = [&](void** p, uint64_t rows, uint32_t n, unsigned long long seed) {
        if (!fmt) return;
        const uint64_t vals = fmt == 1 ? rows * (n / 32) : rows * (n / 256) * 16;
        CK(g4_malloc(p, vals * 2));
        hipLaunchKernelGGL(k_fill_f16, dim3(64), dim3(256), 0, st, (_Float16*)*p, vals, seed);
    };
    for (int s = 0; s < sets; s++) {
        alloc_fill(&wq[s], (uint64_t)NQ * H, 100ull + s);
        alloc_fill(&wk[s], (uint64_t)NK * H, 200ull + s);
        alloc_fill(&wv[s], (uint64_t)NK * H, 300ull + s);
        alloc_fill(&wo[s], (uint64_t)H * NQ, 400ull + s);
        alloc_meta(&mq[s], NQ, H, 500ull + s);
        alloc_meta(&mk[s], NK, H, 600ull + s);
        alloc_meta(&mv[s], NK, H, 700ull + s);
        alloc_meta(&mo[s], H, NQ, 800ull + s);
    }
    HK(hipGetLastError());
    const bool fused = mode != "chain";
    auto step = [&](int i) {
        const int s = i % sets;
        if (fmt && !qchain) {
            g4_linear_qseg qkv[3] = {{wq[s], (const uint16_t*)mq[s], (float*)q, NQ},
                                     {wk[s], (const uint16_t*)mk[s], (float*)k, NK},
                                     {wv[s], (const uint16_t*)mv[s], (float*)v, NK}};
            CK(g4_linear_quant((const float*)x, H, (uint32_t)fmt, qkv, 3, st));
            g4_linear_qseg o = {wo[s], (const uint16_t*)mo[s], (float*)y, H};
            CK(g4_linear_quant((const float*)attn, NQ, (uint32_t)fmt, &o, 1, st));
            return;
        }
        if (qchain) {
            auto mm = [&](const float* in, void* w, void* m, float* out, uint32_t M, uint32_t N) {
                if (fmt == 1)
                    CK(g4_matmul_q8(in, (const int8_t*)w, (const uint16_t*)m, out, g4_matmul_params{M, N}, st));
                else
                    CK(g4_matmul_q4k(in, (const uint32_t*)w, (const uint16_t*)m, out, g4_matmul_params{M, N}, st));
            };
            mm((const float*)x, wq[s], mq[s], (float*)q, NQ, H);
            mm((const float*)x, wk[s], mk[s], (float*)k, NK, H);
            mm((const float*)x, wv[s], mv[s], (float*)v, NK, H);
            mm((const float*)attn, wo[s], mo[s], (float*)y, H, NQ);
            return;
        }
        if (fused) {
            g4_linear_seg qkv[3] = {{(const uint16_t*)wq[s], (float*)q, NQ}, {(const uint16_t*)wk[s], (float*)k, NK},
                                    {(const uint16_t*)wv[s], (float*)v, NK}};
            CK(g4_linear_f16((const float*)x, H, qkv, 3, st));
            g4_linear_seg o = {(const uint16_t*)wo[s], (float*)y, H};
            CK(g4_linear_f16((const float*)attn, NQ, &o, 1, st));
            return;
        }
        CK(g4_matmul_quant_f16((const float*)x, (const uint16_t*)wq[s], (float*)q, g4_matmul_params{NQ, H}, st));
        CK(g4_matmul_quant_f16((const float*)x, (const uint16_t*)wk[s], (float*)k, g4_matmul_params{NK, H}, st));
        CK(g4_matmul_quant_f16((const float*)x, (const uint16_t*)wv[s], (float*)v, g4_matmul_params{NK, H}, st));
        CK(g4_matmul_quant_f16((const float*)attn, (const uint16_t*)wo[s], (float*)y, g4_matmul_params{H, NQ}, st));
    };
    for (int i = 0; i < 3; i++) step(i);
    CK(g4_stream_synchronize(st));
    hipEvent_t a, b;
    HK(hipEventCreate(&a));
    HK(hipEventCreate(&b));
    HK(hipEventRecord(a, st));
    for (int i = 0; i < iters; i++) step(i);
    HK(hipEventRecord(b, st));
    HK(hipEventSynchronize(b));
    float ms = 0;
    HK(hipEventElapsedTime(&ms, a, b));
    const double us = ms * 1e3 / iters;
    printf("%s [%s]: %.2f us/step (linearQKV + linearOut), %.1f GB/s algorithmic (%d iterations)\n", wl.c_str(),
           mode.c_str(), us, bytes / (us * 1e3), iters);
    return 0;
}

struct Layer {
    unsigned seq, window, pos;
    float theta;
    unsigned divisor;
    unsigned hd = HD;  // head_dim (E2B: 256 on local layers, 512 on global layers)
    int src = -1;      // KV producer layer (E2B's shared layers); -1: its own cache
};

static std::vector<Layer> workload(const std::string& w) {
    std::vector<Layer> L;
    if (w == "stack4k" || w == "stack8k" || w == "stack32k" || w == "stack128k") {
        const unsigned pos = w == "stack4k" ? 4096 : w == "stack8k" ? 8192 : w == "stack32k" ? 32768 : 131071;
        for (int i = 0; i < 35; i++) {
            bool global = (i % 5) == 4;
            L.push_back({pos + 1, global ? 0u : 512u, pos, global ? 1e6f : 1e4f, global ? 1u : 0u});
        }
    } else if (w == "e2b8k" || w == "e2b32k") {  // the real E2B head dims: global layers at 512
        unsigned pos = w == "e2b8k" ? 8192 : 32768;
        for (int i = 0; i < 35; i++) {
            bool global = (i % 5) == 4;
            L.push_back({pos + 1, global ? 0u : 512u, pos, global ? 1e6f : 1e4f, global ? 1u : 0u, global ? 512u : 256u});
        }
    } else if (w == "e2bshared8k" || w == "e2bshared32k") {
        // E2B's cache sharing (src/config/gemma4-e2b.ts:159-178): layers 15..34 read the cache of the
        // last unshared layer of their type (13 local, 14 global) and store nothing
        unsigned pos = w == "e2bshared8k" ? 8192 : 32768;
        for (int i = 0; i < 35; i++) {
            bool global = (i % 5) == 4;
            L.push_back({pos + 1, global ? 0u : 512u, pos, global ? 1e6f : 1e4f, global ? 1u : 0u,
                         global ? 512u : 256u, i < 15 ? -1 : (global ? 14 : 13)});
        }
    } else if (w == "long128k") {
        L.push_back({131072, 0, 131071, 1e6f, 1});
    } else if (w == "long128k_hd512") {
        L.push_back({131072, 0, 131071, 1e6f, 1, 512});
    } else if (w == "layer512") {
        L.push_back({513, 512, 512, 1e4f, 0});
    } else if (w == "ragged64") {
        // lengths uniform in [1024, 32768]: lo + floor(u * (hi - lo + 1)), u the top 53 bits of
        // splitmix64 element i of stream 20261203 (the sequence bench.py draws)
        const uint64_t seed = 20261203;
        for (uint64_t i = 1; i <= 64; i++) {
            uint64_t z = seed + i * 0x9E3779B97F4A7C15ull;
            z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
            z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
            z ^= z >> 31;
            const double u = (double)(z >> 11) * (1.0 / 9007199254740992.0);
            const unsigned len = 1024 + (unsigned)floor(u * (32768 - 1024 + 1));
            L.push_back({len, 0, len - 1, 1e6f, 1});
        }
    } else {
        fprintf(stderr, "unknown workload %s\n", w.c_str());
        exit(2);
    }
    return L;
}

// Causal prefill of a 4096-token prompt: one global and one W=512 local layer.
static int run_prefill(const std::string& wl, const std::string& mode, int iters) {
    const unsigned T = 4096, CH = mode == "whole" ? 4096 : 512, NQ = NQH, NK = NKH;
    // prefill4k512: the global layer alone at head_dim 512 (E2B's global layers)
    const unsigned hd = wl == "prefill4k512" ? 512u : (unsigned)HD;
    const int n_layers = wl == "prefill4k512" ? 1 : 2;
    hipStream_t st;
    HK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    std::vector<g4_prefill_entry> ents;
    double flops = 0;
    for (int layer = 0; layer < n_layers; layer++) {
        const unsigned window = layer ? 512u : 0u;
        void *q, *kc, *vc, *out;
        CK(g4_malloc(&q, (size_t)T * NQ * hd * 2));
        CK(g4_malloc(&kc, (size_t)T * NK * hd * 2));
        CK(g4_malloc(&vc, (size_t)T * NK * hd * 2));
        CK(g4_malloc(&out, (size_t)T * NQ * hd * 4));
        hipLaunchKernelGGL(k_fill_f16, dim3(1024), dim3(256), 0, st, (_Float16*)q, (uint64_t)T * NQ * hd, 11u + layer);
        hipLaunchKernelGGL(k_fill_f16, dim3(1024), dim3(256), 0, st, (_Float16*)kc, (uint64_t)T * NK * hd, 21u + layer);
        hipLaunchKernelGGL(k_fill_f16, dim3(1024), dim3(256), 0, st, (_Float16*)vc, (uint64_t)T * NK * hd, 31u + layer);
        for (unsigned c0 = 0; c0 < T; c0 += CH) {
            g4_prefill_entry e = {(const uint16_t*)q + (size_t)c0 * NQ * hd, (const uint16_t*)kc, (const uint16_t*)vc,
                                  (float*)out + (size_t)c0 * NQ * hd, CH, c0, window, 1.0f};
            ents.push_back(e);
        }
        for (unsigned i = 0; i < T; i++) flops += 4.0 * hd * NQ * (window && i + 1 > window ? window : i + 1);
    }
    HK(hipGetLastError());
    size_t ws_bytes = 0;
    CK(g4_attn_prefill_workspace_size(ents.data(), (uint32_t)ents.size(), NQ, NK, hd, &ws_bytes));
    void* ws;
    CK(g4_malloc(&ws, ws_bytes ? ws_bytes : 256));
    g4_decode_plan plan;
    CK(g4_attn_prefill_prepare(ents.data(), (uint32_t)ents.size(), NQ, NK, hd, ws, ws_bytes, &plan, st));
    for (int i = 0; i < 3; i++) CK(g4_attn_prefill_run(&plan, st));
    CK(g4_stream_synchronize(st));
    hipEvent_t a, b;
    HK(hipEventCreate(&a));
    HK(hipEventCreate(&b));
    HK(hipEventRecord(a, st));
    for (int i = 0; i < iters; i++) CK(g4_attn_prefill_run(&plan, st));
    HK(hipEventRecord(b, st));
    HK(hipEventSynchronize(b));
    float ms = 0;
    HK(hipEventElapsedTime(&ms, a, b));
    const double us = ms * 1e3 / iters;
    printf("flops_per_step: %.0f\n", flops);
    printf("%s [%s]: %zu entries, %.2f us/step, %.1f TFLOP/s algorithmic (%d iterations)\n", wl.c_str(), mode.c_str(),
           ents.size(), us, flops / (us * 1e-6) / 1e12, iters);
    return 0;
}

int main(int argc, char** argv) {
    std::string wl = "stack8k", mode = "step";
    int iters = 50, sets = 0;
    for (int i = 1; i < argc; i++) {
        if (!strcmp(argv[i], "--workload") && i + 1 < argc) wl = argv[++i];
        else if (!strcmp(argv[i], "--iters") && i + 1 < argc) iters = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--sets") && i + 1 < argc) sets = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--mode") && i + 1 < argc) mode = argv[++i];
        else {
            fprintf(stderr, "usage: g4bench [--workload W] [--mode step|unfused] [--iters N] [--sets S]\n");
            return 2;
        }
    }
    CK(g4_set_device(0));
    if (wl == "copy") return run_copy(iters);
    if (wl == "prefill4k" || wl == "prefill4k512") return run_prefill(wl, mode, iters);
    if (wl == "lmhead") return run_lmhead(mode, iters);
    if (wl == "proj256" || wl == "proj512") return run_proj(wl, mode, iters, sets);
    std::vector<Layer> L = workload(wl);
    const bool uniform_pos = wl.rfind("stack", 0) == 0 || L.size() == 1;
    uint64_t step_bytes = 0, total_rows = 0;
    for (auto& l : L) {
        unsigned att = l.window && l.seq > l.window ? l.window : l.seq;
        total_rows += att;
        step_bytes += 2ull * att * NKH * l.hd * 2 + NQH * l.hd * 4 * 2;
    }
    bool all256 = true;
    for (auto& l : L) all256 = all256 && l.hd == HD;
    // Token loops (the position advances every token; every plan is re-prepared inside the timed region):
    // loop: one step per head_dim group per token; layers: the engine's order, every layer's plan from one
    // g4_attn_step_prepare_layers per head_dim group, then layer by layer attention + merge; layers_each:
    // the same order with one g4_attn_step_prepare per layer.
    // chain / chain_each: the same two orders with the layer's projections around its attention (q/k/v in
    // one g4_linear_f16 launch, then o_proj with the merge folded in, g4_attn_step_run_out; f16 weights of
    // E2B's shapes, hidden 1536, distinct per layer), as the engine runs a token.
    // advance / layers_adv / chain_adv: loop / layers / chain with the plans advanced every token
    // (g4_attn_step_advance, host only) and prepared again every kReplan tokens.
    const std::string mode_name = mode;
    const bool advancing = mode == "advance" || mode == "layers_adv" || mode == "chain_adv";
    if (advancing) mode = mode == "advance" ? "loop" : mode == "layers_adv" ? "layers" : "chain";
    constexpr int kReplan = 32;
    const bool chain = mode == "chain" || mode == "chain_each";
    const bool token_loop = mode == "loop" || mode == "layers" || mode == "layers_each" || chain;
    if (mode != "step" && !token_loop && !all256) {
        fprintf(stderr, "workload %s: head_dim 512 layers run on the fused step only (--mode step)\n", wl.c_str());
        return 2;
    }
    if (sets <= 0) sets = step_bytes >= (64ull << 20) ? (int)((512ull << 20) / step_bytes) + 1 : 1;
    printf("workload %s: %zu entries, %.1f MB/step, %d sets\n", wl.c_str(), L.size(), step_bytes / 1e6, sets);
    printf("bytes_per_step: %llu\n", (unsigned long long)step_bytes);

    hipStream_t st;
    HK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    std::vector<uint16_t> rf(256), ones(512, 0x3C00);
    for (int i = 0; i < 256; i++) rf[i] = i < 64 ? 0x3C00 : 0x7C00;
    void *d_rf, *d_ones;
    std::vector<float> h_inv[2][2];  // [head_dim 256 / 512][local theta 1e4 / global 1e6 with divisor]
    CK(g4_malloc(&d_rf, 512));
    CK(g4_malloc(&d_ones, 512 * 2));
    CK(g4_upload(d_rf, 0, rf.data(), 512, st));
    CK(g4_upload(d_ones, 0, ones.data(), 512 * 2, st));
    for (int h = 0; h < 2; h++)
        for (int i = 0; i < 2; i++) {
            const unsigned hd = h ? 512 : 256;
            h_inv[h][i].resize(hd / 2);
            CK(g4_rope_inv_freq_host(i ? 1e6f : 1e4f, hd, i, rf.data(), h_inv[h][i].data()));
        }

    struct Set {
        std::vector<void*> bufs;
        std::vector<g4_step_entry> steps[2];     // the step's entries per head_dim group (token loops bump them)
        std::vector<std::pair<int, int>> order;  // layer -> (head_dim group, index in the group)
        void* layers_ws[2] = {nullptr, nullptr};
        size_t layers_ws_bytes[2] = {0, 0};
        std::vector<g4_decode_plan> layer_plans[2];
        std::vector<void*> wqkv, wo, y;  // chain modes: per layer q/k/v weight rows, o_proj weight, o_proj output
        void* x = nullptr;               // the layers' input (hidden 1536)
        g4_decode_plan plan;          // unfused: prep + split + merge
        g4_decode_plan step_plan[2];  // one-launch step per head_dim group (256, 512)
        bool has_step[2] = {false, false};
        void* ws = nullptr;
        void* step_ws[2] = {nullptr, nullptr};
        void* prep_table = nullptr;
        int since_prepare = -1;  // tokens since the last prepare (-1: never prepared)
    };
    std::vector<Set> S(sets);
    size_t ws_bytes = 0;
    if (all256) CK(g4_attn_decode_many_workspace_size((uint32_t)L.size(), NQH, NKH, HD, total_rows, &ws_bytes));
    uint64_t seed = 1;
    const unsigned extra_rows = token_loop ? (unsigned)(iters / sets + 8) : 0;  // rows the loop's tokens append
    for (int s = 0; s < sets; s++) {
        std::vector<g4_decode_entry> ents;
        std::vector<g4_prep_layer> preps;
        std::vector<g4_step_entry>* steps = S[s].steps;
        std::vector<void*> lkc(L.size()), lvc(L.size()), lk(L.size()), lv(L.size());
        for (size_t li = 0; li < L.size(); li++) {
            const Layer& l = L[li];
            void *kc, *vc, *q, *k, *v, *out;
            const unsigned hd = l.hd;
            const size_t cache_bytes = (size_t)(l.seq + extra_rows) * NKH * hd * 2;
            CK(g4_malloc(&q, NQH * hd * 4));
            CK(g4_malloc(&out, NQH * hd * 4));
            hipLaunchKernelGGL(k_fill_f32, dim3(8), dim3(256), 0, st, (float*)q, (uint64_t)NQH * hd, seed++);
            if (l.src >= 0) {  // a consumer: the producer's cache and raw k/v (the row is recomputed)
                kc = lkc[l.src];
                vc = lvc[l.src];
                k = lk[l.src];
                v = lv[l.src];
                S[s].bufs.insert(S[s].bufs.end(), {q, out});
            } else {
                CK(g4_malloc(&kc, cache_bytes));
                CK(g4_malloc(&vc, cache_bytes));
                CK(g4_malloc(&k, NKH * hd * 4));
                CK(g4_malloc(&v, NKH * hd * 4));
                hipLaunchKernelGGL(k_fill_f16, dim3(1024), dim3(256), 0, st, (_Float16*)kc, (uint64_t)cache_bytes / 2,
                                   seed++);
                hipLaunchKernelGGL(k_fill_f16, dim3(1024), dim3(256), 0, st, (_Float16*)vc, (uint64_t)cache_bytes / 2,
                                   seed++);
                hipLaunchKernelGGL(k_fill_f32, dim3(2), dim3(256), 0, st, (float*)k, (uint64_t)NKH * hd, seed++);
                hipLaunchKernelGGL(k_fill_f32, dim3(2), dim3(256), 0, st, (float*)v, (uint64_t)NKH * hd, seed++);
                S[s].bufs.insert(S[s].bufs.end(), {kc, vc, q, k, v, out});
            }
            lkc[li] = kc;
            lvc[li] = vc;
            lk[li] = k;
            lv[li] = v;
            ents.push_back({(const float*)q, (const uint16_t*)kc, (const uint16_t*)vc, (float*)out, l.seq, l.window,
                            1.0f, 0});
            g4_prep_layer p = {};
            p.q = (float*)q;
            p.k = (float*)k;
            p.v = (float*)v;
            p.q_weight = p.k_weight = (const uint16_t*)d_ones;
            p.rope_freqs = (const uint16_t*)d_rf;
            p.k_cache = (uint16_t*)kc;
            p.v_cache = (uint16_t*)vc;
            p.head_dim = HD;
            p.theta = l.theta;
            p.apply_divisor = l.divisor;
            p.store_kv = 1;
            p.max_seq_len = l.seq;
            preps.push_back(p);
            g4_step_entry se = {};
            se.q = (const float*)q;
            se.k = (const float*)k;
            se.v = (const float*)v;
            se.q_weight = se.k_weight = (const uint16_t*)d_ones;
            se.rope_freqs = (const uint16_t*)d_rf;
            se.rope_inv_freq_host = h_inv[hd == 512 ? 1 : 0][l.divisor ? 1 : 0].data();
            se.k_cache = (uint16_t*)kc;
            se.v_cache = (uint16_t*)vc;
            se.out = (float*)out;
            se.seq_len = l.seq;
            se.position = l.pos;
            se.sliding_window = l.window;
            se.store_kv = l.src >= 0 ? 0 : 1;
            se.theta = l.theta;
            se.apply_divisor = l.divisor;
            se.scale = 1.0f;
            se.eps = 1e-6f;
            if (chain) {  // q, k, v weight rows [(NQH + 2 NKH) hd][1536] and o_proj [1536][NQH hd], f16
                void *wq, *wov, *yv;
                const size_t qkv_bytes = (size_t)(NQH + 2 * NKH) * hd * kHidden * 2;
                const size_t o_bytes = (size_t)kHidden * NQH * hd * 2;
                CK(g4_malloc(&wq, qkv_bytes));
                CK(g4_malloc(&wov, o_bytes));
                CK(g4_malloc(&yv, kHidden * 4));
                hipLaunchKernelGGL(k_fill_f16, dim3(1024), dim3(256), 0, st, (_Float16*)wq, (uint64_t)qkv_bytes / 2, seed++);
                hipLaunchKernelGGL(k_fill_f16, dim3(1024), dim3(256), 0, st, (_Float16*)wov, (uint64_t)o_bytes / 2, seed++);
                S[s].wqkv.push_back(wq);
                S[s].wo.push_back(wov);
                S[s].y.push_back(yv);
                S[s].bufs.insert(S[s].bufs.end(), {wq, wov, yv});
            }
            S[s].order.emplace_back(hd == 512 ? 1 : 0, (int)steps[hd == 512 ? 1 : 0].size());
            steps[hd == 512 ? 1 : 0].push_back(se);
        }
        HK(hipGetLastError());
        if (chain) {
            CK(g4_malloc(&S[s].x, kHidden * 4));
            hipLaunchKernelGGL(k_fill_f32, dim3(2), dim3(256), 0, st, (float*)S[s].x, (uint64_t)kHidden, seed++);
            S[s].bufs.push_back(S[s].x);
        }
        if (all256) {
            CK(g4_malloc(&S[s].ws, ws_bytes));
            CK(g4_malloc(&S[s].prep_table, preps.size() * sizeof(g4_prep_layer)));
            CK(g4_upload(S[s].prep_table, 0, preps.data(), preps.size() * sizeof(g4_prep_layer), st));
            CK(g4_attn_decode_many_prepare(ents.data(), (uint32_t)ents.size(), NQH, NKH, HD, S[s].ws, ws_bytes,
                                           &S[s].plan, st));
        }
        for (int h = 0; h < 2; h++) {  // one step per head_dim group (E2B: local layers, then global layers)
            if (steps[h].empty()) continue;
            const unsigned hd = h ? 512 : 256;
            size_t b = 0;
            CK(g4_attn_step_workspace_size((uint32_t)steps[h].size(), NQH, NKH, hd, &b));
            CK(g4_malloc(&S[s].step_ws[h], b));
            CK(g4_attn_step_prepare(steps[h].data(), (uint32_t)steps[h].size(), NQH, NKH, hd, S[s].step_ws[h], b,
                                    &S[s].step_plan[h], st));
            S[s].has_step[h] = true;
            if (token_loop) {
                CK(g4_attn_step_layers_workspace_size((uint32_t)steps[h].size(), 1, NQH, NKH, hd,
                                                      &S[s].layers_ws_bytes[h]));
                CK(g4_malloc(&S[s].layers_ws[h], S[s].layers_ws_bytes[h]));
                S[s].layer_plans[h].resize(steps[h].size());
            }
        }
    }
    CK(g4_stream_synchronize(st));

    const bool fused = mode == "step";
    // mode graph: each set's step (attention launch + merge launch) captured once as a HIP graph
    // and replayed; the plans' work tables are the same device memory, so replays read them.
    std::vector<hipGraphExec_t> gexec(sets, nullptr);
    if (mode == "graph") {
        for (int si = 0; si < sets; si++) {
            hipGraph_t g;
            HK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
            for (int h = 0; h < 2; h++)
                if (S[si].has_step[h]) CK(g4_attn_step_run(&S[si].step_plan[h], st));
            HK(hipStreamEndCapture(st, &g));
            HK(hipGraphInstantiate(&gexec[si], g, nullptr, nullptr, 0));
            HK(hipGraphDestroy(g));
        }
    }
    auto step = [&](int i) {
        Set& s = S[i % sets];
        if (token_loop) {
            for (int h = 0; h < 2; h++)
                for (g4_step_entry& e : s.steps[h]) {
                    e.seq_len++;
                    e.position++;
                }
            const bool replan = !advancing || s.since_prepare < 0 || s.since_prepare + 1 >= kReplan;
            s.since_prepare = replan ? 0 : s.since_prepare + 1;
            for (int h = 0; h < 2 && !replan; h++) {  // the next token of the prepared plans, on the host
                if (!s.has_step[h]) continue;
                if (mode == "loop") {
                    CK(g4_attn_step_advance(&s.step_plan[h], 1));
                    CK(g4_attn_step_run(&s.step_plan[h], st));
                } else {
                    for (g4_decode_plan& p : s.layer_plans[h]) CK(g4_attn_step_advance(&p, 1));
                }
            }
            for (int h = 0; h < 2 && replan; h++) {
                if (!s.has_step[h]) continue;
                const unsigned hd = h ? 512 : 256;
                const uint32_t n = (uint32_t)s.steps[h].size();
                if (mode == "loop") {
                    size_t b = 0;
                    CK(g4_attn_step_workspace_size(n, NQH, NKH, hd, &b));
                    CK(g4_attn_step_prepare(s.steps[h].data(), n, NQH, NKH, hd, s.step_ws[h], b, &s.step_plan[h], st));
                    CK(g4_attn_step_run(&s.step_plan[h], st));
                } else if (mode == "layers" || mode == "chain") {
                    CK(g4_attn_step_prepare_layers(s.steps[h].data(), n, 1, NQH, NKH, hd, s.layers_ws[h],
                                                   s.layers_ws_bytes[h], s.layer_plans[h].data(), st));
                }
            }
            if (mode == "loop") return;
            for (size_t li = 0; li < s.order.size(); li++) {  // the engine's layer order
                const auto& o = s.order[li];
                const unsigned hd = o.first ? 512 : 256;
                g4_decode_plan& plan = s.layer_plans[o.first][o.second];
                const g4_step_entry& se = s.steps[o.first][o.second];
                if (mode == "layers_each" || mode == "chain_each") {
                    const size_t one = s.layers_ws_bytes[o.first] / s.steps[o.first].size();
                    CK(g4_attn_step_prepare(&se, 1, NQH, NKH, hd, (char*)s.layers_ws[o.first] + (size_t)o.second * one,
                                            one, &plan, st));
                }
                if (chain) {  // attn.linearQKV (a consumer that recomputes its producer's row projects q/k/v too)
                    const uint16_t* w = (const uint16_t*)s.wqkv[li];
                    const g4_linear_seg segs[3] = {
                        {w, (float*)se.q, NQH * hd},
                        {w + (size_t)NQH * hd * kHidden, (float*)se.k, NKH * hd},
                        {w + (size_t)(NQH + NKH) * hd * kHidden, (float*)se.v, NKH * hd}};
                    CK(g4_linear_f16((const float*)s.x, kHidden, segs, se.store_kv ? 3u : 1u, st));
                }
                CK(g4_attn_step_run_attention(&plan, st));
                if (chain) {
                    const g4_linear_seg out = {(const uint16_t*)s.wo[li], (float*)s.y[li], kHidden};
                    CK(g4_attn_step_run_out(&plan, &out, 1, st));  // attn.linearOut with the merge folded in
                } else {
                    CK(g4_attn_step_run_merge(&plan, st));
                }
            }
            return;
        }
        if (mode == "graph") {
            HK(hipGraphLaunch(gexec[i % sets], st));
            return;
        }
        if (fused) {
            for (int h = 0; h < 2; h++)
                if (s.has_step[h]) CK(g4_attn_step_run(&s.step_plan[h], st));
            return;
        }
        if (uniform_pos) CK(g4_attn_prep_many((const g4_prep_layer*)s.prep_table, (uint32_t)L.size(), NQH, NKH, 1e-6f,
                                              L[0].pos, L[0].pos, st));
        CK(g4_attn_decode_many_run_split(&s.plan, st));
        CK(g4_attn_decode_many_run_merge(&s.plan, st));
    };
    const int warm = token_loop ? sets : 5;  // token loops: every set once (its positions advance per use)
    for (int i = 0; i < warm; i++) step(i);
    CK(g4_stream_synchronize(st));
    hipEvent_t a, b;
    HK(hipEventCreate(&a));
    HK(hipEventCreate(&b));
    HK(hipEventRecord(a, st));
    for (int i = 0; i < iters; i++) step(warm + i);
    HK(hipEventRecord(b, st));
    HK(hipEventSynchronize(b));
    float ms = 0;
    HK(hipEventElapsedTime(&ms, a, b));
    const double us = ms * 1e3 / iters;
    printf("%s [%s]: %.2f us/step, %.1f GB/s algorithmic (%d iterations)\n", wl.c_str(), mode_name.c_str(), us,
           step_bytes / (us * 1e3), iters);
    return 0;
}
