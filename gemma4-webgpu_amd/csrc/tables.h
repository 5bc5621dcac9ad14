// Work tables the host builds and the decode kernels read as they are: plain
// data, no HIP, so that the host-side planner (step_plan.h) also builds and
// runs in CPU-only test programs.
#pragma once

#include <stdint.h>

namespace g4 {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kTileKeys = 32;  // rows per decode tile
constexpr int kMaxGroup = 8;   // query heads per kv head served by one MFMA column block

// One problem of the split decode, or one entry of a merge table.
struct DecodeEntryDev {
    const float* q;       // [num_kv_heads][group][HD]
    const uint16_t* k;    // [rows][num_kv_heads][HD]
    const uint16_t* v;
    float* out;           // [num_kv_heads][group][HD]
    uint32_t key_begin;   // first attended row
    uint32_t key_end;     // one past the last attended row
    uint32_t split_base;  // first split index (partial record slot) of this entry
    uint32_t n_splits;
    float qscale;         // attention scale * log2(e)
    uint32_t pad;
};

// One entry of the one-launch decode step.
struct StepEntryDev {
    const float* q;  // raw projections, [num_kv_heads][group][HD] and [num_kv_heads][HD]
    const float* k;
    const float* v;
    const uint16_t* q_weight;
    const uint16_t* k_weight;
    const uint16_t* rope_freqs;
    const float* rope_cs;  // RoPE factors of this token [cos x HD/2][sin x HD/2] (host-computed), or nullptr
    uint16_t* k_cache;  // [rows][num_kv_heads][HD]
    uint16_t* v_cache;
    float* out;         // attnOut [num_kv_heads][group][HD]
    uint32_t key_end;   // one past the last attended row; the current row is key_end - 1
    uint32_t n_parts;   // workgroups on this entry
    uint32_t position;  // RoPE position
    uint32_t flags;     // kStoreKv | kRowCached
    float theta;
    uint32_t apply_divisor;
    float qscale;       // attention scale * log2(e)
    float eps;
};

constexpr uint32_t kStoreKv = 1;    // write the current row's k and v to the caches
constexpr uint32_t kRowCached = 2;  // the current row is already in the cache: read it like the others

// One workgroup's share: attended rows [row_begin, row_end) of entry `entry`,
// with a copy of the entry, so that a workgroup's first loads depend on one
// batch of scalar loads (a kernel starts with cold caches: each dependent
// load in that chain costs a memory round trip).
struct StepWorkDev {
    StepEntryDev ent;
    uint32_t row_begin;
    uint32_t row_end;
    uint32_t part;   // partial record slot, when the entry has more than one workgroup
    uint32_t entry;
};
static_assert(sizeof(StepWorkDev) == 128, "work item size");

}  // namespace g4
