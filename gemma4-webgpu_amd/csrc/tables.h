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
    const float* rope_cs;  // RoPE set of this token: [cos x HD/2][sin x HD/2] at `position` (host-computed),
                           // then the inverse frequencies [HD/2] (for later positions); or nullptr
    uint16_t* k_cache;  // [rows][num_kv_heads][HD]
    uint16_t* v_cache;
    float* out;         // attnOut [num_kv_heads][group][HD]
    uint32_t key_end;   // one past the last attended row; the current row is key_end - 1
    uint32_t n_parts;   // workgroups on this entry
    uint32_t position;  // RoPE position
    uint32_t flags;     // kStoreKv | kRowCached | kApplyDivisor
    float theta;
    uint32_t window;    // sliding window (0 = full): rows [key_end - window, key_end) when key_end > window
    float qscale;       // attention scale * log2(e)
    float eps;
};

constexpr uint32_t kStoreKv = 1;       // write the current row's k and v to the caches
constexpr uint32_t kRowCached = 2;     // the current row is already in the cache: read it like the others
constexpr uint32_t kApplyDivisor = 4;  // RoPE frequencies divided by rope_freqs (global layers)
constexpr uint32_t kQReady = 8;        // q holds the post-norm, post-RoPE query: read as is

// First attended row of an entry whose rows end at key_end. (constexpr: the
// kernels and the host planner share these.)
inline constexpr uint32_t step_key_begin(uint32_t key_end, uint32_t window) {
    return window != 0 && key_end > window ? key_end - window : 0u;
}

// Rows [begin, end) of a part planned as [row_begin, row_end) of an entry
// ending at key_end, once the plan is advanced by `adv` tokens: the part moves
// with the entry's first attended row, and the part that held the last row
// extends to the new end.
struct StepRows {
    uint32_t begin, end;
};
inline constexpr StepRows step_part_rows(uint32_t row_begin, uint32_t row_end, uint32_t key_end, uint32_t window,
                                         uint32_t adv) {
    const uint32_t shift = step_key_begin(key_end + adv, window) - step_key_begin(key_end, window);
    return StepRows{row_begin + shift, row_end == key_end ? key_end + adv : row_end + shift};
}

// One workgroup's share: attended rows [row_begin, row_end) of entry `entry`,
// with a copy of the entry, so that a workgroup's first loads depend on one
// batch of scalar loads (a kernel starts with cold caches: each dependent
// load in that chain costs a memory round trip). The rows are those of the
// token the plan was prepared for. A plan advanced by `a` tokens keeps its
// parts: the entry ends at key_end + a, every part moves with the entry's
// first attended row (by step_key_begin(key_end + a) - step_key_begin(key_end):
// 0 on full layers, up to a on windowed ones), and the part holding the last
// row (row_end == key_end) extends to the new end.
struct StepWorkDev {
    StepEntryDev ent;
    uint32_t row_begin;
    uint32_t row_end;
    uint32_t part;   // partial record slot, when the entry has more than one workgroup
    uint32_t entry;
};
static_assert(sizeof(StepWorkDev) == 128, "work item size");

}  // namespace g4
