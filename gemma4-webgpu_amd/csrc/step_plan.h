// Host-side planning of the one-launch decode step (step.hip): argument
// checks, the partition of every entry's attended rows into workgroups, the
// merge table, the token's RoPE factors and the workspace layout. Plain C++
// (no HIP), so the same code runs in CPU-only test programs.
//
// Partition: each entry's attended rows become 32-row tiles; the planner
// picks the smallest tiles-per-workgroup such that the entries' workgroups
// (sum over entries of ceil(tiles / tpw)) fit one wave of the GPU, and cuts
// each entry into that many balanced, contiguous row ranges. A workgroup never
// spans two entries. An entry cut into more than one part writes partial
// records, listed in the merge table for the log-sum-exp merge launch.
#pragma once

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <utility>
#include <vector>

#include "../../include/g4attn.h"
#include "tables.h"

namespace g4 {

// Partial records: an entry gets more than one workgroup only while the
// workgroups fit one wave of the GPU (at most kStepMaxWgs), so at most that
// many records exist.
constexpr unsigned kStepMaxWgs = 1024;
constexpr unsigned kStepOneWgTiles = 16;  // one workgroup per CU up to this many tiles each

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Floats of one RoPE set in the tables region: the factors at the plan's
// position [cos x hd/2][sin x hd/2], then the inverse frequencies [hd/2] that
// the kernel evaluates later positions from (advanced plans).
inline constexpr uint64_t rope_set_floats(uint64_t hd) { return hd + hd / 2; }

// The tables region holds, packed by each prepare and uploaded in one copy,
// the work table, the merge table, the entry table (every entry's attnOut and
// records, read by the merge folded into the output projection) and the RoPE
// factors (their offsets are in the plan); the partial records follow at a
// fixed offset.
struct StepLayout {
    size_t tables, part_ml, part_o, total;
};

// Bytes from a plan's (m, l) records to its o rows.
inline size_t step_part_o_offset(uint64_t nkh, uint64_t group) {
    return align256((uint64_t)kStepMaxWgs * nkh * group * 2 * 4);
}

inline StepLayout step_layout(uint64_t n, uint64_t nkh, uint64_t group, uint64_t hd) {
    StepLayout L;
    const uint64_t max_items = n > kStepMaxWgs ? n : kStepMaxWgs;
    const uint64_t recs = (uint64_t)kStepMaxWgs * nkh * group;
    size_t off = 0;
    L.tables = off;  // work items, merge entries, all entries, and at most one RoPE set per entry
    off += align256(max_items * sizeof(StepWorkDev)) + 2 * align256(n * sizeof(DecodeEntryDev)) +
           align256(n * rope_set_floats(hd) * 4);
    L.part_ml = off;
    off += step_part_o_offset(nkh, group);
    L.part_o = off;
    off += align256(recs * hd * 4);
    L.total = off;
    return L;
}

// Smallest tiles-per-workgroup with sum_e ceil(tiles_e / tpw) <= cap (cap >= n,
// so tpw = max tiles always fits).
inline uint64_t pick_tiles_per_wg(const std::vector<uint32_t>& tiles, uint64_t total, uint64_t max_tiles,
                                  uint64_t cap) {
    auto wgs = [&](uint64_t tpw) {
        uint64_t s = 0;
        for (uint32_t t : tiles) s += (t + tpw - 1) / tpw;
        return s;
    };
    uint64_t lo = (total + cap - 1) / cap, hi = max_tiles;
    if (lo < 1) lo = 1;
    if (lo > hi) lo = hi;
    while (lo < hi) {
        const uint64_t mid = (lo + hi) / 2;
        if (wgs(mid) <= cap) hi = mid;
        else lo = mid + 1;
    }
    return lo;
}

// Overrides of the grid choice (0 = the default rule; the library passes the
// defaults, the planner's checks and experiments others).
struct StepTuning {
    int waves = 0;       // 4 or 8 waves per workgroup (head_dim 256)
    int wgs_per_cu = 0;  // workgroups per CU
    int max_wgs = 0;     // cap on the workgroups of the launch
};

struct StepPlanHost {
    uint32_t waves = 0;      // waves per workgroup of the attention kernel
    uint32_t n_wgs = 0;      // workgroups (work items)
    uint32_t n_merge = 0;    // entries in the merge table
    uint32_t max_parts = 0;  // largest part count of an entry
    uint32_t parts = 0;      // partial-record slots in use
    size_t off_merge = 0;    // byte offsets in the tables blob
    size_t off_ents = 0;
    size_t off_rope = 0;
    std::vector<char> blob;  // work table | merge table | entry table | RoPE factors, ready to upload to the tables region
    // Working storage of plan_step, kept with the blob between calls: a decode
    // loop that plans every token allocates nothing once its step stops growing.
    std::vector<StepEntryDev> tab;
    std::vector<uint32_t> key_begin, tiles, rope_idx, rope_slot;
    std::vector<std::pair<const float*, uint32_t>> rope_keys;
    std::vector<const float*> rope_dev;  // device address of each distinct pair's factors
    std::vector<uint32_t> rope_set;      // its set in this blob, or ~0 when an earlier plan placed it
};

// Hash of an (inverse-frequency table, position) pair.
inline uint64_t rope_key_hash(const float* table, uint32_t position) {
    return (reinterpret_cast<uintptr_t>(table) >> 4) * 0x9E3779B97F4A7C15ull ^ position * 0xC2B2AE3D27D4EB4Full;
}

// RoPE factor sets already placed by the earlier plans of one upload (the
// layers of a token planned one by one): a later plan that needs the same
// (inverse-frequency table, position) pair points at that set instead of
// carrying its own. Looked up through open addressing (slot: 0 = empty, else
// index + 1; at least twice as many slots as keys), so a batched prepare of
// many sequences and layers stays linear in its entries.
struct StepRopeShare {
    std::vector<std::pair<const float*, uint32_t>> keys;
    std::vector<const float*> dev;
    std::vector<uint32_t> slot;
    void clear() {
        keys.clear();
        dev.clear();
        slot.assign(64, 0u);
    }
    const float* find(const std::pair<const float*, uint32_t>& k) const {
        if (slot.empty()) return nullptr;
        const size_t mask = slot.size() - 1;
        for (size_t i = (size_t)(rope_key_hash(k.first, k.second) >> 32) & mask;; i = (i + 1) & mask) {
            const uint32_t v = slot[i];
            if (!v) return nullptr;
            if (keys[v - 1] == k) return dev[v - 1];
        }
    }
    void add(const std::pair<const float*, uint32_t>& k, const float* d) {
        if (2 * (keys.size() + 1) > slot.size()) {  // grow, then re-insert every key
            slot.assign(slot.empty() ? 64 : 2 * slot.size(), 0u);
            for (size_t j = 0; j < keys.size(); j++) place(j);
        }
        keys.push_back(k);
        dev.push_back(d);
        place(keys.size() - 1);
    }

  private:
    void place(size_t j) {
        const size_t mask = slot.size() - 1;
        size_t i = (size_t)(rope_key_hash(keys[j].first, keys[j].second) >> 32) & mask;
        while (slot[i]) i = (i + 1) & mask;
        slot[i] = (uint32_t)j + 1;
    }
};

// The token's RoPE factors c[p] = f32(cos(a_p)), c[half + p] = f32(sin(a_p))
// with a_p = f32(pos * inv[p]), cos and sin evaluated in f64: bit-identical to
// (float)cos((double)a) and (float)sin((double)a) of the C library.
//
// Each pair comes from one Cody-Waite reduction a = k pi/2 + r (pi/2 in
// three parts of 33, 33 and 53 bits: k P1 and k P2 are exact for |k| < 2^20)
// and Taylor polynomials on |r| <= pi/4 (next terms below 2^-62 relative), a
// few f64 ulps from the exact value. The C library is within one ulp of it,
// so wherever the interval d +- 2^-46 |d| around this value rounds to one f32,
// both round to that f32; the rare value near an f32 rounding boundary, and
// any angle beyond 2^20 or not finite, is taken from the C library instead.
inline void rope_factors(const float* inv, uint32_t pos, uint32_t half, float* c) {
    constexpr double kTwoOverPi = 0x1.45f306dc9c883p-1;
    constexpr double kP1 = 0x1.921fb544p+0, kP2 = 0x1.0b4611a6p-34, kP3 = 0x1.3198a2e037073p-69;
    constexpr double kRound = 0x1.8p52;  // adding and subtracting it rounds to an integer (|x| < 2^51)
    float* s = c + half;
    uint8_t sure[256];  // half <= 256; a branch-free first pass, then the C library where unsure
    uint32_t unsure = 0;
    for (uint32_t p = 0; p < half; p++) {
        const double x = (double)((float)pos * inv[p]);
        const double kr = x * kTwoOverPi + kRound;
        const double k = kr - kRound;
        uint64_t kb;
        memcpy(&kb, &kr, 8);
        const double r = ((x - k * kP1) - k * kP2) - k * kP3;
        const double z = r * r;
        const double sr =
            r + r * z *
                    (-1.0 / 6 +
                     z * (1.0 / 120 +
                          z * (-1.0 / 5040 +
                               z * (1.0 / 362880 +
                                    z * (-1.0 / 39916800 +
                                         z * (1.0 / 6227020800 +
                                              z * (-1.0 / 1307674368000 + z * (1.0 / 355687428096000))))))));
        const double cr =
            1.0 + z * (-0.5 +
                       z * (1.0 / 24 +
                            z * (-1.0 / 720 +
                                 z * (1.0 / 40320 +
                                      z * (-1.0 / 3628800 +
                                           z * (1.0 / 479001600 +
                                                z * (-1.0 / 87178291200 +
                                                     z * (1.0 / 20922789888000 + z * (-1.0 / 6402373705728000)))))))));
        const uint64_t q = kb & 3u;  // quadrant: a = k pi/2 + r
        const double sv = q & 1 ? cr : sr, cv = q & 1 ? sr : cr;
        const double sin_a = q & 2 ? -sv : sv;
        const double cos_a = (q + 1) & 2 ? -cv : cv;
        const double es = 0x1p-46 * fabs(sin_a), ec = 0x1p-46 * fabs(cos_a);
        const bool ok = fabs(x) <= 0x1p20 && (float)(sin_a - es) == (float)(sin_a + es) &&
                        (float)(cos_a - ec) == (float)(cos_a + ec);
        c[p] = (float)cos_a;
        s[p] = (float)sin_a;
        sure[p] = ok;
        unsure += !ok;
    }
    if (unsure)
        for (uint32_t p = 0; p < half; p++)
            if (!sure[p]) {
                const double x = (double)((float)pos * inv[p]);
                c[p] = (float)cos(x);
                s[p] = (float)sin(x);
            }
}

// Index of the (inverse-frequency table, position) pair among the distinct
// pairs seen so far, in order of first appearance (a new pair is appended).
// Open addressing over `slot` (a power of two, at least twice the pairs; 0 =
// empty, else index + 1).
inline uint32_t rope_pair_index(StepPlanHost& ph, const float* table, uint32_t position) {
    const uint64_t h = rope_key_hash(table, position);
    const size_t mask = ph.rope_slot.size() - 1;
    for (size_t i = (size_t)(h >> 32) & mask;; i = (i + 1) & mask) {
        const uint32_t v = ph.rope_slot[i];
        if (!v) {
            ph.rope_keys.emplace_back(table, position);
            ph.rope_slot[i] = (uint32_t)ph.rope_keys.size();
            return (uint32_t)ph.rope_keys.size() - 1;
        }
        if (ph.rope_keys[v - 1].first == table && ph.rope_keys[v - 1].second == position) return v - 1;
    }
}

// Checks the step's arguments and plans it. `tables` is the device address of
// the workspace's tables region (the entries' RoPE-factor pointers point into
// it); `cus` the device's compute units. On failure returns a G4_ status and
// writes a message to err. The blob is written in place, every byte of it
// (the alignment gaps between its tables are zero).
inline int plan_step(const g4_step_entry* entries, uint32_t n_entries, uint32_t num_q_heads, uint32_t num_kv_heads,
                     uint32_t head_dim, uint64_t cus, const StepTuning& tune, const char* tables, StepPlanHost* out,
                     char* err, size_t errlen, StepRopeShare* share = nullptr) {
#define PLAN_FAIL(code, ...)                   \
    do {                                       \
        snprintf(err, errlen, __VA_ARGS__);    \
        return code;                           \
    } while (0)
    if (head_dim != 256 && head_dim != 512) PLAN_FAIL(G4_EINVAL, "attnStep: head_dim %u unsupported (256 or 512)", head_dim);
    if (num_kv_heads == 0 || num_q_heads % num_kv_heads || num_q_heads / num_kv_heads > (uint32_t)kMaxGroup)
        PLAN_FAIL(G4_EINVAL, "attnStep: %u query heads over %u kv heads unsupported", num_q_heads, num_kv_heads);
    if (num_kv_heads > 65535) PLAN_FAIL(G4_EINVAL, "attnStep: %u kv heads (max 65535)", num_kv_heads);
    if (!entries || n_entries == 0) PLAN_FAIL(G4_EINVAL, "attnStep: no entries");
    if (n_entries > 65535) PLAN_FAIL(G4_EINVAL, "attnStep: %u entries (max 65535)", n_entries);
    const uint64_t row_bytes = (uint64_t)num_kv_heads * head_dim * 2;
    StepPlanHost& ph = *out;
    ph.tab.resize(n_entries);
    ph.key_begin.resize(n_entries);
    ph.tiles.resize(n_entries);
    ph.rope_idx.resize(n_entries);
    ph.rope_keys.clear();
    {
        size_t slots = 16;
        while (slots < 2 * (size_t)n_entries) slots *= 2;
        ph.rope_slot.assign(slots, 0u);
    }
    std::vector<uint32_t>& key_begin = ph.key_begin;
    std::vector<uint32_t>& tiles = ph.tiles;
    uint64_t T = 0, max_tiles = 0;
    for (uint32_t i = 0; i < n_entries; i++) {
        const g4_step_entry& s = entries[i];
        if (!s.q || !s.q_weight || !s.k_cache || !s.v_cache || !s.out)
            PLAN_FAIL(G4_EINVAL, "attnStep: entry %u has a NULL pointer", i);
        const bool cached = !s.k && !s.v && !s.k_weight;  // consumer whose producer stored the row already
        if (!cached && (!s.k || !s.v || !s.k_weight))
            PLAN_FAIL(G4_EINVAL, "attnStep: entry %u: k, v and k_weight are all set or all NULL", i);
        if (cached && s.store_kv) PLAN_FAIL(G4_EINVAL, "attnStep: entry %u: store_kv needs the raw k and v", i);
        if (reinterpret_cast<uintptr_t>(s.out) & 15)
            PLAN_FAIL(G4_EINVAL, "attnStep: entry %u out must be 16-byte aligned", i);
        if (s.apply_divisor && !s.rope_freqs) PLAN_FAIL(G4_EINVAL, "attnStep: entry %u needs rope_freqs", i);
        if (s.seq_len == 0) PLAN_FAIL(G4_EINVAL, "attnStep: entry %u seq_len 0", i);
        if ((uint64_t)s.seq_len * row_bytes > 0xffffffffull)
            PLAN_FAIL(G4_EINVAL, "attnStep: entry %u cache exceeds 4 GiB", i);
        StepEntryDev& d = ph.tab[i];
        d.q = s.q;
        // Cached rows: the kernel's unconditional loads of k, v and k_weight read q and q_weight
        // instead (valid addresses; the values are not used).
        d.k = cached ? s.q : s.k;
        d.v = cached ? s.q : s.v;
        d.q_weight = s.q_weight;
        d.k_weight = cached ? s.q_weight : s.k_weight;
        d.rope_freqs = s.rope_freqs;
        d.rope_cs = nullptr;  // set below for entries with a host RoPE table
        d.k_cache = s.k_cache;
        d.v_cache = s.v_cache;
        d.out = s.out;
        d.key_end = s.seq_len;
        d.n_parts = 0;  // set by the partition
        d.position = s.position;
        d.flags = (s.store_kv ? kStoreKv : 0u) | (cached ? kRowCached : 0u) | (s.apply_divisor ? kApplyDivisor : 0u) |
                  (s.q_ready ? kQReady : 0u);
        d.theta = s.theta;
        d.window = s.sliding_window;
        d.qscale = s.scale * kLog2e;
        d.eps = s.eps;
        key_begin[i] = step_key_begin(s.seq_len, s.sliding_window);
        tiles[i] = (s.seq_len - key_begin[i] + kTileKeys - 1) / kTileKeys;
        T += tiles[i];
        if (tiles[i] > max_tiles) max_tiles = tiles[i];
        // RoPE factors: one [cos x hd/2][sin x hd/2] set per distinct (table, position) pair
        ph.rope_idx[i] = s.rope_inv_freq_host ? rope_pair_index(ph, s.rope_inv_freq_host, s.position) : ~0u;
    }
    // Workgroups in one wave of the GPU. Small steps (at most kStepOneWgTiles
    // tiles per workgroup with one workgroup per CU) take one 8-wave
    // workgroup per CU: two tile rounds per wave at most, one partial record
    // per CU. Larger steps take two 4-wave workgroups per CU. Measured (us,
    // two 4-wave / one 4-wave / one 8-wave per CU): stack8k 24.0 / 22.3 / 21.9,
    // long128k 34.4 / 32.0 / 31.5, stack32k 48.9 / 56.0 / 55.7, ragged64
    // 190.9 / 199.6 / 197.8. A second workgroup per CU starts behind the first
    // and is served after it, which only pays off when the per-wave rounds
    // are many; grids between one and two per CU are slower than both (CUs
    // with two workgroups finish last). head_dim 512 has one form: one 4-wave
    // workgroup per CU.
    if (cus < 1) cus = 1;
    const bool small = T <= (uint64_t)kStepOneWgTiles * (cus / num_kv_heads);
    const uint32_t waves = head_dim == 512 ? 4u
                           : tune.waves == 4 || tune.waves == 8 ? (uint32_t)tune.waves
                                                                 : (small ? 8u : 4u);
    const uint64_t per_cu = head_dim == 512 ? 1u
                            : tune.wgs_per_cu > 0 ? (uint64_t)tune.wgs_per_cu
                                                  : (waves == 8 || small ? 1u : 2u);
    uint64_t fit = tune.max_wgs > 0 ? (uint64_t)tune.max_wgs / num_kv_heads : per_cu * cus / num_kv_heads;
    if (fit > kStepMaxWgs) fit = kStepMaxWgs;
    if (fit < 1) fit = 1;
    const uint64_t cap = fit > n_entries ? fit : n_entries;
    uint64_t tpw = pick_tiles_per_wg(tiles, T, max_tiles, cap);
    // An 8-wave workgroup requests up to eight tiles at once, one per wave, so
    // two tiles per workgroup instead of one cost no extra tile round and halve
    // the partial records. Measured on one local layer (16 tiles, us per step
    // with the merge): 16 workgroups 10.82, 8 workgroups 10.20, 4 workgroups 10.47.
    if (waves == 8 && tune.max_wgs <= 0 && tpw < 2 && max_tiles >= 2) tpw = 2;

    // Sizes: work items (tpw tiles each, balanced within an entry), merge
    // entries (entries with partial records: the merge grid covers them alone).
    uint64_t n_work = 0;
    uint32_t n_merge = 0, parts = 0, max_parts = 0;
    for (uint32_t i = 0; i < n_entries; i++) {
        const uint64_t we = (tiles[i] + tpw - 1) / tpw;
        ph.tab[i].n_parts = (uint32_t)we;
        n_work += we;
        if (we > max_parts) max_parts = (uint32_t)we;
        if (we > 1) {
            n_merge++;
            parts += (uint32_t)we;
        }
    }
    if (parts > kStepMaxWgs || n_work > cap)
        PLAN_FAIL(G4_EINVAL, "attnStep: internal: %u partial records, %llu items", parts, (unsigned long long)n_work);

    // Tables blob: work items | merge table | entry table | RoPE factors.
    const size_t off_merge = align256(n_work * sizeof(StepWorkDev));
    const size_t off_ents = off_merge + align256(n_merge * sizeof(DecodeEntryDev));
    const size_t off_rope = off_ents + align256(n_entries * sizeof(DecodeEntryDev));
    // Each distinct pair's factors: a set placed by an earlier plan of the share, or one of this blob's.
    const float* rope_base = reinterpret_cast<const float*>(tables + off_rope);
    size_t rope_sets = 0;
    ph.rope_dev.resize(ph.rope_keys.size());
    ph.rope_set.resize(ph.rope_keys.size());
    for (size_t k = 0; k < ph.rope_keys.size(); k++) {
        const float* shared = share ? share->find(ph.rope_keys[k]) : nullptr;
        ph.rope_set[k] = shared ? ~0u : (uint32_t)rope_sets++;
        ph.rope_dev[k] = shared ? shared : rope_base + (size_t)ph.rope_set[k] * rope_set_floats(head_dim);
    }
    ph.blob.resize(off_rope + rope_sets * rope_set_floats(head_dim) * sizeof(float));
    char* blob = ph.blob.data();
    memset(blob + n_work * sizeof(StepWorkDev), 0, off_merge - n_work * sizeof(StepWorkDev));
    memset(blob + off_merge + n_merge * sizeof(DecodeEntryDev), 0, off_ents - off_merge - n_merge * sizeof(DecodeEntryDev));
    memset(blob + off_ents + n_entries * sizeof(DecodeEntryDev), 0, off_rope - off_ents - n_entries * sizeof(DecodeEntryDev));

    // RoPE factors of each distinct pair: the reference's cos/sin of the f32
    // angle, evaluated in f64 and rounded.
    {
        float* rope = reinterpret_cast<float*>(blob + off_rope);
        for (size_t k = 0; k < ph.rope_keys.size(); k++) {
            if (ph.rope_set[k] == ~0u) continue;  // placed by an earlier plan
            float* set = rope + (size_t)ph.rope_set[k] * rope_set_floats(head_dim);
            rope_factors(ph.rope_keys[k].first, ph.rope_keys[k].second, head_dim / 2, set);
            memcpy(set + head_dim, ph.rope_keys[k].first, head_dim / 2 * sizeof(float));  // the inverse frequencies
            if (share) share->add(ph.rope_keys[k], ph.rope_dev[k]);
        }
    }
    // Work items entry by entry (each with a copy of its entry), the merge
    // table and the entry table (every entry: attnOut, first record, parts).
    StepWorkDev* work = reinterpret_cast<StepWorkDev*>(blob);
    DecodeEntryDev* merge = reinterpret_cast<DecodeEntryDev*>(blob + off_merge);
    DecodeEntryDev* ents = reinterpret_cast<DecodeEntryDev*>(blob + off_ents);
    uint32_t part_next = 0;
    for (uint32_t i = 0; i < n_entries; i++) {
        StepEntryDev& d = ph.tab[i];
        if (ph.rope_idx[i] != ~0u) d.rope_cs = ph.rope_dev[ph.rope_idx[i]];
        const uint64_t ne = tiles[i], we = d.n_parts;
        const uint32_t part_base = we > 1 ? part_next : 0;
        // Part j covers tiles [j ne / we, (j + 1) ne / we): the bounds advance by
        // ne / we and carry the remainder, with no division per part.
        const uint64_t step = ne / we, rem = ne % we;
        uint64_t te = 0, acc = 0;
        for (uint64_t j = 0; j < we; j++) {
            const uint64_t tb = te;
            te += step;
            acc += rem;
            if (acc >= we) {
                acc -= we;
                te++;
            }
            const uint64_t rb = key_begin[i] + tb * kTileKeys;
            const uint64_t re = key_begin[i] + te * kTileKeys;
            StepWorkDev& w = *work++;
            w.ent = d;
            w.row_begin = (uint32_t)rb;
            w.row_end = (uint32_t)(re < d.key_end ? re : d.key_end);
            w.part = we > 1 ? part_base + (uint32_t)j : 0u;
            w.entry = i;
        }
        if (we > 1) {
            part_next += (uint32_t)we;
            *merge++ = DecodeEntryDev{nullptr, nullptr, nullptr, d.out, 0, 0, part_base, (uint32_t)we, 0.0f, 0};
        }
        ents[i] = DecodeEntryDev{nullptr, nullptr, nullptr, d.out, 0, 0, part_base, (uint32_t)we, 0.0f, 0};
    }
    ph.waves = waves;
    ph.n_wgs = (uint32_t)n_work;
    ph.n_merge = n_merge;
    ph.max_parts = max_parts;
    ph.parts = parts;
    ph.off_merge = off_merge;
    ph.off_ents = off_ents;
    ph.off_rope = off_rope;
    return G4_OK;
#undef PLAN_FAIL
}

}  // namespace g4
