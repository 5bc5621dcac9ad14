// CPU check of the one-launch step's host planner (gemma4-webgpu_amd/csrc/step_plan.h), built with g++
// under AddressSanitizer and UndefinedBehaviorSanitizer by tests/test_step_plan.py. Reads scenarios from
// stdin, one per line:
//   nqh nkh hd cus seq:window[:c] ...      (c: a KV-consumer entry whose row is already cached)
// plans each (one planner state for all, as a library thread keeps it) and checks the plan's
// invariants; prints "ok <n_wgs> <n_merge>" per scenario, or an error and exits 1.
// With the argument "rope <stride>", instead compares the planner's RoPE factors with the C library's
// f64 cos and sin over positions 0, stride, 2 stride, ... up to 131071 and a set of large angles.
#include <stdio.h>
#include <string.h>

#include <iostream>
#include <sstream>
#include <string>
#include <vector>

#include "../gemma4-webgpu_amd/csrc/step_plan.h"

using namespace g4;

static int bad(int line, const char* what) {
    printf("FAIL line %d: %s\n", line, what);
    return 1;
}

// Every factor equals (float)cos/sin((double)angle) of the C library; returns the values compared.
static long rope_sweep(uint32_t stride) {
    long n = 0;
    std::vector<float> inv(256), c(512);
    const double thetas[] = {1e4, 1e6};
    for (uint32_t hd : {256u, 512u})
        for (double theta : thetas) {
            for (uint32_t i = 0; i < hd / 2; i++) inv[i] = (float)(1.0 / pow(theta, 2.0 * i / hd));
            std::vector<uint32_t> pos;
            for (uint32_t p = 0; p < 131072; p += stride) pos.push_back(p);
            for (uint32_t p : {131071u, 131072u, 1048575u, 1048576u, 16777216u, 4000000000u}) pos.push_back(p);
            for (uint32_t p : pos) {
                rope_factors(inv.data(), p, hd / 2, c.data());
                for (uint32_t i = 0; i < hd / 2; i++, n++) {
                    const double a = (double)((float)p * inv[i]);
                    if (c[i] != (float)cos(a) || c[hd / 2 + i] != (float)sin(a)) {
                        printf("FAIL rope: hd %u theta %g pos %u pair %u: %a %a, C library %a %a\n", hd, theta, p, i,
                               c[i], c[hd / 2 + i], (float)cos(a), (float)sin(a));
                        return -1;
                    }
                }
            }
        }
    return n;
}

// A token's layers planned one by one into one packed upload (g4_attn_step_prepare_layers with E entries
// per layer): each layer's plan equals the plan of its E entries alone except for the RoPE factors, which
// are its own set at the first (table, position) pair of the upload and the earlier layer's set after that,
// with the C library's values; the packed tables fit the layers' tables regions.
static int check_layers(int line, const std::vector<g4_step_entry>& ents, uint32_t E, uint32_t nqh, uint32_t nkh,
                        uint32_t hd, uint32_t cus, char* dev) {
    const uint32_t n = (uint32_t)ents.size() / E;
    const StepLayout L1 = step_layout(E, nkh, nqh / nkh, hd);
    StepPlanHost ph, one;
    StepRopeShare share;
    std::vector<char> packed;
    char err[256] = "";
    for (uint32_t i = 0; i < n; i++) {
        char* tables = dev + packed.size();
        const g4_step_entry* le = &ents[(size_t)i * E];
        if (plan_step(le, E, nqh, nkh, hd, cus, StepTuning{}, tables, &ph, err, sizeof err, &share) ||
            plan_step(le, E, nqh, nkh, hd, cus, StepTuning{}, tables, &one, err, sizeof err))
            return bad(line, "layer plan failed");
        if (ph.n_wgs != one.n_wgs || ph.off_rope != one.off_rope || ph.waves != one.waves ||
            ph.max_parts != one.max_parts || ph.blob.size() > one.blob.size())
            return bad(line, "layer plan differs from the plan of its entries alone");
        const StepWorkDev* w = reinterpret_cast<const StepWorkDev*>(ph.blob.data());
        const StepWorkDev* w1 = reinterpret_cast<const StepWorkDev*>(one.blob.data());
        for (uint32_t k = 0; k < ph.n_wgs; k++) {
            StepWorkDev a = w[k], b = w1[k];
            a.ent.rope_cs = b.ent.rope_cs = nullptr;
            if (memcmp(&a, &b, sizeof a)) return bad(line, "layer work item differs from the plan of its entries");
        }
        if (memcmp(ph.blob.data() + ph.n_wgs * sizeof(StepWorkDev), one.blob.data() + ph.n_wgs * sizeof(StepWorkDev),
                   ph.off_rope - ph.n_wgs * sizeof(StepWorkDev)))
            return bad(line, "layer merge or entry table differs from the plan of its entries");
        const size_t at = packed.size();
        packed.resize(at + align256(ph.blob.size()), 0);
        memcpy(packed.data() + at, ph.blob.data(), ph.blob.size());
        if (packed.size() > (size_t)(i + 1) * L1.part_ml) return bad(line, "packed tables exceed the layers' regions");
        for (uint32_t k = 0; k < ph.n_wgs; k++) {
            const uint32_t ei = (uint32_t)i * E + w[k].entry;  // the entry in the whole list
            const g4_step_entry& e = ents[ei];
            const float* rc = w[k].ent.rope_cs;
            if (!e.rope_inv_freq_host) {
                if (rc) return bad(line, "layer RoPE factors without a host table");
                continue;
            }
            const char* rp = reinterpret_cast<const char*>(rc);
            if (rp < dev || rp + rope_set_floats(hd) * 4 > dev + packed.size() || (size_t)(rp - dev) % 4)
                return bad(line, "layer RoPE pointer outside the packed tables");
            for (uint32_t j = 0; j < (uint32_t)i * E; j++)  // an earlier layer at the same pair owns the set
                if (ents[j].rope_inv_freq_host == e.rope_inv_freq_host && ents[j].position == e.position) {
                    if (rp >= tables) return bad(line, "layer carries a RoPE set an earlier layer placed");
                    break;
                }
            const float* f = reinterpret_cast<const float*>(packed.data() + (rp - dev));
            for (uint32_t p = 0; p < hd / 2; p++) {
                const double a = (double)((float)e.position * e.rope_inv_freq_host[p]);
                if (f[p] != (float)cos(a) || f[hd / 2 + p] != (float)sin(a))
                    return bad(line, "layer RoPE factors differ from the C library's cos and sin");
                if (f[hd + p] != e.rope_inv_freq_host[p]) return bad(line, "layer RoPE set's inverse frequencies");
            }
        }
    }
    return 0;
}

int main(int argc, char** argv) {
    if (argc == 3 && !strcmp(argv[1], "rope")) {
        const long n = rope_sweep((uint32_t)atoi(argv[2]));
        if (n < 0) return 1;
        printf("ok rope %ld\n", n);
        return 0;
    }
    std::string text;
    StepPlanHost ph;  // reused by every scenario: the storage grows and shrinks between plans
    int line = 0;
    // Fake device addresses: the planner stores them and never dereferences them.
    char* const dev = reinterpret_cast<char*>(uintptr_t(1) << 40);
    while (std::getline(std::cin, text)) {
        line++;
        std::istringstream in(text);
        uint32_t nqh, nkh, hd, cus;
        if (!(in >> nqh >> nkh >> hd >> cus)) continue;
        std::vector<g4_step_entry> ents;
        std::vector<std::vector<float>> inv;  // host RoPE tables (read by the planner)
        std::string tok;
        while (in >> tok) {
            uint32_t seq = 0, win = 0;
            char c = 0;
            sscanf(tok.c_str(), "%u:%u:%c", &seq, &win, &c);
            g4_step_entry e{};
            const uintptr_t base = uintptr_t(ents.size() + 1) << 32;
            e.q = reinterpret_cast<const float*>(base + 0x1000);
            e.q_weight = reinterpret_cast<const uint16_t*>(base + 0x2000);
            if (c != 'c') {
                e.k = reinterpret_cast<const float*>(base + 0x3000);
                e.v = reinterpret_cast<const float*>(base + 0x4000);
                e.k_weight = reinterpret_cast<const uint16_t*>(base + 0x5000);
                e.store_kv = 1;
            }
            e.k_cache = reinterpret_cast<uint16_t*>(base + 0x10000000);
            e.v_cache = reinterpret_cast<uint16_t*>(base + 0x20000000);
            e.out = reinterpret_cast<float*>(base + 0x30000000);
            e.seq_len = seq;
            e.position = seq - 1;
            e.sliding_window = win;
            e.theta = win ? 1e4f : 1e6f;
            e.apply_divisor = win ? 0 : 1;
            e.rope_freqs = reinterpret_cast<const uint16_t*>(base + 0x6000);
            e.scale = 1.0f;
            e.eps = 1e-6f;
            ents.push_back(e);
        }
        // Host RoPE tables: entries 0, 2, 4, ... carry one; entries 0 mod 4 their own, entries 2 mod 4 one of
        // two tables shared by window kind (entries at one position then share factors).
        inv.assign(ents.size() + 2, std::vector<float>(hd / 2));
        for (size_t t = 0; t < inv.size(); t++)
            for (uint32_t i = 0; i < hd / 2; i++) inv[t][i] = 1.0f / (float)(i + 1 + t % 3);
        for (size_t i = 0; i < ents.size(); i += 2)
            ents[i].rope_inv_freq_host =
                i % 4 == 0 ? inv[i].data() : inv[ents.size() + (ents[i].sliding_window ? 1 : 0)].data();
        const uint32_t n = (uint32_t)ents.size();
        const StepLayout L = step_layout(n, nkh, nqh / nkh, hd);
        char err[256] = "";
        const int rc = plan_step(ents.data(), n, nqh, nkh, hd, cus, StepTuning{}, dev + L.tables, &ph, err,
                                 sizeof err);
        if (rc) {
            printf("FAIL line %d: plan_step: %s\n", line, err);
            return 1;
        }
        // the blob fits the tables region, and its parts do not overlap
        if (ph.blob.size() > L.part_ml - L.tables) return bad(line, "tables blob exceeds the tables region");
        if (ph.off_merge < ph.n_wgs * sizeof(StepWorkDev)) return bad(line, "merge table overlaps the work table");
        if (ph.off_ents < ph.off_merge + ph.n_merge * sizeof(DecodeEntryDev)) return bad(line, "entries overlap merge");
        if (ph.off_rope < ph.off_ents + n * sizeof(DecodeEntryDev)) return bad(line, "rope overlaps the entry table");
        const size_t cap = n > kStepMaxWgs ? n : kStepMaxWgs;
        if (ph.n_wgs > cap) return bad(line, "more work items than the workspace holds");
        if (ph.parts > kStepMaxWgs) return bad(line, "more partial records than the workspace holds");
        const StepWorkDev* work = reinterpret_cast<const StepWorkDev*>(ph.blob.data());
        const DecodeEntryDev* merge = reinterpret_cast<const DecodeEntryDev*>(ph.blob.data() + ph.off_merge);
        const DecodeEntryDev* etab = reinterpret_cast<const DecodeEntryDev*>(ph.blob.data() + ph.off_ents);
        const size_t rope_bytes = ph.blob.size() - ph.off_rope;
        std::vector<std::vector<const StepWorkDev*>> per(n);
        for (uint32_t w = 0; w < ph.n_wgs; w++) {
            if (work[w].entry >= n) return bad(line, "work item names no entry");
            per[work[w].entry].push_back(&work[w]);
        }
        std::vector<char> slot_used(ph.parts, 0);
        uint32_t n_split = 0;
        for (uint32_t i = 0; i < n; i++) {
            const g4_step_entry& e = ents[i];
            const uint32_t kb = (e.sliding_window && e.seq_len > e.sliding_window) ? e.seq_len - e.sliding_window : 0;
            const auto& items = per[i];
            if (items.empty()) return bad(line, "entry without workgroups");
            uint32_t next = kb;
            for (size_t j = 0; j < items.size(); j++) {  // items of an entry are consecutive, in row order
                const StepWorkDev& w = *items[j];
                if (w.row_begin != next || w.row_end <= w.row_begin) return bad(line, "rows not covered once, in order");
                if (w.row_end > e.seq_len) return bad(line, "rows past seq_len");
                if (w.ent.n_parts != items.size()) return bad(line, "n_parts disagrees with the work items");
                if (w.ent.key_end != e.seq_len || w.ent.position != e.position || w.ent.out != e.out ||
                    w.ent.k_cache != e.k_cache)
                    return bad(line, "entry copy differs from the entry");
                const bool cached = !e.k;
                if (cached != ((w.ent.flags & kRowCached) != 0) || (w.ent.flags & kStoreKv) != (e.store_kv ? kStoreKv : 0) ||
                    ((w.ent.flags & kApplyDivisor) != 0) != (e.apply_divisor != 0))
                    return bad(line, "flags");
                if (w.ent.window != e.sliding_window) return bad(line, "window");
                if (items.size() > 1) {
                    if (w.part >= ph.parts || slot_used[w.part]) return bad(line, "partial-record slot reused or out of range");
                    slot_used[w.part] = 1;
                }
                if (e.rope_inv_freq_host) {
                    const char* rc_ptr = reinterpret_cast<const char*>(w.ent.rope_cs);
                    const char* r0 = dev + L.tables + ph.off_rope;
                    const size_t set_bytes = rope_set_floats(hd) * 4;
                    if (rc_ptr < r0 || rc_ptr + set_bytes > r0 + rope_bytes || (rc_ptr - r0) % set_bytes)
                        return bad(line, "RoPE factor pointer outside the factors");
                    const float* f = reinterpret_cast<const float*>(ph.blob.data() + (rc_ptr - (dev + L.tables)));
                    for (uint32_t p = 0; p < hd / 2; p++) {
                        const double a = (double)((float)e.position * e.rope_inv_freq_host[p]);
                        if (f[p] != (float)cos(a) || f[hd / 2 + p] != (float)sin(a))
                            return bad(line, "RoPE factors differ from the C library's cos and sin");
                        if (f[hd + p] != e.rope_inv_freq_host[p]) return bad(line, "RoPE set's inverse frequencies");
                    }
                } else if (w.ent.rope_cs) {
                    return bad(line, "RoPE factors without a host table");
                }
                next = w.row_end;
            }
            if (next != e.seq_len) return bad(line, "attended rows not fully covered");
            // The plan advanced by a tokens (the kernel's step_part_rows): the parts still cover the
            // entry's attended rows [key_begin(seq_len + a), seq_len + a) once, in order, and the part
            // that ends there is the one that held the last row (the one that computes the new row).
            for (uint32_t a : {1u, 2u, 31u, 32u, 33u, 100u, 511u, 512u, 513u, 1000u, 4096u}) {
                const uint32_t ke = e.seq_len + a;
                uint32_t at = step_key_begin(ke, e.sliding_window);
                for (size_t j = 0; j < items.size(); j++) {
                    const StepWorkDev& w = *items[j];
                    const StepRows r = step_part_rows(w.row_begin, w.row_end, w.ent.key_end, w.ent.window, a);
                    if (r.begin != at || r.end <= r.begin) return bad(line, "advanced rows not covered once, in order");
                    if ((r.end == ke) != (j + 1 == items.size())) return bad(line, "advanced last row in another part");
                    at = r.end;
                }
                if (at != ke) return bad(line, "advanced rows not fully covered");
            }
            // the entry table: attnOut, parts, and the first record of a split entry
            if (etab[i].out != e.out || etab[i].n_splits != items.size() ||
                (items.size() > 1 && etab[i].split_base != items[0]->part))
                return bad(line, "entry table disagrees with the work items");
            if (items.size() > 1) {
                bool found = false;
                for (uint32_t m = 0; m < ph.n_merge; m++)
                    if (merge[m].out == e.out) {
                        found = merge[m].n_splits == items.size() && merge[m].split_base == items[0]->part;
                        break;
                    }
                if (!found) return bad(line, "split entry missing from the merge table");
                n_split++;
            }
        }
        if (n_split != ph.n_merge) return bad(line, "merge table lists entries that are not split");
        if (check_layers(line, ents, 1, nqh, nkh, hd, cus, dev)) return 1;
        if (n % 2 == 0 && check_layers(line, ents, 2, nqh, nkh, hd, cus, dev)) return 1;
        printf("ok %u %u\n", ph.n_wgs, ph.n_merge);
    }
    return 0;
}
