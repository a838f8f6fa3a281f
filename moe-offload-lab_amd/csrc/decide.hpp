// Decision steps shared by the per-step kernels and the fused batched-decode decision kernel:
// the HOBBIT level rule of one token's slots, the per-expert precision vote and copy choice, and
// the expert-sorted dispatch of one workgroup.

#pragma once

#include "common.hpp"

namespace moehip {

// LDS ordering inside one wave: program order, kept by the compiler
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// HOBBIT level and skip of slot j (< k <= 64) of one token, computed by one wave (lane j; lanes
// j >= k pass wj = 0 and get a meaningless level) in the wave's own LDS (s_w[64], s_sorted[64],
// s_total[1]). policy.py:77-123 (unimportance over the normalised weights, stable descending
// rank), the fixed modes (hi / lo / protected layer) and the weight threshold.
__device__ __forceinline__ void slot_level(int j, int k, float wj, const moehip_policy &pol, float *s_w, float *s_sorted,
                                           float *s_total, int &lvl, bool &skip) {
    const bool act = j < k;
    s_w[j] = wj;
    wave_sync();
    if (j == 0) {
        float tot = 0.f;
        for (int i = 0; i < k; ++i) tot += s_w[i];
        s_total[0] = fmaxf(tot, 1e-12f);
    }
    wave_sync();
    skip = false;
    if (pol.mode == 1 || pol.protect) {
        lvl = 0;
    } else if (pol.mode == 2) {
        lvl = 2;
    } else if (pol.mode == 3) {
        lvl = wj >= pol.t1 ? 0 : 2;  // weight threshold: the expert's own routed weight
    } else {
        // unimportance (policy.py:77-87): stable descending rank, s = cumsum(sorted) - own weight
        const float wn = wj / s_total[0];
        wave_sync();
        s_w[j] = wn;
        wave_sync();
        int rank = 0;
        for (int i = 0; i < k; ++i) {
            const float o = s_w[i];
            rank += (o > wn) || (o == wn && i < j);
        }
        if (act) s_sorted[rank] = wn;
        wave_sync();
        float cs = 0.f;
        for (int r = 0; r <= rank && r < k; ++r) cs += s_sorted[r];
        const float s = cs - wn;
        lvl = 2;
        if (pol.t_mid >= 0.f && s <= pol.t_mid) lvl = 1;
        if (s <= pol.t1) lvl = 0;
        skip = pol.t2 >= 0.f && s > pol.t2 && lvl != 0;
    }
}

struct SharedRecs {
    int64_t r[4];
};

// expert e (of E routed, plus the shared one, id E, when has_shared): the most precise level
// requested by at least hi_vote of its pairs (policy.py:148-154), its precision (lv2p) and
// resident copy (as k_decide_table), the table row of that precision (all other precisions' rows
// 0); an expert with no usable copy gets rank -1 on its pairs (they contribute nothing) and counts
// them in miss. info[e] = chosen precision, -1 = missing, -2 = no pairs.
__device__ __forceinline__ void vote_expert(int e, const int32_t *levels, int E, int has_shared, const int32_t *offsets,
                                            const int32_t *sorted_pos, double hi_vote, int upgrade, int lv0, int lv1,
                                            int lv2, const int64_t *rtab, const SharedRecs &srec, int P,
                                            const int64_t *offs, const int *planned, int64_t *tabs, int32_t *rank,
                                            float *info, float *miss) {
    const int EA = E + (has_shared ? 1 : 0);
    const int p0 = offsets[e], n = offsets[e + 1] - p0;
    int chosen = -1;
    if (n > 0) {
        int c0 = 0, c1 = 0;
        for (int i = 0; i < n; ++i) {
            const int l = levels[sorted_pos[p0 + i]];
            c0 += l <= 0;
            c1 += l <= 1;
        }
        const double need = (hi_vote - 1e-9) * (double)n;
        const int level = (double)c0 >= need ? 0 : ((double)c1 >= need ? 1 : 2);
        const int req = level == 0 ? lv0 : (level == 1 ? lv1 : lv2);
        for (int pi = P - 1; pi >= 0; --pi) {
            const int64_t base = e < E ? rtab[(size_t)pi * E + e] : srec.r[pi];
            if (base != 0 && (upgrade ? req >= pi : req == pi)) chosen = pi;
        }
        if (chosen >= 0 && !planned[chosen]) chosen = -1;
    }
    for (int pi = 0; pi < P; ++pi) {
        const bool sel = chosen == pi;
        const int64_t base = !sel ? 0 : (e < E ? rtab[(size_t)pi * E + e] : srec.r[pi]);
        for (int f = 0; f < 4; ++f) tabs[((size_t)pi * EA + e) * 4 + f] = sel ? base + offs[pi * 4 + f] : 0;
    }
    if (n > 0 && chosen < 0) {
        for (int i = 0; i < n; ++i) rank[sorted_pos[p0 + i]] = -1;
        if (miss != nullptr) atomicAdd(miss, (float)n);
    }
    if (info != nullptr) info[e] = n == 0 ? -2.f : (float)chosen;
}

}  // namespace moehip
