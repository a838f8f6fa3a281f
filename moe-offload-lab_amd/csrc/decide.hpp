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
// rank), the fixed modes (hi / lo / protected layer) and the weight threshold. With one64 and
// pol.f64 set, the one-token float64 rule of levels_one (policy.py:89-98, 125-137) instead.
// s_out (optional) receives the slot's unimportance s (0 in the fixed and weight modes, as
// levels_one returns it), which the cache-miss rule below reads.
__device__ __forceinline__ void slot_level(int j, int k, float wj, const moehip_policy &pol, float *s_w, float *s_sorted,
                                           float *s_total, int &lvl, bool &skip, bool one64 = false,
                                           double *s_out = nullptr) {
    const bool act = j < k;
    s_w[j] = wj;
    // the fixed modes and the weight threshold read nothing of the other slots: no LDS round trip
    // (the weights' total below is a serial sum by one lane between two wave barriers)
    if (pol.mode != 0 || pol.protect) {
        skip = false;
        if (s_out) *s_out = 0.0;
        lvl = (pol.mode == 1 || pol.protect) ? 0 : (pol.mode == 2 ? 2 : (wj >= pol.t1 ? 0 : 2));
        return;
    }
    wave_sync();
    const bool f64 = one64 && pol.f64 != 0 && pol.mode == 0 && !pol.protect;
    if (j == 0 && !f64) {
        float tot = 0.f;
        for (int i = 0; i < k; ++i) tot += s_w[i];
        s_total[0] = fmaxf(tot, 1e-12f);
    }
    wave_sync();
    skip = false;
    if (s_out) *s_out = 0.0;
    if (pol.mode == 1 || pol.protect) {
        lvl = 0;
    } else if (pol.mode == 2) {
        lvl = 2;
    } else if (pol.mode == 3) {
        lvl = wj >= pol.t1 ? 0 : 2;  // weight threshold: the expert's own routed weight
    } else if (f64) {
        // levels_one: total = sum(weights) left to right in float64 ("or 1e-12" when it is 0),
        // s_j = running sum of weight / total over the better-ranked slots (stable descending
        // order of the raw weights), thresholds t + 1e-6 in float64
        double tot = 0.0;
        for (int i = 0; i < k; ++i) tot += (double)s_w[i];
        if (tot == 0.0) tot = 1e-12;
        int rank = 0;
        for (int i = 0; i < k; ++i) {
            const float o = s_w[i];
            rank += (o > wj) || (o == wj && i < j);
        }
        if (act) s_sorted[rank] = wj;
        wave_sync();
        double s = 0.0;
        for (int r = 0; r < rank && r < k; ++r) s += (double)s_sorted[r] / tot;
        lvl = 2;
        if (pol.t_mid_64 >= 0.0 && s <= pol.t_mid_64) lvl = 1;
        if (s <= pol.t1_64) lvl = 0;
        skip = pol.t2_64 >= 0.0 && s > pol.t2_64 && lvl != 0;
        if (s_out) *s_out = s;
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
        if (s_out) *s_out = (double)s;
    }
}

// The cache-miss rule of moelab's one-token decode (runtime.py:600-615, policy.py:36-38): a slot
// at level 0 whose level-0 request no resident copy serves, and whose unimportance s exceeds
// miss_t1 + 1e-6 (float64), is served at level 1 instead. Only the one-token rule (pol.f64)
// applies it, as moelab applies it only in its T == 1 path.
__device__ __forceinline__ bool miss_downgrade(const moehip_policy &pol, int lvl, double s) {
    return pol.f64 != 0 && pol.e3 != 0 && lvl == 0 && s > pol.miss_t1_64;
}

struct SharedRecs {
    int64_t r[4];
};

// what the vote of expert e reads besides its tallies: its copy per precision (rtab, or the shared
// expert's records for e == E), the precisions the layer planned and the per-precision offsets of
// the table fields. None of it depends on the routing, so the decision kernels load it at their
// start and the vote, at the end of their chain, waits for no global load.
struct VoteRecs {
    int64_t base[4];
    int64_t offs[16];
    uint32_t planned;  // bit p: precision p planned
};
__device__ __forceinline__ void vote_recs(VoteRecs &vr, int e, int E, int EA, const int64_t *rtab,
                                          const SharedRecs &srec, int P, const int64_t *offs, const int *planned) {
#pragma unroll
    for (int pi = 0; pi < 4; ++pi)
        vr.base[pi] = pi < P && e < EA ? (e < E ? rtab[(size_t)pi * E + e] : srec.r[pi]) : 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) vr.offs[i] = i < 4 * P ? offs[i] : 0;
    vr.planned = 0u;
    for (int pi = 0; pi < P; ++pi)
        if (planned[pi]) vr.planned |= 1u << pi;
}

// expert e (of E routed, plus the shared one, id E, when has_shared): the most precise level
// requested by at least hi_vote of its pairs (policy.py:148-154), its precision (lv2p) and
// resident copy (as k_decide_table), the table row of that precision (all other precisions' rows
// 0); an expert with no usable copy gets rank -1 on its pairs (they contribute nothing) and counts
// them in miss. info[e] = chosen precision, -1 = missing, -2 = no pairs.
__device__ __forceinline__ int vote_apply(int e, int n, int c0, int c1, const int32_t *offsets, int E, int has_shared,
                                           const int32_t *sorted_pos, double hi_vote, int upgrade, int lv0, int lv1,
                                           int lv2, const VoteRecs &vr, int P, int64_t *tabs, int32_t *rank,
                                           float *info, float *miss) {
    const int EA = E + (has_shared ? 1 : 0);
    int chosen = -1;
    if (n > 0) {
        const double need = (hi_vote - 1e-9) * (double)n;
        const int level = (double)c0 >= need ? 0 : ((double)c1 >= need ? 1 : 2);
        // the shared expert runs from its most precise present copy, as in the one-token kernels
        const bool shared_row = e >= E;
        const int req = shared_row ? P - 1 : (level == 0 ? lv0 : (level == 1 ? lv1 : lv2));
        const bool up = shared_row || upgrade;
#pragma unroll
        for (int pi = 3; pi >= 0; --pi)
            if (pi < P && vr.base[pi] != 0 && (up ? req >= pi : req == pi)) chosen = pi;
        if (chosen >= 0 && !((vr.planned >> chosen) & 1u)) chosen = -1;
    }
#pragma unroll
    for (int pi = 0; pi < 4; ++pi) {
        if (pi >= P) break;
        const bool sel = chosen == pi;
        const int64_t base = sel ? vr.base[pi] : 0;
        for (int f = 0; f < 4; ++f) tabs[((size_t)pi * EA + e) * 4 + f] = sel ? base + vr.offs[pi * 4 + f] : 0;
    }
    if (n > 0 && chosen < 0) {
        const int p0 = offsets[e];
        for (int i = 0; i < n; ++i) rank[sorted_pos[p0 + i]] = -1;
        if (miss != nullptr) atomicAdd(miss, (float)n);
    }
    if (info != nullptr) info[e] = n == 0 ? -2.f : (float)chosen;
    return n == 0 ? -1 : chosen;
}

// the vote of expert e from the levels of its dispatched pairs (global memory)
__device__ __forceinline__ void vote_expert(int e, const int32_t *levels, int E, int has_shared, const int32_t *offsets,
                                            const int32_t *sorted_pos, double hi_vote, int upgrade, int lv0, int lv1,
                                            int lv2, const int64_t *rtab, const SharedRecs &srec, int P,
                                            const int64_t *offs, const int *planned, int64_t *tabs, int32_t *rank,
                                            float *info, float *miss) {
    const int p0 = offsets[e], n = offsets[e + 1] - p0;
    int c0 = 0, c1 = 0;
    for (int i = 0; i < n; ++i) {
        const int l = levels[sorted_pos[p0 + i]];
        c0 += l <= 0;
        c1 += l <= 1;
    }
    VoteRecs vr;
    vote_recs(vr, e, E, E + (has_shared ? 1 : 0), rtab, srec, P, offs, planned);
    (void)vote_apply(e, n, c0, c1, offsets, E, has_shared, sorted_pos, hi_vote, upgrade, lv0, lv1, lv2, vr, P, tabs, rank,
                     info, miss);
}

// per-expert tallies of the kept pairs for the vote, gathered while the levels are made (LDS
// atomics, so the vote needs no walk over each expert's pairs): n, #(level <= 0), #(level <= 1)
constexpr int VT_MAX = 1024;
struct VoteTally {
    int n[VT_MAX], c0[VT_MAX], c1[VT_MAX];
};
__device__ __forceinline__ void tally_clear(VoteTally &vt, int EA) {
    for (int e = threadIdx.x; e < EA; e += blockDim.x) vt.n[e] = 0, vt.c0[e] = 0, vt.c1[e] = 0;
}
__device__ __forceinline__ void tally_add(VoteTally &vt, int e, int lvl) {
    atomicAdd(&vt.n[e], 1);
    if (lvl <= 0) atomicAdd(&vt.c0[e], 1);
    if (lvl <= 1) atomicAdd(&vt.c1[e], 1);
}


// tokens per batched-GEMV work item (the work lists written by the decision kernels and read by
// the GEMV kernels: one list of T * ks + 1 ints per record precision, at most GV_MAXP)
constexpr int GV_TOKENS = 1;
constexpr int GV_MAXP = 4;

// order-preserving 32-bit key of a 16-bit logit (bits16) at index c < 1024: the logit bits above
// 1023 - c, so the largest logit wins and equal logits go to the lowest index; -0 == +0
__device__ __forceinline__ uint32_t topk_key16(uint32_t bits16, int c) {
    const uint32_t b = (bits16 & 0x7fffu) == 0u ? 0u : bits16;
    const uint32_t k16 = (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
    return (k16 << 10) | (uint32_t)(1023 - c);
}

// softmax top-k of one token's E logits (16-bit DT, E <= 1024, k <= 32) by one wave: fp32 softmax,
// k rounds of a DPP wave maximum over the keys, optional renorm (the serial sum in slot order);
// lane j < k gets its expert and its final fp32 weight. s_p: 32 floats of the wave's LDS.
// transformers OlmoeTopKRouter.forward (modeling_olmoe.py:337-346) and Qwen3MoeTopKRouter.
// EPL keys per lane (E <= 64 EPL): the rounds only touch the slots that can hold a key.
template <int DT, int EPL>
__device__ __forceinline__ void topk_wave_n(const void *logits, size_t row, int E, int k, int renorm, float *s_p,
                                            int &myc, float &myp) {
    const int lane = threadIdx.x & 63;
    const uint16_t *lr = reinterpret_cast<const uint16_t *>(logits) + row * E;
    float lv[EPL];
    uint32_t key[EPL];
    float m = -INFINITY;
    // every load unconditional (index clamped): a load under a lane-dependent branch is waited for
    // before the next one is issued, EPL round trips in a row
    uint32_t braw[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) braw[i] = lr[min(lane + 64 * i, E - 1)];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const int c = lane + 64 * i;
        key[i] = 0u;
        lv[i] = -INFINITY;
        if (c < E) {
            const uint32_t b = braw[i];
            lv[i] = DT == MOEHIP_DT_F16 ? f16_to_f32((uint16_t)b) : __uint_as_float(b << 16);
            key[i] = topk_key16(b, c);
        }
        m = fmaxf(m, lv[i]);
    }
    m = wave_max(m);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < EPL; ++i)
        if (lane + 64 * i < E) sum += expf(lv[i] - m);
    sum = wave_sum(sum);
    uint32_t myk = 0u;
    myc = 0;
    for (int j = 0; j < k; ++j) {
        uint32_t lb = 0u;
#pragma unroll
        for (int i = 0; i < EPL; ++i) lb = max(lb, key[i]);
        const uint32_t M = wave_max_u32(lb);
#pragma unroll
        for (int i = 0; i < EPL; ++i)
            if (key[i] == M) key[i] = 0u;  // keys are distinct: exactly one lane clears one
        if (lane == j) {
            myc = 1023 - (int)(M & 1023u);
            myk = M >> 10;
        }
    }
    float p = 0.f;
    if (lane < k) {
        // the logit from its key (the inverse of topk_key16; -0 came back as +0, same value)
        const uint32_t b = (myk & 0x8000u) ? (myk & 0x7fffu) : (~myk & 0xffffu);
        const float v = DT == MOEHIP_DT_F16 ? f16_to_f32((uint16_t)b) : __uint_as_float(b << 16);
        p = expf(v - m) / sum;
        s_p[lane] = p;
    }
    wave_sync();
    float tot = 0.f;
    if (renorm)
        for (int j = 0; j < k; ++j) tot += s_p[j];
    myp = renorm ? p / tot : p;
    wave_sync();  // s_p is free for the wave's next token
}
template <int DT>
__device__ __forceinline__ void topk_wave(const void *logits, size_t row, int E, int k, int renorm, float *s_p,
                                          int &myc, float &myp) {
    if (E <= 64) topk_wave_n<DT, 1>(logits, row, E, k, renorm, s_p, myc, myp);
    else if (E <= 128) topk_wave_n<DT, 2>(logits, row, E, k, renorm, s_p, myc, myp);
    else if (E <= 256) topk_wave_n<DT, 4>(logits, row, E, k, renorm, s_p, myc, myp);
    else if (E <= 512) topk_wave_n<DT, 8>(logits, row, E, k, renorm, s_p, myc, myp);
    else topk_wave_n<DT, 16>(logits, row, E, k, renorm, s_p, myc, myp);
}

// x[t] . g over H values (16-bit DT: 8 per 16-byte load; x and g 16-byte aligned, H % 8 == 0), by
// one wave, fp32, every lane gets the sum
template <int DT>
__device__ __forceinline__ float gate_dot_wave(const void *x, const void *g, int t, int H) {
    const int lane = threadIdx.x & 63;
    float acc = 0.f;
    const uint4 *xr = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(x) + (size_t)t * H);
    const uint4 *gr = reinterpret_cast<const uint4 *>(g);
    // 4 chunks per lane requested before any is used (a loop of one chunk per trip waits for each
    // chunk's round trip in turn); the products are added in the same order as one chunk at a time
    constexpr int U = 4;
    const int nc = H / 8;
    for (int c0 = lane; c0 < nc; c0 += 64 * U) {
        uint4 xv[U], gv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = min(c0 + 64 * u, nc - 1);
            xv[u] = xr[c];
            gv[u] = gr[c];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (c0 + 64 * u >= nc) break;
            const uint32_t xa[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w}, ga[4] = {gv[u].x, gv[u].y, gv[u].z, gv[u].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float x0 = DT == MOEHIP_DT_F16 ? f16_to_f32((uint16_t)xa[i]) : __uint_as_float(xa[i] << 16);
                const float x1 = DT == MOEHIP_DT_F16 ? f16_to_f32((uint16_t)(xa[i] >> 16)) : __uint_as_float(xa[i] & 0xffff0000u);
                const float g0 = DT == MOEHIP_DT_F16 ? f16_to_f32((uint16_t)ga[i]) : __uint_as_float(ga[i] << 16);
                const float g1 = DT == MOEHIP_DT_F16 ? f16_to_f32((uint16_t)(ga[i] >> 16)) : __uint_as_float(ga[i] & 0xffff0000u);
                acc = fmaf(x0, g0, acc);
                acc = fmaf(x1, g1, acc);
            }
        }
    }
    return wave_sum(acc);
}

}  // namespace moehip
