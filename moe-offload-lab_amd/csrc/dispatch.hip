// Token-to-expert dispatch: counting sort of the routed pairs by expert, stable in pair order
// (moelab/runtime.py:471-482: keep = ~skip, argsort(flat_e, stable=True), unique_consecutive).
//
// One workgroup of 16 waves; wave w owns the contiguous pair segment [w * SEG, (w + 1) * SEG) and
// walks it in pair order, 64 pairs at a time. In a 64-pair step the lanes holding the same
// expert are matched by ebits ballots; the group's last lane updates the wave's own count of that
// expert (no atomics, no cross-wave order to enforce). Pass 1 builds the per-wave counts
// cnt[w][e]; one thread per expert turns its column into the wave starts, the experts' totals
// are scanned (a shuffle scan per wave plus the wave totals), and pass 2 walks the segments again,
// placing each pair at start[w][e] + its rank. Positions are stable in pair order.

#include "common.hpp"

namespace moehip {

constexpr int DP_WAVES = 16;
constexpr int DP_PRE = 8;  // 64-pair steps per wave whose expert ids are loaded up front

// expert of pair p if it is kept (p < p1, not skipped, id in range), else -1
__device__ __forceinline__ int pair_expert(const int64_t *__restrict__ idx, const uint8_t *__restrict__ skip, int p,
                                           int p1, int E) {
    if (p >= p1) return -1;
    const int64_t e = idx[p];
    return ((skip == nullptr || skip[p] == 0) && e >= 0 && e < E) ? (int)e : -1;
}

// positions of this 64-pair step: m = lanes with the same expert, r = rank among them
__device__ __forceinline__ void match_lanes(int e, bool valid, int ebits, int lane, uint64_t &m, int &r) {
    m = __ballot(valid);
    for (int b = 0; b < ebits; ++b) {
        const bool bit = (e >> b) & 1;
        const uint64_t bal = __ballot(bit);
        m &= bit ? bal : ~bal;
    }
    const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    r = __popcll(m & lt);
}

__global__ __launch_bounds__(1024) void k_dispatch(const int64_t *__restrict__ idx, const uint8_t *__restrict__ skip,
                                                   int NP, int E, int ebits, int32_t *__restrict__ counts,
                                                   int32_t *__restrict__ offsets, int32_t *__restrict__ sorted_pos,
                                                   int32_t *__restrict__ rank) {
    extern __shared__ int s_cnt[];  // [DP_WAVES][E]: counts, then each wave's start per expert
    __shared__ int s_wtot[DP_WAVES];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int SEG = (NP + DP_WAVES - 1) / DP_WAVES;
    const int p0 = wave * SEG, p1 = min(NP, p0 + SEG);
    for (int i = tid; i < DP_WAVES * E; i += 1024) s_cnt[i] = 0;
    __syncthreads();
    int *mine = s_cnt + wave * E;
    // the expert of each of the first DP_PRE steps' pairs, loaded at once (-1 = not a kept pair)
    int pre[DP_PRE];
#pragma unroll
    for (int i = 0; i < DP_PRE; ++i) pre[i] = pair_expert(idx, skip, p0 + 64 * i + lane, p1, E);
    // pass 1: per-wave counts (only the wave itself touches its row)
    for (int base = p0, step = 0; base < p1; base += 64, ++step) {
        const int p = base + lane;
        int ev = -1;
#pragma unroll
        for (int i = 0; i < DP_PRE; ++i)
            if (step == i) ev = pre[i];
        if (step >= DP_PRE) ev = pair_expert(idx, skip, p, p1, E);
        const bool valid = ev >= 0;
        const int e = valid ? ev : 0;
        uint64_t m;
        int r;
        match_lanes(e, valid, ebits, lane, m, r);
        if (valid && r == __popcll(m) - 1) mine[e] += r + 1;
        __builtin_amdgcn_wave_barrier();  // the row update is seen by the wave's next step
    }
    __syncthreads();
    // per expert: column prefix over the waves (wave starts relative to the expert's offset)
    int tot = 0;  // E <= 1024: thread e owns expert e
    if (tid < E) {
        for (int w = 0; w < DP_WAVES; ++w) {
            const int c = s_cnt[w * E + tid];
            s_cnt[w * E + tid] = tot;
            tot += c;
        }
        counts[tid] = tot;
    }
    // exclusive scan of the experts' totals: 64 experts per wave, then the waves' totals
    int incl = tot;
    for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_up(incl, off, 64);
        if (lane >= off) incl += v;
    }
    if (lane == 63) s_wtot[wave] = incl;
    __syncthreads();
    int wbase = 0;
    for (int w = 0; w < wave; ++w) wbase += s_wtot[w];
    const int excl = wbase + incl - tot;
    if (tid < E) {
        offsets[tid] = excl;
        for (int w = 0; w < DP_WAVES; ++w) s_cnt[w * E + tid] += excl;
        if (tid == E - 1) offsets[E] = excl + tot;
    }
    int total = 0;
    for (int w = 0; w < DP_WAVES; ++w) total += s_wtot[w];
    __syncthreads();
    // pass 2: placement
    for (int base = p0, step = 0; base < p1; base += 64, ++step) {
        const int p = base + lane;
        int ev = -1;
#pragma unroll
        for (int i = 0; i < DP_PRE; ++i)
            if (step == i) ev = pre[i];
        if (step >= DP_PRE) ev = pair_expert(idx, skip, p, p1, E);
        const bool valid = ev >= 0;
        const int e = valid ? ev : 0;
        uint64_t m;
        int r;
        match_lanes(e, valid, ebits, lane, m, r);
        if (valid) {
            const int pos = mine[e] + r;
            sorted_pos[pos] = p;
            rank[p] = pos;
        }
        __builtin_amdgcn_wave_barrier();
        if (valid && r == __popcll(m) - 1) mine[e] += r + 1;
        __builtin_amdgcn_wave_barrier();
        if (p < p1 && !valid) rank[p] = -1;
    }
    for (int i = total + tid; i < NP; i += 1024) sorted_pos[i] = -1;
}

}  // namespace moehip

using namespace moehip;

extern "C" int moehip_dispatch(const int64_t *idx, const uint8_t *skip, int T, int k, int E, int32_t *counts,
                               int32_t *offsets, int32_t *sorted_pos, int32_t *rank, void *stream) {
    MOEHIP_REQUIRE(idx && counts && offsets && sorted_pos && rank, "dispatch: null pointer");
    MOEHIP_REQUIRE(T > 0 && k > 0 && E > 0 && E <= 1024 && (long)T * k <= 65536,
                   "dispatch: bad sizes T=%d k=%d E=%d", T, k, E);
    int ebits = 0;
    while ((1 << ebits) < E) ++ebits;
    const size_t lds = (size_t)DP_WAVES * E * sizeof(int);
    static bool big_lds = false;  // more than 64 KiB of dynamic LDS must be enabled once per kernel
    if (lds > 60 * 1024 && !big_lds) {
        MOEHIP_REQUIRE(hipFuncSetAttribute(reinterpret_cast<const void *>(&k_dispatch),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024) == hipSuccess,
                       "dispatch: cannot enable %zu bytes of LDS", lds);
        big_lds = true;
    }
    hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), lds, as_stream(stream), idx, skip, T * k, E, ebits, counts,
                       offsets, sorted_pos, rank);
    return check_launch("dispatch");
}
