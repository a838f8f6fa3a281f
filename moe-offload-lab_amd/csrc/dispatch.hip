// Token-to-expert dispatch: counting sort of the routed pairs by expert, stable in pair order
// (moelab/runtime.py:471-482: keep = ~skip, argsort(flat_e, stable=True), unique_consecutive).
//
// One workgroup of 1024 threads. Counts come from LDS atomics (exact), offsets from an LDS
// scan, and each pair's rank among the earlier pairs of its expert from wave ballots: lanes of a
// wave that hold the same expert id are matched bit by bit, and the 16 waves of a chunk then
// claim their slots in wave order, so the result does not depend on scheduling.

#include "common.hpp"

namespace moehip {

__global__ __launch_bounds__(1024) void k_dispatch(const int64_t *__restrict__ idx, const uint8_t *__restrict__ skip,
                                                   int NP, int E, int ebits, int32_t *__restrict__ counts,
                                                   int32_t *__restrict__ offsets, int32_t *__restrict__ sorted_pos,
                                                   int32_t *__restrict__ rank) {
    __shared__ int s_cnt[1024];
    __shared__ int s_run[1024];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    for (int e = tid; e < E; e += 1024) s_cnt[e] = 0;
    __syncthreads();
    for (int p = tid; p < NP; p += 1024) {
        const int64_t e = idx[p];
        if ((skip == nullptr || skip[p] == 0) && e >= 0 && e < E) atomicAdd(&s_cnt[(int)e], 1);
    }
    __syncthreads();
    // inclusive Hillis-Steele scan over E entries (in s_run), then exclusive offsets
    for (int e = tid; e < E; e += 1024) s_run[e] = s_cnt[e];
    __syncthreads();
    for (int off = 1; off < E; off <<= 1) {
        int add = 0;
        if (tid < E && tid >= off) add = s_run[tid - off];
        __syncthreads();
        if (tid < E) s_run[tid] += add;
        __syncthreads();
    }
    if (tid < E) {
        const int excl = s_run[tid] - s_cnt[tid];
        counts[tid] = s_cnt[tid];
        offsets[tid] = excl;
        if (tid == E - 1) offsets[E] = s_run[tid];
    }
    __syncthreads();
    const int total = s_run[E - 1];
    __syncthreads();
    if (tid < E) s_run[tid] = s_run[tid] - s_cnt[tid];  // running insertion point per expert
    __syncthreads();
    const unsigned long long lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int base = 0; base < NP; base += 1024) {
        const int p = base + tid;
        const int64_t e64 = p < NP ? idx[p] : -1;
        const bool valid = p < NP && (skip == nullptr || skip[p] == 0) && e64 >= 0 && e64 < E;
        const int e = valid ? (int)e64 : 0;
        unsigned long long m = __ballot(valid);
        for (int b = 0; b < ebits; ++b) {
            const bool bit = (e >> b) & 1;
            const unsigned long long bal = __ballot(bit);
            m &= bit ? bal : ~bal;
        }
        const int r_in_wave = __popcll(m & lt);
        const int c_in_wave = __popcll(m);
        for (int w = 0; w < 16; ++w) {
            __syncthreads();
            if (wave == w && valid) {
                const int pos = s_run[e] + r_in_wave;
                sorted_pos[pos] = p;
                rank[p] = pos;
                if (r_in_wave == c_in_wave - 1) s_run[e] = pos + 1;
            }
        }
        if (p < NP && !valid) rank[p] = -1;
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
    hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), 0, as_stream(stream), idx, skip, T * k, E, ebits, counts,
                       offsets, sorted_pos, rank);
    return check_launch("dispatch");
}
