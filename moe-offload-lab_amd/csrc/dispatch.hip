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

#include "decide.hpp"

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

// kept-pair experts of a decision kernel held in LDS (the levels write them, the dispatch reads
// them: no read-back of this workgroup's own global writes), for batches of up to DP_LDS_PAIRS pairs
constexpr int DP_LDS_PAIRS = 4096;

// the dispatch by one workgroup of 1024 threads; s_cnt: DP_WAVES * E ints of LDS. With s_pe, the
// expert of kept pair p (or -1) is s_pe[p] instead of idx / skip.
__device__ __forceinline__ void dispatch_wg(const int64_t *__restrict__ idx, const uint8_t *__restrict__ skip, int NP,
                                            int E, int ebits, int32_t *__restrict__ counts,
                                            int32_t *__restrict__ offsets, int32_t *__restrict__ sorted_pos,
                                            int32_t *__restrict__ rank, int *s_cnt, int *s_wtot,
                                            const int16_t *s_pe = nullptr) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    auto pair_e = [&](int p, int p1) -> int {
        if (s_pe == nullptr) return pair_expert(idx, skip, p, p1, E);
        return p < p1 ? (int)s_pe[p] : -1;
    };
    // up to 1024 pairs: 64 per wave (one step each), so the per-expert columns span only the
    // NW waves that hold pairs; beyond, the pairs spread over all 16 waves
    const int SEG = NP <= 64 * DP_WAVES ? 64 : (NP + DP_WAVES - 1) / DP_WAVES;
    const int NW = (NP + SEG - 1) / SEG;
    const int p0 = wave * SEG, p1 = min(NP, p0 + SEG);
    for (int i = tid; i < NW * E; i += 1024) s_cnt[i] = 0;
    __syncthreads();
    int *mine = s_cnt + wave * E;
    // the expert of each of the first DP_PRE steps' pairs, loaded at once (-1 = not a kept pair)
    int pre[DP_PRE];
#pragma unroll
    for (int i = 0; i < DP_PRE; ++i) pre[i] = pair_e(p0 + 64 * i + lane, p1);
    // pass 1: per-wave counts (only the wave itself touches its row)
    for (int base = p0, step = 0; base < p1; base += 64, ++step) {
        const int p = base + lane;
        int ev = -1;
#pragma unroll
        for (int i = 0; i < DP_PRE; ++i)
            if (step == i) ev = pre[i];
        if (step >= DP_PRE) ev = pair_e(p, p1);
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
        for (int w = 0; w < NW; ++w) {
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
        for (int w = 0; w < NW; ++w) s_cnt[w * E + tid] += excl;
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
        if (step >= DP_PRE) ev = pair_e(p, p1);
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

// The same dispatch for up to 1024 pairs whose experts are in LDS (s_pe), one pair per thread: the
// experts' counts by LDS atomics and their scan, each pair put at an arbitrary slot of its
// expert's segment, then ranked within the segment by pair index (segments are short: the order
// the atomics gave is undone by one pass over the pair's own segment), so the placement is the
// stable one of dispatch_wg. s_cnt: 2 E + NP ints.
__device__ __forceinline__ void dispatch_lds(int NP, int E, int32_t *__restrict__ counts, int32_t *__restrict__ offsets,
                                             int32_t *__restrict__ sorted_pos, int32_t *__restrict__ rank, int *s_cnt,
                                             int *s_wtot, const int16_t *s_pe) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int *c_n = s_cnt, *c_b = s_cnt + E, *c_t = s_cnt + 2 * E;
    if (tid < E) c_n[tid] = 0;
    __syncthreads();
    const int e = tid < NP ? (int)s_pe[tid] : -1;
    int slot = 0;
    if (e >= 0) slot = atomicAdd(&c_n[e], 1);
    __syncthreads();
    // exclusive scan of the counts (thread e owns expert e: E <= 1024)
    const int n = tid < E ? c_n[tid] : 0;
    int incl = n;
    for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_up(incl, off, 64);
        if (lane >= off) incl += v;
    }
    if (lane == 63) s_wtot[wave] = incl;
    __syncthreads();
    int wb = 0, total = 0;
    for (int w = 0; w < DP_WAVES; ++w) {
        if (w < wave) wb += s_wtot[w];
        total += s_wtot[w];
    }
    const int excl = wb + incl - n;
    if (tid < E) {
        counts[tid] = n;
        offsets[tid] = excl;
        c_b[tid] = excl;
    }
    if (tid == 0) offsets[E] = total;
    __syncthreads();
    if (e >= 0) c_t[c_b[e] + slot] = tid;
    __syncthreads();
    if (e >= 0) {
        const int b = c_b[e], m = c_n[e];
        int r = 0;
        for (int i = 0; i < m; ++i) r += c_t[b + i] < tid ? 1 : 0;
        sorted_pos[b + r] = tid;
        rank[tid] = b + r;
    } else if (tid < NP) {
        rank[tid] = -1;
    }
    for (int i = total + tid; i < NP; i += 1024) sorted_pos[i] = -1;
}

// The same dispatch for at most 64 pairs over at most 64 experts by ONE wave (lane = pair; the
// batched decode's few tokens): the stable rank of a pair is its rank among the lower lanes with the
// same expert (match_lanes), the group's last lane writes the expert's count, one prefix scan over
// the experts gives the offsets. No workgroup barrier: the rest of the workgroup is not involved.
// s_cnt: EA words of LDS.
__device__ __forceinline__ void dispatch_wave64(const int64_t *__restrict__ idx, const uint8_t *__restrict__ skip, int NP,
                                                int EA, int ebits, int32_t *__restrict__ counts,
                                                int32_t *__restrict__ offsets, int32_t *__restrict__ sorted_pos,
                                                int32_t *__restrict__ rank, int *s_cnt, const int16_t *s_pe) {
    const int lane = threadIdx.x & 63;
    const int ev = lane < NP ? (s_pe != nullptr ? (int)s_pe[lane] : pair_expert(idx, skip, lane, NP, EA)) : -1;
    const bool valid = ev >= 0;
    const int e = valid ? ev : 0;
    uint64_t m;
    int r;
    match_lanes(e, valid, ebits, lane, m, r);
    if (lane < EA) s_cnt[lane] = 0;
    wave_sync();
    if (valid && r == __popcll(m) - 1) s_cnt[e] = __popcll(m);
    wave_sync();
    const int c = lane < EA ? s_cnt[lane] : 0;
    int incl = c;
    for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_up(incl, off, 64);
        if (lane >= off) incl += v;
    }
    const int total = __shfl(incl, EA - 1, 64);
    if (lane < EA) {
        counts[lane] = c;
        offsets[lane] = incl - c;
        s_cnt[lane] = incl - c;
    }
    if (lane == EA - 1) offsets[EA] = incl;
    wave_sync();
    if (valid) {
        const int pos = s_cnt[e] + r;
        sorted_pos[pos] = lane;
        rank[lane] = pos;
    } else if (lane < NP) {
        rank[lane] = -1;
    }
    if (lane >= total && lane < NP) sorted_pos[lane] = -1;
}

__global__ __launch_bounds__(1024) void k_dispatch(const int64_t *__restrict__ idx, const uint8_t *__restrict__ skip,
                                                   int NP, int E, int ebits, int32_t *__restrict__ counts,
                                                   int32_t *__restrict__ offsets, int32_t *__restrict__ sorted_pos,
                                                   int32_t *__restrict__ rank) {
    extern __shared__ int s_cnt[];  // [DP_WAVES][E]: counts, then each wave's start per expert
    __shared__ int s_wtot[DP_WAVES];
    dispatch_wg(idx, skip, NP, E, ebits, counts, offsets, sorted_pos, rank, s_cnt, s_wtot);
}

// softmax top-k of token t (one wave) and, when gate != nullptr, the shared expert as slot k:
// idx / w_out / w32 (T, k) and idx_ext / w_ext (T, k + 1) (the same results as moehip_router_topk's
// top-k part and moehip_shared_slot). s_p: 64 floats of this wave's LDS.
template <int DT>
__device__ __forceinline__ void route_topk_part(const void *logits, int E, int k, int renorm, bool shared, int t,
                                                int64_t *idx, void *wout, float *w32, int64_t *idx_ext, float *w_ext,
                                                float *s_p, int *myc_out = nullptr, float *r_out = nullptr) {
    const int lane = threadIdx.x & 63;
    const int ks = k + (shared ? 1 : 0);
    int myc;
    float p;
    topk_wave<DT>(logits, (size_t)t, E, k, renorm, s_p, myc, p);
    const float r = rnd_act<DT>(p);
    if (myc_out != nullptr) *myc_out = myc, *r_out = r;
    if (lane < k) {
        idx[(size_t)t * k + lane] = myc;
        if (wout != nullptr) st_act<DT>(wout, (size_t)t * k + lane, p);
        w32[(size_t)t * k + lane] = r;
        if (shared) {
            idx_ext[(size_t)t * ks + lane] = myc;
            w_ext[(size_t)t * ks + lane] = r;
        }
    }
}
template <int DT>
__device__ __forceinline__ void route_shared_part(const void *x, const void *gate, int H, int E, int k, int t,
                                                  int64_t *idx_ext, float *w_ext) {
    const int lane = threadIdx.x & 63;
    const float l = rnd_act<DT>(gate_dot_wave<DT>(x, gate, t, H));
    if (lane == 0) {
        idx_ext[(size_t)t * (k + 1) + k] = E;
        w_ext[(size_t)t * (k + 1) + k] = rnd_act<DT>(1.0f / (1.0f + expf(-l)));
    }
}
template <int DT>
__device__ __forceinline__ void route_token(const void *logits, int E, int k, int renorm, const void *x,
                                            const void *gate, int H, int t, int64_t *idx, void *wout, float *w32,
                                            int64_t *idx_ext, float *w_ext, float *s_p) {
    route_topk_part<DT>(logits, E, k, renorm, gate != nullptr, t, idx, wout, w32, idx_ext, w_ext, s_p);
    if (gate != nullptr) route_shared_part<DT>(x, gate, H, E, k, t, idx_ext, w_ext);
}

// levels and skip of token t's ks slots (one wave; slot k, when ks > k, is the shared expert:
// level 0, never skipped), and the vote tallies of its kept pairs (expert id in [0, EA), not
// skipped: the pairs the dispatch keeps)
// (token_levels_r: the slot's weight wj (lanes < k) and expert e (lanes < ks) in registers; with s_pe,
// the expert of each kept pair, or -1, also goes to s_pe[t * ks + lane])
__device__ __forceinline__ void token_levels_r(int t, int k, int ks, int EA, float wj, int64_t e,
                                               const moehip_policy &pol, int32_t *levels, uint8_t *skip, float *s_w,
                                               float *s_sorted, float *s_total, VoteTally &vt, int16_t *s_pe) {
    const int lane = threadIdx.x & 63;
    int lvl;
    bool sk;
    slot_level(lane, k, wj, pol, s_w, s_sorted, s_total, lvl, sk);
    if (lane >= k) lvl = 0, sk = false;  // the shared expert
    if (lane < ks) {
        levels[(size_t)t * ks + lane] = lvl;
        skip[(size_t)t * ks + lane] = sk ? 1 : 0;
        const bool kept = !sk && e >= 0 && e < EA;
        if (kept) tally_add(vt, (int)e, lvl);
        if (s_pe != nullptr) s_pe[(size_t)t * ks + lane] = kept ? (int16_t)e : (int16_t)-1;
    }
    wave_sync();  // the wave's LDS is reused for its next token
}
__device__ __forceinline__ void token_levels(int t, int k, int ks, int EA, const float *w, const int64_t *idx,
                                             const moehip_policy &pol, int32_t *levels, uint8_t *skip, float *s_w,
                                             float *s_sorted, float *s_total, VoteTally &vt, int16_t *s_pe = nullptr) {
    const int lane = threadIdx.x & 63;
    const float wj = lane < k ? w[(size_t)t * ks + lane] : 0.f;
    const int64_t e = lane < ks ? idx[(size_t)t * ks + lane] : -1;
    token_levels_r(t, k, ks, EA, wj, e, pol, levels, skip, s_w, s_sorted, s_total, vt, s_pe);
}

// the work lists of the batched GEMVs, one per record precision p < P at items + p * (np + 1): one
// item (e << 8 | z) per GV_TOKENS pairs of every expert voted to p (s_ch[e]), in expert order
// (exclusive scan of ceil(n_e / GV_TOKENS)); [np] = their number. For at most 64 experts by one
// wave (lane = expert)
__device__ __forceinline__ void write_items_wave64(const int *s_n, int EA, int np, int P, const int *s_ch,
                                                   int32_t *items) {
    const int lane = threadIdx.x & 63;
    for (int p = 0; p < P; ++p) {
        int32_t *it = items + (size_t)p * (np + 1);
        const int n = (lane < EA && s_ch[lane] == p) ? s_n[lane] : 0;
        const int nz = (n + GV_TOKENS - 1) / GV_TOKENS;
        int incl = nz;
        for (int off = 1; off < 64; off <<= 1) {
            const int v = __shfl_up(incl, off, 64);
            if (lane >= off) incl += v;
        }
        for (int z = 0; z < nz; ++z) it[incl - nz + z] = (lane << 8) | z;
        if (lane == 63) it[np] = incl;
    }
}

// The same work lists for up to 1024 experts by the workgroup, from the vote's own registers
// (thread e: its chosen precision ch and kept pairs n): one scan per precision, one barrier
__device__ __forceinline__ void write_items_1k(int ch, int n, int EA, int np, int P, int32_t *items,
                                               int (*s_wt)[DP_WAVES]) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nz = tid < EA && ch >= 0 ? (n + GV_TOKENS - 1) / GV_TOKENS : 0;
    int incl[GV_MAXP];
#pragma unroll
    for (int p = 0; p < GV_MAXP; ++p) {
        incl[p] = 0;
        if (p >= P) continue;
        int v = ch == p ? nz : 0;
        for (int off = 1; off < 64; off <<= 1) {
            const int u = __shfl_up(v, off, 64);
            if (lane >= off) v += u;
        }
        incl[p] = v;
        if (lane == 63) s_wt[p][wave] = v;
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < GV_MAXP; ++p) {
        if (p >= P) break;
        int wb = 0, tot = 0;
        for (int w = 0; w < DP_WAVES; ++w) {
            const int c = s_wt[p][w];
            if (w < wave) wb += c;
            tot += c;
        }
        int32_t *it = items + (size_t)p * (np + 1);
        if (ch == p)
            for (int z = 0; z < nz; ++z) it[wb + incl[p] - nz + z] = (tid << 8) | z;
        if (tid == 0) it[np] = tot;
    }
}

// The whole T > 1 decision in one workgroup (batched decode, where every step is latency-bound):
// levels per (token, slot) (one wave per token, slot_level), the dispatch of the kept pairs over
// the E + has_shared experts, and the vote / copy / tables per expert (vote_expert); the same
// results as moehip_batch_levels + moehip_dispatch + moehip_batch_vote.
__global__ __launch_bounds__(1024) void k_batch_decide(const float *__restrict__ w, const int64_t *__restrict__ idx,
                                                       int T, int k, int ks, moehip_policy pol,
                                                       int32_t *__restrict__ levels, uint8_t *__restrict__ skip, int E,
                                                       int has_shared, int ebits, int32_t *__restrict__ counts,
                                                       int32_t *__restrict__ offsets, int32_t *__restrict__ sorted_pos,
                                                       int32_t *__restrict__ rank, double hi_vote, int lv0, int lv1,
                                                       int lv2, const int64_t *__restrict__ rtab, SharedRecs srec, int P,
                                                       const int64_t *__restrict__ offs, const int *__restrict__ planned,
                                                       int64_t *__restrict__ tabs, float *__restrict__ info,
                                                       float *__restrict__ miss, int32_t *__restrict__ items) {
    extern __shared__ int s_cnt[];
    __shared__ int s_wtot[DP_WAVES];
    __shared__ float s_w[DP_WAVES][64], s_sorted[DP_WAVES][64], s_total[DP_WAVES];
    __shared__ VoteTally s_vt;
    __shared__ int16_t s_pe[DP_LDS_PAIRS];
    const int tid = threadIdx.x, wave = tid >> 6;
    const int EA = E + (has_shared ? 1 : 0);
    int16_t *pe = T * ks <= DP_LDS_PAIRS ? s_pe : nullptr;
    VoteRecs vr;  // (thread e votes for expert e: EA <= 1024)
    vote_recs(vr, tid, E, EA, rtab, srec, P, offs, planned);
    tally_clear(s_vt, EA);
    __syncthreads();
    for (int t = wave; t < T; t += DP_WAVES)
        token_levels(t, k, ks, EA, w, idx, pol, levels, skip, s_w[wave], s_sorted[wave], &s_total[wave], s_vt, pe);
    __syncthreads();
    if (T * ks <= 64 && EA <= 64) {
        if (wave == 0) dispatch_wave64(idx, skip, T * ks, EA, ebits, counts, offsets, sorted_pos, rank, s_cnt, pe);
    } else if (pe != nullptr && T * ks <= 1024 && 2 * EA + T * ks <= DP_WAVES * EA) {
        dispatch_lds(T * ks, EA, counts, offsets, sorted_pos, rank, s_cnt, s_wtot, pe);
    } else {
        dispatch_wg(idx, skip, T * ks, EA, ebits, counts, offsets, sorted_pos, rank, s_cnt, s_wtot, pe);
    }
    __syncthreads();
    __shared__ int s_ch[VT_MAX];
    __shared__ int s_wt[GV_MAXP][DP_WAVES];
    int ch = -1;
    if (tid < EA)
        s_ch[tid] = ch = vote_apply(tid, s_vt.n[tid], s_vt.c0[tid], s_vt.c1[tid], offsets, E, has_shared, sorted_pos,
                                    hi_vote, pol.upgrade, lv0, lv1, lv2, vr, P, tabs, rank, info, miss);
    if (items == nullptr) return;
    if (EA <= 64) {
        __syncthreads();  // (s_ch)
        if (wave == 0) write_items_wave64(s_vt.n, EA, T * ks, P, s_ch, items);
    } else {
        write_items_1k(ch, tid < EA ? s_vt.n[tid] : 0, EA, T * ks, P, items, s_wt);
    }
}

}  // namespace moehip

using namespace moehip;

// per-token routing of moehip_batch_route_decide on its own, over many workgroups: for batches
// whose tokens would queue behind each other in the single-workgroup launch. Two waves per token:
// the top-k (and the copy of the routed slots into idx_ext / w_ext) on one, the shared expert's
// gate on the other (their outputs are disjoint, so the two latency chains overlap)
template <int DT>
__global__ __launch_bounds__(256) void k_route_tokens(const void *__restrict__ logits, int E, int k, int renorm,
                                                      const void *__restrict__ x, const void *__restrict__ gate, int H,
                                                      int T, int64_t *__restrict__ idx, void *__restrict__ wout,
                                                      float *__restrict__ w32, int64_t *__restrict__ idx_ext,
                                                      float *__restrict__ w_ext) {
    __shared__ float s_p[4][64];
    const int wave = threadIdx.x >> 6, t = blockIdx.x * 2 + (wave >> 1);
    if (t >= T) return;
    if ((wave & 1) == 0)
        route_topk_part<DT>(logits, E, k, renorm, gate != nullptr, t, idx, wout, w32, idx_ext, w_ext, s_p[wave]);
    else if (gate != nullptr)
        route_shared_part<DT>(x, gate, H, E, k, t, idx_ext, w_ext);
}

// Batched decode, everything between the router logits and the expert products in one workgroup:
// softmax top-k per token (one wave per token, topk_wave), the shared expert as slot k (its gate
// x . g and sigmoid rounded to the activation dtype), levels, dispatch, vote / copy / tables, and
// the work list of the batched GEMVs (one item per GV_TOKENS tokens of an expert, in expert order;
// items[T * ks] = their number). Same results as moehip_router_topk (its top-k part) +
// moehip_shared_slot + moehip_batch_decide + the GEMVs' own work list.
template <int DT>
__global__ __launch_bounds__(1024) void k_batch_route_decide(
    const void *__restrict__ logits, int E, int k, int renorm, const void *__restrict__ x,
    const void *__restrict__ gate, int H, int T, int64_t *__restrict__ idx, void *__restrict__ wout,
    float *__restrict__ w32, int64_t *__restrict__ idx_ext, float *__restrict__ w_ext, moehip_policy pol,
    int32_t *__restrict__ levels, uint8_t *__restrict__ skip, int ebits, int32_t *__restrict__ counts,
    int32_t *__restrict__ offsets, int32_t *__restrict__ sorted_pos, int32_t *__restrict__ rank, double hi_vote,
    int lv0, int lv1, int lv2, const int64_t *__restrict__ rtab, SharedRecs srec, int P,
    const int64_t *__restrict__ offs, const int *__restrict__ planned, int64_t *__restrict__ tabs,
    float *__restrict__ info, float *__restrict__ miss, int32_t *__restrict__ items) {
    extern __shared__ int s_cnt[];
    __shared__ int s_wtot[DP_WAVES];
    __shared__ float s_w[DP_WAVES][64], s_sorted[DP_WAVES][64], s_total[DP_WAVES];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool shared = gate != nullptr;
    const int ks = k + (shared ? 1 : 0), EA = E + (shared ? 1 : 0);
    int64_t *pidx = shared ? idx_ext : idx;
    __shared__ VoteTally s_vt;
    __shared__ int16_t s_pe[DP_LDS_PAIRS];
    int16_t *pe = T * ks <= DP_LDS_PAIRS ? s_pe : nullptr;
    VoteRecs vr;  // (thread e votes for expert e: EA <= 1024)
    vote_recs(vr, tid, E, EA, rtab, srec, P, offs, planned);
    tally_clear(s_vt, EA);
    __syncthreads();  // (the tallies are clear before any token adds to them)
    // routing and levels of every token on one wave, the slot's expert and weight passed on in
    // registers (not read back from this workgroup's own global writes)
    for (int t = wave; t < T; t += DP_WAVES) {
        int myc = -1;
        float r = 0.f;
        route_topk_part<DT>(logits, E, k, renorm, shared, t, idx, wout, w32, idx_ext, w_ext, s_w[wave], &myc, &r);
        if (shared) route_shared_part<DT>(x, gate, H, E, k, t, idx_ext, w_ext);
        wave_sync();  // (s_w is the routing's scratch and then the levels')
        const float wj = lane < k ? r : 0.f;
        const int64_t e = lane < k ? (int64_t)myc : (shared && lane == k ? (int64_t)E : (int64_t)-1);
        token_levels_r(t, k, ks, EA, wj, e, pol, levels, skip, s_w[wave], s_sorted[wave], &s_total[wave], s_vt, pe);
    }
    __syncthreads();
    if (T * ks <= 64 && EA <= 64) {
        if (wave == 0) dispatch_wave64(pidx, skip, T * ks, EA, ebits, counts, offsets, sorted_pos, rank, s_cnt, pe);
    } else if (pe != nullptr && T * ks <= 1024 && 2 * EA + T * ks <= DP_WAVES * EA) {
        dispatch_lds(T * ks, EA, counts, offsets, sorted_pos, rank, s_cnt, s_wtot, pe);
    } else {
        dispatch_wg(pidx, skip, T * ks, EA, ebits, counts, offsets, sorted_pos, rank, s_cnt, s_wtot, pe);
    }
    __syncthreads();
    __shared__ int s_ch[VT_MAX];
    __shared__ int s_wt[GV_MAXP][DP_WAVES];
    int ch = -1;
    if (tid < EA)
        s_ch[tid] = ch = vote_apply(tid, s_vt.n[tid], s_vt.c0[tid], s_vt.c1[tid], offsets, E, shared ? 1 : 0, sorted_pos,
                                    hi_vote, pol.upgrade, lv0, lv1, lv2, vr, P, tabs, rank, info, miss);
    if (items == nullptr) return;
    if (EA <= 64) {
        __syncthreads();  // (s_ch)
        if (wave == 0) write_items_wave64(s_vt.n, EA, T * ks, P, s_ch, items);
    } else {
        write_items_1k(ch, tid < EA ? s_vt.n[tid] : 0, EA, T * ks, P, items, s_wt);
    }
}

// more than 64 KiB of LDS per workgroup (dynamic + the kernels' static ~33 KiB) must be enabled
static bool enable_big_lds(const void *fn, size_t lds) {
    if (lds + 36 * 1024 <= 64 * 1024) return true;
    return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024) == hipSuccess;
}

extern "C" int moehip_batch_decide(const float *w32, const int64_t *idx, int T, int k, int ks, const moehip_policy *pol,
                                   int32_t *levels, uint8_t *skip, int E, int has_shared, int32_t *counts,
                                   int32_t *offsets, int32_t *sorted_pos, int32_t *rank, double hi_vote,
                                   const int *lv2p, const int64_t *rtab, const int64_t *shared_rec, int P,
                                   const int64_t *offs, const int *planned, int64_t *tabs, float *info, float *miss,
                                   int32_t *items, void *stream) {
    MOEHIP_REQUIRE(w32 && idx && pol && levels && skip && counts && offsets && sorted_pos && rank && lv2p && rtab &&
                       offs && planned && tabs,
                   "batch_decide: null pointer");
    MOEHIP_REQUIRE(items == nullptr || T <= 256 * GV_TOKENS,
                   "batch_decide: %d tokens (an expert's work items are numbered in 8 bits: <= %d)", T,
                   256 * GV_TOKENS);
    const int EA = E + (has_shared ? 1 : 0);
    MOEHIP_REQUIRE(T > 0 && k > 0 && k <= 64 && ks >= k && ks <= 64 && (long)T * ks <= 65536 && E > 0 && EA <= 1024 &&
                       P > 0 && P <= 4,
                   "batch_decide: bad sizes T=%d k=%d ks=%d E=%d P=%d", T, k, ks, E, P);
    MOEHIP_REQUIRE(!has_shared || shared_rec != nullptr, "batch_decide: shared expert without records");
    for (int i = 0; i < 3; ++i) MOEHIP_REQUIRE(lv2p[i] >= 0 && lv2p[i] < P, "batch_decide: lv2p[%d]=%d", i, lv2p[i]);
    SharedRecs sr = {{0, 0, 0, 0}};
    if (has_shared)
        for (int p = 0; p < P; ++p) sr.r[p] = shared_rec[p];
    int ebits = 0;
    while ((1 << ebits) < EA) ++ebits;
    const size_t lds = (size_t)DP_WAVES * EA * sizeof(int);
    MOEHIP_REQUIRE(enable_big_lds(reinterpret_cast<const void *>(&k_batch_decide), lds),
                   "batch_decide: cannot enable %zu bytes of LDS", lds);
    hipLaunchKernelGGL(k_batch_decide, dim3(1), dim3(1024), lds, as_stream(stream), w32, idx, T, k, ks, *pol, levels,
                       skip, E, has_shared ? 1 : 0, ebits, counts, offsets, sorted_pos, rank, hi_vote, lv2p[0], lv2p[1],
                       lv2p[2], rtab, sr, P, offs, planned, tabs, info, miss, items);
    return check_launch("batch_decide");
}

extern "C" int moehip_batch_route_decide(const void *logits, int dtype, int T, int E, int k, int renorm, const void *x,
                                         const void *gate, int H, int64_t *idx, void *w_out, float *w32,
                                         int64_t *idx_ext, float *w_ext, const moehip_policy *pol, int32_t *levels,
                                         uint8_t *skip, int32_t *counts, int32_t *offsets, int32_t *sorted_pos,
                                         int32_t *rank, double hi_vote, const int *lv2p, const int64_t *rtab,
                                         const int64_t *shared_rec, int P, const int64_t *offs, const int *planned,
                                         int64_t *tabs, float *info, float *miss, int32_t *items, void *stream) {
    MOEHIP_REQUIRE(logits && idx && w32 && pol && levels && skip && counts && offsets && sorted_pos && rank && lv2p &&
                       rtab && offs && planned && tabs,
                   "batch_route_decide: null pointer");
    MOEHIP_REQUIRE(dtype == MOEHIP_DT_F16 || dtype == MOEHIP_DT_BF16, "batch_route_decide: logits dtype %d", dtype);
    const bool shared = gate != nullptr;
    const int ks = k + (shared ? 1 : 0), EA = E + (shared ? 1 : 0);
    MOEHIP_REQUIRE(T > 0 && k > 0 && k <= 32 && k <= E && EA <= 1024 && (long)T * ks <= 65536 && P > 0 && P <= 4,
                   "batch_route_decide: bad sizes T=%d E=%d k=%d P=%d", T, E, k, P);
    MOEHIP_REQUIRE(!shared || (x && idx_ext && w_ext && shared_rec && H % 8 == 0 && ((uintptr_t)x % 16) == 0 &&
                               ((uintptr_t)gate % 16) == 0),
                   "batch_route_decide: shared expert needs x, aligned gate, idx_ext, w_ext and records");
    MOEHIP_REQUIRE(items == nullptr || T <= 256 * GV_TOKENS,
                   "batch_route_decide: %d tokens (an expert's work items are numbered in 8 bits: <= %d)", T,
                   256 * GV_TOKENS);
    for (int i = 0; i < 3; ++i) MOEHIP_REQUIRE(lv2p[i] >= 0 && lv2p[i] < P, "batch_route_decide: lv2p[%d]=%d", i, lv2p[i]);
    SharedRecs sr = {{0, 0, 0, 0}};
    if (shared)
        for (int p = 0; p < P; ++p) sr.r[p] = shared_rec[p];
    int ebits = 0;
    while ((1 << ebits) < EA) ++ebits;
    const size_t lds = (size_t)DP_WAVES * EA * sizeof(int);
    hipStream_t st = as_stream(stream);
    if (dtype == MOEHIP_DT_F16) {
        MOEHIP_REQUIRE(enable_big_lds(reinterpret_cast<const void *>(&k_batch_route_decide<MOEHIP_DT_F16>), lds),
                       "batch_route_decide: cannot enable %zu bytes of LDS", lds);
        hipLaunchKernelGGL((k_batch_route_decide<MOEHIP_DT_F16>), dim3(1), dim3(1024), lds, st, logits, E, k, renorm, x,
                           gate, H, T, idx, w_out, w32, idx_ext, w_ext, *pol, levels, skip, ebits, counts, offsets,
                           sorted_pos, rank, hi_vote, lv2p[0], lv2p[1], lv2p[2], rtab, sr, P, offs, planned, tabs, info,
                           miss, items);
    } else {
        MOEHIP_REQUIRE(enable_big_lds(reinterpret_cast<const void *>(&k_batch_route_decide<MOEHIP_DT_BF16>), lds),
                       "batch_route_decide: cannot enable %zu bytes of LDS", lds);
        hipLaunchKernelGGL((k_batch_route_decide<MOEHIP_DT_BF16>), dim3(1), dim3(1024), lds, st, logits, E, k, renorm,
                           x, gate, H, T, idx, w_out, w32, idx_ext, w_ext, *pol, levels, skip, ebits, counts, offsets,
                           sorted_pos, rank, hi_vote, lv2p[0], lv2p[1], lv2p[2], rtab, sr, P, offs, planned, tabs, info,
                           miss, items);
    }
    return check_launch("batch_route_decide");
}

extern "C" int moehip_route_tokens(const void *logits, int dtype, int T, int E, int k, int renorm, const void *x,
                                   const void *gate, int H, int64_t *idx, void *w_out, float *w32, int64_t *idx_ext,
                                   float *w_ext, void *stream) {
    MOEHIP_REQUIRE(logits && idx && w32, "route_tokens: null pointer");
    MOEHIP_REQUIRE(dtype == MOEHIP_DT_F16 || dtype == MOEHIP_DT_BF16, "route_tokens: logits dtype %d", dtype);
    MOEHIP_REQUIRE(T > 0 && k > 0 && k <= 32 && k <= E && E <= 1024, "route_tokens: bad sizes T=%d E=%d k=%d", T, E,
                   k);
    MOEHIP_REQUIRE(gate == nullptr || (x && idx_ext && w_ext && H % 8 == 0 && ((uintptr_t)x % 16) == 0 &&
                                       ((uintptr_t)gate % 16) == 0),
                   "route_tokens: shared expert needs x, aligned gate, idx_ext and w_ext");
    const dim3 grid((T + 1) / 2);
    if (dtype == MOEHIP_DT_F16)
        hipLaunchKernelGGL((k_route_tokens<MOEHIP_DT_F16>), grid, dim3(256), 0, as_stream(stream), logits, E, k, renorm,
                           x, gate, H, T, idx, w_out, w32, idx_ext, w_ext);
    else
        hipLaunchKernelGGL((k_route_tokens<MOEHIP_DT_BF16>), grid, dim3(256), 0, as_stream(stream), logits, E, k,
                           renorm, x, gate, H, T, idx, w_out, w32, idx_ext, w_ext);
    return check_launch("route_tokens");
}

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
