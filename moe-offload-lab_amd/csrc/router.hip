// Router (logits -> softmax -> top-k -> renorm) and the decode-time decision/table kernel.
//
// Router numerics follow transformers' *TopKRouter.forward (modeling_olmoe.py:337-346):
// logits are F.linear in the model dtype (here: fp32 accumulation, one rounding to the dtype),
// softmax in fp32, top-k, optional renormalisation in fp32, weights cast to the model dtype.
// Top-k compares the (dtype-exact) logits, lowest expert index first among equal logits, which
// selects the same set as top-k over the probabilities whenever distinct logits give distinct
// probabilities.

#include <limits.h>

#include "decide.hpp"

namespace moehip {

constexpr int ROUTER_TT = 8;  // tokens per block in the logits kernel

// logits[t, e] = round_dt(sum_c x[t, c] * Wr[e, c]); one wave per expert row, 4 waves per block
template <int DT>
__global__ __launch_bounds__(256) void k_router_logits(const void *__restrict__ x, const void *__restrict__ Wr, int T,
                                                       int H, int E, int vec16, void *__restrict__ logits) {
    const int lane = threadIdx.x & 63;
    const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (e >= E) return;
    const int t0 = blockIdx.y * ROUTER_TT;
    const int nt = min(ROUTER_TT, T - t0);
    float acc[ROUTER_TT];
#pragma unroll
    for (int t = 0; t < ROUTER_TT; ++t) acc[t] = 0.f;
    const size_t wrow = (size_t)e * H;
    if (DT != MOEHIP_DT_F32 && vec16) {
        // 16-bit dtypes, 8 values per 16-byte load
        const uint16_t *W16 = reinterpret_cast<const uint16_t *>(Wr);
        const uint16_t *X16 = reinterpret_cast<const uint16_t *>(x);
        for (int c = lane * 8; c < H; c += 512) {
            const uint4 wv = *reinterpret_cast<const uint4 *>(W16 + wrow + c);
            const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
            float wf[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (DT == MOEHIP_DT_F16) {
                    wf[2 * j] = f16_to_f32(wd[j] & 0xffffu);
                    wf[2 * j + 1] = f16_to_f32(wd[j] >> 16);
                } else {
                    wf[2 * j] = __uint_as_float(wd[j] << 16);
                    wf[2 * j + 1] = __uint_as_float(wd[j] & 0xffff0000u);
                }
            }
#pragma unroll
            for (int t = 0; t < ROUTER_TT; ++t) {
                if (t < nt) {
                    const uint4 xv = *reinterpret_cast<const uint4 *>(X16 + (size_t)(t0 + t) * H + c);
                    const uint32_t xd[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        float xa, xb;
                        if constexpr (DT == MOEHIP_DT_F16) {
                            xa = f16_to_f32(xd[j] & 0xffffu);
                            xb = f16_to_f32(xd[j] >> 16);
                        } else {
                            xa = __uint_as_float(xd[j] << 16);
                            xb = __uint_as_float(xd[j] & 0xffff0000u);
                        }
                        acc[t] = fmaf(wf[2 * j], xa, acc[t]);
                        acc[t] = fmaf(wf[2 * j + 1], xb, acc[t]);
                    }
                }
            }
        }
    } else {
        for (int c = lane; c < H; c += 64) {
            const float wv = ld_act<DT>(Wr, wrow + c);
#pragma unroll
            for (int t = 0; t < ROUTER_TT; ++t)
                if (t < nt) acc[t] = fmaf(wv, ld_act<DT>(x, (size_t)(t0 + t) * H + c), acc[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < ROUTER_TT; ++t) {
        const float s = wave_sum(acc[t]);
        if (lane == 0 && t < nt) st_act<DT>(logits, (size_t)(t0 + t) * E + e, s);
    }
}

// logits on MFMA (16-bit activations, T >= 4, H a multiple of 512, 16-byte aligned rows): one
// workgroup per 16 tokens x 16 experts, each of its 4 waves a quarter of H through
// v_mfma_f32_16x16x32 (A = 16 tokens x 32 K: lane row + 16 (k / 8), element k % 8; B likewise for
// the 16 expert rows; D row 4 (lane / 16) + i, column lane % 16), the four partial tiles summed
// in wave order in LDS (fixed order: the result does not depend on scheduling), one rounding
typedef _Float16 rf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 rbf16x8 __attribute__((ext_vector_type(8)));
typedef float rf32x4 __attribute__((ext_vector_type(4)));

template <int DT>
__device__ __forceinline__ rf32x4 router_mfma(const uint4 a, const uint4 b, const rf32x4 c) {
    if constexpr (DT == MOEHIP_DT_F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(rf16x8, a), __builtin_bit_cast(rf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(rbf16x8, a), __builtin_bit_cast(rbf16x8, b), c, 0, 0, 0);
}

template <int DT>
__global__ __launch_bounds__(256) void k_router_logits_mfma(const void *__restrict__ x, const void *__restrict__ Wr,
                                                            int T, int H, int E, void *__restrict__ logits) {
    __shared__ float s_part[4][16][17];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t0 = blockIdx.x * 16, e0 = blockIdx.y * 16;
    const int r = lane & 15, kq = lane >> 4;
    const uint16_t *xr = reinterpret_cast<const uint16_t *>(x) + (size_t)min(t0 + r, T - 1) * H + kq * 8;
    const uint16_t *wr = reinterpret_cast<const uint16_t *>(Wr) + (size_t)min(e0 + r, E - 1) * H + kq * 8;
    const int kw = H >> 2;
    rf32x4 acc = {0.f, 0.f, 0.f, 0.f};
    int k0 = wave * kw;
    const int kend = (wave + 1) * kw;
    for (; k0 + 512 <= kend; k0 += 512) {  // 32 loads in flight at once
        uint4 av[16], bv[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            av[u] = *reinterpret_cast<const uint4 *>(xr + k0 + 32 * u);
            bv[u] = *reinterpret_cast<const uint4 *>(wr + k0 + 32 * u);
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) acc = router_mfma<DT>(av[u], bv[u], acc);
    }
    for (; k0 < kend; k0 += 128) {
        uint4 av[4], bv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            av[u] = *reinterpret_cast<const uint4 *>(xr + k0 + 32 * u);
            bv[u] = *reinterpret_cast<const uint4 *>(wr + k0 + 32 * u);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) acc = router_mfma<DT>(av[u], bv[u], acc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) s_part[wave][4 * kq + i][r] = acc[i];
    __syncthreads();
    const int m = threadIdx.x >> 4, n = threadIdx.x & 15;
    const float v = ((s_part[0][m][n] + s_part[1][m][n]) + s_part[2][m][n]) + s_part[3][m][n];
    if (t0 + m < T && e0 + n < E) st_act<DT>(logits, (size_t)(t0 + m) * E + e0 + n, v);
}

// softmax + top-k + renorm for one token per wave (E <= 1024, k <= 32). 16-bit logits: k rounds of
// a DPP wave maximum over 32-bit keys (order-preserving logit bits above 1023 - index: the largest
// logit, the lowest index among equal logits); fp32 logits: value and index compared separately.

template <int DT>
__global__ __launch_bounds__(64) void k_router_topk(const void *__restrict__ logits, int T, int E, int k, int renorm,
                                                    int64_t *__restrict__ idx, void *__restrict__ wout,
                                                    float *__restrict__ w32) {
    const int t = blockIdx.x;
    const int lane = threadIdx.x;
    __shared__ int s_idx[32];
    __shared__ float s_p[32];
    if constexpr (DT != MOEHIP_DT_F32) {
        int myc;
        float p;
        topk_wave<DT>(logits, (size_t)t, E, k, renorm, s_p, myc, p);
        if (lane < k) {
            idx[(size_t)t * k + lane] = myc;
            if (wout != nullptr) st_act<DT>(wout, (size_t)t * k + lane, p);
            if (w32 != nullptr) w32[(size_t)t * k + lane] = rnd_act<DT>(p);
        }
        return;
    }
    // fp32 logits: value and index compared separately (no 16-bit keys)
    float lv[16];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int c = lane + 64 * i;
        lv[i] = c < E ? ld_act<DT>(logits, (size_t)t * E + c) : -INFINITY;
        m = fmaxf(m, lv[i]);
    }
    m = wave_max(m);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i)
        if (lane + 64 * i < E) sum += expf(lv[i] - m);
    sum = wave_sum(sum);
    uint32_t taken = 0;
    for (int j = 0; j < k; ++j) {
        float bv = -INFINITY;
        int bi = INT_MAX;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int c = lane + 64 * i;
            if (c < E && !((taken >> i) & 1u) && (lv[i] > bv || (lv[i] == bv && c < bi))) {
                bv = lv[i];
                bi = c;
            }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(bv, off, 64);
            const int oi = __shfl_xor(bi, off, 64);
            if (ov > bv || (ov == bv && oi < bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
        if (lane == 0) {
            s_idx[j] = bi;
            s_p[j] = expf(bv - m) / sum;
        }
    }
    __syncthreads();
    if (lane == 0) {
        float tot = 0.f;
        if (renorm)
            for (int j = 0; j < k; ++j) tot += s_p[j];
        for (int j = 0; j < k; ++j) {
            const float p = renorm ? s_p[j] / tot : s_p[j];
            idx[(size_t)t * k + j] = s_idx[j];
            const float r = rnd_act<DT>(p);
            if (wout != nullptr) st_act<DT>(wout, (size_t)t * k + j, p);
            if (w32 != nullptr) w32[(size_t)t * k + j] = r;
        }
    }
}

// HOBBIT levels + resident-copy choice + kernel tables for one token (k <= 64), one wave
__global__ __launch_bounds__(64) void k_decide_table(const int64_t *__restrict__ idx, const float *__restrict__ w32,
                                                     int k, moehip_policy pol, int lv0, int lv1, int lv2,
                                                     const int64_t *__restrict__ rtab, int P, int E,
                                                     const int64_t *__restrict__ offs, const int *__restrict__ planned,
                                                     int64_t *__restrict__ tab, float *__restrict__ wtab,
                                                     float *__restrict__ info, float *__restrict__ miss) {
    const int j = threadIdx.x;
    const bool act = j < k;
    const int e = act ? (int)idx[j] : 0;
    const float wj = act ? w32[j] : 0.f;
    __shared__ float s_w[64], s_sorted[64], s_total[1];
    int lvl;
    bool skip;
    double s;
    slot_level(j, k, wj, pol, s_w, s_sorted, s_total, lvl, skip, true, &s);
    int chosen = -1;
    for (int pass = 0; pass < 2; ++pass) {
        const int req = lvl == 0 ? lv0 : (lvl == 1 ? lv1 : lv2);
        for (int pi = P - 1; pi >= 0; --pi) {
            const bool avail = act && e >= 0 && e < E && rtab[(size_t)pi * E + e] != 0;
            const bool ok = avail && (pol.upgrade ? req >= pi : req == pi);
            if (ok) chosen = pi;
        }
        // a level-0 miss below the cache-miss threshold is looked up again at level 1
        if (chosen >= 0 || !miss_downgrade(pol, lvl, s)) break;
        lvl = 1;
    }
    const bool usable = chosen >= 0 && planned[chosen];
    const bool is_miss = act && !skip && !usable;
    if (act) {
        for (int pi = 0; pi < P; ++pi) {
            const bool sel = (chosen == pi) && !skip && planned[pi];
            const int64_t base = sel ? rtab[(size_t)pi * E + e] : 0;
            for (int f = 0; f < 4; ++f) tab[((size_t)pi * k + j) * 4 + f] = sel ? base + offs[pi * 4 + f] : 0;
            wtab[(size_t)pi * k + j] = sel ? wj : 0.f;
        }
        info[j] = (float)e;
        info[k + j] = skip ? -2.f : (float)chosen;
        info[2 * k + j] = (float)lvl;
    }
    const unsigned long long bal = __ballot(is_miss);
    if (j == 0 && miss != nullptr) miss[0] += (float)__popcll(bal);
}

// ---------------------------------------------------------------------------------------
// T > 1 tokens (moelab/runtime.py:459-492 `_decide_general`): per-token levels and skip, then
// after the expert-sorted dispatch one precision per expert by vote (policy.py:148-154) and the
// per-precision record tables. The optional shared expert is slot k of every token (expert E).
// ---------------------------------------------------------------------------------------

// one block (one wave) per token: levels (T, ks) int32 and skip (T, ks) uint8; slot k < ks (the
// shared expert) is level 0 and never skipped
__global__ __launch_bounds__(64) void k_batch_levels(const float *__restrict__ w32, int k, int ks, moehip_policy pol,
                                                     int32_t *__restrict__ levels, uint8_t *__restrict__ skip) {
    const int t = blockIdx.x, j = threadIdx.x;
    const float wj = j < k ? w32[(size_t)t * ks + j] : 0.f;
    __shared__ float s_w[64], s_sorted[64], s_total[1];
    int lvl;
    bool sk;
    slot_level(j, k, wj, pol, s_w, s_sorted, s_total, lvl, sk);
    if (j < k) {
        levels[(size_t)t * ks + j] = lvl;
        skip[(size_t)t * ks + j] = sk ? 1 : 0;
    } else if (j < ks) {
        levels[(size_t)t * ks + j] = 0;
        skip[(size_t)t * ks + j] = 0;
    }
}

// one thread per expert (E routed + the shared one when has_shared): vote_expert (decide.hpp)
__global__ __launch_bounds__(64) void k_batch_vote(const int32_t *__restrict__ levels, int E, int has_shared,
                                                   const int32_t *__restrict__ offsets,
                                                   const int32_t *__restrict__ sorted_pos, double hi_vote, int upgrade,
                                                   int lv0, int lv1, int lv2, const int64_t *__restrict__ rtab,
                                                   SharedRecs srec, int P, const int64_t *__restrict__ offs,
                                                   const int *__restrict__ planned, int64_t *__restrict__ tabs,
                                                   int32_t *__restrict__ rank, float *__restrict__ info,
                                                   float *__restrict__ miss) {
    const int e = blockIdx.x * 64 + threadIdx.x;
    if (e < E + (has_shared ? 1 : 0))
        vote_expert(e, levels, E, has_shared, offsets, sorted_pos, hi_vote, upgrade, lv0, lv1, lv2, rtab, srec, P, offs,
                    planned, tabs, rank, info, miss);
}

// one wave per token: the routed slots copied into (T, k + 1) arrays and slot k = the shared
// expert (id E) with weight sigmoid(x . g), x . g rounded to the activation dtype like the shared
// gate's output and the sigmoid rounded to it too (transformers modeling_qwen3_next.py:793-796)
template <int DT>
__global__ __launch_bounds__(64) void k_shared_slot(const void *__restrict__ x, const void *__restrict__ g, int H,
                                                    const int64_t *__restrict__ idx, const float *__restrict__ w32,
                                                    int k, int E, int64_t *__restrict__ idx_ext,
                                                    float *__restrict__ w_ext) {
    const int t = blockIdx.x, lane = threadIdx.x;
    float acc = 0.f;
    if constexpr (DT != MOEHIP_DT_F32) {
        if (H % 8 == 0) acc = gate_dot_wave<DT>(x, g, t, H);
    }
    if (DT == MOEHIP_DT_F32 || H % 8 != 0) {
        for (int c = lane; c < H; c += 64) acc += ld_act<DT>(x, (size_t)t * H + c) * ld_act<DT>(g, c);
        acc = wave_sum(acc);
    }
    const int ks = k + 1;
    if (lane < k) {
        idx_ext[(size_t)t * ks + lane] = idx[(size_t)t * k + lane];
        w_ext[(size_t)t * ks + lane] = w32[(size_t)t * k + lane];
    } else if (lane == k) {
        const float l = rnd_act<DT>(acc);
        idx_ext[(size_t)t * ks + k] = E;
        w_ext[(size_t)t * ks + k] = rnd_act<DT>(1.0f / (1.0f + expf(-l)));
    }
}

}  // namespace moehip

using namespace moehip;

// logits (T, E) = x Wr^T rounded to dtype: MFMA tiles from 4 tokens (16-bit, H a multiple of 512,
// 16-byte aligned rows), VALU GEMVs otherwise
void moehip::launch_router_logits(const void *x, const void *Wr, int T, int H, int E, int dtype, void *logits,
                          hipStream_t st) {
    const int vec16 = (H % 8 == 0) && ((uintptr_t)Wr % 16) == 0 && ((uintptr_t)x % 16) == 0;
    const dim3 g1((E + 3) / 4, (T + ROUTER_TT - 1) / ROUTER_TT);
    const bool mf = dtype != MOEHIP_DT_F32 && vec16 && T >= 4 && H % 512 == 0;
    const dim3 gm((T + 15) / 16, (E + 15) / 16);
    switch (dtype) {
        case MOEHIP_DT_F16:
            if (mf) hipLaunchKernelGGL((k_router_logits_mfma<MOEHIP_DT_F16>), gm, dim3(256), 0, st, x, Wr, T, H, E, logits);
            else hipLaunchKernelGGL((k_router_logits<MOEHIP_DT_F16>), g1, dim3(256), 0, st, x, Wr, T, H, E, vec16, logits);
            break;
        case MOEHIP_DT_BF16:
            if (mf) hipLaunchKernelGGL((k_router_logits_mfma<MOEHIP_DT_BF16>), gm, dim3(256), 0, st, x, Wr, T, H, E, logits);
            else hipLaunchKernelGGL((k_router_logits<MOEHIP_DT_BF16>), g1, dim3(256), 0, st, x, Wr, T, H, E, vec16, logits);
            break;
        default:
            hipLaunchKernelGGL((k_router_logits<MOEHIP_DT_F32>), g1, dim3(256), 0, st, x, Wr, T, H, E, 0, logits);
            break;
    }
}

extern "C" int moehip_router_topk(const void *x, const void *Wr, int T, int H, int E, int k, int renorm, int dtype,
                                  void *logits, int64_t *idx, void *w, float *w32, void *stream) {
    MOEHIP_REQUIRE(x && Wr && logits && idx, "router_topk: null pointer");
    MOEHIP_REQUIRE(dtype >= MOEHIP_DT_F16 && dtype <= MOEHIP_DT_F32, "router_topk: bad dtype %d", dtype);
    MOEHIP_REQUIRE(T > 0 && H > 0 && E > 0 && E <= 1024 && k > 0 && k <= 32 && k <= E,
                   "router_topk: bad sizes T=%d H=%d E=%d k=%d", T, H, E, k);
    hipStream_t st = as_stream(stream);
    launch_router_logits(x, Wr, T, H, E, dtype, logits, st);
    switch (dtype) {
        case MOEHIP_DT_F16:
            hipLaunchKernelGGL((k_router_topk<MOEHIP_DT_F16>), dim3(T), dim3(64), 0, st, logits, T, E, k, renorm, idx, w, w32);
            break;
        case MOEHIP_DT_BF16:
            hipLaunchKernelGGL((k_router_topk<MOEHIP_DT_BF16>), dim3(T), dim3(64), 0, st, logits, T, E, k, renorm, idx, w, w32);
            break;
        default:
            hipLaunchKernelGGL((k_router_topk<MOEHIP_DT_F32>), dim3(T), dim3(64), 0, st, logits, T, E, k, renorm, idx, w, w32);
            break;
    }
    return check_launch("router");
}

extern "C" int moehip_router_logits(const void *x, const void *Wr, int T, int H, int E, int dtype, void *logits,
                                    void *stream) {
    MOEHIP_REQUIRE(x && Wr && logits, "router_logits: null pointer");
    MOEHIP_REQUIRE(dtype >= MOEHIP_DT_F16 && dtype <= MOEHIP_DT_F32, "router_logits: bad dtype %d", dtype);
    MOEHIP_REQUIRE(T > 0 && H > 0 && E > 0 && E <= 1024, "router_logits: bad sizes T=%d H=%d E=%d", T, H, E);
    launch_router_logits(x, Wr, T, H, E, dtype, logits, as_stream(stream));
    return check_launch("router_logits");
}

extern "C" int moehip_decide_table(const int64_t *idx, const float *w32, int k, const moehip_policy *pol,
                                   const int *lv2p, const int64_t *rtab, int P, int E, const int64_t *offs,
                                   const int *planned, int64_t *tab, float *wtab, float *info, float *miss,
                                   void *stream) {
    MOEHIP_REQUIRE(idx && w32 && pol && lv2p && rtab && offs && planned && tab && wtab && info,
                   "decide_table: null pointer");
    MOEHIP_REQUIRE(k > 0 && k <= 64 && P > 0 && P <= 8 && E > 0, "decide_table: bad sizes k=%d P=%d E=%d", k, P, E);
    for (int i = 0; i < 3; ++i) MOEHIP_REQUIRE(lv2p[i] >= 0 && lv2p[i] < P, "decide_table: lv2p[%d]=%d", i, lv2p[i]);
    hipLaunchKernelGGL(k_decide_table, dim3(1), dim3(64), 0, as_stream(stream), idx, w32, k, *pol, lv2p[0], lv2p[1],
                       lv2p[2], rtab, P, E, offs, planned, tab, wtab, info, miss);
    return check_launch("decide_table");
}

extern "C" int moehip_batch_levels(const float *w32, int T, int k, int ks, const moehip_policy *pol, int32_t *levels,
                                   uint8_t *skip, void *stream) {
    MOEHIP_REQUIRE(w32 && pol && levels && skip, "batch_levels: null pointer");
    MOEHIP_REQUIRE(T > 0 && k > 0 && k <= 64 && ks >= k && ks <= 64, "batch_levels: T=%d k=%d ks=%d", T, k, ks);
    hipLaunchKernelGGL(k_batch_levels, dim3(T), dim3(64), 0, as_stream(stream), w32, k, ks, *pol, levels, skip);
    return check_launch("batch_levels");
}

extern "C" int moehip_batch_vote(const int32_t *levels, int E, int has_shared, const int32_t *offsets,
                                 const int32_t *sorted_pos, double hi_vote, const moehip_policy *pol, const int *lv2p,
                                 const int64_t *rtab, const int64_t *shared_rec, int P, const int64_t *offs,
                                 const int *planned, int64_t *tabs, int32_t *rank, float *info, float *miss,
                                 void *stream) {
    MOEHIP_REQUIRE(levels && offsets && sorted_pos && pol && lv2p && rtab && offs && planned && tabs && rank,
                   "batch_vote: null pointer");
    MOEHIP_REQUIRE(E > 0 && P > 0 && P <= 4, "batch_vote: E=%d P=%d (1..4 precisions)", E, P);
    MOEHIP_REQUIRE(!has_shared || shared_rec != nullptr, "batch_vote: shared expert without records");
    for (int i = 0; i < 3; ++i) MOEHIP_REQUIRE(lv2p[i] >= 0 && lv2p[i] < P, "batch_vote: lv2p[%d]=%d", i, lv2p[i]);
    SharedRecs sr = {{0, 0, 0, 0}};
    if (has_shared)
        for (int p = 0; p < P; ++p) sr.r[p] = shared_rec[p];
    const int EA = E + (has_shared ? 1 : 0);
    hipLaunchKernelGGL(k_batch_vote, dim3((EA + 63) / 64), dim3(64), 0, as_stream(stream), levels, E, has_shared ? 1 : 0,
                       offsets, sorted_pos, hi_vote, pol->upgrade, lv2p[0], lv2p[1], lv2p[2], rtab, sr, P, offs, planned,
                       tabs, rank, info, miss);
    return check_launch("batch_vote");
}

extern "C" int moehip_shared_slot(const void *x, const void *gate, int T, int H, int dtype, const int64_t *idx,
                                  const float *w32, int k, int E, int64_t *idx_ext, float *w_ext, void *stream) {
    MOEHIP_REQUIRE(x && gate && idx && w32 && idx_ext && w_ext, "shared_slot: null pointer");
    MOEHIP_REQUIRE(T > 0 && H > 0 && k > 0 && k < 64 && E > 0, "shared_slot: T=%d H=%d k=%d E=%d", T, H, k, E);
    MOEHIP_REQUIRE(((uintptr_t)x % 16) == 0 && ((uintptr_t)gate % 16) == 0, "shared_slot: x and gate must be 16-byte aligned");
    hipStream_t st = as_stream(stream);
    switch (dtype) {
        case MOEHIP_DT_F16:
            hipLaunchKernelGGL((k_shared_slot<MOEHIP_DT_F16>), dim3(T), dim3(64), 0, st, x, gate, H, idx, w32, k, E, idx_ext, w_ext);
            break;
        case MOEHIP_DT_BF16:
            hipLaunchKernelGGL((k_shared_slot<MOEHIP_DT_BF16>), dim3(T), dim3(64), 0, st, x, gate, H, idx, w32, k, E, idx_ext, w_ext);
            break;
        case MOEHIP_DT_F32:
            hipLaunchKernelGGL((k_shared_slot<MOEHIP_DT_F32>), dim3(T), dim3(64), 0, st, x, gate, H, idx, w32, k, E, idx_ext, w_ext);
            break;
        default:
            MOEHIP_REQUIRE(false, "shared_slot: dtype %d", dtype);
    }
    return check_launch("shared_slot");
}
