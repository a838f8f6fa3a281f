// One MoE layer for one decode token in ONE launch:
//   router logits -> softmax / top-k / renorm -> HOBBIT levels, resident copy, tables ->
//   kernel-A rows (h = silu(gate x) * up x) -> kernel-B rows (w * down h) -> combine in table order.
//
// Work distribution: every workgroup takes work items from an ordered ticket counter:
//   [router items: 4 expert rows each][up items: (table row, 16 row pairs)][down items: (table row,
//   64 output rows)]. An item only waits on items with SMALLER tickets (up waits for the routing,
//   down for all up items of its table row), and a ticket is only taken by a running workgroup,
//   so every wait is on work that is already resident and itself never waits on a larger ticket:
//   the launch always drains. Every wait is also bounded (WAIT_SPINS polls); on expiry the
//   workgroup records an error in the workspace and moves on, so no launch can hang.
//
// Cross-workgroup data (logits, tables, h, partial rows, counters) is exchanged with agent-scope
// relaxed atomic loads/stores (gfx950: global accesses with the sc1 coherence bit) ordered by the
// workgroup barrier's store wait before each counter update, so no L2 writeback/invalidate is
// needed. The last workgroup to finish resets all counters, leaving the workspace ready for the
// next launch (also under HIP-graph replay).
//
// Determinism: each output row block is summed by the last of its down items, in table order.

#include <limits.h>

#include "gemv_core.hpp"

namespace moehip {

constexpr int DL_MAXP = 4;
constexpr int DL_MAXROW = 2048;  // 64 lanes x 32 vector values per lane
constexpr int DL_MAXH = DL_MAXROW;
constexpr int UP_ROWS = 16;  // row pairs per up item (4 per wave)
constexpr int DN_ROWS = 64;  // output rows per down item (16 per wave)
constexpr int WAIT_SPINS = 1 << 22;  // x ~0.3 us per poll: a wait gives up after ~1 s
// header words, each counter on its own 128-byte line; per-row counters are 32 words apart
enum { W_TICKET = 0, W_ROUTER = 32, W_READY = 64, W_DONE = 96, W_ERR = 128, W_HDR = 160 };
constexpr int CSTRIDE = 32;  // words between consecutive up_done / dn_done counters

struct LayerArgs {
    const void *x;          // (H) activation dtype
    const void *Wr;         // (E, H) router weights, or null when idx_in/w32_in are given
    const int64_t *idx_in;  // (k) routed experts (router skipped) or null
    const float *w32_in;    // (k)
    const int64_t *rtab;    // (P, E) base addresses of this layer's resident records, 0 = absent
    int64_t offs[DL_MAXP][4];
    int prec[DL_MAXP];
    int gs_up[DL_MAXP];
    int gs_dn[DL_MAXP];
    int planned[DL_MAXP];
    int lv2p[3];
    int P, E, k, H, I, renorm, accumulate;
    moehip_policy pol;
    void *out;              // (H) activation dtype
    const void *add;        // (H) activation dtype or null
    void *logits_out;       // (E) activation dtype or null
    int64_t *idx_out;       // (k) or null
    void *w_out;            // (k) activation dtype or null
    float *w32_out;         // (k) or null
    float *info;            // (3, k) or null
    float *miss;            // (1) or null
    uint32_t *ws;           // workspace (zeroed once by the caller)
    int nub, ndb;           // up blocks per table row, down blocks
    uint32_t off_up, off_dn, off_tab, off_wtab, off_logits, off_h, off_part;  // byte offsets in ws
    uint64_t *trace;        // optional per-item trace: [ticket] = (start, end, workgroup) or null
};

// ---------------------------------------------------------------------------------------
// coherent (agent-scope) accesses
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ void st_co(float *p, float v) {
    __hip_atomic_store(reinterpret_cast<uint32_t *>(p), __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_co(const float *p) {
    return __uint_as_float(__hip_atomic_load(reinterpret_cast<uint32_t *>(const_cast<float *>(p)), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ void st_co64(int64_t *p, int64_t v) {
    __hip_atomic_store(reinterpret_cast<unsigned long long *>(p), (unsigned long long)v, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int64_t ld_co64(const int64_t *p) {
    return (int64_t)__hip_atomic_load(reinterpret_cast<unsigned long long *>(const_cast<int64_t *>(p)),
                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_co32(uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t add_co32(uint32_t *p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_co32(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until this wave's outstanding memory operations (the sc1 stores above all) have
// completed; then a workgroup barrier publishes them to the counter update that follows it.
// (__syncthreads alone is a bare s_barrier on gfx950 and does not wait for global stores.)
__device__ __forceinline__ void sync_release() {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
}

// thread 0 polls until *p >= v, backing off exponentially (s_sleep 1 .. 8, i.e. up to ~500
// cycles between polls, so hundreds of waiting workgroups do not congest the flag's memory
// channel); bounded by WAIT_SPINS polls. The caller follows with a barrier.
__device__ __forceinline__ void wait_geq(uint32_t *p, uint32_t v, uint32_t *err) {
    int nap = 1;
    for (int it = 0; it < WAIT_SPINS; ++it) {
        if (ld_co32(p) >= v) return;
        switch (nap) {  // s_sleep takes an immediate
            case 1: __builtin_amdgcn_s_sleep(1); break;
            case 2: __builtin_amdgcn_s_sleep(2); break;
            case 4: __builtin_amdgcn_s_sleep(4); break;
            case 8: __builtin_amdgcn_s_sleep(8); break;
            case 16: __builtin_amdgcn_s_sleep(16); break;
            default: __builtin_amdgcn_s_sleep(8); break;
        }
        if (nap < 8) nap <<= 1;
    }
    __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T>
__device__ __forceinline__ T *ws_ptr(const LayerArgs &a, uint32_t off) {
    return reinterpret_cast<T *>(reinterpret_cast<uint8_t *>(a.ws) + off);
}

// ---------------------------------------------------------------------------------------
// LDS staging of a vector in chunk-piece-major order: piece m (4 floats) of chunk c at
// [(m * C + c) * 4], so that a wave reading piece m of consecutive chunks is conflict free.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ int vec_slot(int idx4, int npc, int C) { return ((idx4 % npc) * C + idx4 / npc) * 4; }

// ---------------------------------------------------------------------------------------
// row engines (one wave): dot products of `nrows` weight rows (or row pairs) with the staged vector
// ---------------------------------------------------------------------------------------
// chunks per lane in the fused kernel: every lane holds 32 vector values (rows <= 2048 values)
template <int PREC> struct FusedCpl { static constexpr int v = 32 / Fmt<PREC>::VPC; };

template <int PREC>
__device__ __forceinline__ void up_rows(const uint8_t *qb, const uint8_t *sb, const float *sv, int r0, int nrows, int I, int H, int gs,
                        int lg, float *hout) {
    constexpr int VPC = Fmt<PREC>::VPC;
    constexpr int NPC = VPC / 4;
    constexpr int CPL = FusedCpl<PREC>::v;
    constexpr int D = CPL >= 4 ? 1 : 4 / CPL;  // passes in flight
    const int lane = threadIdx.x & 63;
    const int G = 1 << lg, RPW = 64 >> lg;
    const int slot = lane >> lg, cl = lane & (G - 1);
    const int C = H / VPC;
    const size_t RB = (size_t)C * 16;
    float v[CPL][VPC];
    float vs[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c = min(cl + i * G, C - 1);
        float acc = 0.f;
#pragma unroll
        for (int m = 0; m < NPC; ++m) {
            const float4 p4 = *reinterpret_cast<const float4 *>(sv + (m * C + c) * 4);
            v[i][4 * m + 0] = p4.x;
            v[i][4 * m + 1] = p4.y;
            v[i][4 * m + 2] = p4.z;
            v[i][4 * m + 3] = p4.w;
            acc += (p4.x + p4.y) + (p4.z + p4.w);
        }
        vs[i] = acc;
    }
    const int npass = (nrows + RPW - 1) / RPW;
    for (int pb = 0; pb < npass; pb += D) {
        uint4 qg[D][CPL], qu[D][CPL];
        float sg[D][CPL], su[D][CPL];
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int rp = (pb + d) * RPW + slot;
            const int r = r0 + rp;
            const bool rok = (pb + d) < npass && rp < nrows && r < I;
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const int c = cl + i * G;
                if (rok && c < C) {
                    qg[d][i] = *reinterpret_cast<const uint4 *>(qb + (size_t)r * RB + (size_t)c * 16);
                    qu[d][i] = *reinterpret_cast<const uint4 *>(qb + (size_t)(r + I) * RB + (size_t)c * 16);
                    sg[d][i] = chunk_scale<PREC>(sb, r, c, H, gs);
                    su[d][i] = chunk_scale<PREC>(sb, r + I, c, H, gs);
                } else {
                    qg[d][i] = make_uint4(0, 0, 0, 0);
                    qu[d][i] = make_uint4(0, 0, 0, 0);
                    sg[d][i] = 0.f;
                    su[d][i] = 0.f;
                }
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
            float pg = 0.f, pu = 0.f;
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                pg = fmaf(sg[d][i], chunk_dot<PREC>(qg[d][i], v[i], vs[i]), pg);
                pu = fmaf(su[d][i], chunk_dot<PREC>(qu[d][i], v[i], vs[i]), pu);
            }
            pg = group_sum(pg, lg);
            pu = group_sum(pu, lg);
            const int rp = (pb + d) * RPW + slot;
            const int r = r0 + rp;
            if (cl == 0 && (pb + d) < npass && rp < nrows && r < I) st_co(hout + r, silu_mul(pg, pu));
        }
    }
}

template <int PREC>
__device__ __forceinline__ void down_rows(const uint8_t *qb, const uint8_t *sb, const float *sv, int r0, int nrows, int H, int I,
                          int gs, int lg, float wt, float *pout) {
    constexpr int VPC = Fmt<PREC>::VPC;
    constexpr int NPC = VPC / 4;
    constexpr int CPL = FusedCpl<PREC>::v;
    constexpr int D = CPL >= 4 ? 1 : 4 / CPL;
    const int lane = threadIdx.x & 63;
    const int G = 1 << lg, RPW = 64 >> lg;
    const int slot = lane >> lg, cl = lane & (G - 1);
    const int C = I / VPC;
    const size_t RB = (size_t)C * 16;
    float v[CPL][VPC];
    float vs[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c = min(cl + i * G, C - 1);
        float acc = 0.f;
#pragma unroll
        for (int m = 0; m < NPC; ++m) {
            const float4 p4 = *reinterpret_cast<const float4 *>(sv + (m * C + c) * 4);
            v[i][4 * m + 0] = p4.x;
            v[i][4 * m + 1] = p4.y;
            v[i][4 * m + 2] = p4.z;
            v[i][4 * m + 3] = p4.w;
            acc += (p4.x + p4.y) + (p4.z + p4.w);
        }
        vs[i] = acc;
    }
    const int npass = (nrows + RPW - 1) / RPW;
    for (int pb = 0; pb < npass; pb += D) {
        uint4 qd[D][CPL];
        float sd[D][CPL];
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int rr = (pb + d) * RPW + slot;
            const int r = r0 + rr;
            const bool rok = (pb + d) < npass && rr < nrows && r < H;
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const int c = cl + i * G;
                if (rok && c < C) {
                    qd[d][i] = *reinterpret_cast<const uint4 *>(qb + (size_t)r * RB + (size_t)c * 16);
                    sd[d][i] = chunk_scale<PREC>(sb, r, c, I, gs);
                } else {
                    qd[d][i] = make_uint4(0, 0, 0, 0);
                    sd[d][i] = 0.f;
                }
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < CPL; ++i) acc = fmaf(sd[d][i], chunk_dot<PREC>(qd[d][i], v[i], vs[i]), acc);
            acc = group_sum(acc, lg);
            const int rr = (pb + d) * RPW + slot;
            const int r = r0 + rr;
            if (cl == 0 && (pb + d) < npass && rr < nrows && r < H) st_co(pout + r, wt * acc);
        }
    }
}

__device__ __forceinline__ int vpc_dev(int prec) {
    return prec == MOEHIP_PREC_INT4 ? 32 : (prec == MOEHIP_PREC_INT8 || prec == MOEHIP_PREC_FP8) ? 16
           : (prec == MOEHIP_PREC_F32 ? 4 : 8);
}

// log2 of the lanes per row for rows of `cols` values (32 values per lane)
__device__ __forceinline__ int row_lg(int cols) {
    const int lanes = (cols + 31) / 32;
    int G = 1, lg = 0;
    while (G < lanes && G < 64) G <<= 1, ++lg;
    return lg;
}

// select element i of a small argument array without dynamic indexing (kernel arguments
// indexed by a run-time value would be copied to private memory)
template <typename T>
__device__ __forceinline__ T pick4(const T (&v)[4], int i) {
    return i == 0 ? v[0] : (i == 1 ? v[1] : (i == 2 ? v[2] : v[3]));
}
__device__ __forceinline__ int64_t pick_off(const int64_t (&v)[4][4], int p, int f) {
    const int64_t r0 = f == 0 ? v[0][0] : (f == 1 ? v[0][1] : (f == 2 ? v[0][2] : v[0][3]));
    const int64_t r1 = f == 0 ? v[1][0] : (f == 1 ? v[1][1] : (f == 2 ? v[1][2] : v[1][3]));
    const int64_t r2 = f == 0 ? v[2][0] : (f == 1 ? v[2][1] : (f == 2 ? v[2][2] : v[2][3]));
    const int64_t r3 = f == 0 ? v[3][0] : (f == 1 ? v[3][1] : (f == 2 ? v[3][2] : v[3][3]));
    return p == 0 ? r0 : (p == 1 ? r1 : (p == 2 ? r2 : r3));
}

// ---------------------------------------------------------------------------------------
// route tail: softmax / top-k / renorm / HOBBIT / resident copy / tables (wave 0 of one WG)
// ---------------------------------------------------------------------------------------
template <int XDT>
__device__ __forceinline__ void route_tail(const LayerArgs &a, int *s_idx, float *s_w, float *s_l, uint64_t *ts) {
    const int lane = threadIdx.x;  // wave 0 only; s_l: E floats of LDS (+ 2 x 32 candidate slots)
    const int k = a.k, E = a.E;
    const unsigned long long lt = (1ull << lane) - 1ull;  // lanes below this one
#define TS(i) do { if (ts != nullptr && lane == 0) ts[i] = __builtin_amdgcn_s_memrealtime(); } while (0)
    TS(0);
    if (a.Wr != nullptr) {
        const float *logits = ws_ptr<float>(a, a.off_logits);
        float m = -INFINITY;
        for (int c = lane; c < E; c += 64) {
            const float v = ld_co(logits + c);
            s_l[c] = v;
            m = fmaxf(m, v);
            if (a.logits_out != nullptr) st_act<XDT>(a.logits_out, c, v);
        }
        m = wave_max(m);
        TS(1);
        float sum = 0.f;
        for (int c = lane; c < E; c += 64) sum += expf(s_l[c] - m);
        sum = wave_sum(sum);
        // k-th largest logit by radix select over order-preserving keys (MSB first)
        uint32_t prefix = 0, mask = 0;
        int need = k;
        for (int b = 31; b >= 0; --b) {
            const uint32_t bit = 1u << b, cand = prefix | bit, m2 = mask | bit;
            int cnt = 0;
            for (int c = lane; c < E; c += 64) cnt += (fkey(s_l[c]) & m2) == cand;
            cnt = wave_sum_i(cnt);
            if (cnt >= need) prefix = cand;
            else need -= cnt;
            mask = m2;
        }
        // the k winners: every key above the k-th, then the `need` lowest-index keys equal to it
        float *cv = s_l + E;                              // candidate values
        int *ci = reinterpret_cast<int *>(s_l + E + 32);  // candidate indices
        int nsel = 0, neq = 0;
        for (int c0 = 0; c0 < E; c0 += 64) {
            const int c = c0 + lane;
            const uint32_t key = c < E ? fkey(s_l[c]) : 0u;
            const bool gt = c < E && key > prefix;
            const bool eq = c < E && key == prefix;
            const unsigned long long eqm = __ballot(eq);
            const bool sel = gt || (eq && neq + __popcll(eqm & lt) < need);
            const unsigned long long sm = __ballot(sel);
            if (sel) {
                const int pos = nsel + __popcll(sm & lt);
                cv[pos] = s_l[c];
                ci[pos] = c;
            }
            nsel += __popcll(sm);
            neq += __popcll(eqm);
        }
        __builtin_amdgcn_wave_barrier();
        // order the winners by (logit desc, index asc), probabilities, renorm, outputs
        float p = 0.f;
        int rank = 0, myidx = 0;
        if (lane < k) {
            const float v = cv[lane];
            myidx = ci[lane];
            for (int i = 0; i < k; ++i) {
                const float o = cv[i];
                rank += (o > v) || (o == v && ci[i] < myidx);
            }
            p = expf(v - m) / sum;
        }
        const float tot = a.renorm ? wave_sum(lane < k ? p : 0.f) : 1.f;
        TS(2);
        if (lane < k) {
            const float pw = a.renorm ? p / tot : p;
            const float r = rnd_act<XDT>(pw);
            s_idx[rank] = myidx;
            s_w[rank] = r;
            if (a.idx_out) a.idx_out[rank] = myidx;
            if (a.w_out) st_act<XDT>(a.w_out, rank, pw);
            if (a.w32_out) a.w32_out[rank] = r;
        }
    } else if (lane < k) {
        s_idx[lane] = (int)a.idx_in[lane];
        s_w[lane] = a.w32_in[lane];
    }
    __builtin_amdgcn_wave_barrier();
    TS(3);
    // HOBBIT levels (moelab/policy.py:77-123), resident copy, tables (moelab/fullgraph.py:149-171)
    float *s_sorted = s_l;  // reused: k floats
    const int j = lane;
    const bool act = j < k;
    const int e = act ? s_idx[j] : 0;
    const float wj = act ? s_w[j] : 0.f;
    float tot = 0.f;
    for (int i = 0; i < k; ++i) tot += s_w[i];
    tot = fmaxf(tot, 1e-12f);
    int lvl;
    bool skip = false;
    const moehip_policy pol = a.pol;
    if (pol.mode == 1 || pol.protect) {
        lvl = 0;
    } else if (pol.mode == 2) {
        lvl = 2;
    } else {
        const float wn = wj / tot;
        int rank = 0;
        for (int i = 0; i < k; ++i) {
            const float o = s_w[i] / tot;
            rank += (o > wn) || (o == wn && i < j);
        }
        __builtin_amdgcn_wave_barrier();
        if (act) s_sorted[rank] = wn;
        __builtin_amdgcn_wave_barrier();
        float cs = 0.f;
        for (int r = 0; r <= rank && r < k; ++r) cs += s_sorted[r];
        const float s = cs - wn;
        lvl = 2;
        if (pol.t_mid >= 0.f && s <= pol.t_mid) lvl = 1;
        if (s <= pol.t1) lvl = 0;
        skip = pol.t2 >= 0.f && s > pol.t2 && lvl != 0;
    }
    TS(4);
    const int req = lvl == 0 ? a.lv2p[0] : (lvl == 1 ? a.lv2p[1] : a.lv2p[2]);
    int chosen = -1;
    for (int pi = a.P - 1; pi >= 0; --pi) {
        const bool avail = act && e >= 0 && e < E && a.rtab[(size_t)pi * E + e] != 0;
        if (avail && (pol.upgrade ? req >= pi : req == pi)) chosen = pi;
    }
    TS(5);
    const bool usable = chosen >= 0 && pick4(a.planned, chosen) != 0;
    const bool is_miss = act && !skip && !usable;
    int64_t *tab = ws_ptr<int64_t>(a, a.off_tab);
    float *wtab = ws_ptr<float>(a, a.off_wtab);
    if (act) {
        for (int pi = 0; pi < a.P; ++pi) {
            const bool sel = chosen == pi && !skip && pick4(a.planned, pi) != 0;
            const int64_t base = sel ? a.rtab[(size_t)pi * E + e] : 0;
            for (int f = 0; f < 4; ++f)
                st_co64(tab + ((size_t)pi * k + j) * 4 + f, sel ? base + pick_off(a.offs, pi, f) : 0);
            st_co(wtab + (size_t)pi * k + j, sel ? wj : 0.f);
        }
        if (a.info) {
            a.info[j] = (float)e;
            a.info[k + j] = skip ? -2.f : (float)chosen;
            a.info[2 * k + j] = (float)lvl;
        }
    }
    TS(6);
    const unsigned long long bal = __ballot(is_miss);
    if (j == 0 && a.miss != nullptr) a.miss[0] += (float)__popcll(bal);
    TS(7);
#undef TS
}

// ---------------------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------------------
template <int XDT>
__global__ __launch_bounds__(256) void k_decode_layer(LayerArgs a) {
    __shared__ __align__(16) float s_vec[DL_MAXH];  // x (up items) or h (down items), piece-major
    __shared__ int s_item, s_next, s_flag, s_fmt, s_routed;
    __shared__ int s_idx[64];
    __shared__ float s_w[64];
    __shared__ float s_wt[DL_MAXP * 32];          // route cached per workgroup: table weights
    __shared__ uint64_t s_tab[DL_MAXP * 32 * 4];  // and addresses
    const int tid = threadIdx.x, wave = tid >> 6;
    uint32_t *ws = a.ws;
    uint32_t *err = ws + W_ERR;
    const int PK = a.P * a.k;
    const int NR = a.Wr != nullptr ? (a.E + 3) / 4 : 1;
    const int NU = PK * a.nub;
    const int ND = PK * a.ndb;
    const int total = NR + NU + ND;
    uint32_t *up_done = ws_ptr<uint32_t>(a, a.off_up);
    uint32_t *dn_done = ws_ptr<uint32_t>(a, a.off_dn);
    int64_t *tab = ws_ptr<int64_t>(a, a.off_tab);
    float *wtab = ws_ptr<float>(a, a.off_wtab);
    float *hbuf = ws_ptr<float>(a, a.off_h);
    float *part = ws_ptr<float>(a, a.off_part);
    if (tid == 0) {
        s_fmt = -1;  // which layout s_vec holds: VPC of staged x, or -1
        s_routed = 0;
        s_next = (int)add_co32(ws + W_TICKET, 1u);
    }
    for (;;) {
        __syncthreads();
        if (tid == 0) {
            // take the reserved ticket and reserve the next one (its round trip overlaps the work)
            s_item = s_next;
            s_next = s_item < total ? (int)add_co32(ws + W_TICKET, 1u) : total;
        }
        __syncthreads();
        const int t = s_item;
        if (t >= total) break;
        uint64_t t_start = 0;
        if (a.trace != nullptr && tid == 0) t_start = __builtin_amdgcn_s_memrealtime();
        if (t < NR) {
            // ---------------- router rows ----------------
            if (a.Wr != nullptr) {
                const int e = t * 4 + wave;
                const int lane = tid & 63;
                if (e < a.E) {
                    // each lane: 32 consecutive values (H <= 2048), all loads issued before use
                    constexpr int ESZ = XDT == MOEHIP_DT_F32 ? 4 : 2;
                    constexpr int NV = 32 * ESZ / 16;  // 16-byte vectors per lane
                    const int c0 = lane * 32;
                    float acc = 0.f;
                    if (c0 < a.H) {
                        const uint8_t *wp = reinterpret_cast<const uint8_t *>(a.Wr) + ((size_t)e * a.H + c0) * ESZ;
                        const uint8_t *xp = reinterpret_cast<const uint8_t *>(a.x) + (size_t)c0 * ESZ;
                        uint4 wv[NV], xv[NV];
#pragma unroll
                        for (int i = 0; i < NV; ++i) {
                            wv[i] = reinterpret_cast<const uint4 *>(wp)[i];
                            xv[i] = reinterpret_cast<const uint4 *>(xp)[i];
                        }
#pragma unroll
                        for (int i = 0; i < NV; ++i) {
                            const uint32_t wd[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
                            const uint32_t xd[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                if constexpr (XDT == MOEHIP_DT_F32) {
                                    acc = fmaf(__uint_as_float(wd[q]), __uint_as_float(xd[q]), acc);
                                } else if constexpr (XDT == MOEHIP_DT_F16) {
                                    acc = fmaf(f16_to_f32(wd[q] & 0xffffu), f16_to_f32(xd[q] & 0xffffu), acc);
                                    acc = fmaf(f16_to_f32(wd[q] >> 16), f16_to_f32(xd[q] >> 16), acc);
                                } else {
                                    acc = fmaf(__uint_as_float(wd[q] << 16), __uint_as_float(xd[q] << 16), acc);
                                    acc = fmaf(__uint_as_float(wd[q] & 0xffff0000u), __uint_as_float(xd[q] & 0xffff0000u), acc);
                                }
                            }
                        }
                    }
                    acc = wave_sum(acc);
                    if (lane == 0) st_co(ws_ptr<float>(a, a.off_logits) + e, rnd_act<XDT>(acc));
                }
            }
            sync_release();
            if (tid == 0) s_flag = (add_co32(ws + W_ROUTER, 1u) == (uint32_t)(NR - 1));
            __syncthreads();
            if (s_flag) {
                if (wave == 0) route_tail<XDT>(a, s_idx, s_w, s_vec, a.trace ? a.trace + 3 * total : nullptr);
                sync_release();
                if (tid == 0) {
                    if (a.trace) a.trace[3 * total + 8] = __builtin_amdgcn_s_memrealtime();
                    st_co32(ws + W_READY, 1u);
                    s_fmt = -1;  // s_vec held the logits: no staged x any more
                }
            }
        } else if (t < NR + NU) {
            // ---------------- kernel-A rows ----------------
            const int u = t - NR;
            const int jj = u / a.nub, rb = u % a.nub;
            const int pi = jj / a.k;
            const int prec = pick4(a.prec, pi);
            const int vpc = vpc_dev(prec);
            if (s_fmt != vpc) {  // stage x in the piece-major layout of this format
                const int C = a.H / vpc;
                const int npc = vpc / 4;
                for (int i4 = tid; i4 < a.H / 4; i4 += 256) {
                    const int dst = vec_slot(i4, npc, C);
                    float4 p4;
                    if constexpr (XDT == MOEHIP_DT_F32) {
                        p4 = reinterpret_cast<const float4 *>(a.x)[i4];
                    } else {
                        const uint2 r = reinterpret_cast<const uint2 *>(a.x)[i4];
                        if constexpr (XDT == MOEHIP_DT_F16) {
                            p4 = make_float4(f16_to_f32(r.x & 0xffffu), f16_to_f32(r.x >> 16), f16_to_f32(r.y & 0xffffu),
                                             f16_to_f32(r.y >> 16));
                        } else {
                            p4 = make_float4(__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u),
                                             __uint_as_float(r.y << 16), __uint_as_float(r.y & 0xffff0000u));
                        }
                    }
                    *reinterpret_cast<float4 *>(s_vec + dst) = p4;
                }
                __syncthreads();
                if (tid == 0) s_fmt = vpc;
            }
            if (!s_routed) {  // first item after the routing: cache the tables in LDS
                if (tid == 0) wait_geq(ws + W_READY, 1u, err);
                __syncthreads();
                for (int i = tid; i < PK; i += 256) s_wt[i] = ld_co(wtab + i);
                for (int i = tid; i < PK * 4; i += 256) s_tab[i] = (uint64_t)ld_co64(tab + i);
                __syncthreads();
                if (tid == 0) s_routed = 1;
            }
            const float wt = s_wt[jj];
            if (wt != 0.f) {
                const uint8_t *qb = reinterpret_cast<const uint8_t *>(s_tab[(size_t)jj * 4 + 0]);
                const uint8_t *sb = reinterpret_cast<const uint8_t *>(s_tab[(size_t)jj * 4 + 1]);
                const int lg = row_lg(a.H);
                const int r0 = rb * UP_ROWS + wave * (UP_ROWS / 4);
                float *hout = hbuf + (size_t)jj * a.I;
                const int gs = pick4(a.gs_up, pi);
                constexpr int NR4 = UP_ROWS / 4;
                switch (prec) {
                    case MOEHIP_PREC_INT4: up_rows<MOEHIP_PREC_INT4>(qb, sb, s_vec, r0, NR4, a.I, a.H, gs, lg, hout); break;
                    case MOEHIP_PREC_INT8: up_rows<MOEHIP_PREC_INT8>(qb, sb, s_vec, r0, NR4, a.I, a.H, gs, lg, hout); break;
                    case MOEHIP_PREC_F16: up_rows<MOEHIP_PREC_F16>(qb, sb, s_vec, r0, NR4, a.I, a.H, gs, lg, hout); break;
                    case MOEHIP_PREC_BF16: up_rows<MOEHIP_PREC_BF16>(qb, sb, s_vec, r0, NR4, a.I, a.H, gs, lg, hout); break;
                    default: up_rows<MOEHIP_PREC_FP8>(qb, sb, s_vec, r0, NR4, a.I, a.H, gs, lg, hout); break;
                }
                sync_release();
                if (tid == 0) add_co32(up_done + jj * CSTRIDE, 1u);
            }
        } else {
            // ---------------- kernel-B rows + ordered combine ----------------
            const int d = t - NR - NU;
            const int jj = d / a.ndb, rb = d % a.ndb;
            const int pi = jj / a.k;
            const int prec = pick4(a.prec, pi);
            if (!s_routed) {
                if (tid == 0) wait_geq(ws + W_READY, 1u, err);
                __syncthreads();
                for (int i = tid; i < PK; i += 256) s_wt[i] = ld_co(wtab + i);
                for (int i = tid; i < PK * 4; i += 256) s_tab[i] = (uint64_t)ld_co64(tab + i);
                __syncthreads();
                if (tid == 0) s_routed = 1;
            }
            const float wt = s_wt[jj];
            if (wt != 0.f) {
                if (tid == 0) wait_geq(up_done + jj * CSTRIDE, (uint32_t)a.nub, err);
                __syncthreads();
                const int vpc = vpc_dev(prec);
                const int C = a.I / vpc;
                const int npc = vpc / 4;
                const float *hj = hbuf + (size_t)jj * a.I;
                for (int i4 = tid; i4 < a.I / 4; i4 += 256) {
                    const int dst = vec_slot(i4, npc, C);
                    s_vec[dst + 0] = ld_co(hj + 4 * i4 + 0);
                    s_vec[dst + 1] = ld_co(hj + 4 * i4 + 1);
                    s_vec[dst + 2] = ld_co(hj + 4 * i4 + 2);
                    s_vec[dst + 3] = ld_co(hj + 4 * i4 + 3);
                }
                if (tid == 0) s_fmt = -1;
                __syncthreads();
                const uint8_t *qb = reinterpret_cast<const uint8_t *>(s_tab[(size_t)jj * 4 + 2]);
                const uint8_t *sb = reinterpret_cast<const uint8_t *>(s_tab[(size_t)jj * 4 + 3]);
                const int lg = row_lg(a.I);
                const int r0 = rb * DN_ROWS + wave * (DN_ROWS / 4);
                float *pout = part + (size_t)jj * a.H;
                const int gs = pick4(a.gs_dn, pi);
                constexpr int NR4 = DN_ROWS / 4;
                switch (prec) {
                    case MOEHIP_PREC_INT4: down_rows<MOEHIP_PREC_INT4>(qb, sb, s_vec, r0, NR4, a.H, a.I, gs, lg, wt, pout); break;
                    case MOEHIP_PREC_INT8: down_rows<MOEHIP_PREC_INT8>(qb, sb, s_vec, r0, NR4, a.H, a.I, gs, lg, wt, pout); break;
                    case MOEHIP_PREC_F16: down_rows<MOEHIP_PREC_F16>(qb, sb, s_vec, r0, NR4, a.H, a.I, gs, lg, wt, pout); break;
                    case MOEHIP_PREC_BF16: down_rows<MOEHIP_PREC_BF16>(qb, sb, s_vec, r0, NR4, a.H, a.I, gs, lg, wt, pout); break;
                    default: down_rows<MOEHIP_PREC_FP8>(qb, sb, s_vec, r0, NR4, a.H, a.I, gs, lg, wt, pout); break;
                }
            }
            sync_release();
            if (tid == 0) s_flag = (add_co32(dn_done + rb * CSTRIDE, 1u) == (uint32_t)(PK - 1));
            __syncthreads();
            if (s_flag && tid < DN_ROWS) {
                const int r = rb * DN_ROWS + tid;
                if (r < a.H) {
                    float s = 0.f;
                    for (int q = 0; q < PK; ++q)
                        if (s_wt[q] != 0.f) s += ld_co(part + (size_t)q * a.H + r);
                    if (a.accumulate) s += ld_act<XDT>(a.out, r);
                    if (a.add != nullptr) s += ld_act<XDT>(a.add, r);
                    st_act<XDT>(a.out, r, s);
                }
            }
        }
        if (a.trace != nullptr && tid == 0) {
            a.trace[3 * t + 0] = t_start;
            a.trace[3 * t + 1] = __builtin_amdgcn_s_memrealtime();
            a.trace[3 * t + 2] = blockIdx.x;
        }
    }
    // every workgroup has taken its last ticket; the last one resets the counters
    if (tid == 0) s_flag = (add_co32(ws + W_DONE, 1u) == gridDim.x - 1);
    __syncthreads();
    if (s_flag) {
        for (int i = tid; i < PK; i += 256) st_co32(up_done + i * CSTRIDE, 0u);
        for (int i = tid; i < a.ndb; i += 256) st_co32(dn_done + i * CSTRIDE, 0u);
        if (tid == 0) {
            st_co32(ws + W_TICKET, 0u);
            st_co32(ws + W_ROUTER, 0u);
            st_co32(ws + W_READY, 0u);
            st_co32(ws + W_DONE, 0u);
        }
    }
}

// workspace layout (bytes)
struct DlLayout {
    uint32_t up, dn, tab, wtab, logits, h, part, total;
    int nub, ndb;
};

static inline uint32_t al256(size_t v) { return (uint32_t)((v + 255) / 256 * 256); }

static DlLayout dl_layout(int P, int k, int E, int H, int I) {
    DlLayout L;
    const int PK = P * k;
    L.nub = (I + UP_ROWS - 1) / UP_ROWS;
    L.ndb = (H + DN_ROWS - 1) / DN_ROWS;
    size_t off = W_HDR * 4;
    L.up = (uint32_t)off;
    off += (size_t)PK * CSTRIDE * 4;
    L.dn = (uint32_t)off;
    off += (size_t)L.ndb * CSTRIDE * 4;
    off = al256(off);
    L.tab = (uint32_t)off;
    off += (size_t)PK * 32;
    L.wtab = (uint32_t)off;
    off += (size_t)PK * 4;
    L.logits = (uint32_t)off;
    off += (size_t)E * 4;
    off = al256(off);
    L.h = (uint32_t)off;
    off += (size_t)PK * I * 4;
    off = al256(off);
    L.part = (uint32_t)off;
    off += (size_t)PK * H * 4;
    L.total = al256(off);
    return L;
}

}  // namespace moehip

using namespace moehip;

extern "C" size_t moehip_decode_layer_workspace_bytes(int P, int k, int E, int H, int I) {
    if (P <= 0 || k <= 0 || E <= 0 || H <= 0 || I <= 0) return 0;
    return dl_layout(P, k, E, H, I).total;
}

extern "C" int moehip_decode_layer(const moehip_layer_desc *d, const void *x, const void *Wr, const int64_t *idx_in,
                                   const float *w32_in, const int64_t *rtab, void *out, const void *add,
                                   int accumulate, void *logits_out, int64_t *idx_out, void *w_out, float *w32_out,
                                   float *info, float *miss, void *ws, size_t ws_bytes, int grid, uint64_t *trace,
                                   void *stream) {
    MOEHIP_REQUIRE(d && x && rtab && out && ws, "decode_layer: null pointer");
    MOEHIP_REQUIRE(Wr != nullptr || (idx_in != nullptr && w32_in != nullptr),
                   "decode_layer: need router weights or precomputed idx/w32");
    MOEHIP_REQUIRE(d->P > 0 && d->P <= DL_MAXP, "decode_layer: P=%d (1..%d)", d->P, DL_MAXP);
    MOEHIP_REQUIRE(d->k > 0 && d->k <= 32 && d->k <= d->E && d->E <= 1024, "decode_layer: k=%d E=%d", d->k, d->E);
    MOEHIP_REQUIRE(d->H > 0 && d->H <= DL_MAXROW && d->H % 32 == 0, "decode_layer: H=%d (multiple of 32, <= %d)",
                   d->H, DL_MAXROW);
    MOEHIP_REQUIRE(d->I > 0 && d->I <= DL_MAXROW && d->I % 32 == 0, "decode_layer: I=%d (multiple of 32, <= %d)",
                   d->I, DL_MAXROW);
    MOEHIP_REQUIRE(d->dtype >= MOEHIP_DT_F16 && d->dtype <= MOEHIP_DT_F32, "decode_layer: dtype %d", d->dtype);
    for (int i = 0; i < 3; ++i)
        MOEHIP_REQUIRE(d->lv2p[i] >= 0 && d->lv2p[i] < d->P, "decode_layer: lv2p[%d]=%d", i, d->lv2p[i]);
    for (int p = 0; p < d->P; ++p) {
        const int pr = d->prec[p];
        MOEHIP_REQUIRE(pr >= MOEHIP_PREC_INT4 && pr <= MOEHIP_PREC_FP8 && pr != MOEHIP_PREC_F32,
                       "decode_layer: precision %d (fp32 records use the grouped kernels)", pr);
        const int vpc = pr == MOEHIP_PREC_INT4 ? 32 : (pr == MOEHIP_PREC_INT8 || pr == MOEHIP_PREC_FP8) ? 16
                        : (pr == MOEHIP_PREC_F32 ? 4 : 8);
        (void)vpc;
        if (pr == MOEHIP_PREC_INT4 || pr == MOEHIP_PREC_INT8) {
            const int vpc = pr == MOEHIP_PREC_INT4 ? 32 : 16;
            MOEHIP_REQUIRE(d->gs_up[p] > 0 && d->gs_up[p] % vpc == 0 && d->H % d->gs_up[p] == 0 && d->gs_dn[p] > 0 &&
                               d->gs_dn[p] % vpc == 0 && d->I % d->gs_dn[p] == 0,
                           "decode_layer: group sizes %d/%d need multiples of %d dividing H/I", d->gs_up[p],
                           d->gs_dn[p], vpc);
        }
    }
    const DlLayout L = dl_layout(d->P, d->k, d->E, d->H, d->I);
    MOEHIP_REQUIRE(ws_bytes >= L.total, "decode_layer: workspace %zu bytes < %u", ws_bytes, L.total);
    MOEHIP_REQUIRE(((uintptr_t)ws % 256) == 0, "decode_layer: workspace must be 256-byte aligned");
    MOEHIP_REQUIRE(((uintptr_t)x % 16) == 0 && ((uintptr_t)Wr % 16) == 0, "decode_layer: x and Wr must be 16-byte aligned");
    LayerArgs a;
    a.x = x;
    a.Wr = Wr;
    a.idx_in = idx_in;
    a.w32_in = w32_in;
    a.rtab = rtab;
    for (int p = 0; p < DL_MAXP; ++p) {
        for (int f = 0; f < 4; ++f) a.offs[p][f] = p < d->P ? d->offs[p][f] : 0;
        a.prec[p] = p < d->P ? d->prec[p] : 0;
        a.gs_up[p] = p < d->P ? d->gs_up[p] : 0;
        a.gs_dn[p] = p < d->P ? d->gs_dn[p] : 0;
        a.planned[p] = p < d->P ? d->planned[p] : 0;
    }
    for (int i = 0; i < 3; ++i) a.lv2p[i] = d->lv2p[i];
    a.P = d->P;
    a.E = d->E;
    a.k = d->k;
    a.H = d->H;
    a.I = d->I;
    a.renorm = d->renorm;
    a.accumulate = accumulate;
    a.pol = d->pol;
    a.out = out;
    a.add = add;
    a.logits_out = logits_out;
    a.idx_out = idx_out;
    a.w_out = w_out;
    a.w32_out = w32_out;
    a.info = info;
    a.miss = miss;
    a.ws = reinterpret_cast<uint32_t *>(ws);
    a.nub = L.nub;
    a.ndb = L.ndb;
    a.off_up = L.up;
    a.off_dn = L.dn;
    a.off_tab = L.tab;
    a.off_wtab = L.wtab;
    a.off_logits = L.logits;
    a.off_h = L.h;
    a.off_part = L.part;
    a.trace = trace;
    const int PK = d->P * d->k;
    const int total = (Wr != nullptr ? (d->E + 3) / 4 : 1) + PK * (L.nub + L.ndb);
    const int g = grid > 0 ? (grid < total ? grid : total) : total;
    hipStream_t st = as_stream(stream);
    switch (d->dtype) {
        case MOEHIP_DT_F16: hipLaunchKernelGGL((k_decode_layer<MOEHIP_DT_F16>), dim3(g), dim3(256), 0, st, a); break;
        case MOEHIP_DT_BF16: hipLaunchKernelGGL((k_decode_layer<MOEHIP_DT_BF16>), dim3(g), dim3(256), 0, st, a); break;
        default: hipLaunchKernelGGL((k_decode_layer<MOEHIP_DT_F32>), dim3(g), dim3(256), 0, st, a); break;
    }
    return check_launch("decode_layer");
}

extern "C" int moehip_decode_layer_error(const void *ws, void *flag_out, void *stream) {
    MOEHIP_REQUIRE(ws && flag_out, "decode_layer_error: null pointer");
    const hipError_t e = hipMemcpyAsync(flag_out, reinterpret_cast<const uint32_t *>(ws) + W_ERR, 4,
                                        hipMemcpyDeviceToDevice, as_stream(stream));
    if (e != hipSuccess) {
        set_error("decode_layer_error: %s", hipGetErrorString(e));
        return MOEHIP_ELAUNCH;
    }
    return MOEHIP_OK;
}
