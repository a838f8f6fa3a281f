// One MoE layer for one decode token in ONE launch, organised XCD by XCD (one record precision,
// 16-bit activations: every benchmarked bs=1 configuration).
//
// The MI355X dispatches workgroup b to XCD b % 8 (checked once per device by
// moehip_device_check; where it does not hold, the item-loop kernel of decode_layer.hip runs).
// A word written by a CU is seen by another CU of the same XCD through that XCD's L2 in ~0.2 us
// (plain store, non-temporal load), while an agent-scope exchange between XCDs takes ~0.7-1 us
// under the load of hundreds of pollers. So every exchange but the last stays inside an XCD:
//
//   1. routing, replicated per XCD: the workgroups of an XCD compute the E router logits (and the
//      Qwen3-Next shared gate) between them, each into its XCD's copy, and every workgroup reads
//      all of them back and ranks them itself (softmax, top-k, renorm, HOBBIT, the record of each
//      table row);
//   2. the table rows' h values (k routed + shared, I each, flattened row after row) are cut into
//      8 contiguous segments, one per XCD; the XCD's up items produce its segment's
//      h = w * silu(gate x) * (up x) into the XCD's h area (w = the row's routed weight);
//   3. the XCD's down items each hold DR output rows and multiply the down columns of the segment
//      with h: a partial output of the whole layer restricted to the segment;
//   4. the one exchange between XCDs: the partial rows of the 8 XCDs, summed in XCD order by the
//      down item of XCD d % 8 for its row block d, plus add / accumulate, cast to the output dtype.
//
// Cross-workgroup words are tagged ((launch tag << 32) | payload): inside an XCD written with
// plain stores and polled with non-temporal loads (which do not allocate in the CU's L1, so each
// poll reaches the XCD's L2); between XCDs written and read at agent scope. A launch's tag is the
// workspace generation + 1, read by every workgroup at start; workgroups 0..15 advance it once
// every workgroup has counted itself as having read it (the scheme of the item-loop kernel, same
// header words). Every wait is bounded: on expiry the workspace error flag is set and NaN goes where
// the missing data would have gone (routed weights, partial rows, output rows), so a launch never
// hangs and never returns a plausible wrong answer.
//
// Co-residency: the grid (8 x items per XCD) never exceeds what the GPU holds at once.

#include "decide.hpp"
#include "lanevec.hpp"

namespace moehip {

constexpr int XC_N = 8;            // XCDs
constexpr int XC_SPIN = 1 << 21;   // polls before a wait gives up (~1 s)
constexpr int XC_NGEN = 16;        // header as in decode_layer.hip: reader counters, error flag,
constexpr int XC_NSUB = 16;        // drained count, generation copies 1 KB apart
enum { XC_READ = 0, XC_ERR = XC_NSUB * 32, XC_TOP = XC_NSUB * 32 + 32, XC_GEN = 1024, XC_HDR = XC_GEN + 256 * XC_NGEN };
constexpr int XC_MAXE = 1024;
constexpr int XC_MAXKS = 33;
constexpr int XC_LDS_H = 8192;     // h values of one XCD's segment staged in LDS (fp32)
constexpr int XC_MAXDR = 512;      // output rows of one down item

struct XcArgs {
    const void *x;            // (H) activation dtype, 16-byte aligned
    const void *Wr;           // (E, H) router weights or null
    const void *sgate;        // (H) shared-expert gate or null
    const int64_t *idx_in;    // (k) routing given (router skipped) or null
    const float *w32_in;
    const int64_t *rows_b;    // (ks) explicit table rows (no routing, no decision) or null
    const float *rows_w;
    const int64_t *rtab;      // (E) record bases of this layer, 0 = absent
    int64_t srec;             // shared-expert record, 0 = absent
    int64_t off_gq, off_gs, off_dq, off_ds;
    moehip_policy pol;
    void *out;
    const void *add;
    void *logits_out;
    int64_t *idx_out;
    void *w_out;
    float *w32_out;
    float *info;
    float *miss;
    uint32_t *ws;
    uint64_t *trace;          // 8 stamps per workgroup or null
    uint32_t off_lg, off_h, off_part;  // byte offsets of the tagged areas in ws
    uint32_t lg_stride, h_stride;      // 64-bit words between two XCDs' copies
    uint32_t defer;           // real-time ticks (10 ns) the down items wait before loading
    int E, k, ks, H, I, gs_up, gs_dn, renorm, accumulate, planned;
    int unit, units;          // h values per segment unit, units over all table rows
    int nu, nd;               // up / down items per XCD
    int hpi;                  // h values per up item
    int lg_up, lg_dn;         // log2 lanes per gate/up row and per down row
    int dr;                   // output rows per down item
};

struct XcShared {
    uint32_t tag;
    int poison;
    int idx[64];
    float w[64];
    float sorted[64];
    float tot;
    float rw[64];             // table rows: weight (0 = nothing to run)
    int64_t rb[64];           //             record base
    int lvl[64];
    int chosen[64];
    uint64_t st[8];           // trace stamps of this workgroup
    float part[XC_MAXDR];     // a combiner's own partial rows
    union {
        struct {
            int64_t rt[XC_MAXE];
            float lv[XC_MAXE + 64];
            uint32_t key[XC_MAXE + 64];
        } r;
        __align__(16) float h[XC_LDS_H];
    } u;
};

__device__ __forceinline__ void xc_stamp(const XcArgs &a, XcShared &sh, int i) {
    if (a.trace != nullptr && threadIdx.x == 0) sh.st[i] = __builtin_amdgcn_s_memrealtime();
}

// XCD-local words: plain stores (through to the XCD's L2), non-temporal polls (L1 not allocated).
// The empty asm keeps each poll inside its loop.
__device__ __forceinline__ void st_local(uint64_t *p, uint32_t payload, uint32_t tag) {
    *p = ((uint64_t)tag << 32) | payload;
}
__device__ __forceinline__ uint64_t ld_local(const uint64_t *p) {
    const uint64_t v = __builtin_nontemporal_load(p);
    asm volatile("" ::: "memory");
    return v;
}

__device__ __forceinline__ int xc_seg_begin(int x, int units) { return (x * units) / XC_N; }

// ---------------------------------------------------------------------------------------
// generation: count this workgroup as having read the tag; workgroups 0..15 drain the counters
// and the last one advances the generation (bounded, advanced all the same on expiry)
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ void xc_gen_read(uint32_t *ws) {
    if (threadIdx.x == 64)
        __hip_atomic_fetch_add(ws + XC_READ + 32 * (blockIdx.x % XC_NSUB), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void xc_gen_manage(uint32_t *ws, uint32_t tag) {
    const int G = gridDim.x, b = blockIdx.x;
    if (b >= XC_NSUB || b >= G || threadIdx.x != 0) return;
    const uint32_t nq = (uint32_t)((G - b + XC_NSUB - 1) / XC_NSUB);
    int nap = 1;
    for (int it = 0; it < XC_SPIN; ++it) {
        if (ld_co32(ws + XC_READ + 32 * b) >= nq) break;
        backoff(nap);
        if (it == XC_SPIN - 1) flag_error(ws + XC_ERR);
    }
    st_co32(ws + XC_READ + 32 * b, 0u);
    const uint32_t used = (uint32_t)min(G, XC_NSUB);
    if (add_co32(ws + XC_TOP, 1u) == used - 1u) {
        const uint32_t gen = tag - 1u, next = gen + 1u == 0xFFFFFFFFu ? 0u : gen + 1u;
        st_co32(ws + XC_TOP, 0u);
        for (int c = 0; c < XC_NGEN; ++c) st_co32(ws + XC_GEN + 256 * c, next);
    }
}

// ---------------------------------------------------------------------------------------
// router rows of this workgroup (every wave): rows id = q + NQ * (4 m + wave) < nrows, logit index
// first + id: Wr's row when < E, the shared gate at E. Each lane holds 32 values (H <= 2048). The logit is
// rounded to the activation dtype (the gate's F.linear output) and stored in the XCD's copy.
// ---------------------------------------------------------------------------------------
template <int XDT>
__device__ __forceinline__ void xc_router(const XcArgs &a, int q, int NQ, int first, int nrows, uint64_t *lg, uint32_t tag) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int c0 = lane * 32;
    const bool on = c0 < a.H;
    uint4 xv[4];
    if (on) {
        const uint4 *xp = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint8_t *>(a.x) + (size_t)c0 * 2);
#pragma unroll
        for (int i = 0; i < 4; ++i) xv[i] = xp[i];
    }
    for (int id = q + NQ * wave; id < nrows; id += 4 * NQ) {
        const int r = first + id;  // logit index: Wr row r < E, the shared gate at E
        float acc = 0.f;
        if (on) {
            const uint8_t *wp = r < a.E ? reinterpret_cast<const uint8_t *>(a.Wr) + ((size_t)r * a.H + c0) * 2
                                        : reinterpret_cast<const uint8_t *>(a.sgate) + (size_t)c0 * 2;
            uint4 wv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) wv[i] = reinterpret_cast<const uint4 *>(wp)[i];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t wd[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
                const uint32_t xd[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    if constexpr (XDT == MOEHIP_DT_F16) {
                        acc = fmaf(f16_to_f32(wd[m] & 0xffffu), f16_to_f32(xd[m] & 0xffffu), acc);
                        acc = fmaf(f16_to_f32(wd[m] >> 16), f16_to_f32(xd[m] >> 16), acc);
                    } else {
                        acc = fmaf(__uint_as_float(wd[m] << 16), __uint_as_float(xd[m] << 16), acc);
                        acc = fmaf(__uint_as_float(wd[m] & 0xffff0000u), __uint_as_float(xd[m] & 0xffff0000u), acc);
                    }
                }
            }
        }
        acc = wave_sum(acc);
        if (lane == 0) st_local(lg + r, __float_as_uint(rnd_act<XDT>(acc)), tag);
    }
}

// ---------------------------------------------------------------------------------------
// routing of this launch, computed by wave 0 of every workgroup into LDS: sh.rw / sh.rb for the
// ks table rows (k routed + the shared row), and for the report: idx, w, levels, choices.
// ---------------------------------------------------------------------------------------
template <int XDT>
__device__ __forceinline__ void xc_route(const XcArgs &a, XcShared &sh, const uint64_t *lg, uint32_t tag,
                                         int64_t idx_pre, float w_pre) {
    const int lane = threadIdx.x & 63;
    const int k = a.k, E = a.E, ks = a.ks;
    const bool has_sh = a.sgate != nullptr;
    const bool routed = a.Wr != nullptr;
    if (a.rows_b != nullptr) {  // explicit rows
        if (lane < ks) {
            const int64_t b = a.rows_b[lane];
            sh.rb[lane] = b;
            sh.rw[lane] = b != 0 ? a.rows_w[lane] : 0.f;
        }
        return;
    }
    float *s_lv = sh.u.r.lv;
    uint32_t *s_key = sh.u.r.key;
    const int nlog = (routed ? E : 0) + (has_sh ? 1 : 0);
    const int first = routed ? 0 : E;  // the shared gate alone sits at index E
    bool poisoned = false;
    if (nlog > 0) {
        const int epl = (nlog + 63) >> 6;
        uint32_t need = 0;
        for (int i = 0; i < epl; ++i)
            if (lane + 64 * i < nlog) need |= 1u << i;
        int nap = 1;
        for (int it = 0; it < XC_SPIN && __ballot(need != 0) != 0ull; ++it) {
            for (int i0 = 0; i0 < epl; i0 += 4) {  // up to 4 words per lane in flight at a time
                uint64_t v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (i0 + i < epl && (need & (1u << (i0 + i)))) v[i] = ld_local(lg + first + lane + 64 * (i0 + i));
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int ii = i0 + i;
                    if (ii < epl && (need & (1u << ii)) && tag_ok(v[i], tag)) {
                        const int c = first + lane + 64 * ii;
                        const float l = __uint_as_float((uint32_t)v[i]);
                        s_lv[c] = l;
                        if (c < E) s_key[c] = logit_key<XDT>(l, c);
                        need &= ~(1u << ii);
                    }
                }
            }
            if (__ballot(need != 0) != 0ull) backoff(nap, 2);
        }
        if (__ballot(need != 0) != 0ull) {  // expired: NaN weights, the rest routes on what arrived
            poisoned = true;
            if (lane == 0) flag_error(a.ws + XC_ERR);
            for (int i = 0; i < epl; ++i)
                if (need & (1u << i)) {
                    const int c = first + lane + 64 * i;
                    s_lv[c] = c < E ? -INFINITY : __uint_as_float(0x7fc00000u);
                    if (c < E) s_key[c] = 0u;
                }
        }
        if (routed)
            for (int c = E + lane; c < ((E + 63) & ~63) + 64; c += 64) s_key[c] = 0u;
    }
    __builtin_amdgcn_wave_barrier();
    int myc = 0;
    float myw = 0.f, myp = 0.f;
    if (routed) {
        float myv = 0.f;
        if (E <= 64) {
            // one logit per lane; its rank is the number of larger keys (16-bit keys are distinct)
            const uint32_t key = lane < E ? s_key[lane] : 0u;
            const float lvv = lane < E ? s_lv[lane] : -INFINITY;
            int rank = 0;
#pragma unroll
            for (int q0 = 0; q0 < 64; q0 += 4) {
                const uint4 o = *reinterpret_cast<const uint4 *>(s_key + q0);
                rank += (o.x > key) + (o.y > key) + (o.z > key) + (o.w > key);
            }
            __builtin_amdgcn_wave_barrier();
            if (lane < E && rank < k) {
                s_key[XC_MAXE + rank] = (uint32_t)lane;
                sh.sorted[rank] = lvv;
            }
            __builtin_amdgcn_wave_barrier();
            if (lane < k) {
                myc = (int)s_key[XC_MAXE + lane];
                myv = sh.sorted[lane];
            }
            __builtin_amdgcn_wave_barrier();
        } else {
            const int epl = (E + 63) >> 6;
            for (int r = 0; r < k; ++r) {
                uint32_t lb = 0u;
                for (int i = 0; i < epl; ++i) {
                    const int c = lane + 64 * i;
                    const uint32_t kk = c < E ? s_key[c] : 0u;
                    lb = kk > lb ? kk : lb;
                }
                const uint32_t M = wave_max_u32(lb);
                const int c = min(1023 - (int)(M & 1023u), E - 1);
                const float v = s_lv[c];
                __builtin_amdgcn_wave_barrier();
                if (lane == (c & 63)) s_key[c] = 0u;
                __builtin_amdgcn_wave_barrier();
                if (lane == r) {
                    myc = c;
                    myv = v;
                }
            }
        }
        // softmax over the E logits (fp32), the top-k weights, renormalised when asked
        const float m = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(myv), 0));
        float sum = 0.f;
        for (int c = lane; c < E; c += 64) sum += expf(s_lv[c] - m);
        sum = wave_sum(sum);
        const float p = lane < k ? expf(myv - m) / sum : 0.f;
        const float tot = a.renorm ? wave_sum(p) : 1.f;
        if (lane < k) {
            myp = a.renorm ? p / tot : p;
            myw = poisoned ? __uint_as_float(0x7fc00000u) : rnd_act<XDT>(myp);
        }
    } else if (lane < k) {
        myc = (int)idx_pre;
        myw = w_pre;
    }
    // HOBBIT levels and skip of the routed rows; the shared row is level 0, never skipped
    const bool act = lane < k, shr = has_sh && lane == k;
    int lvl;
    bool skip;
    slot_level(lane, k, act ? myw : 0.f, a.pol, sh.w, sh.sorted, &sh.tot, lvl, skip, true);
    if (shr) lvl = 0, skip = false;
    int64_t base = 0;
    float wt = 0.f;
    if (act && myc >= 0 && myc < E) base = sh.u.r.rt[myc];
    if (shr) {
        base = a.srec;
        const float l = s_lv[E];
        wt = l != l ? l : rnd_act<XDT>(1.0f / (1.0f + expf(-l)));
    } else {
        wt = myw;
    }
    const bool usable = base != 0 && a.planned;
    const bool sel = (act || shr) && !skip && usable;
    if (lane < ks) {
        sh.rb[lane] = sel ? base : 0;
        sh.rw[lane] = sel ? wt : 0.f;
        sh.idx[lane] = myc;
        sh.w[lane] = myp;  // (slot_level is done with sh.w)
        sh.lvl[lane] = lvl;
        sh.chosen[lane] = skip ? -2 : (usable ? 0 : -1);
    }
    if (act) sh.sorted[lane] = myw;
}

// ---------------------------------------------------------------------------------------
// the report of the launch (workgroup 0, after its own work): logits, indices, weights, info, miss
// ---------------------------------------------------------------------------------------
template <int XDT>
__device__ __forceinline__ void xc_report(const XcArgs &a, XcShared &sh) {
    const int tid = threadIdx.x;
    if (a.rows_b != nullptr) return;
    const bool routed = a.Wr != nullptr;
    if (a.logits_out != nullptr && routed)
        for (int c = tid; c < a.E; c += 256) st_act<XDT>(a.logits_out, c, sh.u.r.lv[c]);
    if (tid < 64) {
        const int j = tid;
        const bool act = j < a.k;
        if (act && routed) {
            if (a.idx_out) a.idx_out[j] = sh.idx[j];
            if (a.w_out) st_act<XDT>(a.w_out, j, sh.w[j]);
            if (a.w32_out) a.w32_out[j] = sh.sorted[j];
        }
        if (a.info && act) {
            a.info[j] = (float)sh.idx[j];
            a.info[a.k + j] = (float)sh.chosen[j];
            a.info[2 * a.k + j] = (float)sh.lvl[j];
        }
        const bool is_miss = j < a.ks && sh.chosen[j] == -1;
        const unsigned long long bal = __ballot(is_miss);
        if (j == 0 && a.miss != nullptr && bal != 0ull) atomicAdd(a.miss, (float)__popcll(bal));
    }
}

// ---------------------------------------------------------------------------------------
// up item: h values [f0, f0 + hpi) of the flattened table rows (one row j), written weighted by
// the row's routed weight into the XCD's h area at local index f - seg0
// ---------------------------------------------------------------------------------------
template <int PREC, int XDT>
__device__ __forceinline__ void xc_up(const XcArgs &a, XcShared &sh, int f0, int seg0, uint64_t *hx, uint32_t tag) {
    constexpr int CPL = DlFmt<PREC>::CPL, NPU = DlFmt<PREC>::NPU, VPC = DlFmt<PREC>::VPC;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int lg = a.lg_up, G = 1 << lg, RPW = 64 >> lg;
    const int slot = lane >> lg, cl = lane & (G - 1);
    const int I = a.I, H = a.H;
    const int j = f0 / I, i0 = f0 % I;
    const int per_wave = NPU * RPW;
    const int pair0 = i0 + wave * per_wave;
    const float wj = sh.rw[j];
    const int64_t base = sh.rb[j];
    if (base == 0 || wj == 0.f) {  // a row that does not run: zeros, so the down items never wait
        if (cl == G - 1)
#pragma unroll
            for (int p = 0; p < NPU; ++p) {
                const int r = pair0 + p * RPW + slot;
                if (r < i0 + a.hpi) st_local(hx + (j * I + r - seg0), 0u, tag);
            }
        return;
    }
    gbyte *qb = gbytes(base + a.off_gq);
    gbyte *sb = gbytes(base + a.off_gs);
    const int C = H / VPC;
    const size_t RB = (size_t)C * 16;
    // x first (raw), then every weight and scale load, and only then the lane vector: no load
    // waits on another one's result before all of them are in flight
    uint4 xr[CPL][VPC / 8 > 0 ? VPC / 8 : 1];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c = min(cl + i * G, C - 1);
        const uint4 *src = reinterpret_cast<const uint4 *>(a.x) + (size_t)c * (VPC / 8);
#pragma unroll
        for (int m = 0; m < VPC / 8; ++m) xr[i][m] = src[m];
    }
    uint4 qg[NPU][CPL], qu[NPU][CPL];
    uint32_t sg[NPU][CPL], su[NPU][CPL];
    uint32_t okm = 0;  // chunk (p, i) inside the row: bit p * CPL + i
#pragma unroll
    for (int p = 0; p < NPU; ++p) {
        const int r = pair0 + p * RPW + slot;  // within the item (hpi divides the unit)
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c0 = cl + i * G;
            const int c = min(c0, C - 1);
            okm |= (c0 < C ? 1u : 0u) << (p * CPL + i);
            qg[p][i] = gld16_nt(qb + (size_t)r * RB + (size_t)c * 16);
            qu[p][i] = gld16_nt(qb + (size_t)(r + I) * RB + (size_t)c * 16);
            sg[p][i] = scale_bits<PREC>(sb, r, c, H, a.gs_up);
            su[p][i] = scale_bits<PREC>(sb, r + I, c, H, a.gs_up);
        }
    }
    LaneVec<PREC, XDT> lv;
    prep_x<PREC, XDT>(xr, lv);
    float v[2 * NPU];
#pragma unroll
    for (int p = 0; p < NPU; ++p) {
        float pg = 0.f, pu = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const bool ok = (okm >> (p * CPL + i)) & 1u;
            const float s0 = ok ? scale_val<PREC>(sg[p][i]) : 0.f, s1 = ok ? scale_val<PREC>(su[p][i]) : 0.f;
            pg = fmaf(s0 * lv.p2e[i], lane_dot<PREC, XDT>(qg[p][i], lv, i), pg);
            pu = fmaf(s1 * lv.p2e[i], lane_dot<PREC, XDT>(qu[p][i], lv, i), pu);
        }
        v[2 * p] = pg;
        v[2 * p + 1] = pu;
    }
    grp_total_n<2 * NPU>(v, lg);
    if (cl == G - 1) {
#pragma unroll
        for (int p = 0; p < NPU; ++p) {
            const int r = pair0 + p * RPW + slot;
            st_local(hx + (j * I + r - seg0), __float_as_uint(wj * silu_mul(v[2 * p], v[2 * p + 1])), tag);
        }
    }
}

// ---------------------------------------------------------------------------------------
// down item: output rows [row0w, ...) of each wave over the XCD's segment (nch chunks of VPC
// values, flattened over the table rows it spans)
// ---------------------------------------------------------------------------------------
template <int PREC>
struct XcDown {
    uint4 q[DlFmt<PREC>::NPD][DlFmt<PREC>::CPL];
    uint32_t s[DlFmt<PREC>::NPD][DlFmt<PREC>::CPL];
    uint32_t ok;  // bit p * CPL + i: chunk (p, i) counts (the others multiply by scale 0)
};

template <int PREC>
__device__ __forceinline__ void xc_down_load(const XcArgs &a, const XcShared &sh, int row0, int seg0, int nch,
                                             XcDown<PREC> &d) {
    constexpr int CPL = DlFmt<PREC>::CPL, NPD = DlFmt<PREC>::NPD, VPC = DlFmt<PREC>::VPC;
    const int lane = threadIdx.x & 63;
    const int lg = a.lg_dn, G = 1 << lg, RPW = 64 >> lg;
    const int slot = lane >> lg, cl = lane & (G - 1);
    const int I = a.I, H = a.H;
    const size_t RB = (size_t)(I / VPC) * 16;  // bytes of one down row
    d.ok = 0;
#pragma unroll
    for (int p = 0; p < NPD; ++p) {
        const int r0 = row0 + p * RPW + slot;
        const int r = min(r0, H - 1);
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c0 = cl + i * G;
            const int c = min(c0, max(nch - 1, 0));
            const int f = seg0 + c * VPC;  // flattened h index of the chunk's first value
            const int j = min(f / I, a.ks - 1), col = f - j * I;
            const int64_t base = nch > 0 ? sh.rb[j] : 0;
            const bool ok = c0 < nch && r0 < H && base != 0;
            // rows without a record read the activation vector instead (in bounds) at scale 0
            gbyte *qp = base != 0 ? gbytes(base + a.off_dq) + (size_t)r * RB + (size_t)(col / VPC) * 16 : gbytes(a.x);
            d.q[p][i] = gld16_nt(qp);
            // (the scale of a row without a record is read from x too; the bit drops it)
            d.s[p][i] = scale_bits<PREC>(base != 0 ? gbytes(base + a.off_ds) : gbytes(a.x), base != 0 ? r : 0,
                                         base != 0 ? col / VPC : 0, I, a.gs_dn);
            d.ok |= (ok ? 1u : 0u) << (p * CPL + i);
        }
    }
}

// the down rows' partial sums (valid in the last lane of each lane group)
template <int PREC, int XDT>
__device__ __forceinline__ void xc_down_rows(const XcArgs &a, const XcDown<PREC> &d, const LaneVec<PREC, XDT> &lv,
                                             float (&v)[DlFmt<PREC>::NPD]) {
    constexpr int CPL = DlFmt<PREC>::CPL, NPD = DlFmt<PREC>::NPD;
#pragma unroll
    for (int p = 0; p < NPD; ++p) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const float sc = ((d.ok >> (p * CPL + i)) & 1u) ? scale_val<PREC>(d.s[p][i]) : 0.f;
            acc = fmaf(sc * lv.p2e[i], lane_dot<PREC, XDT>(d.q[p][i], lv, i), acc);
        }
        v[p] = acc;
    }
    grp_total_n<NPD>(v, a.lg_dn);
}

// ---------------------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------------------
template <int XDT, int PREC>
__global__ __launch_bounds__(256) void k_decode_xcd(XcArgs a) {
    __shared__ XcShared sh;
    constexpr int VPC = DlFmt<PREC>::VPC, NPD = DlFmt<PREC>::NPD;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int b = blockIdx.x, x = b % XC_N, q = b / XC_N, NQ = gridDim.x / XC_N;
    uint8_t *wsb = reinterpret_cast<uint8_t *>(a.ws);
    uint64_t *lg = reinterpret_cast<uint64_t *>(wsb + a.off_lg) + (size_t)x * a.lg_stride;
    uint64_t *hx = reinterpret_cast<uint64_t *>(wsb + a.off_h) + (size_t)x * a.h_stride;
    uint64_t *part = reinterpret_cast<uint64_t *>(wsb + a.off_part);
    xc_stamp(a, sh, 0);
    // the launch tag, read by every wave (one of 16 copies; never 0), used from the first store on
    const uint32_t tag = (uint32_t)uni((int)(ld_co32(a.ws + XC_GEN + 256 * (b % XC_NGEN)) + 1u));
    if (tid == 0) sh.poison = 0;
    // the record table into LDS (the k chosen records are looked up after the routing)
    const bool routed = a.Wr != nullptr;
    if (a.rows_b == nullptr)
        for (int e = tid; e < a.E; e += 256) sh.u.r.rt[e] = a.rtab[e];
    int64_t idx_pre = 0;
    float w_pre = 0.f;
    if (!routed && a.rows_b == nullptr && tid < a.k) {
        idx_pre = a.idx_in[tid];
        w_pre = a.w32_in[tid];
    }
    // 1. router rows of this XCD (logits, shared gate), then the routing (wave 0)
    const int nrows = a.rows_b != nullptr ? 0 : (routed ? a.E : 0) + (a.sgate != nullptr ? 1 : 0);
    if (nrows > 0) xc_router<XDT>(a, q, NQ, routed ? 0 : a.E, nrows, lg, tag);
    if (tag != 0u) xc_gen_read(a.ws);  // (after the tag has arrived)
    xc_stamp(a, sh, 1);
    const int seg0u = xc_seg_begin(x, a.units), seg1u = xc_seg_begin(x + 1, a.units);
    const int seg0 = seg0u * a.unit, seg_len = (seg1u - seg0u) * a.unit;
    const bool is_up = q < a.nu;
    const int f0 = seg0 + q * a.hpi;
    const bool up_work = is_up && q * a.hpi < seg_len;
    xc_stamp(a, sh, 2);
    __syncthreads();  // the record table is in LDS
    if (wave == 0) xc_route<XDT>(a, sh, lg, tag, idx_pre, w_pre);
    __syncthreads();
    xc_stamp(a, sh, 3);
    if (is_up) {
        // 2. h of this item's rows (x is requested with the weights: it arrives no later)
        if (up_work) xc_up<PREC, XDT>(a, sh, f0, seg0, hx, tag);
        xc_stamp(a, sh, 5);
    } else {
        // 3. the down rows over the segment
        const int d = q - a.nu;
        const int lgd = a.lg_dn, G = 1 << lgd, RPW = 64 >> lgd;
        const int per_wave = NPD * RPW;
        const int row0 = d * a.dr + wave * per_wave;
        const int nch = seg_len / VPC;
        {  // the gate/up weights first: they are needed before these can be used
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            const uint32_t defer = (uint32_t)uni((int)a.defer);
            while (__builtin_amdgcn_s_memrealtime() - t0 < defer) __builtin_amdgcn_s_sleep(8);
        }
        XcDown<PREC> dd;
        xc_down_load<PREC>(a, sh, row0, seg0, nch, dd);
        xc_stamp(a, sh, 4);
        // h of the segment -> LDS (piece-major: piece m of chunk c at (m * C + c) * 4)
        float *s_h = sh.u.h;
        const int C = nch > 0 ? nch : 1;
        bool h_ok = true;
        for (int w0 = 0; w0 < seg_len; w0 += 256 * 8) {
            uint32_t need = 0;
#pragma unroll
            for (int m = 0; m < 8; ++m)
                if (w0 + tid + 256 * m < seg_len) need |= 1u << m;
            int nap = 1;
            for (int it = 0; it < XC_SPIN; ++it) {
                uint64_t v[8];
#pragma unroll
                for (int m = 0; m < 8; ++m)
                    if (need & (1u << m)) v[m] = ld_local(hx + w0 + tid + 256 * m);
#pragma unroll
                for (int m = 0; m < 8; ++m) {
                    if ((need & (1u << m)) && tag_ok(v[m], tag)) {
                        const int i = w0 + tid + 256 * m;
                        const int c = i / VPC, qq = i - c * VPC;
                        s_h[((qq >> 2) * C + c) * 4 + (qq & 3)] = __uint_as_float((uint32_t)v[m]);
                        need &= ~(1u << m);
                    }
                }
                if (!__syncthreads_or(need != 0)) break;
                backoff(nap, 2);
                if (it == XC_SPIN - 1) {
                    h_ok = false;
                    if (tid == 0) flag_error(a.ws + XC_ERR);
                }
            }
        }
        LaneVec<PREC, XDT> lh;
        load_h<PREC, XDT>(s_h, lane & (G - 1), G, C, lh);
        float v[NPD];
        xc_down_rows<PREC, XDT>(a, dd, lh, v);
        if (!h_ok)
#pragma unroll
            for (int p = 0; p < NPD; ++p) v[p] = __uint_as_float(0x7fc00000u);
        xc_stamp(a, sh, 5);
        // 4. the partial rows: the combiner of this row block keeps its own, the others send theirs
        const bool combiner = (d % XC_N) == x;
        const int cl = lane & (G - 1), slot = lane >> lgd;
        if (cl == G - 1) {
#pragma unroll
            for (int p = 0; p < NPD; ++p) {
                const int r = row0 + p * RPW + slot;
                if (r < a.H) {
                    if (combiner) sh.part[r - d * a.dr] = v[p];
                    else st_tag(part + (size_t)x * a.H + r, __float_as_uint(v[p]), tag);
                }
            }
        }
        if (combiner) {
            __syncthreads();
            const int r0 = d * a.dr, nrow = min(a.dr, a.H - r0);
            for (int rr = tid; rr < nrow; rr += 256) {
                float val[XC_N];
                uint32_t need = 0;
#pragma unroll
                for (int xx = 0; xx < XC_N; ++xx) {
                    if (xx == x) val[xx] = sh.part[rr];
                    else need |= 1u << xx;
                }
                int nap = 1;
                for (int it = 0; it < XC_SPIN && need != 0; ++it) {
                    uint64_t w8[XC_N];
#pragma unroll
                    for (int xx = 0; xx < XC_N; ++xx)
                        if (need & (1u << xx)) w8[xx] = ld_tag(part + (size_t)xx * a.H + r0 + rr);
#pragma unroll
                    for (int xx = 0; xx < XC_N; ++xx)
                        if ((need & (1u << xx)) && tag_ok(w8[xx], tag)) {
                            val[xx] = __uint_as_float((uint32_t)w8[xx]);
                            need &= ~(1u << xx);
                        }
                    if (need != 0) backoff(nap, 2);
                }
                float acc = 0.f;
#pragma unroll
                for (int xx = 0; xx < XC_N; ++xx) acc += (need & (1u << xx)) ? __uint_as_float(0x7fc00000u) : val[xx];
                if (need != 0) flag_error(a.ws + XC_ERR);
                if (a.accumulate) acc += ld_act<XDT>(a.out, r0 + rr);
                if (a.add != nullptr) acc += ld_act<XDT>(a.add, r0 + rr);
                st_act<XDT>(a.out, r0 + rr, acc);
            }
        }
        xc_stamp(a, sh, 6);
    }
    if (b == 0) {
        __syncthreads();
        xc_report<XDT>(a, sh);
    }
    xc_gen_manage(a.ws, tag);
    if (a.trace != nullptr) {
        __syncthreads();
        if (tid == 0) {
            sh.st[7] = __builtin_amdgcn_s_memrealtime();
            for (int i = 0; i < 8; ++i) a.trace[(size_t)b * 8 + i] = sh.st[i];
        }
    }
}

// ---------------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------------
typedef void (*XcKernel)(XcArgs);

template <int XDT>
static XcKernel xc_kernel_x(int prec) {
    switch (prec) {
        case MOEHIP_PREC_INT4: return k_decode_xcd<XDT, MOEHIP_PREC_INT4>;
        case MOEHIP_PREC_INT8: return k_decode_xcd<XDT, MOEHIP_PREC_INT8>;
        case MOEHIP_PREC_F16: return k_decode_xcd<XDT, MOEHIP_PREC_F16>;
        case MOEHIP_PREC_BF16: return k_decode_xcd<XDT, MOEHIP_PREC_BF16>;
        case MOEHIP_PREC_FP8: return k_decode_xcd<XDT, MOEHIP_PREC_FP8>;
        default: return nullptr;
    }
}
static XcKernel xc_kernel(int dtype, int prec) {
    if (dtype == MOEHIP_DT_F16) return xc_kernel_x<MOEHIP_DT_F16>(prec);
    if (dtype == MOEHIP_DT_BF16) return xc_kernel_x<MOEHIP_DT_BF16>(prec);
    return nullptr;
}

static inline int xc_vpc(int prec) { return vpc_of(prec); }
static inline int xc_cpl(int prec) { return 32 / vpc_of(prec); }
static inline int xc_lg(int chunks, int prec) {  // log2 lanes for `chunks` chunks, CPL per lane
    const int lanes = (chunks + xc_cpl(prec) - 1) / xc_cpl(prec);
    int G = 1, lg = 0;
    while (G < lanes && G < 64) G <<= 1, ++lg;
    return lg;
}

struct XcPlan {
    int ok;
    int unit, units, nu, nd, hpi, lg_up, lg_dn, dr, grid;
    uint32_t lg_stride, h_stride, off_lg, off_h, off_part, total;
};

static inline uint32_t xc_al256(size_t v) { return (uint32_t)((v + 255) / 256 * 256); }

// the launch shape of a layer, or ok = 0 when this kernel cannot take it
static XcPlan xc_plan(int prec, int ks, int E, int H, int I) {
    XcPlan p{};
    const int vpc = xc_vpc(prec), cpl = xc_cpl(prec);
    if (vpc == 0 || prec == MOEHIP_PREC_F32 || H > 2048 || H % 32 || I % 32 || E > XC_MAXE || ks > XC_MAXKS) return p;
    const int npu = 4 / cpl, npd = 8 / cpl;
    p.lg_up = xc_lg(H / vpc, prec);
    p.hpi = npu * (64 >> p.lg_up) * 4;
    p.unit = p.hpi > 32 ? p.hpi : 32;
    if (I % p.unit) return p;
    p.units = ks * I / p.unit;
    const int seg_max = ((p.units + XC_N - 1) / XC_N) * p.unit;
    if (seg_max > XC_LDS_H) return p;
    p.nu = (seg_max + p.hpi - 1) / p.hpi;
    p.lg_dn = xc_lg(seg_max / vpc, prec);
    p.dr = npd * (64 >> p.lg_dn) * 4;
    if (p.dr > XC_MAXDR) return p;
    p.nd = (H + p.dr - 1) / p.dr;
    p.grid = XC_N * (p.nu + p.nd);
    // workspace: header, 8 logit copies, 8 h segments, 8 partial rows
    p.lg_stride = (uint32_t)(((size_t)(E + 1) * 8 + 255) / 256 * 32 + 32);
    p.h_stride = (uint32_t)(((size_t)seg_max * 8 + 255) / 256 * 32);
    size_t off = xc_al256((size_t)XC_HDR * 4);
    p.off_lg = (uint32_t)off;
    off = xc_al256(off + (size_t)XC_N * p.lg_stride * 8);
    p.off_h = (uint32_t)off;
    off = xc_al256(off + (size_t)XC_N * p.h_stride * 8);
    p.off_part = (uint32_t)off;
    off = xc_al256(off + (size_t)XC_N * H * 8);
    p.total = (uint32_t)off;
    p.ok = 1;
    return p;
}

// 1 once moehip_device_check confirmed the round-robin XCD dispatch on a device (per device)
static int g_xcd_ok[64];

__global__ void k_xcd_probe(uint32_t *out) {
    if (threadIdx.x == 0) {
        uint32_t v;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
        out[blockIdx.x] = v & 15u;
    }
}

// Called by moehip_device_check: launch a probe grid and record whether workgroup b runs on XCD
// b % 8 on this device (synchronous; the library's only synchronising call, made once at set-up).
int xcd_probe(int dev) {
    if (dev < 0 || dev >= 64) return 0;
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess) return 0;
    if (hipSetDevice(dev) != hipSuccess) return 0;
    int ok = 0;
    uint32_t *d = nullptr;
    const int NB = 4096;
    if (hipMalloc(&d, NB * 4) == hipSuccess) {
        hipLaunchKernelGGL(k_xcd_probe, dim3(NB), dim3(64), 0, 0, d);
        uint32_t *h = (uint32_t *)malloc(NB * 4);
        if (h != nullptr && hipMemcpy(h, d, NB * 4, hipMemcpyDeviceToHost) == hipSuccess) {
            ok = 1;
            for (int b = 0; b < NB; ++b) ok &= (int)(h[b] == (uint32_t)(b % XC_N));
        }
        free(h);
        hipFree(d);
    }
    hipGetLastError();
    g_xcd_ok[dev] = ok;
    hipSetDevice(prev);
    return ok;
}

size_t xcd_workspace_bytes(int prec, int ks, int E, int H, int I) {
    const XcPlan p = xc_plan(prec, ks, E, H, I);
    return p.ok ? p.total : 0;
}

// the XCD kernel for one launch when it applies: returns MOEHIP_OK after launching, 1 when the
// layer does not fit this kernel (the caller then runs the item-loop kernel), or an error code
int xcd_launch(const moehip_layer_desc *d, const void *x, const void *Wr, const int64_t *idx_in,
                      const float *w32_in, const int64_t *rows_b, const float *rows_w, const int64_t *rtab,
                      void *out, const void *add, int accumulate, void *logits_out, int64_t *idx_out, void *w_out,
                      float *w32_out, float *info, float *miss, void *ws, size_t ws_bytes, uint64_t *trace,
                      void *stream, int *used) {
    *used = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64 || !g_xcd_ok[dev]) return MOEHIP_OK;
    if (d->P != 1 || (d->dtype != MOEHIP_DT_F16 && d->dtype != MOEHIP_DT_BF16)) return MOEHIP_OK;
    const int ks = d->k + (d->shared_gate != nullptr ? 1 : 0);
    const XcPlan p = xc_plan(d->prec[0], ks, d->E, d->H, d->I);
    if (!p.ok || ws_bytes < p.total) return MOEHIP_OK;
    XcKernel kern = xc_kernel(d->dtype, d->prec[0]);
    if (kern == nullptr) return MOEHIP_OK;
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(kern), 256, 0) != hipSuccess)
        return MOEHIP_OK;
    if (p.grid > per_cu * cus) return MOEHIP_OK;  // every workgroup must be resident at once
    XcArgs a{};
    a.x = x;
    a.Wr = Wr;
    a.sgate = d->shared_gate;
    a.idx_in = idx_in;
    a.w32_in = w32_in;
    a.rows_b = rows_b;
    a.rows_w = rows_w;
    a.rtab = rtab;
    a.srec = d->shared_rec[0];
    a.off_gq = d->offs[0][0];
    a.off_gs = d->offs[0][1];
    a.off_dq = d->offs[0][2];
    a.off_ds = d->offs[0][3];
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
    a.trace = trace;
    a.off_lg = p.off_lg;
    a.off_h = p.off_h;
    a.off_part = p.off_part;
    a.lg_stride = p.lg_stride;
    a.h_stride = p.h_stride;
    // the time the HBM needs for the ks gate/up blocks (q + scales) at 8 TB/s, in 10 ns ticks
    const double gu = (double)(d->offs[0][2] - d->offs[0][0]);
    a.defer = (uint32_t)(ks * gu / 8.0e12 * 1.0e8);
    a.E = d->E;
    a.k = d->k;
    a.ks = ks;
    a.H = d->H;
    a.I = d->I;
    a.gs_up = d->gs_up[0];
    a.gs_dn = d->gs_dn[0];
    a.renorm = d->renorm;
    a.accumulate = accumulate;
    a.planned = d->planned[0];
    a.unit = p.unit;
    a.units = p.units;
    a.nu = p.nu;
    a.nd = p.nd;
    a.hpi = p.hpi;
    a.lg_up = p.lg_up;
    a.lg_dn = p.lg_dn;
    a.dr = p.dr;
    hipLaunchKernelGGL(kern, dim3(p.grid), dim3(256), 0, as_stream(stream), a);
    *used = 1;
    return check_launch("decode_layer (xcd)");
}

}  // namespace moehip
