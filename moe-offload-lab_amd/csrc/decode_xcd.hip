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
//      all of them back and ranks them itself (top-k and the record of each table row, the keys
//      in registers; the weights, renorm and HOBBIT decision follow while the other waves'
//      expert weights load);
//   2. the table rows' h values (k routed + shared, I each, flattened row after row) are cut into
//      8 contiguous segments, one per XCD; workgroup q of an XCD holds up part q (hpi h values
//      of its segment: h = w * silu(gate x) * (up x), w = the row's routed weight, into the XCD's
//      h area) and down part q (output rows [q * DR, q * DR + DR) times the segment's down
//      columns: a partial output of the layer restricted to the segment). Every wave requests the
//      weights of its up part, then those of its down part, as soon as the rows are ranked: the
//      whole layer's expert bytes are in flight at once, up part first;
//   3. once the XCD's h values are in (polled from the XCD's L2), the down part's products;
//   4. the one exchange between XCDs: the partial rows of the 8 XCDs, summed in XCD order by the
//      workgroup of XCD q % 8 for row block q, plus add / accumulate, cast to the output dtype.
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
// Co-residency: the grid (8 x workgroups per XCD) never exceeds what the GPU holds at once.

#include "decide.hpp"
#include "lanevec.hpp"

namespace moehip {

constexpr int XC_N = 8;            // XCDs
constexpr int XC_SPIN = 1 << 21;   // polls before a wait gives up (~1 s)
constexpr int XC_NGEN = 16;        // header as in decode_layer.hip: reader counters, error flag,
constexpr int XC_NSUB = 16;        // drained count, generation copies 1 KB apart
enum { XC_READ = 0, XC_ERR = XC_NSUB * 32, XC_TOP = XC_NSUB * 32 + 32, XC_TEST = XC_NSUB * 32 + 64, XC_GEN = 1024,
       XC_HDR = XC_GEN + 256 * XC_NGEN };
// XC_TEST: a word the library never writes (zero from the workspace's first zero-fill). When a test
// sets it, the data waits of every later launch on that workspace give up after XC_TEST_SPIN polls and
// the logits are polled for a tag that is never written: an expired wait, forced from the host, in a
// launch whose every workgroup still exits normally (the generation's own counting keeps its full
// bound, so the launch after the test word is cleared runs normally).
constexpr int XC_TEST_SPIN = 8;
constexpr int XC_MAXE = 1024;
constexpr int XC_MAXKS = 33;
constexpr int XC_LDS_H = 8192;     // h values of one XCD's segment staged in LDS (fp32)
constexpr int XC_MAXDR = 512;      // output rows of one down item
constexpr int XC_NST = 16;         // trace stamps per workgroup
constexpr int XC_SPLIT_E = 256;    // from this many experts on, the router rows are split over the XCDs
constexpr uint64_t XC_RELAY_TICKS = 260;  // the split router's first logit poll: 2.6 us of the 100 MHz real-time counter

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
    uint64_t *trace;          // XC_NST stamps per workgroup or null
    uint32_t off_lg, off_h, off_part;  // byte offsets of the tagged areas in ws
    uint32_t off_glg;                  // the agent-scope logit area (router rows split over the XCDs)
    uint32_t lg_stride, h_stride;      // 64-bit words between two XCDs' copies
    int E, k, ks, H, I, gs_up, gs_dn, renorm, accumulate, planned;
    int unit, units;          // h values per segment unit, units over all table rows
    int nu, nd;               // up / down items per XCD
    int hpi;                  // h values per up item
    int lg_up, lg_dn;         // log2 lanes per gate/up row and per down row
    int dr;                   // output rows per down item
    uint32_t defer;           // real-time ticks (10 ns) the down items wait before loading
    int split;                // router rows split over the XCDs (E / 8 each), logits relayed between them
};

struct XcShared {
    int idx[64];
    float w[64];
    float sorted[64];
    float tot;
    float rw[64];             // table rows: weight (0 = nothing to run)
    int64_t rb[64];           //             record base
    int lvl[64];
    int chosen[64];
    uint64_t st[XC_NST];      // trace stamps of this workgroup
    float part[XC_MAXDR];     // a combiner's own partial rows
    union {  // (up items use the routing arrays to the end: the report; down items stage h here)
        struct {
            int64_t rt[XC_MAXE];
            float lv[XC_MAXE + 64];
            uint32_t key[XC_MAXE + 64];
            uint32_t lmax[64];            // top-k of E > 64 keys: the lanes' largest keys
            uint32_t cand[XC_MAXE + 4];   //                       the candidates
        } r;
        __align__(16) float h[XC_LDS_H];
    } u;
};

// down rows per lane group and wave pass
template <int PREC> struct XcFmt {
    static constexpr int NPD = DlFmt<PREC>::NPD;
};

__device__ __forceinline__ void xc_stamp(const XcArgs &a, XcShared &sh, int i) {
    if (a.trace != nullptr && threadIdx.x == 0) sh.st[i] = __builtin_amdgcn_s_memrealtime();
}
// (inside the routing, by the routing wave's first lane)
__device__ __forceinline__ void xc_stamp_r(const XcArgs &a, XcShared &sh, int i) {
    if (a.trace != nullptr && (threadIdx.x & 63) == 0) sh.st[i] = __builtin_amdgcn_s_memrealtime();
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

// the launch tag from the generation word as loaded: computed at the point of use (the opaque
// step keeps the compiler from computing it, and so waiting for the load, any earlier)
__device__ __forceinline__ uint32_t xc_tag_of(uint32_t gen) {
    asm volatile("" : "+v"(gen));
    return gen + 1u;
}

// ---------------------------------------------------------------------------------------
// generation: count this workgroup as having read the tag; workgroups 0..15 drain the counters
// and the last one advances the generation (bounded, advanced all the same on expiry)
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ void xc_gen_read(uint32_t *ws) {
    if (threadIdx.x == 0)
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
// router rows of this workgroup (every wave): rows id = q + NQ * (4 m + wave) < nrows; row id < nr is
// logit r0 + id (Wr's row), row nr the shared gate (logit index E). Each lane holds 32 values
// (H <= 2048). The logit is rounded to the activation dtype (the gate's F.linear output) and stored
// in the XCD's copy, and, when the rows are split over the XCDs (glg), at agent scope for the others.
// ---------------------------------------------------------------------------------------
template <int XDT>
__device__ __forceinline__ void xc_router(const XcArgs &a, int q, int NQ, int r0, int nr, int nrows, uint64_t *lg,
                                          uint64_t *glg, uint32_t gen) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int c0 = lane * 32;
    const bool on = c0 < a.H;
    // the first row's weights are requested before x is used (both loads in flight together)
    auto row_ptr = [&](int id) {
        const int r = id < nr ? r0 + id : a.E;  // logit index: Wr row r < E, the shared gate at E
        return r < a.E ? reinterpret_cast<const uint4 *>(reinterpret_cast<const uint8_t *>(a.Wr) + ((size_t)r * a.H + c0) * 2)
                       : reinterpret_cast<const uint4 *>(reinterpret_cast<const uint8_t *>(a.sgate) + (size_t)c0 * 2);
    };
    int id = q + NQ * wave;
    if (id >= nrows) return;
    uint4 wv[4], xv[4];
    if (on) {
        const uint4 *wp = row_ptr(id);
#pragma unroll
        for (int i = 0; i < 4; ++i) wv[i] = wp[i];
        const uint4 *xp = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint8_t *>(a.x) + (size_t)c0 * 2);
#pragma unroll
        for (int i = 0; i < 4; ++i) xv[i] = xp[i];
    }
    while (true) {
        float acc = 0.f;
        if (on) {
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
        if (lane == 0) {
            const int r = id < nr ? r0 + id : a.E;
            const uint32_t v = __float_as_uint(rnd_act<XDT>(acc));
            st_local(lg + r, v, xc_tag_of(gen));
            if (glg != nullptr && r < a.E) st_tag(glg + r, v, xc_tag_of(gen));
        }
        id += 4 * NQ;
        if (id >= nrows) break;
        if (on) {
            const uint4 *wp = row_ptr(id);
#pragma unroll
            for (int i = 0; i < 4; ++i) wv[i] = wp[i];
        }
    }
}

// ---------------------------------------------------------------------------------------
// relay (router rows split over the XCDs): one wave copies the E / 8 logits of XCD y from the
// agent-scope area into this XCD's copy, each as soon as it is there (bounded; on expiry the error
// flag is set and the word is not copied, so this XCD's pollers expire too and route on NaN)
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ void xc_relay(const XcArgs &a, int y, const uint64_t *glg, uint64_t *lg, uint32_t tag) {
    const int lane = threadIdx.x & 63;
    const int nr = a.E / XC_N, r0 = y * nr;
    for (int i0 = 0; i0 < nr; i0 += 64) {
        const int r = r0 + i0 + lane;
        bool need = i0 + lane < nr;
        int nap = 1;
        for (int it = 0; it < XC_SPIN && __ballot(need) != 0ull; ++it) {
            if (need) {
                const uint64_t v = ld_tag(glg + r);
                if (tag_ok(v, tag)) {
                    st_local(lg + r, (uint32_t)v, tag);
                    need = false;
                }
            }
            if (__ballot(need) != 0ull) backoff(nap, 2);
        }
        if (__ballot(need) != 0ull && lane == 0) flag_error(a.ws + XC_ERR);
    }
}

// ---------------------------------------------------------------------------------------
// routing, part 1, by wave 0 of every workgroup: the k routed experts in rank order (lanes < k:
// expert myc, logit myv) and the record base of every table row (k routed + the shared row) in
// sh.rb. The rows' weight loads start from these; the weights and the HOBBIT decision (part 2)
// follow while they are in flight. A row with no resident copy (or an unplanned layer) has
// base 0 and never runs; a row that part 2 skips runs with weight 0.
// ---------------------------------------------------------------------------------------
// r[i] += (k.i > b) for unsigned values: each compare's lane mask added straight into a count as the
// carry (two VALU operations per key, no select), four independent chains so that no compare waits
// for the count before it; every mask is read three instructions after it is written
__device__ __forceinline__ void count_gt4(const uint4 kk, uint32_t b, int (&r)[4]) {
    uint64_t m0, m1, m2, m3;
    asm(
        "v_cmp_gt_u32_e64 %4, %8, %12\n\t"
        "v_cmp_gt_u32_e64 %5, %9, %12\n\t"
        "v_cmp_gt_u32_e64 %6, %10, %12\n\t"
        "v_cmp_gt_u32_e64 %7, %11, %12\n\t"
        "v_addc_co_u32_e64 %0, %4, 0, %0, %4\n\t"
        "v_addc_co_u32_e64 %1, %5, 0, %1, %5\n\t"
        "v_addc_co_u32_e64 %2, %6, 0, %2, %6\n\t"
        "v_addc_co_u32_e64 %3, %7, 0, %3, %7"
        : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "=&s"(m0), "=&s"(m1), "=&s"(m2), "=&s"(m3)
        : "v"(kk.x), "v"(kk.y), "v"(kk.z), "v"(kk.w), "v"(b));
}
// the number of the n (a multiple of 4) words of LDS array s greater than b
__device__ __forceinline__ int count_greater(const uint32_t *s, int n, uint32_t b) {
    int r[4] = {0, 0, 0, 0};
    for (int j = 0; j < n; j += 4) count_gt4(*reinterpret_cast<const uint4 *>(s + j), b, r);
    return (r[0] + r[1]) + (r[2] + r[3]);
}
template <int N>
__device__ __forceinline__ int count_greater_n(const uint32_t *s, uint32_t b) {
    uint4 kv[N / 4];  // (every read issued before the first compare)
#pragma unroll
    for (int j = 0; j < N / 4; ++j) kv[j] = *reinterpret_cast<const uint4 *>(s + 4 * j);
    int r[4] = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < N / 4; ++j) count_gt4(kv[j], b, r);
    return (r[0] + r[1]) + (r[2] + r[3]);
}

// top-k of E > 64 keys by one wave, EPL keys per lane (key c at lane c % 64, slot c / 64): T = the
// k-th largest of the 64 lanes' largest keys, ranked by counting; only the k lanes whose largest key
// is >= T hold keys >= T, so there are at most k * EPL candidates (about k + a few for routing
// logits), compacted into LDS and ranked by counting among themselves. Keys are distinct (the expert
// index is part of the key); zero keys (padding, expired polls) are never candidates, and a rank that
// no key reaches keeps E - 1, as k rounds of a maximum over zero keys would give it.
template <int EPL>
__device__ __forceinline__ void xc_topk(XcShared &sh, const uint32_t *s_key, int E, int k, int lane, int &myc) {
    uint32_t key[EPL];
    uint32_t lm = 0u;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const int c = lane + 64 * i;
        key[i] = c < E ? s_key[c] : 0u;
        lm = max(lm, key[i]);
    }
    uint32_t *s_lm = sh.u.r.lmax, *s_c = sh.u.r.cand;
    s_lm[lane] = lm;
    if (lane < k) sh.idx[lane] = E - 1;
    wave_sync();
    const int r = count_greater_n<64>(s_lm, lm);
    const unsigned long long bt = __ballot(r == k - 1 && lm != 0u);
    const uint32_t T = bt != 0ull ? (uint32_t)__builtin_amdgcn_readlane((int)lm, __builtin_ffsll((long long)bt) - 1) : 1u;
    int base = 0;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const bool sel = key[i] >= T && key[i] != 0u;
        const unsigned long long b = __ballot(sel);
        const int pos = base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
        if (sel) s_c[pos] = key[i];
        base += __popcll(b);
    }
    if (lane < 4) s_c[base + lane] = 0u;  // (the last uint4 read past the candidates sees zeros)
    wave_sync();
    const int C = uni(base);
    for (int j0 = 0; j0 < C; j0 += 64) {
        const uint32_t mine = j0 + lane < C ? s_c[j0 + lane] : 0u;
        const int rr = count_greater(s_c, (C + 3) & ~3, mine);
        if (mine != 0u && rr < k) sh.idx[rr] = min(1023 - (int)(mine & 1023u), E - 1);
    }
    wave_sync();
    if (lane < k) myc = sh.idx[lane];
}

// the logits of this XCD's copy, polled by one wave (word first + lane + 64 i for the bits i of need):
// every word a lane still needs is requested before any is looked at (one round trip per poll; NB
// words per lane at a time); returns the words that never arrived (bounded by spin)
template <int XDT, int NB>
__device__ __forceinline__ uint32_t xc_poll_logits(const uint64_t *lg, int first, int E, int epl, int lane, uint32_t tag,
                                                   int spin, uint32_t need, float *s_lv, uint32_t *s_key) {
    int nap = 1;
    for (int it = 0; it < spin && __ballot(need != 0) != 0ull; ++it) {
        for (int i0 = 0; i0 < epl; i0 += NB) {
            uint64_t v[NB];
#pragma unroll
            for (int i = 0; i < NB; ++i)
                if (i0 + i < epl && (need & (1u << (i0 + i)))) v[i] = ld_local(lg + first + lane + 64 * (i0 + i));
#pragma unroll
            for (int i = 0; i < NB; ++i) {
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
    return need;
}

template <int XDT>
__device__ __forceinline__ void xc_rank(const XcArgs &a, XcShared &sh, const uint64_t *lg, uint32_t tag, int spin,
                                        int64_t idx_pre, int &myc, float &myv, bool &poisoned, uint64_t t_in) {
    const int lane = threadIdx.x & 63;
    const int k = a.k, E = a.E, ks = a.ks;
    const bool has_sh = a.sgate != nullptr;
    const bool routed = a.Wr != nullptr;
    myc = 0;
    myv = 0.f;
    poisoned = false;
    if (a.rows_b != nullptr) {  // explicit rows: bases and weights as given
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
    if (nlog > 0) {
        const int epl = (nlog + 63) >> 6;
        uint32_t need = 0;
        for (int i = 0; i < epl; ++i)
            if (lane + 64 * i < nlog) need |= 1u << i;
        // with the rows split over the XCDs, the first poll waits until XC_RELAY_TICKS after the
        // workgroup started: the relayed blocks land at ~2.6-3.0 us, and a poll round of words
        // written moments before takes 1.4-1.7 us, so polling earlier costs a round (Qwen3-Next
        // E = 512: int4 18.9 -> 18.7, fp8 21.0 -> 20.6-20.8 us per layer with 2.4-2.8 us)
        if (a.split != 0 && routed)
            while (__builtin_amdgcn_s_memrealtime() - t_in < XC_RELAY_TICKS) __builtin_amdgcn_s_sleep(2);
        if (epl == 1) need = xc_poll_logits<XDT, 1>(lg, first, E, epl, lane, tag, spin, need, s_lv, s_key);
        else if (epl <= 4) need = xc_poll_logits<XDT, 4>(lg, first, E, epl, lane, tag, spin, need, s_lv, s_key);
        else need = xc_poll_logits<XDT, 16>(lg, first, E, epl, lane, tag, spin, need, s_lv, s_key);
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
    xc_stamp_r(a, sh, 2);
    __builtin_amdgcn_wave_barrier();
    if (routed) {
        if (E <= 64) {
            // one key per lane, ranked by counting the larger keys (keys are distinct: the
            // expert index is part of the key): 64 independent compares against the keys read
            // back from LDS, not a chain of k wave maxima. The experts ranked below k write
            // their index into their slot; a slot that no key reaches (expired waits left fewer
            // than k logits) keeps E - 1, as the rounds of a maximum over zero keys give it.
            wave_sync();  // (every lane's keys, written while polling)
            const uint32_t key = lane < E ? s_key[lane] : 0u;
            const int rank = count_greater_n<64>(s_key, key);
            if (lane < k) sh.idx[lane] = E - 1;
            wave_sync();
            if (key != 0u && rank < k) sh.idx[rank] = lane;
            wave_sync();
            if (lane < k) myc = sh.idx[lane];
        } else {
            const int epl = (E + 63) >> 6;
            wave_sync();  // (every lane's keys, written while polling)
            if (epl <= 2) xc_topk<2>(sh, s_key, E, k, lane, myc);
            else if (epl <= 4) xc_topk<4>(sh, s_key, E, k, lane, myc);
            else if (epl <= 8) xc_topk<8>(sh, s_key, E, k, lane, myc);
            else xc_topk<XC_MAXE / 64>(sh, s_key, E, k, lane, myc);
        }
        if (lane < k) myv = s_lv[myc];
    } else if (lane < k) {
        myc = (int)idx_pre;
    }
    xc_stamp_r(a, sh, 3);
    const bool act = lane < k, shr = has_sh && lane == k;
    int64_t base = 0;
    if (act && myc >= 0 && myc < E) base = sh.u.r.rt[myc];
    if (shr) base = a.srec;
    if (lane < ks) {
        sh.rb[lane] = a.planned ? base : 0;
        sh.idx[lane] = myc;
    }
}

// ---------------------------------------------------------------------------------------
// routing, part 2, by the routing wave of the up items before it requests its own weights (the
// other waves' weights load meanwhile): softmax over the E logits
// (fp32), the top-k weights (renormalised when asked), the HOBBIT levels and skips (the shared
// row: level 0, never skipped, weight sigmoid(shared gate logit)); sh.rw[j] = the weight of table
// row j, 0 for a row that does not run; the report's indices, weights, levels and choices.
// ---------------------------------------------------------------------------------------
template <int XDT>
__device__ __forceinline__ void xc_weigh(const XcArgs &a, XcShared &sh, int myc, float myv, bool poisoned, float w_pre) {
    if (a.rows_b != nullptr) return;
    const int lane = threadIdx.x & 63;
    const int k = a.k, E = a.E, ks = a.ks;
    const bool has_sh = a.sgate != nullptr;
    const float *s_lv = sh.u.r.lv;
    float myw = 0.f, myp = 0.f;
    if (a.Wr != nullptr) {
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
        myw = w_pre;
    }
    xc_stamp_r(a, sh, 4);
    const bool act = lane < k, shr = has_sh && lane == k;
    int lvl;
    bool skip;
    double s;
    slot_level(lane, k, act ? myw : 0.f, a.pol, sh.w, sh.sorted, &sh.tot, lvl, skip, true, &s);
    if (shr) lvl = 0, skip = false;
    xc_stamp_r(a, sh, 5);
    float wt = myw;
    if (shr) {
        const float l = s_lv[E];
        wt = l != l ? l : rnd_act<XDT>(1.0f / (1.0f + expf(-l)));
    }
    if (lane < ks) {
        const bool usable = sh.rb[lane] != 0;
        // one record precision: a level-0 miss below the cache-miss threshold is looked up again
        // at level 1, i.e. the same precision, and stays a miss at level 1
        if (act && !usable && miss_downgrade(a.pol, lvl, s)) lvl = 1;
        sh.rw[lane] = (act || shr) && !skip && usable ? wt : 0.f;
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
// the row's routed weight into the XCD's h area at local index f - seg0. Two steps: the loads
// (x raw, every weight and scale: no load waits on another one's result), issued as soon as the
// row's record is known, then, once routing part 2 has weighed the row, the dot products.
// ---------------------------------------------------------------------------------------
template <int PREC>
struct XcX {
    uint4 r[DlFmt<PREC>::CPL][DlFmt<PREC>::VPC / 8 > 0 ? DlFmt<PREC>::VPC / 8 : 1];
};
template <int PREC>
struct XcUp {
    uint4 qg[DlFmt<PREC>::NPU][DlFmt<PREC>::CPL], qu[DlFmt<PREC>::NPU][DlFmt<PREC>::CPL];
    uint32_t sg[DlFmt<PREC>::NPU][DlFmt<PREC>::CPL], su[DlFmt<PREC>::NPU][DlFmt<PREC>::CPL];
    uint32_t okm;  // chunk (p, i) inside the row: bit p * CPL + i
};

// the item's h values as zeros (a row that does not run), so the down items never wait
template <int PREC>
__device__ __forceinline__ void xc_up_zero(const XcArgs &a, int f0, int seg0, uint64_t *hx, uint32_t tag) {
    constexpr int NPU = DlFmt<PREC>::NPU;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int lg = a.lg_up, G = 1 << lg, RPW = 64 >> lg;
    const int slot = lane >> lg, cl = lane & (G - 1);
    const int I = a.I, j = f0 / I, i0 = f0 % I;
    const int pair0 = i0 + wave * NPU * RPW;
    if (cl == G - 1)
#pragma unroll
        for (int p = 0; p < NPU; ++p) {
            const int r = pair0 + p * RPW + slot;
            if (r < i0 + a.hpi) st_local(hx + (j * I + r - seg0), 0u, tag);
        }
}

// the lane's x chunks of a gate/up row (raw), loaded at the start of the launch with the router's
template <int PREC>
__device__ __forceinline__ void xc_up_x(const XcArgs &a, XcX<PREC> &xr) {
    constexpr int CPL = DlFmt<PREC>::CPL, VPC = DlFmt<PREC>::VPC;
    const int lane = threadIdx.x & 63;
    const int G = 1 << a.lg_up, cl = lane & (G - 1);
    const int C = a.H / VPC;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c = min(cl + i * G, C - 1);
        const uint4 *src = reinterpret_cast<const uint4 *>(a.x) + (size_t)c * (VPC / 8);
#pragma unroll
        for (int m = 0; m < VPC / 8; ++m) xr.r[i][m] = src[m];
    }
}

// step 1: false (after writing the zeros) when row j has no record
template <int PREC, int XDT>
__device__ __forceinline__ bool xc_up_issue(const XcArgs &a, const XcShared &sh, int f0, int seg0, uint64_t *hx,
                                            uint32_t tag, XcUp<PREC> &u) {
    constexpr int CPL = DlFmt<PREC>::CPL, NPU = DlFmt<PREC>::NPU, VPC = DlFmt<PREC>::VPC;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int lg = a.lg_up, G = 1 << lg, RPW = 64 >> lg;
    const int slot = lane >> lg, cl = lane & (G - 1);
    const int I = a.I, H = a.H;
    const int j = f0 / I, i0 = f0 % I;
    const int pair0 = i0 + wave * NPU * RPW;
    const int64_t base = uni64(sh.rb[j]);  // (j is the same for the whole workgroup)
    if (base == 0) {
        xc_up_zero<PREC>(a, f0, seg0, hx, tag);
        return false;
    }
    // uniform bases, 32-bit lane offsets stepped row by row (no 64-bit products per load)
    gbyte *qb = gbytes(base + a.off_gq);
    gbyte *sb = gbytes(base + a.off_gs);
    const int C = H / VPC;
    const uint32_t RB = (uint32_t)C * 16;
    const uint32_t step = (uint32_t)RPW * RB, upo = (uint32_t)I * RB;
    const int ng = sc_cols<PREC>(H, a.gs_up);
    const int r0 = pair0 + slot;  // row of pass 0 (within the item: hpi divides the unit)
    u.okm = 0;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c0 = cl + i * G;
        const int c = min(c0, C - 1);
        const uint32_t qo = __umul24(r0, RB) + (uint32_t)c * 16;
        const int cg = sc_col<PREC>(c, a.gs_up);
#pragma unroll
        for (int p = 0; p < NPU; ++p) {
            u.okm |= (c0 < C ? 1u : 0u) << (p * CPL + i);
            u.qg[p][i] = gld16_nt(qb + (qo + p * step));
            u.qu[p][i] = gld16_nt(qb + (qo + upo + p * step));
            u.sg[p][i] = sc_load<PREC>(sb, sc_off<PREC>(r0 + p * RPW, cg, ng));
            u.su[p][i] = sc_load<PREC>(sb, sc_off<PREC>(r0 + p * RPW + I, cg, ng));
        }
    }
    return true;
}

// step 2: h = w * silu(gate x) * (up x); zeros when routing part 2 gave the row weight 0 (skipped)
template <int PREC, int XDT>
__device__ __forceinline__ void xc_up_finish(const XcArgs &a, XcShared &sh, int f0, int seg0, uint64_t *hx,
                                             uint32_t tag, const XcUp<PREC> &u, const XcX<PREC> &xr) {
    constexpr int CPL = DlFmt<PREC>::CPL, NPU = DlFmt<PREC>::NPU;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int lg = a.lg_up, G = 1 << lg, RPW = 64 >> lg;
    const int slot = lane >> lg, cl = lane & (G - 1);
    const int I = a.I, j = f0 / I, i0 = f0 % I;
    const int pair0 = i0 + wave * NPU * RPW;
    const float wj = sh.rw[j];
    if (wj == 0.f) {
        xc_up_zero<PREC>(a, f0, seg0, hx, tag);
        return;
    }
    // the loaded scales pass through opaque steps here, so that no conversion of them is moved
    // before routing part 2 (which would wait for the loads there)
    XcUp<PREC> w = u;
#pragma unroll
    for (int p = 0; p < NPU; ++p)
#pragma unroll
        for (int i = 0; i < CPL; ++i) asm volatile("" : "+v"(w.sg[p][i]), "+v"(w.su[p][i]));
    LaneVec<PREC, XDT> lv;
    prep_x<PREC, XDT>(xr.r, lv);
    xc_stamp(a, sh, 8);
    float v[2 * NPU];
#pragma unroll
    for (int p = 0; p < NPU; ++p) {
        float pg = 0.f, pu = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const bool ok = (w.okm >> (p * CPL + i)) & 1u;
            const float s0 = ok ? scale_val<PREC>(w.sg[p][i]) : 0.f, s1 = ok ? scale_val<PREC>(w.su[p][i]) : 0.f;
            pg = fmaf(s0 * lv.p2e[i], lane_dot<PREC, XDT>(w.qg[p][i], lv, i), pg);
            pu = fmaf(s1 * lv.p2e[i], lane_dot<PREC, XDT>(w.qu[p][i], lv, i), pu);
        }
        v[2 * p] = pg;
        v[2 * p + 1] = pu;
    }
    grp_total_n<2 * NPU>(v, lg);
    if (cl == G - 1) {
#pragma unroll
        for (int p = 0; p < NPU; ++p) {
            const int r = pair0 + p * RPW + slot;
            st_local(hx + (j * I + r - seg0), __float_as_uint(wj * silu_mul_fast(v[2 * p], v[2 * p + 1])), tag);
        }
    }
}

// ---------------------------------------------------------------------------------------
// down item: output rows [row0w, ...) of each wave over the XCD's segment (nch chunks of VPC
// values, flattened over the table rows it spans)
// ---------------------------------------------------------------------------------------
template <int PREC>
struct XcDown {
    uint4 q[XcFmt<PREC>::NPD][DlFmt<PREC>::CPL];
    uint32_t s[XcFmt<PREC>::NPD][DlFmt<PREC>::CPL];
    uint32_t ok;  // bit p * CPL + i: chunk (p, i) counts (the others multiply by scale 0)
};

template <int PREC>
__device__ __forceinline__ void xc_down_load(const XcArgs &a, const XcShared &sh, int row0, int seg0, int nch,
                                             bool on, XcDown<PREC> &d) {
    constexpr int CPL = DlFmt<PREC>::CPL, NPD = XcFmt<PREC>::NPD, VPC = DlFmt<PREC>::VPC;
    const int lane = threadIdx.x & 63;
    const int lg = a.lg_dn, G = 1 << lg, RPW = 64 >> lg;
    const int slot = lane >> lg, cl = lane & (G - 1);
    const int I = a.I, H = a.H;
    const uint32_t RB = (uint32_t)(I / VPC) * 16;  // bytes of one down row
    const int ng = sc_cols<PREC>(I, a.gs_dn);
    d.ok = 0;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        // the chunk's table row j and column: one base per chunk, 32-bit offsets row by row
        const int c0 = cl + i * G;
        const int c = min(c0, max(nch - 1, 0));
        const int f = seg0 + c * VPC;  // flattened h index of the chunk's first value
        const int j = min(f / I, a.ks - 1), col = f - j * I;
        const int64_t base = nch > 0 && on ? sh.rb[j] : 0;
        // rows without a record (and a workgroup without a down part) read the activation vector
        // (in bounds) at offset 0, scale 0
        gbyte *qb = base != 0 ? gbytes(base + a.off_dq) : gbytes(a.x);
        gbyte *sb = base != 0 ? gbytes(base + a.off_ds) : gbytes(a.x);
        const uint32_t co = base != 0 ? (uint32_t)(col / VPC) * 16 : 0u;
        const int cg = sc_col<PREC>(col / VPC, a.gs_dn);
#pragma unroll
        for (int p = 0; p < NPD; ++p) {
            const int r0 = row0 + p * RPW + slot;
            const int r = min(r0, H - 1);
            const bool ok = c0 < nch && r0 < H && base != 0;
            d.q[p][i] = gld16_nt(qb + (base != 0 ? __umul24(r, RB) + co : 0u));
            d.s[p][i] = sc_load<PREC>(sb, base != 0 ? sc_off<PREC>(r, cg, ng) : 0u);
            d.ok |= (ok ? 1u : 0u) << (p * CPL + i);
        }
    }
}

// the down rows' partial sums (valid in the last lane of each lane group)
template <int PREC, int XDT>
__device__ __forceinline__ void xc_down_rows(const XcArgs &a, const XcDown<PREC> &d, const LaneVec<PREC, XDT> &lv,
                                             float (&v)[XcFmt<PREC>::NPD]) {
    constexpr int CPL = DlFmt<PREC>::CPL, NPD = XcFmt<PREC>::NPD;
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
// ---------------------------------------------------------------------------------------
// down item `item` of XCD x: output rows [d * dr, ...) (d = item - nu) over the XCD's segment
// [seg0, seg0 + seg_len) of h: the down weights (after the gate/up weights' head start, for a
// first item), the segment's h from the XCD's L2 into LDS, the products, then the partial rows:
// the combiner of the row block (d % 8 == x) sums the 8 XCDs' partials and writes the output
// ---------------------------------------------------------------------------------------
template <int XDT, int PREC>
__device__ __forceinline__ void xc_down_item(const XcArgs &a, XcShared &sh, const int item, const bool first, const int x,
                                             const int seg0, const int seg_len, uint64_t *hx, uint64_t *part,
                                             const uint32_t tag, const int spin) {
    constexpr int VPC = DlFmt<PREC>::VPC, NPD = XcFmt<PREC>::NPD;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // 3. the down rows over the segment: their weights (after the gate/up weights' head start),
    //    the segment's h -> LDS (piece-major: piece m of chunk c at (m * C + c) * 4), the products
    const int d = item - a.nu;
    const int lgd = a.lg_dn, G = 1 << lgd, RPW = 64 >> lgd;
    const int row0 = d * a.dr + wave * NPD * RPW;
    const int nch = seg_len / VPC;
    if (first && a.defer != 0u) {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        const uint32_t defer = (uint32_t)uni((int)a.defer);
        while (__builtin_amdgcn_s_memrealtime() - t0 < defer) __builtin_amdgcn_s_sleep(8);
    }
    XcDown<PREC> dd;
    xc_down_load<PREC>(a, sh, row0, seg0, nch, true, dd);
    if (first && tag != 0u) xc_gen_read(a.ws);
    xc_stamp(a, sh, 8);
    float *s_h = sh.u.h;
    const int C = nch > 0 ? nch : 1;
    bool h_ok = true;
    for (int w0 = 0; w0 < seg_len; w0 += 256 * 8) {
        // two rounds of 8 words in flight (every round loads all 8, at clamped indices, so the
        // wait for the older round is exact)
        uint32_t need = 0;
#pragma unroll
        for (int m = 0; m < 8; ++m)
            if (w0 + tid + 256 * m < seg_len) need |= 1u << m;
        const uint64_t *hs = hx + w0 + tid;
        const int lim = seg_len - 1 - w0 - tid;  // (index of the last word, relative)
        auto take = [&](const uint64_t (&v)[8]) {
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                if ((need & (1u << m)) && tag_ok(v[m], tag)) {
                    const int i = w0 + tid + 256 * m;
                    const int c = i / VPC, qq = i - c * VPC;
                    s_h[((qq >> 2) * C + c) * 4 + (qq & 3)] = __uint_as_float((uint32_t)v[m]);
                    need &= ~(1u << m);
                }
            }
        };
        uint64_t va[8], vb[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) va[m] = ld_local(hs + min(256 * m, max(lim, 0)));
        int it = 0;
        for (; it < spin; it += 2) {
#pragma unroll
            for (int m = 0; m < 8; ++m) vb[m] = ld_local(hs + min(256 * m, max(lim, 0)));
            take(va);
            if (!__syncthreads_or(need != 0)) break;
#pragma unroll
            for (int m = 0; m < 8; ++m) va[m] = ld_local(hs + min(256 * m, max(lim, 0)));
            take(vb);
            if (!__syncthreads_or(need != 0)) break;
        }
        if (it >= spin) {
            h_ok = false;
            if (tid == 0) flag_error(a.ws + XC_ERR);
        }
    }
    xc_stamp(a, sh, 10);
    LaneVec<PREC, XDT> lh;
    load_h<PREC, XDT>(s_h, lane & (G - 1), G, C, lh);
    float v[NPD];
    xc_down_rows<PREC, XDT>(a, dd, lh, v);
    if (!h_ok)
#pragma unroll
        for (int p = 0; p < NPD; ++p) v[p] = __uint_as_float(0x7fc00000u);
    xc_stamp(a, sh, 11);
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
            // two rounds of the 8 words in flight at once (each round loads all 8, so the
            // compiler's wait for the older round is exact): a new round every poll, not every
            // round trip
            const uint64_t *src = part + r0 + rr;
            float val[XC_N];
            uint32_t need = 0xFFu & ~(1u << x);
            val[x] = sh.part[rr];
            uint64_t wa[XC_N], wb[XC_N];
#pragma unroll
            for (int xx = 0; xx < XC_N; ++xx) wa[xx] = ld_tag(src + (size_t)xx * a.H);
            for (int it = 0; it < spin; it += 2) {
#pragma unroll
                for (int xx = 0; xx < XC_N; ++xx) wb[xx] = ld_tag(src + (size_t)xx * a.H);
#pragma unroll
                for (int xx = 0; xx < XC_N; ++xx)
                    if ((need & (1u << xx)) && tag_ok(wa[xx], tag)) {
                        val[xx] = __uint_as_float((uint32_t)wa[xx]);
                        need &= ~(1u << xx);
                    }
                if (need == 0) break;
#pragma unroll
                for (int xx = 0; xx < XC_N; ++xx) wa[xx] = ld_tag(src + (size_t)xx * a.H);
#pragma unroll
                for (int xx = 0; xx < XC_N; ++xx)
                    if ((need & (1u << xx)) && tag_ok(wb[xx], tag)) {
                        val[xx] = __uint_as_float((uint32_t)wb[xx]);
                        need &= ~(1u << xx);
                    }
                if (need == 0) break;
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
    xc_stamp(a, sh, 12);
}

// TWO: a second pass of down items (its own instantiation: the single-pass kernel's registers and
// schedule stay those of a kernel without it)
template <int XDT, int PREC, bool TWO>
__global__ __launch_bounds__(256) void k_decode_xcd(XcArgs a) {
    __shared__ XcShared sh;
    const uint64_t t_in = __builtin_amdgcn_s_memrealtime();
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int b = blockIdx.x, x = b % XC_N, q = b / XC_N, NQ = gridDim.x / XC_N;
    uint8_t *wsb = reinterpret_cast<uint8_t *>(a.ws);
    uint64_t *lg = reinterpret_cast<uint64_t *>(wsb + a.off_lg) + (size_t)x * a.lg_stride;
    uint64_t *hx = reinterpret_cast<uint64_t *>(wsb + a.off_h) + (size_t)x * a.h_stride;
    uint64_t *part = reinterpret_cast<uint64_t *>(wsb + a.off_part);
    if (a.trace != nullptr && tid == 0)
        for (int i = 0; i < XC_NST; ++i) sh.st[i] = 0;
    xc_stamp(a, sh, 0);
    // every independent load first: the launch tag (one of 16 copies; never 0), the layer's record
    // table, the given routing, x for the up part; the router rows' x and weights follow; nothing
    // waits before these are all in flight
    const uint32_t gen = ld_co32(a.ws + XC_GEN + 256 * (b % XC_NGEN));
    uint32_t test = ld_co32(a.ws + XC_TEST);
    const bool routed = a.Wr != nullptr, tab = a.rows_b == nullptr;
    int64_t rtv[XC_MAXE / 256];
#pragma unroll
    for (int i = 0; i < XC_MAXE / 256; ++i) {
        const int e = tid + 256 * i;
        rtv[i] = tab && e < a.E ? a.rtab[e] : 0;
    }
    const bool is_up = q < a.nu;
    XcX<PREC> xr;
    if (is_up) xc_up_x<PREC>(a, xr);
    int64_t idx_pre = 0;
    float w_pre = 0.f;
    if (!routed && tab && lane < a.k) {  // (lane: any wave may be the routing wave)
        idx_pre = a.idx_in[lane];
        w_pre = a.w32_in[lane];
    }
    // 1. router rows of this XCD (logits, shared gate), then the routing, by one wave chosen by
    //    workgroup: the workgroups q, q + 32, q + 64 of an XCD usually share a CU, and route on
    //    different SIMDs
    //    With the rows split over the XCDs (E / 8 each), every logit also goes out at agent scope and
    //    one wave of workgroups 0..6 of every XCD relays another XCD's block into this XCD's copy.
    const bool split = tab && routed && a.split != 0;
    const int nr = tab && routed ? (split ? a.E / XC_N : a.E) : 0;
    const int nrows = tab ? nr + (a.sgate != nullptr ? 1 : 0) : 0;
    uint64_t *glg = split ? reinterpret_cast<uint64_t *>(wsb + a.off_glg) : nullptr;
    if (nrows > 0) xc_router<XDT>(a, q, NQ, split ? x * (a.E / XC_N) : 0, nr, nrows, lg, glg, gen);
#pragma unroll
    for (int i = 0; i < XC_MAXE / 256; ++i) {
        const int e = tid + 256 * i;
        if (tab && e < a.E) sh.u.r.rt[e] = rtv[i];
    }
    // (the relay wave is never the routing wave below, nor wave 0, which holds a router row)
    if (split && q < XC_N - 1 && wave == 3 - (q & 1)) xc_relay(a, (x + 1 + q) % XC_N, glg, lg, xc_tag_of(gen));
    const uint32_t tag = (uint32_t)uni((int)xc_tag_of(gen));
    xc_stamp(a, sh, 1);
    const int seg0u = xc_seg_begin(x, a.units), seg1u = xc_seg_begin(x + 1, a.units);
    const int seg0 = seg0u * a.unit, seg_len = (seg1u - seg0u) * a.unit;
    const int f0 = seg0 + q * a.hpi;
    const bool up_work = is_up && q * a.hpi < seg_len;
    const int rwave = (q ^ (q >> 5)) & 3;
    __syncthreads();  // the record table is in LDS
    int myc = 0;
    float myv = 0.f;
    bool poisoned = false;
    asm volatile("" : "+v"(test));  // (read here, long after its load was issued)
    const bool forced = uni((int)test) != 0;
    const int spin = forced ? XC_TEST_SPIN : XC_SPIN;
    if (wave == rwave) xc_rank<XDT>(a, sh, lg, forced ? tag + 0x40000000u : tag, spin, idx_pre, myc, myv, poisoned, t_in);
    __syncthreads();
    xc_stamp(a, sh, 6);
    if (is_up) {
        // 2. h of this item's rows: the loads, routing part 2 meanwhile, then the products
        XcUp<PREC> u;
        // the routing wave weighs the rows before requesting its own weights: behind them, its
        // softmax would wait for the CU's queue of weight requests to drain, and every product
        // waits for the weights it decides
        if (wave == rwave) xc_weigh<XDT>(a, sh, myc, myv, poisoned, w_pre);
        const bool run = up_work && xc_up_issue<PREC, XDT>(a, sh, f0, seg0, hx, tag, u);
        xc_stamp(a, sh, 7);
        __syncthreads();
        if (run) xc_up_finish<PREC, XDT>(a, sh, f0, seg0, hx, tag, u, xr);
        if (tag != 0u) xc_gen_read(a.ws);  // (counted once this item's loads are all used)
        xc_stamp(a, sh, 9);
    } else {
        xc_down_item<XDT, PREC>(a, sh, q, true, x, seg0, seg_len, hx, part, tag, spin);
    }
    if constexpr (TWO) {
        if (b == 0) {  // (the report reads the routing's LDS, which a second item reuses for h)
            __syncthreads();
            xc_report<XDT>(a, sh);
        }
        // a second pass only where the layer has more items than the GPU holds workgroups: every
        // up item is a first item and every second item is a down item of a workgroup whose first
        // item was an up item, so no wait depends on an item that has not started
        if (q + NQ < a.nu + a.nd) {
            __syncthreads();
            xc_down_item<XDT, PREC>(a, sh, q + NQ, false, x, seg0, seg_len, hx, part, tag, spin);
        }
        xc_stamp(a, sh, 13);
    } else {
        xc_stamp(a, sh, 13);
        if (b == 0) {
            __syncthreads();
            xc_report<XDT>(a, sh);
        }
    }
    xc_gen_manage(a.ws, tag);
    if (a.trace != nullptr) {
        __syncthreads();
        if (tid == 0) {
            sh.st[14] = __builtin_amdgcn_s_memrealtime();
            for (int i = 0; i < XC_NST; ++i) a.trace[(size_t)b * XC_NST + i] = sh.st[i];
        }
    }
}

// ---------------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------------
typedef void (*XcKernel)(XcArgs);

template <int XDT, bool TWO>
static XcKernel xc_kernel_x(int prec) {
    switch (prec) {
        case MOEHIP_PREC_INT4: return k_decode_xcd<XDT, MOEHIP_PREC_INT4, TWO>;
        case MOEHIP_PREC_INT8: return k_decode_xcd<XDT, MOEHIP_PREC_INT8, TWO>;
        case MOEHIP_PREC_F16: return k_decode_xcd<XDT, MOEHIP_PREC_F16, TWO>;
        case MOEHIP_PREC_BF16: return k_decode_xcd<XDT, MOEHIP_PREC_BF16, TWO>;
        case MOEHIP_PREC_FP8: return k_decode_xcd<XDT, MOEHIP_PREC_FP8, TWO>;
        default: return nullptr;
    }
}
static XcKernel xc_kernel(int dtype, int prec, bool two) {
    if (dtype == MOEHIP_DT_F16) return two ? xc_kernel_x<MOEHIP_DT_F16, true>(prec) : xc_kernel_x<MOEHIP_DT_F16, false>(prec);
    if (dtype == MOEHIP_DT_BF16) return two ? xc_kernel_x<MOEHIP_DT_BF16, true>(prec) : xc_kernel_x<MOEHIP_DT_BF16, false>(prec);
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
    uint32_t lg_stride, h_stride, off_lg, off_h, off_part, off_glg, total;
    int split;
};

static inline uint32_t xc_al256(size_t v) { return (uint32_t)((v + 255) / 256 * 256); }

// the launch shape of a layer, or ok = 0 when this kernel cannot take it
static XcPlan xc_plan(int prec, int ks, int E, int H, int I) {
    XcPlan p{};
    const int vpc = xc_vpc(prec), cpl = xc_cpl(prec);
    if (vpc == 0 || prec == MOEHIP_PREC_F32 || H > 2048 || H % 32 || I % 32 || E > XC_MAXE || ks > XC_MAXKS) return p;
    const int npu = 4 / cpl, npd = 8 / cpl;  // (XcFmt::NPD)
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
    p.grid = XC_N * (p.nu + p.nd);  // workgroup q: up item q < nu, else down item q - nu
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
    // router rows split over the XCDs from E = XC_SPLIT_E on (E / 8 rows each instead of E per XCD)
    p.split = E >= XC_SPLIT_E && E % XC_N == 0 ? 1 : 0;
    p.off_glg = (uint32_t)off;
    if (p.split) off = xc_al256(off + (size_t)E * 8);
    p.total = (uint32_t)off;
    p.ok = 1;
    return p;
}

// 1 once moehip_device_check confirmed the round-robin XCD dispatch on a device (per device)
static int g_xcd_ok[64];

int xcd_dispatch_ok() {
    int dev = 0;
    return hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64 && g_xcd_ok[dev];
}

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
        (void)hipFree(d);
    }
    (void)hipGetLastError();
    g_xcd_ok[dev] = ok;
    (void)hipSetDevice(prev);
    return ok;
}

size_t xcd_workspace_bytes(int prec, int ks, int E, int H, int I) {
    const XcPlan p = xc_plan(prec, ks, E, H, I);
    return p.ok ? p.total : 0;
}

// the XCD kernel for one launch when it applies: returns MOEHIP_OK, with *used = the kernel
// launched (MOEHIP_KERNEL_XCD or MOEHIP_KERNEL_XCD_TWO) or 0 when the layer or the device does
// not fit this kernel (the caller then runs the item kernels), or an error code
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
    XcKernel kern = xc_kernel(d->dtype, d->prec[0], false);
    XcKernel kern2 = xc_kernel(d->dtype, d->prec[0], true);
    if (kern == nullptr || kern2 == nullptr) return MOEHIP_OK;
    int cus = 0, per_cu = 0, per_cu2 = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(kern), 256, 0) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu2, reinterpret_cast<const void *>(kern2), 256, 0) != hipSuccess)
        return MOEHIP_OK;
    // every workgroup must be resident at once; a layer with more items than that (fp8 rows at the
    // Qwen3-Next shape: 152 items per XCD) runs the two-pass kernel, when every up item can be a
    // first item and no workgroup whose first item is a down item needs a second
    int grid = p.grid;
    int which = MOEHIP_KERNEL_XCD;
    if (grid > per_cu * cus) {
        const int nq = per_cu2 * cus / XC_N;
        if (nq < p.nu || nq < p.nd || p.nu + p.nd > 2 * nq) return MOEHIP_OK;
        grid = nq * XC_N;
        kern = kern2;
        which = MOEHIP_KERNEL_XCD_TWO;
    }
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
    a.off_glg = p.off_glg;
    a.split = p.split && Wr != nullptr && rows_b == nullptr && grid / XC_N >= XC_N ? 1 : 0;
    a.lg_stride = p.lg_stride;
    a.h_stride = p.h_stride;
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
    // 0.85 of the time the HBM needs for the ks gate/up blocks (q + scales) at 8 TB/s, in 10 ns
    // ticks: the down items request theirs after it (measured at the OLMoE int4 bs=1 shape, ms per
    // 16-layer token, one box: 0.2323 with 0.8-0.9 of it, 0.2339 with all of it, 0.2344 with 0.7,
    // 0.2404 with 1.25, 15.1 us per layer without a head start; another box: 0.2314 with 0.8 and
    // 0.85, 0.2319 with 0.9, 0.2332 with 0.99)
    const double gu = (double)(d->offs[0][2] - d->offs[0][0]);
    a.defer = (uint32_t)(ks * gu / 8.0e12 * 1.0e8 * 0.85);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256), 0, as_stream(stream), a);
    *used = which;
    return check_launch("decode_layer (xcd)");
}

}  // namespace moehip
