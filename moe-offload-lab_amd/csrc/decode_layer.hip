// One MoE layer for one decode token in ONE launch:
//   router logits -> softmax / top-k / renorm -> HOBBIT levels, resident copy, tables ->
//   kernel-A rows (h = silu(gate x) * up x) -> kernel-B rows (w * down h) -> combine in table order.
//
// Work distribution: the work items are ordered [router items: 4 expert rows each][up items]
//   [down items], and workgroup b runs items b, b + grid, b + 2 grid, ... in that order. An item
//   only waits on SMALLER items (up and down items for the router rows, down items for the h rows
//   of their table row, the combining down items for the other rows' partial sums). The grid is at
//   most what the GPU holds at once (occupancy x CUs), so every workgroup is, or eventually
//   becomes, resident (other kernels' workgroups drain), and the smallest unfinished item always
//   belongs to a resident workgroup whose earlier items are done: the launch always drains, with
//   no shared counter to take items from. Every wait is also bounded (WAIT_SPINS polls); on expiry
//   the workgroup records an error in the workspace and writes NaN where the missing data would
//   have gone (routed weights, partial rows, output rows), so no launch can hang and none returns
//   a plausible wrong answer.
//
// Routing is computed by EVERY workgroup that runs an up or down item, from the logits: wave 0
// polls the E logits, ranks them, applies softmax / renorm / HOBBIT and picks each table row's
// resident copy (from the record table, prefetched into LDS by the other waves while the logits
// are awaited). Every workgroup computes the same routing bit for bit, so no routing record has
// to travel between workgroups: the only exchange before the weight loads is the logits.
//
// Items are sized so that every lane holds its whole share of the item's weights (8 x 16 bytes)
// in registers: an up item issues all its loads as soon as its routing is known, and a down
// item issues its loads BEFORE waiting for h, so the layer's weight bytes are all requested
// right after the routing and the dependency waits overlap the HBM transfers.
//
// Cross-workgroup data is TAGGED instead of guarded by counters: every exchanged value (logit,
// h element, partial output row) is one 64-bit word (launch tag << 32 | payload) written with one
// agent-scope (sc1) atomic store, and a consumer polls the words it needs (all of them at once,
// then the missing ones again) until they carry this launch's tag. The logits are written in
// NLC copies on different memory channels, so that hundreds of polling workgroups do not queue on
// one channel. A producer never waits for its stores and nothing needs resetting between
// launches: the tag is the workspace's launch generation + 1, read by every workgroup at start
// (from one of NGEN copies). Each workgroup then counts itself in one of NSUB reader counters
// (no return value, so nothing waits on it; one counter per workgroup would serialise ~10 ns
// per workgroup on one address), and the router items, which finish early, wait until their
// counters hold every workgroup of the grid, clear them, and the last of them advances the
// generation: every workgroup of this launch holds its tag by then.
//
// Arithmetic (16-bit activations): weights are turned into fp16 pairs with the 1024 + n
// magic-exponent trick (int4: n in the mantissa low bits, or 16 n for the odd nibble; int8:
// q + 128) and multiplied with fp16 pairs of the vector by v_dot2_f32_f16 (exact products, fp32
// accumulation); the constant 1024-offsets are removed with one per-chunk correction term.
// bf16 vectors and h are scaled per 16-byte weight chunk by a power of two into fp16's range.
// fp8 / bf16 records and fp32 activations use fp32 FMAs.
//
// Determinism: output rows are summed by the down items of the last table row, in table order.

#include <limits.h>

#include "decide.hpp"
#include "lanevec.hpp"

namespace moehip {

constexpr int DL_MAXP = 4;
constexpr int DL_MAXROW = 2048;       // 64 lanes x 32 vector values per lane
constexpr int WAIT_SPINS = 1 << 22;   // x ~0.3 us per poll: a wait gives up after ~1 s
// header words (each on its own 128-byte line): NSUB reader counters of the launch generation,
// sticky error flag, the count of drained reader counters, and NGEN copies of the launch
// generation 1 KB apart (read by every workgroup at start)
constexpr int NGEN = 16;
constexpr int NSUB = 16;
enum { W_READ = 0, W_ERR = NSUB * 32, W_TOP = NSUB * 32 + 32, W_TEST = NSUB * 32 + 64, W_GEN = 1024,
       W_HDR = W_GEN + 256 * NGEN };
// W_TEST: a word the library never writes (zero from the workspace's first zero-fill; the XCD
// kernel reads the same word). When a test sets it, every later launch on that workspace polls
// the logits for a tag that is never written and gives up after TEST_SPINS polls: an expired wait
// forced from the host, in a launch whose every workgroup still exits normally (the routing is
// then poisoned, so every other wait is still satisfied, and the generation's counting keeps its
// full bound).
constexpr int TEST_SPINS = 8;
constexpr int NLC = 1;         // copies of the logits
constexpr int RT_LDS = 1024;   // record-table entries (P * E) prefetched into LDS
constexpr int REC_SHARED = 0xFFF;  // expert field of the shared row in a routing record
constexpr int NRC = 8;             // copies of the routing record, REC_STRIDE words apart (4 KB + 128 B:
constexpr int REC_STRIDE = 528;    // different pages and lines, so the pollers spread over channels)
// 64-bit words between two copies of the logits (E routed + the shared gate): a whole number of
// 256-byte blocks plus one, so that consecutive copies start on different channels
__host__ __device__ __forceinline__ size_t logit_stride_words(int E) { return ((size_t)(E + 1) * 8 + 255) / 256 * 32 + 32; }

struct LayerArgs {
    const void *x;          // (H) activation dtype
    const void *Wr;         // (E, H) router weights, or null when idx_in/w32_in are given
    const int64_t *idx_in;  // (k) routed experts (router skipped) or null
    const float *w32_in;    // (k)
    const int64_t *rows_b;  // (P, k) explicit table rows (record bases, 0 = unused) or null:
    const float *rows_w;    //        routing and decision skipped (moehip_decode_rows)
    const int64_t *rtab;    // (P, E) base addresses of this layer's resident records, 0 = absent
    int64_t offs[DL_MAXP][4];
    int prec[DL_MAXP];
    int gs_up[DL_MAXP];
    int gs_dn[DL_MAXP];
    int planned[DL_MAXP];
    int lg_up[DL_MAXP];     // log2 lanes per gate/up row and per down row
    int lg_dn[DL_MAXP];
    int nub[DL_MAXP];       // up / down items per table row of precision p
    int ndb[DL_MAXP];
    int up_base[DL_MAXP];   // first up / down item of precision p (relative)
    int dn_base[DL_MAXP];
    int lv2p[3];
    int P, E, k, H, I, renorm, accumulate;
    int ks;                 // table rows per precision: k routed (+ 1 shared)
    const void *sgate;      // (H) shared-expert gate vector or null
    int64_t srec[DL_MAXP];  // shared-expert record per precision (0 = absent)
    int NU, ND;             // up / down items
    uint32_t defer;         // one-item kernel: down items request their weights this many real-time
                            // ticks (10 ns) after the routing, when the gate/up weights have streamed
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
    uint32_t off_rec, off_logits, off_h, off_part;  // byte offsets in ws of the tagged arrays
    uint64_t *trace;        // optional per-item trace: [ticket] = (start, end, workgroup) or null
    uint64_t *stage;        // with trace: 8 stage stamps per item after the trace rows
};

template <typename T>
__device__ __forceinline__ T *ws_ptr(const LayerArgs &a, uint32_t off) {
    return reinterpret_cast<T *>(reinterpret_cast<uint8_t *>(a.ws) + off);
}

// profiling stamp i of the current item (thread 0, trace runs only)
// Stamps are kept in LDS and written out once at the end of the item (stamp_flush): a global
// store per stamp would make the wave's next memory wait also wait for that store's
// acknowledgement (vmcnt counts stores), which distorts exactly the polls being timed.
// Slots 0-7: the item's stages; 8-15: the routing stamps of the reporting workgroup.
__device__ __forceinline__ uint64_t *stamp_buf() {
    __shared__ uint64_t buf[16];
    return buf;
}
__device__ __forceinline__ void stamp(uint64_t *st, int i) {
    if (st != nullptr && threadIdx.x == 0) stamp_buf()[i] = __builtin_amdgcn_s_memrealtime();
}
__device__ __forceinline__ void stamp_clear() {
    if (threadIdx.x < 16) stamp_buf()[threadIdx.x] = 0;
}
// after a barrier: thread 0 copies the item's stamps (and the routing stamps, if any) out
__device__ __forceinline__ void stamp_flush(uint64_t *st, uint64_t *ts) {
    if (threadIdx.x != 0) return;
    const uint64_t *b = stamp_buf();
    for (int i = 0; i < 8; ++i)
        if (st != nullptr && b[i] != 0) st[i] = b[i];
    for (int i = 0; i < 8; ++i)
        if (ts != nullptr && b[8 + i] != 0) ts[i] = b[8 + i];
}

__device__ __forceinline__ int pick4(const int (&v)[4], int i) {
    const int v0 = uni(v[0]), v1 = uni(v[1]), v2 = uni(v[2]), v3 = uni(v[3]);
    return i == 0 ? v0 : (i == 1 ? v1 : (i == 2 ? v2 : v3));
}
__device__ __forceinline__ int64_t pick_off(const int64_t (&v)[4][4], int p, int f) {
    int64_t r[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int64_t a0 = uni64(v[q][0]), a1 = uni64(v[q][1]), a2 = uni64(v[q][2]), a3 = uni64(v[q][3]);
        r[q] = f == 0 ? a0 : (f == 1 ? a1 : (f == 2 ? a2 : a3));
    }
    return p == 0 ? r[0] : (p == 1 ? r[1] : (p == 2 ? r[2] : r[3]));
}
// the precision block holding relative item u (base[] ascending, base[0] = 0)
__device__ __forceinline__ int block_of(const int (&base)[4], int P, int u) {
    int p = 0;
    if (P > 1 && u >= uni(base[1])) p = 1;
    if (P > 2 && u >= uni(base[2])) p = 2;
    if (P > 3 && u >= uni(base[3])) p = 3;
    return p;
}

// ---------------------------------------------------------------------------------------
// up item (one wave's share): NPU passes of RPW row pairs, h[r] = silu(gate_r . x) * (up_r . x)
// ---------------------------------------------------------------------------------------
template <int PREC, int XDT>
__device__ __forceinline__ void up_rows(gbyte *qb, gbyte *sb, const LaneVec<PREC, XDT> &lv, int pair0,
                                        int I, int H, int gs, int lg, uint64_t *hout, uint32_t tag, uint64_t *st) {
    constexpr int VPC = DlFmt<PREC>::VPC, CPL = DlFmt<PREC>::CPL, NPU = DlFmt<PREC>::NPU;
    const int lane = threadIdx.x & 63;
    const int G = 1 << lg, RPW = 64 >> lg;
    const int slot = lane >> lg, cl = lane & (G - 1);
    const int C = H / VPC;
    const size_t RB = (size_t)C * 16;
    uint4 qg[NPU][CPL], qu[NPU][CPL];
    uint32_t sg[NPU][CPL], su[NPU][CPL];
    // branch-free: out-of-range lanes load an in-range chunk and get a zero scale
#pragma unroll
    for (int p = 0; p < NPU; ++p) {
        const int r0 = pair0 + p * RPW + slot;
        const int r = min(r0, I - 1);
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c0 = cl + i * G;
            const int c = min(c0, C - 1);
            const bool ok = r0 < I && c0 < C;
            qg[p][i] = gld16_nt(qb + (size_t)r * RB + (size_t)c * 16);
            qu[p][i] = gld16_nt(qb + (size_t)(r + I) * RB + (size_t)c * 16);
            const uint32_t a0 = scale_bits<PREC>(sb, r, c, H, gs), a1 = scale_bits<PREC>(sb, r + I, c, H, gs);
            sg[p][i] = ok ? a0 : 0u;
            su[p][i] = ok ? a1 : 0u;
        }
    }
    if (st != nullptr) {  // profiling: separate the load latency from the arithmetic
        __builtin_amdgcn_s_waitcnt(0);
        stamp(st, 2);
    }
    // every pass's dot products first (independent: the compiler interleaves them), then the
    // lane-group reductions step by step over all values, then h = silu(g) * u
    float v[2 * NPU];
#pragma unroll
    for (int p = 0; p < NPU; ++p) {
        float pg = 0.f, pu = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            pg = fmaf(scale_val<PREC>(sg[p][i]) * lv.p2e[i], lane_dot<PREC, XDT>(qg[p][i], lv, i), pg);
            pu = fmaf(scale_val<PREC>(su[p][i]) * lv.p2e[i], lane_dot<PREC, XDT>(qu[p][i], lv, i), pu);
        }
        v[2 * p] = pg;
        v[2 * p + 1] = pu;
    }
    grp_total_n<2 * NPU>(v, lg);
    if (cl == G - 1) {
#pragma unroll
        for (int p = 0; p < NPU; ++p) {
            const int r = pair0 + p * RPW + slot;
            if (r < I) st_tag(hout + r, __float_as_uint(silu_mul(v[2 * p], v[2 * p + 1])), tag);
        }
    }
    stamp(st, 3);
}

// ---------------------------------------------------------------------------------------
// down item (one wave's share): weights loaded first, then (after the caller's wait) h and
// NPD passes of RPW rows, partial[r] = wt * (down_r . h)
// ---------------------------------------------------------------------------------------
template <int PREC>
struct DownRegs {
    uint4 q[DlFmt<PREC>::NPD][DlFmt<PREC>::CPL];
    uint32_t s[DlFmt<PREC>::NPD][DlFmt<PREC>::CPL];
};

template <int PREC>
__device__ __forceinline__ void down_load(gbyte *qb, gbyte *sb, int row0, int H, int I, int gs, int lg,
                                          DownRegs<PREC> &d) {
    constexpr int VPC = DlFmt<PREC>::VPC, CPL = DlFmt<PREC>::CPL, NPD = DlFmt<PREC>::NPD;
    const int lane = threadIdx.x & 63;
    const int G = 1 << lg, RPW = 64 >> lg;
    const int slot = lane >> lg, cl = lane & (G - 1);
    const int C = I / VPC;
    const size_t RB = (size_t)C * 16;
    // branch-free: out-of-range lanes load an in-range chunk and get a zero scale
#pragma unroll
    for (int p = 0; p < NPD; ++p) {
        const int r0 = row0 + p * RPW + slot;
        const int r = min(r0, H - 1);
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c0 = cl + i * G;
            const int c = min(c0, C - 1);
            d.q[p][i] = gld16_nt(qb + (size_t)r * RB + (size_t)c * 16);
            const uint32_t sv = scale_bits<PREC>(sb, r, c, I, gs);
            d.s[p][i] = (r0 < H && c0 < C) ? sv : 0u;
        }
    }
}

template <int PREC, int XDT>
__device__ __forceinline__ void down_rows(const DownRegs<PREC> &d, const LaneVec<PREC, XDT> &lv, int row0, int H,
                                          int lg, float wt, uint64_t *pout, uint32_t tag) {
    constexpr int CPL = DlFmt<PREC>::CPL, NPD = DlFmt<PREC>::NPD;
    const int lane = threadIdx.x & 63;
    const int G = 1 << lg, RPW = 64 >> lg;
    const int slot = lane >> lg, cl = lane & (G - 1);
    float v[NPD];
#pragma unroll
    for (int p = 0; p < NPD; ++p) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; ++i)
            acc = fmaf(scale_val<PREC>(d.s[p][i]) * lv.p2e[i], lane_dot<PREC, XDT>(d.q[p][i], lv, i), acc);
        v[p] = acc;
    }
    grp_total_n<NPD>(v, lg);
    if (cl == G - 1) {
#pragma unroll
        for (int p = 0; p < NPD; ++p) {
            const int r = row0 + p * RPW + slot;
            if (r < H) st_tag(pout + r, __float_as_uint(wt * v[p]), tag);
        }
    }
}

// ---------------------------------------------------------------------------------------
// routing of this launch, computed by each workgroup that runs up / down items (all threads
// call; waves 1-3 prefetch the record table into LDS while wave 0 polls the logits).
// Softmax / top-k / renorm / HOBBIT / resident copy; the result is each table row's weight and
// record address in LDS (s_rw / s_rb, P * ks rows precision-major; weight 0 = nothing to run).
// Logits and keys are staged in LDS (lane l handles l, l + 64, ...). Top-k: for E <= 64 every
// lane counts the keys above its own; otherwise k rounds of a wave-wide maximum over 32-bit keys.
// For 16-bit activations the key packs the order-preserving bits of the logit above
// (1023 - index), so the largest key is the largest logit and, among equal logits, the lowest
// index (torch.topk / the reference order); fp32 logits break ties on the index explicitly.
// The reporting workgroup (report = true) also writes the optional readouts.
// ---------------------------------------------------------------------------------------
// LDS of one workgroup
struct DlShared {
    uint32_t tag;
    int routed;
    int poison;
    int forced;                    // the workspace's test word was set (see W_TEST)
    int idx[64];
    float w[64];
    float sorted[64];
    float tot;
    float gl;                      // shared-expert gate logit
    float rw[DL_MAXP * 32];        // table rows: weight (0 = nothing to run)
    uint64_t rb[DL_MAXP * 32];     //             record address
    float wk[DL_MAXP * 32];
    int64_t rt[RT_LDS];            // prefetched record table (P, E)
    __align__(16) float h[DL_MAXROW];  // staged h; logits and keys during the routing
};

template <int XDT>
__device__ __forceinline__ void route_local(const LayerArgs &a, uint32_t tag, DlShared &sh, uint32_t *err, bool report,
                            uint64_t *ts, uint64_t *ist = nullptr, bool publish = false) {
    // the routing wave: blockIdx % 4, so that the routing waves of the workgroups sharing a CU
    // run on different SIMDs; the other three waves prefetch the record table
    const int tid = threadIdx.x, rwave = (tid >> 6) - (int)(blockIdx.x & 3u), lane = tid & 63;
    const int k = a.k, E = a.E, ks = a.ks, P = a.P;
    const bool has_sh = a.sgate != nullptr;
    if (a.rows_b != nullptr) {  // explicit rows: read, nothing to decide
        for (int j = tid; j < P * ks; j += blockDim.x) {
            const int64_t b = a.rows_b[j];
            const float w = a.rows_w[j];
            sh.rb[j] = (uint64_t)b;
            sh.rw[j] = b != 0 ? w : 0.f;
        }
        if (tid == 0) sh.routed = 1;
        __syncthreads();
        return;
    }
    const bool pre = P * E <= RT_LDS;
    const int epl = (E + 63) >> 6;
    float *s_lv = sh.h;
    uint32_t *s_key = reinterpret_cast<uint32_t *>(sh.h + 1024);
#define TS(i) do { if (ts != nullptr && lane == 0) stamp_buf()[8 + (i)] = __builtin_amdgcn_s_memrealtime(); } while (0)
    if (rwave != 0) {
        if (pre) {
            const int o = (tid + 256 - 64 * (int)(blockIdx.x & 3u)) & 255;  // 64 .. 255 in the other waves
            for (int i = o - 64; i < P * E; i += 192) sh.rt[i] = a.rtab[i];
        }
    } else {
        TS(0);
        if (a.Wr != nullptr || has_sh) {
            // every logit of this launch (written by the router items, smaller tickets), all
            // requested at once, then the missing ones again
            const uint64_t *logits = ws_ptr<uint64_t>(a, a.off_logits) + (size_t)(blockIdx.x % NLC) * logit_stride_words(E);
            uint32_t need = 0;
            if (a.Wr != nullptr)
                for (int i = 0; i < epl; ++i)
                    if (lane + 64 * i < E) need |= 1u << i;
            if (has_sh && lane == 0) need |= 1u << 31;
            int nap = 1;
            const bool forced = sh.forced != 0;
            const uint32_t ptag = forced ? tag + 0x40000000u : tag;  // (forced: never written)
            const int spin = forced ? TEST_SPINS : WAIT_SPINS;
            for (int it = 0; it < spin && __ballot(need != 0) != 0ull; ++it) {
                uint64_t v[16];
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (i < epl && (need & (1u << i))) v[i] = ld_tag(logits + lane + 64 * i);
                const uint64_t vg = (need >> 31) ? ld_tag(logits + E) : 0ull;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    if (i < epl && (need & (1u << i)) && tag_ok(v[i], ptag)) {
                        const int c = lane + 64 * i;
                        const float l = __uint_as_float((uint32_t)v[i]);
                        s_lv[c] = l;
                        s_key[c] = logit_key<XDT>(l, c);
                        need &= ~(1u << i);
                    }
                }
                if ((need >> 31) && tag_ok(vg, ptag)) {
                    sh.gl = __uint_as_float((uint32_t)vg);
                    need &= ~(1u << 31);
                }
                if (__ballot(need != 0) != 0ull) backoff(nap, 2);
                if (it == spin - 1 && lane == 0) flag_error(err);
            }
            if (a.Wr != nullptr)
                for (int i = 0; i < epl; ++i) {  // logits still missing after the wait: never chosen
                    if (need & (1u << i)) {
                        s_lv[lane + 64 * i] = -INFINITY;
                        s_key[lane + 64 * i] = 0u;
                    }
                }
            if (need >> 31) sh.gl = __uint_as_float(0x7fc00000u);  // gate weight NaN
            // an expired wait must not give a plausible answer: every routed weight becomes NaN,
            // so the output of this launch is NaN (and the workspace error flag is set)
            if (lane == 0) sh.poison = __ballot(need != 0) != 0ull ? 1 : 0;
            if (a.Wr != nullptr && E <= 64)
                for (int c = E + lane; c < 64 + 3; c += 64) s_key[c] = 0u;  // pad to whole quads
        }
        if (ist != nullptr && lane == 0) stamp_buf()[6] = __builtin_amdgcn_s_memrealtime();
    }
    __syncthreads();
    // E <= 64 with 16-bit logits (distinct keys below 2^26): every wave counts, for each lane's
    // key, the larger keys among its 16 ((key - other) >> 31 is 1 exactly when other > key);
    // the routing wave adds the four counts up
    int *s_prt = reinterpret_cast<int *>(sh.h + 256);
    const bool rank4 = XDT != MOEHIP_DT_F32 && a.Wr != nullptr && E <= 64;
    if (rank4) {
        const int wv = tid >> 6;
        const uint32_t key = lane < E ? s_key[lane] : 0u;
        uint32_t part = 0;
#pragma unroll
        for (int q = 0; q < 16; q += 4) {
            const uint4 o = *reinterpret_cast<const uint4 *>(s_key + 16 * wv + q);
            part += ((key - o.x) >> 31) + ((key - o.y) >> 31) + ((key - o.z) >> 31) + ((key - o.w) >> 31);
        }
        s_prt[wv * 64 + lane] = (int)part;
        __syncthreads();
    }
    if (rwave == 0) {
        TS(1);
        int myc = 0;      // lane j < k: expert of rank j
        float myw = 0.f;  // and its fp32 weight (rounded to the activation dtype)
        float myp = 0.f;  // (its weight before the rounding, for w_out)
        int64_t rt[DL_MAXP] = {0, 0, 0, 0};  // and the addresses of its resident records
        if (a.Wr != nullptr) {
            float myv = 0.f;
            if (E <= 64) {
                // one logit per lane: its rank is the number of larger keys (keys are distinct for
                // 16-bit logits; fp32 ties go to the lower index)
                const uint32_t key = lane < E ? s_key[lane] : 0u;
                const float lvv = lane < E ? s_lv[lane] : -INFINITY;
                int rank = 0;
                if (rank4) {
                    rank = s_prt[lane] + s_prt[64 + lane] + s_prt[128 + lane] + s_prt[192 + lane];
                } else {
#pragma unroll
                    for (int q = 0; q < 64; q += 4) {  // every lane reads the same 4 keys (LDS
                                                       // broadcast); keys past E are 0, never counted
                        const uint4 o = *reinterpret_cast<const uint4 *>(s_key + q);
                        const uint32_t ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            if constexpr (XDT == MOEHIP_DT_F32) rank += (ov[u] > key) || (ov[u] == key && q + u < lane);
                            else rank += ov[u] > key;
                        }
                    }
                }
                // a slot that no key reaches (an expired wait left fewer than k logits, whose keys
                // are 0) keeps E - 1, as the rounds of a maximum over zero keys give it: every
                // workgroup routes the same way, so every other wait of the launch is still met
                if (lane < k) {
                    s_key[512 + lane] = (uint32_t)(E - 1);
                    s_lv[512 + lane] = -INFINITY;
                }
                __builtin_amdgcn_wave_barrier();
                if (lane < E && rank < k && key != 0u) {
                    s_key[512 + rank] = (uint32_t)lane;
                    s_lv[512 + rank] = lvv;
                }
                __builtin_amdgcn_wave_barrier();
                if (lane < k) {
                    myc = (int)s_key[512 + lane];
                    myv = s_lv[512 + lane];
                }
            }
            for (int r = 0; r < k && E > 64; ++r) {
                uint32_t lb = 0u;
                int lc = lane;
                for (int i = 0; i < epl; ++i) {
                    const int c = lane + 64 * i;
                    const uint32_t kk = c < E ? s_key[c] : 0u;
                    if (kk > lb) lb = kk, lc = c;
                }
                const uint32_t M = wave_max_u32(lb);
                int c;
                if constexpr (XDT == MOEHIP_DT_F32) {
                    // among lanes holding the maximum key, the lowest expert index
                    const uint32_t cand = lb == M ? (uint32_t)(1023 - lc) : 0u;
                    c = 1023 - (int)wave_max_u32(cand);
                } else {
                    (void)lc;
                    c = 1023 - (int)(M & 1023u);
                }
                c = min(c, E - 1);
                const float v = s_lv[c];
                __builtin_amdgcn_wave_barrier();
                if (lane == (c & 63)) s_key[c] = 0u;
                __builtin_amdgcn_wave_barrier();
                if (lane == r) {
                    myc = c;
                    myv = v;
                }
            }
            TS(2);
            if (lane < k && myc >= 0 && myc < E) {  // record-table reads overlap the softmax below
#pragma unroll
                for (int pi = 0; pi < DL_MAXP; ++pi)
                    rt[pi] = pi < P ? (pre ? sh.rt[pi * E + myc] : a.rtab[(size_t)pi * E + myc]) : 0;
            }
            const float m = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(myv), 0));
            float sum = 0.f;
            for (int i = 0; i < epl; ++i)
                if (lane + 64 * i < E) sum += expf(s_lv[lane + 64 * i] - m);
            sum = wave_sum(sum);
            const float p = lane < k ? expf(myv - m) / sum : 0.f;
            const float tot = a.renorm ? wave_sum(p) : 1.f;
            if (lane < k) {
                myp = a.renorm ? p / tot : p;
                myw = sh.poison ? __uint_as_float(0x7fc00000u) : rnd_act<XDT>(myp);
            }
        } else if (lane < k) {
            myc = (int)a.idx_in[lane];
            myw = a.w32_in[lane];
            if (myc >= 0 && myc < E) {
#pragma unroll
                for (int pi = 0; pi < DL_MAXP; ++pi)
                    rt[pi] = pi < P ? (pre ? sh.rt[pi * E + myc] : a.rtab[(size_t)pi * E + myc]) : 0;
            }
        }
        if (has_sh && lane == k) {
            // the shared expert (row k): weight sigmoid(x . g) with x . g rounded to the activation
            // dtype like the gate's output (modeling_qwen3_next.py:793-796), record from srec
            const float l = sh.gl;
            myc = -1;
            myw = l == -INFINITY ? 0.f : (l != l ? l : rnd_act<XDT>(1.0f / (1.0f + expf(-l))));
#pragma unroll
            for (int pi = 0; pi < DL_MAXP; ++pi) rt[pi] = pi < P ? a.srec[pi] : 0;
        }
        TS(3);
        // HOBBIT levels (moelab/policy.py:77-123), resident copy, tables (moelab/fullgraph.py:149-171)
        const int j = lane;
        const bool act = j < k;                  // a routed row
        const bool shr = has_sh && j == k;       // the shared row: level 0, never skipped
        const bool row = act || shr;
        const int e = act ? myc : 0;
        if (act) sh.idx[j] = e;
        const float wj = act ? myw : 0.f;
        int lvl;
        bool skip;
        double s;
        slot_level(j, k, wj, a.pol, sh.w, sh.sorted, &sh.tot, lvl, skip, true, &s);
        if (shr) {
            lvl = 0;
            skip = false;
        }
        TS(4);
        const int l2p0 = uni(a.lv2p[0]), l2p1 = uni(a.lv2p[1]), l2p2 = uni(a.lv2p[2]);
        const bool upg = shr || a.pol.upgrade;
        int chosen = -1;
        for (int pass = 0; pass < 2; ++pass) {
            // the shared row takes its most precise present copy
            const int req = shr ? DL_MAXP - 1 : (lvl == 0 ? l2p0 : (lvl == 1 ? l2p1 : l2p2));
#pragma unroll
            for (int pi = DL_MAXP - 1; pi >= 0; --pi) {
                const bool avail = pi < P && rt[pi] != 0;
                if (avail && (upg ? req >= pi : req == pi)) chosen = pi;
            }
            // a routed level-0 miss below the cache-miss threshold is looked up again at level 1
            if (chosen >= 0 || shr || !miss_downgrade(a.pol, lvl, s)) break;
            lvl = 1;
        }
        const bool usable = chosen >= 0 && pick4(a.planned, chosen) != 0;
        const bool is_miss = row && !skip && !usable;
        // the chosen copy (address, weight) of this row
        const bool sel = row && chosen >= 0 && !skip && usable;
        const int64_t base = !sel ? 0 : (chosen == 0 ? rt[0] : (chosen == 1 ? rt[1] : (chosen == 2 ? rt[2] : rt[3])));
        if (row) {
            for (int pi = 0; pi < P; ++pi) {
                const bool mine = sel && chosen == pi;
                sh.rw[pi * ks + j] = mine ? myw : 0.f;
                sh.rb[pi * ks + j] = mine ? (uint64_t)base : 0ull;
            }
        }
        if (publish && row) {
            // the routing record of a single-precision launch (route_fetch): valid bit, expert
            // (REC_SHARED for the shared row) and the weight's bits in the activation dtype
            const uint32_t wb = XDT == MOEHIP_DT_F16 ? (uint32_t)f32_to_f16_rne(myw) : (__float_as_uint(myw) >> 16);
            const uint32_t pay = (sel ? 0x80000000u : 0u) | ((uint32_t)(shr ? REC_SHARED : e) << 16) | (sel ? wb : 0u);
            for (int c = 0; c < NRC; ++c) st_tag(ws_ptr<uint64_t>(a, a.off_rec) + (size_t)c * REC_STRIDE + j, pay, tag);
        }
        // the readouts, after the record: a store makes the wave's next memory wait also wait for
        // the store's acknowledgement, so none may precede the polls and the record
        const unsigned long long bal = __ballot(is_miss);
        if (report) {
            if (a.logits_out != nullptr && a.Wr != nullptr)
                for (int c = lane; c < E; c += 64) st_act<XDT>(a.logits_out, c, s_lv[c]);
            if (act && a.Wr != nullptr) {
                if (a.idx_out) a.idx_out[j] = myc;
                if (a.w_out) st_act<XDT>(a.w_out, j, myp);
                if (a.w32_out) a.w32_out[j] = myw;
            }
            if (a.info && act) {
                a.info[j] = (float)e;
                a.info[k + j] = skip ? -2.f : (float)chosen;
                a.info[2 * k + j] = (float)lvl;
            }
            if (j == 0 && a.miss != nullptr) a.miss[0] += (float)__popcll(bal);
        }
        if (j == 0) sh.routed = 1;
        TS(5);
        if (ist != nullptr && lane == 0) stamp_buf()[7] = __builtin_amdgcn_s_memrealtime();
    }
    __syncthreads();
#undef TS
}

// this workgroup holds its launch tag: count it in reader counter blockIdx % NSUB (a wave
// other than wave 0, which routes; no return value)
__device__ __forceinline__ void gen_read_done(uint32_t *ws) {
    if (threadIdx.x == 192)
        __hip_atomic_fetch_add(ws + W_READ + 32 * (blockIdx.x % NSUB), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// router item r of NR: wait until the reader counters q = r, r + NR, ... hold every workgroup of
// the grid that counts there, clear them, and count them drained; the last drained counter
// advances the launch generation (every workgroup of the launch has read it by then). Bounded:
// on expiry the error flag is set and the generation is advanced all the same (a tag must never
// be reused).
__device__ __forceinline__ void gen_manage(uint32_t *ws, int r, int NR, uint32_t tag) {
    const int q = threadIdx.x;
    const int G = gridDim.x;
    if (q >= NSUB || q >= G || q % NR != r) return;
    const uint32_t nq = (uint32_t)((G - q + NSUB - 1) / NSUB);
    int nap = 1;
    for (int it = 0; it < WAIT_SPINS; ++it) {
        if (ld_co32(ws + W_READ + 32 * q) >= nq) break;
        backoff(nap);
        if (it == WAIT_SPINS - 1) flag_error(ws + W_ERR);
    }
    st_co32(ws + W_READ + 32 * q, 0u);
    const uint32_t used = (uint32_t)min(G, NSUB);
    if (add_co32(ws + W_TOP, 1u) == used - 1u) {
        const uint32_t gen = tag - 1u, next = gen + 1u == 0xFFFFFFFFu ? 0u : gen + 1u;
        st_co32(ws + W_TOP, 0u);
        for (int c = 0; c < NGEN; ++c) st_co32(ws + W_GEN + 256 * c, next);
    }
}

// ---------------------------------------------------------------------------------------
// routing of a single-precision launch as published by the gathering workgroup (route_local
// with publish): wave blockIdx % 4 polls the ks record words, the other waves prefetch the
// record table into LDS, and each table row's weight and record address land in s_rw / s_rb.
// On expiry a row counts as not routed (weight 0) and the error flag is set.
// ---------------------------------------------------------------------------------------
template <int XDT>
__device__ __forceinline__ void route_fetch(const LayerArgs &a, uint32_t tag, DlShared &sh, uint32_t *err,
                                            uint64_t *ist) {
    const int tid = threadIdx.x, rwave = (tid >> 6) - (int)(blockIdx.x & 3u), lane = tid & 63;
    const int E = a.E, ks = a.ks;
    const bool pre = E <= RT_LDS;
    if (rwave != 0) {
        if (pre) {
            const int o = (tid + 256 - 64 * (int)(blockIdx.x & 3u)) & 255;  // 64 .. 255 in the other waves
            for (int i = o - 64; i < E; i += 192) sh.rt[i] = a.rtab[i];
        }
    } else {
        const uint64_t *rec = ws_ptr<uint64_t>(a, a.off_rec) + (size_t)(blockIdx.x % NRC) * REC_STRIDE;
        bool need = lane < ks;
        uint32_t pay = 0;
        int nap = 1;
        for (int it = 0; it < WAIT_SPINS; ++it) {
            if (need) {
                const uint64_t v = ld_tag(rec + lane);
                if (tag_ok(v, tag)) {
                    pay = (uint32_t)v;
                    need = false;
                }
            }
            if (__ballot(need) == 0ull) break;
            backoff(nap, 8);  // the record is microseconds away: poll gently
            if (it == WAIT_SPINS - 1 && lane == 0) flag_error(err);
        }
        if (lane < ks) sh.idx[lane] = (int)(need ? 0u : pay);
        if (lane == 0 && __ballot(need) != 0ull) sh.poison = 1;  // the output will be NaN
        if (ist != nullptr && lane == 0) stamp_buf()[6] = __builtin_amdgcn_s_memrealtime();
    }
    __syncthreads();
    if (rwave == 0) {
        if (lane < ks) {
            const uint32_t pay = (uint32_t)sh.idx[lane];
            const int e = (int)((pay >> 16) & 0xFFFu);
            const bool valid = (pay >> 31) != 0u && (e == REC_SHARED || e < E);
            const float w = XDT == MOEHIP_DT_F16 ? f16_to_f32(pay & 0xFFFFu) : bf16_to_f32(pay & 0xFFFFu);
            const int64_t base = !valid ? 0 : (e == REC_SHARED ? a.srec[0] : (pre ? sh.rt[e] : a.rtab[e]));
            sh.rw[lane] = base != 0 ? w : 0.f;
            sh.rb[lane] = (uint64_t)base;
        }
        if (lane == 0) sh.routed = 1;
        if (ist != nullptr && lane == 0) stamp_buf()[7] = __builtin_amdgcn_s_memrealtime();
    }
    __syncthreads();
    gen_read_done(a.ws);  // after the routing exchange, whose words it would otherwise queue with
}

// ---------------------------------------------------------------------------------------
// router item: 4 expert rows (one per wave), each lane 32 consecutive values (H <= 2048)
// ---------------------------------------------------------------------------------------
template <int XDT>
__device__ __forceinline__ void router_rows(const LayerArgs &a, int t, uint32_t tag, uint64_t *st, DlShared &sh) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    // rows: the E router rows (with Wr), then the shared-expert gate as row E (with sgate)
    const int r = t * 4 + wave;
    const int nrows = (a.Wr != nullptr ? a.E : 0) + (a.sgate != nullptr ? 1 : 0);
    const int e = a.Wr != nullptr ? r : a.E;  // logit index of this wave's row
    constexpr int ESZ = XDT == MOEHIP_DT_F32 ? 4 : 2;
    constexpr int NV = 32 * ESZ / 16;  // 16-byte vectors per lane
    const int c0 = lane * 32;
    float acc = 0.f;
    if (r < nrows && c0 < a.H) {
        const uint8_t *wp = e < a.E ? reinterpret_cast<const uint8_t *>(a.Wr) + ((size_t)e * a.H + c0) * ESZ
                                    : reinterpret_cast<const uint8_t *>(a.sgate) + (size_t)c0 * ESZ;
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
    if (lane == 0) sh.wk[wave] = rnd_act<XDT>(acc);
    stamp(st, 0);
    __syncthreads();
    // the item's (up to) 4 logits leave in ONE coalesced store (lanes 0..3 of wave 0): fewer
    // partial-line writes to the lines every poller reads. The shared gate (row E) is the last
    // router row, so its item holds no routed row after it.
    const int rr = t * 4 + lane;
    if (wave == 0 && lane < 4 && rr < nrows) {
        const int ee = a.Wr != nullptr ? rr : a.E;
        uint64_t *lg = ws_ptr<uint64_t>(a, a.off_logits);
        for (int c = 0; c < NLC; ++c)
            st_tag(lg + (size_t)c * logit_stride_words(a.E) + ee, __float_as_uint(sh.wk[lane]), tag);
    }
    stamp(st, 1);
}

// ---------------------------------------------------------------------------------------
// up / down items of one precision
// ---------------------------------------------------------------------------------------
struct Route {
    float w;
    uint64_t base;
};

// routing of table row jj (this launch's routing is in LDS): weight 0 = nothing to run
template <int XDT>
__device__ __forceinline__ Route wg_route(const LayerArgs &a, uint32_t tag, int jj, DlShared &sh, uint32_t *err) {
    (void)tag;
    (void)err;
    Route r;
    r.w = sh.rw[jj];
    r.base = sh.rb[jj];
    if (r.base == 0) r.w = 0.f;
    return r;
}

// LAZY: this workgroup fetches the published routing here, after requesting x (one-item kernel)
template <int PREC, int XDT, bool LAZY>
__device__ __forceinline__ void up_item(const LayerArgs &a, uint32_t tag, int pi, int jj, int b, DlShared &sh,
                                        uint32_t *err, int item) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lg = pick4(a.lg_up, pi);
    const int G = 1 << lg, RPW = 64 >> lg;
    const int C = a.H / DlFmt<PREC>::VPC;
    LaneVec<PREC, XDT> lv;
    uint64_t *st = a.stage != nullptr ? a.stage + 8 * (size_t)item : nullptr;
    load_x<PREC, XDT>(a.x, lane & (G - 1), G, C, lv);  // before the routing wait
    stamp(st, 0);
    if (LAZY) route_fetch<XDT>(a, tag, sh, err, st);
    const Route rt = wg_route<XDT>(a, tag, jj, sh, err);
    stamp(st, 1);
    if (rt.w == 0.f) return;
    const int per_wave = DlFmt<PREC>::NPU * RPW;
    const int pair0 = b * per_wave * 4 + wave * per_wave;
    gbyte *qb = gbytes(rt.base + pick_off(a.offs, pi, 0));
    gbyte *sb = gbytes(rt.base + pick_off(a.offs, pi, 1));
    uint64_t *hout = ws_ptr<uint64_t>(a, a.off_h) + (size_t)jj * a.I;
    up_rows<PREC, XDT>(qb, sb, lv, pair0, a.I, a.H, pick4(a.gs_up, pi), lg, hout, tag, st);
}

// h row jj of this launch -> LDS (piece-major for chunks of VPC values); false on expiry.
// Every thread requests all its words at once, then only the missing ones again.
template <int VPC>
__device__ __forceinline__ bool stage_h(const uint64_t *h, int I, uint32_t tag, float *s_h, uint32_t *err) {
    const int tid = threadIdx.x;
    const int C = I / VPC;
    constexpr int PER = DL_MAXROW / 256;  // words per thread (I <= 2048)
    uint32_t need = 0;
#pragma unroll
    for (int m = 0; m < PER; ++m)
        if (tid + 256 * m < I) need |= 1u << m;
    int nap = 1;
    for (int it = 0; it < WAIT_SPINS; ++it) {
        uint64_t v[PER];
#pragma unroll
        for (int m = 0; m < PER; ++m)
            if (need & (1u << m)) v[m] = ld_tag(h + tid + 256 * m);
#pragma unroll
        for (int m = 0; m < PER; ++m) {
            if ((need & (1u << m)) && tag_ok(v[m], tag)) {
                const int i = tid + 256 * m;
                const int c = i / VPC, q = i % VPC;
                s_h[((q >> 2) * C + c) * 4 + (q & 3)] = __uint_as_float((uint32_t)v[m]);
                need &= ~(1u << m);
            }
        }
        if (!__syncthreads_or(need != 0)) return true;
        backoff(nap, 2);
    }
    if (tid == 0) flag_error(err);
    return false;
}

template <int PREC, int XDT, bool LAZY>
__device__ __forceinline__ void down_item(const LayerArgs &a, uint32_t tag, int pi, int jj, int b, DlShared &sh,
                                          uint32_t *err, int item) {
    uint64_t *st = a.stage != nullptr ? a.stage + 8 * (size_t)item : nullptr;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lg = pick4(a.lg_dn, pi);
    const int G = 1 << lg, RPW = 64 >> lg;
    const int per_wave = DlFmt<PREC>::NPD * RPW;
    const int row0 = b * per_wave * 4 + wave * per_wave;
    const int PK = a.P * a.ks;
    if (LAZY) {
        route_fetch<XDT>(a, tag, sh, err, st);
        // the gate/up weights first: requested together with these, they would share the HBM
        // with weights that cannot be used before h exists anyway
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        const uint32_t defer = (uint32_t)uni((int)a.defer);
        while (__builtin_amdgcn_s_memrealtime() - t0 < defer) __builtin_amdgcn_s_sleep(10);
    }
    const Route rt0 = wg_route<XDT>(a, tag, jj, sh, err);
    stamp(st, 1);
    const bool run = rt0.w != 0.f;
    uint64_t *part = ws_ptr<uint64_t>(a, a.off_part);
    if (run) {
        DownRegs<PREC> d;
        down_load<PREC>(gbytes(rt0.base + pick_off(a.offs, pi, 2)), gbytes(rt0.base + pick_off(a.offs, pi, 3)), row0,
                        a.H, a.I,
                        pick4(a.gs_dn, pi), lg, d);
        // h is polled only once this wave's weights are in registers: polling earlier would
        // compete with the weight stream and cannot let the rows start any sooner
        __builtin_amdgcn_s_waitcnt(0);
        stamp(st, 2);
        if (stage_h<DlFmt<PREC>::VPC>(ws_ptr<uint64_t>(a, a.off_h) + (size_t)jj * a.I, a.I, tag, sh.h, err)) {
            stamp(st, 3);
            LaneVec<PREC, XDT> lv;
            load_h<PREC, XDT>(sh.h, lane & (G - 1), G, a.I / DlFmt<PREC>::VPC, lv);
            down_rows<PREC, XDT>(d, lv, row0, a.H, lg, rt0.w, part + (size_t)jj * a.H, tag);
            stamp(st, 4);
        } else {  // h never arrived: this row's partials are NaN, so the output cannot look valid
            const int rows = per_wave * 4;
            for (int i = tid; i < rows; i += 256)
                if (b * rows + i < a.H) st_tag(part + (size_t)jj * a.H + b * rows + i, 0x7fc00000u, tag);
        }
        __syncthreads();  // sh.h is reused below and by the next item
    }
    if (jj != PK - 1) return;
    // the last table row's items sum every row's partials in table order. Table rows are taken
    // in chunks that fit the LDS buffer; every thread requests its (table row, row) words of a
    // chunk at once, then only the missing ones again.
    const int rows = per_wave * 4;
    const int r0 = b * rows;
    float *s_part = sh.h;  // (chunk, rows)
    constexpr int PER = DL_MAXROW / 256;
    float acc[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) acc[u] = 0.f;
    const int QC = max(1, DL_MAXROW / rows);
    for (int q0 = 0; q0 < PK; q0 += QC) {
        const int nq = min(QC, PK - q0), nw = nq * rows;
        uint32_t need = 0;
#pragma unroll
        for (int m = 0; m < PER; ++m) {
            const int i = tid + 256 * m;
            if (i >= nw) continue;
            const int q = q0 + i / rows, rr = i % rows;
            if (sh.rw[q] != 0.f && sh.rb[q] != 0 && r0 + rr < a.H) need |= 1u << m;
            else s_part[i] = 0.f;
        }
        int nap = 1;
        for (int it = 0; it < WAIT_SPINS; ++it) {
            uint64_t v[PER];
#pragma unroll
            for (int m = 0; m < PER; ++m) {
                const int i = tid + 256 * m;
                if (need & (1u << m)) v[m] = ld_tag(part + (size_t)(q0 + i / rows) * a.H + r0 + i % rows);
            }
#pragma unroll
            for (int m = 0; m < PER; ++m) {
                if ((need & (1u << m)) && tag_ok(v[m], tag)) {
                    s_part[tid + 256 * m] = __uint_as_float((uint32_t)v[m]);
                    need &= ~(1u << m);
                }
            }
            if (!__syncthreads_or(need != 0)) break;
            backoff(nap, 2);
            if (it == WAIT_SPINS - 1) {  // give up: the missing partials make the output NaN
                flag_error(err);
#pragma unroll
                for (int m = 0; m < PER; ++m)
                    if (need & (1u << m)) s_part[tid + 256 * m] = __uint_as_float(0x7fc00000u);
                __syncthreads();
            }
        }
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int rr = tid + 256 * u;
            if (rr < rows)
                for (int qq = 0; qq < nq; ++qq) acc[u] += s_part[qq * rows + rr];
        }
        __syncthreads();  // s_part is rewritten by the next chunk
    }
    if (sh.poison) {  // this workgroup's routing wait expired: no plausible output
#pragma unroll
        for (int u = 0; u < PER; ++u) acc[u] = __uint_as_float(0x7fc00000u);
    }
    // the optional terms: each one's loads issued together under a uniform branch (clamped rows
    // of this workgroup's own range), so they cost one round trip, not one per row
    if (a.accumulate) {
        float v[PER];
#pragma unroll
        for (int u = 0; u < PER; ++u) v[u] = ld_act<XDT>(a.out, min(r0 + min(tid + 256 * u, rows - 1), a.H - 1));
#pragma unroll
        for (int u = 0; u < PER; ++u) acc[u] += v[u];
    }
    if (a.add != nullptr) {
        float v[PER];
#pragma unroll
        for (int u = 0; u < PER; ++u) v[u] = ld_act<XDT>(a.add, min(r0 + min(tid + 256 * u, rows - 1), a.H - 1));
#pragma unroll
        for (int u = 0; u < PER; ++u) acc[u] += v[u];
    }
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        const int rr = tid + 256 * u, r = r0 + rr;
        if (rr >= rows || r >= a.H) continue;
        st_act<XDT>(a.out, r, acc[u]);
    }
    stamp(st, 5);
    __syncthreads();  // sh.h is reused by the next item
}

// work items of the router stage: 4 rows each (E router rows, + the shared gate row); at least
// one, which also runs the route tail
__host__ __device__ __forceinline__ int router_items(bool with_router, bool shared, int E) {
    const int rows = (with_router ? E : 0) + (shared ? 1 : 0);
    return rows > 0 ? (rows + 3) / 4 : 1;
}

// rows per down item / row pairs per up item of a precision (host and device)
__host__ __device__ __forceinline__ int down_item_rows(int prec, int lg) {
    const int npd = prec == MOEHIP_PREC_INT4 ? 8 : ((prec == MOEHIP_PREC_F16 || prec == MOEHIP_PREC_BF16) ? 2 : 4);
    return npd * (64 >> lg) * 4;
}

// ---------------------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------------------
// PR = the record precision of a single-precision launch (its code only), or -1 for any mix
template <int XDT, int PR>
__global__ __launch_bounds__(256) void k_decode_layer(LayerArgs a) {
    __shared__ DlShared sh;
    const int tid = threadIdx.x;
    uint32_t *ws = a.ws;
    uint32_t *err = ws + W_ERR;
    const int NR = router_items(a.Wr != nullptr, a.sgate != nullptr, a.E);
    const int total = NR + a.NU + a.ND;
    if (tid == 0) {
        sh.tag = ld_co32(ws + W_GEN + 256 * (blockIdx.x % NGEN)) + 1u;  // launch tag (never 0)
        sh.routed = 0;
        sh.poison = 0;
        sh.forced = ld_co32(ws + W_TEST) != 0u ? 1 : 0;
    }
    __syncthreads();
    const uint32_t tag = uni((int)sh.tag);
    gen_read_done(ws);
    for (int t = blockIdx.x; t < total; t += gridDim.x) {
        __syncthreads();  // LDS of the previous item is free
        uint64_t t_start = 0;
        if (a.trace != nullptr) {
            stamp_clear();
            __syncthreads();
            if (tid == 0) t_start = __builtin_amdgcn_s_memrealtime();
        }
        if (t < NR) {
            // ---------------- router rows; the last router item also reports the routing ----------------
            if (a.Wr != nullptr || a.sgate != nullptr) router_rows<XDT>(a, t, tag, a.stage != nullptr ? a.stage + 8 * (size_t)t : nullptr, sh);
            if (t == NR - 1) route_local<XDT>(a, tag, sh, err, true, a.trace ? a.stage + 8 * (size_t)total : nullptr);
            gen_manage(ws, t, NR, tag);
        } else if (t < NR + a.NU) {
            if (!sh.routed) route_local<XDT>(a, tag, sh, err, false, nullptr);
            // ---------------- kernel-A rows ----------------
            const int u = t - NR;
            const int pi = block_of(a.up_base, a.P, u);
            const int rem = u - pick4(a.up_base, pi);
            const int nub = pick4(a.nub, pi);
            const int jj = pi * a.ks + rem / nub, b = rem % nub;
            if constexpr (PR >= 0) {
                up_item<PR, XDT, false>(a, tag, pi, jj, b, sh, err, t);
            } else {
                switch (pick4(a.prec, pi)) {
                    case MOEHIP_PREC_INT4: up_item<MOEHIP_PREC_INT4, XDT, false>(a, tag, pi, jj, b, sh, err, t); break;
                    case MOEHIP_PREC_INT8: up_item<MOEHIP_PREC_INT8, XDT, false>(a, tag, pi, jj, b, sh, err, t); break;
                    case MOEHIP_PREC_F16: up_item<MOEHIP_PREC_F16, XDT, false>(a, tag, pi, jj, b, sh, err, t); break;
                    case MOEHIP_PREC_BF16: up_item<MOEHIP_PREC_BF16, XDT, false>(a, tag, pi, jj, b, sh, err, t); break;
                    default: up_item<MOEHIP_PREC_FP8, XDT, false>(a, tag, pi, jj, b, sh, err, t); break;
                }
            }
        } else {
            if (!sh.routed) route_local<XDT>(a, tag, sh, err, false, nullptr);
            // ---------------- kernel-B rows (+ ordered combine) ----------------
            const int dd = t - NR - a.NU;
            const int pi = block_of(a.dn_base, a.P, dd);
            const int rem = dd - pick4(a.dn_base, pi);
            const int ndb = pick4(a.ndb, pi);
            const int jj = pi * a.ks + rem / ndb, b = rem % ndb;
            if constexpr (PR >= 0) {
                down_item<PR, XDT, false>(a, tag, pi, jj, b, sh, err, t);
            } else {
                switch (pick4(a.prec, pi)) {
                    case MOEHIP_PREC_INT4: down_item<MOEHIP_PREC_INT4, XDT, false>(a, tag, pi, jj, b, sh, err, t); break;
                    case MOEHIP_PREC_INT8: down_item<MOEHIP_PREC_INT8, XDT, false>(a, tag, pi, jj, b, sh, err, t); break;
                    case MOEHIP_PREC_F16: down_item<MOEHIP_PREC_F16, XDT, false>(a, tag, pi, jj, b, sh, err, t); break;
                    case MOEHIP_PREC_BF16: down_item<MOEHIP_PREC_BF16, XDT, false>(a, tag, pi, jj, b, sh, err, t); break;
                    default: down_item<MOEHIP_PREC_FP8, XDT, false>(a, tag, pi, jj, b, sh, err, t); break;
                }
            }
        }
        if (a.trace != nullptr) {
            __syncthreads();
            stamp_flush(a.stage + 8 * (size_t)t, t == NR - 1 ? a.stage + 8 * (size_t)total : nullptr);
            if (tid == 0) {
                a.trace[3 * t + 0] = t_start;
                a.trace[3 * t + 1] = __builtin_amdgcn_s_memrealtime();
                a.trace[3 * t + 2] = blockIdx.x;
            }
        }
    }
}

// ---------------------------------------------------------------------------------------
// one-item kernel: a single-precision launch whose items all fit on the GPU at once runs one
// item per workgroup (grid = items), with the code of its precision only and no item loop (the
// compiler then keeps no loop state live across the items' code: fewer registers, more
// workgroups per CU). Same items, routing, exchanges and generation handling as above.
// ---------------------------------------------------------------------------------------
// the kernel's argument block, re-derived from the kernarg segment pointer behind an empty asm
// so that the compiler loads each argument where a phase uses it instead of at kernel entry
// (arguments loaded at entry stay live in SGPRs through the whole kernel)
typedef const __attribute__((address_space(4))) LayerArgs KLayerArgs;
__device__ __forceinline__ const LayerArgs &kargs() {
    KLayerArgs *p = (KLayerArgs *)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(p));
    return *(const LayerArgs *)p;
}

template <int XDT, int PR>
__global__ __launch_bounds__(256) void k_decode_tok(LayerArgs) {
    __shared__ DlShared sh;
    const int tid = threadIdx.x;
    int NR, NU, total;
    {
        const LayerArgs &a = kargs();
        NR = uni(router_items(a.Wr != nullptr, a.sgate != nullptr, a.E));
        NU = uni(a.NU);
        total = NR + NU + uni(a.ND);
        if (tid == 0) {
            sh.tag = ld_co32(a.ws + W_GEN + 256 * (blockIdx.x % NGEN)) + 1u;  // launch tag (never 0)
            sh.routed = 0;
            sh.poison = 0;
            sh.forced = ld_co32(a.ws + W_TEST) != 0u ? 1 : 0;
        }
    }
    __syncthreads();
    const uint32_t tag = uni((int)sh.tag);
    const int t = blockIdx.x;
    uint64_t t_start = 0;
    if (kargs().trace != nullptr) {
        stamp_clear();
        __syncthreads();
    }
    if (t < NR) {
        const LayerArgs &a = kargs();
        if (a.trace != nullptr && tid == 0) t_start = __builtin_amdgcn_s_memrealtime();
        if (a.Wr != nullptr || a.sgate != nullptr) router_rows<XDT>(a, t, tag, a.stage != nullptr ? a.stage + 8 * (size_t)t : nullptr, sh);
        if (t == NR - 1)
            route_local<XDT>(a, tag, sh, a.ws + W_ERR, true, a.trace ? a.stage + 8 * (size_t)total : nullptr, nullptr, true);
        gen_read_done(a.ws);
        gen_manage(a.ws, t, NR, tag);
    } else if (t < NR + NU) {
        const LayerArgs &a = kargs();
        if (a.trace != nullptr && tid == 0) t_start = __builtin_amdgcn_s_memrealtime();
        const int u = t - NR;
        const int nub = uni(a.nub[0]);
        up_item<PR, XDT, true>(a, tag, 0, u / nub, u % nub, sh, a.ws + W_ERR, t);
    } else {
        const LayerArgs &a = kargs();
        if (a.trace != nullptr && tid == 0) t_start = __builtin_amdgcn_s_memrealtime();
        const int dd = t - NR - NU;
        const int ndb = uni(a.ndb[0]);
        down_item<PR, XDT, true>(a, tag, 0, dd / ndb, dd % ndb, sh, a.ws + W_ERR, t);
    }
    const LayerArgs &a = kargs();
    if (a.trace != nullptr) {
        __syncthreads();
        stamp_flush(a.stage + 8 * (size_t)t, t == NR - 1 ? a.stage + 8 * (size_t)total : nullptr);
        if (tid == 0) {
            a.trace[3 * t + 0] = t_start;
            a.trace[3 * t + 1] = __builtin_amdgcn_s_memrealtime();
            a.trace[3 * t + 2] = blockIdx.x;
        }
    }
}

// ---------------------------------------------------------------------------------------
// host side: item plans and workspace layout
// ---------------------------------------------------------------------------------------
static inline int cpl_host(int prec) { return 32 / vpc_of(prec); }
// log2 of the lanes per row of `cols` values (CPL chunks of VPC values per lane)
static inline int lg_for(int cols, int prec) {
    const int lanes = (cols / vpc_of(prec) + cpl_host(prec) - 1) / cpl_host(prec);
    int G = 1, lg = 0;
    while (G < lanes && G < 64) G <<= 1, ++lg;
    return lg;
}
static inline int up_item_pairs(int prec, int lg) { return (4 / cpl_host(prec)) * (64 >> lg) * 4; }

struct DlLayout {
    uint32_t rec, logits, h, part, total;
};

static inline uint32_t al256(size_t v) { return (uint32_t)((v + 255) / 256 * 256); }

static DlLayout dl_layout(int P, int k, int E, int H, int I) {
    DlLayout L;
    const int PK = P * k;
    size_t off = W_HDR * 4;
    off = al256(off);
    L.rec = (uint32_t)off;  // the routing record: one tagged word per table row, NRC copies
    off += ((size_t)(NRC - 1) * REC_STRIDE + PK) * 8;
    off = al256(off) + 4096;  // the logits on other pages than the record copies
    L.logits = (uint32_t)off;
    off += (size_t)NLC * logit_stride_words(E) * 8;  // E routed + the shared-expert gate, NLC copies
    off = al256(off);
    L.h = (uint32_t)off;
    off += (size_t)PK * I * 8;
    off = al256(off);
    L.part = (uint32_t)off;
    off += (size_t)PK * H * 8;
    L.total = al256(off);
    return L;
}

// item plan of a layer: fills the plan fields of `a`, returns the number of work items
static int dl_plan(const moehip_layer_desc *d, int with_router, LayerArgs *a) {
    int nu = 0, nd = 0;
    const int ks = d->k + (d->shared_gate != nullptr ? 1 : 0);
    for (int p = 0; p < DL_MAXP; ++p) {
        const bool on = p < d->P;
        a->lg_up[p] = on ? lg_for(d->H, d->prec[p]) : 0;
        a->lg_dn[p] = on ? lg_for(d->I, d->prec[p]) : 0;
        a->nub[p] = a->ndb[p] = 1;
        a->up_base[p] = nu;
        a->dn_base[p] = nd;
        if (on) {
            const int upi = up_item_pairs(d->prec[p], a->lg_up[p]);
            const int dpi = down_item_rows(d->prec[p], a->lg_dn[p]);
            a->nub[p] = (d->I + upi - 1) / upi;
            a->ndb[p] = (d->H + dpi - 1) / dpi;
            nu += ks * a->nub[p];
            nd += ks * a->ndb[p];
        }
    }
    a->NU = nu;
    a->ND = nd;
    return router_items(with_router != 0, d->shared_gate != nullptr, d->E) + nu + nd;
}

// the kernel instances of a launch: the one-item kernel of its precision (single-precision
// launches with 16-bit activations), and the item-loop kernel (any mix, fp32 activations, or
// more items than the GPU holds at once)
typedef void (*DlKernel)(LayerArgs);
template <int XDT>
static DlKernel dl_tok_x(int prec0) {
    switch (prec0) {
        case MOEHIP_PREC_INT4: return k_decode_tok<XDT, MOEHIP_PREC_INT4>;
        case MOEHIP_PREC_INT8: return k_decode_tok<XDT, MOEHIP_PREC_INT8>;
        case MOEHIP_PREC_F16: return k_decode_tok<XDT, MOEHIP_PREC_F16>;
        case MOEHIP_PREC_BF16: return k_decode_tok<XDT, MOEHIP_PREC_BF16>;
        case MOEHIP_PREC_FP8: return k_decode_tok<XDT, MOEHIP_PREC_FP8>;
        default: return nullptr;
    }
}
static DlKernel dl_kernel(int dtype, bool tok, int prec0) {
    switch (dtype) {
        case MOEHIP_DT_F16: return tok ? dl_tok_x<MOEHIP_DT_F16>(prec0) : k_decode_layer<MOEHIP_DT_F16, -1>;
        case MOEHIP_DT_BF16: return tok ? dl_tok_x<MOEHIP_DT_BF16>(prec0) : k_decode_layer<MOEHIP_DT_BF16, -1>;
        default: return k_decode_layer<MOEHIP_DT_F32, -1>;  // (the routing record holds 16-bit weights)
    }
}

// workgroups of a kernel instance the current device holds at once (occupancy x CUs)
static int dl_capacity(DlKernel kern, int *cap) {
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess) return -1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return -1;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(kern), 256, 0) !=
        hipSuccess)
        return -1;
    *cap = per_cu * cus;
    return 0;
}

}  // namespace moehip

using namespace moehip;

extern "C" size_t moehip_decode_layer_workspace_bytes(int P, int k, int E, int H, int I) {
    if (P <= 0 || k <= 0 || E <= 0 || H <= 0 || I <= 0) return 0;
    size_t n = dl_layout(P, k, E, H, I).total;
    if (P == 1)  // room for the XCD-local kernel too (any record kind; k counts the shared row)
        for (int pr : {MOEHIP_PREC_INT4, MOEHIP_PREC_INT8, MOEHIP_PREC_F16, MOEHIP_PREC_FP8}) {
            const size_t m = xcd_workspace_bytes(pr, k, E, H, I);
            n = m > n ? m : n;
        }
    return n;
}

// the decode kernel the calling thread's last moehip_decode_layer / moehip_decode_rows call
// launched (MOEHIP_KERNEL_*; 0 before any)
static thread_local int t_last_kernel = 0;

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
        if (pr == MOEHIP_PREC_INT4 || pr == MOEHIP_PREC_INT8) {
            const int vpc = vpc_of(pr);
            MOEHIP_REQUIRE(d->gs_up[p] > 0 && d->gs_up[p] % vpc == 0 && d->H % d->gs_up[p] == 0 && d->gs_dn[p] > 0 &&
                               d->gs_dn[p] % vpc == 0 && d->I % d->gs_dn[p] == 0,
                           "decode_layer: group sizes %d/%d need multiples of %d dividing H/I", d->gs_up[p],
                           d->gs_dn[p], vpc);
        }
    }
    const int ks = d->k + (d->shared_gate != nullptr ? 1 : 0);
    const DlLayout L = dl_layout(d->P, ks, d->E, d->H, d->I);
    MOEHIP_REQUIRE(ws_bytes >= L.total, "decode_layer: workspace %zu bytes < %u", ws_bytes, L.total);
    MOEHIP_REQUIRE(((uintptr_t)ws % 256) == 0, "decode_layer: workspace must be 256-byte aligned");
    MOEHIP_REQUIRE(((uintptr_t)x % 16) == 0 && ((uintptr_t)Wr % 16) == 0 && ((uintptr_t)d->shared_gate % 16) == 0,
                   "decode_layer: x, Wr and the shared gate must be 16-byte aligned");
    MOEHIP_REQUIRE(d->P * ks <= DL_MAXP * 32, "decode_layer: %d precisions x %d rows exceed %d table rows", d->P, ks,
                   DL_MAXP * 32);
    if ((trace == nullptr && grid == 0) || grid < 0) {
        // the XCD-local kernel when the layer and the device fit it (grid > 0, or a trace with
        // grid 0, asks for the item kernels; grid < 0 for the XCD kernel with its own trace format)
        int used = 0;
        const int rc = xcd_launch(d, x, Wr, idx_in, w32_in, nullptr, nullptr, rtab, out, add, accumulate, logits_out,
                                  idx_out, w_out, w32_out, info, miss, ws, ws_bytes, grid < 0 ? trace : nullptr,
                                  stream, &used);
        if (rc != MOEHIP_OK) return rc;
        if (used) {
            t_last_kernel = used;
            return rc;
        }
    }
    if (grid < 0) grid = 0;
    LayerArgs a{};
    a.x = x;
    a.Wr = Wr;
    a.idx_in = idx_in;
    a.w32_in = w32_in;
    a.rtab = rtab;
    for (int p = 0; p < DL_MAXP; ++p) {
        const bool on = p < d->P;
        for (int f = 0; f < 4; ++f) a.offs[p][f] = on ? d->offs[p][f] : 0;
        a.prec[p] = on ? d->prec[p] : 0;
        a.gs_up[p] = on ? d->gs_up[p] : 0;
        a.gs_dn[p] = on ? d->gs_dn[p] : 0;
        a.planned[p] = on ? d->planned[p] : 0;
    }
    const int total = dl_plan(d, Wr != nullptr, &a);
    {
        // the time the HBM needs for the k routed gate/up blocks (q + scales) at 8 TB/s, in 10 ns
        // ticks: single-precision launches only (one record kind)
        const double gu = (double)(d->offs[0][2] - d->offs[0][0]);
        a.defer = d->P == 1 ? (uint32_t)(d->k * gu / 8.0e12 * 1.0e8) : 0u;
    }
    for (int i = 0; i < 3; ++i) a.lv2p[i] = d->lv2p[i];
    a.P = d->P;
    a.E = d->E;
    a.k = d->k;
    a.ks = ks;
    a.sgate = d->shared_gate;
    for (int p = 0; p < DL_MAXP; ++p) a.srec[p] = p < d->P ? d->shared_rec[p] : 0;
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
    a.off_rec = L.rec;
    a.off_logits = L.logits;
    a.off_h = L.h;
    a.off_part = L.part;
    a.trace = trace;
    a.stage = trace != nullptr ? trace + 3 * (size_t)(total + 3) : nullptr;
    // the one-item kernel when the launch has one precision, no grid was requested and all its
    // items fit on the GPU at once; otherwise the item loop over at most that many workgroups
    DlKernel kern = nullptr;
    int cap = 0;
    // (external routing runs the item-loop kernel: every workgroup reads the fp32 weights itself,
    // where the one-item kernel's routing record carries them in 16 bits)
    if (d->P == 1 && Wr != nullptr && (grid <= 0 || grid >= total)) {
        kern = dl_kernel(d->dtype, true, d->prec[0]);
        if (kern == nullptr || dl_capacity(kern, &cap) != 0 || cap < total) kern = nullptr;
    }
    int g = total;
    if (kern == nullptr) {
        kern = dl_kernel(d->dtype, false, 0);
        if (dl_capacity(kern, &cap) != 0 || cap <= 0) {
            set_error("decode_layer: occupancy query failed");
            return MOEHIP_ELAUNCH;
        }
        g = grid > 0 ? (grid < total ? grid : total) : total;
        if (g > cap) g = cap;  // every workgroup must fit on the GPU at once (see the kernel's header)
        t_last_kernel = MOEHIP_KERNEL_ITEM_LOOP;
    } else {
        t_last_kernel = MOEHIP_KERNEL_ONE_ITEM;
    }
    hipLaunchKernelGGL(kern, dim3(g), dim3(256), 0, as_stream(stream), a);
    return check_launch("decode_layer");
}

extern "C" int moehip_decode_last_kernel(void) { return t_last_kernel; }

extern "C" const char *moehip_decode_kernel_name(int kernel) {
    switch (kernel) {
        case MOEHIP_KERNEL_XCD: return "k_decode_xcd";
        case MOEHIP_KERNEL_XCD_TWO: return "k_decode_xcd (two passes)";
        case MOEHIP_KERNEL_ONE_ITEM: return "k_decode_tok";
        case MOEHIP_KERNEL_ITEM_LOOP: return "k_decode_layer";
        default: return "none";
    }
}

extern "C" int moehip_decode_rows(const moehip_layer_desc *d, const void *x, const int64_t *rows_b, const float *rows_w,
                                  void *out, const void *add, int accumulate, void *ws, size_t ws_bytes, void *stream) {
    MOEHIP_REQUIRE(d && x && rows_b && rows_w && out && ws, "decode_rows: null pointer");
    MOEHIP_REQUIRE(d->shared_gate == nullptr, "decode_rows: a shared expert is one of the explicit rows here");
    MOEHIP_REQUIRE(d->P > 0 && d->P <= DL_MAXP, "decode_rows: P=%d (1..%d)", d->P, DL_MAXP);
    MOEHIP_REQUIRE(d->k > 0 && d->k <= 32, "decode_rows: k=%d (1..32 rows per precision)", d->k);
    MOEHIP_REQUIRE(d->H > 0 && d->H <= DL_MAXROW && d->H % 32 == 0 && d->I > 0 && d->I <= DL_MAXROW && d->I % 32 == 0,
                   "decode_rows: H=%d I=%d (multiples of 32, <= %d)", d->H, d->I, DL_MAXROW);
    MOEHIP_REQUIRE(d->dtype >= MOEHIP_DT_F16 && d->dtype <= MOEHIP_DT_F32, "decode_rows: dtype %d", d->dtype);
    for (int p = 0; p < d->P; ++p) {
        const int pr = d->prec[p];
        MOEHIP_REQUIRE(pr >= MOEHIP_PREC_INT4 && pr <= MOEHIP_PREC_FP8 && pr != MOEHIP_PREC_F32,
                       "decode_rows: precision %d (fp32 records use the grouped kernels)", pr);
        if (pr == MOEHIP_PREC_INT4 || pr == MOEHIP_PREC_INT8) {
            const int vpc = vpc_of(pr);
            MOEHIP_REQUIRE(d->gs_up[p] > 0 && d->gs_up[p] % vpc == 0 && d->H % d->gs_up[p] == 0 && d->gs_dn[p] > 0 &&
                               d->gs_dn[p] % vpc == 0 && d->I % d->gs_dn[p] == 0,
                           "decode_rows: group sizes %d/%d need multiples of %d dividing H/I", d->gs_up[p],
                           d->gs_dn[p], vpc);
        }
    }
    const DlLayout L = dl_layout(d->P, d->k, 1, d->H, d->I);
    MOEHIP_REQUIRE(ws_bytes >= L.total, "decode_rows: workspace %zu bytes < %u", ws_bytes, L.total);
    MOEHIP_REQUIRE(((uintptr_t)ws % 256) == 0 && ((uintptr_t)x % 16) == 0,
                   "decode_rows: workspace 256-byte and x 16-byte aligned");
    moehip_layer_desc dd = *d;
    dd.E = 1;
    for (int p = 0; p < DL_MAXP; ++p) dd.planned[p] = p < d->P ? 1 : 0;
    LayerArgs a{};
    a.x = x;
    a.rows_b = rows_b;
    a.rows_w = rows_w;
    for (int p = 0; p < DL_MAXP; ++p) {
        const bool on = p < d->P;
        for (int f = 0; f < 4; ++f) a.offs[p][f] = on ? d->offs[p][f] : 0;
        a.prec[p] = on ? d->prec[p] : 0;
        a.gs_up[p] = on ? d->gs_up[p] : 0;
        a.gs_dn[p] = on ? d->gs_dn[p] : 0;
        a.planned[p] = on ? 1 : 0;
    }
    const int total = dl_plan(&dd, 0, &a);
    a.P = d->P;
    a.E = 1;
    a.k = d->k;
    a.ks = d->k;
    a.H = d->H;
    a.I = d->I;
    a.accumulate = accumulate;
    a.out = out;
    a.add = add;
    a.ws = reinterpret_cast<uint32_t *>(ws);
    a.off_rec = L.rec;
    a.off_logits = L.logits;
    a.off_h = L.h;
    a.off_part = L.part;
    DlKernel kern = dl_kernel(d->dtype, false, 0);
    int cap = 0;
    if (dl_capacity(kern, &cap) != 0 || cap <= 0) {
        set_error("decode_rows: occupancy query failed");
        return MOEHIP_ELAUNCH;
    }
    hipLaunchKernelGGL(kern, dim3(total < cap ? total : cap), dim3(256), 0, as_stream(stream), a);
    t_last_kernel = MOEHIP_KERNEL_ITEM_LOOP;
    return check_launch("decode_rows");
}

extern "C" size_t moehip_decode_rows_workspace_bytes(int P, int k, int H, int I) {
    if (P <= 0 || k <= 0 || H <= 0 || I <= 0) return 0;
    return dl_layout(P, k, 1, H, I).total;
}

extern "C" int moehip_decode_layer_work_items(const moehip_layer_desc *d, int with_router) {
    if (d == nullptr || d->P <= 0 || d->P > DL_MAXP) return -1;
    LayerArgs a;
    return dl_plan(d, with_router, &a);
}

extern "C" int moehip_decode_layer_error(const void *ws, void *flag_out, void *stream) {
    MOEHIP_REQUIRE(flag_out, "decode_layer_error: null flag_out");
    if (ws == nullptr) {  // the current device's scratch array of moehip_decode_layer_noalloc
        int dev = -1;
        MOEHIP_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0, "decode_layer_error: no current device");
        ws = noalloc_scratch(dev);
        MOEHIP_REQUIRE(ws != nullptr, "decode_layer_error: no workspace given and device %d's scratch array is not "
                       "set up (moehip_device_check(%d) sets it up)", dev, dev);
    }
    const hipError_t e = hipMemcpyAsync(flag_out, reinterpret_cast<const uint32_t *>(ws) + W_ERR, 4,
                                        hipMemcpyDeviceToDevice, as_stream(stream));
    if (e != hipSuccess) {
        set_error("decode_layer_error: %s", hipGetErrorString(e));
        return MOEHIP_ELAUNCH;
    }
    return MOEHIP_OK;
}
