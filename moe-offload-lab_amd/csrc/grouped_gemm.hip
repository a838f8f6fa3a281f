// Expert-sorted grouped GEMM for T > 1 tokens (prefill chunks, batched decode) on MFMA.
//
// Replaces the reference's prefill expert path (moelab/runtime.py:418-436 `_run_grouped_tokens`
// and :352-353: per expert y = expert_ffn(x[tok]), out.index_add_(tok, y * w)) for int4 gs64
// records. The (token, slot) pairs are sorted by expert (moehip_dispatch); per expert the tokens
// form the M dimension of two GEMMs:
//   up:   h (n_e, I) = silu(X_e gate^T) * (X_e up^T)     K = H, weight rows 2I (gate; up)
//   down: y (n_e, H) = w_pair * (h down^T)               K = I, weight rows H
// followed by an ordered combine out[t] = sum over the token's slots in slot order.
//
// MFMA: v_mfma_f32_32x32x16_f16: A = 32 tokens x 16 K (lane i + 32 (k / 8), element k % 8),
// B = 16 K x 32 weight rows (same lane rule), D = 32 x 32 fp32 (row i at lane
// j + 32 ((i / 4) % 2), element 4 (i / 8) + i % 4), accumulated over the whole K. In one int4
// scale group (64 K) lane half h of weight row j holds bytes 16 h .. 16 h + 15 (one 16-byte
// load) and dword m of them feeds MFMA m: its 8 nibbles become fp16 1024 + n (exact), then
// n - 8 (exact) and s * (n - 8) (one fp16 rounding, relative error <= 2^-11; the reference's own
// prefill path rounds the dequantised weights to the model dtype, 2^-8 for bf16).
//
// Operand A is fp16 in LDS: fp16 activations as they are, bf16 activations scaled per token by a
// power of two 2^-e (the row's largest |x| in [2^14, 2^15), exact for bf16 values), h (fp32,
// written by the up kernel with a per-pair maximum gathered by atomics) scaled per pair the
// same way; the outputs are scaled back by 2^e.
//
// Each workgroup (4 waves) owns one expert and 256 weight rows (up: 128 gate + 128 up rows =
// 128 h columns; down: 256 output rows); a wave owns 2 subtiles of 32 rows, for up to 64
// tokens per pass (two 32-token M tiles). K advances in chunks (up: 4 groups, down: 2): a wave
// keeps a ring of chunks of its weight rows in registers (16 KB in flight while it computes),
// and the workgroup stages the activation chunk into LDS (double buffered, rows padded by 16
// bytes, permuted into operand order) one chunk ahead. Workgroups of one expert land on one XCD
// (its L2 then serves the expert's activation rows to all of them).

#include "decide.hpp"
#include "lanevec.hpp"

namespace moehip {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef gbyte gu8;  // record bytes, global address space (common.hpp)
__device__ __forceinline__ gu8 *record_ptr(int64_t a) { return gbytes((uint64_t)a); }

constexpr int GG_KG = 64;     // K per scale group
constexpr int GG_TOK = 64;    // tokens per pass (two 32-token M tiles)
constexpr int GG_ROWS = 256;  // weight rows per workgroup

// chunk geometry: CK values of K per chunk; a lane half covers CK / 2 of them, which is 32 bytes
// of its weight row for every record precision (int4: CK 128 = two scale groups, one per half;
// int8 / fp8: 64; fp16 / bf16: 32). Each of the 256 threads stages CK / 4 fp16 activation values
// of one token (NV 16-byte loads).
template <int CKV> struct GgChunk {
    static constexpr int CK = CKV;          // K per chunk
    static constexpr int LDA = CK + 8;      // LDS row stride in halves
    static constexpr int VPT = CK / 4;      // values staged per thread
    static constexpr int NV = VPT / 8;      // 16-byte loads per thread
};
template <int PREC> struct GgPrec;
template <> struct GgPrec<MOEHIP_PREC_INT4> { static constexpr int CK = 128, BITS = 4; };
template <> struct GgPrec<MOEHIP_PREC_INT8> { static constexpr int CK = 64, BITS = 8; };
template <> struct GgPrec<MOEHIP_PREC_FP8> { static constexpr int CK = 64, BITS = 8; };
template <> struct GgPrec<MOEHIP_PREC_F16> { static constexpr int CK = 32, BITS = 16; };
template <> struct GgPrec<MOEHIP_PREC_BF16> { static constexpr int CK = 32, BITS = 16; };

// ---------------------------------------------------------------------------------------
// weights -> fp16 B operands in operand order c0 c4 c1 c5 c2 c6 c3 c7 (the order the activation
// chunks are stored in). int4: dword d of a row (K elements c0..c7 as nibbles) and the group
// scale s (fp16, both halves): (d & mask) | magic = fp16 1024 + n in one v_and_or_b32 (common.hpp
// and_or; its result feeds the compiler's packed fp16 add, never an MFMA operand directly) for the
// nibbles at bits 0-3 of each half; for those at bits 4-7 the magic is fp16 64, whose unit in the
// last place is 1/16, so the same mask-and-or gives 64 + n with no shift; - 1032 or - 72 (exact),
// * s (one rounding). 13 VALU operations per 8 weights.
// ---------------------------------------------------------------------------------------
struct DeqK {
    uint32_t mask, magic;  // 0x000F000F, 0x64006400
};

__device__ __forceinline__ f16x8 wdeq8(uint32_t d, half2_t s2, DeqK k) {
#pragma clang fp contract(off)
    const half2_t off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const half2_t off_hi = {(_Float16)-72.0f, (_Float16)-72.0f};
    const uint32_t t = d >> 8;
    const uint32_t u0 = and_or(d, k.mask, k.magic);           // 1024 + n (c0, c4)
    const uint32_t u1 = and_or(d, 0x00F000F0u, 0x54005400u);  // 64 + n   (c1, c5)
    const uint32_t u2 = and_or(t, k.mask, k.magic);           // 1024 + n (c2, c6)
    const uint32_t u3 = and_or(t, 0x00F000F0u, 0x54005400u);  // 64 + n   (c3, c7)
    const half2_t h0 = (__builtin_bit_cast(half2_t, u0) + off) * s2;
    const half2_t h1 = (__builtin_bit_cast(half2_t, u1) + off_hi) * s2;
    const half2_t h2 = (__builtin_bit_cast(half2_t, u2) + off) * s2;
    const half2_t h3 = (__builtin_bit_cast(half2_t, u3) + off_hi) * s2;
    const uint4 u = make_uint4(__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1),
                               __builtin_bit_cast(uint32_t, h2), __builtin_bit_cast(uint32_t, h3));
    return __builtin_bit_cast(f16x8, u);
}

// int8: bytes b0..b7 (K c0..c7) in dwords lo, hi. Pair i = (b_i, b_i+4) moved into the low bytes
// of two halves by one v_perm_b32, the sign bit flipped and fp16 1024's high byte set by one xor
// (fp16 1024 + q + 128, exact), - 1152 (exact), * s (one rounding).
__device__ __forceinline__ f16x8 wdeq8_i8(uint32_t lo, uint32_t hi, half2_t s2) {
#pragma clang fp contract(off)
    const half2_t off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    uint32_t r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t sel = 0x0C000C00u | ((uint32_t)(4 + i) << 16) | (uint32_t)i;
        const uint32_t u = __builtin_amdgcn_perm(hi, lo, sel) ^ 0x64806480u;
        r[i] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(half2_t, u) + off) * s2);
    }
    return __builtin_bit_cast(f16x8, make_uint4(r[0], r[1], r[2], r[3]));
}

// fp8 e4m3fn: pair i moved into the HIGH bytes of two halves (b << 8); (v & sign) | ((v >> 1) &
// 0x3F80) is the fp16 of value * 2^-8 exactly (exponent bias 15 vs 7, subnormals included; the
// format's only NaN code never occurs in a record), * fp16(block scale * 2^8) (one rounding).
__device__ __forceinline__ f16x8 wdeq8_fp8(uint32_t lo, uint32_t hi, half2_t s2) {
    uint32_t r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t sel = 0x000C000Cu | ((uint32_t)(4 + i) << 24) | ((uint32_t)i << 8);
        const uint32_t v = __builtin_amdgcn_perm(hi, lo, sel);
        const uint32_t u = and_or(v >> 1, 0x3F803F80u, v & 0x80008000u);
        r[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, u) * s2);
    }
    return __builtin_bit_cast(f16x8, make_uint4(r[0], r[1], r[2], r[3]));
}

// fp16 / bf16: halves c0..c7 in dwords d0..d3; pair i = (c_i, c_i+4) by one v_perm_b32; bf16 pairs
// become fp16 through fp32 (exact for every value in fp16's normal range)
template <int PREC>
__device__ __forceinline__ f16x8 wdeq8_16(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3) {
    uint32_t r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = (i >> 1) == 0 ? d0 : d1, hi = (i >> 1) == 0 ? d2 : d3;
        const uint32_t v = __builtin_amdgcn_perm(hi, lo, (i & 1) ? 0x07060302u : 0x05040100u);
        if constexpr (PREC == MOEHIP_PREC_BF16) {
            r[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(__uint_as_float(v << 16),
                                                                          __uint_as_float(v & 0xffff0000u)));
        } else {
            r[i] = v;
        }
    }
    return __builtin_bit_cast(f16x8, make_uint4(r[0], r[1], r[2], r[3]));
}

// one chunk of weights in registers: per subtile this lane half's 32 bytes of its row and the
// raw scale (int4 / int8: fp16 group scale bits; fp8: fp32 block scale bits; fp16 / bf16: none)
struct WChunk {
    uint4 q[2][2];
    uint32_t s[2];
};

// qp[t]: the lane's row (subtile t) + 32 * half; sp[t]: its scale row (see gemm_rows)
template <int PREC>
__device__ __forceinline__ void load_chunk(WChunk &w, gu8 *const (&qp)[2], gu8 *const (&sp)[2], int c) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        gu8 *q = qp[t] + (size_t)c * 64;  // 64 bytes of a row per chunk for every precision
        w.q[t][0] = gld16(q);
        w.q[t][1] = gld16(q + 16);
        if constexpr (PREC == MOEHIP_PREC_INT4)
            w.s[t] = *(const __attribute__((address_space(1))) uint16_t *)(sp[t] + (size_t)c * 4);
        else if constexpr (PREC == MOEHIP_PREC_INT8)
            w.s[t] = *(const __attribute__((address_space(1))) uint16_t *)(sp[t] + (size_t)c * 2);
        else if constexpr (PREC == MOEHIP_PREC_FP8)
            w.s[t] = *(const __attribute__((address_space(1))) uint32_t *)(sp[t] + (size_t)(c >> 1) * 4);
        else
            w.s[t] = 0u;
    }
}

// row pointers of one lane: q row `row` of a (rows, K) weight matrix at qb, offset by the lane
// half's 32 bytes; scale row at sb (int4 / int8: fp16 (rows, K / 64); fp8: fp32 (rows / 128,
// K / 128) blocks)
template <int PREC>
__device__ __forceinline__ void gemm_rows(gu8 *qb, gu8 *sb, int row, int K, int h, gu8 *&q, gu8 *&sc) {
    q = qb + (size_t)row * ((size_t)K * GgPrec<PREC>::BITS / 8) + 32 * h;
    if constexpr (PREC == MOEHIP_PREC_INT4) sc = sb + (size_t)row * (K / GG_KG) * 2 + 2 * h;
    else if constexpr (PREC == MOEHIP_PREC_INT8) sc = sb + (size_t)row * (K / GG_KG) * 2;
    else if constexpr (PREC == MOEHIP_PREC_FP8) sc = sb + (size_t)(row >> 7) * (K >> 7) * 4;
    else sc = sb;
}

// B operand of MFMA step m of a chunk for one subtile (the lane's 8 dwords, natural K order)
template <int PREC, int M>
__device__ __forceinline__ f16x8 b_operand(const uint4 (&q)[2], uint32_t sraw, DeqK dk) {
    const uint32_t dw[8] = {q[0].x, q[0].y, q[0].z, q[0].w, q[1].x, q[1].y, q[1].z, q[1].w};
    if constexpr (PREC == MOEHIP_PREC_INT4) {
        const uint32_t sw = sraw & 0xffffu;
        return wdeq8(dw[M], __builtin_bit_cast(half2_t, sw | (sw << 16)), dk);
    } else if constexpr (PREC == MOEHIP_PREC_INT8) {
        const uint32_t sw = sraw & 0xffffu;
        return wdeq8_i8(dw[2 * M], dw[2 * M + 1], __builtin_bit_cast(half2_t, sw | (sw << 16)));
    } else if constexpr (PREC == MOEHIP_PREC_FP8) {
        const uint32_t sw = f32_to_f16_rne(__uint_as_float(sraw) * 256.0f);
        return wdeq8_fp8(dw[2 * M], dw[2 * M + 1], __builtin_bit_cast(half2_t, sw | (sw << 16)));
    } else {
        return wdeq8_16<PREC>(dw[4 * M], dw[4 * M + 1], dw[4 * M + 2], dw[4 * M + 3]);
    }
}

// ---------------------------------------------------------------------------------------
// activation chunks (fp16): thread tid stages token tid / 4 of the pass, values VPT * (tid % 4) ..
// of the chunk, permuted per 8 values into operand order (c0 c4 c1 c5 c2 c6 c3 c7), into LDS row
// `tok`. Threads past the pass's tokens load a valid row too (no branch around the loads, which
// keeps the compiler's load counting exact): MFMA rows are independent and those rows are never
// stored.
// ---------------------------------------------------------------------------------------
template <int CK>
__device__ __forceinline__ void xs_load(const uint16_t *row, int c, uint4 (&v)[GgChunk<CK>::NV]) {
    const uint4 *p = reinterpret_cast<const uint4 *>(row + (size_t)c * CK + (threadIdx.x & 3) * GgChunk<CK>::VPT);
#pragma unroll
    for (int m = 0; m < GgChunk<CK>::NV; ++m) v[m] = p[m];
}

template <int CK>
__device__ __forceinline__ void xs_store(const uint4 (&v)[GgChunk<CK>::NV], uint16_t *s_a) {
    const int tok = threadIdx.x >> 2, part = threadIdx.x & 3;
    uint4 *dst = reinterpret_cast<uint4 *>(s_a + tok * GgChunk<CK>::LDA + part * GgChunk<CK>::VPT);
#pragma unroll
    for (int m = 0; m < GgChunk<CK>::NV; ++m) {
        const uint4 u = v[m];
        dst[m] = make_uint4(lo_lo(u.x, u.z), hi_hi(u.x, u.z), lo_lo(u.y, u.w), hi_hi(u.y, u.w));
    }
}

// ---------------------------------------------------------------------------------------
// one chunk of MFMAs for a wave: CK / 16 steps x NM M tiles x 2 subtiles. Step m of lane half h
// covers K h * CK / 2 + 8 m .. + 7 of the chunk, in A (LDS) and B (registers) alike.
// ---------------------------------------------------------------------------------------
template <int PREC, int NM, int M = 0>
__device__ __forceinline__ void mma_steps(const WChunk &w, const uint16_t *ap, DeqK dk, f32x16 (&d)[2][2]) {
    constexpr int CK = GgPrec<PREC>::CK;
    if constexpr (M < CK / 16) {
        const f16x8 b0 = b_operand<PREC, M>(w.q[0], w.s[0], dk);
        const f16x8 b1 = b_operand<PREC, M>(w.q[1], w.s[1], dk);
#pragma unroll
        for (int mt = 0; mt < NM; ++mt) {
            const f16x8 a = *reinterpret_cast<const f16x8 *>(ap + mt * 32 * GgChunk<CK>::LDA + 8 * M);
            d[mt][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b0, d[mt][0], 0, 0, 0);
            d[mt][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b1, d[mt][1], 0, 0, 0);
        }
        mma_steps<PREC, NM, M + 1>(w, ap, dk, d);
    }
}

template <int PREC, int NM>
__device__ __forceinline__ void mma_chunk(const WChunk &w, const uint16_t *s_a, DeqK dk, f32x16 (&d)[2][2]) {
    constexpr int CK = GgPrec<PREC>::CK;
    const int lane = threadIdx.x & 63, i = lane & 31, h = lane >> 5;
    mma_steps<PREC, NM>(w, s_a + i * GgChunk<CK>::LDA + h * (CK / 2), dk, d);
}

// fp16 bits of 2^d for d <= 0 (subnormal below 2^-14, 0 below 2^-24)
__device__ __forceinline__ uint32_t pow2_h(int d) {
    return d >= -14 ? (uint32_t)(d + 15) << 10 : (d >= -24 ? 1u << (d + 24) : 0u);
}

// h chunks staged by the down tiles: h is fp16 scaled by 2^-eb per (pair, 32 columns) (the up
// wave of those columns chose eb); a staging thread multiplies its part of a chunk (CK / 4
// columns, within one block of 32) by 2^(eb - emax), emax the pair's largest eb (exact unless the
// product is subnormal), so one power per pair remains
template <int CK>
__device__ __forceinline__ void xs_scale(uint4 (&v)[GgChunk<CK>::NV], int eb, int emax) {
    const uint32_t fb = pow2_h(eb - emax);
    const half2_t f2 = __builtin_bit_cast(half2_t, fb | (fb << 16));
#pragma unroll
    for (int m = 0; m < GgChunk<CK>::NV; ++m) {
        v[m].x = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, v[m].x) * f2);
        v[m].y = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, v[m].y) * f2);
        v[m].z = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, v[m].z) * f2);
        v[m].w = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, v[m].w) * f2);
    }
}

// ---------------------------------------------------------------------------------------
// the K loop of one pass (nch chunks): queue order of the loads is X0, R0 .. R(RING-2), X1,
// R(RING-1) | per chunk c: X(c + 2), R(c + RING): waiting for an activation chunk never waits
// for the weight chunks issued after it, so RING - 1 weight chunks stay in flight. Every load
// is issued unconditionally (chunk indices clamped to the last chunk: a few repeated loads at
// the end hit L2): with loads under branches the compiler cannot count them and waits for all.
// ---------------------------------------------------------------------------------------
template <int PREC, int RING, int NM, bool SC = false>
__device__ __forceinline__ void k_loop(gu8 *const (&qp)[2], gu8 *const (&sp)[2], int nch, const uint16_t *srcrow,
                                       uint16_t *s_a, DeqK dk, f32x16 (&d)[2][2], const int *ebrow = nullptr,
                                       int emax = 0) {
    constexpr int CK = GgPrec<PREC>::CK;
    constexpr int ABUF = GG_TOK * GgChunk<CK>::LDA;
    const int cl = nch - 1;
    WChunk wr[RING];
    uint4 xv[GgChunk<CK>::NV];
    int xeb = 0;  // SC: the block exponent of the chunk in xv
    auto xload = [&](int c) {
        xs_load<CK>(srcrow, c, xv);
        if constexpr (SC) xeb = ebrow[(c * CK + (threadIdx.x & 3) * GgChunk<CK>::VPT) / 32];
    };
    auto xstore = [&](uint16_t *dst) {
        if constexpr (SC) xs_scale<CK>(xv, xeb, emax);
        xs_store<CK>(xv, dst);
    };
    xload(0);
#pragma unroll
    for (int u = 0; u + 1 < RING; ++u) load_chunk<PREC>(wr[u], qp, sp, min(u, cl));
    xstore(s_a);
    xload(min(1, cl));
    load_chunk<PREC>(wr[RING - 1], qp, sp, min(RING - 1, cl));
    __syncthreads();
#pragma unroll 1
    for (int c0 = 0; c0 < nch; c0 += RING) {
#pragma unroll
        for (int u = 0; u < RING; ++u) {
            const int c = c0 + u;
            const int b = c & 1;
            if (c < nch) mma_chunk<PREC, NM>(wr[u], s_a + b * ABUF, dk, d);
            // unconditional: under a branch the compiler sinks the activation load of the previous
            // step down to this store, and waiting for it then waits for every weight load too.
            // The other buffer was last read before the previous barrier; a store past the last
            // chunk is overwritten by the same thread in the next pass's prologue.
            xstore(s_a + (b ^ 1) * ABUF);
            xload(min(c + 2, cl));
            load_chunk<PREC>(wr[u], qp, sp, min(c + RING, cl));
            if (c < nch) __syncthreads();
        }
    }
}

// tile t -> (expert, block): the blocks of 8 consecutive experts interleave so that every tile of
// one expert has the same t % 8 (workgroups go round-robin over the 8 XCDs)
__device__ __forceinline__ bool tile_of(int t, int E, int NB, int &e, int &nb) {
    const int eg = t / (8 * NB), r = t % (8 * NB);
    e = eg * 8 + (r & 7);
    nb = r >> 3;
    return e < E;
}

// exponent e with max * 2^-e in [2^14, 2^15) (0 for 0, inf or nan)
__device__ __forceinline__ int row_exp(float m) {
    // ilogb(m) = frexp exponent - 1 (v_frexp_exp_i32_f32; subnormal m included)
    return (m > 0.f && m <= 3.0e38f) ? max(__builtin_amdgcn_frexp_expf(m) - 15, -100) : 0;
}

// bf16 activations, one wave per row: xe[r] = row_exp(max |x[r]|) and x16[r] = fp16(x[r] * 2^-xe[r])
// (exact for bf16 values in range), 8 values per 16-byte load and store.
// H is a multiple of 8.
__device__ __forceinline__ float bf16_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

__global__ __launch_bounds__(256) void k_prep(const uint16_t *__restrict__ x, int T, int H, int *__restrict__ xe,
                                              uint16_t *__restrict__ x16) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= T || x == nullptr) return;
    const uint4 *src = reinterpret_cast<const uint4 *>(x + (size_t)r * H);
    uint4 *dst = reinterpret_cast<uint4 *>(x16 + (size_t)r * H);
    const int nv = H / 8;
    float m = 0.f;
    for (int c = lane; c < nv; c += 64) {
        const uint4 v = src[c];
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) m = fmaxf(m, fmaxf(fabsf(bf16_lo(w[i])), fabsf(bf16_hi(w[i]))));
    }
    m = wave_max(m);
    const int e = row_exp(m);
    const float sc = ldexpf(1.0f, -e);
    for (int c = lane; c < nv; c += 64) {
        const uint4 v = src[c];
        dst[c] = make_uint4(pack_h2(bf16_lo(v.x) * sc, bf16_hi(v.x) * sc), pack_h2(bf16_lo(v.y) * sc, bf16_hi(v.y) * sc),
                            pack_h2(bf16_lo(v.z) * sc, bf16_hi(v.z) * sc), pack_h2(bf16_lo(v.w) * sc, bf16_hi(v.w) * sc));
    }
    if (lane == 0) xe[r] = e;
}

// ---------------------------------------------------------------------------------------
// up: tiles (expert, 128 h columns); wave w: h columns nb*128 + 32 w + (lane % 32), subtile 0 =
// gate rows, subtile 1 = up rows. Writes h (pairs, I) fp32.
// ---------------------------------------------------------------------------------------
// x: fp16 activations (the caller's, or x16 with exponents xe for bf16 input; xe null = 0)
// largest of a non-negative float over each 32-lane half of the wave, in every lane of the half
// (every lane active), on the float's bits (their order is the values' for v >= 0; 0 is the
// identity of the unsigned max, so each DPP move folds into its max): butterflies within rows of
// 16, then lane i against lane i ^ 16 (ds_swizzle, bit-mask mode: and 0x1f, or 0, xor 0x10)
__device__ __forceinline__ float half_max(float f) {
    uint32_t v = __float_as_uint(f);
    v = max(v, (uint32_t)dpp_i<0xB1>((int)v));
    v = max(v, (uint32_t)dpp_i<0x4E>((int)v));
    v = max(v, (uint32_t)dpp_i<0x141>((int)v));
    v = max(v, (uint32_t)dpp_i<0x140>((int)v));
    v = max(v, (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x401F));
    return __uint_as_float(v);
}

template <int PREC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_up(
    const uint16_t *__restrict__ x, const int *__restrict__ xe, int H, int I, int k, int E,
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ sorted_pos, const int64_t *__restrict__ tab,
    uint16_t *__restrict__ h16, int *__restrict__ hbe, DeqK dk) {
    constexpr int CK = GgPrec<PREC>::CK;
    __shared__ __align__(16) uint16_t s_a[2 * GG_TOK * GgChunk<CK>::LDA];
    __shared__ int s_e[GG_TOK];
    const int NB = I / 128;
    int e, nb;
    if (!tile_of(blockIdx.x, E, NB, e, nb)) return;
    const int p0 = offsets[e], ne = offsets[e + 1] - p0;
    gu8 *qb = record_ptr(tab[4 * e + 0]);
    gu8 *sb = record_ptr(tab[4 * e + 1]);
    if (ne <= 0 || qb == nullptr) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 31, h = lane >> 5;
    const int col = nb * 128 + 32 * wave + j;
    gu8 *qp[2], *sp[2];
    gemm_rows<PREC>(qb, sb, col, H, h, qp[0], sp[0]);
    gemm_rows<PREC>(qb, sb, I + col, H, h, qp[1], sp[1]);
    const int nch = H / CK;
    for (int m0 = 0; m0 < ne; m0 += GG_TOK) {
        const int mn = min(GG_TOK, ne - m0), nm = (mn + 31) / 32;
        const int stok = tid >> 2;
        const bool sok = stok < mn;
        const int xr = sok ? sorted_pos[p0 + m0 + stok] / k : 0;
        const int ex = (sok && xe != nullptr) ? xe[xr] : 0;
        if ((tid & 3) == 0) s_e[stok] = ex;
        f32x16 d[2][2];
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b) d[a][b] = f32x16{};
        if (nm == 2) k_loop<PREC, 2, 2>(qp, sp, nch, x + (size_t)xr * H, s_a, dk, d);
        else k_loop<PREC, 2, 1>(qp, sp, nch, x + (size_t)xr * H, s_a, dk, d);
        // epilogue: h = silu(gate) * up (scaled back by the token's 2^e); per token the largest
        // |h| of the wave's 32 columns (one half of the wave) sets the block exponent eb; h is
        // stored fp16 times 2^-eb, eb beside it
        // (branch-free first loop: the 16 lane reductions of a tile interleave)
        const int NB32 = I / 32;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            if (mt >= nm) break;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int tok = mt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                const float f = ldexpf(1.0f, s_e[tok]);
                const float hv = silu_mul(d[mt][0][r] * f, d[mt][1][r] * f);
                d[mt][0][r] = hv;
                d[mt][1][r] = half_max(fabsf(hv));
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int tok = mt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                const int eb = row_exp(d[mt][1][r]);
                if (tok < mn) {
                    const size_t p = (size_t)(p0 + m0 + tok);
                    h16[p * I + col] = f32_to_f16_rne(d[mt][0][r] * ldexpf(1.0f, -eb));
                    if (j == 0) hbe[p * NB32 + (col >> 5)] = eb;
                }
            }
        }
        __syncthreads();  // s_e of the next pass
    }
}

// ---------------------------------------------------------------------------------------
// Batched GEMV for few tokens per expert (batched decode): the same h / y as the MFMA kernels,
// computed with v_dot2_f32_f16 against weights streamed in whole rows. A row of K values is
// C = K / VPC chunks of 16 bytes; G = 2^lg lanes share a row, lane cl owning chunks cl + i G
// (i < CPL), so RPW = 64 / G rows per wave pass and P passes per wave, every load of the P passes
// issued before any is used. A chunk's B values come from the MFMA path's converters (operand
// order c0 c4 c1 c5 c2 c6 c3 c7 per 8 values, one fp16 rounding of the scaled weight); the lane's
// activation slice of each token is permuted the same way when it is loaded. The expert's tokens
// run GV_NT at a time against the weights held in registers (weights are read once however many
// tokens the expert has).
// ---------------------------------------------------------------------------------------
constexpr int GV_NT = GV_TOKENS;  // tokens per work item (decide.hpp: the decision kernels write the same list)
constexpr int GV_TG = GV_NT;  // tokens of one expert per workgroup (more tokens: more work items)
constexpr int GV_MAXROWS = 512; // rows of one workgroup (their outputs are staged in LDS)

// raw scale of chunk c of a row (int4 / int8: fp16 bits of its group; fp8: fp32 bits of its block)
template <int PREC>
__device__ __forceinline__ uint32_t gv_scale(gu8 *sb, int row, int c, int K) {
    constexpr int VPC = Fmt<PREC>::VPC;
    if constexpr (PREC == MOEHIP_PREC_INT4 || PREC == MOEHIP_PREC_INT8)
        return *(const __attribute__((address_space(1))) uint16_t *)(sb + ((size_t)row * (K / GG_KG) + (c * VPC) / GG_KG) * 2);
    else if constexpr (PREC == MOEHIP_PREC_FP8)
        return *(const __attribute__((address_space(1))) uint32_t *)(sb + ((size_t)(row >> 7) * (K >> 7) + ((c * VPC) >> 7)) * 4);
    else
        return 0u;
}

// the chunk's VPC values as fp16 pairs in operand order (VPC / 2 dwords)
template <int PREC>
__device__ __forceinline__ void gv_deq(const uint4 q, uint32_t sraw, DeqK dk, uint32_t *wv) {
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
    if constexpr (PREC == MOEHIP_PREC_INT4) {
        const uint32_t sw = sraw & 0xffffu;
        const half2_t s2 = __builtin_bit_cast(half2_t, sw | (sw << 16));
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const uint4 u = __builtin_bit_cast(uint4, wdeq8(d[b], s2, dk));
            wv[4 * b] = u.x, wv[4 * b + 1] = u.y, wv[4 * b + 2] = u.z, wv[4 * b + 3] = u.w;
        }
    } else if constexpr (PREC == MOEHIP_PREC_INT8 || PREC == MOEHIP_PREC_FP8) {
        uint32_t sw;
        if constexpr (PREC == MOEHIP_PREC_INT8) sw = sraw & 0xffffu;
        else sw = f32_to_f16_rne(__uint_as_float(sraw) * 256.0f);
        const half2_t s2 = __builtin_bit_cast(half2_t, sw | (sw << 16));
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const uint4 u = __builtin_bit_cast(uint4, PREC == MOEHIP_PREC_INT8 ? wdeq8_i8(d[2 * b], d[2 * b + 1], s2)
                                                                              : wdeq8_fp8(d[2 * b], d[2 * b + 1], s2));
            wv[4 * b] = u.x, wv[4 * b + 1] = u.y, wv[4 * b + 2] = u.z, wv[4 * b + 3] = u.w;
        }
    } else {
        const uint4 u = __builtin_bit_cast(uint4, wdeq8_16<PREC>(d[0], d[1], d[2], d[3]));
        wv[0] = u.x, wv[1] = u.y, wv[2] = u.z, wv[3] = u.w;
    }
}

// activation slice of chunk c of a row of K fp16 values (VPC / 8 16-byte loads), and its
// permutation into operand order (VPC / 2 dwords), done once the weight loads are issued
template <int VPC>
__device__ __forceinline__ void gv_slice_load(const uint16_t *row, int c, uint4 *raw) {
    const uint4 *p = reinterpret_cast<const uint4 *>(row + (size_t)c * VPC);
#pragma unroll
    for (int b = 0; b < VPC / 8; ++b) raw[b] = p[b];
}
// (int8 records: the pairs of the integer dot instead, (v0,v2) (v1,v3) per 4 values)
template <int VPC, bool I8 = false>
__device__ __forceinline__ void gv_slice_perm(const uint4 *raw, uint32_t *xv) {
#pragma unroll
    for (int b = 0; b < VPC / 8; ++b) {
        const uint4 u = raw[b];
        if constexpr (I8) {
            xv[4 * b] = lo_lo(u.x, u.y), xv[4 * b + 1] = hi_hi(u.x, u.y);
            xv[4 * b + 2] = lo_lo(u.z, u.w), xv[4 * b + 3] = hi_hi(u.z, u.w);
        } else {
            xv[4 * b] = lo_lo(u.x, u.z), xv[4 * b + 1] = hi_hi(u.x, u.z);
            xv[4 * b + 2] = lo_lo(u.y, u.w), xv[4 * b + 3] = hi_hi(u.y, u.w);
        }
    }
}
// the first value of pair q of 8 (the second is 4 further, or 2 further for the int8 pairs)
template <bool I8>
__device__ __forceinline__ constexpr int gv_pair_first(int q) { return I8 ? 4 * (q >> 1) + (q & 1) : q; }

// NG row groups of 4 P RPW rows from r0 (gate and up rows for UP) of one expert, against up to
// GV_NT of its tokens; UP: h[pair, r] = silu(gate . x) * (up . x); else y[pair, r] = w 2^he (down . h).
// The loads of group g + 1 are issued before group g is computed (two register buffers).
template <int PREC, int CPL, int P, bool UP, bool XBF = false>
__device__ __forceinline__ void gv_rows(const void *act, const int *ae, int K, int rows, int I, int k, int p0,
                                        int nt, const int32_t *sorted_pos, gu8 *qb, gu8 *sb, int lg, int r0, int NG,
                                        const float *w, float *out, int ostride, DeqK dk) {
    constexpr int VPC = Fmt<PREC>::VPC, ND = VPC / 2, NM = UP ? 2 : 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int G = 1 << lg, RPW = 64 >> lg, slot = lane >> lg, cl = lane & (G - 1);
    const int C = K / VPC;
    const size_t RB = (size_t)C * 16;
    const int GROWS = 4 * P * RPW;  // rows per group
    __shared__ float s_out[GV_NT][GV_MAXROWS];
    // the tokens first (their loads do not queue behind the weights'), then the activation slices
    int pr[GV_NT], src[GV_NT];
#pragma unroll
    for (int t = 0; t < GV_NT; ++t) {
        pr[t] = p0 + min(t, nt - 1);
        src[t] = UP ? sorted_pos[pr[t]] / k : pr[t];  // UP: the token's row of x; else the pair's h
    }
    // UP: fp16 activation slices (the token's power of two in f); DOWN: fp32 h slices, each chunk
    // scaled into fp16 by its own power of two (fe) once the weights are requested
    constexpr int XW = UP ? VPC / 8 : VPC / 4;  // 16-byte loads per chunk
    uint4 xr[GV_NT][CPL][XW];
    float f[GV_NT];
#pragma unroll
    for (int t = 0; t < GV_NT; ++t) {
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = min(cl + i * G, C - 1);
            const uint4 *p = UP ? reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(act) + (size_t)src[t] * K + (size_t)c * VPC)
                                : reinterpret_cast<const uint4 *>(reinterpret_cast<const float *>(act) + (size_t)src[t] * K + (size_t)c * VPC);
#pragma unroll
            for (int b = 0; b < XW; ++b) xr[t][i][b] = p[b];
        }
        if constexpr (UP) f[t] = ldexpf(1.0f, ae != nullptr ? ae[src[t]] : 0);
        else f[t] = w[sorted_pos[pr[t]]];
    }
    uint4 q[2][P][NM][CPL];
    uint32_t sr[2][P][NM][CPL];
    auto load = [&](int buf, int g) {
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int r = min(r0 + g * GROWS + (wave * P + p) * RPW + slot, rows - 1);
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const int row = r + m * I;  // UP: gate row r, up row I + r
#pragma unroll
                for (int i = 0; i < CPL; ++i) {
                    // every load unconditional (clamped chunk): a load under a lane-dependent
                    // branch is waited for before the next one is issued
                    const int c = min(cl + i * G, C - 1);
                    q[buf][p][m][i] = gld16(qb + (size_t)row * RB + (size_t)c * 16);
                    sr[buf][p][m][i] = gv_scale<PREC>(sb, row, c, K);
                }
            }
        }
    };
    load(0, 0);
    uint32_t xv[GV_NT][CPL][ND];
    float fe[GV_NT][CPL];
    // int4 / int8: the weights' integers straight into dot2 (offsets removed by the per-chunk
    // correction, the group scale applied to the chunk sum in fp32)
    constexpr bool IDOT = PREC == MOEHIP_PREC_INT4 || PREC == MOEHIP_PREC_INT8;
    constexpr bool XS = !UP || XBF;  // activation slices scaled per chunk (fe), not per token
    float corr[GV_NT][CPL];
#pragma unroll
    for (int t = 0; t < GV_NT; ++t)
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            if constexpr (UP && !XBF) {
                gv_slice_perm<VPC, PREC == MOEHIP_PREC_INT8>(xr[t][i], xv[t][i]);
                fe[t][i] = 1.0f;
            } else {
                // fp32 h (down) or bf16 x (XBF: up without the activation preparation pass)
                float v[VPC];
                if constexpr (UP) {
                    const uint32_t *wd = reinterpret_cast<const uint32_t *>(xr[t][i]);
#pragma unroll
                    for (int q = 0; q < VPC / 2; ++q) {
                        v[2 * q] = __uint_as_float(wd[q] << 16);
                        v[2 * q + 1] = __uint_as_float(wd[q] & 0xffff0000u);
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < VPC; ++q) v[q] = reinterpret_cast<const float *>(xr[t][i])[q];
                }
                float m = 0.f;
#pragma unroll
                for (int q = 0; q < VPC; ++q) m = fmaxf(m, fabsf(v[q]));
                const int e = row_exp(m);
                const float sc = ldexpf(1.0f, -e);
                fe[t][i] = ldexpf(1.0f, e);
#pragma unroll
                for (int b = 0; b < VPC / 8; ++b)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        constexpr bool I8 = PREC == MOEHIP_PREC_INT8;
                        const int f = 8 * b + gv_pair_first<I8>(q);
                        xv[t][i][4 * b + q] = pack_h2(v[f] * sc, v[f + (I8 ? 2 : 4)] * sc);
                    }
            }
            // lanes past the row's chunks (G > C / CPL) load the clamped last chunk: a zero slice
            // makes their products zero, so the weights need no select
            if (cl + i * G >= C)
#pragma unroll
                for (int j = 0; j < ND; ++j) xv[t][i][j] = 0u;
            if constexpr (IDOT) corr[t][i] = chunk_corr<PREC>(xv[t][i]);
        }
    auto compute = [&](int buf, int g) {
#pragma unroll
        for (int p = 0; p < P; ++p) {
            float acc[NM][GV_NT];
#pragma unroll
            for (int m = 0; m < NM; ++m) {
#pragma unroll
                for (int t = 0; t < GV_NT; ++t) acc[m][t] = 0.f;
#pragma unroll
                for (int i = 0; i < CPL; ++i) {
                    if constexpr (PREC == MOEHIP_PREC_FP8) {
                        // the exact fp16 pairs of value * 2^-8, the block scale * 2^8 on the sum
                        const float sc = __uint_as_float(sr[buf][p][m][i]) * 256.0f;
                        const uint4 qq = q[buf][p][m][i];
                        const uint32_t d[4] = {qq.x, qq.y, qq.z, qq.w};
                        uint32_t wv[8];
#pragma unroll
                        for (int b = 0; b < 2; ++b)
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                const uint32_t sel = 0x000C000Cu | ((uint32_t)(4 + j) << 24) | ((uint32_t)j << 8);
                                const uint32_t v = __builtin_amdgcn_perm(d[2 * b + 1], d[2 * b], sel);
                                wv[4 * b + j] = and_or(v >> 1, 0x3F803F80u, v & 0x80008000u);
                            }
#pragma unroll
                        for (int t = 0; t < GV_NT; ++t) {
                            if (t < nt) {
                                float pc = 0.f;
#pragma unroll
                                for (int j = 0; j < 8; ++j) pc = dot2h(wv[j], xv[t][i][j], pc);
                                acc[m][t] = fmaf(pc, XS ? sc * fe[t][i] : sc, acc[m][t]);
                            }
                        }
                    } else if constexpr (IDOT) {
                        const float sc = f16_to_f32(sr[buf][p][m][i] & 0xffffu);
#pragma unroll
                        for (int t = 0; t < GV_NT; ++t) {
                            if (t < nt) {
                                const float cd = dot2_chunk<PREC>(q[buf][p][m][i], xv[t][i], corr[t][i]);
                                acc[m][t] = fmaf(cd, XS ? sc * fe[t][i] : sc, acc[m][t]);
                            }
                        }
                    } else {
                    uint32_t wv[ND];
                    gv_deq<PREC>(q[buf][p][m][i], sr[buf][p][m][i], dk, wv);
#pragma unroll
                    for (int t = 0; t < GV_NT; ++t) {
                        if (t < nt) {
                            if constexpr (!XS) {
#pragma unroll
                                for (int j = 0; j < ND; ++j) acc[m][t] = dot2h(wv[j], xv[t][i][j], acc[m][t]);
                            } else {
                                float pc = 0.f;
#pragma unroll
                                for (int j = 0; j < ND; ++j) pc = dot2h(wv[j], xv[t][i][j], pc);
                                acc[m][t] = fmaf(pc, fe[t][i], acc[m][t]);
                            }
                        }
                    }
                    }
                }
            }
            const int r = r0 + g * GROWS + (wave * P + p) * RPW + slot;
#pragma unroll
            for (int t = 0; t < GV_NT; ++t) {
                if (t < nt) {
                    const float a0 = group_sum(acc[0][t], lg);
                    if constexpr (UP) {
                        const float a1 = group_sum(acc[NM - 1][t], lg);
                        const float hv = silu_mul(a0 * f[t], a1 * f[t]);
                        if (cl == 0) s_out[t][r - r0] = hv;
                    } else {
                        if (cl == 0) s_out[t][r - r0] = f[t] * a0;
                    }
                }
            }
        }
    };
    // steady state with unconditional loads (a load under a branch makes the wait for the other
    // buffer a wait for every load), then the last one or two groups
    int g = 0;
    for (; g + 2 < NG; g += 2) {
        load(1, g + 1);
        compute(0, g);
        load(0, g + 2);
        compute(1, g + 1);
    }
    if (g + 1 < NG) {
        load(1, g + 1);
        compute(0, g);
        compute(1, g + 1);
    } else {
        compute(0, g);
    }
    // the outputs, written once the weight stream is done (a store makes every later wait for
    // a load also wait for the store's acknowledgement)
    __syncthreads();
    const int nrows = min(NG * GROWS, rows - r0);
    for (int i = threadIdx.x; i < nt * nrows; i += 256) {
        const int t = i / nrows, rr = i - t * nrows;
        out[(size_t)(p0 + t) * ostride + r0 + rr] = s_out[t][rr];
    }
}

// work lists of the batched GEMVs when the decision did not write them: one per record precision
// p < P at items + p * (NP + 1), the (expert, token group of GV_TG) items of every expert whose
// table row of precision p is set, in expert order (one workgroup, exclusive scan of
// ceil(n_e / GV_TG)); [NP] = their number
__global__ __launch_bounds__(1024) void k_gv_items(const int32_t *__restrict__ offsets, int E, int NP,
                                                   const int64_t *__restrict__ tabs, int P, int32_t *__restrict__ items) {
    __shared__ int s_w[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int p = 0; p < P; ++p) {
        int32_t *it = items + (size_t)p * (NP + 1);
        int base = 0;
        for (int e0 = 0; e0 < E; e0 += 1024) {
            const int e = e0 + tid;
            const int n = (e < E && tabs[((size_t)p * E + e) * 4] != 0) ? offsets[e + 1] - offsets[e] : 0;
            const int nz = (n + GV_TG - 1) / GV_TG;
            int incl = nz;
            for (int off = 1; off < 64; off <<= 1) {
                const int v = __shfl_up(incl, off, 64);
                if (lane >= off) incl += v;
            }
            if (lane == 63) s_w[wave] = incl;
            __syncthreads();
            int wb = base, tot = base;
            for (int w = 0; w < 16; ++w) {
                if (w < wave) wb += s_w[w];
                tot += s_w[w];
            }
            for (int z = 0; z < nz; ++z) it[wb + incl - nz + z] = (e << 8) | z;
            base = tot;
            __syncthreads();
        }
        if (tid == 0) it[NP] = base;
    }
}

// grid (row blocks, NP): block (b, i) covers rows [b * NG * 4 P RPW, ...) of work item i (expert e,
// its tokens [z * GV_TG, (z + 1) * GV_TG)) when i < items[NP]
template <int PREC, int CPL, int P, bool XBF>
__global__ __launch_bounds__(256) void k_gemv_up(const uint16_t *__restrict__ x, const int *__restrict__ xe, int H,
                                                 int I, int k, const int32_t *__restrict__ items, int NP,
                                                 const int32_t *__restrict__ offsets,
                                                 const int32_t *__restrict__ sorted_pos,
                                                 const int64_t *__restrict__ tab, float *__restrict__ hb, DeqK dk,
                                                 int lg, int NG) {
    if ((int)blockIdx.y >= items[NP]) return;
    const int it = items[blockIdx.y], e = it >> 8;
    const int p0 = offsets[e] + (it & 255) * GV_TG, ne = min(GV_TG, offsets[e + 1] - p0);
    gu8 *qb = record_ptr(tab[4 * e + 0]);
    if (ne <= 0 || qb == nullptr) return;
    const int r0 = blockIdx.x * NG * 4 * P * (64 >> lg);
    if (r0 >= I) return;  // a row block of the padding to a multiple of 8
    gv_rows<PREC, CPL, P, true, XBF>(x, xe, H, I, I, k, p0, ne, sorted_pos, qb, record_ptr(tab[4 * e + 1]), lg, r0, NG,
                                nullptr, hb, I, dk);
}

template <int PREC, int CPL, int P>
__global__ __launch_bounds__(256) void k_gemv_down(const float *__restrict__ hb, int H,
                                                   int I, const int32_t *__restrict__ items, int NP,
                                                   const int32_t *__restrict__ offsets,
                                                   const int32_t *__restrict__ sorted_pos,
                                                   const int64_t *__restrict__ tab, const float *__restrict__ w,
                                                   float *__restrict__ y, DeqK dk, int lg, int NG) {
    if ((int)blockIdx.y >= items[NP]) return;
    const int it = items[blockIdx.y], e = it >> 8;
    const int p0 = offsets[e] + (it & 255) * GV_TG, ne = min(GV_TG, offsets[e + 1] - p0);
    gu8 *qb = record_ptr(tab[4 * e + 2]);
    if (ne <= 0 || qb == nullptr) return;
    const int r0 = blockIdx.x * NG * 4 * P * (64 >> lg);
    if (r0 >= H) return;  // a row block of the padding to a multiple of 8
    gv_rows<PREC, CPL, P, false>(hb, nullptr, I, H, 0, 1, p0, ne, sorted_pos, qb, record_ptr(tab[4 * e + 3]), lg, r0, NG,
                                 w, y, H, dk);
}

// Both record precisions of a two-precision store in ONE launch (a mixed store's per-precision
// launches mostly find few or no experts at one of the precisions, and an empty launch still
// costs its dispatch and every workgroup's read of the count): items i < n0 of the grid's y run
// precision 0's list, the next n1 precision 1's, each side with its own row geometry (grid.x is
// the larger of the two sides' row-block counts; a side's surplus blocks exit).
struct GvSide {
    const int32_t *items;  // the precision's work list ([NP] = its length)
    const int64_t *tab;    // its record table
    int lg, NG, gx;        // lanes per row (log2), row groups per workgroup, row blocks
};
template <int PA, int CA, int QA, int PB, int CB, int QB, bool XBF>
__global__ __launch_bounds__(256) void k_gemv_up2(const uint16_t *__restrict__ x, const int *__restrict__ xe, int H,
                                                  int I, int k, int NP, const int32_t *__restrict__ offsets,
                                                  const int32_t *__restrict__ sorted_pos, float *__restrict__ hb,
                                                  DeqK dk, GvSide sa, GvSide sb) {
    const int n0 = sa.items[NP], n1 = sb.items[NP];
    int i = blockIdx.y;
    const bool first = i < n0;
    if (!first) i -= n0;
    if (!first && i >= n1) return;
    const GvSide &sd = first ? sa : sb;
    if ((int)blockIdx.x >= sd.gx) return;
    const int it = sd.items[i], e = it >> 8;
    const int p0 = offsets[e] + (it & 255) * GV_TG, ne = min(GV_TG, offsets[e + 1] - p0);
    gu8 *qb = record_ptr(sd.tab[4 * e + 0]);
    if (ne <= 0 || qb == nullptr) return;
    gu8 *sc = record_ptr(sd.tab[4 * e + 1]);
    if (first) {
        const int r0 = blockIdx.x * sa.NG * 4 * QA * (64 >> sa.lg);
        if (r0 < I) gv_rows<PA, CA, QA, true, XBF>(x, xe, H, I, I, k, p0, ne, sorted_pos, qb, sc, sa.lg, r0, sa.NG, nullptr, hb, I, dk);
    } else {
        const int r0 = blockIdx.x * sb.NG * 4 * QB * (64 >> sb.lg);
        if (r0 < I) gv_rows<PB, CB, QB, true, XBF>(x, xe, H, I, I, k, p0, ne, sorted_pos, qb, sc, sb.lg, r0, sb.NG, nullptr, hb, I, dk);
    }
}

template <int PA, int CA, int QA, int PB, int CB, int QB>
__global__ __launch_bounds__(256) void k_gemv_down2(const float *__restrict__ hb, int H, int I, int NP,
                                                    const int32_t *__restrict__ offsets,
                                                    const int32_t *__restrict__ sorted_pos, const float *__restrict__ w,
                                                    float *__restrict__ y, DeqK dk, GvSide sa, GvSide sb) {
    const int n0 = sa.items[NP], n1 = sb.items[NP];
    int i = blockIdx.y;
    const bool first = i < n0;
    if (!first) i -= n0;
    if (!first && i >= n1) return;
    const GvSide &sd = first ? sa : sb;
    if ((int)blockIdx.x >= sd.gx) return;
    const int it = sd.items[i], e = it >> 8;
    const int p0 = offsets[e] + (it & 255) * GV_TG, ne = min(GV_TG, offsets[e + 1] - p0);
    gu8 *qb = record_ptr(sd.tab[4 * e + 2]);
    if (ne <= 0 || qb == nullptr) return;
    gu8 *sc = record_ptr(sd.tab[4 * e + 3]);
    if (first) {
        const int r0 = blockIdx.x * sa.NG * 4 * QA * (64 >> sa.lg);
        if (r0 < H) gv_rows<PA, CA, QA, false>(hb, nullptr, I, H, 0, 1, p0, ne, sorted_pos, qb, sc, sa.lg, r0, sa.NG, w, y, H, dk);
    } else {
        const int r0 = blockIdx.x * sb.NG * 4 * QB * (64 >> sb.lg);
        if (r0 < H) gv_rows<PB, CB, QB, false>(hb, nullptr, I, H, 0, 1, p0, ne, sorted_pos, qb, sc, sb.lg, r0, sb.NG, w, y, H, dk);
    }
}

// ---------------------------------------------------------------------------------------
// down: tiles (expert, 256 output rows); wave w: rows nb*256 + 64 w + 32 t + (lane % 32).
// y[pair, row] = w[pair] * (down_row . h_pair); h is read as the up tiles left it (fp16 times
// 2^-eb per 32 columns) and rescaled to the pair's largest exponent Emax while staged
// ---------------------------------------------------------------------------------------
template <int PREC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_down(
    const uint16_t *__restrict__ h16, const int *__restrict__ hbe, int H, int I, int E,
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ sorted_pos, const int64_t *__restrict__ tab,
    const float *__restrict__ w, float *__restrict__ y, DeqK dk, int zero_missing) {
    constexpr int CK = GgPrec<PREC>::CK;
    __shared__ __align__(16) uint16_t s_a[2 * GG_TOK * GgChunk<CK>::LDA];
    __shared__ float s_f[GG_TOK];  // w[pair] * 2^Emax
    const int NB = H / GG_ROWS;
    int e, nb;
    if (!tile_of(blockIdx.x, E, NB, e, nb)) return;
    const int p0 = offsets[e], ne = offsets[e + 1] - p0;
    if (ne <= 0) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 31, h = lane >> 5;
    gu8 *qb = record_ptr(tab[4 * e + 2]);
    gu8 *sb = record_ptr(tab[4 * e + 3]);
    const int row0 = nb * GG_ROWS + 64 * wave + j;
    if (qb == nullptr) {  // expert not resident (single-table launches): its pairs contribute nothing
        if (zero_missing)
            for (int i = tid; i < ne * GG_ROWS; i += 256)
                y[(size_t)(p0 + i / GG_ROWS) * H + nb * GG_ROWS + i % GG_ROWS] = 0.f;
        return;
    }
    gu8 *qp[2], *sp[2];
    gemm_rows<PREC>(qb, sb, row0, I, h, qp[0], sp[0]);
    gemm_rows<PREC>(qb, sb, row0 + 32, I, h, qp[1], sp[1]);
    const int nch = I / CK;
    for (int m0 = 0; m0 < ne; m0 += GG_TOK) {
        const int mn = min(GG_TOK, ne - m0), nm = (mn + 31) / 32;
        const int stok = tid >> 2;
        const bool sok = stok < mn;
        const size_t pr = (size_t)(p0 + m0 + (sok ? stok : 0));
        // the pair's largest block exponent: the 4 staging threads of the pair take every 4th
        // block (independent loads, issued together), then the largest over the 4 (DPP)
        const int NB32 = I / 32;
        const int *ebrow = hbe + pr * NB32;
        int emax = -1000;
        for (int i0 = tid & 3; i0 < NB32; i0 += 32) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (i0 + 4 * i < NB32) emax = max(emax, ebrow[i0 + 4 * i]);
        }
        emax = max(emax, dpp_i<0xB1>(emax));
        emax = max(emax, dpp_i<0x4E>(emax));
        if ((tid & 3) == 0) s_f[stok] = sok ? w[sorted_pos[pr]] * ldexpf(1.0f, emax) : 0.f;
        f32x16 d[2][2];
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b) d[a][b] = f32x16{};
        if (nm == 2) k_loop<PREC, 2, 2, true>(qp, sp, nch, h16 + pr * I, s_a, dk, d, ebrow, emax);
        else k_loop<PREC, 2, 1, true>(qp, sp, nch, h16 + pr * I, s_a, dk, d, ebrow, emax);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            if (mt >= nm) break;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int tok = mt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (tok >= mn) continue;
                const size_t p = (size_t)(p0 + m0 + tok);
                const float f = s_f[tok];
                y[p * H + row0] = f * d[mt][0][r];
                y[p * H + row0 + 32] = f * d[mt][1][r];
            }
        }
        __syncthreads();  // s_f of the next pass
    }
}

// ---------------------------------------------------------------------------------------
// Persistent expert FFN: the gate/up and down GEMMs of one record table in ONE launch.
//
// Work units: (expert e, pass m) = up to 64 of the expert's pairs. Unit u (numbered in expert
// order over the experts with pairs) belongs to XCD u % 8. Its tiles: NBU = I / 128 up tiles
// (128 h columns each) and NBD = H / 256 down tiles (256 output rows each). k_ffn_plan writes
// one queue per XCD (a unit's down tiles about a round of up tiles after its up tiles). The
// grid is what the GPU holds at once (or less); workgroup b takes tickets from the queue of XCD
// b % 8 (the XCD it runs on: the MI355X deals workgroups to XCDs round robin, checked once per
// device), so an expert's activation rows and h rows are re-read from that XCD's L2.
//
// An up tile writes h = silu(gate x) * (up x) as fp16 scaled by a power of two per (pair, up
// tile) (2^-eb, eb from the largest |h| of the pair's 128 columns), the exponents beside, then
// counts itself done on the unit (agent-scope counter, after its stores are acknowledged). A
// down tile waits for its unit's NBU up tiles (bounded wait; on expiry its outputs are NaN and
// the error word is set), rescales each h block to the pair's largest exponent while staging it
// (2^(eb - Emax), exact for all but subnormal results) and writes y = w 2^Emax (down h). The
// waits cannot deadlock: a down tile's up tiles were handed out earlier, to running workgroups,
// and up tiles wait for nothing. Reads of h and its exponents bypass the CU's L1 (non-temporal
// loads), which may hold lines fetched before a neighbouring pair's h was written.
//
// K loop: the activation (or h) chunk of a pass is loaded two chunks ahead into registers and
// stored into LDS one chunk ahead (two LDS buffers, one barrier per chunk); the weights of RING
// chunks are in flight in registers per wave.
// ---------------------------------------------------------------------------------------
constexpr int FP_TICK = 0;     // ticket counter of XCD x at FP_TICK + FP_TSTRIDE x (2 KB apart: no shared channel);
constexpr int FP_TSTRIDE = 512; // those of the down phase of a two-phase run at FP_TICK + FP_TSTRIDE (8 + x)
constexpr int FP_NALL = 8192;  // all tiles of XCD x
constexpr int FP_NUP = 8208;   // up tiles of XCD x (the first ones of its queue when the lag covers every unit)
constexpr int FP_ERR = 8200;   // error word: a bounded wait expired
constexpr int FP_DONE = 8448;  // flag[u * NBU + nb]: up tile nb of unit u has stored its h
constexpr int FF_SKIP = 1 << 30;  // entry flag: expert without a record (no tile to run)
constexpr int FF_ZERO = 1 << 29;  // entry flag: down tile of an expert without a record: y = 0
constexpr int FF_SPIN = 1 << 21;  // polls before a wait gives up (~1 s)
constexpr int FF_DUMMY = 512;     // bytes of the workgroup's own line pair read past a pass's last chunk
constexpr int FF_DUMMY_WGS = 4096; // workgroups with a line pair of their own (more share them)

// units over every expert with pairs: at most NP (one per pair) plus one per 64 pairs
__host__ __device__ inline int ffn_max_units(int NP) { return NP + (NP + 63) / 64 + 8; }
// entries per XCD queue: up and down tiles of its units
__host__ __device__ inline int ffn_lmax(int NP, int NBU, int NBD) { return (ffn_max_units(NP) + 7) / 8 * (NBU + NBD); }

// One workgroup: unit numbers by an exclusive scan of the experts' pass counts (twice: the
// first pass counts the units), then every expert writes the entries of its units (32 bytes:
// {e, p0, pairs, nb | flags} {u}, bit 31 of the third word set for down tiles) and zeroes their
// flags; per pair it writes the token's row of x, its exponent and the routed weight. Queue of
// XCD x (its nu units, local index l = u / 8): the up tiles of units 0 .. L - 1, then per unit
// l the up tiles of unit l + L and the down tiles of unit l, L = min(nu, lag): a unit's down
// tiles are handed out about a round of up tiles (lag units: the workgroups of an XCD over its
// NBU up tiles per unit, plus one) after its own up tiles, when those have mostly finished.
__global__ __launch_bounds__(1024) void k_ffn_plan(const int32_t *__restrict__ offsets, const int64_t *__restrict__ tab,
                                                   int E, int NBU, int NBD, int lmax, int zero_missing, int lag,
                                                   int *__restrict__ plan, int4 *__restrict__ list,
                                                   const int32_t *__restrict__ sorted_pos, int k,
                                                   const float *__restrict__ w, const int *__restrict__ xe,
                                                   int *__restrict__ xrow, float *__restrict__ wp,
                                                   int *__restrict__ xep) {
    __shared__ int s_w[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int U = 0;
    for (int pass = 0; pass < 2; ++pass) {
        int base = 0;  // units of the experts before this chunk (the same in every thread)
        for (int e0 = 0; e0 < E; e0 += 1024) {
            const int e = e0 + tid;
            const int ne = e < E ? offsets[e + 1] - offsets[e] : 0;
            const int np = (ne + 63) >> 6;
            int incl = np;
            for (int off = 1; off < 64; off <<= 1) {
                const int v = __shfl_up(incl, off, 64);
                if (lane >= off) incl += v;
            }
            // the wave's total written by every lane (no lane-divergent branch next to the barriers)
            s_w[wave] = __builtin_amdgcn_readlane(incl, 63);
            __syncthreads();
            int ub = base, tot = base;
            for (int w = 0; w < 16; ++w) {
                if (w < wave) ub += s_w[w];
                tot += s_w[w];
            }
            ub += incl - np;
            if (pass == 1 && np > 0) {
                const bool res = tab[4 * (size_t)e] != 0;
                const int fu = res ? 0 : FF_SKIP;
                const int fd = (int)(1u << 31) | (res ? 0 : (zero_missing ? FF_ZERO : FF_SKIP));
                for (int m = 0; m < np; ++m) {
                    const int u = ub + m, x = u & 7, l = u >> 3;
                    const int nu = (U - x + 7) >> 3, L = min(nu, lag);
                    // start of block b: the up tiles of unit b + L (if any), then the down tiles of unit b
                    auto blk = [&](int b) { return L * NBU + b * NBD + NBU * min(b, nu - L); };
                    const int up0 = l < L ? l * NBU : blk(l - L);
                    const int dn0 = blk(l) + (l + L < nu ? NBU : 0);
                    for (int nb = 0; nb < NBU; ++nb) plan[FP_DONE + u * NBU + nb] = 0;
                    int4 *q = list + (size_t)x * lmax * 2;
                    const int p0 = offsets[e] + m * GG_TOK, mn = min(GG_TOK, ne - m * GG_TOK);
                    for (int nb = 0; nb < NBU; ++nb) {
                        q[2 * (up0 + nb)] = make_int4(e, p0, mn, nb | fu);
                        q[2 * (up0 + nb) + 1] = make_int4(u, 0, 0, 0);
                    }
                    for (int nb = 0; nb < NBD; ++nb) {
                        q[2 * (dn0 + nb)] = make_int4(e, p0, mn, nb | fd);
                        q[2 * (dn0 + nb) + 1] = make_int4(u, 0, 0, 0);
                    }
                }
            }
            __syncthreads();  // s_w of the next chunk
            base = tot;
        }
        U = base;
    }
    // per pair (expert-sorted order): its token's row of x, that row's exponent, its routed weight
    const int np_all = offsets[E];
    for (int p = tid; p < np_all; p += 1024) {
        const int sp = sorted_pos[p], r = sp / k;
        xrow[p] = r;
        xep[p] = xe != nullptr ? xe[r] : 0;
        wp[p] = w[sp];
    }
    if (tid < 8) {
        const int nu = U > tid ? (U - tid + 7) >> 3 : 0;  // units u < U with u % 8 == tid
        plan[FP_TICK + FP_TSTRIDE * tid] = 0;
        plan[FP_TICK + FP_TSTRIDE * (8 + tid)] = nu * NBU;
        plan[FP_NALL + tid] = nu * (NBU + NBD);
        plan[FP_NUP + tid] = nu * NBU;
    }
    if (tid == 0) plan[FP_ERR] = 0;
}

struct FfnArgs {
    const uint16_t *x;  // fp16 activations (the caller's, or x16 of bf16 input)
    const int *xe;      // per-token exponents of x16, or null
    int H, I, k, NBU, NBD, lmax;
    const int32_t *offsets, *sorted_pos;
    const int64_t *tab;
    const float *w;     // routed weight of pair-slot t * k + j
    uint16_t *h16;      // (pairs, I) fp16 h, scaled by 2^-eb per (pair, up tile)
    int *hbe;           // (pairs, NBU) those exponents
    float *y;           // (pairs, H) fp32 expert outputs times the routed weight
    int *plan;
    const int4 *list;   // 2 int4 per entry
    const int *xrow;    // per pair: the token's row of x
    const int *xep;     // per pair: that row's exponent (0 without)
    const float *wp;    // per pair: the routed weight
    gu8 *dummy;         // FF_DUMMY bytes per workgroup, read by the loads past a pass's last chunk
    int phase;          // -1: the whole queue; 0: its up tiles; 1: its down tiles (after a phase-0 launch)
    DeqK dk;
};

__device__ __forceinline__ uint4 ld16_nt(const void *p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}


// activation staging of one pass: NT tokens (64, or 32 for a single 32-token M tile) over the
// 256 threads, TPT threads per token, VPT values each (NV 16-byte loads)
template <int CK, int NT> struct Stg {
    static constexpr int TPT = 256 / NT;
    static constexpr int VPT = CK / TPT;
    static constexpr int NV = VPT / 8;
};
// tokens staged for NMT M tiles of 16 (32 when that covers them and still gives 16 bytes per load)
template <int CK, int NMT> struct StgOf {
    static constexpr int NT = (NMT <= 2 && CK >= 64) ? 32 : 64;
};

// one activation chunk of a thread in registers (and, for h, its block exponent)
template <int CK, int NT> struct XStage {
    uint4 v[Stg<CK, NT>::NV];
    int eb;
};

template <int CK, int NT, bool DOWN>
__device__ __forceinline__ void stage_load(const uint16_t *row, const int *ebrow, int c, XStage<CK, NT> &s) {
    const uint16_t *p = row + (size_t)c * CK + (threadIdx.x % Stg<CK, NT>::TPT) * Stg<CK, NT>::VPT;
#pragma unroll
    for (int m = 0; m < Stg<CK, NT>::NV; ++m) s.v[m] = DOWN ? ld16_nt(p + 8 * m) : reinterpret_cast<const uint4 *>(p)[m];
    if constexpr (DOWN) s.eb = __builtin_nontemporal_load(ebrow + (c * CK) / 128);
}

template <int CK, int NT, bool DOWN>
__device__ __forceinline__ void stage_store(const XStage<CK, NT> &s, int emax, uint16_t *s_a) {
    const int tok = threadIdx.x / Stg<CK, NT>::TPT, part = threadIdx.x % Stg<CK, NT>::TPT;
    uint4 *dst = reinterpret_cast<uint4 *>(s_a + tok * GgChunk<CK>::LDA + part * Stg<CK, NT>::VPT);
    half2_t f2;
    if constexpr (DOWN) {
        const uint32_t fb = pow2_h(s.eb - emax);
        f2 = __builtin_bit_cast(half2_t, fb | (fb << 16));
    }
#pragma unroll
    for (int m = 0; m < Stg<CK, NT>::NV; ++m) {
        uint4 u = s.v[m];
        if constexpr (DOWN) {
            u.x = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, u.x) * f2);
            u.y = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, u.y) * f2);
            u.z = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, u.z) * f2);
            u.w = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, u.w) * f2);
        }
        dst[m] = make_uint4(lo_lo(u.x, u.z), hi_hi(u.x, u.z), lo_lo(u.y, u.w), hi_hi(u.y, u.w));
    }
}

// ---------------------------------------------------------------------------------------
// v_mfma_f32_16x16x32_f16 tiles: A = 16 tokens x 32 K (lane l: token l % 16, K 8 (l / 16) + e),
// B = 32 K x 16 weight rows (lane l: row l % 16, K 8 (l / 16) + e), D = 16 x 16 fp32 (lane l:
// tokens 4 (l / 16) + r, row l % 16). A wave holds 64 weight rows as 4 subtiles of 16. Per
// 64-byte chunk of a row, lane l loads bytes 16 (l / 16) .. + 15 (the four lanes of a row read
// its 64 bytes: one load instruction covers 16 rows x 64 contiguous bytes); step s of the
// chunk's CK / 32 MFMA steps takes the lane's s-th group of 8 values, i.e. K positions
// (CK / 4) (l / 16) + 8 s + (c0 c4 c1 c5 c2 c6 c3 c7), which is LDS block (CK / 32) (l / 16) + s
// of the staged activation rows (the same layout as the 32 x 32 tiles').
// ---------------------------------------------------------------------------------------
typedef float f32x4 __attribute__((ext_vector_type(4)));

// byte offsets (32-bit, from the field bases) of the lane's row data (bytes 16 q16 .. of each
// chunk) and of its scale, for `row` of K values
template <int PREC>
__device__ __forceinline__ void rows16(int row, int K, int q16, uint32_t &qo, uint32_t &so) {
    qo = (uint32_t)row * (uint32_t)(K * GgPrec<PREC>::BITS / 8) + 16u * q16;
    if constexpr (PREC == MOEHIP_PREC_INT4) so = (uint32_t)row * (K / GG_KG) * 2 + 2u * (q16 >> 1);
    else if constexpr (PREC == MOEHIP_PREC_INT8) so = (uint32_t)row * (K / GG_KG) * 2;
    else if constexpr (PREC == MOEHIP_PREC_FP8) so = (uint32_t)(row >> 7) * (K >> 7) * 4;
    else so = 0u;
}

struct WChunk16 {
    uint4 q[4];
    uint32_t s[4];
};

// chunk c at uniform field bases (qb, sb) + the lane's offsets; `live` false: the same loads at
// `dum` with offset 0 (the workgroup's own dummy lines)
template <int PREC>
__device__ __forceinline__ void load_chunk16(WChunk16 &w, gu8 *qb, gu8 *sb, const uint32_t (&qo)[4],
                                             const uint32_t (&so)[4], int c, bool live, gu8 *dum) {
    gu8 *qbase = live ? qb : dum;
    gu8 *sbase = live ? sb : dum;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t q = live ? qo[t] + (uint32_t)c * 64u : 0u;
        w.q[t] = gld16(qbase + q);
        uint32_t so2 = 0u;
        if constexpr (PREC == MOEHIP_PREC_INT4) so2 = so[t] + (uint32_t)c * 4u;
        else if constexpr (PREC == MOEHIP_PREC_INT8) so2 = so[t] + (uint32_t)c * 2u;
        else if constexpr (PREC == MOEHIP_PREC_FP8) so2 = so[t] + (uint32_t)(c >> 1) * 4u;
        so2 = live ? so2 : 0u;
        if constexpr (PREC == MOEHIP_PREC_INT4 || PREC == MOEHIP_PREC_INT8)
            w.s[t] = *(const __attribute__((address_space(1))) uint16_t *)(sbase + so2);
        else if constexpr (PREC == MOEHIP_PREC_FP8)
            w.s[t] = *(const __attribute__((address_space(1))) uint32_t *)(sbase + so2);
        else
            w.s[t] = 0u;
    }
}

// one chunk of MFMAs for a wave: CK / 32 steps x NMT token tiles x 4 subtiles. A step reads its
// A operands from LDS first, converts the 4 subtiles' weights while they arrive, then issues its
// MFMAs; the scheduler is kept from moving work across steps (which would hold more registers).
template <int PREC, int NMT>
__device__ __forceinline__ void mma_chunk16(const WChunk16 &w, const uint16_t *s_a, DeqK dk, f32x4 (&d)[4][4]) {
    constexpr int CK = GgPrec<PREC>::CK, S = CK / 32;
    const int lane = threadIdx.x & 63;
    const uint16_t *ap = s_a + (lane & 15) * GgChunk<CK>::LDA + 8 * S * (lane >> 4);
#pragma unroll
    for (int M = 0; M < S; ++M) {
        f16x8 a[4];
#pragma unroll
        for (int mt = 0; mt < NMT; ++mt) a[mt] = *reinterpret_cast<const f16x8 *>(ap + mt * 16 * GgChunk<CK>::LDA + 8 * M);
        f16x8 b[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint4 qq[2] = {w.q[t], w.q[t]};
            switch (M) {  // b_operand takes the step as a template argument
                case 0: b[t] = b_operand<PREC, 0>(qq, w.s[t], dk); break;
                case 1: b[t] = b_operand<PREC, (S > 1 ? 1 : 0)>(qq, w.s[t], dk); break;
                case 2: b[t] = b_operand<PREC, (S > 2 ? 2 : 0)>(qq, w.s[t], dk); break;
                default: b[t] = b_operand<PREC, (S > 3 ? 3 : 0)>(qq, w.s[t], dk); break;
            }
        }
#pragma unroll
        for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
            for (int t = 0; t < 4; ++t) d[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mt], b[t], d[mt][t], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Single-thread work of the persistent kernel (tickets, flags, waits) is done by wave 0 under a
// branch on the wave index made uniform by v_readfirstlane. A branch on threadIdx.x == 0 is
// lane-divergent: the compiler may then thread the other lanes of wave 0 past a later
// thread-0 block straight into the next barrier, splitting the wave around the ticket loop.
__device__ __forceinline__ bool ffn_wave0() { return uni((int)(threadIdx.x >> 6)) == 0; }

// An up tile's flag: a plain store once every store of the workgroup so far is acknowledged (the
// waiting down tiles run on the same XCD and poll its L2). Every lane of wave 0 writes the same
// word: one write, no lane-divergent branch.
__device__ __forceinline__ void ffn_flag(int *plan, int f) {
    if (ffn_wave0()) *reinterpret_cast<volatile int *>(plan + FP_DONE + f) = 1;
}
__device__ __forceinline__ void ffn_release_now(int *plan, int f) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    ffn_flag(plan, f);
}

// The K loop of one pass (RING = 2). Queue order: X0 W0 X1 W1 | X2 | per chunk c: X(c + 3),
// W(c + 2). Chunk c is in LDS buffer c % 2; X(c + 1) is stored during chunk c from the register
// set it was loaded into two chunks earlier. Every load is issued (the compiler can then count
// them); those past the last chunk read the workgroup's own lines at `dummy` (no weight or
// activation traffic). `rel` >= 0: the flag of the previous tile, set once the prologue has
// waited for its first activation chunk (every store issued before it by this workgroup is then
// acknowledged).
template <int PREC, int NMT, bool DOWN>
__device__ __forceinline__ void k_loop16(gu8 *qb, gu8 *sb, const uint32_t (&qo)[4], const uint32_t (&so)[4], int nch,
                                         const uint16_t *srcrow,
                                         const int *ebrow, int emax, uint16_t *s_a, DeqK dk, f32x4 (&d)[4][4],
                                         int *plan, int rel, gu8 *dummy) {
    constexpr int CK = GgPrec<PREC>::CK;
    constexpr int NT = StgOf<CK, NMT>::NT;
    constexpr int ABUF = GG_TOK * GgChunk<CK>::LDA;
    WChunk16 wr[2];
    XStage<CK, NT> xs[2];
    // this workgroup's own lines: a line shared by every workgroup would be a hot spot
    dummy += (size_t)(blockIdx.x % FF_DUMMY_WGS) * FF_DUMMY;
    const uint16_t *xdum = (const uint16_t *)(uintptr_t)dummy;
    const int *edum = (const int *)(uintptr_t)dummy;
    // chunk c of the weights / activations, or the dummy lines past the last chunk
    auto wload = [&](WChunk16 &w, int c) { load_chunk16<PREC>(w, qb, sb, qo, so, c, c < nch, dummy); };
    auto xload = [&](XStage<CK, NT> &x, int c) {
        const bool live = c < nch;
        stage_load<CK, NT, DOWN>(live ? srcrow : xdum, live ? ebrow : edum, live ? c : 0, x);
    };
    xload(xs[0], 0);
    wload(wr[0], 0);
    xload(xs[1], 1);
    wload(wr[1], 1);
    stage_store<CK, NT, DOWN>(xs[0], emax, s_a);
    xload(xs[0], 2);
    __syncthreads();
    if (rel >= 0) ffn_flag(plan, rel);
#pragma unroll 1
    for (int c0 = 0; c0 < nch; c0 += 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int c = c0 + u;
            if (c < nch) mma_chunk16<PREC, NMT>(wr[u], s_a + u * ABUF, dk, d);
            // the buffer of chunk c + 1 was last read before the previous barrier
            stage_store<CK, NT, DOWN>(xs[(u + 1) & 1], emax, s_a + ((u + 1) & 1) * ABUF);
            xload(xs[(u + 1) & 1], c + 3);
            wload(wr[u], c + 2);
            if (c < nch) __syncthreads();
        }
    }
}

// the 4 subtiles' K loop for NMT = ceil(tokens / 16) token tiles (a uniform switch)
template <int PREC, bool DOWN>
__device__ __forceinline__ void k_loop16_n(int nmt, gu8 *qb, gu8 *sb, const uint32_t (&qo)[4], const uint32_t (&so)[4],
                                           int nch,
                                           const uint16_t *src32, const int *eb32, int emax32,
                                           const uint16_t *src64, const int *eb64, int emax64, uint16_t *s_a, DeqK dk,
                                           f32x4 (&d)[4][4], int *plan, int rel, gu8 *dummy) {
    constexpr int CK = GgPrec<PREC>::CK;
#define FF_LOOP(N)                                                                                         \
    k_loop16<PREC, N, DOWN>(qb, sb, qo, so, nch, StgOf<CK, N>::NT == 32 ? src32 : src64,                   \
                            StgOf<CK, N>::NT == 32 ? eb32 : eb64, StgOf<CK, N>::NT == 32 ? emax32 : emax64, \
                            s_a, dk, d, plan, rel, dummy)
    if (nmt == 1) FF_LOOP(1);
    else if (nmt == 2) FF_LOOP(2);
    else if (nmt == 3) FF_LOOP(3);
    else FF_LOOP(4);
#undef FF_LOOP
}

// largest value over each aligned row of 16 lanes, in every lane of the row (v >= 0)
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    return fmaxf(v, dpp_f<0x140>(v));
}

template <int PREC>
struct FfnShared {
    uint16_t a[2 * GG_TOK * GgChunk<GgPrec<PREC>::CK>::LDA];
    float f[GG_TOK];
    int i[GG_TOK];
    float mx[4][GG_TOK];
    int t, ok;
};

// up tile: h columns nb * 128 + 32 w + 16 t + (lane % 16), t = 0, 1, of unit (e, m); subtiles
// 0, 1 = their gate rows, 2, 3 = their up rows. Its stores are released later (the caller passes
// its flag on as `rel`).
// the next tile's entry, read once the ticket taken at this tile's start is published (wave 0
// holds it in tn); the caller's loop ends at t >= nall
struct FfnNext {
    int t;
    int4 e0, e1;
};
template <int PREC>
__device__ __forceinline__ void ffn_next_publish(FfnShared<PREC> &sh, int tn) {
    if (ffn_wave0()) sh.t = uni(tn);
}
__device__ __forceinline__ void ffn_next_read(const FfnArgs &a, int t, int nall, int vx, FfnNext &nx) {
    nx.t = t;
    const int tc = t < nall ? t : 0;
    const int4 *q = a.list + ((size_t)vx * a.lmax + tc) * 2;
    nx.e0 = q[0];
    nx.e1 = q[1];
}

template <int PREC>
__device__ __forceinline__ void ffn_up(const FfnArgs &a, int4 en, int u, FfnShared<PREC> &sh, int rel, int tn,
                                       int nall, int vx, FfnNext &nx) {
    constexpr int CK = GgPrec<PREC>::CK;
    const int e = en.x, p0 = en.y, mn = en.z, nb = en.w & 0xffff;
    const int nmt = (mn + 15) >> 4;
    gu8 *qb = record_ptr(uni64(a.tab[4 * e + 0]));
    gu8 *sb = record_ptr(uni64(a.tab[4 * e + 1]));
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 15, g = lane >> 4;
    const int col0 = nb * 128 + 32 * wave;
    uint32_t qo[4], so[4];
    rows16<PREC>(col0 + j, a.H, g, qo[0], so[0]);
    rows16<PREC>(col0 + 16 + j, a.H, g, qo[1], so[1]);
    rows16<PREC>(a.I + col0 + j, a.H, g, qo[2], so[2]);
    rows16<PREC>(a.I + col0 + 16 + j, a.H, g, qo[3], so[3]);
    // the token of this thread for 64-token staging (tid / 4: also its exponent slot) and 32-token
    const int s64 = tid >> 2, s32 = tid >> 3;
    const int x64 = a.xrow[p0 + (s64 < mn ? s64 : 0)];
    const int x32 = a.xrow[p0 + (s32 < mn ? s32 : 0)];
    if ((tid & 3) == 0) sh.i[s64] = s64 < mn ? a.xep[p0 + s64] : 0;
    f32x4 d[4][4];
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
        for (int q = 0; q < 4; ++q) d[p][q] = f32x4{};
    k_loop16_n<PREC, false>(nmt, qb, sb, qo, so, a.H / CK, a.x + (size_t)x32 * a.H, nullptr, 0, a.x + (size_t)x64 * a.H,
                            nullptr, 0, sh.a, a.dk, d, a.plan, rel, a.dummy);
    ffn_next_publish(sh, tn);
    // h = silu(gate) * up with the token's 2^xe, then the largest |h| per token over the tile
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        if (mt >= nmt) break;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tok = 16 * mt + 4 * g + r;
            const float f = ldexpf(1.0f, sh.i[tok]);
            const float h0 = silu_mul(d[mt][0][r] * f, d[mt][2][r] * f);
            const float h1 = silu_mul(d[mt][1][r] * f, d[mt][3][r] * f);
            d[mt][0][r] = h0;
            d[mt][1][r] = h1;
            const float mx = row16_max(fmaxf(fabsf(h0), fabsf(h1)));
            if (j == 0) sh.mx[wave][tok] = mx;
        }
    }
    __syncthreads();
    ffn_next_read(a, uni(sh.t), nall, vx, nx);
    if (ffn_wave0()) {  // tid < GG_TOK
        const float mx = fmaxf(fmaxf(sh.mx[0][tid], sh.mx[1][tid]), fmaxf(sh.mx[2][tid], sh.mx[3][tid]));
        const int eb = row_exp(mx);
        sh.i[tid] = eb;
        if (tid < mn) a.hbe[(size_t)(p0 + tid) * a.NBU + nb] = eb;
    }
    __syncthreads();
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        if (mt >= nmt) break;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tok = 16 * mt + 4 * g + r;
            if (tok < mn) {
                const float sc = ldexpf(1.0f, -sh.i[tok]);
                uint16_t *hr = a.h16 + (size_t)(p0 + tok) * a.I + col0 + j;
                hr[0] = f32_to_f16_rne(d[mt][0][r] * sc);
                hr[16] = f32_to_f16_rne(d[mt][1][r] * sc);
            }
        }
    }
    // the tile's flag once its stores are acknowledged: the down tiles of the unit wait for it
    ffn_release_now(a.plan, u * a.NBU + nb);
}

// down tile: output rows nb * 256 + 64 w + 16 t + (lane % 16), t = 0 .. 3, of unit (e, m)
template <int PREC>
__device__ __forceinline__ void ffn_down(const FfnArgs &a, int4 en, int u, FfnShared<PREC> &sh, int tn, int nall,
                                         int vx, FfnNext &nx) {
    constexpr int CK = GgPrec<PREC>::CK;
    const int e = en.x, p0 = en.y, mn = en.z, nb = en.w & 0xffff;
    const int nmt = (mn + 15) >> 4;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 15, g = lane >> 4;
    if (en.w & FF_ZERO) {  // expert without a record: its pairs contribute nothing
        for (int i = tid; i < mn * GG_ROWS; i += 256)
            a.y[(size_t)(p0 + i / GG_ROWS) * a.H + nb * GG_ROWS + i % GG_ROWS] = 0.f;
        ffn_next_publish(sh, tn);
        __syncthreads();
        ffn_next_read(a, uni(sh.t), nall, vx, nx);
        return;
    }
    gu8 *qb = record_ptr(uni64(a.tab[4 * e + 2]));
    gu8 *sb = record_ptr(uni64(a.tab[4 * e + 3]));
    const int row0 = nb * GG_ROWS + 64 * wave;
    uint32_t qo[4], so[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) rows16<PREC>(row0 + 16 * t + j, a.I, g, qo[t], so[t]);
    if (ffn_wave0()) {  // lane nb polls the flag of up tile nb (non-temporal: through the XCD's L2)
        const int *fl = a.plan + FP_DONE + u * a.NBU + min(lane, a.NBU - 1);
        int ok = 0, nap = 1;
        for (int it = 0; it < FF_SPIN; ++it) {
            const int v = __builtin_nontemporal_load(fl);
            asm volatile("" ::: "memory");
            if (__builtin_amdgcn_ballot_w64(v != 1) == 0ull) {
                ok = 1;
                break;
            }
            backoff(nap, 2);
        }
        if (!ok) flag_error(reinterpret_cast<uint32_t *>(a.plan + FP_ERR));
        sh.ok = ok;
    }
    __syncthreads();
    const bool ok = sh.ok != 0;
    // per token (tid / 4): the largest block exponent of its h and w * 2^that; a 32-token staging
    // thread (tid / 8) reads the exponent of its token back from LDS
    const int s64 = tid >> 2, s32 = tid >> 3;
    const size_t pr = (size_t)(p0 + (s64 < mn ? s64 : 0));
    int emax = -1000;
    for (int c = 0; c < a.NBU; ++c) emax = max(emax, __builtin_nontemporal_load(a.hbe + pr * a.NBU + c));
    if ((tid & 3) == 0) {
        sh.i[s64] = emax;
        sh.f[s64] = !ok ? __builtin_nanf("") : (s64 < mn ? a.wp[pr] * ldexpf(1.0f, emax) : 0.f);
    }
    __syncthreads();
    const size_t p32 = (size_t)(p0 + (s32 < mn ? s32 : 0));
    f32x4 d[4][4];
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
        for (int q = 0; q < 4; ++q) d[p][q] = f32x4{};
    k_loop16_n<PREC, true>(nmt, qb, sb, qo, so, a.I / CK, a.h16 + p32 * a.I, a.hbe + p32 * a.NBU, sh.i[s32],
                           a.h16 + pr * a.I, a.hbe + pr * a.NBU, emax, sh.a, a.dk, d, a.plan, -1, a.dummy);
    ffn_next_publish(sh, tn);
    __syncthreads();
    ffn_next_read(a, uni(sh.t), nall, vx, nx);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        if (mt >= nmt) break;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tok = 16 * mt + 4 * g + r;
            if (tok >= mn) continue;
            const float f = sh.f[tok];
            float *yr = a.y + (size_t)(p0 + tok) * a.H + row0 + j;
#pragma unroll
            for (int t = 0; t < 4; ++t) yr[16 * t] = f * d[mt][t][r];
        }
    }
}

// Tickets are taken one tile ahead: wave 0 requests the next one when a tile starts (the whole
// wave runs the atomic, lane 0 adding 1) and passes it through LDS when the tile ends. No wait
// can deadlock: a down tile's up tiles are earlier in the queue, and the waiting workgroup with
// the earliest down tile waits only for tiles held (run or reserved) by workgroups whose current
// tiles are earlier still, none of them waiting. An up tile's release is deferred into the next
// tile's prologue; before a down tile (which may wait) or without a next K loop it is done at once.
template <int PREC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_ffn(FfnArgs a) {
    __shared__ __align__(16) FfnShared<PREC> sh;
    const int vx = blockIdx.x & 7;
    const int nall = a.phase == 0 ? a.plan[FP_NUP + vx] : a.plan[FP_NALL + vx];
    uint32_t *ctr = reinterpret_cast<uint32_t *>(a.plan + FP_TICK + FP_TSTRIDE * (a.phase == 1 ? 8 + vx : vx));
    const uint32_t one = (threadIdx.x & 63) == 0 ? 1u : 0u;
    if (ffn_wave0()) sh.t = uni((int)add_co32(ctr, one));
    __syncthreads();
    FfnNext cur;
    ffn_next_read(a, uni(sh.t), nall, vx, cur);
    int pend = -1;  // flag of this workgroup's last up tile, not yet set
    while (cur.t < nall) {
        __syncthreads();  // every thread has read sh.t
        int tn = 0;
        if (ffn_wave0()) tn = (int)add_co32(ctr, one);
        const int4 en = cur.e0;
        const int u = cur.e1.x;
        FfnNext nx;
        if (en.w >= 0 && (en.w & FF_SKIP) == 0) {
            ffn_up<PREC>(a, en, u, sh, -1, tn, nall, vx, nx);
        } else {
            if (pend >= 0) ffn_release_now(a.plan, pend);
            pend = -1;
            if ((en.w & FF_SKIP) == 0) {
                ffn_down<PREC>(a, en, u, sh, tn, nall, vx, nx);
            } else {
                ffn_next_publish(sh, tn);
                __syncthreads();
                ffn_next_read(a, uni(sh.t), nall, vx, nx);
            }
        }
        cur = nx;
    }
    if (pend >= 0) ffn_release_now(a.plan, pend);
}

// out[t] = sum over slots j (in order) of y[rank[t k + j]] (+ out if accumulate) (+ add):
// one workgroup per token, 8 consecutive columns per thread
template <int DT>
__global__ __launch_bounds__(256) void k_combine_pairs(const float *__restrict__ y, const int32_t *__restrict__ rank,
                                                       int T, int k, int H, const void *__restrict__ add,
                                                       void *__restrict__ out, int accumulate, int *__restrict__ clear,
                                                       int nclear, int cstride) {
    // token t, columns [blockIdx.y * 1024, + 1024): 4 per thread
    const int t = blockIdx.x, c0 = blockIdx.y * 1024 + threadIdx.x * 4;
    // words left zero for the next launch (a prefill layer's routing counters, read before this one)
    if (clear != nullptr && t == 0 && blockIdx.y == 0)
        for (int i = threadIdx.x; i < nclear; i += 256) clear[(size_t)i * cstride] = 0;
    if (c0 >= H) return;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    const int32_t *rk = rank + (size_t)t * k;
    // 8 slots at a time: their ranks, then their rows, all requested before any is added (a slot
    // past k or without a pair loads row 0 and is not added); the sums stay in slot order
    for (int j0 = 0; j0 < k; j0 += 8) {
        int p[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) p[u] = rk[min(j0 + u, k - 1)];
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = *reinterpret_cast<const float4 *>(y + (size_t)max(p[u], 0) * H + c0);
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (j0 + u < k && p[u] >= 0) s[0] += v[u].x, s[1] += v[u].y, s[2] += v[u].z, s[3] += v[u].w;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float o = s[q];
        if (accumulate) o += ld_act<DT>(out, (size_t)t * H + c0 + q);
        if (add != nullptr) o += ld_act<DT>(add, (size_t)t * H + c0 + q);
        st_act<DT>(out, (size_t)t * H + c0 + q, o);
    }
}

// ---------------------------------------------------------------------------------------
// Routing of a prefill chunk once its logits are in (16-bit activations, E <= 1024, k <= 32): one
// wave per token takes the softmax top-k (renormalised or not) exactly as moehip_router_topk,
// appends the token's slots to its experts' buckets (agent-scope counters: slot order within an
// expert depends on scheduling, the results do not, since every pair's products and every
// token's slot-order sum are independent of it), and for bf16 activations writes the fp16 copy
// of the token's row scaled by its power of two (the MFMA tiles' operand, as k_prep). The next
// launch (k_route_place) turns the buckets into the expert-sorted pair order of moehip_dispatch;
// the combine at the end of the layer leaves the counters at zero again.
// ---------------------------------------------------------------------------------------
constexpr int RP_MAXE = 1024;   // experts at most
constexpr int RP_STRIDE = 32;   // words between two experts' counters: a 128-byte line each (returning
                                // atomics on counters sharing lines queue on one memory channel)
constexpr int RP_DONE = RP_MAXE * RP_STRIDE;  // words of the counter area

// exclusive scan of v over the 256 threads of a workgroup (s: 4 words of LDS), total in tot
__device__ __forceinline__ int block_excl_scan256(int v, int *s, int &tot) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int incl = v;
    for (int off = 1; off < 64; off <<= 1) {
        const int o = __shfl_up(incl, off, 64);
        if (lane >= off) incl += o;
    }
    s[wave] = __builtin_amdgcn_readlane(incl, 63);
    __syncthreads();
    int base = 0;
    tot = 0;
    for (int w = 0; w < 4; ++w) {
        if (w < wave) base += s[w];
        tot += s[w];
    }
    __syncthreads();
    return base + incl - v;
}

template <int DT>
__global__ __launch_bounds__(256) void k_route_post(const void *__restrict__ logits, const uint16_t *__restrict__ x,
                                                    int T, int H, int E, int k, int renorm, int64_t *__restrict__ idx,
                                                    void *__restrict__ wout, float *__restrict__ w32,
                                                    int *__restrict__ cnt, int *__restrict__ bucket,
                                                    int *__restrict__ xe, uint16_t *__restrict__ x16, int prep) {
    __shared__ float s_p[4][32];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + wave;
    if (t < T) {  // the whole wave
        int myc;
        float p;
        topk_wave<DT>(logits, (size_t)t, E, k, renorm, s_p[wave], myc, p);
        if (lane < k) {
            const size_t q = (size_t)t * k + lane;
            idx[q] = myc;
            if (wout != nullptr) st_act<DT>(wout, q, p);
            w32[q] = rnd_act<DT>(p);
            const int r = (int)add_co32(reinterpret_cast<uint32_t *>(cnt + myc * RP_STRIDE), 1u);
            // r < T whenever the counters started at zero (each token takes an expert once); the
            // test keeps a corrupted counter from writing past the bucket
            if (r < T) bucket[(size_t)myc * T + r] = (int)q;
        }
        if (prep) {  // the token's row: fp16 with max |x| in [2^14, 2^15) (k_prep's rule)
            const uint4 *src = reinterpret_cast<const uint4 *>(x + (size_t)t * H);
            uint4 *dst = reinterpret_cast<uint4 *>(x16 + (size_t)t * H);
            float m = 0.f;
            for (int c = lane; c < H / 8; c += 64) {
                const uint4 v = src[c];
                const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) m = fmaxf(m, fmaxf(fabsf(bf16_lo(wd[i])), fabsf(bf16_hi(wd[i]))));
            }
            m = wave_max(m);
            const int e = row_exp(m);
            const float sc = ldexpf(1.0f, -e);
            for (int c = lane; c < H / 8; c += 64) {
                const uint4 v = src[c];
                dst[c] = make_uint4(pack_h2(bf16_lo(v.x) * sc, bf16_hi(v.x) * sc), pack_h2(bf16_lo(v.y) * sc, bf16_hi(v.y) * sc),
                                    pack_h2(bf16_lo(v.z) * sc, bf16_hi(v.z) * sc), pack_h2(bf16_lo(v.w) * sc, bf16_hi(v.w) * sc));
            }
            if (lane == 0) xe[t] = e;
        }
    }
}

// the expert-sorted pair order of moehip_dispatch from the buckets (counts, offsets, sorted_pos,
// rank): every workgroup scans the E counters (thread i holds experts 4 i .. 4 i + 3) and places
// its 256 positions, q belonging to the expert e with offsets[e] <= q < offsets[e + 1]
__global__ __launch_bounds__(256) void k_route_place(const int *__restrict__ cnt, const int *__restrict__ bucket,
                                                     int T, int k, int E, int32_t *__restrict__ counts,
                                                     int32_t *__restrict__ offsets, int32_t *__restrict__ sorted_pos,
                                                     int32_t *__restrict__ rank) {
    __shared__ int s_off[RP_MAXE + 1];
    __shared__ int s_scan[4];
    int c4[4], loc = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = 4 * threadIdx.x + i;
        c4[i] = e < E ? min(cnt[e * RP_STRIDE], T) : 0;
        loc += c4[i];
    }
    int total = 0;
    int run = block_excl_scan256(loc, s_scan, total);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = 4 * threadIdx.x + i;
        if (e < E) {
            s_off[e] = run;
            if (blockIdx.x == 0) {
                offsets[e] = run;
                counts[e] = c4[i];
            }
        }
        run += c4[i];
    }
    if (threadIdx.x == 0) {
        s_off[E] = total;
        if (blockIdx.x == 0) offsets[E] = total;
    }
    __syncthreads();
    const int q = blockIdx.x * 256 + threadIdx.x;
    if (q >= T * k) return;
    if (q >= total) {
        sorted_pos[q] = -1;
        return;
    }
    int lo = 0, hi = E;  // s_off[lo] <= q < s_off[hi]
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (s_off[mid] <= q) lo = mid;
        else hi = mid;
    }
    const int pr = bucket[(size_t)lo * T + (q - s_off[lo])];
    const bool ok = pr >= 0 && pr < T * k;
    sorted_pos[q] = ok ? pr : -1;
    if (ok) rank[pr] = q;
}

struct GgLayout {
    size_t xe, x16, h, h16, y, items, hbe, plan, list, pairs, dummy, total;
    int lmax;
};
static GgLayout gg_layout(int T, int k, int H, int I) {
    auto al = [](size_t v) { return (v + 255) / 256 * 256; };
    GgLayout L;
    const size_t NP = (size_t)T * k;
    size_t off = 0;
    L.xe = off;
    off = al(off + (size_t)T * 4);
    L.x16 = off;
    off = al(off + (size_t)T * H * 2);
    L.h = off;
    off = al(off + NP * I * 4);
    L.h16 = off;
    off = al(off + NP * I * 2);
    L.y = off;
    off = al(off + NP * H * 4);
    L.items = off;  // one work list per record precision
    off = al(off + (size_t)GV_MAXP * (NP + 1) * 4);
    // the block exponents of h (one per pair and 32 columns; the persistent FFN's one per 128),
    // the persistent FFN's plan words and tile queues
    const int NBU = I / 128, NBD = H / GG_ROWS;
    L.lmax = ffn_lmax((int)NP, NBU, NBD);
    L.hbe = off;
    off = al(off + NP * (I / 32) * 4);
    L.plan = off;
    off = al(off + (size_t)(FP_DONE + (size_t)ffn_max_units((int)NP) * max(NBU, 1)) * 4);
    L.list = off;
    off = al(off + (size_t)8 * L.lmax * 32);
    L.pairs = off;  // xrow, xep, wp: NP words each
    off = al(off + NP * 12);
    L.dummy = off;
    off = al(off + (size_t)FF_DUMMY_WGS * FF_DUMMY);
    L.total = off;
    return L;
}

}  // namespace moehip

using namespace moehip;

extern "C" size_t moehip_grouped_gemm_workspace_bytes(int T, int k, int H, int I) {
    if (T <= 0 || k <= 0 || H <= 0 || I <= 0) return 0;
    return gg_layout(T, k, H, I).total;
}

template <int PREC>
static void launch_up(dim3 g, hipStream_t st, const uint16_t *x, const int *xe, int H, int I, int k, int E,
                      const int32_t *offsets, const int32_t *sorted_pos, const int64_t *tab, uint16_t *h16, int *hbe,
                      DeqK dk) {
    hipLaunchKernelGGL((k_gemm_up<PREC>), g, dim3(256), 0, st, x, xe, H, I, k, E, offsets, sorted_pos, tab, h16, hbe, dk);
}
template <int PREC>
static void launch_down(dim3 g, hipStream_t st, const uint16_t *h16, const int *hbe, int H, int I, int E,
                        const int32_t *offsets, const int32_t *sorted_pos, const int64_t *tab, const float *w, float *y,
                        DeqK dk, int zero_missing) {
    hipLaunchKernelGGL((k_gemm_down<PREC>), g, dim3(256), 0, st, h16, hbe, H, I, E, offsets, sorted_pos, tab, w, y, dk,
                       zero_missing);
}

// the persistent FFN of one record table: plan, then one workgroup per CU slot (at most)
template <int PREC>
static int ffn_grid() {
    static int grid[64];  // per device, computed once
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (grid[dev] == 0) {
        int cus = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(k_ffn<PREC>), 256, 0) !=
                hipSuccess)
            return 0;
        grid[dev] = max(8, cus * per_cu / 8 * 8);
    }
    return grid[dev];
}

template <int PREC>
static void launch_ffn(hipStream_t st, FfnArgs a, const int64_t *tab, int E, int zero_missing) {
    a.tab = tab;
    const int grid = ffn_grid<PREC>();
    const bool one = getenv("MOEHIP_FFN_TWO_LAUNCHES") == nullptr;
    // one launch: a unit's down tiles a round of up tiles after its own; two: every up tile first
    int lag = one ? (grid / 8 + a.NBU - 1) / a.NBU + 1 : (1 << 30);
    if (const char *lv = getenv("MOEHIP_FFN_LAG")) lag = atoi(lv);
    hipLaunchKernelGGL(k_ffn_plan, dim3(1), dim3(1024), 0, st, a.offsets, tab, E, a.NBU, a.NBD, a.lmax, zero_missing,
                       lag, a.plan, const_cast<int4 *>(a.list), a.sorted_pos, a.k, a.w, a.xe,
                       const_cast<int *>(a.xrow), const_cast<float *>(a.wp), const_cast<int *>(a.xep));
    if (one) {
        a.phase = -1;
        hipLaunchKernelGGL(k_ffn<PREC>, dim3(grid), dim3(256), 0, st, a);
    } else {
        a.phase = 0;
        hipLaunchKernelGGL(k_ffn<PREC>, dim3(grid), dim3(256), 0, st, a);
        a.phase = 1;
        hipLaunchKernelGGL(k_ffn<PREC>, dim3(grid), dim3(256), 0, st, a);
    }
}

// batched GEMV launch geometry for rows of K values: G = 2^lg lanes per row, CPL chunks per lane,
// P passes per wave (gv_passes: P * CPL 16-byte loads per lane and matrix in flight)
struct GvGeo {
    int lg, cpl, p, rows_per_block;
};
// passes per wave: 4 / CPL, but 2 at one chunk per lane (int4 rows of up to 2048 values): four
// passes there held 140 registers (3 waves per SIMD), two hold 94 (5), and the extra waves hide
// more of each item's dependent loads (table, offsets, token) than the deeper ring did (OLMoE mixed
// bs=8 61.8 -> 59.2 us per layer, Qwen3-Next int4 bs=32 125.9 -> 120.0); and 1 for int4 rows of
// two chunks per lane (the wide gate/up rows below)
constexpr int gv_passes(int prec, int cpl) {
    return cpl >= 4 ? 1 : (cpl == 1 ? 2 : (prec == MOEHIP_PREC_INT4 ? 1 : 4 / cpl));
}
// wide: int4 gate/up rows of 2048 values on 32 lanes, two chunks each (one pass), not 64 lanes
// of one: Qwen3-Next int4 bs=32 119.8 -> 116.9 us per layer, OLMoE mixed bs=8 59.3 -> 57.1 (the
// int4 side of the two-precision up launch)
static GvGeo gv_geo(int prec, int K, bool wide = false) {
    const int vpc = prec == MOEHIP_PREC_INT4 ? 32 : ((prec == MOEHIP_PREC_INT8 || prec == MOEHIP_PREC_FP8) ? 16 : 8);
    const int C = K / vpc;
    int lg = 0;
    while ((1 << lg) < C && lg < 6) ++lg;
    if (wide && prec == MOEHIP_PREC_INT4 && C == 64) --lg;
    GvGeo g;
    g.lg = lg;
    g.cpl = (C + (1 << lg) - 1) >> lg;
    g.p = gv_passes(prec, g.cpl);
    g.rows_per_block = 4 * g.p * (64 >> lg);
    return g;
}

constexpr int GV_WG_BYTES = 128 << 10;  // weight bytes per workgroup at most
constexpr int GV_MIN_WGS = 2048;        // workgroups per launch at least (about two per CU slot)
// row groups per workgroup (ng) and row blocks per item (gx) of one precision's GEMV launch
static void gv_grid(int prec, bool up, int rows, int NP, const GvGeo &g, int H, int I, int &ng, int &gx) {
    // row groups per workgroup: up to 128 KiB of weights and GV_MAXROWS rows, while the pairs
    // (an upper bound of the work items) still give about two workgroups per CU slot
    const int groups = (rows + g.rows_per_block - 1) / g.rows_per_block;
    const int row_bytes = (up ? 2 : 1) * (up ? H : I) *
                          (prec == MOEHIP_PREC_INT4 ? 1 : (prec == MOEHIP_PREC_INT8 || prec == MOEHIP_PREC_FP8 ? 2 : 4)) / 2;
    ng = max(1, min(groups, GV_WG_BYTES / max(1, g.rows_per_block * row_bytes)));
    ng = max(1, min(ng, GV_MAXROWS / g.rows_per_block));
    ng = max(1, min(ng, groups * NP / GV_MIN_WGS));
    // row blocks per item a multiple of the 8 XCDs: workgroups are dealt to the XCDs round robin,
    // so row block b of every item (the items of one expert, one per token, are adjacent) then
    // runs on XCD b % 8 and the re-reads of its rows hit that XCD's L2
    gx = (groups + ng - 1) / ng;
    gx = (gx + 7) & ~7;
    ng = (groups + gx - 1) / gx;
    gx = (groups + ng - 1) / ng;
    gx = (gx + 7) & ~7;
}

template <int PREC, int CPL>
static void launch_gv_cpl(int mode, int rows, const int32_t *items, int NP, const GvGeo &g, hipStream_t st, const void *act, const int *ae,
                          int H, int I, int k, const int32_t *offsets, const int32_t *sorted_pos, const int64_t *tab,
                          float *out, const float *w, DeqK dk) {
    constexpr int P = gv_passes(PREC, CPL);
    int ng = 1, gx = 8;
    gv_grid(PREC, mode != 0, rows, NP, g, H, I, ng, gx);
    const dim3 grid(gx, NP);
    if (mode == 2)  // bf16 activations, scaled into fp16 per chunk by the kernel
        hipLaunchKernelGGL((k_gemv_up<PREC, CPL, P, true>), grid, dim3(256), 0, st, reinterpret_cast<const uint16_t *>(act),
                           nullptr, H, I, k, items, NP, offsets, sorted_pos, tab, out, dk, g.lg, ng);
    else if (mode == 1)
        hipLaunchKernelGGL((k_gemv_up<PREC, CPL, P, false>), grid, dim3(256), 0, st, reinterpret_cast<const uint16_t *>(act), ae,
                           H, I, k, items, NP, offsets,
                           sorted_pos, tab, out, dk, g.lg, ng);
    else
        hipLaunchKernelGGL((k_gemv_down<PREC, CPL, P>), grid, dim3(256), 0, st, reinterpret_cast<const float *>(act), H, I,
                           items, NP, offsets,
                           sorted_pos, tab, w, out, dk, g.lg, ng);
}

template <int PREC>
static void launch_gv(int mode, const int32_t *items, int NP, hipStream_t st, const void *act, const int *ae, int H, int I, int k,
                      const int32_t *offsets, const int32_t *sorted_pos, const int64_t *tab, float *out,
                      const float *w, DeqK dk) {
    const GvGeo g = gv_geo(PREC, mode != 0 ? H : I, mode != 0);
    const int rows = mode != 0 ? I : H;
    if (g.rows_per_block > GV_MAXROWS) return;  // unreachable for K >= 128 (checked by the caller)
    switch (g.cpl) {
        case 1: launch_gv_cpl<PREC, 1>(mode, rows, items, NP, g, st, act, ae, H, I, k, offsets, sorted_pos, tab, out, w, dk); break;
        case 2: launch_gv_cpl<PREC, 2>(mode, rows, items, NP, g, st, act, ae, H, I, k, offsets, sorted_pos, tab, out, w, dk); break;
        case 3:
        case 4: launch_gv_cpl<PREC, 4>(mode, rows, items, NP, g, st, act, ae, H, I, k, offsets, sorted_pos, tab, out, w, dk); break;
        default: launch_gv_cpl<PREC, 8>(mode, rows, items, NP, g, st, act, ae, H, I, k, offsets, sorted_pos, tab, out, w, dk); break;
    }
}

static void launch_gv_prec(int prec, int mode, const int32_t *items, int NP, hipStream_t st, const void *act, const int *ae, int H, int I,
                           int k, const int32_t *offsets, const int32_t *sorted_pos, const int64_t *tab, float *out,
                           const float *w, DeqK dk) {
    switch (prec) {
        case MOEHIP_PREC_INT4: launch_gv<MOEHIP_PREC_INT4>(mode, items, NP, st, act, ae, H, I, k, offsets, sorted_pos, tab, out, w, dk); break;
        case MOEHIP_PREC_INT8: launch_gv<MOEHIP_PREC_INT8>(mode, items, NP, st, act, ae, H, I, k, offsets, sorted_pos, tab, out, w, dk); break;
        case MOEHIP_PREC_FP8: launch_gv<MOEHIP_PREC_FP8>(mode, items, NP, st, act, ae, H, I, k, offsets, sorted_pos, tab, out, w, dk); break;
        case MOEHIP_PREC_F16: launch_gv<MOEHIP_PREC_F16>(mode, items, NP, st, act, ae, H, I, k, offsets, sorted_pos, tab, out, w, dk); break;
        default: launch_gv<MOEHIP_PREC_BF16>(mode, items, NP, st, act, ae, H, I, k, offsets, sorted_pos, tab, out, w, dk); break;
    }
}

// one launch for both precisions of a two-precision store, when the pair is one this library
// instantiates (a 16-bit record with int4 or int8, each with the chunks per lane its K gives);
// false: the caller launches per precision
template <int PA, int CA, int PB, int CB>
static void launch_gv2_t(int mode, const GvSide &a, const GvSide &b, int NP, hipStream_t st, const void *act, const int *ae,
                         int H, int I, int k, const int32_t *offsets, const int32_t *sorted_pos, float *out,
                         const float *w, DeqK dk) {
    constexpr int QA = gv_passes(PA, CA), QB = gv_passes(PB, CB);
    const dim3 grid(max(a.gx, b.gx), NP);
    if (mode == 2)
        hipLaunchKernelGGL((k_gemv_up2<PA, CA, QA, PB, CB, QB, true>), grid, dim3(256), 0, st,
                           reinterpret_cast<const uint16_t *>(act), nullptr, H, I, k, NP, offsets, sorted_pos, out, dk, a, b);
    else if (mode == 1)
        hipLaunchKernelGGL((k_gemv_up2<PA, CA, QA, PB, CB, QB, false>), grid, dim3(256), 0, st,
                           reinterpret_cast<const uint16_t *>(act), ae, H, I, k, NP, offsets, sorted_pos, out, dk, a, b);
    else
        hipLaunchKernelGGL((k_gemv_down2<PA, CA, QA, PB, CB, QB>), grid, dim3(256), 0, st,
                           reinterpret_cast<const float *>(act), H, I, NP, offsets, sorted_pos, w, out, dk, a, b);
}
static bool launch_gv2(const int *precs, int mode, const int32_t *items, int NP, hipStream_t st, const void *act,
                       const int *ae, int H, int I, int k, const int32_t *offsets, const int32_t *sorted_pos,
                       const int64_t *tabs, int E, float *out, const float *w, DeqK dk) {
    const int K = mode != 0 ? H : I, rows = mode != 0 ? I : H;
    const GvGeo g0 = gv_geo(precs[0], K), g1 = gv_geo(precs[1], K, mode != 0);
    if (g0.rows_per_block > GV_MAXROWS || g1.rows_per_block > GV_MAXROWS) return false;
    GvSide a{items, tabs, g0.lg, 1, 8}, b{items + (NP + 1), tabs + (size_t)E * 4, g1.lg, 1, 8};
    gv_grid(precs[0], mode != 0, rows, NP, g0, H, I, a.NG, a.gx);
    gv_grid(precs[1], mode != 0, rows, NP, g1, H, I, b.NG, b.gx);
    const bool p16 = precs[0] == MOEHIP_PREC_F16 || precs[0] == MOEHIP_PREC_BF16;
    if (!p16 || (precs[1] != MOEHIP_PREC_INT4 && precs[1] != MOEHIP_PREC_INT8)) return false;
    // (16-bit records: K = 2048 gives 4 chunks per lane, 1024 gives 2; int4 / int8: 1, and 2 for
    // the wide int4 gate/up rows)
    const bool w4 = g1.cpl == 2 && precs[1] == MOEHIP_PREC_INT4 && mode != 0;
    if ((g1.cpl != 1 && !w4) || (g0.cpl != 2 && g0.cpl != 4)) return false;
#define GV2(P0, C0, P1) launch_gv2_t<P0, C0, P1, 1>(mode, a, b, NP, st, act, ae, H, I, k, offsets, sorted_pos, out, w, dk)
#define GV2W(P0, C0, P1) launch_gv2_t<P0, C0, P1, 2>(mode, a, b, NP, st, act, ae, H, I, k, offsets, sorted_pos, out, w, dk)
    if (w4 && precs[0] == MOEHIP_PREC_F16) {
        if (g0.cpl == 4) GV2W(MOEHIP_PREC_F16, 4, MOEHIP_PREC_INT4); else GV2W(MOEHIP_PREC_F16, 2, MOEHIP_PREC_INT4);
    } else if (w4) {
        if (g0.cpl == 4) GV2W(MOEHIP_PREC_BF16, 4, MOEHIP_PREC_INT4); else GV2W(MOEHIP_PREC_BF16, 2, MOEHIP_PREC_INT4);
    } else if (precs[0] == MOEHIP_PREC_F16 && precs[1] == MOEHIP_PREC_INT4) {
        if (g0.cpl == 4) GV2(MOEHIP_PREC_F16, 4, MOEHIP_PREC_INT4); else GV2(MOEHIP_PREC_F16, 2, MOEHIP_PREC_INT4);
    } else if (precs[0] == MOEHIP_PREC_BF16 && precs[1] == MOEHIP_PREC_INT4) {
        if (g0.cpl == 4) GV2(MOEHIP_PREC_BF16, 4, MOEHIP_PREC_INT4); else GV2(MOEHIP_PREC_BF16, 2, MOEHIP_PREC_INT4);
    } else if (precs[0] == MOEHIP_PREC_F16 && precs[1] == MOEHIP_PREC_INT8) {
        if (g0.cpl == 4) GV2(MOEHIP_PREC_F16, 4, MOEHIP_PREC_INT8); else GV2(MOEHIP_PREC_F16, 2, MOEHIP_PREC_INT8);
    } else {
        if (g0.cpl == 4) GV2(MOEHIP_PREC_BF16, 4, MOEHIP_PREC_INT8); else GV2(MOEHIP_PREC_BF16, 2, MOEHIP_PREC_INT8);
    }
#undef GV2
#undef GV2W
    return true;
}

static bool gg_prec_ok(int prec) {
    return prec == MOEHIP_PREC_INT4 || prec == MOEHIP_PREC_INT8 || prec == MOEHIP_PREC_FP8 ||
           prec == MOEHIP_PREC_F16 || prec == MOEHIP_PREC_BF16;
}

// the layer on P record tables (one per precision, rows of experts not run at that precision 0)
static int gg_run(int P, const int *precs, const int64_t *tabs, const void *x, int xdtype, int T, int H, int I, int k,
                  int E, int gs, const int32_t *offsets, const int32_t *sorted_pos, const int32_t *rank, const float *w,
                  void *out, const void *add, int accumulate, void *ws, size_t ws_bytes, void *stream, int zero_missing,
                  int gemv, const int32_t *items_in = nullptr, bool x16_ready = false, int *clear = nullptr,
                  int nclear = 0, int cstride = 1) {
    MOEHIP_REQUIRE(tabs && x && offsets && sorted_pos && rank && w && out && ws && precs, "grouped_gemm: null pointer");
    MOEHIP_REQUIRE(P >= 1 && P <= 4, "grouped_gemm: %d record tables (1..4)", P);
    for (int p = 0; p < P; ++p) MOEHIP_REQUIRE(gg_prec_ok(precs[p]), "grouped_gemm: record precision %d", precs[p]);
    MOEHIP_REQUIRE(gs == GG_KG, "grouped_gemm: group size %d (64)", gs);
    MOEHIP_REQUIRE(T > 0 && k > 0 && E > 0 && H > 0 && I > 0 && H % GG_ROWS == 0 && I % 128 == 0,
                   "grouped_gemm: T=%d k=%d E=%d H=%d I=%d (H a multiple of 256, I of 128)", T, k, E, H, I);
    MOEHIP_REQUIRE(xdtype == MOEHIP_DT_F16 || xdtype == MOEHIP_DT_BF16, "grouped_gemm: activation dtype %d", xdtype);
    MOEHIP_REQUIRE(((uintptr_t)x % 16) == 0, "grouped_gemm: x must be 16-byte aligned");
    const GgLayout L = gg_layout(T, k, H, I);
    MOEHIP_REQUIRE(ws_bytes >= L.total && ((uintptr_t)ws % 256) == 0, "grouped_gemm: workspace %zu < %zu bytes (or unaligned)",
                   ws_bytes, L.total);
    uint8_t *wsb = reinterpret_cast<uint8_t *>(ws);
    int *xe = reinterpret_cast<int *>(wsb + L.xe);
    float *hb = reinterpret_cast<float *>(wsb + L.h);
    float *y = reinterpret_cast<float *>(wsb + L.y);
    const int NP = T * k;
    hipStream_t st = as_stream(stream);
    const int E8 = (E + 7) / 8 * 8;
    const dim3 gu(E8 * (I / 128)), gd(E8 * (H / GG_ROWS));
    const uint16_t *xs = reinterpret_cast<const uint16_t *>(x);
    uint16_t *x16 = reinterpret_cast<uint16_t *>(wsb + L.x16);
    const DeqK dk = {0x000F000Fu, 0x64006400u};
    const bool bf = xdtype == MOEHIP_DT_BF16;
    const uint16_t *xa = bf ? x16 : xs;
    const int *xea = bf ? xe : nullptr;
    // bf16 activations: fp16 with a per-token power of two for the MFMA tiles; the GEMVs read
    // the bf16 rows themselves and scale each chunk
    if (bf && !gemv && !x16_ready) hipLaunchKernelGGL(k_prep, dim3((T + 3) / 4), dim3(256), 0, st, xs, T, H, xe, x16);
    // MFMA tiles: the separate up / h / down launches below, or (MOEHIP_GEMM_FUSED set, where
    // workgroups are dealt to the XCDs round robin) the persistent FFN, one launch per record table
    const bool fused = !gemv && xcd_dispatch_ok() && getenv("MOEHIP_GEMM_FUSED") != nullptr;
    if (fused) {
        FfnArgs fa{};
        fa.x = xa;
        fa.xe = xea;
        fa.H = H;
        fa.I = I;
        fa.k = k;
        fa.NBU = I / 128;
        fa.NBD = H / GG_ROWS;
        fa.lmax = L.lmax;
        fa.offsets = offsets;
        fa.sorted_pos = sorted_pos;
        fa.w = w;
        fa.h16 = reinterpret_cast<uint16_t *>(wsb + L.h16);
        fa.hbe = reinterpret_cast<int *>(wsb + L.hbe);
        fa.y = y;
        fa.plan = reinterpret_cast<int *>(wsb + L.plan);
        fa.list = reinterpret_cast<const int4 *>(wsb + L.list);
        fa.dummy = (gu8 *)(uintptr_t)(wsb + L.dummy);
        fa.xrow = reinterpret_cast<const int *>(wsb + L.pairs);
        fa.xep = reinterpret_cast<const int *>(wsb + L.pairs + (size_t)NP * 4);
        fa.wp = reinterpret_cast<const float *>(wsb + L.pairs + (size_t)NP * 8);
        fa.dk = dk;
        for (int p = 0; p < P; ++p) {
            const int64_t *tab = tabs + (size_t)p * E * 4;
            const int zm = zero_missing && P == 1;
            switch (precs[p]) {
                case MOEHIP_PREC_INT4: launch_ffn<MOEHIP_PREC_INT4>(st, fa, tab, E, zm); break;
                case MOEHIP_PREC_INT8: launch_ffn<MOEHIP_PREC_INT8>(st, fa, tab, E, zm); break;
                case MOEHIP_PREC_FP8: launch_ffn<MOEHIP_PREC_FP8>(st, fa, tab, E, zm); break;
                case MOEHIP_PREC_F16: launch_ffn<MOEHIP_PREC_F16>(st, fa, tab, E, zm); break;
                default: launch_ffn<MOEHIP_PREC_BF16>(st, fa, tab, E, zm); break;
            }
        }
    }
    // the work list: the caller's (written by moehip_batch_route_decide) or built here
    int32_t *items = reinterpret_cast<int32_t *>(wsb + L.items);
    if (gemv && items_in == nullptr)
        hipLaunchKernelGGL(k_gv_items, dim3(1), dim3(1024), 0, st, offsets, E, NP, tabs, P, items);
    if (items_in != nullptr) items = const_cast<int32_t *>(items_in);
    // a two-precision store: both precisions in one up and one down launch where the pair is instantiated
    const bool two = gemv && P == 2 &&
                     launch_gv2(precs, bf ? 2 : 1, items, NP, st, bf ? xs : xa, bf ? nullptr : xea, H, I, k, offsets,
                                sorted_pos, tabs, E, hb, nullptr, dk);
    for (int p = 0; p < P && gemv && !two; ++p)
        launch_gv_prec(precs[p], bf ? 2 : 1, items + (size_t)p * (NP + 1), NP, st, bf ? xs : xa, bf ? nullptr : xea, H, I, k, offsets, sorted_pos, tabs + (size_t)p * E * 4, hb, nullptr,
                       dk);
    // the MFMA up tiles write h as fp16 with a power of two per (pair, 32 columns); the GEMVs fp32
    uint16_t *h16 = reinterpret_cast<uint16_t *>(wsb + L.h16);
    int *hbe = reinterpret_cast<int *>(wsb + L.hbe);
    for (int p = 0; p < P && !gemv && !fused; ++p) {
        const int64_t *tab = tabs + (size_t)p * E * 4;
        switch (precs[p]) {
            case MOEHIP_PREC_INT4: launch_up<MOEHIP_PREC_INT4>(gu, st, xa, xea, H, I, k, E, offsets, sorted_pos, tab, h16, hbe, dk); break;
            case MOEHIP_PREC_INT8: launch_up<MOEHIP_PREC_INT8>(gu, st, xa, xea, H, I, k, E, offsets, sorted_pos, tab, h16, hbe, dk); break;
            case MOEHIP_PREC_FP8: launch_up<MOEHIP_PREC_FP8>(gu, st, xa, xea, H, I, k, E, offsets, sorted_pos, tab, h16, hbe, dk); break;
            case MOEHIP_PREC_F16: launch_up<MOEHIP_PREC_F16>(gu, st, xa, xea, H, I, k, E, offsets, sorted_pos, tab, h16, hbe, dk); break;
            default: launch_up<MOEHIP_PREC_BF16>(gu, st, xa, xea, H, I, k, E, offsets, sorted_pos, tab, h16, hbe, dk); break;
        }
    }
    if (two) launch_gv2(precs, 0, items, NP, st, hb, nullptr, H, I, k, offsets, sorted_pos, tabs, E, y, w, dk);
    for (int p = 0; p < P && gemv && !two; ++p)
        launch_gv_prec(precs[p], 0, items + (size_t)p * (NP + 1), NP, st, hb, nullptr, H, I, k, offsets, sorted_pos, tabs + (size_t)p * E * 4,
                       y, w, dk);
    for (int p = 0; p < P && !gemv && !fused; ++p) {
        const int64_t *tab = tabs + (size_t)p * E * 4;
        const int zm = zero_missing && P == 1;
        switch (precs[p]) {
            case MOEHIP_PREC_INT4: launch_down<MOEHIP_PREC_INT4>(gd, st, h16, hbe, H, I, E, offsets, sorted_pos, tab, w, y, dk, zm); break;
            case MOEHIP_PREC_INT8: launch_down<MOEHIP_PREC_INT8>(gd, st, h16, hbe, H, I, E, offsets, sorted_pos, tab, w, y, dk, zm); break;
            case MOEHIP_PREC_FP8: launch_down<MOEHIP_PREC_FP8>(gd, st, h16, hbe, H, I, E, offsets, sorted_pos, tab, w, y, dk, zm); break;
            case MOEHIP_PREC_F16: launch_down<MOEHIP_PREC_F16>(gd, st, h16, hbe, H, I, E, offsets, sorted_pos, tab, w, y, dk, zm); break;
            default: launch_down<MOEHIP_PREC_BF16>(gd, st, h16, hbe, H, I, E, offsets, sorted_pos, tab, w, y, dk, zm); break;
        }
    }
    if (xdtype == MOEHIP_DT_F16)
        hipLaunchKernelGGL((k_combine_pairs<MOEHIP_DT_F16>), dim3(T, (H + 1023) / 1024), dim3(256), 0, st, y, rank, T, k, H, add, out,
                           accumulate, clear, nclear, cstride);
    else
        hipLaunchKernelGGL((k_combine_pairs<MOEHIP_DT_BF16>), dim3(T, (H + 1023) / 1024), dim3(256), 0, st, y, rank, T, k, H, add, out,
                           accumulate, clear, nclear, cstride);
    return check_launch("grouped_gemm");
}

extern "C" int moehip_grouped_gemm(int prec, const int64_t *tab, const void *x, int xdtype, int T, int H, int I, int k,
                                   int E, int gs, const int32_t *offsets, const int32_t *sorted_pos,
                                   const int32_t *rank, const float *w, void *out, const void *add, int accumulate,
                                   void *ws, size_t ws_bytes, void *stream) {
    return gg_run(1, &prec, tab, x, xdtype, T, H, I, k, E, gs, offsets, sorted_pos, rank, w, out, add, accumulate, ws,
                  ws_bytes, stream, 1, 0);
}

// A prefill layer's workspace: the routing counters at offset 0 (zero at first use; every launch
// leaves them zero; at a fixed place whatever the chunk's length), the buckets, counts, offsets,
// sorted_pos and rank of the chunk, then the grouped GEMM's workspace
struct RpLayout {
    size_t cnt, bucket, counts, offsets, sorted, rank, gg, total;
};
static RpLayout rp_layout(int T, int k, int H, int I, int E) {
    auto al = [](size_t v) { return (v + 255) / 256 * 256; };
    RpLayout L;
    size_t off = 0;
    L.cnt = off;
    off = al(off + (RP_DONE + 64) * 4);
    L.bucket = off;
    off = al(off + (size_t)E * T * 4);
    L.counts = off;
    off = al(off + (size_t)E * 4);
    L.offsets = off;
    off = al(off + (size_t)(E + 1) * 4);
    L.sorted = off;
    off = al(off + (size_t)T * k * 4);
    L.rank = off;
    off = al(off + (size_t)T * k * 4);
    L.gg = off;
    off = al(off + gg_layout(T, k, H, I).total);
    L.total = off;
    return L;
}

extern "C" size_t moehip_prefill_layer_workspace_bytes(int T, int k, int H, int I, int E) {
    if (T <= 0 || k <= 0 || H <= 0 || I <= 0 || E <= 0) return 0;
    return rp_layout(T, k, H, I, E).total;
}

extern "C" int moehip_prefill_layer(int prec, const int64_t *tab, const void *x, const void *Wr, int xdtype, int T,
                                    int H, int I, int k, int E, int gs, int renorm, void *logits, int64_t *idx,
                                    void *w, float *w32, void *out, const void *add, int accumulate, void *ws,
                                    size_t ws_bytes, void *stream) {
    MOEHIP_REQUIRE(tab && x && Wr && logits && idx && w32 && out && ws, "prefill_layer: null pointer");
    MOEHIP_REQUIRE(xdtype == MOEHIP_DT_F16 || xdtype == MOEHIP_DT_BF16, "prefill_layer: activation dtype %d", xdtype);
    MOEHIP_REQUIRE(T > 0 && E > 0 && E <= RP_MAXE && k > 0 && k <= 32 && k <= E && H % 512 == 0 && H % GG_ROWS == 0 &&
                       I % 128 == 0,
                   "prefill_layer: T=%d E=%d k=%d H=%d I=%d (E <= 1024, k <= 32, H a multiple of 512, I of 128)", T, E,
                   k, H, I);
    MOEHIP_REQUIRE(((uintptr_t)x % 16) == 0 && ((uintptr_t)Wr % 16) == 0, "prefill_layer: x and Wr must be 16-byte aligned");
    // everything the grouped GEMM checks is checked here, before the routing launches bump the
    // per-expert counters (only this call's combine clears them again)
    MOEHIP_REQUIRE(gg_prec_ok(prec), "prefill_layer: record precision %d", prec);
    MOEHIP_REQUIRE(gs == GG_KG, "prefill_layer: group size %d (64)", gs);
    const RpLayout R = rp_layout(T, k, H, I, E);
    const GgLayout G = gg_layout(T, k, H, I);
    MOEHIP_REQUIRE(ws_bytes >= R.total && ((uintptr_t)ws % 256) == 0, "prefill_layer: workspace %zu < %zu bytes (or unaligned)",
                   ws_bytes, R.total);
    hipStream_t st = as_stream(stream);
    uint8_t *wsb = reinterpret_cast<uint8_t *>(ws);
    uint8_t *wgg = wsb + R.gg;  // the grouped GEMM's workspace (its x16 / xe written by the routing launch)
    launch_router_logits(x, Wr, T, H, E, xdtype, logits, st);
    int *cnt = reinterpret_cast<int *>(wsb + R.cnt);
    int *bucket = reinterpret_cast<int *>(wsb + R.bucket);
    int32_t *counts = reinterpret_cast<int32_t *>(wsb + R.counts);
    int32_t *offsets = reinterpret_cast<int32_t *>(wsb + R.offsets);
    int32_t *sorted = reinterpret_cast<int32_t *>(wsb + R.sorted);
    int32_t *rank = reinterpret_cast<int32_t *>(wsb + R.rank);
    int *xe = reinterpret_cast<int *>(wgg + G.xe);
    uint16_t *x16 = reinterpret_cast<uint16_t *>(wgg + G.x16);
    const uint16_t *xs = reinterpret_cast<const uint16_t *>(x);
    const int prep = xdtype == MOEHIP_DT_BF16;
    const dim3 grid((T + 3) / 4);
    if (xdtype == MOEHIP_DT_F16)
        hipLaunchKernelGGL((k_route_post<MOEHIP_DT_F16>), grid, dim3(256), 0, st, logits, xs, T, H, E, k, renorm, idx, w,
                           w32, cnt, bucket, xe, x16, prep);
    else
        hipLaunchKernelGGL((k_route_post<MOEHIP_DT_BF16>), grid, dim3(256), 0, st, logits, xs, T, H, E, k, renorm, idx, w,
                           w32, cnt, bucket, xe, x16, prep);
    hipLaunchKernelGGL(k_route_place, dim3((T * k + 255) / 256), dim3(256), 0, st, cnt, bucket, T, k, E, counts, offsets,
                       sorted, rank);
    // the combine (after every reader of the counters) leaves them zero
    return gg_run(1, &prec, tab, x, xdtype, T, H, I, k, E, gs, offsets, sorted, rank, w32, out, add, accumulate, wgg,
                  G.total, stream, 1, 0, nullptr, true, cnt, E, RP_STRIDE);
}

extern "C" int moehip_grouped_gemm_multi(int P, const int *precs, const int64_t *tabs, const void *x, int xdtype, int T,
                                         int H, int I, int k, int E, int gs, const int32_t *offsets,
                                         const int32_t *sorted_pos, const int32_t *rank, const float *w, void *out,
                                         const void *add, int accumulate, void *ws, size_t ws_bytes, void *stream) {
    return gg_run(P, precs, tabs, x, xdtype, T, H, I, k, E, gs, offsets, sorted_pos, rank, w, out, add, accumulate, ws,
                  ws_bytes, stream, 0, 0);
}

extern "C" int moehip_grouped_gemv_multi(int P, const int *precs, const int64_t *tabs, const void *x, int xdtype, int T,
                                         int H, int I, int k, int E, int gs, const int32_t *offsets,
                                         const int32_t *sorted_pos, const int32_t *rank, const float *w, void *out,
                                         const void *add, int accumulate, void *ws, size_t ws_bytes,
                                         const int32_t *items, void *stream) {
    MOEHIP_REQUIRE(T <= 256 * GV_TOKENS, "grouped_gemv: %d tokens (an expert's work items are numbered in 8 bits: <= %d)",
                   T, 256 * GV_TOKENS);
    return gg_run(P, precs, tabs, x, xdtype, T, H, I, k, E, gs, offsets, sorted_pos, rank, w, out, add, accumulate, ws,
                  ws_bytes, stream, 0, 1, items);
}
