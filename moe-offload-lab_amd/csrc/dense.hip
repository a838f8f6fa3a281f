// The dense part in int8 (attention projections, shared experts, the LM head): one-token GEMV and
// the row-block dequantisation of the multi-token path. Weights (O, K) int8, group scales (O, K/gs)
// fp16, symmetric (the store's int8 format).

#include "lanevec.hpp"

namespace moehip {

// ---------------------------------------------------------------------------------------
// y (O) = W x, one token. Lane groups of G = 2^lg lanes per row; a lane holds CPL chunks of 16
// int8 values (32 values) of a row segment of G * 32 values; NP row passes per wave, every
// weight and scale load of a segment issued before the first product; fp16 pairs and the
// 1024-offset dot (fp32 accumulation), the group scale per chunk. Rows and chunks past the end
// read valid memory and are dropped.
// ---------------------------------------------------------------------------------------
template <int XDT, int G8_NP>
__global__ __launch_bounds__(256) void k_gemv8(gbyte *q, gbyte *s, const void *x, void *y, int O, int K, int gs,
                                               int lg, int nseg) {
    constexpr int PREC = MOEHIP_PREC_INT8;
    constexpr int CPL = DlFmt<PREC>::CPL, VPC = DlFmt<PREC>::VPC;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int G = 1 << lg, RPW = 64 >> lg;
    const int slot = lane >> lg, cl = lane & (G - 1);
    const int C = K / VPC;                     // chunks per row
    const int CS = G * CPL;                    // chunks per segment
    const uint32_t RB = (uint32_t)K;           // bytes per row
    const int ng = K / gs;
    const int r0 = (blockIdx.x * 4 + wave) * RPW * G8_NP + slot;  // row of pass 0
    float acc[G8_NP];
#pragma unroll
    for (int p = 0; p < G8_NP; ++p) acc[p] = 0.f;
    for (int sg = 0; sg < nseg; ++sg) {
        const int c0 = sg * CS;  // first chunk of the segment
        uint4 qd[G8_NP][CPL];
        uint32_t sd[G8_NP][CPL];
        uint32_t okm = 0;
#pragma unroll
        for (int p = 0; p < G8_NP; ++p) {
            const int rr = r0 + p * RPW;
            const int r = min(rr, O - 1);
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const int cc = c0 + cl + i * G;
                const int c = min(cc, C - 1);
                okm |= (cc < C && rr < O ? 1u : 0u) << (p * CPL + i);
                qd[p][i] = gld16(q + (size_t)r * RB + (size_t)c * 16);
                sd[p][i] = gld2(s + 2 * ((size_t)r * ng + (c * VPC) / gs));
            }
        }
        LaneVec<PREC, XDT> lv;
        load_x<PREC, XDT>(reinterpret_cast<const uint8_t *>(x) + (size_t)c0 * VPC * (XDT == MOEHIP_DT_F32 ? 4 : 2),
                          cl, G, C - c0, lv);
#pragma unroll
        for (int p = 0; p < G8_NP; ++p)
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const float sc = ((okm >> (p * CPL + i)) & 1u) ? f16_to_f32(sd[p][i]) : 0.f;
                acc[p] = fmaf(sc * lv.p2e[i], lane_dot<PREC, XDT>(qd[p][i], lv, i), acc[p]);
            }
    }
    grp_total_n<G8_NP>(acc, lg);
    if (cl == G - 1)
#pragma unroll
        for (int p = 0; p < G8_NP; ++p) {
            const int r = r0 + p * RPW;
            if (r < O) st_act<XDT>(y, r, acc[p]);
        }
}

// ---------------------------------------------------------------------------------------
// W (rows [r0, r0 + n), K) in the activation dtype: q * round(s), rounded once (as the store's
// dequantisation in that dtype); 16 values per thread
// ---------------------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void k_dequant8(gbyte *q, gbyte *s, int n, int K, int gs, void *w) {
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t nchunk = (size_t)n * (K / 16);
    if (t >= nchunk) return;
    const size_t r = t / (size_t)(K / 16);
    const int c = (int)(t - r * (size_t)(K / 16));
    const uint4 v = gld16(q + t * 16);
    const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
    const int ng = K / gs;
    float out[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int col = c * 16 + j;
        float sc = f16_to_f32(gld2(s + 2 * (r * ng + col / gs)));
        if constexpr (DT == MOEHIP_DT_BF16) sc = rnd_act<MOEHIP_DT_BF16>(sc);
        const int qv = (int)(int8_t)((wd[j >> 2] >> (8 * (j & 3))) & 0xffu);
        out[j] = (float)qv * sc;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) st_act<DT>(w, (size_t)r * K + (size_t)c * 16 + j, out[j]);
}

}  // namespace moehip

using namespace moehip;

static bool dense_dt(int d) { return d >= MOEHIP_DT_F16 && d <= MOEHIP_DT_F32; }

extern "C" int moehip_dense_gemv_int8(const void *q, const void *s, const void *x, void *y, int O, int K, int gs,
                                      int dtype, void *stream) {
    MOEHIP_REQUIRE(q && s && x && y, "dense_gemv_int8: null pointer");
    MOEHIP_REQUIRE(dense_dt(dtype), "dense_gemv_int8: bad dtype %d", dtype);
    MOEHIP_REQUIRE(O > 0 && K > 0 && K % 32 == 0 && gs > 0 && gs % 16 == 0 && K % gs == 0,
                   "dense_gemv_int8: O=%d K=%d gs=%d (K a multiple of 32, gs of 16 dividing K)", O, K, gs);
    MOEHIP_REQUIRE(((uintptr_t)q % 16) == 0 && ((uintptr_t)x % 16) == 0,
                   "dense_gemv_int8: q and x must be 16-byte aligned");
    const int chunks = K / 16, cpl = 2;
    int G = 1, lg = 0;
    while (G < (chunks + cpl - 1) / cpl && G < 64) G <<= 1, ++lg;
    const int nseg = (chunks + G * cpl - 1) / (G * cpl);
    // row passes per wave: 4, unless the grid would then hold fewer than 2 workgroups per CU (a
    // small matrix: an attention projection, a shared expert), where 2 or 1 give more workgroups
    int cus = 256;
    {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            n > 0)
            cus = n;
    }
    int np = 1;
    for (int cand : {4, 2})
        if ((O + 4 * (64 >> lg) * cand - 1) / (4 * (64 >> lg) * cand) >= 2 * cus) {
            np = cand;
            break;
        }
    const int rows_per_block = 4 * (64 >> lg) * np;
    const dim3 grid((unsigned)((O + rows_per_block - 1) / rows_per_block));
    hipStream_t st = as_stream(stream);
    gbyte *qb = (gbyte *)(uintptr_t)q, *sb = (gbyte *)(uintptr_t)s;
#define G8_LAUNCH(DT, NP) hipLaunchKernelGGL((k_gemv8<DT, NP>), grid, dim3(256), 0, st, qb, sb, x, y, O, K, gs, lg, nseg)
#define G8_NPS(DT)           \
    if (np == 4)             \
        G8_LAUNCH(DT, 4);    \
    else if (np == 2)        \
        G8_LAUNCH(DT, 2);    \
    else                     \
        G8_LAUNCH(DT, 1)
    switch (dtype) {
        case MOEHIP_DT_F16: G8_NPS(MOEHIP_DT_F16); break;
        case MOEHIP_DT_BF16: G8_NPS(MOEHIP_DT_BF16); break;
        default: G8_NPS(MOEHIP_DT_F32); break;
    }
#undef G8_NPS
#undef G8_LAUNCH
    return check_launch("dense_gemv_int8");
}

extern "C" int moehip_dense_dequant_int8(const void *q, const void *s, int rows, int K, int gs, int dtype, void *w,
                                         void *stream) {
    MOEHIP_REQUIRE(q && s && w, "dense_dequant_int8: null pointer");
    MOEHIP_REQUIRE(dense_dt(dtype), "dense_dequant_int8: bad dtype %d", dtype);
    MOEHIP_REQUIRE(rows > 0 && K > 0 && K % 16 == 0 && gs > 0 && K % gs == 0,
                   "dense_dequant_int8: rows=%d K=%d gs=%d (K a multiple of 16)", rows, K, gs);
    MOEHIP_REQUIRE(((uintptr_t)q % 16) == 0, "dense_dequant_int8: q must be 16-byte aligned");
    const size_t nchunk = (size_t)rows * (K / 16);
    const dim3 grid((unsigned)((nchunk + 255) / 256));
    hipStream_t st = as_stream(stream);
    gbyte *qb = (gbyte *)(uintptr_t)q, *sb = (gbyte *)(uintptr_t)s;
    switch (dtype) {
        case MOEHIP_DT_F16: hipLaunchKernelGGL(k_dequant8<MOEHIP_DT_F16>, grid, dim3(256), 0, st, qb, sb, rows, K, gs, w); break;
        case MOEHIP_DT_BF16: hipLaunchKernelGGL(k_dequant8<MOEHIP_DT_BF16>, grid, dim3(256), 0, st, qb, sb, rows, K, gs, w); break;
        default: hipLaunchKernelGGL(k_dequant8<MOEHIP_DT_F32>, grid, dim3(256), 0, st, qb, sb, rows, K, gs, w); break;
    }
    return check_launch("dense_dequant_int8");
}
