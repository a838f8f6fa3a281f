// Grouped expert FFN for decode (one activation row): dequant-fused GEMV kernels.
//
// Data layout (the store's record format, moelab/store.py:76-115): for each table row e,
// tab[4e+0..3] = device addresses of [gate_up.q, gate_up.s, down.q, down.s]. A weight row is
// streamed as 16-byte chunks; a chunk holds VPC values (int4: 32, int8/fp8: 16, f16/bf16: 8,
// f32: 4) and always lies inside one scale group (int: gs % VPC == 0; fp8: 128-column blocks).
//
// Lane mapping: a row of C chunks is handled by G = min(64, pow2ceil(C)) lanes, each lane owning
// chunks cl, cl+G, ... (CPL of them). A wave therefore covers RPW = 64/G rows per pass and P
// passes; all 16-byte loads of the P passes are issued before any is consumed, so every lane has
// 2P (up) or P (down) loads in flight. The lane's slice of the vector (x for kernel A, h[e] for
// kernel B) is converted to fp32 once and kept in registers for all its rows.
//
// Nibble -> value: int4 bytes hold (q+8) | (q'+8) << 4 (moelab/quant.py:96-101). A dword of
// 8 nibbles is masked into two dwords of 4 bytes each, converted with the unsigned byte
// converts, and the +8 offset is removed once per chunk as -8 * sum(vector slice).
//
// Determinism: kernel B writes per-expert partial rows; the reduce kernel adds them in table
// order (moelab's v1 kernel order, kernels.py:132-146), so results do not depend on scheduling.

#include "gemv_core.hpp"

namespace moehip {

// ---------------------------------------------------------------------------------------
// kernel A (fast path): h[e, r] = silu(gate_e[r] . x) * (up_e[r] . x)
// grid (ceil(I / rows_per_block), n), block 256
// ---------------------------------------------------------------------------------------
template <int PREC, int XDT, int CPL, int P>
__global__ __launch_bounds__(256) void k_up(const int64_t *__restrict__ tab, const float *__restrict__ w,
                                            const void *__restrict__ x, float *__restrict__ h,
                                            float *__restrict__ acc_zero, int I, int H, int gs, int lg) {
    constexpr int VPC = Fmt<PREC>::VPC;
    const int e = blockIdx.y;
    const int tid = threadIdx.x;
    if (acc_zero != nullptr && e == 0) {
        for (int i = blockIdx.x * 256 + tid; i < H; i += gridDim.x * 256) acc_zero[i] = 0.f;
    }
    if (w[e] == 0.f) return;
    const int lane = tid & 63, wave = tid >> 6;
    const int G = 1 << lg, RPW = 64 >> lg;
    const int slot = lane >> lg, cl = lane & (G - 1);
    const int C = H / VPC;
    const size_t RB = (size_t)C * 16;
    const uint8_t *qb = reinterpret_cast<const uint8_t *>(tab[4 * e + 0]);
    const uint8_t *sb = reinterpret_cast<const uint8_t *>(tab[4 * e + 1]);

    float v[CPL][VPC];
    float vs[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c = min(cl + i * G, C - 1);  // lanes past the row read a valid chunk and drop it below
        const size_t base = (size_t)c * VPC;
        float acc = 0.f;
#pragma unroll
        for (int t = 0; t < VPC; ++t) {
            const float val = ld_act<XDT>(x, base + t);
            v[i][t] = val;
            acc += val;
        }
        vs[i] = acc;
    }

    const int rbase = (blockIdx.x * 4 + wave) * RPW * P;
    uint4 qg[P][CPL], qu[P][CPL];
    float sg[P][CPL], su[P][CPL];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const int r = rbase + p * RPW + slot;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = cl + i * G;
            if (r < I && c < C) {
                qg[p][i] = *reinterpret_cast<const uint4 *>(qb + (size_t)r * RB + (size_t)c * 16);
                qu[p][i] = *reinterpret_cast<const uint4 *>(qb + (size_t)(r + I) * RB + (size_t)c * 16);
                sg[p][i] = chunk_scale<PREC>(sb, r, c, H, gs);
                su[p][i] = chunk_scale<PREC>(sb, r + I, c, H, gs);
            } else {
                qg[p][i] = make_uint4(0, 0, 0, 0);
                qu[p][i] = make_uint4(0, 0, 0, 0);
                sg[p][i] = 0.f;
                su[p][i] = 0.f;
            }
        }
    }
#pragma unroll
    for (int p = 0; p < P; ++p) {
        float pg = 0.f, pu = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            pg = fmaf(sg[p][i], chunk_dot<PREC>(qg[p][i], v[i], vs[i]), pg);
            pu = fmaf(su[p][i], chunk_dot<PREC>(qu[p][i], v[i], vs[i]), pu);
        }
        pg = group_sum(pg, lg);
        pu = group_sum(pu, lg);
        const int r = rbase + p * RPW + slot;
        if (cl == 0 && r < I) h[(size_t)e * I + r] = silu_mul(pg, pu);
    }
}

// ---------------------------------------------------------------------------------------
// kernel B (fast path): partial[e, j] = w[e] * (down_e[j] . h[e])   or, for a single matrix
// (tab == nullptr), y[j] = W[j] . vec in dtype ydt.   grid (ceil(rows / rows_per_block), n)
// ---------------------------------------------------------------------------------------
template <int PREC, int VDT, int CPL, int P>
__global__ __launch_bounds__(256) void k_down(const int64_t *__restrict__ tab, const float *__restrict__ w,
                                              const uint8_t *__restrict__ q1, const uint8_t *__restrict__ s1,
                                              const void *__restrict__ vec, float *__restrict__ partial,
                                              void *__restrict__ y, int rows, int cols, int gs, int lg) {
    constexpr int VPC = Fmt<PREC>::VPC;
    const int e = blockIdx.y;
    const int tid = threadIdx.x;
    float we = 1.f;
    const uint8_t *qb = q1;
    const uint8_t *sb = s1;
    size_t voff = 0;
    if (tab != nullptr) {
        we = w[e];
        if (we == 0.f) return;
        qb = reinterpret_cast<const uint8_t *>(tab[4 * e + 2]);
        sb = reinterpret_cast<const uint8_t *>(tab[4 * e + 3]);
        voff = (size_t)e * cols;
    }
    const int lane = tid & 63, wave = tid >> 6;
    const int G = 1 << lg, RPW = 64 >> lg;
    const int slot = lane >> lg, cl = lane & (G - 1);
    const int C = cols / VPC;
    const size_t RB = (size_t)C * 16;

    float v[CPL][VPC];
    float vs[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c = min(cl + i * G, C - 1);  // lanes past the row read a valid chunk and drop it below
        const size_t base = voff + (size_t)c * VPC;
        float acc = 0.f;
#pragma unroll
        for (int t = 0; t < VPC; ++t) {
            const float val = ld_act<VDT>(vec, base + t);
            v[i][t] = val;
            acc += val;
        }
        vs[i] = acc;
    }

    const int rbase = (blockIdx.x * 4 + wave) * RPW * P;
    uint4 qd[P][CPL];
    float sd[P][CPL];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const int r = rbase + p * RPW + slot;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = cl + i * G;
            if (r < rows && c < C) {
                qd[p][i] = *reinterpret_cast<const uint4 *>(qb + (size_t)r * RB + (size_t)c * 16);
                sd[p][i] = chunk_scale<PREC>(sb, r, c, cols, gs);
            } else {
                qd[p][i] = make_uint4(0, 0, 0, 0);
                sd[p][i] = 0.f;
            }
        }
    }
#pragma unroll
    for (int p = 0; p < P; ++p) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) acc = fmaf(sd[p][i], chunk_dot<PREC>(qd[p][i], v[i], vs[i]), acc);
        acc = group_sum(acc, lg);
        const int r = rbase + p * RPW + slot;
        if (cl == 0 && r < rows) {
            if (tab != nullptr) partial[(size_t)e * rows + r] = we * acc;
            else st_act<VDT>(y, r, acc);
        }
    }
}

// ---------------------------------------------------------------------------------------
// generic kernels (any shape / group size): one wave per row, lanes stride over columns
// ---------------------------------------------------------------------------------------
template <int PREC, int XDT>
__global__ __launch_bounds__(256) void k_up_generic(const int64_t *__restrict__ tab, const float *__restrict__ w,
                                                    const void *__restrict__ x, float *__restrict__ h,
                                                    float *__restrict__ acc_zero, int I, int H, int gs) {
    const int e = blockIdx.y;
    const int tid = threadIdx.x;
    if (acc_zero != nullptr && e == 0) {
        for (int i = blockIdx.x * 256 + tid; i < H; i += gridDim.x * 256) acc_zero[i] = 0.f;
    }
    if (w[e] == 0.f) return;
    const int lane = tid & 63;
    const int r = blockIdx.x * 4 + (tid >> 6);
    if (r >= I) return;
    const uint8_t *qb = reinterpret_cast<const uint8_t *>(tab[4 * e + 0]);
    const uint8_t *sb = reinterpret_cast<const uint8_t *>(tab[4 * e + 1]);
    float g = 0.f, u = 0.f;
    for (int c = lane; c < H; c += 64) {
        const float xv = ld_act<XDT>(x, c);
        g = fmaf(weight_at<PREC>(qb, sb, r, c, H, gs), xv, g);
        u = fmaf(weight_at<PREC>(qb, sb, r + I, c, H, gs), xv, u);
    }
    g = wave_sum(g);
    u = wave_sum(u);
    if (lane == 0) h[(size_t)e * I + r] = silu_mul(g, u);
}

template <int PREC, int VDT>
__global__ __launch_bounds__(256) void k_down_generic(const int64_t *__restrict__ tab, const float *__restrict__ w,
                                                      const uint8_t *__restrict__ q1, const uint8_t *__restrict__ s1,
                                                      const void *__restrict__ vec, float *__restrict__ partial,
                                                      void *__restrict__ y, int rows, int cols, int gs) {
    const int e = blockIdx.y;
    const int tid = threadIdx.x;
    float we = 1.f;
    const uint8_t *qb = q1;
    const uint8_t *sb = s1;
    size_t voff = 0;
    if (tab != nullptr) {
        we = w[e];
        if (we == 0.f) return;
        qb = reinterpret_cast<const uint8_t *>(tab[4 * e + 2]);
        sb = reinterpret_cast<const uint8_t *>(tab[4 * e + 3]);
        voff = (size_t)e * cols;
    }
    const int lane = tid & 63;
    const int r = blockIdx.x * 4 + (tid >> 6);
    if (r >= rows) return;
    float acc = 0.f;
    for (int c = lane; c < cols; c += 64) acc = fmaf(weight_at<PREC>(qb, sb, r, c, cols, gs), ld_act<VDT>(vec, voff + c), acc);
    acc = wave_sum(acc);
    if (lane == 0) {
        if (tab != nullptr) partial[(size_t)e * rows + r] = we * acc;
        else st_act<VDT>(y, r, acc);
    }
}

// acc[j] += sum_e (w[e] != 0) partial[e, j], e in table order
__global__ __launch_bounds__(256) void k_reduce(const float *__restrict__ partial, const float *__restrict__ w, int n,
                                                int H, float *__restrict__ acc) {
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j >= H) return;
    float s = 0.f;
    for (int e = 0; e < n; ++e)
        if (w[e] != 0.f) s += partial[(size_t)e * H + j];
    acc[j] += s;
}

template <int DT>
__global__ __launch_bounds__(256) void k_combine(const float *__restrict__ acc, const void *__restrict__ add,
                                                 void *__restrict__ out, size_t N, int accumulate) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= N) return;
    float v = acc[i];
    if (accumulate) v += ld_act<DT>(out, i);
    if (add != nullptr) v += ld_act<DT>(add, i);
    st_act<DT>(out, i, v);
}

// ---------------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------------
struct RowPlan {
    bool fast;
    int lg;   // log2 lanes per row
    int cpl;  // chunks per lane
    int rpw;  // rows per wave pass
};

// cols values per row; gs group size (int formats); requires 16-byte aligned rows
static RowPlan plan_rows(int prec, int cols, int gs, bool aligned) {
    RowPlan rp{false, 6, 1, 1};
    const int vpc = vpc_of(prec);
    if (!aligned || cols % vpc != 0) return rp;
    if ((prec == MOEHIP_PREC_INT4 || prec == MOEHIP_PREC_INT8) && (gs <= 0 || gs % vpc != 0)) return rp;
    const int C = cols / vpc;
    int G = 1, lg = 0;
    while (G < C && G < 64) G <<= 1, ++lg;
    const int cpl = (C + G - 1) / G;
    if (cpl > 4) return rp;
    rp.fast = true;
    rp.lg = lg;
    rp.cpl = cpl == 3 ? 4 : cpl;
    rp.rpw = 64 >> lg;
    return rp;
}

constexpr int UP_P = 4;
constexpr int DOWN_P = 4;

#define MOEHIP_DT_SWITCH(dt, FN, ...)                                  \
    switch (dt) {                                                      \
        case MOEHIP_DT_F16: FN<MOEHIP_DT_F16>(__VA_ARGS__); break;      \
        case MOEHIP_DT_BF16: FN<MOEHIP_DT_BF16>(__VA_ARGS__); break;    \
        default: FN<MOEHIP_DT_F32>(__VA_ARGS__); break;                \
    }

#define MOEHIP_PREC_SWITCH(prec, FN, ...)                                  \
    switch (prec) {                                                        \
        case MOEHIP_PREC_INT4: FN<MOEHIP_PREC_INT4>(__VA_ARGS__); break;    \
        case MOEHIP_PREC_INT8: FN<MOEHIP_PREC_INT8>(__VA_ARGS__); break;    \
        case MOEHIP_PREC_F16: FN<MOEHIP_PREC_F16>(__VA_ARGS__); break;      \
        case MOEHIP_PREC_BF16: FN<MOEHIP_PREC_BF16>(__VA_ARGS__); break;    \
        case MOEHIP_PREC_F32: FN<MOEHIP_PREC_F32>(__VA_ARGS__); break;      \
        default: FN<MOEHIP_PREC_FP8>(__VA_ARGS__); break;                  \
    }

template <int PREC, int XDT>
static void launch_up_dt(const RowPlan &rp, dim3 grid, hipStream_t st, const int64_t *tab, const float *w,
                         const void *x, float *h, float *acc_zero, int I, int H, int gs) {
    if (!rp.fast) {
        hipLaunchKernelGGL((k_up_generic<PREC, XDT>), grid, dim3(256), 0, st, tab, w, x, h, acc_zero, I, H, gs);
        return;
    }
    switch (rp.cpl) {
        case 1: hipLaunchKernelGGL((k_up<PREC, XDT, 1, UP_P>), grid, dim3(256), 0, st, tab, w, x, h, acc_zero, I, H, gs, rp.lg); break;
        case 2: hipLaunchKernelGGL((k_up<PREC, XDT, 2, UP_P>), grid, dim3(256), 0, st, tab, w, x, h, acc_zero, I, H, gs, rp.lg); break;
        default: hipLaunchKernelGGL((k_up<PREC, XDT, 4, UP_P>), grid, dim3(256), 0, st, tab, w, x, h, acc_zero, I, H, gs, rp.lg); break;
    }
}

template <int PREC>
static void launch_up(int xdt, const RowPlan &rp, dim3 grid, hipStream_t st, const int64_t *tab, const float *w,
                      const void *x, float *h, float *acc_zero, int I, int H, int gs) {
    switch (xdt) {
        case MOEHIP_DT_F16: launch_up_dt<PREC, MOEHIP_DT_F16>(rp, grid, st, tab, w, x, h, acc_zero, I, H, gs); break;
        case MOEHIP_DT_BF16: launch_up_dt<PREC, MOEHIP_DT_BF16>(rp, grid, st, tab, w, x, h, acc_zero, I, H, gs); break;
        default: launch_up_dt<PREC, MOEHIP_DT_F32>(rp, grid, st, tab, w, x, h, acc_zero, I, H, gs); break;
    }
}

template <int PREC, int VDT>
static void launch_down(const RowPlan &rp, dim3 grid, hipStream_t st, const int64_t *tab, const float *w,
                        const uint8_t *q1, const uint8_t *s1, const void *vec, float *partial, void *y, int rows,
                        int cols, int gs) {
    if (!rp.fast) {
        hipLaunchKernelGGL((k_down_generic<PREC, VDT>), grid, dim3(256), 0, st, tab, w, q1, s1, vec, partial, y, rows, cols, gs);
        return;
    }
    switch (rp.cpl) {
        case 1: hipLaunchKernelGGL((k_down<PREC, VDT, 1, DOWN_P>), grid, dim3(256), 0, st, tab, w, q1, s1, vec, partial, y, rows, cols, gs, rp.lg); break;
        case 2: hipLaunchKernelGGL((k_down<PREC, VDT, 2, DOWN_P>), grid, dim3(256), 0, st, tab, w, q1, s1, vec, partial, y, rows, cols, gs, rp.lg); break;
        default: hipLaunchKernelGGL((k_down<PREC, VDT, 4, DOWN_P>), grid, dim3(256), 0, st, tab, w, q1, s1, vec, partial, y, rows, cols, gs, rp.lg); break;
    }
}

template <int PREC>
static void launch_down_f32(const RowPlan &rp, dim3 grid, hipStream_t st, const int64_t *tab, const float *w,
                            const float *h, float *partial, int rows, int cols, int gs) {
    launch_down<PREC, MOEHIP_DT_F32>(rp, grid, st, tab, w, nullptr, nullptr, h, partial, nullptr, rows, cols, gs);
}

template <int DT>
static void launch_gemv_int4(const RowPlan &rp, dim3 grid, hipStream_t st, const uint8_t *q, const uint8_t *s,
                             const void *x, void *y, int rows, int cols, int gs) {
    launch_down<MOEHIP_PREC_INT4, DT>(rp, grid, st, nullptr, nullptr, q, s, x, nullptr, y, rows, cols, gs);
}

template <int DT>
static void launch_combine(dim3 grid, hipStream_t st, const float *acc, const void *add, void *out, size_t N,
                           int accumulate) {
    hipLaunchKernelGGL((k_combine<DT>), grid, dim3(256), 0, st, acc, add, out, N, accumulate);
}

static bool valid_prec(int p) { return p >= MOEHIP_PREC_INT4 && p <= MOEHIP_PREC_FP8; }
static bool valid_dt(int d) { return d >= MOEHIP_DT_F16 && d <= MOEHIP_DT_F32; }
static bool int_prec(int p) { return p == MOEHIP_PREC_INT4 || p == MOEHIP_PREC_INT8; }

}  // namespace moehip

using namespace moehip;

extern "C" int moehip_grouped_up(int prec, const int64_t *tab, const float *w, const void *x, int xdtype, float *h,
                                 float *acc_zero, int n, int I, int H, int gs, void *stream) {
    MOEHIP_REQUIRE(valid_prec(prec) && valid_dt(xdtype), "grouped_up: bad precision %d or dtype %d", prec, xdtype);
    MOEHIP_REQUIRE(tab && w && x && h, "grouped_up: null pointer");
    MOEHIP_REQUIRE(n > 0 && I > 0 && H > 0, "grouped_up: bad sizes n=%d I=%d H=%d", n, I, H);
    MOEHIP_REQUIRE(!int_prec(prec) || (gs > 0 && gs % 2 == 0 && H % gs == 0), "grouped_up: group size %d vs H=%d", gs, H);
    MOEHIP_REQUIRE(prec != MOEHIP_PREC_INT4 || H % 2 == 0, "grouped_up: int4 needs an even H");
    hipStream_t st = as_stream(stream);
    const RowPlan rp = plan_rows(prec, H, gs, true);
    const int rows_per_block = rp.fast ? 4 * rp.rpw * UP_P : 4;
    dim3 grid((I + rows_per_block - 1) / rows_per_block, n);
    MOEHIP_PREC_SWITCH(prec, launch_up, xdtype, rp, grid, st, tab, w, x, h, acc_zero, I, H, gs);
    return check_launch("grouped_up");
}

extern "C" size_t moehip_down_workspace_floats(int n, int H) { return (size_t)(n > 0 ? n : 0) * (size_t)(H > 0 ? H : 0); }

extern "C" int moehip_grouped_down(int prec, const int64_t *tab, const float *w, const float *h, float *acc, int n,
                                   int H, int I, int gs, float *partial, void *stream) {
    MOEHIP_REQUIRE(valid_prec(prec), "grouped_down: bad precision %d", prec);
    MOEHIP_REQUIRE(tab && w && h && acc && partial, "grouped_down: null pointer");
    MOEHIP_REQUIRE(n > 0 && I > 0 && H > 0, "grouped_down: bad sizes n=%d H=%d I=%d", n, H, I);
    MOEHIP_REQUIRE(!int_prec(prec) || (gs > 0 && gs % 2 == 0 && I % gs == 0), "grouped_down: group size %d vs I=%d", gs, I);
    MOEHIP_REQUIRE(prec != MOEHIP_PREC_INT4 || I % 2 == 0, "grouped_down: int4 needs an even I");
    hipStream_t st = as_stream(stream);
    const RowPlan rp = plan_rows(prec, I, gs, true);
    const int rows_per_block = rp.fast ? 4 * rp.rpw * DOWN_P : 4;
    dim3 grid((H + rows_per_block - 1) / rows_per_block, n);
    MOEHIP_PREC_SWITCH(prec, launch_down_f32, rp, grid, st, tab, w, h, partial, H, I, gs);
    int rc = check_launch("grouped_down");
    if (rc) return rc;
    hipLaunchKernelGGL(k_reduce, dim3((H + 255) / 256), dim3(256), 0, st, partial, w, n, H, acc);
    return check_launch("grouped_down reduce");
}

extern "C" int moehip_gemv_int4(const void *q, const void *s, const void *x, void *y, int O, int I, int gs, int dtype,
                                void *stream) {
    MOEHIP_REQUIRE(q && s && x && y, "gemv_int4: null pointer");
    MOEHIP_REQUIRE(valid_dt(dtype), "gemv_int4: bad dtype %d", dtype);
    MOEHIP_REQUIRE(O > 0 && I > 0 && I % 2 == 0 && gs > 0 && gs % 2 == 0 && I % gs == 0,
                   "gemv_int4: bad sizes O=%d I=%d gs=%d", O, I, gs);
    hipStream_t st = as_stream(stream);
    const bool aligned = ((uintptr_t)q % 16) == 0;
    const RowPlan rp = plan_rows(MOEHIP_PREC_INT4, I, gs, aligned);
    const uint8_t *qb = reinterpret_cast<const uint8_t *>(q);
    const uint8_t *sb = reinterpret_cast<const uint8_t *>(s);
    const int rows_per_block = rp.fast ? 4 * rp.rpw * DOWN_P : 4;
    dim3 grid((O + rows_per_block - 1) / rows_per_block, 1);
    MOEHIP_DT_SWITCH(dtype, launch_gemv_int4, rp, grid, st, qb, sb, x, y, O, I, gs);
    return check_launch("gemv_int4");
}

extern "C" int moehip_combine(const float *acc, const void *add, void *out, int T, int H, int dtype, int accumulate,
                              void *stream) {
    MOEHIP_REQUIRE(acc && out, "combine: null pointer");
    MOEHIP_REQUIRE(valid_dt(dtype) && T > 0 && H > 0, "combine: bad args");
    const size_t N = (size_t)T * H;
    MOEHIP_DT_SWITCH(dtype, launch_combine, dim3((unsigned)((N + 255) / 256)), as_stream(stream), acc, add, out, N,
                     accumulate);
    return check_launch("combine");
}
