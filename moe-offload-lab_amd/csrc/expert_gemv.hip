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

#include "common.hpp"

namespace moehip {

template <int PREC> struct Fmt;
template <> struct Fmt<MOEHIP_PREC_INT4> { static constexpr int VPC = 32; };
template <> struct Fmt<MOEHIP_PREC_INT8> { static constexpr int VPC = 16; };
template <> struct Fmt<MOEHIP_PREC_F16> { static constexpr int VPC = 8; };
template <> struct Fmt<MOEHIP_PREC_BF16> { static constexpr int VPC = 8; };
template <> struct Fmt<MOEHIP_PREC_F32> { static constexpr int VPC = 4; };
template <> struct Fmt<MOEHIP_PREC_FP8> { static constexpr int VPC = 16; };

static inline int vpc_of(int prec) {
    switch (prec) {
        case MOEHIP_PREC_INT4: return 32;
        case MOEHIP_PREC_INT8: return 16;
        case MOEHIP_PREC_F16: return 8;
        case MOEHIP_PREC_BF16: return 8;
        case MOEHIP_PREC_F32: return 4;
        case MOEHIP_PREC_FP8: return 16;
    }
    return 0;
}

// ---------------------------------------------------------------------------------------
// chunk dot products: sum over the chunk's VPC values of weight * v (int formats unscaled)
// ---------------------------------------------------------------------------------------
template <int PREC>
__device__ __forceinline__ float chunk_dot(const uint4 q, const float *v, float vsum);

template <>
__device__ __forceinline__ float chunk_dot<MOEHIP_PREC_INT4>(const uint4 q, const float *v, float vsum) {
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t lo = d[j] & 0x0F0F0F0Fu;         // even columns 0,2,4,6 of this dword
        const uint32_t hi = (d[j] >> 4) & 0x0F0F0F0Fu;  // odd columns 1,3,5,7
        a0 = fmaf((float)(lo & 0xffu), v[8 * j + 0], a0);
        a1 = fmaf((float)(hi & 0xffu), v[8 * j + 1], a1);
        a0 = fmaf((float)((lo >> 8) & 0xffu), v[8 * j + 2], a0);
        a1 = fmaf((float)((hi >> 8) & 0xffu), v[8 * j + 3], a1);
        a0 = fmaf((float)((lo >> 16) & 0xffu), v[8 * j + 4], a0);
        a1 = fmaf((float)((hi >> 16) & 0xffu), v[8 * j + 5], a1);
        a0 = fmaf((float)(lo >> 24), v[8 * j + 6], a0);
        a1 = fmaf((float)(hi >> 24), v[8 * j + 7], a1);
    }
    return (a0 + a1) - 8.0f * vsum;
}

template <>
__device__ __forceinline__ float chunk_dot<MOEHIP_PREC_INT8>(const uint4 q, const float *v, float vsum) {
    const uint32_t d[4] = {q.x ^ 0x80808080u, q.y ^ 0x80808080u, q.z ^ 0x80808080u, q.w ^ 0x80808080u};
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // byte b holds q + 128 as an unsigned value
        a0 = fmaf((float)(d[j] & 0xffu), v[4 * j + 0], a0);
        a1 = fmaf((float)((d[j] >> 8) & 0xffu), v[4 * j + 1], a1);
        a0 = fmaf((float)((d[j] >> 16) & 0xffu), v[4 * j + 2], a0);
        a1 = fmaf((float)(d[j] >> 24), v[4 * j + 3], a1);
    }
    return (a0 + a1) - 128.0f * vsum;
}

template <>
__device__ __forceinline__ float chunk_dot<MOEHIP_PREC_F16>(const uint4 q, const float *v, float) {
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        a0 = fmaf(f16_to_f32(d[j] & 0xffffu), v[2 * j + 0], a0);
        a1 = fmaf(f16_to_f32(d[j] >> 16), v[2 * j + 1], a1);
    }
    return a0 + a1;
}

template <>
__device__ __forceinline__ float chunk_dot<MOEHIP_PREC_BF16>(const uint4 q, const float *v, float) {
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        a0 = fmaf(__uint_as_float(d[j] << 16), v[2 * j + 0], a0);
        a1 = fmaf(__uint_as_float(d[j] & 0xffff0000u), v[2 * j + 1], a1);
    }
    return a0 + a1;
}

template <>
__device__ __forceinline__ float chunk_dot<MOEHIP_PREC_F32>(const uint4 q, const float *v, float) {
    float a = __uint_as_float(q.x) * v[0];
    a = fmaf(__uint_as_float(q.y), v[1], a);
    a = fmaf(__uint_as_float(q.z), v[2], a);
    return fmaf(__uint_as_float(q.w), v[3], a);
}

template <>
__device__ __forceinline__ float chunk_dot<MOEHIP_PREC_FP8>(const uint4 q, const float *v, float) {
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        a0 = fmaf(__builtin_amdgcn_cvt_f32_fp8((int)d[j], 0), v[4 * j + 0], a0);
        a1 = fmaf(__builtin_amdgcn_cvt_f32_fp8((int)d[j], 1), v[4 * j + 1], a1);
        a0 = fmaf(__builtin_amdgcn_cvt_f32_fp8((int)d[j], 2), v[4 * j + 2], a0);
        a1 = fmaf(__builtin_amdgcn_cvt_f32_fp8((int)d[j], 3), v[4 * j + 3], a1);
    }
    return a0 + a1;
}

// scale of chunk c of row `row` (cols = row length in values)
template <int PREC>
__device__ __forceinline__ float chunk_scale(const uint8_t *sb, int row, int c, int cols, int gs) {
    if constexpr (PREC == MOEHIP_PREC_INT4 || PREC == MOEHIP_PREC_INT8) {
        const int ng = cols / gs;
        const int g = (c * Fmt<PREC>::VPC) / gs;
        return f16_to_f32(reinterpret_cast<const uint16_t *>(sb)[(size_t)row * ng + g]);
    } else if constexpr (PREC == MOEHIP_PREC_FP8) {
        const int sc = (cols + 127) >> 7;
        return reinterpret_cast<const float *>(sb)[(size_t)(row >> 7) * sc + ((c * 16) >> 7)];
    } else {
        return 1.0f;
    }
}

// scalar weight (row, col) for the generic kernels
template <int PREC>
__device__ __forceinline__ float weight_at(const uint8_t *qb, const uint8_t *sb, int row, int col, int cols, int gs) {
    if constexpr (PREC == MOEHIP_PREC_INT4) {
        const uint32_t b = qb[(size_t)row * (cols >> 1) + (col >> 1)];
        const int n = (int)((col & 1) ? (b >> 4) : (b & 15u)) - 8;
        return (float)n * f16_to_f32(reinterpret_cast<const uint16_t *>(sb)[(size_t)row * (cols / gs) + col / gs]);
    } else if constexpr (PREC == MOEHIP_PREC_INT8) {
        const int n = (int)(int8_t)qb[(size_t)row * cols + col];
        return (float)n * f16_to_f32(reinterpret_cast<const uint16_t *>(sb)[(size_t)row * (cols / gs) + col / gs]);
    } else if constexpr (PREC == MOEHIP_PREC_F16) {
        return f16_to_f32(reinterpret_cast<const uint16_t *>(qb)[(size_t)row * cols + col]);
    } else if constexpr (PREC == MOEHIP_PREC_BF16) {
        return bf16_to_f32(reinterpret_cast<const uint16_t *>(qb)[(size_t)row * cols + col]);
    } else if constexpr (PREC == MOEHIP_PREC_F32) {
        return reinterpret_cast<const float *>(qb)[(size_t)row * cols + col];
    } else {
        const int sc = (cols + 127) >> 7;
        return fp8_to_f32(qb[(size_t)row * cols + col]) *
               reinterpret_cast<const float *>(sb)[(size_t)(row >> 7) * sc + (col >> 7)];
    }
}

// ---------------------------------------------------------------------------------------
// kernel A (fast path): h[e, r] = silu(gate_e[r] . x) * (up_e[r] . x)
// grid (ceil(I / rows_per_block), n), block 256
// ---------------------------------------------------------------------------------------
template <int PREC, int CPL, int P>
__global__ __launch_bounds__(256) void k_up(const int64_t *__restrict__ tab, const float *__restrict__ w,
                                            const void *__restrict__ x, int xdt, float *__restrict__ h,
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
        const int c = cl + i * G;
        float acc = 0.f;
#pragma unroll
        for (int t = 0; t < VPC; ++t) {
            const float val = (c < C) ? load_act(x, (size_t)c * VPC + t, xdt) : 0.f;
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
template <int PREC, int CPL, int P>
__global__ __launch_bounds__(256) void k_down(const int64_t *__restrict__ tab, const float *__restrict__ w,
                                              const uint8_t *__restrict__ q1, const uint8_t *__restrict__ s1,
                                              const void *__restrict__ vec, int vdt, float *__restrict__ partial,
                                              void *__restrict__ y, int ydt, int rows, int cols, int gs, int lg) {
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
        const int c = cl + i * G;
        float acc = 0.f;
#pragma unroll
        for (int t = 0; t < VPC; ++t) {
            const float val = (c < C) ? load_act(vec, voff + (size_t)c * VPC + t, vdt) : 0.f;
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
            else store_act(y, r, ydt, acc);
        }
    }
}

// ---------------------------------------------------------------------------------------
// generic kernels (any shape / group size): one wave per row, lanes stride over columns
// ---------------------------------------------------------------------------------------
template <int PREC>
__global__ __launch_bounds__(256) void k_up_generic(const int64_t *__restrict__ tab, const float *__restrict__ w,
                                                    const void *__restrict__ x, int xdt, float *__restrict__ h,
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
        const float xv = load_act(x, c, xdt);
        g = fmaf(weight_at<PREC>(qb, sb, r, c, H, gs), xv, g);
        u = fmaf(weight_at<PREC>(qb, sb, r + I, c, H, gs), xv, u);
    }
    g = wave_sum(g);
    u = wave_sum(u);
    if (lane == 0) h[(size_t)e * I + r] = silu_mul(g, u);
}

template <int PREC>
__global__ __launch_bounds__(256) void k_down_generic(const int64_t *__restrict__ tab, const float *__restrict__ w,
                                                      const uint8_t *__restrict__ q1, const uint8_t *__restrict__ s1,
                                                      const void *__restrict__ vec, int vdt,
                                                      float *__restrict__ partial, void *__restrict__ y, int ydt,
                                                      int rows, int cols, int gs) {
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
    for (int c = lane; c < cols; c += 64) acc = fmaf(weight_at<PREC>(qb, sb, r, c, cols, gs), load_act(vec, voff + c, vdt), acc);
    acc = wave_sum(acc);
    if (lane == 0) {
        if (tab != nullptr) partial[(size_t)e * rows + r] = we * acc;
        else store_act(y, r, ydt, acc);
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

__global__ __launch_bounds__(256) void k_combine(const float *__restrict__ acc, const void *__restrict__ add,
                                                 void *__restrict__ out, size_t N, int dt, int accumulate) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= N) return;
    float v = acc[i];
    if (accumulate) v += load_act(out, i, dt);
    if (add != nullptr) v += load_act(add, i, dt);
    store_act(out, i, dt, v);
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

template <int PREC>
static void launch_up(const RowPlan &rp, dim3 grid, hipStream_t st, const int64_t *tab, const float *w,
                      const void *x, int xdt, float *h, float *acc_zero, int I, int H, int gs) {
    switch (rp.cpl) {
        case 1: hipLaunchKernelGGL((k_up<PREC, 1, UP_P>), grid, dim3(256), 0, st, tab, w, x, xdt, h, acc_zero, I, H, gs, rp.lg); break;
        case 2: hipLaunchKernelGGL((k_up<PREC, 2, UP_P>), grid, dim3(256), 0, st, tab, w, x, xdt, h, acc_zero, I, H, gs, rp.lg); break;
        default: hipLaunchKernelGGL((k_up<PREC, 4, UP_P>), grid, dim3(256), 0, st, tab, w, x, xdt, h, acc_zero, I, H, gs, rp.lg); break;
    }
}

template <int PREC>
static void launch_down(const RowPlan &rp, dim3 grid, hipStream_t st, const int64_t *tab, const float *w,
                        const uint8_t *q1, const uint8_t *s1, const void *vec, int vdt, float *partial, void *y,
                        int ydt, int rows, int cols, int gs) {
    switch (rp.cpl) {
        case 1: hipLaunchKernelGGL((k_down<PREC, 1, DOWN_P>), grid, dim3(256), 0, st, tab, w, q1, s1, vec, vdt, partial, y, ydt, rows, cols, gs, rp.lg); break;
        case 2: hipLaunchKernelGGL((k_down<PREC, 2, DOWN_P>), grid, dim3(256), 0, st, tab, w, q1, s1, vec, vdt, partial, y, ydt, rows, cols, gs, rp.lg); break;
        default: hipLaunchKernelGGL((k_down<PREC, 4, DOWN_P>), grid, dim3(256), 0, st, tab, w, q1, s1, vec, vdt, partial, y, ydt, rows, cols, gs, rp.lg); break;
    }
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

template <int PREC>
static void launch_up_generic(dim3 grid, hipStream_t st, const int64_t *tab, const float *w, const void *x, int xdt,
                              float *h, float *acc_zero, int I, int H, int gs) {
    hipLaunchKernelGGL((k_up_generic<PREC>), grid, dim3(256), 0, st, tab, w, x, xdt, h, acc_zero, I, H, gs);
}

template <int PREC>
static void launch_down_generic(dim3 grid, hipStream_t st, const int64_t *tab, const float *w, const uint8_t *q1,
                                const uint8_t *s1, const void *vec, int vdt, float *partial, void *y, int ydt,
                                int rows, int cols, int gs) {
    hipLaunchKernelGGL((k_down_generic<PREC>), grid, dim3(256), 0, st, tab, w, q1, s1, vec, vdt, partial, y, ydt,
                       rows, cols, gs);
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
    if (rp.fast) {
        const int rows_per_block = 4 * rp.rpw * UP_P;
        dim3 grid((I + rows_per_block - 1) / rows_per_block, n);
        MOEHIP_PREC_SWITCH(prec, launch_up, rp, grid, st, tab, w, x, xdtype, h, acc_zero, I, H, gs);
    } else {
        dim3 grid((I + 3) / 4, n);
        MOEHIP_PREC_SWITCH(prec, launch_up_generic, grid, st, tab, w, x, xdtype, h, acc_zero, I, H, gs);
    }
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
    if (rp.fast) {
        const int rows_per_block = 4 * rp.rpw * DOWN_P;
        dim3 grid((H + rows_per_block - 1) / rows_per_block, n);
        MOEHIP_PREC_SWITCH(prec, launch_down, rp, grid, st, tab, w, nullptr, nullptr, h, MOEHIP_DT_F32, partial,
                           nullptr, MOEHIP_DT_F32, H, I, gs);
    } else {
        dim3 grid((H + 3) / 4, n);
        MOEHIP_PREC_SWITCH(prec, launch_down_generic, grid, st, tab, w, nullptr, nullptr, h, MOEHIP_DT_F32, partial,
                           nullptr, MOEHIP_DT_F32, H, I, gs);
    }
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
    if (rp.fast) {
        const int rows_per_block = 4 * rp.rpw * DOWN_P;
        dim3 grid((O + rows_per_block - 1) / rows_per_block, 1);
        launch_down<MOEHIP_PREC_INT4>(rp, grid, st, nullptr, nullptr, qb, sb, x, dtype, nullptr, y, dtype, O, I, gs);
    } else {
        dim3 grid((O + 3) / 4, 1);
        launch_down_generic<MOEHIP_PREC_INT4>(grid, st, nullptr, nullptr, qb, sb, x, dtype, nullptr, y, dtype, O, I, gs);
    }
    return check_launch("gemv_int4");
}

extern "C" int moehip_combine(const float *acc, const void *add, void *out, int T, int H, int dtype, int accumulate,
                              void *stream) {
    MOEHIP_REQUIRE(acc && out, "combine: null pointer");
    MOEHIP_REQUIRE(valid_dt(dtype) && T > 0 && H > 0, "combine: bad args");
    const size_t N = (size_t)T * H;
    hipLaunchKernelGGL(k_combine, dim3((unsigned)((N + 255) / 256)), dim3(256), 0, as_stream(stream), acc, add, out, N,
                       dtype, accumulate);
    return check_launch("combine");
}
