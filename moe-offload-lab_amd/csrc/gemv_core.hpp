// Dequantising dot products over 16-byte chunks of an expert record row, shared by the
// grouped kernels and the fused decode-layer kernel.
//
// A weight row is streamed as 16-byte chunks; a chunk holds VPC values (int4: 32, int8/fp8: 16,
// f16/bf16: 8, f32: 4) and always lies inside one scale group (int: gs % VPC == 0; fp8:
// 128-column blocks). int4 bytes hold (q+8) | (q'+8) << 4 (moelab/quant.py:96-101): a dword of
// 8 nibbles is masked into two dwords of 4 bytes each, converted with the unsigned byte
// converts, and the +8 offset is removed once per chunk as -8 * sum(vector slice).
#pragma once

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
// dot2 chunk products of the integer records against fp16 activation pairs in operand order
// (per 8 values (v0,v4) (v1,v5) (v2,v6) (v3,v7) for int4, (v0,v2) (v1,v3) per 4 for int8).
// The weights enter as fp16 1024 + n (int4 low nibble), 1024 + 16 n (int4 high nibble, the sum
// scaled by 1/16) or 1024 + q + 128 (int8), each from one v_and_or_b32; the offsets are taken
// out by a per-chunk correction that depends on the activations only:
//   int4: corr = -1032 * sum(even pairs) - 72 * sum(odd pairs);  int8: corr = -1152 * sum.
// The result is sum(q * v) before the group scale (fp32 accumulation).
// ---------------------------------------------------------------------------------------
constexpr uint32_t H2_M1032 = 0xE408E408u;  // (-1032, -1032)
constexpr uint32_t H2_M72 = 0xD480D480u;    // (-72, -72)
constexpr uint32_t H2_M1152 = 0xE480E480u;  // (-1152, -1152)

template <int PREC>
__device__ __forceinline__ float chunk_corr(const uint32_t *xp) {
    float c = 0.f;
    if constexpr (PREC == MOEHIP_PREC_INT4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            c = dot2h(H2_M1032, xp[4 * j + 0], c);
            c = dot2h(H2_M72, xp[4 * j + 1], c);
            c = dot2h(H2_M1032, xp[4 * j + 2], c);
            c = dot2h(H2_M72, xp[4 * j + 3], c);
        }
    } else if constexpr (PREC == MOEHIP_PREC_INT8) {
#pragma unroll
        for (int j = 0; j < 8; ++j) c = dot2h(H2_M1152, xp[j], c);
    }
    return c;
}

template <int PREC>
__device__ __forceinline__ float dot2_chunk(const uint4 q, const uint32_t *xp, float corr) {
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
    if constexpr (PREC == MOEHIP_PREC_INT4) {
        float ae = corr, ao = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t t = d[j] >> 8;
            ae = dot2h(and_or(d[j], 0x000F000Fu, 0x64006400u), xp[4 * j + 0], ae);
            ao = dot2h(and_or(d[j], 0x00F000F0u, 0x64006400u), xp[4 * j + 1], ao);
            ae = dot2h(and_or(t, 0x000F000Fu, 0x64006400u), xp[4 * j + 2], ae);
            ao = dot2h(and_or(t, 0x00F000F0u, 0x64006400u), xp[4 * j + 3], ao);
        }
        return fmaf(ao, 0.0625f, ae);
    } else if constexpr (PREC == MOEHIP_PREC_INT8) {
        float a0 = corr, a1 = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t b = d[j] ^ 0x80808080u, t = b >> 8;
            a0 = dot2h(and_or(b, 0x00FF00FFu, 0x64006400u), xp[2 * j + 0], a0);
            a1 = dot2h(and_or(t, 0x00FF00FFu, 0x64006400u), xp[2 * j + 1], a1);
        }
        return a0 + a1;
    } else {
        float a = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) a = dot2h(d[j], xp[j], a);
        return a;
    }
}

}  // namespace moehip
