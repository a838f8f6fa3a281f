// Shared device helpers for the moehip kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/moehip.h"

namespace moehip {

// ---------------------------------------------------------------------------------------
// error reporting (thread-local message, returned through moehip_last_error)
// ---------------------------------------------------------------------------------------
void set_error(const char *fmt, ...);
int check_launch(const char *what);

#define MOEHIP_REQUIRE(cond, ...)                                                                            \
    do {                                                                                                     \
        if (!(cond)) {                                                                                       \
            ::moehip::set_error(__VA_ARGS__);                                                                \
            return MOEHIP_EINVAL;                                                                            \
        }                                                                                                    \
    } while (0)

static inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// ---------------------------------------------------------------------------------------
// scalar conversions
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;  // NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
    return (float)h;
}

__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
    _Float16 h = (_Float16)f;  // round-to-nearest-even
    return __builtin_bit_cast(uint16_t, h);
}

// typed activation access: DT is a compile-time MOEHIP_DT_* code, so kernels carry no runtime
// dtype switches (each instantiation is straight-line code for one dtype)
template <int DT>
__device__ __forceinline__ float ld_act(const void *p, size_t i) {
    if constexpr (DT == MOEHIP_DT_F16) return f16_to_f32(reinterpret_cast<const uint16_t *>(p)[i]);
    else if constexpr (DT == MOEHIP_DT_BF16) return bf16_to_f32(reinterpret_cast<const uint16_t *>(p)[i]);
    else return reinterpret_cast<const float *>(p)[i];
}

template <int DT>
__device__ __forceinline__ void st_act(void *p, size_t i, float v) {
    if constexpr (DT == MOEHIP_DT_F16) reinterpret_cast<uint16_t *>(p)[i] = f32_to_f16_rne(v);
    else if constexpr (DT == MOEHIP_DT_BF16) reinterpret_cast<uint16_t *>(p)[i] = f32_to_bf16_rne(v);
    else reinterpret_cast<float *>(p)[i] = v;
}

template <int DT>
__device__ __forceinline__ float rnd_act(float v) {
    if constexpr (DT == MOEHIP_DT_F16) return f16_to_f32(f32_to_f16_rne(v));
    else if constexpr (DT == MOEHIP_DT_BF16) return bf16_to_f32(f32_to_bf16_rne(v));
    else return v;
}

// OCP e4m3fn byte -> fp32 (gfx950's fp8 conversion is the OCP format)
__device__ __forceinline__ float fp8_to_f32(uint32_t byte) {
    return __builtin_amdgcn_cvt_f32_fp8((int)byte, 0);
}

// ---------------------------------------------------------------------------------------
// wave64 reductions
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// sum across aligned groups of G = 2^lg lanes (every lane of the group gets the total)
__device__ __forceinline__ float group_sum(float v, int lg) {
    for (int off = (1 << lg) >> 1; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

}  // namespace moehip
