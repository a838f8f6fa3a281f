// Shared device helpers for the moehip kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

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

// the XCD-local one-token layer kernel (decode_xcd.hip): the dispatch check of a device (run once
// by moehip_device_check), its workspace size (0 = the layer does not fit it) and its launch
// (*used = 0 when the layer does not fit it or the device was not confirmed)
int xcd_probe(int dev);
// 1 once xcd_probe confirmed that workgroup b runs on XCD b % 8 on the current device
int xcd_dispatch_ok();
// logits (T, E) = x Wr^T in dtype (router.hip): MFMA tiles for 16-bit rows when the shape allows
void launch_router_logits(const void *x, const void *Wr, int T, int H, int E, int dtype, void *logits, hipStream_t st);
int noalloc_init(int dev);
void *noalloc_scratch(int dev);
size_t xcd_workspace_bytes(int prec, int ks, int E, int H, int I);
int xcd_launch(const moehip_layer_desc *d, const void *x, const void *Wr, const int64_t *idx_in, const float *w32_in,
               const int64_t *rows_b, const float *rows_w, const int64_t *rtab, void *out, const void *add,
               int accumulate, void *logits_out, int64_t *idx_out, void *w_out, float *w32_out, float *info,
               float *miss, void *ws, size_t ws_bytes, uint64_t *trace, void *stream, int *used);

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
// wave64 reductions with DPP: quad_perm [1,0,3,2] and [2,3,0,1] (xor 1, xor 2), row_half_mirror
// and row_mirror (after the previous steps every lane of an aligned group of 8 / 16 holds the
// group's sum), then v_readlane of the four row results for groups of 32 / 64. Every lane must
// be active when these are called.
// ---------------------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float lane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// sum over aligned groups of G = 2^lg lanes; every lane of a group gets the group total
__device__ __forceinline__ float group_sum(float v, int lg) {
    if (lg >= 1) v += dpp_f<0xB1>(v);
    if (lg >= 2) v += dpp_f<0x4E>(v);
    if (lg >= 3) v += dpp_f<0x141>(v);
    if (lg >= 4) v += dpp_f<0x140>(v);
    if (lg >= 5) {
        const float r0 = lane_f(v, 0), r1 = lane_f(v, 16), r2 = lane_f(v, 32), r3 = lane_f(v, 48);
        if (lg == 5) v = (threadIdx.x & 32) ? (r2 + r3) : (r0 + r1);
        else v = (r0 + r1) + (r2 + r3);
    }
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum(v, 6); }

__device__ __forceinline__ int wave_sum_i(int v) {
    v += dpp_i<0xB1>(v);
    v += dpp_i<0x4E>(v);
    v += dpp_i<0x141>(v);
    v += dpp_i<0x140>(v);
    return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
           (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

// order-preserving 32-bit key of a non-NaN float: a > b <=> key(a) > key(b), key(-0) == key(+0)
__device__ __forceinline__ uint32_t fkey(float f) {
    const uint32_t u = f == 0.f ? 0u : __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// sum over aligned groups of G = 2^lg lanes (lg <= 6), valid in the LAST lane of each group:
// within 16-lane rows by quad_perm / mirrors, then DPP row_bcast:15 (rows 1, 3 += lane 15 of
// rows 0, 2) and row_bcast:31 (rows 2, 3 += lane 31). Six DPP adds for a whole wave.
__device__ __forceinline__ float grp_total(float v, int lg) {
    if (lg >= 1) v += dpp_f<0xB1>(v);
    if (lg >= 2) v += dpp_f<0x4E>(v);
    if (lg >= 3) v += dpp_f<0x141>(v);
    if (lg >= 4) v += dpp_f<0x140>(v);
    if (lg >= 5) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));
    if (lg >= 6) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));
    return v;
}

// grp_total of N independent values, step-interleaved so the DPP chains overlap
template <int N>
__device__ __forceinline__ void grp_total_n(float (&v)[N], int lg) {
#pragma unroll
    for (int i = 0; i < N; ++i) if (lg >= 1) v[i] += dpp_f<0xB1>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) if (lg >= 2) v[i] += dpp_f<0x4E>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) if (lg >= 3) v[i] += dpp_f<0x141>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) if (lg >= 4) v[i] += dpp_f<0x140>(v[i]);
#pragma unroll
    for (int i = 0; i < N; ++i)
        if (lg >= 5) v[i] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[i]), 0x142, 0xA, 0xF, false));
#pragma unroll
    for (int i = 0; i < N; ++i)
        if (lg >= 6) v[i] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[i]), 0x143, 0xC, 0xF, false));
}

// maximum of an unsigned value over the wave, uniform result
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)dpp_i<0xB1>((int)v));
    v = max(v, (uint32_t)dpp_i<0x4E>((int)v));
    v = max(v, (uint32_t)dpp_i<0x141>((int)v));
    v = max(v, (uint32_t)dpp_i<0x140>((int)v));
    const uint32_t a = max((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16));
    const uint32_t b = max((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48));
    return max(a, b);
}

// ---------------------------------------------------------------------------------------
// packed half2 arithmetic: v_dot2_f32_f16 (two fp16 products, exact, accumulated in fp32)
// ---------------------------------------------------------------------------------------
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2h(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b), c, false);
}
// half2 bits of (lo, hi), each rounded to nearest even
__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
    return (uint32_t)f32_to_f16_rne(lo) | ((uint32_t)f32_to_f16_rne(hi) << 16);
}
// low halves / high halves of two dwords: (a.lo, b.lo) and (a.hi, b.hi)
__device__ __forceinline__ uint32_t lo_lo(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ __forceinline__ uint32_t hi_hi(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

// (d & mask) | magic in one v_and_or_b32 (the compiler otherwise splits it into two
// instructions: gfx9 VOP3 encodings take no literal constants). Never feed the result straight
// into an MFMA operand: the compiler does not insert hazard wait states for inline asm.
__device__ __forceinline__ uint32_t and_or(uint32_t d, uint32_t mask, uint32_t magic) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(d), "s"(mask), "v"(magic));
    return r;
}

// Record bytes in the global address space. Record addresses come from integer tables; loads
// through generic pointers would be flat loads, which also count against the LDS / scalar wait
// counter (every LDS wait would then also wait for the weight loads in flight).
typedef const __attribute__((address_space(1))) uint8_t gbyte;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ gbyte *gbytes(uint64_t a) { return (gbyte *)(uintptr_t)a; }
__device__ __forceinline__ gbyte *gbytes(const void *p) { return (gbyte *)(uintptr_t)p; }
__device__ __forceinline__ uint4 gld16(gbyte *p) {
    const u32x4_t v = *(const __attribute__((address_space(1))) u32x4_t *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
// streaming load (non-temporal hint) for weight bytes read once per launch: they then do not
// displace the small, reused data (router weights, activations, exchange words) from the caches
__device__ __forceinline__ uint4 gld16_nt(gbyte *p) {
    const u32x4_t v = __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4_t *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t gld4(gbyte *p) { return *(const __attribute__((address_space(1))) uint32_t *)p; }
__device__ __forceinline__ uint32_t gld2(gbyte *p) { return *(const __attribute__((address_space(1))) uint16_t *)p; }

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }
// the same from the hardware's exp2 and reciprocal (about 1 ulp each): 6 instructions instead of ~30,
// for kernels whose every lane evaluates it (exp2(+large) = inf gives g * 0 = -0, as g / inf)
__device__ __forceinline__ float silu_mul_fast(float g, float u) {
    const float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
    return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

}  // namespace moehip
