// Store-side quantisation on the GPU, bit-exact. absmax (moelab/quant.py:57-61, 74-76, 96-127):
// scale = fp16(max(absmax / qmax, 1e-7)) (fp16(1e-7) if that rounds to 0), q = rint(w / scale)
// clamped to [qmin, qmax], int4 packed as (q+8) | (q'+8) << 4 with the even column low.
// One wave per (row, group), one lane per column of the group (gs <= 64).

#include "common.hpp"

namespace moehip {

__global__ __launch_bounds__(256) void k_quantize(const float *__restrict__ w, int O, int I, int bits, int gs,
                                                  uint8_t *__restrict__ q, uint16_t *__restrict__ s) {
    const int lane = threadIdx.x & 63;
    const int ng = I / gs;
    const long gid = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (gid >= (long)O * ng) return;
    const int row = (int)(gid / ng), g = (int)(gid % ng);
    const bool act = lane < gs;
    const float v = act ? w[(size_t)row * I + (size_t)g * gs + lane] : 0.f;
    const float amax = wave_max(fabsf(v));
    const float qmax = bits == 4 ? 7.f : 127.f;
    const float qmin = bits == 4 ? -8.f : -127.f;
    const float sc = fmaxf(amax / qmax, 1e-7f);
    uint16_t s16 = f32_to_f16_rne(sc);
    if ((s16 & 0x7fffu) == 0) s16 = f32_to_f16_rne(1e-7f);
    const float sf = f16_to_f32(s16);
    const float qf = fminf(fmaxf(rintf(v / sf), qmin), qmax);
    const int qi = (int)qf;
    if (lane == 0) s[(size_t)row * ng + g] = s16;
    if (bits == 8) {
        if (act) reinterpret_cast<int8_t *>(q)[(size_t)row * I + (size_t)g * gs + lane] = (int8_t)qi;
    } else {
        const int partner = __shfl_down(qi, 1, 64);
        if (act && (lane & 1) == 0)
            q[(size_t)row * (I / 2) + ((size_t)g * gs + lane) / 2] = (uint8_t)((qi + 8) | ((partner + 8) << 4));
    }
}

// ---------------------------------------------------------------------------------------
// Store-side mse scale search (moelab/quant.py:64-93, method="mse"; the int4 store default,
// store.py:84-85), bit-exact with the oracle's restatement: candidates b * f for the bases
// absmax / qmax and (int4 only) w[argmax |w|] / -8 (the first index of the largest magnitude), f
// = 1.00, 0.98, ..., 0.70 (the double 1 - 0.02 i rounded to float), each rounded to fp16 (0 ->
// fp16(1e-7)); error = sum over the group of (rint(w / s) clamped * s - w)^2 in float32, summed
// in numpy's pairwise order for <= 128 values (8 running sums over the first gs - gs % 8 values,
// ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7)), then the rest one by one; fewer than 8
// values: one by one from 0); the first candidate with the strictly smallest error wins. Every
// product, difference, quotient and fp16 conversion is rounded on its own: plain operators under
// `fp contract(off)` (the __f*_rn helpers inline library code that may still be fused).
//
// 8 lanes per group (8 groups per wave): lane j holds the columns j, j + 8, ... below
// gs - gs % 8, in the order of its running sum; every lane of the group also holds the last
// gs % 8 columns. The group's lanes combine through DPP within their 8 lanes (xor 1, xor 2, the
// mirror of the 8: each step adds two equal-shaped partial sums, in either order the same float).
// Lanes past the last group work on group 0 and store nothing (every lane stays active).
// ---------------------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp8_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp8_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
// (|w|, index, w) of the first largest magnitude, against the lane CTRL names
template <int CTRL>
__device__ __forceinline__ void argmax_step(float &a, int &ix, float &sv) {
    const float oa = dpp8_f<CTRL>(a), osv = dpp8_f<CTRL>(sv);
    const int oix = dpp8_i<CTRL>(ix);
    if (oa > a || (oa == a && oix < ix)) {
        a = oa;
        ix = oix;
        sv = osv;
    }
}
// sum of the group's 8 running sums in numpy's pairing
__device__ __forceinline__ float tree8(float r) {
#pragma clang fp contract(off)
    r = r + dpp8_f<0xB1>(r);   // quad_perm [1,0,3,2]: r0 + r1
    r = r + dpp8_f<0x4E>(r);   // quad_perm [2,3,0,1]: (r0 + r1) + (r2 + r3)
    return r + dpp8_f<0x141>(r);  // row_half_mirror: the other 4 of the 8
}

// the factors: float(1.0 - 0.02 i) for i = 0..15 (the double expression rounded once)
__constant__ const float kMseGrid[16] = {0x1p+0f, 0x1.f5c29p-1f, 0x1.eb851ep-1f, 0x1.e147aep-1f, 0x1.d70a3ep-1f, 0x1.ccccccp-1f, 0x1.c28f5cp-1f, 0x1.b851ecp-1f, 0x1.ae147ap-1f, 0x1.a3d70ap-1f, 0x1.99999ap-1f, 0x1.8f5c28p-1f, 0x1.851eb8p-1f, 0x1.7ae148p-1f, 0x1.70a3d8p-1f, 0x1.666666p-1f};

__global__ __launch_bounds__(256) void k_quantize_mse(const float *__restrict__ w, int O, int I, int bits, int gs,
                                                      uint8_t *__restrict__ q, uint16_t *__restrict__ s) {
    // no contraction: every product, difference and fp16 conversion rounds on its own
#pragma clang fp contract(off)
    const int j = threadIdx.x & 7;
    const int ng = I / gs;
    const long total = (long)O * ng;
    const long gid = (long)blockIdx.x * 32 + (threadIdx.x >> 3);
    const bool live = gid < total;
    const long gg = live ? gid : 0;
    const int row = (int)(gg / ng), g = (int)(gg % ng);
    const float *src = w + (size_t)row * I + (size_t)g * gs;
    const int n8 = gs >> 3, rem = gs & 7, base = gs - rem;
    float v[8], t[7];
#pragma unroll
    for (int m = 0; m < 8; ++m) v[m] = m < n8 ? src[j + 8 * m] : 0.f;
#pragma unroll
    for (int i = 0; i < 7; ++i) t[i] = i < rem ? src[base + i] : 0.f;
    // the largest magnitude and the signed value at its first index
    float a = -1.f, sv = 0.f;
    int ix = 1 << 30;
#pragma unroll
    for (int m = 0; m < 8; ++m)
        if (m < n8 && fabsf(v[m]) > a) {
            a = fabsf(v[m]);
            ix = j + 8 * m;
            sv = v[m];
        }
#pragma unroll
    for (int i = 0; i < 7; ++i)
        if (i < rem && fabsf(t[i]) > a) {  // held by every lane, behind every lane's own columns
            a = fabsf(t[i]);
            ix = base + i;
            sv = t[i];
        }
    argmax_step<0xB1>(a, ix, sv);
    argmax_step<0x4E>(a, ix, sv);
    argmax_step<0x141>(a, ix, sv);
    const float qmax = bits == 4 ? 7.f : 127.f, qmin = bits == 4 ? -8.f : -127.f;
    const uint16_t tiny = f32_to_f16_rne(1e-7f);
    const int nb = bits == 4 ? 2 : 1;
    uint16_t best_s = 0;
    float best_e = 0.f;
    for (int b = 0; b < nb; ++b) {
        const float bs = b == 0 ? a / qmax : sv / qmin;
        for (int i = 0; i < 16; ++i) {
            const float f = kMseGrid[i];
            float bf = bs * f;
            asm volatile("" : "+v"(bf));  // the fp32 product itself (else fused into one fp16 rounding)
            uint16_t s16 = f32_to_f16_rne(bf);
            if ((s16 & 0x7fffu) == 0) s16 = tiny;
            const float sf = f16_to_f32(s16);
            auto sq = [&](float x) {
                const float qv = fminf(fmaxf(rintf(x / sf), qmin), qmax);
                const float p = qv * sf;
                const float d = p - x;
                return d * d;
            };
            float r = sq(v[0]);
#pragma unroll
            for (int m = 1; m < 8; ++m)
                if (m < n8) r = r + sq(v[m]);
            float e = tree8(r);
            if (n8 == 0) e = 0.f;
#pragma unroll
            for (int k = 0; k < 7; ++k)
                if (k < rem) e = e + sq(t[k]);
            if ((b == 0 && i == 0) || e < best_e) {
                best_e = e;
                best_s = s16;
            }
        }
    }
    // quantise with the chosen scale, store in the record's packing
    const float sf = f16_to_f32(best_s);
    auto qz = [&](float x) { return (int)fminf(fmaxf(rintf(x / sf), qmin), qmax); };
    if (live && j == 0) s[(size_t)row * ng + g] = best_s;
    const size_t c0 = (size_t)row * I + (size_t)g * gs;  // first column of the group
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        if (m >= n8) break;
        const int qi = qz(v[m]);
        if (bits == 8) {
            if (live) reinterpret_cast<int8_t *>(q)[c0 + j + 8 * m] = (int8_t)qi;
        } else {
            const int partner = dpp8_i<0xB1>(qi);  // column j + 8m + 1 (j even)
            if (live && (j & 1) == 0) q[(c0 + j + 8 * m) / 2] = (uint8_t)((qi + 8) | ((partner + 8) << 4));
        }
    }
    if (live && j == 0) {
        for (int k = 0; k < rem; ++k) {
            const int qi = qz(t[k]);
            if (bits == 8) reinterpret_cast<int8_t *>(q)[c0 + base + k] = (int8_t)qi;
            else if ((k & 1) == 0) q[(c0 + base + k) / 2] = (uint8_t)((qi + 8) | ((qz(t[k + 1]) + 8) << 4));
        }
    }
}

// fp32 -> OCP e4m3fn code, round to nearest even, |x| saturating at 448 (code 0x7E)
__device__ __forceinline__ uint32_t f32_to_e4m3fn(float x) {
    const uint32_t sign = (__float_as_uint(x) >> 24) & 0x80u;
    const float a = fabsf(x);
    if (a != a) return 0x7Fu | sign;
    uint32_t code;
    if (a < 0.015625f) {  // below 2^-6: subnormal, step 2^-9
        code = (uint32_t)rintf(a * 512.0f);  // 8 rounds up to the smallest normal (code 8)
    } else {
        int e;
        const float m = frexpf(a, &e);            // a = m * 2^e, m in [0.5, 1)
        const float f = rintf((m * 2.0f - 1.0f) * 8.0f);  // 3 mantissa bits, exact operands
        int ex = e - 1 + 7;
        uint32_t mant = (uint32_t)f;
        if (mant == 8u) { mant = 0u; ++ex; }
        code = ex > 15 ? 0x7Fu : ((uint32_t)ex << 3) | mant;
        if (code > 0x7Eu) code = 0x7Eu;
    }
    return code == 0u ? 0u : (code | sign);
}

// Checkpoint-style FP8 block quantisation: one workgroup per 128 x 128 block,
// scale = amax / 448 (1 for an all-zero block), code = e4m3fn(w / scale).
__global__ __launch_bounds__(256) void k_quantize_fp8_block(const float *__restrict__ w, int O, int I,
                                                            uint8_t *__restrict__ q, float *__restrict__ s) {
    __shared__ float s_max[4];
    const int bo = blockIdx.y, bi = blockIdx.x;
    const int sc = (I + 127) >> 7;
    const int tid = threadIdx.x;
    float m = 0.f;
    for (int t = tid; t < 128 * 128; t += 256) {
        const int r = bo * 128 + (t >> 7), c = bi * 128 + (t & 127);
        if (r < O && c < I) m = fmaxf(m, fabsf(w[(size_t)r * I + c]));
    }
    m = wave_max(m);
    if ((tid & 63) == 0) s_max[tid >> 6] = m;
    __syncthreads();
    const float amax = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
    const float scale = amax > 0.f ? amax / 448.0f : 1.0f;
    if (tid == 0) s[(size_t)bo * sc + bi] = scale;
    for (int t = tid; t < 128 * 128; t += 256) {
        const int r = bo * 128 + (t >> 7), c = bi * 128 + (t & 127);
        if (r < O && c < I) q[(size_t)r * I + c] = (uint8_t)f32_to_e4m3fn(w[(size_t)r * I + c] / scale);
    }
}

}  // namespace moehip

using namespace moehip;

extern "C" int moehip_quantize_fp8_block(const float *w, int O, int I, void *q, float *s, void *stream) {
    MOEHIP_REQUIRE(w && q && s, "quantize_fp8_block: null pointer");
    MOEHIP_REQUIRE(O > 0 && I > 0, "quantize_fp8_block: bad sizes O=%d I=%d", O, I);
    hipLaunchKernelGGL(k_quantize_fp8_block, dim3((I + 127) / 128, (O + 127) / 128), dim3(256), 0, as_stream(stream), w,
                       O, I, reinterpret_cast<uint8_t *>(q), s);
    return check_launch("quantize_fp8_block");
}

extern "C" int moehip_quantize(const float *w, int O, int I, int bits, int gs, void *q, void *s, void *stream) {
    MOEHIP_REQUIRE(w && q && s, "quantize: null pointer");
    MOEHIP_REQUIRE(bits == 4 || bits == 8, "quantize: bits must be 4 or 8, got %d", bits);
    MOEHIP_REQUIRE(O > 0 && I > 0 && gs > 0 && gs <= 64 && gs % 2 == 0 && I % gs == 0,
                   "quantize: bad sizes O=%d I=%d gs=%d", O, I, gs);
    const long groups = (long)O * (I / gs);
    hipLaunchKernelGGL(k_quantize, dim3((unsigned)((groups + 3) / 4)), dim3(256), 0, as_stream(stream), w, O, I, bits, gs,
                       reinterpret_cast<uint8_t *>(q), reinterpret_cast<uint16_t *>(s));
    return check_launch("quantize");
}

extern "C" int moehip_quantize_mse(const float *w, int O, int I, int bits, int gs, void *q, void *s, void *stream) {
    MOEHIP_REQUIRE(w && q && s, "quantize_mse: null pointer");
    MOEHIP_REQUIRE(bits == 4 || bits == 8, "quantize_mse: bits must be 4 or 8, got %d", bits);
    MOEHIP_REQUIRE(O > 0 && I > 0 && gs > 0 && gs <= 64 && gs % 2 == 0 && I % gs == 0,
                   "quantize_mse: bad sizes O=%d I=%d gs=%d", O, I, gs);
    const long groups = (long)O * (I / gs);
    hipLaunchKernelGGL(k_quantize_mse, dim3((unsigned)((groups + 31) / 32)), dim3(256), 0, as_stream(stream), w, O, I,
                       bits, gs, reinterpret_cast<uint8_t *>(q), reinterpret_cast<uint16_t *>(s));
    return check_launch("quantize_mse");
}
