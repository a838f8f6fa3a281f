// Store-side absmax quantisation (moelab/quant.py:57-61, 74-76, 96-127) on the GPU, bit-exact:
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
