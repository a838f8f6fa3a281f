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

}  // namespace moehip

using namespace moehip;

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
