// GPTQ (moelab/quant.py:130-188) on the GPU: the column sweep of one block of at most 128
// columns, one lane per weight row. The Hessian preparation, its Cholesky factors and the lazy
// update of the columns right of a block (one float32 matrix product per block) are the host's
// (library linear algebra); this kernel does the part that is sequential in the columns.
//
// Per row, left to right over the block (quant.py:172-186): at a group's first column its scale
// is chosen from the row's weights as corrected so far (mse search or absmax, the arithmetic of
// k_quantize_mse / k_quantize: numpy's pairwise error sums, the first strictly smallest error);
// q = rint(w / s) clamped; err = (w - q s) / Hi[i][i]; every later column j of the block loses
// err * Hi[i][j]. Each product, difference and quotient rounds on its own (no contraction), so
// the sweep is bit-exact with the oracle's for the same Hinv block. The block of Hinv sits in LDS
// (every lane reads the same element: a broadcast), and so do the rows' weights.

#include "common.hpp"

namespace moehip {

constexpr int GQ_NB = 128;  // columns per block, at most

// float(1.0 - 0.02 i), i = 0..15 (quant.py:46)
__constant__ const float kGqGrid[16] = {0x1p+0f,       0x1.f5c29p-1f,  0x1.eb851ep-1f, 0x1.e147aep-1f,
                                        0x1.d70a3ep-1f, 0x1.ccccccp-1f, 0x1.c28f5cp-1f, 0x1.b851ecp-1f,
                                        0x1.ae147ap-1f, 0x1.a3d70ap-1f, 0x1.99999ap-1f, 0x1.8f5c28p-1f,
                                        0x1.851eb8p-1f, 0x1.7ae148p-1f, 0x1.70a3d8p-1f, 0x1.666666p-1f};

__device__ __forceinline__ uint16_t gq_f16(float v) {
    asm volatile("" : "+v"(v));  // round the float32 value itself (no fused product-to-fp16)
    return f32_to_f16_rne(v);
}

// fp16 scale of the GS values v[0..GS) (GS a multiple of 8): absmax (quant.py:74-76) or the mse
// search (quant.py:77-93)
template <int GS>
__device__ __forceinline__ uint16_t gq_scale(const float *v, int bits, int mse) {
#pragma clang fp contract(off)
    const float qmax = bits == 4 ? 7.f : 127.f, qmin = bits == 4 ? -8.f : -127.f;
    float a = -1.f, sv = 0.f;
#pragma unroll
    for (int k = 0; k < GS; ++k)
        if (fabsf(v[k]) > a) {  // strict: the first index of the largest magnitude
            a = fabsf(v[k]);
            sv = v[k];
        }
    const uint16_t tiny = f32_to_f16_rne(1e-7f);
    if (!mse) return gq_f16(fmaxf(a / qmax, 1e-7f));
    uint16_t best_s = 0;
    float best_e = 0.f;
    const int nbase = bits == 4 ? 2 : 1;
    for (int b = 0; b < nbase; ++b) {
        const float bs = b == 0 ? a / qmax : sv / qmin;
        for (int i = 0; i < 16; ++i) {
            uint16_t s16 = gq_f16(bs * kGqGrid[i]);
            if ((s16 & 0x7fffu) == 0) s16 = tiny;
            const float sf = f16_to_f32(s16);
            float r[8];
#pragma unroll
            for (int m = 0; m < GS / 8; ++m)
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const float x = v[8 * m + k];
                    const float qv = fminf(fmaxf(rintf(x / sf), qmin), qmax);
                    const float p = qv * sf;
                    const float d = p - x;
                    const float e2 = d * d;
                    r[k] = m == 0 ? e2 : r[k] + e2;
                }
            const float e = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
            if ((b == 0 && i == 0) || e < best_e) {
                best_e = e;
                best_s = s16;
            }
        }
    }
    return best_s;
}

// One workgroup = one wave of 64 rows. W (O, ldw) float32: columns i1 .. i1 + nb - 1 are read
// (not written); Hinv (ldh) the upper Cholesky factor of H^-1 (its block at (i1, i1) is used);
// q: int4 packed (row stride ldq bytes, byte (i1 + i) / 2 of a row) or int8; s (lds per row)
// fp16 scales of the block's groups; E (lde per row) the block's scaled errors (columns 0..nb-1).
// The rows' corrected weights live in LDS, column-major (sw[c][lane]: each lane reads and writes
// only its own column of it, conflict-free), beside the Hinv block (96 KB in all).
template <int GS>
__global__ __launch_bounds__(64) void k_gptq_block(const float *__restrict__ W, int ldw, const float *__restrict__ Hinv,
                                                   int ldh, int O, int i1, int nb, int bits, int mse,
                                                   uint8_t *__restrict__ q, int ldq, uint16_t *__restrict__ s,
                                                   int lds, float *__restrict__ E, int lde) {
#pragma clang fp contract(off)
    __shared__ __align__(16) float sh[GQ_NB * GQ_NB];
    __shared__ float sw[GQ_NB * 64];
    const int tid = threadIdx.x;
    for (int t = tid; t < GQ_NB * GQ_NB; t += 64) {
        const int a = t / GQ_NB, b = t % GQ_NB;
        sh[t] = (a < nb && b < nb) ? Hinv[(size_t)(i1 + a) * ldh + i1 + b] : 0.f;
    }
    const int r = blockIdx.x * 64 + tid;
    const bool live = r < O;
    const int rr = live ? r : O - 1;
    const float *src = W + (size_t)rr * ldw + i1;
    for (int c = 0; c < nb; ++c) sw[c * 64 + tid] = src[c];
    __syncthreads();
    const float qmax = bits == 4 ? 7.f : 127.f, qmin = bits == 4 ? -8.f : -127.f;
    float sf = 1.f;
    int qprev = 0;
    for (int i = 0; i < nb; ++i) {
        if (i % GS == 0) {
            float v[GS];
#pragma unroll
            for (int k = 0; k < GS; ++k) v[k] = sw[(i + k) * 64 + tid];
            const uint16_t s16 = gq_scale<GS>(v, bits, mse);
            sf = f16_to_f32(s16);
            if (live) s[(size_t)r * lds + (i1 + i) / GS] = s16;
        }
        const float wi = sw[i * 64 + tid];
        const float qv = fminf(fmaxf(rintf(wi / sf), qmin), qmax);
        const int qi = (int)qv;
        if (bits == 8) {
            if (live) reinterpret_cast<int8_t *>(q)[(size_t)r * ldq + i1 + i] = (int8_t)qi;
        } else if (i & 1) {
            if (live) q[(size_t)r * ldq + (i1 + i) / 2] = (uint8_t)((qprev + 8) | ((qi + 8) << 4));
        } else {
            qprev = qi;
        }
        const float p = qv * sf;
        const float d = wi - p;
        const float err = d / sh[i * GQ_NB + i];
        if (live) E[(size_t)r * lde + i] = err;
        const float *hrow = sh + i * GQ_NB;
        for (int j = i + 1; j < nb; ++j) {
            const float t = err * hrow[j];
            sw[j * 64 + tid] = sw[j * 64 + tid] - t;
        }
    }
}

}  // namespace moehip

using namespace moehip;

extern "C" int moehip_gptq_block(const float *W, int ldw, const float *Hinv, int ldh, int O, int i1, int nb, int bits,
                                 int gs, int method, void *q, int ldq, void *s, int lds, float *E, int lde,
                                 void *stream) {
    MOEHIP_REQUIRE(W && Hinv && q && s && E, "gptq_block: null pointer");
    MOEHIP_REQUIRE(bits == 4 || bits == 8, "gptq_block: bits must be 4 or 8, got %d", bits);
    MOEHIP_REQUIRE(gs == 32 || gs == 64, "gptq_block: group size %d (32 or 64)", gs);
    MOEHIP_REQUIRE(method == 0 || method == 1, "gptq_block: method %d (0 absmax, 1 mse)", method);
    MOEHIP_REQUIRE(O > 0 && nb > 0 && nb <= GQ_NB && nb % gs == 0 && i1 >= 0 && i1 % gs == 0 && i1 + nb <= ldw &&
                       i1 + nb <= ldh && lde >= nb && lds >= (i1 + nb) / gs && ldq >= (bits == 4 ? (i1 + nb) / 2 : i1 + nb),
                   "gptq_block: O=%d i1=%d nb=%d (nb <= %d, multiples of gs=%d) ldw=%d ldh=%d ldq=%d lds=%d lde=%d", O, i1,
                   nb, GQ_NB, gs, ldw, ldh, ldq, lds, lde);
    const dim3 grid((unsigned)((O + 63) / 64));
    hipStream_t st = as_stream(stream);
    uint8_t *qb = reinterpret_cast<uint8_t *>(q);
    uint16_t *sb = reinterpret_cast<uint16_t *>(s);
    if (gs == 64)
        hipLaunchKernelGGL(k_gptq_block<64>, grid, dim3(64), 0, st, W, ldw, Hinv, ldh, O, i1, nb, bits, method, qb, ldq, sb,
                           lds, E, lde);
    else
        hipLaunchKernelGGL(k_gptq_block<32>, grid, dim3(64), 0, st, W, ldw, Hinv, ldh, O, i1, nb, bits, method, qb, ldq, sb,
                           lds, E, lde);
    return check_launch("gptq_block");
}
