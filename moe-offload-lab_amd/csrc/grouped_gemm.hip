// Expert-sorted grouped GEMM for T > 1 tokens (prefill chunks, batched decode) on MFMA.
//
// Replaces the reference's prefill expert path (moelab/runtime.py:418-436 `_run_grouped_tokens`
// and :352-353: per expert y = expert_ffn(x[tok]), out.index_add_(tok, y * w)) for int4 gs64
// records. The pairs (token, slot) are sorted by expert (moehip_dispatch); per expert the tokens
// form the M dimension of two GEMMs:
//   up:   h (n_e, I) = silu(X_e gate^T) * (X_e up^T)     K = H, weight rows 2I (gate; up)
//   down: y (n_e, H) = w_pair * (h down^T)               K = I, weight rows H
// followed by an ordered combine out[t] = sum over the token's slots in slot order.
//
// MFMA: v_mfma_f32_16x16x32_f16. A = activations (16 tokens x 32 K), B = weights (32 K x 16
// rows), D = 16 tokens x 16 rows in fp32. One K step of 64 = one int4 scale group: each lane
// loads 8 bytes (16 nibbles) of its weight row, turns each 8 nibbles into fp16 1024 + n with
// one v_and_or_b32 per pair (exact), runs the group's two MFMAs, and folds the group into its
// fp32 accumulators as acc += scale * (D - 1032 * sum_k x_k) (the offset 1024 + 8 removed with
// the group sum of the activations, the scale applied in fp32): the products and the scale are
// exact, as in the reference's dequantise-then-matmul path.
//
// Activations: every token row is scaled by a power of two into fp16 range (exact for fp16 and
// bf16 inputs; the factor is applied back to the outputs). h enters the down GEMM as an fp16
// hi + lo pair (two MFMAs per step), i.e. ~22 bits of its fp32 value.
//
// Each workgroup (4 waves) owns one expert and a block of weight rows (up: 128 h columns =
// 128 gate + 128 up rows; down: 256 output rows), every wave 4 subtiles of 16 rows, for up to
// 64 tokens per pass; activations of the next K step are staged into LDS (double buffered,
// rows padded to 144 bytes so the fragment reads are bank-conflict free) while the current
// step computes.

#include "gemv_core.hpp"

namespace moehip {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int GG_MT = 4;            // 16-token M tiles per pass
constexpr int GG_TOK = GG_MT * 16;  // tokens per pass
constexpr int GG_NS = 4;            // 16-row N subtiles per wave
constexpr int GG_KG = 64;           // K per step (= the int4 group size)
constexpr int GG_LDW = 72;          // LDS row stride in halves (64 + 8: 144 bytes)

// exponent e of a row so that max|row| * 2^-e lies in [2^14, 2^15) (0 for an all-zero row)
__device__ __forceinline__ int row_exp(float m) {
    return (m > 0.f && m <= 3.0e38f) ? max(ilogbf(m) - 14, -100) : 0;
}

// one wave per row: ex[r] = row_exp(max |x[r, :]|)
template <int DT>
__global__ __launch_bounds__(256) void k_row_exp(const void *__restrict__ x, int R, int C, int *__restrict__ ex) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= R) return;
    float m = 0.f;
    for (int c = lane; c < C; c += 64) m = fmaxf(m, fabsf(ld_act<DT>(x, (size_t)r * C + c)));
    m = wave_max(m);
    if (lane == 0) ex[r] = row_exp(m);
}

// 8 nibbles (one dword of an int4 row) -> fp16 (1024 + n) in the order c0 c4 c1 c5 c2 c6 c3 c7.
// Plain C on purpose (not the inline-asm and_or of the GEMV kernels): the results feed MFMA
// operands, and only compiler-generated instructions get the VALU-write -> MFMA-read wait
// states inserted by the compiler's hazard recognizer.
__device__ __forceinline__ f16x8 deq8(uint32_t d) {
    uint4 u;
    u.x = (d & 0x000F000Fu) | 0x64006400u;
    u.y = ((d >> 4) & 0x000F000Fu) | 0x64006400u;
    u.z = ((d >> 8) & 0x000F000Fu) | 0x64006400u;
    u.w = ((d >> 12) & 0x000F000Fu) | 0x64006400u;
    return __builtin_bit_cast(f16x8, u);
}

// 8 consecutive activation values -> fp16 pairs in the same order (c0,c4) (c1,c5) (c2,c6) (c3,c7)
__device__ __forceinline__ uint4 perm8(const float *v) {
    return make_uint4(pack_h2(v[0], v[4]), pack_h2(v[1], v[5]), pack_h2(v[2], v[6]), pack_h2(v[3], v[7]));
}

// Activation staging for one K step: thread tid -> token tid / 4, K values 16 * (tid % 4) ..+16
// of the step (one lane-group slice: LDS positions 16 q .. 16 q + 16, two halves of 8), written
// permuted as the MFMA fragments expect; the group sum of the fp16 values goes to xg[token].
struct StageRegs {
    float v[16];
};

// loads of the next step (activations x (DT) or h (fp32), row `row` scaled by 2^-e)
template <int DT>
__device__ __forceinline__ void stage_load(const void *src, size_t row, int ld, int k0, bool ok, StageRegs &r) {
    const int part = threadIdx.x & 3;
    const size_t base = row * (size_t)ld + k0 + 16 * part;
    if constexpr (DT == MOEHIP_DT_F32) {
        const float4 *p = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(src) + base);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const float4 f = ok ? p[m] : make_float4(0.f, 0.f, 0.f, 0.f);
            r.v[4 * m + 0] = f.x;
            r.v[4 * m + 1] = f.y;
            r.v[4 * m + 2] = f.z;
            r.v[4 * m + 3] = f.w;
        }
    } else {
        const uint4 *p = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(src) + base);
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const uint4 u = ok ? p[m] : make_uint4(0, 0, 0, 0);
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                r.v[8 * m + 2 * q] = DT == MOEHIP_DT_F16 ? f16_to_f32(w[q] & 0xffffu) : bf16_to_f32(w[q] & 0xffffu);
                r.v[8 * m + 2 * q + 1] = DT == MOEHIP_DT_F16 ? f16_to_f32(w[q] >> 16) : bf16_to_f32(w[q] >> 16);
            }
        }
    }
}

// scaled fp16 (hi, and lo = the rounding remainder when LO) into LDS + group sums
template <bool LO>
__device__ __forceinline__ void stage_store(const StageRegs &r, float down, _Float16 *s_hi, _Float16 *s_lo,
                                            float *s_sum) {
    const int tok = threadIdx.x >> 2, part = threadIdx.x & 3;
    float hv[16], lv[16];
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float v = r.v[i] * down;
        hv[i] = f16_to_f32(f32_to_f16_rne(v));
        lv[i] = LO ? f16_to_f32(f32_to_f16_rne(v - hv[i])) : 0.f;
        sum += hv[i] + lv[i];
    }
    uint4 *dh = reinterpret_cast<uint4 *>(s_hi + tok * GG_LDW + 16 * part);
    dh[0] = perm8(hv);
    dh[1] = perm8(hv + 8);
    if constexpr (LO) {
        uint4 *dl = reinterpret_cast<uint4 *>(s_lo + tok * GG_LDW + 16 * part);
        dl[0] = perm8(lv);
        dl[1] = perm8(lv + 8);
    }
    sum += dpp_f<0xB1>(sum);  // the 4 threads of a token are one quad
    sum += dpp_f<0x4E>(sum);
    if (part == 0) s_sum[tok] = sum;
}

// one K step of MFMAs for a wave: nm valid M tiles, GG_NS weight subtiles
template <bool LO>
__device__ __forceinline__ void mma_step(const _Float16 *s_hi, const _Float16 *s_lo, const float *s_sum, const uint2 (&bq)[GG_NS],
                                         const float (&sc)[GG_NS], int nm, f32x4 (&acc)[GG_MT][GG_NS]) {
    const int lane = threadIdx.x & 63;
    const int m = lane & 15, q = lane >> 4;
    f16x8 b0[GG_NS], b1[GG_NS];
#pragma unroll
    for (int j = 0; j < GG_NS; ++j) {
        b0[j] = deq8(bq[j].x);
        b1[j] = deq8(bq[j].y);
    }
#pragma unroll
    for (int mt = 0; mt < GG_MT; ++mt) {
        if (mt >= nm) break;
        const _Float16 *ah = s_hi + (mt * 16 + m) * GG_LDW + 16 * q;
        const f16x8 a0 = *reinterpret_cast<const f16x8 *>(ah);
        const f16x8 a1 = *reinterpret_cast<const f16x8 *>(ah + 8);
        f16x8 l0, l1;
        if constexpr (LO) {
            const _Float16 *al = s_lo + (mt * 16 + m) * GG_LDW + 16 * q;
            l0 = *reinterpret_cast<const f16x8 *>(al);
            l1 = *reinterpret_cast<const f16x8 *>(al + 8);
        }
        const float4 xg = *reinterpret_cast<const float4 *>(s_sum + mt * 16 + 4 * q);
        const float xgv[4] = {xg.x, xg.y, xg.z, xg.w};
#pragma unroll
        for (int j = 0; j < GG_NS; ++j) {
            f32x4 d = {0.f, 0.f, 0.f, 0.f};
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b0[j], d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b1[j], d, 0, 0, 0);
            if constexpr (LO) {
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(l0, b0[j], d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(l1, b1[j], d, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[mt][j][r] = fmaf(sc[j], fmaf(-1032.0f, xgv[r], d[r]), acc[mt][j][r]);
        }
    }
}

// ---------------------------------------------------------------------------------------
// up: grid (ceil(I / 128), E). Wave w: h columns c0 = 128 bx + 32 w .. +32; subtiles 0, 1 =
// gate rows c0 + 16 j, subtiles 2, 3 = up rows I + c0 + 16 (j - 2).
// ---------------------------------------------------------------------------------------
template <int XDT>
__global__ __launch_bounds__(256) void k_gemm_up(const void *__restrict__ x, const int *__restrict__ xe, int H, int I,
                                                 int k, const int32_t *__restrict__ offsets,
                                                 const int32_t *__restrict__ sorted_pos, const int64_t *__restrict__ tab,
                                                 int gs, float *__restrict__ h) {
    __shared__ __align__(16) _Float16 s_x[2][GG_TOK * GG_LDW];
    __shared__ __align__(16) float s_sum[2][GG_TOK];
    const int e = blockIdx.y;
    const int p0 = offsets[e], ne = offsets[e + 1] - p0;
    const uint8_t *qb = reinterpret_cast<const uint8_t *>(tab[4 * e + 0]);
    const uint16_t *sb = reinterpret_cast<const uint16_t *>(tab[4 * e + 1]);
    if (ne <= 0 || qb == nullptr) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int c0 = blockIdx.x * 128 + wave * 32;
    const size_t RB = (size_t)H / 2;
    const int ng = H / gs;
    const int nsteps = H / GG_KG;
    int rowj[GG_NS];
    bool okj[GG_NS];
#pragma unroll
    for (int j = 0; j < GG_NS; ++j) {
        const int col = c0 + 16 * (j & 1) + (lane & 15);
        okj[j] = col < I;
        rowj[j] = (j < 2 ? 0 : I) + min(col, I - 1);
    }
    for (int m0 = 0; m0 < ne; m0 += GG_TOK) {
        const int mn = min(GG_TOK, ne - m0);
        const int nm = (mn + 15) / 16;
        // this thread's staging token
        const int stok = tid >> 2;
        const bool sok = stok < mn;
        const int t_row = sok ? sorted_pos[p0 + m0 + stok] / k : 0;
        const float sdown = sok ? ldexpf(1.0f, -xe[t_row]) : 0.f;
        f32x4 acc[GG_MT][GG_NS];
#pragma unroll
        for (int mt = 0; mt < GG_MT; ++mt)
#pragma unroll
            for (int j = 0; j < GG_NS; ++j) acc[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        StageRegs sr;
        uint2 bq[GG_NS], bn[GG_NS];
        uint32_t sraw[GG_NS], snext[GG_NS];
        stage_load<XDT>(x, (size_t)t_row, H, 0, sok, sr);
#pragma unroll
        for (int j = 0; j < GG_NS; ++j) {
            bq[j] = *reinterpret_cast<const uint2 *>(qb + (size_t)rowj[j] * RB + 8 * (lane >> 4));
            sraw[j] = sb[(size_t)rowj[j] * ng];
        }
        stage_store<false>(sr, sdown, s_x[0], nullptr, s_sum[0]);
        __syncthreads();
        for (int st = 0; st < nsteps; ++st) {
            const int buf = st & 1;
            const bool more = st + 1 < nsteps;
            if (more) {  // next step's loads are in flight while this one computes
                stage_load<XDT>(x, (size_t)t_row, H, (st + 1) * GG_KG, sok, sr);
#pragma unroll
                for (int j = 0; j < GG_NS; ++j) {
                    bn[j] = *reinterpret_cast<const uint2 *>(qb + (size_t)rowj[j] * RB + (size_t)(st + 1) * 32 +
                                                              8 * (lane >> 4));
                    snext[j] = sb[(size_t)rowj[j] * ng + (st + 1) * GG_KG / gs];
                }
            }
            float sc[GG_NS];
#pragma unroll
            for (int j = 0; j < GG_NS; ++j) sc[j] = okj[j] ? f16_to_f32(sraw[j]) : 0.f;
            mma_step<false>(s_x[buf], nullptr, s_sum[buf], bq, sc, nm, acc);
            if (more) {
                stage_store<false>(sr, sdown, s_x[buf ^ 1], nullptr, s_sum[buf ^ 1]);
#pragma unroll
                for (int j = 0; j < GG_NS; ++j) {
                    bq[j] = bn[j];
                    sraw[j] = snext[j];
                }
            }
            __syncthreads();
        }
        // epilogue: h = silu(gate) * up, scaled back by the token's 2^e
#pragma unroll
        for (int mt = 0; mt < GG_MT; ++mt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tok = mt * 16 + 4 * (lane >> 4) + r;
                if (tok >= mn) continue;
                const int p = p0 + m0 + tok;
                const float up = ldexpf(1.0f, xe[sorted_pos[p] / k]);
#pragma unroll
                for (int jp = 0; jp < 2; ++jp) {
                    const int col = c0 + 16 * jp + (lane & 15);
                    if (col < I) h[(size_t)p * I + col] = silu_mul(acc[mt][jp][r] * up, acc[mt][jp + 2][r] * up);
                }
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------------------
// down: grid (ceil(H / 256), E). Wave w: output rows r0 = 256 bx + 64 w + 16 j. h rows enter as
// fp16 hi + lo scaled by the pair's 2^-e; y[p, row] = w[pair] * (down_row . h_p).
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_gemm_down(const float *__restrict__ h, const int *__restrict__ he, int H, int I,
                                                   const int32_t *__restrict__ offsets,
                                                   const int32_t *__restrict__ sorted_pos, const int64_t *__restrict__ tab,
                                                   const float *__restrict__ w, int gs, float *__restrict__ y) {
    __shared__ __align__(16) _Float16 s_hi[2][GG_TOK * GG_LDW];
    __shared__ __align__(16) _Float16 s_lo[2][GG_TOK * GG_LDW];
    __shared__ __align__(16) float s_sum[2][GG_TOK];
    const int e = blockIdx.y;
    const int p0 = offsets[e], ne = offsets[e + 1] - p0;
    if (ne <= 0) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint8_t *qb = reinterpret_cast<const uint8_t *>(tab[4 * e + 2]);
    const uint16_t *sb = reinterpret_cast<const uint16_t *>(tab[4 * e + 3]);
    if (qb == nullptr) {  // expert not resident: its pairs contribute nothing
        for (int i = tid; i < ne * 256; i += 256) {
            const int p = p0 + i / 256, row = blockIdx.x * 256 + i % 256;
            if (row < H) y[(size_t)p * H + row] = 0.f;
        }
        return;
    }
    const size_t RB = (size_t)I / 2;
    const int ng = I / gs;
    const int nsteps = I / GG_KG;
    int rowj[GG_NS];
    bool okj[GG_NS];
#pragma unroll
    for (int j = 0; j < GG_NS; ++j) {
        const int row = blockIdx.x * 256 + wave * 64 + 16 * j + (lane & 15);
        okj[j] = row < H;
        rowj[j] = min(row, H - 1);
    }
    for (int m0 = 0; m0 < ne; m0 += GG_TOK) {
        const int mn = min(GG_TOK, ne - m0);
        const int nm = (mn + 15) / 16;
        const int stok = tid >> 2;
        const bool sok = stok < mn;
        const size_t prow = (size_t)(p0 + m0 + min(stok, mn - 1));
        const float sdown = sok ? ldexpf(1.0f, -he[prow]) : 0.f;
        f32x4 acc[GG_MT][GG_NS];
#pragma unroll
        for (int mt = 0; mt < GG_MT; ++mt)
#pragma unroll
            for (int j = 0; j < GG_NS; ++j) acc[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        StageRegs sr;
        uint2 bq[GG_NS], bn[GG_NS];
        uint32_t sraw[GG_NS], snext[GG_NS];
        stage_load<MOEHIP_DT_F32>(h, prow, I, 0, sok, sr);
#pragma unroll
        for (int j = 0; j < GG_NS; ++j) {
            bq[j] = *reinterpret_cast<const uint2 *>(qb + (size_t)rowj[j] * RB + 8 * (lane >> 4));
            sraw[j] = sb[(size_t)rowj[j] * ng];
        }
        stage_store<true>(sr, sdown, s_hi[0], s_lo[0], s_sum[0]);
        __syncthreads();
        for (int st = 0; st < nsteps; ++st) {
            const int buf = st & 1;
            const bool more = st + 1 < nsteps;
            if (more) {
                stage_load<MOEHIP_DT_F32>(h, prow, I, (st + 1) * GG_KG, sok, sr);
#pragma unroll
                for (int j = 0; j < GG_NS; ++j) {
                    bn[j] = *reinterpret_cast<const uint2 *>(qb + (size_t)rowj[j] * RB + (size_t)(st + 1) * 32 +
                                                              8 * (lane >> 4));
                    snext[j] = sb[(size_t)rowj[j] * ng + (st + 1) * GG_KG / gs];
                }
            }
            float sc[GG_NS];
#pragma unroll
            for (int j = 0; j < GG_NS; ++j) sc[j] = okj[j] ? f16_to_f32(sraw[j]) : 0.f;
            mma_step<true>(s_hi[buf], s_lo[buf], s_sum[buf], bq, sc, nm, acc);
            if (more) {
                stage_store<true>(sr, sdown, s_hi[buf ^ 1], s_lo[buf ^ 1], s_sum[buf ^ 1]);
#pragma unroll
                for (int j = 0; j < GG_NS; ++j) {
                    bq[j] = bn[j];
                    sraw[j] = snext[j];
                }
            }
            __syncthreads();
        }
#pragma unroll
        for (int mt = 0; mt < GG_MT; ++mt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tok = mt * 16 + 4 * (lane >> 4) + r;
                if (tok >= mn) continue;
                const int p = p0 + m0 + tok;
                const float f = w[sorted_pos[p]] * ldexpf(1.0f, he[p]);
#pragma unroll
                for (int j = 0; j < GG_NS; ++j)
                    if (okj[j]) y[(size_t)p * H + rowj[j]] = f * acc[mt][j][r];
            }
        }
        __syncthreads();
    }
}

// out[t] = sum over slots j (in order) of y[rank[t k + j]] (+ out if accumulate) (+ add)
template <int DT>
__global__ __launch_bounds__(256) void k_combine_pairs(const float *__restrict__ y, const int32_t *__restrict__ rank,
                                                       int T, int k, int H, const void *__restrict__ add,
                                                       void *__restrict__ out, int accumulate) {
    const int t = blockIdx.x;
    for (int c = threadIdx.x; c < H; c += 256) {
        float s = 0.f;
        for (int j = 0; j < k; ++j) {
            const int p = rank[(size_t)t * k + j];
            if (p >= 0) s += y[(size_t)p * H + c];
        }
        if (accumulate) s += ld_act<DT>(out, (size_t)t * H + c);
        if (add != nullptr) s += ld_act<DT>(add, (size_t)t * H + c);
        st_act<DT>(out, (size_t)t * H + c, s);
    }
}

struct GgLayout {
    size_t xe, he, h, y, total;
};
static GgLayout gg_layout(int T, int k, int H, int I) {
    auto al = [](size_t v) { return (v + 255) / 256 * 256; };
    GgLayout L;
    const size_t NP = (size_t)T * k;
    size_t off = 0;
    L.xe = off;
    off = al(off + (size_t)T * 4);
    L.he = off;
    off = al(off + NP * 4);
    L.h = off;
    off = al(off + NP * I * 4);
    L.y = off;
    off = al(off + NP * H * 4);
    L.total = off;
    return L;
}

}  // namespace moehip

using namespace moehip;

extern "C" size_t moehip_grouped_gemm_workspace_bytes(int T, int k, int H, int I) {
    if (T <= 0 || k <= 0 || H <= 0 || I <= 0) return 0;
    return gg_layout(T, k, H, I).total;
}

extern "C" int moehip_grouped_gemm(int prec, const int64_t *tab, const void *x, int xdtype, int T, int H, int I, int k,
                                   int E, int gs, const int32_t *offsets, const int32_t *sorted_pos,
                                   const int32_t *rank, const float *w, void *out, const void *add, int accumulate,
                                   void *ws, size_t ws_bytes, void *stream) {
    MOEHIP_REQUIRE(tab && x && offsets && sorted_pos && rank && w && out && ws, "grouped_gemm: null pointer");
    MOEHIP_REQUIRE(prec == MOEHIP_PREC_INT4, "grouped_gemm: precision %d (int4 records)", prec);
    MOEHIP_REQUIRE(gs == GG_KG, "grouped_gemm: group size %d (64)", gs);
    MOEHIP_REQUIRE(T > 0 && k > 0 && E > 0 && H > 0 && I > 0 && H % GG_KG == 0 && I % GG_KG == 0,
                   "grouped_gemm: T=%d k=%d E=%d H=%d I=%d (H, I multiples of 64)", T, k, E, H, I);
    MOEHIP_REQUIRE(xdtype == MOEHIP_DT_F16 || xdtype == MOEHIP_DT_BF16, "grouped_gemm: activation dtype %d", xdtype);
    MOEHIP_REQUIRE(((uintptr_t)x % 16) == 0, "grouped_gemm: x must be 16-byte aligned");
    const GgLayout L = gg_layout(T, k, H, I);
    MOEHIP_REQUIRE(ws_bytes >= L.total && ((uintptr_t)ws % 256) == 0, "grouped_gemm: workspace %zu < %zu bytes (or unaligned)",
                   ws_bytes, L.total);
    uint8_t *wsb = reinterpret_cast<uint8_t *>(ws);
    int *xe = reinterpret_cast<int *>(wsb + L.xe);
    int *he = reinterpret_cast<int *>(wsb + L.he);
    float *h = reinterpret_cast<float *>(wsb + L.h);
    float *y = reinterpret_cast<float *>(wsb + L.y);
    const int NP = T * k;
    hipStream_t st = as_stream(stream);
    if (xdtype == MOEHIP_DT_F16) {
        hipLaunchKernelGGL((k_row_exp<MOEHIP_DT_F16>), dim3((T + 3) / 4), dim3(256), 0, st, x, T, H, xe);
        hipLaunchKernelGGL((k_gemm_up<MOEHIP_DT_F16>), dim3((I + 127) / 128, E), dim3(256), 0, st, x, xe, H, I, k,
                           offsets, sorted_pos, tab, gs, h);
    } else {
        hipLaunchKernelGGL((k_row_exp<MOEHIP_DT_BF16>), dim3((T + 3) / 4), dim3(256), 0, st, x, T, H, xe);
        hipLaunchKernelGGL((k_gemm_up<MOEHIP_DT_BF16>), dim3((I + 127) / 128, E), dim3(256), 0, st, x, xe, H, I, k,
                           offsets, sorted_pos, tab, gs, h);
    }
    hipLaunchKernelGGL((k_row_exp<MOEHIP_DT_F32>), dim3((NP + 3) / 4), dim3(256), 0, st, h, NP, I, he);
    hipLaunchKernelGGL(k_gemm_down, dim3((H + 255) / 256, E), dim3(256), 0, st, h, he, H, I, offsets, sorted_pos, tab, w,
                       gs, y);
    if (xdtype == MOEHIP_DT_F16)
        hipLaunchKernelGGL((k_combine_pairs<MOEHIP_DT_F16>), dim3(T), dim3(256), 0, st, y, rank, T, k, H, add, out,
                           accumulate);
    else
        hipLaunchKernelGGL((k_combine_pairs<MOEHIP_DT_BF16>), dim3(T), dim3(256), 0, st, y, rank, T, k, H, add, out,
                           accumulate);
    return check_launch("grouped_gemm");
}
