// Per-lane pieces shared by the one-token layer kernels: record formats, the lane's slice of
// the activation vector in the operand order of the chunk dot products, tagged cross-workgroup
// words, and the order-preserving keys of the router's top-k.
#pragma once

#include "gemv_core.hpp"

namespace moehip {

// ---------------------------------------------------------------------------------------
// formats: values per 16-byte chunk, chunks per lane (32 values per lane), passes per item
// (so that a lane holds 8 chunks of an item: 2 * NPU * CPL for gate/up rows, NPD * CPL for
// down rows), vector pairs per chunk, and whether the fp16 dot2 path applies.
// ---------------------------------------------------------------------------------------
template <int PREC> struct DlFmt {
    static constexpr int VPC = Fmt<PREC>::VPC;
    static constexpr int CPL = 32 / VPC;
    static constexpr int NPU = 4 / CPL;
    static constexpr int NPD = 8 / CPL;
    static constexpr int XPC = VPC / 2;
};
template <int PREC, int XDT> struct UseDot2 {
    static constexpr bool v = XDT != MOEHIP_DT_F32 &&
                              (PREC == MOEHIP_PREC_INT4 || PREC == MOEHIP_PREC_INT8 || PREC == MOEHIP_PREC_F16);
};

// ---------------------------------------------------------------------------------------
// coherent (agent-scope) accesses
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ void st_co(float *p, float v) {
    __hip_atomic_store(reinterpret_cast<uint32_t *>(p), __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_co(const float *p) {
    return __uint_as_float(__hip_atomic_load(reinterpret_cast<uint32_t *>(const_cast<float *>(p)), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ void st_co64(int64_t *p, int64_t v) {
    __hip_atomic_store(reinterpret_cast<unsigned long long *>(p), (unsigned long long)v, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int64_t ld_co64(const int64_t *p) {
    return (int64_t)__hip_atomic_load(reinterpret_cast<unsigned long long *>(const_cast<int64_t *>(p)),
                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_co32(uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t add_co32(uint32_t *p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_co32(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// tagged words: (tag << 32) | payload, one atomic 64-bit store / load each
__device__ __forceinline__ void st_tag(uint64_t *p, uint32_t payload, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_tag(const uint64_t *p) {
    return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool tag_ok(uint64_t v, uint32_t tag) { return (uint32_t)(v >> 32) == tag; }

// exponential backoff between polls: s_sleep 1 .. 8 (up to ~500 cycles), so hundreds of
// polling workgroups do not congest a memory channel
__device__ __forceinline__ void backoff(int &nap, int cap = 8) {
    switch (nap) {  // s_sleep takes an immediate
        case 1: __builtin_amdgcn_s_sleep(1); break;
        case 2: __builtin_amdgcn_s_sleep(2); break;
        case 4: __builtin_amdgcn_s_sleep(4); break;
        case 8: __builtin_amdgcn_s_sleep(8); break;
        default: __builtin_amdgcn_s_sleep(16); break;
    }
    if (nap < cap) nap <<= 1;
}
__device__ __forceinline__ void flag_error(uint32_t *err) {
    __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Select element i of a small argument array without dynamic indexing. The elements pass
// through v_readfirstlane (they are uniform) so that the compiler cannot turn the select of
// loads into a load from a selected address: that would copy the whole kernel-argument
// struct to private memory.
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int64_t uni64(int64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}
// ---------------------------------------------------------------------------------------
// vector preparation: the 32 vector values of a lane (CPL chunks of VPC values) as fp16 pairs
// in the order the chunk dot consumes them, plus per chunk the correction of the weights'
// 1024-offsets and the power of two the chunk was scaled by.
//   int4: per 8 values (v0,v4) (v1,v5) (v2,v6) (v3,v7); corr = -1032 * sum(even) - 72 * sum(odd)
//   int8: per 4 values (v0,v2) (v1,v3);                 corr = -1152 * sum
//   fp16: natural pairs;                                corr = 0
// ---------------------------------------------------------------------------------------
// pairs of one chunk from 32-bit words w[0 .. VPC/2) (each word = 2 consecutive fp16 values)
template <int PREC>
__device__ __forceinline__ void pair_chunk(const uint32_t *w, uint32_t *xp, float &corr) {
    if constexpr (PREC == MOEHIP_PREC_INT4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t d0 = w[4 * j + 0], d1 = w[4 * j + 1], d2 = w[4 * j + 2], d3 = w[4 * j + 3];
            xp[4 * j + 0] = lo_lo(d0, d2);
            xp[4 * j + 1] = hi_hi(d0, d2);
            xp[4 * j + 2] = lo_lo(d1, d3);
            xp[4 * j + 3] = hi_hi(d1, d3);
        }
    } else if constexpr (PREC == MOEHIP_PREC_INT8) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t d0 = w[2 * j + 0], d1 = w[2 * j + 1];
            xp[2 * j + 0] = lo_lo(d0, d1);
            xp[2 * j + 1] = hi_hi(d0, d1);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) xp[j] = w[j];
    }
    corr = chunk_corr<PREC>(xp);
}

// fp32 values -> fp16 words scaled by 2^-e (e from the chunk's largest magnitude, so that it
// lands in [2^14, 2^15)); returns 2^e
template <int VPC>
__device__ __forceinline__ float scale_to_h(const float *v, uint32_t *w) {
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < VPC; ++i) m = fmaxf(m, fabsf(v[i]));
    int e = 0;
    if (m > 0.f && m <= 3.0e38f) e = max(ilogbf(m) - 14, -100);
    const float down = ldexpf(1.0f, -e);
#pragma unroll
    for (int i = 0; i < VPC / 2; ++i) w[i] = pack_h2(v[2 * i] * down, v[2 * i + 1] * down);
    return ldexpf(1.0f, e);
}

// vector registers of one lane for one item format
template <int PREC, int XDT>
struct LaneVec {
    static constexpr bool D2 = UseDot2<PREC, XDT>::v;
    static constexpr int CPL = DlFmt<PREC>::CPL;
    uint32_t xp[D2 ? 16 : 1];
    float corr[CPL];
    float p2e[CPL];
    float v[D2 ? 1 : 32];
    float vs[CPL];
};

// x (activation dtype, global) -> lane vector; chunk i of the lane is chunk cl + i * G of the row
template <int PREC, int XDT>
__device__ __forceinline__ void load_x(const void *x, int cl, int G, int C, LaneVec<PREC, XDT> &lv) {
    constexpr int VPC = DlFmt<PREC>::VPC, CPL = DlFmt<PREC>::CPL;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c = min(cl + i * G, C - 1);  // lanes past the row end compute on a copy, never stored
        lv.p2e[i] = 1.0f;
        lv.corr[i] = 0.f;
        lv.vs[i] = 0.f;
        if constexpr (XDT == MOEHIP_DT_F32) {
            const float4 *src = reinterpret_cast<const float4 *>(x) + (size_t)c * (VPC / 4);
            float acc = 0.f;
#pragma unroll
            for (int m = 0; m < VPC / 4; ++m) {
                const float4 f = src[m];
                lv.v[i * VPC + 4 * m + 0] = f.x;
                lv.v[i * VPC + 4 * m + 1] = f.y;
                lv.v[i * VPC + 4 * m + 2] = f.z;
                lv.v[i * VPC + 4 * m + 3] = f.w;
                acc += (f.x + f.y) + (f.z + f.w);
            }
            lv.vs[i] = acc;
        } else {
            const uint4 *src = reinterpret_cast<const uint4 *>(x) + (size_t)c * (VPC / 8);
            uint32_t w[VPC / 2];
#pragma unroll
            for (int m = 0; m < VPC / 8; ++m) {
                const uint4 u = src[m];
                w[4 * m + 0] = u.x;
                w[4 * m + 1] = u.y;
                w[4 * m + 2] = u.z;
                w[4 * m + 3] = u.w;
            }
            if constexpr (LaneVec<PREC, XDT>::D2) {
                if constexpr (XDT == MOEHIP_DT_F16) {
                    pair_chunk<PREC>(w, lv.xp + i * DlFmt<PREC>::XPC, lv.corr[i]);
                } else {  // bf16 -> fp16 scaled by a power of two
                    float f[VPC];
#pragma unroll
                    for (int m = 0; m < VPC / 2; ++m) {
                        f[2 * m] = bf16_to_f32(w[m] & 0xffffu);
                        f[2 * m + 1] = bf16_to_f32(w[m] >> 16);
                    }
                    uint32_t hw[VPC / 2];
                    lv.p2e[i] = scale_to_h<VPC>(f, hw);
                    pair_chunk<PREC>(hw, lv.xp + i * DlFmt<PREC>::XPC, lv.corr[i]);
                }
            } else {
                float acc = 0.f;
#pragma unroll
                for (int m = 0; m < VPC / 2; ++m) {
                    const float a0 = XDT == MOEHIP_DT_F16 ? f16_to_f32(w[m] & 0xffffu) : bf16_to_f32(w[m] & 0xffffu);
                    const float a1 = XDT == MOEHIP_DT_F16 ? f16_to_f32(w[m] >> 16) : bf16_to_f32(w[m] >> 16);
                    lv.v[i * VPC + 2 * m] = a0;
                    lv.v[i * VPC + 2 * m + 1] = a1;
                    acc += a0 + a1;
                }
                lv.vs[i] = acc;
            }
        }
    }
}

// the lane vector from raw 16-bit activation chunks already in registers (xr[i] = the VPC values
// of the lane's chunk i, VPC / 8 uint4 each), as load_x prepares them
template <int PREC, int XDT>
__device__ __forceinline__ void prep_x(const uint4 (&xr)[DlFmt<PREC>::CPL][DlFmt<PREC>::VPC / 8 > 0 ? DlFmt<PREC>::VPC / 8 : 1],
                                       LaneVec<PREC, XDT> &lv) {
    static_assert(XDT != MOEHIP_DT_F32, "16-bit activations");
    constexpr int VPC = DlFmt<PREC>::VPC, CPL = DlFmt<PREC>::CPL;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        lv.p2e[i] = 1.0f;
        lv.corr[i] = 0.f;
        lv.vs[i] = 0.f;
        uint32_t w[VPC / 2];
#pragma unroll
        for (int m = 0; m < VPC / 8; ++m) {
            w[4 * m + 0] = xr[i][m].x;
            w[4 * m + 1] = xr[i][m].y;
            w[4 * m + 2] = xr[i][m].z;
            w[4 * m + 3] = xr[i][m].w;
        }
        if constexpr (LaneVec<PREC, XDT>::D2) {
            if constexpr (XDT == MOEHIP_DT_F16) {
                pair_chunk<PREC>(w, lv.xp + i * DlFmt<PREC>::XPC, lv.corr[i]);
            } else {
                float f[VPC];
#pragma unroll
                for (int m = 0; m < VPC / 2; ++m) {
                    f[2 * m] = bf16_to_f32(w[m] & 0xffffu);
                    f[2 * m + 1] = bf16_to_f32(w[m] >> 16);
                }
                uint32_t hw[VPC / 2];
                lv.p2e[i] = scale_to_h<VPC>(f, hw);
                pair_chunk<PREC>(hw, lv.xp + i * DlFmt<PREC>::XPC, lv.corr[i]);
            }
        } else {
            float acc = 0.f;
#pragma unroll
            for (int m = 0; m < VPC / 2; ++m) {
                const float a0 = XDT == MOEHIP_DT_F16 ? f16_to_f32(w[m] & 0xffffu) : bf16_to_f32(w[m] & 0xffffu);
                const float a1 = XDT == MOEHIP_DT_F16 ? f16_to_f32(w[m] >> 16) : bf16_to_f32(w[m] >> 16);
                lv.v[i * VPC + 2 * m] = a0;
                lv.v[i * VPC + 2 * m + 1] = a1;
                acc += a0 + a1;
            }
            lv.vs[i] = acc;
        }
    }
}

// h staged in LDS (piece-major: piece m of chunk c at (m * C + c) * 4) -> lane vector
template <int PREC, int XDT>
__device__ __forceinline__ void load_h(const float *s_h, int cl, int G, int C, LaneVec<PREC, XDT> &lv) {
    constexpr int VPC = DlFmt<PREC>::VPC, CPL = DlFmt<PREC>::CPL;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c = min(cl + i * G, C - 1);
        lv.p2e[i] = 1.0f;
        lv.corr[i] = 0.f;
        lv.vs[i] = 0.f;
        float f[VPC];
#pragma unroll
        for (int m = 0; m < VPC / 4; ++m) {
            const float4 u = *reinterpret_cast<const float4 *>(s_h + (m * C + c) * 4);
            f[4 * m + 0] = u.x;
            f[4 * m + 1] = u.y;
            f[4 * m + 2] = u.z;
            f[4 * m + 3] = u.w;
        }
        if constexpr (LaneVec<PREC, XDT>::D2) {
            uint32_t hw[VPC / 2];
            lv.p2e[i] = scale_to_h<VPC>(f, hw);
            pair_chunk<PREC>(hw, lv.xp + i * DlFmt<PREC>::XPC, lv.corr[i]);
        } else {
            float acc = 0.f;
#pragma unroll
            for (int m = 0; m < VPC; ++m) {
                lv.v[i * VPC + m] = f[m];
                acc += f[m];
            }
            lv.vs[i] = acc;
        }
    }
}

// sum over the lane's chunk i of weight * vector (before the group scale and 2^e)
template <int PREC, int XDT>
__device__ __forceinline__ float lane_dot(const uint4 q, const LaneVec<PREC, XDT> &lv, int i) {
    if constexpr (LaneVec<PREC, XDT>::D2) {
        return dot2_chunk<PREC>(q, lv.xp + i * DlFmt<PREC>::XPC, lv.corr[i]);
    } else {
        return chunk_dot<PREC>(q, lv.v + i * DlFmt<PREC>::VPC, lv.vs[i]);
    }
}

// raw scale bits of chunk c of row `row` (int: fp16 group scale; fp8: fp32 block scale)
template <int PREC>
__device__ __forceinline__ uint32_t scale_bits(gbyte *sb, int row, int c, int cols, int gs) {
    if constexpr (PREC == MOEHIP_PREC_INT4 || PREC == MOEHIP_PREC_INT8) {
        const int ng = cols / gs;
        return gld2(sb + 2 * ((size_t)row * ng + (c * Fmt<PREC>::VPC) / gs));
    } else if constexpr (PREC == MOEHIP_PREC_FP8) {
        const int sc = (cols + 127) >> 7;
        return gld4(sb + 4 * ((size_t)(row >> 7) * sc + ((c * 16) >> 7)));
    } else {
        return 0x3f800000u;
    }
}
// the same scale addressing in three parts, for kernels that step over rows: scale columns per
// row-group (ng), the chunk's scale column (cg), and the byte offset of (row, cg) from the scale base
template <int PREC>
__device__ __forceinline__ int sc_cols(int cols, int gs) {
    if constexpr (PREC == MOEHIP_PREC_INT4 || PREC == MOEHIP_PREC_INT8) return cols / gs;
    else if constexpr (PREC == MOEHIP_PREC_FP8) return (cols + 127) >> 7;
    else return 0;
}
template <int PREC>
__device__ __forceinline__ int sc_col(int c, int gs) {
    if constexpr (PREC == MOEHIP_PREC_INT4 || PREC == MOEHIP_PREC_INT8) return (c * Fmt<PREC>::VPC) / gs;
    else if constexpr (PREC == MOEHIP_PREC_FP8) return (c * 16) >> 7;
    else return 0;
}
template <int PREC>
__device__ __forceinline__ uint32_t sc_off(int row, int cg, int ng) {
    if constexpr (PREC == MOEHIP_PREC_INT4 || PREC == MOEHIP_PREC_INT8) return 2u * (__umul24(row, ng) + (uint32_t)cg);
    else if constexpr (PREC == MOEHIP_PREC_FP8) return 4u * (__umul24(row >> 7, ng) + (uint32_t)cg);
    else return 0u;
}
template <int PREC>
__device__ __forceinline__ uint32_t sc_load(gbyte *sb, uint32_t off) {
    if constexpr (PREC == MOEHIP_PREC_INT4 || PREC == MOEHIP_PREC_INT8) return gld2(sb + off);
    else if constexpr (PREC == MOEHIP_PREC_FP8) return gld4(sb + off);
    else return 0x3f800000u;
}
template <int PREC>
__device__ __forceinline__ float scale_val(uint32_t bits) {
    if constexpr (PREC == MOEHIP_PREC_INT4 || PREC == MOEHIP_PREC_INT8) return f16_to_f32(bits);
    else return __uint_as_float(bits);
}

template <int XDT>
__device__ __forceinline__ uint32_t logit_key(float v, int c) {
    if constexpr (XDT == MOEHIP_DT_F32) {
        (void)c;
        return fkey(v);
    } else {
        uint32_t b = XDT == MOEHIP_DT_F16 ? (uint32_t)f32_to_f16_rne(v) : (__float_as_uint(v) >> 16);
        if (v == 0.f) b = 0u;
        const uint32_t k16 = (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
        return (k16 << 10) | (uint32_t)(1023 - c);
    }
}

}  // namespace moehip
