// A dependency-free streaming read: the floor that ONE launch moving a decode layer's bytes can
// reach on this device. It plays the part of moelab's read floor (profiling.py:81-120: the
// expert bytes at the bandwidth a plain streaming product reaches), measured here at the
// decode kernel's own grid and bytes so the decode kernel's time can be set against it.
//
// The bytes are n segments of equal size (records) and an optional last segment of its own size
// (the router matrix), addresses passed by value in the kernel arguments (no load waits on
// another). Workgroup b reads the 16-byte words [b * per_wg, (b + 1) * per_wg) of their
// concatenation, every load issued before any is used; the words are folded together and a
// workgroup writes its fold only when it equals a value that arbitrary data does not hit by
// chance (the loads stay, nothing is written; `sink` holds `grid` words). With `stamps`
// (2 * grid words), workgroup b writes two
// s_memrealtime stamps (100 MHz): its start and the moment all its words are in.

#include "common.hpp"

namespace moehip {

constexpr int PROBE_MAXSEG = 32;

struct ProbeArgs {
    const uint4 *seg[PROBE_MAXSEG + 1];  // n segments of seg_words words, then the extra one
    uint32_t nseg, seg_words, extra_words, per_wg;
    uint32_t *sink;
    uint64_t *stamps;
};

template <int NV>
__global__ __launch_bounds__(256) void k_stream_read(ProbeArgs a) {
    const uint64_t t0 = a.stamps != nullptr ? __builtin_amdgcn_s_memrealtime() : 0;
    const uint32_t total = a.nseg * a.seg_words + a.extra_words;
    // a workgroup past the end reads the last word (every address stays in bounds)
    const uint32_t w0 = min(blockIdx.x * a.per_wg, total - 1u);
    // a workgroup spans at most two segments (per_wg <= seg_words, checked on the host)
    const uint32_t s0 = min(w0 / a.seg_words, a.nseg);
    const uint32_t s1 = min(s0 + 1u, a.nseg);
    const uint32_t split = s0 < a.nseg ? (s0 + 1u) * a.seg_words : 0xFFFFFFFFu;
    const uint4 *b0 = a.seg[s0];
    const uint4 *b1 = a.seg[s1];
    const uint32_t o0 = s0 * a.seg_words, o1 = s1 * a.seg_words;
    uint4 v[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const uint32_t r = (uint32_t)i * 256u + threadIdx.x;
        // clamped to the workgroup's and the data's last word: every load is unconditional and in bounds
        const uint32_t w = min(w0 + min(r, a.per_wg - 1u), total - 1u);
        const uint4 *p = w < split ? b0 + (w - o0) : b1 + (w - o1);
        v[i] = *p;
    }
    uint32_t f = 0;
#pragma unroll
    for (int i = 0; i < NV; ++i) f ^= (v[i].x + v[i].y) ^ (v[i].z + v[i].w);
    if (a.stamps != nullptr) {
        __syncthreads();
        if (threadIdx.x == 0) {
            a.stamps[2 * blockIdx.x] = t0;
            a.stamps[2 * blockIdx.x + 1] = __builtin_amdgcn_s_memrealtime();
        }
    }
    if (f == 0x9E3779B9u) a.sink[blockIdx.x] = f;
}

}  // namespace moehip

using namespace moehip;

extern "C" int moehip_stream_read(const int64_t *seg_base, int nseg, int64_t seg_bytes, const void *extra,
                                  int64_t extra_bytes, int grid, uint32_t *sink, uint64_t *stamps, void *stream) {
    MOEHIP_REQUIRE(seg_base && sink && nseg > 0 && nseg <= PROBE_MAXSEG && grid > 0,
                   "stream_read: %d segments (1..%d), grid %d, sink and bases needed", nseg, PROBE_MAXSEG, grid);
    MOEHIP_REQUIRE(seg_bytes > 0 && seg_bytes % 16 == 0 && extra_bytes >= 0 && extra_bytes % 16 == 0 &&
                       (extra_bytes == 0 || extra != nullptr),
                   "stream_read: sizes must be multiples of 16 bytes");
    const int64_t total = (nseg * seg_bytes + extra_bytes) / 16;
    MOEHIP_REQUIRE(total < (int64_t)1 << 31, "stream_read: %lld words (< 2^31)", (long long)total);
    ProbeArgs a{};
    for (int i = 0; i < nseg; ++i) {
        MOEHIP_REQUIRE(seg_base[i] != 0 && seg_base[i] % 16 == 0, "stream_read: segment %d not 16-byte aligned", i);
        a.seg[i] = reinterpret_cast<const uint4 *>(seg_base[i]);
    }
    a.seg[nseg] = extra_bytes > 0 ? reinterpret_cast<const uint4 *>(extra) : a.seg[nseg - 1];
    a.nseg = (uint32_t)nseg;
    a.seg_words = (uint32_t)(seg_bytes / 16);
    a.extra_words = (uint32_t)(extra_bytes / 16);
    a.per_wg = (uint32_t)((total + grid - 1) / grid);
    a.sink = sink;
    a.stamps = stamps;
    MOEHIP_REQUIRE(a.per_wg <= a.seg_words, "stream_read: %u words per workgroup exceed a segment (%u): raise the grid",
                   a.per_wg, a.seg_words);
    const int nv = (int)((a.per_wg + 255) / 256);
    hipStream_t st = as_stream(stream);
    if (nv <= 4) hipLaunchKernelGGL(k_stream_read<4>, dim3(grid), dim3(256), 0, st, a);
    else if (nv <= 8) hipLaunchKernelGGL(k_stream_read<8>, dim3(grid), dim3(256), 0, st, a);
    else if (nv <= 16) hipLaunchKernelGGL(k_stream_read<16>, dim3(grid), dim3(256), 0, st, a);
    else if (nv <= 32) hipLaunchKernelGGL(k_stream_read<32>, dim3(grid), dim3(256), 0, st, a);
    else MOEHIP_REQUIRE(false, "stream_read: %d words per lane (<= 32): raise the grid", nv);
    return check_launch("stream_read");
}
