// Offload staging: pinned host records -> device record slots, and device pointer-table updates.
//
// Replaces moelab/runtime.py:310-326 `_to_fast` (torch.empty + copy_(non_blocking) on the copy
// stream, one record at a time) and the table upload of moelab/fullgraph.py:87-98
// `DeviceTable.upload` (host table -> device after every change). Here:
//   * one call stages a batch of records (a layer's misses or its prefetch list) on the copy
//     stream, either as one gather kernel that reads pinned host memory directly over the host
//     link (16-byte loads, 64 KiB per workgroup, every record of the batch in one launch) or as
//     one SDMA copy per record (hipMemcpyAsync);
//   * pointer-table entries are written by a small kernel on the same stream right after the
//     copies, so an entry becomes non-zero only once its record's bytes are in device memory.

#include "common.hpp"

namespace moehip {

constexpr int STAGE_MAX = 32;          // records per gather launch (descriptor passed by value)
constexpr int STAGE_CHUNK = 64 << 10;  // bytes per workgroup
constexpr int STAGE_VEC = STAGE_CHUNK / (256 * 16);  // 16-byte vectors per thread (16)
constexpr int TABLE_MAX = 64;          // entries per table update

struct StageBatch {
    const uint4 *src[STAGE_MAX];
    uint4 *dst[STAGE_MAX];
    uint32_t nvec[STAGE_MAX];           // record length in 16-byte vectors
    uint32_t first[STAGE_MAX + 1];      // first workgroup of each record (prefix sum of chunks)
    int n;
};

// workgroup b copies chunk (b - first[i]) of record i: every thread issues its 16 loads before
// its 16 stores, so 64 KiB per workgroup are in flight over the host link
__global__ __launch_bounds__(256) void k_stage_gather(const StageBatch b) {
    const uint32_t wg = blockIdx.x;
    int i = 0;
    while (i + 1 < b.n && b.first[i + 1] <= wg) ++i;
    const uint32_t v0 = (wg - b.first[i]) * (uint32_t)(STAGE_CHUNK / 16);
    const uint32_t nv = b.nvec[i];
    const uint4 *__restrict__ src = b.src[i];
    uint4 *__restrict__ dst = b.dst[i];
    uint4 r[STAGE_VEC];
#pragma unroll
    for (int j = 0; j < STAGE_VEC; ++j) {
        const uint32_t v = v0 + j * 256 + threadIdx.x;
        r[j] = v < nv ? src[v] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < STAGE_VEC; ++j) {
        const uint32_t v = v0 + j * 256 + threadIdx.x;
        if (v < nv) dst[v] = r[j];
    }
}

struct TableSet {
    int64_t idx[TABLE_MAX];
    int64_t val[TABLE_MAX];
    int n;
};

__global__ __launch_bounds__(64) void k_table_set(int64_t *__restrict__ tab, const TableSet s) {
    const int i = threadIdx.x;
    if (i < s.n) tab[s.idx[i]] = s.val[i];
}

// true if [p, p + bytes) starts and ends in host memory the device can read (pinned)
static bool host_readable(const void *p, uint64_t bytes) {
    const char *c = reinterpret_cast<const char *>(p);
    const void *ends[2] = {c, c + bytes - 1};
    for (const void *q : ends) {
        hipPointerAttribute_t a;
        if (hipPointerGetAttributes(&a, q) != hipSuccess) {
            (void)hipGetLastError();
            return false;
        }
        if (a.type != hipMemoryTypeHost || a.devicePointer == nullptr) return false;
    }
    return true;
}

}  // namespace moehip

using namespace moehip;

extern "C" int moehip_stage_records(const moehip_copy *items, int n, int mode, void *stream) {
    MOEHIP_REQUIRE(items != nullptr && n >= 0 && n <= STAGE_MAX, "stage_records: n = %d (0..%d)", n, STAGE_MAX);
    MOEHIP_REQUIRE(mode == MOEHIP_STAGE_KERNEL || mode == MOEHIP_STAGE_SDMA, "stage_records: mode %d", mode);
    if (n == 0) return MOEHIP_OK;
    hipStream_t st = as_stream(stream);
    StageBatch b = {};
    uint32_t wg = 0;
    for (int i = 0; i < n; ++i) {
        const moehip_copy &c = items[i];
        MOEHIP_REQUIRE(c.src != nullptr && c.dst != nullptr && c.bytes > 0, "stage_records: item %d is empty", i);
        MOEHIP_REQUIRE(((uintptr_t)c.src % 16) == 0 && ((uintptr_t)c.dst % 16) == 0 && c.bytes % 16 == 0,
                       "stage_records: item %d not 16-byte aligned (src %p dst %p bytes %llu)", i, c.src, c.dst,
                       (unsigned long long)c.bytes);
        MOEHIP_REQUIRE(c.bytes <= ((uint64_t)1 << 34), "stage_records: item %d too large", i);
        if (mode == MOEHIP_STAGE_KERNEL) {
            MOEHIP_REQUIRE(host_readable(c.src, c.bytes),
                           "stage_records: item %d source is not pinned host memory (kernel staging reads it "
                           "from the device)", i);
            b.src[i] = reinterpret_cast<const uint4 *>(c.src);
            b.dst[i] = reinterpret_cast<uint4 *>(c.dst);
            b.nvec[i] = (uint32_t)(c.bytes / 16);
            b.first[i] = wg;
            wg += (uint32_t)((c.bytes + STAGE_CHUNK - 1) / STAGE_CHUNK);
        }
    }
    if (mode == MOEHIP_STAGE_SDMA) {
        for (int i = 0; i < n; ++i) {
            const hipError_t e = hipMemcpyAsync(items[i].dst, items[i].src, items[i].bytes, hipMemcpyHostToDevice, st);
            MOEHIP_REQUIRE(e == hipSuccess, "stage_records: hipMemcpyAsync item %d: %s", i, hipGetErrorString(e));
        }
        return MOEHIP_OK;
    }
    b.first[n] = wg;
    b.n = n;
    hipLaunchKernelGGL(k_stage_gather, dim3(wg), dim3(256), 0, st, b);
    return check_launch("stage_records");
}

extern "C" int moehip_table_set(int64_t *tab, int64_t tab_len, const int64_t *idx, const int64_t *val, int n,
                                void *stream) {
    MOEHIP_REQUIRE(tab != nullptr && idx != nullptr && val != nullptr && n >= 0 && n <= TABLE_MAX,
                   "table_set: n = %d (0..%d)", n, TABLE_MAX);
    if (n == 0) return MOEHIP_OK;
    TableSet s = {};
    for (int i = 0; i < n; ++i) {
        MOEHIP_REQUIRE(idx[i] >= 0 && idx[i] < tab_len, "table_set: index %lld outside [0, %lld)", (long long)idx[i],
                       (long long)tab_len);
        s.idx[i] = idx[i];
        s.val[i] = val[i];
    }
    s.n = n;
    hipLaunchKernelGGL(k_table_set, dim3(1), dim3(64), 0, as_stream(stream), tab, s);
    return check_launch("table_set");
}
