// The one entry point that allocates nothing: moehip_decode_layer on a workspace that is a device
// array of this library (no caller workspace, no allocation of any kind), for callers that cannot
// allocate (code under HIP graph capture, tight serving loops).
//
// The array, `scratch`, is a file-scope __device__ variable: every GPU the library runs on holds
// its own copy, at its own address, until the process ends. Host code never passes `scratch` itself
// (in host code the name is a host-side stand-in, not a device address): moehip_device_check(dev),
// the library's set-up call, finds device dev's copy with hipGetSymbolAddress, zero-fills it with a
// kernel (the workspace starts at zero; every launch leaves it ready for the next) and keeps its
// address per device. Every call on a GPU shares that GPU's copy: calls that overlap on one GPU
// (two streams at once) race; one stream at a time.

#include "common.hpp"

namespace moehip {

constexpr size_t NOALLOC_BYTES = (size_t)2 << 20;  // 2 MiB: every layer shape up to 4 precisions x 33 rows
static __device__ __align__(256) uint8_t scratch[NOALLOC_BYTES];

static void *g_scratch[64];  // device address of `scratch` per device, null until set up

__global__ void k_zero_words(uint32_t *p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

// Called by moehip_device_check(dev) (set-up: never under capture): device dev's copy of `scratch`
// (its address from hipGetSymbolAddress, with dev current), zero-filled, kept for every later call.
int noalloc_init(int dev) {
    if (dev < 0 || dev >= 64) {
        set_error("device %d out of range", dev);
        return MOEHIP_EINVAL;
    }
    if (g_scratch[dev] != nullptr) return MOEHIP_OK;
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess || hipSetDevice(dev) != hipSuccess) {
        set_error("device %d cannot be made current", dev);
        return MOEHIP_ENODEV;
    }
    int rc = MOEHIP_OK;
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
        set_error("hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
        rc = MOEHIP_ELAUNCH;
    } else {
        hipLaunchKernelGGL(k_zero_words, dim3(256), dim3(256), 0, nullptr, reinterpret_cast<uint32_t *>(ptr),
                           NOALLOC_BYTES / 4);
        const hipError_t e2 = hipStreamSynchronize(nullptr);
        if (e2 != hipSuccess) {
            set_error("zero-filling the scratch array on device %d: %s", dev, hipGetErrorString(e2));
            rc = MOEHIP_ELAUNCH;
        } else {
            g_scratch[dev] = ptr;
        }
    }
    (void)hipSetDevice(prev);
    return rc;
}

// device dev's copy of `scratch` (null before noalloc_init(dev)): the workspace whose error word
// moehip_decode_layer_error reads when it is given no workspace
void *noalloc_scratch(int dev) { return dev >= 0 && dev < 64 ? g_scratch[dev] : nullptr; }

}  // namespace moehip

using namespace moehip;

extern "C" int moehip_decode_layer_noalloc(const moehip_layer_desc *d, const void *x, const void *Wr,
                                           const int64_t *idx_in, const float *w32_in, const int64_t *rtab, void *out,
                                           const void *add, int accumulate, void *logits_out, int64_t *idx_out,
                                           void *w_out, float *w32_out, float *info, float *miss, void *stream) {
    MOEHIP_REQUIRE(d != nullptr, "decode_layer_noalloc: null description");
    int dev = -1;
    MOEHIP_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64, "decode_layer_noalloc: no current device");
    MOEHIP_REQUIRE(g_scratch[dev] != nullptr, "decode_layer_noalloc: call moehip_device_check(%d) first (it sets up "
                   "this device's scratch array)", dev);
    const int ks = d->k + (d->shared_gate != nullptr ? 1 : 0);
    const size_t need = moehip_decode_layer_workspace_bytes(d->P, ks, d->E, d->H, d->I);
    MOEHIP_REQUIRE(need > 0 && need <= NOALLOC_BYTES,
                   "decode_layer_noalloc: this layer needs %zu workspace bytes, the scratch array holds %zu "
                   "(use moehip_decode_layer with a workspace)", need, NOALLOC_BYTES);
    return moehip_decode_layer(d, x, Wr, idx_in, w32_in, rtab, out, add, accumulate, logits_out, idx_out, w_out,
                               w32_out, info, miss, g_scratch[dev], NOALLOC_BYTES, 0, nullptr, stream);
}
