// Library-wide entry points: version, error text, device check.

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "common.hpp"

namespace moehip {

static thread_local char g_err[512] = "";

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

int check_launch(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: %s", what, hipGetErrorString(e));
        return MOEHIP_ELAUNCH;
    }
    return MOEHIP_OK;
}

}  // namespace moehip

extern "C" int moehip_abi_version(void) { return MOEHIP_ABI_VERSION; }

extern "C" const char *moehip_last_error(void) { return moehip::g_err; }

extern "C" size_t moehip_layer_desc_bytes(void) { return sizeof(moehip_layer_desc); }

extern "C" int moehip_device_check(int dev) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        moehip::set_error("no HIP device %d", dev);
        return MOEHIP_ENODEV;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        moehip::set_error("device %d is %s, this library is built for gfx950", dev, prop.gcnArchName);
        return MOEHIP_ENODEV;
    }
    moehip::xcd_probe(dev);  // whether the XCD-local decode kernel may run on this device
    return moehip::noalloc_init(dev);  // this device's copy of moehip_decode_layer_noalloc's scratch array
}
