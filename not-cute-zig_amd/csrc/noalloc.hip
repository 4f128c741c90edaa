// noalloc.hip — the static scratch of the pair-split kernels, and nc_flash_launch_noalloc: the flash
// launch for callers that cannot allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc).
//
// The pair-split kernels (query blocks p and nqb-1-p shared by two workgroups that exchange partials)
// need scratch memory. Launches through nc_flash_launch[_async] and nc_flash_launch_noalloc take it
// from the file-scope device array `scratch` below. The array is part of this library's code object,
// so each GPU holds its own copy for the life of the process and no launch allocates anything.
// nc_flash_launch_noalloc states that contract in its interface (it rejects a launch that would need
// more than the array holds); the dispatcher only picks the pair split for shapes whose scratch fits.
//
// `scratch` in host code is only a host-side stand-in for the symbol: its device address is taken
// once per device with hipGetSymbolAddress (at nc_init for every visible device, else on the first
// call on a device) and only that address is used from then on. The counter region of the pair
// exchange must start at zero; it is cleared then (and again by every nc_init after nc_deinit, and by
// nc_flash_reset_scratch), and every launch leaves it even (as it found it). All launches on one GPU
// share the array: launches of the pair-split kernels that overlap in time on one GPU (e.g. on two
// streams) race.

#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "notcute_flash.h"

extern "C" int nc_internal_flash_launch_scratch(nc_module module, const uint16_t *q, size_t q_len,
                                                const uint16_t *k, size_t k_len, const uint16_t *v, size_t v_len,
                                                float *o, size_t o_len, const nc_flash_options *opts,
                                                nc_stream stream, void *scratch, size_t cap);
extern "C" int nc_internal_check(int hip_error, const char *what);
extern "C" int nc_internal_fail(int status, const char *what);
extern "C" int nc_internal_module_reset_workspace(nc_module module);

static __device__ __align__(256) unsigned char scratch[NC_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_lock;
void *g_scratch_ptr[kMaxDevices];  // device address of `scratch` on each device, once set up

// Zero the pair-exchange counters of device `dev`'s copy (hipMemset, then waited for: a fill on the
// null stream is not ordered with non-blocking streams). Caller holds g_lock, `dev` is current.
int clear_counters(int dev) {
    int st = nc_internal_check(hipMemset(g_scratch_ptr[dev], 0, NC_XS_COUNTER_BYTES), "hipMemset(scratch counters)");
    if (!st) st = nc_internal_check(hipDeviceSynchronize(), "hipDeviceSynchronize(scratch)");
    return st;
}

// Device `dev` (current) set up: the address of its copy of `scratch`, and, when it is new or
// `rezero` is set, its counters cleared. Caller holds g_lock.
int setup_device(int dev, bool rezero) {
    if (dev < 0 || dev >= kMaxDevices) return nc_internal_fail(NC_ERROR_INVALID_DEVICE, "scratch: device index");
    const bool fresh = g_scratch_ptr[dev] == nullptr;
    if (fresh) {
        void *p = nullptr;
        int st = nc_internal_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (st) return st;
        if (!p) return nc_internal_fail(NC_ERROR_NOT_FOUND, "hipGetSymbolAddress(scratch): null");
        g_scratch_ptr[dev] = p;
    }
    if (fresh || rezero) {
        const int st = clear_counters(dev);
        if (st) {
            if (fresh) g_scratch_ptr[dev] = nullptr;
            return st;
        }
    }
    return NC_SUCCESS;
}

// The current device's copy of `scratch` (set up here on first use if nc_init did not).
int device_scratch(void **out) {
    int dev = 0;
    int st = nc_internal_check(hipGetDevice(&dev), "hipGetDevice");
    if (st) return st;
    std::lock_guard<std::mutex> guard(g_lock);
    st = setup_device(dev, false);
    if (st) return st;
    *out = g_scratch_ptr[dev];
    return NC_SUCCESS;
}

}  // namespace

// Called by nc_init: every visible device (up to kMaxDevices) set up, counters cleared; device 0 is
// current afterwards.
extern "C" int nc_internal_noalloc_setup(void) {
    int n = 0;
    int st = nc_internal_check(hipGetDeviceCount(&n), "hipGetDeviceCount");
    if (st) return st;
    std::lock_guard<std::mutex> guard(g_lock);
    for (int dev = 0; dev < n && dev < kMaxDevices && !st; ++dev) {
        st = nc_internal_check(hipSetDevice(dev), "hipSetDevice");
        if (!st) st = setup_device(dev, true);
    }
    const int st0 = nc_internal_check(hipSetDevice(0), "hipSetDevice(0)");
    return st ? st : st0;
}

// For flash.cpp: the current device's static scratch and its size.
extern "C" int nc_internal_static_scratch(void **out, size_t *cap) {
    if (!out || !cap) return nc_internal_fail(NC_ERROR_INVALID_VALUE, "static scratch: null argument");
    *cap = NC_NOALLOC_SCRATCH_BYTES;
    return device_scratch(out);
}

extern "C" int nc_flash_reset_scratch(nc_module module) {
    int dev = 0;
    int st = nc_internal_check(hipGetDevice(&dev), "hipGetDevice");
    if (st) return st;
    {
        std::lock_guard<std::mutex> guard(g_lock);
        st = setup_device(dev, true);
    }
    if (!st) st = nc_internal_module_reset_workspace(module);
    if (!st) st = nc_internal_check(hipDeviceSynchronize(), "hipDeviceSynchronize(reset)");
    return st;
}

extern "C" int nc_flash_launch_noalloc(nc_module module, const uint16_t *q, size_t q_len, const uint16_t *k,
                                       size_t k_len, const uint16_t *v, size_t v_len, float *o, size_t o_len,
                                       const nc_flash_options *opts, nc_stream stream) {
    nc_flash_kernel_selection sel;
    int st = nc_flash_select_kernel_for(opts, q, k, v, o, &sel);
    if (st) return st;
    if (sel.scratch_bytes > NC_NOALLOC_SCRATCH_BYTES) {
        char msg[200];
        std::snprintf(msg, sizeof msg,
                      "nc_flash_launch_noalloc: %s needs %llu bytes of scratch, more than the %u-byte static buffer",
                      sel.name, (unsigned long long)sel.scratch_bytes, NC_NOALLOC_SCRATCH_BYTES);
        return nc_internal_fail(NC_ERROR_INVALID_VALUE, msg);
    }
    void *p = nullptr;
    st = device_scratch(&p);
    if (st) return st;
    return nc_internal_flash_launch_scratch(module, q, q_len, k, k_len, v, v_len, o, o_len, opts, stream, p,
                                            NC_NOALLOC_SCRATCH_BYTES);
}
