// noalloc.hip — nc_flash_launch_noalloc: the flash launch for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// It is nc_flash_launch_async with one difference: a kernel that needs scratch memory (the
// pair-split kernels: query blocks p and nqb-1-p shared by two workgroups that exchange partials)
// gets it from the file-scope device array `scratch` below instead of the module's workspace, which
// the library allocates on first need. The array is part of this library's code object, so each
// GPU holds its own copy for the life of the process and no call allocates anything.
//
// `scratch` in host code is only a host-side stand-in for the symbol: its device address is taken
// once per device with hipGetSymbolAddress (at nc_init for device 0, else on the first call on a
// device) and only that address is used from then on. The counter region of the pair exchange must
// start at zero; it is cleared once, then, and every launch leaves it even (as it found it). All
// calls on one GPU share the array: calls that overlap in time on one GPU (e.g. on two streams) race.

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

static __device__ __align__(256) unsigned char scratch[NC_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_lock;
void *g_scratch_ptr[kMaxDevices];  // device address of `scratch` on each device, once set up

// The current device's copy of `scratch`, set up on first use: its address, and the pair-exchange
// counters cleared (hipMemset, synchronised: it is not ordered with non-blocking streams).
int device_scratch(void **out) {
    int dev = 0;
    int st = nc_internal_check(hipGetDevice(&dev), "hipGetDevice");
    if (st) return st;
    if (dev < 0 || dev >= kMaxDevices) return nc_internal_fail(NC_ERROR_INVALID_DEVICE, "noalloc: device index");
    std::lock_guard<std::mutex> guard(g_lock);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        st = nc_internal_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (st) return st;
        if (!p) return nc_internal_fail(NC_ERROR_NOT_FOUND, "hipGetSymbolAddress(scratch): null");
        st = nc_internal_check(hipMemset(p, 0, NC_XS_COUNTER_BYTES), "hipMemset(scratch counters)");
        if (!st) st = nc_internal_check(hipDeviceSynchronize(), "hipDeviceSynchronize(scratch)");
        if (st) return st;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return NC_SUCCESS;
}

}  // namespace

// Called by nc_init with device 0 current.
extern "C" int nc_internal_noalloc_setup(void) {
    void *p = nullptr;
    return device_scratch(&p);
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
