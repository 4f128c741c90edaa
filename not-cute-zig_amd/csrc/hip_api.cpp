// hip_api.cpp — the HIP host wrapper behind the C ABI (the role of src/cuda.zig in the reference).
//
// Mirrors the subset of src/cuda.zig the flash path uses: error mapping and check()
// (src/cuda.zig:134-178), init/deinit (:181-204), malloc/free/memcpy (:259-290), Module (:293-316),
// Stream (:319-341), LaunchConfig + Function.launch (:344-424), Function.Attributes (:362-388) and
// Event (:427-460). HIP has no context object: init selects device 0 with hipSetDevice, and the
// module keeps a name -> hipFunction_t cache so a launch does not repeat the symbol lookup that
// flash.launch performs on every call in the reference (src/flash.zig:46).

#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "notcute_flash.h"

struct nc_function_st {
    hipFunction_t fn = nullptr;
    std::string name;
};

struct nc_module_st {
    hipModule_t mod = nullptr;
    // Guards `functions`: several host threads may launch through one module (hipModuleGetFunction,
    // the lookup the cache saves, is itself thread-safe). Entries are never removed before unload,
    // so a returned nc_function stays valid without the lock.
    std::mutex lock;
    std::unordered_map<std::string, std::unique_ptr<nc_function_st>> functions;
    // Scratch for callers that launch the pair-split flash kernels by name
    // (nc_flash_reserve_workspace), zeroed when allocated: their exchange counters rely on starting
    // from zero. Growing it allocates a larger one and keeps the old one in `retired` until unload,
    // because graphs captured earlier and by-name callers may still hold its address. Guarded by
    // `lock`.
    void *workspace = nullptr;
    size_t workspace_bytes = 0;
    std::vector<void *> retired;
};

extern "C" const unsigned char nc_embedded_code_object[];
extern "C" const unsigned char nc_embedded_code_object_end[];

namespace {

thread_local std::string g_last_error;
bool g_initialized = false;

const char *const kStatusNames[] = {
    "Success",         "OutOfMemory",  "Overflow",           "SharedObjectInitFailed", "NotFound",
    "InvalidValue",    "InvalidContext", "InvalidDevice",    "InvalidImage",           "ContextIsDestroyed",
    "LaunchFailed",    "LaunchOutOfResources", "LaunchTimeout", "IllegalAddress",      "NoDevice",
    "NotInitialized",  "UnknownError",
};

int map_hip(hipError_t e) {
    switch (e) {
    case hipSuccess: return NC_SUCCESS;
    case hipErrorOutOfMemory: return NC_ERROR_OUT_OF_MEMORY;
    case hipErrorSharedObjectInitFailed: return NC_ERROR_SHARED_OBJECT_INIT_FAILED;
    case hipErrorNotFound: return NC_ERROR_NOT_FOUND;
    case hipErrorInvalidValue: return NC_ERROR_INVALID_VALUE;
    case hipErrorInvalidContext: return NC_ERROR_INVALID_CONTEXT;
    case hipErrorInvalidDevice: return NC_ERROR_INVALID_DEVICE;
    case hipErrorInvalidImage: return NC_ERROR_INVALID_IMAGE;
    case hipErrorContextIsDestroyed: return NC_ERROR_CONTEXT_IS_DESTROYED;
    case hipErrorLaunchFailure: return NC_ERROR_LAUNCH_FAILED;
    case hipErrorLaunchOutOfResources: return NC_ERROR_LAUNCH_OUT_OF_RESOURCES;
    case hipErrorLaunchTimeOut: return NC_ERROR_LAUNCH_TIMEOUT;
    case hipErrorIllegalAddress: return NC_ERROR_ILLEGAL_ADDRESS;
    case hipErrorNoDevice: return NC_ERROR_NO_DEVICE;
    case hipErrorNotInitialized: return NC_ERROR_NOT_INITIALIZED;
    default: return NC_ERROR_UNKNOWN;
    }
}

// check(): map the HIP status and remember the failing call, as src/cuda.zig:156-178 logs it.
int check(hipError_t e, const char *what) {
    if (e == hipSuccess) return NC_SUCCESS;
    char buf[256];
    std::snprintf(buf, sizeof buf, "%s: %s (%d)", what, hipGetErrorName(e), (int)e);
    g_last_error = buf;
    return map_hip(e);
}

int fail(int status, const char *what) {
    g_last_error = what;
    return status;
}

}  // namespace

// Error helpers for the library's other translation units (flash.cpp, noalloc.hip).
extern "C" int nc_internal_check(int hip_error, const char *what) { return check((hipError_t)hip_error, what); }
extern "C" int nc_internal_fail(int status, const char *what) { return fail(status, what); }
// noalloc.hip: sets up the static scratch on every visible device (device 0 current afterwards).
extern "C" int nc_internal_noalloc_setup(void);

extern "C" {

const char *nc_status_name(int status) {
    if (status < 0 || status > NC_ERROR_UNKNOWN) return "UnknownError";
    return kStatusNames[status];
}

const char *nc_last_error_string(void) { return g_last_error.c_str(); }

int nc_status_from_hip(int hip_error) { return map_hip((hipError_t)hip_error); }

const char *nc_version(void) { return "not-cute-zig_amd 0.1 (gfx950)"; }

int nc_device_count(int *count) {
    if (!count) return fail(NC_ERROR_INVALID_VALUE, "nc_device_count: null output");
    *count = 0;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice) return NC_SUCCESS;
    int st = check(e, "hipGetDeviceCount");
    if (st) return st;
    *count = n;
    return NC_SUCCESS;
}

int nc_init(void) {
    if (g_initialized) return NC_SUCCESS;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice || (e == hipSuccess && n <= 0))
        return fail(NC_ERROR_NO_DEVICE, "nc_init: no GPU visible");
    int st = check(e, "hipGetDeviceCount");
    if (st) return st;
    st = check(hipSetDevice(0), "hipSetDevice(0)");
    if (st) return st;
    // The static scratch of the pair-split kernels on every visible GPU: its address, and its exchange
    // counters zeroed (again after an nc_deinit), so that no launch sets anything up later.
    st = nc_internal_noalloc_setup();
    if (st) return st;
    g_initialized = true;
    return NC_SUCCESS;
}

void nc_deinit(void) {
    if (!g_initialized) return;
    (void)hipDeviceSynchronize();
    g_initialized = false;
}

int nc_device_synchronize(void) { return check(hipDeviceSynchronize(), "hipDeviceSynchronize"); }

int nc_malloc(void **dptr, size_t bytes) {
    if (!dptr) return fail(NC_ERROR_INVALID_VALUE, "nc_malloc: null output");
    *dptr = nullptr;
    return check(hipMalloc(dptr, bytes), "hipMalloc");
}

void nc_free(void *dptr) {
    if (!dptr) return;
    int st = check(hipFree(dptr), "hipFree");
    if (st) std::fprintf(stderr, "not-cute: failed to free device memory: %s\n", nc_status_name(st));
}

// A copy from pageable host memory may return once the bytes are staged, before they reach the
// device, and it is ordered only on the null stream: waited for here, so kernels launched next on
// any stream read the copied bytes.
int nc_memcpy_htod(void *dst, const void *src, size_t bytes) {
    int st = check(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy(HtoD)");
    if (st) return st;
    return check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
}

int nc_memcpy_dtoh(void *dst, const void *src, size_t bytes) {
    return check(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy(DtoH)");
}

// The fill runs on the null stream, which the library's non-blocking streams do not wait for, so
// it is waited for here: work submitted afterwards to any stream sees the filled bytes.
int nc_memset(void *dst, int byte_value, size_t bytes) {
    int st = check(hipMemset(dst, byte_value, bytes), "hipMemset");
    if (st) return st;
    return check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
}

static int module_from(hipModule_t m, nc_module *out) {
    auto *mod = new (std::nothrow) nc_module_st;
    if (!mod) {
        (void)hipModuleUnload(m);
        return fail(NC_ERROR_OUT_OF_MEMORY, "nc_module: host allocation failed");
    }
    mod->mod = m;
    *out = mod;
    return NC_SUCCESS;
}

int nc_module_load_data(nc_module *out, const void *code_object) {
    if (!out || !code_object) return fail(NC_ERROR_INVALID_VALUE, "nc_module_load_data: null argument");
    *out = nullptr;
    hipModule_t m = nullptr;
    int st = check(hipModuleLoadData(&m, code_object), "hipModuleLoadData");
    if (st) return st;
    return module_from(m, out);
}

int nc_module_load_file(nc_module *out, const char *path) {
    if (!out || !path) return fail(NC_ERROR_INVALID_VALUE, "nc_module_load_file: null argument");
    *out = nullptr;
    hipModule_t m = nullptr;
    int st = check(hipModuleLoad(&m, path), "hipModuleLoad");
    if (st) return st;
    return module_from(m, out);
}

int nc_module_load_embedded(nc_module *out) {
    if (nc_embedded_code_object_end <= nc_embedded_code_object)
        return fail(NC_ERROR_INVALID_IMAGE, "nc_module_load_embedded: library built without a code object");
    return nc_module_load_data(out, nc_embedded_code_object);
}

int nc_module_unload(nc_module module) {
    if (!module) return fail(NC_ERROR_INVALID_VALUE, "nc_module_unload: null module");
    int st = NC_SUCCESS;
    if (module->workspace) st = check(hipFree(module->workspace), "hipFree(workspace)");
    for (void *p : module->retired) {
        const int s2 = check(hipFree(p), "hipFree(retired workspace)");
        if (!st) st = s2;
    }
    int st2 = check(hipModuleUnload(module->mod), "hipModuleUnload");
    delete module;
    return st ? st : st2;
}

// The module's workspace, at least `bytes` long (used by nc_flash_reserve_workspace). A larger one
// replaces it as the current workspace; the old one stays allocated until nc_module_unload, since
// graphs captured earlier and by-name callers may still use its address. A new workspace is zeroed
// (and the zeroing waited for) before it is returned.
extern "C" int nc_internal_module_workspace(nc_module module, size_t bytes, void **out) {
    if (!module || !out) return fail(NC_ERROR_INVALID_VALUE, "workspace: null argument");
    std::lock_guard<std::mutex> guard(module->lock);
    if (module->workspace_bytes < bytes) {
        // room to keep the current workspace before anything is allocated (no throw past the C ABI)
        try {
            module->retired.reserve(module->retired.size() + 1);
        } catch (...) {
            return fail(NC_ERROR_OUT_OF_MEMORY, "workspace: host allocation failed");
        }
        void *p = nullptr;
        int st = check(hipMalloc(&p, bytes), "hipMalloc(workspace)");
        if (st) return st;
        // hipMemset may return before it completes and is not ordered with non-blocking streams.
        st = check(hipMemset(p, 0, bytes), "hipMemset(workspace)");
        if (!st) st = check(hipDeviceSynchronize(), "hipDeviceSynchronize(workspace)");
        if (st) {
            (void)hipFree(p);
            return st;
        }
        if (module->workspace) module->retired.push_back(module->workspace);  // capacity reserved above
        module->workspace = p;
        module->workspace_bytes = bytes;
    }
    *out = module->workspace;
    return NC_SUCCESS;
}

// Re-zero the exchange counters of the module's workspaces (current and retired).
extern "C" int nc_internal_module_reset_workspace(nc_module module) {
    if (!module) return NC_SUCCESS;
    std::lock_guard<std::mutex> guard(module->lock);
    int st = NC_SUCCESS;
    if (module->workspace) st = check(hipMemset(module->workspace, 0, NC_XS_COUNTER_BYTES), "hipMemset(workspace)");
    for (void *p : module->retired)
        if (!st) st = check(hipMemset(p, 0, NC_XS_COUNTER_BYTES), "hipMemset(retired workspace)");
    return st;
}

int nc_module_get_function(nc_function *out, nc_module module, const char *name) {
    if (!out || !module || !name) return fail(NC_ERROR_INVALID_VALUE, "nc_module_get_function: null argument");
    *out = nullptr;
    std::lock_guard<std::mutex> guard(module->lock);
    auto it = module->functions.find(name);
    if (it != module->functions.end()) {
        *out = it->second.get();
        return NC_SUCCESS;
    }
    hipFunction_t f = nullptr;
    int st = check(hipModuleGetFunction(&f, module->mod, name), "hipModuleGetFunction");
    if (st) return st;
    auto fn = std::make_unique<nc_function_st>();
    fn->fn = f;
    fn->name = name;
    *out = fn.get();
    module->functions.emplace(name, std::move(fn));
    return NC_SUCCESS;
}

int nc_function_launch(nc_function fn, const nc_launch_config *cfg, void **kernel_params) {
    if (!fn || !cfg) return fail(NC_ERROR_INVALID_VALUE, "nc_function_launch: null argument");
    return check(hipModuleLaunchKernel(fn->fn, cfg->grid[0], cfg->grid[1], cfg->grid[2], cfg->block[0],
                                       cfg->block[1], cfg->block[2], cfg->shared_mem_bytes,
                                       (hipStream_t)cfg->stream, kernel_params, nullptr),
                 "hipModuleLaunchKernel");
}

int nc_function_get_attributes(nc_function fn, nc_function_attributes *out) {
    if (!fn || !out) return fail(NC_ERROR_INVALID_VALUE, "nc_function_get_attributes: null argument");
    std::memset(out, 0, sizeof *out);
    struct {
        hipFunction_attribute attr;
        int32_t *dst;
    } items[] = {
        {HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, &out->max_threads_per_block},
        {HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES, &out->shared_size_bytes},
        {HIP_FUNC_ATTRIBUTE_CONST_SIZE_BYTES, &out->const_size_bytes},
        {HIP_FUNC_ATTRIBUTE_LOCAL_SIZE_BYTES, &out->local_size_bytes},
        {HIP_FUNC_ATTRIBUTE_NUM_REGS, &out->num_regs},
        {HIP_FUNC_ATTRIBUTE_PTX_VERSION, &out->ptx_version},
        {HIP_FUNC_ATTRIBUTE_BINARY_VERSION, &out->binary_version},
    };
    for (auto &it : items) {
        int v = 0;
        int st = check(hipFuncGetAttribute(&v, it.attr, fn->fn), "hipFuncGetAttribute");
        if (st) return st;
        *it.dst = v;
    }
    return NC_SUCCESS;
}

int nc_device_get_attributes(nc_device_attributes *out) {
    if (!out) return fail(NC_ERROR_INVALID_VALUE, "nc_device_get_attributes: null output");
    std::memset(out, 0, sizeof *out);
    int st = nc_init();
    if (st) return st;
    hipDeviceProp_t p;
    st = check(hipGetDeviceProperties(&p, 0), "hipGetDeviceProperties");
    if (st) return st;
    out->max_threads_per_block = p.maxThreadsPerBlock;
    out->max_shared_memory_per_block = (int32_t)p.sharedMemPerBlock;
    out->max_registers_per_sm = p.regsPerMultiprocessor;
    out->max_threads_per_sm = p.maxThreadsPerMultiProcessor;
    out->sm_count = p.multiProcessorCount;
    out->warp_size = p.warpSize;
    out->max_shared_memory_per_sm = (int32_t)p.maxSharedMemoryPerMultiProcessor;
    out->clock_khz = p.clockRate;
    std::snprintf(out->name, sizeof out->name, "%.63s", p.gcnArchName);
    return NC_SUCCESS;
}

int nc_function_max_active_blocks(nc_function fn, int block_threads, size_t dynamic_shared_bytes, int *blocks) {
    if (!fn || !blocks || block_threads <= 0)
        return fail(NC_ERROR_INVALID_VALUE, "nc_function_max_active_blocks: invalid argument");
    *blocks = 0;
    int n = 0;
    int st = check(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn->fn, block_threads, dynamic_shared_bytes),
                   "hipModuleOccupancyMaxActiveBlocksPerMultiprocessor");
    if (st) return st;
    *blocks = n;
    return NC_SUCCESS;
}

int nc_stream_create(nc_stream *out) {
    if (!out) return fail(NC_ERROR_INVALID_VALUE, "nc_stream_create: null output");
    hipStream_t s = nullptr;
    int st = check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags");
    *out = s;
    return st;
}

int nc_stream_destroy(nc_stream stream) { return check(hipStreamDestroy((hipStream_t)stream), "hipStreamDestroy"); }

int nc_stream_synchronize(nc_stream stream) {
    return check(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
}

int nc_event_create(nc_event *out) {
    if (!out) return fail(NC_ERROR_INVALID_VALUE, "nc_event_create: null output");
    hipEvent_t e = nullptr;
    int st = check(hipEventCreate(&e), "hipEventCreate");
    *out = e;
    return st;
}

int nc_event_create_timing(nc_event *out) {
    if (!out) return fail(NC_ERROR_INVALID_VALUE, "nc_event_create_timing: null output");
    hipEvent_t e = nullptr;
    int st = check(hipEventCreateWithFlags(&e, hipEventDisableSystemFence), "hipEventCreateWithFlags");
    *out = e;
    return st;
}

int nc_event_destroy(nc_event ev) { return check(hipEventDestroy((hipEvent_t)ev), "hipEventDestroy"); }

int nc_event_record(nc_event ev, nc_stream stream) {
    return check(hipEventRecord((hipEvent_t)ev, (hipStream_t)stream), "hipEventRecord");
}

int nc_event_record_node(nc_event ev, nc_stream stream) {
    return check(hipEventRecordWithFlags((hipEvent_t)ev, (hipStream_t)stream, hipEventRecordExternal),
                 "hipEventRecordWithFlags(external)");
}

int nc_event_synchronize(nc_event ev) { return check(hipEventSynchronize((hipEvent_t)ev), "hipEventSynchronize"); }

int nc_event_elapsed(float *ms, nc_event start, nc_event stop) {
    if (!ms) return fail(NC_ERROR_INVALID_VALUE, "nc_event_elapsed: null output");
    return check(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop), "hipEventElapsedTime");
}

}  // extern "C"

// ---------------------------------------------------------------------------------------------
// HIP graphs (extension; the reference has none).
// ---------------------------------------------------------------------------------------------

struct nc_graph_st {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

extern "C" {

int nc_stream_begin_capture(nc_stream stream) {
    if (!stream) return fail(NC_ERROR_INVALID_VALUE, "nc_stream_begin_capture: NULL stream cannot be captured");
    return check(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeRelaxed), "hipStreamBeginCapture");
}

int nc_stream_end_capture(nc_stream stream, nc_graph *out) {
    if (!stream || !out) return fail(NC_ERROR_INVALID_VALUE, "nc_stream_end_capture: null argument");
    *out = nullptr;
    auto g = std::make_unique<nc_graph_st>();
    int st = check(hipStreamEndCapture((hipStream_t)stream, &g->graph), "hipStreamEndCapture");
    if (st) return st;
    st = check(hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    if (st) {
        (void)hipGraphDestroy(g->graph);
        return st;
    }
    *out = g.release();
    return NC_SUCCESS;
}

int nc_graph_launch(nc_graph graph, nc_stream stream) {
    if (!graph) return fail(NC_ERROR_INVALID_VALUE, "nc_graph_launch: null graph");
    return check(hipGraphLaunch(static_cast<nc_graph_st *>(graph)->exec, (hipStream_t)stream), "hipGraphLaunch");
}

int nc_graph_destroy(nc_graph graph) {
    if (!graph) return fail(NC_ERROR_INVALID_VALUE, "nc_graph_destroy: null graph");
    auto *g = static_cast<nc_graph_st *>(graph);
    int st = check(hipGraphExecDestroy(g->exec), "hipGraphExecDestroy");
    int st2 = check(hipGraphDestroy(g->graph), "hipGraphDestroy");
    delete g;
    return st ? st : st2;
}

}  // extern "C"
