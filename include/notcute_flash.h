/*
 * notcute_flash.h — C ABI of the MI355X (gfx950) flash-attention forward path.
 *
 * This header is the drop-in boundary that replaces the Zig host layer of
 * not-cute-zig for its flash-attention forward:
 *   - the CUDA driver wrapper   src/cuda.zig      (-> nc_init, nc_malloc, nc_module_*, nc_stream_*, nc_event_*)
 *   - the flash host API        src/flash.zig     (-> nc_flash_options, nc_flash_validate,
 *                                                    nc_flash_select_kernel, nc_flash_launch)
 *   - the benchmark helper      src/benchmark.zig (-> nc_benchmark_run_kernel)
 * Every entry point below names the reference declaration it replaces (file:line).
 *
 * Conventions
 *   - All functions return an nc_status (0 = success) unless stated otherwise.
 *   - Device buffers are plain pointers plus element counts; no C++ or torch types cross the ABI.
 *   - Q/K/V are IEEE binary16 stored as uint16_t bit patterns, O is float32.
 *   - Like the reference, launches are asynchronous; results become visible after a synchronising
 *     copy or an nc_stream_synchronize / nc_device_synchronize. A launch allocates nothing and does
 *     not synchronise: the kernels that need scratch memory (the pair-split kernels,
 *     selection.scratch_bytes > 0) use a static device buffer compiled into this library, one per
 *     GPU, which nc_init sets up on every visible GPU.
 *   - One process, one GPU (device 0), one calling thread, as in the reference.
 *
 * The same header is included by the device code (flash_fwd.hip) for the kernel argument block.
 */
#ifndef NOTCUTE_FLASH_H
#define NOTCUTE_FLASH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------------------------------
 * Status codes. One code per member of the reference's CudaError set (src/cuda.zig:134-151),
 * in the same order, so a Zig binding can map them 1:1 back to `CudaError`.
 * ---------------------------------------------------------------------------------------------- */
typedef enum nc_status {
    NC_SUCCESS = 0,
    NC_ERROR_OUT_OF_MEMORY = 1,
    NC_ERROR_OVERFLOW = 2,
    NC_ERROR_SHARED_OBJECT_INIT_FAILED = 3,
    NC_ERROR_NOT_FOUND = 4,
    NC_ERROR_INVALID_VALUE = 5,
    NC_ERROR_INVALID_CONTEXT = 6,
    NC_ERROR_INVALID_DEVICE = 7,
    NC_ERROR_INVALID_IMAGE = 8,
    NC_ERROR_CONTEXT_IS_DESTROYED = 9,
    NC_ERROR_LAUNCH_FAILED = 10,
    NC_ERROR_LAUNCH_OUT_OF_RESOURCES = 11,
    NC_ERROR_LAUNCH_TIMEOUT = 12,
    NC_ERROR_ILLEGAL_ADDRESS = 13,
    NC_ERROR_NO_DEVICE = 14,
    NC_ERROR_NOT_INITIALIZED = 15,
    NC_ERROR_UNKNOWN = 16
} nc_status;

/* Name of a status code, e.g. "InvalidValue" (the Zig error name). Never NULL. */
const char *nc_status_name(int status);
/* Text of the last failing HIP call on this thread (hipGetErrorName + call site), or "". Mirrors the
 * log line written by check() in src/cuda.zig:156-178. */
const char *nc_last_error_string(void);
/* Map a raw hipError_t value to an nc_status (check(), src/cuda.zig:156-178). */
int nc_status_from_hip(int hip_error);

/* ------------------------------------------------------------------------------------------------
 * Device, memory, module, stream, event: the subset of src/cuda.zig the flash path uses.
 * ---------------------------------------------------------------------------------------------- */
typedef struct nc_module_st *nc_module;     /* CUmodule   -> hipModule_t (+ function cache) */
typedef struct nc_function_st *nc_function; /* CUfunction -> hipFunction_t */
typedef void *nc_stream;                    /* CUstream   -> hipStream_t, NULL = default stream */
typedef void *nc_event;                     /* CUevent    -> hipEvent_t */

/* cuda.init (src/cuda.zig:181-196): select device 0. NC_ERROR_NO_DEVICE without a GPU. Idempotent.
 * Also sets up the pair-split kernels' static scratch on every visible GPU (its address, and its
 * exchange counters zeroed; zeroed again by an nc_init that follows nc_deinit). */
int nc_init(void);
/* cuda.deinit (src/cuda.zig:198-204). */
void nc_deinit(void);
/* Number of visible GPUs (0 when none); never initialises a context beyond hipGetDeviceCount. */
int nc_device_count(int *count);
/* cuCtxSynchronize equivalent. */
int nc_device_synchronize(void);

/* cuda.malloc / free / memcpy (src/cuda.zig:259-290). Sizes are in bytes. Both copies return once
 * the bytes are at their destination, so work submitted afterwards to any stream sees them. */
int nc_malloc(void **dptr, size_t bytes);
void nc_free(void *dptr);
int nc_memcpy_htod(void *dst_device, const void *src_host, size_t bytes);
int nc_memcpy_dtoh(void *dst_host, const void *src_device, size_t bytes);
/* Fills `bytes` bytes with `byte_value` and returns once the fill is complete, so work submitted
 * afterwards to any stream (streams here are non-blocking) sees it. An extension: the reference
 * clears its host arrays before copying them over (src/main.zig:994-995). */
int nc_memset(void *dst_device, int byte_value, size_t bytes);

/* Module (src/cuda.zig:293-316). */
int nc_module_load_data(nc_module *out, const void *code_object); /* hipModuleLoadData */
int nc_module_load_file(nc_module *out, const char *path);        /* hipModuleLoad */
/* The gfx950 flash code object compiled into this library (the @embedFile("cuda-module") of
 * src/main.zig:32). */
int nc_module_load_embedded(nc_module *out);
int nc_module_unload(nc_module module);
/* cuModuleGetFunction (src/cuda.zig:311-315). Results are cached per module. */
int nc_module_get_function(nc_function *out, nc_module module, const char *name);

/* LaunchConfig + Dim3 (src/cuda.zig:344-356). */
typedef struct nc_launch_config {
    uint32_t grid[3];
    uint32_t block[3];
    uint32_t shared_mem_bytes;
    nc_stream stream;
} nc_launch_config;

/* Function.launch (src/cuda.zig:391-423): `kernel_params` is the cuLaunchKernel-style array of
 * pointers to each argument. */
int nc_function_launch(nc_function fn, const nc_launch_config *cfg, void **kernel_params);

/* Function.Attributes (src/cuda.zig:362-388), extended with the gfx950 resource counts that
 * rocprof and the code-object metadata report. */
typedef struct nc_function_attributes {
    int32_t max_threads_per_block;
    int32_t shared_size_bytes;
    int32_t const_size_bytes;
    int32_t local_size_bytes;
    int32_t num_regs;
    int32_t ptx_version;    /* HIP reports 0 on AMD */
    int32_t binary_version; /* gfx target major*10+minor as reported by HIP */
} nc_function_attributes;
int nc_function_get_attributes(nc_function fn, nc_function_attributes *out);

/* cuda.OccupancyCalculator.init (src/cuda.zig:228-245) over cuda.getDevice: the device limits the
 * reference's profile-flash occupancy arithmetic uses (src/main.zig:96-104), for device 0, plus the
 * gfx950 facts that arithmetic needs here (LDS per CU, SIMDs per CU, name). "SM" is a CU. */
typedef struct nc_device_attributes {
    int32_t max_threads_per_block;
    int32_t max_shared_memory_per_block; /* bytes of LDS one workgroup may use */
    int32_t max_registers_per_sm;        /* 32-bit VGPR lanes per CU (hipDeviceProp regsPerMultiprocessor) */
    int32_t max_threads_per_sm;
    int32_t sm_count;                    /* CUs */
    int32_t warp_size;                   /* 64 */
    int32_t max_shared_memory_per_sm;    /* LDS per CU, bytes */
    int32_t clock_khz;                   /* peak shader clock */
    char name[64];                       /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
} nc_device_attributes;
int nc_device_get_attributes(nc_device_attributes *out);
/* Workgroups of `block_threads` threads that fit on one CU at once
 * (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor). An extension: the reference derives this by
 * hand from the function attributes and the device limits (src/main.zig:96-104). */
int nc_function_max_active_blocks(nc_function fn, int block_threads, size_t dynamic_shared_bytes, int *blocks);

/* Stream (src/cuda.zig:319-341). Created non-blocking at the default priority. */
int nc_stream_create(nc_stream *out);
int nc_stream_destroy(nc_stream stream);
int nc_stream_synchronize(nc_stream stream);

/* Event (src/cuda.zig:427-460). */
int nc_event_create(nc_event *out);
/* Extension: an event used only to time the stream between two records (nc_event_elapsed). Its
 * record skips the system-scope cache writeback and invalidate that a default event's record
 * performs (hipEventDisableSystemFence), so the event pair brackets the kernels between them and not
 * a cache flush; work after it still runs in stream order. */
int nc_event_create_timing(nc_event *out);
int nc_event_destroy(nc_event ev);
int nc_event_record(nc_event ev, nc_stream stream);
/* Extension: record `ev` on `stream` as a node of the graph being captured there (hipEventRecordExternal;
 * outside a capture, the same as nc_event_record). Each replay of the graph records the event at that
 * point of the graph, so a pair of such nodes times the launches between them without the graph's
 * own launch cost. */
int nc_event_record_node(nc_event ev, nc_stream stream);
int nc_event_synchronize(nc_event ev);
int nc_event_elapsed(float *ms, nc_event start, nc_event stop);

/* HIP graphs (extension, no counterpart in the reference): capture a sequence of launches issued on
 * `stream` (which must not be the NULL stream) and replay it with one call. Used to time
 * back-to-back kernels without host launch gaps and by callers whose inner loop is launch-bound. */
typedef void *nc_graph;
int nc_stream_begin_capture(nc_stream stream);
int nc_stream_end_capture(nc_stream stream, nc_graph *out); /* capture + instantiate */
int nc_graph_launch(nc_graph graph, nc_stream stream);
int nc_graph_destroy(nc_graph graph);

/* Name of the plain 16-byte copy kernel in the embedded code object, launched by the benchmark to
 * calibrate rocprofv3 FETCH_SIZE / WRITE_SIZE counters against a known byte count:
 * nc_util_copy_b128(const uint4 *src, uint4 *dst, uint64_t n16), grid-stride loop over n16 items. */
#define NC_UTIL_COPY_KERNEL "nc_util_copy_b128"

/* Name of an empty kernel taking the flash kernels' argument block, launched by the benchmark with
 * a flash kernel's grid and block to time the fixed dispatch-and-completion cost of one launch:
 * nc_util_empty(nc_flash_kernel_args), does nothing. */
#define NC_UTIL_EMPTY_KERNEL "nc_util_empty"

/* ------------------------------------------------------------------------------------------------
 * Flash-attention forward (src/flash.zig:5-100).
 * ---------------------------------------------------------------------------------------------- */

/* Element type of Q/K/V (O is always f32). The reference computes in f16 only; bf16 is an
 * extension served by the `_bf16` kernels. */
#define NC_ELEMENT_F16 0u
#define NC_ELEMENT_BF16 1u

/* flash.Options (src/flash.zig:5-14). The first nine fields are the reference's, in order and
 * meaning (element strides between (batch, head) slices). The four row strides are an extension:
 * elements between consecutive rows inside a slice; 0 means head_dim, which is exactly the
 * reference's layout (every reference kernel indexes row*head_dim+col). element_type is an
 * extension too: NC_ELEMENT_F16 (0, the reference's type and the default) or NC_ELEMENT_BF16. */
typedef struct nc_flash_options {
    uint64_t batch_heads; /* default 1 */
    uint64_t seq_len;
    uint64_t head_dim;    /* 16, 32 or 64 */
    uint64_t q_stride;
    uint64_t k_stride;
    uint64_t v_stride;
    uint64_t o_stride;
    float scale;
    uint32_t causal;      /* bool, default 0 */
    uint64_t q_row_stride; /* 0 => head_dim */
    uint64_t k_row_stride;
    uint64_t v_row_stride;
    uint64_t o_row_stride;
    uint32_t element_type; /* NC_ELEMENT_F16 (default) or NC_ELEMENT_BF16 */
} nc_flash_options;

/* Field defaults of flash.Options: batch_heads = 1, causal = false, row strides = head_dim;
 * everything else zero. */
void nc_flash_options_init(nc_flash_options *opts);

/* Options.validate (src/flash.zig:16-28): NC_ERROR_INVALID_VALUE when batch_heads == 0,
 * seq_len == 0, head_dim not in {16,32,64}, a row stride below head_dim, a slice stride below
 * (seq_len-1)*row_stride + head_dim (= seq_len*head_dim for the reference layout), or an unknown
 * element_type.
 * NC_ERROR_OVERFLOW when batch_heads*stride does not fit in 64 bits. */
int nc_flash_validate(const nc_flash_options *opts);

/* flash.KernelSelection (src/flash.zig:72-76), extended with the launch geometry: the reference's
 * callers re-derive the grid as (ceil(S/16), BH) (src/main.zig:822-828, 1024-1030); here the
 * selection carries it, because the gfx950 kernels tile differently. */
typedef struct nc_flash_kernel_selection {
    const char *name;           /* code-object symbol */
    const char *label;          /* human-readable label */
    const char *reference_name; /* the kernel the reference's selectKernel picks for these options */
    uint32_t threads;           /* block size (multiple of 64: wave64) */
    uint32_t grid[3];           /* the launch grid (x, y, z) for `name` with these options; the kernels
                                   derive each workgroup's slice and query block from its id and
                                   do not re-check it, so a by-name launch with a larger grid
                                   reads and writes outside the tensors */
    uint32_t block_m;           /* query rows per workgroup */
    uint32_t block_n;           /* keys staged per workgroup iteration */
    uint32_t kv_splits;         /* waves that share one query tile and split its keys */
    uint32_t lds_bytes;         /* static LDS of the kernel */
    uint32_t aligned;           /* 1: 16-byte vector path, 0: element-wise path for odd strides */
    uint64_t scratch_bytes;     /* device scratch the kernel needs (pair-split kernels), else 0 */
} nc_flash_kernel_selection;

/* selectKernel (src/flash.zig:78-96), re-tuned for MI355X. Assumes 16-byte aligned base pointers
 * (what nc_malloc returns); nc_flash_launch re-checks the actual pointers. Calls nc_flash_validate
 * first and fails with its status; NC_ERROR_OVERFLOW when the launch grid would exceed 2^32 - 1
 * work-items in a dimension (about 2^23 workgroups of 512 threads: batch_heads * ceil(seq_len/32)
 * at that size, where no packed-slice 3-D grid applies). */
int nc_flash_select_kernel(const nc_flash_options *opts, nc_flash_kernel_selection *out);

/* Same, for the actual buffers: picks the element-wise variant when a pointer or stride breaks
 * 16-byte alignment (the reference's smoke cases use odd slice pads, src/main.zig:190-193). */
int nc_flash_select_kernel_for(const nc_flash_options *opts, const void *q, const void *k,
                               const void *v, const void *o, nc_flash_kernel_selection *out);

/* Kernel argument block (the kernarg segment of every nc_flash_fwd_* kernel). Its first 88 bytes
 * are the reference kernels' parameter list in order (q, k, v, o, seq_len, head_dim, q_stride,
 * k_stride, v_stride, o_stride: u64, scale: f32, causal: u32; src/flash.zig:55-68). */
typedef struct nc_flash_kernel_args {
    const uint16_t *q;
    const uint16_t *k;
    const uint16_t *v;
    float *o;
    uint64_t seq_len;
    uint64_t head_dim;
    uint64_t q_stride;
    uint64_t k_stride;
    uint64_t v_stride;
    uint64_t o_stride;
    float scale;
    uint32_t causal;
    /* extension */
    uint64_t q_row_stride;
    uint64_t k_row_stride;
    uint64_t v_row_stride;
    uint64_t o_row_stride;
    uint32_t batch_heads;
    uint32_t num_q_blocks; /* ceil(seq_len / block_m) */
    void *scratch;         /* device scratch of kernels that need one (selection.scratch_bytes), else NULL */
    /* Performance only, results do not depend on it: the number of the grid's last workgroups that
     * order their waves by remaining work so that co-resident ones finish together (non-causal
     * shared-staging kernels; 0: none). nc_flash_pack_args sets it from the current device's CU count
     * when the grid has more workgroups than the device has CUs. */
    uint32_t balance_tail;
} nc_flash_kernel_args;

/* Layout of the scratch of the pair-split kernels (selection.scratch_bytes): a fixed region of
 * NC_XS_COUNTER_BYTES holding one u32 exchange counter per pair of workgroups (at most
 * NC_XS_MAX_PAIRS = batch_heads * (ceil(seq_len/32) / 2) pairs), then two slots per pair of
 * 32 x head_dim f32 partial outputs plus 32 (max, sum) f32 pairs. The counter region is the same for
 * every shape, so shapes that share a workspace never see each other's partial data as counters;
 * the counters must start at zero (even) and every launch leaves them even. */
#define NC_XS_COUNTER_BYTES 65536u
#define NC_XS_MAX_PAIRS (NC_XS_COUNTER_BYTES / 4u)

/* Scratch bytes the kernel `name` needs for a launch with these options (0 for every kernel but the
 * pair-split ones), for callers that launch a kernel by name with their own scratch buffer, which
 * must be zeroed before its first use. NC_ERROR_NOT_FOUND for a name that is not a flash kernel;
 * NC_ERROR_INVALID_VALUE for a pair-split launch with more than NC_XS_MAX_PAIRS pairs (such a
 * by-name launch writes nothing). */
int nc_flash_kernel_scratch_bytes(const char *name, const nc_flash_options *opts, uint64_t *bytes);

/* The kernel-parameter array (cuLaunchKernel style, for nc_function_launch and nc_benchmark_run_kernel)
 * that launches the flash kernel `name` with the argument block `args`. Most kernels declare the block
 * as one parameter: params[0] = args, *count = 1. The dense-layout kernels (`q1s8p1d`, `q1s8p2d`;
 * packed slices: every slice
 * stride seq_len*head_dim, every row stride head_dim; selected by nc_flash_select_kernel for such
 * layouts) declare one parameter per field of the block, in order, so that their first seven are
 * preloaded into SGPRs: params[i] = the address of field i, *count = NC_FLASH_MAX_KERNEL_PARAMS. Either
 * way the kernarg segment is the block's bytes. `params` must hold `capacity` >= *count entries and
 * stays valid while `args` does. NC_ERROR_NOT_FOUND for a name that is not a flash kernel. */
#define NC_FLASH_MAX_KERNEL_PARAMS 20u
int nc_flash_kernel_params(const char *name, nc_flash_kernel_args *args, void **params, uint32_t capacity,
                           uint32_t *count);

/* Fill the argument block for `sel` (row strides resolved, num_q_blocks derived). */
int nc_flash_pack_args(const nc_flash_options *opts, const nc_flash_kernel_selection *sel,
                       const uint16_t *q, const uint16_t *k, const uint16_t *v, float *o,
                       nc_flash_kernel_args *out);

/* flash.launch (src/flash.zig:31-70) + requireLen (src/flash.zig:98-100): validate, require
 * q_len >= batch_heads*q_stride (and likewise k, v, o; lengths in elements), select, look the
 * kernel up in `module`, launch on the default stream. Asynchronous; allocates nothing and does not
 * synchronise (so it may be captured into a HIP graph, first launch included). */
int nc_flash_launch(nc_module module, const uint16_t *q, size_t q_len, const uint16_t *k, size_t k_len,
                    const uint16_t *v, size_t v_len, float *o, size_t o_len, const nc_flash_options *opts);
/* Same on an explicit stream (a strict superset: the reference always uses the null stream).
 * Launches whose kernel uses scratch (selection.scratch_bytes > 0) must not overlap in time with
 * another such launch on the same GPU (e.g. on two streams): they share the GPU's static scratch
 * (with nc_flash_launch_noalloc). */
int nc_flash_launch_async(nc_module module, const uint16_t *q, size_t q_len, const uint16_t *k,
                          size_t k_len, const uint16_t *v, size_t v_len, float *o, size_t o_len,
                          const nc_flash_options *opts, nc_stream stream);

/* No counterpart in the reference (whose kernels use no scratch memory): for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The same launch as nc_flash_launch_async, with the contract stated: a kernel needing
 * scratch gets the static device buffer of NC_NOALLOC_SCRATCH_BYTES compiled into this library (one
 * per GPU, held until the process ends); it never allocates or frees anything, and returns
 * NC_ERROR_INVALID_VALUE when the selected kernel would need more scratch than that. Every
 * pair-split launch on one GPU shares the buffer: launches that overlap in time on one GPU (e.g. on
 * two streams) race. */
#define NC_NOALLOC_SCRATCH_BYTES (4u << 20)
int nc_flash_launch_noalloc(nc_module module, const uint16_t *q, size_t q_len, const uint16_t *k,
                            size_t k_len, const uint16_t *v, size_t v_len, float *o, size_t o_len,
                            const nc_flash_options *opts, nc_stream stream);

/* Extension (no counterpart in the reference, whose kernels use no scratch memory), for callers that
 * launch the selected kernel by name themselves: make the module's workspace large enough for a
 * launch with these options (allocating and zeroing device memory, and synchronising the device,
 * when it must grow) and store it in *workspace (may be NULL); they put it in
 * nc_flash_kernel_args.scratch. Stores NULL, allocating
 * nothing, when the selected kernel needs no scratch. A returned workspace stays valid until
 * nc_module_unload: growing it allocates a new one and keeps the old. nc_flash_launch does not use it. */
int nc_flash_reserve_workspace(nc_module module, const nc_flash_options *opts, void **workspace);

/* Extension (no counterpart in the reference): zero the pair-split exchange counters again, in the
 * current GPU's static scratch and in `module`'s workspaces (module may be NULL), then synchronise the
 * device. The counters are even between launches; a launch that overlapped another pair-split
 * launch on the same GPU, or one that was aborted, can leave them odd, which breaks later pair-split
 * results until this is called. Call it with no launch in flight and outside a stream capture. */
int nc_flash_reset_scratch(nc_module module);

/* Work model of one launch: flops and bytes as the reference's harness counts them
 * (src/main.zig:843-845, 1032-1034: causal keys = S(S+1)/2), and the half-square causal count
 * 4*BH*S*S*d/2 used for the MI355X roofline figures. */
typedef struct nc_flash_work {
    uint64_t flops_reference; /* BH * 4 * eff * d, eff = S(S+1)/2 causal, S*S otherwise */
    uint64_t flops_halfsquare; /* 4*BH*S*S*d, halved when causal */
    uint64_t bytes;           /* BH*S*d*(3*2 + 4): Q,K,V read once, O written once */
} nc_flash_work;
int nc_flash_work_model(const nc_flash_options *opts, nc_flash_work *out);

/* ------------------------------------------------------------------------------------------------
 * Benchmark helper (src/benchmark.zig:6-92).
 * ---------------------------------------------------------------------------------------------- */
typedef struct nc_benchmark_options {   /* BenchmarkOptions, src/benchmark.zig:26-32 */
    uint32_t warmup_iters;              /* reference default 3 */
    uint32_t iters;                     /* reference default 10 */
    uint64_t bytes_processed;           /* 0 = not reported */
    uint64_t flops_processed;           /* 0 = not reported */
    nc_stream stream;
} nc_benchmark_options;

typedef struct nc_benchmark_result {    /* BenchmarkResult, src/benchmark.zig:6-11 */
    float mean_ms;
    float min_ms;
    float max_ms;
    float throughput_gbps;              /* valid when has_gbps */
    float tflops;                       /* valid when has_tflops */
    uint32_t has_gbps;
    uint32_t has_tflops;
} nc_benchmark_result;

void nc_benchmark_options_init(nc_benchmark_options *opts);
/* runKernel (src/benchmark.zig:35-92): warmup launches, sync, then per iteration
 * record(start) -> launch -> record(stop) -> synchronize(stop) -> elapsed; mean/min/max;
 * GB/s = bytes/(mean_ms*1e6), TFLOP/s = flops/(mean_ms*1e9). */
int nc_benchmark_run_kernel(const nc_benchmark_options *opts, nc_function fn, const nc_launch_config *cfg,
                            void **kernel_params, nc_benchmark_result *out);
/* Metric arithmetic of runKernel, exposed for host tests (src/benchmark.zig:80-89). */
void nc_benchmark_finish(const float *iter_ms, uint32_t iters, uint64_t bytes, uint64_t flops,
                         nc_benchmark_result *out);

/* ------------------------------------------------------------------------------------------------
 * Host-side input generation (no GPU needed).
 * ---------------------------------------------------------------------------------------------- */
/* fillFlashInput (src/main.zig:1207-1211): data[i] = f16(((i*mul + add) % 17) * scale). */
void nc_fill_flash_input(uint16_t *data, size_t n, uint64_t mul, uint64_t add, float scale);
/* Seeded synthetic inputs: SplitMix64 keyed by (seed, tensor_id), element i uses counter i, so any
 * slice can be regenerated independently. Uniform in [lo, hi) from the top 24 bits; normal via
 * Box-Muller on element pairs; every value rounded to f16 round-to-nearest-even. */
void nc_fill_uniform_f16(uint16_t *out, size_t n, uint64_t seed, uint32_t tensor_id, float lo, float hi);
void nc_fill_normal_f16(uint16_t *out, size_t n, uint64_t seed, uint32_t tensor_id, float mean, float sigma);
/* The same draws rounded to bfloat16 (round-to-nearest-even) for the bf16 extension. */
void nc_fill_uniform_bf16(uint16_t *out, size_t n, uint64_t seed, uint32_t tensor_id, float lo, float hi);
void nc_fill_normal_bf16(uint16_t *out, size_t n, uint64_t seed, uint32_t tensor_id, float mean, float sigma);
/* IEEE binary16 <-> binary32 (round-to-nearest-even, overflow to inf, subnormals kept). */
uint16_t nc_f32_to_f16(float x);
float nc_f16_to_f32(uint16_t h);
/* bfloat16 (the upper half of a binary32) <-> binary32; rounding to nearest even, NaN kept quiet. */
uint16_t nc_f32_to_bf16(float x);
float nc_bf16_to_f32(uint16_t h);

/* Library version string. */
const char *nc_version(void);

#ifdef __cplusplus
}
#endif

#endif /* NOTCUTE_FLASH_H */
