// benchmark.cpp — event-timed kernel benchmark (the role of src/benchmark.zig in the reference).
//
// nc_benchmark_run_kernel follows runKernel (src/benchmark.zig:35-92) step for step: warmup
// launches, a stream (or device) synchronize, then per iteration record(start) -> launch ->
// record(stop) -> synchronize(stop) -> elapsed, and mean/min/max with the GB/s and TFLOP/s
// formulas of src/benchmark.zig:80-89 (f32 arithmetic, as the reference accumulates in f32).

#include <cmath>
#include <cstring>
#include <vector>

#include "notcute_flash.h"

extern "C" {

void nc_benchmark_options_init(nc_benchmark_options *opts) {
    if (!opts) return;
    std::memset(opts, 0, sizeof *opts);
    opts->warmup_iters = 3;  // src/benchmark.zig:27
    opts->iters = 10;        // src/benchmark.zig:28
}

void nc_benchmark_finish(const float *iter_ms, uint32_t iters, uint64_t bytes, uint64_t flops,
                         nc_benchmark_result *out) {
    if (!out) return;
    std::memset(out, 0, sizeof *out);
    if (!iter_ms || iters == 0) return;
    float total = 0.f, mn = INFINITY, mx = -INFINITY;
    for (uint32_t i = 0; i < iters; ++i) {
        total += iter_ms[i];
        if (iter_ms[i] < mn) mn = iter_ms[i];
        if (iter_ms[i] > mx) mx = iter_ms[i];
    }
    const float mean = total / (float)iters;
    out->mean_ms = mean;
    out->min_ms = mn;
    out->max_ms = mx;
    if (bytes) {
        out->throughput_gbps = (float)bytes / (mean * 1000000.0f);
        out->has_gbps = 1;
    }
    if (flops) {
        out->tflops = (float)flops / (mean * 1000000000.0f);
        out->has_tflops = 1;
    }
}

int nc_benchmark_run_kernel(const nc_benchmark_options *opts, nc_function fn, const nc_launch_config *cfg,
                            void **kernel_params, nc_benchmark_result *out) {
    if (!opts || !fn || !cfg || !out || opts->iters == 0) return NC_ERROR_INVALID_VALUE;
    nc_event start = nullptr, stop = nullptr;
    int st = nc_event_create(&start);
    if (st) return st;
    st = nc_event_create(&stop);
    if (st) {
        nc_event_destroy(start);
        return st;
    }
    nc_launch_config c = *cfg;
    c.stream = opts->stream;
    std::vector<float> ms(opts->iters, 0.f);
    for (uint32_t i = 0; i < opts->warmup_iters && !st; ++i) st = nc_function_launch(fn, &c, kernel_params);
    if (!st) st = opts->stream ? nc_stream_synchronize(opts->stream) : nc_device_synchronize();
    for (uint32_t i = 0; i < opts->iters && !st; ++i) {
        st = nc_event_record(start, opts->stream);
        if (!st) st = nc_function_launch(fn, &c, kernel_params);
        if (!st) st = nc_event_record(stop, opts->stream);
        if (!st) st = nc_event_synchronize(stop);
        if (!st) st = nc_event_elapsed(&ms[i], start, stop);
    }
    nc_event_destroy(start);
    nc_event_destroy(stop);
    if (st) return st;
    nc_benchmark_finish(ms.data(), opts->iters, opts->bytes_processed, opts->flops_processed, out);
    return NC_SUCCESS;
}

}  // extern "C"
