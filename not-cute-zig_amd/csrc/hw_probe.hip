// hw_probe.hip — single-wave probes of the gfx950 instruction semantics flash_fwd.hip is built on.
//
// Not part of the flash path: the GPU tests load this code object and compare each probe's output
// with the layout the kernels assume, so a change of hardware or compiler behaviour shows up as a
// named failure instead of a parity mismatch somewhere in a kernel. Each kernel is launched with
// one workgroup of 64 threads and touches only the buffers the test sizes for it.
//
//   nc_probe_mfma32x32x16   v_mfma_f32_32x32x16_{f16,bf16}: operand and accumulator lane layout
//   nc_probe_ds_read_tr     ds_read_b64_tr_b16: which LDS elements each lane of a 16-lane group gets
//   nc_probe_permlane32     v_permlane32_swap: the lane-pair exchange used for row max / row sum

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

}  // namespace

// a: 32x16 row-major (A), b: 16x32 row-major (B), 16-bit payloads; d: 64 lanes x 16 floats.
// Lane l supplies A[l % 32][8 * (l / 32) + j] and B[8 * (l / 32) + j][l % 32] for j = 0..7 (the
// operand layout the flash kernels load K rows and Q^T columns in) and stores its 16 accumulator
// registers of D = A * B in order.
extern "C" __global__ __launch_bounds__(64) void nc_probe_mfma32x32x16(const uint16_t *a, const uint16_t *b,
                                                                        float *d, int bf16) {
    const int l = threadIdx.x;
    const int row = l % 32, k0 = 8 * (l / 32);
    u16x8 av, bv;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        av[j] = a[row * 16 + k0 + j];
        bv[j] = b[(k0 + j) * 32 + row];
    }
    floatx16 acc = {};
    if (bf16)
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bv),
                                                       acc, 0, 0, 0);
    else
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, av), __builtin_bit_cast(half8, bv), acc,
                                                      0, 0, 0);
#pragma unroll
    for (int r = 0; r < 16; ++r) d[l * 16 + r] = acc[r];
}

// LDS holds a 16 x 64 tile of 16-bit values, element (row, col) = row * 64 + col. In 16-lane group
// g = l / 16, lane m = l % 16 points at (4g + m / 4, 8g + 4 (m % 4)) — the address pattern of the
// flash kernels' V^T reads — and out[l * 4 + j] receives the j-th 16-bit value the lane gets back.
extern "C" __global__ __launch_bounds__(64) void nc_probe_ds_read_tr(uint16_t *out) {
    __shared__ __attribute__((aligned(16))) uint16_t tile[16 * 64];
    const int l = threadIdx.x;
    for (int i = l; i < 16 * 64; i += 64) tile[i] = (uint16_t)i;
    __syncthreads();
    const int g = l / 16, m = l % 16;
    const uint32_t addr = (uint32_t)(uintptr_t)tile + (uint32_t)(((4 * g + m / 4) * 64 + 8 * g + 4 * (m % 4)) * 2);
    u32x2 v;
    asm volatile("ds_read_b64_tr_b16 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        out[l * 4 + 2 * j] = (uint16_t)(v[j] & 0xffffu);
        out[l * 4 + 2 * j + 1] = (uint16_t)(v[j] >> 16);
    }
}

// out[l * 2 + 0/1] = the two results of v_permlane32_swap(x, x) with x = 1000 + lane, in the form
// the kernels' pair_max / pair_sum consume them.
extern "C" __global__ __launch_bounds__(64) void nc_probe_permlane32(uint32_t *out) {
    const uint32_t x = 1000u + threadIdx.x;
    auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    out[threadIdx.x * 2] = r[0];
    out[threadIdx.x * 2 + 1] = r[1];
}
