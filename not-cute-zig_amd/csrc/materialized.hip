// Materialized-attention baseline: the `cublas_materialized` case of the reference's baseline
// program (tools/cuda_baselines.cu:689-759) on MI355X. Two rocBLAS strided-batched GEMMs (f16 in,
// f32 accumulate/out) around a row-softmax kernel of this file:
//
//   scores[b][q][key] = sum_c Q[b][q][c] K[b][key][c]                      (f32, BH x S x S)
//   probs[b][q][key]  = f16(f16(exp(scale*s - m_q)) * (1 / sum_key exp(scale*s - m_q)))
//                       over the keys visible to q (all, or key <= q when causal); 0 elsewhere
//   O[b][q][c]        = sum_key probs[b][q][key] V[b][key][c]               (f32)
//
// Both GEMMs run over the full S x S matrices, causal or not, as the reference's do. This is a
// baseline to time the fused flash path against; the flash path itself never calls it. With
// element_type NC_ELEMENT_BF16 the inputs and probabilities are bf16 instead of f16.

#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <cmath>
#include <cstdio>
#include <limits>
#include <string>

#include "notcute_baselines.h"

namespace {

thread_local std::string g_error;

int fail(int status, const char *what, const char *detail) {
    char buf[256];
    std::snprintf(buf, sizeof buf, "%s: %s", what, detail);
    g_error = buf;
    return status;
}

int check_rocblas(rocblas_status rs, const char *what) {
    if (rs == rocblas_status_success) return NC_SUCCESS;
    int st = NC_ERROR_UNKNOWN;
    switch (rs) {
    case rocblas_status_memory_error: st = NC_ERROR_OUT_OF_MEMORY; break;
    case rocblas_status_invalid_handle:
    case rocblas_status_invalid_pointer:
    case rocblas_status_invalid_size:
    case rocblas_status_invalid_value:
    case rocblas_status_size_unchanged:
    case rocblas_status_size_increased:
    case rocblas_status_size_query_mismatch: st = NC_ERROR_INVALID_VALUE; break;
    case rocblas_status_not_implemented: st = NC_ERROR_NOT_FOUND; break;
    default: break;
    }
    return fail(st, what, rocblas_status_to_string(rs));
}

int check_hip(hipError_t e, const char *what) {
    if (e == hipSuccess) return NC_SUCCESS;
    return fail(nc_status_from_hip((int)e), what, hipGetErrorName(e));
}

uint64_t row_of(uint64_t row_stride, uint64_t d) { return row_stride ? row_stride : d; }

// ---------------------------------------------------------------------------------------------
// Row softmax (attention_softmax_kernel, tools/cuda_baselines.cu:459-505). One workgroup per
// (slice, query row): blockDim.x lanes hold NV scores each in registers, so each score is read
// once (only the visible ones) and each probability written once. Block-wide max and sum go
// through cross-lane exchanges within each wave and one LDS slot per wave.
// ---------------------------------------------------------------------------------------------
template <bool MAX>
__device__ float block_reduce(float v, float *red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(v, off, 64);
        v = MAX ? fmaxf(v, o) : v + o;
    }
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();  // the previous reduction's readers are done with red[]
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    v = red[0];
    for (int i = 1; i < nw; ++i) v = MAX ? fmaxf(v, red[i]) : v + red[i];
    return v;
}

// Round to the probability type (f16, or bf16 when BF) and back to f32.
template <bool BF>
__device__ float round_elem(float x) {
    if constexpr (BF)
        return (float)(__bf16)x;
    else
        return (float)(_Float16)x;
}
template <bool BF>
__device__ uint16_t elem_bits(float x) {
    if constexpr (BF)
        return __builtin_bit_cast(uint16_t, (__bf16)x);
    else
        return __builtin_bit_cast(uint16_t, (_Float16)x);
}

template <int NV, bool BF>
__global__ __launch_bounds__(1024) void nc_materialized_softmax(const float *__restrict__ scores,
                                                                 uint16_t *__restrict__ probs, uint32_t S,
                                                                 float scale, uint32_t causal) {
    __shared__ float red[16];
    const uint32_t row = blockIdx.x % S;
    const size_t base = (size_t)blockIdx.x * S;  // (slice * S + row) * S
    const float *src = scores + base;
    uint16_t *dst = probs + base;
    const uint32_t T = blockDim.x;
    const uint32_t last = causal ? row : S - 1;  // last visible key

    float x[NV];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const uint32_t j = threadIdx.x + i * T;
        x[i] = j <= last ? src[j] * scale : -INFINITY;
        m = fmaxf(m, x[i]);
    }
    m = block_reduce<true>(m, red);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const uint32_t j = threadIdx.x + i * T;
        x[i] = j <= last ? expf(x[i] - m) : 0.f;
        sum += x[i];
    }
    sum = block_reduce<false>(sum, red);
    const float inv = 1.f / sum;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const uint32_t j = threadIdx.x + i * T;
        // The weight is rounded to the probability type before it is normalised, and again after.
        if (j < S) dst[j] = elem_bits<BF>(round_elem<BF>(x[i]) * inv);
    }
}

// Lanes per row and scores per lane: 64 x {1..8} up to S = 512, 256 x {4..32} up to 8192,
// 1024 x 32 up to 32768.
int softmax_geometry(uint32_t S, uint32_t *threads) {
    const uint32_t T = S <= 512 ? 64u : (S <= 8192 ? 256u : 1024u);
    const uint32_t need = (S + T - 1) / T;
    int nv = 1;
    while ((uint32_t)nv < need) nv <<= 1;
    *threads = T;
    return nv;
}

template <bool BF>
hipError_t launch_softmax_t(const float *scores, uint16_t *probs, uint32_t S, uint32_t bh, float scale,
                            uint32_t causal, hipStream_t stream) {
    uint32_t T = 0;
    const int nv = softmax_geometry(S, &T);
    const dim3 grid((uint32_t)((uint64_t)S * bh)), block(T);
    switch (nv) {
    case 1: hipLaunchKernelGGL((nc_materialized_softmax<1, BF>), grid, block, 0, stream, scores, probs, S, scale, causal); break;
    case 2: hipLaunchKernelGGL((nc_materialized_softmax<2, BF>), grid, block, 0, stream, scores, probs, S, scale, causal); break;
    case 4: hipLaunchKernelGGL((nc_materialized_softmax<4, BF>), grid, block, 0, stream, scores, probs, S, scale, causal); break;
    case 8: hipLaunchKernelGGL((nc_materialized_softmax<8, BF>), grid, block, 0, stream, scores, probs, S, scale, causal); break;
    case 16: hipLaunchKernelGGL((nc_materialized_softmax<16, BF>), grid, block, 0, stream, scores, probs, S, scale, causal); break;
    case 32: hipLaunchKernelGGL((nc_materialized_softmax<32, BF>), grid, block, 0, stream, scores, probs, S, scale, causal); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_softmax(const float *scores, uint16_t *probs, uint32_t S, uint32_t bh, float scale, uint32_t causal,
                          bool bf16, hipStream_t stream) {
    return bf16 ? launch_softmax_t<true>(scores, probs, S, bh, scale, causal, stream)
                : launch_softmax_t<false>(scores, probs, S, bh, scale, causal, stream);
}

bool fits_i32(uint64_t x) { return x <= (uint64_t)std::numeric_limits<int32_t>::max(); }

}  // namespace

struct nc_materialized_st {
    rocblas_handle handle;
    hipStream_t stream;
};

extern "C" {

const char *nc_materialized_last_error(void) { return g_error.c_str(); }

int nc_materialized_create(nc_materialized *out, nc_stream stream) {
    if (!out) return fail(NC_ERROR_INVALID_VALUE, "nc_materialized_create", "null output");
    *out = nullptr;
    rocblas_handle h = nullptr;
    int st = check_rocblas(rocblas_create_handle(&h), "rocblas_create_handle");
    if (st) return st;
    st = check_rocblas(rocblas_set_stream(h, (hipStream_t)stream), "rocblas_set_stream");
    if (st) {
        rocblas_destroy_handle(h);
        return st;
    }
    *out = new nc_materialized_st{h, (hipStream_t)stream};
    return NC_SUCCESS;
}

int nc_materialized_destroy(nc_materialized plan) {
    if (!plan) return NC_SUCCESS;
    const int st = check_rocblas(rocblas_destroy_handle(plan->handle), "rocblas_destroy_handle");
    delete plan;
    return st;
}

uint64_t nc_materialized_workspace_bytes(const nc_flash_options *opts) {
    if (nc_flash_validate(opts) != NC_SUCCESS) return 0;
    const uint64_t S = opts->seq_len, bh = opts->batch_heads;
    uint64_t ss = 0, n = 0, bytes = 0;
    if (__builtin_mul_overflow(S, S, &ss) || __builtin_mul_overflow(ss, bh, &n) ||
        __builtin_mul_overflow(n, (uint64_t)(sizeof(float) + sizeof(uint16_t)), &bytes))
        return 0;
    return bytes;
}

int nc_materialized_attention(nc_materialized plan, const uint16_t *q, size_t q_len, const uint16_t *k, size_t k_len,
                              const uint16_t *v, size_t v_len, float *o, size_t o_len, void *workspace,
                              uint64_t workspace_bytes, const nc_flash_options *opts) {
    const char *me = "nc_materialized_attention";
    int st = nc_flash_validate(opts);
    if (st) return fail(st, me, "options rejected by nc_flash_validate");
    if (!plan || !q || !k || !v || !o || !workspace) return fail(NC_ERROR_INVALID_VALUE, me, "null pointer");
    const nc_flash_options &op = *opts;
    const uint64_t need[4] = {op.batch_heads * op.q_stride, op.batch_heads * op.k_stride,
                              op.batch_heads * op.v_stride, op.batch_heads * op.o_stride};
    const uint64_t have[4] = {q_len, k_len, v_len, o_len};
    for (int i = 0; i < 4; ++i)
        if (have[i] < need[i]) return fail(NC_ERROR_INVALID_VALUE, me, "buffer shorter than batch_heads slices");
    if (op.seq_len > NC_MATERIALIZED_MAX_SEQ) return fail(NC_ERROR_INVALID_VALUE, me, "seq_len above the softmax limit");
    const uint64_t ws = nc_materialized_workspace_bytes(opts);
    if (ws == 0 || workspace_bytes < ws) return fail(NC_ERROR_INVALID_VALUE, me, "workspace too small");

    const uint64_t S = op.seq_len, d = op.head_dim, bh = op.batch_heads;
    const uint64_t qr = row_of(op.q_row_stride, d), kr = row_of(op.k_row_stride, d);
    const uint64_t vr = row_of(op.v_row_stride, d), orow = row_of(op.o_row_stride, d);
    // rocBLAS takes 32-bit sizes, leading dimensions and batch counts; the flat softmax grid is
    // 32-bit too.
    if (!fits_i32(bh) || !fits_i32(qr) || !fits_i32(kr) || !fits_i32(vr) || !fits_i32(orow) || !fits_i32(S * bh))
        return fail(NC_ERROR_INVALID_VALUE, me, "dimension beyond 32 bits");

    float *scores = static_cast<float *>(workspace);
    uint16_t *probs = reinterpret_cast<uint16_t *>(static_cast<char *>(workspace) + S * S * bh * sizeof(float));
    const bool bf16 = op.element_type == NC_ELEMENT_BF16;
    const rocblas_datatype et = bf16 ? rocblas_datatype_bf16_r : rocblas_datatype_f16_r;
    const rocblas_int n = (rocblas_int)S, kd = (rocblas_int)d, batch = (rocblas_int)bh;
    const rocblas_stride ss = (rocblas_stride)(S * S);
    const float one = 1.f, zero = 0.f;

    // Column-major view: K as a d x S matrix (ld = K row pitch) is K^T, Q likewise Q^T; the
    // S x S result C = (K^T)^T Q^T = K Q^T, column q holding query q's scores, i.e. row-major
    // scores[q][key].
    st = check_rocblas(rocblas_set_pointer_mode(plan->handle, rocblas_pointer_mode_host), "rocblas_set_pointer_mode");
    if (st) return st;
    st = check_rocblas(
        rocblas_gemm_strided_batched_ex(plan->handle, rocblas_operation_transpose, rocblas_operation_none, n, n, kd,
                                        &one, k, et, (rocblas_int)kr, (rocblas_stride)op.k_stride,
                                        q, et, (rocblas_int)qr, (rocblas_stride)op.q_stride, &zero,
                                        scores, rocblas_datatype_f32_r, n, ss, scores, rocblas_datatype_f32_r, n, ss,
                                        batch, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0),
        "rocblas_gemm_strided_batched_ex (Q K^T)");
    if (st) return st;
    st = check_hip(launch_softmax(scores, probs, (uint32_t)S, (uint32_t)bh, op.scale, op.causal ? 1u : 0u, bf16,
                                  plan->stream),
                   "nc_materialized_softmax launch");
    if (st) return st;
    // V as a d x S column-major matrix is V^T, probs as an S x S one is P^T: C = V^T P^T = (P V)^T,
    // a d x S column-major matrix with ld = O row pitch, i.e. row-major O[q][c]. Only the d
    // leading elements of each O row are written.
    return check_rocblas(
        rocblas_gemm_strided_batched_ex(plan->handle, rocblas_operation_none, rocblas_operation_none, kd, n, n, &one, v,
                                        et, (rocblas_int)vr, (rocblas_stride)op.v_stride, probs,
                                        et, n, ss, &zero, o, rocblas_datatype_f32_r,
                                        (rocblas_int)orow, (rocblas_stride)op.o_stride, o, rocblas_datatype_f32_r,
                                        (rocblas_int)orow, (rocblas_stride)op.o_stride, batch, rocblas_datatype_f32_r,
                                        rocblas_gemm_algo_standard, 0, 0),
        "rocblas_gemm_strided_batched_ex (P V)");
}

}  // extern "C"
