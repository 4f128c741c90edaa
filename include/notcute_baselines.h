/*
 * notcute_baselines.h — C ABI of the materialized-attention baseline (libnotcute_baselines.so).
 *
 * Replaces the `cublas_materialized` case of the reference's baseline program
 * (tools/cuda_baselines.cu:689-759): QK^T by one strided-batched GEMM into an f32 score matrix,
 * a row softmax (scale, causal mask, normalisation) into f16 probabilities, and PV by a second
 * strided-batched GEMM into f32 O. Here the GEMMs are rocBLAS (f16 inputs, f32 accumulate and
 * output) and the softmax is a gfx950 kernel of this library. It is a baseline to time the flash
 * path against, not part of that path: it reads and writes the full BH x S x S score and
 * probability matrices (for causal too, as the reference does).
 *
 * Conventions as in notcute_flash.h: nc_status return codes, plain device pointers, Q/K/V f16 bit
 * patterns (bf16 with element_type NC_ELEMENT_BF16, probabilities then bf16 too), O f32,
 * asynchronous on the plan's stream, one process / one GPU / one calling thread.
 * Layout and validation are those of nc_flash_options / nc_flash_validate, row strides included.
 * The library links libnotcute_flash.so (validation, status names) and librocblas.so.
 */
#ifndef NOTCUTE_BASELINES_H
#define NOTCUTE_BASELINES_H

#include <stddef.h>
#include <stdint.h>

#include "notcute_flash.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Largest seq_len the softmax kernel holds in one workgroup (32 scores per lane, 1024 lanes). */
#define NC_MATERIALIZED_MAX_SEQ 32768u

typedef struct nc_materialized_st *nc_materialized; /* rocBLAS handle + stream */

/* cublasCreate (tools/cuda_baselines.cu:694-695), bound to `stream` (NULL = default stream).
 * Needs nc_init() first. */
int nc_materialized_create(nc_materialized *out, nc_stream stream);
/* cublasDestroy (tools/cuda_baselines.cu:760). NULL is accepted. */
int nc_materialized_destroy(nc_materialized plan);

/* Workspace the caller provides: BH*S*S f32 scores followed by BH*S*S 16-bit probabilities
 * (scores_len * (sizeof(float) + sizeof(half)), tools/cuda_baselines.cu:683-686, 757). Returns 0
 * when the options are invalid or the size overflows 64 bits. */
uint64_t nc_materialized_workspace_bytes(const nc_flash_options *opts);

/* The materialized lambda (tools/cuda_baselines.cu:700-752): GEMM S = Q K^T (f32), softmax of
 * scale*S per query row over its visible keys (all keys, or keys <= row when causal) with
 * P = f16(f16(exp(x - max)) / sum), GEMM O = P V (f32). Lengths are element counts as in
 * nc_flash_launch; NC_ERROR_INVALID_VALUE for invalid options, short buffers, a workspace smaller
 * than nc_materialized_workspace_bytes, or seq_len > NC_MATERIALIZED_MAX_SEQ. Only the S x d
 * active elements of each O slice are written. */
int nc_materialized_attention(nc_materialized plan, const uint16_t *q, size_t q_len, const uint16_t *k, size_t k_len,
                              const uint16_t *v, size_t v_len, float *o, size_t o_len, void *workspace,
                              uint64_t workspace_bytes, const nc_flash_options *opts);

/* Text of the last failure in this library on this thread (rocBLAS or HIP status and call), or "". */
const char *nc_materialized_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* NOTCUTE_BASELINES_H */
