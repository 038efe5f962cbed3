/*
 * kd_mm.h - C ABI of the gfx950 matrix product for the CrossDiT linear
 * layers: ops::linear (src/core/ops.hpp:27-43), i.e. the GGML_OP_MUL_MAT
 * node ggml_mul_mat(w, x) followed by ggml_add(bias) when the Linear has a
 * bias (src/core/module.hpp:87-110).  w is a Linear weight,
 * [in_features, out_features] in ggml order, stored as Q4_0 or Q8_0 (the
 * formats scripts/convert_to_gguf.py:90-146 writes), BF16, F16 or F32
 * (src/core/module.hpp:97-99 falls back to F32 when in_features is not a
 * multiple of the block size).  Exported by libkd_fa.so next to kd_fa.h.
 *
 * Tensor views are kd_fa_tensor (ggml's type / ne / nb / data).
 *   w    [K, N]  Q4_0, Q8_0, BF16, F16 or F32; K % 32 == 0
 *   x    [K, M, M2, M3]  F32 or BF16; rows flattened as ops::linear's
 *                reshape does (nb[2] = nb[1]*ne[1], nb[3] = nb[2]*ne[2])
 *   bias [N] F32, or data == NULL
 *   dst  [N, M, M2, M3] F32, rows flattened the same way
 *   dst[m][n] = sum_k w[n][k] * x[m][k] (+ bias[n])
 *
 * Arithmetic: w is expanded to BF16 (w_bf16 = round_bf16(value), value =
 * d * q for Q8_0, d * (nibble - 8) for Q4_0, exactly as ggml's
 * dequantize_row_q8_0 / _q4_0 compute it in F32), x is rounded to BF16,
 * the products are accumulated in F32 on the matrix cores, the bias is
 * added in F32.  ggml's own CPU path instead rounds x to Q8_0 blocks; both
 * stay within the rounding of the 8-bit formats of the exact product.
 *
 * All device pointers belong to the caller; nothing is allocated, freed,
 * synchronised or retained.  Work is enqueued on the given HIP stream.
 * Status codes are the KD_FA_* codes of kd_fa.h.
 */
#ifndef KD_MM_H
#define KD_MM_H

#include "kd_fa.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ggml_type ids of the weight formats (ggml.h enum ggml_type). */
enum {
    KD_MM_TYPE_F32  = 0,
    KD_MM_TYPE_F16  = 1,
    KD_MM_TYPE_Q4_0 = 2,
    KD_MM_TYPE_Q8_0 = 8,
    KD_MM_TYPE_BF16 = 30
};

/* The GGML_OP_MUL_MAT node of ops::linear plus its optional bias add. */
typedef struct kd_mm_desc {
    kd_fa_tensor w;      /* src0 */
    kd_fa_tensor x;      /* src1 */
    kd_fa_tensor bias;   /* F32 [N] or data == NULL */
    kd_fa_tensor dst;
} kd_mm_desc;

/*
 * kd_mm_supports - replaces ggml_backend_supports_op for the node.  Returns
 * 1 when kd_mm_run can execute it; 0 otherwise, with the first failed
 * condition's KD_FA_ERR_* code in *reason (when reason != NULL).
 * Host-only.
 */
int kd_mm_supports(const kd_mm_desc *desc, int *reason);

/*
 * kd_mm_workspace_size - bytes of workspace kd_mm_run needs: 0 when w is
 * BF16 with 16-byte aligned rows (used as stored), else N * K * 2 (w
 * expanded to BF16 rows).  0 for an invalid node.
 */
size_t kd_mm_workspace_size(const kd_mm_desc *desc);

/*
 * kd_mm_dequant - expands a weight tensor w ([K, N], any accepted type) to
 * BF16 rows out[n][k] (N * K * 2 bytes, row stride K * 2, 16-byte
 * aligned).  The values are those kd_mm_run multiplies with, so a caller
 * that keeps the result (for example from model load on) passes it as a
 * BF16 w and needs no workspace.  Asynchronous on `stream`.
 */
int kd_mm_dequant(const kd_fa_tensor *w, void *out, size_t out_bytes, void *stream);

/*
 * kd_mm_run - executes the node: w BF16 with 16-byte aligned rows is used
 * as stored; any other w is first expanded into `workspace` (at least
 * kd_mm_workspace_size bytes, 16-byte aligned; it holds the BF16 rows
 * afterwards) and the product reads it from there.  Asynchronous on
 * `stream`; returns KD_FA_OK or a negative KD_FA_ERR_* code, in which case
 * nothing is enqueued.
 */
int kd_mm_run(const kd_mm_desc *desc, void *workspace, size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* KD_MM_H */
