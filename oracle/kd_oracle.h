/*
 * kd_oracle.h - CPU oracle for the CrossDiT flash-attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Results are checked against this library: only the test
 * suite, the smoke check and the CPU-baseline leg of the benchmark load it.
 * The product library (libkd_fa.so) never links or calls it.
 *
 * Contents (each function cites the reference code it restates):
 *   - IEEE half / bfloat16 conversions (round to nearest even);
 *   - rope::get_freqs, compute_text_rope, compute_visual_rope, apply
 *     (src/rope.hpp:23-155);
 *   - ops::rms_norm: ggml_rms_norm + ggml_mul (src/core/ops.hpp:76-80);
 *   - kdo_fa_ggml: a restatement of ggml's per-row CPU flash-attention
 *     algorithm (ggml_compute_forward_flash_attn_ext_f16, the kernel the
 *     reference's CPU backend runs for the node built at
 *     src/core/ops.hpp:176), multithreaded over query rows;
 *   - kdo_fa_f64: textbook softmax(scale*QK^T + mask) V in double.
 *
 * The descriptors are the product's C-ABI structs (include/kd_fa.h), so a
 * test hands the same views to the oracle and to the GPU path.
 */
#ifndef KD_ORACLE_H
#define KD_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/kd_fa.h"

#ifdef __cplusplus
extern "C" {
#endif

float    kdo_f16_to_f32(uint16_t h);
uint16_t kdo_f32_to_f16(float f);
float    kdo_bf16_to_f32(uint16_t h);
uint16_t kdo_f32_to_bf16(float f);
/* Round a float to `type` (F32: identity) and back. */
float    kdo_round_to(float f, int type);

void kdo_f32_to_f16_n(const float *src, uint16_t *dst, int64_t n);
void kdo_f32_to_bf16_n(const float *src, uint16_t *dst, int64_t n);
void kdo_f16_to_f32_n(const uint16_t *src, float *dst, int64_t n);
void kdo_bf16_to_f32_n(const uint16_t *src, float *dst, int64_t n);

/* rope::get_freqs (src/rope.hpp:23-29). */
void kdo_rope_freqs(int dim, float max_period, float *out);
/* rope::compute_text_rope (src/rope.hpp:36-49): out[L][D]. */
void kdo_rope_text_table(int L, int D, float theta, float *out);
/* rope::compute_visual_rope (src/rope.hpp:56-102): out[T*Hp*Wp][sum axes]. */
void kdo_rope_visual_table(int T, int Hp, int Wp, const int axes[3],
                           const float scale_factor[3], float theta,
                           float *out);
/*
 * rope::apply (src/rope.hpp:109-155) on an F32 tensor laid out as the
 * reference passes it, x[B][L][H][D] (ggml [D, H, L, B]), with
 * table[L][D] of interleaved (cos, sin).  out may alias x.
 */
void kdo_rope_apply_f32(const float *x, int64_t D, int64_t H, int64_t L,
                        int64_t B, const float *table, float *out);

/* Flat query-row id used by both oracle entry points (ggml's ir order). */
/* ggml_rms_norm + ggml_mul by the weight over rows of D (ops.hpp:76-80). */
void kdo_rms_norm_mul(const float *x, int64_t rows, int64_t D, const float *w,
                      float eps, float *out);

/* F16C (VCVTPS2PH round-to-nearest-even / VCVTPH2PS) forms of the F16
 * conversions, used by kdo_fa_ggml's F16 V accumulator as ggml's SIMD paths
 * convert; kdo_f16_codec_mismatches counts where they differ from the
 * software codec: all 65,536 F16 patterns decoded, and `count` F32 bit
 * patterns from `start` in steps of `stride` encoded. */
void kdo_f32_to_f16_hw_n(const float *src, uint16_t *dst, int64_t n);
void kdo_f16_to_f32_hw_n(const uint16_t *src, float *dst, int64_t n);
int64_t kdo_f16_codec_mismatches(uint32_t start, uint32_t stride, int64_t count);

static inline int64_t kdo_row_id(int64_t b, int64_t h, int64_t i,
                                 int64_t H, int64_t Lq) {
    return i + Lq * (h + H * b);
}

/*
 * kdo_fa_ggml - ggml's per-row CPU algorithm, restated:
 *   Q row -> F32 -> (RoPE) -> K's dot type; for each key j: skip when
 *   mask == -inf, s = dot(k_j, q)*scale (+ softcap), s += mask; online
 *   softmax with expf and a running max M and sum S; V accumulated in F16
 *   (f16_vacc != 0 and V is F16, as ggml does) or F32; O = VKQ / S with
 *   O = 0 when S == 0.  Writes the selected rows of desc->dst (F32
 *   [Dv, H, Lq, B]).  rows == NULL computes every row.  n_threads <= 0
 *   uses every online CPU.  Returns the number of threads used, or a
 *   negative KD_FA_ERR_* code.
 */
int kdo_fa_ggml(const kd_fa_desc *desc, const kd_fa_rope *rope,
                int f16_vacc, const int64_t *rows, int64_t n_rows,
                int n_threads);

/*
 * kdo_fa_f64 - textbook attention in double on the same (type-rounded,
 * RoPE-rotated) operands: out[r][0..Dv) for each requested row, in the
 * order given (rows == NULL: every row in kdo_row_id order).  Fully masked
 * rows give zeros.  Returns threads used or a negative KD_FA_ERR_* code.
 */
int kdo_fa_f64(const kd_fa_desc *desc, const kd_fa_rope *rope,
               const int64_t *rows, int64_t n_rows, double *out,
               int n_threads);

#ifdef __cplusplus
}
#endif

#endif /* KD_ORACLE_H */
