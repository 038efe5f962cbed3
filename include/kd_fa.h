/*
 * kd_fa.h - C ABI of the gfx950 flash-attention backend hook for
 *           kandinsky.cpp's CrossDiT attention (GGML_OP_FLASH_ATTN_EXT).
 *
 * The reference builds exactly one flash-attention node:
 *     kqv = ggml_flash_attn_ext(ctx, q, k, v_perm, mask_f16, scale, 0, 0);
 *     ggml_flash_attn_ext_set_prec(kqv, GGML_PREC_F32);
 * (src/core/ops.hpp:176-177), asks the backend whether it can run it
 * (ggml_backend_supports_op, src/core/ops.hpp:179) and executes it inside
 * ggml_backend_graph_compute (src/core/executor.hpp:241).  This header is
 * the drop-in for that one node: kd_fa_supports replaces the supports_op
 * answer for GGML_OP_FLASH_ATTN_EXT, kd_fa_run replaces the backend's
 * kernel for the node, and kd_fa_rope_run additionally fuses the
 * rope::apply rotation of Q and K (src/rope.hpp:109-155, called at
 * src/models/crossdit.hpp:139-142) into the operand loads.
 *
 * Tensor views follow ggml's model: ne[0] is the innermost (contiguous)
 * dimension, nb[] are byte strides, type ids are ggml's ggml_type values,
 * so a ggml adaptor passes tensor->type / ne / nb / data through unchanged.
 *
 * Op contract (ggml GGML_OP_FLASH_ATTN_EXT, as ops.hpp:122-183 builds it):
 *   q    [Dk, Lq, H,   B ]  F32, F16 or BF16 (converted to K's type)
 *   k    [Dk, Lk, Hkv, Bk]  F16 or BF16 (F32 in the workspace forms)
 *   v    [Dv, Lk, Hkv, Bk]  same type as k, not transposed (F32 in the
 *                           workspace forms; see desc->cast_type)
 *   mask [Lk', Lq', Hm, Bm] F16, optional; Lk' >= Lk, Lq' >= Lq,
 *                           broadcast over heads (H % Hm == 0) and
 *                           batch (B % Bm == 0); row of query i is ne1 = i
 *   dst  [Dv, H, Lq, B]     F32 (ggml's permuted result); or BF16 / F16,
 *                           O rounded to nearest even on store -- the cast
 *                           the reference's out_layer input takes, fused
 *   Dk = Dv = 128 (the DiT heads, src/models/crossdit.hpp:121-160) or 512
 *   (the VAE's one-head attention block, src/models/vae.hpp:60-101: no
 *   mask, no RoPE and no norm on that size); other sizes: KD_FA_ERR_SHAPE.
 *   dst[b][i][h][:] = sum_j softmax_j(scale * <q_bhi, k_j> + mask[b,h,i,j]) v_j
 *   with h_kv = h / (H / Hkv) and b_kv = b / (B / Bk).  A row whose keys
 *   are all masked (-inf) is written as zeros.
 *
 * All device pointers belong to the caller; no entry point allocates,
 * frees, synchronises or retains a pointer.  Work is enqueued on the given
 * HIP stream (NULL = the legacy default stream).
 *
 * dst must not overlap q, k, v, the mask, the RoPE table, the norm weights
 * or the workspace: the kernels write output rows while other rows'
 * operands are still being read, and without a workspace kd_fa_rope_run and
 * kd_fa_dit_run also keep the transformed K of some heads in output rows of
 * later heads during the call (those rows hold O when the call ends).
 *
 * ABI: the structs below only ever grow at their end.  A binding compiled
 * against this header checks kd_fa_abi_version() == KD_FA_ABI_VERSION once,
 * before its first call (a library with another value lays the structs out
 * differently).
 */
#ifndef KD_FA_H
#define KD_FA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml_type ids (ggml.h enum ggml_type) for the types this op accepts. */
enum {
    KD_FA_TYPE_F32  = 0,
    KD_FA_TYPE_F16  = 1,
    KD_FA_TYPE_BF16 = 30
};

/* ggml_prec (ggml.h enum ggml_prec). */
enum {
    KD_FA_PREC_DEFAULT = 0,
    KD_FA_PREC_F32     = 10
};

/* Status codes.  Every entry point returns one of these; none aborts. */
enum {
    KD_FA_OK             = 0,
    KD_FA_ERR_NULL       = -1,   /* NULL descriptor or data pointer       */
    KD_FA_ERR_TYPE       = -2,   /* unsupported tensor type               */
    KD_FA_ERR_SHAPE      = -3,   /* shapes inconsistent with the op       */
    KD_FA_ERR_LAYOUT     = -4,   /* stride / alignment not supported      */
    KD_FA_ERR_PARAM      = -5,   /* max_bias, softcap, sinks or scale unsupported */
    KD_FA_ERR_ROPE       = -6,   /* invalid RoPE or norm descriptor       */
    KD_FA_ERR_LAUNCH     = -7,   /* HIP launch failed                     */
    KD_FA_ERR_DEVICE     = -8,   /* no gfx950 device / runtime error      */
    KD_FA_ERR_SCRATCH    = -9    /* F32 K or V exceeds the static scratch
                                    of kd_fa_dit_run_static               */
};

/* A ggml tensor view: struct ggml_tensor's type, ne, nb and data. */
typedef struct kd_fa_tensor {
    int32_t type;
    int64_t ne[4];
    size_t  nb[4];
    void   *data;
} kd_fa_tensor;

/*
 * The GGML_OP_FLASH_ATTN_EXT node: src[0..4] = q, k, v, mask, sinks and the
 * op params {scale, max_bias, logit_softcap, prec}
 * (ggml_flash_attn_ext + ggml_flash_attn_ext_set_prec, ops.hpp:176-177).
 * mask.data == NULL means "no mask" (ops.hpp:171-174 passes nullptr).
 * sinks is newer ggml's src[4] (per-head F32 logits added to each row's
 * softmax denominator); ops.hpp:176 never sets it, and a node that carries
 * one (sinks.data != NULL) is refused with KD_FA_ERR_PARAM so that the
 * caller keeps its fallback.  Zero-initialise it.
 */
typedef struct kd_fa_desc {
    kd_fa_tensor q;
    kd_fa_tensor k;
    kd_fa_tensor v;
    kd_fa_tensor mask;
    kd_fa_tensor sinks;
    kd_fa_tensor dst;
    float   scale;
    float   max_bias;
    float   logit_softcap;
    int32_t prec;
    /* The type an F32 K and V are cast to (the workspace forms of
     * kd_fa_rope_run_ws and kd_fa_dit_run only): KD_FA_TYPE_F16 -- or 0,
     * a zero-initialised field -- as ggml_cast(k, GGML_TYPE_F16) and
     * ggml_cast(v_perm, GGML_TYPE_F16) in ops::attention
     * (src/core/ops.hpp:167-169), or KD_FA_TYPE_BF16.  When only one of K
     * and V is F32 it is cast to the other's type instead.  Ignored when K
     * and V are both 16-bit.                                              */
    int32_t cast_type;
} kd_fa_desc;

/* Layout version of the structs in this header. */
#define KD_FA_ABI_VERSION 3
int kd_fa_abi_version(void);

/* RoPE operand rotation modes for kd_fa_rope_run. */
enum {
    KD_FA_ROPE_NONE  = 0,
    /* table: F32 [D, L'] view with interleaved (cos_i, sin_i) pairs, one
     * row per token, shared by all heads and batches -- exactly the
     * rope_cos_sin tensor that rope::apply consumes (src/rope.hpp:109-111)
     * and compute_visual_rope / compute_text_rope fill
     * (src/rope.hpp:36-102).  Token i of Q and of K uses row i.          */
    KD_FA_ROPE_TABLE = 1,
    /* axes: the same values factorised per axis of a (T, Hp, Wp) token
     * grid (src/rope.hpp:56-102): a contiguous F32 buffer holding
     * [T][axes[0]] ++ [Hp][axes[1]] ++ [Wp][axes[2]] interleaved
     * (cos, sin) pairs, built by kd_fa_rope_axes_fill.  Token index
     * idx = (t*Hp + h)*Wp + w (rope.hpp:74).                             */
    KD_FA_ROPE_AXES  = 2
};

typedef struct kd_fa_rope {
    int32_t      mode;
    kd_fa_tensor table;      /* KD_FA_ROPE_TABLE                         */
    const float *axes_data;  /* KD_FA_ROPE_AXES: device pointer           */
    int32_t      grid[3];    /* KD_FA_ROPE_AXES: T, Hp, Wp                */
    int32_t      axes[3];    /* KD_FA_ROPE_AXES: per-axis dims, sum = Dk  */
} kd_fa_rope;

/*
 * kd_fa_supports - replaces ggml_backend_supports_op for the node
 * (src/core/ops.hpp:179).  Returns 1 when kd_fa_run can execute it, 0 when
 * the caller must take its fallback (ops.hpp:187-202).  Host-only: never
 * touches the GPU.  When the answer is 0 and reason != NULL, *reason gets
 * the KD_FA_ERR_* code naming the first failed condition.
 */
int kd_fa_supports(const kd_fa_desc *desc, int *reason);

/*
 * kd_fa_run - executes the GGML_OP_FLASH_ATTN_EXT node on a gfx950 GPU,
 * replacing the backend kernel that ggml_backend_graph_compute dispatches
 * for it (src/core/executor.hpp:241; node built at src/core/ops.hpp:176).
 * Asynchronous on `stream` (a hipStream_t).  Returns KD_FA_OK or a
 * negative KD_FA_ERR_* code; on error nothing is enqueued.
 */
int kd_fa_run(const kd_fa_desc *desc, void *stream);

/*
 * kd_fa_run_ws - kd_fa_run with a caller workspace, as ggml's backend
 * kernels take scratch from the backend's buffer pool while the node runs
 * (ggml_backend_graph_compute, src/core/executor.hpp:241): a masked node
 * whose key set is short (Lk <= 256: the text cross-attention,
 * src/models/crossdit.hpp:174-200) with at least 65,536 query rows in all
 * (Lq * H * B) keeps in it a summary of which 64-key
 * tiles of its mask hold finite values for each 32-row block of queries,
 * written by a pass over the mask on `stream`, so that the attention skips
 * the fully masked tiles of a block without loading their mask rows; the
 * result is bitwise kd_fa_run's.  The VAE's one-head D = 512 node
 * (src/models/vae.hpp:60-101) at short token counts (fewer than 512 blocks
 * of 32 query rows: the 64x64 latent) splits every row's keys into ranges
 * computed side by side, their partial results kept in the workspace and
 * merged by a second pass; the result then differs from kd_fa_run's only
 * by F32 rounding (the ranges' sums are combined in another order).  With
 * workspace_bytes below kd_fa_workspace_size(desc, NULL, NULL), or for
 * other nodes, the call is kd_fa_run.  workspace must be 16-byte aligned (KD_FA_ERR_LAYOUT); its
 * contents need not be initialised, and calls that overlap on one buffer
 * race.  The library still allocates nothing.
 */
int kd_fa_run_ws(const kd_fa_desc *desc, void *workspace, size_t workspace_bytes, void *stream);

/*
 * kd_fa_rope_run - rope::apply(q), rope::apply(k) (src/rope.hpp:109-155,
 * as DiTSelfAttention::forward calls it, src/models/crossdit.hpp:139-142)
 * fused into kd_fa_run.  The result is defined as kd_fa_run on
 * q' = round_K(rot(q)), k' = round_K(rot(k)): each interleaved pair
 * (x0, x1) = (x[2i], x[2i+1]) of a token's row becomes
 * (x0*c - x1*s, x0*s + x1*c) in F32, then is rounded to K's type
 * (round to nearest even), as if the caller had materialised rope::apply's
 * F32 output and cast it to K's type (src/core/ops.hpp:167).
 * rope == NULL or mode KD_FA_ROPE_NONE is kd_fa_run.
 */
int kd_fa_rope_run(const kd_fa_desc *desc, const kd_fa_rope *rope, void *stream);

/*
 * kd_fa_rope_run_ws - kd_fa_rope_run for callers that can lend a K-sized
 * buffer (in a ggml graph: the tensor the unfused graph casts the rotated
 * K into, src/core/ops.hpp:167): K is rotated once per call into
 * `workspace` (contiguous [Dk, Lk, Hkv, Bk] in K's type) by a separate
 * pass on `stream`, and the attention then rotates only Q on load.  The
 * result is bitwise equal to kd_fa_rope_run's; the workspace holds the
 * rotated K afterwards.  workspace_bytes must be at least
 * kd_fa_rope_workspace_size(desc) and workspace 16-byte aligned
 * (KD_FA_ERR_LAYOUT otherwise, KD_FA_ERR_NULL when it is NULL).  The library
 * still allocates nothing.  K and V may also be F32 here (the rotation's
 * F32 output and the V projection that ops::attention casts,
 * src/core/ops.hpp:167-169): the same pass casts them, K after its
 * rotation, to desc->cast_type, V into the workspace after K (at a 256-byte
 * boundary); the result is kd_fa_rope_run's on the cast operands.
 */
int kd_fa_rope_run_ws(const kd_fa_desc *desc, const kd_fa_rope *rope, void *workspace,
                      size_t workspace_bytes, void *stream);

/* Bytes of workspace kd_fa_rope_run_ws needs: the rotated K, plus the cast
 * V when V is F32 (0 for an invalid node). */
size_t kd_fa_rope_workspace_size(const kd_fa_desc *desc);

/*
 * RMSNorm of the Q and K head rows ahead of RoPE: the query_norm / key_norm
 * modules of DiTSelfAttention and DiTCrossAttention
 * (src/models/crossdit.hpp:135-136, 192-193; RMSNorm,
 * src/core/module.hpp:163-180, computed by ops::rms_norm =
 * ggml_rms_norm + ggml_mul, src/core/ops.hpp:76-80).  For a row x of Dk
 * elements: mean = (float)(sum of the F32 squares, in double) / Dk, then
 * x * (1.0f / sqrtf(mean + eps)) * weight, each product rounded to F32.
 */
typedef struct kd_fa_qk_norm {
    const float *q_weight;   /* F32 [Dk] device pointer; NULL: Q not normalised */
    const float *k_weight;   /* F32 [Dk] device pointer; NULL: K not normalised */
    float        eps;        /* 1e-6 in the reference                            */
} kd_fa_qk_norm;

/*
 * kd_fa_dit_run - the attention of DiTSelfAttention::forward and
 * DiTCrossAttention::forward from the projections on
 * (src/models/crossdit.hpp:134-150, 191-199): each head row of Q and K is
 * normalised (norm != NULL, per weight given), then rotated (rope != NULL
 * and mode != KD_FA_ROPE_NONE; the self-attention), then rounded to K's
 * type and fed to the node.  The result is defined as kd_fa_run on
 * q' = round_K(rot(rms(q) * wq)), k' = round_K(rot(rms(k) * wk)), with
 * every step in F32 as kd_fa_qk_norm and kd_fa_rope_run state.
 * workspace != NULL: K is transformed once into it (as kd_fa_rope_run_ws,
 * same size rule; it holds k' afterwards); NULL: K tiles are transformed
 * on load.  The two give bitwise equal results.  K and V may be F32 -- the
 * projection outputs as ops::attention receives them: K normalised and
 * rotated before its one rounding, the reference's order (ops.hpp:167
 * casts after RoPE), V cast as stored (ops.hpp:168-169), both to
 * desc->cast_type by the one pre-pass launch that writes the transformed K
 * (V after K in the workspace).  The workspace is then mandatory
 * (KD_FA_ERR_NULL without one); kd_fa_dit_supports answers for this
 * workspace form, so it accepts F32 K and V.  With
 * kd_fa_workspace_size(desc, rope, norm) bytes, a masked short-key node
 * (the cross-attention) also keeps its mask summary there, after K and V
 * (as kd_fa_run_ws).  norm == NULL and rope == NULL with 16-bit K and V is
 * kd_fa_run (kd_fa_run_ws with a workspace).
 */
int kd_fa_dit_run(const kd_fa_desc *desc, const kd_fa_rope *rope, const kd_fa_qk_norm *norm,
                  void *workspace, size_t workspace_bytes, void *stream);

/*
 * Bytes of workspace kd_fa_run_ws, kd_fa_rope_run_ws and kd_fa_dit_run can
 * use for the node (0 for an invalid node or one that uses none): the
 * transformed K when rope or a key norm transforms K or K is F32, then,
 * 256-byte aligned, the cast V when V is F32 (together
 * kd_fa_rope_workspace_size bytes), then, 256-byte aligned, the mask
 * summary of a masked short-key node (4 bytes per mask batch, mask head and
 * 32 query rows); for a D = 512 node with a key split, its partial results
 * (2,056 bytes per query row and key range).
 */
size_t kd_fa_workspace_size(const kd_fa_desc *desc, const kd_fa_rope *rope, const kd_fa_qk_norm *norm);

/* kd_fa_rope_supports plus the checks of the norm descriptor.  Host-only. */
int kd_fa_dit_supports(const kd_fa_desc *desc, const kd_fa_rope *rope,
                       const kd_fa_qk_norm *norm, int *reason);

/*
 * kd_fa_rope_supports - kd_fa_supports plus the checks of the RoPE
 * descriptor.  Host-only.
 */
int kd_fa_rope_supports(const kd_fa_desc *desc, const kd_fa_rope *rope, int *reason);

/*
 * kd_fa_rope_visual_table - host-side mirror of rope::compute_visual_rope
 * (src/rope.hpp:56-102, with get_freqs src/rope.hpp:23-29): fills
 * out[(t*Hp + h)*Wp + w][Dk] (Dk = sum of axes) with interleaved
 * (cos, sin) pairs of pos * freq_i / scale_factor[axis].  The values are
 * computed in F32 exactly as the reference computes them.  Returns
 * KD_FA_OK or KD_FA_ERR_ROPE.
 */
int kd_fa_rope_visual_table(int T, int Hp, int Wp, const int axes[3],
                            const float scale_factor[3], float theta,
                            float *out);

/*
 * kd_fa_rope_axes_size / kd_fa_rope_axes_fill - the factorised form of
 * the same table for KD_FA_ROPE_AXES: (T*axes[0] + Hp*axes[1] +
 * Wp*axes[2]) floats, whose entries are bitwise equal to the columns of
 * kd_fa_rope_visual_table's rows.  Host buffers; the caller copies the
 * result to the device.
 */
size_t kd_fa_rope_axes_size(int T, int Hp, int Wp, const int axes[3]);
int kd_fa_rope_axes_fill(int T, int Hp, int Wp, const int axes[3],
                         const float scale_factor[3], float theta,
                         float *out);

/*
 * kd_fa_rope_text_table - host-side mirror of rope::compute_text_rope
 * (src/rope.hpp:36-49), the 1-D table TextBlock self-attention rotates
 * with: out[pos][D] interleaved (cos, sin) of pos * freq_i.
 */
int kd_fa_rope_text_table(int L, int D, float theta, float *out);

/*
 * kd_fa_dit_run_static - kd_fa_dit_run with the K workspace taken from a
 * device array of the library instead of a caller buffer.  It has no
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under stream capture, tight serving loops, harnesses
 * that forbid hipMalloc).  The caller passes inputs and outputs only; the
 * library allocates nothing, and the array (KD_FA_STATIC_SCRATCH_BYTES per
 * GPU, held until the process ends) is looked up (hipGetSymbolAddress) on
 * the first call on each device; make that first call outside stream
 * capture (a lookup that fails is retried on the next call).  A node whose
 * transformed K and cast V (the kd_fa_rope_workspace_size bytes) exceed the
 * array runs as kd_fa_dit_run without a workspace when K and V are 16-bit
 * (K then transformed in staged groups or on load: the same result,
 * bitwise), and is refused with KD_FA_ERR_SCRATCH before any device work
 * when K or V is F32 (their cast needs the workspace); a node that
 * transforms no K needs no K workspace and always runs.  The array also
 * holds what kd_fa_workspace_size counts beyond K and V (the mask summary,
 * the D = 512 key split's partial results) when that fits; else the call
 * runs without it.  The result is bitwise equal to kd_fa_dit_run's with a
 * caller workspace of the same size.
 * Every call on a GPU shares that GPU's array: calls that overlap on one
 * GPU (two streams, two host threads) race and must be serialised by the
 * caller.
 */
#define KD_FA_STATIC_SCRATCH_BYTES ((size_t)64 << 20)
int kd_fa_dit_run_static(const kd_fa_desc *desc, const kd_fa_rope *rope, const kd_fa_qk_norm *norm,
                         void *stream);

/*
 * kd_fa_set_routing - comparison hook for tests and tuning; it has no
 * counterpart in the reference.  Without it the kernel that runs a node is
 * a function of the node alone.  The specialised kernels compute every row
 * with the same arithmetic as the general 32-row kernel (bitwise equal
 * results), and these flags take them out of the choice so that a test can
 * compare the two.  Process-wide (an atomic read once per call); returns
 * the previous flags.  Production callers never call it.
 */
enum {
    KD_FA_ROUTE_DEFAULT = 0,
    KD_FA_ROUTE_NO_W64  = 1,   /* unmasked calls: the 32-row kernel, not the 64-row or
                                  the persistent long-prompt one                       */
    KD_FA_ROUTE_NO_XRES = 2,   /* short key sets: the 32-row kernel, not the LDS-resident */
    KD_FA_ROUTE_D512_R1 = 4,   /* D = 512: one 32-row block per workgroup                 */
    KD_FA_ROUTE_NO_SPLIT = 8,  /* D = 512, short query sets: no key split (one pass)     */
    KD_FA_ROUTE_W64_SHORT = 16, /* unmasked key sets <= 896 too: the 64-row kernel       */
    KD_FA_ROUTE_STAGED = 32,    /* K transformed without a workspace: staged whenever the
                                   shape allows, also where one on-load launch is cheaper */
    KD_FA_ROUTE_SUMMARY = 64,   /* mask summary for every masked short-key node with the
                                   workspace, also below 65,536 query rows             */
    KD_FA_ROUTE_NO_XLONG = 128, /* unmasked key sets of more than 256 keys: not the
                                   persistent kernels (the 32-row kernel up to 896
                                   keys, the 64-row one above)                         */
    KD_FA_ROUTE_NO_XLONG64 = 256 /* those with F32 Q: not the persistent 64-row kernel
                                   (the persistent 32-row one up to 1,024 keys, the
                                   64-row one above)                                   */
};
int kd_fa_set_routing(int flags);

/* Human-readable text for a KD_FA_* status code. */
const char *kd_fa_strerror(int status);

/* Library version, as MAJOR*10000 + MINOR*100 + PATCH. */
int kd_fa_version(void);

#ifdef __cplusplus
}
#endif

#endif /* KD_FA_H */
