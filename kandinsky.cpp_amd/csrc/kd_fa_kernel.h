// kd_fa_kernel.h - launch arguments shared by the host glue (kd_fa_host.cpp)
// and the gfx950 kernels (kd_fa_kernel.hip).  Internal to libkd_fa.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kd_fa.h"

namespace kdfa {

// Byte strides are ggml's nb[1..3]; element strides nb[0] are the element
// size (checked by kd_fa_supports).
struct Args {
    const char *q;
    const char *k;
    const char *v;
    const char *m;      // F16 mask or nullptr
    char *o;            // F32 dst [Dv, H, Lq, B]
    int64_t q_nb1, q_nb2, q_nb3;
    int64_t k_nb1, k_nb2, k_nb3;
    int64_t v_nb1, v_nb2, v_nb3;
    int64_t m_nb1, m_nb2, m_nb3;
    int64_t o_nb1, o_nb2, o_nb3;
    int32_t Lq, Lk, H, B;
    int32_t rk2, rk3;   // H / Hk, B / Bk  (ggml broadcast ratios)
    int32_t rv2, rv3;   // H / Hv, B / Bv
    int32_t m_ne2, m_ne3;
    int32_t q_type;     // KD_FA_TYPE_*
    int32_t k_type;     // K as stored (F32 only for the K pre-pass; V is F32 when cast)
    int32_t mask_vec;   // mask rows are 16-byte aligned
    float scale_log2;   // scale * log2(e)
    int32_t rope_mode;  // KD_FA_ROPE_*
    const float *rope_tab;
    int64_t rope_nb1;
    const float *axes;
    int32_t grid_t, grid_h, grid_w;
    int32_t axis0, axis1, axis2;
    float rcp_h, rcp_w;   // 1.0f / grid_h, 1.0f / grid_w
    int32_t n_qt;       // query tiles per (b, h) (fa_fwd_xres: query ranges)
    int32_t n_blocks;   // n_qt * H * B
    int32_t x_blocks;   // fa_fwd_xres: 32-row query blocks per range
    int32_t heads_inner;  // block order: heads fastest (mask shared by all heads)
    int32_t o_type;       // dst element type: F32, F16 or BF16
    const float *qn_w;    // RMSNorm weight of Q (F32 [128]) or nullptr
    const float *kn_w;    // RMSNorm weight of K (F32 [128]) or nullptr
    float norm_eps;
    // fa_fwd_xres with a mask: per (mask batch, mask head, 32-row query
    // block), bit t set when key tile t holds a finite mask value for a row
    // of the block (launch_mask_live), or nullptr (every tile checked by
    // loading its mask chunks)
    const uint32_t *m_live;
    int32_t m_live_nqb;   // 32-row query blocks per (mask batch, mask head)
    // fa_fwd_d512 key split (kd_fa_run_ws): with n_split > 1 each row's keys
    // are cut into ranges of split_keys (a multiple of 32), and range s of
    // every row leaves its unnormalised O (F32 [n_split][rows][512]), then
    // its running max and row sum (F32 [n_split][rows][2]) in `part`, which
    // launch_d512_combine merges into dst; rows = B * Lq * H, row
    // (b * Lq + i) * H + h
    float *part;
    int32_t n_split, split_keys;
};

// KD_FA_OK when the current device is a gfx950 (checked once per device),
// else KD_FA_ERR_DEVICE.
int device_gfx950();

// kd_fa_dit_run's body: validation, kernel choice and launch(es).
int run_node(const kd_fa_desc *d, const kd_fa_rope *r, const kd_fa_qk_norm *n, void *ws, size_t ws_bytes,
             void *stream);

// Bytes of workspace the node needs for its transformed K and cast V (0
// when K is not transformed and V is not F32); *status gets the node's
// validation status in the workspace form, *f32_kv whether K or V is F32
// (then the workspace is mandatory).  Host-only.
size_t cast_workspace_need(const kd_fa_desc *d, const kd_fa_rope *r, const kd_fa_qk_norm *n, int *status,
                           bool *f32_kv);

// Bytes of workspace the node can use (kd_fa_workspace_size): the
// transformed K and cast V, then the mask summary of a masked short-key call.
size_t workspace_need(const kd_fa_desc *d, const kd_fa_rope *r, const kd_fa_qk_norm *n, int *status);

// Enqueue the 32-row kernel for K/V element type kv_type on `stream`, with
// `waves` waves of 32 query rows per workgroup (d128_waves; a.n_qt and
// a.n_blocks counted in 32 * waves rows).  Q is normalised (qn_w) and
// rotated (RoPE mode) on load; K too (kn_w, RoPE mode) when k_rope.
hipError_t launch(const Args &a, int kv_type, bool k_rope, int waves, hipStream_t stream);

// Enqueue the 64-rows-per-wave kernel (no mask, K as stored, Lk >= 64; a
// partial last key tile runs in the loop, which needs a scale other than 0;
// query tiles of 256 rows like the unmasked launch).
hipError_t launch_w64(const Args &a, int kv_type, hipStream_t stream);

// Enqueue the short-key kernel (K as stored, no RoPE, Lk <= kXresMaxKeys):
// K and V of a (batch, head) held in LDS, n_qt ranges of x_blocks 32-row
// query blocks per (b, h).
constexpr int kXresMaxKeys = 256;
hipError_t launch_xres(const Args &a, int kv_type, hipStream_t stream);

// Enqueue the persistent long-prompt kernel (no mask, K as stored, Q F32 or
// in K's type and neither rotated nor normalised, kXresMaxKeys < Lk <=
// kXlongMaxKeys, Q row offsets of a unit within 32 bits): units of
// kXlongRows query rows of one (b, h), a.n_qt per (b, h) and a.n_blocks in
// all, walked by at most one workgroup per CU.  (Above 1,024 keys the
// 64-row kernel's faster key loop outweighs the overlapped memory phases:
// Q F32 [128, 31744, 32, 2] with F16 K/V, 1,024 keys 1.20 against 1.22 ms,
// 1,536 keys 1.66 against 1.61.)
constexpr int kXlongRows = 256;
constexpr int kXlongMaxKeys = 1024;
hipError_t launch_xlong(const Args &a, int kv_type, hipStream_t stream);
// Unmasked key sets of more than kXresMaxKeys keys (any number) with F32 Q
// on fa_fwd_w64's key loop (fa_fwd_xlong64): units of kXlongRows rows as
// above; a wave's Q and O rows (64) within 31-bit offsets of its first row,
// K and V as fa_fwd_w64's.
hipError_t launch_xlong64(const Args &a, int kv_type, hipStream_t stream);

// Enqueue the mask summary fa_fwd_xres reads through a.m_live: one 32-bit
// word per (mask batch, mask head, 32-row query block) of the call's mask
// (rows past Lq clamped to Lq - 1, keys below Lk, Lk <= kXresMaxKeys, rows
// 16-byte aligned), bit t set when 64-key tile t holds a value other than
// -inf; written to `out` (mask_live_words(a) words).
int64_t mask_live_words(const Args &a);
hipError_t launch_mask_live(const Args &a, uint32_t *out, hipStream_t stream);

// Enqueue the D = 512 kernel (no mask, no RoPE; 32-row query tiles).
// rows: query rows per workgroup, 32 or 64 (a.n_qt and a.n_blocks counted in
// those)
hipError_t launch_d512(const Args &a, int kv_type, int rows, hipStream_t stream);
// Merge the key ranges of a split D = 512 call (a.part, a.n_split) into dst.
hipError_t launch_d512_combine(const Args &a, hipStream_t stream);

// Byte strides of the transformed K the pre-pass writes: per key, per K
// head, per K batch (contiguous [D, Lk, Hk, Bk]: 256, 256 Lk, 256 Lk Hk).
struct KStrides {
    int64_t key, head, batch;
};

// The pre-pass: normalise (kn_w), rotate (RoPE mode) and round K
// ([D, Lk, H/rk2, B/rk3] through a.k and its strides, a.k_type) into `out`
// with strides `st`, and cast an F32 V (through a.v) into `vout` with
// strides `vst`, both in the operand type kv_type; `heads` x `batch` (b, h)
// pairs of K (of V when out is nullptr; with both, K and V have the same
// heads and batches).  Either output may be nullptr.
hipError_t launch_rope_k(const Args &a, int kv_type, int heads, int batch, void *out, const KStrides &st,
                         void *vout, const KStrides &vst, hipStream_t stream);
inline hipError_t launch_rope_k(const Args &a, int kv_type, int heads, int batch, void *out, const KStrides &st,
                                hipStream_t stream) {
    return launch_rope_k(a, kv_type, heads, batch, out, st, nullptr, st, stream);
}

// Waves per workgroup of the 32-row kernel (32 query rows each): 8 (two per
// SIMD, one workgroup per CU) when it transforms K tiles on load and for
// unmasked key sets longer than kShortKeys; else 4 -- one wave per SIMD,
// two independent workgroups per CU, each one's Q load and O store
// overlapping the other's key loop (the masked text cross-attention, and
// the unmasked one with a long prompt).
constexpr int kShortKeys = 896;
constexpr int d128_waves(bool masked, bool k_on_load, int Lk) {
    return k_on_load ? 8 : (masked || Lk <= kShortKeys) ? 4 : 8;
}
constexpr int kMinBlockRows = 128;
// query rows per workgroup of the 64-row kernel
constexpr int kW64Rows = 256;

}  // namespace kdfa
