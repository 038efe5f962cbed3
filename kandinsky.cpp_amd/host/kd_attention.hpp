// kd_attention.hpp - C++ host mirror of kandinsky.cpp's ops::attention flash
// branch (src/core/ops.hpp:107-207) on top of the libkd_fa C ABI.
//
// The reference reshapes the activations q [C, Lq, N] and k/v [C_kv, Lk, N]
// (C = n_head * d_head) into per-head tensors with cont(permute(...)) copies
// (ops.hpp:122-131), casts K/V to F16 (ops.hpp:167-169), transposes and casts
// the mask (ops.hpp:173), builds GGML_OP_FLASH_ATTN_EXT with scale
// 1/sqrt(d_head) (ops.hpp:161, 176-177), asks supports_op (ops.hpp:179) and
// falls back to mul_mat + soft_max when the backend says no (ops.hpp:187-202).
// Here the per-head views are strided views of the same memory -- no copy --
// since the kernel reads any 16-byte-aligned row stride, and the result is
// written straight into the [C, Lq, N] layout the out_layer consumes
// (ops.hpp:204-206), for any N (the reference's view at ops.hpp:183 is only
// correct for N = 1).
//
// Header-only; link against libkd_fa.so.
#pragma once

#include <cmath>
#include <cstddef>
#include <cstdint>

#include "../../include/kd_fa.h"

namespace kd {

// A dense row-major activation as the reference holds it: ggml [C, L, N]
// (ne0 = C contiguous), element type `type`, row stride `row_bytes`
// (>= C * element size), batch stride `batch_bytes`.
struct Activation {
    void *data = nullptr;
    int32_t type = KD_FA_TYPE_F32;
    int64_t C = 0, L = 0, N = 1;
    size_t row_bytes = 0;
    size_t batch_bytes = 0;
};

inline size_t type_size(int32_t t) { return t == KD_FA_TYPE_F32 ? 4 : 2; }

// ggml view [d_head, L, n_head, N] of an activation [n_head * d_head, L, N]:
// head h of token l is the d_head elements at l*row + h*d_head*elem.
inline kd_fa_tensor head_view(const Activation &x, int64_t n_head) {
    kd_fa_tensor t{};
    const int64_t d = x.C / n_head;
    const size_t es = type_size(x.type);
    t.type = x.type;
    t.ne[0] = d;
    t.ne[1] = x.L;
    t.ne[2] = n_head;
    t.ne[3] = x.N;
    t.nb[0] = es;
    t.nb[1] = x.row_bytes;
    t.nb[2] = (size_t)d * es;
    t.nb[3] = x.batch_bytes;
    t.data = x.data;
    return t;
}

// F32 output [C, Lq, N] written as ggml's permuted [d_head, n_head, Lq, N].
inline kd_fa_tensor out_view(void *data, int64_t d_head, int64_t n_head, int64_t Lq, int64_t N) {
    kd_fa_tensor t{};
    t.type = KD_FA_TYPE_F32;
    t.ne[0] = d_head;
    t.ne[1] = n_head;
    t.ne[2] = Lq;
    t.ne[3] = N;
    t.nb[0] = 4;
    t.nb[1] = (size_t)d_head * 4;
    t.nb[2] = t.nb[1] * (size_t)n_head;
    t.nb[3] = t.nb[2] * (size_t)Lq;
    t.data = data;
    return t;
}

// Optional additive mask: F16 [Lk, Lq', 1, N'] rows per query (the layout
// ops.hpp:173 produces with cast(transpose(mask))).
struct Mask {
    const void *data = nullptr;
    int64_t Lk = 0, Lq = 0, N = 1;
    size_t row_bytes = 0;
    size_t batch_bytes = 0;
};

// Status of attention(): KD_FA_OK, or why the node was not run (the
// caller then takes its own fallback, as ops.hpp:187-202 does).
struct Result {
    int status = KD_FA_OK;
    bool ran() const { return status == KD_FA_OK; }
};

// The GGML_OP_FLASH_ATTN_EXT node ops::attention builds (ops.hpp:159-177),
// as strided views of the activations.  Returns false for a bad head split.
inline bool make_node(const Activation &q, const Activation &k, const Activation &v,
                      int64_t n_head, void *out, const Mask *mask, kd_fa_desc *node) {
    if (n_head <= 0 || q.C % n_head) return false;
    const int64_t d_head = q.C / n_head;
    if (k.C % d_head || v.C != k.C) return false;
    const int64_t n_kv_head = k.C / d_head;
    kd_fa_desc d{};
    d.q = head_view(q, n_head);
    d.k = head_view(k, n_kv_head);
    d.v = head_view(v, n_kv_head);
    if (mask && mask->data) {
        d.mask.type = KD_FA_TYPE_F16;
        d.mask.ne[0] = mask->Lk;
        d.mask.ne[1] = mask->Lq;
        d.mask.ne[2] = 1;
        d.mask.ne[3] = mask->N;
        d.mask.nb[0] = 2;
        d.mask.nb[1] = mask->row_bytes;
        d.mask.nb[2] = mask->row_bytes * (size_t)mask->Lq;
        d.mask.nb[3] = mask->batch_bytes;
        d.mask.data = const_cast<void *>(mask->data);
    }
    d.dst = out_view(out, d_head, n_head, q.L, q.N);
    d.scale = 1.0f / std::sqrt((float)d_head);   // ops.hpp:161
    d.max_bias = 0.0f;
    d.logit_softcap = 0.0f;
    d.prec = KD_FA_PREC_F32;                     // ops.hpp:177
    *node = d;
    return true;
}

// ops::attention(ctx, backend, q, k, v, n_head, mask, flash=true,
// causal=false) for one GPU stream.  q: [C, Lq, N]; k, v: [C_kv, Lk, N]
// with C_kv = n_kv_head * d_head (grouped heads are broadcast by the op,
// no repeat copies as ops.hpp:135-157 make); out: [C, Lq, N], F32 (the
// node's type) or, with out_type F16 / BF16, rounded to that type.
// rope (optional): rotate Q and K on load (rope::apply, src/rope.hpp:109).
// norm (optional): the query_norm / key_norm RMSNorm of the attention
// modules before RoPE (crossdit.hpp:135-136, 192-193).
// k_workspace (optional, kd_fa_workspace_size bytes): the transformed K,
// and for a masked cross-attention its mask summary (kd_fa_run_ws).
inline Result attention(const Activation &q, const Activation &k, const Activation &v,
                        int64_t n_head, void *out, const Mask *mask = nullptr,
                        const kd_fa_rope *rope = nullptr, void *stream = nullptr,
                        void *k_workspace = nullptr, size_t k_workspace_bytes = 0,
                        const kd_fa_qk_norm *norm = nullptr, int32_t out_type = KD_FA_TYPE_F32) {
    Result r;
    kd_fa_desc d{};
    if (!make_node(q, k, v, n_head, out, mask, &d)) {
        r.status = KD_FA_ERR_SHAPE;
        return r;
    }
    if (out_type != KD_FA_TYPE_F32) {
        d.dst.type = out_type;
        d.dst.nb[0] = 2;
        d.dst.nb[1] = (size_t)d.dst.ne[0] * 2;
        d.dst.nb[2] = d.dst.nb[1] * (size_t)d.dst.ne[1];
        d.dst.nb[3] = d.dst.nb[2] * (size_t)d.dst.ne[2];
    }
    int reason = KD_FA_OK;
    const bool ok = norm ? kd_fa_dit_supports(&d, rope, norm, &reason)
                  : rope ? kd_fa_rope_supports(&d, rope, &reason)
                         : kd_fa_supports(&d, &reason);
    if (!ok) {
        r.status = reason;
        return r;
    }
    if (norm)
        r.status = kd_fa_dit_run(&d, rope, norm, k_workspace, k_workspace_bytes, stream);
    else if (rope && k_workspace)
        r.status = kd_fa_rope_run_ws(&d, rope, k_workspace, k_workspace_bytes, stream);
    else if (rope)
        r.status = kd_fa_rope_run(&d, rope, stream);
    else if (k_workspace)
        r.status = kd_fa_run_ws(&d, k_workspace, k_workspace_bytes, stream);
    else
        r.status = kd_fa_run(&d, stream);
    return r;
}

}  // namespace kd
