// kd_fa_host.cpp - C ABI of libkd_fa.so (include/kd_fa.h): operator
// validation (the supports_op answer), RoPE table helpers and the launch of
// the gfx950 kernels.  Nothing here allocates device memory, synchronises or
// keeps pointers past the call.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <vector>

#include "../../include/kd_fa.h"
#include "kd_fa_kernel.h"

namespace {

constexpr int64_t kHeadDim = 128;
// D of the 2-D VAE's single-head attention (src/models/vae.hpp:60-101)
constexpr int64_t kHeadDimVae = 512;
constexpr int64_t kI32Max = 0x7fffffff;
// A 64-row tile is addressed with 32-bit offsets from a per-tile base.
constexpr uint64_t kMaxRowStride = (uint64_t)1 << 25;

size_t elem_size(int type) { return type == KD_FA_TYPE_F32 ? 4 : 2; }
bool is_16b(uint64_t x) { return (x & 15u) == 0; }
bool is_16b(const void *p) { return is_16b(reinterpret_cast<uintptr_t>(p)); }

bool is_16bit(int type) { return type == KD_FA_TYPE_F16 || type == KD_FA_TYPE_BF16; }

// The MFMA operand type of the call: K's and V's when they are 16-bit; an
// F32 K or V (the workspace forms) is cast to the other's 16-bit type, or,
// when both are F32, to desc->cast_type (F16 unless BF16 is asked for: the
// ggml_cast of ops.hpp:167-169).
int op_type(const kd_fa_desc *d) {
    if (is_16bit(d->v.type)) return d->v.type;
    if (is_16bit(d->k.type)) return d->k.type;
    return d->cast_type == KD_FA_TYPE_BF16 ? KD_FA_TYPE_BF16 : KD_FA_TYPE_F16;
}

// Conditions of kd_fa_supports (and of the RoPE and norm descriptors when
// given).  `mask_vec` reports whether the mask rows can be read 16 bytes at
// a time.
// kv_f32: an F32 K and V are accepted (the workspace forms, whose pre-pass
// casts them; run() then also requires the workspace).
int validate(const kd_fa_desc *d, const kd_fa_rope *r, const kd_fa_qk_norm *n, bool *mask_vec,
             bool kv_f32 = false) {
    if (!d) return KD_FA_ERR_NULL;
    const kd_fa_tensor &q = d->q, &k = d->k, &v = d->v, &m = d->mask, &o = d->dst;
    if (!q.data || !k.data || !v.data || !o.data) return KD_FA_ERR_NULL;

    // types: Q is converted to K's type on load; K and V share one MFMA type
    // (an F32 K or V is cast to it by the workspace pre-pass)
    if (q.type != KD_FA_TYPE_F32 && q.type != KD_FA_TYPE_F16 && q.type != KD_FA_TYPE_BF16) return KD_FA_ERR_TYPE;
    const bool k32 = kv_f32 && k.type == KD_FA_TYPE_F32, v32 = kv_f32 && v.type == KD_FA_TYPE_F32;
    if ((!is_16bit(k.type) && !k32) || (!is_16bit(v.type) && !v32)) return KD_FA_ERR_TYPE;
    if (k.type != v.type && !k32 && !v32) return KD_FA_ERR_TYPE;
    if ((k32 || v32) && d->cast_type != 0 && !is_16bit(d->cast_type)) return KD_FA_ERR_TYPE;
    // dst: the node's F32, or a 16-bit cast of it
    if (o.type != KD_FA_TYPE_F32 && o.type != KD_FA_TYPE_F16 && o.type != KD_FA_TYPE_BF16) return KD_FA_ERR_TYPE;
    if (m.data && m.type != KD_FA_TYPE_F16) return KD_FA_ERR_TYPE;

    // op params: plain softmax attention only (ops.hpp:176 passes 0, 0 and
    // no sinks)
    if (d->max_bias != 0.0f || d->logit_softcap != 0.0f) return KD_FA_ERR_PARAM;
    if (d->sinks.data) return KD_FA_ERR_PARAM;
    if (!std::isfinite(d->scale)) return KD_FA_ERR_PARAM;

    // shapes
    for (int i = 0; i < 4; ++i)
        if (q.ne[i] < 0 || k.ne[i] < 0 || v.ne[i] < 0 || o.ne[i] < 0) return KD_FA_ERR_SHAPE;
    const int64_t D = q.ne[0];
    if (k.ne[0] != D || v.ne[0] != D || (D != kHeadDim && D != kHeadDimVae)) return KD_FA_ERR_SHAPE;
    const int64_t Lq = q.ne[1], Lk = k.ne[1], H = q.ne[2], B = q.ne[3];
    if (v.ne[1] != Lk) return KD_FA_ERR_SHAPE;
    // at least one key: the kernels clamp key rows to Lk - 1 (the reference
    // never builds the node without keys; the caller's fallback takes it)
    if (Lk == 0) return KD_FA_ERR_SHAPE;
    if (k.ne[2] == 0 || v.ne[2] == 0 || k.ne[3] == 0 || v.ne[3] == 0) return KD_FA_ERR_SHAPE;
    if (H % k.ne[2] || H % v.ne[2] || B % k.ne[3] || B % v.ne[3]) return KD_FA_ERR_SHAPE;
    if (o.ne[0] != v.ne[0] || o.ne[1] != H || o.ne[2] != Lq || o.ne[3] != B) return KD_FA_ERR_SHAPE;
    if (Lq > kI32Max || Lk > kI32Max || H > kI32Max || B > kI32Max) return KD_FA_ERR_SHAPE;
    const int64_t n_qt = (Lq + kdfa::kMinBlockRows - 1) / kdfa::kMinBlockRows;
    if (H > 0 && B > 0 && n_qt > kI32Max / H / B) return KD_FA_ERR_SHAPE;
    if (m.data) {
        if (m.ne[0] < Lk || m.ne[1] < Lq || m.ne[2] <= 0 || m.ne[3] <= 0) return KD_FA_ERR_SHAPE;
        if (H % m.ne[2] || B % m.ne[3]) return KD_FA_ERR_SHAPE;
    }

    // layouts: unit element stride; 16-byte rows for Q/K/V/dst vector access
    const kd_fa_tensor *vec_t[4] = {&q, &k, &v, &o};
    for (const kd_fa_tensor *t : vec_t) {
        if (t->nb[0] != elem_size(t->type)) return KD_FA_ERR_LAYOUT;
        if (t->nb[1] > kMaxRowStride) return KD_FA_ERR_LAYOUT;
        if (!is_16b(t->data) || !is_16b(t->nb[1]) || !is_16b(t->nb[2]) || !is_16b(t->nb[3])) return KD_FA_ERR_LAYOUT;
    }
    bool mv = false;
    if (m.data) {
        if (m.nb[0] != 2) return KD_FA_ERR_LAYOUT;
        if ((reinterpret_cast<uintptr_t>(m.data) | m.nb[1] | m.nb[2] | m.nb[3]) & 1u) return KD_FA_ERR_LAYOUT;
        mv = is_16b(m.data) && is_16b(m.nb[1]) && is_16b(m.nb[2]) && is_16b(m.nb[3]);
    }
    if (mask_vec) *mask_vec = mv;

    // D = 512 (the VAE attention block): the plain node only -- no mask, no
    // RoPE, no RMSNorm; 32-row query tiles; 32-bit V row offsets
    if (D == kHeadDimVae) {
        if (k32 || v32) return KD_FA_ERR_TYPE;
        if (m.data) return KD_FA_ERR_SHAPE;
        if ((r && r->mode != KD_FA_ROPE_NONE) || (n && (n->q_weight || n->k_weight))) return KD_FA_ERR_ROPE;
        if (H > 0 && B > 0 && (Lq + 31) / 32 > kI32Max / H / B) return KD_FA_ERR_SHAPE;
        if (Lk > 0 && (Lk - 1) * v.nb[1] + 1024 >= (int64_t)1 << 32) return KD_FA_ERR_LAYOUT;
        return KD_FA_OK;
    }

    // RoPE
    if (r && r->mode != KD_FA_ROPE_NONE) {
        const int64_t L = Lq > Lk ? Lq : Lk;
        if (r->mode == KD_FA_ROPE_TABLE) {
            const kd_fa_tensor &t = r->table;
            if (!t.data || t.type != KD_FA_TYPE_F32) return KD_FA_ERR_ROPE;
            if (t.ne[0] != kHeadDim || t.ne[1] < L || t.nb[0] != 4) return KD_FA_ERR_ROPE;
            if (!is_16b(t.data) || !is_16b(t.nb[1])) return KD_FA_ERR_ROPE;
            if (t.nb[1] > kMaxRowStride) return KD_FA_ERR_ROPE;
        } else if (r->mode == KD_FA_ROPE_AXES) {
            if (!r->axes_data || !is_16b(r->axes_data)) return KD_FA_ERR_ROPE;
            for (int i = 0; i < 3; ++i) {
                if (r->axes[i] < 0 || r->axes[i] % 8) return KD_FA_ERR_ROPE;
                if (r->grid[i] <= 0) return KD_FA_ERR_ROPE;
            }
            if (r->axes[0] + r->axes[1] + r->axes[2] != kHeadDim) return KD_FA_ERR_ROPE;
            const int64_t cells = (int64_t)r->grid[0] * r->grid[1] * r->grid[2];
            if (cells < L || L > (int64_t)1 << 24) return KD_FA_ERR_ROPE;
        } else {
            return KD_FA_ERR_ROPE;
        }
    }

    // RMSNorm weights: F32 [Dk], read 16 bytes at a time
    if (n) {
        if (!std::isfinite(n->eps) || n->eps < 0.0f) return KD_FA_ERR_ROPE;
        if ((n->q_weight && !is_16b(n->q_weight)) || (n->k_weight && !is_16b(n->k_weight))) return KD_FA_ERR_LAYOUT;
    }
    return KD_FA_OK;
}

// gfx950 check, once per device.
std::atomic<int> g_dev_state[64];

// KD_FA_ROUTE_* flags of kd_fa_set_routing (tests and tuning only).
std::atomic<int> g_route{KD_FA_ROUTE_DEFAULT};

int device_ok() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return KD_FA_ERR_DEVICE;
    if (dev < 0 || dev >= 64) return KD_FA_ERR_DEVICE;
    int st = g_dev_state[dev].load(std::memory_order_acquire);
    if (st == 0) {
        hipDeviceProp_t prop;
        st = -1;
        if (hipGetDeviceProperties(&prop, dev) == hipSuccess &&
            std::strncmp(prop.gcnArchName, "gfx950", 6) == 0)
            st = 1;
        g_dev_state[dev].store(st, std::memory_order_release);
    }
    return st == 1 ? KD_FA_OK : KD_FA_ERR_DEVICE;
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

// Key split of the D = 512 kernel through the workspace (kd_fa_run_ws):
// when its 32-row workgroups (two per CU) would leave CUs idle (fewer than
// 512: the VAE's 64x64 latent, 4,096 tokens, gives 128) and there are at least four key
// tiles (at two, 9.1 against 11.5 us), each row block's keys are cut into
// S ranges of whole 32-key tiles (S <= 8, one workgroup per range), whose
// unnormalised partial results a second pass merges.  `bytes`: the partial
// O (F32, 512 per row) and running max / row sum of every range and row.
struct D512Split {
    int S = 1;
    int keys = 0;
    size_t bytes = 0;
};
constexpr int64_t kD512Slots = 512;   // 32-row workgroups resident at once: two per CU
D512Split d512_split(int64_t Lq, int64_t Lk, int64_t H, int64_t B, int route) {
    D512Split r;
    const int64_t nb32 = (Lq + 31) / 32 * H * B;
    if ((route & KD_FA_ROUTE_NO_SPLIT) || nb32 >= kD512Slots || nb32 == 0) return r;
    const int64_t tiles = (Lk + 31) / 32;
    if (tiles < 4) return r;   // the merge's launch outweighs splitting one to three tiles
    int64_t S = std::min<int64_t>(std::min<int64_t>(8, kD512Slots / nb32), tiles);
    if (S < 2) return r;
    const int64_t per = (tiles + S - 1) / S;   // tiles per range
    S = (tiles + per - 1) / per;
    if (S < 2) return r;
    r.S = (int)S;
    r.keys = (int)(per * 32);
    r.bytes = (size_t)S * (size_t)(Lq * H * B) * (size_t)(kHeadDimVae * 4 + 8);
    return r;
}

// The summary pass costs a launch and one read of the mask (~9 us at the
// 31,744-token cross-attention, whose kernel it shortens by ~33 us); below
// 65,536 query rows in all (2,048 tokens x 32 heads) the launch is not paid
// back, and the call runs without it.  KD_FA_ROUTE_SUMMARY builds it for every
// masked short-key node that has the workspace (for comparisons).
bool summary_pays(int64_t rows, int route) { return (route & KD_FA_ROUTE_SUMMARY) || rows >= 65536; }

// The workspace of a D = 128 node, each part at a 256-byte boundary: the
// transformed K (when K is normalised, rotated or F32: contiguous
// [D, Lk, Hk, Bk] in the operand type), the cast V (when V is F32:
// contiguous [D, Lk, Hv, Bv]), then the mask summary of a masked call whose
// key set the short-key kernel can hold (one 32-bit word per mask batch,
// mask head and 32-row query block).  `cast` is the end of the K and V
// parts (kd_fa_rope_workspace_size).
struct WsLayout {
    bool k_ws = false, v_ws = false;
    size_t k_bytes = 0, v_off = 0, v_bytes = 0, cast = 0, s_off = 0, s_bytes = 0, total = 0;
};
// (force_k: K has a part whatever the descriptors say -- the rotated K of
// kd_fa_rope_run_ws, sized before its RoPE descriptor is known.)
WsLayout ws_layout(const kd_fa_desc *d, const kd_fa_rope *r, const kd_fa_qk_norm *n, bool force_k = false) {
    WsLayout w;
    const bool rope_on = r && r->mode != KD_FA_ROPE_NONE;
    w.k_ws = force_k || rope_on || (n && n->k_weight) || d->k.type == KD_FA_TYPE_F32;
    w.v_ws = d->v.type == KD_FA_TYPE_F32;
    const size_t row = (size_t)kHeadDim * 2, lk = (size_t)d->k.ne[1];
    if (w.k_ws) w.k_bytes = row * lk * (size_t)d->k.ne[2] * (size_t)d->k.ne[3];
    w.v_off = w.k_ws ? align256(w.k_bytes) : 0;
    if (w.v_ws) w.v_bytes = row * lk * (size_t)d->v.ne[2] * (size_t)d->v.ne[3];
    w.cast = w.v_ws ? w.v_off + w.v_bytes : w.k_bytes;
    if (d->mask.data && !rope_on && d->k.ne[1] <= kdfa::kXresMaxKeys) {
        w.s_off = w.cast ? align256(w.cast) : 0;
        w.s_bytes = 4 * (size_t)d->mask.ne[3] * (size_t)d->mask.ne[2] * (size_t)((d->q.ne[1] + 31) / 32);
    }
    w.total = w.s_bytes ? w.s_off + w.s_bytes : w.cast;
    return w;
}

// K is transformed (normalised and / or rotated) when a norm weight or a
// RoPE mode asks for it: with ws != nullptr once into ws (contiguous, K's
// type), after which the attention transforms only Q on load; without, group
// by group into output rows of later heads (run_staged) where staged_ok
// allows, else by the attention kernel on every K tile it loads.

// The 64-row kernel runs a partial last tile in its key loop with the
// scores of the keys past Lk set to -inf, which gives them weight 0 only
// while the scale is not 0 (-inf * 0 is NaN): with scale 0 and a partial
// tile the call goes to the 32-row kernel, which zeroes those weights after
// the exponent.
static bool w64_tail_ok(const kdfa::Args &a) { return a.Lk % 64 == 0 || a.scale_log2 != 0.0f; }

// The 64-rows-per-wave kernel takes the unmasked calls whose K streams from
// memory as stored (no transform on load) and that have more than
// kShortKeys keys and that the persistent kernels do not take (use_xlong64
// and use_xlong are asked first); its buffer-resource offsets are 32-bit.  (With one
// workgroup per CU, all CUs load Q, run the few key steps of a short key set
// and store O in step, while the 32-row kernel's 4-wave workgroups, two per
// CU, overlap one's memory phases with the other's key loop: cross-attention
// with Q F32 [128, 31744, 32, 2] and 320 keys 0.62 against 0.72 ms, 512
// keys 0.78 against 0.85, 896 keys 1.14 against 1.15, 1,024 keys even --
// the range where the persistent kernels now run when they can.)
// For comparisons, KD_FA_ROUTE_NO_W64 routes every call to the 32-row
// kernel and KD_FA_ROUTE_W64_SHORT the short key sets too to this one.
static bool use_w64(const kdfa::Args &a, bool k_on_load, int route) {
    if ((route & KD_FA_ROUTE_NO_W64) || a.m || k_on_load || a.Lk < 64 || !w64_tail_ok(a)) return false;
    if (a.Lk <= kdfa::kShortKeys && !(route & KD_FA_ROUTE_W64_SHORT)) return false;
    const int64_t lim = (int64_t)1 << 31;
    return (int64_t)(a.Lk - 1) * a.k_nb1 + 256 < lim && (int64_t)(a.Lk - 1) * a.v_nb1 + 256 < lim;
}

// Short key sets (the text cross-attention) go to the kernel that keeps K
// and V in LDS, when K is read as stored, Q is not rotated and stored as F32
// or in K's type, and a mask's rows are 16-byte aligned and hold every
// 8-key chunk that starts below Lk.  KD_FA_ROUTE_NO_XRES routes them to the
// 32-row kernel (for comparisons).
static bool use_xres(const kdfa::Args &a, int op, const kd_fa_desc *d, bool k_on_load, int route) {
    if ((route & KD_FA_ROUTE_NO_XRES) || k_on_load || a.rope_mode != KD_FA_ROPE_NONE) return false;
    if (a.Lk > kdfa::kXresMaxKeys) return false;
    if (a.q_type != KD_FA_TYPE_F32 && a.q_type != op) return false;
    if (a.m && (!a.mask_vec || d->mask.ne[0] < ((int64_t)a.Lk + 7) / 8 * 8)) return false;
    return true;
}

// Unmasked key sets past the LDS-resident kernel's (the text cross-attention
// of a long prompt as ops::attention hands it over, with F32 Q, and any
// longer unmasked node) go to the persistent kernel on the 64-row loop,
// fa_fwd_xlong64, when K is read as stored, Q is neither rotated nor
// normalised and is F32 or in K's type (then with a scale >= 0: it does not
// negate 16-bit Q), the 64-row kernel's limits hold (the partial last tile's
// weights, 31-bit K/V offsets) and a wave's 64 Q and O rows lie within
// 31-bit offsets of its first row.  (It beats fa_fwd_w64, whose workgroups
// load Q, run the key loop and store O in sequence, at every length
// measured: 1,024 keys 1.14 against 1.24 ms, 2,048 keys 1.99 against 2.07,
// 8,192 keys 7.14 against 7.16, Q F32 [128, 31744, 32, 2].)
// KD_FA_ROUTE_NO_XLONG64 routes them as if it did not exist,
// KD_FA_ROUTE_NO_XLONG, KD_FA_ROUTE_NO_W64 and KD_FA_ROUTE_W64_SHORT keep
// them off the persistent kernels (for comparisons).
static bool use_xlong64(const kdfa::Args &a, int op, bool k_on_load, int route) {
    if (route & (KD_FA_ROUTE_NO_XLONG | KD_FA_ROUTE_NO_XLONG64 | KD_FA_ROUTE_NO_W64 | KD_FA_ROUTE_W64_SHORT))
        return false;
    if (a.m || k_on_load || a.rope_mode != KD_FA_ROPE_NONE || a.qn_w) return false;
    if (a.Lk <= kdfa::kXresMaxKeys || !w64_tail_ok(a)) return false;
    if (a.q_type != KD_FA_TYPE_F32 && !(a.q_type == op && a.scale_log2 >= 0.0f)) return false;
    const int64_t lim = (int64_t)1 << 31;
    return (int64_t)(a.Lk - 1) * a.k_nb1 + 256 < lim && (int64_t)(a.Lk - 1) * a.v_nb1 + 256 < lim &&
           63 * a.q_nb1 + 512 < lim && 63 * a.o_nb2 + 512 < lim;
}

// The other unmasked key sets of up to 1,024 keys (Q in K's type with a
// negative scale, or scale 0 and a partial last tile) go to the persistent
// kernel on the 32-row step, fa_fwd_xlong, when K is read as stored, Q is
// neither rotated nor normalised and is stored as F32 or in K's type, and a
// unit's Q rows lie within 32-bit offsets of its first row.  KD_FA_ROUTE_NO_XLONG and
// KD_FA_ROUTE_NO_W64 route them to the 32-row kernel, KD_FA_ROUTE_W64_SHORT
// to the 64-row one (for comparisons).
static bool use_xlong(const kdfa::Args &a, int op, bool k_on_load, int route) {
    if (route & (KD_FA_ROUTE_NO_XLONG | KD_FA_ROUTE_NO_W64 | KD_FA_ROUTE_W64_SHORT)) return false;
    if (a.m || k_on_load || a.rope_mode != KD_FA_ROPE_NONE || a.qn_w) return false;
    if (a.Lk <= kdfa::kXresMaxKeys || a.Lk > kdfa::kXlongMaxKeys) return false;
    if (a.q_type != KD_FA_TYPE_F32 && a.q_type != op) return false;
    return (int64_t)(kdfa::kXlongRows - 1) * a.q_nb1 + 512 < ((int64_t)1 << 32);
}

// Query ranges per (b, h) for fa_fwd_xres: about one workgroup per CU
// (256 on MI355X) in all, at least four 32-row blocks (one per wave) each.
// (Two to four workgroups per CU, which would let the dispatcher balance
// batches whose masks leave different numbers of live key tiles, measured
// no faster: each workgroup first loads its K and V.)
static void xres_split(kdfa::Args &a) {
    const int64_t n_qb = ((int64_t)a.Lq + 31) / 32;
    const int64_t bh = (int64_t)a.H * a.B;
    int64_t ranges = (256 + bh - 1) / bh;
    ranges = std::min<int64_t>(ranges, (n_qb + 3) / 4);
    ranges = std::max<int64_t>(ranges, 1);
    const int64_t per = (n_qb + ranges - 1) / ranges;
    a.x_blocks = (int32_t)per;
    a.n_qt = (int32_t)((n_qb + per - 1) / per);
    a.n_blocks = (int32_t)(a.n_qt * bh);
}

// Staged calls: K transformed (normalised and / or rotated) without a
// workspace.  Rotating K on load costs every query tile of a head the whole
// rotation again; instead the (b, h) pairs are processed in groups, and each
// group's transformed K is written by the pre-pass into the output rows of
// the NEXT group -- rows that group's attention overwrites only later, in
// stream order -- so that the group runs on the 64-row kernel with K read as
// stored.  A transformed K row (256 bytes) takes half of an F32 output row,
// so a group may hold up to twice as many heads as the next (as many, for a
// 16-bit output); the sizes shrink geometrically towards the last group
// (one or two heads), which has no later rows to borrow and rotates K on
// load.  The transformed values are the pre-pass's, so the result is
// bitwise that of the workspace path.  Groups stay within one batch.
// Byte range [lo, hi) a tensor view spans (empty for a NULL or empty view).
struct Range {
    uintptr_t lo = 0, hi = 0;
};
Range view_range(const kd_fa_tensor &t) {
    Range r;
    if (!t.data) return r;
    uint64_t span = elem_size(t.type);
    for (int i = 0; i < 4; ++i) {
        if (t.ne[i] <= 0) return r;
        span += (uint64_t)(t.ne[i] - 1) * t.nb[i];
    }
    r.lo = reinterpret_cast<uintptr_t>(t.data);
    r.hi = r.lo + span;
    return r;
}
Range ptr_range(const void *p, size_t bytes) {
    Range r;
    if (p) {
        r.lo = reinterpret_cast<uintptr_t>(p);
        r.hi = r.lo + bytes;
    }
    return r;
}
bool overlaps(const Range &a, const Range &b) { return a.lo < b.hi && b.lo < a.hi; }

// Whether dst shares bytes with an operand of the call.  The header requires
// that it does not; the staged path, which writes transformed K into output
// rows ahead of the attention, is only taken when this is checked false.
bool dst_overlaps_operands(const kd_fa_desc *d, const kd_fa_rope *r, const kd_fa_qk_norm *n) {
    const Range o = view_range(d->dst);
    if (overlaps(o, view_range(d->q)) || overlaps(o, view_range(d->k)) || overlaps(o, view_range(d->v)) ||
        overlaps(o, view_range(d->mask)))
        return true;
    if (r && r->mode == KD_FA_ROPE_TABLE && overlaps(o, view_range(r->table))) return true;
    if (r && r->mode == KD_FA_ROPE_AXES) {
        const size_t floats = (size_t)r->grid[0] * r->axes[0] + (size_t)r->grid[1] * r->axes[1] +
                              (size_t)r->grid[2] * r->axes[2];
        if (overlaps(o, ptr_range(r->axes_data, floats * 4))) return true;
    }
    if (n && (overlaps(o, ptr_range(n->q_weight, kHeadDim * 4)) || overlaps(o, ptr_range(n->k_weight, kHeadDim * 4))))
        return true;
    return false;
}

bool staged_ok(const kdfa::Args &a, const kd_fa_desc *d, const kd_fa_rope *r, const kd_fa_qk_norm *n, int route) {
    if ((route & KD_FA_ROUTE_NO_W64) || a.m) return false;
    if (dst_overlaps_operands(d, r, n)) return false;
    if (a.rk2 != 1 || a.rk3 != 1 || a.rv2 != 1 || a.rv3 != 1) return false;
    if (a.Lk < 64 || a.Lq < a.Lk || !w64_tail_ok(a)) return false;
    const int64_t row = kHeadDim * (int64_t)elem_size(d->dst.type);
    if ((int64_t)d->dst.nb[1] != row) return false;   // the heads of an output row are contiguous
    if ((int64_t)a.H * a.B < 4) return false;
    const int64_t lim = (int64_t)1 << 31;            // the 64-row kernel's 32-bit buffer offsets
    return (int64_t)(a.Lk - 1) * (int64_t)d->dst.nb[2] + 256 < lim && (int64_t)(a.Lk - 1) * a.v_nb1 + 256 < lim;
}

// a's view restricted to heads [h0, h0 + n) of batch b (no broadcast)
kdfa::Args head_range(const kdfa::Args &a, int b, int h0, int n) {
    kdfa::Args s = a;
    s.q = a.q + (int64_t)b * a.q_nb3 + (int64_t)h0 * a.q_nb2;
    s.k = a.k + (int64_t)b * a.k_nb3 + (int64_t)h0 * a.k_nb2;
    s.v = a.v + (int64_t)b * a.v_nb3 + (int64_t)h0 * a.v_nb2;
    s.o = a.o + (int64_t)b * a.o_nb3 + (int64_t)h0 * a.o_nb1;
    s.H = n;
    s.B = 1;
    return s;
}

// Group sizes for run_staged, first to last (the last one rotates K on
// load), and their cost.  A launch fills the GPU in rounds of one workgroup
// per CU (256 on MI355X), one workgroup per 256 query rows and head, and its
// last round may be partial; the sizes minimise the rounds of all launches
// (plus a small cost per launch pair; the on-load kernel's rounds count 1.4
// times) under the constraints: each group at most `ratio` times the heads
// of the next (whose output rows hold its transformed K) and within one
// batch; the last group has 1 to 8 heads.  A dynamic program over (pairs
// left, size of the next group): a group never spans batches, so the next
// group's size is at most H, and the program takes O(P H^2) steps and
// O(P H) memory per last-group size for P (b, h) pairs.  Calls with more
// than kStagedMaxPairs pairs are not staged (an empty plan: K on load).
// The last few plans of the calling thread are remembered.  The cost is in
// the same units as onload_cost's, the one launch that rotates K on load
// for every pair.
constexpr double kStagedLaunch = 0.05, kStagedOnLoad = 1.4;
constexpr int kStagedMaxPairs = 4096;
double launch_rounds(int heads, int wg_head) { return (double)(((int64_t)heads * wg_head + 255) / 256); }
double onload_cost(int P, int wg_head) { return kStagedOnLoad * launch_rounds(P, wg_head); }
struct StagedPlan {
    std::vector<int> sizes;
    double cost = 1e300;
};
StagedPlan staged_groups(int P, int H, int wg_head, int ratio) {
    struct Memo {
        int P = -1, H = -1, wg = -1, ratio = -1;
        StagedPlan plan;
    };
    constexpr int kMemo = 4;
    thread_local Memo memo[kMemo];
    thread_local int memo_next = 0;
    for (const Memo &m : memo)
        if (m.P == P && m.H == H && m.wg == wg_head && m.ratio == ratio) return m.plan;
    StagedPlan plan;
    if (P <= kStagedMaxPairs && H >= 1) {
        auto rounds = [wg_head](int h) { return launch_rounds(h, wg_head); };
        constexpr double kLaunch = kStagedLaunch, kOnLoad = kStagedOnLoad;
        const size_t W = (size_t)H + 1;   // next-group sizes 1..H
        std::vector<double> dp((size_t)(P + 1) * W);
        std::vector<int> pick((size_t)(P + 1) * W);
        for (int n_last = 1; n_last <= 8; ++n_last) {
            if (n_last > H || n_last >= P) continue;
            const int E = P - n_last;
            for (int s = 1; s <= H; ++s) dp[s] = 0.0;   // e = 0
            for (int e = 1; e <= E; ++e) {
                const int avail = e - ((e - 1) / H) * H;   // pairs of its batch before e
                for (int s = 1; s <= H; ++s) {
                    double b = 1e300;
                    int bh = 0;
                    const int top = std::min(ratio * s, avail);
                    for (int h = 1; h <= top; ++h) {
                        const double c = rounds(h) + kLaunch + dp[(size_t)(e - h) * W + h];
                        if (c < b - 1e-12 || (c < b + 1e-12 && h > bh)) { b = c; bh = h; }
                    }
                    dp[(size_t)e * W + s] = b;
                    pick[(size_t)e * W + s] = bh;
                }
            }
            const double cost = dp[(size_t)E * W + n_last] + kOnLoad * rounds(n_last);
            if (cost < plan.cost) {
                plan.cost = cost;
                plan.sizes.clear();
                for (int e = E, s = n_last; e > 0;) {
                    const int h = pick[(size_t)e * W + s];
                    plan.sizes.push_back(h);
                    e -= h;
                    s = h;
                }
                std::reverse(plan.sizes.begin(), plan.sizes.end());
                plan.sizes.push_back(n_last);
            }
        }
    }
    memo[memo_next] = {P, H, wg_head, ratio, plan};
    memo_next = (memo_next + 1) % kMemo;
    return plan;
}

// The staged plan of a call that staged_ok allows.
StagedPlan staged_plan(const kdfa::Args &a) {
    const int ratio = a.o_type == KD_FA_TYPE_F32 ? 2 : 1;   // transformed K rows per output row
    return staged_groups(a.H * a.B, a.H, (a.Lq + 255) / 256, ratio);
}

// Staging pays when its launches take fewer rounds than one launch that
// rotates K on load for every pair.  When the whole call fits one round
// (the 1,280-token self-attention: 160 workgroups), each staged launch still
// takes a whole workgroup lifetime: its five launches took 144 us there, one
// on-load launch for all 32 heads 55 us.  KD_FA_ROUTE_STAGED stages whenever the shape
// allows (for comparisons).
bool staged_pays(const kdfa::Args &a, const StagedPlan &plan, int route) {
    if (plan.sizes.empty()) return false;
    return (route & KD_FA_ROUTE_STAGED) || plan.cost < onload_cost(a.H * a.B, (a.Lq + 255) / 256);
}

int run_staged(const kdfa::Args &a, const std::vector<int> &sizes, int kv_type, hipStream_t hs) {
    const int H = a.H;
    std::vector<int> start(1, 0);
    for (int n : sizes) start.push_back(start.back() + n);
    const int n_last = sizes.back();
    const int n_groups = (int)start.size() - 1;   // the last one rotates K on load
    const int64_t krow = kHeadDim * (int64_t)elem_size(kv_type);
    for (int g = 0; g + 1 < n_groups; ++g) {
        const int p0 = start[g], n = start[g + 1] - p0;
        const int p1 = start[g + 1];   // the next group: its output rows hold this group's K
        kdfa::Args s = head_range(a, p0 / H, p0 % H, n);
        char *kst = a.o + (int64_t)(p1 / H) * a.o_nb3 + (int64_t)(p1 % H) * a.o_nb1;
        const kdfa::KStrides st = {a.o_nb2, krow, 0};
        if (kdfa::launch_rope_k(s, kv_type, n, 1, kst, st, hs) != hipSuccess) return KD_FA_ERR_LAUNCH;
        s.k = kst;
        s.k_nb1 = a.o_nb2;
        s.k_nb2 = krow;
        s.k_nb3 = 0;
        s.n_qt = (a.Lq + kdfa::kW64Rows - 1) / kdfa::kW64Rows;
        s.n_blocks = s.n_qt * n;
        if (kdfa::launch_w64(s, kv_type, hs) != hipSuccess) return KD_FA_ERR_LAUNCH;
    }
    const int p0 = start[n_groups - 1];
    kdfa::Args s = head_range(a, p0 / H, p0 % H, n_last);
    const int waves = kdfa::d128_waves(false, true, a.Lk);
    s.n_qt = (a.Lq + 32 * waves - 1) / (32 * waves);
    s.n_blocks = s.n_qt * n_last;
    return kdfa::launch(s, kv_type, true, waves, hs) == hipSuccess ? KD_FA_OK : KD_FA_ERR_LAUNCH;
}

// kv_f32: the entry point accepts an F32 K and V (the workspace forms).
int run(const kd_fa_desc *d, const kd_fa_rope *r, const kd_fa_qk_norm *n, void *ws, size_t ws_bytes,
        void *stream, bool kv_f32) {
    bool mask_vec = false;
    int st = validate(d, r, n, &mask_vec, kv_f32);
    if (st != KD_FA_OK) return st;
    const bool v32 = d->v.type == KD_FA_TYPE_F32;
    const WsLayout wl = ws_layout(d, r, n);
    const bool k_xform = wl.k_ws;   // normalised, rotated or cast from F32
    // an F32 K or V is cast to the operand type by the workspace pre-pass only
    if (!ws && (d->k.type == KD_FA_TYPE_F32 || v32)) return KD_FA_ERR_NULL;
    if (ws && !is_16b(ws)) return KD_FA_ERR_LAYOUT;
    if (ws && wl.cast && ws_bytes < wl.cast) return KD_FA_ERR_LAYOUT;
    const int T = op_type(d);   // the MFMA operand type
    const int route = g_route.load(std::memory_order_relaxed);
    const int64_t Lq = d->q.ne[1], H = d->q.ne[2], B = d->q.ne[3];
    if (Lq == 0 || H == 0 || B == 0) return KD_FA_OK;
    st = device_ok();
    if (st != KD_FA_OK) return st;

    kdfa::Args a;
    std::memset(&a, 0, sizeof(a));
    a.q = static_cast<const char *>(d->q.data);
    a.k = static_cast<const char *>(d->k.data);
    a.v = static_cast<const char *>(d->v.data);
    a.m = static_cast<const char *>(d->mask.data);
    a.o = static_cast<char *>(d->dst.data);
    a.q_nb1 = d->q.nb[1]; a.q_nb2 = d->q.nb[2]; a.q_nb3 = d->q.nb[3];
    a.k_nb1 = d->k.nb[1]; a.k_nb2 = d->k.nb[2]; a.k_nb3 = d->k.nb[3];
    a.v_nb1 = d->v.nb[1]; a.v_nb2 = d->v.nb[2]; a.v_nb3 = d->v.nb[3];
    if (a.m) {
        a.m_nb1 = d->mask.nb[1]; a.m_nb2 = d->mask.nb[2]; a.m_nb3 = d->mask.nb[3];
        a.m_ne2 = (int32_t)d->mask.ne[2]; a.m_ne3 = (int32_t)d->mask.ne[3];
    }
    a.o_nb1 = d->dst.nb[1]; a.o_nb2 = d->dst.nb[2]; a.o_nb3 = d->dst.nb[3];
    a.o_type = d->dst.type;
    if (n) {
        a.qn_w = n->q_weight;
        a.kn_w = n->k_weight;
        a.norm_eps = n->eps;
    }
    a.Lq = (int32_t)Lq;
    a.Lk = (int32_t)d->k.ne[1];
    a.H = (int32_t)H;
    a.B = (int32_t)B;
    a.rk2 = (int32_t)(H / d->k.ne[2]); a.rk3 = (int32_t)(B / d->k.ne[3]);
    a.rv2 = (int32_t)(H / d->v.ne[2]); a.rv3 = (int32_t)(B / d->v.ne[3]);
    a.q_type = d->q.type;
    a.k_type = d->k.type;
    a.mask_vec = mask_vec ? 1 : 0;
    a.scale_log2 = d->scale * 1.4426950408889634f;
    a.rope_mode = r ? r->mode : KD_FA_ROPE_NONE;
    if (a.rope_mode == KD_FA_ROPE_TABLE) {
        a.rope_tab = static_cast<const float *>(r->table.data);
        a.rope_nb1 = (int64_t)r->table.nb[1];
    } else if (a.rope_mode == KD_FA_ROPE_AXES) {
        a.axes = r->axes_data;
        a.grid_t = r->grid[0]; a.grid_h = r->grid[1]; a.grid_w = r->grid[2];
        a.axis0 = r->axes[0]; a.axis1 = r->axes[1]; a.axis2 = r->axes[2];
        a.rcp_h = 1.0f / (float)r->grid[1];
        a.rcp_w = 1.0f / (float)r->grid[2];
    }
    hipStream_t hs = static_cast<hipStream_t>(stream);
    if (d->q.ne[0] == kHeadDimVae) {
        // 64 query rows per workgroup (half the key stream per row) when that
        // still gives every CU a workgroup, else 32; KD_FA_ROUTE_D512_R1
        // forces 32 (for comparisons)
        const int rows = ((route & KD_FA_ROUTE_D512_R1) || (Lq + 63) / 64 * H * B < 256) ? 32 : 64;
        a.n_qt = (int32_t)((Lq + rows - 1) / rows);
        a.n_blocks = (int32_t)(a.n_qt * H * B);
        // with a workspace, the key split of short query sets (the partial
        // results, then the merge into dst)
        const D512Split sp = rows == 32 ? d512_split(Lq, a.Lk, H, B, route) : D512Split{};
        if (sp.S > 1 && ws && ws_bytes >= sp.bytes) {
            a.part = static_cast<float *>(ws);
            a.n_split = sp.S;
            a.split_keys = sp.keys;
            if (kdfa::launch_d512(a, T, rows, hs) != hipSuccess) return KD_FA_ERR_LAUNCH;
            return kdfa::launch_d512_combine(a, hs) == hipSuccess ? KD_FA_OK : KD_FA_ERR_LAUNCH;
        }
        return kdfa::launch_d512(a, T, rows, hs) == hipSuccess ? KD_FA_OK : KD_FA_ERR_LAUNCH;
    }
    bool k_rope = k_xform && !ws;
    if (k_rope && staged_ok(a, d, r, n, route)) {
        const StagedPlan plan = staged_plan(a);
        if (staged_pays(a, plan, route)) return run_staged(a, plan.sizes, T, hs);
    }
    // a mask row block shared by every head is read once per q-tile when the
    // heads of a q-tile run back to back (K and V of all heads then share the
    // L2 instead, which the short text keys of the cross-attention allow)
    a.heads_inner = (a.m && d->mask.ne[2] == 1 && H > 1 && d->k.ne[1] <= 1024) ? 1 : 0;

    if (ws && (k_xform || v32)) {
        // the pre-pass: K normalised / rotated / cast and an F32 V cast, in
        // one launch when K and V have the same heads and batches
        char *const wsc = static_cast<char *>(ws);
        const int hk = (int)d->k.ne[2], bk = (int)d->k.ne[3];
        const int hv = (int)d->v.ne[2], bv = (int)d->v.ne[3];
        const int64_t row = kHeadDim * 2;
        const kdfa::KStrides kst = {row, row * a.Lk, row * a.Lk * hk};
        const kdfa::KStrides vst = {row, row * a.Lk, row * a.Lk * hv};
        char *const kout = k_xform ? wsc : nullptr;
        char *const vout = v32 ? wsc + wl.v_off : nullptr;
        hipError_t e = hipSuccess;
        if (kout && vout && (hk != hv || bk != bv)) {
            e = kdfa::launch_rope_k(a, T, hk, bk, kout, kst, nullptr, vst, hs);
            if (e == hipSuccess) e = kdfa::launch_rope_k(a, T, hv, bv, nullptr, kst, vout, vst, hs);
        } else {
            e = kout ? kdfa::launch_rope_k(a, T, hk, bk, kout, kst, vout, vst, hs)
                     : kdfa::launch_rope_k(a, T, hv, bv, nullptr, kst, vout, vst, hs);
        }
        if (e != hipSuccess) return KD_FA_ERR_LAUNCH;
        if (kout) {
            a.k = kout;
            a.k_nb1 = row;
            a.k_nb2 = row * a.Lk;
            a.k_nb3 = row * a.Lk * hk;
        }
        if (vout) {
            a.v = vout;
            a.v_nb1 = row;
            a.v_nb2 = row * a.Lk;
            a.v_nb3 = row * a.Lk * hv;
        }
    }
    hipError_t e;
    if (use_xres(a, T, d, k_rope, route)) {
        xres_split(a);
        // with room in the workspace, the mask summary: tiles that are -inf
        // for all rows of a block are then skipped without loading their
        // mask chunks (one L2 round trip per dead tile and block)
        if (a.m && ws && wl.s_bytes && ws_bytes >= wl.s_off + wl.s_bytes && summary_pays(Lq * H * B, route)) {
            uint32_t *sum = reinterpret_cast<uint32_t *>(static_cast<char *>(ws) + wl.s_off);
            if (kdfa::launch_mask_live(a, sum, hs) != hipSuccess) return KD_FA_ERR_LAUNCH;
            a.m_live = sum;
            a.m_live_nqb = (int32_t)((Lq + 31) / 32);
        }
        e = kdfa::launch_xres(a, T, hs);
    } else if (use_xlong64(a, T, k_rope, route)) {
        a.n_qt = (int32_t)((Lq + kdfa::kXlongRows - 1) / kdfa::kXlongRows);
        a.n_blocks = (int32_t)(a.n_qt * H * B);
        e = kdfa::launch_xlong64(a, T, hs);
    } else if (use_xlong(a, T, k_rope, route)) {
        a.n_qt = (int32_t)((Lq + kdfa::kXlongRows - 1) / kdfa::kXlongRows);
        a.n_blocks = (int32_t)(a.n_qt * H * B);
        e = kdfa::launch_xlong(a, T, hs);
    } else if (use_w64(a, k_rope, route)) {
        a.n_qt = (int32_t)((Lq + kdfa::kW64Rows - 1) / kdfa::kW64Rows);
        a.n_blocks = (int32_t)(a.n_qt * H * B);
        e = kdfa::launch_w64(a, T, hs);
    } else {
        const int waves = kdfa::d128_waves(a.m != nullptr, k_rope, a.Lk);
        a.n_qt = (int32_t)((Lq + 32 * waves - 1) / (32 * waves));
        a.n_blocks = (int32_t)(a.n_qt * H * B);
        e = kdfa::launch(a, T, k_rope, waves, hs);
    }
    if (e != hipSuccess) return KD_FA_ERR_LAUNCH;
    return KD_FA_OK;
}

// rope::get_freqs (src/rope.hpp:23-29), same float expression order.
void rope_freqs(int dim, float max_period, float *out) {
    for (int i = 0; i < dim; i++) out[i] = expf(-logf(max_period) * (float)i / (float)dim);
}

bool axes_ok(int T, int Hp, int Wp, const int axes[3]) {
    if (!axes || T <= 0 || Hp <= 0 || Wp <= 0) return false;
    for (int i = 0; i < 3; ++i)
        if (axes[i] < 0 || axes[i] % 2) return false;
    return true;
}

}  // namespace

namespace kdfa {
int device_gfx950() { return device_ok(); }

int run_node(const kd_fa_desc *d, const kd_fa_rope *r, const kd_fa_qk_norm *n, void *ws, size_t ws_bytes,
             void *stream) {
    return run(d, r, n, ws, ws_bytes, stream, true);
}

size_t cast_workspace_need(const kd_fa_desc *d, const kd_fa_rope *r, const kd_fa_qk_norm *n, int *status,
                           bool *f32_kv) {
    *status = validate(d, r, n, nullptr, true);
    *f32_kv = false;
    if (*status != KD_FA_OK || d->q.ne[0] != kHeadDim) return 0;
    *f32_kv = d->k.type == KD_FA_TYPE_F32 || d->v.type == KD_FA_TYPE_F32;
    return ws_layout(d, r, n).cast;
}

size_t workspace_need(const kd_fa_desc *d, const kd_fa_rope *r, const kd_fa_qk_norm *n, int *status) {
    *status = validate(d, r, n, nullptr, true);
    if (*status != KD_FA_OK) return 0;
    if (d->q.ne[0] == kHeadDimVae) return d512_split(d->q.ne[1], d->k.ne[1], d->q.ne[2], d->q.ne[3], 0).bytes;
    return ws_layout(d, r, n).total;
}
}  // namespace kdfa

extern "C" {

int kd_fa_supports(const kd_fa_desc *desc, int *reason) {
    const int st = validate(desc, nullptr, nullptr, nullptr);
    if (reason) *reason = st;
    return st == KD_FA_OK ? 1 : 0;
}

int kd_fa_rope_supports(const kd_fa_desc *desc, const kd_fa_rope *rope, int *reason) {
    const int st = validate(desc, rope, nullptr, nullptr);
    if (reason) *reason = st;
    return st == KD_FA_OK ? 1 : 0;
}

int kd_fa_run(const kd_fa_desc *desc, void *stream) {
    return run(desc, nullptr, nullptr, nullptr, 0, stream, false);
}

int kd_fa_run_ws(const kd_fa_desc *desc, void *workspace, size_t workspace_bytes, void *stream) {
    return run(desc, nullptr, nullptr, workspace, workspace_bytes, stream, false);
}

size_t kd_fa_workspace_size(const kd_fa_desc *desc, const kd_fa_rope *rope, const kd_fa_qk_norm *norm) {
    if (!desc) return 0;
    int st = KD_FA_OK;
    const size_t need = kdfa::workspace_need(desc, rope, norm, &st);
    return st == KD_FA_OK ? need : 0;
}

int kd_fa_rope_run(const kd_fa_desc *desc, const kd_fa_rope *rope, void *stream) {
    return run(desc, rope, nullptr, nullptr, 0, stream, false);
}

int kd_fa_dit_supports(const kd_fa_desc *desc, const kd_fa_rope *rope, const kd_fa_qk_norm *norm,
                       int *reason) {
    // the workspace form: an F32 K and V are cast by its pre-pass
    const int st = validate(desc, rope, norm, nullptr, true);
    if (reason) *reason = st;
    return st == KD_FA_OK ? 1 : 0;
}

int kd_fa_dit_run(const kd_fa_desc *desc, const kd_fa_rope *rope, const kd_fa_qk_norm *norm,
                  void *workspace, size_t workspace_bytes, void *stream) {
    return run(desc, rope, norm, workspace, workspace_bytes, stream, true);
}

size_t kd_fa_rope_workspace_size(const kd_fa_desc *desc) {
    if (!desc || validate(desc, nullptr, nullptr, nullptr, true) != KD_FA_OK || desc->q.ne[0] != kHeadDim) return 0;
    return ws_layout(desc, nullptr, nullptr, true).cast;
}

int kd_fa_rope_run_ws(const kd_fa_desc *desc, const kd_fa_rope *rope, void *workspace,
                      size_t workspace_bytes, void *stream) {
    if (!workspace && rope && rope->mode != KD_FA_ROPE_NONE && desc && desc->k.ne[1] > 0)
        return KD_FA_ERR_NULL;
    return run(desc, rope, nullptr, workspace, workspace_bytes, stream, true);
}

// rope::compute_visual_rope (src/rope.hpp:56-102).
int kd_fa_rope_visual_table(int T, int Hp, int Wp, const int axes[3], const float sf[3],
                            float theta, float *out) {
    if (!axes_ok(T, Hp, Wp, axes) || !sf || !out) return KD_FA_ERR_ROPE;
    const int D = axes[0] + axes[1] + axes[2];
    std::vector<float> f[3];
    for (int a = 0; a < 3; ++a) {
        f[a].resize(axes[a] / 2 + 1);
        rope_freqs(axes[a] / 2, theta, f[a].data());
    }
    for (int t = 0; t < T; t++)
        for (int h = 0; h < Hp; h++)
            for (int w = 0; w < Wp; w++) {
                float *row = out + (size_t)((t * Hp + h) * Wp + w) * D;
                const int pos[3] = {t, h, w};
                int off = 0;
                for (int a = 0; a < 3; ++a) {
                    for (int i = 0; i < axes[a] / 2; i++) {
                        const float angle = (float)pos[a] * f[a][i] / sf[a];
                        row[off + 2 * i] = cosf(angle);
                        row[off + 2 * i + 1] = sinf(angle);
                    }
                    off += axes[a];
                }
            }
    return KD_FA_OK;
}

size_t kd_fa_rope_axes_size(int T, int Hp, int Wp, const int axes[3]) {
    if (!axes_ok(T, Hp, Wp, axes)) return 0;
    return (size_t)T * axes[0] + (size_t)Hp * axes[1] + (size_t)Wp * axes[2];
}

// The per-axis factors of compute_visual_rope: the t block of row
// (t, h, w) equals axes-table row t of axis 0, and likewise for h and w.
int kd_fa_rope_axes_fill(int T, int Hp, int Wp, const int axes[3], const float sf[3],
                         float theta, float *out) {
    if (!axes_ok(T, Hp, Wp, axes) || !sf || !out) return KD_FA_ERR_ROPE;
    const int n[3] = {T, Hp, Wp};
    float *dst = out;
    for (int a = 0; a < 3; ++a) {
        std::vector<float> f(axes[a] / 2 + 1);
        rope_freqs(axes[a] / 2, theta, f.data());
        for (int p = 0; p < n[a]; ++p) {
            for (int i = 0; i < axes[a] / 2; ++i) {
                const float angle = (float)p * f[i] / sf[a];
                dst[2 * i] = cosf(angle);
                dst[2 * i + 1] = sinf(angle);
            }
            dst += axes[a];
        }
    }
    return KD_FA_OK;
}

// rope::compute_text_rope (src/rope.hpp:36-49).
int kd_fa_rope_text_table(int L, int D, float theta, float *out) {
    if (L < 0 || D <= 0 || D % 2 || !out) return KD_FA_ERR_ROPE;
    std::vector<float> f(D / 2 + 1);
    rope_freqs(D / 2, theta, f.data());
    for (int pos = 0; pos < L; pos++)
        for (int i = 0; i < D / 2; i++) {
            const float angle = (float)pos * f[i];
            out[(size_t)pos * D + 2 * i] = cosf(angle);
            out[(size_t)pos * D + 2 * i + 1] = sinf(angle);
        }
    return KD_FA_OK;
}

const char *kd_fa_strerror(int status) {
    switch (status) {
    case KD_FA_OK: return "ok";
    case KD_FA_ERR_NULL: return "null descriptor or data pointer";
    case KD_FA_ERR_TYPE: return "unsupported tensor type";
    case KD_FA_ERR_SHAPE: return "tensor shapes inconsistent with GGML_OP_FLASH_ATTN_EXT";
    case KD_FA_ERR_LAYOUT: return "unsupported stride or alignment";
    case KD_FA_ERR_PARAM: return "unsupported op parameter (max_bias, logit_softcap, sinks, scale)";
    case KD_FA_ERR_ROPE: return "invalid RoPE descriptor";
    case KD_FA_ERR_LAUNCH: return "HIP kernel launch failed";
    case KD_FA_ERR_DEVICE: return "current device is not a gfx950 GPU";
    case KD_FA_ERR_SCRATCH: return "transformed K larger than the library's static scratch (KD_FA_STATIC_SCRATCH_BYTES)";
    default: return "unknown status";
    }
}

int kd_fa_version(void) { return 302; }

int kd_fa_abi_version(void) { return KD_FA_ABI_VERSION; }

int kd_fa_set_routing(int flags) { return g_route.exchange(flags); }

}  // extern "C"
