// kd_mm_host.cpp - C ABI of the linear-layer product (include/kd_mm.h):
// validation of the GGML_OP_MUL_MAT node as ops::linear builds it
// (src/core/ops.hpp:27-43), the weight expansion and the product launch.
// Nothing here allocates device memory, synchronises or keeps pointers past
// the call.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/kd_mm.h"
#include "kd_fa_kernel.h"
#include "kd_mm_kernel.h"

namespace {

constexpr int64_t kI32Max = 0x7fffffff;
constexpr uint64_t kU32Max = 0xffffffffull;

bool is_16b(uint64_t x) { return (x & 15u) == 0; }
bool is_16b(const void *p) { return is_16b(reinterpret_cast<uintptr_t>(p)); }

// bytes of one 32-element block of a weight row
int64_t block_bytes(int type) {
    switch (type) {
    case KD_MM_TYPE_Q8_0: return 34;
    case KD_MM_TYPE_Q4_0: return 18;
    case KD_MM_TYPE_F16:
    case KD_MM_TYPE_BF16: return 64;
    case KD_MM_TYPE_F32: return 128;
    default: return 0;
    }
}

// Weight tensor [K, N]: a known type, K a multiple of 32, rows of at least
// K/32 blocks; quantized rows 2-byte aligned, float rows 16-byte aligned.
int check_w(const kd_fa_tensor &w) {
    if (!w.data) return KD_FA_ERR_NULL;
    const int64_t bb = block_bytes(w.type);
    if (bb == 0) return KD_FA_ERR_TYPE;
    const int64_t K = w.ne[0], N = w.ne[1];
    if (K <= 0 || N < 0 || w.ne[2] != 1 || w.ne[3] != 1) return KD_FA_ERR_SHAPE;
    if (K % 32 != 0 || K > kI32Max || N > kI32Max) return KD_FA_ERR_SHAPE;
    const bool quant = w.type == KD_MM_TYPE_Q8_0 || w.type == KD_MM_TYPE_Q4_0;
    const uint64_t row = (uint64_t)(K / 32) * (uint64_t)bb;
    if (quant) {
        if (w.nb[0] != (size_t)bb) return KD_FA_ERR_LAYOUT;
        if ((w.nb[1] & 1u) || (reinterpret_cast<uintptr_t>(w.data) & 1u)) return KD_FA_ERR_LAYOUT;
    } else {
        if (w.nb[0] != (size_t)(bb / 32)) return KD_FA_ERR_LAYOUT;
        if (!is_16b(w.nb[1]) || !is_16b(w.data)) return KD_FA_ERR_LAYOUT;
    }
    if (w.nb[1] < row) return KD_FA_ERR_LAYOUT;
    return KD_FA_OK;
}

// rows of a [ne0, ne1, ne2, ne3] view flattened as ops::linear's reshape
// (contiguous beyond the rows); 0 on a layout it cannot flatten
int64_t flat_rows(const kd_fa_tensor &t) {
    if (t.ne[1] < 0 || t.ne[2] < 1 || t.ne[3] < 1) return -1;
    if (t.ne[2] > 1 && t.nb[2] != t.nb[1] * (size_t)t.ne[1]) return -1;
    if (t.ne[3] > 1 && t.nb[3] != t.nb[2] * (size_t)t.ne[2]) return -1;
    return t.ne[1] * t.ne[2] * t.ne[3];
}

int validate(const kd_mm_desc *d) {
    if (!d) return KD_FA_ERR_NULL;
    int st = check_w(d->w);
    if (st != KD_FA_OK) return st;
    const kd_fa_tensor &x = d->x, &o = d->dst, &b = d->bias;
    if (!x.data || !o.data) return KD_FA_ERR_NULL;
    if (x.type != KD_MM_TYPE_F32 && x.type != KD_MM_TYPE_BF16) return KD_FA_ERR_TYPE;
    if (o.type != KD_MM_TYPE_F32) return KD_FA_ERR_TYPE;
    if (b.data && b.type != KD_MM_TYPE_F32) return KD_FA_ERR_TYPE;
    const int64_t K = d->w.ne[0], N = d->w.ne[1];
    if (x.ne[0] != K || o.ne[0] != N) return KD_FA_ERR_SHAPE;
    const int64_t M = flat_rows(x);
    if (M < 0 || flat_rows(o) != M) return KD_FA_ERR_LAYOUT;
    if (o.ne[1] != x.ne[1] || o.ne[2] != x.ne[2] || o.ne[3] != x.ne[3]) return KD_FA_ERR_SHAPE;
    if (M > kI32Max) return KD_FA_ERR_SHAPE;
    if (N % 4 != 0) return KD_FA_ERR_SHAPE;
    if (b.data && (b.ne[0] != N || b.ne[1] != 1 || b.ne[2] != 1 || b.ne[3] != 1)) return KD_FA_ERR_SHAPE;
    // rows 16-byte aligned, elements contiguous
    const size_t xe = x.type == KD_MM_TYPE_F32 ? 4 : 2;
    if (x.nb[0] != xe || o.nb[0] != 4) return KD_FA_ERR_LAYOUT;
    if (!is_16b(x.data) || !is_16b(x.nb[1]) || !is_16b(o.data) || !is_16b(o.nb[1])) return KD_FA_ERR_LAYOUT;
    if (b.data && (!is_16b(b.data) || b.nb[0] != 4)) return KD_FA_ERR_LAYOUT;
    // a 256-row tile is addressed with 32-bit offsets from its first row
    if ((uint64_t)x.nb[1] * kdfa::kMmBM > kU32Max) return KD_FA_ERR_LAYOUT;
    if ((uint64_t)K * 2 * kdfa::kMmBN > kU32Max) return KD_FA_ERR_LAYOUT;
    if (d->w.type == KD_MM_TYPE_BF16 && (uint64_t)d->w.nb[1] * kdfa::kMmBN > kU32Max) return KD_FA_ERR_LAYOUT;
    return KD_FA_OK;
}

// w BF16 with 16-byte aligned rows is multiplied as stored
bool w_direct(const kd_fa_tensor &w) {
    return w.type == KD_MM_TYPE_BF16 && is_16b(w.data) && is_16b(w.nb[1]);
}

size_t ws_bytes(const kd_mm_desc *d) {
    return w_direct(d->w) ? 0 : (size_t)d->w.ne[0] * (size_t)d->w.ne[1] * 2;
}

hipError_t dequant(const kd_fa_tensor &w, void *out, hipStream_t s) {
    kdfa::DqArgs a;
    a.w = static_cast<const char *>(w.data);
    a.w_nb1 = (int64_t)w.nb[1];
    a.type = w.type;
    a.K = (int32_t)w.ne[0];
    a.N = (int32_t)w.ne[1];
    a.out = static_cast<char *>(out);
    a.out_nb1 = w.ne[0] * 2;
    return kdfa::launch_dequant(a, s);
}

}  // namespace

extern "C" {

int kd_mm_supports(const kd_mm_desc *desc, int *reason) {
    const int st = validate(desc);
    if (reason) *reason = st;
    return st == KD_FA_OK ? 1 : 0;
}

size_t kd_mm_workspace_size(const kd_mm_desc *desc) {
    if (validate(desc) != KD_FA_OK) return 0;
    return ws_bytes(desc);
}

int kd_mm_dequant(const kd_fa_tensor *w, void *out, size_t out_bytes, void *stream) {
    if (!w || !out) return KD_FA_ERR_NULL;
    const int st = check_w(*w);
    if (st != KD_FA_OK) return st;
    if (!is_16b(out) || out_bytes < (size_t)w->ne[0] * (size_t)w->ne[1] * 2) return KD_FA_ERR_LAYOUT;
    if (w->ne[1] == 0) return KD_FA_OK;
    const int dv = kdfa::device_gfx950();
    if (dv != KD_FA_OK) return dv;
    return dequant(*w, out, static_cast<hipStream_t>(stream)) == hipSuccess ? KD_FA_OK : KD_FA_ERR_LAUNCH;
}

int kd_mm_run(const kd_mm_desc *desc, void *workspace, size_t workspace_bytes, void *stream) {
    int st = validate(desc);
    if (st != KD_FA_OK) return st;
    const size_t need = ws_bytes(desc);
    if (need) {
        if (!workspace) return KD_FA_ERR_NULL;
        if (!is_16b(workspace) || workspace_bytes < need) return KD_FA_ERR_LAYOUT;
    }
    const int64_t K = desc->w.ne[0], N = desc->w.ne[1], M = flat_rows(desc->x);
    if (M == 0 || N == 0) return KD_FA_OK;
    st = kdfa::device_gfx950();
    if (st != KD_FA_OK) return st;
    hipStream_t hs = static_cast<hipStream_t>(stream);

    kdfa::MmArgs a;
    if (need) {
        if (dequant(desc->w, workspace, hs) != hipSuccess) return KD_FA_ERR_LAUNCH;
        a.w = static_cast<const char *>(workspace);
        a.w_nb1 = K * 2;
    } else {
        a.w = static_cast<const char *>(desc->w.data);
        a.w_nb1 = (int64_t)desc->w.nb[1];
    }
    a.x = static_cast<const char *>(desc->x.data);
    a.x_nb1 = (int64_t)desc->x.nb[1];
    a.bias = static_cast<const float *>(desc->bias.data);
    a.dst = static_cast<char *>(desc->dst.data);
    a.d_nb1 = (int64_t)desc->dst.nb[1];
    a.M = (int32_t)M;
    a.N = (int32_t)N;
    a.K = (int32_t)K;
    a.tiles_m = (int32_t)((M + kdfa::kMmBM - 1) / kdfa::kMmBM);
    a.tiles_n = (int32_t)((N + kdfa::kMmBN - 1) / kdfa::kMmBN);
    if ((int64_t)a.tiles_m * a.tiles_n > kI32Max) return KD_FA_ERR_SHAPE;
    a.n_blocks = a.tiles_m * a.tiles_n;
    return kdfa::launch_mm(a, desc->x.type == KD_MM_TYPE_F32, hs) == hipSuccess ? KD_FA_OK : KD_FA_ERR_LAUNCH;
}

}  // extern "C"
