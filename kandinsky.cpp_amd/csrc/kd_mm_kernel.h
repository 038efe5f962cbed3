// kd_mm_kernel.h - launch arguments shared by the host glue (kd_mm_host.cpp)
// and the gfx950 matrix-product kernels (kd_mm_kernel.hip).  Internal to
// libkd_fa.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kdfa {

// Workgroup tile of the product: 256 rows of x (tokens) by 256 rows of w
// (outputs), 32 k per stage.
constexpr int kMmBM = 256;
constexpr int kMmBN = 256;
constexpr int kMmBK = 32;

struct MmArgs {
    const char *w;       // BF16 rows [N][K], row stride w_nb1 bytes
    const char *x;       // F32 or BF16 rows [M][K], row stride x_nb1 bytes
    const float *bias;   // F32 [N] or nullptr
    char *dst;           // F32 rows [M][N], row stride d_nb1 bytes
    int64_t w_nb1, x_nb1, d_nb1;
    int32_t M, N, K;
    int32_t tiles_m, tiles_n, n_blocks;
};

// Enqueue the product (x F32 when x_f32, else BF16).
hipError_t launch_mm(const MmArgs &a, bool x_f32, hipStream_t stream);

struct DqArgs {
    const char *w;       // weight rows [N], row stride w_nb1 bytes
    int64_t w_nb1;
    int32_t type;        // KD_MM_TYPE_*
    int32_t N, K;
    char *out;           // BF16 rows [N][K], row stride out_nb1 bytes
    int64_t out_nb1;
};

// Enqueue the expansion of a weight to BF16 rows.
hipError_t launch_dequant(const DqArgs &a, hipStream_t stream);

}  // namespace kdfa
