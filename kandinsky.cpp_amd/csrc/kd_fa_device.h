// kd_fa_device.h - device helpers shared by the gfx950 attention kernels:
// element-type traits (MFMA, F32 <-> storage conversions), operand loads,
// the RoPE rotation (src/rope.hpp:109-155), the LDS swizzles, the DMA
// instruction and the lane-pair reductions.  Internal to libkd_fa.so.
//
// Operand layouts of v_mfma_f32_32x32x16 (wave64):
//   A (32 x 16): lane l holds row l%32, k = (l/32)*8 .. +7
//   B (16 x 32): lane l holds column l%32, k = (l/32)*8 .. +7
//   C (32 x 32): lane l, element i holds row 8*(i/4) + 4*(l/32) + i%4,
//                column l%32
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kd_fa_kernel.h"

namespace kdfa {

// a compile-time flag passed to generic lambdas (BC<true>(), BC<false>())
template <bool B> struct BC { static constexpr bool value = B; };
// a compile-time integer passed the same way
template <int I> struct IC { static constexpr int value = I; };

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

#define LDS_PTR(T, p) ((__attribute__((address_space(3))) T *)(p))
// LDS addresses are handled as 32-bit address-space-3 pointers throughout
// (generic pointers would cost two registers each)
typedef __attribute__((address_space(3))) char lds_t;

constexpr int kD = 128;          // head dim (Dk = Dv)
constexpr float kLog2e = 1.4426950408889634f;
// Lazy rescale, masked path: a row's running max moves only when the row's
// tile max exceeds it by more than kTau (log2 units), so P <= 2^kTau before
// normalisation.
constexpr float kTau = 8.0f;
// Unmasked path: a row's weights of one 64-key tile, taken against the
// running max, may sum up to Elem<T>::kSumCap; the row's max moves (to the
// exact max) only when its own sum leaves [0, kSumCap].  Both rules are
// decided per row, so a row's result depends on its own scores only, not on
// which rows share its wave.
// Every weight is at most that sum and is rounded to T for the PV product,
// so the cap must stay inside T's finite range: BF16 2^64 (no F32 overflow
// of O for any |V| < 2^40 and Lk < 2^20); F16 2^15, below its largest
// finite value 65504 -- a weight of 2^16 would round to +inf.

// ---------------------------------------------------------------------
// element-type traits: MFMA and F32 <-> storage conversions
// ---------------------------------------------------------------------
template <typename T> struct Elem;

template <> struct Elem<__bf16> {
    typedef bf16x8 vec8;
    static constexpr float kSumCap = 18446744073709551616.0f;   // 2^64
    static __device__ __forceinline__ f32x16 mfma(vec8 a, vec8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
        bf16x2 v = __builtin_convertvector((f32x4){lo, hi, 0.f, 0.f}.xy, bf16x2);
        return __builtin_bit_cast(uint32_t, v);
    }
    static __device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
    static __device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
};

template <> struct Elem<_Float16> {
    typedef f16x8 vec8;
    static constexpr float kSumCap = 32768.0f;                  // 2^15
    static __device__ __forceinline__ f32x16 mfma(vec8 a, vec8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
        f16x2 v = __builtin_convertvector((f32x4){lo, hi, 0.f, 0.f}.xy, f16x2);
        return __builtin_bit_cast(uint32_t, v);
    }
    static __device__ __forceinline__ float lo(uint32_t w) { return (float)__builtin_bit_cast(f16x2, w).x; }
    static __device__ __forceinline__ float hi(uint32_t w) { return (float)__builtin_bit_cast(f16x2, w).y; }
};

static __device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
static __device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
static __device__ __forceinline__ float f16_lo(uint32_t w) { return (float)__builtin_bit_cast(f16x2, w).x; }
static __device__ __forceinline__ float f16_hi(uint32_t w) { return (float)__builtin_bit_cast(f16x2, w).y; }

static __device__ __forceinline__ u32x4 ld16(const void *p) { return *reinterpret_cast<const u32x4 *>(p); }

// Eight consecutive elements of a row (16-byte aligned) as F32.
static __device__ __forceinline__ void load8_f32(const char *p, int type, float x[8]) {
    if (type == KD_FA_TYPE_F32) {
        const f32x4 a = *reinterpret_cast<const f32x4 *>(p);
        const f32x4 b = *reinterpret_cast<const f32x4 *>(p + 16);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    } else {
        const u32x4 w = ld16(p);
        if (type == KD_FA_TYPE_BF16) {
            for (int j = 0; j < 4; ++j) { x[2 * j] = bf16_lo(w[j]); x[2 * j + 1] = bf16_hi(w[j]); }
        } else {
            for (int j = 0; j < 4; ++j) { x[2 * j] = f16_lo(w[j]); x[2 * j + 1] = f16_hi(w[j]); }
        }
    }
}

// n / d for 0 <= n < 2^24, d >= 1, given rd = 1.0f / d: the float quotient
// is within one of the true one, and one correction step each way fixes it.
static __device__ __forceinline__ int div_small(int n, int d, float rd) {
    int q = (int)((float)n * rd);
    const int r = n - q * d;
    q += (r >= d) - (r < 0);
    return q;
}

// (cos, sin) pairs for columns d0 .. d0+7 of token `tok`: TABLE reads row
// `tok` of the [D, L] table; AXES reads the row of the token's t, h or w
// coordinate from the per-axis table holding that column block.
template <int RM>
static __device__ __forceinline__ const float *rope_ptr(const Args &a, int tok, int d0) {
    if (RM == KD_FA_ROPE_TABLE)
        return reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.rope_tab) +
                                               (int64_t)tok * a.rope_nb1) + d0;
    const int tw = div_small(tok, a.grid_w, a.rcp_w);          // t*Hp + h
    if (d0 < a.axis0) return a.axes + div_small(tw, a.grid_h, a.rcp_h) * a.axis0 + d0;
    if (d0 < a.axis0 + a.axis1) {
        const int h = tw - div_small(tw, a.grid_h, a.rcp_h) * a.grid_h;
        return a.axes + a.grid_t * a.axis0 + h * a.axis1 + (d0 - a.axis0);
    }
    const int w = tok - tw * a.grid_w;
    return a.axes + a.grid_t * a.axis0 + a.grid_h * a.axis1 + w * a.axis2 + (d0 - a.axis0 - a.axis1);
}

// rope::apply's pair rotation (src/rope.hpp:137-138): every product and
// every sum rounded to F32 on its own, as the separate ggml ops do.
static __device__ __forceinline__ void rotate8(float x[8], f32x4 c0, f32x4 c1) {
#pragma clang fp contract(off)
    const float cs[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    for (int j = 0; j < 4; ++j) {
        const float x0 = x[2 * j], x1 = x[2 * j + 1];
        const float c = cs[2 * j], s = cs[2 * j + 1];
        const float p0 = x0 * c, p1 = x1 * s, p2 = x0 * s, p3 = x1 * c;
        x[2 * j] = p0 - p1;
        x[2 * j + 1] = p2 + p3;
    }
}

// K tile: LDS row r holds key k_row_of(r) (bits 2 and 3 exchanged, its own
// inverse); 16-byte chunk c of a row is stored at c ^ (r & 15).
// V tile: row r holds key r; chunk c is stored at c ^ v_swz(r).  Both keep
// the MFMA operand reads free of bank conflicts on 32- and 64-bank LDS.
static __device__ __forceinline__ int k_row_of(int key) {
    return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
}
static __device__ __forceinline__ int v_swz(int r) { return ((r & 3) << 2) | (r & 2); }

// One wave-wide 16-byte-per-lane DMA: global (base + lane offset) -> LDS
// (wave-uniform destination + 16 * lane).  Written as the instruction itself
// so that the uniform base stays in SGPRs with a 32-bit lane offset (no
// per-lane 64-bit address registers); the compiler does not track it, so
// every consumer waits with an explicit s_waitcnt vmcnt(0) + barrier.
static __device__ __forceinline__ void dma16(const char *base, uint32_t lane_off, lds_t *lds_wave_base) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_wave_base);
    asm volatile("global_load_lds_dwordx4 %0, %1" :: "v"(lane_off), "s"(base), "{m0}"(m0));
}

// v_max3_f32 directly: the maxnum builtins would first canonicalise every
// input (one extra v_max_f32 each) to quiet signalling NaNs, which the
// scores never are
static __device__ __forceinline__ float max3(float a, float b, float c) {
    float d;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
    return d;
}

// max of 32 values: two interleaved chains of v_max3_f32
static __device__ __forceinline__ float max32(const float *p) {
    float x = max3(p[0], p[1], p[2]);
    float y = max3(p[3], p[4], p[5]);
#pragma unroll
    for (int i = 6; i < 30; i += 4) {
        x = max3(x, p[i], p[i + 1]);
        y = max3(y, p[i + 2], p[i + 3]);
    }
    return max3(x, y, __builtin_fmaxf(p[30], p[31]));
}

// max32 for scores fresh from the matrix unit: max3 is inline asm, whose
// operands the compiler does not check against the wait states that an MFMA
// result needs before a vector instruction reads it; these v_max it sees.
// The same value as max32 (a max is exact; either zero may stand for a
// +-0 tie, which gives every weight and rescale factor the same value).
static __device__ __forceinline__ float max32_mfma(const float *p) {
    float x = __builtin_fmaxf(p[0], p[1]);
    float y = __builtin_fmaxf(p[2], p[3]);
#pragma unroll
    for (int i = 4; i < 32; i += 4) {
        x = __builtin_fmaxf(x, __builtin_fmaxf(p[i], p[i + 1]));
        y = __builtin_fmaxf(y, __builtin_fmaxf(p[i + 2], p[i + 3]));
    }
    return __builtin_fmaxf(x, y);
}

// max over the lane pair (l, l ^ 32) that shares one query row
static __device__ __forceinline__ float pair_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
static __device__ __forceinline__ float pair_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ---------------------------------------------------------------------
// RMSNorm of a head row (ops::rms_norm = ggml_rms_norm + ggml_mul,
// src/core/ops.hpp:76-80): the squares rounded to F32 and summed in double,
// mean = (float)(sum / 128), scale = 1.0f / sqrtf(mean + eps) (both
// correctly rounded), then x * scale * w with each product rounded to F32.
// A row's squares are spread over several lanes; the caller reduces the
// partial double sums over them before rms_scale.
// ---------------------------------------------------------------------
static __device__ __forceinline__ double sum_sq8(const float x[8]) {
#pragma clang fp contract(off)
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float sq = x[i] * x[i];
        s += (double)sq;
    }
    return s;
}

// sqrtf as the C library computes it (correctly rounded): v_sqrt_f32 alone
// is within 1 ulp only, so the root is taken in double -- whose square root
// sequence is exact to well under a double ulp -- and rounded once; rounding
// a square root from 53 to 24 bits cannot round twice (53 >= 2*24 + 2).
static __device__ __forceinline__ float sqrt_rn(float x) { return (float)__builtin_sqrt((double)x); }

static __device__ __forceinline__ float rms_scale(double sum, float eps) {
    const float mean = (float)(sum * (1.0 / 128.0));
    return 1.0f / sqrt_rn(mean + eps);
}

// x = x * scale * w[0..7] (two roundings per element)
static __device__ __forceinline__ void rms_apply8(float x[8], float scale, f32x4 w0, f32x4 w1) {
#pragma clang fp contract(off)
    const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float y = x[i] * scale;
        x[i] = y * w[i];
    }
}

// sum of a double over the lane pair (l, l ^ 32)
static __device__ __forceinline__ double pair_sum_f64(double x) {
    const uint64_t u = __builtin_bit_cast(uint64_t, x);
    const auto lo = __builtin_amdgcn_permlane32_swap((uint32_t)u, (uint32_t)u, false, false);
    const auto hi = __builtin_amdgcn_permlane32_swap((uint32_t)(u >> 32), (uint32_t)(u >> 32), false, false);
    const double a = __builtin_bit_cast(double, (uint64_t)lo[0] | ((uint64_t)hi[0] << 32));
    const double b = __builtin_bit_cast(double, (uint64_t)lo[1] | ((uint64_t)hi[1] << 32));
    return a + b;
}

// sum of a double over the 16 lanes of each aligned 16-lane group
static __device__ __forceinline__ double sum16_f64(double x) {
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) x += __shfl_xor(x, m, 64);
    return x;
}

// O / l of query row q_row -> dst[b][q_row][h][d_base + :128] (F32, or
// rounded to F16 / BF16).  o holds O^T of the row's 32-row block in MFMA
// accumulator order (element i of d block dblk: d = dblk*32 + 8*(i/4) +
// 4*hi + i%4); l_run is the row's weight sum (the kernels that hold half of
// it per lane add the lane pair first).
static __device__ __forceinline__ void store_o_row_l(const Args &a, int q_row, int h, int b, int hi, const f32x16 o[4],
                                              float l_run, int d_base) {
    if (q_row < a.Lq) {
        const float inv = l_run == 0.0f ? 0.0f : 1.0f / l_run;
        char *op = a.o + (int64_t)b * a.o_nb3 + (int64_t)q_row * a.o_nb2 + (int64_t)h * a.o_nb1 +
                   (int64_t)d_base * (a.o_type == KD_FA_TYPE_F32 ? 4 : 2);
        const int ot = a.o_type;
#pragma unroll
        for (int dblk = 0; dblk < 4; ++dblk)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = dblk * 32 + 8 * g + 4 * hi;
                const f32x4 v = {o[dblk][4 * g] * inv, o[dblk][4 * g + 1] * inv,
                                 o[dblk][4 * g + 2] * inv, o[dblk][4 * g + 3] * inv};
                if (ot == KD_FA_TYPE_F32) {
                    *reinterpret_cast<f32x4 *>(op + d * 4) = v;
                } else if (ot == KD_FA_TYPE_BF16) {
                    const u32x2 w = {Elem<__bf16>::pack2(v.x, v.y), Elem<__bf16>::pack2(v.z, v.w)};
                    *reinterpret_cast<u32x2 *>(op + d * 2) = w;
                } else {
                    const u32x2 w = {Elem<_Float16>::pack2(v.x, v.y), Elem<_Float16>::pack2(v.z, v.w)};
                    *reinterpret_cast<u32x2 *>(op + d * 2) = w;
                }
            }
    }
}

}  // namespace kdfa
