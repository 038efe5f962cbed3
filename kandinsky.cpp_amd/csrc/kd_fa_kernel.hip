// kd_fa_kernel.hip - gfx950 flash-attention forward for the CrossDiT
// attention node (GGML_OP_FLASH_ATTN_EXT as src/core/ops.hpp:176 builds it),
// with optional RoPE (src/rope.hpp:109-155) fused into the Q/K operand loads.
//
// One workgroup = 4 waves = 128 query rows of one (batch, head); each wave
// owns 32 query rows for the whole key loop.  Per 64-key tile:
//   S^T[key][query] = K Q^T   on v_mfma_f32_32x32x16_{bf16,f16}
//   online softmax in F32 (exp2 domain, one cross-lane exchange per row)
//   O^T[d][query]  += V^T P^T on the same MFMA shape
// K and V tiles are double-buffered in LDS (2 x 32 KiB), written through
// registers so that RoPE (K) and the transpose (V) happen on the way in.
//
// Operand layouts of v_mfma_f32_32x32x16 (wave64):
//   A (32 x 16): lane l holds row l%32, k = (l/32)*8 .. +7
//   B (16 x 32): lane l holds column l%32, k = (l/32)*8 .. +7
//   C (32 x 32): lane l, element i holds row 8*(i/4) + 4*(l/32) + i%4,
//                column l%32
// The S^T product uses A = K (keys on M) and B = Q^T (queries on N), so
// each lane holds 16 scores of one query per 32-key block.  The K rows of
// each 32-key block sit in LDS in "swapped" order (bits 2 and 3 of the key
// index exchanged), which makes score element i of lane l belong to key
// 16*(i/8) + 8*(l/32) + i%8: elements 0..7 and 8..15 are then exactly the
// B operands (P^T, keys on K) of the two 16-key PV steps.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kd_fa_kernel.h"

namespace kdfa {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kD = 128;        // head dim (Dk = Dv)
constexpr int kBM = 128;       // query rows per workgroup
constexpr int kBN = 64;        // keys per tile
constexpr int kThreads = 256;  // 4 waves
constexpr int kKBytes = kBN * kD * 2;   // one K tile in LDS
constexpr int kVBytes = kD * kBN * 2;   // one V^T tile in LDS
constexpr int kBufBytes = kKBytes + kVBytes;
constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------
// element-type traits: MFMA and F32 <-> storage conversions
// ---------------------------------------------------------------------
template <typename T> struct Elem;

template <> struct Elem<__bf16> {
    typedef bf16x8 vec8;
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
    static __device__ __forceinline__ f32x16 mfma(vec8 a, vec8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
        f16x2 v = __builtin_convertvector((f32x4){lo, hi, 0.f, 0.f}.xy, f16x2);
        return __builtin_bit_cast(uint32_t, v);
    }
    static __device__ __forceinline__ float lo(uint32_t w) {
        return (float)__builtin_bit_cast(f16x2, w).x;
    }
    static __device__ __forceinline__ float hi(uint32_t w) {
        return (float)__builtin_bit_cast(f16x2, w).y;
    }
};

static __device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
static __device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
static __device__ __forceinline__ float f16_lo(uint32_t w) { return (float)__builtin_bit_cast(f16x2, w).x; }
static __device__ __forceinline__ float f16_hi(uint32_t w) { return (float)__builtin_bit_cast(f16x2, w).y; }

static __device__ __forceinline__ u32x4 ld16(const void *p) {
    return *reinterpret_cast<const u32x4 *>(p);
}

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

// (cos, sin) pairs for columns d0 .. d0+7 of token `tok`.
static __device__ __forceinline__ void rope_cs8(const Args &a, int tok, int d0, float cs[8]) {
    const float *p;
    if (a.rope_mode == KD_FA_ROPE_TABLE) {
        p = reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.rope_tab) +
                                            (int64_t)tok * a.rope_nb1) + d0;
    } else {
        const int hw = a.grid_h * a.grid_w;
        if (d0 < a.axis0) {
            p = a.axes + (tok / hw) * a.axis0 + d0;
        } else if (d0 < a.axis0 + a.axis1) {
            p = a.axes + a.grid_t * a.axis0 + ((tok / a.grid_w) % a.grid_h) * a.axis1 + (d0 - a.axis0);
        } else {
            p = a.axes + a.grid_t * a.axis0 + a.grid_h * a.axis1 + (tok % a.grid_w) * a.axis2 +
                (d0 - a.axis0 - a.axis1);
        }
    }
    const f32x4 u = *reinterpret_cast<const f32x4 *>(p);
    const f32x4 v = *reinterpret_cast<const f32x4 *>(p + 4);
    cs[0] = u.x; cs[1] = u.y; cs[2] = u.z; cs[3] = u.w;
    cs[4] = v.x; cs[5] = v.y; cs[6] = v.z; cs[7] = v.w;
}

// rope::apply's pair rotation (src/rope.hpp:137-138): every product and
// every sum rounded to F32 on its own, as the separate ggml ops do.
static __device__ __forceinline__ void rotate8(float x[8], const float cs[8]) {
#pragma clang fp contract(off)
    for (int j = 0; j < 4; ++j) {
        const float x0 = x[2 * j], x1 = x[2 * j + 1];
        const float c = cs[2 * j], s = cs[2 * j + 1];
        const float p0 = x0 * c, p1 = x1 * s, p2 = x0 * s, p3 = x1 * c;
        x[2 * j] = p0 - p1;
        x[2 * j + 1] = p2 + p3;
    }
}

// Key index inside a 64-key tile <-> LDS row of the K tile (bits 2 and 3
// exchanged; the map is its own inverse).
static __device__ __forceinline__ int k_row_of(int key) {
    return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
}

// XOR swizzles of the 16-byte chunks of a K row (16 chunks) and of a V^T
// row (8 chunks): every group of 16 (or 8) lanes that reads one logical
// chunk column hits distinct banks.
static __device__ __forceinline__ int k_chunk(int row, int c) { return c ^ (row & 15); }
static __device__ __forceinline__ int v_chunk(int d, int c) { return c ^ ((d & 7) ^ ((d >> 3) & 1)); }

template <typename T, bool HAS_MASK, bool ROPE>
__global__ __launch_bounds__(kThreads) void fa_fwd_d128(Args a) {
    typedef Elem<T> E;
    typedef typename E::vec8 vec8;
    __shared__ __attribute__((aligned(16))) char smem[2 * kBufBytes];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l32 = lane & 31;
    const int hi = lane >> 5;

    // Workgroups are dealt to the 8 XCDs round-robin; give each XCD a
    // contiguous range of (b, h, q-tile) so the tiles of one head share
    // that XCD's L2.
    const int pid = blockIdx.x;
    const int per = a.n_blocks >> 3;
    const int lid = pid < per * 8 ? (pid & 7) * per + (pid >> 3) : pid;
    const int qt = lid % a.n_qt;
    const int bh = lid / a.n_qt;
    const int h = bh % a.H;
    const int b = bh / a.H;

    const char *kbase = a.k + (int64_t)(h / a.rk2) * a.k_nb2 + (int64_t)(b / a.rk3) * a.k_nb3;
    const char *vbase = a.v + (int64_t)(h / a.rv2) * a.v_nb2 + (int64_t)(b / a.rv3) * a.v_nb3;

    // ---- Q fragment (B operand of S^T): row q_row, k-steps of 16 -------
    const int q_row = qt * kBM + wave * 32 + l32;
    const int q_ld = q_row < a.Lq ? q_row : a.Lq - 1;
    vec8 qf[8];
    {
        const char *qp = a.q + (int64_t)q_ld * a.q_nb1 + (int64_t)h * a.q_nb2 + (int64_t)b * a.q_nb3;
        const int esz = a.q_type == KD_FA_TYPE_F32 ? 4 : 2;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const int d0 = ks * 16 + hi * 8;
            float x[8];
            load8_f32(qp + d0 * esz, a.q_type, x);
            if (ROPE) {
                float cs[8];
                rope_cs8(a, q_ld, d0, cs);
                rotate8(x, cs);
            }
            u32x4 w;
            for (int j = 0; j < 4; ++j) w[j] = E::pack2(x[2 * j], x[2 * j + 1]);
            qf[ks] = __builtin_bit_cast(vec8, w);
        }
    }

    const uint16_t *mrow = nullptr;
    if (HAS_MASK) {
        mrow = reinterpret_cast<const uint16_t *>(a.m + (int64_t)q_ld * a.m_nb1 +
                                                  (int64_t)(h % a.m_ne2) * a.m_nb2 +
                                                  (int64_t)(b % a.m_ne3) * a.m_nb3);
    }

    f32x16 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (f32x16){};
    float m_run = -INFINITY;
    float l_run = 0.0f;

    // ---- tile staging: global -> registers -> (RoPE / transpose) -> LDS --
    // K: thread handles chunks u = tid + 256*j: key u/16, 16-byte chunk u%16.
    // V: thread handles keys 4*(tid%16) .. +3 at d-chunk tid/16.
    const int v_kq = tid & 15;
    const int v_dc = tid >> 4;
    u32x4 kr[4], vr[4];

    auto load_tile = [&](int t) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int u = tid + kThreads * j;
            const int gk = t * kBN + (u >> 4);
            kr[j] = gk < a.Lk ? ld16(kbase + (int64_t)gk * a.k_nb1 + (u & 15) * 16) : (u32x4){0, 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int gk = t * kBN + 4 * v_kq + j;
            vr[j] = gk < a.Lk ? ld16(vbase + (int64_t)gk * a.v_nb1 + v_dc * 16) : (u32x4){0, 0, 0, 0};
        }
    };

    auto store_tile = [&](int t, int buf) {
        char *ks_ = smem + buf * kBufBytes;
        char *vt_ = ks_ + kKBytes;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int u = tid + kThreads * j;
            const int key = u >> 4, c = u & 15;
            u32x4 w = kr[j];
            if (ROPE) {
                const int gk = t * kBN + key;
                if (gk < a.Lk) {
                    float x[8], cs[8];
                    for (int e = 0; e < 4; ++e) { x[2 * e] = E::lo(w[e]); x[2 * e + 1] = E::hi(w[e]); }
                    rope_cs8(a, gk, c * 8, cs);
                    rotate8(x, cs);
                    for (int e = 0; e < 4; ++e) w[e] = E::pack2(x[2 * e], x[2 * e + 1]);
                }
            }
            const int row = k_row_of(key);
            *reinterpret_cast<u32x4 *>(ks_ + row * 256 + k_chunk(row, c) * 16) = w;
        }
        // V^T: for d = 8*v_dc + e, keys 4*v_kq .. +3 -> 8 bytes
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int d = v_dc * 8 + e;
            const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
            const uint32_t w0 = __builtin_amdgcn_perm(vr[1][e >> 1], vr[0][e >> 1], sel);
            const uint32_t w1 = __builtin_amdgcn_perm(vr[3][e >> 1], vr[2][e >> 1], sel);
            const int c = v_kq >> 1;
            *reinterpret_cast<u32x2 *>(vt_ + d * 128 + v_chunk(d, c) * 16 + (v_kq & 1) * 8) = (u32x2){w0, w1};
        }
    };

    const int n_tiles = (a.Lk + kBN - 1) / kBN;
    if (n_tiles > 0) {
        load_tile(0);
        store_tile(0, 0);
    }
    __syncthreads();

    const float c2 = a.scale_log2;
    for (int t = 0; t < n_tiles; ++t) {
        const int buf = t & 1;
        const bool has_next = t + 1 < n_tiles;
        if (has_next) load_tile(t + 1);

        const char *ks_ = smem + buf * kBufBytes;
        const char *vt_ = ks_ + kKBytes;

        // mask values of this lane's 32 keys (keys 16*hh + 8*hi + e of each
        // 32-key block mb), as F32; -inf also marks keys >= Lk
        float mv[32];
        bool live = true;
        if (HAS_MASK) {
            bool any = false;
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int k0 = t * kBN + mb * 32 + hh * 16 + hi * 8;
                    float x[8];
                    if (a.mask_vec && k0 + 8 <= a.Lk) {
                        const u32x4 w = ld16(mrow + k0);
                        for (int j = 0; j < 4; ++j) { x[2 * j] = f16_lo(w[j]); x[2 * j + 1] = f16_hi(w[j]); }
                    } else {
                        for (int e = 0; e < 8; ++e) {
                            if (k0 + e < a.Lk) {
                                const uint16_t hb = mrow[k0 + e];
                                x[e] = (float)__builtin_bit_cast(_Float16, hb);
                            } else {
                                x[e] = -INFINITY;
                            }
                        }
                    }
                    for (int e = 0; e < 8; ++e) {
                        mv[mb * 16 + hh * 8 + e] = x[e];
                        any |= x[e] != -INFINITY;
                    }
                }
            live = __builtin_amdgcn_ballot_w64(any) != 0;
        }

        if (live) {
            // ---- S^T = K Q^T ------------------------------------------------
            f32x16 s[2];
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) {
                s[mb] = (f32x16){};
                const int row = mb * 32 + l32;
#pragma unroll
                for (int ks = 0; ks < 8; ++ks) {
                    const int c = ks * 2 + hi;
                    const vec8 ka = *reinterpret_cast<const vec8 *>(ks_ + row * 256 + k_chunk(row, c) * 16);
                    s[mb] = E::mfma(ka, qf[ks], s[mb]);
                }
            }

            // ---- online softmax (log2 domain) -------------------------------
            float x[32];
            const bool tail = (t + 1) * kBN > a.Lk;
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    float v = s[mb][i] * c2;
                    if (HAS_MASK) {
                        const float m = mv[mb * 16 + i];
                        v = m == -INFINITY ? -INFINITY : __builtin_fmaf(m, kLog2e, v);
                    }
                    if (tail) {
                        const int key = t * kBN + mb * 32 + 16 * (i >> 3) + 8 * hi + (i & 7);
                        if (key >= a.Lk) v = -INFINITY;
                    }
                    x[mb * 16 + i] = v;
                }
            float mx = x[0];
#pragma unroll
            for (int i = 1; i < 32; ++i) mx = fmaxf(mx, x[i]);
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float m_new = fmaxf(m_run, mx);
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                x[i] = __builtin_amdgcn_exp2f(x[i] - m_use);
                sum += x[i];
            }
            sum += __shfl_xor(sum, 32);
            l_run = l_run * alpha + sum;
            m_run = m_new;
            if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
                for (int dblk = 0; dblk < 4; ++dblk)
#pragma unroll
                    for (int i = 0; i < 16; ++i) o[dblk][i] *= alpha;
            }

            // ---- O^T += V^T P^T ----------------------------------------------
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    u32x4 pw;
                    const int base = mb * 16 + kk * 8;
                    for (int j = 0; j < 4; ++j) pw[j] = E::pack2(x[base + 2 * j], x[base + 2 * j + 1]);
                    const vec8 pb = __builtin_bit_cast(vec8, pw);
                    const int c = mb * 4 + kk * 2 + hi;
#pragma unroll
                    for (int dblk = 0; dblk < 4; ++dblk) {
                        const int d = dblk * 32 + l32;
                        const vec8 va = *reinterpret_cast<const vec8 *>(vt_ + d * 128 + v_chunk(d, c) * 16);
                        o[dblk] = E::mfma(va, pb, o[dblk]);
                    }
                }
        }

        if (has_next) store_tile(t + 1, buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue: O / l -> dst[b][q][h][:] (F32) ---------------------------
    if (q_row < a.Lq) {
        const float inv = l_run == 0.0f ? 0.0f : 1.0f / l_run;
        char *op = a.o + (int64_t)b * a.o_nb3 + (int64_t)q_row * a.o_nb2 + (int64_t)h * a.o_nb1;
#pragma unroll
        for (int dblk = 0; dblk < 4; ++dblk)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = dblk * 32 + 8 * g + 4 * hi;
                const f32x4 v = {o[dblk][4 * g] * inv, o[dblk][4 * g + 1] * inv,
                                 o[dblk][4 * g + 2] * inv, o[dblk][4 * g + 3] * inv};
                *reinterpret_cast<f32x4 *>(op + d * 4) = v;
            }
    }
}

template <typename T, bool M, bool R>
static hipError_t launch_t(const Args &a, hipStream_t stream) {
    hipLaunchKernelGGL((fa_fwd_d128<T, M, R>), dim3(a.n_blocks), dim3(kThreads), 0, stream, a);
    return hipGetLastError();
}

template <typename T>
static hipError_t launch_m(const Args &a, bool mask, bool rope, hipStream_t s) {
    if (mask) return rope ? launch_t<T, true, true>(a, s) : launch_t<T, true, false>(a, s);
    return rope ? launch_t<T, false, true>(a, s) : launch_t<T, false, false>(a, s);
}

hipError_t launch(const Args &a, int kv_type, hipStream_t stream) {
    const bool mask = a.m != nullptr;
    const bool rope = a.rope_mode != KD_FA_ROPE_NONE;
    if (kv_type == KD_FA_TYPE_BF16) return launch_m<__bf16>(a, mask, rope, stream);
    return launch_m<_Float16>(a, mask, rope, stream);
}

}  // namespace kdfa
