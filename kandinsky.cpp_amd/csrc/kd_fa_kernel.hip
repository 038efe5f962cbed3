// kd_fa_kernel.hip - gfx950 flash-attention forward for the CrossDiT
// attention node (GGML_OP_FLASH_ATTN_EXT as src/core/ops.hpp:176 builds it),
// with optional RoPE (src/rope.hpp:109-155) fused into the Q/K operand loads.
//
// One workgroup = 8 waves = 256 query rows of one (batch, head); each wave
// owns 32 query rows for the whole key loop, and two waves share each SIMD
// so that one wave's softmax (VALU) overlaps the other's matrix products.
// Per 64-key tile:
//   S^T[key][query] = K Q^T   on v_mfma_f32_32x32x16_{bf16,f16}
//   online softmax in F32 (exp2 domain, row max shared by a lane pair)
//   O^T[d][query]  += V^T P^T on the same MFMA shape
// K and V tiles are double-buffered in LDS (2 x 32 KiB) and streamed
// global -> LDS by the DMA path (global_load_lds, 16 bytes per lane) while
// the previous tile is being computed.  With RoPE, K instead passes through
// registers, where it is rotated on its way into LDS.
//
// Operand layouts of v_mfma_f32_32x32x16 (wave64):
//   A (32 x 16): lane l holds row l%32, k = (l/32)*8 .. +7
//   B (16 x 32): lane l holds column l%32, k = (l/32)*8 .. +7
//   C (32 x 32): lane l, element i holds row 8*(i/4) + 4*(l/32) + i%4,
//                column l%32
// S^T uses A = K (keys on M) and B = Q^T (queries on N): each lane holds 16
// scores of one query per 32-key block.  The K rows of each 32-key block sit
// in LDS with bits 2 and 3 of the key index exchanged, which makes score
// element i of lane l belong to key 16*(i/8) + 8*(l/32) + i%8: elements
// 0..7 and 8..15 are then exactly the B operands (P^T) of the two 16-key PV
// steps.  The PV A operand (V^T) is read from row-major V with
// ds_read_b64_tr_b16: within each 16-lane group, source lane s supplies 4
// elements and result lane j receives element j%4 of source lanes j/4 + 4r,
// r = 0..3 -- one column of 4 consecutive keys per lane.
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
typedef short s16x4 __attribute__((ext_vector_type(4)));

#define LDS_PTR(T, p) ((__attribute__((address_space(3))) T *)(p))

constexpr int kD = 128;          // head dim (Dk = Dv)
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kBM = 32 * kWaves; // query rows per workgroup
constexpr int kBN = 64;          // keys per tile
constexpr int kTileBytes = kBN * kD * 2;   // one K or V tile
constexpr float kLog2e = 1.4426950408889634f;
// Lazy rescale: the running max moves only when a row max exceeds it by
// more than kTau (log2 units), so P <= 2^kTau before normalisation.
constexpr float kTau = 8.0f;

static_assert(kBM == kBlockM, "block rows");

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

// Address of the (cos, sin) pairs for columns d0 .. d0+7 of token `tok`.
static __device__ __forceinline__ const float *rope_ptr(const Args &a, int tok, int d0) {
    if (a.rope_mode == KD_FA_ROPE_TABLE)
        return reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.rope_tab) +
                                               (int64_t)tok * a.rope_nb1) + d0;
    const int hw = a.grid_h * a.grid_w;
    if (d0 < a.axis0) return a.axes + (tok / hw) * a.axis0 + d0;
    if (d0 < a.axis0 + a.axis1)
        return a.axes + a.grid_t * a.axis0 + ((tok / a.grid_w) % a.grid_h) * a.axis1 + (d0 - a.axis0);
    return a.axes + a.grid_t * a.axis0 + a.grid_h * a.axis1 + (tok % a.grid_w) * a.axis2 +
           (d0 - a.axis0 - a.axis1);
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

static __device__ __forceinline__ void dma16(const void *g, char *lds_wave_base) {
    __builtin_amdgcn_global_load_lds(g, LDS_PTR(void, lds_wave_base), 16, 0, 0);
}

static __device__ __forceinline__ float max3(float a, float b, float c) {
    return __builtin_fmaxf(a, __builtin_fmaxf(b, c));
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

template <typename T, bool HAS_MASK, bool ROPE>
__global__ __launch_bounds__(kThreads) void fa_fwd_d128(Args a) {
    typedef Elem<T> E;
    typedef typename E::vec8 vec8;
    // four distinct LDS objects (not one array) so that the compiler can
    // tell the tile being computed from the tile the DMA is filling
    __shared__ __attribute__((aligned(1024))) char sK0[kTileBytes];
    __shared__ __attribute__((aligned(1024))) char sK1[kTileBytes];
    __shared__ __attribute__((aligned(1024))) char sV0[kTileBytes];
    __shared__ __attribute__((aligned(1024))) char sV1[kTileBytes];

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
    const int Lk = a.Lk;

    // ---- Q fragment (B operand of S^T): row q_row, k-steps of 16 -----------
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
                const float *cp = rope_ptr(a, q_ld, d0);
                rotate8(x, *reinterpret_cast<const f32x4 *>(cp), *reinterpret_cast<const f32x4 *>(cp + 4));
            }
            u32x4 w;
            for (int j = 0; j < 4; ++j) w[j] = E::pack2(x[2 * j], x[2 * j + 1]);
            // scale < 0: use -q (exact) and |scale|, so that every score
            // below is s * c2 with c2 >= 0 and its max is max(s) * c2
            if (a.scale_log2 < 0.0f) w ^= (u32x4){0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
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
    float m_run = -INFINITY;   // running max (log2 units), same in both lanes of a pair
    float l_half = 0.0f;       // running sum over this lane's half of the keys

    // ---- tile staging -------------------------------------------------------
    // DMA: each wave fills 1 KiB (4 rows) of a tile per instruction; wave w
    // covers rows 4*(w + 8j) .. +3, j = 0, 1, for K and for V.
    const int dma_row = lane >> 4;        // row within the wave's 4 rows
    const int dma_pc = lane & 15;         // physical chunk this lane fills
    auto issue_tile = [&](int t, char *dK, char *dV) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int r = 4 * (wave + 8 * j) + dma_row;
            int gk = t * kBN + r;
            gk = gk < Lk ? gk : Lk - 1;
            dma16(vbase + (int64_t)gk * a.v_nb1 + ((dma_pc ^ v_swz(r)) << 4),
                  dV + (wave + 8 * j) * 1024);
        }
        if (!ROPE) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int r = 4 * (wave + 8 * j) + dma_row;
                int gk = t * kBN + k_row_of(r);
                gk = gk < Lk ? gk : Lk - 1;
                dma16(kbase + (int64_t)gk * a.k_nb1 + ((dma_pc ^ (r & 15)) << 4),
                      dK + (wave + 8 * j) * 1024);
            }
        }
    };
    // RoPE: K chunk u = tid + 512*j -> LDS row u/16, physical chunk u%16.
    u32x4 kreg[2];
    f32x4 kcs[2][2];
    auto rope_load = [&](int t) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int u = tid + kThreads * j;
            const int r = u >> 4;
            const int c = (u & 15) ^ (r & 15);
            int gk = t * kBN + k_row_of(r);
            gk = gk < Lk ? gk : Lk - 1;
            kreg[j] = ld16(kbase + (int64_t)gk * a.k_nb1 + c * 16);
            const float *cp = rope_ptr(a, gk, c * 8);
            kcs[j][0] = *reinterpret_cast<const f32x4 *>(cp);
            kcs[j][1] = *reinterpret_cast<const f32x4 *>(cp + 4);
        }
    };
    auto rope_store = [&](char *dK) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int u = tid + kThreads * j;
            float x[8];
            for (int e = 0; e < 4; ++e) { x[2 * e] = E::lo(kreg[j][e]); x[2 * e + 1] = E::hi(kreg[j][e]); }
            rotate8(x, kcs[j][0], kcs[j][1]);
            u32x4 w;
            for (int e = 0; e < 4; ++e) w[e] = E::pack2(x[2 * e], x[2 * e + 1]);
            *reinterpret_cast<u32x4 *>(dK + u * 16) = w;
        }
    };

    // mask values of this lane's 32 keys (key 16*hh + 8*hi + e of 32-key
    // block mb at index mb*16 + hh*8 + e), prefetched one tile ahead
    u32x4 mraw[4];
    auto mask_load = [&](int t) {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int k0 = t * kBN + mb * 32 + hh * 16 + hi * 8;
                u32x4 w;
                if (a.mask_vec && k0 + 8 <= Lk) {
                    w = ld16(mrow + k0);
                } else {
                    uint16_t e16[8];
                    for (int e = 0; e < 8; ++e) e16[e] = k0 + e < Lk ? mrow[k0 + e] : (uint16_t)0xfc00u;
                    for (int e = 0; e < 4; ++e) w[e] = (uint32_t)e16[2 * e] | ((uint32_t)e16[2 * e + 1] << 16);
                }
                mraw[mb * 2 + hh] = w;
            }
    };

    const int n_tiles = (Lk + kBN - 1) / kBN;
    if (n_tiles > 0) {
        issue_tile(0, sK0, sV0);
        if (ROPE) {
            rope_load(0);
            rope_store(sK0);
        }
        if (HAS_MASK) mask_load(0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    const float c2 = __builtin_fabsf(a.scale_log2);
    // K-operand LDS offset of this lane (rows l32 and 32 + l32 share the swizzle)
    const int k_off = l32 * 256;
    const int k_swz = lane & 15;
    // V-operand (ds_read_b64_tr_b16) LDS offsets of this lane
    const int v_sub = (lane & 15) >> 2;            // row within a 4-row group
    const int v_g1 = (lane >> 4) & 1;
    const int v_c_lo = 2 * v_g1 + ((lane & 3) >> 1);
    const int v_byte = 8 * (lane & 1);

    auto step = [&](int t, const char *ks_, const char *vs_, char *nK, char *nV) {
        const bool has_next = t + 1 < n_tiles;
        if (has_next) {
            issue_tile(t + 1, nK, nV);
            if (ROPE) rope_load(t + 1);
        }

        float mv[32];
        bool live = true;
        if (HAS_MASK) {
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    mv[q4 * 8 + 2 * e] = f16_lo(mraw[q4][e]);
                    mv[q4 * 8 + 2 * e + 1] = f16_hi(mraw[q4][e]);
                }
            bool any = false;
#pragma unroll
            for (int i = 0; i < 32; ++i) any |= mv[i] != -INFINITY;
            live = __builtin_amdgcn_ballot_w64(any) != 0;
            if (has_next) mask_load(t + 1);
        }

        if (live) {
            // ---- S^T = K Q^T ------------------------------------------------
            f32x16 s0 = (f32x16){}, s1 = (f32x16){};
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                const int off = k_off + (((2 * ks + hi) ^ k_swz) << 4);
                const vec8 a0 = *reinterpret_cast<const vec8 *>(ks_ + off);
                const vec8 a1 = *reinterpret_cast<const vec8 *>(ks_ + off + 32 * 256);
                s0 = E::mfma(a0, qf[ks], s0);
                s1 = E::mfma(a1, qf[ks], s1);
            }

            // ---- online softmax (log2 domain) -------------------------------
            float p[32];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                p[i] = s0[i];
                p[16 + i] = s1[i];
            }
            if (!HAS_MASK) {
                // keys past Lk (last tile only): -inf raw scores for the max
                // (each lane pair still holds the tile's first key, which is
                // valid) and -inf exponents below
                const bool tail = (t + 1) * kBN > Lk;
                if (tail) {
#pragma unroll
                    for (int i = 0; i < 32; ++i) {
                        const int key = t * kBN + (i >> 4) * 32 + 16 * ((i >> 3) & 1) + 8 * hi + (i & 7);
                        p[i] = key < Lk ? p[i] : -INFINITY;
                    }
                }
                float mx = max3(p[0], p[1], p[2]);
#pragma unroll
                for (int i = 3; i < 31; i += 2) mx = max3(mx, p[i], p[i + 1]);
                mx = __builtin_fmaxf(mx, p[31]);
                mx = pair_max(mx) * c2;
                if (__builtin_amdgcn_ballot_w64(mx > m_run + kTau) != 0) {
                    const float m_new = __builtin_fmaxf(m_run, mx);
                    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
                    m_run = m_new;
                    l_half *= alpha;
#pragma unroll
                    for (int dblk = 0; dblk < 4; ++dblk)
#pragma unroll
                        for (int i = 0; i < 16; ++i) o[dblk][i] *= alpha;
                }
                const float nm = -m_run;
#pragma unroll
                for (int i = 0; i < 32; ++i) p[i] = __builtin_fmaf(p[i], c2, nm);
                if (tail) {
#pragma unroll
                    for (int i = 0; i < 32; ++i) {
                        const int key = t * kBN + (i >> 4) * 32 + 16 * ((i >> 3) & 1) + 8 * hi + (i & 7);
                        p[i] = key < Lk ? p[i] : -INFINITY;
                    }
                }
#pragma unroll
                for (int i = 0; i < 32; ++i) p[i] = __builtin_amdgcn_exp2f(p[i]);
            } else {
                // log2-domain logits s*c2 + mask*log2(e); -inf mask entries
                // (and keys past Lk, filled with -inf) stay -inf
#pragma unroll
                for (int i = 0; i < 32; ++i)
                    p[i] = mv[i] == -INFINITY ? -INFINITY : __builtin_fmaf(mv[i], kLog2e, p[i] * c2);
                float mx = max3(p[0], p[1], p[2]);
#pragma unroll
                for (int i = 3; i < 31; i += 2) mx = max3(mx, p[i], p[i + 1]);
                mx = __builtin_fmaxf(mx, p[31]);
                mx = pair_max(mx);
                if (__builtin_amdgcn_ballot_w64(mx > m_run + kTau) != 0) {
                    const float m_new = __builtin_fmaxf(m_run, mx);
                    const float alpha = m_new == m_run ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
                    m_run = m_new;
                    l_half *= alpha;
#pragma unroll
                    for (int dblk = 0; dblk < 4; ++dblk)
#pragma unroll
                        for (int i = 0; i < 16; ++i) o[dblk][i] *= alpha;
                }
                const float mu = m_run == -INFINITY ? 0.0f : m_run;
#pragma unroll
                for (int i = 0; i < 32; ++i) p[i] = __builtin_amdgcn_exp2f(p[i] - mu);
            }
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; ++i) sum += p[i];
            l_half += sum;

            // ---- O^T += V^T P^T ----------------------------------------------
            vec8 pb[4];
#pragma unroll
            for (int kst = 0; kst < 4; ++kst) {
                u32x4 w;
                for (int j = 0; j < 4; ++j) w[j] = E::pack2(p[8 * kst + 2 * j], p[8 * kst + 2 * j + 1]);
                pb[kst] = __builtin_bit_cast(vec8, w);
            }
#pragma unroll
            for (int kst = 0; kst < 4; ++kst) {
#pragma unroll
                for (int dblk = 0; dblk < 4; ++dblk) {
                    const int c = 4 * dblk + v_c_lo;
                    const int r0 = 16 * kst + 8 * hi + v_sub;
                    const int r1 = r0 + 4;
                    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        LDS_PTR(s16x4, vs_ + r0 * 256 + ((c ^ v_swz(r0)) << 4) + v_byte));
                    const s16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        LDS_PTR(s16x4, vs_ + r1 * 256 + ((c ^ v_swz(r1)) << 4) + v_byte));
                    const vec8 va = __builtin_bit_cast(vec8, __builtin_shufflevector(lo, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
                    o[dblk] = E::mfma(va, pb[kst], o[dblk]);
                }
            }
        }

        if (ROPE && has_next) rope_store(nK);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    };
    for (int t = 0; t < n_tiles; t += 2) {
        step(t, sK0, sV0, sK1, sV1);
        if (t + 1 < n_tiles) step(t + 1, sK1, sV1, sK0, sV0);
    }

    // ---- epilogue: O / l -> dst[b][q][h][:] (F32) ---------------------------
    const float l_run = pair_sum(l_half);
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
