// kd_mm_kernel.hip - gfx950 kernels of the CrossDiT linear layers
// (ops::linear, src/core/ops.hpp:27-43: ggml_mul_mat(w, x) + bias):
//
//   dequant_kernel  expands Q4_0 / Q8_0 / F16 / F32 weight rows to BF16,
//                   one 32-element block per thread, in the F32 arithmetic
//                   of ggml's dequantize_row_q4_0 / _q8_0
//   mm_bf16         dst[m][n] = sum_k w[n][k] x[m][k] (+ bias[n]) on
//                   v_mfma_f32_32x32x16_bf16, F32 accumulation
//
// The product computes D^T = W X^T: A = W (outputs on M), B = X^T (tokens
// on N), so that each lane ends with 4 consecutive outputs of one token --
// 16-byte pieces of a dst row.  Both operands are k-contiguous rows, which
// is exactly the MFMA operand form (A: lane l holds row l%32, k 8*(l/32)..
// +7; B: column l%32, the same k) -- no transposes anywhere.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/kd_mm.h"
#include "kd_fa_device.h"
#include "kd_mm_kernel.h"

namespace kdfa {

// ---------------------------------------------------------------------------
// dequant_kernel: weight rows -> BF16 rows (F32 value, then round to
// nearest even).  Q8_0 block: F16 d, 32 x int8 q; value = q * d.  Q4_0
// block: F16 d, 16 bytes whose low nibble is element j and high nibble
// element j + 16; value = (nibble - 8) * d (convert_to_gguf.py:121-123 and
// ggml's dequantize_row_q4_0 use this layout).  Blocks are 2-byte aligned
// (34 and 18 bytes), so they are read 16 bits at a time.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dequant_kernel(DqArgs a) {
    const int nbk = a.K / 32;
    const int64_t n_blocks = (int64_t)a.N * nbk;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_blocks;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int n = (int)(i / nbk);
        const int blk = (int)(i % nbk);
        const char *row = a.w + (int64_t)n * a.w_nb1;
        float v[32];
        if (a.type == KD_MM_TYPE_Q8_0 || a.type == KD_MM_TYPE_Q4_0) {
            const int bsize = a.type == KD_MM_TYPE_Q8_0 ? 34 : 18;
            const uint16_t *b16 = reinterpret_cast<const uint16_t *>(row + (int64_t)blk * bsize);
            const float d = (float)__builtin_bit_cast(_Float16, b16[0]);
            if (a.type == KD_MM_TYPE_Q8_0) {
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const uint16_t w = b16[1 + j];
                    v[2 * j] = (float)(int8_t)(w & 0xff) * d;
                    v[2 * j + 1] = (float)(int8_t)(w >> 8) * d;
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint16_t w = b16[1 + j];
                    const int b0 = w & 0xff, b1 = w >> 8;
                    v[2 * j] = (float)((b0 & 15) - 8) * d;
                    v[2 * j + 16] = (float)((b0 >> 4) - 8) * d;
                    v[2 * j + 1] = (float)((b1 & 15) - 8) * d;
                    v[2 * j + 17] = (float)((b1 >> 4) - 8) * d;
                }
            }
        } else if (a.type == KD_MM_TYPE_F16) {
            const f16x8 *p = reinterpret_cast<const f16x8 *>(row + (int64_t)blk * 64);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const f16x8 h = p[c];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[8 * c + e] = (float)h[e];
            }
        } else if (a.type == KD_MM_TYPE_BF16) {
            const u32x4 *p = reinterpret_cast<const u32x4 *>(row + (int64_t)blk * 64);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const u32x4 w = p[c];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[8 * c + 2 * e] = Elem<__bf16>::lo(w[e]);
                    v[8 * c + 2 * e + 1] = Elem<__bf16>::hi(w[e]);
                }
            }
        } else {   // F32
            const f32x4 *p = reinterpret_cast<const f32x4 *>(row + (int64_t)blk * 128);
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const f32x4 f = p[c];
                v[4 * c] = f.x; v[4 * c + 1] = f.y; v[4 * c + 2] = f.z; v[4 * c + 3] = f.w;
            }
        }
        u32x4 *o = reinterpret_cast<u32x4 *>(a.out + (int64_t)n * a.out_nb1 + (int64_t)blk * 64);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            u32x4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] = Elem<__bf16>::pack2(v[8 * c + 2 * e], v[8 * c + 2 * e + 1]);
            o[c] = w;
        }
    }
}

hipError_t launch_dequant(const DqArgs &a, hipStream_t s) {
    const int64_t n_blocks = (int64_t)a.N * (a.K / 32);
    const int64_t want = (n_blocks + 255) / 256;
    const int grid = (int)(want < 8192 ? want : 8192);
    hipLaunchKernelGGL(dequant_kernel, dim3(grid > 0 ? grid : 1), dim3(256), 0, s, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// mm_bf16: one workgroup = 4 waves (one per SIMD, 512 registers each) = a
// 256 (outputs) x 256 (tokens) tile of dst; wave w holds the 128 x 128
// quarter (w & 1, w >> 1) as 4 x 4 MFMA accumulator blocks (256 AGPRs).
//
// K advances 32 per stage through S LDS stages (4 with BF16 X, 3 with F32
// X: 128 / 144 KiB), each filled by DMA (global_load_lds_dwordx4) S - 1
// stages ahead of its use:
//   W stage: 256 rows x 64 bytes (BF16); 16-byte chunk c of row r at
//            c ^ ((r >> 2) & 3)
//   X stage: 256 rows x 128 bytes (F32) or 64 bytes (BF16); chunk c of row
//            r at c ^ ((r >> 1) & 7) (F32) or c ^ ((r >> 2) & 3) (BF16)
// -- so that the 16 rows one 16-lane group of an operand read touches fill
// the 256 bytes of the 64 banks exactly once.  F32 X is rounded to BF16
// next to the MFMAs that use its fragments.  Per stage a wave reads 8 W and
// 8 X fragments and issues 32 MFMAs, with the DMAs of a later stage spread
// over the first 16; the only barrier is the one that publishes a stage.
// Rows past M or N read clamped (repeated) rows and are not stored; the
// workgroups an XCD runs at once cover 8 token tiles x 4 output tiles, so
// its L2 serves their shared W and X stages.  The output goes through LDS so
// that its stores are whole 128-byte lines.
// ---------------------------------------------------------------------------
constexpr int kMmWaves = 4;
constexpr int kMmWTile = kMmBN * kMmBK * 2;   // 16 KiB

template <bool XF32>
__global__ __launch_bounds__(64 * kMmWaves) __attribute__((amdgpu_waves_per_eu(1, 1)))
void mm_bf16(MmArgs a) {
    typedef Elem<__bf16> E;
    typedef E::vec8 vec8;
    constexpr int kXRow = XF32 ? 128 : 64;               // bytes of one X row per stage
    constexpr int kXTile = kMmBM * kXRow;
    constexpr int kStage = kMmWTile + kXTile;
    constexpr int kThreads = 64 * kMmWaves;
    constexpr int kWRounds = kMmWTile / (kThreads * 16);   // 4
    constexpr int kXRounds = kXTile / (kThreads * 16);     // 8 (F32) or 4
    constexpr int kWRowsPerRound = 1024 / 64;              // 16 rows per wave DMA
    constexpr int kXRowsPerRound = 1024 / kXRow;           // 8 or 16
    constexpr int kS = XF32 ? 3 : 4;                       // LDS stages
    constexpr int kPer = kWRounds + kXRounds;              // DMAs per stage per wave
    __shared__ __attribute__((aligned(1024))) char lds[kS * kStage];
    lds_t *const sbase = LDS_PTR(char, lds);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int hi = lane >> 5;

    // tile: XCD-contiguous runs of tiles, dealt in columns of 4 output tiles
    // (m fastest within a column): the 32 workgroups an XCD runs at once
    // then share 4 W tiles and 8 X tiles in its L2, where n-fastest order
    // (16 W, 2 X) spread them over more (3-8% at the DiT's shapes)
    const int pid = blockIdx.x;
    const int per = a.n_blocks >> 3;
    const int lid = pid < per * 8 ? (pid & 7) * per + (pid >> 3) : pid;
    int nt, mt;
    if (a.tiles_n % 4 == 0) {
        const int col = lid / (a.tiles_m * 4), rem = lid % (a.tiles_m * 4);
        mt = rem / 4;
        nt = col * 4 + rem % 4;
    } else {
        nt = lid % a.tiles_n;
        mt = lid / a.tiles_n;
    }
    const int n0 = nt * kMmBN;
    const int m0 = mt * kMmBM;

    // DMA lane offsets, relative to the tile's first row (the stage base
    // moves by 64 / kXRow bytes per stage)
    uint32_t w_off[kWRounds], x_off[kXRounds];
#pragma unroll
    for (int j = 0; j < kWRounds; ++j) {
        const int r = kWRowsPerRound * (wave + kMmWaves * j) + (lane >> 2);
        const int c = (lane & 3) ^ ((r >> 2) & 3);
        const int rr = n0 + r < a.N ? r : a.N - 1 - n0;
        w_off[j] = (uint32_t)rr * (uint32_t)a.w_nb1 + (uint32_t)(c << 4);
    }
#pragma unroll
    for (int j = 0; j < kXRounds; ++j) {
        const int r = kXRowsPerRound * (wave + kMmWaves * j) + (XF32 ? (lane >> 3) : (lane >> 2));
        const int c = XF32 ? ((lane & 7) ^ ((r >> 1) & 7)) : ((lane & 3) ^ ((r >> 2) & 3));
        const int rr = m0 + r < a.M ? r : a.M - 1 - m0;
        x_off[j] = (uint32_t)rr * (uint32_t)a.x_nb1 + (uint32_t)(c << 4);
    }
    const char *const wtile = a.w + (int64_t)n0 * a.w_nb1;
    const char *const xtile = a.x + (int64_t)m0 * a.x_nb1;
    // DMA j (of kPer) of stage kt into LDS stage buffer st: W rounds first
    auto dma_j = [&](int kt, int st, int j) __attribute__((always_inline)) {
        lds_t *sw = sbase + st * kStage;
        if (j < kWRounds)
            dma16(wtile + kt * 64, w_off[j], sw + (wave + kMmWaves * j) * 1024);
        else
            dma16(xtile + kt * kXRow, x_off[j - kWRounds], sw + kMmWTile + (wave + kMmWaves * (j - kWRounds)) * 1024);
    };
    auto issue = [&](int kt, int st) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < kPer; ++j) dma_j(kt, st, j);
    };

    // fragment read offsets within a stage (the row part of the swizzle is
    // l32's, since every block starts at a multiple of 32 rows)
    const int wn = wave & 1;
    const int wm = wave >> 1;
    uint32_t a_rd[2], b_rd[2][2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        a_rd[ks] = (uint32_t)((128 * wn + l32) * 64 + (((2 * ks + hi) ^ ((l32 >> 2) & 3)) << 4));
        if (XF32) {
            b_rd[ks][0] = (uint32_t)(kMmWTile + (128 * wm + l32) * 128 + (((4 * ks + 2 * hi) ^ ((l32 >> 1) & 7)) << 4));
            b_rd[ks][1] = (uint32_t)(kMmWTile + (128 * wm + l32) * 128 + (((4 * ks + 2 * hi + 1) ^ ((l32 >> 1) & 7)) << 4));
        } else {
            b_rd[ks][0] = (uint32_t)(kMmWTile + (128 * wm + l32) * 64 + (((2 * ks + hi) ^ ((l32 >> 2) & 3)) << 4));
            b_rd[ks][1] = 0;
        }
    }

    f32x16 acc[4][4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) acc[nb][mb] = (f32x16){};

    // operand fragments, two sets: the reads of one k-step are issued before
    // the 16 MFMAs of the previous one, so their LDS latency hides behind
    // 512 cycles of matrix work instead of stalling each group of four.  F32
    // X fragments are kept as read and rounded to BF16 next to the products
    // that use them, so that no rounding waits on a read just issued.
    struct XFragBf16 { vec8 b[4]; };
    struct XFragF32 { f32x4 u[4], v[4]; };
    typedef typename std::conditional<XF32, XFragF32, XFragBf16>::type XFrag;
    vec8 fa0[4], fa1[4];
    XFrag fb0, fb1;
    auto read = [&](int st, int ks, vec8 fa[4], XFrag &fb) __attribute__((always_inline)) {
        const lds_t *s = sbase + st * kStage;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
            fa[nb] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(s + a_rd[ks] + nb * 32 * 64);
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
            if constexpr (XF32) {
                fb.u[mb] = *reinterpret_cast<const __attribute__((address_space(3))) f32x4 *>(s + b_rd[ks][0] + mb * 32 * 128);
                fb.v[mb] = *reinterpret_cast<const __attribute__((address_space(3))) f32x4 *>(s + b_rd[ks][1] + mb * 32 * 128);
            } else {
                fb.b[mb] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(s + b_rd[ks][0] + mb * 32 * 64);
            }
        }
    };
    // the 16 MFMAs of one k-step; with dma, the DMAs of stage dkt (into
    // buffer dst) spread over them, one group after every two MFMAs, so that
    // their data does not reach the LDS in one burst that holds up the
    // fragment reads (5-10% over issuing a stage's DMAs together)
    auto mfmas = [&](const vec8 fa[4], const XFrag &fb, bool dma, int dkt, int dst) __attribute__((always_inline)) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
            vec8 b;
            if constexpr (XF32) {
                const f32x4 u = fb.u[mb], v = fb.v[mb];
                const u32x4 w = {E::pack2(u.x, u.y), E::pack2(u.z, u.w), E::pack2(v.x, v.y), E::pack2(v.z, v.w)};
                b = __builtin_bit_cast(vec8, w);
            } else {
                b = fb.b[mb];
            }
#pragma unroll
            for (int hp = 0; hp < 2; ++hp) {
#pragma unroll
                for (int nb = 2 * hp; nb < 2 * hp + 2; ++nb) acc[nb][mb] = E::mfma(fa[nb], b, acc[nb][mb]);
                __builtin_amdgcn_sched_barrier(0);
                if (dma) {
#pragma unroll
                    for (int j = 0; j < kPer; ++j)
                        if (j * 8 / kPer == 2 * mb + hp) dma_j(dkt, dst, j);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    // a stage is complete in LDS for every wave: this wave's DMAs of it have
    // landed (the `later` stages issued after it may be in flight; DMAs
    // complete in issue order), then the barrier
    auto publish = [&](int later) __attribute__((always_inline)) {
        static_assert(3 * kPer <= 63, "vmcnt range");
        if (later >= 3)
            asm volatile("s_waitcnt vmcnt(%0)" :: "n"(3 * kPer) : "memory");
        else if (later == 2)
            asm volatile("s_waitcnt vmcnt(%0)" :: "n"(2 * kPer) : "memory");
        else if (later == 1)
            asm volatile("s_waitcnt vmcnt(%0)" :: "n"(kPer) : "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    };

    // Step kt (stage st = kt % S): 16 MFMAs of k-step 0 while the fragments
    // of k-step 1 load, the DMAs of stage kt+S-1 spread over them; publish
    // stage kt+1 (its DMAs landed, later stages' may be in flight); 16 MFMAs
    // of k-step 1 while the fragments of stage kt+1's k-step 0 load.
    constexpr int kLead = kS - 1;
    const int nk = a.K / kMmBK;
#pragma unroll
    for (int j = 0; j < kLead; ++j)
        if (j < nk) issue(j, j);
    publish(min(kLead, nk) - 1);
    read(0, 0, fa0, fb0);
    int st = 0;
    // The last step is peeled so that every step of the loop issues the same
    // LDS reads (a read under a branch makes the wait counts conservative);
    // sched_barrier keeps the compiler from moving reads next to their uses.
    for (int kt = 0; kt + 1 < nk; ++kt) {
        const int st1 = st == kS - 1 ? 0 : st + 1;
        // stage kt+S-1 goes into the buffer of stage kt-1, whose reads all
        // completed before the previous barrier (its fence drains them)
        read(st, 1, fa1, fb1);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(fa0, fb0, kt + kLead < nk, kt + kLead, st == 0 ? kS - 1 : st - 1);
        __builtin_amdgcn_sched_barrier(0);
        publish(min(kLead, nk - 1 - kt) - 1);
        read(st1, 0, fa0, fb0);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(fa1, fb1, false, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        st = st1;
    }
    read(st, 1, fa1, fb1);
    __builtin_amdgcn_sched_barrier(0);
    mfmas(fa0, fb0, false, 0, 0);
    mfmas(fa1, fb1, false, 0, 0);
    static_assert(kPer == (XF32 ? 12 : 8), "per-stage DMA count");

    // ---- epilogue: dst[m][n .. n+3] = acc (+ bias) ----------------------------
    // Through LDS, one 32-output block (128 bytes of each of the wave's 128
    // token rows) at a time: the lanes leave their 16-byte pieces in the
    // wave's own 16 KiB (chunk index XOR (row >> 1) & 7: no bank conflicts),
    // then lane L reads chunk L % 8 of row 8j + L / 8, so that every store
    // instruction writes eight whole 128-byte lines of dst instead of
    // 32-byte pieces of 32 rows, as streaming (nontemporal) stores: dst is
    // not read again here (1%).  The stage buffers are free once every wave
    // is past its last read; after that a wave touches only its own region
    // (its LDS operations complete in order).
    __syncthreads();
    lds_t *const sO = sbase + wave * 32768;
    const int rr = lane >> 3;
    const int rc = lane & 7;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
        lds_t *const so = sO + (nb & 1) * 16384;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
            const int row = 32 * mb + l32;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 v = {acc[nb][mb][4 * g], acc[nb][mb][4 * g + 1], acc[nb][mb][4 * g + 2],
                                 acc[nb][mb][4 * g + 3]};
                *reinterpret_cast<__attribute__((address_space(3))) f32x4 *>(
                    so + row * 128 + (((2 * g + hi) ^ ((row >> 1) & 7)) << 4)) = v;
            }
        }
        const int n = n0 + 128 * wn + 32 * nb + 4 * rc;
        f32x4 bias = {0.f, 0.f, 0.f, 0.f};
        if (a.bias && n < a.N) bias = *reinterpret_cast<const f32x4 *>(a.bias + n);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int row = 8 * j + rr;
            f32x4 v = *reinterpret_cast<const __attribute__((address_space(3))) f32x4 *>(
                so + row * 128 + ((rc ^ ((row >> 1) & 7)) << 4));
            const int m = m0 + 128 * wm + row;
            if (m < a.M && n < a.N) {
                v.x += bias.x; v.y += bias.y; v.z += bias.z; v.w += bias.w;
                __builtin_nontemporal_store(v, reinterpret_cast<f32x4 *>(a.dst + (int64_t)m * a.d_nb1 + (int64_t)n * 4));
            }
        }
    }
}

hipError_t launch_mm(const MmArgs &a, bool x_f32, hipStream_t s) {
    if (x_f32)
        hipLaunchKernelGGL(mm_bf16<true>, dim3(a.n_blocks), dim3(64 * kMmWaves), 0, s, a);
    else
        hipLaunchKernelGGL(mm_bf16<false>, dim3(a.n_blocks), dim3(64 * kMmWaves), 0, s, a);
    return hipGetLastError();
}

}  // namespace kdfa
