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
// (MFMA operand layouts: kd_fa_device.h.)
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

#include "kd_fa_device.h"

namespace kdfa {


constexpr int kBN = 64;                             // keys per tile
constexpr int kTileBytes = kBN * kD * 2;            // one K or V tile

// Instruction order of one S^T product for the scheduler: PRE pairs of K
// fragment reads ahead, then per k-step two MFMAs and the next pair of reads.
// (sched_group_barrier masks: 0x008 MFMA, 0x100 DS read.)
template <int KS, int PRE> __device__ __forceinline__ void sched_qk_step() {
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    if constexpr (KS + PRE < 8) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
}
template <int PRE> __device__ __forceinline__ void sched_qk() {
    for (int i = 0; i < PRE; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    sched_qk_step<0, PRE>(); sched_qk_step<1, PRE>(); sched_qk_step<2, PRE>(); sched_qk_step<3, PRE>();
    sched_qk_step<4, PRE>(); sched_qk_step<5, PRE>(); sched_qk_step<6, PRE>(); sched_qk_step<7, PRE>();
}

// Instruction order of the pipelined step's first half: the S^T product of
// the next tile (16 MFMA, 16 K-fragment reads) with the softmax of the
// current tile spread between its MFMAs, VPM VALU instructions after each.
// (0x402: VALU or transcendental.)
template <int KS, int PRE, int VPM> __device__ __forceinline__ void sched_pipe_step() {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x402, VPM, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x402, VPM, 0);
    if constexpr (KS + PRE < 8) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
}
template <int PRE, int VPM> __device__ __forceinline__ void sched_pipe() {
    for (int i = 0; i < PRE; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    sched_pipe_step<0, PRE, VPM>(); sched_pipe_step<1, PRE, VPM>(); sched_pipe_step<2, PRE, VPM>();
    sched_pipe_step<3, PRE, VPM>(); sched_pipe_step<4, PRE, VPM>(); sched_pipe_step<5, PRE, VPM>();
    sched_pipe_step<6, PRE, VPM>(); sched_pipe_step<7, PRE, VPM>();
}

// K-fragment prefetch distance (k-steps ahead of their MFMAs) of the
// kernels that stream K by DMA, and the VALU instructions placed after each
// MFMA of the pipelined step (sched_pipe).  The kernel that transforms K
// tiles on load holds more registers and reads its fragments with no
// prefetch and no explicit interleave.
constexpr int kKPreDma = 2;
constexpr int kPipeVpm = 6;

// Q fragments of query row q_ld (B operands of S^T = K Q^T, k-steps of 16):
// this lane holds elements ks*16 + hi*8 .. +7 of each k-step; the lane
// l ^ 32 the other half.  RMSNorm (qn_w) and RoPE (RM) are applied in F32
// first; scale < 0 negates Q (exact) so that every score is s * |scale|.
// Every load of the row is issued before any is used, unconditionally, so
// the row costs one memory round trip (a branch on Q's type per chunk put
// each chunk's load and its wait in a block of its own): two 16-byte loads
// per 8-element chunk, both halves of an F32 chunk or the 16-bit chunk
// twice, and the values chosen by the type afterwards.  TABS: the rotation
// table's pairs and the norm weights are loaded up front too (64 registers
// each; where the registers are free), else per chunk.  !QUP: Q too is
// loaded per chunk (for the kernel that rotates K tiles on load, whose
// registers are short).
template <typename T, int RM, bool TABS = false, bool QUP = true>
__device__ __forceinline__ void load_q_frags(const Args &a, int q_ld, int h, int b, int hi,
                                             typename Elem<T>::vec8 qf[8]) {
    typedef Elem<T> E;
    typedef typename E::vec8 vec8;
    constexpr bool ROPE = RM != KD_FA_ROPE_NONE;
    const char *qp = a.q + (int64_t)q_ld * a.q_nb1 + (int64_t)h * a.q_nb2 + (int64_t)b * a.q_nb3;
    const bool q32 = a.q_type == KD_FA_TYPE_F32;
    const bool q_bf16 = a.q_type == KD_FA_TYPE_BF16;
    u32x4 ra[QUP ? 8 : 1], rb[QUP ? 8 : 1];
    if constexpr (QUP) {
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const int d0 = ks * 16 + hi * 8;
            ra[ks] = ld16(qp + (q32 ? d0 * 4 : d0 * 2));
            rb[ks] = ld16(qp + (q32 ? d0 * 4 + 16 : d0 * 2));
        }
    }
    // the rotation's (cos, sin) pairs and the norm weights
    f32x4 rc[ROPE && TABS ? 16 : 1];
    if constexpr (ROPE && TABS) {
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const float *cp = rope_ptr<RM>(a, q_ld, ks * 16 + hi * 8);
            rc[2 * ks] = *reinterpret_cast<const f32x4 *>(cp);
            rc[2 * ks + 1] = *reinterpret_cast<const f32x4 *>(cp + 4);
        }
    }
    const bool qnorm = a.qn_w != nullptr;
    f32x4 wn[TABS ? 16 : 1];
    if (TABS && qnorm) {
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            wn[2 * ks] = *reinterpret_cast<const f32x4 *>(a.qn_w + ks * 16 + hi * 8);
            wn[2 * ks + 1] = *reinterpret_cast<const f32x4 *>(a.qn_w + ks * 16 + hi * 8 + 4);
        }
    }
    auto elems = [&](int ks, float x[8]) __attribute__((always_inline)) {
        if constexpr (!QUP) {
            load8_f32(qp + (ks * 16 + hi * 8) * (q32 ? 4 : 2), a.q_type, x);
            return;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t w16 = ra[ks][j];
            const float lo16 = q_bf16 ? bf16_lo(w16) : f16_lo(w16);
            const float hi16 = q_bf16 ? bf16_hi(w16) : f16_hi(w16);
            // F32: elements 0-3 from the first load, 4-7 from the second
            const float e0 = __uint_as_float(j < 2 ? ra[ks][2 * j] : rb[ks][2 * j - 4]);
            const float e1 = __uint_as_float(j < 2 ? ra[ks][2 * j + 1] : rb[ks][2 * j - 3]);
            x[2 * j] = q32 ? e0 : lo16;
            x[2 * j + 1] = q32 ? e1 : hi16;
        }
    };
    // RMSNorm of the row (query_norm): this lane holds 64 of its 128
    // elements, the lane l ^ 32 the rest
    float qscale = 1.0f;
    if (qnorm) {
        double ss = 0.0;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            float x[8];
            elems(ks, x);
            ss += sum_sq8(x);
        }
        qscale = rms_scale(pair_sum_f64(ss), a.norm_eps);
    }
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
        float x[8];
        elems(ks, x);
        const int d0 = ks * 16 + hi * 8;
        if (qnorm) {
            if constexpr (TABS)
                rms_apply8(x, qscale, wn[2 * ks], wn[2 * ks + 1]);
            else
                rms_apply8(x, qscale, *reinterpret_cast<const f32x4 *>(a.qn_w + d0),
                           *reinterpret_cast<const f32x4 *>(a.qn_w + d0 + 4));
        }
        if constexpr (ROPE) {
            if constexpr (TABS) {
                rotate8(x, rc[2 * ks], rc[2 * ks + 1]);
            } else {
                const float *cp = rope_ptr<RM>(a, q_ld, d0);
                rotate8(x, *reinterpret_cast<const f32x4 *>(cp), *reinterpret_cast<const f32x4 *>(cp + 4));
            }
        }
        u32x4 w;
        for (int j = 0; j < 4; ++j) w[j] = E::pack2(x[2 * j], x[2 * j + 1]);
        if (a.scale_log2 < 0.0f) w ^= (u32x4){0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
        qf[ks] = __builtin_bit_cast(vec8, w);
    }
}

__device__ __forceinline__ void store_o_row(const Args &a, int q_row, int h, int b, int hi, const f32x16 o[4],
                                            float l_half) {
    store_o_row_l(a, q_row, h, b, hi, o, pair_sum(l_half), 0);
}

template <typename T, bool HAS_MASK, int RM, bool KROPE, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2)))
void fa_fwd_d128(Args a) {
    constexpr bool ROPE = RM != KD_FA_ROPE_NONE;   // rotate Q on load
    constexpr bool KR = KROPE;                      // transform K tiles on load
    constexpr int kWaves = NW;
    constexpr int kThreads = 64 * kWaves;
    constexpr int kBM = 32 * kWaves;                // query rows per workgroup
    constexpr int kRounds = kTileBytes / (kThreads * 16);  // 16-byte DMA rounds per thread per tile
    static_assert(kRounds * kThreads * 16 == kTileBytes, "tile shape");
    typedef Elem<T> E;
    typedef typename E::vec8 vec8;
    // four distinct LDS objects (not one array) so that the compiler can
    // tell the tile being computed from the tile the DMA is filling
    __shared__ __attribute__((aligned(1024))) char lK0[kTileBytes];
    __shared__ __attribute__((aligned(1024))) char lK1[kTileBytes];
    __shared__ __attribute__((aligned(1024))) char lV0[kTileBytes];
    __shared__ __attribute__((aligned(1024))) char lV1[kTileBytes];
    lds_t *const sK0 = LDS_PTR(char, lK0), *const sK1 = LDS_PTR(char, lK1);
    lds_t *const sV0 = LDS_PTR(char, lV0), *const sV1 = LDS_PTR(char, lV1);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: SGPR
    const int l32 = lane & 31;
    const int hi = lane >> 5;

    // Workgroups are dealt to the 8 XCDs round-robin; give each XCD a
    // contiguous range of (b, h, q-tile) so the tiles of one head share
    // that XCD's L2.
    const int pid = blockIdx.x;
    const int per = a.n_blocks >> 3;
    const int lid = pid < per * 8 ? (pid & 7) * per + (pid >> 3) : pid;
    // Logical order: the q-tiles of one head in a row (they share K and V),
    // or, for a mask shared by all heads, the heads of one q-tile in a row
    // (they share the mask tile).
    int qt, h, b;
    if (a.heads_inner) {
        h = lid % a.H;
        const int r = lid / a.H;
        qt = r % a.n_qt;
        b = r / a.n_qt;
    } else {
        qt = lid % a.n_qt;
        const int bh = lid / a.n_qt;
        h = bh % a.H;
        b = bh / a.H;
    }

    const char *kbase = a.k + (int64_t)(h / a.rk2) * a.k_nb2 + (int64_t)(b / a.rk3) * a.k_nb3;
    const char *vbase = a.v + (int64_t)(h / a.rv2) * a.v_nb2 + (int64_t)(b / a.rv3) * a.v_nb3;
    const int Lk = a.Lk;

    // ---- Q fragment (B operand of S^T): row q_row, k-steps of 16 -----------
    const int q_row = qt * kBM + wave * 32 + l32;
    const int q_ld = q_row < a.Lq ? q_row : a.Lq - 1;
    vec8 qf[8];
    load_q_frags<T, RM, false, !KR>(a, q_ld, h, b, hi, qf);

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
    // covers rows 4*(w + kWaves*j) .. +3, j < kRounds, for K and for V.  The source
    // is a uniform tile base plus a fixed per-lane offset; only a partial
    // last tile clamps its rows to Lk - 1.
    const int dma_row = lane >> 4;        // row within the wave's 4 rows
    const int dma_pc = lane & 15;         // physical chunk this lane fills
    uint32_t k_dma[kRounds], v_dma[kRounds];
#pragma unroll
    for (int j = 0; j < kRounds; ++j) {
        const int r = 4 * (wave + kWaves * j) + dma_row;
        v_dma[j] = (uint32_t)r * (uint32_t)a.v_nb1 + ((dma_pc ^ v_swz(r)) << 4);
        k_dma[j] = (uint32_t)k_row_of(r) * (uint32_t)a.k_nb1 + ((dma_pc ^ (r & 15)) << 4);
    }
    auto issue_v = [&](int t, lds_t *dV) __attribute__((always_inline)) {
        const char *vt = vbase + (int64_t)t * kBN * a.v_nb1;
        if ((t + 1) * kBN <= Lk) {
            // round j covers rows 4*kWaves*j + (row of round 0): only the
            // uniform base moves
#pragma unroll
            for (int j = 0; j < kRounds; ++j)
                dma16(vt + (int64_t)j * 4 * kWaves * a.v_nb1, v_dma[0], dV + (wave + kWaves * j) * 1024);
        } else {
#pragma unroll
            for (int j = 0; j < kRounds; ++j) {
                const int r = 4 * (wave + kWaves * j) + dma_row;
                const int vr = t * kBN + r < Lk ? r : Lk - 1 - t * kBN;
                dma16(vt, (uint32_t)vr * (uint32_t)a.v_nb1 + ((dma_pc ^ v_swz(r)) << 4),
                      dV + (wave + kWaves * j) * 1024);
            }
        }
    };
    auto issue_k = [&](int t, lds_t *dK) __attribute__((always_inline)) {   // K without RoPE
        const char *kt = kbase + (int64_t)t * kBN * a.k_nb1;
        if ((t + 1) * kBN <= Lk) {
#pragma unroll
            for (int j = 0; j < kRounds; ++j)
                dma16(kt + (int64_t)j * 4 * kWaves * a.k_nb1, k_dma[0], dK + (wave + kWaves * j) * 1024);
        } else {
#pragma unroll
            for (int j = 0; j < kRounds; ++j) {
                const int r = 4 * (wave + kWaves * j) + dma_row;
                const int kr = t * kBN + k_row_of(r) < Lk ? k_row_of(r) : Lk - 1 - t * kBN;
                dma16(kt, (uint32_t)kr * (uint32_t)a.k_nb1 + ((dma_pc ^ (r & 15)) << 4),
                      dK + (wave + kWaves * j) * 1024);
            }
        }
    };
    auto issue_tile = [&](int t, lds_t *dK, lds_t *dV) __attribute__((always_inline)) {
        issue_v(t, dV);
        if (!KR) issue_k(t, dK);
    };
    // RoPE: K chunk u = tid + kThreads*j -> LDS row u/16, physical chunk
    // u%16 -- the same rows and chunks as the DMA lanes, so the K source
    // offsets are k_dma[]; TABLE mode reads the table row of the same key.
    u32x4 kreg[kRounds];
    f32x4 kcs[kRounds][2];
    uint32_t tab_off[kRounds];
#pragma unroll
    for (int j = 0; j < kRounds; ++j) {
        const int r = 4 * (wave + kWaves * j) + dma_row;
        tab_off[j] = (uint32_t)k_row_of(r) * (uint32_t)a.rope_nb1 + (((dma_pc ^ (r & 15)) << 5));
    }
    auto rope_load = [&](int t) __attribute__((always_inline)) {
        const char *kt = kbase + (int64_t)t * kBN * a.k_nb1;
        const bool full = (t + 1) * kBN <= Lk;
#pragma unroll
        for (int j = 0; j < kRounds; ++j) {
            const int r = 4 * (wave + kWaves * j) + dma_row;
            const int c = dma_pc ^ (r & 15);
            int kr = k_row_of(r);
            if (!full && t * kBN + kr >= Lk) kr = Lk - 1 - t * kBN;
            if (RM == KD_FA_ROPE_NONE) {
                kreg[j] = ld16(kt + (full ? k_dma[j] : (uint32_t)kr * (uint32_t)a.k_nb1 + (c << 4)));
            } else if (RM == KD_FA_ROPE_TABLE) {
                const char *tt = reinterpret_cast<const char *>(a.rope_tab) + (int64_t)t * kBN * a.rope_nb1;
                const uint32_t ko = full ? k_dma[j] : (uint32_t)kr * (uint32_t)a.k_nb1 + (c << 4);
                const uint32_t to = full ? tab_off[j] : (uint32_t)kr * (uint32_t)a.rope_nb1 + (c << 5);
                kreg[j] = ld16(kt + ko);
                kcs[j][0] = *reinterpret_cast<const f32x4 *>(tt + to);
                kcs[j][1] = *reinterpret_cast<const f32x4 *>(tt + to + 16);
            } else {
                kreg[j] = ld16(kt + ((uint32_t)kr * (uint32_t)a.k_nb1 + (c << 4)));
                const float *cp = rope_ptr<RM>(a, t * kBN + kr, c * 8);
                kcs[j][0] = *reinterpret_cast<const f32x4 *>(cp);
                kcs[j][1] = *reinterpret_cast<const f32x4 *>(cp + 4);
            }
        }
    };
    // key_norm weights of this lane's chunk (the chunk a lane handles is the
    // same in every round: the row's low four bits do not change)
    f32x4 kw0 = {}, kw1 = {};
    if (KR && a.kn_w) {
        const int c = dma_pc ^ ((4 * wave + dma_row) & 15);
        kw0 = *reinterpret_cast<const f32x4 *>(a.kn_w + c * 8);
        kw1 = *reinterpret_cast<const f32x4 *>(a.kn_w + c * 8 + 4);
    }
    auto rope_store = [&](lds_t *dK) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < kRounds; ++j) {
            const int u = tid + kThreads * j;
            float x[8];
            for (int e = 0; e < 4; ++e) { x[2 * e] = E::lo(kreg[j][e]); x[2 * e + 1] = E::hi(kreg[j][e]); }
            // RMSNorm: the 16 lanes of a 16-lane group hold the 16 chunks of one row
            if (a.kn_w) rms_apply8(x, rms_scale(sum16_f64(sum_sq8(x)), a.norm_eps), kw0, kw1);
            if (ROPE) rotate8(x, kcs[j][0], kcs[j][1]);
            u32x4 w;
            for (int e = 0; e < 4; ++e) w[e] = E::pack2(x[2 * e], x[2 * e + 1]);
            *reinterpret_cast<__attribute__((address_space(3))) u32x4 *>(dK + u * 16) = w;
        }
    };

    // mask values of this lane's 32 keys (key 16*hh + 8*hi + e of 32-key
    // block mb at index mb*16 + hh*8 + e), prefetched one tile ahead
    u32x4 mraw[4];
    auto mask_load = [&](int t) __attribute__((always_inline)) {
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

    const float c2 = __builtin_fabsf(a.scale_log2);
    // K-operand LDS offsets of this lane, one per 16-wide k-step (rows l32
    // and 32 + l32 share the swizzle)
    uint32_t k_rd[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) k_rd[ks] = l32 * 256 + (((2 * ks + hi) ^ (lane & 15)) << 4);
    // V-operand (ds_read_b64_tr_b16) LDS offsets of this lane, one per
    // 32-wide d block: row 16*kst + 8*hi + v_sub (+4), chunk 4*dblk + v_c_lo;
    // the swizzle depends on the row only through v_sub
    const int v_sub = (lane & 15) >> 2;
    const int v_c_lo = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
    uint32_t v_rd[4];
#pragma unroll
    for (int dblk = 0; dblk < 4; ++dblk)
        v_rd[dblk] = 2048 * hi + 256 * v_sub + (((4 * dblk + v_c_lo) ^ v_swz(v_sub)) << 4) + 8 * (lane & 1);

    // ---- S^T = K Q^T for one 64-key tile ---------------------------------------
    // K fragments are read kKPre k-steps ahead of the MFMAs that use them,
    // so that LDS latency overlaps the products instead of stalling each
    // pair of them
    auto qk = [&](const lds_t *ks_, f32x16 &s0, f32x16 &s1) __attribute__((always_inline)) {
        constexpr int kKPre = KR ? 0 : kKPreDma;
        s0 = (f32x16){};
        s1 = (f32x16){};
        vec8 ka[8][2];
#pragma unroll
        for (int ks = 0; ks < kKPre; ++ks) {
            ka[ks][0] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(ks_ + k_rd[ks]);
            ka[ks][1] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(ks_ + k_rd[ks] + 32 * 256);
        }
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            if (ks + kKPre < 8) {
                ka[ks + kKPre][0] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(ks_ + k_rd[ks + kKPre]);
                ka[ks + kKPre][1] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(ks_ + k_rd[ks + kKPre] + 32 * 256);
            }
            s0 = E::mfma(ka[ks][0], qf[ks], s0);
            s1 = E::mfma(ka[ks][1], qf[ks], s1);
        }
        if constexpr (!KR) sched_qk<kKPre>();
    };

    // the running max of a row moves to mx when `up` (a decision per row, so
    // that every row's result depends on its own scores only: the ballot
    // just skips the rescale when no row of the wave moves); O and the sums
    // of a moved row are rescaled.  Masked rows move when the tile max
    // exceeds the running max by more than kTau, unmasked rows when their
    // own weight sum left [0, E::kSumCap].
    auto move_max = [&](float mx, bool up) __attribute__((always_inline)) {
        if (__builtin_amdgcn_ballot_w64(up) != 0) {
            const float m_new = up ? __builtin_fmaxf(m_run, mx) : m_run;
            const float alpha = m_new == m_run ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
            l_half *= alpha;
#pragma unroll
            for (int dblk = 0; dblk < 4; ++dblk)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[dblk][i] *= alpha;
        }
    };
    auto update_max = [&](float mx) __attribute__((always_inline)) { move_max(mx, mx > m_run + kTau); };

    // P rounded to the operand type (the PV B operands).  The row sum adds the F32 weights (before rounding): each 16-key step's
    // 8 weights of this lane in order, the four steps combined as
    // (s0 + s1) + (s2 + s3).  (Plain adds: a dot2 on the rounded pairs would
    // stall the matrix pipe.)
    auto pack_sum = [&](const float *p, vec8 pb[4]) -> float {
        float part[4];
#pragma unroll
        for (int kst = 0; kst < 4; ++kst) {
            u32x4 w;
            for (int j = 0; j < 4; ++j) w[j] = E::pack2(p[8 * kst + 2 * j], p[8 * kst + 2 * j + 1]);
            part[kst] = p[8 * kst] + p[8 * kst + 1];
            for (int i = 2; i < 8; ++i) part[kst] += p[8 * kst + i];
            pb[kst] = __builtin_bit_cast(vec8, w);
        }
        return (part[0] + part[1]) + (part[2] + part[3]);
    };
    auto pack_p = [&](const float *p, vec8 pb[4]) __attribute__((always_inline)) { l_half += pack_sum(p, pb); };

    // online softmax with the additive mask: logits s*c2 + mask*log2(e);
    // -inf mask entries (and keys past Lk, filled with -inf) stay -inf
    auto softmax_masked = [&](const f32x16 &s0, const f32x16 &s1, const float *mv, vec8 pb[4]) __attribute__((always_inline)) {
        float p[32];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            p[i] = s0[i];
            p[16 + i] = s1[i];
        }
#pragma unroll
        for (int i = 0; i < 32; ++i)
            p[i] = mv[i] == -INFINITY ? -INFINITY : __builtin_fmaf(mv[i], kLog2e, p[i] * c2);
        update_max(pair_max(max32(p)));
        const float mu = m_run == -INFINITY ? 0.0f : m_run;
#pragma unroll
        for (int i = 0; i < 32; ++i) p[i] = __builtin_amdgcn_exp2f(p[i] - mu);
        pack_p(p, pb);
    };

    // ---- O^T += V^T P^T ------------------------------------------------------
    auto pv = [&](const lds_t *vs_, const vec8 pb[4]) __attribute__((always_inline)) {
#pragma unroll
        for (int kst = 0; kst < 4; ++kst) {
#pragma unroll
            for (int dblk = 0; dblk < 4; ++dblk) {
                const lds_t *vp = vs_ + v_rd[dblk] + 4096 * kst;
                const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)(vp));
                const s16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)(vp + 1024));
                const vec8 va = __builtin_bit_cast(vec8, __builtin_shufflevector(lo, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
                o[dblk] = E::mfma(va, pb[kst], o[dblk]);
            }
        }
    };

    auto load_tile_sync = [&](int t, lds_t *dK, lds_t *dV) __attribute__((always_inline)) {
        issue_tile(t, dK, dV);
        if (KR) {
            rope_load(t);
            rope_store(dK);
        }
    };

    const int n_tiles = (Lk + kBN - 1) / kBN;

    // Unmasked softmax of one 64-key step (scores s0, s1 of keys key0 ..
    // key0+63) and O^T += V^T P^T with the V rows at vs_.  The running max
    // m_run is not refreshed every step: the exponents are taken against the
    // current m_run, and only when a row's sum of weights leaves
    // [0, E::kSumCap] (a score far above m_run, or the first step with
    // m_run = -inf) is the step's exact row max computed, O rescaled and the
    // exponents redone.  Weights stay <= E::kSumCap, inside T's finite range
    // once rounded for the PV product.  TAIL: keys past Lk (last tile only) read clamped K rows,
    // i.e. copies of key Lk-1 -- finite scores that never raise the row
    // max; their weights are zeroed after the exponent.
    auto soft_pv = [&](auto tail_c, int key0, const f32x16 &s0, const f32x16 &s1, const lds_t *vs_) __attribute__((always_inline)) {
        constexpr bool TAIL = decltype(tail_c)::value;
        auto drop_tail = [&](float *p) __attribute__((always_inline)) {
            if (TAIL) {
#pragma unroll
                for (int i = 0; i < 32; ++i) {
                    const int key = key0 + (i >> 4) * 32 + 16 * ((i >> 3) & 1) + 8 * hi + (i & 7);
                    p[i] = key < Lk ? p[i] : 0.0f;
                }
            }
        };
        vec8 pb[4];
        float p[32];
        float nm = -m_run;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[i], c2, nm));
            p[16 + i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[i], c2, nm));
        }
        drop_tail(p);
        float sum = pack_sum(p, pb);
        const float pair = pair_sum(sum);
        // !(x <= cap) also catches NaN (inf - inf with m_run = -inf)
        if (__builtin_amdgcn_ballot_w64(!(pair <= E::kSumCap)) != 0) {
            float q[32];
#pragma unroll
            for (int i = 0; i < 16; ++i) { q[i] = s0[i]; q[16 + i] = s1[i]; }
            move_max(pair_max(max32_mfma(q)) * c2, !(pair <= E::kSumCap));
            nm = -m_run;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[i], c2, nm));
                p[16 + i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[i], c2, nm));
            }
            drop_tail(p);
            sum = pack_sum(p, pb);
        }
        l_half += sum;
        pv(vs_, pb);
    };

    if constexpr (!HAS_MASK && !KR) {
        // Pipelined: while step t computes the softmax of tile t, the same
        // wave issues the S^T products of tile t+1 between its VALU
        // instructions; the PV products of tile t follow.  K is staged one
        // tile ahead of V: during step t the LDS holds K(t+1) and V(t), and
        // the DMA fills K(t+2) (into the buffer K(t) left) and V(t+1).
        if (n_tiles > 0) {
            issue_k(0, sK0);
            issue_v(0, sV0);
            if (n_tiles > 1) issue_k(1, sK1);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        f32x16 sa0, sa1, sb0, sb1;
        if (n_tiles > 0) qk(sK0, sa0, sa1);
        __syncthreads();   // every wave is done with K(0) before K(2) lands in its buffer
        if (n_tiles > 0) {
            // step 0 against m_run = -inf would give every weight +inf and
            // redo the step against its exact max: take that max here (O
            // and the row sums are still 0: nothing to rescale)
            float q[32];
#pragma unroll
            for (int i = 0; i < 16; ++i) { q[i] = sa0[i]; q[16 + i] = sa1[i]; }
            m_run = __builtin_fmaxf(m_run, pair_max(max32_mfma(q)) * c2);
        }
        // c0, c1: scores of tile t; n0, n1 <- scores of tile t+1 (NEXT)
        auto pstep = [&](auto next_c, auto tail_c, int t, const f32x16 &c0, const f32x16 &c1, f32x16 &n0,
                         f32x16 &n1, const lds_t *kn_, const lds_t *vs_, lds_t *dK, lds_t *dV)
                         __attribute__((always_inline)) {
            constexpr bool NEXT = decltype(next_c)::value;
            constexpr bool TAIL = decltype(tail_c)::value;
            constexpr int kKPre = kKPreDma;
            if (NEXT) {
                issue_v(t + 1, dV);
                if (t + 2 < n_tiles) issue_k(t + 2, dK);
            }
            const int key0 = t * kBN;
            auto drop_tail = [&](float *p) __attribute__((always_inline)) {
                if (TAIL) {
#pragma unroll
                    for (int i = 0; i < 32; ++i) {
                        const int key = key0 + (i >> 4) * 32 + 16 * ((i >> 3) & 1) + 8 * hi + (i & 7);
                        p[i] = key < Lk ? p[i] : 0.0f;
                    }
                }
            };
            vec8 pb[4];
            float p[32];
            float nm = -m_run;
            vec8 ka[8][2];
            if (NEXT) {
                n0 = (f32x16){};
                n1 = (f32x16){};
#pragma unroll
                for (int ks = 0; ks < kKPre; ++ks) {
                    ka[ks][0] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(kn_ + k_rd[ks]);
                    ka[ks][1] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(kn_ + k_rd[ks] + 32 * 256);
                }
#pragma unroll
                for (int ks = 0; ks < 8; ++ks) {
                    if (ks + kKPre < 8) {
                        ka[ks + kKPre][0] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(kn_ + k_rd[ks + kKPre]);
                        ka[ks + kKPre][1] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(kn_ + k_rd[ks + kKPre] + 32 * 256);
                    }
                    n0 = E::mfma(ka[ks][0], qf[ks], n0);
                    n1 = E::mfma(ka[ks][1], qf[ks], n1);
                }
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(c0[i], c2, nm));
                p[16 + i] = __builtin_amdgcn_exp2f(__builtin_fmaf(c1[i], c2, nm));
            }
            drop_tail(p);
            float sum = pack_sum(p, pb);
            if (NEXT) sched_pipe<kKPre, kPipeVpm>();
            const float pair = pair_sum(sum);
            // the weight sum left [0, E::kSumCap]: exact max, rescale, redo
            if (__builtin_amdgcn_ballot_w64(!(pair <= E::kSumCap)) != 0) {
                float q[32];
#pragma unroll
                for (int i = 0; i < 16; ++i) { q[i] = c0[i]; q[16 + i] = c1[i]; }
                move_max(pair_max(max32_mfma(q)) * c2, !(pair <= E::kSumCap));
                nm = -m_run;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(c0[i], c2, nm));
                    p[16 + i] = __builtin_amdgcn_exp2f(__builtin_fmaf(c1[i], c2, nm));
                }
                drop_tail(p);
                sum = pack_sum(p, pb);
            }
            l_half += sum;
            pv(vs_, pb);
            if (NEXT) {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                __syncthreads();
            }
        };
        // steps 0 .. n_tiles-2 have a next tile (and are full tiles); the
        // last step may be partial.  Step t: K(t+1) in sK[(t+1)&1], V(t) in
        // sV[t&1].
        int t = 0;
        for (; t + 2 < n_tiles; t += 2) {
            pstep(BC<true>(), BC<false>(), t, sa0, sa1, sb0, sb1, sK1, sV0, sK0, sV1);
            pstep(BC<true>(), BC<false>(), t + 1, sb0, sb1, sa0, sa1, sK0, sV1, sK1, sV0);
        }
        const bool tail = Lk % kBN != 0;
        if (t + 1 < n_tiles) {   // two steps left: t (even) and t+1 (last)
            pstep(BC<true>(), BC<false>(), t, sa0, sa1, sb0, sb1, sK1, sV0, sK0, sV1);
            if (tail)
                pstep(BC<false>(), BC<true>(), t + 1, sb0, sb1, sa0, sa1, sK0, sV1, sK1, sV0);
            else
                pstep(BC<false>(), BC<false>(), t + 1, sb0, sb1, sa0, sa1, sK0, sV1, sK1, sV0);
        } else if (t < n_tiles) {   // one step left: t (even, last)
            if (tail)
                pstep(BC<false>(), BC<true>(), t, sa0, sa1, sb0, sb1, sK1, sV0, sK0, sV1);
            else
                pstep(BC<false>(), BC<false>(), t, sa0, sa1, sb0, sb1, sK1, sV0, sK0, sV1);
        }
    } else if constexpr (!HAS_MASK) {
        // Two LDS stages; tile t+1 streams in while tile t is computed.
        if (n_tiles > 0) load_tile_sync(0, sK0, sV0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        // TAIL: the last, partial tile (a compile-time variant, so that full
        // tiles carry no branch around the weights)
        auto step = [&](auto tail_c, int t, const lds_t *ks_, const lds_t *vs_, lds_t *nK, lds_t *nV) __attribute__((always_inline)) {
            const bool has_next = t + 1 < n_tiles;
            if (has_next) {
                issue_tile(t + 1, nK, nV);
                if (KR) rope_load(t + 1);
            }
            f32x16 s0, s1;
            qk(ks_, s0, s1);
            soft_pv(tail_c, t * kBN, s0, s1, vs_);
            if (KR && has_next) rope_store(nK);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
        };
        const int n_full = Lk / kBN;
        for (int t = 0; t < n_full; t += 2) {
            step(BC<false>(), t, sK0, sV0, sK1, sV1);
            if (t + 1 < n_full) step(BC<false>(), t + 1, sK1, sV1, sK0, sV0);
        }
        if (n_full < n_tiles) {
            if (n_full & 1)
                step(BC<true>(), n_full, sK1, sV1, sK0, sV0);
            else
                step(BC<true>(), n_full, sK0, sV0, sK1, sV1);
        }
    } else {
        // masked: two LDS stages; a tile whose mask is -inf for all of this
        // wave's rows is skipped (no MFMA, no softmax)
        if (n_tiles > 0) {
            load_tile_sync(0, sK0, sV0);
            mask_load(0);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        auto mstep = [&](int t, const lds_t *ks_, const lds_t *vs_, lds_t *nK, lds_t *nV) __attribute__((always_inline)) {
            const bool has_next = t + 1 < n_tiles;
            if (has_next) {
                issue_tile(t + 1, nK, nV);
                if (KR) rope_load(t + 1);
            }
            float mv[32];
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
            const bool live = __builtin_amdgcn_ballot_w64(any) != 0;
            if (has_next) mask_load(t + 1);
            if (live) {
                f32x16 s0, s1;
                qk(ks_, s0, s1);
                vec8 pb[4];
                softmax_masked(s0, s1, mv, pb);
                pv(vs_, pb);
            }
            if (KR && has_next) rope_store(nK);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
        };
        for (int t = 0; t < n_tiles; t += 2) {
            mstep(t, sK0, sV0, sK1, sV1);
            if (t + 1 < n_tiles) mstep(t + 1, sK1, sV1, sK0, sV0);
        }
    }

    // ---- epilogue: O / l -> dst[b][q][h][:] (F32, or rounded to F16 / BF16) --
    store_o_row(a, q_row, h, b, hi, o, l_half);
}

// ---------------------------------------------------------------------------
// fa_fwd_xres: short key sets held in LDS -- the text cross-attention
// (src/models/crossdit.hpp:174-200: a few hundred prompt tokens as keys
// against every visual token as a query).  With Lk <= 256, K and V of one
// (batch, head) are at most 2 x 64 KiB, and the call's cost is streaming Q
// rows in and O rows out (plus the mask rows, which all heads share).
//
// One workgroup = 8 waves, two per SIMD = one (batch, head) and a range of
// 32-row query blocks (a.x_blocks of them); wave w takes blocks w, w+8, ...
// K and V are loaded into LDS once, in fa_fwd_d128's tile layout; after that
// the waves never synchronise again, and while one wave of a SIMD waits for
// its next block's Q and mask rows, the other computes.  Within a block the
// mask chunks of tile t+1 are loaded while tile t's products are computed.  Workgroups
// are dealt heads-fastest and XCD-contiguous: the heads of one query range
// run on one XCD and share its L2 for the mask rows.
//
// Per row the arithmetic is fa_fwd_d128's -- the same products, the same
// online softmax (masked: exact running max; unmasked: the lazy max with the
// weight-sum check), the same sums and the same store -- so the two kernels
// give bitwise equal results.
constexpr int kXNT = 4;      // key tiles held in LDS: Lk <= 256
constexpr int kXWaves = 8;
constexpr int kXStage = 4096;   // per wave: 32 rows x 128 bytes of O
static_assert(kXNT * kBN == kXresMaxKeys, "LDS holds every key");

template <typename T, bool HAS_MASK, bool Q32>
__global__ __launch_bounds__(64 * kXWaves) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fa_fwd_xres(Args a) {
    constexpr int kThreads = 64 * kXWaves;
    constexpr int kRounds = kTileBytes / (kThreads * 16);
    static_assert(kRounds * kThreads * 16 == kTileBytes, "tile shape");
    typedef Elem<T> E;
    typedef typename E::vec8 vec8;
    // one LDS object: K tiles at 0, V tiles at 64 KiB, a 4 KiB staging area
    // per wave for its O rows (160 KiB in all) -- so that every K fragment
    // address is one base register plus an immediate offset (and every V
    // address one more base)
    __shared__ __attribute__((aligned(1024))) char lds[2 * kXNT * kTileBytes + kXWaves * kXStage];
    lds_t *const sK = LDS_PTR(char, lds);
    lds_t *const sV = sK + kXNT * kTileBytes;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int hi = lane >> 5;

    // unit (range, b, h), heads fastest, then batches; each XCD a contiguous
    // run of units (so that one XCD's ranges mix the batches, whose masks
    // may leave different numbers of live key tiles)
    const int pid = blockIdx.x;
    const int per = a.n_blocks >> 3;
    const int lid = pid < per * 8 ? (pid & 7) * per + (pid >> 3) : pid;
    const int h = lid % a.H;
    const int rest = lid / a.H;
    const int b = rest % a.B;
    const int range = rest / a.B;

    const char *kbase = a.k + (int64_t)(h / a.rk2) * a.k_nb2 + (int64_t)(b / a.rk3) * a.k_nb3;
    const char *vbase = a.v + (int64_t)(h / a.rv2) * a.v_nb2 + (int64_t)(b / a.rv3) * a.v_nb3;
    const int Lk = a.Lk;
    const int n_tiles = (Lk + kBN - 1) / kBN;

    // ---- K, V -> LDS (rows past Lk repeat key Lk - 1, as in fa_fwd_d128) ----
    {
        const int dma_row = lane >> 4;
        const int dma_pc = lane & 15;
#pragma unroll
        for (int t = 0; t < kXNT; ++t) {
            if (t < n_tiles) {
                const char *kt = kbase + (int64_t)t * kBN * a.k_nb1;
                const char *vt = vbase + (int64_t)t * kBN * a.v_nb1;
#pragma unroll
                for (int j = 0; j < kRounds; ++j) {
                    const int r = 4 * (wave + kXWaves * j) + dma_row;
                    const int kr = t * kBN + k_row_of(r) < Lk ? k_row_of(r) : Lk - 1 - t * kBN;
                    const int vr = t * kBN + r < Lk ? r : Lk - 1 - t * kBN;
                    dma16(kt, (uint32_t)kr * (uint32_t)a.k_nb1 + ((dma_pc ^ (r & 15)) << 4),
                          sK + t * kTileBytes + (wave + kXWaves * j) * 1024);
                    dma16(vt, (uint32_t)vr * (uint32_t)a.v_nb1 + ((dma_pc ^ v_swz(r)) << 4),
                          sV + t * kTileBytes + (wave + kXWaves * j) * 1024);
                }
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    const int n_qb = (a.Lq + 31) >> 5;
    const int qb_end = min((range + 1) * a.x_blocks, n_qb);
    int qb = range * a.x_blocks + wave;
    if (qb >= qb_end) return;   // no barrier follows

    // Per-lane LDS operand offsets.  The masked kernel computes them from an
    // opaque copy of the lane index in each tile's products: hoisted out of
    // the block loop, its 12 offsets were spilled to scratch and reloaded
    // behind the loop's memory waits (a round trip per block).  The unmasked
    // kernel has the registers and keeps them.
    auto k_off = [](int ln, int ks) __attribute__((always_inline)) -> uint32_t {
        return (uint32_t)((ln & 31) * 256 + (((2 * ks + (ln >> 5)) ^ (ln & 15)) << 4));
    };
    auto v_off = [](int ln, int dblk) __attribute__((always_inline)) -> uint32_t {
        const int sub = (ln & 15) >> 2;
        const int c_lo = 2 * ((ln >> 4) & 1) + ((ln & 3) >> 1);
        return (uint32_t)(2048 * (ln >> 5) + 256 * sub + (((4 * dblk + c_lo) ^ v_swz(sub)) << 4) + 8 * (ln & 1));
    };
    uint32_t k_rd[8], v_rd[4];
    if constexpr (!HAS_MASK) {
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) k_rd[ks] = k_off(lane, ks);
#pragma unroll
        for (int dblk = 0; dblk < 4; ++dblk) v_rd[dblk] = v_off(lane, dblk);
    }
    auto k_at = [&](int ln, int ks) __attribute__((always_inline)) -> uint32_t {
        if constexpr (HAS_MASK) return k_off(ln, ks);
        return k_rd[ks];
    };
    auto v_at = [&](int ln, int dblk) __attribute__((always_inline)) -> uint32_t {
        if constexpr (HAS_MASK) return v_off(ln, dblk);
        return v_rd[dblk];
    };

    // ---- operands of a block ----------------------------------------------
    // Q: this lane's 64 elements of its row as stored (Q32: F32, 16 x 16
    // bytes; else K's type, 8 x 16 bytes).  Mask: this lane's 32 keys of a
    // tile as four 16-byte chunks.  The mask rows hold every chunk that
    // starts below Lk; chunks past it re-read the last one and, like the
    // keys of a partial chunk past Lk, count as -inf.
    // The block's uniform values (row bases, strides, flags).  The masked
    // kernel reads them again at the top of every block from the kernel
    // argument segment, through a pointer made opaque there: kept live across
    // the block loop they overflowed the scalar registers, were parked in
    // vector registers and spilled, and the reload waited behind the previous
    // block's stores.
    const char *qbase, *mbase;
    char *obase;
    int64_t q_nb1, m_nb1, o_nb2;
    int Lq, o_type;
    const float *qn_w;
    bool qnorm, qneg;
    float norm_eps, c2;
    auto load_uniforms = [&](const auto *ap) __attribute__((always_inline)) {
        qbase = ap->q + (int64_t)h * ap->q_nb2 + (int64_t)b * ap->q_nb3;
        q_nb1 = ap->q_nb1;
        mbase = HAS_MASK ? ap->m + (int64_t)(h % ap->m_ne2) * ap->m_nb2 + (int64_t)(b % ap->m_ne3) * ap->m_nb3
                         : nullptr;
        m_nb1 = ap->m_nb1;
        Lq = ap->Lq;
        o_type = ap->o_type;
        obase = ap->o + (int64_t)b * ap->o_nb3 + (int64_t)h * ap->o_nb1;
        o_nb2 = ap->o_nb2;
        qn_w = ap->qn_w;
        qnorm = qn_w != nullptr;
        norm_eps = ap->norm_eps;
        qneg = ap->scale_log2 < 0.0f;
        c2 = __builtin_fabsf(ap->scale_log2);
    };
    lds_t *const sO = sV + kXNT * kTileBytes + wave * kXStage;
    // the query-norm weights, in the first 512 bytes of the wave's staging
    // area from the start of a block to its epilogue: each block loads its
    // lane's 8 bytes ahead of the Q rows and leaves them there (read from
    // memory at their use, they queued behind the Q and mask loads: 4% of
    // the normalised cross-attention)
    const __attribute__((address_space(3))) float *const lQw =
        reinterpret_cast<const __attribute__((address_space(3))) float *>(sO);
    u32x4 qraw[Q32 ? 16 : 8];
    u32x4 mraw[4];
    // hi_b, lk_b: hi and Lk, made opaque once per block so that the
    // per-lane address offsets and per-key tests below are computed inside
    // the block loop (hoisted out of it, they would hold dozens of registers
    // for the whole loop)
    int hi_b = hi, lk_b = Lk;
    auto issue_q = [&](int q_ld) __attribute__((always_inline)) {
        const char *qp = qbase + (int64_t)q_ld * q_nb1 + (Q32 ? 32 : 16) * hi_b;
        if constexpr (Q32) {
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                qraw[2 * ks] = ld16(qp + ks * 64);
                qraw[2 * ks + 1] = ld16(qp + ks * 64 + 16);
            }
        } else {
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) qraw[ks] = ld16(qp + ks * 32);
        }
    };
    auto issue_m = [&](const uint16_t *mrow, int t, u32x4 dst[4]) __attribute__((always_inline)) {
        const int last_chunk = (lk_b - 1) & ~7;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int k0 = t * kBN + (c >> 1) * 32 + (c & 1) * 16 + hi_b * 8;
            dst[c] = ld16(mrow + (k0 < last_chunk ? k0 : last_chunk));
        }
    };
    // elements ks*16 + hi*8 .. +7 of the row as F32 (load8_f32 on the raw bytes)
    auto q_elems = [&](int ks, float x[8]) __attribute__((always_inline)) {
        if constexpr (Q32) {
            const f32x4 u = __builtin_bit_cast(f32x4, qraw[2 * ks]);
            const f32x4 w = __builtin_bit_cast(f32x4, qraw[2 * ks + 1]);
            x[0] = u.x; x[1] = u.y; x[2] = u.z; x[3] = u.w;
            x[4] = w.x; x[5] = w.y; x[6] = w.z; x[7] = w.w;
        } else {
            for (int j = 0; j < 4; ++j) { x[2 * j] = E::lo(qraw[ks][j]); x[2 * j + 1] = E::hi(qraw[ks][j]); }
        }
    };
    // load_q_frags' arithmetic (RMSNorm, rounding, sign) on the raw bytes
    vec8 qf[8];
    auto q_frags = [&](u32x2 qw) __attribute__((always_inline)) {
        float qscale = 1.0f;
        if (qnorm) {
            *reinterpret_cast<__attribute__((address_space(3))) u32x2 *>(sO + 8 * lane) = qw;
            double ss = 0.0;
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                float x[8];
                q_elems(ks, x);
                ss += sum_sq8(x);
            }
            qscale = rms_scale(pair_sum_f64(ss), norm_eps);
        }
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const int d0 = ks * 16 + hi * 8;
            float x[8];
            q_elems(ks, x);
            if (qnorm)
                rms_apply8(x, qscale, *reinterpret_cast<const __attribute__((address_space(3))) f32x4 *>(lQw + d0),
                           *reinterpret_cast<const __attribute__((address_space(3))) f32x4 *>(lQw + d0 + 4));
            u32x4 w;
            for (int j = 0; j < 4; ++j) w[j] = E::pack2(x[2 * j], x[2 * j + 1]);
            if (qneg) w ^= (u32x4){0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
            qf[ks] = __builtin_bit_cast(vec8, w);
        }
    };

    f32x16 o[4];
    float m_run, l_half;
    // true until the block's first PV: O and l_half are still 0 in every
    // row, so moving the running max needs no rescale (0 * alpha = 0 for
    // the alpha in [0, 1] it would apply).  Wave-uniform.
    bool o_zero;
    // the block's live key tiles (bit t: tile t holds a finite mask value
    // for one of its rows), from the mask summary when the call has one,
    // else every tile (each is then checked on its mask chunks); the mask
    // chunks of the next live tile are loaded while a tile is computed
    uint32_t live = 0xfu;
    auto next_live = [&](int t) __attribute__((always_inline)) -> int {
        const uint32_t rest = live >> (t + 1);
        return rest ? t + 1 + (int)__builtin_ctz(rest) : kXNT;
    };

    auto qk = [&](const lds_t *ks_, f32x16 &s0, f32x16 &s1) __attribute__((always_inline)) {
        constexpr int kKPre = HAS_MASK ? 1 : kKPreDma;
        s0 = (f32x16){};
        s1 = (f32x16){};
        int ln = lane;
        if constexpr (HAS_MASK) asm volatile("" : "+v"(ln));
        vec8 ka[8][2];
#pragma unroll
        for (int ks = 0; ks < kKPre; ++ks) {
            ka[ks][0] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(ks_ + k_at(ln, ks));
            ka[ks][1] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(ks_ + k_at(ln, ks) + 32 * 256);
        }
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            if (ks + kKPre < 8) {
                ka[ks + kKPre][0] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(ks_ + k_at(ln, ks + kKPre));
                ka[ks + kKPre][1] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(ks_ + k_at(ln, ks + kKPre) + 32 * 256);
            }
            s0 = E::mfma(ka[ks][0], qf[ks], s0);
            s1 = E::mfma(ka[ks][1], qf[ks], s1);
        }
        sched_qk<kKPre>();
    };
    auto move_max = [&](float mx, bool up) __attribute__((always_inline)) {   // fa_fwd_d128's rules, per row
        if (__builtin_amdgcn_ballot_w64(up) != 0) {
            const float m_new = up ? __builtin_fmaxf(m_run, mx) : m_run;
            if (o_zero) {
                m_run = m_new;
            } else {
                const float alpha = m_new == m_run ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
                m_run = m_new;
                l_half *= alpha;
#pragma unroll
                for (int dblk = 0; dblk < 4; ++dblk)
#pragma unroll
                    for (int i = 0; i < 16; ++i) o[dblk][i] *= alpha;
            }
        }
    };
    auto update_max = [&](float mx) __attribute__((always_inline)) { move_max(mx, mx > m_run + kTau); };
    auto pack_sum = [&](const float *p, vec8 pb[4]) -> float {
        float part[4];
#pragma unroll
        for (int kst = 0; kst < 4; ++kst) {
            u32x4 w;
            for (int j = 0; j < 4; ++j) w[j] = E::pack2(p[8 * kst + 2 * j], p[8 * kst + 2 * j + 1]);
            part[kst] = p[8 * kst] + p[8 * kst + 1];
            for (int i = 2; i < 8; ++i) part[kst] += p[8 * kst + i];
            pb[kst] = __builtin_bit_cast(vec8, w);
        }
        return (part[0] + part[1]) + (part[2] + part[3]);
    };
    auto pv = [&](const lds_t *vs_, const vec8 pb[4]) __attribute__((always_inline)) {
        int ln = lane;
        if constexpr (HAS_MASK) asm volatile("" : "+v"(ln));
#pragma unroll
        for (int kst = 0; kst < 4; ++kst) {
#pragma unroll
            for (int dblk = 0; dblk < 4; ++dblk) {
                const lds_t *vp = vs_ + v_at(ln, dblk) + 4096 * kst;
                const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)(vp));
                const s16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)(vp + 1024));
                const vec8 va = __builtin_bit_cast(vec8, __builtin_shufflevector(lo, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
                o[dblk] = E::mfma(va, pb[kst], o[dblk]);
            }
        }
    };
    // masked tile t with its mask chunks mr: logits s*c2 + mask*log2(e),
    // -inf entries (and keys past Lk) stay -inf; a tile that is -inf for all
    // 32 rows is skipped.  Element i of this lane is key
    // t*64 + 32*(i/16) + 16*((i/8)%2) + 8*hi + i%8, chunk i/8.
    auto tile_masked = [&](auto part_c, int t, u32x4 mr[4], const uint16_t *mrow) __attribute__((always_inline)) {
        constexpr bool part = decltype(part_c)::value;
        auto mval = [&](int i) __attribute__((always_inline)) -> float {
            const uint32_t w = mr[i >> 3][(i & 7) >> 1];
            const float v = (i & 1) ? f16_hi(w) : f16_lo(w);
            if constexpr (part) {
                const int key = t * kBN + (i >> 4) * 32 + ((i >> 3) & 1) * 16 + hi_b * 8 + (i & 7);
                return key < lk_b ? v : -INFINITY;
            }
            return v;
        };
        bool any = false;
        if constexpr (part) {
#pragma unroll
            for (int i = 0; i < 32; ++i) any |= mval(i) != -INFINITY;
        } else {
            // on the F16 bits: -inf is exactly 0xfc00
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    any |= (mr[c][e] & 0xffffu) != 0xfc00u || (mr[c][e] >> 16) != 0xfc00u;
        }
        const int tn = next_live(t);
        if (__builtin_amdgcn_ballot_w64(any) == 0) {
            if (tn < n_tiles) issue_m(mrow, tn, mr);
            return;
        }
        f32x16 s0, s1;
        qk(sK + t * kTileBytes, s0, s1);
        float p[32];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            p[i] = s0[i];
            p[16 + i] = s1[i];
        }
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const float mv = mval(i);
            p[i] = mv == -INFINITY ? -INFINITY : __builtin_fmaf(mv, kLog2e, p[i] * c2);
        }
        // the mask chunks are consumed: the registers take the next live tile's
        if (tn < n_tiles) issue_m(mrow, tn, mr);
        update_max(pair_max(max32(p)));
        const float mu = m_run == -INFINITY ? 0.0f : m_run;
#pragma unroll
        for (int i = 0; i < 32; ++i) p[i] = __builtin_amdgcn_exp2f(p[i] - mu);
        vec8 pb[4];
        l_half += pack_sum(p, pb);
        pv(sV + t * kTileBytes, pb);
        o_zero = false;
    };
    // unmasked tile: weights against the current running max, the exact max
    // and a redo only when a row's weight sum leaves [0, E::kSumCap]; keys past
    // Lk (repeats of key Lk - 1) get weight 0
    auto tile_plain = [&](auto part_c, int t) __attribute__((always_inline)) {
        constexpr bool tail = decltype(part_c)::value;
        f32x16 s0, s1;
        qk(sK + t * kTileBytes, s0, s1);
        const int key0 = t * kBN;
        auto drop_tail = [&](float *p) __attribute__((always_inline)) {
            if constexpr (tail) {
#pragma unroll
                for (int i = 0; i < 32; ++i) {
                    const int key = key0 + (i >> 4) * 32 + 16 * ((i >> 3) & 1) + 8 * hi_b + (i & 7);
                    p[i] = key < lk_b ? p[i] : 0.0f;
                }
            }
        };
        vec8 pb[4];
        float p[32];
        if (o_zero) {
            // the block's first tile: every row's running max is -inf, so
            // its weights would all be +inf, leave [0, cap] and take the
            // exact max below; take it here, before the one pass of exp2
            float q[32];
#pragma unroll
            for (int i = 0; i < 16; ++i) { q[i] = s0[i]; q[16 + i] = s1[i]; }
            move_max(pair_max(max32_mfma(q)) * c2, true);
        }
        float nm = -m_run;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[i], c2, nm));
            p[16 + i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[i], c2, nm));
        }
        drop_tail(p);
        float sum = pack_sum(p, pb);
        const float pair = pair_sum(sum);
        if (__builtin_amdgcn_ballot_w64(!(pair <= E::kSumCap)) != 0) {
            float q[32];
#pragma unroll
            for (int i = 0; i < 16; ++i) { q[i] = s0[i]; q[16 + i] = s1[i]; }
            move_max(pair_max(max32_mfma(q)) * c2, !(pair <= E::kSumCap));
            nm = -m_run;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[i], c2, nm));
                p[16 + i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[i], c2, nm));
            }
            drop_tail(p);
            sum = pack_sum(p, pb);
        }
        l_half += sum;
        pv(sV + t * kTileBytes, pb);
        o_zero = false;
    };

    if constexpr (!HAS_MASK) load_uniforms(&a);
    for (; qb < qb_end; qb += kXWaves) {
        if constexpr (HAS_MASK) {
            typedef const __attribute__((address_space(4))) Args *args_ptr;
            args_ptr ap = (args_ptr)__builtin_amdgcn_kernarg_segment_ptr();
            asm volatile("" : "+s"(ap));
            load_uniforms(ap);
            // the block's word of the mask summary (read here, from the
            // argument segment, like the other uniforms of the block)
            const uint32_t *ml = ap->m_live;
            live = ml ? ml[((int64_t)(b % ap->m_ne3) * ap->m_ne2 + h % ap->m_ne2) * ap->m_live_nqb + qb] : 0xfu;
        }
        lk_b = Lk;
        hi_b = hi;
        asm volatile("" : "+s"(lk_b), "+v"(hi_b));
        const int q_row = qb * 32 + l32;
        const int q_ld = q_row < Lq ? q_row : Lq - 1;
        u32x2 qw = {};
        if (qnorm) {
            int ln = lane;   // the offset computed here, not held (and spilled) across the loop
            asm volatile("" : "+v"(ln));
            qw = *reinterpret_cast<const u32x2 *>(qn_w + 2 * ln);
        }
        issue_q(q_ld);
        const uint16_t *mrow = nullptr;
        if (HAS_MASK) {
            mrow = reinterpret_cast<const uint16_t *>(mbase + (int64_t)q_ld * m_nb1);
            const int t0 = live ? (int)__builtin_ctz(live) : kXNT;
            if (t0 < n_tiles) issue_m(mrow, t0, mraw);
        }
        q_frags(qw);
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = (f32x16){};
        m_run = -INFINITY;
        l_half = 0.0f;
        o_zero = true;
#pragma unroll
        for (int t = 0; t < kXNT; ++t) {
            if (t < n_tiles && ((live >> t) & 1u)) {
                const bool part = (t + 1) * kBN > lk_b;   // the last tile, keys past Lk
                if (HAS_MASK) {
                    if (part)
                        tile_masked(BC<true>(), t, mraw, mrow);
                    else
                        tile_masked(BC<false>(), t, mraw, mrow);
                } else {
                    if (part)
                        tile_plain(BC<true>(), t);
                    else
                        tile_plain(BC<false>(), t);
                }
            }
        }
        // O / l -> the rows (store_o_row_l's arithmetic), through the wave's
        // 4 KiB staging area, all 32 rows at a time: each lane leaves its
        // 16-byte pieces of its row there (chunk index XOR the row's low
        // bits: no bank conflicts), then lane L reads chunk L%8 of rows
        // 8j + L/8, so that every store instruction writes eight whole
        // 128-byte lines (one per row) instead of 32-byte pieces of 32 rows.
        // F32: one 32-column block per round (4 rounds); 16-bit: two (2
        // rounds).  Half that area took twice the rounds, each an LDS write
        // and read in sequence: 2-3% of C2.  (LDS operations of a wave
        // complete in order, so a round's reads see its writes and precede
        // the next round's writes.)
        {
            const float l_run = pair_sum(l_half);
            const float inv = l_run == 0.0f ? 0.0f : 1.0f / l_run;
            const int rr = lane >> 3;
            const int rc = lane & 7;
            // row 8j + rr, chunk rc ^ rr: one base per lane, computed here
            // from an opaque copy of the lane index (hoisted out of the
            // block loop, the per-row addresses went to scratch)
            int ln_f = lane;
            asm volatile("" : "+v"(ln_f));
            const lds_t *const fbase = sO + (ln_f >> 3) * 128 + (((ln_f & 7) ^ (ln_f >> 3 & 7)) << 4);
            auto flush = [&](int col_byte) __attribute__((always_inline)) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int r = 8 * j + rr;
                    const u32x4 w = *reinterpret_cast<const __attribute__((address_space(3))) u32x4 *>(fbase + j * 1024);
                    const int row = qb * 32 + r;
                    // streaming store: O is not read again here (2-3%)
                    if (row < Lq) __builtin_nontemporal_store(w, reinterpret_cast<u32x4 *>(obase + (int64_t)row * o_nb2 + col_byte + rc * 16));
                }
            };
            if (o_type == KD_FA_TYPE_F32) {
#pragma unroll
                for (int dblk = 0; dblk < 4; ++dblk) {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const f32x4 v = {o[dblk][4 * g] * inv, o[dblk][4 * g + 1] * inv,
                                         o[dblk][4 * g + 2] * inv, o[dblk][4 * g + 3] * inv};
                        *reinterpret_cast<__attribute__((address_space(3))) f32x4 *>(
                            sO + l32 * 128 + (((2 * g + hi_b) ^ (l32 & 7)) << 4)) = v;
                    }
                    flush(dblk * 128);
                }
            } else {
                const bool bf = o_type == KD_FA_TYPE_BF16;
#pragma unroll
                for (int rnd = 0; rnd < 2; ++rnd) {
#pragma unroll
                    for (int dd = 0; dd < 2; ++dd)
#pragma unroll
                        for (int g = 0; g < 4; ++g) {
                            const int dblk = 2 * rnd + dd;
                            const float v0 = o[dblk][4 * g] * inv, v1 = o[dblk][4 * g + 1] * inv;
                            const float v2 = o[dblk][4 * g + 2] * inv, v3 = o[dblk][4 * g + 3] * inv;
                            const u32x2 w = bf ? (u32x2){Elem<__bf16>::pack2(v0, v1), Elem<__bf16>::pack2(v2, v3)}
                                               : (u32x2){Elem<_Float16>::pack2(v0, v1), Elem<_Float16>::pack2(v2, v3)};
                            *reinterpret_cast<__attribute__((address_space(3))) u32x2 *>(
                                sO + l32 * 128 + (((dd * 4 + g) ^ (l32 & 7)) << 4) + 8 * hi_b) = w;
                        }
                    flush(rnd * 128);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// fa_fwd_xlong: unmasked key sets of kXresMaxKeys + 1 .. kXlongMaxKeys keys,
// K read as stored, Q neither rotated nor normalised -- the text
// cross-attention of a long prompt (src/models/crossdit.hpp:198 calls
// ops::attention without a mask; the tokenizer keeps up to 512 prompt
// tokens, src/models/qwen_tokenizer.hpp:128,183-186).  K and V of 512 keys
// (256 KiB in 16 bits) do not fit the LDS, so they stream through it tile by
// tile, in fa_fwd_d128's pipelined unmasked loop (the scores of tile t+1
// computed between the softmax instructions of tile t; K two tiles and V one
// tile ahead by DMA).  What this kernel adds is that a workgroup's memory
// phases overlap its key loop instead of running in sequence with it:
//
// * Persistent workgroups.  One 8-wave workgroup per CU walks units of 256
//   query rows of one (b, h): XCD x (workgroups are dealt to the XCDs
//   round-robin) owns a contiguous range of units and its workgroup j takes
//   units j, j + w, j + 2w, ... of it (w workgroups per XCD), so that an
//   XCD's workgroups run neighbouring query tiles of one head together and
//   share its K and V in the L2.
// * Q by DMA during the key loop.  In the first kPieces steps of a unit,
//   each wave brings 128 bytes of each of its 32 rows of the next unit into
//   its raw area (one piece per step) and, a step later, rounds them to the
//   operand type into its fragment area, from which the next unit loads its
//   Q fragments with eight LDS reads.
// * The next unit's first tiles ahead of the O stores.  The last step of a
//   unit fetches the next unit's K(0) and K(1) (its K buffers are free by
//   then), V(0) follows once the step's products are done, and only then
//   are the unit's O stores issued: the wait before the next unit's first
//   step counts the stores issued after V(0) and does not wait for them
//   (loads and stores complete in issue order).
//
// Each unit starts like fa_fwd_d128's loop (the exact max of its first
// tile's scores, then the lazy running max), and per row the arithmetic is
// that loop's, so the two kernels give bitwise equal results.
//
// LDS (one object, the tiles first so that every fragment address is a lane
// offset plus an immediate below 64 KiB): K and V tiles 2 x 2 x 16 KiB, then
// per wave 8 KiB of Q fragments (lane l's fragment of k-step ks at
// ks * 1024 + 16 l) and 4 KiB of raw Q rows (row r of the wave at 128 r, its
// 16-byte chunk c at c ^ (r & 7)), which also stage the O rows of the
// epilogue: 160 KiB.
// ---------------------------------------------------------------------------
constexpr int kLWaves = 8;
constexpr int kLRows = 32 * kLWaves;   // query rows per unit
constexpr int kLFrag = 8192;           // per wave: 8 k-steps x 64 lanes x 16 bytes
constexpr int kLRaw = 4096;            // per wave: 128 bytes of each of its 32 rows
static_assert(kLRows == kXlongRows, "unit size");

template <typename T, bool Q32>
__global__ __launch_bounds__(64 * kLWaves) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fa_fwd_xlong(Args a) {
    constexpr int kThreads = 64 * kLWaves;
    constexpr int kRounds = kTileBytes / (kThreads * 16);
    static_assert(kRounds * kThreads * 16 == kTileBytes, "tile shape");
    constexpr int kPieces = Q32 ? 4 : 2;   // 128-byte pieces of a Q row
    constexpr int kKPre = kKPreDma;
    typedef Elem<T> E;
    typedef typename E::vec8 vec8;
    __shared__ __attribute__((aligned(1024))) char lds[4 * kTileBytes + kLWaves * (kLFrag + kLRaw)];
    lds_t *const sK0 = LDS_PTR(char, lds), *const sK1 = sK0 + kTileBytes;
    lds_t *const sV0 = sK0 + 2 * kTileBytes, *const sV1 = sK0 + 3 * kTileBytes;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int hi = lane >> 5;
    lds_t *const sQf = sK0 + 4 * kTileBytes + wave * (kLFrag + kLRaw);
    lds_t *const sRaw = sQf + kLFrag;

    // this workgroup's units: j, j + wpx, ... within its XCD's range
    const int n_units = a.n_blocks;
    const int wpx = (int)(gridDim.x >> 3);
    const int per = (n_units + 7) >> 3;
    const int xcd = (int)(blockIdx.x & 7);
    const int u_end = min((xcd + 1) * per, n_units);
    int u = xcd * per + (int)(blockIdx.x >> 3);
    if (u >= u_end) return;   // before any barrier

    const int Lk = a.Lk, Lq = a.Lq;
    const int n_tiles = (Lk + kBN - 1) / kBN;   // >= 5
    const float c2 = __builtin_fabsf(a.scale_log2);

    // A unit's values come from the kernel arguments read again through a
    // pointer made opaque at each use, so that the arguments the key loop
    // does not need are not held in scalar registers across it.
    typedef const __attribute__((address_space(4))) Args *args_ptr;
    auto kargs = []() __attribute__((always_inline)) {
        args_ptr ap = (args_ptr)__builtin_amdgcn_kernarg_segment_ptr();
        asm volatile("" : "+s"(ap));
        return ap;
    };
    struct Unit {
        const char *k, *v, *q;   // K, V of its (b, h); Q from its first row
        char *o;                 // O from its first row
        int row0;
    };
    auto unit_at = [&](int uu) __attribute__((always_inline)) {
        const args_ptr ap = kargs();
        Unit r;
        const int qt = uu % ap->n_qt;
        const int bh = uu / ap->n_qt;
        const int h = bh % ap->H;
        const int b = bh / ap->H;
        r.row0 = qt * kLRows;
        r.o = ap->o + (int64_t)b * ap->o_nb3 + (int64_t)h * ap->o_nb1 + (int64_t)r.row0 * ap->o_nb2;
        r.k = ap->k + (int64_t)(h / ap->rk2) * ap->k_nb2 + (int64_t)(b / ap->rk3) * ap->k_nb3;
        r.v = ap->v + (int64_t)(h / ap->rv2) * ap->v_nb2 + (int64_t)(b / ap->rv3) * ap->v_nb3;
        r.q = ap->q + (int64_t)h * ap->q_nb2 + (int64_t)b * ap->q_nb3 + (int64_t)r.row0 * ap->q_nb1;
        return r;
    };
    // a fresh opaque copy of the lane index at each use outside the key
    // products: what is derived from it (the partial tile's key tests and
    // clamped DMA offsets, the Q pieces' and O rows' addresses) is computed
    // at its use instead of being held across the loops
    auto fresh_lane = [&]() __attribute__((always_inline)) {
        int x = lane;
        asm volatile("" : "+v"(x));
        return x;
    };

    // ---- K/V tile DMA (fa_fwd_d128's lanes, rows and swizzles) ---------------
    const uint32_t v_dma0 = (uint32_t)(4 * wave + (lane >> 4)) * (uint32_t)a.v_nb1 +
                            (((lane & 15) ^ v_swz(4 * wave + (lane >> 4))) << 4);
    const uint32_t k_dma0 = (uint32_t)k_row_of(4 * wave + (lane >> 4)) * (uint32_t)a.k_nb1 +
                            (((lane & 15) ^ ((4 * wave + (lane >> 4)) & 15)) << 4);
    auto issue_v = [&](const char *vb, int t, lds_t *dV) __attribute__((always_inline)) {
        const char *vt = vb + (int64_t)t * kBN * a.v_nb1;
        if ((t + 1) * kBN <= Lk) {
#pragma unroll
            for (int j = 0; j < kRounds; ++j)
                dma16(vt + (int64_t)j * 4 * kLWaves * a.v_nb1, v_dma0, dV + (wave + kLWaves * j) * 1024);
        } else {
            const int ln = fresh_lane();
#pragma unroll
            for (int j = 0; j < kRounds; ++j) {
                const int r = 4 * (wave + kLWaves * j) + (ln >> 4);
                const int vr = t * kBN + r < Lk ? r : Lk - 1 - t * kBN;
                dma16(vt, (uint32_t)vr * (uint32_t)a.v_nb1 + (((ln & 15) ^ v_swz(r)) << 4),
                      dV + (wave + kLWaves * j) * 1024);
            }
        }
    };
    auto issue_k = [&](const char *kb, int t, lds_t *dK) __attribute__((always_inline)) {
        const char *kt = kb + (int64_t)t * kBN * a.k_nb1;
        if ((t + 1) * kBN <= Lk) {
#pragma unroll
            for (int j = 0; j < kRounds; ++j)
                dma16(kt + (int64_t)j * 4 * kLWaves * a.k_nb1, k_dma0, dK + (wave + kLWaves * j) * 1024);
        } else {
            const int ln = fresh_lane();
#pragma unroll
            for (int j = 0; j < kRounds; ++j) {
                const int r = 4 * (wave + kLWaves * j) + (ln >> 4);
                const int kr = t * kBN + k_row_of(r) < Lk ? k_row_of(r) : Lk - 1 - t * kBN;
                dma16(kt, (uint32_t)kr * (uint32_t)a.k_nb1 + (((ln & 15) ^ (r & 15)) << 4),
                      dK + (wave + kLWaves * j) * 1024);
            }
        }
    };

    // ---- the next unit's Q -----------------------------------------------------
    // Piece p of a row is its bytes 128 p .. +127 (F32: k-steps 2p, 2p+1;
    // 16-bit: k-steps 4p .. 4p+3).  DMA instruction jj of a piece fills rows
    // 8 jj .. +7 of the raw area: lane l fills slot l % 8 of row 8 jj + l / 8
    // with the chunk that belongs there.  Rows past Lq read row Lq - 1.
    auto issue_piece = [&](const Unit &un, int p) __attribute__((always_inline)) {
        const int ln = fresh_lane();
        const int pr = ln >> 3;
        const uint32_t pc16 = (uint32_t)(((ln & 7) ^ (pr & 7)) << 4);
        const char *qb = un.q + p * 128;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int r = un.row0 + wave * 32 + 8 * jj + pr;
            const int rc = (r < Lq ? r : Lq - 1) - un.row0;
            dma16(qb, (uint32_t)rc * (uint32_t)a.q_nb1 + pc16, sRaw + jj * 1024);
        }
    };
    // piece p of this lane's row -> its fragments in the fragment area, with
    // load_q_frags' rounding and sign (scale < 0 negates Q)
    auto convert_piece = [&](int p) __attribute__((always_inline)) {
        const int ln = fresh_lane();
        const int r32 = ln & 31, h2 = ln >> 5;
        const lds_t *rp = sRaw + r32 * 128;
        const int sw = r32 & 7;
        const uint32_t ng = a.scale_log2 < 0.0f ? 0x80008000u : 0u;
        if constexpr (Q32) {
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const f32x4 x0 = *reinterpret_cast<const __attribute__((address_space(3))) f32x4 *>(
                    rp + (((4 * e + 2 * h2) ^ sw) << 4));
                const f32x4 x1 = *reinterpret_cast<const __attribute__((address_space(3))) f32x4 *>(
                    rp + (((4 * e + 2 * h2 + 1) ^ sw) << 4));
                const u32x4 w = {E::pack2(x0.x, x0.y) ^ ng, E::pack2(x0.z, x0.w) ^ ng, E::pack2(x1.x, x1.y) ^ ng,
                                 E::pack2(x1.z, x1.w) ^ ng};
                *reinterpret_cast<__attribute__((address_space(3))) u32x4 *>(sQf + (2 * p + e) * 1024 + ln * 16) = w;
                // both reads have returned before what follows (the next
                // piece's DMA into the raw area)
                asm volatile("" ::"v"(x0.w), "v"(x1.w));
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const u32x4 r = *reinterpret_cast<const __attribute__((address_space(3))) u32x4 *>(
                    rp + (((2 * e + h2) ^ sw) << 4));
                u32x4 w;
#pragma unroll
                for (int j = 0; j < 4; ++j) w[j] = E::pack2(E::lo(r[j]), E::hi(r[j])) ^ ng;
                *reinterpret_cast<__attribute__((address_space(3))) u32x4 *>(sQf + (4 * p + e) * 1024 + ln * 16) = w;
                asm volatile("" ::"v"(r[3]));   // the read has returned
            }
        }
    };

    // ---- per-row state and fa_fwd_d128's arithmetic ------------------------------
    vec8 qf[8];
    f32x16 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (f32x16){};
    float m_run = -INFINITY;
    float l_half = 0.0f;

    uint32_t k_rd[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) k_rd[ks] = l32 * 256 + (((2 * ks + hi) ^ (lane & 15)) << 4);
    const int v_sub = (lane & 15) >> 2;
    const int v_c_lo = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
    uint32_t v_rd[4];
#pragma unroll
    for (int dblk = 0; dblk < 4; ++dblk)
        v_rd[dblk] = 2048 * hi + 256 * v_sub + (((4 * dblk + v_c_lo) ^ v_swz(v_sub)) << 4) + 8 * (lane & 1);

    auto qk = [&](const lds_t *ks_, f32x16 &s0, f32x16 &s1) __attribute__((always_inline)) {
        s0 = (f32x16){};
        s1 = (f32x16){};
        vec8 ka[8][2];
#pragma unroll
        for (int ks = 0; ks < kKPre; ++ks) {
            ka[ks][0] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(ks_ + k_rd[ks]);
            ka[ks][1] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(ks_ + k_rd[ks] + 32 * 256);
        }
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            if (ks + kKPre < 8) {
                ka[ks + kKPre][0] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(ks_ + k_rd[ks + kKPre]);
                ka[ks + kKPre][1] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(ks_ + k_rd[ks + kKPre] + 32 * 256);
            }
            s0 = E::mfma(ka[ks][0], qf[ks], s0);
            s1 = E::mfma(ka[ks][1], qf[ks], s1);
        }
        sched_qk<kKPre>();
    };
    auto move_max = [&](float mx, bool up) __attribute__((always_inline)) {
        if (__builtin_amdgcn_ballot_w64(up) != 0) {
            const float m_new = up ? __builtin_fmaxf(m_run, mx) : m_run;
            const float alpha = m_new == m_run ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
            l_half *= alpha;
#pragma unroll
            for (int dblk = 0; dblk < 4; ++dblk)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[dblk][i] *= alpha;
        }
    };
    auto pack_sum = [&](const float *p, vec8 pb[4]) -> float {
        float part[4];
#pragma unroll
        for (int kst = 0; kst < 4; ++kst) {
            u32x4 w;
            for (int j = 0; j < 4; ++j) w[j] = E::pack2(p[8 * kst + 2 * j], p[8 * kst + 2 * j + 1]);
            part[kst] = p[8 * kst] + p[8 * kst + 1];
            for (int i = 2; i < 8; ++i) part[kst] += p[8 * kst + i];
            pb[kst] = __builtin_bit_cast(vec8, w);
        }
        return (part[0] + part[1]) + (part[2] + part[3]);
    };
    auto pv = [&](const lds_t *vs_, const vec8 pb[4]) __attribute__((always_inline)) {
#pragma unroll
        for (int kst = 0; kst < 4; ++kst) {
#pragma unroll
            for (int dblk = 0; dblk < 4; ++dblk) {
                const lds_t *vp = vs_ + v_rd[dblk] + 4096 * kst;
                const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)(vp));
                const s16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)(vp + 1024));
                const vec8 va = __builtin_bit_cast(vec8, __builtin_shufflevector(lo, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
                o[dblk] = E::mfma(va, pb[kst], o[dblk]);
            }
        }
    };

    // ---- O of a unit: fa_fwd_xres's whole-line stores through LDS ----------------
    // (the wave's raw area, free once the next unit's last piece is
    // converted).  F32: 16 store instructions per wave, 16-bit: 8, each
    // issued unless all of its 8 rows are past Lq.  The next unit's first
    // wait leaves that many outstanding when every row of the unit lies
    // below Lq: the fence before the flush keeps all of them after the V(0)
    // DMA, and no global store is wider than 16 bytes per lane, so the
    // compiler can only split them (a longer wait), never merge them.  (The
    // stores written as the instructions themselves measured 1-1.5% slower.)
    auto flush_unit = [&](const Unit &un) __attribute__((always_inline)) {
        const int ln = fresh_lane();
        const int r32 = ln & 31, h2 = ln >> 5;
        const float l_run = pair_sum(l_half);
        const float inv = l_run == 0.0f ? 0.0f : 1.0f / l_run;
        const int rr = ln >> 3;
        const int rc = ln & 7;
        const lds_t *const fbase = sRaw + rr * 128 + ((rc ^ rr) << 4);
        const args_ptr ap = kargs();
        const int64_t o_nb2 = ap->o_nb2;
        // row row0 + 32 wave + 8 j + rr at obase + 8 j * o_nb2
        char *const obase = un.o + (int64_t)(wave * 32 + rr) * o_nb2 + rc * 16;
        const int rowb = un.row0 + wave * 32 + rr;
        auto flush = [&](int col_byte) __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u32x4 w = *reinterpret_cast<const __attribute__((address_space(3))) u32x4 *>(fbase + j * 1024);
                if (rowb + 8 * j < Lq)
                    __builtin_nontemporal_store(w, reinterpret_cast<u32x4 *>(obase + (int64_t)(8 * j) * o_nb2 + col_byte));
            }
        };
        if (ap->o_type == KD_FA_TYPE_F32) {
#pragma unroll
            for (int dblk = 0; dblk < 4; ++dblk) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const f32x4 v = {o[dblk][4 * g] * inv, o[dblk][4 * g + 1] * inv, o[dblk][4 * g + 2] * inv,
                                     o[dblk][4 * g + 3] * inv};
                    *reinterpret_cast<__attribute__((address_space(3))) f32x4 *>(
                        sRaw + r32 * 128 + (((2 * g + h2) ^ (r32 & 7)) << 4)) = v;
                }
                flush(dblk * 128);
            }
        } else {
            const bool bf = ap->o_type == KD_FA_TYPE_BF16;
#pragma unroll
            for (int rnd = 0; rnd < 2; ++rnd) {
#pragma unroll
                for (int dd = 0; dd < 2; ++dd)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int dblk = 2 * rnd + dd;
                        const float v0 = o[dblk][4 * g] * inv, v1 = o[dblk][4 * g + 1] * inv;
                        const float v2 = o[dblk][4 * g + 2] * inv, v3 = o[dblk][4 * g + 3] * inv;
                        const u32x2 w = bf ? (u32x2){Elem<__bf16>::pack2(v0, v1), Elem<__bf16>::pack2(v2, v3)}
                                           : (u32x2){Elem<_Float16>::pack2(v0, v1), Elem<_Float16>::pack2(v2, v3)};
                        *reinterpret_cast<__attribute__((address_space(3))) u32x2 *>(
                            sRaw + r32 * 128 + (((dd * 4 + g) ^ (r32 & 7)) << 4) + 8 * h2) = w;
                    }
                flush(rnd * 128);
            }
        }
    };

    // ---- the first unit: Q from memory, K(0), V(0), K(1) ---------------------------
    Unit cur = unit_at(u);
    {
        const int q_row = cur.row0 + wave * 32 + l32;
        const int bh = u / a.n_qt;
        load_q_frags<T, KD_FA_ROPE_NONE>(a, q_row < Lq ? q_row : Lq - 1, bh % a.H, bh / a.H, hi, qf);
    }
    u += wpx;
    bool has_nxt = u < u_end;
    Unit nxt = has_nxt ? unit_at(u) : cur;
    issue_k(cur.k, 0, sK0);
    issue_v(cur.v, 0, sV0);
    issue_k(cur.k, 1, sK1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // the previous unit's O stores were all issued after this unit's V(0):
    // its first wait then counts them (16 with F32 O, 8 with 16-bit O)
    int n_after = 0;

    for (;;) {
        // ---- the unit: the scores of tile 0 (K(0) in its buffer), then the
        // pipelined steps of fa_fwd_d128 --------------------------------------------
        f32x16 sa0, sa1, sb0, sb1;   // scores of the tiles of even / odd index
        qk(sK0, sa0, sa1);
        // V(0) is in, and every wave is done with K(0) before K(2) lands in
        // its buffer
        if (n_after == 16)
            asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        else if (n_after == 8)
            asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        {
            float q[32];
#pragma unroll
            for (int i = 0; i < 16; ++i) { q[i] = sa0[i]; q[16 + i] = sa1[i]; }
            m_run = __builtin_fmaxf(m_run, pair_max(max32_mfma(q)) * c2);
        }
        // step t: softmax and PV of tile t (scores c0, c1; V(t) at vs_) and,
        // when NEXT, the scores n0, n1 of tile t+1 (K at kn_); DMAs of V(t+1)
        // into dV and K(t+2) into dK.  The last step (!NEXT) fetches the next
        // unit's K(0), K(1) instead.  TAIL: tile t is the last, partial one.
        auto pstep = [&](auto next_c, auto tail_c, int t, const f32x16 &c0, const f32x16 &c1, f32x16 &n0,
                         f32x16 &n1, const lds_t *kn_, const lds_t *vs_, lds_t *dK, lds_t *dV)
                         __attribute__((always_inline)) {
            constexpr bool NEXT = decltype(next_c)::value;
            constexpr bool TAIL = decltype(tail_c)::value;
            if (NEXT) {
                issue_v(cur.v, t + 1, dV);
                if (t + 2 < n_tiles) issue_k(cur.k, t + 2, dK);
            } else if (has_nxt) {
                issue_k(nxt.k, 0, sK0);
                issue_k(nxt.k, 1, sK1);
            }
            if (has_nxt) {
                // the raw area's reads (the conversion's, which end in
                // registers the DMA is ordered after, or the previous unit's
                // O staging, consumed by its stores) come before the DMA
                // refills it
                if (t >= 1 && t <= kPieces) convert_piece(t - 1);
                if (t < kPieces) issue_piece(nxt, t);
            }
            const int key0 = t * kBN;
            auto drop_tail = [&](float *p) __attribute__((always_inline)) {
                if (TAIL) {
                    // key key0 + 8 hi + off of this lane is below Lk
                    const int lim = Lk - key0 - 8 * (fresh_lane() >> 5);
#pragma unroll
                    for (int i = 0; i < 32; ++i) {
                        const int off = (i >> 4) * 32 + 16 * ((i >> 3) & 1) + (i & 7);
                        p[i] = off < lim ? p[i] : 0.0f;
                    }
                }
            };
            vec8 pb[4];
            float p[32];
            float nm = -m_run;
            vec8 ka[8][2];
            if (NEXT) {
                n0 = (f32x16){};
                n1 = (f32x16){};
#pragma unroll
                for (int ks = 0; ks < kKPre; ++ks) {
                    ka[ks][0] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(kn_ + k_rd[ks]);
                    ka[ks][1] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(kn_ + k_rd[ks] + 32 * 256);
                }
#pragma unroll
                for (int ks = 0; ks < 8; ++ks) {
                    if (ks + kKPre < 8) {
                        ka[ks + kKPre][0] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(kn_ + k_rd[ks + kKPre]);
                        ka[ks + kKPre][1] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(kn_ + k_rd[ks + kKPre] + 32 * 256);
                    }
                    n0 = E::mfma(ka[ks][0], qf[ks], n0);
                    n1 = E::mfma(ka[ks][1], qf[ks], n1);
                }
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(c0[i], c2, nm));
                p[16 + i] = __builtin_amdgcn_exp2f(__builtin_fmaf(c1[i], c2, nm));
            }
            drop_tail(p);
            float sum = pack_sum(p, pb);
            if (NEXT) sched_pipe<kKPre, kPipeVpm>();
            const float pair = pair_sum(sum);
            if (__builtin_amdgcn_ballot_w64(!(pair <= E::kSumCap)) != 0) {
                float q[32];
#pragma unroll
                for (int i = 0; i < 16; ++i) { q[i] = c0[i]; q[16 + i] = c1[i]; }
                move_max(pair_max(max32_mfma(q)) * c2, !(pair <= E::kSumCap));
                nm = -m_run;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(c0[i], c2, nm));
                    p[16 + i] = __builtin_amdgcn_exp2f(__builtin_fmaf(c1[i], c2, nm));
                }
                drop_tail(p);
                sum = pack_sum(p, pb);
            }
            l_half += sum;
            pv(vs_, pb);
            if (NEXT || has_nxt) {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                __syncthreads();
            }
        };
        // steps 0 .. n_tiles-2 have a next tile (and are full tiles); step t:
        // K(t+1) in sK[(t+1)&1], V(t) in sV[t&1]
        const bool tail = Lk % kBN != 0;
        int t = 0;
        for (; t + 2 < n_tiles; t += 2) {
            pstep(BC<true>(), BC<false>(), t, sa0, sa1, sb0, sb1, sK1, sV0, sK0, sV1);
            pstep(BC<true>(), BC<false>(), t + 1, sb0, sb1, sa0, sa1, sK0, sV1, sK1, sV0);
        }
        if (t + 1 < n_tiles) {   // two steps left: t (even) and t+1 (last)
            pstep(BC<true>(), BC<false>(), t, sa0, sa1, sb0, sb1, sK1, sV0, sK0, sV1);
            if (tail)
                pstep(BC<false>(), BC<true>(), t + 1, sb0, sb1, sa0, sa1, sK0, sV1, sK1, sV0);
            else
                pstep(BC<false>(), BC<false>(), t + 1, sb0, sb1, sa0, sa1, sK0, sV1, sK1, sV0);
        } else {   // one step left: t (even, last)
            if (tail)
                pstep(BC<false>(), BC<true>(), t, sa0, sa1, sb0, sb1, sK1, sV0, sK0, sV1);
            else
                pstep(BC<false>(), BC<false>(), t, sa0, sa1, sb0, sb1, sK1, sV0, sK0, sV1);
        }
        // ---- the next unit's V(0), then this unit's O -------------------------
        if (has_nxt) issue_v(nxt.v, 0, sV0);
        asm volatile("" ::: "memory");
        flush_unit(cur);
        if (!has_nxt) break;
        n_after = cur.row0 + kLRows <= Lq ? (a.o_type == KD_FA_TYPE_F32 ? 16 : 8) : 0;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
            qf[ks] = *reinterpret_cast<const __attribute__((address_space(3))) vec8 *>(sQf + ks * 1024 + lane * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = (f32x16){};
        m_run = -INFINITY;
        l_half = 0.0f;
        cur = nxt;
        u += wpx;
        has_nxt = u < u_end;
        if (has_nxt) nxt = unit_at(u);
    }
}

// ---------------------------------------------------------------------------
// mask_live_kernel: the mask summary of fa_fwd_xres.  One wave per (mask
// batch, mask head, 32-row query block); each load instruction reads whole
// rows: lane l takes 16-byte chunk l % 32 (keys 8 (l % 32) .. +7, tile
// (l % 32) / 8) of rows 2i + l / 32, i = 0..15 (rows past Lq clamped to
// Lq - 1, as the attention reads them; chunks that start at or past Lk are
// not read -- the mask rows hold every chunk that starts below Lk -- and
// keys past Lk in the last chunk do not count).  The wave's ballot sets bit
// t of the block's word when one of tile t's F16 values is not -inf
// (0xfc00): the test fa_fwd_xres applies to a tile's chunks, so a tile the
// summary marks dead is exactly one it would skip after loading them.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void mask_live_kernel(Args a, uint32_t *out, int64_t n_words) {
    const int lane = threadIdx.x & 63;
    const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (w >= n_words) return;
    const int qb = (int)(w % a.m_live_nqb);
    const int64_t hb = w / a.m_live_nqb;
    const int mh = (int)(hb % a.m_ne2);
    const int mb = (int)(hb / a.m_ne2);
    const int c = lane & 31;
    const int k0 = 8 * c;
    bool any = false;
    if (k0 < a.Lk) {
        const char *base = a.m + (int64_t)mb * a.m_nb3 + (int64_t)mh * a.m_nb2 + (int64_t)k0 * 2;
        u32x4 v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = min(qb * 32 + 2 * i + (lane >> 5), a.Lq - 1);
            v[i] = ld16(base + (int64_t)row * a.m_nb1);
        }
        const int n_keys = min(8, a.Lk - k0);
#pragma unroll
        for (int i = 0; i < 16; ++i)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t h16 = (v[i][e >> 1] >> (16 * (e & 1))) & 0xffffu;
                any |= e < n_keys && h16 != 0xfc00u;
            }
    }
    const uint64_t bal = __builtin_amdgcn_ballot_w64(any);
    const uint32_t per_chunk = (uint32_t)bal | (uint32_t)(bal >> 32);   // bit c: chunk c of some row
    uint32_t bits = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) bits |= ((per_chunk >> (8 * t)) & 0xffu ? 1u : 0u) << t;
    if (lane == 0) out[w] = bits;
}

int64_t mask_live_words(const Args &a) {
    return (int64_t)a.m_ne3 * a.m_ne2 * (((int64_t)a.Lq + 31) / 32);
}

hipError_t launch_mask_live(const Args &a, uint32_t *out, hipStream_t stream) {
    const int64_t n = mask_live_words(a);
    if (n == 0) return hipSuccess;
    Args s = a;
    s.m_live_nqb = (int32_t)((a.Lq + 31) / 32);
    hipLaunchKernelGGL(mask_live_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, stream, s, out, n);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// fa_fwd_w64: the unmasked kernel with 64 query rows per wave.
//
// One workgroup = 4 waves = 256 query rows of one (batch, head), one wave per
// SIMD with 512 registers: O^T (128 floats per lane) and the Q fragments
// (64) stay in AGPRs as MFMA operands.  A K or V^T fragment read from LDS
// now feeds two MFMAs (one per 32-row block), which halves the LDS operand
// traffic per flop of fa_fwd_d128, and the softmax of one tile runs between
// the matrix products of the next tile in the same wave.  The key loop is
// hand-scheduled ISA (kd_fa_w64_loop.inc, written by gen_w64_loop.py);
// its arithmetic is fa_fwd_d128's step for step, so that both kernels give
// bitwise identical results.  K and V stream global -> LDS through buffer
// resources whose record count stops at the last key (a DMA past it reads
// zeros).  The loop runs every 64-key tile (Lk >= 64); in a partial last
// tile the scores of the keys past Lk (zero rows) are set to -inf before
// any softmax reads them, which gives them fa_fwd_d128's tail weights (0)
// and row max (the valid keys').
// LDS: K and V tiles double-buffered (0 .. 64 KiB), the Q fragments handed
// to the loop (64 .. 128 KiB).  The loop ends by storing O / l itself: each
// wave stages its rows in 8 KiB over the K/V tiles and stores whole 128-byte
// lines through a buffer resource that ends at the last valid row.
#include "kd_fa_w64_loop.inc"

constexpr int kW64Lds = 131072;
constexpr int kW64QOff = 65536;

template <typename T, int RM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void fa_fwd_w64(Args a) {
    typedef Elem<T> E;
    typedef typename E::vec8 vec8;
    __shared__ __attribute__((aligned(1024))) char lds_arr[kW64Lds];
    lds_t *const lds = LDS_PTR(char, lds_arr);
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int hi = lane >> 5;

    // block order as in fa_fwd_d128 (unmasked: the q-tiles of one head in a
    // row, each XCD a contiguous range)
    const int pid = blockIdx.x;
    const int per = a.n_blocks >> 3;
    const int lid = pid < per * 8 ? (pid & 7) * per + (pid >> 3) : pid;
    const int qt = lid % a.n_qt;
    const int bh = lid / a.n_qt;
    const int h = bh % a.H;
    const int b = bh / a.H;

    // DMA: round j of wave w fills tile rows 4*(w + 4j) .. +3 (1 KiB at
    // LDS (w + 4j) * 1024); lane: row 4*(w + 4j) + lane/16, chunk lane%16
    const int r0 = 4 * wave + (lane >> 4);
    const int pc = lane & 15;
    uint32_t kdma[4], vdma[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        kdma[j] = (uint32_t)(k_row_of(r0) + 16 * j) * (uint32_t)a.k_nb1 + ((pc ^ (r0 & 15)) << 4);
        vdma[j] = (uint32_t)(r0 + 16 * j) * (uint32_t)a.v_nb1 + ((pc ^ v_swz(r0)) << 4);
    }
    const uint32_t dmab = __builtin_amdgcn_readfirstlane(lds0 + wave * 1024);
    // buffer resources of this head's K and V: base, no stride, records up to
    // the end of key Lk-1, raw dword access
    const char *kbase = a.k + (int64_t)(h / a.rk2) * a.k_nb2 + (int64_t)(b / a.rk3) * a.k_nb3;
    const char *vbase = a.v + (int64_t)(h / a.rv2) * a.v_nb2 + (int64_t)(b / a.rv3) * a.v_nb3;
    const uint64_t ka = (uint64_t)(uintptr_t)kbase, va = (uint64_t)(uintptr_t)vbase;
    const uint32_t kw0 = __builtin_amdgcn_readfirstlane((uint32_t)ka);
    const uint32_t kw1 = __builtin_amdgcn_readfirstlane((uint32_t)(ka >> 32) & 0xffffu);
    const uint32_t kw2 = __builtin_amdgcn_readfirstlane((uint32_t)(a.Lk - 1) * (uint32_t)a.k_nb1 + 256u);
    const uint32_t vw0 = __builtin_amdgcn_readfirstlane((uint32_t)va);
    const uint32_t vw1 = __builtin_amdgcn_readfirstlane((uint32_t)(va >> 32) & 0xffffu);
    const uint32_t vw2 = __builtin_amdgcn_readfirstlane((uint32_t)(a.Lk - 1) * (uint32_t)a.v_nb1 + 256u);
    const uint32_t rw3 = 0x00020000u;
    const uint32_t ktile = __builtin_amdgcn_readfirstlane(64u * (uint32_t)a.k_nb1);
    const uint32_t vtile = __builtin_amdgcn_readfirstlane(64u * (uint32_t)a.v_nb1);
    // K(0), V(0) and K(1) by DMA ahead of the Q loads, so that the two round
    // trips overlap (the wait for Q, later in the same in-order counter,
    // covers them; the tiles land below the Q fragments' LDS)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile(KD_W64_PRE
                 :
                 : [kdma0] "v"(kdma[0]), [kdma1] "v"(kdma[1]), [kdma2] "v"(kdma[2]), [kdma3] "v"(kdma[3]),
                   [vdma0] "v"(vdma[0]), [vdma1] "v"(vdma[1]), [vdma2] "v"(vdma[2]), [vdma3] "v"(vdma[3]),
                   [dmab] "s"(dmab), [kw0] "s"(kw0), [kw1] "s"(kw1), [kw2] "s"(kw2), [kw3] "s"(rw3),
                   [vw0] "s"(vw0), [vw1] "s"(vw1), [vw2] "s"(vw2), [vw3] "s"(rw3), [ktile] "s"(ktile),
                   [vtile] "s"(vtile)
                 : KD_W64_PRE_CLOBBERS);
#pragma clang diagnostic pop

    // Q fragments of the wave's two 32-row blocks -> LDS, lane-major
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const int q_row = qt * 256 + wave * 64 + qb * 32 + l32;
        const int q_ld = q_row < a.Lq ? q_row : a.Lq - 1;
        vec8 qf[8];
        load_q_frags<T, RM, true>(a, q_ld, h, b, hi, qf);
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
            *reinterpret_cast<__attribute__((address_space(3))) vec8 *>(
                lds + kW64QOff + wave * 16384 + (qb * 8 + ks) * 1024 + lane * 16) = qf[ks];
    }

    // per-lane LDS offsets of the operand reads (fa_fwd_d128's k_rd / v_rd)
    uint32_t krd[8], vrd[4];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) krd[ks] = lds0 + l32 * 256 + (((2 * ks + hi) ^ (lane & 15)) << 4);
    const int v_sub = (lane & 15) >> 2;
    const int v_c_lo = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
#pragma unroll
    for (int dblk = 0; dblk < 4; ++dblk)
        vrd[dblk] = lds0 + 2048 * hi + 256 * v_sub + (((4 * dblk + v_c_lo) ^ v_swz(v_sub)) << 4) + 8 * (lane & 1);
    const uint32_t qrd = lds0 + kW64QOff + wave * 16384 + lane * 16;
    // O: this wave's 64 rows from a buffer resource whose record count ends
    // at the last valid row (0 when none is), staged per wave in 8 KiB of the
    // K/V tiles
    const uint32_t rawb = __builtin_amdgcn_readfirstlane(lds0 + wave * 8192);
    const uint32_t ot = a.o_type == KD_FA_TYPE_F32 ? 0u : a.o_type == KD_FA_TYPE_BF16 ? 1u : 2u;
    const uint32_t onb2 = (uint32_t)a.o_nb2;
    const uint32_t o8 = 8u * onb2;
    const int orow = qt * 256 + wave * 64;
    const char *ob = a.o + (int64_t)b * a.o_nb3 + (int64_t)h * a.o_nb1 + (int64_t)orow * a.o_nb2;
    const int o_valid = min(a.Lq - orow, 64);
    const uint32_t ow0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)ob);
    const uint32_t ow1 = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)(uintptr_t)ob >> 32) & 0xffffu);
    const uint32_t ow2 = __builtin_amdgcn_readfirstlane(
        o_valid > 0 ? (uint32_t)(o_valid - 1) * onb2 + (ot == 0 ? 512u : 256u) : 0u);

    // every tile, a partial last one included: the loop sets the scores of
    // its keys past Lk to -inf in step mstep (= n - 2; none when the last
    // tile is whole), against thr = its valid keys - 8 * (lane / 32)
    const uint32_t n_tiles = __builtin_amdgcn_readfirstlane((uint32_t)((a.Lk + kBN - 1) / kBN));
    const int rem = a.Lk - kBN * ((int)n_tiles - 1);
    const uint32_t mstep = __builtin_amdgcn_readfirstlane(rem < kBN ? n_tiles - 2 : 0xffffffffu);
    const int thr = rem - 8 * hi;
    const float c2 = __builtin_fabsf(a.scale_log2);

    __syncthreads();
#define KD_W64_OPERANDS                                                                              \
    [krd0] "v"(krd[0]), [krd1] "v"(krd[1]), [krd2] "v"(krd[2]), [krd3] "v"(krd[3]), [krd4] "v"(krd[4]), \
        [krd5] "v"(krd[5]), [krd6] "v"(krd[6]), [krd7] "v"(krd[7]), [vrd0] "v"(vrd[0]), [vrd1] "v"(vrd[1]), \
        [vrd2] "v"(vrd[2]), [vrd3] "v"(vrd[3]), [kdma0] "v"(kdma[0]), [kdma1] "v"(kdma[1]),                \
        [kdma2] "v"(kdma[2]), [kdma3] "v"(kdma[3]), [vdma0] "v"(vdma[0]), [vdma1] "v"(vdma[1]),            \
        [vdma2] "v"(vdma[2]), [vdma3] "v"(vdma[3]), [qrd] "v"(qrd), [kw0] "s"(kw0), [kw1] "s"(kw1),        \
        [kw2] "s"(kw2), [kw3] "s"(rw3), [vw0] "s"(vw0), [vw1] "s"(vw1), [vw2] "s"(vw2), [vw3] "s"(rw3),    \
        [rw3] "s"(rw3), [ktile] "s"(ktile), [vtile] "s"(vtile), [n] "s"(n_tiles), [c2] "s"(c2),              \
        [dmab] "s"(dmab), [mstep] "s"(mstep), [thr] "v"(thr), [rawb] "s"(rawb), [ow0] "s"(ow0),             \
        [ow1] "s"(ow1), [ow2] "s"(ow2), [o8] "s"(o8), [onb2] "s"(onb2), [ot] "s"(ot)
// (m0 is in the clobber list for the reader; the compiler reserves it and
// uses it nowhere in this kernel)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    if constexpr (__is_same(T, __bf16))
        asm volatile(KD_W64_LOOP_BF16 : : KD_W64_OPERANDS : KD_W64_CLOBBERS);
    else
        asm volatile(KD_W64_LOOP_F16 : : KD_W64_OPERANDS : KD_W64_CLOBBERS);
#pragma clang diagnostic pop
#undef KD_W64_OPERANDS
}

template <typename T>
static hipError_t launch_w64_t(const Args &a, hipStream_t s) {
    switch (a.rope_mode) {
    case KD_FA_ROPE_TABLE:
        hipLaunchKernelGGL((fa_fwd_w64<T, KD_FA_ROPE_TABLE>), dim3(a.n_blocks), dim3(256), 0, s, a);
        break;
    case KD_FA_ROPE_AXES:
        hipLaunchKernelGGL((fa_fwd_w64<T, KD_FA_ROPE_AXES>), dim3(a.n_blocks), dim3(256), 0, s, a);
        break;
    default:
        hipLaunchKernelGGL((fa_fwd_w64<T, KD_FA_ROPE_NONE>), dim3(a.n_blocks), dim3(256), 0, s, a);
        break;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// fa_fwd_xlong64: the persistent long-prompt kernel on fa_fwd_w64's key loop,
// for F32 Q (the text cross-attention as ops::attention hands it over:
// src/core/ops.hpp:122-124, src/models/crossdit.hpp:198) and Q in K's type
// (Q16: its fragments are its rows' 16-byte chunks, DMA'd straight into the
// fragment area; a negative scale, which load_q_frags applies by negating Q,
// is not taken then).
//
// One 4-wave workgroup per CU walks units of 256 query rows of one (b, h),
// as fa_fwd_xlong does (XCD-contiguous unit ranges, workgroup j of an XCD
// takes units j, j + w, ...).  Each unit runs one hand-scheduled block
// (kd_fa_xlong64_loop.inc, written by gen_w64_loop.py): fa_fwd_w64's loop
// with
//   * the next unit's Q brought in during steps 0-4: each wave DMAs 128
//     bytes of each of its 64 F32 rows per step into its raw area and, a step
//     later, rounds them to the operand type into its Q fragment area, from
//     which the next unit loads its fragments;
//   * the next unit's K(0), K(1) fetched by the unit's last step and V(0)
//     once every wave is done with the V buffers, before the O stores, so
//     that the next unit's first wait is for those three tiles and not for
//     the stores (loads and stores complete in issue order: the end of its
//     first step, which waits for that step's tiles, waits for them);
//   * the O epilogue in the block: O / l staged per 32 rows in the raw area
//     and stored, non-temporal, as whole 128-byte lines through a buffer
//     resource that ends at the last valid row (rows past Lq are not
//     written).
// Per row the arithmetic is fa_fwd_w64's (and so fa_fwd_d128's): the
// results are bitwise equal.
//
// LDS: K and V tiles 2 x 2 x 16 KiB, per wave 16 KiB of Q fragments (64 ..
// 128 KiB) and 8 KiB of raw Q pieces / O staging (128 .. 160 KiB).
// ---------------------------------------------------------------------------
#include "kd_fa_xlong64_loop.inc"

constexpr int kX64QOff = 65536;
constexpr int kX64RawOff = 131072;
constexpr int kX64Raw = 8192;
constexpr int kX64Lds = 163840;
static_assert(kX64RawOff + 4 * kX64Raw == kX64Lds, "LDS plan");

template <typename T, bool Q16>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void fa_fwd_xlong64(Args a) {
    typedef Elem<T> E;
    typedef typename E::vec8 vec8;
    __shared__ __attribute__((aligned(1024))) char lds_arr[kX64Lds];
    lds_t *const lds = LDS_PTR(char, lds_arr);
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int hi = lane >> 5;

    // this workgroup's units: j, j + wpx, ... within its XCD's range
    const int n_units = a.n_blocks;
    const int wpx = (int)(gridDim.x >> 3);
    const int per = (n_units + 7) >> 3;
    const int xcd = (int)(blockIdx.x & 7);
    const int u_end = min((xcd + 1) * per, n_units);
    int u = xcd * per + (int)(blockIdx.x >> 3);
    if (u >= u_end) return;   // before any barrier

    // the first unit's Q fragments -> LDS (load_q_frags: rounding and sign)
    {
        const int qt = u % a.n_qt, bh = u / a.n_qt;
        const int h = bh % a.H, b = bh / a.H;
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            const int q_row = qt * 256 + wave * 64 + qb * 32 + l32;
            const int q_ld = q_row < a.Lq ? q_row : a.Lq - 1;
            vec8 qf[8];
            load_q_frags<T, KD_FA_ROPE_NONE, true>(a, q_ld, h, b, hi, qf);
#pragma unroll
            for (int ks = 0; ks < 8; ++ks)
                *reinterpret_cast<__attribute__((address_space(3))) vec8 *>(
                    lds + kX64QOff + wave * 16384 + (qb * 8 + ks) * 1024 + lane * 16) = qf[ks];
        }
    }

    // per-lane LDS offsets of the operand reads and the K/V DMA (fa_fwd_w64's)
    uint32_t krd[8], vrd[4];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) krd[ks] = lds0 + l32 * 256 + (((2 * ks + hi) ^ (lane & 15)) << 4);
    const int v_sub = (lane & 15) >> 2;
    const int v_c_lo = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
#pragma unroll
    for (int dblk = 0; dblk < 4; ++dblk)
        vrd[dblk] = lds0 + 2048 * hi + 256 * v_sub + (((4 * dblk + v_c_lo) ^ v_swz(v_sub)) << 4) + 8 * (lane & 1);
    const int r0 = 4 * wave + (lane >> 4);
    const int pc = lane & 15;
    uint32_t kdma[4], vdma[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        kdma[j] = (uint32_t)(k_row_of(r0) + 16 * j) * (uint32_t)a.k_nb1 + ((pc ^ (r0 & 15)) << 4);
        vdma[j] = (uint32_t)(r0 + 16 * j) * (uint32_t)a.v_nb1 + ((pc ^ v_swz(r0)) << 4);
    }
    const uint32_t qrd = lds0 + kX64QOff + wave * 16384 + lane * 16;
    const uint32_t dmab = __builtin_amdgcn_readfirstlane(lds0 + wave * 1024);
    const uint32_t rawb = __builtin_amdgcn_readfirstlane(lds0 + kX64RawOff + wave * kX64Raw);
    const uint32_t rawdelta = __builtin_amdgcn_readfirstlane((uint32_t)(kX64RawOff - kX64QOff) - wave * 8192u);
    // the next unit's Q rows: lane l reads row 32 qb + l % 32 of its wave
    // (F32: the 16-byte halves of its 32-byte chunk; 16-bit: its fragment's
    // 16-byte chunk)
    const uint32_t qoff0 = (uint32_t)l32 * (uint32_t)a.q_nb1 + (Q16 ? 16u : 32u) * (uint32_t)hi;
    const uint32_t qoff1 = qoff0 + 32u * (uint32_t)a.q_nb1;
    const uint32_t qfb = __builtin_amdgcn_readfirstlane(lds0 + kX64QOff + wave * 16384);
    const uint32_t qrow_bytes = Q16 ? 256u : 512u;

    const uint32_t rw3 = 0x00020000u;
    const uint32_t kw2 = __builtin_amdgcn_readfirstlane((uint32_t)(a.Lk - 1) * (uint32_t)a.k_nb1 + 256u);
    const uint32_t vw2 = __builtin_amdgcn_readfirstlane((uint32_t)(a.Lk - 1) * (uint32_t)a.v_nb1 + 256u);
    const uint32_t ktile = __builtin_amdgcn_readfirstlane(64u * (uint32_t)a.k_nb1);
    const uint32_t vtile = __builtin_amdgcn_readfirstlane(64u * (uint32_t)a.v_nb1);
    const uint32_t n_tiles = __builtin_amdgcn_readfirstlane((uint32_t)((a.Lk + kBN - 1) / kBN));
    const int rem = a.Lk - kBN * ((int)n_tiles - 1);
    const uint32_t mstep = __builtin_amdgcn_readfirstlane(rem < kBN ? n_tiles - 2 : 0xffffffffu);
    const int thr = rem - 8 * hi;
    const float c2 = __builtin_fabsf(a.scale_log2);
    const uint32_t qsgn = a.scale_log2 < 0.0f ? 0x80008000u : 0u;
    const uint32_t ot = a.o_type == KD_FA_TYPE_F32 ? 0u : a.o_type == KD_FA_TYPE_BF16 ? 1u : 2u;
    const uint32_t orow_bytes = ot == 0 ? 512u : 256u;
    const uint32_t onb2 = (uint32_t)a.o_nb2;
    const uint32_t o8 = 8u * onb2;

    // buffer resource words of a unit's K, V (from its (b, h)), Q and O
    // (from this wave's first row; the record count ends at the last valid
    // row, 0 when none is)
    auto res_lo = [](const char *p) { return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p); };
    auto res_hi = [](const char *p) {
        return __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)(uintptr_t)p >> 32) & 0xffffu);
    };
    uint32_t first = 1;
    for (;;) {
        const int nu = u + wpx;
        const bool has_next = nu < u_end;
        const int qt = u % a.n_qt, bh = u / a.n_qt;
        const int h = bh % a.H, b = bh / a.H;
        const char *kb = a.k + (int64_t)(h / a.rk2) * a.k_nb2 + (int64_t)(b / a.rk3) * a.k_nb3;
        const char *vb = a.v + (int64_t)(h / a.rv2) * a.v_nb2 + (int64_t)(b / a.rv3) * a.v_nb3;
        const int orow = qt * 256 + wave * 64;
        const char *ob = a.o + (int64_t)b * a.o_nb3 + (int64_t)h * a.o_nb1 + (int64_t)orow * a.o_nb2;
        const int o_valid = min(a.Lq - orow, 64);
        const uint32_t ow2 = o_valid > 0 ? (uint32_t)(o_valid - 1) * onb2 + orow_bytes : 0u;
        const char *nkb = kb, *nvb = vb, *nqb = a.q;
        uint32_t nkw2 = 0, nvw2 = 0, nqw2 = 0;
        if (has_next) {
            const int nqt = nu % a.n_qt, nbh = nu / a.n_qt;
            const int nh = nbh % a.H, nb = nbh / a.H;
            nkb = a.k + (int64_t)(nh / a.rk2) * a.k_nb2 + (int64_t)(nb / a.rk3) * a.k_nb3;
            nvb = a.v + (int64_t)(nh / a.rv2) * a.v_nb2 + (int64_t)(nb / a.rv3) * a.v_nb3;
            const int qrow = nqt * 256 + wave * 64;
            nqb = a.q + (int64_t)nh * a.q_nb2 + (int64_t)nb * a.q_nb3 + (int64_t)qrow * a.q_nb1;
            const int q_valid = min(a.Lq - qrow, 64);
            nkw2 = kw2;
            nvw2 = vw2;
            nqw2 = q_valid > 0 ? (uint32_t)(q_valid - 1) * (uint32_t)a.q_nb1 + qrow_bytes : 0u;
        }
        const uint32_t kw0 = res_lo(kb), kw1 = res_hi(kb), vw0 = res_lo(vb), vw1 = res_hi(vb);
        const uint32_t ow0 = res_lo(ob), ow1 = res_hi(ob);
        const uint32_t nkw0 = res_lo(nkb), nkw1 = res_hi(nkb), nvw0 = res_lo(nvb), nvw1 = res_hi(nvb);
        const uint32_t nqw0 = res_lo(nqb), nqw1 = res_hi(nqb);
        const uint32_t ow2u = __builtin_amdgcn_readfirstlane(ow2);
        const uint32_t nkw2u = __builtin_amdgcn_readfirstlane(nkw2), nvw2u = __builtin_amdgcn_readfirstlane(nvw2);
        const uint32_t nqw2u = __builtin_amdgcn_readfirstlane(nqw2);
#define KD_XL64_OPERANDS                                                                                      \
    [krd0] "v"(krd[0]), [krd1] "v"(krd[1]), [krd2] "v"(krd[2]), [krd3] "v"(krd[3]), [krd4] "v"(krd[4]),       \
        [krd5] "v"(krd[5]), [krd6] "v"(krd[6]), [krd7] "v"(krd[7]), [vrd0] "v"(vrd[0]), [vrd1] "v"(vrd[1]),   \
        [vrd2] "v"(vrd[2]), [vrd3] "v"(vrd[3]), [kdma0] "v"(kdma[0]), [kdma1] "v"(kdma[1]),                  \
        [kdma2] "v"(kdma[2]), [kdma3] "v"(kdma[3]), [vdma0] "v"(vdma[0]), [vdma1] "v"(vdma[1]),              \
        [vdma2] "v"(vdma[2]), [vdma3] "v"(vdma[3]), [qrd] "v"(qrd), [thr] "v"(thr), [qoff0] "v"(qoff0),     \
        [qoff1] "v"(qoff1), [kw0] "s"(kw0), [kw1] "s"(kw1), [kw2] "s"(kw2), [rw3] "s"(rw3), [vw0] "s"(vw0),   \
        [vw1] "s"(vw1), [vw2] "s"(vw2), [ktile] "s"(ktile), [vtile] "s"(vtile), [n] "s"(n_tiles),            \
        [c2] "s"(c2), [dmab] "s"(dmab), [mstep] "s"(mstep), [first] "s"(first), [nkw0] "s"(nkw0),            \
        [nkw1] "s"(nkw1), [nkw2] "s"(nkw2u), [nvw0] "s"(nvw0), [nvw1] "s"(nvw1), [nvw2] "s"(nvw2u),           \
        [nqw0] "s"(nqw0), [nqw1] "s"(nqw1), [nqw2] "s"(nqw2u), [ow0] "s"(ow0), [ow1] "s"(ow1),               \
        [ow2] "s"(ow2u), [o8] "s"(o8), [onb2] "s"(onb2), [ot] "s"(ot), [qsgn] "s"(qsgn), [rawb] "s"(rawb),     \
        [rawdelta] "s"(rawdelta), [qfb] "s"(qfb)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
        if constexpr (__is_same(T, __bf16) && !Q16)
            asm volatile(KD_XL64_UNIT_BF16 : : KD_XL64_OPERANDS : KD_XL64_CLOBBERS);
        else if constexpr (!Q16)
            asm volatile(KD_XL64_UNIT_F16 : : KD_XL64_OPERANDS : KD_XL64_CLOBBERS);
        else if constexpr (__is_same(T, __bf16))
            asm volatile(KD_XL64_UNIT_BF16_Q16 : : KD_XL64_OPERANDS : KD_XL64_CLOBBERS);
        else
            asm volatile(KD_XL64_UNIT_F16_Q16 : : KD_XL64_OPERANDS : KD_XL64_CLOBBERS);
#pragma clang diagnostic pop
#undef KD_XL64_OPERANDS
        if (!has_next) break;
        u = nu;
        first = 0;
    }
}

template <typename T>
static void launch_xlong64_t(const Args &a, hipStream_t s) {
    // at most one workgroup per CU (256), a multiple of the 8 XCDs
    const int g = a.n_blocks < 256 ? (a.n_blocks + 7) / 8 * 8 : 256;
    if (a.q_type == KD_FA_TYPE_F32)
        hipLaunchKernelGGL((fa_fwd_xlong64<T, false>), dim3(g), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((fa_fwd_xlong64<T, true>), dim3(g), dim3(256), 0, s, a);
}

hipError_t launch_xlong64(const Args &a, int kv_type, hipStream_t s) {
    if (kv_type == KD_FA_TYPE_BF16)
        launch_xlong64_t<__bf16>(a, s);
    else
        launch_xlong64_t<_Float16>(a, s);
    return hipGetLastError();
}

template <typename T>
static void launch_xres_t(const Args &a, hipStream_t s) {
    const dim3 g(a.n_blocks), b(64 * kXWaves);
    const bool q32 = a.q_type == KD_FA_TYPE_F32;
    if (a.m) {
        if (q32) hipLaunchKernelGGL((fa_fwd_xres<T, true, true>), g, b, 0, s, a);
        else hipLaunchKernelGGL((fa_fwd_xres<T, true, false>), g, b, 0, s, a);
    } else {
        if (q32) hipLaunchKernelGGL((fa_fwd_xres<T, false, true>), g, b, 0, s, a);
        else hipLaunchKernelGGL((fa_fwd_xres<T, false, false>), g, b, 0, s, a);
    }
}

hipError_t launch_xres(const Args &a, int kv_type, hipStream_t s) {
    if (kv_type == KD_FA_TYPE_BF16)
        launch_xres_t<__bf16>(a, s);
    else
        launch_xres_t<_Float16>(a, s);
    return hipGetLastError();
}

template <typename T>
static void launch_xlong_t(const Args &a, hipStream_t s) {
    // at most one workgroup per CU (256), a multiple of the 8 XCDs
    const int g = a.n_blocks < 256 ? (a.n_blocks + 7) / 8 * 8 : 256;
    if (a.q_type == KD_FA_TYPE_F32)
        hipLaunchKernelGGL((fa_fwd_xlong<T, true>), dim3(g), dim3(64 * kLWaves), 0, s, a);
    else
        hipLaunchKernelGGL((fa_fwd_xlong<T, false>), dim3(g), dim3(64 * kLWaves), 0, s, a);
}

hipError_t launch_xlong(const Args &a, int kv_type, hipStream_t s) {
    if (kv_type == KD_FA_TYPE_BF16)
        launch_xlong_t<__bf16>(a, s);
    else
        launch_xlong_t<_Float16>(a, s);
    return hipGetLastError();
}

hipError_t launch_w64(const Args &a, int kv_type, hipStream_t stream) {
    return kv_type == KD_FA_TYPE_BF16 ? launch_w64_t<__bf16>(a, stream) : launch_w64_t<_Float16>(a, stream);
}

template <typename T, bool M, int R, bool KR, int NW>
static hipError_t launch_t(const Args &a, hipStream_t stream) {
    hipLaunchKernelGGL((fa_fwd_d128<T, M, R, KR, NW>), dim3(a.n_blocks), dim3(64 * NW), 0, stream, a);
    return hipGetLastError();
}

// the instances d128_waves chooses: K transformed on load 8 waves, masked 4,
// unmasked 4 or 8
template <typename T, bool M, int R>
static hipError_t launch_w(const Args &a, bool k_rope, int waves, hipStream_t s) {
    if (k_rope) return waves == 8 ? launch_t<T, M, R, true, 8>(a, s) : hipErrorInvalidValue;
    if constexpr (M) return waves == 4 ? launch_t<T, M, R, false, 4>(a, s) : hipErrorInvalidValue;
    else
        return waves == 4 ? launch_t<T, M, R, false, 4>(a, s)
                          : waves == 8 ? launch_t<T, M, R, false, 8>(a, s) : hipErrorInvalidValue;
}

template <typename T, bool M>
static hipError_t launch_r(const Args &a, bool k_rope, int waves, hipStream_t s) {
    switch (a.rope_mode) {
    case KD_FA_ROPE_TABLE:
        return launch_w<T, M, KD_FA_ROPE_TABLE>(a, k_rope, waves, s);
    case KD_FA_ROPE_AXES:
        return launch_w<T, M, KD_FA_ROPE_AXES>(a, k_rope, waves, s);
    default:
        return launch_w<T, M, KD_FA_ROPE_NONE>(a, k_rope, waves, s);
    }
}

hipError_t launch(const Args &a, int kv_type, bool k_rope, int waves, hipStream_t stream) {
    const bool mask = a.m != nullptr;
    if (kv_type == KD_FA_TYPE_BF16)
        return mask ? launch_r<__bf16, true>(a, k_rope, waves, stream)
                    : launch_r<__bf16, false>(a, k_rope, waves, stream);
    return mask ? launch_r<_Float16, true>(a, k_rope, waves, stream)
                : launch_r<_Float16, false>(a, k_rope, waves, stream);
}

// ---------------------------------------------------------------------------
// Pre-pass of the workspace entry points: ops::rms_norm (kn_w) and
// rope::apply (src/rope.hpp:109-155) on K with the same F32 arithmetic as the
// in-kernel transform, rounded to the operand type T (K may be stored in
// F32), written to out + key * o.key + head * o.head + batch * o.batch: a
// contiguous [D, Lk, Hkv, Bk] workspace, or rows of the call's own output
// buffer that the attention writes later (the staged path).  In the same
// pass, an F32 V (the projection output ops::attention casts,
// src/core/ops.hpp:168-169) is rounded to T into vout.  One thread per
// 8-element chunk; the 16 chunks of a row are 16 consecutive lanes, which
// reduce the row's squares together.
// ---------------------------------------------------------------------------
template <typename T, int RM, int kRopeKPairs>
__global__ __launch_bounds__(256) void rope_k_kernel(Args a, char *out, KStrides o, char *vout, KStrides vo,
                                                     int n_hb) {
    typedef Elem<T> E;
    // heads of the (b, h) pairs: K's, or V's in a pass that casts V only
    // (when both are written, K and V have the same heads and batches)
    const int nh = out ? a.H / a.rk2 : a.H / a.rv2;
    // x: 16 keys per workgroup, 16 lanes per key (one 16-byte output chunk
    // each); y: groups of kRopeKPairs (b, h) pairs (1 or 4), uniform per workgroup
    // (no division per chunk).  The chunk's rotation pairs and norm weights
    // are the same for every (b, h): loaded once.  The group's K (and V)
    // chunks are loaded before any is used, branch-free (both 16-byte halves
    // of an F32 chunk, or the 16-bit chunk twice; past the last pair, the
    // last pair again, not stored).
    const int key = (int)blockIdx.x * 16 + (int)(threadIdx.x >> 4);
    const int c = (int)(threadIdx.x & 15);
    if (key >= a.Lk) return;
    const bool k32 = a.k_type == KD_FA_TYPE_F32;
    const bool kbf = a.k_type == KD_FA_TYPE_BF16;
    f32x4 cs0 = {}, cs1 = {};
    if (RM != KD_FA_ROPE_NONE) {
        const float *cp = rope_ptr<RM>(a, key, c * 8);
        cs0 = *reinterpret_cast<const f32x4 *>(cp);
        cs1 = *reinterpret_cast<const f32x4 *>(cp + 4);
    }
    const bool knorm = a.kn_w != nullptr;
    f32x4 wn0 = {}, wn1 = {};
    if (knorm) {
        wn0 = *reinterpret_cast<const f32x4 *>(a.kn_w + c * 8);
        wn1 = *reinterpret_cast<const f32x4 *>(a.kn_w + c * 8 + 4);
    }
    const char *const kkey = a.k + (int64_t)key * a.k_nb1 + (k32 ? c * 32 : c * 16);
    const char *const vkey = a.v + (int64_t)key * a.v_nb1 + c * 32;
    for (int g0 = (int)blockIdx.y * kRopeKPairs; g0 < n_hb; g0 += (int)gridDim.y * kRopeKPairs) {
        u32x4 ra[kRopeKPairs], rb[kRopeKPairs], va[kRopeKPairs], vb[kRopeKPairs];
        if (out) {
#pragma unroll
            for (int i = 0; i < kRopeKPairs; ++i) {
                const int hb = min(g0 + i, n_hb - 1);
                const char *src = kkey + (int64_t)(hb % nh) * a.k_nb2 + (int64_t)(hb / nh) * a.k_nb3;
                ra[i] = ld16(src);
                rb[i] = ld16(src + (k32 ? 16 : 0));
            }
        }
        if (vout) {
#pragma unroll
            for (int i = 0; i < kRopeKPairs; ++i) {
                const int hb = min(g0 + i, n_hb - 1);
                const char *src = vkey + (int64_t)(hb % nh) * a.v_nb2 + (int64_t)(hb / nh) * a.v_nb3;
                va[i] = ld16(src);
                vb[i] = ld16(src + 16);
            }
        }
        if (out) {
#pragma unroll
            for (int i = 0; i < kRopeKPairs; ++i) {
                const int hb = g0 + i;
                if (hb >= n_hb) break;
                float x[8];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t w16 = ra[i][j];
                    const float lo16 = kbf ? bf16_lo(w16) : f16_lo(w16);
                    const float hi16 = kbf ? bf16_hi(w16) : f16_hi(w16);
                    const float e0 = __uint_as_float(j < 2 ? ra[i][2 * j] : rb[i][2 * j - 4]);
                    const float e1 = __uint_as_float(j < 2 ? ra[i][2 * j + 1] : rb[i][2 * j - 3]);
                    x[2 * j] = k32 ? e0 : lo16;
                    x[2 * j + 1] = k32 ? e1 : hi16;
                }
                if (knorm) rms_apply8(x, rms_scale(sum16_f64(sum_sq8(x)), a.norm_eps), wn0, wn1);
                if (RM != KD_FA_ROPE_NONE) rotate8(x, cs0, cs1);
                u32x4 w;
                for (int e = 0; e < 4; ++e) w[e] = E::pack2(x[2 * e], x[2 * e + 1]);
                *reinterpret_cast<u32x4 *>(out + (int64_t)key * o.key + (int64_t)(hb % nh) * o.head +
                                           (int64_t)(hb / nh) * o.batch + c * 16) = w;
            }
        }
        if (vout) {
#pragma unroll
            for (int i = 0; i < kRopeKPairs; ++i) {
                const int hb = g0 + i;
                if (hb >= n_hb) break;
                u32x4 w;
                w[0] = E::pack2(__uint_as_float(va[i][0]), __uint_as_float(va[i][1]));
                w[1] = E::pack2(__uint_as_float(va[i][2]), __uint_as_float(va[i][3]));
                w[2] = E::pack2(__uint_as_float(vb[i][0]), __uint_as_float(vb[i][1]));
                w[3] = E::pack2(__uint_as_float(vb[i][2]), __uint_as_float(vb[i][3]));
                *reinterpret_cast<u32x4 *>(vout + (int64_t)key * vo.key + (int64_t)(hb % nh) * vo.head +
                                           (int64_t)(hb / nh) * vo.batch + c * 16) = w;
            }
        }
    }
}

template <typename T, int P>
static void launch_rope_k_p(const Args &a, dim3 grid, char *o, const KStrides &st, char *vo, const KStrides &vst,
                            int n_hb, hipStream_t stream) {
    switch (o ? a.rope_mode : KD_FA_ROPE_NONE) {   // a V-only pass rotates nothing
    case KD_FA_ROPE_TABLE:
        hipLaunchKernelGGL((rope_k_kernel<T, KD_FA_ROPE_TABLE, P>), grid, dim3(256), 0, stream, a, o, st, vo, vst,
                           n_hb);
        break;
    case KD_FA_ROPE_AXES:
        hipLaunchKernelGGL((rope_k_kernel<T, KD_FA_ROPE_AXES, P>), grid, dim3(256), 0, stream, a, o, st, vo, vst,
                           n_hb);
        break;
    default:
        hipLaunchKernelGGL((rope_k_kernel<T, KD_FA_ROPE_NONE, P>), grid, dim3(256), 0, stream, a, o, st, vo, vst,
                           n_hb);
        break;
    }
}

hipError_t launch_rope_k(const Args &a, int kv_type, int heads, int batch, void *out, const KStrides &st,
                         void *vout, const KStrides &vst, hipStream_t stream) {
    const int64_t n_hb = (int64_t)heads * batch;
    if (a.Lk == 0 || n_hb == 0 || (!out && !vout)) return hipSuccess;
    // x: 16 keys per workgroup; y: groups of P (b, h) pairs, at most 65,535
    // (a workgroup takes every gridDim.y-th group beyond that).  P = 4 --
    // the rotation pairs loaded once for four heads, four loads in flight
    // per thread -- when that still leaves 2,048 workgroups (62,464 keys x
    // 32 heads: 0.267 -> 0.200 ms), else 1 (short key sets: more
    // workgroups rather than more work per thread).
    const int64_t nx = (a.Lk + 15) / 16;
    const int P = nx * ((n_hb + 3) / 4) >= 2048 ? 4 : 1;
    const int64_t n_g = (n_hb + P - 1) / P;
    const dim3 grid((unsigned)nx, (unsigned)(n_g < 65535 ? n_g : 65535));
    char *o = static_cast<char *>(out);
    char *vo = static_cast<char *>(vout);
    if (kv_type == KD_FA_TYPE_BF16) {
        if (P == 4) launch_rope_k_p<__bf16, 4>(a, grid, o, st, vo, vst, (int)n_hb, stream);
        else launch_rope_k_p<__bf16, 1>(a, grid, o, st, vo, vst, (int)n_hb, stream);
    } else {
        if (P == 4) launch_rope_k_p<_Float16, 4>(a, grid, o, st, vo, vst, (int)n_hb, stream);
        else launch_rope_k_p<_Float16, 1>(a, grid, o, st, vo, vst, (int)n_hb, stream);
    }
    return hipGetLastError();
}

}  // namespace kdfa
