// kd_fa_d512.hip - the D = 512 attention of the 2-D VAE's attention block
// (src/models/vae.hpp:60-101 -> ops::attention, one head, D = channels).
//
// Built with VGPR-form MFMAs (-mllvm -amdgpu-mfma-vgpr-form, see the
// Makefile): O is rescaled by the vector unit every tile, and with the
// accumulators in AGPRs the compiler would copy all of O through VGPRs on
// every tile.  Internal to libkd_fa.so.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kd_fa_device.h"

namespace kdfa {

// fa_fwd_d512: the attention of the 2-D VAE's attention block
// (src/models/vae.hpp:60-101 -> ops::attention with one head, D = channels =
// 512), no mask, no RoPE.
//
// A workgroup is 4 waves and covers R blocks of 32 query rows of one (b, h);
// wave w owns the 128 columns 128w .. 128w+127 of D for both products, so
// that its O (32R rows x 128) and Q (32R rows x 128) stay in registers.  Per
// 32-key tile:
//   S_w^T = K_w Q_w^T over the wave's 128 columns (8 MFMA per row block), K
//           fragments straight from global memory (each wave reads only its
//           columns, once for all R blocks);
//   the four partial scores meet in LDS; wave w runs the online softmax of
//           rows 8Rw .. 8Rw+8R-1 (exact running max, exp2 domain) and writes
//           the weights P (rounded to the operand type), the rescale factor
//           and, at the end, the row sum to LDS for all waves;
//   O_w^T = alpha * O_w^T + V_w^T P^T (8 MFMA per row block), V_w staged by
//           DMA in the wave's own LDS region (NB buffers, no barrier: only
//           that wave reads it) and read transposed with ds_read_b64_tr_b16,
//           each fragment once for all R blocks.
// NB = 2 (R = 2): V(t+1) staged during tile t, one workgroup per CU.  NB = 1
// (R = 1, 54 KB of LDS, 228 registers): two workgroups per CU, so that one
// hides the other's barrier and LDS round trips; V(t+1) is staged once
// PV(t) has read V(t), and K is loaded two tiles ahead instead.
// Two barriers per tile.  Keys past Lk (last tile) load clamped rows and get
// weight 0.  Every K and V byte a workgroup streams serves 32R query rows:
// with R = 2 the key stream of the long latents (16,384 keys, all of them
// re-read by every workgroup) halves.  R = 1 and R = 2 give bitwise equal
// results: the same products, the same sums of the partial scores, and the
// row sums combined in the same tree (4 keys per leaf).
// With a key split (a.n_split > 1, short query sets with a workspace), a
// workgroup runs only its range of key tiles and leaves the unnormalised O,
// running max and row sum of its rows for d512_combine.
constexpr int kD5 = 512;                     // D, four 128-column slices
constexpr int kD5Keys = 32;                    // keys per tile
constexpr int kD5SStride = kD5Keys + 4;        // floats per row of a partial-score block (pad)
constexpr int kD5PStride = kD5Keys + 8;        // 16-bit weights per row of P (pad)
constexpr int kD5VTile = kD5Keys * 256;        // one wave's V tile: 32 keys x 128 columns

static_assert(kD5 == 4 * 128, "one 128-column slice per wave");

template <typename T, int R, int NB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NB == 1 ? 2 : 1, NB == 1 ? 2 : 1)))
void fa_fwd_d512(Args a) {
    typedef Elem<T> E;
    typedef typename E::vec8 vec8;
    constexpr int kRows = 32 * R;                  // query rows per workgroup
    constexpr int kLanesPerRow = 8 / R;            // softmax lanes per row
    constexpr int kKeysPerLane = 4 * R;
    __shared__ __attribute__((aligned(16))) float sS[4][kRows][kD5SStride];
    __shared__ __attribute__((aligned(16))) uint16_t sP[kRows][kD5PStride];
    __shared__ float sAlpha[kRows];
    __shared__ float sL[kRows];
    __shared__ __attribute__((aligned(1024))) char sV[4][NB][kD5VTile];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int hi = lane >> 5;
    // key split (a.n_split > 1): the grid holds n_split copies of the
    // unsplit grid, copy s taking keys [s * split_keys, (s + 1) * split_keys)
    const int split = a.n_split > 1 ? (int)blockIdx.x / a.n_blocks : 0;
    const int blk = (int)blockIdx.x - split * a.n_blocks;
    const int qt = blk % a.n_qt;
    const int bh = blk / a.n_qt;
    const int h = bh % a.H;
    const int b = bh / a.H;
    const int Lk = a.Lk;
    const int k_end = a.n_split > 1 ? min((split + 1) * a.split_keys, Lk) : Lk;
    const int t_begin = a.n_split > 1 ? split * a.split_keys / kD5Keys : 0;
    const int n_tiles = (k_end + kD5Keys - 1) / kD5Keys;   // one past the range's last tile
    const int col0 = 128 * wave;                  // this wave's columns of D

    // Q fragments of the wave's columns (B operands of S_w^T = K_w Q_w^T)
    vec8 qf[R][8];
#pragma unroll
    for (int rb = 0; rb < R; ++rb) {
        const int q_row = qt * kRows + 32 * rb + l32;
        const int q_ld = q_row < a.Lq ? q_row : a.Lq - 1;
        const char *qp = a.q + (int64_t)q_ld * a.q_nb1 + (int64_t)h * a.q_nb2 + (int64_t)b * a.q_nb3;
        const int esz = a.q_type == KD_FA_TYPE_F32 ? 4 : 2;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            float x[8];
            load8_f32(qp + (col0 + ks * 16 + hi * 8) * esz, a.q_type, x);
            u32x4 w;
            for (int j = 0; j < 4; ++j) w[j] = E::pack2(x[2 * j], x[2 * j + 1]);
            if (a.scale_log2 < 0.0f) w ^= (u32x4){0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
            qf[rb][ks] = __builtin_bit_cast(vec8, w);
        }
    }
    const float c2 = __builtin_fabsf(a.scale_log2);

    const char *kbase = a.k + (int64_t)(h / a.rk2) * a.k_nb2 + (int64_t)(b / a.rk3) * a.k_nb3 + col0 * 2;
    const char *vbase = a.v + (int64_t)(h / a.rv2) * a.v_nb2 + (int64_t)(b / a.rv3) * a.v_nb3 + col0 * 2;
    // K fragment of k-step ks: key (tile row) l32, columns ks*16 + hi*8 .. +7
    auto load_k = [&](int t, vec8 kf[8]) __attribute__((always_inline)) {
        int key = t * kD5Keys + l32;
        key = key < Lk ? key : Lk - 1;
        const char *kp = kbase + (int64_t)key * a.k_nb1 + hi * 16;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) kf[ks] = __builtin_bit_cast(vec8, ld16(kp + ks * 32));
    };
    // V tile of this wave: LDS row r (key t*32 + r, clamped) holds the wave's
    // 128 columns, 16-byte chunk c at c ^ v_swz(r); 8 DMA rounds of 4 rows
    const int dma_row = lane >> 4, dma_pc = lane & 15;
    auto issue_v = [&](int t, int buf) __attribute__((always_inline)) {
        lds_t *dst = LDS_PTR(char, sV[wave][buf]);
#pragma unroll
        for (int j = 0; j < kD5Keys / 4; ++j) {
            const int r = 4 * j + dma_row;
            int key = t * kD5Keys + r;
            key = key < Lk ? key : Lk - 1;
            dma16(vbase, (uint32_t)key * (uint32_t)a.v_nb1 + ((dma_pc ^ v_swz(r)) << 4), dst + j * 1024);
        }
    };
    const int v_sub = (lane & 15) >> 2;
    const int v_c_lo = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
    uint32_t v_rd[4];
#pragma unroll
    for (int dblk = 0; dblk < 4; ++dblk)
        v_rd[dblk] = 2048 * hi + 256 * v_sub + (((4 * dblk + v_c_lo) ^ v_swz(v_sub)) << 4) + 8 * (lane & 1);

    f32x16 o[R][4];
#pragma unroll
    for (int rb = 0; rb < R; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[rb][i] = (f32x16){};
    // softmax state of row 8R*wave + lane / (8/R) (the lanes of a row agree);
    // the lane's keys are 4R consecutive ones
    const int srow = 8 * R * wave + lane / kLanesPerRow;
    const int skey = kKeysPerLane * (lane % kLanesPerRow);
    float m_run = -INFINITY, l_run = 0.0f;

    // VMEM order per tile: the V DMA (inline asm, invisible to the
    // compiler's vmcnt bookkeeping) before the K loads, so that the
    // compiler's own waits for K stay exact (loads complete in order) and
    // V(t) has landed once at most the 16 newer loads are in flight
    // NB = 1 (one V buffer per wave, two workgroups per CU): K fragments
    // two tiles ahead in two register sets, V(t+1) staged once PV(t) has
    // read V(t); VMEM order K(t+2) .. V(t+1), so the compiler's wait for K
    // never waits for the V DMA issued after it
    vec8 kf[NB == 1 ? 2 : 1][8];
    if (n_tiles > t_begin) {
        if constexpr (NB == 2) {
            issue_v(t_begin, t_begin & 1);
            load_k(t_begin, kf[0]);
        } else {
            load_k(t_begin, kf[0]);
            if (t_begin + 1 < n_tiles) load_k(t_begin + 1, kf[1]);
            issue_v(t_begin, 0);
        }
    }
    auto tile = [&](int t, auto kb_c) __attribute__((always_inline)) {
        constexpr int kb = decltype(kb_c)::value ? 1 : 0;
        // the Q fragments (read by the matrix unit only) live in AGPRs, so
        // that O, S and the K fragments have the VGPRs to themselves
#pragma unroll
        for (int rb = 0; rb < R; ++rb)
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) asm volatile("" : "+a"(qf[rb][ks]));
        // ---- partial scores over this wave's columns
        f32x16 s[R];
#pragma unroll
        for (int rb = 0; rb < R; ++rb) {
            s[rb] = (f32x16){};
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) s[rb] = E::mfma(kf[kb][ks], qf[rb][ks], s[rb]);
        }
        if constexpr (NB == 2) {
            if (t + 1 < n_tiles) {
                issue_v(t + 1, (t + 1) & 1);
                load_k(t + 1, kf[0]);
            }
        } else {
            if (t + 2 < n_tiles) load_k(t + 2, kf[kb]);
        }
        // element i of lane l: key 8*(i/4) + 4*hi + i%4, query l32
#pragma unroll
        for (int rb = 0; rb < R; ++rb)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *reinterpret_cast<f32x4 *>(&sS[wave][32 * rb + l32][8 * g + 4 * hi]) =
                    (f32x4){s[rb][4 * g], s[rb][4 * g + 1], s[rb][4 * g + 2], s[rb][4 * g + 3]};
        __syncthreads();
        // ---- softmax of the wave's rows: 4R keys per lane
        {
            float sc[kKeysPerLane];
#pragma unroll
            for (int c = 0; c < R; ++c) {
                f32x4 x = *reinterpret_cast<const f32x4 *>(&sS[0][srow][skey + 4 * c]);
#pragma unroll
                for (int w = 1; w < 4; ++w)
                    x += *reinterpret_cast<const f32x4 *>(&sS[w][srow][skey + 4 * c]);
                sc[4 * c] = x.x * c2; sc[4 * c + 1] = x.y * c2; sc[4 * c + 2] = x.z * c2; sc[4 * c + 3] = x.w * c2;
            }
#pragma unroll
            for (int e = 0; e < kKeysPerLane; ++e)
                if (t * kD5Keys + skey + e >= k_end) sc[e] = -INFINITY;
            float mx = sc[0];
#pragma unroll
            for (int e = 1; e < kKeysPerLane; ++e) mx = __builtin_fmaxf(mx, sc[e]);
#pragma unroll
            for (int d = 1; d < kLanesPerRow; d <<= 1) mx = __builtin_fmaxf(mx, __shfl_xor(mx, d));
            const float m_new = __builtin_fmaxf(m_run, mx);
            const float alpha = m_new == m_run ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
            const float mu = m_new == -INFINITY ? 0.0f : m_new;
            float p[kKeysPerLane];
#pragma unroll
            for (int e = 0; e < kKeysPerLane; ++e) p[e] = __builtin_amdgcn_exp2f(sc[e] - mu);
            // row sum: 4-key leaves (p0 + p1) + (p2 + p3) combined pairwise,
            // the pairs within the lane first, then across lanes
            float ps = (p[0] + p[1]) + (p[2] + p[3]);
            if constexpr (R == 2) ps = ps + ((p[4] + p[5]) + (p[6] + p[7]));
#pragma unroll
            for (int d = 1; d < kLanesPerRow; d <<= 1) ps += __shfl_xor(ps, d);
            l_run = l_run * alpha + ps;
#pragma unroll
            for (int c = 0; c < R; ++c) {
                const u32x2 w = {E::pack2(p[4 * c], p[4 * c + 1]), E::pack2(p[4 * c + 2], p[4 * c + 3])};
                *reinterpret_cast<u32x2 *>(&sP[srow][skey + 4 * c]) = w;
            }
            if (lane % kLanesPerRow == 0) sAlpha[srow] = alpha;
        }
        __syncthreads();
        // ---- O_w^T = alpha * O_w^T + V_w^T P^T
#pragma unroll
        for (int rb = 0; rb < R; ++rb) {
            const float al = sAlpha[32 * rb + l32];
            if (__builtin_amdgcn_ballot_w64(al != 1.0f) != 0) {
#pragma unroll
                for (int dblk = 0; dblk < 4; ++dblk)
#pragma unroll
                    for (int i = 0; i < 16; ++i) o[rb][dblk][i] *= al;
            }
        }
        if constexpr (NB == 2) {
            if (t + 1 < n_tiles)
                asm volatile("s_waitcnt vmcnt(16)" ::: "memory");   // V(t) landed; V(t+1), K(t+1) may fly
            else
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        } else {
            if (t + 2 < n_tiles)
                asm volatile("s_waitcnt vmcnt(8)" ::: "memory");    // V(t) landed; K(t+2) may fly
            else
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        const lds_t *vs_ = LDS_PTR(char, sV[wave][NB == 2 ? (t & 1) : 0]);
#pragma unroll
        for (int kst = 0; kst < kD5Keys / 16; ++kst) {
            vec8 pb[R];
#pragma unroll
            for (int rb = 0; rb < R; ++rb) pb[rb] = *reinterpret_cast<const vec8 *>(&sP[32 * rb + l32][16 * kst + 8 * hi]);
#pragma unroll
            for (int dblk = 0; dblk < 4; ++dblk) {
                const lds_t *vp = vs_ + v_rd[dblk] + 4096 * kst;
                const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)(vp));
                const s16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)(vp + 1024));
                const vec8 va = __builtin_bit_cast(vec8, __builtin_shufflevector(lo, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
                for (int rb = 0; rb < R; ++rb) o[rb][dblk] = E::mfma(va, pb[rb], o[rb][dblk]);
            }
        }
        if constexpr (NB == 1) {
            if (t + 1 < n_tiles) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // this wave's V(t) reads are done
                issue_v(t + 1, 0);
            }
        }
    };
    for (int t = t_begin; t < n_tiles; t += NB == 1 ? 2 : 1) {
        tile(t, BC<false>());
        if constexpr (NB == 1)
            if (t + 1 < n_tiles) tile(t + 1, BC<true>());
    }
    if (a.n_split > 1) {
        // this range's unnormalised O (times exactly 1), running max and row
        // sum, for launch_d512_combine
        const int64_t rows = (int64_t)a.B * a.Lq * a.H;
        Args pa = a;
        pa.o = reinterpret_cast<char *>(a.part + (int64_t)split * rows * kD5);
        pa.o_type = KD_FA_TYPE_F32;
        pa.o_nb1 = kD5 * 4;
        pa.o_nb2 = (int64_t)a.H * kD5 * 4;
        pa.o_nb3 = (int64_t)a.Lq * a.H * kD5 * 4;
#pragma unroll
        for (int rb = 0; rb < R; ++rb) store_o_row_l(pa, qt * kRows + 32 * rb + l32, h, b, hi, o[rb], 1.0f, col0);
        const int q_row = qt * kRows + srow;
        if (lane % kLanesPerRow == 0 && q_row < a.Lq) {   // the softmax lanes of the wave's rows
            float *ml = a.part + (int64_t)a.n_split * rows * kD5 +
                        2 * ((int64_t)split * rows + ((int64_t)b * a.Lq + q_row) * a.H + h);
            ml[0] = m_run;
            ml[1] = l_run;
        }
        return;
    }
    if (lane % kLanesPerRow == 0) sL[srow] = l_run;
    __syncthreads();
#pragma unroll
    for (int rb = 0; rb < R; ++rb)
        store_o_row_l(a, qt * kRows + 32 * rb + l32, h, b, hi, o[rb], sL[32 * rb + l32], col0);
}

// d512_combine: dst row r = sum_s w_s O_s / sum_s w_s l_s with
// w_s = 2^(m_s - max_s m_s) over the key ranges of a split call (running
// maxima in the exp2 domain, as the kernel keeps them); 128 threads per row,
// four columns each, F32 arithmetic, then the store_o_row_l rounding.
__global__ __launch_bounds__(256) void d512_combine(Args a) {
    const int64_t rows = (int64_t)a.B * a.Lq * a.H;
    const int64_t r = (int64_t)blockIdx.x * 2 + (threadIdx.x >> 7);
    if (r >= rows) return;
    const int c = (int)(threadIdx.x & 127) * 4;
    const int S = a.n_split;
    const float *ml = a.part + (int64_t)S * rows * kD5;
    float M = -INFINITY;
    for (int s = 0; s < S; ++s) M = __builtin_fmaxf(M, ml[2 * ((int64_t)s * rows + r)]);
    float L = 0.0f;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s = 0; s < S; ++s) {
        const float m = ml[2 * ((int64_t)s * rows + r)];
        const float w = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - M);
        L += w * ml[2 * ((int64_t)s * rows + r) + 1];
        const f32x4 v = *reinterpret_cast<const f32x4 *>(a.part + ((int64_t)s * rows + r) * kD5 + c);
        acc.x += w * v.x; acc.y += w * v.y; acc.z += w * v.z; acc.w += w * v.w;
    }
    const float inv = L == 0.0f ? 0.0f : 1.0f / L;
    const f32x4 v = {acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv};
    const int h = (int)(r % a.H);
    const int i = (int)((r / a.H) % a.Lq);
    const int b = (int)(r / ((int64_t)a.H * a.Lq));
    char *op = a.o + (int64_t)b * a.o_nb3 + (int64_t)i * a.o_nb2 + (int64_t)h * a.o_nb1;
    if (a.o_type == KD_FA_TYPE_F32) {
        *reinterpret_cast<f32x4 *>(op + c * 4) = v;
    } else if (a.o_type == KD_FA_TYPE_BF16) {
        *reinterpret_cast<u32x2 *>(op + c * 2) = (u32x2){Elem<__bf16>::pack2(v.x, v.y), Elem<__bf16>::pack2(v.z, v.w)};
    } else {
        *reinterpret_cast<u32x2 *>(op + c * 2) =
            (u32x2){Elem<_Float16>::pack2(v.x, v.y), Elem<_Float16>::pack2(v.z, v.w)};
    }
}

template <typename T, int R, int NB>
static hipError_t launch_d512_t(const Args &a, hipStream_t s) {
    const int64_t grid = (int64_t)a.n_blocks * (a.n_split > 1 ? a.n_split : 1);
    hipLaunchKernelGGL((fa_fwd_d512<T, R, NB>), dim3((unsigned)grid), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_d512_combine(const Args &a, hipStream_t s) {
    const int64_t rows = (int64_t)a.B * a.Lq * a.H;
    hipLaunchKernelGGL(d512_combine, dim3((unsigned)((rows + 1) / 2)), dim3(256), 0, s, a);
    return hipGetLastError();
}

// 64-row workgroups (R = 2): one per CU, V double-buffered; 32-row ones
// (R = 1): two per CU, one V buffer per wave (4,096 tokens with the key
// split 0.115 -> 0.106 ms, without 0.188 -> 0.181; 1,024 tokens 0.053 ->
// 0.050; the same bits)
hipError_t launch_d512(const Args &a, int kv_type, int rows, hipStream_t stream) {
    if (rows == 64)
        return kv_type == KD_FA_TYPE_BF16 ? launch_d512_t<__bf16, 2, 2>(a, stream) : launch_d512_t<_Float16, 2, 2>(a, stream);
    return kv_type == KD_FA_TYPE_BF16 ? launch_d512_t<__bf16, 1, 1>(a, stream) : launch_d512_t<_Float16, 1, 1>(a, stream);
}

}  // namespace kdfa
