// kd_probe.hip - HBM streaming probes for the benchmark's ceiling figures
// (libkd_probe.so, not part of the attention library).  They measure what
// this GPU sustains for the byte mixes of the attention's HBM-bound cases:
//   widen: read a 16-bit array, write it as F32 (the text cross-attention's
//          Q-in / F32-O-out mix: 2 bytes read per 4 written);
//   read:  read an array, write one value per workgroup;
//   write: write an array.
// Each thread moves whole 16-byte pieces, grid-stride, stores streaming
// (nontemporal) like the attention kernels' O stores.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kThreads = 256;

// U pieces per thread per round: all U loads are issued before any store
// (loads and stores complete in issue order, so a load issued after a store
// also waits for it); NT: streaming (nontemporal) loads and stores.
template <int U, bool NT>
__global__ __launch_bounds__(kThreads) void widen_bf16(const u32x4 *__restrict__ src, u32x4 *__restrict__ dst,
                                                       int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i0 = (int64_t)blockIdx.x * kThreads * U + threadIdx.x; i0 < n16; i0 += stride * U) {
        u32x4 w[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = i0 + (int64_t)u * kThreads;
            if (i < n16) w[u] = NT ? __builtin_nontemporal_load(src + i) : src[i];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = i0 + (int64_t)u * kThreads;
            if (i < n16) {
                u32x4 lo, hi;
                lo.x = w[u].x << 16; lo.y = w[u].x & 0xffff0000u; lo.z = w[u].y << 16; lo.w = w[u].y & 0xffff0000u;
                hi.x = w[u].z << 16; hi.y = w[u].z & 0xffff0000u; hi.z = w[u].w << 16; hi.w = w[u].w & 0xffff0000u;
                if (NT) {
                    __builtin_nontemporal_store(lo, dst + 2 * i);
                    __builtin_nontemporal_store(hi, dst + 2 * i + 1);
                } else {
                    dst[2 * i] = lo;
                    dst[2 * i + 1] = hi;
                }
            }
        }
    }
}

__global__ __launch_bounds__(kThreads) void read_all(const u32x4 *__restrict__ src, u32x4 *__restrict__ sink,
                                                     int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n16; i += stride) acc ^= src[i];
    // one value per workgroup keeps the loads live
    __shared__ u32x4 red[kThreads];
    red[threadIdx.x] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        u32x4 s = red[0];
        for (int t = 1; t < kThreads; ++t) s ^= red[t];
        sink[blockIdx.x] = s;
    }
}

__global__ __launch_bounds__(kThreads) void write_all(u32x4 *__restrict__ dst, int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    const u32x4 z = {0u, 0u, 0u, 0u};
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n16; i += stride)
        __builtin_nontemporal_store(z, dst + i);
}

}  // namespace

// n16: 16-byte pieces of the source (widen, read) or of dst (write); all
// pointers 16-byte aligned; sink holds `blocks` 16-byte values.
// variant: unroll 1, 4 or 8 pieces per thread (x10 for streaming loads and
// stores: 11, 14, 18)
extern "C" int kd_probe_widen(const void *src, void *dst, int64_t n16, int blocks, int variant, void *stream) {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const u32x4 *a = static_cast<const u32x4 *>(src);
    u32x4 *d = static_cast<u32x4 *>(dst);
    switch (variant) {
    case 1: hipLaunchKernelGGL((widen_bf16<1, false>), dim3(blocks), dim3(kThreads), 0, s, a, d, n16); break;
    case 4: hipLaunchKernelGGL((widen_bf16<4, false>), dim3(blocks), dim3(kThreads), 0, s, a, d, n16); break;
    case 8: hipLaunchKernelGGL((widen_bf16<8, false>), dim3(blocks), dim3(kThreads), 0, s, a, d, n16); break;
    case 11: hipLaunchKernelGGL((widen_bf16<1, true>), dim3(blocks), dim3(kThreads), 0, s, a, d, n16); break;
    case 14: hipLaunchKernelGGL((widen_bf16<4, true>), dim3(blocks), dim3(kThreads), 0, s, a, d, n16); break;
    case 18: hipLaunchKernelGGL((widen_bf16<8, true>), dim3(blocks), dim3(kThreads), 0, s, a, d, n16); break;
    default: return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int kd_probe_read(const void *src, void *sink, int64_t n16, int blocks, void *stream) {
    hipLaunchKernelGGL(read_all, dim3(blocks), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                       static_cast<const u32x4 *>(src), static_cast<u32x4 *>(sink), n16);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int kd_probe_write(void *dst, int64_t n16, int blocks, void *stream) {
    hipLaunchKernelGGL(write_all, dim3(blocks), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                       static_cast<u32x4 *>(dst), n16);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
