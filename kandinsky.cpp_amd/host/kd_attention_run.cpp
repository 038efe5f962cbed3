// kd_attention_run - runs kd::attention (the ops::attention mirror) once on
// a GPU from raw files, as the reference's DiT attention would call it.
//
//   kd_attention_run <n_head> <Lq> <Lk> <N> <bf16|f16> <q.bin> <k.bin> <v.bin> <out.bin>
//       [rope.bin|-] [wq.bin wk.bin]
//
// q.bin: [N][Lq][C] F32 activations (C = n_head * 128); k.bin, v.bin:
// [N][Lk][C] in the storage type (raw 16-bit); out.bin receives F32
// [N][Lq][C].  With rope.bin (F32 [max(Lq,Lk)][128] table) Q and K are
// rotated on load.  With wq.bin, wk.bin (F32 [128] RMSNorm weights, eps
// 1e-6) Q and K are normalised first, K once into a workspace.  Exit status
// 0 on success, otherwise the KD_FA status or 100+ for I/O and runtime
// errors.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "kd_attention.hpp"

static bool read_file(const char *path, std::vector<char> &buf) {
    FILE *f = std::fopen(path, "rb");
    if (!f) return false;
    std::fseek(f, 0, SEEK_END);
    const long n = std::ftell(f);
    std::fseek(f, 0, SEEK_SET);
    buf.resize((size_t)n);
    const bool ok = std::fread(buf.data(), 1, buf.size(), f) == buf.size();
    std::fclose(f);
    return ok;
}

int main(int argc, char **argv) {
    if (argc != 10 && argc != 11 && argc != 13) {
        std::fprintf(stderr, "usage: %s n_head Lq Lk N bf16|f16 q.bin k.bin v.bin out.bin [rope.bin|- [wq.bin wk.bin]]\n",
                     argv[0]);
        return 100;
    }
    const int64_t n_head = std::atoll(argv[1]), Lq = std::atoll(argv[2]), Lk = std::atoll(argv[3]),
                  N = std::atoll(argv[4]);
    const int32_t kt = std::strcmp(argv[5], "bf16") == 0 ? KD_FA_TYPE_BF16 : KD_FA_TYPE_F16;
    const int64_t C = n_head * 128;
    std::vector<char> hq, hk, hv, hr;
    if (!read_file(argv[6], hq) || !read_file(argv[7], hk) || !read_file(argv[8], hv)) return 101;
    if (hq.size() != (size_t)(N * Lq * C * 4) || hk.size() != (size_t)(N * Lk * C * 2) || hv.size() != hk.size())
        return 102;
    const bool rope_on = argc >= 11 && std::strcmp(argv[10], "-") != 0;
    if (rope_on && !read_file(argv[10], hr)) return 101;
    const bool norm_on = argc == 13;
    std::vector<char> hwq, hwk;
    if (norm_on && (!read_file(argv[11], hwq) || !read_file(argv[12], hwk) || hwq.size() != 512 || hwk.size() != 512))
        return 101;

    void *dq, *dk, *dv, *dout, *dr = nullptr;
    const size_t out_bytes = (size_t)(N * Lq * C * 4);
    if (hipMalloc(&dq, hq.size()) != hipSuccess || hipMalloc(&dk, hk.size()) != hipSuccess ||
        hipMalloc(&dv, hv.size()) != hipSuccess || hipMalloc(&dout, out_bytes) != hipSuccess)
        return 103;
    if (hipMemcpy(dq, hq.data(), hq.size(), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(dk, hk.data(), hk.size(), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(dv, hv.data(), hv.size(), hipMemcpyHostToDevice) != hipSuccess)
        return 104;
    kd_fa_rope rope{};
    if (rope_on) {
        if (hipMalloc(&dr, hr.size()) != hipSuccess) return 103;
        if (hipMemcpy(dr, hr.data(), hr.size(), hipMemcpyHostToDevice) != hipSuccess) return 104;
        rope.mode = KD_FA_ROPE_TABLE;
        rope.table.type = KD_FA_TYPE_F32;
        rope.table.ne[0] = 128;
        rope.table.ne[1] = (int64_t)(hr.size() / 512);
        rope.table.ne[2] = rope.table.ne[3] = 1;
        rope.table.nb[0] = 4;
        rope.table.nb[1] = 512;
        rope.table.nb[2] = rope.table.nb[3] = hr.size();
        rope.table.data = dr;
    }
    kd_fa_qk_norm norm{};
    void *dw = nullptr, *dws = nullptr;
    if (norm_on) {
        if (hipMalloc(&dw, 1024) != hipSuccess || hipMalloc(&dws, hk.size()) != hipSuccess) return 103;
        if (hipMemcpy(dw, hwq.data(), 512, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(static_cast<char *>(dw) + 512, hwk.data(), 512, hipMemcpyHostToDevice) != hipSuccess)
            return 104;
        norm.q_weight = static_cast<const float *>(dw);
        norm.k_weight = static_cast<const float *>(dw) + 128;
        norm.eps = 1e-6f;
    }
    kd::Activation q{dq, KD_FA_TYPE_F32, C, Lq, N, (size_t)C * 4, (size_t)(Lq * C * 4)};
    kd::Activation k{dk, kt, C, Lk, N, (size_t)C * 2, (size_t)(Lk * C * 2)};
    kd::Activation v{dv, kt, C, Lk, N, (size_t)C * 2, (size_t)(Lk * C * 2)};
    const kd::Result r = kd::attention(q, k, v, n_head, dout, nullptr, rope_on ? &rope : nullptr, nullptr,
                                       dws, norm_on ? hk.size() : 0, norm_on ? &norm : nullptr);
    if (!r.ran()) {
        std::fprintf(stderr, "kd::attention: %s\n", kd_fa_strerror(r.status));
        return -r.status;
    }
    if (hipDeviceSynchronize() != hipSuccess) return 105;
    std::vector<char> ho(out_bytes);
    if (hipMemcpy(ho.data(), dout, out_bytes, hipMemcpyDeviceToHost) != hipSuccess) return 104;
    FILE *f = std::fopen(argv[9], "wb");
    if (!f || std::fwrite(ho.data(), 1, ho.size(), f) != ho.size()) return 101;
    std::fclose(f);
    (void)hipFree(dq);
    (void)hipFree(dk);
    (void)hipFree(dv);
    (void)hipFree(dout);
    if (dr) (void)hipFree(dr);
    if (dw) (void)hipFree(dw);
    if (dws) (void)hipFree(dws);
    return 0;
}
