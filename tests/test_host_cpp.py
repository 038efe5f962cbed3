"""The C++ host mirror of ops::attention (kandinsky.cpp_amd/host/
kd_attention.hpp): built with g++ against libkd_fa.so, it must turn the
reference's activation layout q [C, Lq, N], k/v [C_kv, Lk, N]
(src/core/ops.hpp:107-183) into the op's per-head strided views without
copies, with scale 1/sqrt(d_head) and F32 precision, and be accepted by
kd_fa_supports; a bad head split is rejected before any GPU work."""
import os
import subprocess
import tempfile

import kd_fa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# tests/run_sanitized.sh: the mirror is compiled under ASan + UBSan as well,
# with the compiler whose runtime the sanitized library uses
SANITIZE = os.environ.get("KD_SANITIZE") == "1"
CXX = (["/opt/rocm/llvm/bin/clang++", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
        "-shared-libsan", "-g"] if SANITIZE else ["g++"])

SRC = r"""
#include <cstdio>
#include <cstdlib>
#include "kd_attention.hpp"
#define CHECK(c) do { if (!(c)) { std::printf("FAIL %s:%d %s\n", __FILE__, __LINE__, #c); return 1; } } while (0)
int main() {
  alignas(256) static char buf[1 << 16];
  // Pro CrossDiT: C = 4096 (32 heads x 128), Lq = Lk = 40 tokens, N = 2
  kd::Activation q{buf, KD_FA_TYPE_F32, 4096, 40, 2, 4096 * 4, 40 * 4096 * 4};
  kd::Activation k{buf, KD_FA_TYPE_BF16, 4096, 40, 2, 4096 * 2, 40 * 4096 * 2};
  kd::Activation v = k;
  kd_fa_desc d;
  CHECK(kd::make_node(q, k, v, 32, buf, nullptr, &d));
  CHECK(d.q.ne[0] == 128 && d.q.ne[1] == 40 && d.q.ne[2] == 32 && d.q.ne[3] == 2);
  CHECK(d.q.nb[0] == 4 && d.q.nb[1] == 4096 * 4 && d.q.nb[2] == 128 * 4 && d.q.nb[3] == 40 * 4096 * 4);
  CHECK(d.k.nb[1] == 4096 * 2 && d.k.nb[2] == 256);
  CHECK(d.dst.ne[0] == 128 && d.dst.ne[1] == 32 && d.dst.ne[2] == 40 && d.dst.ne[3] == 2);
  CHECK(d.dst.nb[1] == 512 && d.dst.nb[2] == 4096 * 4 && d.dst.nb[3] == 40 * 4096 * 4);
  CHECK(d.scale > 0.0883883f && d.scale < 0.0883884f && d.prec == KD_FA_PREC_F32);
  CHECK(d.max_bias == 0.0f && d.logit_softcap == 0.0f && d.mask.data == nullptr);
  int reason = -99;
  CHECK(kd_fa_supports(&d, &reason) == 1 && reason == KD_FA_OK);
  // grouped K/V heads (C_kv = 4 x 128) are broadcast, not repeated
  kd::Activation kg{buf, KD_FA_TYPE_BF16, 512, 40, 2, 512 * 2, 40 * 512 * 2};
  CHECK(kd::make_node(q, kg, kg, 32, buf, nullptr, &d) && d.k.ne[2] == 4);
  CHECK(kd_fa_supports(&d, &reason) == 1);
  // 4096 is not a multiple of 48 heads: rejected before any GPU work
  CHECK(kd::attention(q, k, v, 48, buf).status == KD_FA_ERR_SHAPE);
  std::printf("ok\n");
  return 0;
}
"""


def test_ops_attention_mirror_builds_views():
    lib_dir = os.path.dirname(kd_fa.LIB_PATH)
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "t.cpp")
        exe = os.path.join(d, "t")
        with open(src, "w") as f:
            f.write(SRC)
        subprocess.run(CXX + ["-std=c++17", "-Wall", "-Werror",
                        "-I", os.path.join(ROOT, "kandinsky.cpp_amd", "host"), src,
                        "-L", lib_dir, "-lkd_fa", f"-Wl,-rpath,{lib_dir}", "-o", exe], check=True)
        out = subprocess.run([exe], capture_output=True, text=True)
        assert out.returncode == 0 and out.stdout.strip() == "ok", out.stdout + out.stderr
