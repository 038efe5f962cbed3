#!/bin/bash
# The CPU test suite against host builds under AddressSanitizer and
# UndefinedBehaviorSanitizer: the oracle (oracle/_asan/libkd_oracle.so) and
# the product library's host code -- the C-ABI validation, kernel choice and
# launch glue -- (kandinsky.cpp_amd/_asan/libkd_fa.so).  Both are built with
# ROCm's clang, so one sanitizer runtime (preloaded into the Python process)
# serves both.  CPU only: no test here launches a kernel.
#   bash tests/run_sanitized.sh [extra pytest args]
set -e
ROOT=$(cd "$(dirname "$0")/.." && pwd)
make -s -C "$ROOT/oracle" asan
make -s -C "$ROOT/kandinsky.cpp_amd" asan
RT=$(ls /opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so | head -1)
export LD_PRELOAD="$RT"
export ASAN_OPTIONS=detect_leaks=0:halt_on_error=1:abort_on_error=1
export UBSAN_OPTIONS=halt_on_error=1:print_stacktrace=1
export KD_FA_LIB="$ROOT/kandinsky.cpp_amd/_asan/libkd_fa.so"
export KD_ORACLE_LIB="$ROOT/oracle/_asan/libkd_oracle.so"
export KD_SANITIZE=1
cd "$ROOT"
export PYTHONPATH="$ROOT/oracle:$ROOT/kandinsky.cpp_amd${PYTHONPATH:+:$PYTHONPATH}"
python -m pytest tests -m "not gpu" -q -p no:cacheprovider "$@"
# The sanitizers are live: the oracle's rotation called on the CPU with an
# output buffer one row short must be stopped as a heap-buffer-overflow.
set +e
out=$(python - 2>&1 <<'PY'
import ctypes
import numpy as np
import kd_oracle as orc
L, D = 8, 128
x = np.zeros((1, L, 1, D), dtype=np.float32)
t = np.zeros((L, D), dtype=np.float32)
short = np.zeros((1, L - 1, 1, D), dtype=np.float32)
fp = ctypes.POINTER(ctypes.c_float)
orc.lib().kdo_rope_apply_f32(x.ctypes.data_as(fp), D, 1, L, 1, t.ctypes.data_as(fp), short.ctypes.data_as(fp))
print("not caught")
PY
)
set -e
if echo "$out" | grep -q "heap-buffer-overflow"; then
    echo "sanitizer liveness: planted overflow caught"
else
    echo "sanitizer liveness check FAILED: $out" | tail -5
    exit 1
fi
