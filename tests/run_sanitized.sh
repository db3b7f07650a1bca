#!/bin/bash
# The CPU test suite (pytest -m "not gpu") against AddressSanitizer +
# UndefinedBehaviorSanitizer builds of the oracle and of the backend
# library's host code: the ONNX wire decoder and its fuzz tests, the passes,
# the executor's planning (dry runs), the profiler and the ABI checks.
# Both builds use the ROCm clang, so one ASan runtime (preloaded into the
# uninstrumented Python interpreter) serves both libraries. Leak checking is
# off: the interpreter itself leaks by design. Any sanitizer report aborts
# the run with a non-zero status.
# Usage: tests/run_sanitized.sh [extra pytest arguments]
set -euo pipefail
cd "$(dirname "$0")/.."
python -m inferc_amd.build --sanitize
make -s -C oracle sanitize
RT=$(ls /opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so | head -n 1)
export INFERC_HIP_LIB="$PWD/inferc_amd/libinferc_hip_san.so"
export ORACLE_LIB="$PWD/oracle/build/liboracle_san.so"
export LD_LIBRARY_PATH="/opt/rocm/llvm/lib${LD_LIBRARY_PATH:+:$LD_LIBRARY_PATH}"
export ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1:detect_odr_violation=0"
export UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1"
LD_PRELOAD="$RT" python -m pytest tests -m "not gpu" -q -p no:cacheprovider "$@"
