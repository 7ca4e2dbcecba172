#!/bin/bash
# Runs the CPU tests (pytest -m "not gpu") against the sanitized builds of
# the library's host code: first ASan + UBSan, then TSan. Build them first
# with `make -C mini-serve-rs_amd/csrc -j16 sanitize`. The sanitizer runtime
# is preloaded into the (uninstrumented) Python interpreter; leak checking is
# off, since the interpreter's own allocations would be reported.
set -eo pipefail
HERE=$(cd "$(dirname "$0")" && pwd)
ROOT=$(cd "$HERE/../.." && pwd)
PKG=$ROOT/mini-serve-rs_amd
RT=$(/opt/rocm/llvm/bin/clang++ -print-resource-dir)/lib/linux
cd "$ROOT"
echo "== ASan + UBSan"
RLSE_KV_LIB=$PKG/librlse_kv_asan.so \
LD_PRELOAD=$RT/libclang_rt.asan-x86_64.so \
ASAN_OPTIONS=detect_leaks=0:abort_on_error=1:halt_on_error=1 \
UBSAN_OPTIONS=halt_on_error=1:print_stacktrace=1 \
  python -m pytest tests -q -m "not gpu" -p no:cacheprovider "$@"
echo "== TSan"
# One OpenMP thread: the oracle's OpenMP regions synchronise inside libgomp,
# which TSan does not see, so its worker threads would be reported as racing
# with the caller (the library's own threads are the tests' Python threads).
OMP_NUM_THREADS=1 \
RLSE_KV_LIB=$PKG/librlse_kv_tsan.so \
LD_PRELOAD=$RT/libclang_rt.tsan-x86_64.so \
TSAN_OPTIONS=halt_on_error=1:second_deadlock_stack=1 \
  python -m pytest tests -q -m "not gpu" -p no:cacheprovider "$@"
