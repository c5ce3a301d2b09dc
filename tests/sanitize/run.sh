#!/bin/bash
# The CPU ASan/UBSan pass:  bash tests/sanitize/run.sh
# Builds the sanitized libdsx.so (host code) and C oracle, then runs the CPU
# tests that reach them -- the ABI and host-logic tests plus a fuzz of the
# chunk-table builder against libdsx.so, the oracle tests against the oracle
# -- each in its own process with its compiler's ASan runtime preloaded
# (Python itself is not instrumented). Any sanitizer report fails the run.
set -euo pipefail
HERE="$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)"
ROCM="${ROCM:-/opt/rocm}"
make -s -C "$HERE"
clang_rt=""
for f in "$ROCM"/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so \
         "$ROCM"/llvm/lib/clang/*/lib/x86_64-unknown-linux-gnu/libclang_rt.asan.so; do
  if [ -f "$f" ]; then clang_rt="$f"; break; fi
done
if [ -z "$clang_rt" ]; then echo "[sanitize] clang's ASan runtime not found under $ROCM/llvm" >&2; exit 1; fi
gcc_rt="$(gcc -print-file-name=libasan.so)"
export ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1"
export UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1"
echo "[sanitize] canary: a planted host-side overflow must be reported"
if LD_PRELOAD="$clang_rt" python "$HERE/canary.py" "$HERE/_build/libdsx.so" 2> "$HERE/_build/canary.err"; then
  echo "[sanitize] the canary ran clean: the sanitizer is not active" >&2; exit 1
fi
grep -q "heap-buffer-overflow" "$HERE/_build/canary.err" || { tail -20 "$HERE/_build/canary.err" >&2; exit 1; }
echo "[sanitize] libdsx.so (host code) with $clang_rt"
LD_PRELOAD="$clang_rt" python "$HERE/run_tests.py" libdsx "$HERE/_build/libdsx.so"
echo "[sanitize] C oracle with $gcc_rt"
LD_PRELOAD="$gcc_rt" python "$HERE/run_tests.py" oracle "$HERE/_build/libdsx_oracle.so"
echo "[sanitize] clean"
