#!/bin/bash
# The CPU test suite (pytest -m "not gpu") under AddressSanitizer and
# UndefinedBehaviorSanitizer.  Instrumented: the host code of libaether_weaver.so
# (planner, parameter validation, the .aether fabric's file, loom and checkpoint
# code, the dense ops' argument checks; the gfx950 device code is not) and the CPU oracle, both built with ROCm's
# clang into a scratch directory and loaded through AETHER_WEAVER_LIB and
# WEAVER_ORACLE_LIB.  Usage: tests/run_sanitized.sh [scratch-dir]
set -euo pipefail
ROOT=$(cd "$(dirname "$0")/.." && pwd)
OUT=${1:-$(mktemp -d)}
mkdir -p "$OUT/lib"
RT=$(ls /opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so | head -1)
RTDIR=$(dirname "$RT")
SAN_HOST="-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined -Xarch_host -fno-sanitize-recover=undefined -Xarch_host -fno-omit-frame-pointer"
echo "building the host-instrumented library into $OUT/lib"
/opt/rocm/bin/hipcc --offload-arch=gfx950 -O1 -g -std=c++17 -fPIC -shared \
    -Xclang -target-feature -Xclang -packed-fp32-ops $SAN_HOST -shared-libsan -Wl,-rpath,"$RTDIR" \
    -I "$ROOT/include" -o "$OUT/lib/libaether_weaver.so" \
    "$ROOT/aether_nexus_amd/csrc/weaver_engine.hip" "$ROOT/aether_nexus_amd/csrc/fabric.hip" \
    "$ROOT/aether_nexus_amd/csrc/ops.hip" 2>&1 |
    { grep -v "packed-fp32-ops\|argument unused" || true; }
echo "building the instrumented oracle"
/opt/rocm/llvm/bin/clang -O1 -g -std=c11 -ffp-contract=off -march=x86-64-v3 -fPIC -shared \
    -fsanitize=address,undefined -fno-sanitize-recover=undefined -fno-omit-frame-pointer -shared-libsan \
    -Wl,-rpath,"$RTDIR" -o "$OUT/libweaver_oracle.so" "$ROOT/oracle/weaver_oracle.c" -lm -lpthread
cd "$ROOT"
rm -f "$OUT"/asan.* "$OUT"/ubsan.*
# Leak checking is off: the Python interpreter and torch keep allocations to exit.
status=0
LD_PRELOAD="$RT" ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:log_path=$OUT/asan" \
    UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1:log_path=$OUT/ubsan" \
    AETHER_WEAVER_LIB="$OUT/lib/libaether_weaver.so" WEAVER_ORACLE_LIB="$OUT/libweaver_oracle.so" \
    python -m pytest tests -q -m "not gpu" -p no:cacheprovider || status=$?
for f in "$OUT"/asan.* "$OUT"/ubsan.*; do
    [ -e "$f" ] && { echo "== sanitizer report $f"; cat "$f"; status=1; }
done
exit $status
