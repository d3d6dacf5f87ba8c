#!/usr/bin/env bash
# Builds oracle/_ref/libmlvc_ref_kernels.so from the reference CPU kernel
# sources and core/src/yuv.cpp where they lie (default /root/reference) plus
# oracle/ref_harness.cpp.
# Test infrastructure only; the output stays out of git history.
# Flags follow the reference's backends/cpu/CMakeLists.txt: the AVX2 file is
# built with -mavx2 -mfma -mf16c, the scalar file without (so its multiply
# and add round separately), Release -O3.
set -euo pipefail
REF="${1:-/root/reference}"
HERE="$(cd "$(dirname "$0")" && pwd)"
OUT="$HERE/_ref"
if [ ! -d "$REF/backends/cpu/src" ]; then
    echo "reference checkout not found at $REF; skipping oracle/_ref" >&2
    exit 0
fi
mkdir -p "$OUT/obj"
INC="-I$REF/core/include -I$REF/runtime/include -I$REF/backends/cpu/src"
CXX="g++ -std=c++20 -O3 -fPIC -DMLVC_CPU_ENABLE_X86_AVX2=1 $INC"
pids=()
$CXX -c "$REF/backends/cpu/src/kernels_scalar.cpp" -o "$OUT/obj/kernels_scalar.o" & pids+=($!)
$CXX -mavx2 -mfma -mf16c -c "$REF/backends/cpu/src/kernels_x86_avx2.cpp" -o "$OUT/obj/kernels_x86_avx2.o" & pids+=($!)
$CXX -c "$REF/backends/cpu/src/thread_pool.cpp" -o "$OUT/obj/thread_pool.o" & pids+=($!)
$CXX -c "$REF/backends/cpu/src/cpu_features.cpp" -o "$OUT/obj/cpu_features.o" & pids+=($!)
$CXX -c "$REF/core/src/yuv.cpp" -o "$OUT/obj/yuv.o" & pids+=($!)
$CXX -c "$HERE/ref_harness.cpp" -o "$OUT/obj/ref_harness.o" & pids+=($!)
for p in "${pids[@]}"; do wait "$p"; done
g++ -shared -o "$OUT/libmlvc_ref_kernels.so" "$OUT"/obj/*.o -lpthread
rm -rf "$OUT/obj"
echo "built $OUT/libmlvc_ref_kernels.so"
