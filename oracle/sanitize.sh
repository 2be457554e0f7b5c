#!/bin/bash
# AddressSanitizer + UndefinedBehaviorSanitizer over the host-side C++ on the CPU: the oracle
# (oracle.cpp), and the library's host code (host.cpp bookkeeping, plan.cpp's work-list planner,
# sched.cpp, sha256.cpp, pool.h).
# Instrumented copies go to oracle/_san/ (git-ignored); the library's device objects are the
# regular build's (llmario_amd/_build, built first). Then the CPU tests that drive this code run
# with clang's sanitizer runtime preloaded, against the instrumented libraries:
#   tests/test_sched.py, tests/test_oracle_*.py, tests/test_golden.py, tests/test_native_abi.py,
#   tests/test_plan.py (the work-list planner on random calls)
# Usage: bash oracle/sanitize.sh   (exit status: pytest's; any sanitizer report fails the run)
set -euo pipefail
ROOT="$(cd "$(dirname "$0")/.." && pwd)"
OUT="$ROOT/oracle/_san"
LLVM=/opt/rocm/lib/llvm/bin
HIPCC=/opt/rocm/bin/hipcc
RT=$(ls /opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so | head -1)
SAN="-fsanitize=address,undefined -fno-sanitize-recover=undefined -fno-omit-frame-pointer -shared-libsan"
mkdir -p "$OUT/obj"
[ -f "$ROOT/llmario_amd/_build/decode.hip.o" ] || python3 -c "import sys; sys.path.insert(0, '$ROOT'); from llmario_amd import build; build.build()"
# the oracle, as its Makefile builds it, instrumented
$LLVM/clang++ -O1 -g -std=c++17 -fPIC -mavx2 -mfma -ffp-contract=off -pthread $SAN -shared \
  -o "$OUT/liboracle.so" "$ROOT/oracle/oracle.cpp"
# the library's host-only sources
for f in plan sched sha256; do
  $LLVM/clang++ -O1 -g -std=c++17 -fPIC $SAN -I "$ROOT/include" -c "$ROOT/llmario_amd/csrc/$f.cpp" -o "$OUT/obj/$f.o"
done
# host.cpp carries device structures: its host pass instrumented, device pass as usual
$HIPCC --offload-arch=gfx950 -O1 -g -std=c++17 -fPIC -I "$ROOT/include" \
  -Xarch_host -fsanitize=address,undefined -Xarch_host -fno-sanitize-recover=undefined \
  -Xarch_host -fno-omit-frame-pointer -x hip -c "$ROOT/llmario_amd/csrc/host.cpp" -o "$OUT/obj/host.o" 2>/dev/null
$HIPCC --offload-arch=gfx950 -shared -fPIC -shared-libsan -Xarch_host -fsanitize=address,undefined -o "$OUT/libllmario_hip.so" \
  "$OUT/obj/host.o" "$OUT/obj/plan.o" "$OUT/obj/sched.o" "$OUT/obj/sha256.o" \
  "$ROOT/llmario_amd/_build/kv_kernels.hip.o" "$ROOT/llmario_amd/_build/decode.hip.o" "$ROOT/llmario_amd/_build/prefill.hip.o"
cd "$ROOT"
LD_PRELOAD="$RT" ASAN_OPTIONS=detect_leaks=0:halt_on_error=1 UBSAN_OPTIONS=halt_on_error=1:print_stacktrace=1 \
  LLMARIO_HIP_LIB="$OUT/libllmario_hip.so" LLMARIO_ORACLE_LIB="$OUT/liboracle.so" \
  python3 -m pytest -q -p no:cacheprovider tests/test_sched.py tests/test_oracle_attend.py tests/test_oracle_codecs.py \
  tests/test_oracle_pool.py tests/test_oracle_rope.py tests/test_oracle_sched.py tests/test_oracle_snapshot.py \
  tests/test_oracle_window.py tests/test_golden.py tests/test_native_abi.py tests/test_plan.py -m "not gpu"
