#!/usr/bin/env bash
# Host-side AddressSanitizer + UndefinedBehaviorSanitizer run of the C ABI.
#
# Compiles the library's sources host-only (--cuda-host-only: the extern "C"
# entry points, argument checks, launch dispatch and error reporting; no
# device code: an empty GPU binary is embedded in its place, so every launch
# fails with a HIP error) with the sanitizers on
# the host pass, links them with abi_host_check.cpp into one executable and
# runs it.  Output goes to fused-turboquant_amd/_build/asan/.  Runs on a
# machine without a GPU; a sanitizer report or a failed check exits non-zero.
set -euo pipefail
HERE="$(cd "$(dirname "$0")" && pwd)"
REPO="$(cd "$HERE/../.." && pwd)"
SRC="$REPO/fused-turboquant_amd/csrc"
OUT="$REPO/fused-turboquant_amd/_build/asan"
mkdir -p "$OUT"
: > "$OUT/empty.fatbin"
SAN=(-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined -Xarch_host -fno-sanitize-recover=all)
FLAGS=(--cuda-host-only -Xclang -fcuda-include-gpubinary -Xclang "$OUT/empty.fatbin" -O1 -g -fno-omit-frame-pointer -std=c++17 -I"$REPO/include" -Wall -Wno-unused-function)
pids=()
for f in "$SRC"/*.hip "$SRC"/ftq_capi.cpp "$HERE/abi_host_check.cpp"; do
  b="$(basename "$f")"
  hipcc -x hip "${FLAGS[@]}" "${SAN[@]}" -c "$f" -o "$OUT/$b.o" 2> "$OUT/$b.log" &
  pids+=($!)
done
rc=0
for p in "${pids[@]}"; do wait "$p" || rc=1; done
for l in "$OUT"/*.log; do grep -v "packed-fp32-ops" "$l" | grep -v "^$" || true; done
[[ $rc -eq 0 ]] || { echo "asan compile failed" >&2; exit 1; }
hipcc "${SAN[@]}" -fno-omit-frame-pointer "$OUT"/*.o -o "$OUT/abi_host_check"
export ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:strict_string_checks=1:detect_stack_use_after_return=1"
export UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1"
"$OUT/abi_host_check"
