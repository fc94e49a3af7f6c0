#!/usr/bin/env bash
# Build libfused_tq.so (gfx950) in-tree, next to the Python package that loads it.
set -euo pipefail
HERE="$(cd "$(dirname "$0")" && pwd)"
SRC="$HERE/csrc"
OUT="$HERE/fused_turboquant/libfused_tq.so"
OBJ="$HERE/_build"
mkdir -p "$OBJ"
FLAGS=(-O3 -std=c++17 -fPIC --offload-arch=gfx950 -ffp-contract=off
       -Xclang -target-feature -Xclang -packed-fp32-ops -mllvm -amdgpu-mfma-vgpr-form
       -I"$HERE/../include" -Wall -Wno-unused-function)
pids=()
for f in "$SRC"/*.hip "$SRC"/*.cpp; do
  b="$(basename "$f")"
  if [[ "$f" == *.cpp ]]; then
    hipcc -x hip "${FLAGS[@]}" -c "$f" -o "$OBJ/$b.o" 2> "$OBJ/$b.log" &
  else
    hipcc "${FLAGS[@]}" -c "$f" -o "$OBJ/$b.o" 2> "$OBJ/$b.log" &
  fi
  pids+=($!)
done
rc=0
for p in "${pids[@]}"; do wait "$p" || rc=1; done
for l in "$OBJ"/*.log; do grep -v "packed-fp32-ops" "$l" | grep -v "^$" || true; done
[[ $rc -eq 0 ]] || { echo "compile failed" >&2; exit 1; }
hipcc --offload-arch=gfx950 -shared -fPIC "$OBJ"/*.o -o "$OUT.tmp"
mv "$OUT.tmp" "$OUT"
echo "built $OUT"
