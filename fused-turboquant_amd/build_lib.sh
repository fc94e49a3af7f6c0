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
  [[ "$b" == ftq_torch_ops.cpp ]] && continue  # the PyTorch operator library, built below
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
rm -f "$OBJ/ftq_torch_ops.cpp.o"
hipcc --offload-arch=gfx950 -shared -fPIC "$OBJ"/*.o -o "$OUT.tmp"
mv "$OUT.tmp" "$OUT"
echo "built $OUT"

# torch.ops.fused_tq: the PyTorch operators over the C ABI (host code only),
# linked against libfused_tq.so next to it and torch's own libraries
TORCH_DIR="$(python3 -c 'import os, torch; print(os.path.dirname(torch.__file__))')"
TOUT="$HERE/fused_turboquant/libfused_tq_torch.so"
ABI="$(python3 -c 'import torch; print(int(torch._C._GLIBCXX_USE_CXX11_ABI))')"
hipcc -std=c++17 -O2 -fPIC -shared "$SRC/ftq_torch_ops.cpp" -I"$HERE/../include" \
  -I"$TORCH_DIR/include" -I"$TORCH_DIR/include/torch/csrc/api/include" -D_GLIBCXX_USE_CXX11_ABI="$ABI" \
  -L"$TORCH_DIR/lib" -lc10 -lc10_hip -ltorch_cpu -ltorch_hip -ltorch \
  -L"$HERE/fused_turboquant" -lfused_tq -Wl,-rpath,'$ORIGIN' -o "$TOUT.tmp"
mv "$TOUT.tmp" "$TOUT"
echo "built $TOUT"
