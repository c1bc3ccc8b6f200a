#!/bin/bash
# Host-side AddressSanitizer + UndefinedBehaviorSanitizer build of the C-ABI layer
# (deepgemm-amd_amd/csrc/dg_api.cpp: argument validation, layout/recipe checks,
# descriptor handling), linked with the regular objects of the HIP sources from the
# in-tree build. GPU code is not sanitized (no device sanitizer on this stack).
# Usage: build_asan.sh OUT_DIR   -- prints the ASan runtime to preload on its last line.
set -euo pipefail
HERE=$(cd "$(dirname "$0")" && pwd)
ROOT=$(dirname "$(dirname "$HERE")")
ROCM=${ROCM_PATH:-/opt/rocm}
OUT=$1
mkdir -p "$OUT"
"$ROCM/llvm/bin/clang++" -O1 -g -std=c++20 -fPIC -fsanitize=address,undefined -fno-omit-frame-pointer \
    -fno-sanitize-recover=undefined -D__HIP_PLATFORM_AMD__ -I "$ROCM/include" -I "$ROOT/include" \
    -I "$ROOT/deepgemm-amd_amd/csrc" -c "$ROOT/deepgemm-amd_amd/csrc/dg_api.cpp" -o "$OUT/dg_api.asan.o"
"$ROCM/bin/hipcc" --offload-arch=gfx950 -shared -fPIC -Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined \
    -o "$OUT/libdeepgemm_mi355x_asan.so" "$OUT/dg_api.asan.o" "$ROOT"/deepgemm-amd_amd/_build/*.hip.o
ls "$ROCM"/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so | head -1
