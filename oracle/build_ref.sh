#!/usr/bin/env bash
# Builds the test-infrastructure libraries of the oracle:
#   oracle/lib/libxtu_oracle.so     the C restatement (xtu_oracle.c)
#   oracle/_ref/libxref_<isa>.so    the reference CPU engine, compiled from its
#                                   own headers where they lie in the reference
#                                   checkout, behind the harness ref_engine.cpp
# The reference libraries are built only when the checkout is present; on a
# machine without it the prebuilt files under oracle/_ref/ are used as they are.
set -euo pipefail
HERE="$(cd "$(dirname "${BASH_SOURCE[0]}")" && pwd)"
REF_ROOT="${XTU_REFERENCE_ROOT:-/root/reference}"
mkdir -p "$HERE/lib" "$HERE/_ref"

gcc -std=c11 -O2 -fPIC -shared -ffp-contract=off -fno-fast-math \
    "$HERE/xtu_oracle.c" -o "$HERE/lib/libxtu_oracle.so" -lm

SRC="$REF_ROOT/xiaotu_moe/csrc"
if [[ -d "$SRC/moe" ]]; then
  # Same optimisation flags as the reference's own engine build
  # (scripts/build_engine_variants.sh COMMON), NO_CUDA engine.
  COMMON="-std=c++17 -fPIC -O3 -ffast-math -fno-finite-math-only -DXIAOTU_MOE_NO_CUDA -w"
  VNNI="-mavx512f -mavx512bw -mavx512vl -mavx512dq -mavx512bf16 -mavx512vbmi -mavx512vnni -mfma"
  AVX512="-mavx512f -mavx512bw -mavx512vl -mavx512dq -mfma"
  g++ $COMMON $VNNI -I"$SRC" -c "$HERE/ref_engine.cpp" -o "$HERE/_ref/ref_vnni.o" &
  g++ $COMMON $AVX512 -I"$SRC" -c "$HERE/ref_engine.cpp" -o "$HERE/_ref/ref_avx512.o" &
  wait
  # link without -ffast-math so loading the library does not switch the process to
  # flush-to-zero / denormals-are-zero
  g++ -shared "$HERE/_ref/ref_vnni.o" -o "$HERE/_ref/libxref_avx512_vnni.so.tmp" -lpthread
  mv "$HERE/_ref/libxref_avx512_vnni.so.tmp" "$HERE/_ref/libxref_avx512_vnni.so"
  g++ -shared "$HERE/_ref/ref_avx512.o" -o "$HERE/_ref/libxref_avx512.so.tmp" -lpthread
  mv "$HERE/_ref/libxref_avx512.so.tmp" "$HERE/_ref/libxref_avx512.so"
  rm -f "$HERE/_ref/ref_vnni.o" "$HERE/_ref/ref_avx512.o"
  echo "built reference engine harness into $HERE/_ref"
else
  echo "reference checkout not found at $REF_ROOT; using prebuilt oracle/_ref if present"
fi
