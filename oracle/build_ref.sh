#!/bin/sh
# Builds the reference's own CPU twins (route, combine, SwiGLU, the Q8_1 quantizer and the
# Q8_0 / Q4_K mat-vecs over Q8_1) from the sources where they lie in the reference checkout,
# plus this repo's C-ABI shim, into oracle/_ref/. q4_k_mv.cpp calls std::fma without
# including <cmath> (it compiles only where another header brings it in), so <cmath> is
# force-included.
# Test infrastructure only. Usage: oracle/build_ref.sh [reference_root]
set -e
REF=${1:-/root/reference}
HERE=$(cd "$(dirname "$0")" && pwd)
[ -d "$REF/tests/metal/oracles" ] || { echo "reference checkout not found at $REF" >&2; exit 1; }
mkdir -p "$HERE/_ref"
O="$REF/tests/metal/oracles"
g++ -std=c++20 -O2 -fPIC -shared -ffp-contract=off -include cmath -I"$REF/tests/metal" -I"$REF/include" \
    "$O/common.cpp" "$O/moe_route.cpp" "$O/moe_combine.cpp" "$O/moe_swiglu.cpp" \
    "$O/q8_1.cpp" "$O/q8_0_mv.cpp" "$O/q4_k_mv.cpp" \
    "$HERE/ref_driver.cpp" -o "$HERE/_ref/libref_twins.so"
