#!/bin/sh
# Builds the reference's own CPU twins (route, combine, SwiGLU) from the sources where they
# lie in the reference checkout, plus this repo's C-ABI shim, into oracle/_ref/.
# Test infrastructure only. Usage: oracle/build_ref.sh [reference_root]
set -e
REF=${1:-/root/reference}
HERE=$(cd "$(dirname "$0")" && pwd)
[ -d "$REF/tests/metal/oracles" ] || { echo "reference checkout not found at $REF" >&2; exit 1; }
mkdir -p "$HERE/_ref"
g++ -std=c++20 -O2 -fPIC -shared -ffp-contract=off -I"$REF/tests/metal" \
    "$REF/tests/metal/oracles/common.cpp" "$REF/tests/metal/oracles/moe_route.cpp" \
    "$REF/tests/metal/oracles/moe_combine.cpp" "$REF/tests/metal/oracles/moe_swiglu.cpp" \
    "$HERE/ref_driver.cpp" -o "$HERE/_ref/libref_twins.so"
