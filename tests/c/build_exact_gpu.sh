#!/bin/sh
# Builds tests/c/exact_rounding_gpu.hip with the library's device flags:
# build_exact_gpu.sh OUTPUT
set -e
ROOT=$(cd "$(dirname "$0")/../.." && pwd)
HIPCC=${HIPCC:-/opt/rocm/bin/hipcc}
$HIPCC -O3 -std=c++17 --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops \
    -fhip-fp32-correctly-rounded-divide-sqrt -ffp-contract=off \
    "$ROOT/tests/c/exact_rounding_gpu.hip" -o "$1" 2>&1 | grep -v "packed-fp32-ops" || true
test -x "$1"
