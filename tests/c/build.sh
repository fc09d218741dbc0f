#!/bin/sh
# Builds tests/c/kvm_abi_decode.c (C99, gcc) against include/kvm_hotpath.h,
# the library, the C oracle and the HIP runtime: build.sh OUTPUT
set -e
ROOT=$(cd "$(dirname "$0")/../.." && pwd)
ROCM=${ROCM_PATH:-/opt/rocm}
LIB=$ROOT/kvmem-llama.cpp_amd/lib
gcc -std=c99 -O2 -Wall -Wextra -Werror -D__HIP_PLATFORM_AMD__ \
    -I"$ROOT/include" -I"$ROOT/oracle" -I"$ROCM/include" \
    "$ROOT/tests/c/kvm_abi_decode.c" -o "$1" \
    -L"$LIB" -lkvm_hotpath -L"$ROOT/oracle" -lkvm_oracle -L"$ROCM/lib" -lamdhip64 -lm \
    -Wl,-rpath,"$LIB" -Wl,-rpath,"$ROOT/oracle" -Wl,-rpath,"$ROCM/lib"
