#!/bin/sh
# Builds tests/native/host_status (the host runtime, the CPU oracle and the
# status driver) with AddressSanitizer and UndefinedBehaviorSanitizer on the
# host side.  Usage: build_host_status.sh OUT_DIR
set -e
ROOT=$(cd "$(dirname "$0")/../.." && pwd)
OUT=$1
mkdir -p "$OUT"
HIPCC=${HIPCC:-/opt/rocm/bin/hipcc}
SAN="-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined -Xarch_host -fno-sanitize-recover=undefined -Xarch_host -fno-omit-frame-pointer"
FLAGS="--offload-arch=gfx950 -O1 -g -std=c++17 -Wno-unused-result -Xclang -target-feature -Xclang -packed-fp32-ops -I$ROOT/include"
objs=""
for src in "$ROOT"/qwen38-metal_amd/csrc/*.hip "$ROOT"/qwen38-metal_amd/csrc/*.cpp; do
  obj="$OUT/$(basename "$src").o"
  "$HIPCC" $FLAGS $SAN -c "$src" -o "$obj" &
  objs="$objs $obj"
done
"$HIPCC" $FLAGS $SAN -fopenmp -c "$ROOT/oracle/qm_oracle.cpp" -o "$OUT/qm_oracle.o" &
"$HIPCC" $FLAGS $SAN -c "$ROOT/tests/native/host_status.cpp" -o "$OUT/host_status.o" &
wait
"$HIPCC" --offload-arch=gfx950 $SAN -fopenmp $objs "$OUT/qm_oracle.o" "$OUT/host_status.o" -o "$OUT/host_status"
