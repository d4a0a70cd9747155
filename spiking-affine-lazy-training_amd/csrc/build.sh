#!/usr/bin/env bash
# Builds libsalt_hip.so (gfx950) next to the Python package.  Packed-FP32 codegen is
# disabled on purpose (see the project notes on this GPU pool).
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"
root="$(cd "$here/../.." && pwd)"
out="$here/../salt_amd/libsalt_hip.so"
/opt/rocm/bin/hipcc -O3 -std=c++17 --offload-arch=gfx950 -shared -fPIC \
  -Xclang -target-feature -Xclang -packed-fp32-ops \
  -Wall -Wno-unused-function \
  -I "$root/include" -o "$out.tmp" "$here/salt_hip.hip"
mv "$out.tmp" "$out"
echo "built $out"
