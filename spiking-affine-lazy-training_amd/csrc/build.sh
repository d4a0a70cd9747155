#!/usr/bin/env bash
# Builds libsalt_hip.so (gfx950) next to the Python package.  The kernel families are
# instantiated in separate objects (conv_inst.hip per iteration count, fc_inst.hip per
# weight width) compiled in parallel.  Packed-FP32 codegen is disabled on purpose.
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"
root="$(cd "$here/../.." && pwd)"
out="$here/../salt_amd/libsalt_hip.so"
obj="$(mktemp -d "${TMPDIR:-/tmp}/salt_build.XXXXXX")"
trap 'rm -rf "$obj"' EXIT
flags=(-O3 -std=c++17 --offload-arch=gfx950 -fPIC
       -Xclang -target-feature -Xclang -packed-fp32-ops
       -Wall -Wno-unused-function -I "$root/include" -I "$here")
hipcc=/opt/rocm/bin/hipcc

pids=()
"$hipcc" "${flags[@]}" -c "$here/salt_hip.hip" -o "$obj/salt_hip.o" & pids+=($!)
"$hipcc" "${flags[@]}" -c "$here/trace_kernel.hip" -o "$obj/trace.o" & pids+=($!)
for n in 1 2 3 4 8; do
  "$hipcc" "${flags[@]}" -DSALT_NIT=$n -c "$here/conv_inst.hip" -o "$obj/conv_$n.o" & pids+=($!)
done
for n in 1 2 3 4 5 6 7 8; do
  "$hipcc" "${flags[@]}" -DSALT_PACK_IMAX=$n -c "$here/conv_packed_inst.hip" -o "$obj/pack_$n.o" & pids+=($!)
done
for q in 8 16 32; do
  "$hipcc" "${flags[@]}" -DSALT_QBITS=$q -c "$here/fc_inst.hip" -o "$obj/fc_$q.o" & pids+=($!)
done
status=0
for p in "${pids[@]}"; do wait "$p" || status=1; done
if [ "$status" -ne 0 ]; then echo "build failed" >&2; exit 1; fi
"$hipcc" --offload-arch=gfx950 -shared -fPIC -o "$out.tmp" "$obj"/*.o
mv "$out.tmp" "$out"
echo "built $out"
# The LDS bandwidth probe bench.py's roofline uses: a library of its own, not linked into
# the forward path.
probe="$here/../salt_amd/libsalt_probe.so"
"$hipcc" "${flags[@]}" -shared -o "$probe.tmp" "$here/lds_probe.hip"
mv "$probe.tmp" "$probe"
echo "built $probe"
