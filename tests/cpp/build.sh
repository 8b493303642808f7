#!/bin/bash
# Builds tests/cpp/build/facade_parity against the in-tree libraries.
set -e
HERE="$(cd "$(dirname "$0")" && pwd)"
ROOT="$(cd "$HERE/../.." && pwd)"
mkdir -p "$HERE/build"
g++ -std=c++17 -O2 -Wno-unused-result -D__HIP_PLATFORM_AMD__ -I/opt/rocm/include -I"$ROOT/include" \
  "$HERE/facade_parity.cpp" -o "$HERE/build/facade_parity" \
  -L"$ROOT/hierarchicalkv-ascend_amd/lib" -lhkv_amd -L"$ROOT/oracle" -loracle \
  -L/opt/rocm/lib -lamdhip64 \
  -Wl,-rpath,"\$ORIGIN/../../../hierarchicalkv-ascend_amd/lib:\$ORIGIN/../../../oracle:/opt/rocm/lib"
# The functor APIs instantiate their kernels in the caller's code: hipcc.
/opt/rocm/bin/hipcc --offload-arch=gfx950 -std=c++17 -O2 -Wno-unused-value -Xclang -target-feature -Xclang -packed-fp32-ops \
  -I"$ROOT/include" "$HERE/facade_predicates.hip" -o "$HERE/build/facade_predicates" \
  -L"$ROOT/hierarchicalkv-ascend_amd/lib" -lhkv_amd -L"$ROOT/oracle" -loracle \
  -Wl,-rpath,"\$ORIGIN/../../../hierarchicalkv-ascend_amd/lib:\$ORIGIN/../../../oracle:/opt/rocm/lib"
