#!/bin/bash
# Builds trace/lib/libitts_trace.so: the product library with the persistent decode step
# replaced by its instrumented copy (instrument.py).  The other objects come from the
# product build, so run `make -C index-tts-rs_amd` first.
set -e
cd "$(dirname "$0")"
HIPCC=${HIPCC:-/opt/rocm/bin/hipcc}
mkdir -p _gen lib
python3 instrument.py ../csrc/kernels_persist.hip _gen/kernels_persist_trace.hip
# the generated file sits outside csrc; headers resolve to the product's
$HIPCC --offload-arch=gfx950 -O3 -std=c++17 -fPIC -Wall -Wno-unused-function \
  -Xclang -target-feature -Xclang -packed-fp32-ops -I../csrc -c _gen/kernels_persist_trace.hip -o _gen/kp_trace.o
B=../_build
$HIPCC --offload-arch=gfx950 -shared -fPIC -o lib/libitts_trace.so $B/kernels_decode.o $B/kernels_prefill.o \
  $B/kernels_sampler.o _gen/kp_trace.o $B/kernels_attn.o $B/kernels_cfm.o $B/runtime.o $B/loader.o $B/cfm.o -lpthread
echo "built trace/lib/libitts_trace.so"
