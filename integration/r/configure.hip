# configure.hip -- the HIP (gfx950) branch of fastEmbedR's configure.
#
# Sourced by configure after its CUDA branch (configure:67-113), with
#     . ./configure.hip
# It mirrors that branch: it detects hipcc, chooses the implementation or the
# stub object, and prepares the Makevars rules that compile the HIP sources.
# configure then adds "embedding_hip_bridge.o $hip_objects" to OBJECTS and
# prints "$hip_rule" into src/Makevars when hip_enabled is 1, as it does for
# $cuda_objects and $cuda_rule (configure:312-327).
#
# Environment:
#   FASTEMBEDR_USE_HIP   auto (default): build the HIP backend when hipcc is
#                        found; 1: require it; 0: never (stub only)
#   HIPCC                hipcc to use (default $ROCM_PATH/bin/hipcc)
#   ROCM_PATH, HIP_PATH  ROCm installation (default /opt/rocm)
#   FASTEMBEDR_HIP_ARCH  offload target; the kernels are written for CDNA4,
#                        so only gfx950 is accepted
#   FASTEMBEDR_HIP_SRC   directory of the HIP sources, relative to src/
#                        (default hip: fastembedr_hip.h and the files of
#                        fastembedr_amd/csrc/)
#
# Sets: hip_enabled (0/1), hip_objects, hip_rule, hip_device_flags,
# hip_host_flags; extends cppflags and libs.  The device and host flags are
# those of fastembedr_amd/build.py: the perplexity search keeps denormals
# (-fno-gpu-flush-denormals-to-zero) for its bit-level agreement with the CPU
# search, and packed fp32 instructions stay off.

use_hip=${FASTEMBEDR_USE_HIP:-auto}
hip_enabled=0
hip_objects="embedding_hip_stub.o"
hip_rule=""
hip_units="embedding_hip_kernels attraction_tiles_hip transform_hip interp_grid_hip knn_hip metrics_hip"
hip_host_units="embedding_hip_session"
rocm_home=${ROCM_PATH:-${HIP_PATH:-/opt/rocm}}
hipcc=${HIPCC:-}
if [ -z "$hipcc" ] && [ -x "$rocm_home/bin/hipcc" ]; then
  hipcc="$rocm_home/bin/hipcc"
fi
hip_arch=${FASTEMBEDR_HIP_ARCH:-gfx950}
hip_src=${FASTEMBEDR_HIP_SRC:-hip}
hip_device_flags="--offload-arch=$hip_arch -O3 -std=c++17 -fPIC -fvisibility=hidden -fno-gpu-flush-denormals-to-zero -Xclang -target-feature -Xclang -packed-fp32-ops -Wall"
hip_host_flags="-O2 -std=c++17 -fPIC -fvisibility=hidden -Wall -D__HIP_PLATFORM_AMD__"

if [ "$use_hip" = "1" ] && [ -z "$hipcc" ]; then
  echo "FASTEMBEDR_USE_HIP=1 but no hipcc was found (set HIPCC or ROCM_PATH)." >&2
  exit 1
fi
if [ "$use_hip" != "0" ] && [ -n "$hipcc" ]; then
  if [ "$hip_arch" != "gfx950" ]; then
    echo "FASTEMBEDR_HIP_ARCH=$hip_arch: the HIP kernels are written for gfx950 (MI355X) only." >&2
    exit 1
  fi
  hip_enabled=1
  hip_objects="embedding_hip_impl.o"
  for unit in $hip_host_units $hip_units; do
    hip_objects="$hip_objects $unit.o"
  done
  # embedding_hip_impl.cpp is compiled by R's C++ compiler: it needs the
  # C ABI header and the HIP runtime API header (device buffers of the KNN).
  cppflags="$cppflags -DFASTEMBEDR_HAS_HIP -D__HIP_PLATFORM_AMD__ -I$hip_src -I$rocm_home/include"
  libs="$libs -L$rocm_home/lib -Wl,-rpath,$rocm_home/lib -lamdhip64"
  # the object rules below must not become make's default goal when the
  # CUDA rule (which sets it too) is absent
  hip_rule="
.DEFAULT_GOAL := all

HIPCC = $hipcc
HIP_DEVICE_FLAGS = $hip_device_flags -I$hip_src
HIP_HOST_FLAGS = $hip_host_flags -I$hip_src
"
  for unit in $hip_units; do
    hip_rule="$hip_rule
$unit.o: $hip_src/$unit.hip
	\$(HIPCC) \$(HIP_DEVICE_FLAGS) -c \$< -o \$@
"
  done
  for unit in $hip_host_units; do
    hip_rule="$hip_rule
$unit.o: $hip_src/$unit.cpp
	\$(HIPCC) \$(HIP_HOST_FLAGS) -c \$< -o \$@
"
  done
fi
