#!/bin/sh
# Builds the reference with the HIP backend dropped in, the way a maintainer
# would: a temporary copy of the reference's src/ tree,
# guanaco_amd/host/reference-hip.patch applied, hip_backend.c / .h added, all
# compiled with -DUSE_HIP=1 against libgq_hip.so.  Outputs, and nothing else,
# go to oracle/_ref/ (or $1):
#   libref_hip.so  the patched engine, loader, sessions, CPU kernels, factory
#                  and the HIP backend (the tests drive it through ctypes);
#   guanaco_hip    the patched command-line program (main.c).
# The temporary copy is removed on exit; no reference source is kept.
set -eu
HERE=$(cd "$(dirname "$0")" && pwd)
ROOT=$(dirname "$HERE")
REF=${REF:-/root/reference}
OUT=${1:-$HERE/_ref}
CC=${CC:-gcc}
T=$(mktemp -d)
trap 'rm -rf "$T"' EXIT
cp -r "$REF/src" "$T/src"
(cd "$T/src" && patch -p1 --quiet --forward --no-backup-if-mismatch < "$ROOT/guanaco_amd/host/reference-hip.patch")
cp "$ROOT/guanaco_amd/host/hip_backend.c" "$T/src/backend/"
cp "$ROOT/guanaco_amd/host/hip_backend.h" "$T/src/include/"
S="$T/src"
SRCS="$S/engine/loader.c $S/engine/engine.c $S/engine/generate.c $S/engine/chat.c $S/engine/session.c
      $S/engine/gpu_prefill.c $S/kernels/cpu/kernels_cpu.c $S/kernels/cpu/quant_matvec_q8_0.c
      $S/kernels/cpu/quant_matvec_q4_k.c $S/kernels/cpu/quant_matvec_q6_k.c $S/memory/arena.c
      $S/memory/scratch.c $S/memory/kv_cache.c $S/tokenizer/tokenizer.c $S/backend/backend.c
      $S/backend/cpu_backend.c $S/backend/cuda_backend.c $S/threadpool/threadpool.c"
# the reference's flags (Makefile:16, USE_PTHREAD per build.sh:57) plus USE_HIP
FLAGS="-std=c11 -D_GNU_SOURCE -O2 -mavx2 -mfma -DUSE_PTHREAD=1 -DUSE_HIP=1 -pthread -fPIC -I$S/include -I$S/backend -I$ROOT/include"
LINK="-L$ROOT/guanaco_amd -Wl,-rpath,$ROOT/guanaco_amd -Wl,-rpath,\$ORIGIN/../../guanaco_amd -lgq_hip -lm"
mkdir -p "$OUT"
# the HIP backend with every warning on; the reference's files as it builds them
$CC $FLAGS -Wall -Wextra -Werror -c "$S/backend/hip_backend.c" -o "$T/hip_backend.o"
$CC $FLAGS -w -shared -o "$OUT/libref_hip.so" $SRCS "$T/hip_backend.o" $LINK -Wl,-Bsymbolic
$CC $FLAGS -w -o "$OUT/guanaco_hip" $SRCS "$S/main.c" "$T/hip_backend.o" $LINK
