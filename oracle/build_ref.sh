#!/bin/sh
# Compiles the reference's own hot-path translation units, where they lie, into oracle/_ref/.
# Used only to pin the oracle and as the CPU baseline (test infrastructure; nothing in the product
# links it). No reference source is copied. Sources compiled: ds_quantize.c, ds_kernels.c,
# ds_kernels_avx.c, ds_kernels_generic.c (without -DUSE_BLAS; every cblas call in them is under
# #ifdef USE_BLAS) plus oracle/ref_harness.c, which defines the two mode globals the reference
# defines in ds_ocr.c (ds_ocr.c itself needs the Darwin-only Metal backend, so it is not built).
# The reference's ds_kernels.c does not compile on x86-64 as shipped: it uses the function-pointer
# types ds_bf16_matvec_fused_fn_t / ds_argmax_bf16_range_fn_t unconditionally (ds_kernels.c:59-60)
# but ds_kernels_impl.h:44-51 declares them only under __ARM_NEON. FIXTYPES names those two types on
# the command line as the types of the reference's own generic kernels (same signatures); no file
# is added and no reference source is changed.
# Flags: the reference Makefile's -O3 with -march=x86-64-v4 instead of -march=native, so the binary
# runs on any AVX-512F/BW host (the reference only branches on __AVX512F__/__AVX512BW__/__AVX2__/
# __FMA__, all of which x86-64-v4 defines). An AVX2-only variant (x86-64-v3) is built beside it.
set -e
REF=${DS_REF_DIR:-/root/reference}
HERE=$(cd "$(dirname "$0")" && pwd)
OUT="$HERE/_ref"
if [ ! -f "$REF/ds_quantize.c" ]; then
  echo "build_ref.sh: reference sources not found at $REF; skipping" >&2
  exit 0
fi
mkdir -p "$OUT"
FIXTYPES="-Dds_bf16_matvec_fused_fn_t=__typeof__(&ds_bf16_matvec_fused_generic) -Dds_argmax_bf16_range_fn_t=__typeof__(&ds_argmax_bf16_range_generic)"
SRCS="$REF/ds_quantize.c $REF/ds_kernels.c $REF/ds_kernels_avx.c $REF/ds_kernels_generic.c $HERE/ref_harness.c"
gcc -O3 -march=x86-64-v4 -fPIC -shared -w $FIXTYPES -I"$REF" $SRCS -o "$OUT/libdsref_v4.so" -lm -lpthread
gcc -O3 -march=x86-64-v3 -fPIC -shared -w $FIXTYPES -I"$REF" $SRCS -o "$OUT/libdsref_v3.so" -lm -lpthread
echo "built $OUT/libdsref_v4.so $OUT/libdsref_v3.so"
