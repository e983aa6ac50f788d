#!/bin/sh
# Compiles the reference's CPU path from its own sources, where they lie
# (read-only), into oracle/_ref/libref_moe.so for golden-vector generation.
# Test infrastructure only.  Flags: the reference's Makefile:29-33 (clang,
# -O3, FLASH_ATTENTION FUSED_GEMV Q8_DOT) with the ISA pinned to AVX2
# (-mavx2 -mfma -mf16c) instead of -march=native, so the fp32 lane order is the
# 8-lane one on every host.  Exits 0 without building when the tree is absent.
set -e
REF=${REF:-/root/reference}
HERE=$(cd "$(dirname "$0")" && pwd)
OUT=$HERE/../_ref
if [ ! -f "$REF/matmul.c" ]; then
	echo "build_ref: $REF not present, nothing built"
	exit 0
fi
CC=${REF_CC:-clang}
mkdir -p "$OUT/obj"
FLAGS="-O3 -mavx2 -mfma -mf16c -DFLASH_ATTENTION -DFUSED_GEMV -DQ8_DOT -fPIC -w \
 -I$REF -I$REF/models/olmoe -I$REF/models/llama -I$REF/models/gpt2"
OBJS=""
for f in tensor quant matmul thread_pool nn kvcache gguf vocab json tensor_trace \
	 model prompt tools tools/time tools/calculate; do
	o="$OUT/obj/$(echo "$f" | tr / _).o"
	$CC $FLAGS -c "$REF/$f.c" -o "$o"
	OBJS="$OBJS $o"
done
for f in ref_olmoe ref_llama ref_ops ref_q4; do
	$CC $FLAGS -c "$HERE/$f.c" -o "$OUT/obj/$f.o"
	OBJS="$OBJS $OUT/obj/$f.o"
done
$CC -shared -o "$OUT/libref_moe.so" $OBJS -lm -lpthread
echo "build_ref: built $OUT/libref_moe.so"

# The integration lines of INTEGRATION.md around the reference's olmoe.c,
# linked against the product library (tests/test_dropin.py).
LIBDIR=$HERE/../../llm.c_amd
if [ -f "$LIBDIR/libhip_moe.so" ]; then
	$CC $FLAGS -I$HERE/../../include -c "$HERE/../../tests/native/dropin_olmoe.c" \
		-o "$OUT/obj/dropin_olmoe.o"
	DOBJS=""
	for o in $OBJS; do
		case "$o" in */ref_*) ;; *) DOBJS="$DOBJS $o" ;; esac
	done
	$CC -shared -o "$OUT/libdropin_olmoe.so" $DOBJS "$OUT/obj/dropin_olmoe.o" \
		-L"$LIBDIR" -lhip_moe -Wl,-rpath,"\$ORIGIN/../../llm.c_amd" -lm -lpthread
	echo "build_ref: built $OUT/libdropin_olmoe.so"
fi
