#!/bin/sh
# Builds the reference pieces that compile from their own sources (header-only
# routing / f32 MoE, and the safetensors container reader) into oracle/_ref/.
# Nothing is copied: the sources are compiled where they lie.  Used only as a
# checker of the oracle and of the product's host-side parsing.
set -e
REF=${FLOYD_REFERENCE:-/root/reference}
HERE=$(cd "$(dirname "$0")" && pwd)
OUT="$HERE/_ref"
if [ ! -f "$REF/moe_route.h" ]; then
    echo "build_ref: $REF not present, skipping" >&2
    exit 0
fi
mkdir -p "$OUT"
CFLAGS="-O2 -fPIC -shared -std=gnu11 -ffp-contract=off -w"
gcc $CFLAGS -I"$REF" -o "$OUT/libref_moe.so" "$HERE/ref_wrap_moe.c" -lm
gcc $CFLAGS -I"$REF" -o "$OUT/libref_model.so" "$HERE/ref_wrap_model.c" \
    "$REF/moonlight_model.c" -lm
echo "build_ref: built $OUT/libref_moe.so $OUT/libref_model.so"
