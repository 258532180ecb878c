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

# The reference's own boundary tests, compiled unchanged from their sources
# and linked against libfloyd_amd.so in place of moonlight_metal.m /
# backend_metal.m: proof that the C ABI is a drop-in.  They run on the GPU
# (tests/test_reference_link_gpu.py, tests/test_reference_moonlight_gpu.py)
# against fixtures written by the CPU oracle (tests/golden/).  The runtime
# test asserts an Apple device name (test_moonlight_metal_runtime.c:94); its
# runnable build is made from a copy with that one string changed to
# "gfx950", written into this build directory only.
LIB="$HERE/../floyd_amd/lib"
if [ -f "$LIB/libfloyd_amd.so" ]; then
    LINK="-L$LIB -lfloyd_amd -Wl,-rpath,\$ORIGIN/../../floyd_amd/lib -lm"
    gcc -O2 -w -I"$REF" -o "$OUT/test_backend_metal" "$REF/tests/test_backend_metal.c" $LINK
    for t in runtime primitives mla moe; do
        gcc -O2 -w -fopenmp -I"$REF" -o "$OUT/test_moonlight_metal_$t" \
            "$REF/tests/test_moonlight_metal_$t.c" "$REF/moonlight_model.c" $LINK
    done
    sed 's/moonlight_device_name(model), "Apple"/moonlight_device_name(model), "gfx950"/' \
        "$REF/tests/test_moonlight_metal_runtime.c" > "$OUT/runtime_device_patched.c"
    grep -q '"gfx950"' "$OUT/runtime_device_patched.c"
    gcc -O2 -w -fopenmp -I"$REF" -I"$REF/tests" -o "$OUT/test_moonlight_metal_runtime_gfx950" \
        "$OUT/runtime_device_patched.c" "$REF/moonlight_model.c" $LINK
    rm -f "$OUT/runtime_device_patched.c"
    echo "build_ref: linked the reference's backend and Moonlight tests against libfloyd_amd.so"
    # The real callers: floyd's CLI (floyd.c, moonlight_chat.c, moonlight_model.c
    # and the HTTP layer it links) compiled unchanged with the reference's own
    # flags (Makefile:26-29) and linked against the library in place of
    # moonlight_metal.o / backend_metal.o; dsv4_stub.c stands in for the
    # DeepSeek-V4 objects, which are not part of this path.
    gcc -O3 -fopenmp -w -I"$REF" -o "$OUT/floyd" "$REF/floyd.c" "$REF/moonlight_chat.c" \
        "$REF/moonlight_model.c" "$REF/openai_http.c" "$REF/openai_responses.c" \
        "$HERE/dsv4_stub.c" $LINK -pthread
    echo "build_ref: linked floyd (floyd.c + moonlight_chat.c, unchanged) against libfloyd_amd.so"
fi
