"""Writes tests/golden/quant_golden.npz: packing vectors from the reference's own
quantizer.

The reference packs weights with quant_int8 / quant_int4 in
tools/convert_moonlight.py:46-66 (numpy float32 arithmetic).  No test or file in
the reference holds their output, so this script imports those two functions
from the reference tree (in the build container only; nothing here runs on the
GPU box) and records input -> (bytes, scales) pairs.  The committed .npz is
plain data: float32 inputs, uint8 packed bytes, float32 per-row scales.

Run:  python tests/golden/make_golden.py [--reference /root/reference]
"""
import argparse
import importlib.util
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def load_converter(reference):
    path = os.path.join(reference, "tools", "convert_moonlight.py")
    spec = importlib.util.spec_from_file_location("convert_moonlight_ref", path)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def bf16_round(a):
    """float32 -> nearest-even bfloat16 -> float32 (as the container's source)."""
    u = a.astype(np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def cases():
    rng = np.random.default_rng(20261201)
    out = {}
    out["rand_16x64"] = bf16_round(rng.normal(0, 0.02, (16, 64)))
    out["rand_64x2048"] = bf16_round(rng.normal(0, 0.02, (64, 2048)))
    out["odd_7x33"] = bf16_round(rng.normal(0, 1.0, (7, 33)))
    out["odd_3x1"] = np.array([[0.5], [-3.0], [0.0]], np.float32)
    out["wide_range_4x257"] = bf16_round(
        rng.normal(0, 1.0, (4, 257)) * np.array([[1e-3], [1.0], [1e3], [1e-9]]))
    special = np.zeros((8, 16), np.float32)
    special[1, 3] = 0.25                              # single non-zero
    special[2] = np.arange(16) - 7.5                  # exact .5 quotients (q4)
    special[3] = (np.arange(16) - 8) * (127.0 / 8)    # amax at the negative end
    special[4, :] = 1e-12                             # scale floor 1e-8
    special[5] = [127, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5,
                  126.5, -126.5, 63.5, -63.5, 0, 1, -1, 64.5]  # q8 ties
    special[6] = [7, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5,
                  6.5, -6.5, 5.5, -5.5, 0, 4.5, -4.5, -7]       # q4 ties
    special[7] = -special[6]
    out["special_8x16"] = special
    return out


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument("--reference", default="/root/reference")
    args = parser.parse_args()
    conv = load_converter(args.reference)
    arrays = {}
    for name, w in cases().items():
        w = np.ascontiguousarray(w, dtype=np.float32)
        arrays[name + ".w"] = w
        for bits in (8, 4):
            fn = conv.quant_int8 if bits == 8 else conv.quant_int4
            q, s = fn(w, bits)
            arrays[f"{name}.q{bits}"] = np.asarray(q, np.uint8)
            arrays[f"{name}.s{bits}"] = np.asarray(s, np.float32)
    dest = os.path.join(HERE, "quant_golden.npz")
    np.savez_compressed(dest, **arrays)
    print(f"wrote {dest}: {len(arrays)} arrays")


if __name__ == "__main__":
    main()
