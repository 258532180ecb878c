"""Pins the oracle's packing (quant_int8 / quant_int4 restatement) and its
synthetic-input helpers.

Reference: tools/convert_moonlight.py:46-66.  The golden vectors in
tests/golden/quant_golden.npz were produced by the reference's own functions
(tests/golden/make_golden.py); the closed-form cases below fail for the
plausible slips (scale from mean instead of amax, truncation instead of
round-half-even, swapped nibbles, pad nibble 8 instead of 0, 1e-8 floor lost).
"""
import os

import numpy as np
import pytest

import oracle_lib as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quant_golden.npz")


def golden_cases():
    g = np.load(GOLDEN, allow_pickle=False)
    names = sorted({k.rsplit(".", 1)[0] for k in g.files})
    return g, names


@pytest.mark.parametrize("bits", [8, 4])
def test_quant_matches_reference_golden(bits):
    g, names = golden_cases()
    assert len(names) >= 6
    for name in names:
        q, s = O.quant(g[name + ".w"], bits)
        assert np.array_equal(q, g[f"{name}.q{bits}"]), name
        assert np.array_equal(s.view(np.uint32), g[f"{name}.s{bits}"].view(np.uint32)), name


def test_q8_closed_forms():
    w = np.array([[127.0, -63.5, 63.5, 0.5, 1.5, -0.5, -127.0, 0.0],
                  [0.0] * 8,
                  [2.0, 0, 0, 0, 0, 0, 0, 0]], np.float32)
    q, s = O.quant(w, 8)
    q = q.view(np.int8).reshape(3, 8)
    assert s[0] == np.float32(1.0)
    # round half to even: -63.5 -> -64, 63.5 -> 64, 0.5 -> 0, 1.5 -> 2, -0.5 -> -0
    assert list(q[0]) == [127, -64, 64, 0, 2, 0, -127, 0]
    assert s[1] == np.float32(1e-8) and not q[1].any()      # all-zero row: 1e-8 floor
    assert s[2] == np.float32(2.0) / np.float32(127.0)      # f32 division
    assert q[2, 0] == 127                                     # amax element -> qmax


def test_q4_closed_forms():
    w = np.array([[7.0, -7.0, 3.5, -3.5, 0.5, 1.0, 2.0]], np.float32)  # odd width
    q, s = O.quant(w, 4)
    assert s[0] == np.float32(1.0)
    assert q.size == 4
    nib = [(b & 15, b >> 4) for b in q]
    # values + 8, even column in the low nibble
    assert nib[0] == (15, 1)           # 7, -7
    assert nib[1] == (12, 4)           # 3.5 -> 4, -3.5 -> -4
    assert nib[2] == (8, 9)            # 0.5 -> 0, 1.0 -> 1
    assert nib[3] == (10, 0)           # 2.0 -> 2; pad nibble stays 0
    zero_q, zero_s = O.quant(np.zeros((1, 4), np.float32), 4)
    assert zero_s[0] == np.float32(1e-8) and list(zero_q) == [0x88, 0x88]


def test_bf16_round_and_normal_stream():
    assert O.lib().orc_bf16_round(1.0) == 1.0
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7: even mantissa (1.0) wins
    assert O.lib().orc_bf16_round(1.0 + 2.0 ** -8) == 1.0
    assert O.lib().orc_bf16_round(1.0 + 3 * 2.0 ** -8) == 1.0 + 2.0 ** -6
    x = O.fill_normal(200000, seed=7)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    y = O.fill_normal(200000, seed=7, std=0.02, bf16=True)
    assert np.all((y.view(np.uint32) & 0xFFFF) == 0)
    assert abs(y.std() - 0.02) < 0.001
    assert np.array_equal(O.fill_normal(1000, seed=7), x[:1000])  # index-addressable
