"""Pins the oracle's matmul, RMSNorm, RoPE and routing pieces on the CPU.

References: moonlight_kernels.metal:23-130 (matmul, rmsnorm),
:132-200 (RoPE), :469-512 and moe_route.h:12-99 (routing),
moonlight_metal.m:525-559 (route tables), tests/test_moe_route.c:16-112 (KATs).
"""
import ctypes
import os

import numpy as np
import pytest

import oracle_lib as O
from conftest import rel_l2


def dequant(fmt, q, s, out_width, in_width):
    if fmt == 1:
        return q.view(np.int8).reshape(out_width, in_width).astype(np.float64) * s[:, None]
    rb = (in_width + 1) // 2
    b = q.reshape(out_width, rb)
    vals = np.empty((out_width, 2 * rb), np.float64)
    vals[:, 0::2] = (b & 15).astype(np.int64) - 8
    vals[:, 1::2] = (b >> 4).astype(np.int64) - 8
    return vals[:, :in_width] * s[:, None]


@pytest.mark.parametrize("fmt,out_width,in_width,rows", [
    (1, 128, 257, 4), (2, 128, 257, 4), (1, 64, 2048, 1), (2, 96, 2048, 3),
    (0, 33, 100, 2)])
def test_matmul_matches_f64_bruteforce(fmt, out_width, in_width, rows):
    rng = np.random.default_rng(fmt * 1000 + in_width)
    w = rng.normal(0, 0.02, (out_width, in_width)).astype(np.float32)
    x = rng.normal(0, 1, (rows, in_width)).astype(np.float32)
    if fmt == 0:
        q, s, dense = w, None, w.astype(np.float64)
    else:
        q, s = O.quant(w, 8 if fmt == 1 else 4)
        dense = dequant(fmt, q, s, out_width, in_width)
    y = O.matmul(fmt, q, s, x, out_width, in_width)
    ref = x.astype(np.float64) @ dense.T
    assert rel_l2(y, ref) < 1e-6
    # the multithreaded split is the same per-row arithmetic
    assert np.array_equal(O.matmul(fmt, q, s, x, out_width, in_width, threads=4), y)


def test_matmul_closed_forms():
    rng = np.random.default_rng(3)
    w = rng.normal(0, 0.02, (16, 64)).astype(np.float32)
    q, s = O.quant(w, 8)
    qi = q.view(np.int8).reshape(16, 64)
    e5 = np.zeros((1, 64), np.float32)
    e5[0, 5] = 1.0
    y = O.matmul(1, q, s, e5, 16, 64)[0]
    assert np.array_equal(y, qi[:, 5].astype(np.float32) * s)   # unit vector picks a column
    ones = np.ones((1, 64), np.float32)
    y = O.matmul(1, q, s, ones, 16, 64)[0]
    assert np.array_equal(y, qi.sum(axis=1).astype(np.float32) * s)  # row sums (exact ints)
    q4, s4 = O.quant(w, 4)
    y4 = O.matmul(2, q4, s4, e5, 16, 64)[0]
    nib = (q4.reshape(16, 32)[:, 2] >> 4).astype(np.int32) - 8   # column 5 = high nibble of byte 2
    assert np.array_equal(y4, nib.astype(np.float32) * s4)
    assert O.lib().orc_detect_format(16 * 64, 16, 64) == 1
    assert O.lib().orc_detect_format(16 * 32, 16, 64) == 2
    assert O.lib().orc_detect_format(16 * 33, 16, 65) == 2
    assert O.lib().orc_detect_format(100, 16, 64) == -1


def test_rmsnorm_closed_form():
    x = np.array([[3.0, 4.0], [0.0, 0.0]], np.float32)
    w = np.array([1.0, 2.0], np.float32)
    y = np.empty_like(x)
    O.lib().orc_rmsnorm(O.fptr(x), O.fptr(w), O.fptr(y), 2, 2, 0.0)
    r = np.float32(1.0) / np.sqrt(np.float32(12.5))
    assert np.allclose(y[0], [3 * r, 8 * r], rtol=1e-7)
    y_eps = np.empty_like(x)
    O.lib().orc_rmsnorm(O.fptr(x), O.fptr(w), O.fptr(y_eps), 2, 2, 1e-5)
    assert np.all(y_eps[1] == 0)


def test_rope_closed_forms():
    rng = np.random.default_rng(5)
    v = rng.normal(0, 1, 64).astype(np.float32)
    out = np.empty(64, np.float32)
    O.lib().orc_rope(O.fptr(v), O.fptr(out), 64, 0, 50000.0)
    # position 0: identity up to the interleaved -> half layout permutation
    assert np.array_equal(out[:32], v[0::2]) and np.array_equal(out[32:], v[1::2])
    O.lib().orc_rope(O.fptr(v), O.fptr(out), 64, 1234, 50000.0)
    # each pair is rotated: norms preserved, angle = pos * theta^(-2p/64)
    n_in = v[0::2].astype(np.float64) ** 2 + v[1::2].astype(np.float64) ** 2
    n_out = out[:32].astype(np.float64) ** 2 + out[32:].astype(np.float64) ** 2
    assert np.allclose(n_in, n_out, rtol=1e-5)
    ang = 1234 * 50000.0 ** (-2.0 * np.arange(32) / 64)
    z = (v[0::2] + 1j * v[1::2]) * np.exp(1j * ang)
    assert np.allclose(out[:32], z.real, atol=2e-3) and np.allclose(out[32:], z.imag, atol=2e-3)
    assert O.lib().orc_rope_inv_freq(50000.0, 0, 64) == 1.0


def test_route_kats_of_reference_tests():
    # tests/test_moe_route.c:16-33: sigmoid bias changes selection only
    ids, w = O.route(np.array([[0.0, 2.0, -2.0]], np.float32),
                     np.array([0.0, -1.5, 2.0], np.float32), 2, normalize=0)
    assert list(ids[0]) == [2, 0]
    assert abs(w[0, 0] - 1.0 / (1.0 + np.exp(2.0))) < 1e-6 and abs(w[0, 1] - 0.5) < 1e-6
    # :69-81: ties keep the lower index
    ids, _ = O.route(np.zeros((1, 3), np.float32), np.zeros(3, np.float32), 2)
    assert list(ids[0]) == [0, 1]
    # :83-94 finalize: normalise over the selected weights then scale
    ids, w = O.route(np.array([[0.0, 0.0, -50.0]], np.float32), np.zeros(3, np.float32), 2,
                     normalize=1, scale=2.0)
    assert np.allclose(w[0], [1.0, 1.0], rtol=1e-6)
    # :35-38: sigmoid(-100) underflows to 0 through expf
    _, w = O.route(np.array([[-100.0, 5.0]], np.float32), np.zeros(2, np.float32), 2,
                   normalize=0)
    assert w[0, 1] == 0.0


REF_MOE = os.path.join(O.REF_DIR, "libref_moe.so")


def ulp_diff(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return int(np.max(np.abs(a - b))) if a.size else 0


def test_route_score_is_correctly_rounded_sigmoid():
    """K = 1, no normalisation, scale 1: the weight is the score itself,
    1 / (1 + e^-x) with e^-x rounded once to f32 (numpy's f64 exp)."""
    rng = np.random.default_rng(13)
    x = rng.normal(0, 4.0, (4000, 1)).astype(np.float32)
    ids, w = O.route(x, np.zeros(1, np.float32), 1, normalize=0, scale=1.0)
    e = np.exp(-x.astype(np.float64)).astype(np.float32)
    expect = np.float32(1.0) / (np.float32(1.0) + e)
    assert (ids == 0).all() and np.array_equal(w.view(np.uint32), expect.view(np.uint32))


@pytest.mark.skipif(not os.path.exists(REF_MOE), reason="oracle/_ref not built")
def test_route_bit_exact_with_reference_moe_route_h():
    ref = ctypes.CDLL(REF_MOE)
    rng = np.random.default_rng(11)
    experts, top_k = 64, 6
    bias = np.linspace(-0.1, 0.1, experts).astype(np.float32)
    logits = rng.normal(0, 1.0, (500, experts)).astype(np.float32)
    logits[0, :] = 0.0                      # all ties
    logits[1, 10] = logits[1, 20] = 3.0     # tie between two experts after bias? no: bias differs
    logits[2, :] = np.float32(-100.0)       # underflowed scores
    ids, w = O.route(logits, bias, top_k, normalize=1, scale=2.446)
    for r in range(logits.shape[0]):
        ind = np.zeros(top_k, np.int32)
        wt = np.zeros(top_k, np.float32)
        sc = np.zeros(experts, np.float32)
        sel = np.zeros(experts, np.float32)
        n = ref.ref_route_select(O.fptr(logits[r].copy()), O.fptr(bias), experts, top_k, 1,
                                 O.iptr(ind), O.fptr(wt), O.fptr(sc), O.fptr(sel))
        ref.ref_route_finalize.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_int,
                                           ctypes.c_int, ctypes.c_float]
        ref.ref_route_finalize(O.fptr(wt), n, 1, ctypes.c_float(2.446))
        assert np.array_equal(ids[r], ind), r
        # glibc expf (the reference twin) is not correctly rounded for ~0.06 %
        # of inputs; the oracle's score is: weights agree to a few ulp
        assert ulp_diff(w[r], wt) <= 4, r


def test_route_tables_first_appearance_order():
    ids = np.array([[3, 7], [5, 3], [7, 1]], np.int32)
    n, unique, counts, er, es = O.route_tables(ids, experts=8, max_batch=4)
    assert n == 4 and list(unique) == [3, 7, 5, 1]
    assert counts[3] == 2 and counts[7] == 2 and counts[5] == 1 and counts[1] == 1
    assert list(er[3 * 4:3 * 4 + 2]) == [0, 1] and list(es[3 * 4:3 * 4 + 2]) == [0, 1]
    assert list(er[7 * 4:7 * 4 + 2]) == [0, 2] and list(es[7 * 4:7 * 4 + 2]) == [1, 0]
    bad = np.array([[3, 9]], np.int32)
    assert O.route_tables(bad, experts=8, max_batch=4)[0] == -1


def test_route_tables_bruteforce_random():
    rng = np.random.default_rng(2)
    for trial in range(20):
        rows, top_k, experts = int(rng.integers(1, 9)), 3, 12
        ids = np.stack([rng.choice(experts, top_k, replace=False) for _ in range(rows)]).astype(np.int32)
        n, unique, counts, er, es = O.route_tables(ids, experts, max_batch=rows)
        flat = ids.ravel()
        expect_unique = list(dict.fromkeys(flat.tolist()))
        assert list(unique) == expect_unique
        for e in range(experts):
            pos = [(p // top_k, p % top_k) for p in range(flat.size) if flat[p] == e]
            assert counts[e] == len(pos)
            assert [(er[e * rows + j], es[e * rows + j]) for j in range(len(pos))] == pos


@pytest.mark.skipif(not os.path.exists(REF_MOE), reason="oracle/_ref not built")
def test_route_fixed_bit_exact_with_reference():
    ref = ctypes.CDLL(REF_MOE)
    ref.ref_route_finalize.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_int,
                                       ctypes.c_int, ctypes.c_float]
    rng = np.random.default_rng(12)
    experts, top_k, rows = 64, 6, 300
    logits = rng.normal(0, 2.0, (rows, experts)).astype(np.float32)
    ids = O.zipf_routes(rows, experts, top_k, seed=5)
    w = np.empty((rows, top_k), np.float32)
    assert O.lib().orc_route_fixed(O.fptr(logits), rows, experts, top_k, 1, 2.446, O.iptr(ids),
                                   O.fptr(w))
    for r in range(rows):
        wt = np.zeros(top_k, np.float32)
        sc = np.zeros(experts, np.float32)
        n = ref.ref_route_fixed(O.fptr(logits[r].copy()), experts, O.iptr(ids[r].copy()), top_k,
                                1, O.fptr(wt), O.fptr(sc))
        assert n == top_k
        ref.ref_route_finalize(O.fptr(wt), n, 1, ctypes.c_float(2.446))
        assert ulp_diff(w[r], wt) <= 4, r
    bad = ids.copy()
    bad[3, 2] = experts
    assert not O.lib().orc_route_fixed(O.fptr(logits), rows, experts, top_k, 1, 2.446,
                                       O.iptr(bad), O.fptr(w))


def test_zipf_routes_are_distinct_and_skewed():
    ids = O.zipf_routes(2048, 64, 6, seed=3)
    assert all(len(set(r)) == 6 for r in ids)
    counts = np.bincount(ids.ravel(), minlength=64)
    assert counts.sum() == 2048 * 6 and counts.max() > 10 * counts.min()
