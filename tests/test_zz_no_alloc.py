"""GPU test of fm_matmul_static (include/fm_backend.h), the allocation-free
variant of fm_matmul_q8 / fm_matmul_q4: through the C ABI, two calls in a row
(the second with a smaller input, so stale bytes of the first would show)
return exactly what fm_matmul_q8 / _q4 return on the same inputs, and sizes
beyond the static scratch are refused before any device work."""
import numpy as np
import pytest

import oracle_lib as O
from conftest import rel_l2
from floyd_amd import native

pytestmark = pytest.mark.gpu

SCRATCH = 32 << 20


@pytest.fixture(scope="module")
def fm(device):
    lib = native.load()  # binds the include/*.h signatures (void pointers)
    assert lib.fm_init() == 1
    return lib


def fptr(a):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def case(bits, O_, I, S, seed):
    w = O.fill_normal(O_ * I, seed, std=0.02, bf16=True).reshape(O_, I)
    q, s = O.quant(w, bits)
    x = O.fill_normal(S * I, seed + 1).reshape(S, I)
    return q, s, x


def run_pair(fm, bits, O_, I, S, seed):
    q, s, x = case(bits, O_, I, S, seed)
    ref = np.empty((S, O_), np.float32)
    getattr(fm, f"fm_matmul_q{bits}")(fptr(ref), fptr(x), q.ctypes.data, fptr(s), O_, I, S, 0)
    got = np.full((S, O_), 7.0, np.float32)
    assert fm.fm_matmul_static(bits, fptr(got), fptr(x), q.ctypes.data, fptr(s), O_, I, S) == 1
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (bits, O_, I, S)
    expect = O.matmul(native.MLK_Q8 if bits == 8 else native.MLK_Q4, q, s, x, O_, I)
    assert rel_l2(got, expect) < 1e-5
    return got


@pytest.mark.parametrize("bits", [8, 4])
def test_static_matches_fm_matmul(fm, bits):
    print(f"[gpu] fm_matmul_static q{bits}: large then small call", flush=True)
    # a Moonlight dense projection (23 MB of q8 weights), then a smaller one
    # with a ragged width: the second call runs on the first call's leftovers
    run_pair(fm, bits, 11264, 2048, 4, 31 + bits)
    run_pair(fm, bits, 577, 1031, 3, 57 + bits)


def test_static_refuses_oversize(fm):
    q, s, x = case(8, 64, 2048, 1, 5)
    y = np.zeros((1, 16384), np.float32)
    big_o = 16384  # 16384 x 2048 q8 = 32 MiB of weights alone: over the limit
    w = np.zeros((big_o, 2048), np.int8)
    s_big = np.ones(big_o, np.float32)
    assert fm.fm_matmul_static(8, fptr(y), fptr(x), w.ctypes.data, fptr(s_big), big_o, 2048,
                               1) == 0
    assert np.isnan(y).all()
    assert b"static scratch" in fm.mlk_last_error()
    assert fm.fm_matmul_static(3, fptr(y), fptr(x), q.ctypes.data, fptr(s), 64, 2048, 1) == 0
    # the array still serves a valid call afterwards
    run_pair(fm, 8, 64, 2048, 1, 5)
