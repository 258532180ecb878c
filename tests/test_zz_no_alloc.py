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
_CACHED = []  # host weights handed to fm_matmul_q8 with cache = 1


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


def hip_runtime():
    """The HIP runtime instance libfloyd_amd.so runs on (the one already
    mapped into this process)."""
    import ctypes
    with open("/proc/self/maps") as f:
        paths = {line.split()[-1] for line in f if "libamdhip64" in line}
    assert paths, "libamdhip64 is not loaded"
    return ctypes.CDLL(sorted(paths)[0])


def device_free_bytes(hip):
    import ctypes
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_static_calls_allocate_nothing(fm):
    """Free device memory is the same before and after a series of
    fm_matmul_static calls (each shape called once beforehand, so the HIP
    runtime's own lazy loading of the kernels' code is not counted).  As a
    control, fm_matmul_q8 with cache = 1 on a new weight (a device copy kept
    by host pointer) shows up in the same measurement."""
    print("[gpu] fm_matmul_static: device free bytes across calls", flush=True)
    hip = hip_runtime()
    shapes = [(8, 11264, 2048, 4, 91), (4, 11264, 2048, 1, 92), (8, 577, 1031, 3, 93)]
    cases = [(bits, O_, I, S) + case(bits, O_, I, S, seed) for bits, O_, I, S, seed in shapes]
    for bits, O_, I, S, q, s, x in cases:
        y = np.empty((S, O_), np.float32)
        assert fm.fm_matmul_static(bits, fptr(y), fptr(x), q.ctypes.data, fptr(s), O_, I, S) == 1
    before = device_free_bytes(hip)
    for _ in range(3):
        for bits, O_, I, S, q, s, x in cases:
            y = np.empty((S, O_), np.float32)
            assert fm.fm_matmul_static(bits, fptr(y), fptr(x), q.ctypes.data, fptr(s), O_, I,
                                       S) == 1
            assert np.isfinite(y).all()
    after = device_free_bytes(hip)
    assert after == before, (before, after)
    # control: a cached fm_matmul_q8 weight (11264 x 2048 q8, 22 MiB) is a
    # device allocation the measurement sees
    bits, O_, I, S, q, s, x = cases[0]
    q_new = q.copy()
    _CACHED.append(q_new)  # the cache is keyed by host pointer: keep it alive
    y = np.empty((S, O_), np.float32)
    fm.fm_matmul_q8(fptr(y), fptr(x), q_new.ctypes.data, fptr(s), O_, I, S, 1)
    assert np.isfinite(y).all()
    assert device_free_bytes(hip) <= after - q_new.nbytes
