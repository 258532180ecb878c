"""GPU parity of the dequant GEMV (include/moonlight_kernels.h mlk_gemv*,
include/fm_backend.h) against the CPU oracle on the same seeded inputs.

Tolerances: the path computes in fp32 with a different summation order than
the oracle's serial loop, so results agree to rounding; the contract is
rel-L2 <= 1e-3, checked here at 1e-5, and the
reference's own kernel gate of max relative error <= 1e-3
(tests/test_backend_metal.c:50-77).
"""
import numpy as np
import pytest

import oracle_lib as O
from conftest import rel_l2
from floyd_amd import native
from floyd_amd.native import DeviceBuffer

pytestmark = pytest.mark.gpu

TOL = 1e-5


def make_weights(fmt, out_width, in_width, seed):
    w = O.fill_normal(out_width * in_width, seed, std=0.02, bf16=True).reshape(out_width, in_width)
    if fmt == 0:
        return w, None
    return O.quant(w, 8 if fmt == 1 else 4)


SHAPES = [
    # (fmt, out, in, rows): benchmark configs 0-1 and the Moonlight decode shapes
    (1, 11264, 2048, 1), (1, 11264, 2048, 4), (2, 11264, 2048, 1), (2, 2048, 11264, 1),
    (1, 2048, 11264, 1), (1, 3072, 2048, 1), (1, 576, 2048, 2), (1, 2048, 1408, 1),
    (1, 2048, 2816, 3), (2, 1408, 2048, 1), (2, 2048, 1408, 1), (1, 128, 512, 1),
    (2, 128, 512, 1), (0, 64, 2048, 1), (0, 4096, 2048, 1), (0, 1000, 2048, 4),
    # tiny-fixture widths (hidden 256, expert 64) and odd shapes (generic path)
    (1, 192, 256, 5), (2, 80, 256, 3), (1, 256, 64, 2), (2, 256, 64, 1),
    (1, 128, 257, 4), (2, 128, 257, 4), (0, 7, 33, 2), (1, 33, 48, 9),
    # split-k kernel (I > 4096, O <= 4096): 2 and 4 token rows, a last k
    # chunk with only 1 or 2 of its 4 wave ranges (5120, 11264), row blocks
    # past O (1000, 2040)
    (1, 2048, 11264, 4), (2, 2048, 11264, 2), (1, 512, 5120, 1), (2, 1000, 6144, 4),
    (1, 2040, 8192, 2),
    # wide kernel (one row, I a multiple of 1024 in (4096, 16384], O 2048 or
    # 4096; config 1's 2048 x 11264 above): 16 and 5 waves, O = 4096; O =
    # 2053 and 3000 take split-k
    (2, 2048, 16384, 1), (1, 2048, 5120, 1), (2, 4096, 11264, 1), (1, 3000, 7168, 1),
    (1, 2053, 5120, 1),
]


@pytest.mark.parametrize("fmt,out_width,in_width,rows", SHAPES)
def test_gemv_matches_oracle(device, fmt, out_width, in_width, rows):
    print(f"[gpu] gemv fmt={fmt} O={out_width} I={in_width} rows={rows}", flush=True)
    q, s = make_weights(fmt, out_width, in_width, seed=out_width * 7 + in_width)
    x = O.fill_normal(rows * in_width, 99 + rows).reshape(rows, in_width)
    expect = O.matmul(fmt, q, s, x, out_width, in_width)
    dw, dx = DeviceBuffer.from_array(q), DeviceBuffer.from_array(x)
    ds = DeviceBuffer.from_array(s) if s is not None else None
    dy = DeviceBuffer(rows * out_width * 4)
    native.gemv(fmt, dw, ds, dx, dy, out_width, in_width, rows)
    got = dy.download(np.float32).reshape(rows, out_width)
    assert np.isfinite(got).all()
    assert rel_l2(got, expect) < TOL


@pytest.mark.parametrize("fmt,out_width,in_width,rows", [
    (1, 3072, 2048, 1), (2, 3648, 2048, 2), (0, 64, 2048, 3), (1, 192, 256, 4),
    (0, 163840 // 16, 2048, 1),
    # narrow rows with a partially filled last wave (lane groups past O)
    (1, 80, 256, 2), (2, 80, 256, 1), (1, 40, 128, 3), (2, 72, 256, 2), (1, 20, 64, 1),
    # wide kernel: the sum of squares adds up over the waves; split-k: over
    # the k chunks
    (1, 2048, 11264, 1), (2, 2048, 5120, 1), (2, 1024, 5120, 4)])
def test_gemv_rmsnorm_prologue(device, fmt, out_width, in_width, rows):
    print(f"[gpu] gemv+norm fmt={fmt} O={out_width} I={in_width} rows={rows}", flush=True)
    q, s = make_weights(fmt, out_width, in_width, seed=5 + out_width)
    x = O.fill_normal(rows * in_width, 3).reshape(rows, in_width) * 3.0
    nw = O.fill_normal(in_width, 4, mean=1.0, std=0.1)
    xn = np.empty_like(x)
    O.lib().orc_rmsnorm(O.fptr(x), O.fptr(nw), O.fptr(xn), rows, in_width, 1e-5)
    expect = O.matmul(fmt, q, s, xn, out_width, in_width)
    dw, dx, dn = (DeviceBuffer.from_array(a) for a in (q, x, nw))
    ds = DeviceBuffer.from_array(s) if s is not None else None
    dy = DeviceBuffer(rows * out_width * 4)
    native.gemv(fmt, dw, ds, dx, dy, out_width, in_width, rows, norm_w=dn, eps=1e-5)
    assert rel_l2(dy.download(np.float32), expect) < TOL


@pytest.mark.parametrize("fmt,out_width,in_width,rows", [
    (1, 2048, 2048, 1), (1, 2048, 11264, 2), (2, 2048, 1408, 1), (1, 256, 64, 3),
    (1, 2048, 11264, 1)])
def test_gemv_residual_epilogue(device, fmt, out_width, in_width, rows):
    q, s = make_weights(fmt, out_width, in_width, seed=17)
    x = O.fill_normal(rows * in_width, 8).reshape(rows, in_width)
    res = O.fill_normal(rows * out_width, 9).reshape(rows, out_width)
    expect = res + O.matmul(fmt, q, s, x, out_width, in_width)
    dw, ds, dx, dr = (DeviceBuffer.from_array(a) for a in (q, s, x, res))
    dy = DeviceBuffer(rows * out_width * 4)
    native.gemv(fmt, dw, ds, dx, dy, out_width, in_width, rows, resid=dr)
    assert rel_l2(dy.download(np.float32), expect) < TOL


@pytest.mark.parametrize("fmt,width,in_width,rows,norm", [
    (1, 11264, 2048, 1, True), (1, 1408, 2048, 2, True), (2, 2816, 2048, 1, False),
    (1, 64, 256, 4, True), (2, 1408, 2048, 5, True), (1, 50, 257, 2, False)])
def test_gemv_swiglu_pair(device, fmt, width, in_width, rows, norm):
    print(f"[gpu] swiglu fmt={fmt} W={width} I={in_width} rows={rows}", flush=True)
    qg, sg = make_weights(fmt, width, in_width, seed=21)
    qu, su = make_weights(fmt, width, in_width, seed=22)
    x = O.fill_normal(rows * in_width, 23).reshape(rows, in_width)
    nw = O.fill_normal(in_width, 24, mean=1.0, std=0.1)
    xn = x
    if norm:
        xn = np.empty_like(x)
        O.lib().orc_rmsnorm(O.fptr(x), O.fptr(nw), O.fptr(xn), rows, in_width, 1e-5)
    g = O.matmul(fmt, qg, sg, xn, width, in_width)
    u = O.matmul(fmt, qu, su, xn, width, in_width)
    expect = g / (1.0 + np.exp(-g.astype(np.float64))) * u
    bufs = [DeviceBuffer.from_array(a) for a in (qg, sg, qu, su, x, nw)]
    dh = DeviceBuffer(rows * width * 4)
    native.gemv_swiglu(fmt, bufs[0], bufs[1], bufs[2], bufs[3], bufs[4], dh, width, in_width,
                       rows, norm_w=bufs[5] if norm else None, eps=1e-5)
    assert rel_l2(dh.download(np.float32), expect) < TOL


@pytest.mark.parametrize("bits,rows,cols", [(8, 11264, 2048), (4, 2048, 11264), (4, 33, 257),
                                            (8, 5, 33), (4, 7, 1)])
def test_device_quantizer_bit_exact(device, bits, rows, cols):
    w = O.fill_normal(rows * cols, 31 + bits, std=0.02, bf16=True).reshape(rows, cols)
    w[0, :] = 0.0
    if cols > 4:
        w[1, :4] = [0.5, -1.5, 2.5, 127.0]
    q_ref, s_ref = O.quant(w, bits)
    dw = DeviceBuffer.from_array(w)
    dq, ds = DeviceBuffer(q_ref.nbytes), DeviceBuffer(s_ref.nbytes)
    native.quantize(bits, dw, rows, cols, dq, ds)
    assert np.array_equal(dq.download(np.uint8), q_ref)
    assert np.array_equal(ds.download(np.float32).view(np.uint32), s_ref.view(np.uint32))


def test_device_fill_normal_distribution(device):
    n = 1 << 20
    d = DeviceBuffer(n * 4)
    native.fill_normal(d, n, 1234, 0.0, 0.02, bf16=True)
    v = d.download(np.float32)
    assert np.all((v.view(np.uint32) & 0xFFFF) == 0)
    assert abs(v.mean()) < 1e-4 and abs(v.std() - 0.02) < 2e-4
    host = O.fill_normal(4096, 1234, std=0.02, bf16=True)
    # same counter stream; device libm may differ in the last double ulp
    assert np.mean(host == v[:4096]) > 0.99


def test_fm_backend_reference_kernel_gate(device):
    """tests/test_backend_metal.c:35-80: O=128, I=257 (odd, q4 tail), S=4,
    max relative error vs f64 <= 1e-3 for cache=0 (twice) and cache=1 (twice)."""
    lib = native.load()
    assert lib.fm_init() == 1
    assert b"gfx950" in lib.fm_device_name()
    rng = np.random.default_rng(42)
    O_, I_, S_ = 128, 257, 4
    w8 = rng.integers(-127, 128, O_ * I_).astype(np.int8)
    s = (rng.uniform(-1, 1, O_) * 0.01 + 0.02).astype(np.float32)
    x = rng.uniform(-1, 1, S_ * I_).astype(np.float32)
    y = np.empty(S_ * O_, np.float32)

    def maxrel(y, dense):
        ref = x.reshape(S_, I_).astype(np.float64) @ dense.T
        return np.max(np.abs(y.reshape(S_, O_) - ref) / (np.abs(ref) + 1e-6))

    dense8 = w8.reshape(O_, I_).astype(np.float64) * s[:, None]
    for _ in range(2):
        lib.fm_matmul_q8(y.ctypes.data, x.ctypes.data, w8.ctypes.data, s.ctypes.data,
                         O_, I_, S_, 0)
        assert maxrel(y, dense8) <= 1e-3
        x[:] = rng.uniform(-1, 1, S_ * I_)
    ib = (I_ + 1) // 2
    w4 = rng.integers(0, 256, O_ * ib).astype(np.uint8)
    vals = np.empty((O_, 2 * ib))
    b = w4.reshape(O_, ib)
    vals[:, 0::2] = (b & 15).astype(np.int64) - 8
    vals[:, 1::2] = (b >> 4).astype(np.int64) - 8
    dense4 = vals[:, :I_] * s[:, None]
    for _ in range(2):
        lib.fm_matmul_q4(y.ctypes.data, x.ctypes.data, w4.ctypes.data, s.ctypes.data,
                         O_, I_, S_, 1)
        assert maxrel(y, dense4) <= 1e-3
        x[:] = rng.uniform(-1, 1, S_ * I_)
    assert lib.fm_matmul_deepseek_v4_fp8(None, None, None, None, 128, 128, 1, 128) == 0


@pytest.mark.parametrize("fmt,rows", [(1, 1), (2, 4)])
def test_splitk_repeat_deterministic(device, fmt, rows):
    """The split-k kernel's arrival counters reset themselves: back-to-back
    launches (with a different shape in between) return the same bits, the
    splits added in a fixed order whatever order the workgroups finish in.
    (At one row 2048 x 11264 takes the wide kernel, whose sums stay inside
    a workgroup, and 1000 x 6144 the split-k kernel.)"""
    q, s = make_weights(fmt, 2048, 11264, seed=123)
    x = O.fill_normal(rows * 11264, 77).reshape(rows, 11264)
    dw, dx, ds = DeviceBuffer.from_array(q), DeviceBuffer.from_array(x), DeviceBuffer.from_array(s)
    q2, s2 = make_weights(fmt, 1000, 6144, seed=9)
    x2 = O.fill_normal(6144, 78).reshape(1, 6144)
    dw2, dx2, ds2 = (DeviceBuffer.from_array(a) for a in (q2, x2, s2))
    dy, dy2 = DeviceBuffer(rows * 2048 * 4), DeviceBuffer(1000 * 4)
    first = None
    for _ in range(4):
        native.gemv(fmt, dw, ds, dx, dy, 2048, 11264, rows)
        got = dy.download(np.float32)
        if first is None:
            first = got
            assert rel_l2(got, O.matmul(fmt, q, s, x, 2048, 11264).ravel()) < TOL
        assert np.array_equal(got.view(np.uint32), first.view(np.uint32))
        native.gemv(fmt, dw2, ds2, dx2, dy2, 1000, 6144, 1)
        assert rel_l2(dy2.download(np.float32), O.matmul(fmt, q2, s2, x2, 1000, 6144).ravel()) < TOL


@pytest.mark.parametrize("fmt,out_width,in_width,rows,norm", [
    (1, 2048, 2048, 1, False),   # LDS-DMA kernel (q8, one row): o_proj
    (2, 11264, 2048, 1, False),  # register-direct kernel (q4)
    (1, 3072, 2048, 2, False),   # register-direct kernel (q8, two rows)
    (1, 2048, 11264, 1, False),  # wide kernel
    (1, 1000, 6144, 1, False),   # split-k kernel
    (2, 2048, 11264, 4, False),
    (1, 3072, 2048, 2, True),    # RMSNorm: the normalised row is NaN
])
def test_gemv_nonfinite_inputs(device, fmt, out_width, in_width, rows, norm):
    """A NaN or an infinity in x makes the token row's outputs NaN wherever
    the reference's fp32 dot (x . q, then the scale) is NaN, and NaN or the
    reference's infinity where that is infinite: never a finite value (the
    limb split cannot carry them).  Rows without one are unaffected.  Row 0:
    one +inf; row 1: a +inf and a -inf; row 2: a NaN; row 3: finite."""
    print(f"[gpu] gemv non-finite x fmt={fmt} O={out_width} I={in_width} rows={rows}", flush=True)
    q, s = make_weights(fmt, out_width, in_width, seed=4242)
    x = O.fill_normal(rows * in_width, 17).reshape(rows, in_width)
    x[0, 7] = np.inf
    if rows > 1:
        x[1, 100], x[1, in_width - 3] = np.inf, -np.inf
    if rows > 2:
        x[2, 555] = np.nan
    dw, dx = DeviceBuffer.from_array(q), DeviceBuffer.from_array(x)
    ds = DeviceBuffer.from_array(s)
    dy = DeviceBuffer(rows * out_width * 4)
    if norm:
        nw = O.fill_normal(in_width, 4, mean=1.0, std=0.1)
        dn = DeviceBuffer.from_array(nw)
        native.gemv(fmt, dw, ds, dx, dy, out_width, in_width, rows, norm_w=dn, eps=1e-5)
        xn = np.empty_like(x)
        O.lib().orc_rmsnorm(O.fptr(x), O.fptr(nw), O.fptr(xn), rows, in_width, 1e-5)
        expect = O.matmul(fmt, q, s, xn, out_width, in_width)
    else:
        native.gemv(fmt, dw, ds, dx, dy, out_width, in_width, rows)
        with np.errstate(invalid="ignore", over="ignore"):
            expect = O.matmul(fmt, q, s, x, out_width, in_width)
    got = dy.download(np.float32).reshape(rows, out_width)
    assert np.array_equal(np.isfinite(got), np.isfinite(expect))
    assert np.isnan(got[np.isnan(expect)]).all()
    inf = np.isinf(expect)
    assert (np.isnan(got[inf]) | (got[inf] == expect[inf])).all()
    assert not np.isfinite(expect[0]).all()  # the case is exercised
    fin = np.isfinite(expect)
    if rows > 3:
        assert fin[3].all() and rel_l2(got[3], expect[3]) < TOL
    assert rel_l2(got[fin], expect[fin]) < TOL
