"""ctypes binding of libfloyd_amd.so (the HIP product library).

Raises NativeError when the library is not built: there is no host-side or
PyTorch fallback for any entry point.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(HERE, "lib", "libfloyd_amd.so")

MLK_F32, MLK_Q8, MLK_Q4 = 0, 1, 2

_c = ctypes
_vp = _c.c_void_p
_fp = _c.POINTER(_c.c_float)


class NativeError(RuntimeError):
    pass


# (name, restype, argtypes) of every exported C entry point.
SIGNATURES = {
    # include/moonlight_kernels.h
    "mlk_init": (_c.c_int, []),
    "mlk_device_name": (_c.c_char_p, []),
    "mlk_last_error": (_c.c_char_p, []),
    "mlk_malloc": (_vp, [_c.c_size_t]),
    "mlk_free": (_c.c_int, [_vp]),
    "mlk_memcpy_h2d": (_c.c_int, [_vp, _vp, _c.c_size_t]),
    "mlk_memcpy_d2h": (_c.c_int, [_vp, _vp, _c.c_size_t]),
    "mlk_memcpy_d2d": (_c.c_int, [_vp, _vp, _c.c_size_t]),
    "mlk_memset": (_c.c_int, [_vp, _c.c_int, _c.c_size_t]),
    "mlk_synchronize": (_c.c_int, []),
    "mlk_gemv": (_c.c_int, [_c.c_int, _vp, _vp, _vp, _vp, _c.c_int, _c.c_int, _c.c_int,
                            _vp, _c.c_float, _vp]),
    "mlk_gemv_swiglu": (_c.c_int, [_c.c_int, _vp, _vp, _vp, _vp, _vp, _vp, _c.c_int,
                                   _c.c_int, _c.c_int, _vp, _c.c_float]),
    "mlk_gemv_kernel_name": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int, _c.c_int,
                                        _c.c_char_p, _c.c_size_t]),
    "mlk_time_gemv": (_c.c_int, [_c.c_int, _c.POINTER(_vp), _c.POINTER(_vp), _c.c_int, _vp,
                                 _vp, _c.c_int, _c.c_int, _c.c_int, _c.c_int, _c.c_int,
                                 _c.c_int, _c.POINTER(_c.c_double)]),
    "mlk_time_copy": (_c.c_int, [_c.POINTER(_vp), _c.POINTER(_vp), _c.c_int, _c.c_size_t,
                                 _c.c_int, _c.c_int, _c.POINTER(_c.c_double)]),
    "mlk_time_read": (_c.c_int, [_c.POINTER(_vp), _c.c_int, _c.c_size_t, _c.c_int, _vp,
                                 _c.c_int, _c.c_int, _c.POINTER(_c.c_double)]),
    "mlk_route_topk": (_c.c_int, [_vp, _vp, _c.c_int, _c.c_int, _c.c_int, _c.c_int,
                                  _c.c_float, _vp, _vp]),
    "mlk_sample": (_c.c_int, [_vp, _c.c_int, _c.c_float, _c.c_float, _c.c_double,
                              _c.POINTER(_c.c_int)]),
    "mlk_quantize": (_c.c_int, [_c.c_int, _vp, _c.c_int, _c.c_int, _vp, _vp]),
    "mlk_fill_normal": (_c.c_int, [_vp, _c.c_int64, _c.c_uint64, _c.c_float, _c.c_float,
                                   _c.c_int]),
    # include/fm_backend.h
    "fm_init": (_c.c_int, []),
    "fm_device_name": (_c.c_char_p, []),
    "fm_matmul_q8": (None, [_vp, _vp, _vp, _vp, _c.c_int, _c.c_int, _c.c_int, _c.c_int]),
    "fm_matmul_q4": (None, [_vp, _vp, _vp, _vp, _c.c_int, _c.c_int, _c.c_int, _c.c_int]),
    "fm_matmul_deepseek_v4_fp8": (_c.c_int, [_vp, _vp, _vp, _vp, _c.c_int, _c.c_int,
                                             _c.c_int, _c.c_int]),
    "fm_matmul_deepseek_v4_fp4": (_c.c_int, [_vp, _vp, _vp, _vp, _c.c_int, _c.c_int,
                                             _c.c_int]),
    "fm_matmul_static": (_c.c_int, [_c.c_int, _vp, _vp, _vp, _vp, _c.c_int, _c.c_int,
                                    _c.c_int]),
}

_lib = None


def load():
    """Loads libfloyd_amd.so once; raises NativeError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIBRARY_PATH):
        raise NativeError(
            f"{LIBRARY_PATH} is missing: build it with `python -m floyd_amd.build` "
            "(there is no CPU fallback)")
    lib = _c.CDLL(LIBRARY_PATH)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


def last_error():
    msg = load().mlk_last_error()
    return msg.decode() if msg else ""


def check(status, what):
    if status != 0:
        raise NativeError(f"{what} failed ({status}): {last_error()}")


def init():
    check(load().mlk_init(), "mlk_init")
    return load().mlk_device_name().decode()


def synchronize():
    check(load().mlk_synchronize(), "mlk_synchronize")


class DeviceBuffer:
    """Device allocation from mlk_malloc, freed on close / garbage collection."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        ptr = load().mlk_malloc(max(self.nbytes, 1))
        if not ptr:
            raise NativeError(f"mlk_malloc({self.nbytes}) failed: {last_error()}")
        self.ptr = ptr

    @classmethod
    def from_array(cls, array):
        array = np.ascontiguousarray(array)
        buf = cls(array.nbytes)
        buf.upload(array)
        return buf

    def upload(self, array, offset=0):
        array = np.ascontiguousarray(array)
        assert offset + array.nbytes <= self.nbytes
        check(load().mlk_memcpy_h2d(self.ptr + offset, array.ctypes.data, array.nbytes),
              "mlk_memcpy_h2d")

    def download(self, dtype, count=None, offset=0):
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype)
        assert offset + out.nbytes <= self.nbytes
        check(load().mlk_memcpy_d2h(out.ctypes.data, self.ptr + offset, out.nbytes),
              "mlk_memcpy_d2h")
        return out

    def zero(self):
        check(load().mlk_memset(self.ptr, 0, self.nbytes), "mlk_memset")

    def close(self):
        if getattr(self, "ptr", None):
            load().mlk_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _ptr(buf):
    if buf is None:
        return None
    if isinstance(buf, DeviceBuffer):
        return buf.ptr
    return int(buf)


def gemv(fmt, w, s, x, y, out_width, in_width, rows, norm_w=None, eps=1e-5, resid=None):
    check(load().mlk_gemv(fmt, _ptr(w), _ptr(s), _ptr(x), _ptr(y), out_width, in_width,
                          rows, _ptr(norm_w), eps, _ptr(resid)), "mlk_gemv")


def gemv_swiglu(fmt, wg, sg, wu, su, x, h, out_width, in_width, rows, norm_w=None,
                eps=1e-5):
    check(load().mlk_gemv_swiglu(fmt, _ptr(wg), _ptr(sg), _ptr(wu), _ptr(su), _ptr(x),
                                 _ptr(h), out_width, in_width, rows, _ptr(norm_w), eps),
          "mlk_gemv_swiglu")


def gemv_kernel_name(fmt, out_width, in_width, rows, swiglu=False):
    buf = _c.create_string_buffer(128)
    check(load().mlk_gemv_kernel_name(fmt, out_width, in_width, rows, int(swiglu), buf, 128),
          "mlk_gemv_kernel_name")
    return buf.value.decode()


def time_gemv(fmt, w_list, s_list, x, y, out_width, in_width, rows, warmup, iters,
              use_graph=True):
    n = len(w_list)
    wa = (_vp * n)(*[_ptr(w) for w in w_list])
    sa = (_vp * n)(*[_ptr(s) for s in s_list]) if s_list else None
    out = _c.c_double()
    check(load().mlk_time_gemv(fmt, wa, sa, n, _ptr(x), _ptr(y), out_width, in_width, rows,
                               warmup, iters, int(use_graph), _c.byref(out)), "mlk_time_gemv")
    return out.value


def time_copy(src_list, dst_list, nbytes, warmup, iters):
    n = len(src_list)
    sa = (_vp * n)(*[_ptr(b) for b in src_list])
    da = (_vp * n)(*[_ptr(b) for b in dst_list])
    out = _c.c_double()
    check(load().mlk_time_copy(sa, da, n, nbytes, warmup, iters, _c.byref(out)),
          "mlk_time_copy")
    return out.value


def time_read(src_list, nbytes, blocks, scratch, warmup, iters):
    n = len(src_list)
    sa = (_vp * n)(*[_ptr(b) for b in src_list])
    out = _c.c_double()
    check(load().mlk_time_read(sa, n, nbytes, blocks, _ptr(scratch), warmup, iters,
                               _c.byref(out)), "mlk_time_read")
    return out.value


def route_topk(logits, bias, rows, experts, top_k, normalize, routed_scale, ids, weights):
    check(load().mlk_route_topk(_ptr(logits), _ptr(bias), rows, experts, top_k, normalize,
                                routed_scale, _ptr(ids), _ptr(weights)), "mlk_route_topk")


def sample(logits, vocab, temperature, top_p, u):
    """The device sampler's token for `vocab` device logits (mlk_sample)."""
    tok = _c.c_int(-1)
    check(load().mlk_sample(_ptr(logits), vocab, temperature, top_p, u, _c.byref(tok)),
          "mlk_sample")
    return tok.value


def quantize(bits, w, rows, cols, q, s):
    check(load().mlk_quantize(bits, _ptr(w), rows, cols, _ptr(q), _ptr(s)), "mlk_quantize")


def fill_normal(out, n, seed, mean=0.0, std=1.0, bf16=False):
    check(load().mlk_fill_normal(_ptr(out), n, seed, mean, std, int(bf16)),
          "mlk_fill_normal")
