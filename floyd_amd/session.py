"""ctypes binding of the Moonlight session C API (include/moonlight_hip.h,
include/moonlight_hip_ext.h) exported by libfloyd_amd.so.

Mirrors floyd's moonlight_metal.h interface: the same functions, argument
meaning and 1/0 return convention; failures raise SessionError carrying the
library's message.
"""
import ctypes as C

import numpy as np

from . import native


class Options(C.Structure):
    _fields_ = [("context_size", C.c_int), ("max_batch", C.c_int)]


class ModelInfo(C.Structure):
    _fields_ = [(n, C.c_int) for n in (
        "hidden_size", "layer_count", "vocab_size", "head_count", "kv_lora_rank",
        "qk_nope_dim", "qk_rope_dim", "value_dim", "expert_count", "experts_per_token",
        "moe_intermediate_size", "shared_expert_count", "first_dense_layer_count")] + [
        (n, C.c_float) for n in ("rms_norm_epsilon", "rope_theta", "routed_scale")] + [
        ("resident_bytes", C.c_uint64)]


class Stats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "command_buffers", "prefill_tokens", "decode_tokens", "cpu_fallbacks",
        "buffer_allocations", "resident_bytes")] + [("prefill_ms", C.c_double),
                                                    ("decode_ms", C.c_double)]


class SyntheticConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in (
        "hidden_size", "layer_count", "head_count", "expert_count", "experts_per_token",
        "dense_intermediate_size", "moe_intermediate_size", "first_dense_layer_count",
        "kv_lora_rank", "qk_nope_dim", "qk_rope_dim", "value_dim", "shared_expert_count",
        "normalize_topk", "vocab_size")] + [
        (n, C.c_float) for n in ("rms_norm_epsilon", "rope_theta", "routed_scale")] + [
        ("expert_bits", C.c_int), ("dense_bits", C.c_int), ("weight_std", C.c_float),
        ("seed", C.c_uint64)]


CONFIG_INT_FIELDS = (
    "hidden_size", "layer_count", "head_count", "expert_count", "experts_per_token",
    "dense_intermediate_size", "moe_intermediate_size", "first_dense_layer_count",
    "q_lora_rank", "kv_lora_rank", "qk_nope_dim", "qk_rope_dim", "value_dim",
    "shared_expert_count", "normalize_topk", "vocab_size")
CONFIG_FLOAT_FIELDS = ("rms_norm_epsilon", "rope_theta", "routed_scale")

_vp, _cp, _sz = C.c_void_p, C.c_char_p, C.c_size_t
_pp = C.POINTER(C.c_void_p)

SIGNATURES = {
    "moonlight_model_open": (C.c_int, [_pp, _cp, _cp, _sz]),
    "moonlight_model_close": (None, [_vp]),
    "moonlight_device_name": (_cp, [_vp]),
    "moonlight_model_info": (ModelInfo, [_vp]),
    "moonlight_session_create": (C.c_int, [_pp, _vp, C.POINTER(Options), _cp, _sz]),
    "moonlight_session_destroy": (None, [_vp]),
    "moonlight_session_reset": (None, [_vp]),
    "moonlight_session_position": (C.c_int, [_vp]),
    "moonlight_session_stats": (Stats, [_vp]),
    "moonlight_session_prefill": (C.c_int, [_vp, _vp, C.c_int, _vp, _cp, _sz]),
    "moonlight_session_append": (C.c_int, [_vp, _vp, C.c_int, _vp, _cp, _sz]),
    "moonlight_session_decode": (C.c_int, [_vp, C.c_int, _vp, _cp, _sz]),
    "moonlight_test_prefill_layers": (C.c_int, [_vp, _vp, C.c_int, _vp, _vp, _cp, _sz]),
    "moonlight_test_embed": (C.c_int, [_vp, _vp, C.c_int, _vp]),
    "moonlight_test_rmsnorm": (C.c_int, [_vp, _vp, _cp, C.c_int, C.c_int, _vp]),
    "moonlight_test_matmul": (C.c_int, [_vp, _cp, _vp, C.c_int, C.c_int, C.c_int, _vp]),
    "moonlight_test_attention": (C.c_int, [_vp, C.c_int, _vp, C.c_int, C.c_int, _vp]),
    "moonlight_test_kv_length": (C.c_int, [_vp, C.c_int]),
    "moonlight_test_copy_kv": (C.c_int, [_vp, C.c_int, _vp, _vp, C.c_int]),
    "moonlight_test_moe": (C.c_int, [_vp, C.c_int, _vp, C.c_int, _vp, _vp, _vp, _vp, _vp,
                                     _vp]),
    "moonlight_test_dense_mlp": (C.c_int, [_vp, C.c_int, _vp, C.c_int, _vp]),
    "moonlight_test_copy_routes": (C.c_int, [_vp, C.c_int, _vp, C.c_int]),
    "moonlight_container_probe": (C.c_int, [_cp, _vp, _vp, _cp, _sz]),
    "moonlight_container_tensor": (C.c_int, [_cp, _cp, _vp, _vp, _vp]),
    "moonlight_synthetic_moonlight_config": (SyntheticConfig, []),
    "moonlight_model_create_synthetic": (C.c_int, [_pp, C.POINTER(SyntheticConfig), _cp, _sz]),
    "moonlight_model_read_tensor": (_sz, [_vp, _cp, _vp, _sz]),
    "moonlight_model_tensor_info": (C.c_int, [_vp, _cp, _vp, _vp, _vp]),
    "moonlight_session_fill_kv": (C.c_int, [_vp, C.c_int, C.c_int, C.c_uint64]),
    "moonlight_session_device_time": (C.c_int, [_vp, C.POINTER(C.c_double)]),
    "moonlight_session_decode_graph": (C.c_int, [_vp, C.c_int]),
    "moonlight_session_sample": (C.c_int, [_vp, C.c_float, C.c_float,
                                           C.POINTER(C.c_uint64), C.POINTER(C.c_int), _cp, _sz]),
    "moonlight_session_decode_sample": (C.c_int, [_vp, C.c_int, C.c_float, C.c_float,
                                                  C.POINTER(C.c_uint64), C.POINTER(C.c_int),
                                                  _cp, _sz]),
    "moonlight_session_fix_routes": (C.c_int, [_vp, _vp, C.c_int]),
    "moonlight_session_copy_route_tables": (C.c_int, [_vp, C.c_int, _vp, _vp, _vp, _vp, _vp,
                                                      _vp, _vp]),
    "moonlight_session_trace_router": (C.c_int, [_vp, C.c_int]),
    "moonlight_session_copy_router_trace": (C.c_int, [_vp, C.c_int, _vp, C.c_int]),
    "moonlight_session_time_moe": (C.c_int, [_vp, C.c_int, C.c_int, C.c_uint64, C.c_int,
                                             C.c_int, C.POINTER(C.c_double),
                                             C.POINTER(C.c_int)]),
    "moonlight_session_time_attention": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.c_uint64,
                                                   C.c_int, C.c_int, C.POINTER(C.c_double)]),
}

_bound = False


def lib():
    global _bound
    L = native.load()
    if not _bound:
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _bound = True
    return L


class SessionError(RuntimeError):
    pass


def _arr(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a, a.ctypes.data


def probe_container(path):
    """Config (dict) and tensor count of a container directory, without a GPU."""
    ints = np.zeros(16, np.int32)
    floats = np.zeros(3, np.float32)
    err = C.create_string_buffer(512)
    n = lib().moonlight_container_probe(path.encode(), ints.ctypes.data, floats.ctypes.data,
                                        err, 512)
    if n < 0:
        raise SessionError(err.value.decode())
    cfg = dict(zip(CONFIG_INT_FIELDS, ints.tolist()))
    cfg.update(zip(CONFIG_FLOAT_FIELDS, floats.tolist()))
    return cfg, n


def container_tensor(path, name):
    dtype, numel, nbytes = C.c_int(), C.c_int64(), C.c_int64()
    ok = lib().moonlight_container_tensor(path.encode(), name.encode(), C.byref(dtype),
                                          C.byref(numel), C.byref(nbytes))
    return (dtype.value, numel.value, nbytes.value) if ok else None


class Model:
    def __init__(self, handle):
        self.handle = handle

    @classmethod
    def open(cls, path):
        h = C.c_void_p()
        err = C.create_string_buffer(1024)
        if not lib().moonlight_model_open(C.byref(h), path.encode(), err, 1024):
            raise SessionError(err.value.decode())
        return cls(h.value)

    @classmethod
    def synthetic(cls, **overrides):
        cfg = lib().moonlight_synthetic_moonlight_config()
        for k, v in overrides.items():
            setattr(cfg, k, v)
        h = C.c_void_p()
        err = C.create_string_buffer(1024)
        if not lib().moonlight_model_create_synthetic(C.byref(h), C.byref(cfg), err, 1024):
            raise SessionError(err.value.decode())
        return cls(h.value)

    def info(self):
        i = lib().moonlight_model_info(self.handle)
        return {f: getattr(i, f) for f, _ in ModelInfo._fields_}

    def device_name(self):
        return lib().moonlight_device_name(self.handle).decode()

    def tensor_info(self, name):
        dtype, numel, nbytes = C.c_int(), C.c_int64(), C.c_int64()
        if not lib().moonlight_model_tensor_info(self.handle, name.encode(), C.byref(dtype),
                                                 C.byref(numel), C.byref(nbytes)):
            return None
        return dtype.value, numel.value, nbytes.value

    def read_tensor(self, name, dtype):
        info = self.tensor_info(name)
        if info is None:
            raise KeyError(name)
        out = np.empty(info[2], np.uint8)
        n = lib().moonlight_model_read_tensor(self.handle, name.encode(), out.ctypes.data,
                                              out.nbytes)
        if n != info[2]:
            raise SessionError(f"read of {name} failed")
        return out.view(dtype)

    def close(self):
        if self.handle:
            lib().moonlight_model_close(self.handle)
            self.handle = None


class Session:
    def __init__(self, model, context_size, max_batch):
        self.model = model
        h = C.c_void_p()
        err = C.create_string_buffer(1024)
        opts = Options(context_size, max_batch)
        if not lib().moonlight_session_create(C.byref(h), model.handle, C.byref(opts), err,
                                              1024):
            raise SessionError(err.value.decode())
        self.handle = h.value
        self.info = model.info()

    def close(self):
        if self.handle:
            lib().moonlight_session_destroy(self.handle)
            self.handle = None

    def _call(self, fn, *args):
        err = C.create_string_buffer(1024)
        if not fn(self.handle, *args, err, 1024):
            raise SessionError(err.value.decode())

    def prefill(self, ids):
        ids, p = _arr(ids, np.int32)
        out = np.empty(self.info["vocab_size"], np.float32)
        self._call(lib().moonlight_session_prefill, p, ids.size, out.ctypes.data)
        return out

    def append(self, ids):
        ids, p = _arr(ids, np.int32)
        out = np.empty(self.info["vocab_size"], np.float32)
        self._call(lib().moonlight_session_append, p, ids.size, out.ctypes.data)
        return out

    def decode(self, token, out=None):
        """Logits of one decode step; `out` (float32 [vocab], C-contiguous) is
        reused when given, as a serving loop would."""
        if out is None:
            out = np.empty(self.info["vocab_size"], np.float32)
        elif (out.dtype != np.float32 or out.shape != (self.info["vocab_size"],) or
              not out.flags["C_CONTIGUOUS"]):
            raise ValueError("out must be a C-contiguous float32 array of vocab_size")
        self._call(lib().moonlight_session_decode, int(token), out.ctypes.data)
        return out

    def sample(self, temperature=0.0, top_p=1.0, rng=None):
        """Next token from the last forward's logits, chosen on the device
        (choose_token, moonlight_chat.c:96-131).  `rng` is the caller's
        xorshift64 state as an int; returns (token, advanced state)."""
        state = C.c_uint64(rng or 0)
        tok = C.c_int(-1)
        self._call(lib().moonlight_session_sample, float(temperature), float(top_p),
                   C.byref(state), C.byref(tok))
        return tok.value, state.value

    def decode_sample(self, token, temperature=0.0, top_p=1.0, rng=None):
        """One decode step ending in a device-side token choice: only the
        token id comes back.  Returns (next token, advanced rng state)."""
        state = C.c_uint64(rng or 0)
        tok = C.c_int(-1)
        self._call(lib().moonlight_session_decode_sample, int(token), float(temperature),
                   float(top_p), C.byref(state), C.byref(tok))
        return tok.value, state.value

    def prefill_layers(self, ids):
        ids, p = _arr(ids, np.int32)
        layers = np.empty((self.info["layer_count"], ids.size, self.info["hidden_size"]),
                          np.float32)
        out = np.empty(self.info["vocab_size"], np.float32)
        self._call(lib().moonlight_test_prefill_layers, p, ids.size, layers.ctypes.data,
                   out.ctypes.data)
        return layers, out

    def reset(self):
        lib().moonlight_session_reset(self.handle)

    def position(self):
        return lib().moonlight_session_position(self.handle)

    def stats(self):
        s = lib().moonlight_session_stats(self.handle)
        return {f: getattr(s, f) for f, _ in Stats._fields_}

    def device_time_ms(self):
        v = C.c_double()
        lib().moonlight_session_device_time(self.handle, C.byref(v))
        return v.value

    def decode_graph(self, enable=None):
        """Switches the decode-step graph on / off (None: query); returns
        whether decode steps replay a captured graph."""
        return bool(lib().moonlight_session_decode_graph(
            self.handle, -1 if enable is None else int(bool(enable))))

    def fill_kv(self, length, seed, layer=-1):
        if not lib().moonlight_session_fill_kv(self.handle, layer, length, seed):
            raise SessionError("fill_kv failed")

    def fix_routes(self, ids):
        """Expert ids [rows, top_k] used by test_moe / time_moe (None: top-k)."""
        if ids is None:
            ok = lib().moonlight_session_fix_routes(self.handle, None, 0)
        else:
            ids, p = _arr(ids, np.int32)
            ok = lib().moonlight_session_fix_routes(self.handle, p, ids.shape[0])
        if not ok:
            raise SessionError("fix_routes failed")

    def route_tables(self, rows):
        """Device route tables of the last routing of `rows` token rows:
        dict(n_unique, unique, counts, offsets, list_rows, list_slots, list_pos)."""
        e, k = self.info["expert_count"], self.info["experts_per_token"]
        n = np.zeros(1, np.int32)
        t = {name: np.full(e, -7, np.int32) for name in ("unique", "counts", "offsets")}
        t.update({name: np.full(rows * k, -7, np.int32)
                  for name in ("list_rows", "list_slots", "list_pos")})
        ok = lib().moonlight_session_copy_route_tables(
            self.handle, rows, n.ctypes.data, t["unique"].ctypes.data, t["counts"].ctypes.data,
            t["offsets"].ctypes.data, t["list_rows"].ctypes.data, t["list_slots"].ctypes.data,
            t["list_pos"].ctypes.data)
        if not ok:
            raise SessionError("copy_route_tables failed")
        t["n_unique"] = int(n[0])
        return t

    def trace_router(self, enable=True):
        if not lib().moonlight_session_trace_router(self.handle, int(bool(enable))):
            raise SessionError("trace_router failed")

    def router_trace(self, layer, rows):
        out = np.empty((rows, self.info["expert_count"]), np.float32)
        ok = lib().moonlight_session_copy_router_trace(self.handle, layer, out.ctypes.data, rows)
        return out if ok else None

    def time_moe(self, layer, rows, seed=7, warmup=5, iters=50):
        """(us per pass, mean distinct experts per timed pass); layer -1
        cycles through every MoE layer with a fresh input per pass."""
        us, uniq = C.c_double(), C.c_int()
        if not lib().moonlight_session_time_moe(self.handle, layer, rows, seed, warmup, iters,
                                                C.byref(us), C.byref(uniq)):
            raise SessionError("time_moe failed")
        return us.value, uniq.value / iters

    def time_attention(self, layer, rows, position, seed=7, warmup=5, iters=50):
        """us per pass; layer -1 cycles through every layer (each layer's
        cache filled up to `position`) with a fresh input per pass."""
        us = C.c_double()
        if not lib().moonlight_session_time_attention(self.handle, layer, rows, position, seed,
                                                      warmup, iters, C.byref(us)):
            raise SessionError("time_attention failed")
        return us.value

    # ---- test hooks (0 = failure, no message) ----
    def test_embed(self, ids):
        ids, p = _arr(ids, np.int32)
        out = np.empty((ids.size, self.info["hidden_size"]), np.float32)
        ok = lib().moonlight_test_embed(self.handle, p, ids.size, out.ctypes.data)
        return out if ok else None

    def test_rmsnorm(self, x, weight_name):
        x, p = _arr(x, np.float32)
        out = np.empty_like(x)
        ok = lib().moonlight_test_rmsnorm(self.handle, p, weight_name.encode(), x.shape[0],
                                          x.shape[1], out.ctypes.data)
        return out if ok else None

    def test_matmul(self, name, x, out_width):
        x, p = _arr(x, np.float32)
        out = np.empty((x.shape[0], out_width), np.float32)
        ok = lib().moonlight_test_matmul(self.handle, name.encode(), p, x.shape[0], x.shape[1],
                                         out_width, out.ctypes.data)
        return out if ok else None

    def test_attention(self, layer, x, position):
        x, p = _arr(x, np.float32)
        out = np.empty_like(x)
        ok = lib().moonlight_test_attention(self.handle, layer, p, x.shape[0], position,
                                            out.ctypes.data)
        return out if ok else None

    def test_kv_length(self, layer):
        return lib().moonlight_test_kv_length(self.handle, layer)

    def test_copy_kv(self, layer, capacity):
        lat = np.empty((capacity, self.info["kv_lora_rank"]), np.float32)
        rope = np.empty((capacity, self.info["qk_rope_dim"]), np.float32)
        ok = lib().moonlight_test_copy_kv(self.handle, layer, lat.ctypes.data, rope.ctypes.data,
                                          capacity)
        return (lat, rope) if ok else None

    def test_moe(self, layer, x):
        x, p = _arr(x, np.float32)
        rows, k, e = x.shape[0], self.info["experts_per_token"], self.info["expert_count"]
        ids = np.empty((rows, k), np.int32)
        w = np.empty((rows, k), np.float32)
        scores = np.empty((rows, e), np.float32)
        routed = np.empty_like(x)
        shared = np.empty_like(x)
        out = np.empty_like(x)
        ok = lib().moonlight_test_moe(self.handle, layer, p, rows, ids.ctypes.data,
                                      w.ctypes.data, scores.ctypes.data, routed.ctypes.data,
                                      shared.ctypes.data, out.ctypes.data)
        if not ok:
            return None
        return dict(ids=ids, weights=w, logits=scores, routed=routed, shared=shared, out=out)

    def test_dense_mlp(self, layer, x):
        x, p = _arr(x, np.float32)
        out = np.empty_like(x)
        ok = lib().moonlight_test_dense_mlp(self.handle, layer, p, x.shape[0], out.ctypes.data)
        return out if ok else None

    def test_copy_routes(self, layer, rows):
        out = np.empty((rows, self.info["experts_per_token"]), np.int32)
        ok = lib().moonlight_test_copy_routes(self.handle, layer, out.ctypes.data, rows)
        return out if ok else None
