"""ctypes binding of the CPU oracle (oracle/moonlight_oracle.c).

Test infrastructure: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg load this.  The product library never does.
"""
import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "_build", "libmoonlight_oracle.so")
REF_DIR = os.path.join(ORACLE_DIR, "_ref")

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int)
_u8p = ctypes.POINTER(ctypes.c_uint8)


def fptr(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_f32p)


def iptr(a):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(_i32p)


def u8ptr(a):
    assert a.dtype == np.uint8 and a.flags.c_contiguous
    return a.ctypes.data_as(_u8p)


def vptr(a):
    assert a.flags.c_contiguous
    return ctypes.c_void_p(a.ctypes.data)


class OrcConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "hidden_size", "layer_count", "head_count", "expert_count",
        "experts_per_token", "dense_intermediate_size", "moe_intermediate_size",
        "first_dense_layer_count", "q_lora_rank", "kv_lora_rank", "qk_nope_dim",
        "qk_rope_dim", "value_dim", "shared_expert_count", "normalize_topk",
        "vocab_size")] + [(n, ctypes.c_float) for n in (
            "rms_norm_epsilon", "rope_theta", "routed_scale")]


_lib = None


def build():
    subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            build()
        L = ctypes.CDLL(ORACLE_SO)
        L.orc_splitmix64_at.restype = ctypes.c_uint64
        L.orc_splitmix64_at.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        L.orc_fill_normal.argtypes = [_f32p, ctypes.c_int64, ctypes.c_uint64,
                                      ctypes.c_double, ctypes.c_double, ctypes.c_int]
        L.orc_bf16_round.restype = ctypes.c_float
        L.orc_bf16_round.argtypes = [ctypes.c_float]
        L.orc_quant_int8.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, _u8p, _f32p]
        L.orc_quant_int4.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, _u8p, _f32p]
        L.orc_matmul.argtypes = [ctypes.c_int, ctypes.c_void_p, _f32p, _f32p, _f32p,
                                 ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.orc_set_threads.argtypes = [ctypes.c_int]
        L.orc_random_unit.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        L.orc_random_unit.restype = ctypes.c_double
        L.orc_choose_token.argtypes = [_f32p, ctypes.c_int, ctypes.c_float, ctypes.c_float,
                                       ctypes.POINTER(ctypes.c_uint64)]
        L.orc_detect_format.argtypes = [ctypes.c_int64, ctypes.c_int, ctypes.c_int]
        L.orc_rmsnorm.argtypes = [_f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_float]
        L.orc_rope.argtypes = [_f32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_float]
        L.orc_rope_inv_freq.restype = ctypes.c_float
        L.orc_rope_inv_freq.argtypes = [ctypes.c_float, ctypes.c_int, ctypes.c_int]
        L.orc_silu_mul.restype = ctypes.c_float
        L.orc_silu_mul.argtypes = [ctypes.c_float, ctypes.c_float]
        L.orc_route_sigmoid_topk.argtypes = [_f32p, _f32p, ctypes.c_int, ctypes.c_int,
                                             ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                             _i32p, _f32p]
        L.orc_route_tables.argtypes = [_i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int, _i32p, _i32p, _i32p, _i32p]
        L.orc_model_create.restype = ctypes.c_void_p
        L.orc_model_create.argtypes = [ctypes.POINTER(OrcConfig), ctypes.c_int]
        L.orc_model_destroy.argtypes = [ctypes.c_void_p]
        L.orc_model_add_tensor.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int,
                                           ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64]
        L.orc_model_reset.argtypes = [ctypes.c_void_p]
        L.orc_model_kv_length.argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.orc_model_set_kv.argtypes = [ctypes.c_void_p, ctypes.c_int, _f32p, _f32p,
                                       ctypes.c_int]
        L.orc_model_copy_kv.argtypes = [ctypes.c_void_p, ctypes.c_int, _f32p, _f32p,
                                        ctypes.c_int]
        L.orc_named_matmul.argtypes = [ctypes.c_void_p, ctypes.c_char_p, _f32p,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p]
        L.orc_attention.argtypes = [ctypes.c_void_p, ctypes.c_int, _f32p, ctypes.c_int,
                                    ctypes.c_int, _f32p]
        L.orc_moe_layer.argtypes = [ctypes.c_void_p, ctypes.c_int, _f32p, ctypes.c_int,
                                    _i32p, _f32p, _f32p, _f32p, _f32p, _f32p]
        L.orc_route_fixed.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_float, _i32p, _f32p]
        L.orc_moe_layer_fixed.argtypes = [ctypes.c_void_p, ctypes.c_int, _f32p, ctypes.c_int,
                                          _i32p, _f32p, _f32p]
        L.orc_forward_routes.argtypes = [ctypes.c_void_p, _i32p, ctypes.c_int, ctypes.c_int,
                                         _i32p, _f32p, _f32p]
        L.orc_dense_mlp.argtypes = [ctypes.c_void_p, ctypes.c_int, _f32p, ctypes.c_int,
                                    _f32p]
        L.orc_forward.argtypes = [ctypes.c_void_p, _i32p, ctypes.c_int, ctypes.c_int,
                                  _f32p, _i32p, _f32p]
        _lib = L
    return _lib


# ---- convenience wrappers ---------------------------------------------------

def fill_normal(n, seed, std=1.0, mean=0.0, bf16=False):
    out = np.empty(n, np.float32)
    lib().orc_fill_normal(fptr(out), n, seed, mean, std, int(bf16))
    return out


def quant(w, bits):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    s = np.empty(rows, np.float32)
    if bits == 8:
        q = np.empty(rows * cols, np.uint8)
        lib().orc_quant_int8(fptr(w), rows, cols, u8ptr(q), fptr(s))
    else:
        q = np.empty(rows * ((cols + 1) // 2), np.uint8)
        lib().orc_quant_int4(fptr(w), rows, cols, u8ptr(q), fptr(s))
    return q, s


def matmul(fmt, w, s, x, out_width, in_width, threads=1):
    x = np.ascontiguousarray(x, np.float32)
    rows = x.size // in_width
    y = np.empty((rows, out_width), np.float32)
    sp = fptr(s) if s is not None else ctypes.cast(None, _f32p)
    lib().orc_matmul(fmt, vptr(w), sp, fptr(x), fptr(y), out_width, in_width, rows,
                     threads)
    return y


def route(logits, bias, top_k, normalize=1, scale=1.0):
    logits = np.ascontiguousarray(logits, np.float32)
    rows, experts = logits.shape
    ids = np.empty((rows, top_k), np.int32)
    w = np.empty((rows, top_k), np.float32)
    bias = np.ascontiguousarray(bias, np.float32)
    lib().orc_route_sigmoid_topk(fptr(logits), fptr(bias), rows, experts, top_k,
                                 normalize, scale, iptr(ids), fptr(w))
    return ids, w


def route_tables(ids, experts, max_batch):
    ids = np.ascontiguousarray(ids, np.int32)
    rows, top_k = ids.shape
    unique = np.full(experts, -1, np.int32)
    counts = np.zeros(experts, np.int32)
    er = np.full(experts * max_batch, -1, np.int32)
    es = np.full(experts * max_batch, -1, np.int32)
    n = lib().orc_route_tables(iptr(ids), rows, top_k, experts, max_batch,
                               iptr(unique), iptr(counts), iptr(er), iptr(es))
    return n, unique[:max(n, 0)], counts, er, es


class Model:
    """Named-tensor oracle model; keeps references to the registered arrays."""

    def __init__(self, config, context_size):
        self.config = config
        self.cfg = OrcConfig(**config)
        self.handle = lib().orc_model_create(ctypes.byref(self.cfg), context_size)
        assert self.handle
        self._keep = []

    def add(self, name, array, dtype=None):
        array = np.ascontiguousarray(array)
        if dtype is None:
            dtype = 3 if array.dtype == np.uint8 else 2
        if dtype == 2:
            assert array.dtype == np.float32
        self._keep.append(array)
        ok = lib().orc_model_add_tensor(self.handle, name.encode(), dtype, vptr(array),
                                        array.size, array.nbytes)
        assert ok

    def close(self):
        if self.handle:
            lib().orc_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()


def zipf_routes(rows, experts, top_k, seed, s=1.1):
    """Expert ids [rows, top_k]: per row top_k distinct experts drawn without
    replacement with p_e proportional to (rank_e + 1)^-s over a seeded
    permutation of the expert ids (the skewed prefill routing of the MoE
    prefill benchmark)."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(experts)
    p = np.empty(experts)
    p[perm] = (np.arange(experts) + 1.0) ** -s
    p /= p.sum()
    return np.stack([rng.choice(experts, top_k, replace=False, p=p)
                     for _ in range(rows)]).astype(np.int32)



def choose_token(logits, temperature, top_p, rng=0):
    """choose_token (moonlight_chat.c:96-131) on the CPU: (token, new rng)."""
    logits = np.ascontiguousarray(logits, np.float32)
    state = ctypes.c_uint64(rng)
    tok = lib().orc_choose_token(fptr(logits), logits.size, temperature, top_p,
                                 ctypes.byref(state))
    return tok, state.value
