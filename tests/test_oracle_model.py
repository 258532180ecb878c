"""Pins the oracle's composite functions on the CPU against formulations that
do not share its code:

  orc_attention  explicit decompression K_h = W_UK_h lat, V_h = W_UV_h lat and
                 textbook causal softmax attention in f64 (the absorbed form of
                 moonlight_kernels.metal:218-375 is an algebraic rewrite of it);
                 one key gives ctx_h = W_UV_h lat_0; split prefill + append
                 equals one prefill (tests/test_moonlight_metal_mla.c:219-238).
  orc_dense_mlp  f64 SwiGLU on the dequantised weights.
  orc_moe_layer  moe_exec.h built from the reference (moe_f32_forward: experts
                 summed in ascending index order, each shared expert separately)
                 on the dequantised weights.
  orc_forward    split prefill + append equals one prefill
                 (tests/test_moonlight_metal_runtime.c:252-268); layer outputs are
                 the residual stream of the composed pieces.
"""
import ctypes
import os

import numpy as np
import pytest

import oracle_lib as O
from conftest import rel_l2
from container_util import TINY, build_tensors, oracle_model

REF_MOE = os.path.join(O.REF_DIR, "libref_moe.so")


def dequant(tensors, name, rows, cols):
    """f64 [rows, cols] from a stored matrix (f32, or U8 q8/q4 + '.qs')."""
    q = tensors[name]
    if q.dtype == np.float32:
        return q.reshape(rows, cols).astype(np.float64)
    s = tensors[name + ".qs"].astype(np.float64)
    if q.size == rows * cols:
        return q.view(np.int8).reshape(rows, cols).astype(np.float64) * s[:, None]
    rb = (cols + 1) // 2
    b = q.reshape(rows, rb)
    vals = np.empty((rows, 2 * rb), np.float64)
    vals[:, 0::2] = (b & 15).astype(np.int64) - 8
    vals[:, 1::2] = (b >> 4).astype(np.int64) - 8
    return vals[:, :cols] * s[:, None]


def rmsnorm64(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w


def rope64(v, pos, theta):
    """Rotation of the interleaved pairs (2p, 2p+1) by pos * theta^(-2p/n),
    written out in half layout [p] / [n/2 + p] (closed form pinned in
    test_oracle_math.test_rope_closed_forms)."""
    n = v.shape[-1]
    ang = pos * theta ** (-2.0 * np.arange(n // 2) / n)
    z = (v[..., 0::2] + 1j * v[..., 1::2]) * np.exp(1j * ang)
    return np.concatenate([z.real, z.imag], axis=-1)


def attention64(t, cfg, layer, x, position, lat_prev, rope_prev):
    """Explicit (non-absorbed) MLA in f64.  Returns (out, new latent rows, new
    rope rows)."""
    H, heads = cfg["hidden_size"], cfg["head_count"]
    nope, rope, vd, lw = cfg["qk_nope_dim"], cfg["qk_rope_dim"], cfg["value_dim"], cfg["kv_lora_rank"]
    eps, theta = cfg["rms_norm_epsilon"], cfg["rope_theta"]
    p = f"model.layers.{layer}.self_attn."
    wq = dequant(t, p + "q_proj.weight", heads * (nope + rope), H)
    wkva = dequant(t, p + "kv_a_proj_with_mqa.weight", lw + rope, H)
    wkvb = dequant(t, p + "kv_b_proj.weight", heads * (nope + vd), lw).reshape(heads, nope + vd, lw)
    wo = dequant(t, p + "o_proj.weight", H, heads * vd)
    kvn = t[p + "kv_a_layernorm.weight"].astype(np.float64)
    rows = x.shape[0]
    x = x.astype(np.float64)
    q = (x @ wq.T).reshape(rows, heads, nope + rope)
    c = x @ wkva.T
    pos = position + np.arange(rows)
    lat_new = rmsnorm64(c[:, :lw], kvn, eps)
    rope_new = np.stack([rope64(c[r, lw:], pos[r], theta) for r in range(rows)])
    lat = np.concatenate([lat_prev.astype(np.float64), lat_new])
    rp = np.concatenate([rope_prev.astype(np.float64), rope_new])
    k_nope = np.einsum("hnl,kl->hkn", wkvb[:, :nope], lat)   # [heads, keys, nope]
    v = np.einsum("hvl,kl->hkv", wkvb[:, nope:], lat)         # [heads, keys, vdim]
    ctx = np.empty((rows, heads, vd))
    for r in range(rows):
        keys = position + r + 1
        qr = np.stack([rope64(q[r, h, nope:], pos[r], theta) for h in range(heads)])
        s = (np.einsum("hn,hkn->hk", q[r, :, :nope], k_nope[:, :keys]) + qr @ rp[:keys].T)
        s = s / np.sqrt(nope + rope)
        e = np.exp(s - s.max(axis=1, keepdims=True))
        prob = e / e.sum(axis=1, keepdims=True)
        ctx[r] = np.einsum("hk,hkv->hv", prob, v[:, :keys])
    return ctx.reshape(rows, heads * vd) @ wo.T, lat_new, rope_new


@pytest.fixture(scope="module", params=[(8, 8), (4, 4)], ids=["q8", "q4"])
def tiny(request):
    ebits, dbits = request.param
    t = build_tensors(TINY, ebits=ebits, dbits=dbits, seed=4242)
    return t


def kv_of(m, layer, n):
    lat = np.empty((n, TINY["kv_lora_rank"]), np.float32)
    rp = np.empty((n, TINY["qk_rope_dim"]), np.float32)
    assert O.lib().orc_model_copy_kv(m.handle, layer, O.fptr(lat), O.fptr(rp), n)
    return lat, rp


def test_attention_equals_explicit_decompression(tiny):
    cfg, layer, ctx = TINY, 1, 16
    m = oracle_model(cfg, tiny, ctx)
    # 5 cached keys ~N(0,1), then 3 new rows appended at position 5
    lat0 = O.fill_normal(5 * 64, 8).reshape(5, 64)
    rope0 = O.fill_normal(5 * 16, 9).reshape(5, 16)
    assert O.lib().orc_model_set_kv(m.handle, layer, O.fptr(lat0), O.fptr(rope0), 5)
    x = O.fill_normal(3 * 256, 10).reshape(3, 256)
    out = np.empty_like(x)
    assert O.lib().orc_attention(m.handle, layer, O.fptr(x), 3, 5, O.fptr(out))
    expect, lat_new, rope_new = attention64(tiny, cfg, layer, x, 5, lat0, rope0)
    assert rel_l2(out, expect) < 1e-5
    lat, rp = kv_of(m, layer, 8)
    assert np.array_equal(lat[:5], lat0) and np.array_equal(rp[:5], rope0)
    assert rel_l2(lat[5:], lat_new) < 1e-6 and rel_l2(rp[5:], rope_new) < 1e-6
    m.close()


def test_attention_single_key_is_value_projection(tiny):
    cfg, layer = TINY, 2
    m = oracle_model(cfg, tiny, 4)
    x = O.fill_normal(256, 21).reshape(1, 256)
    out = np.empty_like(x)
    assert O.lib().orc_attention(m.handle, layer, O.fptr(x), 1, 0, O.fptr(out))
    lat, _ = kv_of(m, layer, 1)
    p = f"model.layers.{layer}.self_attn."
    heads, nope, vd, lw = 4, 32, 32, 64
    wkvb = dequant(tiny, p + "kv_b_proj.weight", heads * (nope + vd), lw).reshape(heads, nope + vd, lw)
    wo = dequant(tiny, p + "o_proj.weight", 256, heads * vd)
    ctx = np.einsum("hvl,l->hv", wkvb[:, nope:], lat[0].astype(np.float64)).reshape(-1)
    assert rel_l2(out[0], wo @ ctx) < 1e-6
    m.close()


def test_attention_split_prefill_equals_full(tiny):
    x = O.fill_normal(6 * 256, 31).reshape(6, 256)
    full = oracle_model(TINY, tiny, 8)
    out_full = np.empty_like(x)
    assert O.lib().orc_attention(full.handle, 1, O.fptr(x), 6, 0, O.fptr(out_full))
    split = oracle_model(TINY, tiny, 8)
    a, b = np.empty((4, 256), np.float32), np.empty((2, 256), np.float32)
    assert O.lib().orc_attention(split.handle, 1, O.fptr(np.ascontiguousarray(x[:4])), 4, 0, O.fptr(a))
    assert O.lib().orc_attention(split.handle, 1, O.fptr(np.ascontiguousarray(x[4:])), 2, 4, O.fptr(b))
    assert np.array_equal(np.concatenate([a, b]), out_full)
    # the position precondition (moonlight_metal.m:1366-1369) is enforced
    assert not O.lib().orc_attention(split.handle, 1, O.fptr(b), 2, 4, O.fptr(b))
    full.close()
    split.close()


def test_dense_mlp_equals_f64_swiglu(tiny):
    m = oracle_model(TINY, tiny, 4)
    x = O.fill_normal(5 * 256, 41).reshape(5, 256)
    out = np.empty_like(x)
    assert O.lib().orc_dense_mlp(m.handle, 0, O.fptr(x), 5, O.fptr(out))
    p = "model.layers.0.mlp."
    g = x.astype(np.float64) @ dequant(tiny, p + "gate_proj.weight", 512, 256).T
    u = x.astype(np.float64) @ dequant(tiny, p + "up_proj.weight", 512, 256).T
    h = g / (1 + np.exp(-g)) * u
    assert rel_l2(out, h @ dequant(tiny, p + "down_proj.weight", 256, 512).T) < 1e-5
    m.close()


@pytest.mark.skipif(not os.path.exists(REF_MOE), reason="oracle/_ref not built")
def test_moe_layer_equals_reference_moe_exec(tiny):
    cfg, layer, rows = TINY, 2, 7
    H, E, I, K = 256, 64, 64, 6
    m = oracle_model(cfg, tiny, 4)
    x = O.fill_normal(rows * H, 51).reshape(rows, H)
    out = np.empty_like(x)
    ids = np.empty((rows, K), np.int32)
    assert O.lib().orc_moe_layer(m.handle, layer, O.fptr(x), rows, O.iptr(ids), None, None,
                                 None, None, O.fptr(out))
    p = f"model.layers.{layer}.mlp."

    def f32(name, r, c):
        return np.ascontiguousarray(dequant(tiny, name, r, c), np.float32)

    gate = np.stack([f32(p + f"experts.{e}.gate_proj.weight", I, H) for e in range(E)])
    up = np.stack([f32(p + f"experts.{e}.up_proj.weight", I, H) for e in range(E)])
    down = np.stack([f32(p + f"experts.{e}.down_proj.weight", H, I) for e in range(E)])
    sg = f32(p + "shared_experts.gate_proj.weight", 2 * I, H).reshape(2, I, H)
    su = f32(p + "shared_experts.up_proj.weight", 2 * I, H).reshape(2, I, H)
    sd_full = f32(p + "shared_experts.down_proj.weight", H, 2 * I)
    sd = np.ascontiguousarray(np.stack([sd_full[:, :I], sd_full[:, I:]]))
    router = np.ascontiguousarray(tiny[p + "gate.weight"])
    bias = np.ascontiguousarray(tiny[p + "gate.e_score_correction_bias"])
    ref = ctypes.CDLL(REF_MOE)
    ref.ref_moe_forward_flat.argtypes = [ctypes.c_int] * 5 + [ctypes.c_float] * 2 + \
        [ctypes.POINTER(ctypes.c_float)] * 5 + [ctypes.c_int] + \
        [ctypes.POINTER(ctypes.c_float)] * 4 + [ctypes.c_int, ctypes.POINTER(ctypes.c_float)]
    expect = np.empty_like(x)
    assert ref.ref_moe_forward_flat(H, I, E, K, 1, 2.446, 0.0, O.fptr(router), O.fptr(bias),
                                    O.fptr(gate), O.fptr(up), O.fptr(down), 2, O.fptr(sg),
                                    O.fptr(su), O.fptr(sd), O.fptr(x), rows, O.fptr(expect))
    assert rel_l2(out, expect) < 1e-5
    # distinct experts per row, all in range
    assert all(len(set(r)) == K for r in ids) and ids.min() >= 0 and ids.max() < E
    m.close()


@pytest.mark.skipif(not os.path.exists(REF_MOE), reason="oracle/_ref not built")
def test_moe_layer_fixed_equals_reference_moe_exec(tiny):
    cfg, layer, rows = TINY, 3, 9
    H, E, I, K = 256, 64, 64, 6
    m = oracle_model(cfg, tiny, 4)
    x = O.fill_normal(rows * H, 61).reshape(rows, H)
    ids = O.zipf_routes(rows, E, K, seed=8)
    out = np.empty_like(x)
    w = np.empty((rows, K), np.float32)
    assert O.lib().orc_moe_layer_fixed(m.handle, layer, O.fptr(x), rows, O.iptr(ids), O.fptr(w),
                                       O.fptr(out))
    p = f"model.layers.{layer}.mlp."

    def f32(name, r, c):
        return np.ascontiguousarray(dequant(tiny, name, r, c), np.float32)

    gate = np.stack([f32(p + f"experts.{e}.gate_proj.weight", I, H) for e in range(E)])
    up = np.stack([f32(p + f"experts.{e}.up_proj.weight", I, H) for e in range(E)])
    down = np.stack([f32(p + f"experts.{e}.down_proj.weight", H, I) for e in range(E)])
    sg = f32(p + "shared_experts.gate_proj.weight", 2 * I, H).reshape(2, I, H)
    su = f32(p + "shared_experts.up_proj.weight", 2 * I, H).reshape(2, I, H)
    sd_full = f32(p + "shared_experts.down_proj.weight", H, 2 * I)
    sd = np.ascontiguousarray(np.stack([sd_full[:, :I], sd_full[:, I:]]))
    router = np.ascontiguousarray(tiny[p + "gate.weight"])
    fixed = np.ascontiguousarray(ids.astype(np.int64))
    ref = ctypes.CDLL(REF_MOE)
    fp = ctypes.POINTER(ctypes.c_float)
    ref.ref_moe_forward_fixed_flat.argtypes = [ctypes.c_int] * 5 + [ctypes.c_float] + \
        [fp] * 4 + [ctypes.c_int] + [fp] * 4 + [ctypes.c_int, ctypes.c_void_p, fp]
    expect = np.empty_like(x)
    assert ref.ref_moe_forward_fixed_flat(H, I, E, K, 1, 2.446, O.fptr(router), O.fptr(gate),
                                          O.fptr(up), O.fptr(down), 2, O.fptr(sg), O.fptr(su),
                                          O.fptr(sd), O.fptr(x), rows, fixed.ctypes.data,
                                          O.fptr(expect))
    assert rel_l2(out, expect) < 1e-5
    m.close()


def test_forward_split_prefill_equals_full(tiny):
    ids = np.array([5, 77, 300, 12, 511, 0], np.int32)
    L, H, V = TINY["layer_count"], 256, 512

    def run(model, chunk, start):
        n = chunk.size
        layers = np.empty((L, n, H), np.float32)
        trace = np.full((L, n, 6), -1, np.int32)
        logits = np.empty(V, np.float32)
        assert O.lib().orc_forward(model.handle, O.iptr(chunk), n, start, O.fptr(layers),
                                   O.iptr(trace), O.fptr(logits))
        return layers, trace, logits

    full = oracle_model(TINY, tiny, 8)
    lf, tf, gf = run(full, ids, 0)
    split = oracle_model(TINY, tiny, 8)
    run(split, ids[:4].copy(), 0)
    ls, ts, gs = run(split, ids[4:].copy(), 4)
    assert np.array_equal(gs, gf)
    assert np.array_equal(ls, lf[:, 4:]) and np.array_equal(ts, tf[:, 4:])
    assert (tf[0] == -1).all() and (tf[1:] >= 0).all()  # layer 0 is dense
    # the residual stream: layer 0 output = embed + attn + dense ffn of the oracle pieces
    emb = tiny["model.embed_tokens.weight"].reshape(V, H)[ids]
    one = oracle_model(TINY, tiny, 8)
    w_in = tiny["model.layers.0.input_layernorm.weight"]
    w_post = tiny["model.layers.0.post_attention_layernorm.weight"]
    n1 = np.empty_like(emb)
    O.lib().orc_rmsnorm(O.fptr(np.ascontiguousarray(emb)), O.fptr(w_in), O.fptr(n1), 6, H, 1e-5)
    a = np.empty_like(emb)
    assert O.lib().orc_attention(one.handle, 0, O.fptr(n1), 6, 0, O.fptr(a))
    h = emb + a
    n2 = np.empty_like(h)
    O.lib().orc_rmsnorm(O.fptr(h), O.fptr(w_post), O.fptr(n2), 6, H, 1e-5)
    d = np.empty_like(h)
    assert O.lib().orc_dense_mlp(one.handle, 0, O.fptr(n2), 6, O.fptr(d))
    assert np.array_equal(lf[0], h + d)
    for mm in (full, split, one):
        mm.close()
