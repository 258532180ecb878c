"""Parity at the real Moonlight-16B-A3B shapes (benchmark configs 2 and 4) on a
synthetic q8 model generated in HBM (moonlight_model_create_synthetic): the
oracle reads the very same packed weights back from the device.

  test_moe_decode         config 2: one MoE layer, T = 1, 8, 64 token rows
  test_mla_decode_ctx4096 config 4 attention: one layer at position 4096 over
                          a latent cache pre-filled ~N(0, 1)
  test_decode_step        config 4: a full 27-layer decode step at ctx 4096,
                          logits rel-L2 <= 1e-3, routes equal in every layer
"""
import numpy as np
import pytest

import oracle_lib as O
from conftest import rel_l2
from floyd_amd import session as S

pytestmark = pytest.mark.gpu

MOON = dict(hidden_size=2048, layer_count=27, head_count=16, expert_count=64,
            experts_per_token=6, dense_intermediate_size=11264, moe_intermediate_size=1408,
            first_dense_layer_count=1, q_lora_rank=0, kv_lora_rank=512, qk_nope_dim=128,
            qk_rope_dim=64, value_dim=128, shared_expert_count=2, normalize_topk=1,
            vocab_size=163840, rms_norm_epsilon=1e-5, rope_theta=50000.0, routed_scale=2.446)


@pytest.fixture(scope="module")
def moon(device):
    print("[gpu] building the synthetic Moonlight q8 model in HBM", flush=True)
    model = S.Model.synthetic()
    O.lib().orc_set_threads(16)
    yield model
    model.close()


def oracle_with(model, names, context):
    """Oracle model holding the named tensors (and their .qs scales) read back
    from HBM."""
    orc = O.Model(MOON, context)
    for name in names:
        for n in (name, name + ".qs"):
            info = model.tensor_info(n)
            if info is None:
                continue
            arr = model.read_tensor(n, np.uint8 if info[0] == 3 else np.float32)
            orc.add(n, arr, dtype=info[0])
    return orc


def moe_layer_names(layer):
    p = f"model.layers.{layer}.mlp."
    names = [p + "gate.weight", p + "gate.e_score_correction_bias"]
    names += [p + f"shared_experts.{m}_proj.weight" for m in ("gate", "up", "down")]
    names += [p + f"experts.{e}.{m}_proj.weight" for e in range(64) for m in ("gate", "up", "down")]
    return names


@pytest.mark.parametrize("rows", [1, 8, 64])
def test_moe_decode(moon, rows):
    print(f"[gpu] moonlight MoE layer rows={rows}", flush=True)
    sess = S.Session(moon, 128, 64)
    x = O.fill_normal(rows * 2048, 40 + rows).reshape(rows, 2048)
    got = sess.test_moe(1, x)
    assert got is not None
    bias = np.linspace(-0.1, 0.1, 64).astype(np.float32)
    ids, w = O.route(got["logits"], bias, 6, 1, 2.446)
    assert np.array_equal(got["ids"], ids)
    assert np.array_equal(got["weights"].view(np.uint32), w.view(np.uint32))
    orc = oracle_with(moon, moe_layer_names(1), 8)
    e = {k: np.empty_like(x) for k in ("routed", "shared", "out")}
    e_ids = np.empty((rows, 6), np.int32)
    e_w = np.empty((rows, 6), np.float32)
    e_logits = np.empty((rows, 64), np.float32)
    assert O.lib().orc_moe_layer(orc.handle, 1, O.fptr(x), rows, O.iptr(e_ids), O.fptr(e_w),
                                 O.fptr(e_logits), O.fptr(e["routed"]), O.fptr(e["shared"]),
                                 O.fptr(e["out"]))
    assert rel_l2(got["logits"], e_logits) < 1e-5
    same = np.array([set(a) == set(b) for a, b in zip(got["ids"], e_ids)])
    assert same.all(), np.nonzero(~same)
    # fp32-exact GEMV below 5 rows; from 5 rows the int8-limb MFMA GEMM (~2e-4)
    tol = 1e-4 if rows < 5 else 1e-3
    for k in ("routed", "shared", "out"):
        err = rel_l2(got[k], e[k])
        print(f"[gpu] rows={rows} {k} rel-L2 {err:.2e}", flush=True)
        assert err < tol, k
    sess.close()
    orc.close()


def attention_names(layer):
    p = f"model.layers.{layer}.self_attn."
    return [p + n for n in ("q_proj.weight", "kv_a_proj_with_mqa.weight", "kv_b_proj.weight",
                            "o_proj.weight", "kv_a_layernorm.weight")]


def test_mla_decode_ctx4096(moon):
    print("[gpu] moonlight MLA decode at position 4096", flush=True)
    ctx, layer = 4097, 2
    sess = S.Session(moon, ctx, 4)
    sess.fill_kv(4096, seed=99, layer=layer)
    lat, rope = sess.test_copy_kv(layer, 4096)
    orc = oracle_with(moon, attention_names(layer), ctx)
    assert O.lib().orc_model_set_kv(orc.handle, layer, O.fptr(lat), O.fptr(rope), 4096)
    x = O.fill_normal(2048, 77).reshape(1, 2048)
    got = sess.test_attention(layer, x, 4096)
    expect = np.empty_like(x)
    assert O.lib().orc_attention(orc.handle, layer, O.fptr(x), 1, 4096, O.fptr(expect))
    assert rel_l2(got, expect) < 1e-4
    lat2, rope2 = sess.test_copy_kv(layer, 4097)
    elat = np.empty((4097, 512), np.float32)
    erope = np.empty((4097, 64), np.float32)
    assert O.lib().orc_model_copy_kv(orc.handle, layer, O.fptr(elat), O.fptr(erope), 4097)
    assert rel_l2(lat2[4096], elat[4096]) < 1e-5 and rel_l2(rope2[4096], erope[4096]) < 1e-5
    sess.close()
    orc.close()


def all_names(model):
    names = ["model.embed_tokens.weight", "model.norm.weight", "lm_head.weight"]
    for l in range(27):
        p = f"model.layers.{l}."
        names += [p + "input_layernorm.weight", p + "post_attention_layernorm.weight"]
        names += attention_names(l)
        if l == 0:
            names += [p + f"mlp.{m}_proj.weight" for m in ("gate", "up", "down")]
        else:
            names += moe_layer_names(l)
    return names


def test_decode_step(moon):
    print("[gpu] moonlight full decode step at ctx 4096 (oracle reads 17 GB back)", flush=True)
    ctx = 4097
    sess = S.Session(moon, ctx, 1)
    sess.fill_kv(4096, seed=5)
    orc = oracle_with(moon, all_names(moon), ctx)
    for l in range(27):
        lat, rope = sess.test_copy_kv(l, 4096)
        assert O.lib().orc_model_set_kv(orc.handle, l, O.fptr(lat), O.fptr(rope), 4096)
    token = 12345
    logits = sess.decode(token)
    routes = [sess.test_copy_routes(l, 1) for l in range(1, 27)]
    layers = np.empty((27, 1, 2048), np.float32)
    trace = np.full((27, 1, 6), -1, np.int32)
    e_logits = np.empty(163840, np.float32)
    tok = np.array([token], np.int32)
    assert O.lib().orc_forward(orc.handle, O.iptr(tok), 1, 4096, O.fptr(layers), O.iptr(trace),
                               O.fptr(e_logits))
    err = rel_l2(logits, e_logits)
    print(f"[gpu] decode step logits rel-L2 {err:.3e}", flush=True)
    assert err < 1e-3
    assert int(np.argmax(logits)) == int(np.argmax(e_logits))
    for l, r in zip(range(1, 27), routes):
        assert set(r[0]) == set(trace[l, 0]), l
    # the device sampler over the full 163,840-token vocabulary
    from sampler_util import nucleus_choice, xorshift_unit
    assert sess.sample(0.0)[0] == int(np.argmax(logits))
    state, compared = 2024, 0
    for temperature, top_p in ((1.0, 0.9), (0.6, 0.95), (1.0, 1.0)):
        for _ in range(4):
            u = xorshift_unit(state)[0]
            want, margin, _ = nucleus_choice(logits, temperature, top_p, u)
            e_tok, e_state = O.choose_token(logits, temperature, top_p, state)
            tok, state = sess.sample(temperature, top_p, state)
            assert state == e_state
            if margin > 1e-6:
                assert tok == e_tok == want, (temperature, top_p, u)
                compared += 1
    assert compared >= 10
    sess.close()
    orc.close()
