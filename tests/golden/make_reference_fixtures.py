"""Writes the ORACLE_DIR fixture that the reference's own Moonlight tests read
(tests/test_moonlight_metal_{primitives,mla,moe,runtime}.c: `usage: MODEL
ORACLE_DIR`), computed by the CPU oracle on a tiny converter-layout model.

The reference's generator of these files (tools/make_moonlight_oracle.py) is
deleted upstream, so the tensor names and meanings follow the tests that read
them:
  input_ids            I64 [n]                    every test
  embed                embedding rows             primitives.c:123
  final_input          last layer's output        primitives.c:124
  final_norm           RMSNorm(final_input)       primitives.c:125
  logits               lm_head(final_norm) [n, vocab]  primitives.c:128, runtime.c:122
  layer.0.input_norm   RMSNorm(embed)             primitives.c:126, mla.c:150
  layer.0.q            q_proj(input_norm)         primitives.c:127
  layer.0.attn         attention output (o_proj, no residual)  mla.c:151
  layer.0.kv_a         kv_a_proj_with_mqa(input_norm)          mla.c:152
  layer.0.kv_norm      RMSNorm(kv_a[:, :kv_lora_rank])         mla.c:153
  layer.N.post_norm    RMSNorm(h + attn) (N = 0, 1)            runtime.c:129, moe.c:197
  layer.N.mlp          the FFN output, no residual (N = 0, 1)  runtime.c:130, moe.c:205
  layer.1.router_scores / _ids (I64) / _weights, layer.1.routed_mlp,
  layer.1.shared_mlp   one MoE layer               moe.c:198-204
  layer.N.output       h after layer N             runtime.c:157
  layer.N.router_ids   I64 routes of MoE layer N   runtime.c:173
  ref.json             {"greedy_ids": [g0, g1]}: arg-max of the last row's
                       logits, then of the decode of g0 (runtime.c:35-63)

The MODEL directory itself (several MB) is not committed: it is regenerated
from MODEL_SEED by tests/container_util.py (converter layout, q8 experts and
dense) and checked against MODEL_SHA256 before the tests run.

    python tests/golden/make_reference_fixtures.py
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import container_util as CU  # noqa: E402
import oracle_lib as O  # noqa: E402

OUT = os.path.join(HERE, "ref_tiny_e8d8")
MODEL_SEED = 20261202
EBITS, DBITS = 8, 8
N_TOKENS = 20
IDS_SEED = 97


def model_tensors():
    return CU.build_tensors(dict(CU.TINY), ebits=EBITS, dbits=DBITS, seed=MODEL_SEED)


def tensors_sha256(tensors):
    h = hashlib.sha256()
    for name in sorted(tensors):
        h.update(name.encode())
        h.update(np.ascontiguousarray(tensors[name]).tobytes())
    return h.hexdigest()


def rmsnorm(x, w):
    x = np.ascontiguousarray(x, np.float32)
    rows, width = x.shape
    y = np.empty_like(x)
    O.lib().orc_rmsnorm(O.fptr(x), O.fptr(np.ascontiguousarray(w, np.float32)), O.fptr(y),
                        rows, width, CU.TINY["rms_norm_epsilon"])
    return y


def named(orc, name, x, out_width):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty((x.shape[0], out_width), np.float32)
    assert O.lib().orc_named_matmul(orc.handle, name.encode(), O.fptr(x), x.shape[0],
                                    x.shape[1], out_width, O.fptr(y))
    return y


def main():
    from safetensors.numpy import save_file
    cfg = dict(CU.TINY)
    tensors = model_tensors()
    L, H, V = cfg["layer_count"], cfg["hidden_size"], cfg["vocab_size"]
    K, E = cfg["experts_per_token"], cfg["expert_count"]
    ids = np.random.default_rng(IDS_SEED).integers(0, V, N_TOKENS).astype(np.int32)
    n = len(ids)
    orc = CU.oracle_model(cfg, tensors, 64)
    out = {"input_ids": ids.astype(np.int64)}
    h = tensors["model.embed_tokens.weight"][ids].astype(np.float32)
    out["embed"] = h.copy()
    for l in range(L):
        p = f"model.layers.{l}."
        xn = rmsnorm(h, tensors[p + "input_layernorm.weight"])
        attn = np.empty_like(xn)
        assert O.lib().orc_attention(orc.handle, l, O.fptr(xn), n, 0, O.fptr(attn))
        if l == 0:
            out["layer.0.input_norm"] = xn
            qw = cfg["head_count"] * (cfg["qk_nope_dim"] + cfg["qk_rope_dim"])
            out["layer.0.q"] = named(orc, p + "self_attn.q_proj.weight", xn, qw)
            cw = cfg["kv_lora_rank"] + cfg["qk_rope_dim"]
            out["layer.0.kv_a"] = named(orc, p + "self_attn.kv_a_proj_with_mqa.weight", xn, cw)
            lat = np.empty((n, cfg["kv_lora_rank"]), np.float32)
            rope = np.empty((n, cfg["qk_rope_dim"]), np.float32)
            assert O.lib().orc_model_copy_kv(orc.handle, 0, O.fptr(lat), O.fptr(rope), n)
            out["layer.0.kv_norm"] = lat
            out["layer.0.attn"] = attn
        h1 = h + attn
        pn = rmsnorm(h1, tensors[p + "post_attention_layernorm.weight"])
        if l < cfg["first_dense_layer_count"]:
            mlp = np.empty_like(pn)
            assert O.lib().orc_dense_mlp(orc.handle, l, O.fptr(pn), n, O.fptr(mlp))
        else:
            r_ids = np.empty((n, K), np.int32)
            r_w = np.empty((n, K), np.float32)
            r_logits = np.empty((n, E), np.float32)
            routed, shared, mlp = (np.empty_like(pn) for _ in range(3))
            assert O.lib().orc_moe_layer(orc.handle, l, O.fptr(pn), n, O.iptr(r_ids),
                                         O.fptr(r_w), O.fptr(r_logits), O.fptr(routed),
                                         O.fptr(shared), O.fptr(mlp))
            out[f"layer.{l}.router_ids"] = r_ids.astype(np.int64)
            if l == 1:
                out["layer.1.router_scores"] = r_logits
                out["layer.1.router_weights"] = r_w
                out["layer.1.routed_mlp"] = routed
                out["layer.1.shared_mlp"] = shared
        if l <= 1:
            out[f"layer.{l}.post_norm"] = pn
            out[f"layer.{l}.mlp"] = mlp
        h = h1 + mlp
        out[f"layer.{l}.output"] = h.copy()
    out["final_input"] = h.copy()
    fn = rmsnorm(h, tensors["model.norm.weight"])
    out["final_norm"] = fn
    out["logits"] = named(orc, "lm_head.weight", fn, V)
    orc.close()
    # the composition above is the oracle's own forward, bit for bit
    check = CU.oracle_model(cfg, tensors, 64)
    layers = np.empty((L, n, H), np.float32)
    trace = np.full((L, n, K), -1, np.int32)
    last = np.empty(V, np.float32)
    assert O.lib().orc_forward(check.handle, O.iptr(ids), n, 0, O.fptr(layers), O.iptr(trace),
                               O.fptr(last))
    for l in range(L):
        assert np.array_equal(layers[l].view(np.uint32), out[f"layer.{l}.output"].view(np.uint32))
    assert np.array_equal(last.view(np.uint32), out["logits"][-1].view(np.uint32))
    g0 = int(np.argmax(last))
    dec = np.empty(V, np.float32)
    assert O.lib().orc_forward(check.handle, O.iptr(np.array([g0], np.int32)), 1, n, None, None,
                               O.fptr(dec))
    g1 = int(np.argmax(dec))
    check.close()
    os.makedirs(OUT, exist_ok=True)
    save_file({k: np.ascontiguousarray(v) for k, v in out.items()},
              os.path.join(OUT, "oracle.safetensors"))
    with open(os.path.join(OUT, "ref.json"), "w") as f:
        json.dump({"greedy_ids": [g0, g1]}, f)
    with open(os.path.join(OUT, "model.json"), "w") as f:
        json.dump({"config": cfg, "ebits": EBITS, "dbits": DBITS, "seed": MODEL_SEED,
                   "sha256": tensors_sha256(tensors), "tokens": n}, f, indent=1)
    print(f"wrote {OUT}: {len(out)} tensors, greedy {g0}, {g1}")


if __name__ == "__main__":
    main()
