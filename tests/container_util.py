"""Synthetic Moonlight containers for tests: writes config.json + safetensors
shards in exactly the layout tools/convert_moonlight.py emits (U8 packed
weights + F32 `.qs` per-row scales; embed, lm_head, router and 1-D tensors
F32), and registers the same tensors with the CPU oracle.

The default shape is the reference's tiny DeepseekV3 fixture
(tools/make_oracle.py:15-41): hidden 256, 4 layers (first dense), 4 heads,
MLA kv_lora 64 / nope 32 / rope 16 / v 32, 64 experts top-6 + 2 shared,
expert FFN 64, dense FFN 512, vocab 512, theta 50000, routed scale 2.446.
"""
import json
import os

import numpy as np
from safetensors.numpy import save_file

import oracle_lib as O

TINY = dict(hidden_size=256, layer_count=4, head_count=4, expert_count=64,
            experts_per_token=6, dense_intermediate_size=512, moe_intermediate_size=64,
            first_dense_layer_count=1, q_lora_rank=0, kv_lora_rank=64, qk_nope_dim=32,
            qk_rope_dim=16, value_dim=32, shared_expert_count=2, normalize_topk=1,
            vocab_size=512, rms_norm_epsilon=1e-5, rope_theta=50000.0, routed_scale=2.446)


def hf_config(cfg):
    """config.json keys read by moonlight_model.c:84-104."""
    return {
        "architectures": ["DeepseekV3ForCausalLM"], "model_type": "deepseek_v3",
        "hidden_size": cfg["hidden_size"], "num_hidden_layers": cfg["layer_count"],
        "num_attention_heads": cfg["head_count"], "num_key_value_heads": cfg["head_count"],
        "n_routed_experts": cfg["expert_count"], "num_experts_per_tok": cfg["experts_per_token"],
        "intermediate_size": cfg["dense_intermediate_size"],
        "moe_intermediate_size": cfg["moe_intermediate_size"],
        "first_k_dense_replace": cfg["first_dense_layer_count"], "q_lora_rank": None,
        "kv_lora_rank": cfg["kv_lora_rank"], "qk_nope_head_dim": cfg["qk_nope_dim"],
        "qk_rope_head_dim": cfg["qk_rope_dim"], "v_head_dim": cfg["value_dim"],
        "n_shared_experts": cfg["shared_expert_count"],
        "norm_topk_prob": bool(cfg["normalize_topk"]), "vocab_size": cfg["vocab_size"],
        "rms_norm_eps": cfg["rms_norm_epsilon"], "rope_theta": cfg["rope_theta"],
        "routed_scaling_factor": cfg["routed_scale"], "scoring_func": "sigmoid",
        "topk_method": "noaux_tc", "tie_word_embeddings": False,
    }


def tensor_specs(cfg):
    """(name, kind, rows, cols): kind 'm' matrix (quantized unless router /
    embed / lm_head), 'n' norm vector, 'b' selection bias."""
    H = cfg["hidden_size"]
    heads, nope, rope, v = (cfg["head_count"], cfg["qk_nope_dim"], cfg["qk_rope_dim"],
                            cfg["value_dim"])
    lora = cfg["kv_lora_rank"]
    out = [("model.embed_tokens.weight", "f", cfg["vocab_size"], H),
           ("model.norm.weight", "n", 1, H), ("lm_head.weight", "f", cfg["vocab_size"], H)]
    for l in range(cfg["layer_count"]):
        p = f"model.layers.{l}."
        out += [(p + "input_layernorm.weight", "n", 1, H),
                (p + "post_attention_layernorm.weight", "n", 1, H),
                (p + "self_attn.q_proj.weight", "d", heads * (nope + rope), H),
                (p + "self_attn.kv_a_proj_with_mqa.weight", "d", lora + rope, H),
                (p + "self_attn.kv_a_layernorm.weight", "n", 1, lora),
                (p + "self_attn.kv_b_proj.weight", "d", heads * (nope + v), lora),
                (p + "self_attn.o_proj.weight", "d", H, heads * v)]
        if l < cfg["first_dense_layer_count"]:
            I = cfg["dense_intermediate_size"]
            out += [(p + "mlp.gate_proj.weight", "d", I, H), (p + "mlp.up_proj.weight", "d", I, H),
                    (p + "mlp.down_proj.weight", "d", H, I)]
            continue
        E, I = cfg["expert_count"], cfg["moe_intermediate_size"]
        sw = I * cfg["shared_expert_count"]
        out += [(p + "mlp.gate.weight", "f", E, H),
                (p + "mlp.gate.e_score_correction_bias", "b", 1, E),
                (p + "mlp.shared_experts.gate_proj.weight", "d", sw, H),
                (p + "mlp.shared_experts.up_proj.weight", "d", sw, H),
                (p + "mlp.shared_experts.down_proj.weight", "d", H, sw)]
        for e in range(E):
            q = f"{p}mlp.experts.{e}."
            out += [(q + "down_proj.weight", "e", H, I), (q + "gate_proj.weight", "e", I, H),
                    (q + "up_proj.weight", "e", I, H)]
    return out


def build_tensors(cfg, ebits=8, dbits=8, seed=1234, std=0.05):
    """name -> numpy array as stored in the container (plus '.qs' scales)."""
    tensors = {}
    for i, (name, kind, rows, cols) in enumerate(tensor_specs(cfg)):
        s = seed * 1000003 + i
        if kind == "n":
            tensors[name] = O.fill_normal(cols, s, mean=1.0, std=0.1)
        elif kind == "b":
            tensors[name] = np.linspace(-0.1, 0.1, cols).astype(np.float32)
        else:
            w = O.fill_normal(rows * cols, s, std=std, bf16=True).reshape(rows, cols)
            if kind == "f":
                tensors[name] = w
            else:
                bits = ebits if kind == "e" else dbits
                q, sc = O.quant(w, bits)
                tensors[name] = q
                tensors[name + ".qs"] = sc
    return tensors


def write_container(path, cfg, tensors, shards=2):
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(hf_config(cfg), f)
    names = sorted(tensors)
    per = (len(names) + shards - 1) // shards
    for i in range(shards):
        part = {n: tensors[n] for n in names[i * per:(i + 1) * per]}
        if part:
            save_file(part, os.path.join(path, f"out-{i:05d}.safetensors"))
    return path


def oracle_model(cfg, tensors, context_size):
    m = O.Model(cfg, context_size)
    for name, arr in tensors.items():
        m.add(name, arr)
    return m
