"""Host-side container parsing (no GPU): the library's reader against the
reference's own moonlight_model.c / st.h / json.h (compiled into
oracle/_ref/libref_model.so from /root/reference by oracle/build_ref.sh) on
containers written like tools/convert_moonlight.py writes them."""
import ctypes
import json
import os

import numpy as np
import pytest
from safetensors.numpy import save_file

import container_util as CU
import oracle_lib as O
from floyd_amd import session as S

REF_MODEL = os.path.join(O.REF_DIR, "libref_model.so")


def ref_probe(path):
    lib = ctypes.CDLL(REF_MODEL)
    ints = np.zeros(16, np.int32)
    floats = np.zeros(3, np.float32)
    err = ctypes.create_string_buffer(512)
    n = lib.ref_model_probe(path.encode(), ints.ctypes.data_as(ctypes.c_void_p),
                            floats.ctypes.data_as(ctypes.c_void_p), err, 512)
    cfg = dict(zip(S.CONFIG_INT_FIELDS, ints.tolist()))
    cfg.update(zip(S.CONFIG_FLOAT_FIELDS, floats.tolist()))
    return cfg, n, err.value.decode()


def small_container(path, config_overrides=None, drop=()):
    cfg = dict(CU.TINY, layer_count=2, expert_count=8, vocab_size=64)
    tensors = CU.build_tensors(cfg, seed=3)
    conf = CU.hf_config(cfg)
    for k in drop:
        conf.pop(k, None)
    conf.update(config_overrides or {})
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(conf, f)
    names = sorted(tensors)
    save_file({n: tensors[n] for n in names[:40]}, os.path.join(path, "out-00000.safetensors"))
    save_file({n: tensors[n] for n in names[40:]}, os.path.join(path, "out-00001.safetensors"))
    return cfg, tensors


CASES = {
    "plain": ({}, ()),
    "rope_parameters": ({"rope_parameters": {"rope_theta": 12345.0}}, ("rope_theta",)),
    "no_norm_topk": ({"norm_topk_prob": False}, ()),
    "defaults": ({}, ("rms_norm_eps", "routed_scaling_factor", "rope_theta")),
    "float_ints": ({"hidden_size": 256.0, "num_experts_per_tok": 6.9}, ()),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_config_and_table_match_reference_reader(tmp_path, case):
    overrides, drop = CASES[case]
    path = str(tmp_path / case)
    cfg, tensors = small_container(path, overrides, drop)
    got, n = S.probe_container(path)
    assert n == len(tensors)
    if os.path.exists(REF_MODEL):
        ref, ref_n, err = ref_probe(path)
        assert ref_n == n, err
        assert got == ref
    else:
        assert got["hidden_size"] == 256
    for name in ("lm_head.weight", "model.layers.1.mlp.experts.3.up_proj.weight",
                 "model.layers.1.mlp.experts.3.up_proj.weight.qs",
                 "model.layers.0.input_layernorm.weight"):
        dtype, numel, nbytes = S.container_tensor(path, name)
        arr = tensors[name]
        assert nbytes == arr.nbytes and numel == arr.size
        assert dtype == (3 if arr.dtype == np.uint8 else 2)


def test_reader_rejects_bad_containers(tmp_path):
    empty = tmp_path / "empty"
    empty.mkdir()
    with pytest.raises(S.SessionError, match="cannot open"):
        S.probe_container(str(empty))
    (empty / "config.json").write_text("{not json")
    with pytest.raises(S.SessionError, match="invalid JSON"):
        S.probe_container(str(empty))
    (empty / "config.json").write_text(json.dumps({"hidden_size": 0}))
    with pytest.raises(S.SessionError, match="unsupported Moonlight config"):
        S.probe_container(str(empty))
    path = str(tmp_path / "noshards")
    small_container(path)
    for f in os.listdir(path):
        if f.endswith(".safetensors"):
            os.remove(os.path.join(path, f))
    with pytest.raises(S.SessionError, match="no safetensors"):
        S.probe_container(path)
