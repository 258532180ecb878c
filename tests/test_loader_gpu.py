"""GPU check of the staged container upload (moonlight_model_open,
floyd_amd/csrc/runtime.cpp upload_container; the reference uploads tensor by
tensor, moonlight_metal.m:850-871): a container larger than three 64 MiB
staging buffers, with tensors of odd byte counts straddling stage and piece
boundaries, lands in HBM byte for byte, with one reader thread and with the
default pool, and with small stages and odd piece sizes forced through the
MLH_LOAD_STAGE_BYTES / MLH_LOAD_PIECE_BYTES overrides."""
import os

import numpy as np
import pytest

import container_util as CU
from floyd_amd import session as S

pytestmark = pytest.mark.gpu

# odd byte counts: tensors cross the 64 MiB stage and 4 MiB piece boundaries
BLOBS = [70 * 2**20 + 13, 3 * 2**20 + 1, 65 * 2**20 - 5, 7, 60 * 2**20 + 4097, 999_999]


@pytest.fixture(scope="module")
def big(tmp_path_factory):
    cfg = dict(CU.TINY)
    tensors = CU.build_tensors(cfg, ebits=8, dbits=4, seed=2468)
    rng = np.random.default_rng(7)
    for i, n in enumerate(BLOBS):
        tensors[f"model.extra.blob{i}"] = rng.integers(0, 256, n, dtype=np.uint8)
    tensors["model.extra.odd_f32"] = rng.standard_normal(333_331).astype(np.float32)
    total = sum(a.nbytes for a in tensors.values())
    assert total > 3 * 64 * 2**20
    path = CU.write_container(str(tmp_path_factory.mktemp("big_container")), cfg, tensors,
                              shards=3)
    print(f"[gpu] container {path}: {len(tensors)} tensors, {total / 2**20:.1f} MiB",
          flush=True)
    return cfg, tensors, path


def load_and_compare(path, tensors, env):
    saved = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        model = S.Model.open(path)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    try:
        for name, arr in tensors.items():
            got = model.read_tensor(name, np.uint8)
            want = np.ascontiguousarray(arr).view(np.uint8).ravel()
            assert got.size == want.size, name
            assert np.array_equal(got, want), name
        sess = S.Session(model, 16, 4)
        logits = sess.prefill(np.array([1, 2, 3], np.int32))
        sess.close()
        return logits
    finally:
        model.close()


@pytest.mark.parametrize("env", [
    {"MLH_LOAD_THREADS": "1"},
    {"MLH_LOAD_THREADS": "8"},
    {"MLH_LOAD_THREADS": "5", "MLH_LOAD_STAGE_BYTES": str(3 * 2**20 + 512),
     "MLH_LOAD_PIECE_BYTES": str(2**18 + 17)},
], ids=["one_reader", "pool", "small_stages"])
def test_staged_upload(big, env):
    cfg, tensors, path = big
    print(f"[gpu] staged upload with {env}", flush=True)
    logits = load_and_compare(path, tensors, env)
    assert np.isfinite(logits).all()
    # the model in HBM computes what a one-reader load computes, bit for bit
    ref = load_and_compare(path, {k: v for k, v in tensors.items() if "extra" not in k},
                           {"MLH_LOAD_THREADS": "1"})
    assert np.array_equal(logits.view(np.uint32), ref.view(np.uint32))
