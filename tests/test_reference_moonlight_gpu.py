"""The reference's own Moonlight tests (tests/test_moonlight_metal_primitives.c,
_mla.c, _moe.c, _runtime.c), compiled from their sources and linked against
libfloyd_amd.so (oracle/build_ref.sh), run on the GPU with their own gates
(max-abs 3e-6 .. 5e-4, zero route-mismatch rows, greedy tokens, the
command_buffers pins) against:

  MODEL       a tiny converter-layout container (q8 experts and dense)
              regenerated from the seed in tests/golden/ref_tiny_e8d8/model.json
              and checked against its recorded SHA-256;
  ORACLE_DIR  tests/golden/ref_tiny_e8d8 (oracle.safetensors + ref.json),
              written by tests/golden/make_reference_fixtures.py from the CPU
              oracle.

The runtime test runs from the build whose device-name check expects
"gfx950" instead of "Apple" (test_moonlight_metal_runtime.c:94); the other
three run unchanged."""
import json
import os
import subprocess
import sys

import pytest

import container_util as CU

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_BIN = os.path.join(ROOT, "oracle", "_ref")
FIXTURE = os.path.join(ROOT, "tests", "golden", "ref_tiny_e8d8")
sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model_dir(tmp_path_factory):
    import make_reference_fixtures as MF
    meta = json.load(open(os.path.join(FIXTURE, "model.json")))
    assert meta["seed"] == MF.MODEL_SEED
    tensors = MF.model_tensors()
    assert MF.tensors_sha256(tensors) == meta["sha256"]
    path = CU.write_container(str(tmp_path_factory.mktemp("ref_model")), dict(CU.TINY), tensors)
    print(f"[gpu] reference-test model {path}", flush=True)
    return path


@pytest.mark.parametrize("name", ["primitives", "mla", "moe", "runtime_gfx950"])
def test_reference_moonlight_test_passes(model_dir, name):
    binary = os.path.join(REF_BIN, f"test_moonlight_metal_{name}")
    if not os.path.exists(binary):
        pytest.skip("oracle/_ref not built")
    print(f"[gpu] reference test_moonlight_metal_{name} {model_dir} {FIXTURE}", flush=True)
    run = subprocess.run([binary, model_dir, FIXTURE], capture_output=True, text=True,
                         timeout=120)
    print(run.stdout, run.stderr, flush=True)
    assert run.returncode == 0, run.stderr
