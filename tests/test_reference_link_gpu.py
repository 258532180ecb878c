"""The reference's tests/test_backend_metal.c, compiled unchanged and linked
against libfloyd_amd.so (oracle/build_ref.sh), run on the GPU: fm_init,
fm_device_name and fm_matmul_q8/q4 with cache = 0 and 1, odd I = 257, S = 4,
checked by the test's own f64 reference (max rel error <= 1e-3)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "oracle", "_ref", "test_backend_metal")

pytestmark = pytest.mark.gpu


@pytest.mark.skipif(not os.path.exists(BINARY), reason="oracle/_ref not built")
def test_reference_backend_test_passes():
    print("[gpu] reference test_backend_metal against libfloyd_amd.so", flush=True)
    run = subprocess.run([BINARY], capture_output=True, text=True, timeout=120)
    print(run.stdout, run.stderr, flush=True)
    assert run.returncode == 0
    assert run.stdout.strip().endswith("OK")
    assert "gfx950" in run.stdout
