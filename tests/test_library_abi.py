"""CPU checks of the C-ABI boundary: the built library loads without a GPU and
exports every function that include/*.h declares (no compute calls here)."""
import os
import re
import subprocess

import pytest

from floyd_amd import native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def declared_functions():
    names = set()
    for header in sorted(os.listdir(INCLUDE)):
        if not header.endswith(".h"):
            continue
        text = open(os.path.join(INCLUDE, header)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"\b([a-z_][a-z0-9_]*)\s*\(([^;{]*?)\)\s*;", text):
            names.add(m.group(1))
    return names


@pytest.fixture(scope="module")
def exported():
    if not os.path.exists(native.LIBRARY_PATH):
        pytest.fail("libfloyd_amd.so is not built (python -m floyd_amd.build)")
    out = subprocess.run(["nm", "-D", "--defined-only", native.LIBRARY_PATH],
                         capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_headers_declare_entry_points():
    names = declared_functions()
    for expected in ("fm_matmul_q8", "mlk_gemv"):
        assert expected in names


def test_every_declared_function_is_exported(exported):
    missing = sorted(declared_functions() - exported)
    assert not missing, missing


def test_library_loads_and_binds_without_gpu():
    lib = native.load()
    for name in native.SIGNATURES:
        assert hasattr(lib, name)
    assert set(native.SIGNATURES) <= declared_functions()


REF_TESTS = ["test_backend_metal"] + [f"test_moonlight_metal_{t}"
                                      for t in ("runtime", "primitives", "mla", "moe")]


@pytest.mark.parametrize("name", REF_TESTS)
def test_reference_tests_link_against_library(exported, name):
    """The reference's own boundary tests (compiled unchanged by
    oracle/build_ref.sh) take every moonlight_* / fm_* symbol they use from
    libfloyd_amd.so."""
    path = os.path.join(ROOT, "oracle", "_ref", name)
    if not os.path.exists(path):
        pytest.skip("oracle/_ref not built (needs the reference tree)")
    out = subprocess.run(["nm", "-D", "--undefined-only", path], capture_output=True,
                         text=True, check=True).stdout
    used = {line.split()[-1] for line in out.splitlines()}
    boundary = {s for s in used if s.startswith(("moonlight_", "fm_"))}
    assert boundary, "no boundary symbols used"
    assert boundary <= exported, sorted(boundary - exported)
