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


# The production entry points moonlight_chat.c calls (moonlight_chat.c:133-153,
# :173-202, :255-297, :377-413).
CHAT_SYMBOLS = {"moonlight_model_open", "moonlight_model_close", "moonlight_model_info",
                "moonlight_device_name", "moonlight_session_create",
                "moonlight_session_destroy", "moonlight_session_reset",
                "moonlight_session_position", "moonlight_session_stats",
                "moonlight_session_prefill", "moonlight_session_append",
                "moonlight_session_decode"}


def test_floyd_cli_links_against_library(exported):
    """floyd's own CLI -- floyd.c, moonlight_chat.c, moonlight_model.c and the
    HTTP layer, compiled unchanged by oracle/build_ref.sh with a DeepSeek-V4
    stub -- takes every Moonlight session symbol it uses from libfloyd_amd.so
    and runs (its usage text needs no GPU)."""
    path = os.path.join(ROOT, "oracle", "_ref", "floyd")
    if not os.path.exists(path):
        pytest.skip("oracle/_ref not built (needs the reference tree)")
    out = subprocess.run(["nm", "-D", "--undefined-only", path], capture_output=True,
                         text=True, check=True).stdout
    used = {line.split()[-1] for line in out.splitlines()}
    boundary = {s for s in used if s.startswith(("moonlight_", "fm_"))}
    assert boundary == CHAT_SYMBOLS, sorted(boundary ^ CHAT_SYMBOLS)
    assert boundary <= exported
    run = subprocess.run([path, "--help"], capture_output=True, text=True, timeout=60)
    assert run.returncode == 0, run.stderr
    assert "floyd run --model DIR --prompt TEXT" in run.stdout
