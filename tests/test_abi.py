"""The C-ABI library loads, exports what include/cellm_hip.h declares, and
reports errors without a GPU (no compute calls here)."""
from __future__ import annotations

import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "cellm_hip.h"


def declared_symbols(header: Path = HEADER, prefix: str = "cellm_hip_") -> set[str]:
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(" + prefix + r"\w+)\s*\(", text))


def test_library_exports_the_cellm_file_api():
    from cellm_amd import _lib

    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True)
    exported = set(re.findall(r"\bT (cellm_file_\w+)", out.stdout))
    declared = declared_symbols(prefix="cellm_file_")
    assert declared and declared <= exported, sorted(declared - exported)


def test_library_exports_every_declared_symbol():
    from cellm_amd import _lib

    lib_path = _lib.LIB_PATH
    assert lib_path.exists(), "libcellm_hip.so not built"
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib_path)], capture_output=True, text=True, check=True)
    exported = set(re.findall(r"\bT (cellm_hip_\w+)", out.stdout))
    declared = declared_symbols()
    assert declared, "no declarations parsed"
    missing = declared - exported
    assert not missing, f"declared but not exported: {sorted(missing)}"
    # the ctypes binding covers the same set
    assert declared == set(_lib.SIGNATURES), set(_lib.SIGNATURES) ^ declared


def test_library_loads_and_binds():
    from cellm_amd import _lib

    lib = _lib.load()
    for name in _lib.SIGNATURES:
        assert hasattr(lib, name)


def test_error_reporting_without_device():
    """Null-context calls fail with INVALID_ARG and set the thread's message."""
    from cellm_amd import _lib

    lib = _lib.load()
    rc = lib.cellm_hip_synchronize(None)
    assert rc == _lib.ERR_INVALID_ARG
    assert "null context" in _lib.last_error()
    # message length query with a NULL buffer
    n = lib.cellm_hip_last_error_message(None, 0)
    assert n == len("null context")
    # truncation keeps a NUL terminator
    buf = C.create_string_buffer(5)
    lib.cellm_hip_last_error_message(buf, 5)
    assert buf.value == b"null"


def test_null_out_pointers_rejected():
    from cellm_amd import _lib

    lib = _lib.load()
    assert lib.cellm_hip_device_count(None) == _lib.ERR_INVALID_ARG
    assert lib.cellm_hip_create(0, None) == _lib.ERR_INVALID_ARG


def test_product_fails_loudly_without_library(tmp_path):
    """There is no CPU fallback: loading a missing library raises."""
    from cellm_amd import _lib

    saved = _lib._lib
    try:
        _lib._lib = None
        with pytest.raises(ImportError, match="no CPU fallback"):
            _lib.load(tmp_path / "missing.so")
    finally:
        _lib._lib = saved


def test_product_does_not_import_oracle():
    """Nothing in the package or bench's product leg links the oracle."""
    pkg = ROOT / "cellm_amd"
    for p in list(pkg.rglob("*.py")) + list(pkg.rglob("*.cpp")) + list(pkg.rglob("*.hip")) + list(pkg.rglob("*.hpp")):
        text = p.read_text()
        assert "import oracle" not in text and "from oracle" not in text and "liboracle" not in text, p


def test_step_library_exports_its_header():
    from cellm_amd import build

    assert build.STEP_LIB_PATH.exists(), "libcellm_llama_step.so not built"
    out = subprocess.run(["nm", "-D", "--defined-only", str(build.STEP_LIB_PATH)], capture_output=True, text=True,
                         check=True)
    exported = set(re.findall(r"\bT (cellm_llama_\w+)", out.stdout))
    declared = declared_symbols(ROOT / "include" / "cellm_llama_step.h", "cellm_llama_")
    assert declared and not (declared - exported), sorted(declared - exported)


def test_every_header_is_checked():
    headers = {p.name for p in (ROOT / "include").glob("*.h")}
    assert headers == {"cellm_hip.h", "cellm_llama_step.h"}, headers
