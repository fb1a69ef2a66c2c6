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


def test_last_error_message_follows_the_reference_ffi():
    """cellm_last_error_message (crates/cellm-sdk/src/ffi.rs:126-138): a NULL
    or empty buffer returns 0 and leaves the message; otherwise the message is
    taken, truncated to buf_len - 1 bytes plus NUL, and the bytes written are
    returned."""
    from cellm_amd import _lib

    lib = _lib.load()
    assert lib.cellm_hip_synchronize(None) == _lib.ERR_INVALID_ARG
    assert lib.cellm_hip_last_error_message(None, 0) == 0
    assert lib.cellm_hip_last_error_message(C.create_string_buffer(8), 0) == 0
    buf = C.create_string_buffer(5)
    assert lib.cellm_hip_last_error_message(buf, 5) == 4  # "null" + NUL
    assert buf.value == b"null"
    # taken: a second read finds nothing
    buf = C.create_string_buffer(64)
    assert lib.cellm_hip_last_error_message(buf, 64) == 0 and buf.value == b""
    # a full read returns the whole message
    assert lib.cellm_hip_synchronize(None) == _lib.ERR_INVALID_ARG
    assert lib.cellm_hip_last_error_message(buf, 64) == len("null context") and buf.value == b"null context"


def test_messages_are_per_thread():
    """Each thread reads its own last error."""
    import threading

    from cellm_amd import _lib

    lib = _lib.load()
    assert lib.cellm_hip_device_count(None) == _lib.ERR_INVALID_ARG
    seen = {}

    def other():
        assert lib.cellm_hip_synchronize(None) == _lib.ERR_INVALID_ARG
        seen["other"] = _lib.last_error()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["other"] == "null context"
    assert _lib.last_error() == "null out_count"


def test_exception_guard_turns_throws_into_status(tmp_path):
    """The guard every entry point runs in (cellm_amd/csrc/api_guard.hpp):
    std::bad_alloc becomes CELLM_HIP_ERR_OUT_OF_MEMORY, any other exception
    CELLM_HIP_ERR_DEVICE with its message, and nothing propagates (the
    reference catches panics at its FFI, crates/cellm-sdk/src/ffi.rs:142).
    Built and run as a small host program."""
    src = tmp_path / "guard.cpp"
    src.write_text(r"""
#include <cstdio>
#include <stdexcept>
#include <string>
#include <vector>
#include "cellm_hip.h"
#include "api_guard.hpp"
static cellm::ErrorSlot slot = {};
static int32_t report(int32_t code, const char* what) { slot.store(what, strlen(what)); return code; }
static int32_t oom() { CELLM_API_BEGIN std::vector<char> v((size_t)1 << 62); return v.empty() ? 1 : 0; CELLM_API_END(report) }
static int32_t rt() { CELLM_API_BEGIN throw std::runtime_error("boom"); CELLM_API_END(report) }
static int32_t other() { CELLM_API_BEGIN throw 7; CELLM_API_END(report) }
static void vfn(int* hit) { CELLM_API_BEGIN *hit = 1; throw std::string("x"); CELLM_API_END_VOID }
int main() {
    char buf[64];
    if (oom() != CELLM_HIP_ERR_OUT_OF_MEMORY) return 1;
    if (rt() != CELLM_HIP_ERR_DEVICE) return 2;
    slot.take(buf, sizeof buf);
    if (std::string(buf) != "boom") return 3;
    if (other() != CELLM_HIP_ERR_DEVICE) return 4;
    int hit = 0;
    vfn(&hit);
    return hit == 1 ? 0 : 5;
}
""")
    exe = tmp_path / "guard"
    subprocess.run(["g++", "-std=c++17", f"-I{ROOT / 'include'}", f"-I{ROOT / 'cellm_amd' / 'csrc'}", str(src), "-o",
                    str(exe)], check=True)
    assert subprocess.run([str(exe)]).returncode == 0


def _extern_c_bodies(path):
    """(name, first body line) of every multi-line extern "C" definition."""
    lines = path.read_text().split("\n")
    out, in_c = [], False
    for i, ln in enumerate(lines):
        if ln.startswith('extern "C" {'):
            in_c = True
        elif ln.startswith('}  // extern "C"'):
            in_c = False
        m = re.match(r"^(?:int32_t|void|int64_t|size_t) (cellm_\w+)\(", ln) if in_c else None
        if m and not ln.rstrip().endswith("}"):
            j = i
            while lines[j] != "{":
                j += 1
            out.append((m.group(1), lines[j + 1].strip()))
    return out


def test_every_entry_point_is_guarded():
    """Every multi-line extern "C" body of the library opens with the guard."""
    srcs = [ROOT / "cellm_amd" / "csrc" / f for f in ("capi.cpp", "cellm_file.cpp", "llama_device.cpp",
                                                      "llama_step.cpp")]
    bodies = [b for p in srcs for b in _extern_c_bodies(p)]
    assert len(bodies) > 40
    unguarded = [n for n, first in bodies if first != "CELLM_API_BEGIN"]
    assert not unguarded, unguarded


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


def test_argmax_key_decoding():
    """cellm_hip_argmax_f32_keys keys decode as documented (high word: f32 bits in unsigned order,
    non-negative values with the sign bit set, negative ones inverted; low word: 0xffffffff - index),
    in the library and in the Python helper alike; the order of such keys is the order of the
    values, then of the lower index."""
    from cellm_amd import _lib
    from cellm_amd.hipops import argmax_key_index, argmax_key_value

    lib = _lib.load()
    cases = [  # (key, value, index)
        ((0xBF800000 << 32) | 0xFFFFFFFA, 1.0, 5),              # 1.0 = 0x3f800000 | sign bit
        ((0x3FFFFFFF << 32) | 0xFFFFFFFF, -2.0, 0),             # -2.0 = 0xc0000000, inverted
        ((0x007FFFFF << 32) | 0x00000000, float("-inf"), 0xFFFFFFFF),  # -inf = 0xff800000, inverted
        ((0x80000000 << 32) | 0xFFFF0000, 0.0, 0xFFFF),         # +0 (and -0, taken as +0)
        ((0xFF7FFFFF << 32) | 0xFFFFFF00, 3.4028234663852886e38, 0xFF),  # largest finite f32
    ]
    for key, val, idx in cases:
        want_idx = idx - (1 << 32) if idx >= 1 << 31 else idx
        assert lib.cellm_hip_argmax_key_index(key) == want_idx
        assert lib.cellm_hip_argmax_key_value(key) == val
        assert argmax_key_index(key) == idx
        assert argmax_key_value(key) == val
    # ordering: values ascending give keys ascending; at equal values the lower index gives the larger key
    ordered = sorted(cases[:4], key=lambda c: c[0])
    assert [c[1] for c in ordered] == sorted(c[1] for c in cases[:4])
    assert ((0xBF800000 << 32) | (0xFFFFFFFF - 3)) > ((0xBF800000 << 32) | (0xFFFFFFFF - 4))
