"""Host-side argument checks of the sync logits_* wrappers (no GPU): short or
mismatched host arrays are refused in Python before the C ABI copies
rows*cols bytes out of them, and a wrong `out` is refused before results are
copied into it."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest


class _Unreachable:
    """Stands in for the C library: any call means a check was skipped."""

    def __getattr__(self, name):
        raise AssertionError(f"{name} reached the C ABI with bad arguments")


@pytest.fixture()
def ops():
    from cellm_amd.hipops import HipOps

    o = HipOps.__new__(HipOps)  # no device context: every case must fail before the C call
    o._lib = _Unreachable()
    o._h = C.c_void_p()
    return o


def _q4(rows=16, cols=128, dt=np.float16):
    g = (cols + 63) // 64
    return (np.zeros(cols, np.float32), np.zeros((rows, cols // 8), np.uint32), np.ones((rows, g), dt),
            np.zeros((rows, g), dt))


def test_q4_short_arrays_rejected(ops):
    x, wq, s, b = _q4()
    with pytest.raises(ValueError):
        ops.logits_q4_affine(x[:-8], wq, s, b, 16, 128, "k")
    with pytest.raises(ValueError):
        ops.logits_q4_affine(x, wq[:-1], s, b, 16, 128, "k")
    with pytest.raises(ValueError):
        ops.logits_q4_affine(x, wq, s[:-1], b, 16, 128, "k")
    with pytest.raises(ValueError):
        ops.logits_q4_affine(x, wq, s, b[:-1], 16, 128, "k")
    with pytest.raises(ValueError):
        ops.logits_q4_affine(x, wq, s, b, 16, 120, "k")  # cols % 8 == 0 but the arrays are for 128


def test_q4_bias_dtype_must_match_scales(ops):
    """float32 biases beside bf16-bit scales are not silently reinterpreted."""
    x, wq, s, _ = _q4(dt=np.uint16)
    b = np.zeros(s.shape, np.float32)
    with pytest.raises(TypeError, match="biases dtype"):
        ops.logits_q4_affine(x, wq, s, b, 16, 128, "k")


@pytest.mark.parametrize("bad", [np.empty(15, np.float32), np.empty(16, np.float64), np.empty((16, 2), np.float32)[:, 0]])
def test_out_must_be_float32_of_rows(ops, bad):
    x, wq, s, b = _q4()
    with pytest.raises(ValueError, match="out must be"):
        ops.logits_q4_affine(x, wq, s, b, 16, 128, "k", out=bad)
    with pytest.raises(ValueError, match="out must be"):
        ops.logits_i8(np.zeros(64, np.float32), np.zeros((16, 64), np.int8), np.zeros(16, np.uint16), 16, 64, "k",
                      out=bad)
    with pytest.raises(ValueError, match="out must be"):
        ops.logits_i4(np.zeros(64, np.float32), np.zeros((16, 32), np.uint8), np.zeros(16, np.uint16), 16, 64, 64,
                      "k", out=bad)


def test_i8_i4_shape_checks(ops):
    with pytest.raises(ValueError):
        ops.logits_i8(np.zeros(64, np.float32), np.zeros((16, 64), np.int8), np.zeros(15, np.uint16), 16, 64, "k")
    with pytest.raises(ValueError):
        ops.logits_i4(np.zeros(64, np.float32), np.zeros((16, 31), np.uint8), np.zeros(16, np.uint16), 16, 64, 64,
                      "k")
    with pytest.raises(ValueError):  # gs = 32 needs two scales per row
        ops.logits_i4(np.zeros(64, np.float32), np.zeros((16, 32), np.uint8), np.zeros(16, np.uint16), 16, 64, 32,
                      "k")
