"""ctypes binding of libcellm_hip.so (the C ABI declared in include/cellm_hip.h).

Loading fails loudly when the library is missing: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libcellm_hip.so"

OK = 0
ERR_INVALID_ARG = -1
ERR_DEVICE = -2
ERR_OUT_OF_MEMORY = -3
ERR_NOT_FOUND = -4
ERR_UNSUPPORTED = -5

DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2

_vp, _sz, _i32, _i64 = C.c_void_p, C.c_size_t, C.c_int32, C.c_int64

OP_QGEMV_I8, OP_QGEMV_Q4_AFFINE, OP_QGEMV_F16, OP_QGEMV_I2, OP_QGEMV_Q1_0_G128, OP_QGEMV_I4_SYM = 0, 1, 2, 3, 4, 5


class QgemvOp(C.Structure):
    """cellm_hip_qgemv_op_t (include/cellm_hip.h)."""
    _fields_ = [("kind", _i32), ("sb_dtype", _i32), ("x_dtype", _i32), ("group", _i32), ("w", _vp), ("scales", _vp),
                ("biases", _vp), ("n_scales", _i64), ("x", _vp), ("bias", _vp), ("y", _vp), ("m", _i64), ("n", _i64),
                ("k", _i64)]

# name -> (restype, argtypes); the same set include/cellm_hip.h declares
SIGNATURES = {
    "cellm_hip_last_error_message": (_sz, [C.c_char_p, _sz]),
    "cellm_hip_device_count": (_i32, [C.POINTER(_i32)]),
    "cellm_hip_smoke_test": (_i32, [_i32]),
    "cellm_hip_create": (_i32, [_i32, C.POINTER(_vp)]),
    "cellm_hip_destroy": (None, [_vp]),
    "cellm_hip_synchronize": (_i32, [_vp]),
    "cellm_hip_get_stream": (_i32, [_vp, C.POINTER(_vp)]),
    "cellm_hip_weight_upload": (_i32, [_vp, C.c_char_p, _vp, _sz, C.POINTER(_vp)]),
    "cellm_hip_weight_lookup": (_i32, [_vp, C.c_char_p, C.POINTER(_vp), C.POINTER(_sz)]),
    "cellm_hip_weight_evict": (_i32, [_vp, C.c_char_p]),
    "cellm_hip_weight_cache_stats": (_i32, [_vp, C.POINTER(_sz), C.POINTER(_sz)]),
    "cellm_hip_qgemv_i8": (_i32, [_vp, _vp, _vp, _i32, _i64, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _vp]),
    "cellm_hip_qgemv_q4_affine": (_i32, [_vp, _vp, _vp, _vp, _i32, _i64, _vp, _i32, _vp, _i64, _i64, _i64, _vp]),
    "cellm_hip_qgemv_batch": (_i32, [_vp, C.POINTER(QgemvOp), _i64, _vp]),
    "cellm_hip_qgemv_i8_qkv": (_i32, [_vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i32, _vp,
                                      _i32, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "cellm_hip_qgemv_q4_affine_qkv": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32,
                                             _i64, _vp, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "cellm_hip_qgemv_i8_gate_up_silu": (_i32, [_vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i32, _vp, _i32, _vp,
                                               _i64, _i64, _i64, _vp]),
    "cellm_hip_qgemv_q4_affine_gate_up_silu": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _vp, _i32, _vp,
                                                      _i64, _i64, _i64, _vp]),
    "cellm_hip_qgemv_i8_gate_up_gelu": (_i32, [_vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _i32, _vp, _i32, _vp,
                                               _i64, _i64, _i64, _vp]),
    "cellm_hip_qgemv_q4_affine_gate_up_gelu": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _vp, _i32, _vp,
                                                      _i64, _i64, _i64, _vp]),
    "cellm_hip_qgemv_i4_gate_up_gelu": (_i32, [_vp, _vp, _vp, _i64, _vp, _vp, _i64, _i64, _vp, _i32, _vp, _i64, _i64,
                                               _i64, _vp]),
    "cellm_hip_qgemv_i4_sym": (_i32, [_vp, _vp, _vp, _i64, _i64, _vp, _i32, _vp, _i64, _i64, _i64, _vp]),
    "cellm_hip_qgemm_q4_affine": (_i32, [_vp, _vp, _vp, _vp, _i32, _i64, _vp, _vp, _i64, _i64, _i64, _vp]),
    "cellm_hip_qgemm_i8": (_i32, [_vp, _vp, _vp, _i32, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "cellm_hip_dequant_q4_affine": (_i32, [_vp, _vp, _vp, _vp, _i32, _i64, _vp, _i32, _i64, _i64, _vp]),
    "cellm_hip_logits_i8": (_i32, [_vp, _vp, _vp, _vp, _sz, _sz, C.c_char_p, _vp]),
    "cellm_hip_logits_i4": (_i32, [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, C.c_char_p, _vp]),
    "cellm_hip_logits_q4_affine": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _sz, _sz, C.c_char_p, _vp]),
    "cellm_hip_embed_i8": (_i32, [_vp, _vp, _i64, _vp, _vp, _i64, _i64, _vp, _vp]),
    "cellm_hip_embed_f16": (_i32, [_vp, _vp, _i64, _vp, _i64, _i64, _vp, _vp]),
    "cellm_hip_embed_i4": (_i32, [_vp, _vp, _i64, _vp, _vp, _i64, _i64, _vp, _vp]),
    "cellm_hip_rms_norm": (_i32, [_vp, _vp, _vp, _i32, _i64, _i64, C.c_float, _vp, _vp]),
    "cellm_hip_qgemv_f16": (_i32, [_vp, _vp, _vp, _i32, _vp, _i64, _i64, _i64, _vp]),
    "cellm_hip_qgemv_i2": (_i32, [_vp, _vp, _vp, _i32, _vp, _i32, _vp, _i64, _i64, _i64, _vp]),
    "cellm_hip_qgemv_q1_0_g128": (_i32, [_vp, _vp, _vp, _i32, _vp, _i64, _i64, _i64, _vp]),
    "cellm_hip_upload_cellm_file": (_i32, [_vp, _vp, C.c_char_p, _vp, _vp]),
    "cellm_hip_linear_file": (_i32, [_vp, _vp, C.c_char_p, _i32, _vp, _vp, _i64, _i64, _i64, _vp]),
    "cellm_hip_decode_qkv_rope_kv": (_i32, [_vp, _vp, _vp, _vp, _vp, C.c_float, _vp, _vp, _vp, _vp, _vp, _vp, _i64,
                                            _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64,
                                            _i64, _i64, _i64, _vp]),
    "cellm_hip_decode_gate_up_silu": (_i32, [_vp, _vp, _vp, _vp, _vp, C.c_float, _vp, _vp, _vp, _vp, _i64, _i64,
                                             _i64, _vp, _vp]),
    "cellm_hip_decode_q4_affine_qkv_rope_kv": (_i32, [_vp, _vp, _vp, _vp, _vp, C.c_float, _vp, _vp, _vp, _vp, _vp, _vp,
                                                     _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64,
                                                     _i64, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64,
                                                     _i64, _i64, _i64, _vp]),
    "cellm_hip_decode_q4_affine_gate_up_silu": (_i32, [_vp, _vp, _vp, _vp, _vp, C.c_float, _vp, _vp, _vp, _vp, _vp,
                                                      _vp, _i32, _i64, _i64, _i64, _i64, _vp, _vp]),
    "cellm_hip_add_rms_norm": (_i32, [_vp, _vp, _vp, _vp, _i32, _i64, _i64, C.c_float, _vp, _vp]),
    "cellm_hip_rope_half_f32": (_i32, [_vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _vp]),
    "cellm_hip_rope_interleaved_f32": (_i32, [_vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _vp]),
    "cellm_hip_set_rope_interleaved": (_i32, [_vp, _i32]),
    "cellm_hip_rope_kv_write_f16": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _vp,
                                           _i64, _i64, _i64, _i64, _i64, _vp]),
    "cellm_hip_kv_write_f16": (_i32, [_vp, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                      _vp]),
    "cellm_hip_attention_gqa_f16kv": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _i64,
                                             _i64, _i64, C.c_float, C.c_float, _vp, _vp]),
    "cellm_hip_attention_gqa_f16kv_window": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i64,
                                                    _i64, _i64, _i64, C.c_float, C.c_float, _i64, _vp, _vp]),
    "cellm_hip_attention_gqa_f16kv_noalloc": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _i64,
                                                     _i64, _i64, _i64, C.c_float, C.c_float, _vp, _vp]),
    "cellm_hip_silu_mul_f32": (_i32, [_vp, _vp, _vp, _i64, _vp]),
    "cellm_hip_gelu_tanh_mul_f32": (_i32, [_vp, _vp, _vp, _i64, _vp]),
    "cellm_hip_add_f32_inplace": (_i32, [_vp, _vp, _vp, _i64, _vp]),
    "cellm_hip_argmax_f32": (_i32, [_vp, _vp, _i64, _i64, _vp, _vp, _vp]),
    "cellm_hip_argmax_f32_keys": (_i32, [_vp, _vp, _i64, _i64, _vp, _vp]),
    "cellm_hip_argmax_key_index": (_i32, [C.c_uint64]),
    "cellm_hip_argmax_key_value": (C.c_float, [C.c_uint64]),
}

_lib = None


class CellmHipError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"cellm_hip error {code}: {message}")
        self.code = code


def load(path: str | os.PathLike | None = None) -> C.CDLL:
    """Load libcellm_hip.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise ImportError(f"{p} is missing: build it with `python -m cellm_amd.build` "
                          "(there is no CPU fallback for the HIP path)")
    lib = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    """Takes the calling thread's last error message (it is cleared, as
    cellm_last_error_message does, crates/cellm-sdk/src/ffi.rs:126-138)."""
    lib = load()
    buf = C.create_string_buffer(2048)
    n = lib.cellm_hip_last_error_message(buf, len(buf))
    return buf.raw[:n].decode(errors="replace")


def check(rc: int) -> None:
    if rc != OK:
        raise CellmHipError(rc, last_error())
