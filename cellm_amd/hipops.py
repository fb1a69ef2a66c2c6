"""HipOps: the host-side mirror of cellm's MetalOps over libcellm_hip.so.

Method names and argument meaning follow MetalOps
(crates/cellm-kernels/src/metal.rs): `logits_*` take host arrays and a cache
key and return host results (metal.rs:1017-1204); `encode_*` take device
tensors and queue work on a stream (metal.rs:813-1176).  Errors raise
CellmHipError, the analogue of the anyhow::Result the Rust methods return.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import DTYPE_BF16, DTYPE_F16, DTYPE_F32, check

_NP_DT = {np.dtype(np.float32): DTYPE_F32, np.dtype(np.float16): DTYPE_F16}


def _np_ptr(a: np.ndarray):
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("arrays passed to HipOps must be C-contiguous")
    return a.ctypes.data_as(C.c_void_p)


def _torch_dtype_code(t) -> int:
    import torch

    if t.dtype == torch.float32:
        return DTYPE_F32
    if t.dtype == torch.float16:
        return DTYPE_F16
    if t.dtype == torch.bfloat16:
        return DTYPE_BF16
    raise TypeError(f"unsupported tensor dtype {t.dtype}")


def _dev_ptr(t):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("encode_* expects device tensors")
    if not t.is_contiguous():
        raise ValueError("encode_* expects contiguous tensors")
    return C.c_void_p(t.data_ptr())


def _stream_ptr(stream):
    if stream is None:
        return None
    if isinstance(stream, int):
        return C.c_void_p(stream)
    return C.c_void_p(stream.cuda_stream)


def argmax_key_index(key: int) -> int:
    """Index of a cellm_hip_argmax_f32_keys key (the low word holds 0xffffffff - index)."""
    return 0xFFFFFFFF - (int(key) & 0xFFFFFFFF)


def argmax_key_value(key: int) -> float:
    """Value of a cellm_hip_argmax_f32_keys key (the high word holds the f32 bits in unsigned order)."""
    o = (int(key) >> 32) & 0xFFFFFFFF
    u = (o & 0x7FFFFFFF) if o & 0x80000000 else (~o & 0xFFFFFFFF)
    return float(np.array([u], np.uint32).view(np.float32)[0])


def device_count() -> int:
    lib = _lib.load()
    n = C.c_int32(0)
    check(lib.cellm_hip_device_count(C.byref(n)))
    return n.value


def smoke_test(device: int = 0) -> None:
    """MetalKernels::smoke_test_add_f32 analogue (metal.rs:33-93)."""
    check(_lib.load().cellm_hip_smoke_test(device))


class HipOps:
    """One device context: stream, name-keyed weight cache, scratch buffers."""

    def __init__(self, device: int = 0):
        self._lib = _lib.load()
        h = C.c_void_p()
        check(self._lib.cellm_hip_create(device, C.byref(h)))
        self._h = h
        self.device = device

    @classmethod
    def create(cls, device: int = 0) -> "HipOps":
        return cls(device)

    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            self._lib.cellm_hip_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def handle(self):
        return self._h

    def synchronize(self) -> None:
        check(self._lib.cellm_hip_synchronize(self._h))

    def stream(self) -> int:
        s = C.c_void_p()
        check(self._lib.cellm_hip_get_stream(self._h, C.byref(s)))
        return s.value or 0

    # -- weight cache -------------------------------------------------------------
    def weight_upload(self, key: str, host: np.ndarray) -> int:
        out = C.c_void_p()
        check(self._lib.cellm_hip_weight_upload(self._h, key.encode(), _np_ptr(host), host.nbytes, C.byref(out)))
        return out.value

    def weight_lookup(self, key: str):
        out, nb = C.c_void_p(), C.c_size_t()
        check(self._lib.cellm_hip_weight_lookup(self._h, key.encode(), C.byref(out), C.byref(nb)))
        return out.value, nb.value

    def weight_evict(self, key: str) -> None:
        check(self._lib.cellm_hip_weight_evict(self._h, key.encode()))

    def weight_cache_stats(self):
        e, b = C.c_size_t(), C.c_size_t()
        check(self._lib.cellm_hip_weight_cache_stats(self._h, C.byref(e), C.byref(b)))
        return e.value, b.value

    # -- sync: MetalOps::logits_* -----------------------------------------------
    @staticmethod
    def _out_f32(out, rows: int, what: str) -> np.ndarray:
        if out is None:
            return np.empty(rows, np.float32)
        if not isinstance(out, np.ndarray) or out.dtype != np.float32 or out.size != rows or \
                not out.flags["C_CONTIGUOUS"]:
            raise ValueError(f"{what}: out must be a C-contiguous float32 array of {rows} elements")
        return out

    def logits_i8(self, x: np.ndarray, w_i8: np.ndarray, scales_f16_bits: np.ndarray, vocab: int, hidden: int,
                  cache_key: str, out: np.ndarray | None = None) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w_i8, np.int8)
        s = np.ascontiguousarray(scales_f16_bits, np.uint16)
        if x.size != hidden or w.size != vocab * hidden or s.size != vocab:
            raise ValueError("logits_i8: shape mismatch")
        out = self._out_f32(out, vocab, "logits_i8")
        check(self._lib.cellm_hip_logits_i8(self._h, _np_ptr(x), _np_ptr(w), _np_ptr(s), vocab, hidden,
                                            cache_key.encode(), _np_ptr(out)))
        return out

    def logits_i4(self, x: np.ndarray, w_u8: np.ndarray, scales_f16_bits: np.ndarray, vocab: int, hidden: int,
                  gs: int, cache_key: str, out: np.ndarray | None = None) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w_u8, np.uint8)
        s = np.ascontiguousarray(scales_f16_bits, np.uint16)
        if x.size != hidden or w.size != vocab * ((hidden + 1) // 2):
            raise ValueError("logits_i4: shape mismatch")
        if gs < 1 or vocab < 1 or s.size < vocab * (((hidden - 1) // gs + 1) if hidden else 1):
            raise ValueError("logits_i4: need gs >= 1 and ceil(hidden / gs) f16 scales per row")
        out = self._out_f32(out, vocab, "logits_i4")
        check(self._lib.cellm_hip_logits_i4(self._h, _np_ptr(x), _np_ptr(w), _np_ptr(s), s.size, vocab, hidden, gs,
                                            cache_key.encode(), _np_ptr(out)))
        return out

    def logits_q4_affine(self, x: np.ndarray, wq: np.ndarray, scales: np.ndarray, biases: np.ndarray, rows: int,
                         cols: int, cache_key: str, out: np.ndarray | None = None) -> np.ndarray:
        """The LFM affine linear (lfm.rs:985-1066) from host arrays: x [cols],
        wq u32 [rows, cols/8], scales/biases [rows, ceil(cols/64)] of one dtype
        (float32, float16, or uint16 holding bf16 bits)."""
        x = np.ascontiguousarray(x, np.float32)
        wq = np.ascontiguousarray(wq, np.uint32)
        scales = np.ascontiguousarray(scales)
        biases = np.ascontiguousarray(biases)
        if biases.dtype != scales.dtype:
            raise TypeError(f"logits_q4_affine: biases dtype {biases.dtype} differs from scales {scales.dtype}")
        dt = _NP_DT.get(scales.dtype, DTYPE_BF16 if scales.dtype == np.uint16 else None)
        if dt is None:
            raise TypeError(f"unsupported scale dtype {scales.dtype}")
        groups = (cols + 63) // 64
        if rows < 0 or cols < 0 or cols % 8 != 0 or x.size != cols or wq.size * 8 != rows * cols or \
                scales.size != rows * groups or biases.size != rows * groups:
            raise ValueError("logits_q4_affine: shape mismatch (x [cols], wq [rows, cols/8], scales/biases "
                             "[rows, ceil(cols/64)], cols % 8 == 0)")
        out = self._out_f32(out, rows, "logits_q4_affine")
        check(self._lib.cellm_hip_logits_q4_affine(self._h, _np_ptr(x), _np_ptr(wq), _np_ptr(scales), _np_ptr(biases),
                                                   dt, rows, cols, cache_key.encode(), _np_ptr(out)))
        return out

    # -- async: MetalOps::encode_* over torch device tensors ------------------------
    def encode_qgemv_i8(self, w, scales, x, y, bias=None, stream=None) -> None:
        """y[m,n] = (W[n,:] . x[m,:]) * s[n] (+ bias[n]); W int8 [n,k]."""
        n, k = w.shape
        m = x.numel() // k
        check(self._lib.cellm_hip_qgemv_i8(self._h, _dev_ptr(w), _dev_ptr(scales), _torch_dtype_code(scales),
                                           scales.numel(), _dev_ptr(x), _torch_dtype_code(x), _dev_ptr(bias),
                                           _dev_ptr(y), m, n, k, _stream_ptr(stream)))

    def encode_qgemv_q4_affine(self, wq, scales, biases, x, y, group: int = 64, stream=None) -> None:
        """MLX affine; wq int32/uint32 words [n, k/8], scales/biases [n, ceil(k/group)]."""
        n = wq.shape[0]
        k = wq.shape[1] * 8
        m = x.numel() // k
        check(self._lib.cellm_hip_qgemv_q4_affine(self._h, _dev_ptr(wq), _dev_ptr(scales), _dev_ptr(biases),
                                                  _torch_dtype_code(scales), group, _dev_ptr(x), _torch_dtype_code(x),
                                                  _dev_ptr(y), m, n, k, _stream_ptr(stream)))

    def encode_qkv_i8(self, wq, sq, wk, sk, wv, sv, x, q, k_out, v, bq=None, bk=None, bv=None,
                      stream=None) -> None:
        """MetalOps::encode_qkv_i8(_bias): three int8 projections of one x in one launch."""
        rows_q, cols = wq.shape
        rows_kv = wk.shape[0]
        m = x.numel() // cols
        if sq.dtype != sk.dtype or sq.dtype != sv.dtype:
            raise TypeError("q/k/v scales must share a dtype")
        check(self._lib.cellm_hip_qgemv_i8_qkv(
            self._h, _dev_ptr(wq), _dev_ptr(sq), sq.numel(), _dev_ptr(bq), _dev_ptr(wk), _dev_ptr(sk), sk.numel(),
            _dev_ptr(bk), _dev_ptr(wv), _dev_ptr(sv), sv.numel(), _dev_ptr(bv), _torch_dtype_code(sq), _dev_ptr(x),
            _torch_dtype_code(x), _dev_ptr(q), _dev_ptr(k_out), _dev_ptr(v), m, rows_q, rows_kv, cols,
            _stream_ptr(stream)))

    def encode_qkv_q4_affine(self, wq, sq, bq, wk, sk, bk, wv, sv, bv, x, q, k_out, v, biasq=None, biask=None,
                             biasv=None, group: int = 64, stream=None) -> None:
        """Three MLX q4 affine projections of one x (f16 or f32) in one launch, each with an
        optional f32 projection bias added after the row sum (cellm_hip_qgemv_q4_affine_qkv)."""
        rows_q, cols = wq.shape[0], wq.shape[1] * 8
        rows_kv = wk.shape[0]
        m = x.numel() // cols
        if not (sq.dtype == sk.dtype == sv.dtype == bq.dtype == bk.dtype == bv.dtype):
            raise TypeError("q/k/v scales and group biases must share a dtype")
        check(self._lib.cellm_hip_qgemv_q4_affine_qkv(
            self._h, _dev_ptr(wq), _dev_ptr(sq), _dev_ptr(bq), _dev_ptr(biasq), _dev_ptr(wk), _dev_ptr(sk),
            _dev_ptr(bk), _dev_ptr(biask), _dev_ptr(wv), _dev_ptr(sv), _dev_ptr(bv), _dev_ptr(biasv),
            _torch_dtype_code(sq), group, _dev_ptr(x), _torch_dtype_code(x), _dev_ptr(q), _dev_ptr(k_out),
            _dev_ptr(v), m, rows_q, rows_kv, cols, _stream_ptr(stream)))

    def encode_gate_up_silu_i8(self, wg, sg, wu, su, x, h, bg=None, bu=None, stream=None) -> None:
        """h = silu(Wg.x * sg (+bg)) * (Wu.x * su (+bu)); int8 gate/up."""
        n, k = wg.shape
        m = x.numel() // k
        if sg.dtype != su.dtype:
            raise TypeError("gate/up scales must share a dtype")
        check(self._lib.cellm_hip_qgemv_i8_gate_up_silu(
            self._h, _dev_ptr(wg), _dev_ptr(sg), sg.numel(), _dev_ptr(bg), _dev_ptr(wu), _dev_ptr(su), su.numel(),
            _dev_ptr(bu), _torch_dtype_code(sg), _dev_ptr(x), _torch_dtype_code(x), _dev_ptr(h), m, n, k,
            _stream_ptr(stream)))

    def encode_gate_up_silu_q4_affine(self, wg, sg, bg, wu, su, bu, x, h, group: int = 64, stream=None) -> None:
        """h = silu(dequant(Wg).x) * (dequant(Wu).x); MLX 4-bit affine gate/up."""
        n, k = wg.shape[0], wg.shape[1] * 8
        m = x.numel() // k
        check(self._lib.cellm_hip_qgemv_q4_affine_gate_up_silu(
            self._h, _dev_ptr(wg), _dev_ptr(sg), _dev_ptr(bg), _dev_ptr(wu), _dev_ptr(su), _dev_ptr(bu),
            _torch_dtype_code(sg), group, _dev_ptr(x), _torch_dtype_code(x), _dev_ptr(h), m, n, k,
            _stream_ptr(stream)))

    def encode_gate_up_gelu_i8(self, wg, sg, wu, su, x, h, bg=None, bu=None, stream=None) -> None:
        """h = gelu_tanh(Wg.x * sg (+bg)) * (Wu.x * su (+bu)); int8 gate/up (Gemma's MLP)."""
        n, k = wg.shape
        m = x.numel() // k
        if sg.dtype != su.dtype:
            raise TypeError("gate/up scales must share a dtype")
        check(self._lib.cellm_hip_qgemv_i8_gate_up_gelu(
            self._h, _dev_ptr(wg), _dev_ptr(sg), sg.numel(), _dev_ptr(bg), _dev_ptr(wu), _dev_ptr(su), su.numel(),
            _dev_ptr(bu), _torch_dtype_code(sg), _dev_ptr(x), _torch_dtype_code(x), _dev_ptr(h), m, n, k,
            _stream_ptr(stream)))

    def encode_gate_up_gelu_q4_affine(self, wg, sg, bg, wu, su, bu, x, h, group: int = 64, stream=None) -> None:
        """h = gelu_tanh(dequant(Wg).x) * (dequant(Wu).x); MLX 4-bit affine gate/up."""
        n, k = wg.shape[0], wg.shape[1] * 8
        m = x.numel() // k
        check(self._lib.cellm_hip_qgemv_q4_affine_gate_up_gelu(
            self._h, _dev_ptr(wg), _dev_ptr(sg), _dev_ptr(bg), _dev_ptr(wu), _dev_ptr(su), _dev_ptr(bu),
            _torch_dtype_code(sg), group, _dev_ptr(x), _torch_dtype_code(x), _dev_ptr(h), m, n, k,
            _stream_ptr(stream)))

    def encode_gate_up_gelu_i4_sym(self, wg, sg_f16, wu, su_f16, gs: int, x, h, k: int, stream=None) -> None:
        """h = gelu_tanh(i4(Wg).x) * (i4(Wu).x); symmetric i4 gate/up [n, ceil(k/2)] bytes, f16 scales."""
        n = wg.shape[0]
        m = x.numel() // k
        check(self._lib.cellm_hip_qgemv_i4_gate_up_gelu(
            self._h, _dev_ptr(wg), _dev_ptr(sg_f16), sg_f16.numel(), _dev_ptr(wu), _dev_ptr(su_f16), su_f16.numel(),
            gs, _dev_ptr(x), _torch_dtype_code(x), _dev_ptr(h), m, n, k, _stream_ptr(stream)))

    @staticmethod
    def qgemv_op_i8(w, scales, x, y, bias=None) -> "_lib.QgemvOp":
        """One cellm_hip_qgemv_op_t of kind int8 (arguments as encode_qgemv_i8)."""
        n, k = w.shape
        return _lib.QgemvOp(kind=_lib.OP_QGEMV_I8, sb_dtype=_torch_dtype_code(scales), x_dtype=_torch_dtype_code(x),
                            group=0, w=_dev_ptr(w), scales=_dev_ptr(scales), biases=None, n_scales=scales.numel(),
                            x=_dev_ptr(x), bias=_dev_ptr(bias), y=_dev_ptr(y), m=x.numel() // k, n=n, k=k)

    @staticmethod
    def qgemv_op_q4_affine(wq, scales, biases, x, y, group: int = 64) -> "_lib.QgemvOp":
        """One cellm_hip_qgemv_op_t of kind q4 affine (arguments as encode_qgemv_q4_affine)."""
        n, k = wq.shape[0], wq.shape[1] * 8
        return _lib.QgemvOp(kind=_lib.OP_QGEMV_Q4_AFFINE, sb_dtype=_torch_dtype_code(scales),
                            x_dtype=_torch_dtype_code(x), group=group, w=_dev_ptr(wq), scales=_dev_ptr(scales),
                            biases=_dev_ptr(biases), n_scales=0, x=_dev_ptr(x), bias=None, y=_dev_ptr(y),
                            m=x.numel() // k, n=n, k=k)

    @staticmethod
    def qgemv_op_f16(w_f16, x, y) -> "_lib.QgemvOp":
        """One cellm_hip_qgemv_op_t of kind f16 (arguments as encode_qgemv_f16)."""
        n, k = w_f16.shape
        return _lib.QgemvOp(kind=_lib.OP_QGEMV_F16, sb_dtype=0, x_dtype=_torch_dtype_code(x), group=0,
                            w=_dev_ptr(w_f16), scales=None, biases=None, n_scales=0, x=_dev_ptr(x), bias=None,
                            y=_dev_ptr(y), m=x.numel() // k, n=n, k=k)

    @staticmethod
    def qgemv_op_i2(w_u8, scales_f16, scale_mode: int, x, y, k: int) -> "_lib.QgemvOp":
        """One cellm_hip_qgemv_op_t of kind i2 (group carries scale_mode)."""
        return _lib.QgemvOp(kind=_lib.OP_QGEMV_I2, sb_dtype=1, x_dtype=_torch_dtype_code(x), group=scale_mode,
                            w=_dev_ptr(w_u8), scales=_dev_ptr(scales_f16), biases=None, n_scales=scales_f16.numel(),
                            x=_dev_ptr(x), bias=None, y=_dev_ptr(y), m=x.numel() // k, n=w_u8.shape[0], k=k)

    @staticmethod
    def qgemv_op_i4_sym(w_u8, scales_f16, gs: int, x, y, k: int) -> "_lib.QgemvOp":
        """One cellm_hip_qgemv_op_t of kind i4_sym (group carries gs)."""
        return _lib.QgemvOp(kind=_lib.OP_QGEMV_I4_SYM, sb_dtype=1, x_dtype=_torch_dtype_code(x), group=gs,
                            w=_dev_ptr(w_u8), scales=_dev_ptr(scales_f16), biases=None, n_scales=scales_f16.numel(),
                            x=_dev_ptr(x), bias=None, y=_dev_ptr(y), m=x.numel() // k, n=w_u8.shape[0], k=k)

    @staticmethod
    def qgemv_op_q1_0_g128(w_u8, x, y, k: int) -> "_lib.QgemvOp":
        """One cellm_hip_qgemv_op_t of kind q1_0_g128."""
        return _lib.QgemvOp(kind=_lib.OP_QGEMV_Q1_0_G128, sb_dtype=0, x_dtype=_torch_dtype_code(x), group=0,
                            w=_dev_ptr(w_u8), scales=None, biases=None, n_scales=0, x=_dev_ptr(x), bias=None,
                            y=_dev_ptr(y), m=x.numel() // k, n=w_u8.shape[0], k=k)

    def encode_qgemv_batch(self, ops, stream=None) -> None:
        """Enqueue a list of qgemv ops (qgemv_op_*) in order with one call; a
        ctypes array built once may be passed again to re-enqueue it."""
        if not isinstance(ops, C.Array):
            ops = (_lib.QgemvOp * len(ops))(*ops)
        check(self._lib.cellm_hip_qgemv_batch(self._h, ops, len(ops), _stream_ptr(stream)))

    def encode_qgemv_i4_sym(self, w_u8, scales_f16, gs: int, x, y, k: int, stream=None) -> None:
        n = w_u8.shape[0]
        m = x.numel() // k
        check(self._lib.cellm_hip_qgemv_i4_sym(self._h, _dev_ptr(w_u8), _dev_ptr(scales_f16), scales_f16.numel(), gs,
                                               _dev_ptr(x), _torch_dtype_code(x), _dev_ptr(y), m, n, k,
                                               _stream_ptr(stream)))

    def encode_qgemv_f16(self, w_f16, x, y, stream=None) -> None:
        """y[m, n] = sum_k f32(W[n, k]) * x[m, k]; W [n][k] float16 (or int16 holding f16 bits)."""
        n, k = w_f16.shape
        check(self._lib.cellm_hip_qgemv_f16(self._h, _dev_ptr(w_f16), _dev_ptr(x), _torch_dtype_code(x), _dev_ptr(y),
                                            x.numel() // k, n, k, _stream_ptr(stream)))

    def encode_qgemv_i2(self, w_u8, scales_f16, scale_mode: int, x, y, k: int, stream=None) -> None:
        """i2 rows of ceil(k/4) bytes, one f16 scale per row; scale_mode 0 = at the end (Qwen), 1 = per element (Gemma)."""
        check(self._lib.cellm_hip_qgemv_i2(self._h, _dev_ptr(w_u8), _dev_ptr(scales_f16), scale_mode, _dev_ptr(x),
                                           _torch_dtype_code(x), _dev_ptr(y), x.numel() // k, w_u8.shape[0], k,
                                           _stream_ptr(stream)))

    def encode_qgemv_q1_0_g128(self, w_u8, x, y, k: int, stream=None) -> None:
        """q1_0_g128 rows of k/128 blocks of 18 bytes."""
        check(self._lib.cellm_hip_qgemv_q1_0_g128(self._h, _dev_ptr(w_u8), _dev_ptr(x), _torch_dtype_code(x),
                                                  _dev_ptr(y), x.numel() // k, w_u8.shape[0], k, _stream_ptr(stream)))

    def encode_qgemm_q4_affine(self, wq, scales, biases, x_f16, y, group: int = 64, stream=None) -> None:
        n = wq.shape[0]
        k = wq.shape[1] * 8
        m = x_f16.numel() // k
        check(self._lib.cellm_hip_qgemm_q4_affine(self._h, _dev_ptr(wq), _dev_ptr(scales), _dev_ptr(biases),
                                                  _torch_dtype_code(scales), group, _dev_ptr(x_f16), _dev_ptr(y), m, n,
                                                  k, _stream_ptr(stream)))

    def encode_qgemm_i8(self, w, scales, x_f16, y, bias=None, stream=None) -> None:
        n, k = w.shape
        m = x_f16.numel() // k
        check(self._lib.cellm_hip_qgemm_i8(self._h, _dev_ptr(w), _dev_ptr(scales), _torch_dtype_code(scales),
                                           scales.numel(), _dev_ptr(x_f16), _dev_ptr(bias), _dev_ptr(y), m, n, k,
                                           _stream_ptr(stream)))

    def encode_dequant_q4_affine(self, wq, scales, biases, out, group: int = 64, stream=None) -> None:
        n = wq.shape[0]
        k = wq.shape[1] * 8
        check(self._lib.cellm_hip_dequant_q4_affine(self._h, _dev_ptr(wq), _dev_ptr(scales), _dev_ptr(biases),
                                                    _torch_dtype_code(scales), group, _dev_ptr(out),
                                                    _torch_dtype_code(out), n, k, _stream_ptr(stream)))

    # ---- decode-step ops (MetalOps::encode_rms_norm_f16w / encode_rope_half_f32 /
    # encode_add_f32_inplace, MetalKvStorage::encode_write_token_f32 / encode_attention)

    def encode_embed_i8(self, tokens_u32, embed_i8, scales_f16, out, stream=None) -> None:
        vocab, hidden = embed_i8.shape
        check(self._lib.cellm_hip_embed_i8(self._h, _dev_ptr(tokens_u32), tokens_u32.numel(), _dev_ptr(embed_i8),
                                           _dev_ptr(scales_f16), vocab, hidden, _dev_ptr(out), _stream_ptr(stream)))

    def encode_embed_f16(self, tokens_u32, embed_f16, out, stream=None) -> None:
        """embed_token's f16 branch (llama.rs:687-693); embed_f16 f16 [vocab, hidden]."""
        vocab, hidden = embed_f16.shape
        check(self._lib.cellm_hip_embed_f16(self._h, _dev_ptr(tokens_u32), tokens_u32.numel(), _dev_ptr(embed_f16),
                                            vocab, hidden, _dev_ptr(out), _stream_ptr(stream)))

    def encode_embed_i4(self, tokens_u32, embed_i4, scales_f16, hidden: int, out, stream=None) -> None:
        """embed_token's i4 branch (llama.rs:703-718); embed_i4 uint8 [vocab, ceil(hidden/2)]."""
        vocab = embed_i4.shape[0]
        if embed_i4.shape[1] != (hidden + 1) // 2:
            raise ValueError(f"embed_i4 rows hold {embed_i4.shape[1]} bytes, hidden {hidden} needs {(hidden + 1) // 2}")
        check(self._lib.cellm_hip_embed_i4(self._h, _dev_ptr(tokens_u32), tokens_u32.numel(), _dev_ptr(embed_i4),
                                           _dev_ptr(scales_f16), vocab, hidden, _dev_ptr(out), _stream_ptr(stream)))

    def encode_rms_norm(self, x, weight, out, eps: float, stream=None) -> None:
        n = weight.numel()
        check(self._lib.cellm_hip_rms_norm(self._h, _dev_ptr(x), _dev_ptr(weight), _torch_dtype_code(weight),
                                           x.numel() // n, n, eps, _dev_ptr(out), _stream_ptr(stream)))

    def encode_add_rms_norm(self, x, y, weight, out, eps: float, stream=None) -> None:
        n = weight.numel()
        check(self._lib.cellm_hip_add_rms_norm(self._h, _dev_ptr(x), _dev_ptr(y), _dev_ptr(weight),
                                               _torch_dtype_code(weight), x.numel() // n, n, eps, _dev_ptr(out),
                                               _stream_ptr(stream)))

    def encode_rope_kv_write(self, q, k, v, n_heads: int, n_kv_heads: int, head_dim: int, positions_i32, cos_sin,
                             kcache, vcache, block_tables, total_blocks: int, n_layers: int, tokens_per_block: int,
                             layer: int, stream=None) -> None:
        rows = positions_i32.numel()
        check(self._lib.cellm_hip_rope_kv_write_f16(self._h, _dev_ptr(q), _dev_ptr(k), _dev_ptr(v), rows, n_heads,
                                                    n_kv_heads, head_dim, _dev_ptr(positions_i32), _dev_ptr(cos_sin),
                                                    cos_sin.shape[0], _dev_ptr(kcache), _dev_ptr(vcache),
                                                    _dev_ptr(block_tables), block_tables.shape[-1], total_blocks,
                                                    n_layers, tokens_per_block, layer, _stream_ptr(stream)))

    def encode_decode_qkv(self, x_prev, y, x_out, norm_w, eps: float, wq, sq, wk, sk, wv, sv, n_heads: int,
                          n_kv_heads: int, head_dim: int, positions_i32, cos_sin, q_out, kcache, vcache, block_tables,
                          total_blocks: int, n_layers: int, tokens_per_block: int, layer: int, stream=None) -> None:
        rows, hidden = positions_i32.numel(), norm_w.numel()
        check(self._lib.cellm_hip_decode_qkv_rope_kv(
            self._h, _dev_ptr(x_prev), _dev_ptr(y), _dev_ptr(x_out), _dev_ptr(norm_w), eps, _dev_ptr(wq),
            _dev_ptr(sq), _dev_ptr(wk), _dev_ptr(sk), _dev_ptr(wv), _dev_ptr(sv), rows, hidden, n_heads, n_kv_heads,
            head_dim, _dev_ptr(positions_i32), _dev_ptr(cos_sin), cos_sin.shape[0], _dev_ptr(q_out),
            _dev_ptr(kcache), _dev_ptr(vcache), _dev_ptr(block_tables), block_tables.shape[-1], total_blocks,
            n_layers, tokens_per_block, layer, _stream_ptr(stream)))

    def encode_decode_gate_up(self, x_prev, y, x_out, norm_w, eps: float, wg, sg, wu, su, h, stream=None) -> None:
        hidden = norm_w.numel()
        rows = x_prev.numel() // hidden
        check(self._lib.cellm_hip_decode_gate_up_silu(
            self._h, _dev_ptr(x_prev), _dev_ptr(y), _dev_ptr(x_out), _dev_ptr(norm_w), eps, _dev_ptr(wg),
            _dev_ptr(sg), _dev_ptr(wu), _dev_ptr(su), rows, hidden, wg.shape[0], _dev_ptr(h), _stream_ptr(stream)))

    def encode_decode_q4_qkv(self, x_prev, y, x_out, norm_w, eps: float, wq, sq, bq, biasq, wk, sk, bk, biask, wv, sv,
                             bv, biasv, group: int, n_heads: int, n_kv_heads: int, head_dim: int, positions_i32,
                             cos_sin, q_out, kcache, vcache, block_tables, total_blocks: int, n_layers: int,
                             tokens_per_block: int, layer: int, stream=None) -> None:
        """cellm_hip_decode_q4_affine_qkv_rope_kv: u32 weights, f32 scales/biases [out][hidden/group]."""
        rows, hidden = positions_i32.numel(), norm_w.numel()
        check(self._lib.cellm_hip_decode_q4_affine_qkv_rope_kv(
            self._h, _dev_ptr(x_prev), _dev_ptr(y), _dev_ptr(x_out), _dev_ptr(norm_w), eps, _dev_ptr(wq),
            _dev_ptr(sq), _dev_ptr(bq), _dev_ptr(biasq), _dev_ptr(wk), _dev_ptr(sk), _dev_ptr(bk), _dev_ptr(biask),
            _dev_ptr(wv), _dev_ptr(sv), _dev_ptr(bv), _dev_ptr(biasv), _torch_dtype_code(sq), group, rows, hidden,
            n_heads, n_kv_heads, head_dim, _dev_ptr(positions_i32), _dev_ptr(cos_sin), cos_sin.shape[0],
            _dev_ptr(q_out), _dev_ptr(kcache), _dev_ptr(vcache), _dev_ptr(block_tables), block_tables.shape[-1],
            total_blocks, n_layers, tokens_per_block, layer, _stream_ptr(stream)))

    def encode_decode_q4_gate_up(self, x_prev, y, x_out, norm_w, eps: float, wg, sg, bg, wu, su, bu, group: int, h,
                                 stream=None) -> None:
        """cellm_hip_decode_q4_affine_gate_up_silu: u32 weights, f32 scales/biases [inter][hidden/group]."""
        hidden = norm_w.numel()
        rows = x_prev.numel() // hidden
        check(self._lib.cellm_hip_decode_q4_affine_gate_up_silu(
            self._h, _dev_ptr(x_prev), _dev_ptr(y), _dev_ptr(x_out), _dev_ptr(norm_w), eps, _dev_ptr(wg),
            _dev_ptr(sg), _dev_ptr(bg), _dev_ptr(wu), _dev_ptr(su), _dev_ptr(bu), _torch_dtype_code(sg), group,
            rows, hidden, wg.shape[0], _dev_ptr(h), _stream_ptr(stream)))

    def encode_rope_half(self, x, n_heads: int, head_dim: int, positions_i32, cos_sin, stream=None) -> None:
        rows = positions_i32.numel()
        check(self._lib.cellm_hip_rope_half_f32(self._h, _dev_ptr(x), rows, n_heads, head_dim,
                                                _dev_ptr(positions_i32), _dev_ptr(cos_sin), cos_sin.shape[0],
                                                _stream_ptr(stream)))

    def encode_rope_interleaved(self, x, n_heads: int, head_dim: int, positions_i32, cos_sin, stream=None) -> None:
        rows = positions_i32.numel()
        check(self._lib.cellm_hip_rope_interleaved_f32(self._h, _dev_ptr(x), rows, n_heads, head_dim,
                                                       _dev_ptr(positions_i32), _dev_ptr(cos_sin), cos_sin.shape[0],
                                                       _stream_ptr(stream)))

    def set_rope_interleaved(self, interleaved: bool) -> None:
        """RoPE pair layout of encode_rope_kv_write / encode_decode_qkv on this context."""
        check(self._lib.cellm_hip_set_rope_interleaved(self._h, 1 if interleaved else 0))

    def encode_kv_write(self, k, v, positions_i32, kcache, vcache, block_tables, total_blocks: int, n_layers: int,
                        tokens_per_block: int, layer: int, stream=None) -> None:
        rows = positions_i32.numel()
        check(self._lib.cellm_hip_kv_write_f16(self._h, _dev_ptr(k), _dev_ptr(v), rows, k.numel() // rows,
                                               _dev_ptr(positions_i32), _dev_ptr(kcache), _dev_ptr(vcache),
                                               _dev_ptr(block_tables), block_tables.shape[-1], total_blocks, n_layers,
                                               tokens_per_block, layer, _stream_ptr(stream)))

    def encode_attention(self, q, kcache, vcache, block_tables, positions_i32, out, n_heads: int, n_kv_heads: int,
                         head_dim: int, total_blocks: int, n_layers: int, tokens_per_block: int, layer: int,
                         attn_scale: float | None = None, soft_cap: float | None = None, stream=None,
                         window: int | None = None) -> None:
        """attention_single_token_gqa_f32 (kvcache.rs:710-789) per row; attn_scale
        None = 1/sqrt(head_dim), soft_cap None = no cap (the reference's Options).
        window: a Gemma sliding layer's window (gemma.rs:747-751), each row then
        attends to its last `window` positions only; 0 = every position."""
        rows = positions_i32.numel()
        if window is not None:
            check(self._lib.cellm_hip_attention_gqa_f16kv_window(
                self._h, _dev_ptr(q), _dev_ptr(kcache), _dev_ptr(vcache), _dev_ptr(block_tables),
                block_tables.shape[-1], total_blocks, _dev_ptr(positions_i32), rows, n_heads, n_kv_heads, head_dim,
                n_layers, tokens_per_block, layer, 0.0 if attn_scale is None else attn_scale,
                0.0 if soft_cap is None else soft_cap, window, _dev_ptr(out), _stream_ptr(stream)))
            return
        check(self._lib.cellm_hip_attention_gqa_f16kv(self._h, _dev_ptr(q), _dev_ptr(kcache), _dev_ptr(vcache),
                                                      _dev_ptr(block_tables), block_tables.shape[-1], total_blocks,
                                                      _dev_ptr(positions_i32), rows, n_heads, n_kv_heads, head_dim,
                                                      n_layers, tokens_per_block, layer,
                                                      0.0 if attn_scale is None else attn_scale,
                                                      0.0 if soft_cap is None else soft_cap, _dev_ptr(out),
                                                      _stream_ptr(stream)))

    def encode_attention_noalloc(self, q, kcache, vcache, block_tables, positions_i32, out, n_heads: int,
                                 n_kv_heads: int, head_dim: int, total_blocks: int, n_layers: int,
                                 tokens_per_block: int, layer: int, attn_scale: float | None = None,
                                 soft_cap: float | None = None, stream=None) -> None:
        """encode_attention with its partials in the library's static device
        scratch (8 MiB per GPU): allocates nothing; overlapping calls on one
        GPU race."""
        rows = positions_i32.numel()
        check(self._lib.cellm_hip_attention_gqa_f16kv_noalloc(
            self._h, _dev_ptr(q), _dev_ptr(kcache), _dev_ptr(vcache), _dev_ptr(block_tables), block_tables.shape[-1],
            total_blocks, _dev_ptr(positions_i32), rows, n_heads, n_kv_heads, head_dim, n_layers, tokens_per_block,
            layer, 0.0 if attn_scale is None else attn_scale, 0.0 if soft_cap is None else soft_cap, _dev_ptr(out),
            _stream_ptr(stream)))

    def encode_silu_mul(self, gate, up, stream=None) -> None:
        """gate = silu(gate) * up in place (f32), silu_mul_f32_inplace."""
        check(self._lib.cellm_hip_silu_mul_f32(self._h, _dev_ptr(gate), _dev_ptr(up), gate.numel(),
                                               _stream_ptr(stream)))

    def encode_gelu_tanh_mul(self, gate, up, stream=None) -> None:
        """gate = gelu_tanh(gate) * up in place (f32), gelu_tanh_mul_f32_inplace."""
        check(self._lib.cellm_hip_gelu_tanh_mul_f32(self._h, _dev_ptr(gate), _dev_ptr(up), gate.numel(),
                                                    _stream_ptr(stream)))

    def encode_add_inplace(self, x, y, stream=None) -> None:
        check(self._lib.cellm_hip_add_f32_inplace(self._h, _dev_ptr(x), _dev_ptr(y), x.numel(), _stream_ptr(stream)))

    def encode_argmax(self, logits, out_index_i32, out_value, stream=None) -> None:
        rows = out_index_i32.numel()
        check(self._lib.cellm_hip_argmax_f32(self._h, _dev_ptr(logits), rows, logits.numel() // rows,
                                             _dev_ptr(out_index_i32), _dev_ptr(out_value), _stream_ptr(stream)))

    def encode_argmax_keys(self, logits, out_keys_i64, stream=None) -> None:
        """First maximum per row merged into packed keys (int64 tensor, zero before the first call);
        decode with argmax_key_index / argmax_key_value."""
        rows = out_keys_i64.numel()
        check(self._lib.cellm_hip_argmax_f32_keys(self._h, _dev_ptr(logits), rows, logits.numel() // rows,
                                                  _dev_ptr(out_keys_i64), _stream_ptr(stream)))
