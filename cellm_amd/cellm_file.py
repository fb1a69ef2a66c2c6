"""ctypes binding of the .cellm file API of libcellm_hip.so (include/cellm_hip.h,
cellm_file_*), the host side of CellmFile (crates/cellm-model/src/cellm_file.rs).

`CellmFile(path)` maps and validates a file; `.config` holds the model fields
of the header, `.tensors` the tensor index in header order, `.tensor_bytes`
returns a zero-copy numpy view of the mapped bytes, `.upload(ops)` puts
the tensors into a HipOps context's name-keyed device weight cache, and
`.linear(ops, name, family, x, y)` runs one projection by the dtype of its
weight tensor under a runner family's dispatch rules.  `write_cellm` writes a
file in the same layout (synthetic models for tests and bench.py).
"""
from __future__ import annotations

import ctypes as C
import json
import struct
from dataclasses import dataclass

import numpy as np

from ._lib import CellmHipError, load


class FileConfig(C.Structure):
    _fields_ = [("model_type", C.c_char * 64), ("vocab_size", C.c_int64), ("hidden_dim", C.c_int64),
                ("intermediate_size", C.c_int64), ("num_layers", C.c_int64), ("num_heads", C.c_int64),
                ("num_kv_heads", C.c_int64), ("head_dim", C.c_int64), ("bos_token_id", C.c_int64),
                ("eos_token_id", C.c_int64), ("max_position_embeddings", C.c_int64),
                ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float), ("tie_word_embeddings", C.c_int32)]


class FileTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("dtype", C.c_char_p), ("shape", C.c_int64 * 8), ("ndim", C.c_int32),
                ("offset_bytes", C.c_uint64), ("nbytes", C.c_uint64)]


@dataclass(frozen=True)
class TensorInfo:
    name: str
    dtype: str
    shape: tuple
    offset_bytes: int
    nbytes: int


# runner families of cellm_hip_linear_file (CELLM_HIP_FAMILY_*)
FAMILIES = {"llama": 0, "qwen": 1, "gemma": 2, "lfm": 3}

_bound = None


def _lib():
    global _bound
    if _bound is not None:
        return _bound
    lib = load()
    vp = C.c_void_p
    sig = {
        "cellm_file_open": (C.c_int32, [C.c_char_p, C.POINTER(vp)]),
        "cellm_file_close": (None, [vp]),
        "cellm_file_config": (C.c_int32, [vp, C.POINTER(FileConfig)]),
        "cellm_file_header_json": (C.c_int32, [vp, C.POINTER(C.c_char_p), C.POINTER(C.c_size_t)]),
        "cellm_file_tensor_count": (C.c_int64, [vp]),
        "cellm_file_tensor_at": (C.c_int32, [vp, C.c_int64, C.POINTER(FileTensor)]),
        "cellm_file_find": (C.c_int32, [vp, C.c_char_p, C.POINTER(FileTensor)]),
        "cellm_file_tensor_bytes": (C.c_int32, [vp, C.c_char_p, C.POINTER(vp), C.POINTER(C.c_size_t)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _bound = lib
    return lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        from ._lib import last_error

        raise CellmHipError(rc, f"{what}: {last_error()}")


class CellmFile:
    def __init__(self, path):
        self._lib = _lib()
        h = C.c_void_p()
        _check(self._lib.cellm_file_open(str(path).encode(), C.byref(h)), f"cellm_file_open({path})")
        self._h = h
        cfg = FileConfig()
        _check(self._lib.cellm_file_config(h, C.byref(cfg)), "cellm_file_config")
        self.config = {f: getattr(cfg, f) for f, _ in FileConfig._fields_}
        self.config["model_type"] = cfg.model_type.decode()
        self.tensors = []
        t = FileTensor()
        for i in range(self._lib.cellm_file_tensor_count(h)):
            _check(self._lib.cellm_file_tensor_at(h, i, C.byref(t)), "cellm_file_tensor_at")
            self.tensors.append(TensorInfo(t.name.decode(), t.dtype.decode(), tuple(t.shape[:t.ndim]),
                                           int(t.offset_bytes), int(t.nbytes)))
        self._by_name = {ti.name: ti for ti in self.tensors}

    @property
    def handle(self):
        return self._h

    def header_json(self) -> str:
        p = C.c_char_p()
        n = C.c_size_t()
        _check(self._lib.cellm_file_header_json(self._h, C.byref(p), C.byref(n)), "cellm_file_header_json")
        return C.string_at(p, n.value).decode()

    def has_tensor(self, name: str) -> bool:
        return name in self._by_name

    def tensor(self, name: str) -> TensorInfo:
        t = FileTensor()
        _check(self._lib.cellm_file_find(self._h, name.encode(), C.byref(t)), f"cellm_file_find({name})")
        return self._by_name[name]

    def tensor_bytes(self, name: str) -> np.ndarray:
        """The mapped bytes of a tensor as a read-only uint8 view (valid while the file is open)."""
        p = C.c_void_p()
        n = C.c_size_t()
        _check(self._lib.cellm_file_tensor_bytes(self._h, name.encode(), C.byref(p), C.byref(n)),
               f"cellm_file_tensor_bytes({name})")
        if n.value == 0:
            return np.zeros(0, np.uint8)
        buf = (C.c_uint8 * n.value).from_address(p.value)
        a = np.frombuffer(buf, dtype=np.uint8)
        a.flags.writeable = False
        return a

    def upload(self, ops, name_prefix: str | None = None) -> tuple[int, int]:
        """All tensors (or those under name_prefix) into ops' device weight cache; (count, bytes)."""
        count = C.c_int64()
        nbytes = C.c_size_t()
        _check(ops._lib.cellm_hip_upload_cellm_file(ops._h, self._h, name_prefix.encode() if name_prefix else None,
                                                    C.byref(count), C.byref(nbytes)), "cellm_hip_upload_cellm_file")
        return count.value, nbytes.value

    def linear(self, ops, weight_name: str, family: str, x, y, stream=None) -> None:
        """y[m, out] = W x[m, in] with W the tensor `weight_name`, dispatched on its dtype as the
        family's ("llama", "qwen", "gemma", "lfm") linear_f16_out_in does (cellm_hip_linear_file);
        x and y are float32 device tensors of shape [m, in] and [m, out]; enqueued on `stream`.
        The first call for a tensor uploads it into ops' weight cache."""
        from .hipops import _dev_ptr, _stream_ptr
        import torch

        if family not in FAMILIES:
            raise ValueError(f"family must be one of {sorted(FAMILIES)}")
        if x.dtype != torch.float32 or y.dtype != torch.float32 or x.dim() != 2 or y.dim() != 2 \
                or x.shape[0] != y.shape[0]:
            raise ValueError("x and y must be float32 [m, in] and [m, out] device tensors")
        _check(ops._lib.cellm_hip_linear_file(ops._h, self._h, weight_name.encode(), FAMILIES[family], _dev_ptr(x),
                                              _dev_ptr(y), x.shape[0], y.shape[1], x.shape[1], _stream_ptr(stream)),
               f"cellm_hip_linear_file({weight_name})")

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.cellm_file_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        self.close()


def write_cellm(path, header: dict, tensors, version: int = 1, magic: bytes = b"CELLM") -> dict:
    """Writes a .cellm file in the layout the reference's writers use (tools/convert_lfm.py:15-90):
    the magic, a version byte, the u32 little-endian header length, the JSON header (the given
    fields plus the tensor index), then each tensor at an absolute, 64-byte aligned offset, in
    name order.  tensors: (name, array, dtype string, shape) with the array's bytes written as
    they are; returns the header written.  Tensors are written one at a time (no copy of the
    whole model is held)."""
    items = sorted(tensors, key=lambda t: t[0])
    sizes = {name: int(np.asarray(a).nbytes) for name, a, _, _ in items}

    def layout(hlen):
        off = (10 + hlen + 63) & ~63
        offs = {}
        for name, _, _, _ in items:
            off = (off + 63) & ~63
            offs[name] = off
            off += sizes[name]
        return offs

    def build(offs):
        h = dict(header)
        h["tensors"] = [{"name": n, "offset_bytes": offs[n], "nbytes": sizes[n], "shape": list(shape),
                         "dtype": dt} for n, _, dt, shape in items]
        return h, json.dumps(h).encode()

    offs = layout(0)
    for _ in range(8):  # offsets depend on the header length and vice versa: iterate to a fixed point
        h, text = build(offs)
        new = layout(len(text))
        if new == offs:
            break
        offs = new
    h, text = build(offs)
    if layout(len(text)) != offs:
        # a header whose length moved a tensor after the last pass would put the data at other offsets
        # than the header states: refuse instead of writing a corrupt file
        raise ValueError("write_cellm: header offsets did not converge")
    with open(path, "wb") as f:
        f.write(magic)
        f.write(struct.pack("<B", version))
        f.write(struct.pack("<I", len(text)))
        f.write(text)
        for name, a, _, _ in items:
            pos = f.tell()
            f.write(b"\0" * (offs[name] - pos))
            f.write(np.ascontiguousarray(a).tobytes())
    return h


def llama_header(n_layers, hidden, heads, kv_heads, inter, vocab, eps=1e-5, theta=100000.0, head_dim=None,
                 **extra) -> dict:
    """The model fields of a .cellm header (CellmHeader, crates/cellm-model/src/cellm_file.rs:20-48) for a
    Llama-layout model; `extra` adds or overrides fields (model_type, tie_word_embeddings, ...)."""
    h = {"model_type": "llama", "vocab_size": vocab, "hidden_dim": hidden, "intermediate_size": inter,
         "num_layers": n_layers, "num_heads": heads, "num_kv_heads": kv_heads, "head_dim": head_dim,
         "rms_norm_eps": eps, "rope_theta": theta, "bos_token_id": 1, "eos_token_id": 2,
         "tie_word_embeddings": True, "source_quantization": None}
    h.update(extra)
    return h
