"""ctypes binding of libcellm_llama_step.so's device-resident Llama decode
step (include/cellm_llama_step.h, cellm_llama_dev_*).

`LlamaDevice` owns one runner: int8 per-row-scaled projection weights and
the tied int8 embedding uploaded once, a paged f16 K/V cache on the device
(KvCacheLayout, crates/cellm-core/src/kv_cache.rs:62-73), and one captured
HIP graph per session count.  `step` decodes up to max_rows sessions in one
pass over the weights and returns their greedy ids, the device counterpart
of LlamaRunner::step_topk with top_k = 1 (crates/cellm-model/src/llama.rs:189-212).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import build
from ._lib import CellmHipError, load


class Config(C.Structure):
    _fields_ = [("n_layers", C.c_int32), ("hidden", C.c_int32), ("n_heads", C.c_int32), ("n_kv_heads", C.c_int32),
                ("head_dim", C.c_int32), ("intermediate", C.c_int32), ("vocab", C.c_int32),
                ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float), ("tokens_per_block", C.c_int32),
                ("total_blocks", C.c_int32)]


class Layer(C.Structure):
    _fields_ = [("w", C.c_void_p * 7), ("scale_f16", C.c_void_p * 7), ("input_layernorm_f16", C.c_void_p),
                ("post_attention_layernorm_f16", C.c_void_p)]


PROJ_NAMES = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


@dataclass
class LlamaShape:
    n_layers: int
    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    tokens_per_block: int = 16
    total_blocks: int = 64

    def proj_shapes(self) -> list[tuple[int, int]]:
        """[out, in] of q, k, v, o, gate, up, down."""
        h, kv, i = self.hidden, self.n_kv_heads * self.head_dim, self.intermediate
        return [(h, h), (kv, h), (kv, h), (h, h), (i, h), (i, h), (h, i)]

    def kv_elems(self) -> int:
        return self.total_blocks * self.n_layers * self.tokens_per_block * self.n_kv_heads * self.head_dim

    def weight_bytes(self) -> int:
        """int8 projection and embedding bytes plus their f16 row scales."""
        per_layer = sum(o * i + 2 * o for o, i in self.proj_shapes())
        return self.n_layers * per_layer + self.vocab * self.hidden + 2 * self.vocab


_lib = None


def _load():
    global _lib
    if _lib is not None:
        return _lib
    load()  # libcellm_hip.so first: the step library links against it
    if not build.STEP_LIB_PATH.exists():
        raise CellmHipError(-1, f"{build.STEP_LIB_PATH} is not built (run cellm_amd.build)")
    lib = C.CDLL(str(build.STEP_LIB_PATH))
    lib.cellm_llama_dev_create.argtypes = [C.POINTER(Config), C.POINTER(Layer), C.c_void_p, C.c_void_p, C.c_void_p,
                                           C.c_int32, C.c_int32, C.c_int32, C.POINTER(C.c_void_p)]
    lib.cellm_llama_dev_kv_upload.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]
    lib.cellm_llama_dev_kv_download.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]
    lib.cellm_llama_dev_step.argtypes = [C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                         C.c_void_p, C.c_void_p]
    lib.cellm_llama_dev_set_graphs.argtypes = [C.c_void_p, C.c_int32]
    lib.cellm_llama_dev_create_from_file.argtypes = [C.c_char_p, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                                     C.c_int32, C.POINTER(C.c_void_p)]
    lib.cellm_llama_dev_destroy.argtypes = [C.c_void_p]
    lib.cellm_llama_last_error_message.restype = C.c_size_t
    lib.cellm_llama_last_error_message.argtypes = [C.c_char_p, C.c_size_t]
    _lib = lib
    return lib


def _check(lib, rc: int, what: str) -> None:
    if rc != 0:
        b = C.create_string_buffer(2048)
        lib.cellm_llama_last_error_message(b, len(b))
        raise CellmHipError(rc, f"{what}: {b.value.decode(errors='replace')}")


class LlamaDevice:
    """One device-resident runner.  `layers[l]` = (weights[7] int8 [out, in],
    scales[7] f16-as-uint16 [out], input_layernorm f16 [hidden],
    post_attention_layernorm f16 [hidden]); `embed` int8 [vocab, hidden] with
    f16 row scales `embed_scale` (the tied lm_head); `final_norm` f16."""

    def __init__(self, shape: LlamaShape, layers, embed: np.ndarray, embed_scale: np.ndarray,
                 final_norm: np.ndarray, device: int = 0, max_rows: int = 4, max_blocks: int | None = None):
        self.lib = _load()
        self.shape = shape
        self.max_rows = max_rows
        self.max_blocks = max_blocks if max_blocks is not None else shape.total_blocks
        cl = (Layer * shape.n_layers)()
        keep = []
        for l, (ws, ss, n1, n2) in enumerate(layers):
            for j, (o, i) in enumerate(shape.proj_shapes()):
                w = np.ascontiguousarray(ws[j], dtype=np.int8)
                s = np.ascontiguousarray(ss[j]).view(np.uint16)
                if w.shape != (o, i) or s.shape != (o,):
                    raise ValueError(f"layer {l} {PROJ_NAMES[j]}: weight {w.shape} / scale {s.shape}, "
                                     f"want ({o}, {i}) / ({o},)")
                keep += [w, s]
                cl[l].w[j] = w.ctypes.data
                cl[l].scale_f16[j] = s.ctypes.data
            for name, n in (("input_layernorm_f16", n1), ("post_attention_layernorm_f16", n2)):
                a = np.ascontiguousarray(n).view(np.uint16)
                if a.shape != (shape.hidden,):
                    raise ValueError(f"layer {l} {name}: shape {a.shape}")
                keep.append(a)
                setattr(cl[l], name, a.ctypes.data)
        e = np.ascontiguousarray(embed, dtype=np.int8)
        es = np.ascontiguousarray(embed_scale).view(np.uint16)
        fn = np.ascontiguousarray(final_norm).view(np.uint16)
        if e.shape != (shape.vocab, shape.hidden) or es.shape != (shape.vocab,) or fn.shape != (shape.hidden,):
            raise ValueError("embedding / final norm shapes do not match the config")
        cfg = Config(shape.n_layers, shape.hidden, shape.n_heads, shape.n_kv_heads, shape.head_dim,
                     shape.intermediate, shape.vocab, shape.rms_norm_eps, shape.rope_theta,
                     shape.tokens_per_block, shape.total_blocks)
        h = C.c_void_p()
        _check(self.lib, self.lib.cellm_llama_dev_create(C.byref(cfg), cl, e.ctypes.data, es.ctypes.data,
                                                         fn.ctypes.data, device, max_rows, self.max_blocks,
                                                         C.byref(h)), "cellm_llama_dev_create")
        self.h = h

    @classmethod
    def from_file(cls, path, device: int = 0, max_rows: int = 4, max_blocks: int = 64, tokens_per_block: int = 16,
                  total_blocks: int | None = None) -> "LlamaDevice":
        """A runner over a .cellm Llama or Qwen2 model (cellm_llama_dev_create_from_file; the header's
        model_type "qwen*" selects the Qwen2 layer with its optional projection biases): projections
        stored as "i8" (+ .qscale), "u32" MLX affine (+ f32 .scales/.biases), "i4" (+ .qscale) or
        "f16", and for Qwen also "i2" (+ .qscale) and "q1_0_g128"; the embedding (and tied lm_head) as
        "i8" / "i4" (+ .qscale) or "f16"; the shape comes from the file's header, the paged K/V cache
        from the arguments (total_blocks defaults to max_rows * max_blocks)."""
        from .cellm_file import CellmFile

        with CellmFile(path) as f:
            c = f.config
        total = total_blocks if total_blocks is not None else max_rows * max_blocks
        head_dim = c["head_dim"] if c["head_dim"] > 0 else c["hidden_dim"] // c["num_heads"]
        self = cls.__new__(cls)
        self.lib = _load()
        self.shape = LlamaShape(c["num_layers"], c["hidden_dim"], c["num_heads"], c["num_kv_heads"], head_dim,
                                c["intermediate_size"], c["vocab_size"], c["rms_norm_eps"], c["rope_theta"],
                                tokens_per_block, total)
        self.max_rows = max_rows
        self.max_blocks = max_blocks
        h = C.c_void_p()
        _check(self.lib, self.lib.cellm_llama_dev_create_from_file(str(path).encode(), device, max_rows, max_blocks,
                                                                   tokens_per_block, total, C.byref(h)),
               "cellm_llama_dev_create_from_file")
        self.h = h
        return self

    def close(self) -> None:
        if getattr(self, "h", None):
            self.lib.cellm_llama_dev_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def set_graphs(self, enable: bool) -> None:
        _check(self.lib, self.lib.cellm_llama_dev_set_graphs(self.h, int(enable)), "cellm_llama_dev_set_graphs")

    def kv_upload(self, k_f16: np.ndarray, v_f16: np.ndarray) -> None:
        k = np.ascontiguousarray(k_f16).view(np.uint16)
        v = np.ascontiguousarray(v_f16).view(np.uint16)
        if k.size != self.shape.kv_elems() or v.size != k.size:
            raise ValueError(f"K/V need {self.shape.kv_elems()} elements each")
        _check(self.lib, self.lib.cellm_llama_dev_kv_upload(self.h, k.ctypes.data, v.ctypes.data, k.size),
               "cellm_llama_dev_kv_upload")

    def kv_download(self) -> tuple[np.ndarray, np.ndarray]:
        n = self.shape.kv_elems()
        k = np.empty(n, np.uint16)
        v = np.empty(n, np.uint16)
        _check(self.lib, self.lib.cellm_llama_dev_kv_download(self.h, k.ctypes.data, v.ctypes.data, n),
               "cellm_llama_dev_kv_download")
        return k, v

    def step(self, tokens, positions, block_tables, want_logits: bool = False):
        """Greedy ids (uint32 [rows]) and their logits (f32 [rows]); with
        want_logits also the full logits [rows, vocab]."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        p = np.ascontiguousarray(positions, dtype=np.int32)
        rows = t.size
        bt = np.zeros((rows, self.max_blocks), np.uint32)
        src = np.asarray(block_tables, dtype=np.uint32).reshape(rows, -1)
        bt[:, :min(src.shape[1], self.max_blocks)] = src[:, :self.max_blocks]
        ids = np.empty(rows, np.uint32)
        vals = np.empty(rows, np.float32)
        logits = np.empty((rows, self.shape.vocab), np.float32) if want_logits else None
        _check(self.lib, self.lib.cellm_llama_dev_step(self.h, rows, t.ctypes.data, p.ctypes.data, bt.ctypes.data,
                                                       ids.ctypes.data, vals.ctypes.data,
                                                       logits.ctypes.data if want_logits else None),
               "cellm_llama_dev_step")
        return (ids, vals, logits) if want_logits else (ids, vals)
