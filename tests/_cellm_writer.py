"""Writes .cellm files for the tests in the layout the reference's writers use
(tools/convert_lfm.py:15-90): "CELLM", version byte 1, u32 little-endian
header length, the JSON header, then each tensor at an absolute, 64-byte
aligned offset, in name order."""
from __future__ import annotations

import json
import struct

import numpy as np


def write_cellm(path, header: dict, tensors: list[tuple[str, np.ndarray, str, tuple]], version: int = 1,
                magic: bytes = b"CELLM") -> dict:
    """tensors: (name, array, dtype string, shape); returns the header written."""
    items = sorted(tensors, key=lambda t: t[0])
    blobs = {name: np.ascontiguousarray(a).tobytes() for name, a, _, _ in items}

    def layout(hlen):
        off = (10 + hlen + 63) & ~63
        offs = {}
        for name, _, _, _ in items:
            off = (off + 63) & ~63
            offs[name] = off
            off += len(blobs[name])
        return offs

    def build(offs):
        h = dict(header)
        h["tensors"] = [{"name": n, "offset_bytes": offs[n], "nbytes": len(blobs[n]), "shape": list(shape),
                         "dtype": dt} for n, _, dt, shape in items]
        return h, json.dumps(h).encode()

    offs = layout(0)
    for _ in range(4):  # offsets depend on the header length and vice versa: iterate to a fixed point
        h, text = build(offs)
        new = layout(len(text))
        if new == offs:
            break
        offs = new
    h, text = build(offs)
    with open(path, "wb") as f:
        f.write(magic)
        f.write(struct.pack("<B", version))
        f.write(struct.pack("<I", len(text)))
        f.write(text)
        for name, _, _, _ in items:
            pos = f.tell()
            f.write(b"\0" * (offs[name] - pos))
            f.write(blobs[name])
    return h


def llama_header(n_layers, hidden, heads, kv_heads, inter, vocab, eps=1e-5, theta=100000.0, head_dim=None, **extra):
    h = {"model_type": "llama", "vocab_size": vocab, "hidden_dim": hidden, "intermediate_size": inter,
         "num_layers": n_layers, "num_heads": heads, "num_kv_heads": kv_heads, "head_dim": head_dim,
         "rms_norm_eps": eps, "rope_theta": theta, "bos_token_id": 1, "eos_token_id": 2,
         "tie_word_embeddings": True, "source_quantization": None}
    h.update(extra)
    return h
