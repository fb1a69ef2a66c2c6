"""The .cellm reader of libcellm_hip.so (cellm_file_*, no device needed)
against files written in the reference's layout, and its rejections
(cellm_file.rs:58-124: magic, version, header length, JSON, tensor ranges)."""
from __future__ import annotations

import json
import struct

import numpy as np
import pytest

from _cellm_writer import llama_header, write_cellm


@pytest.fixture(scope="module")
def CellmFile():
    from cellm_amd.cellm_file import CellmFile

    return CellmFile


def sample_tensors(rng):
    w = rng.integers(-127, 128, (48, 32)).astype(np.int8)
    s = rng.uniform(0.001, 0.02, 48).astype(np.float16)
    q = rng.integers(0, 2**32, (16, 4), dtype=np.uint64).astype(np.uint32)
    n = rng.standard_normal(32).astype(np.float16)
    e = np.zeros((0,), np.float32)
    return [("model.layers.0.mlp.up_proj.weight", w, "i8", w.shape),
            ("model.layers.0.mlp.up_proj.weight.qscale", s, "f16", s.shape),
            ("model.layers.0.self_attn.q_proj.weight", q, "u32", (16, 32)),
            ("model.norm.weight", n, "f16", n.shape),
            ("empty", e, "f32", (0,))]


def test_reads_header_config_and_tensor_bytes(tmp_path, CellmFile):
    rng = np.random.default_rng(1)
    ts = sample_tensors(rng)
    hdr = llama_header(2, 32, 4, 2, 48, 100, eps=1e-6, theta=500000.0,
                       source_text_config={"a": [1, 2.5, None, True, {"b": "x"}]},
                       note="café \"quoted\" \\ \n tab\t \U0001F600")
    p = tmp_path / "m.cellm"
    written = write_cellm(p, hdr, ts)
    with CellmFile(p) as f:
        c = f.config
        assert c["model_type"] == "llama"
        assert (c["vocab_size"], c["hidden_dim"], c["intermediate_size"], c["num_layers"], c["num_heads"],
                c["num_kv_heads"]) == (100, 32, 48, 2, 4, 2)
        assert c["head_dim"] == -1  # null in the header
        assert (c["bos_token_id"], c["eos_token_id"], c["max_position_embeddings"]) == (1, 2, -1)
        assert c["rms_norm_eps"] == np.float32(1e-6) and c["rope_theta"] == np.float32(500000.0)
        assert c["tie_word_embeddings"] == 1
        # the tensor index in header order, offsets absolute and 64-byte aligned
        assert [t.name for t in f.tensors] == [t["name"] for t in written["tensors"]]
        for t, w in zip(f.tensors, written["tensors"]):
            assert (t.offset_bytes, t.nbytes, list(t.shape), t.dtype) == (w["offset_bytes"], w["nbytes"], w["shape"],
                                                                          w["dtype"])
            assert t.offset_bytes % 64 == 0
        for name, a, _, _ in ts:
            assert f.has_tensor(name)
            np.testing.assert_array_equal(f.tensor_bytes(name), np.frombuffer(a.tobytes(), np.uint8))
        assert json.loads(f.header_json()) == written
        assert json.loads(f.header_json())["note"] == hdr["note"]
        assert not f.has_tensor("model.missing")


def _raw(p, text: bytes, tail: bytes = b"", magic=b"CELLM", version=1, hlen=None):
    with open(p, "wb") as f:
        f.write(magic + struct.pack("<B", version) + struct.pack("<I", len(text) if hlen is None else hlen) + text +
                tail)


@pytest.mark.parametrize("case,needle", [
    ("too_small", "file too small"),
    ("magic", "bad magic"),
    ("version", "unsupported version 2"),
    ("hlen", "header length out of range"),
    ("json", "header json parse failed"),
    ("trailing", "header json parse failed"),
    ("no_tensors", "tensors missing"),
    ("missing_field", "hidden_dim missing"),
    ("range", "out of range"),
    ("bad_shape", "bad shape"),
])
def test_rejects_malformed_files(tmp_path, CellmFile, case, needle):
    from cellm_amd._lib import CellmHipError

    p = tmp_path / f"{case}.cellm"
    good = llama_header(1, 8, 2, 2, 16, 10)
    t = {"name": "w", "offset_bytes": 64, "nbytes": 8, "shape": [8], "dtype": "i8"}
    if case == "too_small":
        p.write_bytes(b"CELLM\x01")
    elif case == "magic":
        _raw(p, b"{}", magic=b"CELLX")
    elif case == "version":
        _raw(p, b"{}", version=2)
    elif case == "hlen":
        _raw(p, b"{}", hlen=4096)
    elif case == "json":
        _raw(p, b'{"model_type": "llama", ')
    elif case == "trailing":
        _raw(p, json.dumps(dict(good, tensors=[])).encode() + b" x")
    elif case == "no_tensors":
        _raw(p, json.dumps(good).encode())
    elif case == "missing_field":
        h = dict(good, tensors=[])
        del h["hidden_dim"]
        _raw(p, json.dumps(h).encode())
    elif case == "range":
        _raw(p, json.dumps(dict(good, tensors=[dict(t, nbytes=1 << 20)])).encode(), b"\0" * 128)
    elif case == "bad_shape":
        _raw(p, json.dumps(dict(good, tensors=[dict(t, shape=[-1])])).encode(), b"\0" * 128)
    with pytest.raises(CellmHipError, match=needle):
        CellmFile(p)


def test_missing_path_and_unknown_tensor(tmp_path, CellmFile):
    from cellm_amd._lib import CellmHipError

    with pytest.raises(CellmHipError, match="open failed"):
        CellmFile(tmp_path / "nope.cellm")
    p = tmp_path / "m.cellm"
    write_cellm(p, llama_header(1, 8, 2, 2, 16, 10), [("a", np.zeros(4, np.int8), "i8", (4,))])
    with CellmFile(p) as f:
        with pytest.raises(CellmHipError, match="unknown tensor"):
            f.tensor_bytes("b")


def test_duplicate_name_keeps_last_entry(tmp_path, CellmFile):
    """cellm_file.rs:89-92 indexes tensors with HashMap::insert: a repeated name
    resolves to its last entry, and every entry is still range-checked."""
    from cellm_amd._lib import CellmHipError

    good = llama_header(1, 8, 2, 2, 16, 10)
    payload = bytes(range(128))
    first = {"name": "w", "offset_bytes": 0, "nbytes": 8, "shape": [8], "dtype": "i8"}
    other = {"name": "v", "offset_bytes": 16, "nbytes": 4, "shape": [4], "dtype": "u8"}
    last = {"name": "w", "offset_bytes": 32, "nbytes": 16, "shape": [4, 4], "dtype": "u8"}
    base = 10 + 4096  # header padded with spaces to 4096 bytes, so offsets are known up front
    for t in (first, other, last):
        t["offset_bytes"] += base
    p = tmp_path / "dup.cellm"
    text = json.dumps(dict(good, tensors=[first, other, last])).encode()
    assert len(text) <= 4096
    _raw(p, text.ljust(4096), payload)
    with CellmFile(p) as f:
        assert [t.name for t in f.tensors] == ["w", "v"]
        w = f.tensors[0]
        assert (w.offset_bytes, w.nbytes, list(w.shape), w.dtype) == (base + 32, 16, [4, 4], "u8")
        np.testing.assert_array_equal(f.tensor_bytes("w"), np.frombuffer(payload[32:48], np.uint8))
    # a shadowed entry that points past the end still fails the load
    bad = dict(first, nbytes=1 << 20)
    _raw(p, json.dumps(dict(good, tensors=[bad, last])).encode().ljust(4096), payload)
    with pytest.raises(CellmHipError, match="out of range"):
        CellmFile(p)
