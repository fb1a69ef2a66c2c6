"""A .cellm file to device-resident weights (cellm_hip_upload_cellm_file) and
to the device decode runner (cellm_llama_dev_create_from_file).

- every uploaded tensor's device bytes equal the file's bytes;
- a runner built from a file decodes bit-identically (ids, logits, K/V) to
  one built from the same tensors in memory;
- with an untied int8 lm_head.weight whose rows are the embedding's rows
  permuted, the logits come out permuted the same way, exactly (each logit
  row depends only on its own weight row).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import oracle
from _cellm_writer import llama_header, write_cellm

pytestmark = pytest.mark.gpu

L, HID, NH, NKV, HD, INTER, VOCAB = 2, 960, 15, 5, 64, 2560, 49152
TPB, CTX, ROWS = 16, 512, 4
KVD = NKV * HD
NAMES = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
         "mlp.up_proj", "mlp.down_proj")


def shapes():
    return [(HID, HID), (KVD, HID), (KVD, HID), (HID, HID), (INTER, HID), (INTER, HID), (HID, INTER)]


def make_model():
    layers = []
    for l in range(L):
        ws, ss = [], []
        for j, (o, i) in enumerate(shapes()):
            sd = 0xCF000000 + l * 64 + j * 4
            ws.append(oracle.gen_i8((o, i), sd))
            ss.append((oracle.gen_uniform((o,), sd + 1, 0.5, 1.5) / (73.3 * np.sqrt(i))).astype(np.float16))
        n1 = (1.0 + 0.1 * oracle.lcg_fill(HID, 0xCF100000 + l, 1.0)).astype(np.float16)
        n2 = (1.0 + 0.1 * oracle.lcg_fill(HID, 0xCF200000 + l, 1.0)).astype(np.float16)
        layers.append((ws, ss, n1, n2))
    embed = oracle.gen_i8((VOCAB, HID), 0xCF300000)
    escale = (oracle.gen_uniform((VOCAB,), 0xCF300001, 0.5, 1.5) / 127.0).astype(np.float16)
    fnorm = (1.0 + 0.1 * oracle.lcg_fill(HID, 0xCF300002, 1.0)).astype(np.float16)
    return layers, embed, escale, fnorm


def file_tensors(model, prefix="", lm_head=None):
    layers, embed, escale, fnorm = model
    ts = []
    for l, (ws, ss, n1, n2) in enumerate(layers):
        pre = f"{prefix}model.layers.{l}."
        for j, name in enumerate(NAMES):
            ts.append((pre + name + ".weight", ws[j], "i8", ws[j].shape))
            ts.append((pre + name + ".weight.qscale", ss[j], "f16", ss[j].shape))
        ts.append((pre + "input_layernorm.weight", n1, "f16", n1.shape))
        ts.append((pre + "post_attention_layernorm.weight", n2, "f16", n2.shape))
    ts.append((prefix + "model.embed_tokens.weight", embed, "i8", embed.shape))
    ts.append((prefix + "model.embed_tokens.weight.qscale", escale, "f16", escale.shape))
    ts.append((prefix + "model.norm.weight", fnorm, "f16", fnorm.shape))
    if lm_head is not None:
        ts.append(("lm_head.weight", lm_head[0], "i8", lm_head[0].shape))
        ts.append(("lm_head.weight.qscale", lm_head[1], "f16", lm_head[1].shape))
    return ts


def header(tied=True):
    return llama_header(L, HID, NH, NKV, INTER, VOCAB, eps=1e-5, theta=100000.0, tie_word_embeddings=tied)


@pytest.fixture(scope="module")
def model():
    return make_model()


def kv_state():
    total = ROWS * CTX // TPB
    n = total * L * TPB * KVD
    k = oracle.gen_normal((n,), 0xCF400000, 0.0, 1.0).astype(np.float16)
    v = oracle.gen_normal((n,), 0xCF400001, 0.0, 1.0).astype(np.float16)
    bts = np.array([[b * ROWS + s for b in range(CTX // TPB)] for s in range(ROWS)], np.uint32)
    return k, v, bts


def run(dev, k, v, bts):
    dev.kv_upload(k, v)
    tokens = np.array([(100 + 7919 * s) % VOCAB for s in range(ROWS)], np.uint32)
    pos = np.array([CTX - 1, 300, 64, 0], np.int32)
    ids, vals, logits = dev.step(tokens, pos, bts, want_logits=True)
    kk, vv = dev.kv_download()
    return ids, logits, kk, vv


def test_upload_puts_file_bytes_on_the_device(tmp_path, model):
    from cellm_amd import HipOps
    from cellm_amd.cellm_file import CellmFile

    p = tmp_path / "m.cellm"
    ts = file_tensors(model)
    write_cellm(p, header(), ts)
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    ops = HipOps(0)
    try:
        with CellmFile(p) as f:
            count, nbytes = f.upload(ops, "model.layers.1.")
            assert count == 7 * 2 + 2
            count2, nbytes2 = f.upload(ops)
            assert count2 == len(ts) and nbytes2 == sum(a.nbytes for _, a, _, _ in ts)
        for name, a, _, _ in ts:
            ptr, nb = ops.weight_lookup(name)
            assert nb == a.nbytes
            host = np.empty(a.nbytes, np.uint8)
            assert hip.hipMemcpy(host.ctypes.data, ptr, nb, 2) == 0  # device to host
            np.testing.assert_array_equal(host, np.frombuffer(a.tobytes(), np.uint8))
    finally:
        ops.close()


@pytest.mark.parametrize("prefix", ["", "language_model."])
def test_runner_from_file_equals_runner_from_memory(tmp_path, model, prefix):
    from cellm_amd.llama_step import LlamaDevice, LlamaShape

    layers, embed, escale, fnorm = model
    p = tmp_path / "m.cellm"
    write_cellm(p, header(), file_tensors(model, prefix))
    k, v, bts = kv_state()
    shape = LlamaShape(L, HID, NH, NKV, HD, INTER, VOCAB, 1e-5, 100000.0, TPB, ROWS * CTX // TPB)
    mem = LlamaDevice(shape, layers, embed, escale, fnorm, 0, max_rows=ROWS, max_blocks=CTX // TPB)
    try:
        a = run(mem, k, v, bts)
    finally:
        mem.close()
    dev = LlamaDevice.from_file(p, 0, max_rows=ROWS, max_blocks=CTX // TPB, tokens_per_block=TPB)
    try:
        b = run(dev, k, v, bts)
    finally:
        dev.close()
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)
    print("ids", a[0].tolist())


def test_untied_lm_head_from_file(tmp_path, model):
    from cellm_amd.llama_step import LlamaDevice

    layers, embed, escale, fnorm = model
    perm = np.random.default_rng(5).permutation(VOCAB)
    k, v, bts = kv_state()
    p1, p2 = tmp_path / "tied.cellm", tmp_path / "untied.cellm"
    write_cellm(p1, header(), file_tensors(model))
    write_cellm(p2, header(tied=False), file_tensors(model, lm_head=(embed[perm], escale[perm])))
    outs = []
    for p in (p1, p2):
        dev = LlamaDevice.from_file(p, 0, max_rows=ROWS, max_blocks=CTX // TPB, tokens_per_block=TPB)
        try:
            outs.append(run(dev, k, v, bts))
        finally:
            dev.close()
    np.testing.assert_array_equal(outs[1][1], outs[0][1][:, perm])


def test_runner_from_file_rejects_other_dtypes(tmp_path, model):
    from cellm_amd._lib import CellmHipError
    from cellm_amd.llama_step import LlamaDevice

    ts = file_tensors(model)
    ts = [(n, a, "bf16" if n == "model.layers.0.self_attn.q_proj.weight" else d, s) for n, a, d, s in ts]
    p = tmp_path / "bad.cellm"
    write_cellm(p, header(), ts)
    with pytest.raises(CellmHipError, match="q_proj.weight is bf16"):
        LlamaDevice.from_file(p, 0, max_rows=ROWS, max_blocks=CTX // TPB, tokens_per_block=TPB)
    ts = [(n, a, "bf16" if n == "model.embed_tokens.weight" else d, s) for n, a, d, s in file_tensors(model)]
    write_cellm(p, header(), ts)
    with pytest.raises(CellmHipError, match="unsupported embed dtype"):
        LlamaDevice.from_file(p, 0, max_rows=ROWS, max_blocks=CTX // TPB, tokens_per_block=TPB)


# ---- other projection formats from a file (the runners' dtype dispatch) ----------

def _q4_proj(o, i, sd):
    """MLX affine u32 words [o, i/8] with f32 scales/biases [o, i/64] whose
    weights q*s + b are centred and variance-preserving."""
    wq = oracle.gen_q4_words((o, i // 8), sd)
    base = 1.0 / (4.6 * np.sqrt(i))
    s = (oracle.gen_uniform((o, i // 64), sd + 1, 0.5, 1.5) * base).astype(np.float32)
    b = (-7.5 * s + oracle.gen_normal((o, i // 64), sd + 2, 0.0, 0.1 * base)).astype(np.float32)
    return wq, s, b


def _i4_proj(o, i, sd):
    """cellm i4: [o, ceil(i/2)] bytes (low nibble even), one f16 scale per row."""
    w = oracle.gen_i8((o, (i + 1) // 2), sd).view(np.uint8)
    s = (oracle.gen_uniform((o,), sd + 1, 0.5, 1.5) / (4.6 * np.sqrt(i))).astype(np.float16)
    return w, s


def _f16_proj(o, i, sd):
    """f16 [o, i] weights with unit-variance outputs for unit inputs."""
    return (oracle.gen_normal((o, i), sd, 0.0, 1.0 / np.sqrt(i))).astype(np.float16), None


def _embed_of(kind, embed, escale):
    """The int8 test embedding in the given format: "i8" as is, "i4" as the
    nibbles q + 8 of a fresh i4 table with per-row scales, "f16" as fresh
    unit-normal rows."""
    if kind == "i8":
        return "i8", embed, escale
    if kind == "i4":
        w, s = _i4_proj(VOCAB, HID, 0xCF700000)
        return "i4", w, (s * np.float16(4.6 * np.sqrt(HID) / 7.0)).astype(np.float16)
    return "f16", oracle.gen_normal((VOCAB, HID), 0xCF700002, 0.0, 1.0).astype(np.float16), None


def _mixed_model(kinds):
    """Layer projections in the given per-projection formats ("u32", "i4",
    "i8", "f16"); the embedding in kinds.get("embed", "i8") (tied unless kinds
    has an "lm" entry)."""
    i8_layers, embed, escale, fnorm = make_model()
    layers = []
    for l, (ws, ss, n1, n2) in enumerate(i8_layers):
        projs = []
        for j, (o, i) in enumerate(shapes()):
            kind, sd = kinds[j], 0xCF500000 + l * 64 + j * 4
            if kind == "u32":
                projs.append(("u32",) + _q4_proj(o, i, sd))
            elif kind == "i4":
                projs.append(("i4",) + _i4_proj(o, i, sd))
            elif kind == "f16":
                projs.append(("f16",) + _f16_proj(o, i, sd))
            else:
                projs.append(("i8", ws[j], ss[j]))
        layers.append((projs, n1, n2))
    lm = None
    if "lm" in kinds:
        lm = ("i4",) + _i4_proj(VOCAB, HID, 0xCF600000) if kinds["lm"] == "i4" else \
            ("u32",) + _q4_proj(VOCAB, HID, 0xCF600000)
    return layers, _embed_of(kinds.get("embed", "i8"), embed, escale), fnorm, lm


def _proj_tensors(name, pr):
    kind = pr[0]
    if kind == "u32":
        _, wq, s, b = pr
        base = name[:-len(".weight")]
        return [(name, wq, "u32", wq.shape), (base + ".scales", s, "f32", s.shape), (base + ".biases", b, "f32", b.shape)]
    w, s = pr[1], pr[2]
    if kind == "f16":
        return [(name, w, "f16", w.shape)]
    shape = (w.shape[0], 2 * w.shape[1]) if kind == "i4" else w.shape  # i4: logical [out, in]
    return [(name, w, kind, shape), (name + ".qscale", s, "f16", s.shape)]


def _mixed_tensors(mm):
    layers, emb, fnorm, lm = mm
    ts = []
    for l, (projs, n1, n2) in enumerate(layers):
        pre = f"model.layers.{l}."
        for j, name in enumerate(NAMES):
            ts += _proj_tensors(pre + name + ".weight", projs[j])
        ts.append((pre + "input_layernorm.weight", n1, "f16", n1.shape))
        ts.append((pre + "post_attention_layernorm.weight", n2, "f16", n2.shape))
    ts += _proj_tensors("model.embed_tokens.weight", emb)
    ts.append(("model.norm.weight", fnorm, "f16", fnorm.shape))
    if lm is not None:
        ts += _proj_tensors("lm_head.weight", lm)
    return ts


def _oracle_proj(pr, x, o, i):
    """The reference's linear for each format: matmul_i8_f32 (cpu_kernels.rs:66-133),
    the LFM affine GEMV (lfm.rs:985-1066), matmul_i4_f32 with gs = in_dim
    (cpu_kernels.rs:219-243, gemma.rs:1471), matmul_f16_f32 (cpu_kernels.rs:135-214)."""
    if pr[0] == "f16":
        return oracle.qgemv_f16(pr[1].view(np.uint16), x.reshape(1, -1))[0]
    if pr[0] == "u32":
        return oracle.qgemv_q4_affine(pr[1], pr[2], pr[3], x.reshape(1, -1), i)[0]
    if pr[0] == "i4":
        return oracle.matmul_i4_f32(pr[1], pr[2].view(np.uint16), o, i, i, x)
    return oracle.matmul_i8_f32(pr[1], pr[2].view(np.uint16), x)


def _oracle_session(mm, kc, vc, token, pos, bt):
    """LlamaRunner::step_inner (llama.rs:235-647) for one session over the
    paged f16 cache (updated in place), projections by format."""
    layers, emb, fnorm, lm = mm
    ekind, ew, es = emb
    x = oracle.embed(ekind, [token], ew.view(np.uint16) if ekind == "f16" else ew,
                     None if es is None else es.view(np.uint16), VOCAB, HID)[0]

    def base_of(tpos, layer):
        return int(bt[tpos // TPB]) * (L * TPB * KVD) + layer * (TPB * KVD) + (tpos % TPB) * KVD

    for l, (projs, n1, n2) in enumerate(layers):
        xn = oracle.rms_norm(x, n1.astype(np.float32), 1e-5)
        q = _oracle_proj(projs[0], xn, HID, HID)
        k = _oracle_proj(projs[1], xn, KVD, HID)
        v = _oracle_proj(projs[2], xn, KVD, HID)
        oracle.rope_half_(q, NH, HD, pos, 100000.0)
        oracle.rope_half_(k, NKV, HD, pos, 100000.0)
        wb = base_of(pos, l)
        kc[wb:wb + KVD] = k.astype(np.float16).view(np.uint16)
        vc[wb:wb + KVD] = v.astype(np.float16).view(np.uint16)
        bases = np.array([base_of(tp, l) for tp in range(pos + 1)], np.uint64)
        attn = oracle.attention_gqa_f16kv(kc, vc, bases, q, NH, NKV, HD)
        x = x + _oracle_proj(projs[3], attn, HID, HID)
        xn = oracle.rms_norm(x, n2.astype(np.float32), 1e-5)
        g = np.ascontiguousarray(_oracle_proj(projs[4], xn, INTER, HID), np.float32)
        oracle.silu_mul_(g, _oracle_proj(projs[5], xn, INTER, HID))
        x = x + _oracle_proj(projs[6], g, HID, INTER)
    xf = oracle.rms_norm(x, fnorm.astype(np.float32), 1e-5)
    if lm is not None:
        logits = _oracle_proj(lm, xf, VOCAB, HID)
    elif ekind == "i8":  # the tied lm_head reads the embedding in its own format (llama.rs:576-646)
        logits = oracle.llama_lm_head_i8(xf, ew, es.view(np.uint16))
    else:
        logits = oracle.llama_lm_head_f16_i4(ekind, xf, ew.view(np.uint16) if ekind == "f16" else ew,
                                             None if es is None else es.view(np.uint16), VOCAB, HID)
    return oracle.argmax_first(logits), logits


@pytest.mark.parametrize("case", ["u32", "i4", "mixed", "f16", "i8_embed_i4", "mixed_embed_f16"])
def test_runner_from_file_other_formats_match_oracle(tmp_path, case):
    """The runners' dtype dispatch from a .cellm file: projections as "u32"
    MLX affine (+ f32 .scales/.biases, as tools/convert_lfm.py writes them),
    "i4" (+ f16 .qscale) or "f16", each dispatched to its HIP GEMV; a mixed
    file also pairs an i8 gate with an i4 up (separate GEMVs + the SiLU
    kernel) and carries an i4 lm_head.  The embedding as "i8", "i4" or "f16"
    (embed_token, llama.rs:676-726) is also the tied lm_head in its own format
    ("i8_embed_i4" keeps the fused int8 launches with an i4 embedding).  Greedy
    ids of 4 sessions equal the oracle step's; logits within 1e-3."""
    from cellm_amd.llama_step import LlamaDevice

    kinds = {"u32": ["u32"] * 7, "i4": ["i4"] * 7, "f16": ["f16"] * 7, "i8_embed_i4": ["i8"] * 7,
             "mixed": ["u32", "i4", "i8", "u32", "i8", "i4", "u32"],
             "mixed_embed_f16": ["f16", "i8", "i4", "f16", "u32", "f16", "i8"]}[case]
    kinds = dict(enumerate(kinds))
    if case == "mixed":
        kinds["lm"] = "i4"
    kinds["embed"] = {"f16": "f16", "mixed_embed_f16": "f16", "i8_embed_i4": "i4"}.get(case, "i8")
    mm = _mixed_model(kinds)
    p = tmp_path / f"{case}.cellm"
    write_cellm(p, header(tied=case != "mixed"), _mixed_tensors(mm))
    k, v, bts = kv_state()
    dev = LlamaDevice.from_file(p, 0, max_rows=ROWS, max_blocks=CTX // TPB, tokens_per_block=TPB)
    try:
        ids, logits, _, _ = run(dev, k, v, bts)
    finally:
        dev.close()
    kc, vc = k.view(np.uint16).copy(), v.view(np.uint16).copy()
    tokens = [(100 + 7919 * s) % VOCAB for s in range(ROWS)]
    pos = [CTX - 1, 300, 64, 0]
    for s in range(ROWS):
        rid, rlog = _oracle_session(mm, kc, vc, tokens[s], pos[s], bts[s])
        assert int(ids[s]) == rid, (case, s)
        err = float(np.max(np.abs(logits[s] - rlog)) / np.max(np.abs(rlog)))
        assert err <= 1e-3, (case, s, err)
