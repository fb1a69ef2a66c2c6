"""The device decode runner over Qwen2-family .cellm files
(cellm_llama_dev_create_from_file with model_type "qwen*").

The Qwen2 layer is the Llama layer plus optional f16 biases on the
projections, added after each one (qwen.rs:1132-1139; the fused Metal step
qwen.rs:1361-1466 uploads them as f32, :232-239), and Qwen's weight formats:
i4 with several scales per row in groups of in / (scales per row)
(qwen.rs:1076-1077), i2 with the row scale on the sum (:1087-1096,
1591-1606) and q1_0_g128 (:1004-1022), also as an lm_head.  RoPE is the
half-split rotation of the fused step (qwen.rs:1401-1402), and the i8
lm_head applies the row scale to the sum (matmul_i8_f32, :592-600).

Each case decodes 4 sessions at Qwen2.5-0.5B layer shapes (hidden 896, 14 q /
2 kv heads, intermediate 4864; 2 layers, vocabulary 32768) and compares the
greedy ids with the oracle's step over the same formats (equal) and the
logits (within 1e-3 of the largest).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from _cellm_writer import llama_header, write_cellm

pytestmark = pytest.mark.gpu

L, HID, NH, NKV, HD, INTER, VOCAB = 2, 896, 14, 2, 64, 4864, 32768
TPB, CTX, ROWS = 16, 256, 4
KVD = NKV * HD
EPS, THETA = 1e-6, 1000000.0
NAMES = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
         "mlp.up_proj", "mlp.down_proj")
SHAPES = [(HID, HID), (KVD, HID), (KVD, HID), (HID, HID), (INTER, HID), (INTER, HID), (HID, INTER)]


def _proj(kind, o, i, sd):
    """(kind, arrays...) of one projection; weights scaled for unit-variance outputs."""
    if kind == "i8":
        return ("i8", oracle.gen_i8((o, i), sd),
                (oracle.gen_uniform((o,), sd + 1, 0.5, 1.5) / (73.3 * np.sqrt(i))).astype(np.float16))
    if kind.startswith("i4"):  # "i4" one scale per row, "i4g4" four groups per row
        g = int(kind[3:]) if len(kind) > 2 else 1
        w = oracle.gen_i8((o, (i + 1) // 2), sd).view(np.uint8)
        s = (oracle.gen_uniform((o * g,), sd + 1, 0.5, 1.5) / (4.6 * np.sqrt(i))).astype(np.float16)
        return ("i4", w, s, g)
    if kind == "i2":
        w = oracle.gen_i8((o, (i + 3) // 4), sd).view(np.uint8)
        s = (oracle.gen_uniform((o,), sd + 1, 0.5, 1.5) / np.sqrt(i)).astype(np.float16)
        return ("i2", w, s)
    if kind == "q1":
        w = oracle.gen_i8((o, i // 128 * 18), sd).view(np.uint8).copy()
        d = (oracle.gen_uniform((o, i // 128), sd + 1, 0.5, 1.5) / np.sqrt(i)).astype(np.float16)
        w.reshape(o, i // 128, 18)[:, :, :2] = d.view(np.uint8).reshape(o, i // 128, 2)
        return ("q1", w)
    if kind == "f16":
        return ("f16", oracle.gen_normal((o, i), sd, 0.0, 1.0 / np.sqrt(i)).astype(np.float16))
    assert kind == "u32"
    wq = oracle.gen_q4_words((o, i // 8), sd)
    base = 1.0 / (4.6 * np.sqrt(i))
    s = (oracle.gen_uniform((o, i // 64), sd + 1, 0.5, 1.5) * base).astype(np.float32)
    b = (-7.5 * s + oracle.gen_normal((o, i // 64), sd + 2, 0.0, 0.1 * base)).astype(np.float32)
    return ("u32", wq, s, b)


def _tensors(name, pr, o, i):
    k = pr[0]
    if k == "u32":
        base = name[:-len(".weight")]
        return [(name, pr[1], "u32", pr[1].shape), (base + ".scales", pr[2], "f32", pr[2].shape),
                (base + ".biases", pr[3], "f32", pr[3].shape)]
    if k == "f16":
        return [(name, pr[1], "f16", (o, i))]
    if k == "q1":
        return [(name, pr[1], "q1_0_g128", (o, i))]
    dt = {"i8": "i8", "i4": "i4", "i2": "i2"}[k]
    return [(name, pr[1], dt, (o, i)), (name + ".qscale", pr[2], "f16", pr[2].shape)]


def _apply(pr, x, o, i):
    """The Qwen runner's linear for each format (qwen.rs:1073-1101; u32 as lfm.rs:985-1066)."""
    k = pr[0]
    if k == "i8":
        return oracle.matmul_i8_f32(pr[1], pr[2].view(np.uint16), x)
    if k == "i4":
        g = pr[3]
        return oracle.matmul_i4_f32(pr[1], pr[2].view(np.uint16), o, i, i // g if g > 1 else i, x)
    if k == "i2":
        return oracle.qgemv_i2(pr[1], pr[2].view(np.uint16), x.reshape(1, -1), i, 0)[0]
    if k == "q1":
        return oracle.qgemv_q1_0_g128(pr[1], x.reshape(1, -1), i)[0]
    if k == "f16":
        return oracle.qgemv_f16(pr[1].view(np.uint16), x.reshape(1, -1))[0]
    return oracle.qgemv_q4_affine(pr[1], pr[2], pr[3], x.reshape(1, -1), i)[0]


def make_model(kinds, biased, embed_kind, lm_kind, base):
    layers = []
    for l in range(L):
        projs, biases = [], []
        for j, (o, i) in enumerate(SHAPES):
            sd = 0xA7000000 + l * 64 + j * 4
            projs.append(_proj(kinds[j], o, i, sd))
            biases.append(oracle.gen_normal((o,), sd + 3, 0.0, 0.5).astype(np.float16) if j in biased else None)
        n1 = (1.0 + 0.1 * oracle.lcg_fill(HID, 0xA7100000 + l, 1.0)).astype(np.float16)
        n2 = (1.0 + 0.1 * oracle.lcg_fill(HID, 0xA7200000 + l, 1.0)).astype(np.float16)
        layers.append((projs, biases, n1, n2))
    if embed_kind == "i8":
        emb = ("i8", oracle.gen_i8((VOCAB, HID), 0xA7300000),
               (oracle.gen_uniform((VOCAB,), 0xA7300001, 0.5, 1.5) / 127.0).astype(np.float16))
    elif embed_kind == "i4":
        w = oracle.gen_i8((VOCAB, HID // 2), 0xA7300000).view(np.uint8)
        emb = ("i4", w, (oracle.gen_uniform((VOCAB,), 0xA7300001, 0.5, 1.5) / 7.0).astype(np.float16), 1)
    else:
        emb = ("f16", oracle.gen_normal((VOCAB, HID), 0xA7300000, 0.0, 1.0).astype(np.float16))
    fnorm = (1.0 + 0.1 * oracle.lcg_fill(HID, 0xA7300002, 1.0)).astype(np.float16)
    lm = None if lm_kind is None else _proj(lm_kind, VOCAB, HID, 0xA7400000)
    return dict(layers=layers, emb=emb, fnorm=fnorm, lm=lm, base=base)


def file_tensors(m):
    base, ts = m["base"], []
    for l, (projs, biases, n1, n2) in enumerate(m["layers"]):
        pre = f"{base}layers.{l}."
        for j, name in enumerate(NAMES):
            o, i = SHAPES[j]
            ts += _tensors(pre + name + ".weight", projs[j], o, i)
            if biases[j] is not None:
                ts.append((pre + name + ".bias", biases[j], "f16", (o,)))
        ts.append((pre + "input_layernorm.weight", n1, "f16", (HID,)))
        ts.append((pre + "post_attention_layernorm.weight", n2, "f16", (HID,)))
    ts += _tensors(base + "embed_tokens.weight", m["emb"], VOCAB, HID)
    ts.append((base + "norm.weight", m["fnorm"], "f16", (HID,)))
    if m["lm"] is not None:
        ts += _tensors("lm_head.weight", m["lm"], VOCAB, HID)
    return ts


def header(tied=True, model_type="qwen2"):
    return llama_header(L, HID, NH, NKV, INTER, VOCAB, eps=EPS, theta=THETA, model_type=model_type,
                        tie_word_embeddings=tied)


def oracle_session(m, kc, vc, token, pos, bt):
    """QwenRunner's step for one session over the paged f16 cache (updated in place)."""
    ek = m["emb"][0]
    w = m["emb"][1].view(np.uint16) if ek == "f16" else m["emb"][1]
    s = None if ek == "f16" else m["emb"][2].view(np.uint16)
    x = oracle.embed(ek, [token], w, s, VOCAB, HID)[0]

    def base_of(tpos, layer):
        return int(bt[tpos // TPB]) * (L * TPB * KVD) + layer * (TPB * KVD) + (tpos % TPB) * KVD

    def lin(l, j, v):
        projs, biases = m["layers"][l][0], m["layers"][l][1]
        o, i = SHAPES[j]
        y = np.asarray(_apply(projs[j], v, o, i), np.float32)
        if biases[j] is not None:
            y = (y + biases[j].astype(np.float32)).astype(np.float32)
        return y

    for l, (_, _, n1, n2) in enumerate(m["layers"]):
        xn = oracle.rms_norm(x, n1.astype(np.float32), EPS)
        q, k, v = lin(l, 0, xn), lin(l, 1, xn), lin(l, 2, xn)
        oracle.rope_half_(q, NH, HD, pos, THETA)
        oracle.rope_half_(k, NKV, HD, pos, THETA)
        wb = base_of(pos, l)
        kc[wb:wb + KVD] = k.astype(np.float16).view(np.uint16)
        vc[wb:wb + KVD] = v.astype(np.float16).view(np.uint16)
        bases = np.array([base_of(tp, l) for tp in range(pos + 1)], np.uint64)
        attn = oracle.attention_gqa_f16kv(kc, vc, bases, q, NH, NKV, HD)
        x = x + lin(l, 3, attn)
        xn = oracle.rms_norm(x, n2.astype(np.float32), EPS)
        g = np.ascontiguousarray(lin(l, 4, xn), np.float32)
        oracle.silu_mul_(g, lin(l, 5, xn))
        x = x + lin(l, 6, g)
    xf = oracle.rms_norm(x, m["fnorm"].astype(np.float32), EPS)
    lm = m["lm"] if m["lm"] is not None else m["emb"]
    logits = np.asarray(_apply(lm, xf, VOCAB, HID), np.float32)
    return oracle.argmax_first(logits), logits


def kv_state():
    total = ROWS * CTX // TPB
    n = total * L * TPB * KVD
    k = oracle.gen_normal((n,), 0xA7500000, 0.0, 1.0).astype(np.float16)
    v = oracle.gen_normal((n,), 0xA7500001, 0.0, 1.0).astype(np.float16)
    bts = np.array([[b * ROWS + s for b in range(CTX // TPB)] for s in range(ROWS)], np.uint32)
    return k, v, bts


CASES = {
    # Qwen2.5 structure: int8 projections, q/k/v biases, tied int8 embedding
    "i8_qkv_bias": (["i8"] * 7, {0, 1, 2}, "i8", None, "model."),
    # every format of the dispatch, biases on all seven projections, i4 embedding, q1_0_g128 lm_head
    "mixed_all_bias": (["u32", "i4g4", "i2", "q1", "f16", "i8", "u32"], set(range(7)), "i4", "q1", "model."),
    # MLX affine projections with q/k/v biases under the "model.language_model." prefix, f16 embedding
    "u32_prefix_f16_embed": (["u32"] * 7, {0, 1, 2}, "f16", None, "model.language_model."),
    # int8 attention with biases, i2 MLP and an i2 lm_head (qwen.rs:611-619)
    "i2_mlp_i2_lm_head": (["i8", "i8", "i8", "i8", "i2", "i2", "i2"], {0, 1, 2}, "i8", "i2", "model."),
}


@pytest.mark.parametrize("case", list(CASES))
def test_qwen_runner_from_file_matches_oracle(tmp_path, case):
    from cellm_amd.llama_step import LlamaDevice

    kinds, biased, ek, lk, base = CASES[case]
    m = make_model(kinds, biased, ek, lk, base)
    p = tmp_path / f"{case}.cellm"
    write_cellm(p, header(tied=lk is None), file_tensors(m))
    k, v, bts = kv_state()
    print(f"case {case}", flush=True)
    dev = LlamaDevice.from_file(p, 0, max_rows=ROWS, max_blocks=CTX // TPB, tokens_per_block=TPB)
    try:
        dev.kv_upload(k, v)
        tokens = np.array([(100 + 7919 * s) % VOCAB for s in range(ROWS)], np.uint32)
        pos = np.array([CTX - 1, 200, 17, 0], np.int32)
        ids, _, logits = dev.step(tokens, pos, bts, want_logits=True)
    finally:
        dev.close()
    kc, vc = k.view(np.uint16).copy(), v.view(np.uint16).copy()
    for s in range(ROWS):
        rid, rlog = oracle_session(m, kc, vc, int(tokens[s]), int(pos[s]), bts[s])
        err = float(np.max(np.abs(logits[s] - rlog)) / np.max(np.abs(rlog)))
        assert err <= 1e-3, (case, s, err)
        assert int(ids[s]) == rid, (case, s)


def test_qwen_runner_refusals(tmp_path):
    from cellm_amd._lib import CellmHipError
    from cellm_amd.llama_step import LlamaDevice

    m = make_model(["i8"] * 7, {0, 1, 2}, "i8", None, "model.")
    ts = file_tensors(m)
    kw = dict(max_rows=ROWS, max_blocks=CTX // TPB, tokens_per_block=TPB)
    p = tmp_path / "r.cellm"
    write_cellm(p, header(model_type="qwen3_5_text"), ts)
    with pytest.raises(CellmHipError, match="qwen3_5_text"):
        LlamaDevice.from_file(p, 0, **kw)
    qn = np.ones(HD, np.float16)
    write_cellm(p, header(), ts + [("model.layers.1.self_attn.k_norm.weight", qn, "f16", (HD,))])
    with pytest.raises(CellmHipError, match="k_norm.weight: q/k norms are not supported"):
        LlamaDevice.from_file(p, 0, **kw)
    # i2 is a Qwen/Gemma arm: a Llama file with it is refused, as llama.rs:935-939 refuses it
    mi = make_model(["i8", "i8", "i8", "i8", "i2", "i8", "i8"], set(), "i8", None, "model.")
    write_cellm(p, header(model_type="llama"), file_tensors(mi))
    with pytest.raises(CellmHipError, match="gate_proj.weight is i2"):
        LlamaDevice.from_file(p, 0, **kw)
    # grouped i4 scales must cover the row: 3 groups of 896 // 3 = 298 leave 2 columns
    mg = make_model(["i4g3", "i8", "i8", "i8", "i8", "i8", "i8"], set(), "i8", None, "model.")
    write_cellm(p, header(), file_tensors(mg))
    with pytest.raises(CellmHipError, match="do not cover"):
        LlamaDevice.from_file(p, 0, **kw)
