"""An independent float64 restatement of one Llama decode step, for tests.

It shares no code with `oracle/` or the runners: RMSNorm, rotate-half RoPE
(angles from numpy's float64 pow/cos/sin), GQA softmax attention over the
f16 K/V pages, SiLU and the int8 row GEMVs are written here in float64 from
their definitions (cpu_kernels.rs:17-34, :264-277; kvcache.rs:710-789;
llama.rs:235-647, :602-643).  The K/V row of the step is rounded to f16 as the
reference stores it.  The CPU-side helpers of the host-step runner and the
oracle's are restatements of each other; this is the check that is not.
"""
from __future__ import annotations

import numpy as np


def _f16(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


def f64_step(model, kcache, vcache, token, pos, bt, dims):
    """model = (layers, embed, escale, fnorm) with f16 scales/norms as uint16
    bits; kcache/vcache f16 bits, updated in place at `pos`; dims = dict of
    L, HID, NH, NKV, HD, VOCAB, EPS, THETA, TPB.  Returns (argmax, logits)."""
    L, NH, NKV, HD, TPB = dims["L"], dims["NH"], dims["NKV"], dims["HD"], dims["TPB"]
    eps, theta, vocab = dims["EPS"], dims["THETA"], dims["VOCAB"]
    kvd, half, G = NKV * HD, HD // 2, NH // NKV
    layers, embed, escale, fnorm = model

    def base(tpos, layer):
        return int(bt[tpos // TPB]) * (L * TPB * kvd) + layer * (TPB * kvd) + (tpos % TPB) * kvd

    def norm(v, w):
        return v / np.sqrt(np.mean(v * v) + eps) * _f16(w)

    def mv(w, s, v):
        return (w.astype(np.float64) @ v) * _f16(s)

    ang = pos * theta ** (-(2.0 * np.arange(half)) / HD)
    c, s = np.cos(ang), np.sin(ang)

    def rope(v, nh):
        v = v.reshape(nh, HD)
        a, b = v[:, :half].copy(), v[:, half:].copy()
        return np.concatenate([a * c - b * s, b * c + a * s], axis=1).reshape(-1)

    t = token % vocab
    x = embed[t].astype(np.float64) * _f16(escale[t:t + 1])[0]
    for layer in range(L):
        ws, ss, n1, n2 = layers[layer]
        xn = norm(x, n1)
        q = rope(mv(ws[0], ss[0], xn), NH)
        k = rope(mv(ws[1], ss[1], xn), NKV)
        v = mv(ws[2], ss[2], xn)
        wb = base(pos, layer)
        kcache[wb:wb + kvd] = k.astype(np.float16).view(np.uint16)
        vcache[wb:wb + kvd] = v.astype(np.float16).view(np.uint16)
        rows = np.array([base(tp, layer) for tp in range(pos + 1)])[:, None] + np.arange(kvd)
        K = kcache.view(np.float16)[rows].astype(np.float64)
        V = vcache.view(np.float16)[rows].astype(np.float64)
        att = np.empty(NH * HD)
        for h in range(NH):
            cols = slice((h // G) * HD, (h // G + 1) * HD)
            sc = K[:, cols] @ q[h * HD:(h + 1) * HD] / np.sqrt(HD)
            p = np.exp(sc - sc.max())
            att[h * HD:(h + 1) * HD] = (p / p.sum()) @ V[:, cols]
        x = x + mv(ws[3], ss[3], att)
        xn = norm(x, n2)
        g, u = mv(ws[4], ss[4], xn), mv(ws[5], ss[5], xn)
        x = x + mv(ws[6], ss[6], g / (1.0 + np.exp(-g)) * u)
    logits = (embed.astype(np.float64) @ norm(x, fnorm)) * _f16(escale)
    return int(np.argmax(logits)), logits
