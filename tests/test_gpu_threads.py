"""One context shared by two host threads on one stream.

The entry points that use a context's per-stream scratch (the split-K qGEMM's
partials, the unfused gate/up's up rows, the attention's softmax partials)
hold the context's mutex from taking the buffer until their last kernel is
enqueued, so calls from several threads queue their scratch users back to
back.  Both threads run every scratch user many times, interleaved, and the
outputs of every repetition of each thread must equal what the same calls
give run alone: a thread that reduced the other's partials, or read its up
rows, would differ.
"""
from __future__ import annotations

import threading

import numpy as np
import pytest

import oracle
from tests._util import make_q4

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    if a.dtype == np.uint32:
        a = a.view(np.int32)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def _case(i):
    """Inputs of one thread: a split-K qGEMM (4864 -> 896 at M = 128: 8 K
    splits), an f32-x q4 gate/up (two GEMVs + SiLU through the up scratch) and
    a paged attention (its partials scratch)."""
    import torch

    c = {}
    wq, s, b, x = make_q4(896, 4864, 128, cfg=4, salt=90 + i)
    c["gemm"] = (_dev(wq), _dev(s).view(torch.float16), _dev(b).view(torch.float16), _dev(x))
    gw, gs, gb, gx = make_q4(2560, 960, 3, x_dtype=np.float32, salt=92 + i)
    uw, us, ub, _ = make_q4(2560, 960, 3, salt=94 + i)
    c["gu"] = (_dev(gw), _dev(gs).view(torch.float16), _dev(gb).view(torch.float16), _dev(uw),
               _dev(us).view(torch.float16), _dev(ub).view(torch.float16), _dev(gx))
    L, tpb, nkv, hd, nh, rows, blocks = 2, 16, 5, 64, 15, 4, 40
    total = rows * blocks + 3
    n = total * L * tpb * nkv * hd
    k = oracle.gen_normal((n,), 0xE000 + i, 0.0, 1.0).astype(np.float16).view(np.uint16)
    v = oracle.gen_normal((n,), 0xE100 + i, 0.0, 1.0).astype(np.float16).view(np.uint16)
    bt = np.array([[bb * rows + r + 3 for bb in range(blocks)] for r in range(rows)], np.uint32)
    q = np.stack([oracle.gen_normal((nh * hd,), 0xE200 + 16 * i + r, 0.0, 1.0) for r in range(rows)]).astype(np.float32)
    pos = np.array([639, 100 + i, 5, 300], np.int32)
    c["attn"] = (_dev(q), _dev(k).view(torch.float16), _dev(v).view(torch.float16), _dev(bt), _dev(pos), nh, nkv, hd,
                 total, L, tpb)
    return c


def _outs():
    import torch

    return {"gemm": torch.empty((128, 896), dtype=torch.float32, device="cuda"),
            "gu": torch.empty((3, 2560), dtype=torch.float32, device="cuda"),
            "attn": torch.empty((4, 15 * 64), dtype=torch.float32, device="cuda")}


def _run(ops, c, o, stream):
    ops.encode_qgemm_q4_affine(*c["gemm"], o["gemm"], stream=stream)
    g = c["gu"]
    ops.encode_gate_up_silu_q4_affine(g[0], g[1], g[2], g[3], g[4], g[5], g[6], o["gu"], stream=stream)
    q, k, v, bt, pos, nh, nkv, hd, total, L, tpb = c["attn"]
    ops.encode_attention(q, k, v, bt, pos, o["attn"], nh, nkv, hd, total, L, tpb, 1, stream=stream)


def test_two_threads_share_one_context_and_stream(ops):
    import torch

    st = torch.cuda.Stream()
    sp = st.cuda_stream
    cases = [_case(0), _case(1)]
    refs = []
    for c in cases:
        o = _outs()
        _run(ops, c, o, sp)
        st.synchronize()
        refs.append({key: t.clone() for key, t in o.items()})
    reps = 40
    outs = [_outs(), _outs()]
    # every repetition's outputs, copied on the same stream right after it: a repetition whose scratch was
    # overwritten by the other thread shows up even if a later one is clean
    hist = [{key: torch.empty((reps,) + tuple(t.shape), dtype=t.dtype, device="cuda") for key, t in o.items()}
            for o in outs]
    errors = []
    start = threading.Barrier(2)

    def work(i):
        try:
            start.wait()
            with torch.cuda.stream(st):
                for r in range(reps):
                    _run(ops, cases[i], outs[i], sp)
                    for key, t in outs[i].items():
                        hist[i][key][r].copy_(t)
        except Exception as e:  # reported below, in the main thread
            errors.append(e)

    threads = [threading.Thread(target=work, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    st.synchronize()
    assert not errors, errors
    for i in range(2):
        for key in refs[i]:
            for r in range(reps):
                assert torch.equal(hist[i][key][r], refs[i][key]), (i, key, r)
    # the two threads' inputs differ, so equal outputs cannot come from a shared mix-up
    assert not torch.equal(refs[0]["gemm"], refs[1]["gemm"])
