"""cellm_hip_attention_gqa_f16kv_noalloc: the allocation-free variant of the
paged GQA attention (softmax partials in the library's static device scratch)
gives the same bits as cellm_hip_attention_gqa_f16kv, call after call, and
refuses inputs whose partials exceed the static array."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _util import rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from cellm_amd import HipOps

    o = HipOps(0)
    yield o
    o.close()


def _dev(a: np.ndarray):
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).cuda()
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda()
    return torch.from_numpy(a).cuda()


def _case(nh, nkv, hd, rows, blocks_per_row, positions, seed, L=3, tpb=16):
    total = rows * blocks_per_row + 3
    kvd = nkv * hd
    n = total * L * tpb * kvd
    k = oracle.gen_normal((n,), seed, 0.0, 1.0).astype(np.float16).view(np.uint16)
    v = oracle.gen_normal((n,), seed + 1, 0.0, 1.0).astype(np.float16).view(np.uint16)
    bt = np.array([[b * rows + r + 3 for b in range(blocks_per_row)] for r in range(rows)], np.uint32)
    q = np.stack([oracle.gen_normal((nh * hd,), seed + 2 + r, 0.0, 1.0) for r in range(rows)]).astype(np.float32)
    return dict(nh=nh, nkv=nkv, hd=hd, total=total, L=L, tpb=tpb, k=k, v=v, bt=bt, q=q,
                pos=np.array(positions, np.int32))


def _run(ops, c, noalloc, out):
    fn = ops.encode_attention_noalloc if noalloc else ops.encode_attention
    fn(_dev(c["q"]), _dev(c["k"]), _dev(c["v"]), _dev(c["bt"]), _dev(c["pos"]), out, c["nh"], c["nkv"], c["hd"],
       c["total"], c["L"], c["tpb"], 1)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_noalloc_matches_allocating_entry_point_twice(ops):
    """Two calls in a row, the second on a smaller input (fewer rows, heads and
    positions): each equals the allocating entry point bit for bit, and the
    oracle within the attention bar."""
    big = _case(15, 5, 64, 4, 34, (0, 31, 300, 543), 0xD0000300)
    small = _case(8, 2, 128, 2, 33, (79, 7), 0xD0000400)  # 528-position tables: the partials path
    for c in (big, small):
        rows, width = c["q"].shape
        out_na = torch.full((rows, width), float("nan"), dtype=torch.float32, device="cuda")
        out_ref = torch.full((rows, width), float("nan"), dtype=torch.float32, device="cuda")
        got = _run(ops, c, True, out_na)
        ref = _run(ops, c, False, out_ref)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        kvd = c["nkv"] * c["hd"]
        for r in range(rows):
            seq = int(c["pos"][r]) + 1
            bases = np.array([int(c["bt"][r][t // c["tpb"]]) * (c["L"] * c["tpb"] * kvd) + 1 * (c["tpb"] * kvd) +
                              (t % c["tpb"]) * kvd for t in range(seq)], np.uint64)
            o = oracle.attention_gqa_f16kv(c["k"], c["v"], bases, c["q"][r], c["nh"], c["nkv"], c["hd"])
            assert rel_err(got[r], o) <= 1e-5


def test_noalloc_refuses_more_than_the_static_scratch(ops):
    """64 heads of 128 over 32768 positions for 4 rows need 68 MB of partials:
    refused with a message that names the limit; nothing is launched."""
    from cellm_amd._lib import CellmHipError

    z = torch.zeros(16, dtype=torch.float32, device="cuda")
    pos = torch.zeros(4, dtype=torch.int32, device="cuda")
    bt = torch.zeros((4, 2048), dtype=torch.int32, device="cuda")
    with pytest.raises(CellmHipError, match="static scratch"):
        ops.encode_attention_noalloc(z, z, z, bt, pos, z, 64, 8, 128, 1, 1, 16, 0)
