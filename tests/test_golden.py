"""The committed golden fixtures: the oracle still reproduces them bit for bit,
and the fixture inputs satisfy the closed forms that pin them."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import oracle

G = np.load(Path(__file__).resolve().parent / "golden" / "golden_v1.npz")


def test_golden_i8():
    assert np.array_equal(oracle.qgemv_i8(G["i8_w"], G["i8_s"], G["i8_x"]), G["i8_y"])
    assert np.array_equal(oracle.matmul_i8_f32(G["i8_w"], G["i8_s16"], G["i8_x"][0]), G["i8_y16"])


def test_golden_q4():
    k = G["q4_wq"].shape[1] * 8
    assert np.array_equal(oracle.qgemv_q4_affine(G["q4_wq"], G["q4_s"], G["q4_b"], G["q4_x"], k), G["q4_y"])
    assert np.array_equal(oracle.dequant_q4_affine_f16(G["q4_wq"], G["q4_s"], G["q4_b"], k), G["q4_deq16"])
    assert np.array_equal(oracle.q4_affine_dequant_f32(G["q4_wq"], G["q4_s"], G["q4_b"], k), G["q4_deq32"])
    # the f16 dequant is the RNE of the f32 dequant (IEEE, numpy)
    assert np.array_equal(G["q4_deq32"].astype(np.float16).view(np.uint16), G["q4_deq16"])


def test_golden_i4():
    n, k = G["i4_w"].shape[0], G["i4_w"].shape[1] * 2
    assert np.array_equal(oracle.matmul_i4_f32(G["i4_w"], G["i4_s"], n, k, 64, G["i4_x"]), G["i4_y"])


@pytest.mark.gpu
def test_golden_on_gpu(ops):
    """The HIP path through the C ABI against the committed fixtures."""
    import torch

    d = lambda a: torch.from_numpy(a.view(np.int32) if a.dtype == np.uint32 else a).cuda()
    y = torch.empty(G["i8_y"].shape, dtype=torch.float32, device="cuda")
    ops.encode_qgemv_i8(d(G["i8_w"]), d(G["i8_s"]), d(G["i8_x"]), y)
    torch.cuda.synchronize()
    r = G["i8_y"]
    assert np.max(np.abs(y.cpu().numpy() - r)) / np.max(np.abs(r)) <= 1e-3
    yq = torch.empty(G["q4_y"].shape, dtype=torch.float32, device="cuda")
    ops.encode_qgemv_q4_affine(d(G["q4_wq"]), d(G["q4_s"]), d(G["q4_b"]), d(G["q4_x"]), yq)
    h = torch.empty(G["q4_deq16"].shape, dtype=torch.float16, device="cuda")
    ops.encode_dequant_q4_affine(d(G["q4_wq"]), d(G["q4_s"]), d(G["q4_b"]), h)
    torch.cuda.synchronize()
    r = G["q4_y"]
    assert np.max(np.abs(yq.cpu().numpy() - r)) / np.max(np.abs(r)) <= 1e-3
    assert np.array_equal(h.cpu().numpy().view(np.uint16), G["q4_deq16"])
