"""f16, i2 and q1_0_g128 GEMVs on the device (cellm_hip_qgemv_f16 / _i2 /
_q1_0_g128) against the CPU oracle.

- Integer-valued x with weights whose products and partial sums are exact in
  f32 (small f16 integers, i2 with a power-of-two scale, q1 with a
  power-of-two d): any summation order gives the same bits, so the device
  result must equal the oracle exactly.
- Random inputs: the device sums in a different order than the reference's
  sequential loop; each output must lie within 2 * gamma_K * sum|w x| of the
  oracle (both are within gamma_K of the exact sum), and the normwise
  relative error within 1e-3.
- Shapes cover the fast kernel (whole 16-byte units, 1..4 activation rows,
  f32 and f16 x) and the generic one (K not a whole number of units, rows too
  long for LDS), plus the batch entry point and argument errors.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _util import rel_err

pytestmark = pytest.mark.gpu

U = 2.0 ** -24
I2_C = np.array([-1.5, -0.5, 0.5, 1.5], np.float64)


def gamma(k: int) -> float:
    return k * U / (1 - k * U)


def dev(a: np.ndarray):
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda()
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def within_bound(got, ref, absprod, k):
    bound = 2.0 * gamma(k) * absprod + 1e-30
    assert np.all(np.abs(got.astype(np.float64) - ref.astype(np.float64)) <= bound), \
        float(np.max(np.abs(got - ref) / bound))
    assert rel_err(got, ref) <= 1e-3


def f16_inputs(n, k, m, seed, xdt=np.float32):
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((n, k)).astype(np.float16)
    x = rng.standard_normal((m, k)).astype(xdt)
    return w, x


def i2_inputs(n, k, m, seed, xdt=np.float32):
    rng = np.random.default_rng(seed)
    w = rng.integers(0, 256, (n, (k + 3) // 4)).astype(np.uint8)
    s = rng.uniform(0.01, 0.05, n).astype(np.float16)
    x = rng.standard_normal((m, k)).astype(xdt)
    return w, s, x


def i2_values(w, k):
    q = (w[:, :, None] >> (2 * np.arange(4, dtype=np.uint8))) & 3
    return I2_C[q.reshape(w.shape[0], -1)[:, :k]]


def q1_inputs(n, k, m, seed, xdt=np.float32):
    rng = np.random.default_rng(seed)
    w = rng.integers(0, 256, (n, k // 128 * 18)).astype(np.uint8)
    d = rng.uniform(0.01, 0.1, (n, k // 128)).astype(np.float16)
    w.reshape(n, k // 128, 18)[:, :, :2] = d.view(np.uint8).reshape(n, k // 128, 2)
    x = rng.standard_normal((m, k)).astype(xdt)
    return w, x


def q1_values(w, k):
    n = w.shape[0]
    blk = w.reshape(n, k // 128, 18)
    d = blk[:, :, :2].copy().view(np.float16).astype(np.float64)[:, :, 0]
    bits = np.unpackbits(blk[:, :, 2:], axis=2, bitorder="little").astype(bool)
    return np.where(bits, d[:, :, None], -d[:, :, None]).reshape(n, k)


def out(m, n):
    return torch.empty((m, n), dtype=torch.float32, device="cuda")


# (k, n, m, x dtype): fast kernel shapes, then the generic kernel's
F16_CASES = [(896, 1152, 1, np.float32), (960, 2560, 4, np.float16), (4864, 896, 2, np.float32),
             (2048, 333, 3, np.float32), (100, 37, 3, np.float32), (12000, 64, 1, np.float16)]


@pytest.mark.parametrize("k,n,m,xdt", F16_CASES)
def test_f16_gemv_random(ops, k, n, m, xdt):
    w, x = f16_inputs(n, k, m, 0xF160 + k, xdt)
    y = out(m, n)
    ops.encode_qgemv_f16(dev(w), dev(x), y)
    torch.cuda.synchronize()
    ref = oracle.qgemv_f16(w.view(np.uint16), x)
    absprod = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    within_bound(y.cpu().numpy(), ref, absprod, k)


@pytest.mark.parametrize("k,n,m", [(1024, 300, 4), (104, 50, 1)])
def test_f16_gemv_exact_integers(ops, k, n, m):
    rng = np.random.default_rng(0xF16E)
    w = rng.integers(-8, 9, (n, k)).astype(np.float16)
    x = rng.integers(-4, 5, (m, k)).astype(np.float32)
    y = out(m, n)
    ops.encode_qgemv_f16(dev(w), dev(x), y)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), oracle.qgemv_f16(w.view(np.uint16), x))


I2_CASES = [(1152, 1536, 1, np.float32), (2048, 1000, 4, np.float16), (6912, 256, 2, np.float32),
            (1023, 77, 3, np.float32), (20000, 40, 1, np.float32), (1152, 6912, 1, np.float16),
            (1152, 700, 3, np.float16)]


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("k,n,m,xdt", I2_CASES)
def test_i2_gemv_random(ops, k, n, m, xdt, mode):
    w, s, x = i2_inputs(n, k, m, 0x120 + k, xdt)
    y = out(m, n)
    ops.encode_qgemv_i2(dev(w), dev(s.view(np.uint16)), mode, dev(x), y, k)
    torch.cuda.synchronize()
    ref = oracle.qgemv_i2(w, s.view(np.uint16), x, k, mode)
    absprod = (np.abs(x.astype(np.float64)) @ np.abs(i2_values(w, k)).T) * s.astype(np.float64)[None, :]
    within_bound(y.cpu().numpy(), ref, absprod, k + 1)


@pytest.mark.parametrize("xdt", [np.float32, np.float16])
@pytest.mark.parametrize("mode", [0, 1])
def test_i2_gemv_exact_integers(ops, mode, xdt):
    """f16 x takes the pair-packed dot2 kernel: (1024 + q) * x and the
    -1025.5 * sum(x) correction stay exact integers (or halves) here."""
    k, n, m = 1024, 500, 4
    rng = np.random.default_rng(0x12E)
    w = rng.integers(0, 256, (n, k // 4)).astype(np.uint8)
    s = np.full(n, 0.5, np.float16)
    x = rng.integers(-4, 5, (m, k)).astype(xdt)
    y = out(m, n)
    ops.encode_qgemv_i2(dev(w), dev(s.view(np.uint16)), mode, dev(x), y, k)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), oracle.qgemv_i2(w, s.view(np.uint16), x, k, mode))


Q1_CASES = [(1152, 1536, 1, np.float32), (2048, 1000, 4, np.float16), (4096, 300, 2, np.float32),
            (128, 9, 3, np.float32), (20480, 40, 1, np.float32), (1152, 6912, 1, np.float16),
            (1152, 700, 3, np.float16),
            # one row, N >= 32768, K <= 1152: the sign-sum table kernel (9, 8, 5 and 1 blocks per row)
            (1152, 40000, 1, np.float32), (1024, 32768, 1, np.float16), (640, 50000, 1, np.float16),
            (128, 65536, 1, np.float32)]


@pytest.mark.parametrize("k,n,m,xdt", Q1_CASES)
def test_q1_gemv_random(ops, k, n, m, xdt):
    w, x = q1_inputs(n, k, m, 0x1A0 + k, xdt)
    y = out(m, n)
    ops.encode_qgemv_q1_0_g128(dev(w), dev(x), y, k)
    torch.cuda.synchronize()
    ref = oracle.qgemv_q1_0_g128(w, x, k)
    absprod = np.abs(x.astype(np.float64)) @ np.abs(q1_values(w, k)).T
    within_bound(y.cpu().numpy(), ref, absprod, k)


@pytest.mark.parametrize("xdt", [np.float32, np.float16])
def test_q1_gemv_exact_integers_odd_row_offset(ops, xdt):
    """d = 0.25 everywhere, integer x: exact; the tensor starts 2 bytes into
    an allocation, so the 18-byte blocks sit on 2-byte boundaries only.  f16 x
    takes the pair-packed dot2 kernel."""
    k, n, m = 1024, 333, 4
    rng = np.random.default_rng(0x1AE)
    w = rng.integers(0, 256, (n, k // 128 * 18)).astype(np.uint8)
    d = np.full((n, k // 128), 0.25, np.float16)
    w.reshape(n, k // 128, 18)[:, :, :2] = d.view(np.uint8).reshape(n, k // 128, 2)
    x = rng.integers(-4, 5, (m, k)).astype(xdt)
    buf = torch.zeros(w.size + 16, dtype=torch.uint8, device="cuda")
    buf[2:2 + w.size] = torch.from_numpy(w.reshape(-1)).cuda()
    y = out(m, n)
    ops.encode_qgemv_q1_0_g128(buf[2:2 + w.size].view(n, -1), dev(x), y, k)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), oracle.qgemv_q1_0_g128(w, x, k))


@pytest.mark.parametrize("xdt", [np.float32, np.float16, "bf16"])
def test_q1_table_kernel_exact_integers(ops, xdt):
    """One row, N >= 32768: the sign-sum table path.  d = 0.25 and integer x
    keep every table entry and partial sum an exact integer (or quarter), so
    the result must equal the oracle bit for bit; N = 33001 leaves a ragged
    last row group (7 rows per group at K = 1152)."""
    k, n = 1152, 33001
    rng = np.random.default_rng(0x1AB)
    w = rng.integers(0, 256, (n, k // 128 * 18)).astype(np.uint8)
    d = np.full((n, k // 128), 0.25, np.float16)
    w.reshape(n, k // 128, 18)[:, :, :2] = d.view(np.uint8).reshape(n, k // 128, 2)
    x = rng.integers(-4, 5, (1, k)).astype(np.float32 if xdt == "bf16" else xdt)
    y = out(1, n)
    xd = dev(x).to(torch.bfloat16) if xdt == "bf16" else dev(x)  # small integers are exact in bf16
    ops.encode_qgemv_q1_0_g128(dev(w), xd, y, k)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), oracle.qgemv_q1_0_g128(w, x, k))


def test_lowbit_batch_matches_single_calls(ops):
    k, n, m = 1024, 640, 2
    wf, x = f16_inputs(n, k, m, 0xBA7)
    wi, si, _ = i2_inputs(n, k, m, 0xBA8)
    wq, _ = q1_inputs(n, k, m, 0xBA9)
    xd = dev(x)
    wfd, wid, sid, wqd = dev(wf), dev(wi), dev(si.view(np.uint16)), dev(wq)
    ys = [out(m, n) for _ in range(4)]
    ops.encode_qgemv_batch([ops.qgemv_op_f16(wfd, xd, ys[0]), ops.qgemv_op_i2(wid, sid, 0, xd, ys[1], k),
                            ops.qgemv_op_i2(wid, sid, 1, xd, ys[2], k), ops.qgemv_op_q1_0_g128(wqd, xd, ys[3], k)])
    zs = [out(m, n) for _ in range(4)]
    ops.encode_qgemv_f16(wfd, xd, zs[0])
    ops.encode_qgemv_i2(wid, sid, 0, xd, zs[1], k)
    ops.encode_qgemv_i2(wid, sid, 1, xd, zs[2], k)
    ops.encode_qgemv_q1_0_g128(wqd, xd, zs[3], k)
    torch.cuda.synchronize()
    for a, b in zip(ys, zs):
        np.testing.assert_array_equal(a.cpu().numpy(), b.cpu().numpy())


def test_lowbit_argument_errors(ops):
    from cellm_amd._lib import CellmHipError

    x = torch.zeros((1, 200), dtype=torch.float32, device="cuda")
    y = out(1, 4)
    w = torch.zeros((4, 200), dtype=torch.uint8, device="cuda")
    with pytest.raises(CellmHipError):  # q1 needs whole 128-element blocks
        ops.encode_qgemv_q1_0_g128(w, x, y, 200)
    s = torch.ones(4, dtype=torch.float16, device="cuda")
    with pytest.raises(CellmHipError):  # scale_mode is 0 or 1
        ops.encode_qgemv_i2(w, s, 2, x, y, 200)
