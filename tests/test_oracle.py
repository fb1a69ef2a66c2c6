"""Pins of the CPU oracle (oracle/cellm_oracle.c) without the reference.

The reference is Rust (no toolchain here) and ships no tests or fixtures for
these kernels, so each oracle function is checked against something the
mathematics fixes, built from different primitives than the oracle's C loops:
  * IEEE-754 conversions from numpy (exhaustive over f16);
  * strict left-to-right f32 sums via np.add.accumulate (sequential in numpy),
    which is the order the reference's x86 loops use;
  * integer closed forms where every partial sum is exact;
  * fp64 error bounds gamma_K * sum|w x|;
  * known-answer nibble/byte words and brute force on tiny shapes.
Each test names the plausible mistake it catches.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle

U = 2.0 ** -24


def seq_sum_f32(p: np.ndarray) -> np.float32:
    """Strict left-to-right f32 sum (np.add.accumulate does not reassociate)."""
    p = np.asarray(p, np.float32)
    if p.size == 0:
        return np.float32(0.0)
    return np.add.accumulate(p, dtype=np.float32)[-1]


def gamma(k: int) -> float:
    return k * U / (1 - k * U)


# ------------------------------------------------------------ conversions ----

def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    ours = oracle.f16_bits_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))  # signed zeros too


def test_f32_to_f16_rne_matches_numpy():
    rng = np.random.default_rng(1)
    vals = [rng.standard_normal(200000).astype(np.float32) * s for s in (1e-6, 1e-3, 1.0, 1e3, 6e4)]
    # every f16 value, the midpoints between neighbours (ties) and one ulp either side
    h = np.arange(0, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((h[:-1] + h[1:]) / 2).astype(np.float32)
    vals += [h.astype(np.float32), mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(0))]
    vals += [np.array([65504.0, 65519.99, 65520.0, 1e9, 2.0 ** -25, 2.0 ** -26, 3 * 2.0 ** -26, 0.0, -0.0, np.inf,
                       -np.inf], np.float32)]
    x = np.concatenate(vals).astype(np.float32)
    x = np.concatenate([x, -x])
    ours = oracle.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


def test_f32_to_f16_nan_is_quiet():
    out = oracle.f32_to_f16_bits(np.array([np.nan], np.float32))
    assert out[0] & 0x7c00 == 0x7c00 and out[0] & 0x3ff


# ------------------------------------------------------------------ LCG ----

def test_lcg_deterministic_and_in_range():
    a = oracle.lcg_fill(1000, 0xA11CE, 0.8)
    b = oracle.lcg_fill(1000, 0xA11CE, 0.8)
    assert np.array_equal(a, b) and np.all(np.abs(a) <= 0.8)
    # first draw by exact integer arithmetic: s1 = seed*6364136223846793005 + 1 mod 2^64
    s1 = (0xA11CE * 6364136223846793005 + 1) % 2 ** 64
    u = np.float32(np.float32(s1 >> 32) / np.float32(2 ** 32 - 1))
    assert a[0] == np.float32((u * np.float32(2.0) - np.float32(1.0)) * np.float32(0.8))
    w = oracle.gen_q4_words((4096,), 3)
    nib = (w[:, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF
    assert set(np.unique(nib)) == set(range(16))
    q = oracle.gen_i8((100000,), 5)
    assert q.min() == -127 and q.max() == 127
    s = oracle.gen_normal((10000,), 9, 0.02, 0.005, positive_only=True)
    assert s.min() > 0 and abs(float(s.mean()) - 0.02) < 5e-4


# ---------------------------------------------------------- int8 per-row ----

def test_i8_closed_form_exact_integers():
    """Integer x in [-4,4], power-of-two scales, K <= 4096: every partial sum is
    exact, so any order gives the integer dot * scale (catches a dropped or
    per-element-misplaced scale, wrong row/column indexing)."""
    rng = np.random.default_rng(2)
    n, k = 37, 4096
    w = rng.integers(-127, 128, (n, k)).astype(np.int8)
    x = rng.integers(-4, 5, k).astype(np.float32)
    e = rng.integers(-12, -4, n)
    s = (2.0 ** e).astype(np.float16)
    y = oracle.matmul_i8_f32(w, s.view(np.uint16), x)
    exact = (w.astype(np.int64) @ x.astype(np.int64)).astype(np.float64) * s.astype(np.float64)
    assert np.array_equal(y.astype(np.float64), exact)


def test_i8_sequential_order_bit_exact():
    """x86 branch: acc += f32(w)*x left to right, then * scale."""
    rng = np.random.default_rng(3)
    n, k = 9, 577
    w = rng.integers(-127, 128, (n, k)).astype(np.int8)
    x = rng.standard_normal(k).astype(np.float32)
    s = rng.uniform(1e-3, 2e-2, n).astype(np.float16)
    y = oracle.matmul_i8_f32(w, s.view(np.uint16), x)
    for r in range(n):
        acc = seq_sum_f32(w[r].astype(np.float32) * x)
        assert y[r] == np.float32(acc * np.float32(s[r]))


def test_i8_fp64_bound_and_batched_rows():
    rng = np.random.default_rng(4)
    n, k, m = 50, 1152, 3
    w = rng.integers(-127, 128, (n, k)).astype(np.int8)
    x = rng.standard_normal((m, k)).astype(np.float16)
    s = rng.uniform(1e-3, 2e-2, n).astype(np.float32)
    y = oracle.qgemv_i8(w, s, x)
    ref = (x.astype(np.float64) @ w.astype(np.float64).T) * s[None, :]
    bound = gamma(k + 1) * (np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T) * s[None, :]
    assert np.all(np.abs(y - ref) <= bound + 1e-30)
    # batched form = the reference row GEMV on each activation row
    for i in range(m):
        yi = oracle.qgemv_i8(w, s, x[i:i + 1])
        assert np.array_equal(yi[0], y[i])


def test_llama_lm_head_i8_per_element_scale_and_nonfinite():
    """llama.rs:602-643: acc += x * (f32(w) * scale); non-finite -> -inf."""
    rng = np.random.default_rng(5)
    v, h = 6, 64
    w = rng.integers(-127, 128, (v, h)).astype(np.int8)
    s = rng.uniform(1e-3, 2e-2, v).astype(np.float16)
    x = rng.standard_normal(h).astype(np.float32)
    y = oracle.llama_lm_head_i8(x, w, s.view(np.uint16))
    for r in range(v):
        assert y[r] == seq_sum_f32(x * (w[r].astype(np.float32) * np.float32(s[r])))
    x[3] = np.inf
    w[0, 3] = 5   # +inf -> -inf
    w[1, 3] = -5  # -inf stays -inf
    w[2, 3] = 0   # inf * 0 = nan -> -inf
    y = oracle.llama_lm_head_i8(x, w, s.view(np.uint16))
    assert np.all(np.isneginf(y))


def test_embed_f16_i8_i4_known_answers_and_wrap():
    """llama.rs:676-726: f16 rows widen exactly (every f16 pattern against
    numpy); i8 rows are f32(w) * scale; i4 byte 0x8F -> [7, 0] (low nibble
    even, q = nib - 8) times the row scale, ceil(hidden/2) bytes per row for
    an odd hidden; the token wraps modulo the vocabulary (:684)."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16).reshape(1, -1)
    got = oracle.embed("f16", [0], bits, None, 1, 65536)[0]
    want = bits[0].view(np.float16).astype(np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    rng = np.random.default_rng(41)
    v, h = 5, 7
    w8 = rng.integers(-127, 128, (v, h)).astype(np.int8)
    s = rng.uniform(1e-3, 2e-2, v).astype(np.float16)
    got = oracle.embed("i8", [3, v + 1], w8, s.view(np.uint16), v, h)
    assert np.array_equal(got[0], w8[3].astype(np.float32) * np.float32(s[3]))
    assert np.array_equal(got[1], w8[1].astype(np.float32) * np.float32(s[1]))
    w4 = np.zeros((v, (h + 1) // 2), np.uint8)
    w4[2, 0], w4[2, 3] = 0x8F, 0xE1  # elements 0, 1 = 7, 0; element 6 = 1 - 8 (its high nibble has no element)
    got = oracle.embed("i4", [2], w4, s.view(np.uint16), v, h)[0]
    sc = np.float32(s[2])
    want = np.array([7, 0, -8, -8, -8, -8, -7], np.float32) * sc
    assert np.array_equal(got, want)
    # every byte value, both nibbles, against numpy's own unpacking
    w4 = np.arange(256, dtype=np.uint8).reshape(1, 256)
    got = oracle.embed("i4", [0], w4, np.array([0x3C00], np.uint16), 1, 512)[0]
    want = np.empty(512, np.float32)
    want[0::2] = (w4[0] & 0xF).astype(np.int32) - 8
    want[1::2] = (w4[0] >> 4).astype(np.int32) - 8
    assert np.array_equal(got, want)


def test_llama_lm_head_f16_i4_order_bounds_and_nonfinite():
    """llama.rs:576-646 for f16 and i4 sources: strict left-to-right sums of
    x * f32(w) and (x * val) * scale; integer data with a power-of-two scale
    is exact; random data within gamma_K of an fp64 dot; non-finite -> -inf."""
    rng = np.random.default_rng(42)
    v, h = 6, 96
    wf = rng.standard_normal((v, h)).astype(np.float16)
    x = rng.standard_normal(h).astype(np.float32)
    y = oracle.llama_lm_head_f16_i4("f16", x, wf.view(np.uint16), None, v, h)
    for r in range(v):
        assert y[r] == seq_sum_f32(x * wf[r].astype(np.float32))
        exact = float(np.dot(x.astype(np.float64), wf[r].astype(np.float64)))
        bound = gamma(h) * float(np.sum(np.abs(x.astype(np.float64) * wf[r].astype(np.float64))))
        assert abs(float(y[r]) - exact) <= bound
    w4 = rng.integers(0, 256, (v, (h + 1) // 2)).astype(np.uint8)
    s = rng.uniform(1e-3, 2e-2, v).astype(np.float16)
    y = oracle.llama_lm_head_f16_i4("i4", x, w4, s.view(np.uint16), v, h)
    q = np.empty((v, h), np.float32)
    q[:, 0::2] = (w4 & 0xF).astype(np.int32) - 8
    q[:, 1::2] = (w4 >> 4).astype(np.int32) - 8
    for r in range(v):
        assert y[r] == seq_sum_f32((x * q[r]) * np.float32(s[r]))
        exact = float(np.dot(x.astype(np.float64), q[r].astype(np.float64))) * float(np.float32(s[r]))
        bound = 2 * gamma(h + 2) * float(np.sum(np.abs(x.astype(np.float64) * q[r]))) * float(np.float32(s[r]))
        assert abs(float(y[r]) - exact) <= bound
    # integer x, power-of-two scale: every partial sum exact
    xi = rng.integers(-4, 5, h).astype(np.float32)
    s2 = np.full(v, 0.25, np.float16)
    y = oracle.llama_lm_head_f16_i4("i4", xi, w4, s2.view(np.uint16), v, h)
    assert np.array_equal(y, (q.astype(np.int64) @ xi.astype(np.int64)).astype(np.float32) * np.float32(0.25))
    x[5] = np.inf
    wf[0, 5], wf[1, 5], wf[2, 5] = 1.0, -1.0, 0.0
    y = oracle.llama_lm_head_f16_i4("f16", x, wf.view(np.uint16), None, v, h)
    assert np.all(np.isneginf(y[:3]))


# ----------------------------------------------------------------- i4 sym ----

def test_i4_known_answer_and_order():
    """byte 0x8F -> elements [7, 0] (low nibble even, q = nib - 8)."""
    w = np.array([[0x8F, 0x08]], np.uint8)  # elements: 7, 0, 0, -8
    s = np.array([1.0], np.float16).view(np.uint16)
    x = np.array([1.0, 10.0, 100.0, 1000.0], np.float32)
    y = oracle.matmul_i4_f32(w, s, 1, 4, 4, x)
    assert y[0] == np.float32(7.0 - 8000.0)
    rng = np.random.default_rng(6)
    n, k, gs = 5, 256, 64
    w = rng.integers(0, 256, (n, k // 2)).astype(np.uint8)
    s = rng.uniform(1e-3, 2e-2, n * (k // gs)).astype(np.float16)
    x = rng.standard_normal(k).astype(np.float32)
    y = oracle.matmul_i4_f32(w, s.view(np.uint16), n, k, gs, x)
    q = np.empty((n, k), np.float32)
    q[:, 0::2] = (w & 0xF).astype(np.int32) - 8
    q[:, 1::2] = (w >> 4).astype(np.int32) - 8
    for r in range(n):
        sc = np.repeat(s[r * (k // gs):(r + 1) * (k // gs)].astype(np.float32), gs)
        assert y[r] == seq_sum_f32((q[r] * sc) * x)


# --------------------------------------------------------------- affine ----

def _unpack(wq: np.ndarray) -> np.ndarray:
    return ((wq[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(wq.shape[0], -1)


def test_affine_nibble_order_known_answer():
    """u32 0x76543210 -> q = 0..7 and 0xFEDCBA98 -> 8..15 (nibble j = bits 4j..4j+3)."""
    wq = np.array([[0x76543210, 0xFEDCBA98] * 4], np.uint32)  # K = 64, one group
    s = np.array([[1.0]], np.float32)
    b = np.array([[0.0]], np.float32)
    w = oracle.q4_affine_dequant_f32(wq, s, b, 64)
    assert np.array_equal(w[0, :16], np.arange(16, dtype=np.float32))
    # exhaustive 16-value sweep through scale and bias
    s = np.array([[0.37]], np.float32)
    b = np.array([[-1.25]], np.float32)
    w = oracle.q4_affine_dequant_f32(wq, s, b, 64)
    qs = np.arange(16, dtype=np.float32)
    assert np.array_equal(w[0, :16], (qs * np.float32(0.37)) + np.float32(-1.25))


def test_affine_dequant_two_roundings_and_groups():
    rng = np.random.default_rng(7)
    n, k = 6, 320  # 5 groups
    wq = rng.integers(0, 2 ** 32, (n, k // 8), dtype=np.uint64).astype(np.uint32)
    s = rng.standard_normal((n, 5)).astype(np.float32)
    b = rng.standard_normal((n, 5)).astype(np.float32)
    w = oracle.q4_affine_dequant_f32(wq, s, b, k)
    q = _unpack(wq).astype(np.float32)
    sg, bg = np.repeat(s, 64, axis=1), np.repeat(b, 64, axis=1)
    assert np.array_equal(w, (q * sg) + bg)  # numpy rounds each op in f32: mul then add
    fused = (q.astype(np.float64) * sg + bg).astype(np.float32)  # one rounding
    assert not np.array_equal(w, fused), "data should separate one and two roundings"


def test_affine_gemv_sequential_bit_exact_and_lm_head_equal():
    rng = np.random.default_rng(8)
    n, k, m = 11, 896, 2
    wq = rng.integers(0, 2 ** 32, (n, k // 8), dtype=np.uint64).astype(np.uint32)
    s = np.abs(rng.normal(0.02, 0.005, (n, k // 64))).astype(np.float16)
    b = rng.normal(0, 0.05, (n, k // 64)).astype(np.float16)
    x = rng.standard_normal((m, k)).astype(np.float16)
    y = oracle.qgemv_q4_affine(wq, s, b, x, k)
    w = oracle.q4_affine_dequant_f32(wq, s, b, k)
    for i in range(m):
        for r in range(n):
            assert y[i, r] == seq_sum_f32(w[r] * x[i].astype(np.float32))
    # the affine lm_head (lfm.rs:700-741) with f32 scale/bias files gives the same bits as the GEMV
    s32, b32 = s.astype(np.float32), b.astype(np.float32)
    lm = oracle.lfm_lm_head_q4_affine(wq, s32, b32, x[0].astype(np.float32), n, k)
    assert np.array_equal(lm, oracle.qgemv_q4_affine(wq, s32, b32, x[0:1].astype(np.float32), k)[0])


def test_affine_gemv_fp64_bound_brute_force_tiny():
    rng = np.random.default_rng(9)
    for k in (8, 16, 64, 128):
        for n in range(1, 8):
            wq = rng.integers(0, 2 ** 32, (n, k // 8), dtype=np.uint64).astype(np.uint32)
            g = (k + 63) // 64
            s = rng.uniform(0.01, 0.03, (n, g)).astype(np.float32)
            b = rng.normal(0, 0.05, (n, g)).astype(np.float32)
            x = rng.standard_normal((1, k)).astype(np.float32)
            y = oracle.qgemv_q4_affine(wq, s, b, x, k)[0]
            q = _unpack(wq).astype(np.float64)
            w64 = q * np.repeat(s, 64, axis=1)[:, :k] + np.repeat(b, 64, axis=1)[:, :k]
            ref = w64 @ x[0].astype(np.float64)
            bound = (gamma(k) + 3 * U) * (np.abs(w64) @ np.abs(x[0].astype(np.float64)))
            assert np.all(np.abs(y - ref) <= bound + 1e-30), (k, n)


def test_dequant_f16_rne_and_double_rounding():
    rng = np.random.default_rng(10)
    n, k = 8, 256
    wq = rng.integers(0, 2 ** 32, (n, k // 8), dtype=np.uint64).astype(np.uint32)
    for dt in (np.float32, np.float16):
        s = rng.normal(0.02, 0.005, (n, 4)).astype(dt)
        b = rng.normal(0, 0.05, (n, 4)).astype(dt)
        h = oracle.dequant_q4_affine_f16(wq, s, b, k)
        w32 = oracle.q4_affine_dequant_f32(wq, s, b, k)
        assert np.array_equal(h, w32.astype(np.float16).view(np.uint16))
    # q=3, s = 1+2^-10 (an f16), b = -2^-24: q*s = 3.0029296875 is an f16 midpoint;
    # f32 rounding of q*s+b lands back on it and RNE picks the even neighbour, the
    # reference's double rounding; a single rounding would pick the lower value.
    wq1 = np.array([[3]], np.uint32)
    s1 = np.array([[1 + 2 ** -10]], np.float16)
    b1 = np.array([[-(2.0 ** -24)]], np.float16)
    h1 = oracle.dequant_q4_affine_f16(wq1, s1, b1, 8, 64)[0, 0]
    single = np.float16(np.float64(3) * np.float64(s1[0, 0]) + np.float64(b1[0, 0])).view(np.uint16)
    double = np.float16(np.float32(3) * np.float32(s1[0, 0]) + np.float32(b1[0, 0])).view(np.uint16)
    assert h1 == double and h1 != single


# ------------------------------------------------------------------- dense ----

def test_matmul_f32_accumulates_into_out_sequentially():
    rng = np.random.default_rng(11)
    m, k, n = 3, 17, 5
    a = rng.standard_normal((m, k)).astype(np.float32)
    bm = rng.standard_normal((k, n)).astype(np.float32)
    out0 = rng.standard_normal((m, n)).astype(np.float32)
    out = oracle.matmul_f32(a, bm, out0.copy())
    for i in range(m):
        for j in range(n):
            p = np.concatenate([[out0[i, j]], a[i] * bm[:, j]]).astype(np.float32)
            assert out[i, j] == seq_sum_f32(p)
    # n == 1 path: row dot
    v = oracle.matmul_f32(a, bm[:, :1].copy())
    for i in range(m):
        assert v[i] == seq_sum_f32(a[i] * bm[:, 0])


def test_gemm_xwT_equals_matmul_over_transposed_weight():
    rng = np.random.default_rng(12)
    m, k, n = 7, 128, 9
    x = rng.standard_normal((m, k)).astype(np.float16)
    w = rng.standard_normal((n, k)).astype(np.float32)
    y = oracle.gemm_xwT(x, w)
    ref = oracle.matmul_f32(x.astype(np.float32), np.ascontiguousarray(w.T))
    assert np.array_equal(y, ref)


# ----------------------------------------------------- decode-step helpers ----

def test_rms_norm_closed_form():
    x = np.full(64, 3.0, np.float32)
    w = np.linspace(0.5, 1.5, 64).astype(np.float32)
    y = oracle.rms_norm(x, w, 1e-5)
    inv = np.float32(1.0) / np.sqrt(np.float32(9.0) + np.float32(1e-5))
    assert np.allclose(y, (x * inv) * w, rtol=0, atol=1e-6)


def test_rope_identity_at_zero_and_rotation():
    rng = np.random.default_rng(13)
    x = rng.standard_normal(4 * 64).astype(np.float32)
    y = oracle.rope_half_(x.copy(), 4, 64, 0, 10000.0)
    assert np.array_equal(x, y)
    y = oracle.rope_half_(x.copy(), 4, 64, 37, 10000.0)
    nx = np.linalg.norm(x.reshape(4, 2, 32), axis=1)
    ny = np.linalg.norm(y.reshape(4, 2, 32), axis=1)
    assert np.allclose(nx, ny, rtol=1e-5)
    # head_dim 2, pos 1: angle 1 rad
    z = oracle.rope_half_(np.array([1.0, 0.0], np.float32), 1, 2, 1, 10000.0)
    assert np.allclose(z, [np.cos(1.0), np.sin(1.0)], atol=1e-6)


def test_rope_interleaved_identity_rotation_and_permutation():
    """rope_interleaved_inplace_f32 (cpu_kernels.rs:279-292): identity at pos 0, each (2i, 2i+1)
    pair keeps its norm, a 2-element head at pos 1 turns by 1 rad, and the interleaved form equals
    the rotate-half form on the permuted head (x[2i] -> i, x[2i+1] -> half + i) bit for bit, so
    the two layouts share every angle and product."""
    rng = np.random.default_rng(14)
    nh, hd = 4, 64
    x = rng.standard_normal(nh * hd).astype(np.float32)
    assert np.array_equal(oracle.rope_interleaved_(x.copy(), nh, hd, 0, 10000.0), x)
    y = oracle.rope_interleaved_(x.copy(), nh, hd, 37, 10000.0)
    assert np.allclose(np.hypot(x[0::2], x[1::2]), np.hypot(y[0::2], y[1::2]), rtol=1e-5)
    z = oracle.rope_interleaved_(np.array([1.0, 0.0], np.float32), 1, 2, 1, 10000.0)
    assert np.allclose(z, [np.cos(1.0), np.sin(1.0)], atol=1e-6)
    perm = np.concatenate([np.arange(0, hd, 2), np.arange(1, hd, 2)])  # half-layout position j <- x[perm[j]]
    for pos in (1, 37, 511):
        xh = np.ascontiguousarray(x.reshape(nh, hd)[:, perm].reshape(-1))
        yh = oracle.rope_half_(xh, nh, hd, pos, 10000.0).reshape(nh, hd)
        back = np.empty((nh, hd), np.float32)
        back[:, perm] = yh
        yi = oracle.rope_interleaved_(x.copy(), nh, hd, pos, 10000.0)
        assert np.array_equal(back.reshape(-1), yi)
    # and the layouts differ: rotate-half on the unpermuted head is another result
    assert not np.array_equal(oracle.rope_half_(x.copy(), nh, hd, 37, 10000.0), y)


def test_gelu_tanh_closed_forms_and_erf_distance():
    """gelu_tanh_f32 * up (gemma.rs:844-846, 1689-1693): gelu(0) = 0; the odd part
    gelu(x) - gelu(-x) = x (the 0.5 and the 1 + tanh); gelu(x) -> x and -> 0 far out; multiplying
    by up = 2 doubles it exactly; against the float64 formula with k = sqrt(2/pi) computed here,
    within f32 rounding; and within 5e-4 of the erf GELU x * Phi(x) over [-8, 8], the tanh form's
    known distance, which a wrong k (0.79: 2.8e-3), c (0.05: 3.0e-3) or a missing cubic (3.4e-2)
    exceeds."""
    import math

    x = np.linspace(-8.0, 8.0, 40001).astype(np.float32)
    one = np.ones_like(x)
    g = oracle.gelu_tanh_mul_(x.copy(), one)
    assert g[len(x) // 2] == 0.0 and x[len(x) // 2] == 0.0
    gn = oracle.gelu_tanh_mul_((-x).copy(), one)
    assert np.max(np.abs((g - gn) - x)) <= 1e-6 * 8
    big = oracle.gelu_tanh_mul_(np.array([12.0, -12.0], np.float32), np.ones(2, np.float32))
    assert big[0] == np.float32(12.0) and abs(big[1]) <= 1e-30
    assert np.array_equal(oracle.gelu_tanh_mul_(x.copy(), 2 * one), 2 * g)
    xd = x.astype(np.float64)
    t = 0.5 * xd * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (xd + 0.044715 * xd ** 3)))
    assert np.max(np.abs(g - t)) <= 1e-6
    erf_gelu = np.array([0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0))) for v in xd])
    assert np.max(np.abs(g - erf_gelu)) <= 5e-4


def test_softmax_attention_argmax():
    s = oracle.softmax_(np.full(8, 2.5, np.float32))
    assert np.allclose(s, 1 / 8)
    # one token: attention returns v exactly (weight 1)
    hd, nh, nkv = 8, 4, 2
    v = np.arange(nkv * hd, dtype=np.float32).astype(np.float16)
    kc = np.ones(nkv * hd, np.float16)
    out = oracle.attention_gqa_f16kv(kc.view(np.uint16), v.view(np.uint16), [0], np.ones(nh * hd, np.float32), nh,
                                     nkv, hd)
    expect = np.concatenate([v[(h // 2) * hd:(h // 2 + 1) * hd] for h in range(nh)]).astype(np.float32)
    assert np.array_equal(out, expect)
    assert oracle.argmax_first(np.array([1.0, 3.0, 3.0, 2.0], np.float32)) == 1
    g = np.array([0.0, 1.0], np.float32)
    oracle.silu_mul_(g, np.array([2.0, 2.0], np.float32))
    assert g[0] == 0.0 and np.isclose(g[1], 2.0 / (1.0 + np.exp(-1.0)))


def test_bf16_to_f32_exhaustive():
    """All 65536 bf16 patterns against torch's bfloat16 -> float32 (a library
    conversion built independently of the oracle's shift).  NaNs keep sign and
    payload; ctypes' float return passes through a double, which sets the
    quiet bit of a signalling NaN, so that bit is compared as set."""
    import torch

    bits = np.arange(65536, dtype=np.uint16)
    L = oracle.lib()
    ours = np.array([L.oracle_bf16_to_f32(int(b)) for b in bits], np.float32).view(np.uint32)
    ref = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to(torch.float32).numpy().view(np.uint32)
    nan = np.isnan(ref.view(np.float32))
    assert nan.sum() == 2 * 127
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.array_equal(ours[nan], ref[nan] | np.uint32(0x00400000))
    ours = ours.view(np.float32)
    # the byte order a wrong shift or a truncating f16 path would break
    assert ours[0x3F80] == 1.0 and ours[0xBF80] == -1.0 and ours[0x4049] == np.float32(3.140625)


def _attention_f64(k, v, q, nh, nkv, hd, scale, cap=None):
    """Softmax attention in float64 from the widened f16 K/V rows [seq, nkv*hd]."""
    g = nh // nkv
    out = np.zeros((nh, hd))
    for h in range(nh):
        kv = h // g
        kh = k[:, kv * hd:(kv + 1) * hd].astype(np.float64)
        vh = v[:, kv * hd:(kv + 1) * hd].astype(np.float64)
        sc = kh @ q[h * hd:(h + 1) * hd].astype(np.float64) * scale
        if cap is not None:
            sc = np.tanh(sc / cap) * cap
        w = np.exp(sc - sc.max())
        out[h] = (w / w.sum()) @ vh
    return out.reshape(-1)


@pytest.mark.parametrize("seq,nh,nkv,hd,attn_scale,cap,qmag", [
    (37, 4, 2, 64, None, None, 2.0),
    (300, 15, 5, 64, None, None, 2.0),     # SmolLM2-360M heads
    (129, 8, 1, 128, 0.0625, None, 2.0),   # explicit attn_scale (Some(s), kvcache.rs:752)
    (64, 4, 4, 64, None, 50.0, 60.0),      # a soft cap of 50 (kvcache.rs:768-770) on scores it bends
    (64, 4, 4, 64, 0.3, 2.0, 1.0),         # a cap that bends most scores
])
def test_attention_multi_token_fp64_bound(seq, nh, nkv, hd, attn_scale, cap, qmag):
    """Many positions with unequal scores against float64 softmax attention,
    within a forward error bound of the f32 arithmetic:
      |ds| <= scale * gamma_hd * max_t sum|q k_t| + rounding of the scale/cap,
      |out - ref| <= max|v| * (2|ds| + 2 gamma_seq + 8u), times 2.
    A wrong 1/sqrt(hd), a missing cap, or a wrong kv-head mapping moves the
    weights by O(1) and is checked to fail that bound by far."""
    rng = np.random.default_rng(seq + nh + hd)
    kvd = nkv * hd
    k = rng.standard_normal((seq, kvd)).astype(np.float16)
    v = rng.standard_normal((seq, kvd)).astype(np.float16)
    q = (qmag * rng.standard_normal(nh * hd)).astype(np.float32)
    bases = np.arange(seq, dtype=np.uint64) * kvd
    out = oracle.attention_gqa_f16kv(k.view(np.uint16).ravel(), v.view(np.uint16).ravel(), bases, q, nh, nkv, hd,
                                     attn_scale=attn_scale, soft_cap=cap)
    scale = attn_scale if attn_scale is not None else float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    ref = _attention_f64(k, v, q, nh, nkv, hd, scale, cap)
    g = nh // nkv
    qk = max(float(np.max(np.abs(k[:, (h // g) * hd:(h // g + 1) * hd]).astype(np.float64) @
                      np.abs(q[h * hd:(h + 1) * hd]).astype(np.float64))) for h in range(nh))
    ds = scale * gamma(hd) * qk + 4 * U * scale * qk + (4 * U * cap if cap else 0.0)
    bound = 2 * float(np.max(np.abs(v.astype(np.float64)))) * (2 * ds + 2 * gamma(seq) + 8 * U)
    err = float(np.max(np.abs(out.astype(np.float64) - ref)))
    assert err <= bound, (err, bound)
    # the plausible mistakes are far outside the bound
    wrong = [_attention_f64(k, v, q, nh, nkv, hd, 1.0 / hd, cap),
             _attention_f64(k, v, q, nh, nkv, hd, scale, None if cap else 1.0)]
    if nkv > 1:
        wrong.append(_attention_f64(k, v, q, nh, nkv, hd, scale, cap)[::-1].copy())
    for w in wrong:
        assert float(np.max(np.abs(out - w))) > 20 * bound


def test_qgemv_i4_sym_rows_equal_matmul_i4():
    """The batched i4 form is matmul_i4_f32 (cpu_kernels.rs:219-243) per
    activation row, bit for bit, with f32 x and with f16 x widened exactly;
    per-row (gs = K) and per-group scales; odd K."""
    rng = np.random.default_rng(44)
    for n, k, gs in ((7, 256, 256), (5, 192, 64), (3, 37, 37), (4, 100, 32)):
        w = rng.integers(0, 256, (n, (k + 1) // 2)).astype(np.uint8)
        spr = (k + gs - 1) // gs
        s = rng.uniform(1e-3, 2e-2, n * spr).astype(np.float16).view(np.uint16)
        for xdt in (np.float32, np.float16):
            x = rng.standard_normal((3, k)).astype(xdt)
            y = oracle.qgemv_i4_sym(w, s, gs, x, n, k)
            for r in range(3):
                ref = oracle.matmul_i4_f32(w, s, n, k, gs, x[r].astype(np.float32))
                assert np.array_equal(y[r].view(np.uint32), ref.view(np.uint32)), (n, k, gs, xdt, r)


# ------------------------------------------------------- f16, i2, q1_0_g128 ----

def test_f16_gemv_known_answer_and_sequential_order():
    """f16 weights: 1.0, -2.0, 0.5 (bits 0x3C00, 0xC000, 0x3800) against x =
    1, 10, 100 is exactly 31; random rows equal the strict left-to-right sum of
    f32(w) * x (catches a transposed weight, a reordered or fused sum)."""
    w = np.array([[0x3C00, 0xC000, 0x3800]], np.uint16)
    assert oracle.qgemv_f16(w, np.array([1.0, 10.0, 100.0], np.float32))[0, 0] == np.float32(31.0)
    rng = np.random.default_rng(21)
    n, k = 7, 300
    wf = rng.standard_normal((n, k)).astype(np.float16)
    x = rng.standard_normal((2, k)).astype(np.float32)
    y = oracle.qgemv_f16(wf.view(np.uint16), x)
    for m in range(2):
        for r in range(n):
            assert y[m, r] == seq_sum_f32(wf[r].astype(np.float32) * x[m])
    # an f16 x is widened exactly
    xh = x.astype(np.float16)
    np.testing.assert_array_equal(oracle.qgemv_f16(wf.view(np.uint16), xh),
                                  oracle.qgemv_f16(wf.view(np.uint16), xh.astype(np.float32)))


def _i2_codes(w: np.ndarray, k: int) -> np.ndarray:
    """numpy decode: element j = bits 2(j%4)..2(j%4)+1 of byte j/4."""
    q = (w[:, :, None] >> (2 * np.arange(4, dtype=np.uint8))) & 3
    return q.reshape(w.shape[0], -1)[:, :k]


I2_CENTROIDS = np.array([-1.5, -0.5, 0.5, 1.5], np.float32)


def test_i2_known_answer_bit_order():
    """byte 0xE4 = codes 0, 1, 2, 3 (low bits first) = -1.5, -0.5, 0.5, 1.5;
    against x = 1, 10, 100, 1000 that is 1543.5, exact in both scale modes,
    times 2 for a scale of 2 (catches reversed lanes or centroids)."""
    w = np.array([[0xE4]], np.uint8)
    x = np.array([1.0, 10.0, 100.0, 1000.0], np.float32)
    for mode in (0, 1):
        assert oracle.qgemv_i2(w, np.array([1.0], np.float16).view(np.uint16), x, 4, mode)[0, 0] == np.float32(1543.5)
        assert oracle.qgemv_i2(w, np.array([2.0], np.float16).view(np.uint16), x, 4, mode)[0, 0] == np.float32(3087.0)


def test_i2_scale_modes_and_ragged_rows():
    """Mode 0 (Qwen) = (left-to-right sum of x * dq) * scale; mode 1 (Gemma) =
    left-to-right sum of x * (dq * scale); the two differ for a scale that is
    not a power of two (catches swapped modes).  K = 1023 leaves the last byte
    partly used: codes past K are ignored."""
    rng = np.random.default_rng(22)
    n, k = 6, 1023
    w = rng.integers(0, 256, (n, (k + 3) // 4)).astype(np.uint8)
    s = rng.uniform(0.01, 0.05, n).astype(np.float16)
    x = rng.standard_normal(k).astype(np.float32)
    dq = I2_CENTROIDS[_i2_codes(w, k)]
    y0 = oracle.qgemv_i2(w, s.view(np.uint16), x, k, 0)[0]
    y1 = oracle.qgemv_i2(w, s.view(np.uint16), x, k, 1)[0]
    for r in range(n):
        sc = np.float32(s[r])
        assert y0[r] == np.float32(seq_sum_f32(x * dq[r]) * sc)
        assert y1[r] == seq_sum_f32(x * (dq[r] * sc))
    assert np.any(y0 != y1)
    # the unused high code bits of the last byte do not matter
    w2 = w.copy()
    w2[:, -1] ^= 0xC0
    np.testing.assert_array_equal(oracle.qgemv_i2(w2, s.view(np.uint16), x, k, 0)[0], y0)


def _q1_values(w: np.ndarray, k: int) -> np.ndarray:
    """numpy decode of q1_0_g128 rows: little-endian f16 d, then 128 bits (bit j of byte b = element 8b+j)."""
    n = w.shape[0]
    blk = w.reshape(n, k // 128, 18)
    d = blk[:, :, :2].copy().view(np.float16).astype(np.float32)[:, :, 0]
    bits = np.unpackbits(blk[:, :, 2:], axis=2, bitorder="little").astype(bool)
    return np.where(bits, d[:, :, None], -d[:, :, None]).reshape(n, k)


def test_q1_known_answer_bit_and_byte_order():
    """d = 1.0 as bytes 00 3C; only bit 3 of sign byte 5 set: element 43 is +1,
    the other 127 are -1, so y = 2 x[43] - sum(x), exact for integer x
    (catches a big-endian d, a reversed bit order or a block offset)."""
    w = np.zeros((1, 18), np.uint8)
    w[0, 0], w[0, 1] = 0x00, 0x3C
    w[0, 2 + 5] = 1 << 3
    x = np.arange(128, dtype=np.float32) - 40.0
    assert oracle.qgemv_q1_0_g128(w, x, 128)[0, 0] == np.float32(2 * x[43] - x.sum())


def test_q1_sequential_order_random():
    """Random blocks: y = left-to-right sum of value * x over the row, values
    from numpy's own unpacking."""
    rng = np.random.default_rng(23)
    n, k = 5, 512
    w = rng.integers(0, 256, (n, k // 128 * 18)).astype(np.uint8)
    d = rng.uniform(0.01, 0.1, (n, k // 128)).astype(np.float16)
    w.reshape(n, k // 128, 18)[:, :, :2] = d.view(np.uint8).reshape(n, k // 128, 2)
    x = rng.standard_normal((3, k)).astype(np.float32)
    y = oracle.qgemv_q1_0_g128(w, x, k)
    v = _q1_values(w, k)
    for m in range(3):
        for r in range(n):
            assert y[m, r] == seq_sum_f32(v[r] * x[m])
