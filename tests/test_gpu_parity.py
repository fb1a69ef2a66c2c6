"""GPU parity: the HIP path (through the C ABI) against the CPU oracle.

Bars:
  * unpack / dequant: bit-exact;
  * GEMV/GEMM with f32 accumulation of exact products: normwise relative error
    max|y - ref| / max|ref| <= 1e-3 against the reference CPU order;
  * GEMM over f16 dequantized tiles: <= 2e-2 against the reference f32 path,
    and <= 1e-3 against the same f16 tiles summed by the oracle.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests._util import make_i8, make_q4, rel_err, seed

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-3
TOL_F16_TILE = 2e-2


def _t(a, dtype=None):
    import torch

    if a.dtype == np.uint32:
        a = a.view(np.int32)
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.to("cuda")


def _sb_tensor(a):
    import torch

    if a.dtype == np.uint16:  # bf16 bits
        return torch.from_numpy(a.view(np.int16)).to("cuda").view(torch.bfloat16)
    return _t(a)


def _check_f16_tiles(y, wq, s, b, x, k, group=64):
    """The MFMA paths multiply f16 tiles RNE_f16(f32(q)*s + b) (the converter's
    dequant, tools/convert/src/main.rs:4435-4436): within the f32 bar of the
    oracle's sum over the same tiles, and within the fp16-tile bar of the
    reference's f32 path."""
    w16 = oracle.f16_bits_to_f32(oracle.dequant_q4_affine_f16(wq, s, b, k, gs=group))
    assert rel_err(y, oracle.gemm_xwT(x, w16)) <= TOL_F32
    assert rel_err(y, oracle.qgemv_q4_affine(wq, s, b, x, k, gs=group)) <= TOL_F16_TILE


def _run_q4(ops, wq, s, b, x, group=64, gemm=False):
    import torch

    n, k = wq.shape[0], wq.shape[1] * 8
    m = x.shape[0]
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    if gemm:
        ops.encode_qgemm_q4_affine(_t(wq), _sb_tensor(s), _sb_tensor(b), _t(x), y, group=group)
    else:
        ops.encode_qgemv_q4_affine(_t(wq), _sb_tensor(s), _sb_tensor(b), _t(x), y, group=group)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def _run_i8(ops, w, s, x, bias=None, gemm=False):
    import torch

    n, k = w.shape
    m = x.shape[0]
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    bt = _t(bias) if bias is not None else None
    if gemm:
        ops.encode_qgemm_i8(_t(w), _t(s), _t(x), y, bias=bt)
    else:
        ops.encode_qgemv_i8(_t(w), _t(s), _t(x), y, bias=bt)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def test_smoke(ops):
    from cellm_amd import smoke_test

    smoke_test(0)


# ---------------------------------------------------------------- dequant ----

@pytest.mark.parametrize("sb", [np.float16, np.float32, "bf16"])
@pytest.mark.parametrize("n,k,group", [(64, 896, 64), (7, 128, 64), (5, 96, 64), (9, 256, 32), (3, 512, 128)])
def test_dequant_bit_exact(ops, sb, n, k, group):
    import torch

    wq, s, b, _ = make_q4(n, k, 1, sb_dtype=sb, group=group, salt=n + k)
    out16 = torch.empty((n, k), dtype=torch.float16, device="cuda")
    ops.encode_dequant_q4_affine(_t(wq), _sb_tensor(s), _sb_tensor(b), out16, group=group)
    out32 = torch.empty((n, k), dtype=torch.float32, device="cuda")
    ops.encode_dequant_q4_affine(_t(wq), _sb_tensor(s), _sb_tensor(b), out32, group=group)
    torch.cuda.synchronize()
    ref16 = oracle.dequant_q4_affine_f16(wq, s, b, k, group)
    ref32 = oracle.q4_affine_dequant_f32(wq, s, b, k, group)
    np.testing.assert_array_equal(out16.cpu().numpy().view(np.uint16), ref16)
    np.testing.assert_array_equal(out32.cpu().numpy().view(np.uint32), ref32.view(np.uint32))


# ------------------------------------------------------------- q4 affine GEMV ----

QWEN_SHAPES = [(896, 1152), (896, 896), (896, 9728), (4864, 896)]  # (K, N), config 2


@pytest.mark.parametrize("k,n", QWEN_SHAPES)
def test_q4_gemv_qwen_shapes(ops, k, n):
    wq, s, b, x = make_q4(n, k, 1)
    y = _run_q4(ops, wq, s, b, x)
    ref = oracle.qgemv_q4_affine(wq, s, b, x, k)
    assert rel_err(y, ref) <= TOL_F32, rel_err(y, ref)


def test_q4_gemv_qwen_lm_head(ops):
    k, n = 896, 151936
    wq, s, b, x = make_q4(n, k, 1, salt=1)
    y = _run_q4(ops, wq, s, b, x)
    ref = oracle.qgemv_q4_affine(wq, s, b, x, k)
    assert rel_err(y, ref) <= TOL_F32
    assert int(np.argmax(y[0])) == int(np.argmax(ref[0]))


@pytest.mark.parametrize("k,n,group,sb", [
    (1024, 40000, 64, "bf16"),      # flat-batch kernel, 8 loads per 16-row batch
    (512, 32768, 64, np.float32),   # flat, 4 loads per batch, f32 scale rows of 32 bytes
    (640, 40000, 64, np.float16),   # flat, 5 loads per batch
    (768, 65536, 128, "bf16"),      # flat, 6 loads per batch, group 128
    (512, 1048576, 32, np.float16), # flat, group 32, 32 batches parked per wave
    (960, 49152, 64, np.float16),   # batched-row ring kernel, 30 of 32 lanes per row (SmolLM2-360M lm_head shape)
    (256, 32768, 32, np.float16),   # ring kernel, 8 chunks per row
    (512, 33001, 128, np.float32),  # N % 16 != 0: persistent kernel, ragged last tile
    (896, 65536, 64, np.float32),   # f32 scale rows of 56 bytes: persistent kernel
])
def test_q4_gemv_long_output(ops, k, n, group, sb):
    wq, s, b, x = make_q4(n, k, 1, sb_dtype=sb, group=group, salt=k + n)
    y = _run_q4(ops, wq, s, b, x, group=group)
    assert rel_err(y, oracle.qgemv_q4_affine(wq, s, b, x, k, gs=group)) <= TOL_F32


@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("sb", [np.float16, np.float32, "bf16"])
def test_q4_gemv_batched_small_m(ops, m, sb):
    k, n = 1152, 1000  # N not a multiple of any rows-per-block
    wq, s, b, x = make_q4(n, k, m, cfg=3, sb_dtype=sb, salt=m)
    y = _run_q4(ops, wq, s, b, x)
    ref = oracle.qgemv_q4_affine(wq, s, b, x, k)
    assert rel_err(y, ref) <= TOL_F32


@pytest.mark.parametrize("k,n,group", [(40, 33, 64), (96, 17, 64), (256, 50, 32), (512, 31, 128)])
def test_q4_gemv_ragged_and_groups(ops, k, n, group):
    wq, s, b, x = make_q4(n, k, 1, group=group, salt=k)
    y = _run_q4(ops, wq, s, b, x, group=group)
    ref = oracle.qgemv_q4_affine(wq, s, b, x, k, group)
    assert rel_err(y, ref) <= TOL_F32


def test_q4_logits_sync_f32_reference_dtypes(ops):
    """The LFM layout as converted by convert_lfm.py: f32 scales/biases, f32 x."""
    k, n = 1024, 2048
    wq, s, b, x = make_q4(n, k, 1, sb_dtype=np.float32, x_dtype=np.float32, salt=7)
    y = ops.logits_q4_affine(x[0], wq, s, b, n, k, "test.lfm.q4")
    ref = oracle.qgemv_q4_affine(wq, s, b, x, k)[0]
    assert rel_err(y, ref) <= TOL_F32
    # second call hits the weight cache
    y2 = ops.logits_q4_affine(x[0], wq, s, b, n, k, "test.lfm.q4")
    np.testing.assert_array_equal(y, y2)


# ------------------------------------------------------------------ int8 GEMV ----

@pytest.mark.parametrize("n", [576, 1536])
def test_i8_gemv_smollm_config1(ops, n):
    k = 576
    w, s, x = make_i8(n, k, 1)
    y = _run_i8(ops, w, s, x)
    ref = oracle.qgemv_i8(w, s, x)
    assert rel_err(y, ref) <= TOL_F32


@pytest.mark.parametrize("k,n", [(1152, 1536), (1024, 1152)])
@pytest.mark.parametrize("m", [1, 4, 16, 64])
def test_i8_gemv_gemma_attn_f16x(ops, k, n, m):
    """Config 3's int8 attention projections (fused QKV 1152 -> 1536, o 1024 ->
    1152) at every M it names: M <= 4 the VALU GEMV, 16 and 64 the batched
    MFMA path (int8 exact in f16: exact products, the f32 bar)."""
    w, s, x = make_i8(n, k, m, cfg=3, x_dtype=np.float16, salt=m)
    y = _run_i8(ops, w, s, x)
    ref = oracle.qgemv_i8(w, s, x)
    assert rel_err(y, ref) <= TOL_F32


def test_i8_logits_sync_reference_dtypes(ops):
    """MetalOps::logits_i8 contract: f16 scales, f32 x, host in/out."""
    k, n = 960, 2560
    w, s, x = make_i8(n, k, 1, cfg=5, scale_dtype=np.float16)
    sbits = s.view(np.uint16)
    y = ops.logits_i8(x[0], w, sbits, n, k, "test.i8.logits")
    ref = oracle.matmul_i8_f32(w, sbits, x[0])
    assert rel_err(y, ref) <= TOL_F32


def test_i8_bias_and_per_tensor_scale(ops):
    import torch

    k, n = 256, 300
    w, s, x = make_i8(n, k, 2, salt=3)
    bias = oracle.gen_normal((n,), seed(1, 5), 0.0, 1.0)
    y = _run_i8(ops, w, s, x, bias=bias)
    ref = oracle.qgemv_i8(w, s, x) + bias[None, :]
    assert rel_err(y, ref) <= TOL_F32
    # per-tensor scale: one scale for the tensor (metal.rs:900: the buffer does not cover every row)
    s1 = s[:1].copy()
    yt = torch.empty((2, n), dtype=torch.float32, device="cuda")
    ops.encode_qgemv_i8(_t(w), _t(s1), _t(x), yt)
    torch.cuda.synchronize()
    ref1 = oracle.qgemv_i8(w, np.full(n, s1[0], np.float32), x)
    assert rel_err(yt.cpu().numpy(), ref1) <= TOL_F32
    # 2..n-1 scales are neither: refused instead of silently using scale[0]
    from cellm_amd import CellmHipError

    with pytest.raises(CellmHipError, match="n_scales=2"):
        ops.encode_qgemv_i8(_t(w), _t(s[:2].copy()), _t(x), yt)


@pytest.mark.parametrize("k,m", [(6912, 4), (4864, 4), (10240, 3), (6912, 2)])
def test_i8_gemv_f32x_long_rows(ops, k, m):
    """f32 activations of long rows at M > 1 (the device runner's down_proj at Gemma-3-1B and Qwen2.5
    widths): x takes more than 64 KB of LDS, so the team kernel runs with the per-kernel limit
    raised (up to 160 KB: K <= 10240 at four rows)."""
    n = 1152
    w, s, x = make_i8(n, k, m, cfg=5, x_dtype=np.float32, salt=k + m)
    y = _run_i8(ops, w, s, x)
    ref = oracle.qgemv_i8(w, s, x)
    assert rel_err(y, ref) <= TOL_F32


@pytest.mark.parametrize("n,k,m,sdt", [
    (49152, 960, 4, np.float16),    # the configs[4] lm_head at four sessions (f16 row scales)
    (49152, 960, 2, np.float32),
    (32768, 128, 3, np.float32),    # two 64-k blocks: one block pair
    (32768, 192, 4, np.float16),    # three blocks: a pair and an odd one
    (40000, 1024, 2, np.float32),   # the longest K; N not a multiple of 64
    (32768, 576, 4, np.float32),
])
def test_i8_f32x_long_output_mfma(ops, n, k, m, sdt):
    """f32 activations at 2..4 rows over a long output (the Llama lm_head of a multi-session step,
    llama.rs:602-643): int8 weights as the B bytes of int8 MFMA, each x row as three signed 8-bit
    digits under one power of two per row, exact integer sums over the whole K, the row scale
    after the sum.  Every row within 3e-5 of the f32 reference order, which one f16 rounding of x
    would miss."""
    w, s, x = make_i8(n, k, m, cfg=5, scale_dtype=sdt, x_dtype=np.float32, salt=300 + m + k % 97)
    y = _run_i8(ops, w, s, x)
    ref = oracle.qgemv_i8(w, s, x)
    for r in range(m):
        assert rel_err(y[r], ref[r]) <= 3e-5, (r, rel_err(y[r], ref[r]))
    xr = x.astype(np.float16).astype(np.float32)
    assert rel_err(oracle.qgemv_i8(w, s, xr), ref) > 3e-5
    # with a bias: added after the scale, as the team kernel does
    bias = oracle.gen_normal((n,), 0xD0000300 + k, 0.0, 1.0).astype(np.float32)
    yb = _run_i8(ops, w, s, x, bias=bias)
    for r in range(m):
        assert rel_err(yb[r], ref[r] + bias) <= 3e-5, r


def test_i8_f32x_long_output_mfma_range(ops):
    """The int8 f32-x MFMA path over x far from N(0,1): rows at ~1e5, ~1e-5 and ~1e-12 and a zero
    row; each row against the f32 oracle to 3e-5, the zero row exactly zero."""
    n, k, m = 32768, 960, 4
    row_scale = np.array([1e5, 1e-5, 1e-12, 0.0], np.float32)
    w, s, x0 = make_i8(n, k, m, cfg=5, x_dtype=np.float32, salt=331)
    x = np.ascontiguousarray(x0 * row_scale[:, None], np.float32)
    y = _run_i8(ops, w, s, x)
    ref = oracle.qgemv_i8(w, s, x)
    assert np.all(np.isfinite(y))
    for r in range(3):
        assert rel_err(y[r], ref[r]) <= 3e-5, (r, rel_err(y[r], ref[r]))
    assert not np.any(y[3])


def test_i8_ragged_k(ops):
    k, n = 40, 19  # k % 16 != 0 -> generic kernel
    w, s, x = make_i8(n, k, 1, salt=9)
    y = _run_i8(ops, w, s, x)
    ref = oracle.qgemv_i8(w, s, x)
    assert rel_err(y, ref) <= TOL_F32


# ------------------------------------------------------------- batched / GEMM ----

@pytest.fixture(scope="module")
def gemma_lm_head():
    """Config 3's int8 lm_head: W [262144, 1152] (302 MB), fp32 row scales."""
    k, n = 1152, 262144
    w, s, _ = make_i8(n, k, 1, cfg=3, x_dtype=np.float16, salt=200)
    return w, s, _t(w), _t(s)


@pytest.mark.parametrize("m", [1, 4])
def test_i8_gemma_lm_head_full(ops, gemma_lm_head, m):
    """The bench's config-3 lm_head at full size: M = 1 runs the 8-lane f16-x
    decode kernel, M = 4 the batched MFMA path (>= 8192 outputs).  Every row
    against the oracle; the greedy id of each activation row as well."""
    import torch

    w, s, wd, sd = gemma_lm_head
    k, n = w.shape[1], w.shape[0]
    x = oracle.gen_normal((m, k), seed(3, 2, 300 + m), 0.0, 1.0).astype(np.float16)
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    ops.encode_qgemv_i8(wd, sd, _t(x), y)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref = oracle.qgemv_i8(w, s, x)
    assert rel_err(got, ref) <= TOL_F32
    assert [int(v) for v in got.argmax(1)] == [int(v) for v in ref.argmax(1)]


@pytest.mark.parametrize("m", [16, 64])
def test_i8_gemma_lm_head_full_n_sampled_rows(ops, gemma_lm_head, m):
    """M = 16 and 64 run over the full 262144 rows; the oracle checks a sample
    of 6144 rows spread over the whole output (every tile position of the
    persistent grid's first, middle and last rounds, plus random rows)."""
    import torch

    w, s, wd, sd = gemma_lm_head
    k, n = w.shape[1], w.shape[0]
    x = oracle.gen_normal((m, k), seed(3, 2, 400 + m), 0.0, 1.0).astype(np.float16)
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    ops.encode_qgemv_i8(wd, sd, _t(x), y)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    rng = np.random.default_rng(m)
    rows = np.unique(np.concatenate([np.arange(2048), np.arange(n // 2 - 1024, n // 2 + 1024), np.arange(n - 1024, n),
                                     rng.choice(n, 1024, replace=False)]))
    ref = oracle.qgemv_i8(np.ascontiguousarray(w[rows]), np.ascontiguousarray(s[rows]), x)
    assert rel_err(got[:, rows], ref) <= TOL_F32


@pytest.mark.parametrize("m,k,n", [(64, 1152, 1000), (49, 1024, 4099), (64, 704, 300), (64, 1216, 2000),
                                   (57, 1152, 262)])
def test_i8_batched_whole_x_in_lds(ops, m, k, n):
    """49..64 rows whose X is 80-152 KB run one 1024-thread block per CU with
    the whole X in LDS (ragged tile counts, a CU count above the tile count);
    K = 1216 is past 152 KB and takes the chunked form."""
    w, s, x = make_i8(n, k, m, cfg=3, x_dtype=np.float16, salt=m + k)
    y = _run_i8(ops, w, s, x)
    assert rel_err(y, oracle.qgemv_i8(w, s, x)) <= TOL_F32


@pytest.mark.parametrize("m,k,n,sb", [(64, 1152, 1000, np.float16), (49, 1024, 4099, "bf16"),
                                      (57, 1152, 262, np.float32), (64, 1280, 300, np.float16)])
def test_q4_batched_whole_x_in_lds(ops, m, k, n, sb):
    """q4 at 49..64 rows whose X is 80-152 KB: one 512-thread block per CU
    with the whole X in LDS (ragged tile counts); K = 1280 is past 152 KB and
    takes the chunked form."""
    wq, s, b, x = make_q4(n, k, m, cfg=3, sb_dtype=sb, salt=m + k)
    y = _run_q4(ops, wq, s, b, x)
    _check_f16_tiles(y, wq, s, b, x, k)


@pytest.mark.parametrize("m", [1, 4, 16, 64])
def test_q4_gemma_gate_up_full_config3(ops, m):
    """Config 3's q4 gate+up 1152 -> 13824 at every M it names, full size.
    M = 1 takes the 16-lanes-per-row VALU kernel (exact products, f32 sums:
    the f32 bar), M = 4 (>= 8192 outputs) and 16 the batched MFMA path, M =
    64 its whole-X-in-LDS form (f16 tiles)."""
    k, n = 1152, 13824
    wq, s, b, x = make_q4(n, k, m, cfg=3, salt=m)
    y = _run_q4(ops, wq, s, b, x)
    if m == 1:
        assert rel_err(y, oracle.qgemv_q4_affine(wq, s, b, x, k)) <= TOL_F32
    else:
        _check_f16_tiles(y, wq, s, b, x, k)


@pytest.mark.parametrize("m,sb,lo,hi", [
    (4, np.float32, 1e-4, 1e-3),     # f32 scales and biases, as convert_lfm.py writes them (lfm.rs:1003-1004)
    (16, np.float16, 1e-4, 1e-3),    # f16 scales below 1e-3: s/16 would be an f16 subnormal
    (64, "bf16", 2e-5, 1e-3),
    (7, np.float32, 1e-4, 1e-3),
])
def test_q4_batched_small_scales(ops, m, sb, lo, hi):
    """Batched decode with small group scales and f32 scale/bias files: the
    tiles are rounded once from the f32 value q*s + b, so scales below 1e-3
    (where s/16 would be an f16 subnormal) keep the tile bars."""
    k, n = 1152, 9000
    wq, _, b, x = make_q4(n, k, m, cfg=3, sb_dtype=np.float32, salt=m + 100)
    s = oracle.gen_uniform(b.shape, seed(3, 7, m), lo, hi)
    b = (b * np.float32(hi / 0.05)).astype(np.float32)  # biases of the same order as the scales
    if sb == np.float16:
        s, b = s.astype(np.float16), b.astype(np.float16)
    elif sb == "bf16":
        s = (s.view(np.uint32) >> 16).astype(np.uint16)
        b = (b.view(np.uint32) >> 16).astype(np.uint16)
    y = _run_q4(ops, wq, s, b, x)
    _check_f16_tiles(y, wq, s, b, x, k)


@pytest.mark.parametrize("m", [2, 3, 7, 33])
def test_i8_batched_mfma_small_m_and_k_chunks(ops, m):
    """5..64 rows (and 2..4 rows with >= 8192 outputs) take the MFMA batched
    path; K=6912 spans several LDS chunks, K=960 and 576 end on an odd
    64-column block (576 at m=33: the odd block opens a fresh X chunk)."""
    for k, n in ((1152, 1000), (6912, 300), (960, 333), (576, 700), (1152, 8200)):
        w, s, x = make_i8(n, k, m, cfg=3, x_dtype=np.float16, salt=m + k)
        y = _run_i8(ops, w, s, x)
        assert rel_err(y, oracle.qgemv_i8(w, s, x)) <= TOL_F32, (m, k)


@pytest.mark.parametrize("m", [1, 4])
def test_q4_gemma_down_config3_small_m(ops, m):
    """Config 3's q4 down projection 6912 -> 1152 at M = 1 and 4: the VALU GEMV
    (64 lanes per row, two register passes), exact products and f32 sums."""
    k, n = 6912, 1152
    wq, s, b, x = make_q4(n, k, m, cfg=3, salt=40 + m)
    y = _run_q4(ops, wq, s, b, x)
    assert rel_err(y, oracle.qgemv_q4_affine(wq, s, b, x, k)) <= TOL_F32


@pytest.mark.parametrize("m,k,n", [(5, 6912, 1152), (16, 6912, 1152), (17, 6912, 1152), (64, 6912, 1152),
                                   (2, 1152, 8200), (4, 1152, 8200)])
def test_q4_batched_mfma_k_chunks(ops, m, k, n):
    """Gemma down projection (several X chunks in LDS) at 5..64 rows; 2..4
    rows take the MFMA path only for >= 8192 outputs."""
    wq, s, b, x = make_q4(n, k, m, cfg=3, salt=m)
    y = _run_q4(ops, wq, s, b, x)
    _check_f16_tiles(y, wq, s, b, x, k)


@pytest.mark.parametrize("kind,m,k,n,sdt,group", [
    ("i8", 8, 2560, 960, np.float16, 0), ("i8", 20, 2496, 700, "bf16", 0), ("i8", 64, 4096, 64, np.float32, 0),
    ("q4", 8, 4864, 896, np.float32, 64), ("q4", 33, 4992, 300, "bf16", 64), ("q4", 64, 6912, 1152, np.float16, 128),
])
def test_batched_mfma_split_k(ops, kind, m, k, n, sdt, group):
    """Few 64-row W tiles over a long K: the batched MFMA kernel splits K over work items
    and a second kernel adds the partial sums in split order.  K = 2496 and 4992 end on
    an odd K block (taken by the last split).  Two calls give the same bits."""
    import torch

    if kind == "i8":
        w, s, x = make_i8(n, k, m, cfg=3, x_dtype=np.float16, salt=m + k)
        if sdt == "bf16":
            s = (s.view(np.uint32) >> 16).astype(np.uint16)
            sref = (s.astype(np.uint32) << 16).view(np.float32)
            st = torch.from_numpy(s.view(np.int16)).to("cuda").view(torch.bfloat16)
        else:
            s = s.astype(sdt)
            sref = s.astype(np.float32)
            st = _t(s)
        bias = oracle.gen_normal((n,), seed(3, 5, m), 0.0, 1.0)
        ys = []
        for _ in range(2):
            y = torch.empty((m, n), dtype=torch.float32, device="cuda")
            ops.encode_qgemv_i8(_t(w), st, _t(x), y, bias=_t(bias))
            torch.cuda.synchronize()
            ys.append(y.cpu().numpy())
        assert rel_err(ys[0], oracle.qgemv_i8(w, sref, x) + bias[None, :]) <= TOL_F32
        # one scale for the tensor
        y1 = torch.empty((m, n), dtype=torch.float32, device="cuda")
        ops.encode_qgemv_i8(_t(w), st[:1].contiguous(), _t(x), y1)
        torch.cuda.synchronize()
        assert rel_err(y1.cpu().numpy(), oracle.qgemv_i8(w, np.full(n, sref[0], np.float32), x)) <= TOL_F32
    else:
        wq, s, b, x = make_q4(n, k, m, cfg=3, sb_dtype=sdt, group=group, salt=m + k)
        ys = [_run_q4(ops, wq, s, b, x, group=group) for _ in range(2)]
        _check_f16_tiles(ys[0], wq, s, b, x, k, group)
    assert np.array_equal(ys[0].view(np.uint32), ys[1].view(np.uint32))


@pytest.mark.parametrize("m,group", [(8, 128), (20, 256), (4, 128), (6, 32)])
def test_q4_batched_mfma_other_groups(ops, m, group):
    """Groups of 32, 128 and 256 on the batched MFMA path."""
    k, n = 1024, 8448
    wq, s, b, x = make_q4(n, k, m, cfg=3, group=group, salt=m + group)
    y = _run_q4(ops, wq, s, b, x, group=group)
    _check_f16_tiles(y, wq, s, b, x, k, group)


@pytest.mark.parametrize("k,n", [(896, 4864), (4864, 896)])
def test_q4_prefill_qgemm_m512(ops, k, n):
    m = 512
    wq, s, b, x = make_q4(n, k, m, cfg=4)
    y = _run_q4(ops, wq, s, b, x, gemm=True)
    w16 = oracle.f16_bits_to_f32(oracle.dequant_q4_affine_f16(wq, s, b, k))
    ref16 = oracle.gemm_xwT(x, w16)
    assert rel_err(y, ref16) <= TOL_F32
    w32 = oracle.q4_affine_dequant_f32(wq, s, b, k)
    ref32 = oracle.gemm_xwT(x, w32)
    assert rel_err(y, ref32) <= TOL_F16_TILE


@pytest.mark.parametrize("n", [64, 224])
@pytest.mark.parametrize("sb", [np.float16, "bf16", np.float32])
def test_qgemm_tiles_are_the_converter_f16_dequant(ops, sb, n):
    """X = identity makes Y[m, n] = W_tile[n, m]: one exact product, zeros
    elsewhere, so the GEMM output exposes the f16 tile values bit for bit.
    Row 0 carries the double-rounding case of the oracle pins (q=3,
    s=1+2^-10, b=-2^-24), where one rounding of q*s+b would differ.  n = 224
    ends in a ragged 96-column tile."""
    import torch

    k = 256
    wq, s, b, _ = make_q4(n, k, 1, cfg=4, sb_dtype=sb, salt=77)
    if sb == np.float16:
        wq[0, 0] = (wq[0, 0] & ~np.uint32(0xF)) | np.uint32(3)
        s[0, 0] = np.float16(1 + 2 ** -10)
        b[0, 0] = np.float16(-(2.0 ** -24))
    x = np.eye(k, dtype=np.float16)
    y = _run_q4(ops, wq, s, b, x, gemm=True)
    ref16 = oracle.f16_bits_to_f32(oracle.dequant_q4_affine_f16(wq, s, b, k))
    np.testing.assert_array_equal(y.T.view(np.uint32), ref16.view(np.uint32))


@pytest.mark.parametrize("m,k,n,group,sb", [
    (37, 192, 77, 64, np.float16),      # K % 128 != 0: register-staged kernel
    (37, 256, 77, 64, np.float16),      # K % 128 == 0: dequant-at-the-MFMA kernel, ragged M and N
    (300, 640, 1000, 128, "bf16"),
    (130, 4864, 200, 64, np.float32),   # split-K through the workspace
    (64, 256, 96, 32, np.float16),
    (130, 896, 300, 64, np.float16),    # dequant-at-the-MFMA kernel, ragged M and N over 7 k-steps
])
def test_qgemm_ragged_m_n(ops, m, k, n, group, sb):
    wq, s, b, x = make_q4(n, k, m, cfg=4, sb_dtype=sb, group=group, salt=5 + k)
    y = _run_q4(ops, wq, s, b, x, group=group, gemm=True)
    w16 = oracle.f16_bits_to_f32(oracle.dequant_q4_affine_f16(wq, s, b, k, gs=group))
    assert rel_err(y, oracle.gemm_xwT(x, w16)) <= TOL_F32


@pytest.mark.parametrize("n,k,m,sb,group", [
    (4864, 896, 1, np.float16, 64),      # Qwen2.5-0.5B gate, as the LFM runner passes f32 x
    (896, 4864, 4, np.float16, 64),      # long rows: 64-lane teams
    (2560, 960, 3, np.float32, 64),      # f32 S/B, as LFM .cellm files hold them
    (960, 2560, 2, "bf16", 128),
    (1000, 1024, 1, np.float16, 32),
    (300, 10240, 2, np.float16, 64),
    (200, 10240, 4, np.float16, 64),
    (151936, 896, 1, np.float16, 64),    # the affine lm_head (lfm.rs:700-741) with its f32 x_final
    (333, 96, 1, np.float16, 32),        # one chunk per row, most lanes idle
])
def test_q4_affine_f32_activations(ops, n, k, m, sb, group):
    """MLX q4 affine GEMV with f32 x (linear_i4_out_in, lfm.rs:985-1066), the
    LFM runner's activations: the team kernel over x split into hi + lo f16
    parts (products with either part exact in f32), within 1e-3 of the
    reference order.  The split keeps x to about 22 bits: the error also stays
    under 3e-5, which one f16 rounding of x (about 2e-4 here) would not."""
    wq, s, b, x = make_q4(n, k, m, sb_dtype=sb, x_dtype=np.float32, group=group, salt=70 + m + k % 97)
    y = _run_q4(ops, wq, s, b, x, group=group)
    ref = oracle.qgemv_q4_affine(wq, s, b, x, k, gs=group)
    assert rel_err(y, ref) <= TOL_F32
    assert rel_err(y, ref) <= 3e-5
    # the same weights with x rounded once to f16 land much further from the f32 reference
    xr = x.astype(np.float16).astype(np.float32)
    assert rel_err(oracle.qgemv_q4_affine(wq, s, b, xr, k, gs=group), ref) > 3e-5


@pytest.mark.parametrize("n,k,m,sb", [
    (32768, 896, 1, np.float16),
    (32768, 896, 2, np.float16),
    (32768, 896, 3, "bf16"),
    (32768, 896, 4, np.float16),
    (32768, 128, 2, np.float32),         # one 128-k block: no block pair, only the odd block
    (35008, 1024, 4, np.float32),        # the longest K; N not a multiple of 64 tiles
    (40000, 384, 3, np.float16),         # three blocks: a pair and an odd one
    (151936, 896, 4, np.float32),        # the Qwen-shape affine lm_head at four sessions, f32 S/B
])
def test_q4_affine_f32_activations_long_output_mfma(ops, n, k, m, sb):
    """The long-output f32-x path (lfm.rs:700-741's x_final on the affine lm_head): nibbles as exact
    f16 integers on MFMA, x as hi + lo f16 parts scaled per (row, group of 64), the group's scale
    and bias folded after the group's sum.  Every row within 3e-5 of the f32 reference order, which
    one f16 rounding of x would miss."""
    wq, s, b, x = make_q4(n, k, m, sb_dtype=sb, x_dtype=np.float32, group=64, salt=90 + m + k % 89)
    y = _run_q4(ops, wq, s, b, x, group=64)
    ref = oracle.qgemv_q4_affine(wq, s, b, x, k, gs=64)
    for r in range(m):
        assert rel_err(y[r], ref[r]) <= 3e-5, (r, rel_err(y[r], ref[r]))
    xr = x.astype(np.float16).astype(np.float32)
    assert rel_err(oracle.qgemv_q4_affine(wq, s, b, xr, k, gs=64), ref) > 3e-5


@pytest.mark.parametrize("n,k,m,group", [
    (896, 896, 1, 64), (896, 896, 2, 64), (896, 896, 4, 64),   # Qwen2 o_proj: one team per row
    (1000, 1024, 3, 32),
    (333, 96, 1, 32),                   # three chunks per row: teams of 16 lanes, most idle
    (700, 2048, 4, 128),                # the longest row on one team (64 chunks)
    (896, 4864, 1, 64), (896, 4864, 2, 64), (896, 4864, 4, 64),  # Qwen2 down_proj: rows split over 3 waves
    (300, 2080, 2, 32),                 # just past 2048: 22 chunks per wave
    (129, 6144, 3, 64),                 # 64 chunks per wave, a ragged last block of rows
])
def test_q4_affine_f32_dot_paths(ops, n, k, m, group):
    """f32 x with f32 scales and biases at 1..4 rows (the u32 runners' o_proj and down_proj,
    linear_i4_out_in, lfm.rs:985-1066): x in LDS as f32 and an f32 FMA dot over the widened
    nibbles, one team per row up to K = 2048, longer rows split over three waves.  No f16 rounding
    of x anywhere: every row within 1e-5 of the f32 reference order."""
    wq, s, b, x = make_q4(n, k, m, sb_dtype=np.float32, x_dtype=np.float32, group=group, salt=200 + m + k % 83)
    y = _run_q4(ops, wq, s, b, x, group=group)
    ref = oracle.qgemv_q4_affine(wq, s, b, x, k, gs=group)
    for r in range(m):
        assert rel_err(y[r], ref[r]) <= 1e-5, (r, rel_err(y[r], ref[r]))


@pytest.mark.parametrize("k", [896, 4864])
def test_q4_affine_f32_dot_range(ops, k):
    """The f32-dot paths over x far from N(0,1) (rows at ~1e5, ~1e-5, ~1e-12 and zero): f32
    throughout, so each row stays within 1e-5 of the f32 oracle and the zero row is exactly zero."""
    n, m = 700, 4
    row_scale = np.array([1e5, 1e-5, 1e-12, 0.0], np.float32)
    wq, s, b, x0 = make_q4(n, k, m, sb_dtype=np.float32, x_dtype=np.float32, salt=230 + k % 7)
    x = np.ascontiguousarray(x0 * row_scale[:, None], np.float32)
    y = _run_q4(ops, wq, s, b, x)
    ref = oracle.qgemv_q4_affine(wq, s, b, x, k)
    assert np.all(np.isfinite(y))
    for r in range(m):
        assert rel_err(y[r], ref[r]) <= 1e-5, (r, rel_err(y[r], ref[r]))
    assert not np.any(y[3])


def test_q4_affine_f32_activation_range_long_output_mfma(ops):
    """The MFMA f32-x path over x far from N(0,1): rows past f16's largest value, at ~1e-5 and
    ~1e-12, and zero; each row against the f32 oracle to 3e-5, the zero row exactly zero."""
    k, n, m = 896, 32768, 4
    row_scale = np.array([1e5, 1e-5, 1e-12, 0.0], np.float32)
    wq, s, b, x0 = make_q4(n, k, m, x_dtype=np.float32, salt=81)
    x = np.ascontiguousarray(x0 * row_scale[:, None], np.float32)
    assert np.max(np.abs(x[0])) > 65504.0
    y = _run_q4(ops, wq, s, b, x)
    ref = oracle.qgemv_q4_affine(wq, s, b, x, k)
    assert np.all(np.isfinite(y))
    for r in range(m):
        assert rel_err(y[r], ref[r]) <= 3e-5, (r, rel_err(y[r], ref[r]))
    assert not np.any(y[3])


@pytest.mark.parametrize("entry", ["gemv", "gate_up_silu", "qkv"])
def test_q4_affine_f32_activation_range(ops, entry):
    """f32 x far from N(0,1) through the three hi + lo f16 kernels (lfm.rs:985-1066 takes any
    f32 x): one row scaled past f16's largest value (|x| up to ~4e5 > 65504, where an
    unscaled split gives hi = inf and a NaN row), one at ~1e-5 and one at ~1e-12 (below
    f16's normal range, where hi, lo and lo/16 lose bits), and a row of zeros.  Each
    row is checked on its own against the f32 oracle, to the 3e-5 of the N(0,1) case."""
    import torch

    k, n, m = 896, 1000, 4
    row_scale = np.array([1e5, 1e-5, 1e-12, 0.0], np.float32)
    mats = [make_q4(n, k, m, x_dtype=np.float32, salt=77 + i) for i in range(3)]
    x = np.ascontiguousarray(mats[0][3] * row_scale[:, None], np.float32)
    assert np.max(np.abs(x[0])) > 65504.0
    refs = [oracle.qgemv_q4_affine(wq, s, b, x, k) for wq, s, b, _ in mats]
    if entry == "gemv":
        wq, s, b, _ = mats[0]
        outs, want = [_run_q4(ops, wq, s, b, x)], refs[:1]
    elif entry == "gate_up_silu":
        (wg, sg, bg, _), (wu, su, bu, _) = mats[0], mats[1]
        h = torch.empty((m, n), dtype=torch.float32, device="cuda")
        ops.encode_gate_up_silu_q4_affine(_t(wg), _t(sg), _t(bg), _t(wu), _t(su), _t(bu), _t(x), h)
        torch.cuda.synchronize()
        outs, want = [h.cpu().numpy()], [oracle.silu_mul_(np.ascontiguousarray(refs[0]), refs[1])]
    else:
        ys = [torch.empty((m, n), dtype=torch.float32, device="cuda") for _ in range(3)]
        args = []
        for wq, s, b, _ in mats:
            args += [_t(wq), _t(s), _t(b)]
        ops.encode_qkv_q4_affine(*args, _t(x), *ys)
        torch.cuda.synchronize()
        outs, want = [y.cpu().numpy() for y in ys], refs
    for y, ref in zip(outs, want):
        assert np.all(np.isfinite(y))
        for r in range(m):
            assert rel_err(y[r], ref[r]) <= 3e-5, (entry, r, rel_err(y[r], ref[r]))
        assert not np.any(y[3])  # x = 0: exactly zero


# ------------------------------------------------------------------- i4 sym ----

def test_i4_sym_logits(ops):
    k, n, gs = 512, 700, 128
    w = oracle.gen_i8((n, k // 2), seed(6, 0)).view(np.uint8)
    s = oracle.gen_uniform((n * (k // gs),), seed(6, 1), 1e-3, 2e-2).astype(np.float16).view(np.uint16)
    x = oracle.gen_normal((k,), seed(6, 2), 0.0, 1.0)
    y = ops.logits_i4(x, w, s, n, k, gs, "test.i4")
    ref = oracle.matmul_i4_f32(w, s, n, k, gs, x)
    assert rel_err(y, ref) <= TOL_F32


def _run_i4(ops, w, s, gs, x):
    import torch

    n, m, k = w.shape[0], x.shape[0], x.shape[1]
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    ops.encode_qgemv_i4_sym(_t(w), _t(s.view(np.int16)), gs, _t(x), y, k)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def _i4_case(n, k, m, gs, salt, xdt=np.float32):
    w = oracle.gen_i8((n, (k + 1) // 2), seed(60 + salt, 0)).view(np.uint8)
    spr = (k + gs - 1) // gs
    s = oracle.gen_uniform((n * spr,), seed(60 + salt, 1), 1e-3, 2e-2).astype(np.float16).view(np.uint16)
    x = oracle.gen_normal((m, k), seed(60 + salt, 2), 0.0, 1.0).astype(xdt)
    return w, s, x


@pytest.mark.parametrize("n,k", [(6912, 1152), (1152, 6912)])
@pytest.mark.parametrize("m", [1, 2, 4])
def test_i4_sym_gemma_mlp_per_row(ops, n, k, m):
    """Gemma-3-1B MLP projections in the reference's i4 format: one f16 scale
    per row, gs = in_dim (gemma.rs:1446-1471), f32 activations."""
    w, s, x = _i4_case(n, k, m, k, salt=m + (k == 6912))
    y = _run_i4(ops, w, s, k, x)
    assert rel_err(y, oracle.qgemv_i4_sym(w, s, k, x, n, k)) <= TOL_F32
    if m == 1:
        assert rel_err(y[0], oracle.matmul_i4_f32(w, s, n, k, k, x[0])) <= TOL_F32


@pytest.mark.parametrize("n,k,m,gs,xdt", [
    (6912, 1152, 1, 1152, np.float16),   # f16 x widened at staging
    (1152, 6912, 4, 6912, np.float16),
    (1000, 1024, 3, 32, np.float32),     # one group per chunk
    (777, 1152, 2, 96, np.float32),      # three chunks per group
    (513, 4096, 1, 2048, np.float32),    # two groups per row, MP passes
    (300, 1152, 1, 4096, np.float32),    # gs > k: still one scale per row
    (200, 1001, 1, 1001, np.float32),    # odd k: one-wave-per-row kernel
    (200, 1024, 1, 48, np.float32),      # gs % 32 != 0: one-wave-per-row kernel
    (200, 1152, 5, 1152, np.float32),    # m > 4: one-wave-per-row kernel
])
def test_i4_sym_shapes_and_groups(ops, n, k, m, gs, xdt):
    w, s, x = _i4_case(n, k, m, gs, salt=n % 97 + m, xdt=xdt)
    y = _run_i4(ops, w, s, gs, x)
    assert rel_err(y, oracle.qgemv_i4_sym(w, s, gs, x, n, k)) <= TOL_F32


# -------------------------------------------------------------- edge cases ----

def test_empty_inputs_are_noops(ops):
    import torch

    w = torch.zeros((0, 64), dtype=torch.int8, device="cuda")
    s = torch.ones(1, dtype=torch.float32, device="cuda")
    x = torch.zeros((1, 64), dtype=torch.float32, device="cuda")
    y = torch.zeros((1, 0), dtype=torch.float32, device="cuda")
    ops.encode_qgemv_i8(w, s, x, y)
    torch.cuda.synchronize()


def test_k_zero_gives_zero(ops):
    import torch

    n = 10
    w = torch.zeros((n, 0), dtype=torch.int8, device="cuda")
    s = torch.ones(n, dtype=torch.float32, device="cuda")
    x = torch.zeros((1, 0), dtype=torch.float32, device="cuda")
    y = torch.full((1, n), 7.0, dtype=torch.float32, device="cuda")
    from cellm_amd._lib import load
    import ctypes as C

    lib = load()
    def ptr(t):
        return C.c_void_p(t.data_ptr()) if t.data_ptr() else None

    rc = lib.cellm_hip_qgemv_i8(ops.handle, ptr(w), ptr(s), 0, n, ptr(x), 0, None, ptr(y), 1, n, 0, None)
    assert rc == 0
    torch.cuda.synchronize()
    assert float(y.abs().max()) == 0.0


def test_bad_k_is_rejected(ops):
    import torch
    from cellm_amd import CellmHipError

    wq = torch.zeros((4, 1), dtype=torch.int32, device="cuda")
    s = torch.ones((4, 1), dtype=torch.float16, device="cuda")
    x = torch.zeros((1, 12), dtype=torch.float16, device="cuda")
    y = torch.zeros((1, 4), dtype=torch.float32, device="cuda")
    import ctypes as C
    from cellm_amd._lib import load, last_error

    rc = load().cellm_hip_qgemv_q4_affine(ops.handle, C.c_void_p(wq.data_ptr()), C.c_void_p(s.data_ptr()),
                                          C.c_void_p(s.data_ptr()), 1, 64, C.c_void_p(x.data_ptr()), 1,
                                          C.c_void_p(y.data_ptr()), 1, 4, 12, None)
    assert rc == -1 and "multiple of 8" in last_error()
    with pytest.raises(CellmHipError):
        ops.weight_lookup("no.such.key")


# ------------------------------------------------------------- HIP graphs ----

def test_graph_replays_match_eager(ops):
    """Each path captured in a HIP graph, replayed several times with eager
    work in between; every replay equals the eager result bit for bit."""
    import torch

    cases = []
    a = [_t(v) if i != 1 and i != 2 else _sb_tensor(v) for i, v in enumerate(make_q4(40000, 896, 1, salt=11))]
    cases.append(lambda y, st: ops.encode_qgemv_q4_affine(a[0], a[1], a[2], a[3], y, stream=st))  # persistent GEMV
    c = [_t(v) for v in make_i8(3000, 1152, 16, cfg=3, x_dtype=np.float16, salt=12)]
    cases.append(lambda y, st: ops.encode_qgemv_i8(c[0], c[1], c[2], y, stream=st))  # batched MFMA decode
    e = [_t(v) if i != 1 and i != 2 else _sb_tensor(v) for i, v in enumerate(make_q4(896, 4864, 512, cfg=4, salt=13))]
    cases.append(lambda y, st: ops.encode_qgemm_q4_affine(e[0], e[1], e[2], e[3], y, stream=st))  # split-K qGEMM
    shapes = [(1, 40000), (16, 3000), (512, 896)]
    cap = torch.cuda.Stream()
    for fn, (m, n) in zip(cases, shapes):
        ref = torch.empty((m, n), dtype=torch.float32, device="cuda")
        fn(ref, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        y = torch.zeros((m, n), dtype=torch.float32, device="cuda")
        with torch.cuda.stream(cap):
            fn(y, cap.cuda_stream)  # warm-up on the capture stream (per-stream scratch)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap):
            fn(y, cap.cuda_stream)
        for rep in range(3):
            y.fill_(float("nan"))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, ref), (m, n, rep)
            _ = (ref * 2).sum().item()  # eager work between replays


def test_qgemv_batch_matches_single_calls(ops):
    """cellm_hip_qgemv_batch enqueues each op as its single-op entry point does."""
    import torch

    from cellm_amd._lib import CellmHipError, QgemvOp

    q = [_t(v) if i not in (1, 2) else _sb_tensor(v) for i, v in enumerate(make_q4(1000, 1152, 1, cfg=3, salt=21))]
    e = [_t(v) for v in make_i8(700, 576, 4, x_dtype=np.float16, salt=22)]
    g = [_t(v) if i not in (1, 2) else _sb_tensor(v) for i, v in enumerate(make_q4(300, 896, 16, cfg=3, salt=23))]
    iw, isc, ix = _i4_case(640, 1152, 2, 1152, salt=24)
    i4 = [_t(iw), _t(isc.view(np.int16)), _t(ix)]
    outs = [torch.empty(shape, dtype=torch.float32, device="cuda")
            for shape in ((1, 1000), (4, 700), (16, 300), (2, 640))]
    refs = [torch.empty_like(o) for o in outs]
    ops.encode_qgemv_q4_affine(q[0], q[1], q[2], q[3], refs[0])
    ops.encode_qgemv_i8(e[0], e[1], e[2], refs[1])
    ops.encode_qgemv_q4_affine(g[0], g[1], g[2], g[3], refs[2])
    ops.encode_qgemv_i4_sym(i4[0], i4[1], 1152, i4[2], refs[3], 1152)
    ops.encode_qgemv_batch([ops.qgemv_op_q4_affine(q[0], q[1], q[2], q[3], outs[0]),
                            ops.qgemv_op_i8(e[0], e[1], e[2], outs[1]),
                            ops.qgemv_op_q4_affine(g[0], g[1], g[2], g[3], outs[2]),
                            ops.qgemv_op_i4_sym(i4[0], i4[1], 1152, i4[2], outs[3], 1152)])
    torch.cuda.synchronize()
    for o, r in zip(outs, refs):
        assert torch.equal(o, r)
    # an unknown op kind fails with its own status after the ops before it
    outs[0].zero_()
    bad = QgemvOp(kind=9)
    with pytest.raises(CellmHipError, match="unknown kind"):
        ops.encode_qgemv_batch([ops.qgemv_op_q4_affine(q[0], q[1], q[2], q[3], outs[0]), bad])
    torch.cuda.synchronize()
    assert torch.equal(outs[0], refs[0])


# ----------------------------------------------------- fused multi-output ----

@pytest.mark.parametrize("m,xdt", [(1, np.float32), (4, np.float16), (8, np.float16), (3, np.float32)])
def test_qkv_i8_fused(ops, m, xdt):
    """SmolLM2-360M attention: q 960 rows, k/v 320 rows, hidden 960; biases,
    and a per-tensor scale on v.  m <= 4 is one launch, m = 8 the fallback."""
    import torch

    k, rq, rkv = 960, 960, 320
    wq, sq, x = make_i8(rq, k, m, cfg=5, scale_dtype=np.float16, x_dtype=xdt, salt=31)
    wk, sk, _ = make_i8(rkv, k, m, cfg=5, scale_dtype=np.float16, salt=32)
    wv, sv, _ = make_i8(rkv, k, m, cfg=5, scale_dtype=np.float16, salt=33)
    sv = sv[:1].copy()  # per-tensor
    bq = oracle.gen_normal((rq,), seed(5, 8, 1), 0.0, 1.0)
    bk = oracle.gen_normal((rkv,), seed(5, 8, 2), 0.0, 1.0)
    outs = [torch.empty((m, n), dtype=torch.float32, device="cuda") for n in (rq, rkv, rkv)]
    ops.encode_qkv_i8(_t(wq), _t(sq), _t(wk), _t(sk), _t(wv), _t(sv), _t(x), *outs, bq=_t(bq), bk=_t(bk))
    torch.cuda.synchronize()
    refs = [oracle.qgemv_i8(wq, sq, x) + bq[None, :], oracle.qgemv_i8(wk, sk, x) + bk[None, :],
            oracle.qgemv_i8(wv, np.full(rkv, sv[0], np.float16), x)]
    for o, r in zip(outs, refs):
        assert rel_err(o.cpu().numpy(), r) <= TOL_F32


@pytest.mark.parametrize("m,xdt", [(1, np.float32), (4, np.float16), (8, np.float16)])
def test_gate_up_silu_i8(ops, m, xdt):
    """SmolLM2-360M MLP: h = silu(Wg.x*sg + bg) * (Wu.x*su) for 2560 rows."""
    import torch

    k, n = 960, 2560
    wg, sg, x = make_i8(n, k, m, cfg=5, scale_dtype=np.float16, x_dtype=xdt, salt=41)
    wu, su, _ = make_i8(n, k, m, cfg=5, scale_dtype=np.float16, salt=42)
    bg = oracle.gen_normal((n,), seed(5, 9, 1), 0.0, 0.5)
    h = torch.empty((m, n), dtype=torch.float32, device="cuda")
    ops.encode_gate_up_silu_i8(_t(wg), _t(sg), _t(wu), _t(su), _t(x), h, bg=_t(bg))
    torch.cuda.synchronize()
    g = np.ascontiguousarray(oracle.qgemv_i8(wg, sg, x) + bg[None, :], np.float32)
    ref = oracle.silu_mul_(g, oracle.qgemv_i8(wu, su, x))
    assert rel_err(h.cpu().numpy(), ref) <= TOL_F32


@pytest.mark.parametrize("k,rq,rkv,m,sb,xdt,biased", [
    (896, 896, 128, 1, np.float16, np.float16, True),    # Qwen2.5-0.5B q/k/v, f16 x
    (896, 896, 128, 4, np.float32, np.float32, True),    # from a .cellm u32 file: f32 S/B and x
    (1152, 1024, 256, 2, "bf16", np.float32, False),     # Gemma-3-1B shapes, no bias
    (4864, 300, 100, 3, np.float16, np.float32, True),   # long rows (two register passes), ragged rows
    (896, 896, 128, 5, np.float16, np.float32, True),    # m > 4: one GEMV per projection + bias kernel
])
def test_qkv_q4_affine(ops, k, rq, rkv, m, sb, xdt, biased):
    """Three MLX q4 projections of one x in one launch with projection biases after the row
    sums (cellm_hip_qgemv_q4_affine_qkv), against the oracle's three GEMVs plus the bias
    (lfm.rs:985-1066, qwen.rs:1132-1139); f32 x within 3e-5 (hi + lo f16 parts)."""
    import torch

    mats = [make_q4(r, k, m, sb_dtype=sb, x_dtype=xdt, salt=90 + i + m) for i, r in enumerate((rq, rkv, rkv))]
    x = mats[0][3]
    biases = [oracle.gen_normal((r,), seed(3, 9, i), 0.0, 1.0) if biased else None
              for i, r in enumerate((rq, rkv, rkv))]
    outs = [torch.empty((m, r), dtype=torch.float32, device="cuda") for r in (rq, rkv, rkv)]
    args = []
    for wq, s, b, _ in mats:
        args += [_t(wq), _sb_tensor(s), _sb_tensor(b)]
    ops.encode_qkv_q4_affine(*args, _t(x), *outs, *[None if bb is None else _t(bb) for bb in biases])
    torch.cuda.synchronize()
    for (wq, s, b, _), bb, y in zip(mats, biases, outs):
        ref = oracle.qgemv_q4_affine(wq, s, b, x, k)
        if bb is not None:
            ref = (ref + bb[None, :]).astype(np.float32)
        err = rel_err(y.cpu().numpy(), ref)
        assert err <= TOL_F32
        if xdt == np.float32:
            assert err <= 3e-5


@pytest.mark.parametrize("k,n,m,sb,group,xdt", [
    (896, 4864, 1, np.float16, 64, np.float16),    # Qwen2.5-0.5B MLP halves, one launch
    (896, 4864, 4, np.float16, 64, np.float16),
    (1152, 6912, 1, np.float32, 64, np.float16),   # Gemma-3-1B MLP halves, f32 S/B as LFM files hold them
    (1152, 6912, 2, "bf16", 128, np.float16),
    (4864, 896, 3, np.float16, 32, np.float16),    # long rows: two register passes per lane
    (896, 1000, 1, np.float16, 64, np.float32),    # f32 x (the LFM runner's): one launch over hi + lo f16 parts
    (896, 4864, 4, np.float32, 64, np.float32),    # Qwen2.5-0.5B MLP halves from a .cellm u32 file, f32 x
    (4864, 896, 3, np.float16, 64, np.float32),    # f32 x of long rows: past 64 KB of LDS
    (896, 4864, 5, np.float16, 64, np.float16),    # m > 4: two GEMVs + SiLU kernel
])
def test_gate_up_silu_q4(ops, k, n, m, sb, group, xdt):
    """h = silu(gate) * up over MLX q4 affine gate/up matrices (the mv2 + silu_mul
    pattern, metal.rs:512-541,232-243), against the oracle's two GEMVs and
    silu_mul_f32_inplace."""
    import torch

    wg, sg, bg, x = make_q4(n, k, m, sb_dtype=sb, x_dtype=xdt, group=group, salt=51 + m)
    wu, su, bu, _ = make_q4(n, k, m, sb_dtype=sb, group=group, salt=52 + m)
    h = torch.empty((m, n), dtype=torch.float32, device="cuda")
    ops.encode_gate_up_silu_q4_affine(_t(wg), _sb_tensor(sg), _sb_tensor(bg), _t(wu), _sb_tensor(su),
                                      _sb_tensor(bu), _t(x), h, group=group)
    torch.cuda.synchronize()
    g = np.ascontiguousarray(oracle.qgemv_q4_affine(wg, sg, bg, x, k, gs=group), np.float32)
    ref = oracle.silu_mul_(g, oracle.qgemv_q4_affine(wu, su, bu, x, k, gs=group))
    assert rel_err(h.cpu().numpy(), ref) <= TOL_F32


# ------------------------------------------------------------ GELU * up ----
# Gemma's MLP activation (gemma.rs:844-846 over gelu_tanh_f32, gemma.rs:1689-1693; Metal
# gelu_tanh_mul_f32_inplace, metal.rs:245-257) at the Gemma-3-1B MLP shape 1152 -> 6912.

def test_gelu_tanh_mul_elementwise(ops):
    """cellm_hip_gelu_tanh_mul_f32 against the oracle: the device tanhf and glibc's differ by an
    ulp or two, so the bar is normwise 1e-6 (1 + tanh cancels for large negative g, where both
    results are ~1e-7 in absolute terms)."""
    import torch

    n = 6912 * 4
    g = np.concatenate([np.linspace(-12.0, 12.0, 4001), oracle.gen_normal((n - 4001,), seed(3, 12), 0.0, 3.0)])
    g = g.astype(np.float32)
    u = oracle.gen_normal((n,), seed(3, 13), 0.0, 1.0)
    gd = _t(g.copy())
    ops.encode_gelu_tanh_mul(gd, _t(u))
    torch.cuda.synchronize()
    ref = oracle.gelu_tanh_mul_(g.copy(), u)
    assert rel_err(gd.cpu().numpy(), ref) <= 1e-6
    # not the SiLU: the two activations differ at this size
    assert rel_err(oracle.silu_mul_(g.copy(), u), ref) > 1e-2


@pytest.mark.parametrize("m,xdt", [(1, np.float16), (4, np.float16), (2, np.float32), (8, np.float16)])
def test_gate_up_gelu_i8(ops, m, xdt):
    """int8 gate/up with the tanh GELU epilogue (cellm_hip_qgemv_i8_gate_up_gelu): one launch for
    m <= 4, the two GEMVs and the elementwise kernel at m = 8; against the oracle's two
    matmul_i8_f32 rows and gelu_tanh_mul."""
    import torch

    k, n = 1152, 6912
    wg, sg, x = make_i8(n, k, m, cfg=3, scale_dtype=np.float16, x_dtype=xdt, salt=141)
    wu, su, _ = make_i8(n, k, m, cfg=3, scale_dtype=np.float16, salt=142)
    h = torch.empty((m, n), dtype=torch.float32, device="cuda")
    ops.encode_gate_up_gelu_i8(_t(wg), _t(sg), _t(wu), _t(su), _t(x), h)
    torch.cuda.synchronize()
    g = np.ascontiguousarray(oracle.qgemv_i8(wg, sg, x), np.float32)
    u = oracle.qgemv_i8(wu, su, x)
    ref = oracle.gelu_tanh_mul_(g.copy(), u)
    got = h.cpu().numpy()
    assert rel_err(got, ref) <= TOL_F32
    # the GELU, not the SiLU: where |g| < 2 the two activations differ by far more than the error
    silu = oracle.silu_mul_(g.copy(), u)
    near = np.abs(g) < 2.0
    assert near.sum() > 10
    assert np.max(np.abs(got - silu)[near]) > 100 * np.max(np.abs(got - ref)[near])


@pytest.mark.parametrize("m,sb,xdt", [(1, np.float16, np.float16), (4, np.float32, np.float16),
                                      (2, np.float16, np.float32), (5, np.float16, np.float16)])
def test_gate_up_gelu_q4(ops, m, sb, xdt):
    """MLX q4 gate/up with the tanh GELU epilogue (cellm_hip_qgemv_q4_affine_gate_up_gelu), Gemma
    MLP halves 1152 -> 6912: one launch for m <= 4 (f16 or f32 x), two GEMVs and the elementwise
    kernel at m = 5."""
    import torch

    k, n = 1152, 6912
    wg, sg, bg, x = make_q4(n, k, m, sb_dtype=sb, x_dtype=xdt, salt=151 + m)
    wu, su, bu, _ = make_q4(n, k, m, sb_dtype=sb, salt=152 + m)
    h = torch.empty((m, n), dtype=torch.float32, device="cuda")
    ops.encode_gate_up_gelu_q4_affine(_t(wg), _sb_tensor(sg), _sb_tensor(bg), _t(wu), _sb_tensor(su),
                                      _sb_tensor(bu), _t(x), h)
    torch.cuda.synchronize()
    g = np.ascontiguousarray(oracle.qgemv_q4_affine(wg, sg, bg, x, k), np.float32)
    ref = oracle.gelu_tanh_mul_(g, oracle.qgemv_q4_affine(wu, su, bu, x, k))
    assert rel_err(h.cpu().numpy(), ref) <= TOL_F32


@pytest.mark.parametrize("m", [1, 4])
def test_gate_up_gelu_i4(ops, m):
    """Symmetric i4 gate/up (gs = in_dim, gemma.rs:1446-1471) with the tanh GELU
    (cellm_hip_qgemv_i4_gate_up_gelu), f32 x, 1152 -> 6912, against the oracle's two
    matmul_i4_f32 rows and gelu_tanh_mul."""
    import torch

    k, n, gs = 1152, 6912, 1152
    wg = oracle.gen_i8((n, k // 2), seed(6, 20, m)).view(np.uint8)
    wu = oracle.gen_i8((n, k // 2), seed(6, 21, m)).view(np.uint8)
    sg = oracle.gen_uniform((n,), seed(6, 22, m), 1e-3, 2e-2).astype(np.float16)
    su = oracle.gen_uniform((n,), seed(6, 23, m), 1e-3, 2e-2).astype(np.float16)
    x = oracle.gen_normal((m, k), seed(6, 24, m), 0.0, 1.0)
    h = torch.empty((m, n), dtype=torch.float32, device="cuda")
    ops.encode_gate_up_gelu_i4_sym(_t(wg), _t(sg.view(np.int16)), _t(wu), _t(su.view(np.int16)), gs, _t(x), h, k)
    torch.cuda.synchronize()
    got = h.cpu().numpy()
    for r in range(m):
        g = np.ascontiguousarray(oracle.matmul_i4_f32(wg, sg.view(np.uint16), n, k, gs, x[r]), np.float32)
        ref = oracle.gelu_tanh_mul_(g, oracle.matmul_i4_f32(wu, su.view(np.uint16), n, k, gs, x[r]))
        assert rel_err(got[r], ref) <= TOL_F32
