"""CPU oracle for cellm's quantized-weight matmul path -- TEST INFRASTRUCTURE.

numpy wrappers over liboracle.so (built from cellm_oracle.c by oracle/Makefile).
Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py may
import this package; it is the checker, never part of the product path.

Every function restates a reference function (file:line in cellm_oracle.c).
Parity pins live in tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB_PATH = _DIR / "liboracle.so"
_lib = None

F32, F16, BF16 = 0, 1, 2


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            subprocess.run(["make", "-C", str(_DIR), "liboracle.so"], check=True, capture_output=True)
        _lib = C.CDLL(str(_LIB_PATH))
        _declare(_lib)
    return _lib


def _declare(L):
    vp, sz, i32, u64, f32 = C.c_void_p, C.c_size_t, C.c_int, C.c_uint64, C.c_float
    sig = {
        "oracle_f16_to_f32": (f32, [C.c_uint16]),
        "oracle_f32_to_f16": (C.c_uint16, [f32]),
        "oracle_bf16_to_f32": (f32, [C.c_uint16]),
        "oracle_f16_to_f32_array": (None, [vp, vp, sz]),
        "oracle_f32_to_f16_array": (None, [vp, vp, sz]),
        "oracle_lcg_fill": (None, [vp, sz, u64, f32]),
        "oracle_lcg_unit": (None, [vp, sz, u64]),
        "oracle_gen_i8": (None, [vp, sz, u64]),
        "oracle_gen_q4_words": (None, [vp, sz, u64]),
        "oracle_gen_uniform": (None, [vp, sz, u64, f32, f32]),
        "oracle_gen_normal": (None, [vp, sz, u64, f32, f32, i32]),
        "oracle_matmul_i8_f32": (None, [vp, vp, sz, sz, vp, vp]),
        "oracle_qgemv_i8": (None, [vp, vp, i32, vp, i32, sz, sz, sz, vp]),
        "oracle_llama_lm_head_i8": (None, [vp, vp, vp, sz, sz, vp]),
        "oracle_embed": (None, [i32, vp, sz, vp, vp, sz, sz, vp]),
        "oracle_llama_lm_head_f16_i4": (None, [i32, vp, vp, vp, sz, sz, vp]),
        "oracle_matmul_i4_f32": (None, [vp, vp, sz, sz, sz, sz, vp, vp]),
        "oracle_qgemv_i4_sym": (None, [vp, vp, sz, sz, vp, i32, sz, sz, sz, vp]),
        "oracle_qgemv_f16": (None, [vp, vp, i32, sz, sz, sz, vp]),
        "oracle_qgemv_i2": (None, [vp, vp, i32, vp, i32, sz, sz, sz, vp]),
        "oracle_qgemv_q1_0_g128": (None, [vp, vp, i32, sz, sz, sz, vp]),
        "oracle_q4_affine_dequant_f32": (None, [vp, vp, vp, i32, sz, sz, sz, vp]),
        "oracle_qgemv_q4_affine": (None, [vp, vp, vp, i32, vp, i32, sz, sz, sz, sz, vp]),
        "oracle_lfm_lm_head_q4_affine": (None, [vp, sz, vp, vp, sz, vp, sz, sz, vp]),
        "oracle_dequant_q4_affine_f16": (None, [vp, vp, vp, i32, sz, sz, sz, vp]),
        "oracle_matmul_f32": (None, [vp, sz, sz, vp, sz, vp]),
        "oracle_gemm_xwT_f32": (None, [vp, i32, vp, sz, sz, sz, vp]),
        "oracle_rms_norm_f32": (None, [vp, vp, sz, f32, vp]),
        "oracle_rope_half_f32": (None, [vp, sz, sz, sz, f32]),
        "oracle_rope_interleaved_f32": (None, [vp, sz, sz, sz, f32]),
        "oracle_gelu_tanh_mul_f32": (None, [vp, vp, sz]),
        "oracle_softmax_f32": (None, [vp, sz]),
        "oracle_attention_gqa_f16kv": (None, [vp, vp, vp, sz, vp, sz, sz, sz, f32, f32, vp, vp]),
        "oracle_silu_mul_f32": (None, [vp, vp, sz]),
        "oracle_argmax_first": (C.c_int64, [vp, sz]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(C.c_void_p)


def _dt(a: np.ndarray) -> int:
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.float16:
        return F16
    if a.dtype == np.uint16:  # raw bf16 bits
        return BF16
    raise TypeError(f"unsupported dtype {a.dtype}")


# --- conversions -----------------------------------------------------------

def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().oracle_f16_to_f32_array(_p(bits), _p(out), bits.size)
    return out


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


# --- generators (reference LCG, metal_parity.rs:17-26) -----------------------

def lcg_fill(n: int, seed: int, scale: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().oracle_lcg_fill(_p(out), n, seed, scale)
    return out


def gen_i8(shape, seed: int) -> np.ndarray:
    out = np.empty(shape, np.int8)
    lib().oracle_gen_i8(_p(out), out.size, seed)
    return out


def gen_q4_words(shape, seed: int) -> np.ndarray:
    out = np.empty(shape, np.uint32)
    lib().oracle_gen_q4_words(_p(out), out.size, seed)
    return out


def gen_uniform(shape, seed: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(shape, np.float32)
    lib().oracle_gen_uniform(_p(out), out.size, seed, lo, hi)
    return out


def gen_normal(shape, seed: int, mu: float, sigma: float, positive_only: bool = False) -> np.ndarray:
    out = np.empty(shape, np.float32)
    lib().oracle_gen_normal(_p(out), out.size, seed, mu, sigma, 1 if positive_only else 0)
    return out


# --- int8 GEMV and the Llama int8 lm_head -----------------------------------

def matmul_i8_f32(w: np.ndarray, scales_f16_bits: np.ndarray, x: np.ndarray) -> np.ndarray:
    """cpu_kernels::matmul_i8_f32 (x86 branch), f16 scales."""
    n, k = w.shape
    w = np.ascontiguousarray(w, np.int8)
    s = np.ascontiguousarray(scales_f16_bits, np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(n, np.float32)
    lib().oracle_matmul_i8_f32(_p(w), _p(s), n, k, _p(x), _p(out))
    return out


def qgemv_i8(w: np.ndarray, scales: np.ndarray, x: np.ndarray) -> np.ndarray:
    """Batched int8 GEMV: x [M,K] (f32 or f16), scales [N] (f32, f16, or uint16 = bf16 bits)."""
    n, k = w.shape
    x2 = np.ascontiguousarray(x.reshape(-1, k))
    m = x2.shape[0]
    w = np.ascontiguousarray(w, np.int8)
    s = np.ascontiguousarray(scales)
    y = np.empty((m, n), np.float32)
    lib().oracle_qgemv_i8(_p(w), _p(s), _dt(s), _p(x2), _dt(x2), m, n, k, _p(y))
    return y


def llama_lm_head_i8(x: np.ndarray, w: np.ndarray, scales_f16_bits: np.ndarray) -> np.ndarray:
    vocab, hidden = w.shape
    out = np.empty(vocab, np.float32)
    lib().oracle_llama_lm_head_i8(_p(np.ascontiguousarray(x, np.float32)), _p(np.ascontiguousarray(w, np.int8)),
                                  _p(np.ascontiguousarray(scales_f16_bits, np.uint16)), vocab, hidden, _p(out))
    return out


# --- Llama embedding and f16 / i4 lm_head sources -----------------------------

EMBED_KINDS = {"f16": 0, "i8": 1, "i4": 2}


def embed(kind: str, tokens, w: np.ndarray, scales_f16_bits: np.ndarray | None, vocab: int, hidden: int) -> np.ndarray:
    """LlamaRunner::embed_token (llama.rs:676-726) for each token: kind "f16"
    (w f16 bits [vocab, hidden]), "i8" (int8 [vocab, hidden]) or "i4" (uint8
    [vocab, ceil(hidden/2)]), the last two with f16 row scales."""
    t = np.ascontiguousarray(tokens, np.uint32)
    out = np.empty((t.size, hidden), np.float32)
    sp = None if scales_f16_bits is None else _p(np.ascontiguousarray(scales_f16_bits, np.uint16))
    lib().oracle_embed(EMBED_KINDS[kind], _p(t), t.size, _p(np.ascontiguousarray(w)), sp, vocab, hidden, _p(out))
    return out


def llama_lm_head_f16_i4(kind: str, x: np.ndarray, w: np.ndarray, scales_f16_bits: np.ndarray | None,
                         vocab: int, hidden: int) -> np.ndarray:
    """The serial lm_head loop of llama.rs:576-646 over an f16 ("f16") or i4
    ("i4", per-row f16 scale) source; non-finite logits -> -inf."""
    out = np.empty(vocab, np.float32)
    sp = None if scales_f16_bits is None else _p(np.ascontiguousarray(scales_f16_bits, np.uint16))
    lib().oracle_llama_lm_head_f16_i4(0 if kind == "f16" else 1, _p(np.ascontiguousarray(x, np.float32)),
                                      _p(np.ascontiguousarray(w)), sp, vocab, hidden, _p(out))
    return out


# --- symmetric i4 ----------------------------------------------------------------

def matmul_i4_f32(w_u8: np.ndarray, scales_f16_bits: np.ndarray, m: int, k: int, gs: int, x: np.ndarray) -> np.ndarray:
    w_u8 = np.ascontiguousarray(w_u8, np.uint8)
    s = np.ascontiguousarray(scales_f16_bits, np.uint16)
    out = np.empty(m, np.float32)
    lib().oracle_matmul_i4_f32(_p(w_u8), _p(s), s.size, m, k, gs, _p(np.ascontiguousarray(x, np.float32)), _p(out))
    return out


def qgemv_i4_sym(w_u8, scales_f16_bits, gs, x, n, k):
    x2 = np.ascontiguousarray(x.reshape(-1, k))
    m = x2.shape[0]
    s = np.ascontiguousarray(scales_f16_bits, np.uint16)
    y = np.empty((m, n), np.float32)
    lib().oracle_qgemv_i4_sym(_p(np.ascontiguousarray(w_u8, np.uint8)), _p(s), s.size, gs, _p(x2), _dt(x2), m, n, k,
                              _p(y))
    return y


# --- f16, i2, q1_0_g128 --------------------------------------------------------

def qgemv_f16(w_f16_bits: np.ndarray, x: np.ndarray) -> np.ndarray:
    """y[m, n] = sum_k f32(W[n, k]) * x[m, k] (matmul_f16_f32, cpu_kernels.rs:135-214)."""
    n, k = w_f16_bits.shape
    x2 = np.ascontiguousarray(x.reshape(-1, k))
    y = np.empty((x2.shape[0], n), np.float32)
    lib().oracle_qgemv_f16(_p(np.ascontiguousarray(w_f16_bits, np.uint16)), _p(x2), _dt(x2), x2.shape[0], n, k, _p(y))
    return y


def qgemv_i2(w_u8: np.ndarray, scales_f16_bits: np.ndarray, x: np.ndarray, k: int, scale_mode: int) -> np.ndarray:
    """i2 rows of ceil(k/4) bytes; scale_mode 0 = Qwen (scale at the end), 1 = Gemma (per element)."""
    n = w_u8.shape[0]
    x2 = np.ascontiguousarray(x.reshape(-1, k))
    y = np.empty((x2.shape[0], n), np.float32)
    lib().oracle_qgemv_i2(_p(np.ascontiguousarray(w_u8, np.uint8)), _p(np.ascontiguousarray(scales_f16_bits, np.uint16)),
                          scale_mode, _p(x2), _dt(x2), x2.shape[0], n, k, _p(y))
    return y


def qgemv_q1_0_g128(w_u8: np.ndarray, x: np.ndarray, k: int) -> np.ndarray:
    """q1_0_g128 rows of k/128 blocks of 18 bytes (f16 d + 128 sign bits)."""
    n = w_u8.shape[0]
    x2 = np.ascontiguousarray(x.reshape(-1, k))
    y = np.empty((x2.shape[0], n), np.float32)
    lib().oracle_qgemv_q1_0_g128(_p(np.ascontiguousarray(w_u8, np.uint8)), _p(x2), _dt(x2), x2.shape[0], n, k, _p(y))
    return y


# --- MLX affine GEMV, lm_head and f16 dequant -----------------------------------

def q4_affine_dequant_f32(wq: np.ndarray, scales: np.ndarray, biases: np.ndarray, k: int, gs: int = 64) -> np.ndarray:
    n = wq.shape[0]
    s = np.ascontiguousarray(scales)
    b = np.ascontiguousarray(biases, s.dtype)
    out = np.empty((n, k), np.float32)
    lib().oracle_q4_affine_dequant_f32(_p(np.ascontiguousarray(wq, np.uint32)), _p(s), _p(b), _dt(s), n, k, gs,
                                       _p(out))
    return out


def qgemv_q4_affine(wq: np.ndarray, scales: np.ndarray, biases: np.ndarray, x: np.ndarray, k: int,
                    gs: int = 64) -> np.ndarray:
    n = wq.shape[0]
    x2 = np.ascontiguousarray(x.reshape(-1, k))
    m = x2.shape[0]
    s = np.ascontiguousarray(scales)
    b = np.ascontiguousarray(biases, s.dtype)
    y = np.empty((m, n), np.float32)
    lib().oracle_qgemv_q4_affine(_p(np.ascontiguousarray(wq, np.uint32)), _p(s), _p(b), _dt(s), _p(x2), _dt(x2), m, n,
                                 k, gs, _p(y))
    return y


def lfm_lm_head_q4_affine(wq, scales_f32, biases_f32, x, vocab, hidden):
    wq = np.ascontiguousarray(wq, np.uint32)
    s = np.ascontiguousarray(scales_f32, np.float32)
    b = np.ascontiguousarray(biases_f32, np.float32)
    out = np.empty(vocab, np.float32)
    lib().oracle_lfm_lm_head_q4_affine(_p(wq), wq.size, _p(s), _p(b), s.size, _p(np.ascontiguousarray(x, np.float32)),
                                       vocab, hidden, _p(out))
    return out


def dequant_q4_affine_f16(wq, scales, biases, k: int, gs: int = 64) -> np.ndarray:
    """Returns f16 bit patterns [N, K] (tools/convert/src/main.rs:4349-4444)."""
    n = wq.shape[0]
    s = np.ascontiguousarray(scales)
    b = np.ascontiguousarray(biases, s.dtype)
    out = np.empty((n, (k // 8) * 8), np.uint16)
    lib().oracle_dequant_q4_affine_f16(_p(np.ascontiguousarray(wq, np.uint32)), _p(s), _p(b), _dt(s), n, k, gs, _p(out))
    return out


# --- dense f32 -------------------------------------------------------------------

def matmul_f32(a: np.ndarray, b: np.ndarray, out: np.ndarray | None = None) -> np.ndarray:
    m, k = a.shape
    k2, n = b.shape if b.ndim == 2 else (b.shape[0], 1)
    assert k == k2
    if out is None:
        out = np.zeros((m, n), np.float32) if n > 1 else np.zeros(m, np.float32)
    lib().oracle_matmul_f32(_p(np.ascontiguousarray(a, np.float32)), m, k, _p(np.ascontiguousarray(b, np.float32)), n,
                            _p(out))
    return out


def gemm_xwT(x: np.ndarray, w_f32: np.ndarray) -> np.ndarray:
    m, k = x.shape
    n = w_f32.shape[0]
    x = np.ascontiguousarray(x)
    y = np.empty((m, n), np.float32)
    lib().oracle_gemm_xwT_f32(_p(x), _dt(x), _p(np.ascontiguousarray(w_f32, np.float32)), m, n, k, _p(y))
    return y


# --- decode-step helpers ----------------------------------------------------------

def rms_norm(x, w, eps):
    out = np.empty_like(x, dtype=np.float32)
    lib().oracle_rms_norm_f32(_p(np.ascontiguousarray(x, np.float32)), _p(np.ascontiguousarray(w, np.float32)), x.size,
                              eps, _p(out))
    return out


def rope_half_(x: np.ndarray, n_heads: int, head_dim: int, pos: int, theta: float) -> np.ndarray:
    assert x.dtype == np.float32 and x.flags["C_CONTIGUOUS"]
    lib().oracle_rope_half_f32(_p(x), n_heads, head_dim, pos, theta)
    return x


def rope_interleaved_(x: np.ndarray, n_heads: int, head_dim: int, pos: int, theta: float) -> np.ndarray:
    """rope_interleaved_inplace_f32 (cpu_kernels.rs:279-292), in place."""
    assert x.dtype == np.float32 and x.flags["C_CONTIGUOUS"]
    lib().oracle_rope_interleaved_f32(_p(x), n_heads, head_dim, pos, theta)
    return x


def softmax_(x: np.ndarray) -> np.ndarray:
    assert x.dtype == np.float32 and x.flags["C_CONTIGUOUS"]
    lib().oracle_softmax_f32(_p(x), x.size)
    return x


def attention_gqa_f16kv(kcache_bits, vcache_bits, bases, q, n_heads, n_kv_heads, head_dim, attn_scale=None,
                        soft_cap=None):
    """attention_single_token_gqa_f32 (kvcache.rs:710-789); attn_scale / soft_cap
    None are the reference's None (1/sqrt(head_dim); no cap)."""
    bases = np.ascontiguousarray(bases, np.uint64)
    scores = np.empty(max(len(bases), 1), np.float32)
    out = np.empty(n_heads * head_dim, np.float32)
    lib().oracle_attention_gqa_f16kv(_p(np.ascontiguousarray(kcache_bits, np.uint16)),
                                     _p(np.ascontiguousarray(vcache_bits, np.uint16)), _p(bases), len(bases),
                                     _p(np.ascontiguousarray(q, np.float32)), n_heads, n_kv_heads, head_dim,
                                     0.0 if attn_scale is None else attn_scale, 0.0 if soft_cap is None else soft_cap,
                                     _p(scores), _p(out))
    return out


def silu_mul_(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    assert gate.dtype == np.float32 and gate.flags["C_CONTIGUOUS"]
    lib().oracle_silu_mul_f32(_p(gate), _p(np.ascontiguousarray(up, np.float32)), gate.size)
    return gate


def gelu_tanh_mul_(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """gate = gelu_tanh_f32(gate) * up in place (gemma.rs:844-846, 1689-1693)."""
    assert gate.dtype == np.float32 and gate.flags["C_CONTIGUOUS"]
    lib().oracle_gelu_tanh_mul_f32(_p(gate), _p(np.ascontiguousarray(up, np.float32)), gate.size)
    return gate


def argmax_first(logits: np.ndarray) -> int:
    return int(lib().oracle_argmax_first(_p(np.ascontiguousarray(logits, np.float32)), logits.size))
