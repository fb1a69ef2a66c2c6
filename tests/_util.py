"""Shared helpers for the parity tests: seeded inputs and error metrics."""
from __future__ import annotations

import numpy as np

import oracle

# One fixed seed per config and tensor: 0xCE11_0000 + cfg*16 + tensor.
def seed(cfg: int, tensor: int, salt: int = 0) -> int:
    return 0xCE110000 + cfg * 16 + tensor + (salt << 20)


def rel_err(y: np.ndarray, ref: np.ndarray) -> float:
    """Normwise max relative error: max|y - ref| / max|ref| (robust to cancellation)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    denom = float(np.max(np.abs(ref))) if ref.size else 1.0
    if denom == 0.0:
        denom = 1.0
    return float(np.max(np.abs(y - ref))) / denom if ref.size else 0.0


def make_i8(n: int, k: int, m: int, cfg: int = 1, scale_dtype=np.float32, x_dtype=np.float32, salt: int = 0):
    """Config 1/3 int8 inputs: W U[-127,127], S U[1e-3,2e-2] per row, x N(0,1)."""
    w = oracle.gen_i8((n, k), seed(cfg, 0, salt))
    s = oracle.gen_uniform((n,), seed(cfg, 1, salt), 1e-3, 2e-2)
    if scale_dtype == np.float16:
        s = s.astype(np.float16)
    x = oracle.gen_normal((m, k), seed(cfg, 2, salt), 0.0, 1.0)
    x = x.astype(x_dtype)
    return w, s, x


def make_q4(n: int, k: int, m: int, cfg: int = 2, sb_dtype=np.float16, x_dtype=np.float16, group: int = 64,
            salt: int = 0):
    """Config 2-4 affine inputs: nibbles U{0..15}; S N(0.02,0.005)>0, B N(0,0.05) per group; x N(0,1)."""
    wq = oracle.gen_q4_words((n, k // 8), seed(cfg, 0, salt))
    groups = (k + group - 1) // group
    s = oracle.gen_normal((n, groups), seed(cfg, 1, salt), 0.02, 0.005, positive_only=True)
    b = oracle.gen_normal((n, groups), seed(cfg, 3, salt), 0.0, 0.05)
    if sb_dtype == np.float16:
        s, b = s.astype(np.float16), b.astype(np.float16)
    elif sb_dtype == "bf16":
        s = (s.view(np.uint32) >> 16).astype(np.uint16)  # truncation to bf16 bits: any bf16 value is a valid input
        b = (b.view(np.uint32) >> 16).astype(np.uint16)
    x = oracle.gen_normal((m, k), seed(cfg, 2, salt), 0.0, 1.0).astype(x_dtype)
    return wq, s, b, x
