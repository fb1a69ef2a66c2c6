"""Writes the golden fixtures in this folder from the CPU oracle.

The reference ships no fixtures for the quantized kernels, so these vectors are
produced by the oracle on inputs drawn with the reference's test LCG
(crates/cellm-kernels/tests/metal_parity.rs:17-26) and are pinned by the closed
forms in tests/test_oracle.py.  They let GPU tests and later rounds check
against fixed bits without rebuilding the oracle.

    python tests/golden/gen_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

import oracle  # noqa: E402


def main():
    out = {}
    # config 1 shape (SmolLM2-135M int8, fp32 scales, fp32 x), trimmed N
    n, k = 64, 576
    w = oracle.gen_i8((n, k), 0xCE110010)
    s = oracle.gen_uniform((n,), 0xCE110011, 1e-3, 2e-2)
    x = oracle.gen_normal((1, k), 0xCE110012, 0.0, 1.0)
    out.update(i8_w=w, i8_s=s, i8_x=x, i8_y=oracle.qgemv_i8(w, s, x))
    # f16 scales, reference-native: cpu_kernels::matmul_i8_f32
    s16 = s.astype(np.float16)
    out.update(i8_s16=s16.view(np.uint16), i8_y16=oracle.matmul_i8_f32(w, s16.view(np.uint16), x[0]))
    # config 2 shape (Qwen q4 affine 896 -> 48 rows), fp16 S/B/x
    n, k = 48, 896
    wq = oracle.gen_q4_words((n, k // 8), 0xCE110020)
    sq = oracle.gen_normal((n, k // 64), 0xCE110021, 0.02, 0.005, True).astype(np.float16)
    bq = oracle.gen_normal((n, k // 64), 0xCE110023, 0.0, 0.05).astype(np.float16)
    xq = oracle.gen_normal((2, k), 0xCE110022, 0.0, 1.0).astype(np.float16)
    out.update(q4_wq=wq, q4_s=sq, q4_b=bq, q4_x=xq, q4_y=oracle.qgemv_q4_affine(wq, sq, bq, xq, k),
               q4_deq16=oracle.dequant_q4_affine_f16(wq, sq, bq, k),
               q4_deq32=oracle.q4_affine_dequant_f32(wq, sq, bq, k))
    # symmetric i4 (cpu_kernels::matmul_i4_f32), gs 64
    n, k, gs = 32, 256, 64
    w4 = oracle.gen_i8((n, k // 2), 0xCE110060).view(np.uint8)
    s4 = oracle.gen_uniform((n * (k // gs),), 0xCE110061, 1e-3, 2e-2).astype(np.float16).view(np.uint16)
    x4 = oracle.gen_normal((k,), 0xCE110062, 0.0, 1.0)
    out.update(i4_w=w4, i4_s=s4, i4_x=x4, i4_y=oracle.matmul_i4_f32(w4, s4, n, k, gs, x4))
    np.savez_compressed(HERE / "golden_v1.npz", **out)
    print("wrote", HERE / "golden_v1.npz", sum(v.nbytes for v in out.values()), "bytes raw")


if __name__ == "__main__":
    main()
