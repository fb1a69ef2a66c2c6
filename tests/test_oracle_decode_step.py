"""The oracle's decode-step helpers (RMSNorm, RoPE, GQA attention over f16
K/V, SiLU, the int8 lm_head loop; oracle/cellm_oracle.c) composed into one
SmolLM2-360M-shape step, against the independent float64 step of
tests/_llama_f64.py: the two share no code, so a wrong formula on either side
(a missing 1/sqrt(head_dim), a swapped RoPE half, an RMSNorm over the wrong
length) moves the logits far beyond f32 rounding."""
from __future__ import annotations

import numpy as np

from tests._llama_f64 import f64_step
from tests.test_gpu_decode_step import CTX, DIMS, F64_TOL, block_table, make_kv, make_model, oracle_step


def test_oracle_step_matches_float64_step():
    model = make_model()
    k0, v0 = make_kv()
    for s in (0, 3):
        token = int(1000 + 7919 * s) % DIMS["VOCAB"]
        bt = block_table(s)
        ok, ov = k0.copy(), v0.copy()
        ref_id, ref_logits = oracle_step(model, ok, ov, token, CTX - 1, bt)
        fk, fv = k0.copy(), v0.copy()
        f64_id, f64_logits = f64_step(model, fk, fv, token, CTX - 1, bt, DIMS)
        rel = float(np.max(np.abs(ref_logits - f64_logits)) / np.max(np.abs(f64_logits)))
        assert ref_id == f64_id
        assert rel <= F64_TOL, rel
        # the K/V row each step wrote: the same f16 values up to one rounding step
        w = np.flatnonzero(ok != k0)
        np.testing.assert_array_equal(w, np.flatnonzero(fk != k0))
        d = np.abs(ok[w].view(np.float16).astype(np.float64) - fk[w].view(np.float16).astype(np.float64))
        assert float(d.max()) <= 2e-3 * float(np.abs(fk[w].view(np.float16).astype(np.float64)).max())
