"""cellm_hip_linear_file: one projection by the dtype of its .cellm weight
tensor, under each runner family's linear_f16_out_in rules
(llama.rs:743-941, qwen.rs:1033-1105, gemma.rs:1358-1499, lfm.rs:924-981).

- every (family, dtype) arm the reference has runs the GEMV of its format and
  matches the oracle's restatement of that arm within 1e-3 of the largest
  output, at a ragged shape and at a Qwen-size shape, two activation rows;
- the arms that differ between families differ here too: Llama's i4 reads the
  row's first scale (gs = in), Qwen's splits the row into groups when
  .qscale holds several scales per row; Qwen's i2 scales the row sum, Gemma's
  each element;
- refusals carry the reference's messages (unknown dtype per family, 2-D and
  [out, in] checks, qscale counts, missing tensors, an LFM u32 tensor without
  scales/biases falling back to the f16 reading);
- the second call for a tensor reuses the cached device copy.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from _cellm_writer import llama_header, write_cellm

pytestmark = pytest.mark.gpu

M = 2
SHAPES = [(37, 256), (1152, 896)]  # (out, in)


def _f16(o, i, sd):
    return oracle.gen_normal((o, i), sd, 0.0, 1.0 / np.sqrt(i)).astype(np.float16)


def _i8(o, i, sd):
    w = oracle.gen_i8((o, i), sd)
    s = (oracle.gen_uniform((o,), sd + 1, 1e-3, 2e-2)).astype(np.float16)
    return w, s


def _i4(o, i, sd, groups=1):
    w = oracle.gen_i8((o, (i + 1) // 2), sd).view(np.uint8)
    s = (oracle.gen_uniform((o * groups,), sd + 1, 0.5, 1.5) / (4.6 * np.sqrt(i))).astype(np.float16)
    return w, s


def _i2(o, i, sd):
    w = oracle.gen_i8((o, (i + 3) // 4), sd).view(np.uint8)
    s = (oracle.gen_uniform((o,), sd + 1, 0.5, 1.5) / np.sqrt(i)).astype(np.float16)
    return w, s


def _q1(o, i, sd):
    w = oracle.gen_i8((o, i // 128 * 18), sd).view(np.uint8).copy()
    d = (oracle.gen_uniform((o, i // 128), sd + 1, 0.5, 1.5) / np.sqrt(i)).astype(np.float16)
    w.reshape(o, i // 128, 18)[:, :, :2] = d.view(np.uint8).reshape(o, i // 128, 2)
    return w


def _u32(o, i, sd):
    wq = oracle.gen_q4_words((o, i // 8), sd)
    base = 1.0 / (4.6 * np.sqrt(i))
    s = (oracle.gen_uniform((o, (i + 63) // 64), sd + 1, 0.5, 1.5) * base).astype(np.float32)
    b = (-7.5 * s + oracle.gen_normal(s.shape, sd + 2, 0.0, 0.1 * base)).astype(np.float32)
    return wq, s, b


def _cases(o, i):
    """(family, tensor name, file tensors, oracle function of x) for every arm."""
    t = f"{o}x{i}"
    cs = []
    w = _f16(o, i, 0xD1000001)
    for fam in ("llama", "qwen", "gemma", "lfm"):
        n = f"{fam}.f16.{t}.weight"
        cs.append((fam, n, [(n, w, "f16", (o, i))], lambda x, w=w: oracle.qgemv_f16(w.view(np.uint16), x)))
    w8, s8 = _i8(o, i, 0xD1000011)
    for fam in ("llama", "qwen", "gemma"):
        n = f"{fam}.i8.{t}.weight"
        cs.append((fam, n, [(n, w8, "i8", (o, i)), (n + ".qscale", s8, "f16", (o,))],
                   lambda x: np.stack([oracle.matmul_i8_f32(w8, s8.view(np.uint16), r) for r in x])))
    # i4: one scale per row everywhere; four per row for Llama (first scale) and Qwen (groups of in/4)
    w4, s4 = _i4(o, i, 0xD1000021)
    for fam in ("llama", "qwen", "gemma"):
        n = f"{fam}.i4.{t}.weight"
        cs.append((fam, n, [(n, w4, "i4", (o, i)), (n + ".qscale", s4, "f16", (o,))],
                   lambda x: np.stack([oracle.matmul_i4_f32(w4, s4.view(np.uint16), o, i, i, r) for r in x])))
    g = 4  # both shapes' in_dim is a multiple of 4
    w4g, s4g = _i4(o, i, 0xD1000031, groups=g)
    n = f"llama.i4g.{t}.weight"
    cs.append(("llama", n, [(n, w4g, "i4", (o, i)), (n + ".qscale", s4g, "f16", (o * g,))],
               lambda x: np.stack([oracle.matmul_i4_f32(w4g, s4g.view(np.uint16), o, i, i, r) for r in x])))
    n = f"qwen.i4g.{t}.weight"
    cs.append(("qwen", n, [(n, w4g, "i4", (o, i)), (n + ".qscale", s4g, "f16", (o * g,))],
               lambda x: np.stack([oracle.matmul_i4_f32(w4g, s4g.view(np.uint16), o, i, i // g, r) for r in x])))
    w2, s2 = _i2(o, i, 0xD1000041)
    for fam, mode in (("qwen", 0), ("gemma", 1)):
        n = f"{fam}.i2.{t}.weight"
        cs.append((fam, n, [(n, w2, "i2", (o, i)), (n + ".qscale", s2, "f16", (o,))],
                   lambda x, mode=mode: oracle.qgemv_i2(w2, s2.view(np.uint16), x, i, mode)))
    if i % 128 == 0:
        w1 = _q1(o, i, 0xD1000051)
        n = f"qwen.q1.{t}.weight"
        cs.append(("qwen", n, [(n, w1, "q1_0_g128", (o, i))], lambda x: oracle.qgemv_q1_0_g128(w1, x, i)))
    wq, s, b = _u32(o, i, 0xD1000061)
    n = f"lfm.u32.{t}"
    cs.append(("lfm", n + ".weight", [(n + ".weight", wq, "u32", wq.shape), (n + ".scales", s, "f32", s.shape),
                                       (n + ".biases", b, "f32", b.shape)],
               lambda x: oracle.qgemv_q4_affine(wq, s, b, x, i)))
    return cs


@pytest.fixture(scope="module")
def fresh_ops():
    """A context of its own: the weight cache is keyed by tensor name."""
    import torch

    if not torch.cuda.is_available():  # torch's HIP runtime first, as the shared ops fixture does
        pytest.fail("GPU test selected but no HIP device is visible")
    from cellm_amd import HipOps

    o = HipOps(0)
    yield o
    o.close()


@pytest.mark.parametrize("o,i", SHAPES)
def test_every_family_arm_matches_the_oracle(tmp_path, fresh_ops, o, i):
    import torch

    from cellm_amd.cellm_file import CellmFile

    cases = _cases(o, i)
    path = tmp_path / "arms.cellm"
    write_cellm(path, llama_header(1, 64, 1, 1, 64, 64), [tt for c in cases for tt in c[2]])
    x = oracle.gen_normal((M, i), 0xD1000100 + i, 0.0, 1.0).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    with CellmFile(path) as f:
        for fam, name, _, ref in cases:
            print(f"case {fam} {name}", flush=True)
            y = torch.full((M, o), float("nan"), dtype=torch.float32, device="cuda")
            f.linear(fresh_ops, name, fam, xd, y)
            got = y.cpu().numpy()
            want = np.asarray(ref(x), np.float32).reshape(M, o)
            err = float(np.max(np.abs(got - want)) / np.max(np.abs(want)))
            assert err <= 1e-3, (fam, name, err)


def test_family_arms_differ_where_the_reference_does(tmp_path, fresh_ops):
    """Llama's i4 with three scales per row uses only the first; Qwen's uses all three:
    the outputs differ unless the scales are equal.  Qwen's i2 and Gemma's i2 differ
    only in rounding (scale at the end or per element)."""
    import torch

    from cellm_amd.cellm_file import CellmFile

    o, i = 64, 384
    w4, s4 = _i4(o, i, 0xD1000201, groups=3)
    w2, s2 = _i2(o, i, 0xD1000211)
    ts = [("a.i4.weight", w4, "i4", (o, i)), ("a.i4.weight.qscale", s4, "f16", (o * 3,)),
          ("a.i2.weight", w2, "i2", (o, i)), ("a.i2.weight.qscale", s2, "f16", (o,))]
    path = tmp_path / "diff.cellm"
    write_cellm(path, llama_header(1, 64, 1, 1, 64, 64), ts)
    x = torch.from_numpy(oracle.gen_normal((1, i), 0xD1000221, 0.0, 1.0).astype(np.float32)).cuda()
    outs = {}
    with CellmFile(path) as f:
        for fam, name in (("llama", "a.i4.weight"), ("qwen", "a.i4.weight"), ("qwen", "a.i2.weight"),
                          ("gemma", "a.i2.weight")):
            y = torch.empty((1, o), dtype=torch.float32, device="cuda")
            f.linear(fresh_ops, name, fam, x, y)
            outs[(fam, name)] = y.cpu().numpy()[0]
    a, b = outs[("llama", "a.i4.weight")], outs[("qwen", "a.i4.weight")]
    assert np.max(np.abs(a - b)) > 1e-2 * np.max(np.abs(a))
    c, d = outs[("qwen", "a.i2.weight")], outs[("gemma", "a.i2.weight")]
    assert np.max(np.abs(c - d)) <= 1e-4 * np.max(np.abs(c))


def test_refusals_and_cache_reuse(tmp_path, fresh_ops):
    import torch

    from cellm_amd._lib import CellmHipError
    from cellm_amd.cellm_file import CellmFile

    o, i = 16, 128
    w8, s8 = _i8(o, i, 0xD1000301)
    w2, s2 = _i2(o, i, 0xD1000311)
    w4, s4 = _i4(o, i, 0xD1000321, groups=2)
    wq, s, _ = _u32(o, i, 0xD1000331)
    ts = [("r.i8.weight", w8, "i8", (o, i)), ("r.i8.weight.qscale", s8, "f16", (o,)),
          ("r.i2.weight", w2, "i2", (o, i)), ("r.i2.weight.qscale", s2, "f16", (o,)),
          ("r.i4.weight", w4, "i4", (o, i)), ("r.i4.weight.qscale", s4, "f16", (2 * o,)),
          ("r.bf.weight", w8.view(np.uint8).reshape(o // 2, 2 * i), "bf16", (o // 2, i)),
          ("r.flat.weight", w8.reshape(-1), "i8", (o * i,)),
          ("r.u32.weight", wq, "u32", wq.shape), ("r.u32.scales", s, "f32", s.shape)]
    path = tmp_path / "bad.cellm"
    write_cellm(path, llama_header(1, 64, 1, 1, 64, 64), ts)
    x = torch.zeros((1, i), dtype=torch.float32, device="cuda")
    y = torch.empty((1, o), dtype=torch.float32, device="cuda")
    with CellmFile(path) as f:
        def refuse(name, fam, msg, out_dim=o, in_dim=i):
            xx = torch.zeros((1, in_dim), dtype=torch.float32, device="cuda")
            yy = torch.empty((1, out_dim), dtype=torch.float32, device="cuda")
            with pytest.raises(CellmHipError, match=msg):
                f.linear(fresh_ops, name, fam, xx, yy)

        refuse("r.i2.weight", "llama", "unsupported weight dtype for r.i2.weight: i2")
        refuse("r.bf.weight", "qwen", "linear fallback unsupported dtype bf16", out_dim=o // 2)
        refuse("r.bf.weight", "gemma", r"shape mismatch: \[8, 128\] expected \[16,128\]")
        refuse("r.flat.weight", "llama", r"expected 2D, got \[2048\]")
        refuse("r.i4.weight", "gemma", "qscale len mismatch: 32 expected 16")
        refuse("r.missing.weight", "llama", "unknown tensor r.missing.weight")
        refuse("r.missing.weight", "qwen", "linear_f16_out_in: unknown tensor 'r.missing.weight'")
        # u32 without .biases is read as f16 by the LFM runner: o*i/2 bytes are not o*i f16 values
        refuse("r.u32.weight", "lfm", "linear_f16_out_in: weight shape mismatch for r.u32.weight")
        refuse("r.i8.weight", "llama", r"shape mismatch: \[16, 128\] expected \[16,64\]", in_dim=64)

        before = fresh_ops.weight_cache_stats()
        f.linear(fresh_ops, "r.i8.weight", "llama", x, y)
        mid = fresh_ops.weight_cache_stats()
        f.linear(fresh_ops, "r.i8.weight", "gemma", x, y)
        after = fresh_ops.weight_cache_stats()
        assert mid[0] == before[0] + 2 and after == mid  # weight + qscale uploaded once
        torch.cuda.synchronize()
        assert float(y.abs().max()) == 0.0
