"""Decode-step ops on the device (cellm_hip.h: embed, RMSNorm, RoPE, K/V write,
paged GQA attention, residual add, greedy argmax) against the CPU oracle.

- embed, K/V write, add, argmax, RoPE: bit-exact (RoPE angles come from
  cellm_llama_rope_table, the same glibc f32 math the oracle's rope uses).
- RMSNorm: the sum of squares is a tree here and sequential in the reference:
  relative error <= 1e-6.
- attention: softmax with the device expf; tables of up to 512 positions in
  one block per query head, longer ones as split-sequence partials combined
  with rescaling: relative error <= 1e-5 of max|out|.
"""
from __future__ import annotations

import ctypes as C

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


@pytest.fixture(scope="module")
def steplib():
    from cellm_amd import build
    from cellm_amd._lib import load

    load()
    lib = C.CDLL(str(build.STEP_LIB_PATH))
    lib.cellm_llama_rope_table.argtypes = [C.c_float, C.c_int32, C.c_int32, C.c_void_p]
    return lib


def dev(a: np.ndarray):
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).cuda()
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda()
    return torch.from_numpy(a).cuda()


def rope_table(lib, theta, hd, positions):
    t = np.empty((positions, hd // 2, 2), np.float32)
    assert lib.cellm_llama_rope_table(theta, hd, positions, t.ctypes.data) == 0
    return t


def test_embed_i8(ops):
    vocab, hid = 1000, 960
    emb = oracle.gen_i8((vocab, hid), 0xD0000001)
    sc = (oracle.gen_uniform((vocab,), 0xD0000002, 0.5, 1.5) / 127).astype(np.float16).view(np.uint16)
    toks = np.array([3, 999, 1000 + 5, 0], np.uint32)  # token % vocab, as embed_token does
    out = torch.empty((4, hid), dtype=torch.float32, device="cuda")
    ops.encode_embed_i8(dev(toks), dev(emb), dev(sc), out)
    torch.cuda.synchronize()
    ref = np.stack([emb[t % vocab].astype(np.float32) * oracle.f16_bits_to_f32(sc[t % vocab:t % vocab + 1])[0]
                    for t in toks])
    np.testing.assert_array_equal(out.cpu().numpy(), ref)


@pytest.mark.parametrize("hid", [960, 7])
def test_embed_f16_and_i4_bit_exact(ops, hid):
    """embed_token's f16 and i4 branches (llama.rs:687-693, 703-718) against
    the oracle, bit for bit; an odd hidden size for i4 rows of ceil(hid/2)
    bytes; tokens wrap modulo the vocabulary."""
    vocab = 1000
    rng = np.random.default_rng(0xD0000003 + hid)
    ef = rng.standard_normal((vocab, hid)).astype(np.float16)
    e4 = rng.integers(0, 256, (vocab, (hid + 1) // 2)).astype(np.uint8)
    sc = (rng.uniform(0.5, 1.5, vocab) / 7).astype(np.float16).view(np.uint16)
    toks = np.array([3, 999, 1000 + 5, 0], np.uint32)
    out = torch.empty((4, hid), dtype=torch.float32, device="cuda")
    ops.encode_embed_f16(dev(toks), dev(ef.view(np.uint16)), out)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), oracle.embed("f16", toks, ef.view(np.uint16), None, vocab, hid))
    ops.encode_embed_i4(dev(toks), dev(e4), dev(sc), hid, out)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), oracle.embed("i4", toks, e4, sc, vocab, hid))


@pytest.mark.parametrize("wdt", ["f32", "f16"])
@pytest.mark.parametrize("n", [960, 1152, 7])
def test_rms_norm(ops, n, wdt):
    rows = 3
    x = np.stack([oracle.gen_normal((n,), 0xD0000010 + r, 0.0, 2.0) for r in range(rows)]).astype(np.float32)
    w = (1.0 + 0.1 * oracle.lcg_fill(n, 0xD0000020, 1.0)).astype(np.float16)
    wd = w.astype(np.float32) if wdt == "f32" else w
    out = torch.empty((rows, n), dtype=torch.float32, device="cuda")
    ops.encode_rms_norm(dev(x), dev(wd), out, 1e-5)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for r in range(rows):
        ref = oracle.rms_norm(x[r], w.astype(np.float32), 1e-5)
        assert rel_err(got[r], ref) <= 1e-6


@pytest.mark.parametrize("heads,hd", [(15, 64), (5, 64), (8, 128)])
def test_rope_half_bit_exact(ops, steplib, heads, hd):
    positions = np.array([0, 1, 511, 2047], np.int32)
    theta = 100000.0
    table = rope_table(steplib, theta, hd, 2048)
    x = np.stack([oracle.gen_normal((heads * hd,), 0xD0000030 + i, 0.0, 1.0) for i in range(4)]).astype(np.float32)
    xd = dev(x.copy())
    ops.encode_rope_half(xd, heads, hd, dev(positions), dev(table))
    torch.cuda.synchronize()
    got = xd.cpu().numpy()
    for r, p in enumerate(positions):
        ref = oracle.rope_half_(x[r].copy(), heads, hd, int(p), theta)
        np.testing.assert_array_equal(got[r], ref)


@pytest.mark.parametrize("heads,hd", [(15, 64), (4, 256)])
def test_rope_interleaved_bit_exact(ops, steplib, heads, hd):
    """cellm_hip_rope_interleaved_f32 against rope_interleaved_inplace_f32 (cpu_kernels.rs:279-292)
    bit for bit, from the same table as the rotate-half form."""
    positions = np.array([0, 1, 511, 2047], np.int32)
    theta = 10000.0
    table = rope_table(steplib, theta, hd, 2048)
    x = np.stack([oracle.gen_normal((heads * hd,), 0xD0000038 + i, 0.0, 1.0) for i in range(4)]).astype(np.float32)
    xd = dev(x.copy())
    ops.encode_rope_interleaved(xd, heads, hd, dev(positions), dev(table))
    torch.cuda.synchronize()
    got = xd.cpu().numpy()
    for r, p in enumerate(positions):
        np.testing.assert_array_equal(got[r], oracle.rope_interleaved_(x[r].copy(), heads, hd, int(p), theta))


def paged_setup(L, tpb, nkv, hd, rows, blocks_per_row, seed):
    total = rows * blocks_per_row + 3
    kvd = nkv * hd
    n = total * L * tpb * kvd
    k = oracle.gen_normal((n,), seed, 0.0, 1.0).astype(np.float16).view(np.uint16)
    v = oracle.gen_normal((n,), seed + 1, 0.0, 1.0).astype(np.float16).view(np.uint16)
    # interleaved, non-contiguous pages per row
    bt = np.array([[b * rows + r + 3 for b in range(blocks_per_row)] for r in range(rows)], np.uint32)
    return total, k, v, bt


def base_of(bt_row, t, layer, L, tpb, kvd):
    return int(bt_row[t // tpb]) * (L * tpb * kvd) + layer * (tpb * kvd) + (t % tpb) * kvd


def test_kv_write_f16(ops):
    L, tpb, nkv, hd, rows = 4, 16, 5, 64, 3
    kvd = nkv * hd
    total, k0, v0, bt = paged_setup(L, tpb, nkv, hd, rows, 8, 0xD0000040)
    pos = np.array([0, 17, 127], np.int32)
    layer = 2
    kn = np.stack([oracle.gen_normal((kvd,), 0xD0000050 + r, 0.0, 3.0) for r in range(rows)]).astype(np.float32)
    vn = np.stack([oracle.gen_normal((kvd,), 0xD0000060 + r, 0.0, 3.0) for r in range(rows)]).astype(np.float32)
    kd, vd = dev(k0.copy()), dev(v0.copy())
    ops.encode_kv_write(dev(kn), dev(vn), dev(pos), kd, vd, dev(bt), total, L, tpb, layer)
    torch.cuda.synchronize()
    k_ref, v_ref = k0.copy(), v0.copy()
    for r in range(rows):
        b = base_of(bt[r], int(pos[r]), layer, L, tpb, kvd)
        k_ref[b:b + kvd] = kn[r].astype(np.float16).view(np.uint16)  # write_token_f32: f16 RNE
        v_ref[b:b + kvd] = vn[r].astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(kd.cpu().numpy().view(np.uint16), k_ref)
    np.testing.assert_array_equal(vd.cpu().numpy().view(np.uint16), v_ref)


@pytest.mark.parametrize("nh,nkv,hd,blocks,pos", [
    (15, 5, 64, 34, (0, 31, 64, 543)),      # G 3: seq 1, half a chunk, chunk + 1, 9 chunks
    (8, 8, 128, 34, (63, 64, 127, 543)),    # G 1, head_dim 128
    (14, 2, 64, 34, (0, 100, 200, 543)),    # G 7
    (8, 4, 64, 8, (5, 127, 0, 64)),         # G 2, a short table
    (16, 2, 128, 132, (2099, 1024, 1, 700)),  # G 8: 33 chunks, past the combine's preloaded 16
    (15, 5, 64, 64, (1023, 960, 15, 511)),   # G 3, 16 chunks: the largest single-launch table
    (15, 5, 64, 80, (1279, 1024, 3, 640)),   # G 3, 20 chunks: split-sequence launches
    (4, 2, 128, 20, (319, 0, 64, 200)),      # G 2 at head_dim 128: single launch
    # tables of up to 512 positions: one block per query head over the whole sequence
    (14, 2, 64, 32, (511, 300, 0, 255)),    # G 7, 512 positions: two sub-chunks, full
    (8, 8, 128, 16, (255, 128, 17, 0)),     # G 1 at head_dim 128, 256 positions: one sub-chunk
    (16, 2, 128, 32, (511, 256, 257, 3)),   # G 8 at head_dim 128, sub-chunk edges
    (15, 5, 64, 33, (527, 511, 512, 0)),    # 528 positions: back to the chunked kernels
])
def test_attention_gqa_f16kv(ops, nh, nkv, hd, blocks, pos):
    L, tpb, rows = 3, 16, 4
    kvd = nkv * hd
    total, k, v, bt = paged_setup(L, tpb, nkv, hd, rows, blocks, 0xD0000070 + nh)
    pos = np.array(pos, np.int32)
    layer = 1
    q = np.stack([oracle.gen_normal((nh * hd,), 0xD0000080 + r, 0.0, 1.0) for r in range(rows)]).astype(np.float32)
    out = torch.empty((rows, nh * hd), dtype=torch.float32, device="cuda")
    ops.encode_attention(dev(q), dev(k), dev(v), dev(bt), dev(pos), out, nh, nkv, hd, total, L, tpb, layer)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for r in range(rows):
        seq = int(pos[r]) + 1
        bases = np.array([base_of(bt[r], t, layer, L, tpb, kvd) for t in range(seq)], np.uint64)
        ref = oracle.attention_gqa_f16kv(k, v, bases, q[r], nh, nkv, hd)
        assert rel_err(got[r], ref) <= 1e-5, (r, rel_err(got[r], ref))


@pytest.mark.parametrize("tpb,blocks,pos", [
    (8, 64, (511, 300, 7, 0)),      # pages of 8: a wave's 16 positions span two pages
    (12, 42, (503, 255, 12, 11)),   # pages of 12: page edges inside the waves' 16-position groups
    (32, 16, (511, 31, 32, 256)),   # pages of 32: two waves' positions per page
    (64, 8, (511, 64, 63, 400)),
    (16, 16, (255, 16, 15, 0)),     # one sub-chunk
])
def test_attention_per_head_page_sizes(ops, tpb, blocks, pos):
    """The per-query-head kernel (tables of up to 512 positions) at page sizes other than 16
    positions, including pages whose edges fall inside a wave's 16 positions: each position's
    element base comes from its own page entry.  Every row against the oracle."""
    nh, nkv, hd, L, rows = 15, 5, 64, 2, 4
    kvd = nkv * hd
    total, k, v, bt = paged_setup(L, tpb, nkv, hd, rows, blocks, 0xD00000C0 + tpb)
    pos = np.array(pos, np.int32)
    layer = 1
    q = np.stack([oracle.gen_normal((nh * hd,), 0xD00000D0 + r, 0.0, 1.0) for r in range(rows)]).astype(np.float32)
    out = torch.empty((rows, nh * hd), dtype=torch.float32, device="cuda")
    ops.encode_attention(dev(q), dev(k), dev(v), dev(bt), dev(pos), out, nh, nkv, hd, total, L, tpb, layer)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for r in range(rows):
        seq = int(pos[r]) + 1
        bases = np.array([base_of(bt[r], t, layer, L, tpb, kvd) for t in range(seq)], np.uint64)
        ref = oracle.attention_gqa_f16kv(k, v, bases, q[r], nh, nkv, hd)
        assert rel_err(got[r], ref) <= 1e-5, (r, rel_err(got[r], ref))


@pytest.mark.parametrize("nh,nkv,hd,blocks,window,pos", [
    (15, 5, 64, 32, 100, (511, 99, 100, 0)),        # per-head kernel, one sub-chunk group: window edges
    (14, 2, 64, 64, 512, (1023, 600, 511, 513)),    # per-head kernel over 1024 positions, Gemma-3's window
    (8, 2, 128, 80, 512, (1279, 700, 512, 5)),      # chunked one-launch form: window starts inside a chunk
    (8, 4, 64, 80, 64, (1279, 1215, 64, 63)),       # chunked: window start on a chunk edge
    (15, 5, 64, 32, 1, (511, 37, 1, 0)),            # window 1, per-head kernel
    (8, 2, 64, 80, 1, (1279, 640, 63, 64)),         # window 1, chunked form
])
def test_attention_sliding_window(ops, nh, nkv, hd, blocks, window, pos):
    """Sliding-window layers (gemma.rs:747-780): each row attends to positions
    max(0, pos + 1 - window) .. pos, the reference's gather bases from
    seq.saturating_sub(window).  Every row against the oracle over exactly
    those bases; at window 1 the softmax has one term, so every query head's
    output is the current position's V of its kv head (the f16 values, exactly);
    window 0 through the same entry equals the full-attention entry bit for bit."""
    L, tpb, rows, layer = 2, 16, 4, 1
    kvd = nkv * hd
    total, k, v, bt = paged_setup(L, tpb, nkv, hd, rows, blocks, 0xD0000600 + blocks + window)
    pos = np.array(pos, np.int32)
    q = np.stack([oracle.gen_normal((nh * hd,), 0xD0000610 + r, 0.0, 1.0) for r in range(rows)]).astype(np.float32)
    args = (dev(q), dev(k), dev(v), dev(bt), dev(pos))
    out = torch.empty((rows, nh * hd), dtype=torch.float32, device="cuda")
    ops.encode_attention(*args, out, nh, nkv, hd, total, L, tpb, layer, window=window)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for r in range(rows):
        seq = int(pos[r]) + 1
        bases = np.array([base_of(bt[r], t, layer, L, tpb, kvd) for t in range(max(0, seq - window), seq)], np.uint64)
        ref = oracle.attention_gqa_f16kv(k, v, bases, q[r], nh, nkv, hd)
        assert rel_err(got[r], ref) <= 1e-5, (r, rel_err(got[r], ref))
        if window == 1:
            b = base_of(bt[r], seq - 1, layer, L, tpb, kvd)
            vrow = v[b:b + kvd].view(np.float16).astype(np.float32).reshape(nkv, hd)
            np.testing.assert_array_equal(got[r].reshape(nh, hd), vrow[np.arange(nh) // (nh // nkv)])
    full = torch.empty_like(out)
    ops.encode_attention(*args, full, nh, nkv, hd, total, L, tpb, layer)
    ops.encode_attention(*args, out, nh, nkv, hd, total, L, tpb, layer, window=0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), full.cpu().numpy().view(np.uint32))
    from cellm_amd._lib import CellmHipError
    with pytest.raises(CellmHipError, match="bad window"):
        ops.encode_attention(*args, out, nh, nkv, hd, total, L, tpb, layer, window=-1)


def test_attention_sliding_window_two_launch_form(ops):
    """The two-launch form (more than 16384 (row, kv head) groups) with a window
    of 10: rows whose window starts in the first chunk and rows whose window
    starts in the second, against the oracle on sampled rows."""
    nh, nkv, hd, L, tpb, layer, bpr, window = 64, 64, 64, 1, 16, 0, 5, 10
    kvd = nkv * hd
    rows = 257
    total = rows * bpr + 3
    rng = np.random.default_rng(0xD0000700)
    k = rng.standard_normal(total * L * tpb * kvd, dtype=np.float32).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(total * L * tpb * kvd, dtype=np.float32).astype(np.float16).view(np.uint16)
    bt = np.array([[b * rows + r + 3 for b in range(bpr)] + [3] * (33 - bpr) for r in range(rows)], np.uint32)
    pos = (64 + (np.arange(rows) * 7) % 16).astype(np.int32)
    q = rng.standard_normal((rows, nh * hd), dtype=np.float32)
    out = torch.empty((rows, nh * hd), dtype=torch.float32, device="cuda")
    ops.encode_attention(dev(q), dev(k), dev(v), dev(bt), dev(pos), out, nh, nkv, hd, total, L, tpb, layer,
                         window=window)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    starts = set()
    for r in (0, 1, 2, 9, 100, 200, rows - 1):
        seq = int(pos[r]) + 1
        starts.add((seq - window) // 64)
        bases = np.array([base_of(bt[r], t, layer, L, tpb, kvd) for t in range(seq - window, seq)], np.uint64)
        ref = oracle.attention_gqa_f16kv(k, v, bases, q[r], nh, nkv, hd)
        assert rel_err(got[r], ref) <= 1e-5, r
    assert starts == {0, 1}


def test_attention_one_launch_and_two_launch_forms(ops):
    """Up to 16384 (row, kv head) groups run in one launch (the group's last
    chunk block combines through coherent stores/loads and a self-resetting
    counter); more groups take the two-launch form.  257 rows x 64 kv heads
    (16448 groups) run the two-launch form, then the first 256 rows (16384
    groups) the one-launch form, twice.  Every row has 65..80 positions (two
    chunks) in a table of 33 pages (528 positions: tables of up to 512 take
    the one-block-per-head kernel instead).  Sampled rows match the oracle; the rows both forms share are equal
    bit for bit, as are the two one-launch calls."""
    nh, nkv, hd, L, tpb, layer, bpr = 64, 64, 64, 1, 16, 0, 5
    kvd = nkv * hd
    rows = 257
    total = rows * bpr + 3
    rng = np.random.default_rng(0xD0000500)
    k = rng.standard_normal(total * L * tpb * kvd, dtype=np.float32).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(total * L * tpb * kvd, dtype=np.float32).astype(np.float16).view(np.uint16)
    bt = np.array([[b * rows + r + 3 for b in range(bpr)] + [3] * (33 - bpr) for r in range(rows)], np.uint32)
    pos = (64 + (np.arange(rows) * 7) % 16).astype(np.int32)
    q = rng.standard_normal((rows, nh * hd), dtype=np.float32)
    kd, vd, qd = dev(k), dev(v), dev(q)
    outs = []
    for r_used in (rows, rows - 1, rows - 1):
        out = torch.empty((r_used, nh * hd), dtype=torch.float32, device="cuda")
        ops.encode_attention(qd[:r_used].contiguous(), kd, vd, dev(np.ascontiguousarray(bt[:r_used])),
                             dev(np.ascontiguousarray(pos[:r_used])), out, nh, nkv, hd, total, L, tpb, layer)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    for r in (0, 1, 100, 200, rows - 2, rows - 1):
        bases = np.array([base_of(bt[r], t, layer, L, tpb, kvd) for t in range(int(pos[r]) + 1)], np.uint64)
        ref = oracle.attention_gqa_f16kv(k, v, bases, q[r], nh, nkv, hd)
        assert rel_err(outs[0][r], ref) <= 1e-5, r
        if r < rows - 1:
            assert rel_err(outs[1][r], ref) <= 1e-5, r
    np.testing.assert_array_equal(outs[1].view(np.uint32), outs[0][:rows - 1].view(np.uint32))
    np.testing.assert_array_equal(outs[2].view(np.uint32), outs[1].view(np.uint32))


@pytest.mark.parametrize("nh,nkv,hd,attn_scale,cap,qmag", [
    (8, 2, 64, 0.0625, None, 1.0),    # explicit attn_scale (kvcache.rs:752)
    (8, 2, 64, None, 50.0, 40.0),     # soft cap 50 on scores it bends (kvcache.rs:768-770)
    (4, 1, 128, 0.3, 2.0, 1.0),       # both; a cap that bends most scores
])
def test_attention_scale_and_soft_cap(ops, nh, nkv, hd, attn_scale, cap, qmag):
    L, tpb, rows = 2, 16, 3
    kvd = nkv * hd
    total, k, v, bt = paged_setup(L, tpb, nkv, hd, rows, 10, 0xD00000A0 + nh)
    pos = np.array([0, 70, 159], np.int32)
    layer = 1
    q = np.stack([oracle.gen_normal((nh * hd,), 0xD00000B0 + r, 0.0, qmag) for r in range(rows)]).astype(np.float32)
    out = torch.empty((rows, nh * hd), dtype=torch.float32, device="cuda")
    ops.encode_attention(dev(q), dev(k), dev(v), dev(bt), dev(pos), out, nh, nkv, hd, total, L, tpb, layer,
                         attn_scale=attn_scale, soft_cap=cap)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for r in range(rows):
        seq = int(pos[r]) + 1
        bases = np.array([base_of(bt[r], t, layer, L, tpb, kvd) for t in range(seq)], np.uint64)
        ref = oracle.attention_gqa_f16kv(k, v, bases, q[r], nh, nkv, hd, attn_scale=attn_scale, soft_cap=cap)
        assert rel_err(got[r], ref) <= 1e-5, (r, rel_err(got[r], ref))
        if seq > 1:  # the options change the result: the test would see them dropped
            plain = oracle.attention_gqa_f16kv(k, v, bases, q[r], nh, nkv, hd)
            assert rel_err(plain, ref) > 1e-3


def test_attention_rejects_bad_scale_or_cap(ops):
    from cellm_amd._lib import CellmHipError

    z = torch.zeros(64, dtype=torch.float32, device="cuda")
    for kw in ({"attn_scale": -1.0}, {"soft_cap": float("nan")}, {"soft_cap": float("inf")}):
        with pytest.raises(CellmHipError, match="attn_scale and soft_cap"):
            ops.encode_attention(z, z, z, torch.zeros((1, 1), dtype=torch.int32, device="cuda"),
                                 torch.zeros(1, dtype=torch.int32, device="cuda"), z, 1, 1, 64, 1, 1, 16, 0, **kw)


def test_attention_rejects_unsupported_head_dim(ops):
    from cellm_amd._lib import CellmHipError

    z = torch.zeros(64, dtype=torch.float32, device="cuda")
    with pytest.raises(CellmHipError):
        ops.encode_attention(z, z, z, torch.zeros((1, 1), dtype=torch.int32, device="cuda"),
                             torch.zeros(1, dtype=torch.int32, device="cuda"), z, 1, 1, 96, 1, 1, 16, 0)


@pytest.mark.parametrize("n", [49152, 49151, 131072, 151936, 262144, 16385, 1000])
def test_argmax_first_and_non_finite(ops, n):
    """First maximum per row over chunk blocks of 16384 elements combined in one launch: ties inside a
    chunk and across chunks keep the first index; NaN and +-inf count as -inf; an all -inf row
    gives index 0; the maximum in the ragged last chunk; three calls in a row (the row counters
    return to zero) with the same results and values."""
    rows = np.stack([oracle.gen_normal((n,), 0xD0000090 + r, 0.0, 1.0) for r in range(5)]).astype(np.float32)
    rows[1, 100] = rows[1, min(40000, n - 1)] = 50.0   # a tie (across chunks when n > 40000): the first index wins
    rows[2, 7] = np.nan                                 # NaN -> -inf
    rows[2, 9] = np.inf                                 # +inf -> -inf too (not finite)
    rows[3, :] = -np.inf                                # all -inf: index 0
    rows[4, n - 1] = 60.0                               # in the last (ragged) chunk
    rows[4, n - 2] = 60.0                               # ... tied with its neighbour: n - 2 wins
    idx = torch.empty(5, dtype=torch.int32, device="cuda")
    val = torch.empty(5, dtype=torch.float32, device="cuda")
    d = dev(rows)
    for _ in range(3):
        idx.fill_(-7)
        ops.encode_argmax(d, idx, val)
        torch.cuda.synchronize()
        got, gv = idx.cpu().numpy(), val.cpu().numpy()
        for r in range(5):
            z = rows[r].copy()
            z[~np.isfinite(z)] = -np.inf
            assert got[r] == oracle.argmax_first(z), r
            assert gv[r] == z[got[r]], r
        assert got[1] == 100 and got[4] == n - 2


@pytest.mark.parametrize("n", [49152, 49151, 151936, 262144, 4097, 1000])
def test_argmax_keys_first_and_non_finite(ops, n):
    """The packed-key argmax (one 64-bit atomic max per 4096-element chunk) gives the oracle's first
    maximum: ties inside and across chunks keep the first index, NaN and +-inf count as -inf, an
    all -inf row gives index 0, -0 and +0 are equal (the first of them wins), the maximum in the
    ragged last chunk; a second call on the same keys leaves them unchanged."""
    rows = np.stack([oracle.gen_normal((n,), 0xD00000B0 + r, 0.0, 1.0) for r in range(6)]).astype(np.float32)
    rows[1, 100] = rows[1, min(40000, n - 1)] = 50.0
    rows[2, 7] = np.nan
    rows[2, 9] = np.inf
    rows[3, :] = -np.inf
    rows[4, n - 1] = 60.0
    rows[4, n - 2] = 60.0
    rows[5, :] = -np.abs(rows[5, :]) - 1.0
    rows[5, 3] = -0.0
    rows[5, min(5000, n - 1)] = 0.0                    # +0 after -0: equal, index 3 wins
    keys = torch.zeros(6, dtype=torch.int64, device="cuda")
    d = dev(rows)
    from cellm_amd.hipops import argmax_key_index, argmax_key_value
    for call in range(3):
        if call != 2:
            keys.zero_()
        ops.encode_argmax_keys(d, keys)
        torch.cuda.synchronize()
        got = [int(k) & 0xFFFFFFFFFFFFFFFF for k in keys.cpu().numpy()]
        for r in range(6):
            z = rows[r].copy()
            z[~np.isfinite(z)] = -np.inf
            i = argmax_key_index(got[r])
            assert i == oracle.argmax_first(z), (r, i)
            assert argmax_key_value(got[r]) == z[i], r
        assert argmax_key_index(got[1]) == 100 and argmax_key_index(got[4]) == n - 2
        assert argmax_key_index(got[5]) == 3


def test_argmax_keys_refusals(ops):
    """Keys that are not 8-byte aligned and empty rows are refused before any launch."""
    from cellm_amd._lib import CellmHipError
    d = torch.zeros((2, 64), dtype=torch.float32, device="cuda")
    k = torch.zeros(3, dtype=torch.int64, device="cuda")
    rc = ops._lib.cellm_hip_argmax_f32_keys(ops._h, C.c_void_p(d.data_ptr()), 2, 64, C.c_void_p(k.data_ptr() + 4),
                                            None)
    assert rc != 0
    with pytest.raises(CellmHipError):
        ops.encode_argmax_keys(torch.zeros((2, 0), dtype=torch.float32, device="cuda"), k[:2])


def test_add_inplace(ops):
    a = oracle.gen_normal((5000,), 0xD00000A0, 0.0, 1.0).astype(np.float32)
    b = oracle.gen_normal((5000,), 0xD00000A1, 0.0, 1.0).astype(np.float32)
    ad = dev(a.copy())
    ops.encode_add_inplace(ad, dev(b))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ad.cpu().numpy(), a + b)


@pytest.mark.parametrize("wdt", ["f32", "f16"])
@pytest.mark.parametrize("n", [960, 2048, 2049, 5])
def test_add_rms_norm(ops, wdt, n):
    """x += y, then rms_norm(x): x is exactly a + b; out is what add followed by
    rms_norm gives (the same kernel arithmetic), within 1e-6 of the oracle.
    n 2048 is the largest row kept in registers, 2049 takes the loop."""
    rows = 4
    a = np.stack([oracle.gen_normal((n,), 0xD00000B0 + r, 0.0, 2.0) for r in range(rows)]).astype(np.float32)
    b = np.stack([oracle.gen_normal((n,), 0xD00000C0 + r, 0.0, 1.0) for r in range(rows)]).astype(np.float32)
    w = (1.0 + 0.1 * oracle.lcg_fill(n, 0xD00000D0, 1.0)).astype(np.float16)
    wd = dev(w.astype(np.float32) if wdt == "f32" else w)
    xd = dev(a.copy())
    out = torch.empty((rows, n), dtype=torch.float32, device="cuda")
    ops.encode_add_rms_norm(xd, dev(b), wd, out, 1e-5)
    x2 = dev(a.copy())
    ops.encode_add_inplace(x2, dev(b))
    out2 = torch.empty_like(out)
    ops.encode_rms_norm(x2, wd, out2, 1e-5)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(xd.cpu().numpy(), a + b)
    np.testing.assert_array_equal(out.cpu().numpy(), out2.cpu().numpy())
    got = out.cpu().numpy()
    for r in range(rows):
        assert rel_err(got[r], oracle.rms_norm(a[r] + b[r], w.astype(np.float32), 1e-5)) <= 1e-6


@pytest.mark.parametrize("interleaved", [False, True])
@pytest.mark.parametrize("nh,nkv,hd", [(15, 5, 64), (16, 2, 128)])
def test_rope_kv_write_matches_rope_then_write(ops, steplib, nh, nkv, hd, interleaved):
    """One launch = rope on q, rope on k, then the K/V write: q and k bit-exact
    against the oracle's RoPE (rotate-half, or interleaved after
    cellm_hip_set_rope_interleaved), the cache rows bit-exact against f16(k), f16(v),
    every other cache element untouched; a negative position writes nothing."""
    L, tpb, rows, layer, theta = 3, 16, 4, 1, 10000.0
    kvd = nkv * hd
    total, k0, v0, bt = paged_setup(L, tpb, nkv, hd, rows, 8, 0xD00000E0 + nh)
    pos = np.array([0, 17, 127, -1], np.int32)
    table = rope_table(steplib, theta, hd, 8 * tpb)
    q = np.stack([oracle.gen_normal((nh * hd,), 0xD00000F0 + r, 0.0, 1.0) for r in range(rows)]).astype(np.float32)
    k = np.stack([oracle.gen_normal((kvd,), 0xD0000100 + r, 0.0, 1.0) for r in range(rows)]).astype(np.float32)
    v = np.stack([oracle.gen_normal((kvd,), 0xD0000110 + r, 0.0, 1.0) for r in range(rows)]).astype(np.float32)
    qd, kd, vd = dev(q.copy()), dev(k.copy()), dev(v.copy())
    kc, vc = dev(k0.copy()), dev(v0.copy())
    ops.set_rope_interleaved(interleaved)
    try:
        ops.encode_rope_kv_write(qd, kd, vd, nh, nkv, hd, dev(pos), dev(table), kc, vc, dev(bt), total, L, tpb, layer)
        torch.cuda.synchronize()
    finally:
        ops.set_rope_interleaved(False)
    rope = oracle.rope_interleaved_ if interleaved else oracle.rope_half_
    gq, gk = qd.cpu().numpy(), kd.cpu().numpy()
    k_ref, v_ref = k0.copy(), v0.copy()
    for r in range(rows):
        p = max(int(pos[r]), 0)
        np.testing.assert_array_equal(gq[r], rope(q[r].copy(), nh, hd, p, theta))
        kr = rope(k[r].copy(), nkv, hd, p, theta)
        np.testing.assert_array_equal(gk[r], kr)
        if pos[r] >= 0:
            b = base_of(bt[r], int(pos[r]), layer, L, tpb, kvd)
            k_ref[b:b + kvd] = kr.astype(np.float16).view(np.uint16)
            v_ref[b:b + kvd] = v[r].astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(kc.cpu().numpy().view(np.uint16), k_ref)
    np.testing.assert_array_equal(vc.cpu().numpy().view(np.uint16), v_ref)


def _i8_layer(out_dims, k, seed):
    ws, ss = [], []
    for j, o in enumerate(out_dims):
        ws.append(oracle.gen_i8((o, k), seed + 4 * j))
        ss.append((oracle.gen_uniform((o,), seed + 4 * j + 1, 0.5, 1.5) / (73.3 * np.sqrt(k))).astype(np.float16))
    return ws, ss


@pytest.mark.parametrize("rows,with_y,interleaved", [(4, True, False), (1, True, False), (3, False, False),
                                                    (4, True, True)])
def test_decode_qkv_matches_separate_ops(ops, steplib, rows, with_y, interleaved):
    """cellm_hip_decode_qkv_rope_kv against add_rms_norm + three int8 GEMVs +
    rope_kv_write, both with the context's RoPE layout: the residual exactly, q
    within 1e-5 (the GEMV sums its row in another order), the written K/V rows
    within f16 rounding, no other cache element touched."""
    ops.set_rope_interleaved(interleaved)
    try:
        _decode_qkv_case(ops, steplib, rows, with_y)
    finally:
        ops.set_rope_interleaved(False)


def test_decode_qkv_negative_position(ops, steplib):
    """A session at position -1 in the fused int8 QKV launch: its q as the separate ops give it, no
    K/V element written for it (the page base the epilogue reads early is -1)."""
    _decode_qkv_case(ops, steplib, 4, True, positions=(127, -1, 64, 17))


def _decode_qkv_case(ops, steplib, rows, with_y, positions=(127, 0, 64, 17)):
    H, nh, nkv, hd, L, tpb, layer = 960, 15, 5, 64, 3, 16, 2
    kvd = nkv * hd
    total, k0, v0, bt = paged_setup(L, tpb, nkv, hd, rows, 8, 0xD0000200)
    pos = np.array(positions[:rows], np.int32)
    table = rope_table(steplib, 100000.0, hd, 8 * tpb)
    xp = np.stack([oracle.gen_normal((H,), 0xD0000210 + r, 0.0, 1.0) for r in range(rows)]).astype(np.float32)
    y = np.stack([oracle.gen_normal((H,), 0xD0000220 + r, 0.0, 0.5) for r in range(rows)]).astype(np.float32)
    nw = (1.0 + 0.1 * oracle.lcg_fill(H, 0xD0000230, 1.0)).astype(np.float32)
    (wq, wk, wv), (sq, sk, sv) = _i8_layer([nh * hd, kvd, kvd], H, 0xD0000240)
    d = [dev(a) for a in (wq, sq.view(np.uint16), wk, sk.view(np.uint16), wv, sv.view(np.uint16))]
    d = [t.view(torch.float16) if t.dtype == torch.int16 else t for t in d]
    # separate ops
    x_sep = dev(xp.copy())
    xn = torch.empty((rows, H), dtype=torch.float32, device="cuda")
    if with_y:
        ops.encode_add_rms_norm(x_sep, dev(y), dev(nw), xn, 1e-5)
    else:
        ops.encode_rms_norm(x_sep, dev(nw), xn, 1e-5)
    q = torch.empty((rows, nh * hd), dtype=torch.float32, device="cuda")
    k = torch.empty((rows, kvd), dtype=torch.float32, device="cuda")
    v = torch.empty((rows, kvd), dtype=torch.float32, device="cuda")
    ops.encode_qgemv_i8(d[0], d[1], xn, q)
    ops.encode_qgemv_i8(d[2], d[3], xn, k)
    ops.encode_qgemv_i8(d[4], d[5], xn, v)
    kc1, vc1 = dev(k0.copy()), dev(v0.copy())
    ops.encode_rope_kv_write(q, k, v, nh, nkv, hd, dev(pos), dev(table), kc1, vc1, dev(bt), total, L, tpb, layer)
    # fused
    x_out = torch.full((rows, H), np.nan, dtype=torch.float32, device="cuda")
    q2 = torch.empty_like(q)
    kc2, vc2 = dev(k0.copy()), dev(v0.copy())
    ops.encode_decode_qkv(dev(xp), dev(y) if with_y else None, x_out, dev(nw), 1e-5, d[0], d[1], d[2], d[3], d[4],
                          d[5], nh, nkv, hd, dev(pos), dev(table), q2, kc2, vc2, dev(bt), total, L, tpb, layer)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(x_out.cpu().numpy(), x_sep.cpu().numpy())
    assert rel_err(q2.cpu().numpy(), q.cpu().numpy()) <= 1e-5
    for got, ref, init in ((kc2, kc1, k0), (vc2, vc1, v0)):
        g = got.cpu().numpy().view(np.uint16)
        r = ref.cpu().numpy().view(np.uint16)
        changed = r != init
        np.testing.assert_array_equal(g[~changed], init[~changed])
        gf, rf = oracle.f16_bits_to_f32(g[changed]), oracle.f16_bits_to_f32(r[changed])
        assert np.max(np.abs(gf - rf)) <= 2e-3 * np.max(np.abs(rf))


@pytest.mark.parametrize("rows", [4, 2, 1])
def test_decode_gate_up_matches_separate_ops(ops, rows):
    H, N = 960, 2560
    xp = np.stack([oracle.gen_normal((H,), 0xD0000300 + r, 0.0, 1.0) for r in range(rows)]).astype(np.float32)
    y = np.stack([oracle.gen_normal((H,), 0xD0000310 + r, 0.0, 0.5) for r in range(rows)]).astype(np.float32)
    nw = (1.0 + 0.1 * oracle.lcg_fill(H, 0xD0000320, 1.0)).astype(np.float32)
    (wg, wu), (sg, su) = _i8_layer([N, N], H, 0xD0000330)
    wgd, wud = dev(wg), dev(wu)
    sgd, sud = dev(sg.view(np.uint16)).view(torch.float16), dev(su.view(np.uint16)).view(torch.float16)
    x_sep = dev(xp.copy())
    xn = torch.empty((rows, H), dtype=torch.float32, device="cuda")
    ops.encode_add_rms_norm(x_sep, dev(y), dev(nw), xn, 1e-5)
    h = torch.empty((rows, N), dtype=torch.float32, device="cuda")
    ops.encode_gate_up_silu_i8(wgd, sgd, wud, sud, xn, h)
    x_out = torch.empty((rows, H), dtype=torch.float32, device="cuda")
    h2 = torch.empty_like(h)
    ops.encode_decode_gate_up(dev(xp), dev(y), x_out, dev(nw), 1e-5, wgd, sgd, wud, sud, h2)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(x_out.cpu().numpy(), x_sep.cpu().numpy())
    assert rel_err(h2.cpu().numpy(), h.cpu().numpy()) <= 1e-5


def _q4_mats(out_dims, k, seed, group=64):
    """MLX q4 affine matrices with f32 group scales/biases (the u32 runners' layout)."""
    ws, ss, bs = [], [], []
    for j, n in enumerate(out_dims):
        ws.append(oracle.gen_q4_words((n, k // 8), seed + 3 * j))
        ss.append(oracle.gen_normal((n, k // group), seed + 3 * j + 1, 0.02, 0.005, positive_only=True))
        bs.append(oracle.gen_normal((n, k // group), seed + 3 * j + 2, 0.0, 0.05))
    return ws, ss, bs


# hidden 896: Qwen2.5-0.5B (28 chunks per row, teams of 32 lanes); 256 (teams of 16);
# 1536 (48 chunks, teams of 64, two float4 groups per thread in the prologue);
# 2560 (80 chunks: two per lane, four float4 groups per thread)
@pytest.mark.parametrize("H,nh,nkv,hd,rows,with_y,interleaved,bias", [
    (896, 14, 2, 64, 4, True, False, True),
    (896, 14, 2, 64, 1, False, False, True),
    (896, 14, 2, 64, 3, True, True, False),
    (256, 4, 2, 64, 2, True, False, True),
    (1536, 12, 2, 128, 4, True, False, True),
    (2560, 20, 4, 128, 4, True, False, False),
    (2560, 20, 4, 128, 1, True, True, True),
])
def test_decode_q4_qkv_matches_separate_ops(ops, steplib, H, nh, nkv, hd, rows, with_y, interleaved, bias):
    """cellm_hip_decode_q4_affine_qkv_rope_kv against add_rms_norm + the q4 QKV
    GEMV (f32 x) + rope_kv_write, and its q against the oracle (RMSNorm, the q4
    affine GEMV, the projection bias and rotate-half/interleaved RoPE): the
    residual exactly, q within 1e-5, written K/V within f16 rounding, no other
    cache element touched."""
    ops.set_rope_interleaved(interleaved)
    try:
        _decode_q4_qkv_case(ops, steplib, H, nh, nkv, hd, rows, with_y, interleaved, bias)
    finally:
        ops.set_rope_interleaved(False)


def _decode_q4_qkv_case(ops, steplib, H, nh, nkv, hd, rows, with_y, interleaved, bias):
    L, tpb, layer, theta = 3, 16, 1, 1000000.0
    kvd = nkv * hd
    total, k0, v0, bt = paged_setup(L, tpb, nkv, hd, rows, 8, 0xD0000500)
    pos = np.array([127, 0, 64, 17][:rows], np.int32)
    table = rope_table(steplib, theta, hd, 8 * tpb)
    xp = np.stack([oracle.gen_normal((H,), 0xD0000510 + r, 0.0, 1.0) for r in range(rows)]).astype(np.float32)
    y = np.stack([oracle.gen_normal((H,), 0xD0000520 + r, 0.0, 0.5) for r in range(rows)]).astype(np.float32)
    nw = (1.0 + 0.1 * oracle.lcg_fill(H, 0xD0000530, 1.0)).astype(np.float32)
    (wq, wk, wv), (sq, sk, sv), (bq, bk, bv) = _q4_mats([nh * hd, kvd, kvd], H, 0xD0000540)
    pb = [oracle.gen_normal((n,), 0xD0000550 + j, 0.0, 0.3).astype(np.float32) if bias else None
          for j, n in enumerate((nh * hd, kvd, kvd))]
    d = [dev(a) for a in (wq, sq, bq, wk, sk, bk, wv, sv, bv)]
    dpb = [dev(b) if b is not None else None for b in pb]
    # separate ops
    x_sep = dev(xp.copy())
    xn = torch.empty((rows, H), dtype=torch.float32, device="cuda")
    if with_y:
        ops.encode_add_rms_norm(x_sep, dev(y), dev(nw), xn, 1e-6)
    else:
        ops.encode_rms_norm(x_sep, dev(nw), xn, 1e-6)
    q = torch.empty((rows, nh * hd), dtype=torch.float32, device="cuda")
    k = torch.empty((rows, kvd), dtype=torch.float32, device="cuda")
    v = torch.empty((rows, kvd), dtype=torch.float32, device="cuda")
    ops.encode_qkv_q4_affine(*d, xn, q, k, v, biasq=dpb[0], biask=dpb[1], biasv=dpb[2])
    kc1, vc1 = dev(k0.copy()), dev(v0.copy())
    ops.encode_rope_kv_write(q, k, v, nh, nkv, hd, dev(pos), dev(table), kc1, vc1, dev(bt), total, L, tpb, layer)
    # fused
    x_out = torch.full((rows, H), np.nan, dtype=torch.float32, device="cuda")
    q2 = torch.full_like(q, np.nan)
    kc2, vc2 = dev(k0.copy()), dev(v0.copy())
    ops.encode_decode_q4_qkv(dev(xp), dev(y) if with_y else None, x_out, dev(nw), 1e-6, d[0], d[1], d[2], dpb[0],
                             d[3], d[4], d[5], dpb[1], d[6], d[7], d[8], dpb[2], 64, nh, nkv, hd, dev(pos),
                             dev(table), q2, kc2, vc2, dev(bt), total, L, tpb, layer)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(x_out.cpu().numpy(), x_sep.cpu().numpy())
    assert rel_err(q2.cpu().numpy(), q.cpu().numpy()) <= 1e-5
    # q against the oracle: x_prev + y, RMSNorm, the affine GEMV in the reference order, bias, RoPE
    xr = xp + y if with_y else xp
    q_ref = np.empty((rows, nh * hd), np.float32)
    for r in range(rows):
        xn_r = oracle.rms_norm(xr[r], nw, 1e-6)
        qr = oracle.qgemv_q4_affine(wq, sq, bq, xn_r, H)[0]
        if bias:
            qr = (qr + pb[0]).astype(np.float32)
        qr = np.ascontiguousarray(qr)
        (oracle.rope_interleaved_ if interleaved else oracle.rope_half_)(qr, nh, hd, int(pos[r]), theta)
        q_ref[r] = qr
    assert rel_err(q2.cpu().numpy(), q_ref) <= 2e-5
    for got, ref, init in ((kc2, kc1, k0), (vc2, vc1, v0)):
        g = got.cpu().numpy().view(np.uint16)
        r = ref.cpu().numpy().view(np.uint16)
        changed = r != init
        assert changed.sum() > 0
        np.testing.assert_array_equal(g[~changed], init[~changed])
        gf, rf = oracle.f16_bits_to_f32(g[changed]), oracle.f16_bits_to_f32(r[changed])
        assert np.max(np.abs(gf - rf)) <= 2e-3 * np.max(np.abs(rf))


@pytest.mark.parametrize("H,N,rows,with_y", [(896, 4864, 4, True), (896, 4864, 1, True), (896, 4864, 2, False),
                                             (256, 704, 3, True), (1536, 8960, 4, True), (2560, 1000, 4, True)])
def test_decode_q4_gate_up_matches_separate_ops(ops, H, N, rows, with_y):
    """cellm_hip_decode_q4_affine_gate_up_silu against add_rms_norm + the q4
    gate/up+SiLU GEMV (f32 x), and h against the oracle (RMSNorm, two q4 affine
    GEMVs, silu * up): the residual exactly, h within 1e-5 / 2e-5."""
    xp = np.stack([oracle.gen_normal((H,), 0xD0000600 + r, 0.0, 1.0) for r in range(rows)]).astype(np.float32)
    y = np.stack([oracle.gen_normal((H,), 0xD0000610 + r, 0.0, 0.5) for r in range(rows)]).astype(np.float32)
    nw = (1.0 + 0.1 * oracle.lcg_fill(H, 0xD0000620, 1.0)).astype(np.float32)
    (wg, wu), (sg, su), (bg, bu) = _q4_mats([N, N], H, 0xD0000630)
    d = [dev(a) for a in (wg, sg, bg, wu, su, bu)]
    x_sep = dev(xp.copy())
    xn = torch.empty((rows, H), dtype=torch.float32, device="cuda")
    if with_y:
        ops.encode_add_rms_norm(x_sep, dev(y), dev(nw), xn, 1e-6)
    else:
        ops.encode_rms_norm(x_sep, dev(nw), xn, 1e-6)
    h = torch.empty((rows, N), dtype=torch.float32, device="cuda")
    ops.encode_gate_up_silu_q4_affine(*d, xn, h)
    x_out = torch.full((rows, H), np.nan, dtype=torch.float32, device="cuda")
    h2 = torch.full_like(h, np.nan)
    ops.encode_decode_q4_gate_up(dev(xp), dev(y) if with_y else None, x_out, dev(nw), 1e-6, *d, 64, h2)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(x_out.cpu().numpy(), x_sep.cpu().numpy())
    assert rel_err(h2.cpu().numpy(), h.cpu().numpy()) <= 1e-5
    xr = xp + y if with_y else xp
    xn_ref = np.stack([oracle.rms_norm(xr[r], nw, 1e-6) for r in range(rows)])
    g = oracle.qgemv_q4_affine(wg, sg, bg, xn_ref, H)
    u = oracle.qgemv_q4_affine(wu, su, bu, xn_ref, H)
    h_ref = oracle.silu_mul_(np.ascontiguousarray(g), u)
    assert rel_err(h2.cpu().numpy(), h_ref) <= 2e-5


def test_decode_q4_fused_rejects_unsupported(ops):
    from cellm_amd._lib import CellmHipError

    H, N = 896, 64
    x = torch.zeros((1, H), dtype=torch.float32, device="cuda")
    nw = torch.ones(H, dtype=torch.float32, device="cuda")
    w = torch.zeros((N, H // 8), dtype=torch.int32, device="cuda")
    s = torch.ones((N, H // 64), dtype=torch.float32, device="cuda")
    h = torch.zeros((1, N), dtype=torch.float32, device="cuda")
    with pytest.raises(CellmHipError, match="alias"):
        ops.encode_decode_q4_gate_up(x, None, x, nw, 1e-5, w, s, s, w, s, s, 64, h)
    with pytest.raises(CellmHipError, match="f32"):
        ops.encode_decode_q4_gate_up(x, None, x.clone(), nw, 1e-5, w, s.half(), s.half(), w, s.half(), s.half(), 64, h)
    with pytest.raises(CellmHipError, match="power-of-two"):
        ops.encode_decode_q4_gate_up(x, None, x.clone(), nw, 1e-5, w, s, s, w, s, s, 96, h)
    xb = torch.zeros((1, 4128), dtype=torch.float32, device="cuda")
    wb = torch.zeros((N, 4128 // 8), dtype=torch.int32, device="cuda")
    sb = torch.ones((N, 4128 // 32), dtype=torch.float32, device="cuda")
    with pytest.raises(CellmHipError, match="4096"):
        ops.encode_decode_q4_gate_up(xb, None, xb.clone(), torch.ones(4128, dtype=torch.float32, device="cuda"), 1e-5,
                                     wb, sb, sb, wb, sb, sb, 32, h)


def test_decode_fused_rejects_aliasing_and_unsupported(ops):
    from cellm_amd._lib import CellmHipError

    H = 960
    x = torch.zeros((1, H), dtype=torch.float32, device="cuda")
    nw = torch.ones(H, dtype=torch.float32, device="cuda")
    w = torch.zeros((64, H), dtype=torch.int8, device="cuda")
    s = torch.ones(64, dtype=torch.float16, device="cuda")
    h = torch.zeros((1, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(CellmHipError, match="alias"):
        ops.encode_decode_gate_up(x, None, x, nw, 1e-5, w, s, w, s, h)
    xb = torch.zeros((1, 5000), dtype=torch.float32, device="cuda")
    with pytest.raises(CellmHipError, match="4096"):
        ops.encode_decode_gate_up(xb, None, xb.clone(), torch.ones(5000, dtype=torch.float32, device="cuda"), 1e-5,
                                  torch.zeros((64, 5000), dtype=torch.int8, device="cuda"), s,
                                  torch.zeros((64, 5000), dtype=torch.int8, device="cuda"), s, h)


def test_attention_workspace_growth():
    """A fresh context whose attention workspace grows through 1, 2, 3 and 4
    rows (a grow frees and reallocates, possibly at the same address) gives
    correct results at every size, twice."""
    from cellm_amd import HipOps

    nh, nkv, hd, L, tpb, layer = 15, 5, 64, 2, 16, 1
    kvd = nkv * hd
    total, k, v, bt = paged_setup(L, tpb, nkv, hd, 4, 34, 0xD0000400)
    o = HipOps(0)
    try:
        for rep in range(2):
            for rows in (1, 2, 3, 4):
                pos = np.array([543, 0, 64, 300][:rows][::-1], np.int32)
                q = np.stack([oracle.gen_normal((nh * hd,), 0xD0000410 + r, 0.0, 1.0) for r in range(rows)])
                q = q.astype(np.float32)
                out = torch.empty((rows, nh * hd), dtype=torch.float32, device="cuda")
                o.encode_attention(dev(q), dev(k), dev(v), dev(np.ascontiguousarray(bt[:rows])), dev(pos), out, nh,
                                   nkv, hd, total, L, tpb, layer)
                torch.cuda.synchronize()
                got = out.cpu().numpy()
                for r in range(rows):
                    bases = np.array([base_of(bt[r], t, layer, L, tpb, kvd) for t in range(int(pos[r]) + 1)],
                                     np.uint64)
                    ref = oracle.attention_gqa_f16kv(k, v, bases, q[r], nh, nkv, hd)
                    assert rel_err(got[r], ref) <= 1e-5, (rep, rows, r)
    finally:
        o.close()
