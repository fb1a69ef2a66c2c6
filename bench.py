#!/usr/bin/env python3
"""Benchmark of the quantized-weight matmul path on one MI355X.

A step is one decode pass (batch 1) over the five Qwen2.5-0.5B-shape MLX 4-bit
affine projections of BASELINE.json configs[1]: 896->1152 (fused QKV),
896->896, 896->9728 (gate+up), 4864->896, 896->151936 (lm_head), fp16 x,
fp16 group-64 scales/biases.  Every step reads a different copy of the weights
(copies total > 512 MB, twice the 256 MB Infinity Cache), so weights stream
from HBM.  `value` = algorithmic bytes of the step / step time (GB/s).

A step is one cellm_hip_qgemv_batch call (the five projections enqueued from C),
so the host's per-call cost does not gate the small projections.  Extra keys
report the other BASELINE.json configs (int8 GEMV, Gemma batched decode, M=512
prefill qGEMM) and the roofline of the dominant kernel (the lm_head GEMV),
whose per-launch duration is measured with HIP events on the launch stream
around batch calls of 100 launches (median of three blocks, after 20 ms of
the same calls).
cpu_baseline times the CPU oracle (a restatement of the reference CPU kernels)
on a bounded sample of the same workload on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, published
BASELINE_METRIC = "int4/int8 qGEMV µs & HBM GB/s (% peak); M=512 qGEMM TFLOP/s (% MFMA)"
WARM_MIN_S = 0.05              # least warm-up time before the timed steps (see main)
CACHE_BYTES = 512 * 2**20      # every timed loop rotates through more weight bytes than this (2x the MALL)

QWEN_SHAPES = [("qkv", 896, 1152), ("o", 896, 896), ("gate_up", 896, 9728), ("down", 4864, 896),
               ("lm_head", 896, 151936)]


def progress(msg: str) -> None:
    """One line per finished phase on stderr (the JSON line stays alone on stdout)."""
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def q4_bytes(m: int, n: int, k: int) -> int:
    """Algorithmic bytes of one q4-affine g64 call: packed W + f16 S,B + f16 x + f32 y."""
    return n * k // 2 + 4 * n * ((k + 63) // 64) + 2 * m * k + 4 * m * n


def i8_bytes(m: int, n: int, k: int, x_bytes: int, s_bytes: int = 4) -> int:
    return n * k + s_bytes * n + x_bytes * m * k + 4 * m * n


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--eager-decode-step", action="store_true",
                    help="time the configs[4] decode step with eager launches only (the same kernels without "
                         "HIP graph replay; for runs under rocprofv3, whose kernel tracer fails on graph launches)")
    ap.add_argument("--no-extra", action="store_true", help="skip the extra configs")
    ap.add_argument("--pmc-sample", nargs="?", const="lm_head_q4", default=None,
                    choices=["lm_head_q4", "lm_head_i8_m1", "lm_head_i8_m64", "qgemm_896x4864", "qgemm_4864x896",
                             "i4_6912x1152", "decode_layer_4", "decode_layer_q4_4",
                             "q4_gate_up_silu_1152x6912", "q4_down_6912x1152_m1", "q4_down_6912x1152_m4",
                             "q4_down_6912x1152_m16", "q4_down_6912x1152_m64", "q4_gate_up_1152x13824_m4",
                             "q4_gate_up_1152x13824_m16", "q4_gate_up_1152x13824_m64"],
                    help="run only a 256 MiB device copy (counter calibration) and 20 launches of one kernel "
                         "(default: the q4 lm_head GEMV), for rocprofv3 --pmc passes")
    return ap.parse_args()


def pmc_sample(torch, ops, stream, gen, which: str):
    """Workload of a counter pass: the plain copy whose counters calibrate
    FETCH_SIZE / WRITE_SIZE against known bytes, then 20 launches of one
    kernel (weights on rotating copies for the GEMVs)."""
    nbytes = 256 * 2**20
    src = torch.randn(nbytes // 4, device="cuda", generator=gen)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    info = {"copy_bytes_read": nbytes, "copy_bytes_written": nbytes, "copy_launches": 3, "workload": which,
            "launches": 20}
    if which == "lm_head_q4":
        k, n, copies = 896, 151936, 8
        ws = [Q4Weights(torch, n, k, gen) for _ in range(copies)]
        x = torch.randn((1, k), device="cuda", generator=gen).to(torch.float16)
        y = torch.empty((1, n), dtype=torch.float32, device="cuda")
        arr = op_array([ops.qgemv_op_q4_affine(ws[i % copies].wq, ws[i % copies].s, ws[i % copies].b, x, y)
                        for i in range(20)])
        ops.encode_qgemv_batch(arr, stream=stream.cuda_stream)
        info.update({"kernel": "qgemv_q4_flat_kernel (q4 affine 896->151936, M=1)",
                     "algorithmic_bytes": q4_bytes(1, n, k)})
    elif which in ("lm_head_i8_m1", "lm_head_i8_m64"):
        k, n, m, copies = 1152, 262144, (1 if which == "lm_head_i8_m1" else 64), 2
        w = torch.randint(-127, 128, (copies, n, k), dtype=torch.int8, device="cuda", generator=gen)
        sc = torch.rand((n,), device="cuda", generator=gen) * 0.019 + 0.001
        x = torch.randn((m, k), device="cuda", generator=gen).to(torch.float16)
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        arr = op_array([ops.qgemv_op_i8(w[i % copies], sc, x, y) for i in range(20)])
        ops.encode_qgemv_batch(arr, stream=stream.cuda_stream)
        info.update({"kernel": f"{'qgemv_i8_kernel' if m == 1 else 'qgemv_mfma_kernel'} (int8 1152->262144, M={m})",
                     "algorithmic_bytes": i8_bytes(m, n, k, 2)})
    elif which == "decode_layer_4":
        # one configs[4] layer for 4 sessions at context 512, eager launches (no runner, no graph): the
        # fused QKV (+ RMSNorm, RoPE, K/V write), attention, o_proj, fused gate/up, down_proj, 20 times
        H, NH, NKV, HD, I, L, TPB, CTX, R = 960, 15, 5, 64, 2560, 1, 16, 512, 4
        kvd, blocks = NKV * HD, CTX // TPB
        w8 = lambda o, i: torch.randint(-127, 128, (o, i), dtype=torch.int8, device="cuda", generator=gen)
        sc = lambda o: (torch.rand((o,), device="cuda", generator=gen) * 0.004 + 0.001).to(torch.float16)
        wq, wk, wv, wo, wg, wu, wd = w8(H, H), w8(kvd, H), w8(kvd, H), w8(H, H), w8(I, H), w8(I, H), w8(H, I)
        sq, sk, sv, so, sg, su, sd = sc(H), sc(kvd), sc(kvd), sc(H), sc(I), sc(I), sc(H)
        norm = torch.ones(H, dtype=torch.float32, device="cuda")
        total = R * blocks
        kc = torch.randn(total * L * TPB * kvd, device="cuda", generator=gen).to(torch.float16)
        vc = torch.randn(total * L * TPB * kvd, device="cuda", generator=gen).to(torch.float16)
        bt = torch.tensor([[b * R + s for b in range(blocks)] for s in range(R)], dtype=torch.int32, device="cuda")
        pos = torch.full((R,), CTX - 1, dtype=torch.int32, device="cuda")
        ang = torch.arange(CTX, device="cuda").float()[:, None] * torch.pow(
            100000.0, -torch.arange(0, HD, 2, device="cuda").float() / HD)[None, :]
        cs = torch.stack([torch.cos(ang), torch.sin(ang)], dim=-1).contiguous()
        xa, xb = torch.randn((R, H), device="cuda", generator=gen), torch.zeros((R, H), device="cuda")
        y = torch.zeros((R, H), device="cuda")
        q = torch.empty((R, NH * HD), device="cuda")
        att = torch.empty((R, NH * HD), device="cuda")
        h = torch.empty((R, I), device="cuda")
        sp = stream.cuda_stream
        for _ in range(20):
            ops.encode_decode_qkv(xa, y, xb, norm, 1e-5, wq, sq, wk, sk, wv, sv, NH, NKV, HD, pos, cs, q, kc, vc, bt,
                                  total, L, TPB, 0, stream=sp)
            ops.encode_attention(q, kc, vc, bt, pos, att, NH, NKV, HD, total, L, TPB, 0, stream=sp)
            ops.encode_qgemv_i8(wo, so, att, y, stream=sp)
            ops.encode_decode_gate_up(xb, y, xa, norm, 1e-5, wg, sg, wu, su, h, stream=sp)
            ops.encode_qgemv_i8(wd, sd, h, y, stream=sp)
        info.update({"kernel": "decode_i8_kernel (QKV, gate/up), attn_head_kernel, qgemv_i8_kernel (o, down)",
                     "algorithmic_bytes": sum(t.numel() for t in (wq, wk, wv, wo, wg, wu, wd))})
    elif which == "decode_layer_q4_4":
        # one configs[1]-shape Qwen2 layer for 4 sessions at context 512, eager launches: the fused q4 QKV
        # (+ RMSNorm, biases, RoPE, K/V write), attention, o_proj, fused q4 gate/up, down_proj (f32 x,
        # MLX q4 g64 with f32 scales and biases, as the u32 runners hold them), 20 times
        H, NH, NKV, HD, I, L, TPB, CTX, R = 896, 14, 2, 64, 4864, 1, 16, 512, 4
        kvd, blocks = NKV * HD, CTX // TPB

        def q4w(o, i):
            wq_ = torch.randint(-2**31, 2**31 - 1, (o, i // 8), dtype=torch.int32, device="cuda", generator=gen)
            s_ = (torch.rand((o, i // 64), device="cuda", generator=gen) + 0.5) / (4.6 * i ** 0.5)
            return wq_, s_, -7.5 * s_

        (wq, sq, bq), (wk, sk, bk), (wv, sv, bv) = q4w(H, H), q4w(kvd, H), q4w(kvd, H)
        (wo, so, bo), (wg, sg, bg), (wu, su, bu), (wd, sd, bd) = q4w(H, H), q4w(I, H), q4w(I, H), q4w(H, I)
        pq, pk, pv = (torch.randn(n, device="cuda", generator=gen) * 0.1 for n in (H, kvd, kvd))
        norm = torch.ones(H, dtype=torch.float32, device="cuda")
        total = R * blocks
        kc = torch.randn(total * L * TPB * kvd, device="cuda", generator=gen).to(torch.float16)
        vc = torch.randn(total * L * TPB * kvd, device="cuda", generator=gen).to(torch.float16)
        bt = torch.tensor([[b * R + s for b in range(blocks)] for s in range(R)], dtype=torch.int32, device="cuda")
        pos = torch.full((R,), CTX - 1, dtype=torch.int32, device="cuda")
        ang = torch.arange(CTX, device="cuda").float()[:, None] * torch.pow(
            1000000.0, -torch.arange(0, HD, 2, device="cuda").float() / HD)[None, :]
        cs = torch.stack([torch.cos(ang), torch.sin(ang)], dim=-1).contiguous()
        xa, xb = torch.randn((R, H), device="cuda", generator=gen), torch.zeros((R, H), device="cuda")
        y = torch.zeros((R, H), device="cuda")
        q = torch.empty((R, NH * HD), device="cuda")
        att = torch.empty((R, NH * HD), device="cuda")
        h = torch.empty((R, I), device="cuda")
        sp = stream.cuda_stream
        for _ in range(20):
            ops.encode_decode_q4_qkv(xa, y, xb, norm, 1e-6, wq, sq, bq, pq, wk, sk, bk, pk, wv, sv, bv, pv, 64, NH,
                                     NKV, HD, pos, cs, q, kc, vc, bt, total, L, TPB, 0, stream=sp)
            ops.encode_attention(q, kc, vc, bt, pos, att, NH, NKV, HD, total, L, TPB, 0, stream=sp)
            ops.encode_qgemv_q4_affine(wo, so, bo, att, y, stream=sp)
            ops.encode_decode_q4_gate_up(xb, y, xa, norm, 1e-6, wg, sg, bg, wu, su, bu, 64, h, stream=sp)
            ops.encode_qgemv_q4_affine(wd, sd, bd, h, y, stream=sp)
        info.update({"kernel": "decode_q4_kernel (QKV, gate/up), attn_head_kernel, qgemv_q4_x32_kernel (o), "
                               "qgemv_q4_x32s_kernel (down)",
                     # packed W + f32 S,B per group of 64 + f32 x + f32 y per projection
                     "algorithmic_bytes": sum(o * i // 2 + 8 * o * (i // 64) + 4 * R * i + 4 * R * o for o, i in
                                              ((H, H), (kvd, H), (kvd, H), (H, H), (I, H), (I, H), (H, I)))})
    elif which == "i4_6912x1152":
        k, n, copies = 6912, 1152, 8
        w = torch.randint(0, 256, (copies, n, k // 2), dtype=torch.uint8, device="cuda", generator=gen)
        sc = (torch.rand((n,), device="cuda", generator=gen) * 0.019 + 0.001).to(torch.float16)
        x = torch.randn((1, k), device="cuda", generator=gen)
        y = torch.empty((1, n), dtype=torch.float32, device="cuda")
        arr = op_array([ops.qgemv_op_i4_sym(w[i % copies], sc, k, x, y, k) for i in range(20)])
        ops.encode_qgemv_batch(arr, stream=stream.cuda_stream)
        info.update({"kernel": "qgemv_i4_kernel (symmetric i4 6912->1152, gs = K, M=1, f32 x)",
                     "algorithmic_bytes": n * k // 2 + 2 * n + 4 * k + 4 * n})
    elif which.startswith(("q4_down_6912x1152_m", "q4_gate_up_1152x13824_m")):
        k, n = (6912, 1152) if "down" in which else (1152, 13824)
        copies, m = 8, int(which.rsplit("_m", 1)[1])
        ws = [Q4Weights(torch, n, k, gen) for _ in range(copies)]
        x = torch.randn((m, k), device="cuda", generator=gen).to(torch.float16)
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        arr = op_array([ops.qgemv_op_q4_affine(ws[i % copies].wq, ws[i % copies].s, ws[i % copies].b, x, y)
                        for i in range(20)])
        ops.encode_qgemv_batch(arr, stream=stream.cuda_stream)
        info.update({"kernel": f"q4 affine {k}->{n}, M={m} (VALU GEMV at M <= 4 and N < 8192, else MFMA)",
                     "algorithmic_bytes": q4_bytes(m, n, k)})
    elif which == "q4_gate_up_silu_1152x6912":
        k, n, copies = 1152, 6912, 8
        ws = [(Q4Weights(torch, n, k, gen), Q4Weights(torch, n, k, gen)) for _ in range(copies)]
        x = torch.randn((1, k), device="cuda", generator=gen).to(torch.float16)
        h = torch.empty((1, n), dtype=torch.float32, device="cuda")
        for i in range(20):
            g_, u_ = ws[i % copies]
            ops.encode_gate_up_silu_q4_affine(g_.wq, g_.s, g_.b, u_.wq, u_.s, u_.b, x, h, stream=stream.cuda_stream)
        info.update({"kernel": "qgemv_q4_gate_up_silu_kernel (q4 affine 1152->6912 x2 + SiLU, M=1)",
                     "algorithmic_bytes": 2 * (n * k // 2 + 4 * n * ((k + 63) // 64)) + 2 * k + 4 * n})
    else:
        k, n = (896, 4864) if which == "qgemm_896x4864" else (4864, 896)
        m = 512
        w = Q4Weights(torch, n, k, gen)
        x = torch.randn((m, k), device="cuda", generator=gen).to(torch.float16)
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        for _ in range(20):
            ops.encode_qgemm_q4_affine(w.wq, w.s, w.b, x, y, stream=stream.cuda_stream)
        info.update({"kernel": f"qgemm_q4_regw_kernel (M=512, {k}->{n})", "flops": 2 * m * n * k,
                     "algorithmic_bytes": q4_bytes(m, n, k)})
    torch.cuda.synchronize()
    print(json.dumps({"pmc_sample": info}))


def q4_copies(torch, n: int, k: int, gen, min_bytes: int = CACHE_BYTES):
    """R copies of one q4 g64 weight (f16 S/B) with R * bytes > min_bytes, allocated as three
    tensors; returns R and the list of (wq, s, b) views."""
    g = (k + 63) // 64
    wbytes = n * k // 2 + 4 * n * g
    r = max(2, -(-min_bytes // wbytes) + 1)
    wq = torch.randint(-2**31, 2**31 - 1, (r, n, k // 8), dtype=torch.int32, device="cuda", generator=gen)
    s = (torch.randn((r, n, g), device="cuda", generator=gen) * 0.005 + 0.02).abs_().to(torch.float16)
    b = (torch.randn((r, n, g), device="cuda", generator=gen) * 0.05).to(torch.float16)
    return r, [(wq[i], s[i], b[i]) for i in range(r)]


class Q4Weights:
    def __init__(self, torch, n: int, k: int, gen):
        self.n, self.k = n, k
        g = (k + 63) // 64
        self.wq = torch.randint(-2**31, 2**31 - 1, (n, k // 8), dtype=torch.int32, device="cuda", generator=gen)
        self.s = (torch.randn((n, g), device="cuda", generator=gen) * 0.005 + 0.02).abs_().to(torch.float16)
        self.b = (torch.randn((n, g), device="cuda", generator=gen) * 0.05).to(torch.float16)


def time_batch(torch, ops, arr, stream, reps: int = 5, warm_s: float = 0.02, trials: int = 3):
    """Mean ms per launch over `reps` cellm_hip_qgemv_batch calls of the
    prebuilt op array `arr`, HIP events on the launch stream; the median of
    `trials` such blocks, after at least `warm_s` seconds of the same calls.
    (Right after a stretch of launch-bound small kernels, the first block of
    a long kernel reads 5-10 % slower than every later one on the box.)"""
    t0 = time.perf_counter()
    while True:
        ops.encode_qgemv_batch(arr, stream=stream.cuda_stream)
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= warm_s:
            break
    out = []
    for _ in range(trials):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            ops.encode_qgemv_batch(arr, stream=stream.cuda_stream)
        e1.record(stream)
        torch.cuda.synchronize()
        out.append(e0.elapsed_time(e1) / (reps * len(arr)))
    return sorted(out)[len(out) // 2]


def isolated_launch_us(torch, ops, arr, stream, reps: int = 20) -> float:
    """Median of `reps` single launches, each alone on an idle GPU: HIP events
    around one op of `arr` (its own weight copy), with a synchronisation before
    and after (the latency one projection adds when nothing is queued)."""
    out = []
    for i in range(reps):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        ops.encode_qgemv_batch(op_array([arr[i % len(arr)]]), stream=stream.cuda_stream)
        e1.record(stream)
        torch.cuda.synchronize()
        out.append(e0.elapsed_time(e1) * 1e3)
    return round(sorted(out)[len(out) // 2], 2)


def time_calls(torch, fn, reps: int, stream):
    """Mean ms per call of fn(i) over `reps` back-to-back calls (used for the
    qGEMM, whose kernels far outlast the host launch cost)."""
    fn(0)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(reps):
        fn(i)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def op_array(ops_list):
    from cellm_amd._lib import QgemvOp

    return (QgemvOp * len(ops_list))(*ops_list)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 (multi-GPU sharding of the "
                                   "path is designed, not implemented)"}))
        sys.exit(2)

    import torch

    from cellm_amd import HipOps

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    ops = HipOps(0)
    stream = torch.cuda.current_stream()
    sptr = stream.cuda_stream
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0xCE11)
    if args.pmc_sample:
        pmc_sample(torch, ops, stream, gen, args.pmc_sample)
        ops.close()
        return

    # ---- the step -------------------------------------------------
    step_bytes = sum(q4_bytes(1, n, k) for _, k, n in QWEN_SHAPES)
    w_bytes_per_set = sum(n * k // 2 + 4 * n * ((k + 63) // 64) for _, k, n in QWEN_SHAPES)
    copies = max(2, -(-512 * 2**20 // w_bytes_per_set) + 1)
    sets = [[Q4Weights(torch, n, k, gen) for _, k, n in QWEN_SHAPES] for _ in range(copies)]
    xs = [torch.randn((1, k), device="cuda", generator=gen).to(torch.float16) for _, k, _ in QWEN_SHAPES]
    ys = [torch.empty((1, n), dtype=torch.float32, device="cuda") for _, _, n in QWEN_SHAPES]

    # one op array per weight copy: a step is one cellm_hip_qgemv_batch call
    step_arrays = [op_array([ops.qgemv_op_q4_affine(w.wq, w.s, w.b, xs[j], ys[j]) for j, w in enumerate(ws)])
                   for ws in sets]

    def step(i):
        ops.encode_qgemv_batch(step_arrays[i % copies], stream=sptr)

    # Warm-up: the W steps asked for, and at least one pass over every weight copy and WARM_MIN_S
    # seconds of steps.  Right after the weights are written, the first steps of a fresh process
    # read 40-55 us where every later one reads ~29 us (first touch of each copy's pages, clocks
    # still rising): W = 5 steps touch only 5 of the copies.  The extra steps are reported.
    warm_steps, t_warm = 0, time.perf_counter()
    while warm_steps < max(args.warmup, copies) or time.perf_counter() - t_warm < WARM_MIN_S:
        step(warm_steps)
        warm_steps += 1
        if warm_steps % 64 == 0:
            torch.cuda.synchronize()  # keep the queue short
    torch.cuda.synchronize()
    warm_s = time.perf_counter() - t_warm
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(args.steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_total = ev0.elapsed_time(ev1)
    ms_per_step = ms_total / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    del step_arrays, sets
    torch.cuda.empty_cache()

    # ---- per-shape latency and the dominant kernel's roofline ---------------------
    # Each shape rotates through its own R weight copies with R * W > CACHE_BYTES (one op per copy
    # in the timed batch), so every launch reads its weights from HBM.
    per_shape = {}
    for j, (name, k, n) in enumerate(QWEN_SHAPES):
        r_copies, wset = q4_copies(torch, n, k, gen)
        arr = op_array([ops.qgemv_op_q4_affine(*wset[i % r_copies], xs[j], ys[j]) for i in range(max(100, r_copies))])
        ms = time_batch(torch, ops, arr, stream, reps=1 if len(arr) > 100 else 5)
        gbs = q4_bytes(1, n, k) / (ms * 1e-3) / 1e9
        per_shape[f"{name}_{k}x{n}"] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
                                        "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                                        "isolated_us": isolated_launch_us(torch, ops, arr, stream),
                                        "weight_copies": r_copies,
                                        "bytes_rotated": r_copies * (n * k // 2 + 4 * n * ((k + 63) // 64))}
        del arr, wset
        torch.cuda.empty_cache()
    dom = per_shape["lm_head_896x151936"]
    traffic = None
    tfile = ROOT / "profiles" / "traffic_q4_gemv_lm_head.json"
    if tfile.exists():
        try:
            traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")
        except Exception:
            traffic = None
    roofline = {"bound": "hbm", "achieved": dom["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(dom["GB/s"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": "qgemv_q4_flat_kernel (896->151936 lm_head, M=1)",
                "algorithmic_bytes": q4_bytes(1, 151936, 896)}

    extra = {}
    if not args.no_extra:
        progress("configs[1] step and per-shape lines done")
        extra = extra_configs(torch, ops, stream, gen, graphs=not args.eager_decode_step)
        rd = extra.get("hbm_stream_read_77MB")
        if rd:
            # the same bytes read by the probe: the lm_head against the box's own streaming ceiling
            roofline["measured_read_peak_GBs"] = rd["GB/s"]
            roofline["frac_of_measured_read_peak"] = round(dom["GB/s"] / rd["GB/s"], 4)

    cpu = None
    if not args.no_cpu:
        progress("extra lines done")
        cpu = cpu_baseline()
        progress("cpu baseline done")

    out = {
        "metric": BASELINE_METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4*f16->f32",
        "data": "synthetic (seeded random weights/activations of the config shapes)",
        "config": {"workload": "qwen2.5-0.5b-shape q4-affine g64 decode GEMV set, batch 1: "
                               "896->1152, 896->896, 896->9728, 4864->896, 896->151936",
                   "weight_copies_rotated": copies, "bytes_per_step": step_bytes,
                   "timing": "HIP events on the launch stream; a step is one cellm_hip_qgemv_batch call",
                   "warmup_steps_run": warm_steps, "warmup_s": round(warm_s, 3),
                   "frac_hbm_peak": round(value / HBM_PEAK_GBS, 4), "wall_s": round(wall, 3)},
        "per_shape": per_shape,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out))
    ops.close()


def extra_configs(torch, ops, stream, gen, graphs: bool = True):
    """configs[0], [2], [3]: int8 GEMV, Gemma batched decode, M=512 prefill qGEMM;
    plus a measured device-to-device copy as the box's practical HBM figure."""
    res = {}

    # plain 512 MiB device copy: read + write bytes over time
    nbytes = 512 * 2**20
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    ms = time_calls(torch, lambda i: dst.copy_(src), 20, stream)
    res["hbm_copy_512MiB"] = {"us": round(ms * 1e3, 1), "GB/s_read_plus_write": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}
    del src, dst

    res.update(launch_floor(torch, ops, stream))
    res.update(measured_ceilings(torch, stream))
    progress("copy and launch floor done")

    # SmolLM2-135M int8, fp32 scale, fp32 x, K=576
    for n in (576, 1536):
        k = 576
        copies = max(2, -(-512 * 2**20 // (n * k)) + 1)
        w = torch.randint(-127, 128, (copies, n, k), dtype=torch.int8, device="cuda", generator=gen)
        s = torch.rand((n,), device="cuda", generator=gen) * 0.019 + 0.001
        x = torch.randn((1, k), device="cuda", generator=gen)
        y = torch.empty((1, n), dtype=torch.float32, device="cuda")
        arr = op_array([ops.qgemv_op_i8(w[i % copies], s, x, y) for i in range(200)])
        ms = time_batch(torch, ops, arr, stream)
        b = i8_bytes(1, n, k, 4)
        res[f"cfg1_i8_576x{n}"] = {"us": round(ms * 1e3, 3), "GB/s": round(b / (ms * 1e-3) / 1e9, 1)}
        del w

    # Gemma-3-1B int8 lm_head 1152->262144 and q4 gate+up 1152->13824 at M in {1,4,16,64}
    k, n = 1152, 262144
    copies = 2
    w = torch.randint(-127, 128, (copies, n, k), dtype=torch.int8, device="cuda", generator=gen)
    s = torch.rand((n,), device="cuda", generator=gen) * 0.019 + 0.001
    for m in (1, 4, 16, 64):
        x = torch.randn((m, k), device="cuda", generator=gen).to(torch.float16)
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        arr = op_array([ops.qgemv_op_i8(w[i % copies], s, x, y) for i in range(20)])
        ms = time_batch(torch, ops, arr, stream, reps=2)
        b = i8_bytes(m, n, k, 2)
        res[f"cfg3_i8_lm_head_1152x262144_m{m}"] = {"us": round(ms * 1e3, 2), "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
                                                    "frac_hbm": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    del w
    k, n = 1152, 13824
    wset = [Q4Weights(torch, n, k, gen) for _ in range(64)]
    for m in (1, 4, 16, 64):
        x = torch.randn((m, k), device="cuda", generator=gen).to(torch.float16)
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        arr = op_array([ops.qgemv_op_q4_affine(wset[i % 64].wq, wset[i % 64].s, wset[i % 64].b, x, y)
                        for i in range(100)])
        ms = time_batch(torch, ops, arr, stream)
        b = q4_bytes(m, n, k)
        res[f"cfg3_q4_gate_up_1152x13824_m{m}"] = {"us": round(ms * 1e3, 2), "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
                                                   "frac_hbm": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    del wset
    # configs[2]'s other projections: int8 fused QKV 1152->1536 and o 1024->1152, q4 down 6912->1152
    for name, kind, k, n in (("i8_attn_qkv", "i8", 1152, 1536), ("i8_attn_o", "i8", 1024, 1152),
                             ("q4_mlp_down", "q4", 6912, 1152)):
        wbytes = n * k if kind == "i8" else n * k // 2 + 4 * n * (k // 64)
        copies = max(2, -(-512 * 2**20 // wbytes) + 1)
        if kind == "i8":
            w8 = torch.randint(-127, 128, (copies, n, k), dtype=torch.int8, device="cuda", generator=gen)
            s8 = torch.rand((n,), device="cuda", generator=gen) * 0.019 + 0.001
        else:
            wset = [Q4Weights(torch, n, k, gen) for _ in range(copies)]
        for m in (1, 4, 16, 64):
            x = torch.randn((m, k), device="cuda", generator=gen).to(torch.float16)
            y = torch.empty((m, n), dtype=torch.float32, device="cuda")
            if kind == "i8":
                arr = op_array([ops.qgemv_op_i8(w8[i % copies], s8, x, y) for i in range(100)])
                bts = i8_bytes(m, n, k, 2)
            else:
                arr = op_array([ops.qgemv_op_q4_affine(wset[i % copies].wq, wset[i % copies].s, wset[i % copies].b,
                                                       x, y) for i in range(100)])
                bts = q4_bytes(m, n, k)
            ms = time_batch(torch, ops, arr, stream)
            res[f"cfg3_{name}_{k}x{n}_m{m}"] = {"us": round(ms * 1e3, 2),
                                                "GB/s": round(bts / (ms * 1e-3) / 1e9, 1),
                                                "frac_hbm": round(bts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        if kind == "i8":
            del w8
        else:
            del wset

    progress("configs[0] and configs[2] done")
    res.update(decode_step_cfg5(graphs))
    progress("configs[4] decode step done")
    res.update(decode_step_cfg2_qwen(graphs))
    progress("configs[4] decode step done")
    res.update(lowbit_gemvs(torch, ops, stream, gen))
    res.update(i4_gemma_mlp(torch, ops, stream, gen))
    res.update(q4_gate_up_silu(torch, ops, stream, gen))
    progress("low-bit, i4 and fused gate/up lines done")

    # M=512 prefill qGEMM (MFMA)
    m = 512
    for k, n in ((896, 4864), (4864, 896)):
        w = Q4Weights(torch, n, k, gen)
        x = torch.randn((m, k), device="cuda", generator=gen).to(torch.float16)
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        fn = lambda i: ops.encode_qgemm_q4_affine(w.wq, w.s, w.b, x, y, stream=stream.cuda_stream)
        ms = time_calls(torch, fn, 100, stream)
        tflops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
        res[f"cfg4_qgemm_m512_{k}x{n}"] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(tflops, 1),
                                           "frac_mfma_f16": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                                           "frac_mfma_f16_measured": round(
                                               tflops / res["mfma_f16_measured"]["TFLOP/s"], 4)}
    return res


def measured_ceilings(torch, stream):
    """The box's own ceilings beside the published peaks (libcellm_probes.so):
    dense f16 MFMA throughput (v_mfma_f32_32x32x16_f16 on register operands, four
    blocks of four waves per CU) and the streaming read rate of a 77,185,280-byte
    buffer, the q4 lm_head's algorithmic bytes (eight rotating copies, 617 MB,
    past the 256 MB MALL)."""
    import ctypes as C

    lib = C.CDLL(str(ROOT / "cellm_amd" / "libcellm_probes.so"))
    lib.cellm_probe_mfma_f16.argtypes = [C.c_int32, C.c_int32, C.c_void_p, C.c_void_p]
    lib.cellm_probe_mfma_f16.restype = C.c_int32
    lib.cellm_probe_mfma_f16_flops.argtypes = [C.c_int32, C.c_int32]
    lib.cellm_probe_mfma_f16_flops.restype = C.c_double
    lib.cellm_probe_stream_read.argtypes = [C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p]
    lib.cellm_probe_stream_read.restype = C.c_int32
    sptr = C.c_void_p(stream.cuda_stream)
    res = {}

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    blocks, iters = 4 * cus, 2000
    sink = torch.empty((blocks,), dtype=torch.float32, device="cuda")

    def mfma(i):
        assert lib.cellm_probe_mfma_f16(blocks, iters, C.c_void_p(sink.data_ptr()), sptr) == 0

    best = min(time_calls(torch, mfma, 5, stream) for _ in range(3))
    tflops = lib.cellm_probe_mfma_f16_flops(blocks, iters) / (best * 1e-3) / 1e12
    res["mfma_f16_measured"] = {"TFLOP/s": round(tflops, 1), "frac_published": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                                "probe": f"{blocks} blocks x 4 waves, {iters} rounds of 8 independent "
                                         "v_mfma_f32_32x32x16_f16 chains per wave"}

    nbytes = q4_bytes(1, 151936, 896)
    nbytes -= nbytes % 16
    copies = 8
    bufs = [torch.empty((nbytes // 4,), dtype=torch.int32, device="cuda").fill_(i) for i in range(copies)]
    isink = torch.empty((1,), dtype=torch.int32, device="cuda")

    def rd(i):
        assert lib.cellm_probe_stream_read(C.c_void_p(bufs[i % copies].data_ptr()), nbytes,
                                           C.c_void_p(isink.data_ptr()), sptr) == 0

    for i in range(20):
        rd(i)
    ms = sorted(time_calls(torch, rd, 100, stream) for _ in range(3))[1]
    res["hbm_stream_read_77MB"] = {"us": round(ms * 1e3, 2), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                                   "frac_published": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                   "probe": "non-temporal 16-byte loads, 4 in flight per lane, grid-stride over "
                                            "one 512-thread block per CU, 8 rotating copies"}
    del bufs
    return res


def launch_floor(torch, ops, stream):
    """The box's floor for one dependent kernel launch, against which the
    small decode shapes are judged launch-bound:
      * eager: 200 back-to-back launches of the smallest int8 GEMV (M=1,
        16x64, one block) from one cellm_hip_qgemv_batch call, as the bench
        step issues its projections;
      * graph: 200 single-block elementwise launches (cellm_hip_add_f32_inplace
        on 64 floats) captured in a HIP graph and replayed.
    Both per launch, HIP events on the stream."""
    res = {}
    w = torch.zeros((16, 64), dtype=torch.int8, device="cuda")
    s = torch.ones((16,), dtype=torch.float32, device="cuda")
    x = torch.zeros((1, 64), dtype=torch.float32, device="cuda")
    y = torch.empty((1, 16), dtype=torch.float32, device="cuda")
    arr = op_array([ops.qgemv_op_i8(w, s, x, y) for _ in range(200)])
    res["launch_floor_eager_us"] = round(time_batch(torch, ops, arr, stream) * 1e3, 3)
    a = torch.zeros(64, dtype=torch.float32, device="cuda")
    b = torch.zeros(64, dtype=torch.float32, device="cuda")
    cap = torch.cuda.Stream()
    with torch.cuda.stream(cap):
        ops.encode_add_inplace(a, b, stream=cap.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        for _ in range(200):
            ops.encode_add_inplace(a, b, stream=cap.cuda_stream)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(5):
        g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    res["launch_floor_graph_us"] = round(e0.elapsed_time(e1) / 1000 * 1e3, 3)
    del g
    return res


def lowbit_gemvs(torch, ops, stream, gen):
    """The remaining .cellm weight formats at batch 1 (f16 x): f16 896->4864
    (Qwen2.5-0.5B gate), i2 1152->6912 (Gemma-3-1B MLP), q1_0_g128
    1152->6912 and 1152->262144 (a Gemma-3-1B-size lm_head).  Weight copies
    rotate past 512 MB so that they stream from HBM.  Bytes per call: weights
    and row scales + x + y."""
    res = {}
    cases = [("f16", 896, 4864), ("i2", 1152, 6912), ("q1_0_g128", 1152, 6912), ("q1_0_g128", 1152, 262144)]
    for fmt, k, n in cases:
        if fmt == "f16":
            wbytes, sbytes = n * k * 2, 0
        elif fmt == "i2":
            wbytes, sbytes = n * k // 4, 2 * n
        else:
            wbytes, sbytes = n * (k // 128) * 18, 0
        copies = max(2, -(-512 * 2**20 // wbytes) + 1)
        w = torch.randint(0, 256, (copies, wbytes), dtype=torch.uint8, device="cuda", generator=gen)
        if fmt == "q1_0_g128":  # finite d in every block
            d = torch.full((copies, n * (k // 128), 1), 0.05, dtype=torch.float16, device="cuda").view(torch.uint8)
            w.view(copies, n * (k // 128), 18)[:, :, :2] = d
        s = (torch.rand((n,), device="cuda", generator=gen) * 0.04 + 0.01).to(torch.float16)
        x = torch.randn((1, k), device="cuda", generator=gen).to(torch.float16)
        y = torch.empty((1, n), dtype=torch.float32, device="cuda")
        if fmt == "f16":
            arr = op_array([ops.qgemv_op_f16(w[i % copies].view(torch.float16).view(n, k), x, y) for i in range(100)])
        elif fmt == "i2":
            arr = op_array([ops.qgemv_op_i2(w[i % copies].view(n, k // 4), s, 0, x, y, k) for i in range(100)])
        else:
            arr = op_array([ops.qgemv_op_q1_0_g128(w[i % copies].view(n, -1), x, y, k) for i in range(100)])
        ms = time_batch(torch, ops, arr, stream)
        b = wbytes + sbytes + 2 * k + 4 * n
        res[f"lowbit_{fmt}_{k}x{n}"] = {"us": round(ms * 1e3, 2), "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
                                         "frac_hbm": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del w
    return res


def i4_gemma_mlp(torch, ops, stream, gen):
    """Gemma-3-1B MLP in the reference's symmetric i4 format (gemma.rs:1446-1471:
    one f16 scale per row, gs = in_dim, f32 activations): gate/up 1152->6912
    and down 6912->1152 at M in {1, 4}.  Weight copies rotate past 512 MB.
    Bytes per call: weights + row scales + x + y."""
    res = {}
    for k, n in ((1152, 6912), (6912, 1152)):
        wbytes = n * k // 2
        copies = max(2, -(-512 * 2**20 // wbytes) + 1)
        w = torch.randint(0, 256, (copies, n, k // 2), dtype=torch.uint8, device="cuda", generator=gen)
        s = (torch.rand((n,), device="cuda", generator=gen) * 0.019 + 0.001).to(torch.float16)
        for m in (1, 4):
            x = torch.randn((m, k), device="cuda", generator=gen)
            y = torch.empty((m, n), dtype=torch.float32, device="cuda")
            arr = op_array([ops.qgemv_op_i4_sym(w[i % copies], s, k, x, y, k) for i in range(100)])
            ms = time_batch(torch, ops, arr, stream)
            b = wbytes + 2 * n + 4 * m * k + 4 * m * n
            res[f"gemma_i4_{k}x{n}_m{m}"] = {"us": round(ms * 1e3, 2), "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
                                              "frac_hbm": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del w
    return res


def _graph_us_per_call(torch, record, calls: int, trials: int = 3) -> float:
    """Capture record() (which enqueues `calls` calls on the capture stream)
    into one HIP graph, replay it, and return the median us per call."""
    cap = torch.cuda.Stream()
    with torch.cuda.stream(cap):
        record(cap.cuda_stream)  # eager pass: buffers and kernel attributes set up outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        record(cap.cuda_stream)
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    out = []
    s = torch.cuda.current_stream()
    for _ in range(trials):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        g.replay()
        e1.record(s)
        torch.cuda.synchronize()
        out.append(e0.elapsed_time(e1) * 1e3 / calls)
    del g
    return sorted(out)[len(out) // 2]


def q4_gate_up_silu(torch, ops, stream, gen):
    """MLX q4 gate/up + SiLU (the reference's mv2 + silu_mul pattern) at the
    Qwen2.5-0.5B (896->4864 x2) and Gemma-3-1B (1152->6912 x2) MLP shapes:
    one cellm_hip_qgemv_q4_affine_gate_up_silu launch against two q4 GEMVs and
    the SiLU kernel.  Each variant is captured once per weight pair into a HIP
    graph (pairs rotate past 512 MB) and replayed; us per gate/up call.  Bytes:
    both matrices' weights and f16 S/B + x + h."""
    res = {}
    for k, n in ((896, 4864), (1152, 6912)):
        pair = 2 * (n * k // 2 + 4 * n * ((k + 63) // 64))
        copies = -(-512 * 2**20 // pair) + 1
        ws = [(Q4Weights(torch, n, k, gen), Q4Weights(torch, n, k, gen)) for _ in range(copies)]
        for m in (1, 4):
            x = torch.randn((m, k), device="cuda", generator=gen).to(torch.float16)
            h = torch.empty((m, n), dtype=torch.float32, device="cuda")
            u = torch.empty((m, n), dtype=torch.float32, device="cuda")

            def fused(st):
                for g_, u_ in ws:
                    ops.encode_gate_up_silu_q4_affine(g_.wq, g_.s, g_.b, u_.wq, u_.s, u_.b, x, h, stream=st)

            def unfused(st):
                for g_, u_ in ws:
                    ops.encode_qgemv_q4_affine(g_.wq, g_.s, g_.b, x, h, stream=st)
                    ops.encode_qgemv_q4_affine(u_.wq, u_.s, u_.b, x, u, stream=st)
                    ops.encode_silu_mul(h, u, stream=st)

            b = pair + 2 * m * k + 4 * m * n
            us_f = _graph_us_per_call(torch, fused, copies)
            us_u = _graph_us_per_call(torch, unfused, copies)
            res[f"q4_gate_up_silu_{k}x{n}x2_m{m}"] = {
                "fused_us": round(us_f, 2), "unfused_us": round(us_u, 2),
                "GB/s": round(b / (us_f * 1e-6) / 1e9, 1), "frac_hbm": round(b / (us_f * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                "launch": "captured HIP graph"}
        del ws
    return res


CFG5_SESSIONS, CFG5_CTX, CFG5_TPB = 4, 512, 16


def cfg5_runner():
    """a random-init SmolLM2-360M-shape int8 model on the device
    runner (cellm_llama_dev_*): 32 layers, hidden 960, 15/5 heads of 64,
    intermediate 2560, vocab 49152, 4 sessions with context 512 of seeded f16
    K/V on interleaved pages.  Returns (runner, shape, block tables)."""
    import numpy as np

    from cellm_amd.llama_step import LlamaDevice, LlamaShape

    sessions, ctx, tpb = CFG5_SESSIONS, CFG5_CTX, CFG5_TPB
    shape = LlamaShape(32, 960, 15, 5, 64, 2560, 49152, 1e-5, 100000.0, tpb, sessions * ctx // tpb)
    rng = np.random.default_rng(0xC5)
    layers = []
    for _ in range(shape.n_layers):
        ws, ss = [], []
        for o, i in shape.proj_shapes():
            ws.append(rng.integers(-127, 128, (o, i), dtype=np.int8))
            ss.append((rng.uniform(0.5, 1.5, o) / (73.3 * np.sqrt(i))).astype(np.float16))
        n1 = (1.0 + 0.1 * rng.standard_normal(shape.hidden)).astype(np.float16)
        n2 = (1.0 + 0.1 * rng.standard_normal(shape.hidden)).astype(np.float16)
        layers.append((ws, ss, n1, n2))
    embed = rng.integers(-127, 128, (shape.vocab, shape.hidden), dtype=np.int8)
    escale = (rng.uniform(0.5, 1.5, shape.vocab) / 127.0).astype(np.float16)
    fnorm = (1.0 + 0.1 * rng.standard_normal(shape.hidden)).astype(np.float16)
    dev = LlamaDevice(shape, layers, embed, escale, fnorm, 0, max_rows=sessions, max_blocks=ctx // tpb)
    del layers, embed
    kv = shape.kv_elems()
    dev.kv_upload(rng.standard_normal(kv, dtype=np.float32).astype(np.float16),
                  rng.standard_normal(kv, dtype=np.float32).astype(np.float16))
    bts = np.array([[b * sessions + s for b in range(ctx // tpb)] for s in range(sessions)], np.uint32)
    return dev, shape, bts


def decode_step_cfg5(graphs: bool = True):
    """The configs[4] decode step: host ids in -> greedy ids out (input/output
    copies and the final synchronisation included), timed on the host clock,
    replaying the captured graph and, for comparison, launching eagerly.
    Bytes per step: every int8 weight and scale once, plus each session's K/V
    over its context."""
    import numpy as np

    dev, shape, bts = cfg5_runner()
    sessions, ctx = CFG5_SESSIONS, CFG5_CTX
    kvd = shape.n_kv_heads * shape.head_dim
    res = {}
    for rows in (sessions, 1):
        tokens = np.array([(1000 + 7919 * s) % shape.vocab for s in range(rows)], np.uint32)
        pos = np.full(rows, ctx - 1, np.int32)
        step_bytes = shape.weight_bytes() + rows * ctx * shape.n_layers * kvd * 2 * 2
        entry = {"sessions": rows, "context": ctx, "bytes_per_step": step_bytes,
                 "launch": "captured HIP graph" if graphs else "eager launches"}
        for replay in ((True, False) if graphs else (False,)):
            dev.set_graphs(replay)
            for _ in range(3):
                dev.step(tokens, pos, bts[:rows])
            n = 50
            t0 = time.perf_counter()
            for _ in range(n):
                ids, _ = dev.step(tokens, pos, bts[:rows])
            us = (time.perf_counter() - t0) / n * 1e6
            if replay or not graphs:
                entry.update({"us_per_step": round(us, 1), "tokens_per_s": round(rows * 1e6 / us, 1),
                              "GB/s": round(step_bytes / (us * 1e-6) / 1e9, 1),
                              "frac_hbm": round(step_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
            else:
                entry["eager_us_per_step"] = round(us, 1)
        res[f"cfg5_llama360m_i8_decode_step_{rows}sessions"] = entry
    dev.close()
    return res


def decode_step_cfg2_qwen(graphs: bool = True):
    """configs[1]'s projections inside a model: a random-init Qwen2.5-0.5B-shape decode step on the
    device runner (cellm_llama_dev_create_from_file, model_type "qwen2"): 24 layers, hidden 896, 14/2
    heads of 64, intermediate 4864, vocabulary 151936; every projection and the untied lm_head MLX
    4-bit affine (u32 words, f32 scales and biases per group of 64, the .cellm layout
    tools/convert_lfm.py writes), f16 q/k/v biases, int8 embedding; 1 and 4 sessions at context 512
    of seeded f16 K/V.  The file is written to a temporary directory and removed.  Timed as the
    configs[4] step; bytes per step: every weight, scale and bias once plus each session's K/V."""
    import tempfile

    import numpy as np

    from cellm_amd.cellm_file import llama_header, write_cellm
    from cellm_amd.llama_step import LlamaDevice

    L, H, NH, NKV, HD, I, V = 24, 896, 14, 2, 64, 4864, 151936
    sessions, ctx, tpb = 4, 512, 16
    kvd = NKV * HD
    rng = np.random.default_rng(0xC2)
    names = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
             "mlp.up_proj", "mlp.down_proj")
    shapes = [(H, H), (kvd, H), (kvd, H), (H, H), (I, H), (I, H), (H, I)]

    def q4(name, o, i):
        # zero-mean weights of std ~1/sqrt(i): q*s + b with s ~ U(0.5,1.5)/(4.6 sqrt(i)), b ~ -7.5 s
        wq = rng.integers(0, 2**32, (o, i // 8), dtype=np.uint32)
        sc = (rng.uniform(0.5, 1.5, (o, i // 64)) / (4.6 * np.sqrt(i))).astype(np.float32)
        bi = (-7.5 * sc).astype(np.float32)
        base = name[:-len(".weight")]
        return [(name, wq, "u32", wq.shape), (base + ".scales", sc, "f32", sc.shape), (base + ".biases", bi, "f32", bi.shape)]

    ts, wbytes = [], 0
    for l in range(L):
        pre = f"model.layers.{l}."
        for j, (o, i) in enumerate(shapes):
            ts += q4(pre + names[j] + ".weight", o, i)
            if j < 3:
                ts.append((pre + names[j] + ".bias", rng.standard_normal(o).astype(np.float16), "f16", (o,)))
        for nm in ("input_layernorm.weight", "post_attention_layernorm.weight"):
            ts.append((pre + nm, (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float16), "f16", (H,)))
    ts.append(("model.embed_tokens.weight", rng.integers(-127, 128, (V, H), dtype=np.int8), "i8", (V, H)))
    ts.append(("model.embed_tokens.weight.qscale", (rng.uniform(0.5, 1.5, V) / 127.0).astype(np.float16), "f16", (V,)))
    ts.append(("model.norm.weight", (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float16), "f16", (H,)))
    ts += q4("lm_head.weight", V, H)
    # bytes a step reads: every projection and lm_head tensor, biases and norms, one embedding row per session
    wbytes = sum(a.nbytes for n, a, _, _ in ts if not n.startswith("model.embed_tokens"))
    res = {}
    with tempfile.TemporaryDirectory() as tmp:
        path = Path(tmp) / "qwen25_05b_q4.cellm"
        write_cellm(path, llama_header(L, H, NH, NKV, I, V, eps=1e-6, theta=1000000.0, model_type="qwen2",
                                       tie_word_embeddings=False), ts)
        del ts
        dev = LlamaDevice.from_file(path, 0, max_rows=sessions, max_blocks=ctx // tpb, tokens_per_block=tpb)
    try:
        kv = dev.shape.kv_elems()
        dev.kv_upload(rng.standard_normal(kv, dtype=np.float32).astype(np.float16),
                      rng.standard_normal(kv, dtype=np.float32).astype(np.float16))
        bts = np.array([[b * sessions + s for b in range(ctx // tpb)] for s in range(sessions)], np.uint32)
        for rows in (sessions, 1):
            tokens = np.array([(1000 + 7919 * s) % V for s in range(rows)], np.uint32)
            pos = np.full(rows, ctx - 1, np.int32)
            step_bytes = wbytes + rows * (H + 2) + rows * ctx * L * kvd * 2 * 2
            entry = {"sessions": rows, "context": ctx, "bytes_per_step": step_bytes,
                     "weights": "u32 MLX affine g64, f32 scales/biases; f16 q/k/v biases; int8 embedding",
                     "launch": "captured HIP graph" if graphs else "eager launches"}
            for replay in ((True, False) if graphs else (False,)):
                dev.set_graphs(replay)
                for _ in range(3):
                    dev.step(tokens, pos, bts[:rows])
                n = 50
                t0 = time.perf_counter()
                for _ in range(n):
                    dev.step(tokens, pos, bts[:rows])
                us = (time.perf_counter() - t0) / n * 1e6
                if replay or not graphs:
                    entry.update({"us_per_step": round(us, 1), "tokens_per_s": round(rows * 1e6 / us, 1),
                                  "GB/s": round(step_bytes / (us * 1e-6) / 1e9, 1),
                                  "frac_hbm": round(step_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
                else:
                    entry["eager_us_per_step"] = round(us, 1)
            res[f"cfg2_qwen25_05b_q4_decode_step_{rows}sessions"] = entry
    finally:
        dev.close()
    return res


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_time(fn, budget_s: float, max_reps: int = 50, min_reps: int = 3) -> tuple[float, int]:
    """Median seconds per call after one warm-up call, within about budget_s."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_reps or (time.perf_counter() < t_end and len(times) < max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2], len(times)


def cpu_baseline():
    """The CPU oracle (a C restatement of the reference CPU kernels, OpenMP over
    rows as rayon does) on the host cores, on bounded samples of the workloads.

    `value` is configs[1]'s decode pass as the reference runs it per token
    (LfmRunner, lfm.rs): the four projections hit the f32 dequant cache and run
    the f32 row GEMV ('warm', lfm.rs:1056-1063); the tied lm_head dequantizes on
    the fly (lfm.rs:700-741).  `legs` time the other reference CPU paths of the
    the same pass 'cold' (the f32 dequant of each projection included,
    lfm.rs:1012-1026), matmul_i8_f32 at configs[0] (cpu_kernels.rs:66-133), the
    configs[2] int8 lm_head row GEMV, and matmul_f32 at configs[3]'s M = 512
    over the dequantized weight (cpu_kernels.rs:36-63).
    """
    import numpy as np

    import oracle

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
    rng = np.random.default_rng(0xCE11)

    def q4(n, k):
        wq = rng.integers(0, 2**32, (n, k // 8), dtype=np.uint32)
        s = (np.abs(rng.normal(0.02, 0.005, (n, k // 64)))).astype(np.float32)
        b = rng.normal(0.0, 0.05, (n, k // 64)).astype(np.float32)
        return wq, s, b

    lin_q = [(k, n) + q4(n, k) for _, k, n in QWEN_SHAPES[:-1]]
    lin = [(oracle.q4_affine_dequant_f32(wq, s, b, k), rng.normal(size=k).astype(np.float32)) for k, n, wq, s, b in lin_q]
    k, n = 896, 151936
    wq, s, b = q4(n, k)
    x = rng.normal(size=k).astype(np.float32)

    def warm_pass():
        for w32, xv in lin:
            oracle.matmul_f32(w32, xv.reshape(-1, 1))
        oracle.lfm_lm_head_q4_affine(wq, s, b, x, n, k)

    def cold_pass():
        for (kk, _, wq_, s_, b_), (_, xv) in zip(lin_q, lin):
            oracle.matmul_f32(oracle.q4_affine_dequant_f32(wq_, s_, b_, kk), xv.reshape(-1, 1))
        oracle.lfm_lm_head_q4_affine(wq, s, b, x, n, k)

    step_bytes = sum(q4_bytes(1, n_, k_) for _, k_, n_ in QWEN_SHAPES)
    med, reps = _median_time(warm_pass, 6.0)
    legs = {}
    cmed, creps = _median_time(cold_pass, 4.0, max_reps=20)
    legs["cfg2_q4_affine_step_cold"] = {"ms": round(cmed * 1e3, 3), "GB/s": round(step_bytes / cmed / 1e9, 3),
                                        "reps": creps}
    for n1 in (576, 1536):
        k1 = 576
        w8 = rng.integers(-127, 128, (n1, k1), dtype=np.int8)
        s8 = rng.uniform(1e-3, 2e-2, n1).astype(np.float32)
        x8 = rng.normal(size=(1, k1)).astype(np.float32)
        t, r = _median_time(lambda: oracle.qgemv_i8(w8, s8, x8), 1.0)
        legs[f"cfg1_i8_576x{n1}"] = {"us": round(t * 1e6, 2), "GB/s": round(i8_bytes(1, n1, k1, 4) / t / 1e9, 3),
                                     "reps": r}
    kg, ng = 1152, 262144
    wg = rng.integers(-127, 128, (ng, kg), dtype=np.int8)
    sg = rng.uniform(1e-3, 2e-2, ng).astype(np.float32)
    xg = rng.normal(size=(1, kg)).astype(np.float16)
    t, r = _median_time(lambda: oracle.qgemv_i8(wg, sg, xg), 3.0, max_reps=20)
    legs["cfg3_i8_lm_head_1152x262144_m1"] = {"ms": round(t * 1e3, 3),
                                              "GB/s": round(i8_bytes(1, ng, kg, 2) / t / 1e9, 3), "reps": r}
    del wg
    for k4, n4 in ((896, 4864), (4864, 896)):
        wq4, s4, b4 = q4(n4, k4)
        w32t = np.ascontiguousarray(oracle.q4_affine_dequant_f32(wq4, s4, b4, k4).T)  # [K, N] as matmul_f32 takes b
        a = rng.normal(size=(512, k4)).astype(np.float32)
        out = np.zeros((512, n4), np.float32)

        def gemm():
            out.fill(0.0)
            oracle.matmul_f32(a, w32t, out)

        t, r = _median_time(gemm, 3.0, max_reps=10)
        legs[f"cfg4_matmul_f32_m512_{k4}x{n4}"] = {"ms": round(t * 1e3, 3),
                                                  "GFLOP/s": round(2.0 * 512 * n4 * k4 / t / 1e9, 2), "reps": r}
    return {"value": round(step_bytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "ms_per_step": round(med * 1e3, 3), "cpu_model": _cpu_model(), "nproc": os.cpu_count(),
            "sample": f"{reps} decode passes over the 5 configs[1] projections (4 warm f32-cache GEMVs + "
                      "on-the-fly affine lm_head, lfm.rs:700-741,1056-1063), median; C oracle, OpenMP over rows; "
                      "legs: medians of the named reference paths at their full sizes",
            "legs": legs}


if __name__ == "__main__":
    main()
