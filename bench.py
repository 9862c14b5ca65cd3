#!/usr/bin/env python3
"""Benchmark of the W4A8 projection path on one MI355X.

Headline: decode MLP gate+up, M=8 tokens, K=5120,
N=2x17408, G=128, BF16 out -> achieved HBM GB/s. A step is one fan-out
projection launch (both weights) over resident int8 activations, as in the
reference's own GEMM/GEMV benches (kernels_dpas.cpp:2146-2195, quantization
outside the timer). The other BASELINE configs are measured the same way and
reported under "configs".

Timing: `steps` launches are captured into one HIP graph (torch's capture on
the stream the library launches on) and replayed once between two
synchronizations, so the timed region is back-to-back kernels; the launches
rotate over weight copies totalling > 512 MB so the 256 MB Infinity Cache
cannot serve them. HIP events on that stream bracket the replay; the kernel's
average duration is that time / steps. The cpu_baseline leg times the CPU
oracle (a scalar C++ restatement of the reference arithmetic, OpenMP over
output rows) on the host cores.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, public spec
INT8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA, public spec
MALL_BYTES = 256 << 20
QUANT_STEPS = 200            # graph-replayed launches per quantizer timing


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def setup(cfg, seed=0):
    import torch
    from knivesysl_xe_amd import ops, workloads
    inp = workloads.generate(cfg, seed)
    ws = []
    for c, s in zip(inp.codes, inp.scales):
        ws.append(ops.W4Weight.from_codes(torch.from_numpy(c).cuda(),
                                          torch.from_numpy(s.view(np.int16)).cuda(), cfg.group))
    x = torch.from_numpy(inp.x_bf16.view(np.int16)).cuda().view(torch.bfloat16)
    act = ops.quantize_act(x, 0)
    torch.cuda.synchronize()
    return inp, ws, x, act


def make_copies(ws, min_bytes=2 * MALL_BYTES + (64 << 20)):
    per = sum(w.codes.numel() + 2 * w.scales.numel() for w in ws)
    n = max(2, math.ceil(min_bytes / per))
    copies = [ws]
    for _ in range(n - 1):
        copies.append([type(w)(w.M, w.K, w.group, w.scale_enc, w.codes.clone(), w.scales.clone())
                       for w in ws])
    return copies, per * n


class launcher:
    """run(copy): one launch of the projection on weight copy `copy`. The
    argument checks and marshalling of each copy are done once, by prepare()
    or on the copy's first call (ops.PreparedGemv / PreparedGemmFanout), so a
    call is one C-ABI call."""

    def __init__(self, cfg, act, outs):
        import torch
        self.cfg, self.act, self.outs = cfg, act, outs
        self.dt = torch.bfloat16 if cfg.out_bf16 else torch.float32
        self.calls = {}

    def prepare(self, copies):
        from knivesysl_xe_amd import ops
        for w in copies:
            if id(w) not in self.calls:
                self.calls[id(w)] = (
                    ops.PreparedGemv(w[0], self.act, self.dt, out=self.outs[0]) if self.cfg.kind == "gemv"
                    else ops.PreparedGemmFanout(w, self.act, self.dt, offsets=self.cfg.offsets, outs=self.outs))

    def __call__(self, w):
        if id(w) not in self.calls:
            self.prepare([w])
        self.calls[id(w)]()


WARM_MS = 20.0      # warm-up GPU time before a timed region (the shader clock's ramp)
# Timed regions of up to EAGER_TIMED_MAX launches (the driver's
# `--steps 20`) are issued one by one behind a hold kernel (ops.probe_hold,
# nvbench's blocking kernel), enqueued after the pre-timing synchronize: one
# wave polls a host-pinned flag that the host sets once it has submitted the
# timed launches, so the start event is stamped with all of them queued.
# Without it the host's submission sometimes lands inside the timed region
# (the headline's 20 launches in one graph replay read 18.9-20.8 us, behind
# the hold 18.4-18.5 us), and a graph replay carries ~10 us of its own on
# the device, which 20 launches share. Longer regions replay one graph right
# after the synchronize: their submission is a small part of the region,
# while a hold idles the GPU for the whole submission (under rocprofv3 ~10
# ms per replay, which lowered the clock the GEMM lines then started on).
# The hold times out after HOLD_MAX_US; the JSON line says whether the flag
# released it.
HOLD_MAX_US = 20000
EAGER_TIMED_MAX = 32


def time_graph(run, copies, steps, warmup, settle_ms=0.0, info=None):
    """Time `steps` launches between HIP events after a synchronize: one
    graph replay, or up to EAGER_TIMED_MAX launches issued one by one behind
    the hold kernel. The `warmup` launches run as one graph
    replay before the synchronize. With warmup=None the warm-up graph holds
    about WARM_MS of launches, sized from a replay of 10 (the clock ramps up
    over the first milliseconds of load, so a fixed small count under-warms
    short kernels). settle_ms > 0 runs about that much GPU time of untimed
    launches of the same kernel right before the `warmup` launches (their
    count goes to info["settle_launches"]), so that a short explicit warm-up
    does not start the timed launches on a clock that is still ramping.
    info["hold_released"] says whether the host's flag, not the time-out,
    ended the hold before the timed launches."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(3):
            run(copies[i % len(copies)])
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()

    def capture(n, offset):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n):
                run(copies[(offset + i) % len(copies)])
        return g

    if warmup is None:
        g10 = capture(10, 0)
        g10.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g10.replay()
        e1.record()
        torch.cuda.synchronize()
        per_ms = max(e0.elapsed_time(e1) / 10, 1e-3)
        warmup = int(min(max(WARM_MS / per_ms, 20), 20000))
        del g10
    eager = steps <= EAGER_TIMED_MAX
    gw = capture(max(warmup, 1), 0)
    gt = None if eager else capture(steps, max(warmup, 1))
    torch.cuda.synchronize()
    if settle_ms > 0:
        g10 = capture(10, 0)
        g10.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g10.replay()
        e1.record()
        torch.cuda.synchronize()
        reps = int(min(max(settle_ms / max(e0.elapsed_time(e1), 1e-3), 1), 2000))
        for _ in range(reps):
            g10.replay()
        if info is not None:
            info["settle_launches"] = 10 * (reps + 2)
    gw.replay()
    torch.cuda.synchronize()
    from knivesysl_xe_amd import ops
    flag = torch.zeros(1, dtype=torch.int32, pin_memory=True)
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    if eager:
        ops.probe_hold(flag, HOLD_MAX_US, status)
    e0.record()
    try:
        if eager:
            for i in range(steps):
                run(copies[(max(warmup, 1) + i) % len(copies)])
        else:
            gt.replay()
        e1.record()
    finally:
        flag.fill_(1)                                   # release the hold
    submit = time.perf_counter() - t0
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    if info is not None:
        info["submit_us"] = submit * 1e6
        if eager:
            info["hold_released"] = int(status.item()) == 1
    return e0.elapsed_time(e1) / 1e3, wall


def check_against_oracle(cfg, inp, outs, rows=512):
    """Bit-exact spot check of the benchmarked outputs on a row subset."""
    import torch
    from oracle import oracle as O
    from knivesysl_xe_amd import workloads
    q, s, sm = O.quantize_act(workloads.bf16_bits_to_f32(inp.x_bf16), 0)
    for c, sc, y in zip(inp.codes, inp.scales, outs):
        N = c.shape[0]
        if cfg.kind == "gemv":
            variant, sp = O.VAR_GEMV, O.gemv_splits(N // 16)
        else:
            variant, sp = O.VAR_GEMM, O.segment_splits(cfg.tokens, N, cfg.K, cfg.offsets)
        r = min(rows, N)
        ref = O.project(c, sc, cfg.group, 0, q, s, sm, 0, variant, sp, out_bf16=cfg.out_bf16,
                        rows=(0, r))
        got = y[:, :r]
        got = got.view(torch.int16).cpu().numpy().view(np.uint16) if cfg.out_bf16 \
            else got.cpu().numpy().view(np.uint32)
        if not np.array_equal(got, ref[:, :r].view(got.dtype)):
            return False
    return True


def time_eager(run, copies, steps, warmup):
    """Back-to-back eager launches bracketed by events on the launch stream
    (for counter collection, which wants one dispatch per launch)."""
    import torch
    for i in range(max(warmup, 1)):
        run(copies[i % len(copies)])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for i in range(steps):
        run(copies[(warmup + i) % len(copies)])
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3, time.perf_counter() - t0


def measure(cfg, steps, warmup, eager=False, settle_ms=0.0):
    import torch
    inp, ws, x, act = setup(cfg)
    dt = torch.bfloat16 if cfg.out_bf16 else torch.float32
    outs = [torch.empty(cfg.tokens, w.M, dtype=dt, device="cuda") for w in ws]
    run = launcher(cfg, act, outs)
    copies, rot_bytes = make_copies(ws)
    run.prepare(copies)
    info = {}
    if eager:
        secs, wall = time_eager(run, copies, steps, warmup)
    else:
        secs, wall = time_graph(run, copies, steps, warmup, settle_ms, info)
    run(copies[0])
    torch.cuda.synchronize()
    exact = check_against_oracle(cfg, inp, outs)
    # activation quantization, timed on its own for reference (graph replay
    # of QUANT_STEPS launches into one reused output, like the projection;
    # with few launches the replay's start-up dominates a few-us kernel)
    from knivesysl_xe_amd import ops
    qa = ops.QuantAct.empty(cfg.tokens, cfg.K, 0)
    qsecs, _ = time_graph(lambda _c: ops.quantize_act(x, 0, out=qa), [None], QUANT_STEPS, None)
    quant_us = qsecs / QUANT_STEPS * 1e6
    per = secs / steps
    res = {
        "kernel_us": per * 1e6,
        "GBps": cfg.algorithmic_bytes() / per / 1e9,
        "TOPS": cfg.ops() / per / 1e12,
        "bytes": cfg.algorithmic_bytes(),
        "ops": cfg.ops(),
        "bound": cfg.bound,
        "bit_exact_vs_oracle_rows0_512": exact,
        "rotated_weight_bytes": rot_bytes,
        "quantize_us": quant_us,
        "wall_s": wall,
    }
    for k in ("settle_launches", "hold_released", "submit_us"):
        if k in info:
            res[k] = info[k]
    res["roofline_frac"] = (res["GBps"] / HBM_PEAK_GBS if cfg.bound == "hbm"
                            else res["TOPS"] / INT8_PEAK_TOPS)
    del copies, ws, outs
    torch.cuda.empty_cache()
    return res


def measure_w4a4(cfg, steps, warmup, eager=False):
    """The W4A4 GEMM (x_gemm_w4a4, the reference's default prefill dispatch for
    K64 weights) on a K64 config's shape: the config's codes, its FP16 scales
    with the low nibble replaced by a seeded zero point (FP16|zp encoding),
    and its BF16 activations quantized to s4 outside the timed region."""
    import torch
    from knivesysl_xe_amd import ops, workloads
    from oracle import oracle as O
    assert cfg.group == 64 and len(cfg.rows) == 1 and not cfg.segments
    inp = workloads.generate(cfg, 0)
    rng = np.random.default_rng(1)
    codes = inp.codes[0]
    scales = ((inp.scales[0] & 0xFFF0) | (rng.integers(-8, 8, inp.scales[0].shape) & 0xF)).astype(np.uint16)
    w = ops.W4Weight.from_codes(torch.from_numpy(codes).cuda(),
                                torch.from_numpy(scales.view(np.int16)).cuda(), 64, O.SCALE_FP16_ZP4)
    x = torch.from_numpy(inp.x_bf16.view(np.int16)).cuda().view(torch.bfloat16)
    act = ops.quantize_act_s4(x)
    dt = torch.bfloat16 if cfg.out_bf16 else torch.float32
    out = torch.empty(cfg.tokens, w.M, dtype=dt, device="cuda")
    copies, rot_bytes = make_copies([w])
    run = lambda ws: ops.gemm_w4a4(ws[0], act, dt, out=out)
    secs, wall = (time_eager if eager else time_graph)(run, copies, steps, warmup)
    run(copies[0])
    torch.cuda.synchronize()
    q, s, sm = O.quantize_act_s4(workloads.bf16_bits_to_f32(inp.x_bf16))
    ref = O.project(codes, scales, 64, O.SCALE_FP16_ZP4, q, s, sm, 64, O.VAR_GEMM, 1,
                    out_bf16=cfg.out_bf16, rows=(0, 512))
    got = out[:, :512]
    got = got.view(torch.int16).cpu().numpy().view(np.uint16) if cfg.out_bf16 \
        else got.cpu().numpy().view(np.uint32)
    exact = bool(np.array_equal(got, ref[:, :512].view(got.dtype)))
    qa = ops.QuantActS4.empty(cfg.tokens, cfg.K)
    qsecs, _ = time_graph(lambda _c: ops.quantize_act_s4(x, out=qa), [None], QUANT_STEPS, None)
    per = secs / steps
    N = sum(cfg.rows)
    res = {
        "kernel_us": per * 1e6,
        "TOPS": cfg.ops() / per / 1e12,
        "ops": cfg.ops(),
        "bound": "mfma",
        "bit_exact_vs_oracle_rows0_512": exact,
        "rotated_weight_bytes": rot_bytes,
        "quantize_s4_us": qsecs / QUANT_STEPS * 1e6,
        "bytes": N * cfg.K // 2 + N * (cfg.K // 64) * 2 + cfg.tokens * cfg.K // 2 + cfg.tokens * N * 4,
        "wall_s": wall,
    }
    res["GBps"] = res["bytes"] / per / 1e9
    res["roofline_frac"] = res["TOPS"] / INT8_PEAK_TOPS
    del copies, w, out
    torch.cuda.empty_cache()
    return res


REFMODE_GROUPS = {"cfg3": 32, "cfg2_m512": 64,   # the reference's K32 / K64 weight tiers
                  "cfg1": 32, "cfg2_m1": 64}


def measure_refmode(cfg, steps, warmup, eager=False, general=False):
    """x_gemv_w4a8 / x_gemm_w4a8 as the reference runs them on a config's
    shape: the config's codes with FP16|zp scales at the reference's weight
    group (K32 for cfg3 and the cfg1 gate/up pair, K64 for the cfg2 down
    projection: |N(0,1)| * 0.02 rounded to FP16, the low nibble replaced by
    a seeded zero point in [-8, 7]), and its BF16 activations quantized per
    (token, K32 block) outside the timed region (x_quantize_act_chunk).
    general=True times the general GEMM kernel on the same inputs (GEMM
    shapes only)."""
    import torch
    from knivesysl_xe_amd import ops, workloads
    from oracle import oracle as O
    assert not cfg.segments
    group = REFMODE_GROUPS[cfg.name]
    inp = workloads.generate(cfg, 0)
    rng = np.random.default_rng(2)
    K, T = cfg.K, cfg.tokens
    ws, scs = [], []
    for codes, N in zip(inp.codes, cfg.rows):
        mags = (np.abs(rng.standard_normal((N, K // group), dtype=np.float32)) * np.float32(0.02))
        scales = ((mags.astype(np.float16).view(np.uint16) & 0xFFF0)
                  | (rng.integers(-8, 8, (N, K // group)) & 0xF)).astype(np.uint16)
        scs.append(scales)
        ws.append(ops.W4Weight.from_codes(torch.from_numpy(codes).cuda(),
                                          torch.from_numpy(scales.view(np.int16)).cuda(), group,
                                          O.SCALE_FP16_ZP4))
    x = torch.from_numpy(inp.x_bf16.view(np.int16)).cuda().view(torch.bfloat16)
    act = ops.quantize_act(x, 32)
    dt = torch.bfloat16 if cfg.out_bf16 else torch.float32
    outs = [torch.empty(T, N, dtype=dt, device="cuda") for N in cfg.rows]
    copies, rot_bytes = make_copies(ws)
    if cfg.kind == "gemv":
        run = lambda wc: ops.gemv(wc[0], act, dt, out=outs[0])
    else:
        run = lambda wc: ops.gemm_fanout(wc, act, dt, outs=outs)
    with ops.option("gemm_kernel", 1 if general else 0):
        secs, wall = (time_eager if eager else time_graph)(run, copies, steps, warmup)
        run(copies[0])
    torch.cuda.synchronize()
    q, s, sm = O.quantize_act(workloads.bf16_bits_to_f32(inp.x_bf16), 32)
    exact = True
    for codes, scales, N, y in zip(inp.codes, scs, cfg.rows, outs):
        if cfg.kind == "gemv":
            variant, sp = O.VAR_GEMV, O.gemv_splits(N // 16)
        else:
            variant, sp = O.VAR_GEMM, O.segment_splits(T, N, K)
        ref = O.project(codes, scales, group, O.SCALE_FP16_ZP4, q, s, sm, 32, variant, sp,
                        out_bf16=cfg.out_bf16, rows=(0, 512))
        got = y[:, :512]
        got = got.view(torch.int16).cpu().numpy().view(np.uint16) if cfg.out_bf16 \
            else got.cpu().numpy().view(np.uint32)
        exact = exact and bool(np.array_equal(got, ref[:, :512].view(got.dtype)))
    per = secs / steps
    NS = sum(cfg.rows)
    hbm = cfg.bound == "hbm"
    res = {
        "kernel_us": per * 1e6,
        "TOPS": cfg.ops() / per / 1e12,
        "ops": cfg.ops(),
        "bound": cfg.bound,
        "bit_exact_vs_oracle_rows0_512": exact,
        "rotated_weight_bytes": rot_bytes,
        # codes, FP16|zp scales, activation input (BF16 for decode, as the
        # per-token lines count it; int8 codes and K32 scales for prefill)
        # and output
        "bytes": NS * K // 2 + NS * (K // group) * 2
                 + (T * K * 2 if hbm else T * K + T * (K // 32) * 4)
                 + T * NS * (2 if cfg.out_bf16 else 4),
        "wall_s": wall,
        "shape": f"T={T}, K={K}, N={'+'.join(str(n) for n in cfg.rows)}, FP16|zp group {group}, "
                 "K32 activation blocks" + (" (general GEMM kernel)" if general else ""),
    }
    res["GBps"] = res["bytes"] / per / 1e9
    res["roofline_frac"] = res["GBps"] / HBM_PEAK_GBS if hbm else res["TOPS"] / INT8_PEAK_TOPS
    del copies, ws, outs
    torch.cuda.empty_cache()
    return res


def measure_k16(steps, warmup, eager=False, rows=5120, K=17408, T=1):
    """The K16 tier (x_gemv_w4a8_core_k16, kernels_dpas.cpp:683-760) on the
    down projection's shape: seeded int4 codes uniform in [-8, 7], one FP16|zp
    scale per (row, K16 half) (|N(0,1)| * 0.02, the low nibble a zero point in
    [-8, 7]), BF16 N(0,1) activations quantized per (token, K32) outside the
    timed region; the default split plan. HBM-bound: codes + scales stream
    once per launch."""
    import torch
    from knivesysl_xe_amd import ops, workloads
    from oracle import oracle as O
    rng = np.random.default_rng(3)
    codes = rng.integers(-8, 8, (rows, K), dtype=np.int8)
    mags = (np.abs(rng.standard_normal((rows, K // 16), dtype=np.float32)) * np.float32(0.02))
    scales = ((mags.astype(np.float16).view(np.uint16) & 0xFFF0)
              | (rng.integers(-8, 8, (rows, K // 16)) & 0xF)).astype(np.uint16)
    w = ops.W4Weight.from_codes(torch.from_numpy(codes).cuda(),
                                torch.from_numpy(scales.view(np.int16)).cuda(), 16, O.SCALE_FP16_ZP4)
    xb = workloads.f32_to_bf16_bits(rng.standard_normal((T, K), dtype=np.float32))
    x = torch.from_numpy(xb.view(np.int16)).cuda().view(torch.bfloat16)
    act = ops.quantize_act(x, 32)
    out = torch.empty(T, rows, dtype=torch.float32, device="cuda")
    copies, rot_bytes = make_copies([w])
    run = lambda ws: ops.gemv(ws[0], act, torch.float32, out=out)
    secs, wall = (time_eager if eager else time_graph)(run, copies, steps, warmup)
    run(copies[0])
    torch.cuda.synchronize()
    q, s, sm = O.quantize_act(workloads.bf16_bits_to_f32(xb), 32)
    ref = O.project(codes, scales, 16, O.SCALE_FP16_ZP4, q, s, sm, 32, O.VAR_GEMV,
                    O.gemv_splits(rows // 16), rows=(0, 512))
    exact = bool(np.array_equal(out[:, :512].cpu().numpy().view(np.uint32), ref[:, :512].view(np.uint32)))
    per = secs / steps
    nbytes = rows * K // 2 + rows * (K // 16) * 2 + T * K * 2 + T * rows * 4
    res = {
        "kernel_us": per * 1e6,
        "GBps": nbytes / per / 1e9,
        "TOPS": 2 * T * rows * K / per / 1e12,
        "bytes": nbytes,
        "bound": "hbm",
        "bit_exact_vs_oracle_rows0_512": exact,
        "rotated_weight_bytes": rot_bytes,
        "wall_s": wall,
        "shape": f"T={T}, K={K}, N={rows}, FP16|zp per K16 half (the down projection)",
    }
    res["roofline_frac"] = res["GBps"] / HBM_PEAK_GBS
    del copies, w, out
    torch.cuda.empty_cache()
    return res


LM_HEAD_ROWS = 248320        # ~1.27 GB of int8 codes at K = 5120 (kernels_dpas.cpp:1576-1577)


def measure_w8a8(steps, warmup, eager=False, rows=LM_HEAD_ROWS, K=5120, T=8):
    """The W8A8 tier on its reference use: x_gemm_w8a8 over the spec wave's 8
    rows against an lm_head-sized int8 weight (decode.cpp:2335-2342), seeded
    synthetic codes (int8 uniform) and FP16 scales |N(0,1)| * 0.002, BF16
    N(0,1) activations quantized per (token, K32) outside the timed region.
    HBM-bound: the weight streams once per launch."""
    import torch
    from knivesysl_xe_amd import ops
    from oracle import oracle as O
    g = torch.Generator(device="cuda").manual_seed(0)
    codes = torch.randint(-128, 128, (rows, K), dtype=torch.int8, device="cuda", generator=g)
    scales = (torch.randn(rows, K // 32, device="cuda", generator=g).abs() * 0.002).half().view(torch.int16)
    w = ops.W4Weight.from_codes_s8(codes, scales)
    x = torch.randn(T, K, device="cuda", generator=g).bfloat16()
    act = ops.quantize_act(x, 32)
    out = torch.empty(T, rows, dtype=torch.float32, device="cuda")
    copies, rot_bytes = make_copies([w])
    run = lambda ws: ops.gemm(ws[0], act, torch.float32, forced_splits=1, out=out)
    secs, wall = (time_eager if eager else time_graph)(run, copies, steps, warmup)
    run(copies[0])
    torch.cuda.synchronize()
    c = codes[:512].cpu().numpy()
    sc = scales[:512].cpu().numpy().view(np.uint16)
    q, s, sm = O.quantize_act(x.float().cpu().numpy(), 32)
    ref = O.project(c, sc, 32, O.SCALE_S8, q, s, sm, 32, O.VAR_GEMM, 1)
    exact = bool(np.array_equal(out[:, :512].cpu().numpy().view(np.uint32), ref.view(np.uint32)))
    per = secs / steps
    nbytes = rows * K + rows * (K // 32) * 2 + T * K + T * rows * 4
    res = {
        "kernel_us": per * 1e6,
        "GBps": nbytes / per / 1e9,
        "TOPS": 2 * T * rows * K / per / 1e12,
        "bytes": nbytes,
        "bound": "hbm",
        "bit_exact_vs_oracle_rows0_512": exact,
        "rotated_weight_bytes": rot_bytes,
        "wall_s": wall,
        "shape": f"T={T} (spec wave), K={K}, N={rows} int8 (lm_head)",
    }
    res["roofline_frac"] = res["GBps"] / HBM_PEAK_GBS
    del copies, w, out, codes
    torch.cuda.empty_cache()
    return res


def cpu_info():
    """CPU model name, the host's logical CPUs and those this process may use."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count()
    return model, os.cpu_count(), usable


def cpu_time_config(cfg, budget_s):
    """The oracle on the host cores for one config: whole weights for the
    decode shapes, else a row subset sized so a pass takes about a tenth of
    the budget; one warm-up pass, then timed passes until the budget is spent;
    the median pass gives GB/s and GOPS of that subset's algorithmic work
    (codes + scales of the rows, all activations, the rows' outputs)."""
    from oracle import oracle as O
    from knivesysl_xe_amd import workloads
    inp = workloads.generate(cfg, 0)
    q, s, sm = O.quantize_act(workloads.bf16_bits_to_f32(inp.x_bf16), 0)
    splits = [O.segment_splits(cfg.tokens, c.shape[0], cfg.K, cfg.offsets) for c in inp.codes]

    def one_pass(rows):
        t0 = time.perf_counter()
        for c, sc, sp in zip(inp.codes, inp.scales, splits):
            r = min(rows, c.shape[0])
            O.project(c, sc, cfg.group, 0, q, s, sm, 0, O.VAR_GEMM, sp, out_bf16=cfg.out_bf16,
                      rows=(0, r))
        return time.perf_counter() - t0

    M = max(c.shape[0] for c in inp.codes)
    if cfg.tokens <= 16:
        rows = M                                         # decode shapes: whole weights
        one_pass(rows)                                   # warm-up
    else:
        rows = min(M, 256)
        t = one_pass(rows)                               # warm-up and calibration
        rows = int(min(M, max(16, rows * (budget_s / 10) / max(t, 1e-6))) // 16 * 16) or 16
    times = []
    t_end = time.perf_counter() + budget_s
    while not times or (time.perf_counter() < t_end and len(times) < 50):
        times.append(one_pass(rows))
    per = float(np.median(times))
    nr = sum(min(rows, c.shape[0]) for c in inp.codes)
    nbytes = nr * cfg.K // 2 + nr * (cfg.K // cfg.group) * 2 + cfg.tokens * cfg.K * 2 + \
        cfg.tokens * nr * (2 if cfg.out_bf16 else 4)
    ops = 2 * cfg.tokens * nr * cfg.K
    return {"GBps": nbytes / per / 1e9, "GOPS": ops / per / 1e9, "rows": nr,
            "rows_total": sum(c.shape[0] for c in inp.codes), "passes": len(times),
            "s_per_pass": per}


def cpu_baseline(head, names, budget_s=3.0):
    """The oracle (scalar C++ restatement of the reference arithmetic, OpenMP
    over output rows) on the host cores for the headline and each config."""
    from oracle import oracle as O
    from knivesysl_xe_amd import workloads
    O.build()
    model, nproc, usable = cpu_info()
    per = {}
    for name in dict.fromkeys(["cfg1"] + list(names)):
        per[name] = cpu_time_config(workloads.CONFIGS[name], budget_s)
        log(f"cpu {name}: {per[name]['GBps']:.2f} GB/s, {per[name]['GOPS']:.1f} GOPS "
            f"({per[name]['rows']}/{per[name]['rows_total']} rows, {per[name]['passes']} passes)")
    h = per["cfg1"]
    return {"value": h["GBps"], "unit": "GB/s", "cores": O.num_threads(), "kind": "port",
            "sample": f"cfg1 whole weights (both, all 8 tokens), median of {h['passes']} passes; "
                      "other configs on the row subsets listed; scalar C++ oracle, OpenMP over "
                      "output rows",
            "cpu_model": model, "nproc": nproc, "usable_cpus": usable,
            "configs": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                        for k, v in per.items()}}


def calibration_copy(mib):
    """A device-to-device copy of `mib` MiB: the known-size kernel the
    FETCH_SIZE / WRITE_SIZE counters are calibrated against."""
    import torch
    src = torch.empty(mib << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"calibration copy: 3 x {mib} MiB")


def machine_probes(head_bytes):
    """Measured ceilings, the MI355X counterpart of the reference's
    xpu/probe/dpas_probe.cpp (DPAS rates with all-ones operands, pure read;
    xpu/PROBE_RESULTS.md:8-33): the int8 MFMA rate of both MFMA shapes, with
    the all-ones check, and the pure HBM read rate over a 2 GiB buffer and
    over slices of the headline's byte count rotated through it."""
    import torch
    from knivesysl_xe_amd import ops
    sink = torch.empty(ops.PROBE_SINK_WORDS, dtype=torch.int32, device="cuda")
    out = {}

    def timed(fn, reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(reps):
            fn(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3 / reps

    for shape, name, k, iters in ((0, "mfma_i8_32x32x32", 32, 20000), (1, "mfma_i8_16x16x64", 64, 40000)):
        ops.probe_mfma_i8(shape, 100, sink)
        res = {}
        secs = timed(lambda _i: res.update(zip(("n", "ops"), ops.probe_mfma_i8(shape, iters, sink))), 3)
        out[f"{name}_TOPS"] = res["ops"] / secs / 1e12
        out[f"{name}_check"] = bool((sink[:res["n"]] == iters * k).all().item())
    # issue mix of the GEMM's inner work: ns per block per SIMD for MFMA only,
    # the FP32 chain only, both in one wave, both in separate waves
    fsink = torch.empty(ops.PROBE_SINK_WORDS, dtype=torch.float32, device="cuda")
    names = ("mfma", "chain", "mfma_chain_same_wave", "mfma_chain_split_waves")
    for mode, wps in ((0, 1), (0, 2), (1, 2), (1, 4), (2, 1), (2, 2), (2, 4), (3, 2), (3, 4)):
        ops.probe_issue(mode, wps, 10, fsink)
        res = {}
        secs = timed(lambda _i: res.update(blocks=ops.probe_issue(mode, wps, 4000, fsink)[1]), 3)
        out[f"issue_{names[mode]}_w{wps}_ns_per_block"] = secs / res["blocks"] * 1e9
    buf = torch.empty(2 << 30, dtype=torch.uint8, device="cuda").fill_(1)
    n = (head_bytes + 4095) // 4096 * 4096
    slices = [buf[i * n:(i + 1) * n] for i in range(buf.numel() // n)]
    best_full, best_head = (0.0, -1), (0.0, -1)
    for shape in range(ops.probe_read_shapes()):
        ops.probe_read(buf, sink, shape)
        secs = timed(lambda _i: ops.probe_read(buf, sink, shape), 5)
        best_full = max(best_full, (buf.numel() / secs / 1e9, shape))
        # the headline's byte count, timed like the headline: launches over
        # rotated slices captured in one graph and replayed between syncs
        secs, _ = time_graph(lambda sl: ops.probe_read(sl, sink, shape), slices, 2 * len(slices), 2)
        best_head = max(best_head, (n * 2 * len(slices) / secs / 1e9, shape))
    out["hbm_read_2GiB_GBps"], out["hbm_read_2GiB_shape"] = best_full
    out["hbm_read_headline_bytes_GBps"], out["hbm_read_headline_bytes_shape"] = best_head
    out["issue_sample"] = ("kxw4_probe_issue, one work-group per CU, 4000 iterations of 4 blocks per wave; "
                           "a block is 4 dependent v_mfma_i32_32x32x32_i8 and/or 16 cvt + 16 fma per lane")
    out["read_sample"] = (f"fastest of {ops.probe_read_shapes()} launch shapes; 2 GiB: 5 sweeps; headline "
                          f"bytes: {len(slices)} slices of {n} bytes rotated through 2 GiB, graph replay of "
                          f"{2 * len(slices)} launches as for the headline")
    del buf
    return out


def source_digest(files):
    """sha256 over the kernel sources a traffic figure was measured on."""
    import hashlib
    h = hashlib.sha256()
    for f in files:
        with open(os.path.join(ROOT, f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()


HEADLINE_SOURCES = ["knivesysl_xe_amd/csrc/kxw4_rowwave.hip", "knivesysl_xe_amd/csrc/kxw4_device.hpp",
                    "knivesysl_xe_amd/csrc/kxw4_internal.hpp"]


def read_traffic(name, sources):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if any:
    fetch_kib * fetch_cal + write_kib * write_cal, where each factor is the
    known size of a plain copy over what the same counter read for it. The
    summary names the sha256 of the kernel sources it was measured on; when
    they have changed since, the figure is stale and (None, reason) is
    returned instead."""
    path = os.path.join(ROOT, "profiles", f"traffic_{name}.txt")
    if not os.path.exists(path):
        return None, "no counter summary"
    vals = {}
    for line in open(path):
        if "=" in line and not line.lstrip().startswith("#"):
            k, v = line.split("=", 1)
            vals[k.strip()] = v.split()[0] if v.split() else ""
    if vals.get("source_sha256") != source_digest(sources):
        return None, "counter summary measured on other kernel sources"
    try:
        kib = float(vals["fetch_kib"]) * float(vals["fetch_cal"]) + float(vals["write_kib"]) * float(vals["write_cal"])
    except (KeyError, ValueError):
        return None, "counter summary incomplete"
    return int(kib * 1024), f"profiles/traffic_{name}.txt"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # (a 20 us launch: 1000 warmup launches are ~20 ms, long enough for the
    # shader clock to settle before the timed region; with 20 the timed
    # region started during the ramp and read up to 8% slow)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=1000)
    ap.add_argument("--configs", default="cfg0,cfg2_m1,cfg2_m512,cfg3,cfg4",
                    help="extra BASELINE configs to report ('' for none)")
    ap.add_argument("--w4a4", default="cfg2_m512",
                    help="K64 configs to also run through the W4A4 GEMM ('' for none)")
    ap.add_argument("--refmode", default="cfg1,cfg2_m1,cfg3,cfg2_m512",
                    help="configs to also run as x_gemv_w4a8 / x_gemm_w4a8 run them: FP16|zp "
                         "K32/K64 weights, K32 activation blocks ('' for none)")
    ap.add_argument("--refmode-general", action="store_true",
                    help="also time the reference-mode lines on the general GEMM kernel")
    ap.add_argument("--no-w8a8", action="store_true", help="skip the W8A8 lm_head line")
    ap.add_argument("--no-k16", action="store_true", help="skip the K16 down-projection GEMV line")
    ap.add_argument("--no-probes", action="store_true", help="skip the MFMA / HBM read probes")
    ap.add_argument("--extra-steps", type=int, default=200,
                    help="timed launches per extra config (each after ~20 ms of warm-up launches)")
    ap.add_argument("--cpu-budget", type=float, default=3.0,
                    help="seconds of CPU-baseline timing per config")
    ap.add_argument("--eager", action="store_true",
                    help="time eager launches instead of a graph replay (for counter runs)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="also run a device copy of this many MiB (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the projection would shard column-parallel over row-groups, or row-parallel "
              "over K with one all-reduce of the FP32 partials)", file=sys.stderr)
        sys.exit(2)

    import torch
    from knivesysl_xe_amd import workloads
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    head = workloads.CONFIGS["cfg1"]
    # The headline is timed last, after the other lines and the probes, so
    # that with a short warm-up (the driver's 5 launches) its timed region
    # does not start on an idle GPU (20 timed launches after 5 warm-up ones:
    # 19.89 us timed first in a process, 19.53 us after other GPU work).
    extra = {}
    for name in [c for c in args.configs.split(",") if c]:
        cfg = workloads.CONFIGS[name]
        log(f"{name}: {cfg.note}")
        extra[name] = measure(cfg, args.extra_steps, 5 if args.eager else None, args.eager)
        e = extra[name]
        log(f"{name}: {e['kernel_us']:.2f} us, {e['GBps']:.1f} GB/s, {e['TOPS']:.1f} TOPS, "
            f"frac {e['roofline_frac']:.3f}, exact={e['bit_exact_vs_oracle_rows0_512']}")
    for name in [c for c in args.w4a4.split(",") if c]:
        cfg = workloads.CONFIGS[name]
        log(f"{name}_w4a4: W4A4 GEMM on the {name} shape (s4 activations, FP16|zp K64 weight)")
        e = extra[f"{name}_w4a4"] = measure_w4a4(cfg, args.extra_steps, 5 if args.eager else None, args.eager)
        log(f"{name}_w4a4: {e['kernel_us']:.2f} us, {e['TOPS']:.1f} TOPS, frac {e['roofline_frac']:.3f}, "
            f"exact={e['bit_exact_vs_oracle_rows0_512']}")
    for name in [c for c in args.refmode.split(",") if c]:
        cfg = workloads.CONFIGS[name]
        for general in ((False, True) if args.refmode_general and cfg.kind != "gemv" else (False,)):
            key = f"{name}_ref" + ("_general" if general else "")
            fn = "x_gemv_w4a8" if cfg.kind == "gemv" else "x_gemm_w4a8"
            log(f"{key}: {fn} on the {name} shape (FP16|zp K{REFMODE_GROUPS[name]} weight, K32 blocks)")
            e = extra[key] = measure_refmode(cfg, args.extra_steps, 5 if args.eager else None, args.eager, general)
            log(f"{key}: {e['kernel_us']:.2f} us, {e['GBps']:.1f} GB/s, {e['TOPS']:.1f} TOPS, "
                f"frac {e['roofline_frac']:.3f}, exact={e['bit_exact_vs_oracle_rows0_512']}")
    if not args.no_w8a8:
        log("lm_head_w8a8: W8A8 GEMM, spec wave T=8, K=5120, N=248320 int8")
        e = extra["lm_head_w8a8"] = measure_w8a8(args.extra_steps, 3 if args.eager else None, args.eager)
        log(f"lm_head_w8a8: {e['kernel_us']:.2f} us, {e['GBps']:.1f} GB/s, frac {e['roofline_frac']:.3f}, "
            f"exact={e['bit_exact_vs_oracle_rows0_512']}")
    if not args.no_k16:
        log("down_k16: K16 GEMV, T=1, K=17408, N=5120, FP16|zp per K16 half")
        e = extra["down_k16"] = measure_k16(args.extra_steps, 3 if args.eager else None, args.eager)
        log(f"down_k16: {e['kernel_us']:.2f} us, {e['GBps']:.1f} GB/s, frac {e['roofline_frac']:.3f}, "
            f"exact={e['bit_exact_vs_oracle_rows0_512']}")
    probes = None
    if not args.no_probes:
        probes = machine_probes(int(head.algorithmic_bytes()))
        log(f"probes: MFMA i8 32x32x32 {probes['mfma_i8_32x32x32_TOPS']:.0f} TOPS "
            f"(check {probes['mfma_i8_32x32x32_check']}), 16x16x64 {probes['mfma_i8_16x16x64_TOPS']:.0f} TOPS "
            f"(check {probes['mfma_i8_16x16x64_check']}); read {probes['hbm_read_2GiB_GBps']:.0f} GB/s (2 GiB), "
            f"{probes['hbm_read_headline_bytes_GBps']:.0f} GB/s (headline bytes); ns per block per SIMD: "
            + ", ".join(f"{k[6:-13]} {v:.1f}" for k, v in probes.items() if k.startswith("issue_") and k.endswith("_ns_per_block")))
    log(f"headline {head.note}")
    # Before its `warmup` launches the headline kernel also runs ~WARM_MS of
    # untimed launches, as every other line does: after the driver's 5
    # warm-up launches alone its 20 timed launches read 19.5-19.9 us, with
    # the settle pass 19.2-19.4 us; issued one by one behind the hold kernel
    # they read as the 1000-launch replay does (~18.3-18.5 us).
    r = measure(head, args.steps, args.warmup, args.eager, settle_ms=WARM_MS)
    log(f"cfg1: {r['kernel_us']:.2f} us/launch, {r['GBps']:.1f} GB/s, exact={r['bit_exact_vs_oracle_rows0_512']}")
    if args.copy_mib:
        calibration_copy(args.copy_mib)
    log("cpu baseline (oracle on host cores)")
    cpu = cpu_baseline(head, ["cfg0", "cfg2_m1", "cfg2_m512", "cfg3", "cfg4"], args.cpu_budget)
    per = r["kernel_us"] / 1e6
    traffic, traffic_src = read_traffic("cfg1", HEADLINE_SOURCES)
    out = {
        "metric": "W4A8 GEMV HBM GB/s (M=1,8) + prefill GEMM int8 TOPS, % of MI355X roofline",
        "value": round(r["GBps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_launches": r.get("settle_launches"),
        "timing": "HIP events around the timed launches after a synchronize: up to 32 issued "
                  "one by one behind a kernel that holds the stream until the host has submitted "
                  "them; more as one graph replay",
        "hold_released": r.get("hold_released"),
        "ms_per_step": round(per * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic, seeded: int4 uniform [-8,7], FP16 |N(0,1)|*0.02 scales, "
                "BF16 N(0,1) activations quantized per token",
        "config": {"workload": "cfg1: decode MLP gate+up fan-out, M=8 tokens, K=5120, "
                               "N=2x17408, G=128, BF16 out",
                   "tokens": 8, "K": 5120, "N": 34816, "group": 128, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(r["GBps"], 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(r["GBps"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "traffic_source": traffic_src},
        "cpu_baseline": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in cpu.items()},
        "bit_exact_vs_oracle": r["bit_exact_vs_oracle_rows0_512"],
        "probes": None if probes is None else dict(
            {k: (round(v, 2) if isinstance(v, float) else v) for k, v in probes.items()},
            headline_frac_of_read_probe=round(r["GBps"] / probes["hbm_read_headline_bytes_GBps"], 4)),
        "quantize_us": round(r["quantize_us"], 2),
        "configs": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in extra.items()},
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
