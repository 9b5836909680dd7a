#!/usr/bin/env python3
"""bench.py -- k-quant linear path on one MI355X.

Headline ("C2"): Q4_K decode GEMV over the seven
Llama-3-8B projections of one decoder layer at batch 1 --
q 4096x4096, k 1024x4096, v 1024x4096, o 4096x4096, gate 14336x4096,
up 14336x4096, down 4096x14336 (out x in).  One step = one pass over the
seven projections of one layer copy, issued as an inference engine issues
them: q+k+v in one launch and gate+up in one launch (each group reads the same
activations; okq_gemv_multi), then o and down, which read activations produced
in between -- 4 launches.  Steps rotate over --copies distinct layer copies
(default 8 = 981 MB of quantized weights, beyond the 256 MB MALL) so weights
stream from HBM.  value = quantized weight bytes per step x steps / wall time of
the timed region, in GB/s; inputs are resident in HBM before timing starts.
Steps are replayed from HIP graphs so host launch overhead does not gate the
GPU.  The same steps as seven single-projection launches are reported in
extra.c2_sequential.

The JSON line also carries:
  roofline      the dominant kernel (the gate+up launch, 2 x 14336x4096 Q4_K,
                54% of the step's bytes): its quantized weight bytes / its
                average launch duration, measured with stream events around
                HIP-graph replays of back-to-back launches over >= 512 MB of
                weight replicas per matrix, vs 8 TB/s; `traffic` is the HBM
                bytes per launch from rocprofv3 FETCH_SIZE and WRITE_SIZE passes
                (profiles/gemv_q4k_gate_up_traffic.md)
  cpu_baseline  the reference CPU path (oracle restatement of
                linear_out_by_in, scalar mode, 1 core since rows < 32) on one
                layer copy, dequantized once outside the timing
  extra         per-launch and per-projection times, the 7-launch step, and
                the secondary configs (C1, C3, C4)

Run: python bench.py [--steps K] [--warmup W] [--copies C] [--no-cpu] ...
     python bench.py --probe gate_up|copy   (bare workload for counter passes)
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X datasheet HBM3E bandwidth
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16/fp16 MFMA
Q4K, Q6K, Q8_0 = 12, 14, 8
BLOCK = {Q4K: (256, 144), Q6K: (256, 210), Q8_0: (32, 34)}
C2_PROJ = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
           ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
METRIC = "Q4_K dequant-GEMV GB/s (% of HBM peak) + prefill dequant-GEMM TFLOPS"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def wbytes(t: int, n: int, k: int) -> int:
    e, b = BLOCK[t]
    return n * (k // e) * b


class Hip:
    """Minimal hipEvent access (the events passed to okq_set_launch_events)."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so")
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventSynchronize.argtypes = [ctypes.c_void_p]

    def event(self) -> int:
        e = ctypes.c_void_p()
        assert self.lib.hipEventCreate(ctypes.byref(e)) == 0
        return e.value

    def elapsed_ms(self, a: int, b: int) -> float:
        assert self.lib.hipEventSynchronize(b) == 0
        ms = ctypes.c_float()
        assert self.lib.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return ms.value

    def destroy(self, e: int) -> None:
        self.lib.hipEventDestroy(e)


class Ctx:
    def __init__(self, torch, okq):
        self.torch = torch
        self.okq = okq
        self.hip = Hip()
        self.tmp = None

    @property
    def stream(self) -> int:
        return self.torch.cuda.current_stream().cuda_stream

    def quantized(self, t: int, n: int, k: int, seed: int, sigma: float = 0.02):
        """Seeded N(0, sigma) weights quantized on the GPU (chunked through a
        reusable f32 scratch tensor)."""
        torch = self.torch
        out = torch.empty(wbytes(t, n, k), dtype=torch.uint8, device="cuda")
        e, b = BLOCK[t]
        total = n * k
        chunk = (1 << 26) // e * e
        if self.tmp is None or self.tmp.numel() < chunk:
            self.tmp = torch.empty(chunk, dtype=torch.float32, device="cuda")
        done = 0
        while done < total:
            m = min(chunk, total - done)
            self.okq.call("okq_fill_normal", seed, done, m, sigma, self.tmp.data_ptr(), self.stream)
            self.okq.call("okq_quantize", t, self.tmp.data_ptr(), m, out.data_ptr() + done // e * b, self.stream)
            done += m
        return out

    def normal(self, n: int, seed: int, sigma: float = 1.0):
        x = self.torch.empty(n, dtype=self.torch.float32, device="cuda")
        self.okq.call("okq_fill_normal", seed, 0, n, sigma, x.data_ptr(), self.stream)
        return x

    def gemv(self, t, x, k, w, n, y, entry="okq_gemv", rows=1):
        self.okq.call(entry, x.data_ptr(), rows, k, t, w.data_ptr(), w.numel(), n, None, y.data_ptr(), self.stream)

    def graph_us(self, launch, n: int, reps: int = 3) -> float:
        """Average duration (µs) of one launch inside a HIP graph of n
        back-to-back launch(i) calls, timed with events on the stream the graph
        is replayed on."""
        torch = self.torch
        launch(0)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n):
                launch(i)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        us = 1000.0 * e0.elapsed_time(e1) / (reps * n)
        del g
        return us

    def replicas(self, w, min_bytes: int = 512 << 20):
        """A pool of copies of w (>= min_bytes) so that rotating launches read
        HBM rather than the 256 MB MALL; returns (pool, copies)."""
        copies = max(2, -(-min_bytes // w.numel()))
        return w.repeat(copies), copies

    def kernel_us(self, launch, reps: int) -> list:
        """Per-launch dispatch duration (µs) of `reps` launches of launch(i)."""
        evs = [(self.hip.event(), self.hip.event()) for _ in range(reps)]
        try:
            for i, (a, b) in enumerate(evs):
                self.okq.call("okq_set_launch_events", a, b)
                launch(i)
        finally:
            self.okq.call("okq_set_launch_events", None, None)
        self.torch.cuda.synchronize()
        us = [1000.0 * self.hip.elapsed_ms(a, b) for a, b in evs]
        for a, b in evs:
            self.hip.destroy(a)
            self.hip.destroy(b)
        return us


def median(v):
    s = sorted(v)
    return s[len(s) // 2]


def pct(v, p):
    s = sorted(v)
    return s[min(len(s) - 1, max(0, int(round(p / 100.0 * (len(s) - 1)))))]


# ---------------------------------------------------------------------------
# C2 headline
# ---------------------------------------------------------------------------

# The launches of one decoder layer's projections as an inference engine
# issues them: projections that read the same activations share a launch
# (okq_gemv_multi); o and down read activations produced in between.
C2_GROUPS = [("qkv", ["q", "k", "v"]), ("o", ["o"]), ("gate_up", ["gate", "up"]), ("down", ["down"])]
C2_SHAPE = {name: (n, k) for name, n, k in C2_PROJ}


def launch_group(ctx, names, ws, x, outs):
    """One launch over the matrices `names` (weights ws[name]) against x."""
    n0, k = C2_SHAPE[names[0]]
    if len(names) == 1:
        w = ws[names[0]]
        ctx.okq.call("okq_gemv", x.data_ptr(), 1, k, Q4K, w.data_ptr(), w.numel(), n0, None,
                     outs[names[0]].data_ptr(), ctx.stream)
        return
    c = len(names)
    ctx.okq.call("okq_gemv_multi", x.data_ptr(), 1, k, Q4K, c,
                 (ctypes.c_void_p * c)(*[ws[m].data_ptr() for m in names]),
                 (ctypes.c_uint64 * c)(*[ws[m].numel() for m in names]),
                 (ctypes.c_int64 * c)(*[C2_SHAPE[m][0] for m in names]), None,
                 (ctypes.c_void_p * c)(*[outs[m].data_ptr() for m in names]), ctx.stream)


def time_steps(ctx, args, step):
    """Wall time of args.steps steps replayed from HIP graphs (one graph per
    pass over all layer copies, single-step graphs for the remainder)."""
    torch = ctx.torch
    step(0)
    torch.cuda.synchronize()
    g_all = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_all):
        for c in range(args.copies):
            step(c)
    g_one = []
    for c in range(args.copies):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step(c)
        g_one.append(g)

    def run_steps(nsteps, start=0):
        i = start
        while nsteps > 0:
            if i % args.copies == 0 and nsteps >= args.copies:
                g_all.replay()
                i += args.copies
                nsteps -= args.copies
            else:
                g_one[i % args.copies].replay()
                i += 1
                nsteps -= 1
        return i

    i = run_steps(args.warmup)
    i = i - i % args.copies  # restart on a copy boundary
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run_steps(args.steps, i)
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def run_c2(ctx: Ctx, args):
    torch = ctx.torch
    log(f"C2: generating {args.copies} Q4_K layer copies")
    layers = []
    for c in range(args.copies):
        layers.append({name: ctx.quantized(Q4K, n, k, seed=10_000 + 100 * c + i)
                       for i, (name, n, k) in enumerate(C2_PROJ)})
    x4096 = ctx.normal(4096, 1)
    x14336 = ctx.normal(14336, 2)
    outs = {name: torch.empty(n, dtype=torch.float32, device="cuda") for name, n, _ in C2_PROJ}
    step_bytes = sum(wbytes(Q4K, n, k) for _, n, k in C2_PROJ)

    def xin(names):
        return x14336 if C2_SHAPE[names[0]][1] == 14336 else x4096

    def step_fused(c):
        lay = layers[c % args.copies]
        for _, names in C2_GROUPS:
            launch_group(ctx, names, lay, xin(names), outs)

    def step_seq(c):
        lay = layers[c % args.copies]
        for name, n, k in C2_PROJ:
            ctx.gemv(Q4K, xin([name]), k, lay[name], n, outs[name])

    log(f"C2: warmup {args.warmup} steps, timing {args.steps} steps (4 launches per layer)")
    sec = time_steps(ctx, args, step_fused)
    log(f"C2: the same steps as 7 single-projection launches")
    sec_seq = time_steps(ctx, args, step_seq)

    # per-launch durations: graphs of back-to-back launches, each launch on the
    # next replica of the group's weights (>= 512 MB of replicas per matrix)
    def group_time(names):
        pools = {m: ctx.replicas(layers[0][m]) for m in names}
        copies = min(cp for _, cp in pools.values())
        x = xin(names)

        def launch(i):
            ws = {}
            for m in names:
                pool, _ = pools[m]
                b = wbytes(Q4K, *C2_SHAPE[m])
                ws[m] = pool.narrow(0, (i % copies) * b, b)
            launch_group(ctx, names, ws, x, outs)

        us = ctx.graph_us(launch, max(64, 2 * copies))
        b = sum(wbytes(Q4K, *C2_SHAPE[m]) for m in names)
        del pools
        return {"matrices": names, "weight_bytes": b, "us_mean": round(us, 3), "gbs": round(b / us / 1e3, 1),
                "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}

    launches = {g: group_time(names) for g, names in C2_GROUPS}
    shapes = {name: group_time([name]) for name, _, _ in C2_PROJ}
    return {"gbs": step_bytes * args.steps / sec / 1e9, "sec": sec,
            "gbs_sequential": step_bytes * args.steps / sec_seq / 1e9, "sec_sequential": sec_seq,
            "step_bytes": step_bytes, "launches": launches, "shapes": shapes, "layers": layers,
            "x4096": x4096, "x14336": x14336}


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_q4k_gate_up_traffic.md")


def measured_traffic():
    """HBM bytes per launch of the roofline kernel from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (line `traffic_bytes_per_launch:
    N`), or None when no such measurement is committed."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip().split()[0])
    except (OSError, ValueError):
        pass
    return None


def roofline_from(launches):
    # dominant kernel: the gate+up launch (two 14336 x 4096 Q4_K matrices, 54%
    # of the step's bytes; gemv_kernel<FQ4K, 2, 1, true, 0, 1, true>, an
    # instantiation no other launch of the step uses, so rocprof's per-kernel
    # average covers exactly these launches and C5's identical batch-1 ones)
    s = launches["gate_up"]
    achieved = s["weight_bytes"] / s["us_mean"] / 1e3
    return {"bound": "hbm", "kernel": "okq::gemv_kernel<okq::FQ4K, 2, 1, true, 0, 1, true> (C2 gate+up, 2 x 14336x4096 Q4_K)",
            "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
            "algorithmic_bytes_per_launch": s["weight_bytes"], "launch_us_mean": s["us_mean"]}


# ---------------------------------------------------------------------------
# secondary configs
# ---------------------------------------------------------------------------

def run_c3(ctx: Ctx, args):
    n, k = 128256, 4096
    log("C3: Q6_K head 128256x4096")
    w = ctx.quantized(Q6K, n, k, seed=31)
    x = ctx.normal(k, 32)
    y = ctx.torch.empty(n, dtype=ctx.torch.float32, device="cuda")
    b = wbytes(Q6K, n, k)
    pool, copies = ctx.replicas(w)
    del w

    def launch(i):
        ctx.okq.call("okq_gemv", x.data_ptr(), 1, k, Q6K, pool.data_ptr() + (i % copies) * b, b, n, None,
                     y.data_ptr(), ctx.stream)

    us = ctx.graph_us(launch, 16)
    del pool
    return {"shape": [n, k], "weight_bytes": b, "us_mean": round(us, 2),
            "gbs": round(b / us / 1e3, 1), "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}


def run_c1(ctx: Ctx, args):
    n, k = 4096, 4096
    log("C1: Q8_0 4096x4096 GEMV (GPU)")
    w = ctx.quantized(Q8_0, n, k, seed=40)
    x = ctx.normal(k, 41)
    y = ctx.torch.empty(n, dtype=ctx.torch.float32, device="cuda")
    b = wbytes(Q8_0, n, k)
    pool, copies = ctx.replicas(w)

    def launch(i):
        ctx.okq.call("okq_gemv", x.data_ptr(), 1, k, Q8_0, pool.data_ptr() + (i % copies) * b, b, n, None,
                     y.data_ptr(), ctx.stream)

    us = ctx.graph_us(launch, max(64, 2 * copies))
    del pool
    return {"shape": [n, k], "weight_bytes": b, "us_mean": round(us, 3),
            "gbs": round(b / us / 1e3, 1), "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}


def run_c4(ctx: Ctx, args, c2):
    """Q4_K prefill GEMM at M in {128, 512, 2048} with bf16 activations.
    us_kernel: the MFMA kernel's own dispatch time; us_call: the whole entry
    point (activation pre-pass + GEMM) timed with stream events."""
    torch = ctx.torch
    res = {}
    lay = c2["layers"]
    for m in (128, 512, 2048):
        log(f"C4: Q4_K GEMM M={m}")
        xf = ctx.normal(m * 14336, 50 + m)
        xb = torch.empty(m * 14336, dtype=torch.int16, device="cuda")
        ctx.okq.call("okq_f32_to_bf16", xf.data_ptr(), xf.numel(), xb.data_ptr(), ctx.stream)
        for name, n, k in C2_PROJ:
            if name in ("k", "o", "up"):
                continue  # same shapes as v, q, gate
            y = torch.empty(m * n, dtype=torch.float32, device="cuda")
            reps = max(8, args.kernel_reps // 8)

            def call(r, name=name, n=n, k=k, y=y):
                ctx.gemv(Q4K, xb, k, lay[r % len(lay)][name], n, y, entry="okq_gemm_bf16", rows=m)

            call(0)
            us = ctx.kernel_us(call, reps)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record()
            for r in range(reps):
                call(r)
            e1.record()
            torch.cuda.synchronize()
            t_call = 1000.0 * e0.elapsed_time(e1) / reps
            t = sum(us) / len(us)
            flops = 2.0 * m * n * k
            res[f"M{m}_{name}"] = {"m": m, "n": n, "k": k, "us_kernel": round(t, 2), "us_call": round(t_call, 2),
                                   "tflops": round(flops / t / 1e6, 1),
                                   "frac_bf16_peak": round(flops / t / 1e6 / BF16_PEAK_TFLOPS, 4),
                                   "tflops_call": round(flops / t_call / 1e6, 1)}
    return res


# ---------------------------------------------------------------------------
# C5: the 32-layer decoder-stack sweep (Q4_K_M mix)
# ---------------------------------------------------------------------------

# Llama-3-8B layer in the Q4_K_M mix: Q6_K for v and down, Q4_K for the rest
C5_PROJ = [("q", Q4K, 4096, 4096), ("k", Q4K, 1024, 4096), ("v", Q6K, 1024, 4096), ("o", Q4K, 4096, 4096),
           ("gate", Q4K, 14336, 4096), ("up", Q4K, 14336, 4096), ("down", Q6K, 4096, 14336)]
C5_LAYERS = 32
C5_HEAD = (Q6K, 128256, 4096)


def run_c5(ctx: Ctx, args):
    """One step = every projection of 32 layers plus the Q6_K head, back to
    back on one stream, replayed from a HIP graph.  `grouped`: the launches
    an engine issues (q+k and gate+up share x in okq_gemv_multi, the other
    projections through okq_linear_out_by_in_q); `auto`: one
    okq_linear_out_by_in_q per projection.  Both dispatches pick the kernel
    by shape: the streaming decode-batch MFMA kernel for Q4_K/Q6_K weights of
    16 MB and more from five rows, and for every Q4_K/Q6_K weight above eight
    rows; the GEMV otherwise (okq_gemv_multi's matrices that stay on the GEMV
    share one launch, each pass over a weight serving up to four rows)."""
    torch = ctx.torch
    log(f"C5: generating {C5_LAYERS} Q4_K_M layers + Q6_K head")
    layers = [{name: ctx.quantized(t, n, k, seed=50_000 + 100 * l + i) for i, (name, t, n, k) in enumerate(C5_PROJ)}
              for l in range(C5_LAYERS)]
    head = ctx.quantized(*C5_HEAD, seed=59_999)
    step_bytes = C5_LAYERS * sum(wbytes(t, n, k) for _, t, n, k in C5_PROJ) + wbytes(*C5_HEAD)
    shape = {name: (t, n, k) for name, t, n, k in C5_PROJ}
    res = {"weight_bytes_per_step": step_bytes, "layers": C5_LAYERS}
    cs = torch.cuda.Stream()  # capture stream: the GEMM workspace is allocated on it before capture
    for rows in (1, 8, 32):
        x4 = ctx.normal(rows * 4096, 60 + rows)
        x14 = ctx.normal(rows * 14336, 61 + rows)
        outs = {name: torch.empty(rows * n, dtype=torch.float32, device="cuda") for name, _, n, _ in C5_PROJ}
        yh = torch.empty(rows * C5_HEAD[1], dtype=torch.float32, device="cuda")

        def one(entry, name, w, s):
            t, n, k = shape[name]
            x = x14 if k == 14336 else x4
            ctx.okq.call(entry, x.data_ptr(), rows, k, t, w.data_ptr(), w.numel(), n, None, outs[name].data_ptr(), s)

        def group(names, lay, s):
            t, _, k = shape[names[0]]
            c = len(names)
            ctx.okq.call("okq_gemv_multi", x4.data_ptr(), rows, k, t, c,
                         (ctypes.c_void_p * c)(*[lay[m].data_ptr() for m in names]),
                         (ctypes.c_uint64 * c)(*[lay[m].numel() for m in names]),
                         (ctypes.c_int64 * c)(*[shape[m][1] for m in names]), None,
                         (ctypes.c_void_p * c)(*[outs[m].data_ptr() for m in names]), s)

        def step(mode, s):
            for lay in layers:
                if mode == "grouped":
                    group(["q", "k"], lay, s)
                    one("okq_linear_out_by_in_q", "v", lay["v"], s)
                    one("okq_linear_out_by_in_q", "o", lay["o"], s)
                    group(["gate", "up"], lay, s)
                    one("okq_linear_out_by_in_q", "down", lay["down"], s)
                else:
                    for name, _, _, _ in C5_PROJ:
                        one("okq_linear_out_by_in_q", name, lay[name], s)
            t, n, k = C5_HEAD
            ctx.okq.call("okq_linear_out_by_in_q", x4.data_ptr(), rows, k, t, head.data_ptr(), head.numel(), n, None,
                         yh.data_ptr(), s)

        modes = ["grouped"] if rows == 1 else ["grouped", "auto"]
        for mode in modes:
            with torch.cuda.stream(cs):
                step(mode, cs.cuda_stream)  # warm: allocates the GEMM workspace of this stream
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=cs):
                step(mode, cs.cuda_stream)
            for _ in range(2):
                g.replay()
            torch.cuda.synchronize()
            reps = args.c5_steps
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                g.replay()
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / reps
            log(f"C5: batch {rows} {mode}: {ms:.3f} ms per step")
            res[f"b{rows}_{mode}"] = {"batch": rows, "ms_per_step": round(ms, 4),
                                     "weight_gbs": round(step_bytes / ms / 1e6, 1),
                                     "frac_hbm": round(step_bytes / ms / 1e6 / HBM_PEAK_GBS, 4),
                                     "tokens_per_s": round(rows * 1000.0 / ms, 1)}
            del g
    del layers, head
    return res


# ---------------------------------------------------------------------------
# CPU baseline (reference CPU path, oracle restatement)
# ---------------------------------------------------------------------------

def run_cpu_baseline(ctx: Ctx, c2, args):
    import numpy as np
    from oracle import oracle as O
    orc = O.Oracle()
    lay = c2["layers"][0]
    log("cpu baseline: dequantizing one layer copy on the host (not timed)")
    w = {name: orc.dequantize(O.Q4_K, lay[name].cpu().numpy(), n * k).reshape(n, k) for name, n, k in C2_PROJ}
    x4096 = c2["x4096"].cpu().numpy()
    x14336 = c2["x14336"].cpu().numpy()
    # sanity: the GPU result of the last timed step equals the CPU path within tolerance
    passes = 0
    t0 = time.perf_counter()
    while True:
        for name, n, k in C2_PROJ:
            orc.linear(x14336 if k == 14336 else x4096, 1, k, w[name], n, None, O.MODE_SCALAR, 1)
        passes += 1
        if time.perf_counter() - t0 >= args.cpu_seconds:
            break
    sec = time.perf_counter() - t0
    gbs = c2["step_bytes"] * passes / sec / 1e9
    cpu = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(gbs, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"C2 layer copy 0 (7 Q4_K projections, {c2['step_bytes']} quantized bytes) dequantized to f32 "
                      f"once (untimed); reference scalar linear_out_by_in, batch 1, serial (rows < 32); "
                      f"{passes} passes in {sec:.2f} s on {cpu}",
            "ms_per_step": round(1000.0 * sec / passes, 2)}


def run_probe(ctx: Ctx, what: str):
    """Bare workloads for `rocprofv3 --pmc` (one dispatch per launch, no graph)."""
    torch = ctx.torch
    if what == "gate_up":
        names = ["gate", "up"]
        ws = {m: ctx.quantized(Q4K, *C2_SHAPE[m], seed=10_004 + i) for i, m in enumerate(names)}
        pools = {m: ctx.replicas(ws[m]) for m in names}
        copies = min(cp for _, cp in pools.values())
        x = ctx.normal(4096, 1)
        outs = {m: torch.empty(C2_SHAPE[m][0], dtype=torch.float32, device="cuda") for m in names}
        b = wbytes(Q4K, *C2_SHAPE["gate"])
        for i in range(20):
            launch_group(ctx, names, {m: pools[m][0].narrow(0, (i % copies) * b, b) for m in names}, x, outs)
        log(f"probe gate_up: 20 launches, {2 * b} weight bytes each")
    else:
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(20):
            torch.mul(src, 1.0, out=dst)
        log(f"probe copy: 20 launches, {src.numel() * 4} bytes read and written each")
    torch.cuda.synchronize()


# ---------------------------------------------------------------------------

def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--copies", type=int, default=8)
    ap.add_argument("--kernel-reps", type=int, default=200)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="only the C2 headline")
    ap.add_argument("--only", default="c1,c3,c4,c5", help="secondary configs to run (comma list of c1,c3,c4,c5)")
    ap.add_argument("--c5-steps", type=int, default=10, help="timed steps per C5 batch size")
    ap.add_argument("--probe", choices=["gate_up", "copy"], default=None,
                    help="run a bare workload for rocprofv3 counter passes and exit: 20 gate+up GEMV launches over "
                         "weight replicas, or 20 launches of a 256 MiB f32 elementwise copy (calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X only: this build has no multi-GPU path "
              "(the sharding design is described in DESIGN.md). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    from ocelotl_amd import okq
    okq.call("okq_init", 0)
    ctx = Ctx(torch, okq)
    if args.probe:
        run_probe(ctx, args.probe)
        return

    c2 = run_c2(ctx, args)
    extra = {"c2_launches": c2["launches"], "c2_shapes": c2["shapes"],
             "c2_sequential": {"what": "the same step as 7 single-projection launches",
                               "gbs": round(c2["gbs_sequential"], 1),
                               "ms_per_step": round(1000.0 * c2["sec_sequential"] / args.steps, 5),
                               "frac_hbm_peak": round(c2["gbs_sequential"] / HBM_PEAK_GBS, 4)}}
    only = set(args.only.split(",")) if not args.no_extra else set()
    if "c1" in only:
        extra["c1_q8_0"] = run_c1(ctx, args)
    if "c3" in only:
        extra["c3_q6_k_head"] = run_c3(ctx, args)
    if "c4" in only:
        extra["c4_q4_k_gemm_bf16"] = run_c4(ctx, args, c2)
    if "c5" in only:
        extra["c5_stack_sweep"] = run_c5(ctx, args)
    cpu = None if args.no_cpu else run_cpu_baseline(ctx, c2, args)

    rec = {
        "metric": METRIC,
        "value": round(c2["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1000.0 * c2["sec"] / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k weights x f32 activations (int8 dot4 -> i32, f32 scale/accumulate)",
        "data": "synthetic: seeded N(0,0.02) weights quantized to Q4_K on the GPU, N(0,1) f32 activations",
        "config": {"workload": "C2: Q4_K decode GEMV, one Llama-3-8B layer per step (q 4096x4096, k/v 1024x4096, "
                               "o 4096x4096, gate/up 14336x4096, down 4096x14336), batch 1, as 4 launches: "
                               "q+k+v and gate+up each in one okq_gemv_multi launch (they share x), o, down",
                   "batch": 1, "layer_copies_rotated": args.copies,
                   "weight_bytes_per_step": c2["step_bytes"],
                   "frac_hbm_peak": round(c2["gbs"] / HBM_PEAK_GBS, 4)},
        "roofline": roofline_from(c2["launches"]),
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
