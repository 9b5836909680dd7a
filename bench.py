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
  roofline_gemm the prefill half of the metric: the Q4_K GEMM kernel of the
                C4 M=512 gate call (14336x4096, bf16 activations), 2*M*N*K
                flops / its average dispatch duration (stream events around
                each launch) vs the 2.5 PFLOP/s dense fp16/bf16 MFMA peak;
                `traffic` from rocprofv3 FETCH_SIZE / WRITE_SIZE passes
                (profiles/gemm_q4k_m512_gate_counters.md)
  cpu_baseline  the reference CPU path (oracle restatement of
                linear_out_by_in, scalar mode, 1 core since rows < 32) on one
                layer copy, dequantized once outside the timing, with a check
                that the GPU's outputs of that step match it; `configs` holds
                bounded samples of C1, C3, C4 (scalar and AVX2, rows chunked
                over the host cores) and C5 (one layer at batch 1, 8, 32)
  extra         per-launch and per-projection times (mean, p10, median,
                p90), the 7-launch step, the secondary configs (C1, C3,
                C4 per call, C5), Q5_K at the MLP shapes (gate+up at
                batch 1 and 8, the M=512 gate prefill call), and the Q6_K
                down projection's M=512 prefill call

Run: python bench.py [--steps K] [--warmup W] [--copies C] [--no-cpu] ...
     python bench.py --probe gate_up|copy|gemm_gate512|gemm_down512|gemm_gate128|gemm_q8_512|gemm_q8_2048|gemm_q6_512|decode_gate_up32|decode_head8
                                                        (bare workloads for counter passes)
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
Q4K, Q5K, Q6K, Q8_0 = 12, 13, 14, 8
BLOCK = {Q4K: (256, 144), Q5K: (256, 176), Q6K: (256, 210), Q8_0: (32, 34)}
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
        self.host = {}  # host copies of workloads for the CPU baseline leg

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

    def graph_us(self, launch, n: int, reps: int = 10):
        """Duration (µs) of one launch inside a HIP graph of n back-to-back
        launch(i) calls, timed with events on the stream the graph is replayed
        on: (mean over `reps` replays, per-replay means)."""
        torch = self.torch
        launch(0)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n):
                launch(i)
        g.replay()
        torch.cuda.synchronize()
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        evs[0].record()
        for r in range(reps):
            g.replay()
            evs[r + 1].record()
        torch.cuda.synchronize()
        per = [1000.0 * evs[r].elapsed_time(evs[r + 1]) / n for r in range(reps)]
        del g
        return sum(per) / reps, per

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
    """Wall time of exactly args.steps steps, and per-step times (for
    p10/median/p90).  The steps (rotating over the layer copies) are captured
    into one HIP graph, so the timed region -- synchronize on both sides -- is
    a single replay.  The percentiles come from a second measurement after it:
    replays of a graph of one pass over all copies, with events between the
    replays."""
    torch = ctx.torch
    step(0)
    torch.cuda.synchronize()

    def capture(n):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for c in range(n):
                step(c)
        return g

    g_all = capture(args.copies)
    g_k = capture(args.steps)
    for _ in range(max(1, -(-args.warmup // args.copies))):
        g_all.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g_k.replay()
    torch.cuda.synchronize()
    sec = time.perf_counter() - t0
    reps = max(4, min(32, args.steps // args.copies))
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    evs[0].record()
    for i in range(reps):
        g_all.replay()
        evs[i + 1].record()
    torch.cuda.synchronize()
    per_step = [evs[i].elapsed_time(evs[i + 1]) / args.copies for i in range(reps)]
    del g_all, g_k
    return sec, per_step


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
    sec, per_step = time_steps(ctx, args, step_fused)
    log(f"C2: the same steps as 7 single-projection launches")
    sec_seq, _ = time_steps(ctx, args, step_seq)

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

        us, per = ctx.graph_us(launch, max(64, 2 * copies))
        b = sum(wbytes(Q4K, *C2_SHAPE[m]) for m in names)
        del pools
        return {"matrices": names, "weight_bytes": b, "us_mean": round(us, 3), "us_p10": round(pct(per, 10), 3),
                "us_median": round(median(per), 3), "us_p90": round(pct(per, 90), 3), "gbs": round(b / us / 1e3, 1),
                "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}

    launches = {g: group_time(names) for g, names in C2_GROUPS}
    shapes = {name: group_time([name]) for name, _, _ in C2_PROJ}
    return {"gbs": step_bytes * args.steps / sec / 1e9, "sec": sec, "per_step_ms": per_step,
            "gbs_sequential": step_bytes * args.steps / sec_seq / 1e9, "sec_sequential": sec_seq,
            "step_bytes": step_bytes, "launches": launches, "shapes": shapes, "layers": layers,
            "x4096": x4096, "x14336": x14336}


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_q4k_gate_up_traffic.md")
GEMM_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemm_q4k_m512_gate_counters.md")


def measured_traffic(path=TRAFFIC_FILE):
    """HBM bytes per launch of a roofline kernel from a committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (line `traffic_bytes_per_launch: N`), or
    None when no such measurement is committed."""
    try:
        with open(path) as f:
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


def roofline_gemm_from(c4):
    """The prefill half of the metric: the Q4_K GEMM kernel of the C4 M=512
    gate call (the dominant prefill shape), algorithmic flops 2*M*N*K per
    launch over the kernel's average dispatch duration."""
    r = c4.get("M512_gate")
    if r is None:
        return None
    flops = 2 * r["m"] * r["n"] * r["k"]
    achieved = flops / r["us_kernel"] / 1e6
    return {"bound": "mfma", "kernel": r.get("kernel", "okq::gemm_wide_q4k_kernel"),
            "shape": "M=512 x N=14336 x K=4096 (C4 gate, bf16 activations)",
            "achieved": round(achieved, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / BF16_PEAK_TFLOPS, 4), "traffic": measured_traffic(GEMM_TRAFFIC_FILE),
            "algorithmic_flops_per_launch": flops, "launch_us_mean": r["us_kernel"],
            "per_call_frac": r["frac_bf16_peak"], "per_call_us": r["us_call"]}


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
    if not args.no_cpu:  # the CPU baseline leg runs the same head and activations
        ctx.host["c3"] = (w.cpu().numpy(), x.cpu().numpy())
    pool, copies = ctx.replicas(w)
    del w

    def launch(i):
        ctx.okq.call("okq_gemv", x.data_ptr(), 1, k, Q6K, pool.data_ptr() + (i % copies) * b, b, n, None,
                     y.data_ptr(), ctx.stream)

    us, per = ctx.graph_us(launch, 16)
    del pool
    return {"shape": [n, k], "weight_bytes": b, "us_mean": round(us, 2), "us_p10": round(pct(per, 10), 2),
            "us_median": round(median(per), 2), "us_p90": round(pct(per, 90), 2),
            "gbs": round(b / us / 1e3, 1), "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}


def run_c1(ctx: Ctx, args):
    n, k = 4096, 4096
    log("C1: Q8_0 4096x4096 GEMV (GPU)")
    w = ctx.quantized(Q8_0, n, k, seed=40)
    x = ctx.normal(k, 41)
    y = ctx.torch.empty(n, dtype=ctx.torch.float32, device="cuda")
    b = wbytes(Q8_0, n, k)
    if not args.no_cpu:
        ctx.host["c1"] = (w.cpu().numpy(), x.cpu().numpy())
    pool, copies = ctx.replicas(w)

    def launch(i):
        ctx.okq.call("okq_gemv", x.data_ptr(), 1, k, Q8_0, pool.data_ptr() + (i % copies) * b, b, n, None,
                     y.data_ptr(), ctx.stream)

    us, per = ctx.graph_us(launch, max(64, 2 * copies))
    del pool
    return {"shape": [n, k], "weight_bytes": b, "us_mean": round(us, 3), "us_p10": round(pct(per, 10), 3),
            "us_median": round(median(per), 3), "us_p90": round(pct(per, 90), 3),
            "gbs": round(b / us / 1e3, 1), "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}


def run_c4(ctx: Ctx, args, c2):
    """Prefill dequant-GEMM at M in {128, 512, 2048} with bf16 activations:
    Q4_K at the Llama-3-8B projection shapes (q/o 4096x4096, k/v 1024x4096,
    gate/up 14336x4096, down 4096x14336; one of each pair) and Q8_0 at
    4096x4096.  us_call: the whole entry point (activation pre-pass + GEMM +
    split-K reduction) as a prefill issues it, back to back: `reps` calls
    rotating over 8 weight copies captured into one HIP graph, stream events
    around each of 10 replays (mean per call; p10, median, p90 over the
    replays' per-call means); us_kernel: the MFMA kernel's own dispatch time.
    frac_bf16_peak is per call."""
    torch = ctx.torch
    res = {}
    lay = c2["layers"]
    q8 = [ctx.quantized(Q8_0, 4096, 4096, seed=70 + c) for c in range(8)]
    shapes = [(Q4K, name, n, k) for name, n, k in C2_PROJ if name not in ("k", "o", "up")] + [(Q8_0, "q8_0", 4096, 4096)]
    for m in (128, 512, 2048):
        log(f"C4: GEMM M={m}")
        xf = ctx.normal(m * 14336, 50 + m)
        xb = torch.empty(m * 14336, dtype=torch.int16, device="cuda")
        ctx.okq.call("okq_f32_to_bf16", xf.data_ptr(), xf.numel(), xb.data_ptr(), ctx.stream)
        for t, name, n, k in shapes:
            y = torch.empty(m * n, dtype=torch.float32, device="cuda")
            reps = max(8, args.kernel_reps // 8)
            ws = [lay[c][name] for c in range(len(lay))] if t == Q4K else q8

            def call(r, t=t, n=n, k=k, y=y, ws=ws):
                ctx.gemv(t, xb, k, ws[r % len(ws)], n, y, entry="okq_gemm_bf16", rows=m)

            call(0)
            us = ctx.kernel_us(call, reps)
            cs = torch.cuda.Stream()  # capture stream: its GEMM workspace is allocated before capture
            with torch.cuda.stream(cs):
                call(0)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=cs):
                for r in range(reps):
                    call(r)
            g.replay()
            torch.cuda.synchronize()
            replays = 10
            evs = [torch.cuda.Event(enable_timing=True) for _ in range(replays + 1)]
            evs[0].record()
            for r in range(replays):
                g.replay()
                evs[r + 1].record()
            torch.cuda.synchronize()
            del g
            per = [1000.0 * evs[r].elapsed_time(evs[r + 1]) / reps for r in range(replays)]
            t_call = sum(per) / replays
            t_k = sum(us) / len(us)
            flops = 2.0 * m * n * k
            key = f"M{m}_{name}" if t == Q4K else f"M{m}_q8_0_4096"
            kernel = None
            if key == "M512_gate":  # the plan's choice at 256 CUs (gemm_plan, okq_gemm.hip)
                kernel = "okq::gemm_wide_q4k_kernel (128x256 tiles, 8 waves, weights dequantised in registers)"
            elif t == Q8_0:  # bf16 Q8_0: no pre-pass; 8-wave tiles where they fill the CUs (gemm_plan)
                kernel = ("okq::gemm_q8_wide_kernel (128x256 tiles, 8 waves)" if m >= 2048 else
                          "okq::gemm_q8_kernel (128x128 tiles, 4 waves, K split)") + \
                    ": bf16 MFMAs on x and q, per-block f32 fold with d, no activation pre-pass"
            res[key] = {"type": "Q4_K" if t == Q4K else "Q8_0", "m": m, "n": n, "k": k,
                        "us_call": round(t_call, 2), "us_call_p10": round(pct(per, 10), 2),
                        "us_call_median": round(median(per), 2), "us_call_p90": round(pct(per, 90), 2),
                        "tflops_call": round(flops / t_call / 1e6, 1),
                        "frac_bf16_peak": round(flops / t_call / 1e6 / BF16_PEAK_TFLOPS, 4),
                        "us_kernel": round(t_k, 2), "tflops_kernel": round(flops / t_k / 1e6, 1),
                        "frac_bf16_peak_kernel": round(flops / t_k / 1e6 / BF16_PEAK_TFLOPS, 4)}
            if kernel:
                res[key]["kernel"] = kernel
    del q8
    return res


def graph_call_us(ctx, call, reps: int, replays: int = 10):
    """Per-call duration (µs) of `reps` back-to-back call(r) captured into one
    HIP graph on a capture stream whose GEMM workspace is allocated before
    capture; stream events around each of `replays` replays: (mean, per-replay
    means)."""
    torch = ctx.torch
    cs = torch.cuda.Stream()
    with torch.cuda.stream(cs):
        call(0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cs):
        for r in range(reps):
            call(r)
    g.replay()
    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(replays + 1)]
    evs[0].record()
    for r in range(replays):
        g.replay()
        evs[r + 1].record()
    torch.cuda.synchronize()
    del g
    per = [1000.0 * evs[r].elapsed_time(evs[r + 1]) / reps for r in range(replays)]
    return sum(per) / replays, per


def run_q5k(ctx: Ctx, args):
    """Q5_K, the linear path's fourth format, at the Llama-3-8B MLP shapes:
    the gate+up pair (2 x 14336x4096) as one okq_gemv_multi call at batch 1
    (the grouped GEMV launch) and at 8 rows (one decode-batch launch), and the
    M=512 gate prefill call with bf16 activations (pre-pass + tiled kernel).
    Each rotates over >= 512 MB of weight replicas inside a HIP graph."""
    torch = ctx.torch
    n, k = 14336, 4096
    b = wbytes(Q5K, n, k)
    log("Q5_K: gate+up at batch 1 and 8, M=512 gate prefill")
    pools = [ctx.replicas(ctx.quantized(Q5K, n, k, seed=900 + i)) for i in range(2)]
    copies = min(cp for _, cp in pools)
    w_at = lambda i, r: pools[i][0].narrow(0, (r % copies) * b, b)
    res = {"weight_bytes_per_matrix": b}
    for rows in (1, 8):
        x = ctx.normal(rows * k, 902 + rows)
        ys = [torch.empty(rows * n, dtype=torch.float32, device="cuda") for _ in range(2)]

        def call(r, rows=rows, x=x, ys=ys):
            ctx.okq.call("okq_gemv_multi", x.data_ptr(), rows, k, Q5K, 2,
                         (ctypes.c_void_p * 2)(w_at(0, r).data_ptr(), w_at(1, r).data_ptr()),
                         (ctypes.c_uint64 * 2)(b, b), (ctypes.c_int64 * 2)(n, n), None,
                         (ctypes.c_void_p * 2)(ys[0].data_ptr(), ys[1].data_ptr()), ctx.stream)

        us, per = graph_call_us(ctx, call, max(64, 2 * copies))
        res[f"gate_up_b{rows}"] = {"rows": rows, "us_mean": round(us, 3), "us_p10": round(pct(per, 10), 3),
                                   "us_median": round(median(per), 3), "us_p90": round(pct(per, 90), 3),
                                   "gbs": round(2 * b / us / 1e3, 1), "frac_hbm": round(2 * b / us / 1e3 / HBM_PEAK_GBS, 4)}
    m = 512
    xf = ctx.normal(m * k, 905)
    xb = torch.empty(m * k, dtype=torch.int16, device="cuda")
    ctx.okq.call("okq_f32_to_bf16", xf.data_ptr(), xf.numel(), xb.data_ptr(), ctx.stream)
    y = torch.empty(m * n, dtype=torch.float32, device="cuda")
    reps = max(8, args.kernel_reps // 8)

    def gcall(r):
        ctx.gemv(Q5K, xb, k, w_at(0, r), n, y, entry="okq_gemm_bf16", rows=m)

    gcall(0)
    us_k = ctx.kernel_us(gcall, reps)
    t_call, per = graph_call_us(ctx, gcall, reps)
    t_k = sum(us_k) / len(us_k)
    flops = 2.0 * m * n * k
    res["M512_gate"] = {"m": m, "n": n, "k": k, "us_call": round(t_call, 2), "us_call_p10": round(pct(per, 10), 2),
                        "us_call_median": round(median(per), 2), "us_call_p90": round(pct(per, 90), 2),
                        "tflops_call": round(flops / t_call / 1e6, 1),
                        "frac_bf16_peak": round(flops / t_call / 1e6 / BF16_PEAK_TFLOPS, 4),
                        "us_kernel": round(t_k, 2), "frac_bf16_peak_kernel": round(flops / t_k / 1e6 / BF16_PEAK_TFLOPS, 4)}
    del pools
    return res


def run_q6k_prefill(ctx: Ctx, args):
    """The Q4_K_M / Q5_K_M files' other format at prefill: the Q6_K down
    projection (4096 x 14336, the largest matrix a Q4_K_M layer stores in
    Q6_K) at M=512 with bf16 activations (pre-pass + gemm_wide_q6k_kernel +
    split-K reduction), rotating over >= 512 MB of weight replicas in a HIP
    graph."""
    torch = ctx.torch
    n, k, m = 4096, 14336, 512
    b = wbytes(Q6K, n, k)
    log("Q6_K: M=512 down prefill")
    pool, copies = ctx.replicas(ctx.quantized(Q6K, n, k, seed=910))
    xf = ctx.normal(m * k, 911)
    xb = torch.empty(m * k, dtype=torch.int16, device="cuda")
    ctx.okq.call("okq_f32_to_bf16", xf.data_ptr(), xf.numel(), xb.data_ptr(), ctx.stream)
    y = torch.empty(m * n, dtype=torch.float32, device="cuda")
    reps = max(8, args.kernel_reps // 8)

    def gcall(r):
        ctx.gemv(Q6K, xb, k, pool.narrow(0, (r % copies) * b, b), n, y, entry="okq_gemm_bf16", rows=m)

    gcall(0)
    us_k = ctx.kernel_us(gcall, reps)
    t_call, per = graph_call_us(ctx, gcall, reps)
    t_k = sum(us_k) / len(us_k)
    flops = 2.0 * m * n * k
    del pool
    return {"M512_down": {"m": m, "n": n, "k": k, "us_call": round(t_call, 2), "us_call_p10": round(pct(per, 10), 2),
                          "us_call_median": round(median(per), 2), "us_call_p90": round(pct(per, 90), 2),
                          "tflops_call": round(flops / t_call / 1e6, 1),
                          "frac_bf16_peak": round(flops / t_call / 1e6 / BF16_PEAK_TFLOPS, 4),
                          "us_kernel": round(t_k, 2),
                          "frac_bf16_peak_kernel": round(flops / t_k / 1e6 / BF16_PEAK_TFLOPS, 4)}}


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
    an engine issues (q, k and v share x in okq_linear_multi_q -- Q4_K and
    Q6_K matrices in one launch at batch sizes -- gate+up in okq_gemv_multi,
    o and down through okq_linear_out_by_in_q); `auto`: one
    okq_linear_out_by_in_q per projection.  Both dispatches pick the kernel
    by shape: the streaming decode-batch MFMA kernel for weights from 2 MB at
    6-8 rows (from 8 MB at 5 rows, down projections and the head from 3
    rows), and for every weight above eight rows; the GEMV otherwise
    (okq_gemv_multi's matrices that stay on the GEMV share one launch, each
    pass over a weight serving up to four rows)."""
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

        def qkv(lay, s):
            names = ["q", "k", "v"]
            c = len(names)
            ctx.okq.call("okq_linear_multi_q", x4.data_ptr(), rows, 4096, c,
                         (ctypes.c_uint32 * c)(*[shape[m][0] for m in names]),
                         (ctypes.c_void_p * c)(*[lay[m].data_ptr() for m in names]),
                         (ctypes.c_uint64 * c)(*[lay[m].numel() for m in names]),
                         (ctypes.c_int64 * c)(*[shape[m][1] for m in names]), None,
                         (ctypes.c_void_p * c)(*[outs[m].data_ptr() for m in names]), s)

        def step(mode, s):
            for lay in layers:
                if mode == "grouped":
                    qkv(lay, s)
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

def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads() -> int:
    """Host threads for the reference's chunked path (rows >= 32): the box's
    CPU share, at most 16."""
    return max(1, min(16, os.cpu_count() or 1))


def cpu_time(fn, seconds: float):
    """Calls fn until `seconds` have elapsed (at least once): (s per call, calls)."""
    calls = 0
    t0 = time.perf_counter()
    while True:
        fn()
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            return el / calls, calls


def run_cpu_baseline(ctx: Ctx, c2, args):
    """The reference CPU path (the oracle's restatement of linear_out_by_in,
    crates/kernels/src/lib.rs:1974-2123, and its AVX2 variant,
    crates/kernels/src/cpu_avx2.rs:58-253) on the host cores of the GPU box,
    weights dequantized to f32 once outside the timing.  The reference runs
    rows < 32 serially and chunks rows >= 32 over all cores (lib.rs:2245,
    :2294-2390); every entry states its threads.  Headline: the C2 step on
    one layer copy (1 core).  `configs`: bounded samples of C1, C3, C4 and C5.
    The C2 outputs of the CPU path are checked against the GPU's for the same
    inputs with the reference rule."""
    import numpy as np
    from oracle import oracle as O
    orc = O.Oracle()
    model = cpu_model()
    lay = c2["layers"][0]
    log("cpu baseline: dequantizing one layer copy on the host (not timed)")
    w = {name: orc.dequantize(O.Q4_K, lay[name].cpu().numpy(), n * k).reshape(n, k) for name, n, k in C2_PROJ}
    x4096 = c2["x4096"].cpu().numpy()
    x14336 = c2["x14336"].cpu().numpy()
    cpu_out = {}

    def c2_pass():
        for name, n, k in C2_PROJ:
            cpu_out[name] = orc.linear(x14336 if k == 14336 else x4096, 1, k, w[name], n, None, O.MODE_SCALAR, 1)

    sec_pass, passes = cpu_time(c2_pass, args.cpu_seconds)
    gbs = c2["step_bytes"] / sec_pass / 1e9
    # the GPU's outputs of the same step (layer copy 0, the same activations)
    gpu_out = {name: ctx.torch.empty(n, dtype=ctx.torch.float32, device="cuda") for name, n, _ in C2_PROJ}
    for _, names in C2_GROUPS:
        launch_group(ctx, names, lay, c2["x14336"] if C2_SHAPE[names[0]][1] == 14336 else c2["x4096"], gpu_out)
    ctx.torch.cuda.synchronize()
    parity = all(O.allclose_ref_rule(gpu_out[name].cpu().numpy(), cpu_out[name], 1e-3)[0] for name, _, _ in C2_PROJ)
    # the timed step's error against the reference CPU path: the largest
    # absolute difference, the largest relative one over outputs with
    # |want| >= 0.1, and the largest min(abs, rel) -- the quantity the
    # reference rule bounds by 1e-3 (outputs are ~N(0, 1.3))
    abs_err, rel_err, rule = 0.0, 0.0, 0.0
    for name, _, _ in C2_PROJ:
        got = gpu_out[name].cpu().numpy().astype(np.float64)
        want = cpu_out[name].astype(np.float64)
        d = np.abs(got - want)
        abs_err = max(abs_err, float(d.max()))
        big = np.abs(want) >= 0.1
        if big.any():
            rel_err = max(rel_err, float((d[big] / np.abs(want[big])).max()))
        rule = max(rule, float(np.minimum(d, d / np.maximum(np.abs(want), 1e-30)).max()))
    head = {"value": round(gbs, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"C2 layer copy 0 (7 Q4_K projections, {c2['step_bytes']} quantized bytes) dequantized to f32 "
                      f"once (untimed); reference scalar linear_out_by_in, batch 1, serial (rows < 32); "
                      f"{passes} passes in {sec_pass * passes:.2f} s on {model}",
            "ms_per_step": round(1000.0 * sec_pass, 2),
            "gpu_outputs_match_cpu_within_rule": bool(parity),
            "gpu_vs_cpu_max_abs_err": float(f"{abs_err:.3g}"),
            "gpu_vs_cpu_max_rel_err_where_abs_want_ge_0.1": float(f"{rel_err:.3g}"),
            "gpu_vs_cpu_max_min_abs_rel": float(f"{rule:.3g}")}
    if args.cpu_configs:
        head["configs"] = run_cpu_configs(ctx, orc, O, args)
    return head


def run_cpu_configs(ctx: Ctx, orc, O, args):
    """Bounded CPU samples of the secondary configs (reference scalar and AVX2
    paths, the reference's threading rule)."""
    import numpy as np
    res = {}
    thr = cpu_threads()
    sec = args.cpu_config_seconds
    # C1: Q8_0 4096 x 4096 at batch 1 (serial)
    if "c1" in ctx.host:
        wq, x = ctx.host["c1"]
        wf = orc.dequantize(O.Q8_0, wq, 4096 * 4096)
        for mode, label in ((O.MODE_SCALAR, "scalar"), (O.MODE_AVX2, "avx2")):
            if mode == O.MODE_AVX2 and not orc.has_avx2():
                continue
            t, calls = cpu_time(lambda: orc.linear(x, 1, 4096, wf, 4096, None, mode, 1), sec)
            res[f"c1_q8_0_{label}"] = {"us_per_call": round(1e6 * t, 1), "gbs": round(wq.size / t / 1e9, 3),
                                       "cores": 1, "calls": calls}
        del wf
    # C3: the Q6_K head at batch 1 (serial)
    if "c3" in ctx.host:
        wq, x = ctx.host["c3"]
        log("cpu baseline: dequantizing the Q6_K head (not timed)")
        wf = orc.dequantize(O.Q6_K, wq, 128256 * 4096)
        t, calls = cpu_time(lambda: orc.linear(x, 1, 4096, wf, 128256, None, O.MODE_SCALAR, 1), sec)
        res["c3_q6_k_head_scalar"] = {"us_per_call": round(1e6 * t, 1), "gbs": round(wq.size / t / 1e9, 3), "cores": 1,
                                      "calls": calls}
        del wf
    # C4: Q4_K prefill at M = 128, 512, 2048 on the q (4096 x 4096), gate
    # (14336 x 4096) and down (4096 x 14336) shapes, rows chunked over the
    # host cores as the reference does at rows >= 32 (each sample at least
    # one whole call)
    c4_cases = [(m, name, n, k, n) for m in (128, 512, 2048)
                for name, n, k in (("q", 4096, 4096), ("gate", 14336, 4096), ("down", 4096, 14336))]
    wcache = {}
    for m, name, n, k, n_s in c4_cases:
        if (name, n_s) not in wcache:
            seed = {"q": 10_000, "gate": 10_004, "down": 10_006}[name]
            rb = (k // 256) * 144
            wq = ctx.quantized(Q4K, n, k, seed=seed).cpu().numpy()[: n_s * rb]
            wcache[(name, n_s)] = orc.dequantize(O.Q4_K, wq, n_s * k).reshape(n_s, k)
        wf = wcache[(name, n_s)]
        xb = orc.f32_to_bf16(orc.normal(50 + m, m * k, 1.0))
        x = orc.bf16_to_f32(xb)
        for mode, label in ((O.MODE_SCALAR, "scalar"), (O.MODE_AVX2, "avx2")):
            if mode == O.MODE_AVX2 and not orc.has_avx2():
                continue
            t, calls = cpu_time(lambda: orc.linear(x, m, k, wf, n_s, None, mode, thr), sec)
            rec = {"us_per_call": round(1e6 * t * n / n_s, 1), "tflops": round(2.0 * m * n_s * k / t / 1e12, 4),
                   "cores": thr, "calls": calls}
            if n_s < n:
                rec["sample"] = f"{n_s} of {n} output features per call, time scaled by {n / n_s:g}"
            res[f"c4_M{m}_{name}_{label}"] = rec
    del wcache
    # C5: one Q4_K_M layer (Q6_K v and down) at batch 1, 8 (serial) and 32 (all cores)
    lay = {name: ctx.quantized(t, n, k, seed=50_000 + i).cpu().numpy() for i, (name, t, n, k) in enumerate(C5_PROJ)}
    wl = {name: orc.dequantize(t, lay[name], n * k).reshape(n, k) for name, t, n, k in C5_PROJ}
    lbytes = sum(wbytes(t, n, k) for _, t, n, k in C5_PROJ)
    for b in (1, 8, 32):
        x4 = orc.normal(60 + b, b * 4096, 1.0)
        x14 = orc.normal(61 + b, b * 14336, 1.0)
        th = thr if b >= 32 else 1

        def layer():
            for name, t, n, k in C5_PROJ:
                orc.linear(x14 if k == 14336 else x4, b, k, wl[name], n, None, O.MODE_SCALAR, th)

        t, calls = cpu_time(layer, sec)
        res[f"c5_layer_b{b}_scalar"] = {"ms_per_layer": round(1e3 * t, 2),
                                        "weight_gbs": round(lbytes / t / 1e9, 3), "cores": th, "calls": calls,
                                        "tokens_per_s_32_layers": round(b / (32 * t), 2)}
    return res


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
        # 100 launches, so that the first (cold) one weighs little in a trace's average
        for i in range(100):
            launch_group(ctx, names, {m: pools[m][0].narrow(0, (i % copies) * b, b) for m in names}, x, outs)
        log(f"probe gate_up: 100 launches, {2 * b} weight bytes each")
    elif what == "decode_gate_up32":
        names = ["gate", "up"]
        ws = {m: ctx.quantized(Q4K, *C2_SHAPE[m], seed=10_004 + i) for i, m in enumerate(names)}
        pools = {m: ctx.replicas(ws[m]) for m in names}
        copies = min(cp for _, cp in pools.values())
        rows, (n, k) = 32, C2_SHAPE["gate"]
        x = ctx.normal(rows * k, 32)
        outs = [torch.empty(rows * n, dtype=torch.float32, device="cuda") for _ in names]
        b = wbytes(Q4K, n, k)
        for i in range(20):
            w = [pools[m][0].narrow(0, (i % copies) * b, b) for m in names]
            ctx.okq.call("okq_gemv_multi", x.data_ptr(), rows, k, Q4K, 2, (ctypes.c_void_p * 2)(*[t.data_ptr() for t in w]),
                         (ctypes.c_uint64 * 2)(b, b), (ctypes.c_int64 * 2)(n, n), None,
                         (ctypes.c_void_p * 2)(*[o.data_ptr() for o in outs]), ctx.stream)
        log(f"probe decode_gate_up32: 20 calls of 32 rows over gate+up ({2 * b} weight bytes each): "
            f"one decode-batch launch and its split-K reduction per call")
    elif what == "decode_head8":
        t, n, k = C5_HEAD
        rows = 8
        w = ctx.quantized(t, n, k, seed=59_999)
        pool, copies = ctx.replicas(w)
        x = ctx.normal(rows * k, 8)
        y = torch.empty(rows * n, dtype=torch.float32, device="cuda")
        b = wbytes(t, n, k)
        for i in range(20):
            ctx.okq.call("okq_linear_out_by_in_q", x.data_ptr(), rows, k, t, pool.narrow(0, (i % copies) * b, b).data_ptr(),
                         b, n, None, y.data_ptr(), ctx.stream)
        log(f"probe decode_head8: 20 calls of 8 rows over the Q6_K head ({b} weight bytes each): "
            f"one decode-batch launch per call")
    elif what.startswith("gemm_"):
        t, m, n, k = {"gemm_gate512": (Q4K, 512, 14336, 4096), "gemm_down512": (Q4K, 512, 4096, 14336),
                      "gemm_gate128": (Q4K, 128, 14336, 4096), "gemm_q8_512": (Q8_0, 512, 4096, 4096),
                      "gemm_q8_2048": (Q8_0, 2048, 4096, 4096), "gemm_q6_512": (Q6K, 512, 4096, 14336)}[what]
        ws = [ctx.quantized(t, n, k, seed=10_004 + c) for c in range(4)]
        xf = ctx.normal(m * k, 562)
        xb = torch.empty(m * k, dtype=torch.int16, device="cuda")
        ctx.okq.call("okq_f32_to_bf16", xf.data_ptr(), xf.numel(), xb.data_ptr(), ctx.stream)
        y = torch.empty(m * n, dtype=torch.float32, device="cuda")
        for i in range(20):
            ctx.gemv(t, xb, k, ws[i % len(ws)], n, y, entry="okq_gemm_bf16", rows=m)
        log(f"probe {what}: 20 {dict([(Q8_0, 'Q8_0'), (Q6K, 'Q6_K')]).get(t, 'Q4_K')} GEMM calls M={m} N={n} K={k} (bf16), "
            f"{2 * m * n * k} flops each")
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
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="C2 CPU baseline sample (seconds)")
    ap.add_argument("--cpu-config-seconds", type=float, default=1.5,
                    help="CPU baseline sample per secondary config (seconds; at least one call)")
    ap.add_argument("--no-cpu-configs", dest="cpu_configs", action="store_false",
                    help="CPU baseline of the C2 headline only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="only the C2 headline")
    ap.add_argument("--only", default="c1,c3,c4,c5,q5k,q6k",
                    help="secondary configs to run (comma list of c1,c3,c4,c5,q5k,q6k)")
    ap.add_argument("--c5-steps", type=int, default=10, help="timed steps per C5 batch size")
    ap.add_argument("--probe", choices=["gate_up", "copy", "gemm_gate512", "gemm_down512", "gemm_gate128",
                                        "gemm_q8_512", "gemm_q8_2048", "gemm_q6_512",
                                        "decode_gate_up32", "decode_head8"], default=None,
                    help="run a bare workload for rocprofv3 counter passes and exit: 20 gate+up GEMV launches over "
                         "weight replicas, 20 launches of a 256 MiB f32 elementwise copy (calibration), 20 Q4_K "
                         "GEMM calls (M=512 gate or down, M=128 gate), or 20 gate+up calls at 32 rows "
                         "(decode-batch kernel)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X only: this build has no multi-GPU path "
              "(each GPU would run the same kernels on its share of the rows). Run with --gpus 1.", file=sys.stderr)
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
    if "q5k" in only:
        extra["q5_k"] = run_q5k(ctx, args)
    if "q6k" in only:
        extra["q6_k_prefill"] = run_q6k_prefill(ctx, args)
    cpu = None if args.no_cpu else run_cpu_baseline(ctx, c2, args)

    rec = {
        "metric": METRIC,
        "value": round(c2["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1000.0 * c2["sec"] / args.steps, 5),
        "ms_per_step_p10_median_p90": [round(pct(c2["per_step_ms"], 10), 5), round(median(c2["per_step_ms"]), 5),
                                       round(pct(c2["per_step_ms"], 90), 5)],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k weights (4-bit ints, 6-bit scales/mins, f16 d/dmin) x f32 activations encoded per 32-run as "
                 "16-bit block integers (two int8 limbs; a third limb, 24 bits, only on outlier runs) with a power-of-2 "
                 "run scale; v_dot4_i32_i8 -> exact i32 sums; f32 scale and accumulate",
        "data": "synthetic: seeded N(0,0.02) weights quantized to Q4_K on the GPU, N(0,1) f32 activations",
        "config": {"workload": "C2: Q4_K decode GEMV, one Llama-3-8B layer per step (q 4096x4096, k/v 1024x4096, "
                               "o 4096x4096, gate/up 14336x4096, down 4096x14336), batch 1, as 4 launches: "
                               "q+k+v and gate+up each in one okq_gemv_multi launch (they share x), o, down",
                   "batch": 1, "layer_copies_rotated": args.copies,
                   "weight_bytes_per_step": c2["step_bytes"],
                   "frac_hbm_peak": round(c2["gbs"] / HBM_PEAK_GBS, 4)},
        "roofline": roofline_from(c2["launches"]),
        "roofline_gemm": roofline_gemm_from(extra["c4_q4_k_gemm_bf16"]) if "c4_q4_k_gemm_bf16" in extra else None,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
