#!/usr/bin/env python3
"""Headline benchmark of the MI355X INT4 weight-only linear path (one GPU).

Metric: "int4_linear M=1 HBM GB/s (% peak) over 7 layers; TFLOPS at M=2048".

A *step* is one pass of the hot path over one batch: the 7 TinyLlama-1.1B
decoder linears (q, k, v, o, gate, up, down; G=128) at M=1, each an
``ops.int4_linear`` call.  ``value`` is the 7-layer
algorithmic bytes (22,779,904 B; bench/bench_gemm.py:80,98) divided by the
measured time per step, in GB/s.

Protocol
* Weights: W ~ 0.02 N(0,1) fp32 per layer (seeded), quantized with the
  package's quantize_weight; x ~ N(0,1) fp16.  Synthetic, resident in HBM.
* Infinity-Cache-cold: R copies of the 7-layer weight set (R * 22.8 MB >= 2x
  the 256 MB MALL) are rotated, step i using copy i % R, so no step finds its
  weights in the MALL or L2.
* The steps are captured in HIP graphs (R steps per graph), so host launch
  cost is excluded as in the reference's CUDA-graph decode; W warm-up steps,
  then exactly K timed steps bracketed by torch.cuda.synchronize().
* roofline: the dominant kernel is the M=1 GEMV on the gate/up shape
  (N=5632, K=2048, 5,962,752 B per launch).  Its average duration is measured
  live with one HIP event pair per launch on the launching stream, launches
  queued behind a GPU spin so only GPU time is inside each pair, MALL-cold.
* ceilings: HBM copy/read peaks measured in the same run with the library's
  dwordx4 kernels on 1 GiB buffers; fp16 MFMA peak measured with torch.matmul
  (hipBLASLt) at 4096/6144/8192.
* M=2048: the GEMM on every TinyLlama shape at M=2048, event-timed; TFLOPS
  (2*M*N*K / time) for gate and for the 7-layer sum.
* cpu_baseline: the oracle's FP32 dequant + matmul (numpy; the reference's
  CPU path restated) on the host cores, over a bounded sample.

--gpus N > 1 is refused: this build measures one GPU.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "kernel-forge_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "int4_linear M=1 HBM GB/s (% peak) over 7 layers; TFLOPS at M=2048"
GROUP = 128
TL_LAYERS = [("q", 2048, 2048), ("k", 256, 2048), ("v", 256, 2048), ("o", 2048, 2048),
             ("gate", 5632, 2048), ("up", 5632, 2048), ("down", 2048, 5632)]
MALL_BYTES = 256 << 20
SPEC_HBM_GBPS = 8000.0
SPEC_FP16_TFLOPS = 2500.0
REFERENCE_PCT_OF_COPY = 79.0  # reference's 7-layer aggregate on its own GPU


def algo_bytes(m: int, n: int, k: int, g: int = GROUP) -> int:
    return n * k // 2 + 2 * n * (k // g) + 2 * m * k + 2 * m * n


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2400)
    ap.add_argument("--warmup", type=int, default=96)
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="bound on the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-m2048", action="store_true", help="skip the M=2048 GEMM leg")
    ap.add_argument("--verbose", action="store_true")
    return ap.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Timer:
    """Per-launch HIP event pairs, launches queued behind a GPU spin (reference bench_utils.py:114-185)."""

    def __init__(self, torch):
        self.torch = torch
        self.cycles_per_ms = self._calibrate()

    def _calibrate(self) -> float | None:
        torch = self.torch
        if not hasattr(torch.cuda, "_sleep"):
            log("torch.cuda._sleep unavailable: per-launch timing runs without a launch guard")
            return None
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        cycles = 2_000_000
        torch.cuda._sleep(cycles)
        torch.cuda.synchronize()
        s.record()
        torch.cuda._sleep(cycles)
        e.record()
        torch.cuda.synchronize()
        return cycles / max(s.elapsed_time(e), 1e-3)

    def per_launch_ms(self, fns, batch: int = 16, guard_ms: float = 2.0) -> list[float]:
        torch = self.torch
        out = []
        for b0 in range(0, len(fns), batch):
            chunk = fns[b0:b0 + batch]
            evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in chunk]
            if self.cycles_per_ms:
                torch.cuda._sleep(int(guard_ms * self.cycles_per_ms))
            for (s, e), fn in zip(evs, chunk):
                s.record()
                fn()
                e.record()
            torch.cuda.synchronize()
            out += [s.elapsed_time(e) for s, e in evs]
        return out

    def batch_avg_ms(self, fn, reps: int) -> float:
        torch = self.torch
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / reps


def measure_hbm(torch, lib, kl, timer) -> dict:
    """Copy and read ceilings over 1 GiB buffers (4x the MALL), best over grid sizes."""
    nbytes = 1 << 30
    a = torch.empty(nbytes // 4, dtype=torch.int32, device="cuda").fill_(1)
    b = torch.empty_like(a)
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    best = {"copy": 0.0, "read": 0.0}
    for grid in (cus * 4, cus * 8, cus * 16, cus * 32):
        def copy():
            kl.check(lib.kf_bw_copy(a.data_ptr(), b.data_ptr(), nbytes, grid, stream), "copy")

        def read():
            kl.check(lib.kf_bw_read(a.data_ptr(), sink.data_ptr(), nbytes, grid, stream), "read")

        copy(), read()
        t_copy = min(timer.batch_avg_ms(copy, 1) for _ in range(5))
        t_read = min(timer.batch_avg_ms(read, 1) for _ in range(5))
        best["copy"] = max(best["copy"], 2 * nbytes / (t_copy * 1e-3) / 1e9)
        best["read"] = max(best["read"], nbytes / (t_read * 1e-3) / 1e9)
    del a, b
    torch.cuda.empty_cache()
    return {"hbm_copy_gbps": best["copy"], "hbm_read_gbps": best["read"], "buffer_bytes": nbytes}


def measure_mfma_peak(torch, timer) -> float:
    best = 0.0
    for s in (4096, 6144, 8192):
        a = torch.randn(s, s, dtype=torch.float16, device="cuda")
        b = torch.randn(s, s, dtype=torch.float16, device="cuda")
        torch.matmul(a, b)
        t = min(timer.batch_avg_ms(lambda: torch.matmul(a, b), 3) for _ in range(3))
        best = max(best, 2 * s ** 3 / (t * 1e-3) / 1e12)
        del a, b
    torch.cuda.empty_cache()
    return best


def make_layers(torch, kq):
    """Seeded fp32 weights quantized by the package (the format producer), plus x per layer."""
    layers = []
    for i, (name, n, k) in enumerate(TL_LAYERS):
        g = torch.Generator().manual_seed(1000 + i)
        w = torch.randn(n, k, generator=g) * 0.02
        qw = kq.quantize_weight(w, GROUP)
        x = torch.randn(1, k, generator=g).half()
        layers.append((name, n, k, qw.packed, qw.scales, x))
    return layers


def main() -> int:
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures a single GPU: --gpus {args.gpus} (WORLD_SIZE={world}) is not supported. "
              "This build has no multi-GPU path; run with --gpus 1.", file=sys.stderr)
        return 2
    import numpy as np
    import torch

    from kernelforge import _lib as kl
    from kernelforge import ops
    from kernelforge import quantize as kq

    lib = kl.load()
    if not torch.cuda.is_available():
        print("bench.py needs a HIP GPU", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)
    props = torch.cuda.get_device_properties(0)
    timer = Timer(torch)
    stream_ptr = torch.cuda.current_stream().cuda_stream

    log("measuring HBM ceilings")
    ceil = measure_hbm(torch, lib, kl, timer)
    log(f"copy {ceil['hbm_copy_gbps']:.0f} GB/s, read {ceil['hbm_read_gbps']:.0f} GB/s")

    log("quantizing TinyLlama-shaped layers")
    layers = make_layers(torch, kq)
    step_bytes = sum(algo_bytes(1, n, k) for _, n, k, *_ in layers)
    set_bytes = sum(p.numel() * 4 + s.numel() * 2 for *_, p, s, _x in layers)
    copies = max(2, -(-(2 * MALL_BYTES) // set_bytes))
    dev_sets = [[(p.cuda(), s.cuda()) for *_, p, s, _x in layers] for _ in range(copies)]
    xs = [x.cuda() for *_, x in layers]

    # --- the timed step: 7 int4_linear calls, graph-captured, rotating weight copies ---------------
    def run_step(r):
        for li, (name, n, k, *_rest) in enumerate(layers):
            p, s = dev_sets[r][li]
            ops.int4_linear(xs[li], p, s, GROUP)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for r in range(copies):
            run_step(r)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graphs = {}

    def graph_for(count):
        if count not in graphs:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for r in range(count):
                    run_step(r)
            graphs[count] = g
        return graphs[count]

    def run_steps(n_steps):
        full, rem = divmod(n_steps, copies)
        for _ in range(full):
            graph_for(copies).replay()
        if rem:
            graph_for(rem).replay()

    log(f"{copies} weight copies ({copies * set_bytes / 2**20:.0f} MiB); warmup {args.warmup} steps")
    run_steps(args.warmup)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run_steps(args.steps)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"7-layer step {ms_per_step * 1e3:.2f} us -> {value:.0f} GB/s")

    # --- dominant kernel: M=1 GEMV on the gate shape, per-launch events, MALL-cold ----------------
    gate_idx = [nm for nm, *_ in layers].index("gate")
    _, gn, gk, *_ = layers[gate_idx]
    y_gate = torch.empty(1, gn, dtype=torch.float16, device="cuda")

    def gemv_launch(r, li=gate_idx, y=None):
        _, n, k, *_r = layers[li]
        p, s = dev_sets[r][li]
        yy = y if y is not None else y_gate
        return lambda: kl.check(lib.kf_int4_gemv(xs[li].data_ptr(), p.data_ptr(), s.data_ptr(), yy.data_ptr(),
                                                 1, n, k, GROUP, stream_ptr), "gemv")

    launches = [gemv_launch(i % copies) for i in range(8 * copies)]
    for f in launches[:copies]:
        f()
    durs = timer.per_launch_ms(launches)
    gate_avg_ms = statistics.fmean(durs)
    gate_bytes = algo_bytes(1, gn, gk)
    achieved = gate_bytes / (gate_avg_ms * 1e-3) / 1e9
    log(f"gate GEMV avg {gate_avg_ms * 1e3:.2f} us over {len(durs)} launches -> {achieved:.0f} GB/s")

    # --- per-layer isolated kernel times (reference protocol: median of per-launch events) ---------
    per_layer = {}
    sum_med = 0.0
    for li, (name, n, k, *_r) in enumerate(layers):
        yl = torch.empty(1, n, dtype=torch.float16, device="cuda")
        fl = [gemv_launch(i % copies, li, yl) for i in range(4 * copies)]
        d = sorted(timer.per_launch_ms(fl))
        med = statistics.median(d)
        sum_med += med
        b = algo_bytes(1, n, k)
        per_layer[name] = {"N": n, "K": k, "bytes": b, "median_us": round(med * 1e3, 3),
                           "p10_us": round(d[len(d) // 10] * 1e3, 3), "p90_us": round(d[(9 * len(d)) // 10] * 1e3, 3),
                           "gbps": round(b / (med * 1e-3) / 1e9, 1),
                           "pct_of_copy": round(100 * b / (med * 1e-3) / 1e9 / ceil["hbm_copy_gbps"], 1)}
    isolated_gbps = step_bytes / (sum_med * 1e-3) / 1e9

    # --- M=2048: MFMA GEMM on every shape ------------------------------------------------------------
    m2048 = None
    if not args.no_m2048:
        log("M=2048 GEMM leg")
        mfma_peak = measure_mfma_peak(torch, timer)
        total_flops, total_ms, per = 0.0, 0.0, {}
        for li, (name, n, k, *_r) in enumerate(layers):
            xm = torch.randn(2048, k, dtype=torch.float16, device="cuda")
            p, s = dev_sets[0][li]
            ops.int4_gemm(xm, p, s, GROUP)
            t = statistics.median(timer.batch_avg_ms(lambda: ops.int4_gemm(xm, p, s, GROUP), 5) for _ in range(5))
            fl = 2.0 * 2048 * n * k
            per[name] = {"us": round(t * 1e3, 1), "tflops": round(fl / (t * 1e-3) / 1e12, 1)}
            total_flops += fl
            total_ms += t
            del xm
        gate_tf = per["gate"]["tflops"]
        m2048 = {"gate_tflops": gate_tf, "seven_layer_tflops": round(total_flops / (total_ms * 1e-3) / 1e12, 1),
                 "measured_fp16_mfma_peak_tflops": round(mfma_peak, 1),
                 "gate_frac_of_measured_peak": round(gate_tf / mfma_peak, 4),
                 "gate_frac_of_spec_peak": round(gate_tf / SPEC_FP16_TFLOPS, 4), "per_layer": per}
        log(f"M=2048 gate {gate_tf} TFLOPS; hipBLASLt fp16 peak {mfma_peak:.0f} TFLOPS")

    # --- CPU baseline: the oracle's FP32 dequant + matmul on the host cores ------------------------
    cpu = None
    if not args.no_cpu:
        from threadpoolctl import threadpool_limits

        from oracle import int4_oracle as o

        threads = min(len(os.sched_getaffinity(0)), 16)
        host = [(p.numpy(), s.numpy(), x.numpy()) for *_, p, s, x in layers]
        with threadpool_limits(limits=threads):
            for p, s, x in host:  # warm-up
                o.linear_ref_fp32(x, p, s, GROUP)
            times = []
            t_end = time.perf_counter() + args.cpu_seconds
            while time.perf_counter() < t_end or len(times) < 3:
                t1 = time.perf_counter()
                for p, s, x in host:
                    o.linear_ref_fp32(x, p, s, GROUP)
                times.append(time.perf_counter() - t1)
        med = statistics.median(times)
        cpu = {"value": round(step_bytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": f"{len(times)} steps of the 7 TinyLlama linears at M=1 (oracle FP32 dequant+matmul, "
                         f"numpy; BLAS on {threads} threads, unpack single-threaded); median {med * 1e3:.1f} ms/step",
               "cpu_model": _cpu_model()}
        log(f"CPU baseline {cpu['value']} GB/s ({med * 1e3:.1f} ms/step)")

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": "tinyllama_7_linears_m1_g128", "shapes_NxK": [[n, k] for _, n, k in TL_LAYERS],
                   "group_size": GROUP, "bytes_per_step": step_bytes, "weight_copies_rotated": copies,
                   "graph_captured": True},
        "pct_of_measured_copy": round(100 * value / ceil["hbm_copy_gbps"], 1),
        "pct_of_measured_read": round(100 * value / ceil["hbm_read_gbps"], 1),
        "reference_pct_of_copy_on_its_gpu": REFERENCE_PCT_OF_COPY,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": SPEC_HBM_GBPS, "unit": "GB/s",
                     "frac": round(achieved / SPEC_HBM_GBPS, 4), "traffic": None,
                     "kernel": "gemv_kernel M=1 gate 5632x2048", "bytes_per_launch": gate_bytes,
                     "avg_launch_us": round(gate_avg_ms * 1e3, 3),
                     "frac_of_measured_copy": round(achieved / ceil["hbm_copy_gbps"], 4)},
        "cpu_baseline": cpu,
        "ceilings": {k: round(v, 1) if isinstance(v, float) else v for k, v in ceil.items()},
        "isolated_sum_of_medians_gbps": round(isolated_gbps, 1),
        "per_layer_m1": per_layer,
        "m2048": m2048,
        "device": props.name, "cu_count": props.multi_processor_count,
    }
    print(json.dumps(line), flush=True)
    return 0


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    sys.exit(main())
