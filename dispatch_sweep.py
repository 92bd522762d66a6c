"""GEMV / GEMM crossover sweep on one GPU, the MI355X counterpart of the
reference's bench/sweep_int4_dispatch.py.

For every layer shape and M it times ``ops.int4_gemv`` (M <= 8) and ``ops.int4_gemm`` with HIP
events around graph replays of back-to-back launches (weights rotated so each launch reads them
from HBM), and applies the reference's rule (bench/sweep_int4_dispatch.py:51-57): GEMV_MAX_M is
the largest M at which the sum of GEMV times over the shapes is below the sum of GEMM times.
With ``--fp16`` it also times ``F.linear`` on fp16 weights of the same shape (hipBLASLt), the
baseline the reference's bench/bench_gemm.py:83 calls ``cublas_fp16``.

    python dispatch_sweep.py [--out sweep.json] [--ms 1,2,4,8,16] [--fp16] [--mfma16]

A measurement harness beside bench.py, not part of the package.
"""

from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parent / "kernel-forge_amd"))

from kernelforge import ops  # noqa: E402
from kernelforge import quantize as kq  # noqa: E402

SHAPES = {  # (N, K)
    "tinyllama_qo": (2048, 2048), "tinyllama_kv": (256, 2048), "tinyllama_gate_up": (5632, 2048),
    "tinyllama_down": (2048, 5632), "qwen_qo": (1536, 1536), "qwen_kv": (256, 1536),
    "qwen_gate_up": (8960, 1536), "qwen_down": (1536, 8960),
}
CONFIG4_MS = [1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 2048]
MALL_BYTES = 256 << 20


def time_us(fn_for_copy, copies: int, reps: int = 3) -> float:
    """Average µs per call over graph replays of `copies` back-to-back calls (one per weight copy)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for c in range(copies):
            fn_for_copy(c)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for c in range(copies):
            fn_for_copy(c)
    g.replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        g.replay()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) * 1e3 / (reps * copies)


def sweep(ms: list[int], shapes: dict, group: int = 128, fp16: bool = False) -> dict:
    res = {}
    for name, (n, k) in shapes.items():
        w = torch.randn(n, k, generator=torch.Generator().manual_seed(n + k)) * 0.02
        qw = kq.quantize_weight(w, group)
        copies = max(2, min(32, -(-(2 * MALL_BYTES) // qw.nbytes)))
        dev = [(qw.packed.cuda(), qw.scales.cuda()) for _ in range(copies)]
        w16 = []
        if fp16:
            copies16 = max(2, min(32, -(-(2 * MALL_BYTES) // (2 * n * k))))
            w16 = [w.half().cuda() for _ in range(copies16)]
        res[name] = {}
        for m in ms:
            x = torch.randn(m, k, device="cuda").half()
            row = {}
            if m <= 8:
                row["gemv_us"] = time_us(lambda c: ops.int4_gemv(x, dev[c][0], dev[c][1], group), copies)
            if n % 64 == 0:
                row["gemm_us"] = time_us(lambda c: ops.int4_gemm(x, dev[c][0], dev[c][1], group), copies)
                plan = ops.gemm_plan(m, n, k, group)
                row["gemm_kernel"] = f"{plan['kernel']}/{plan['splits']}"  # tile-table index (or skinny) / splits
            row["tflops_best"] = 2 * m * n * k / min(v for kk, v in row.items() if kk.endswith("_us")) / 1e6
            if w16:
                row["fp16_us"] = time_us(lambda c: torch.nn.functional.linear(x, w16[c]), len(w16))
                int4_us = min(v for kk, v in row.items() if kk in ("gemv_us", "gemm_us"))
                row["fp16_over_int4"] = row["fp16_us"] / int4_us
            res[name][m] = row
            print(f"{name} M={m}: " + " ".join(f"{kk}={v:.2f}" if isinstance(v, float) else f"{kk}={v}"
                                              for kk, v in row.items()), flush=True)
        del dev, w16
        torch.cuda.empty_cache()
    return res


def crossover(res: dict, ms: list[int]) -> int:
    """Largest M (<= 8) with sum of GEMV times < sum of GEMM times (reference rule)."""
    best = 0
    for m in ms:
        if m > 8:
            continue
        g = sum(r[m]["gemv_us"] for r in res.values() if "gemm_us" in r[m])
        t = sum(r[m]["gemm_us"] for r in res.values() if "gemm_us" in r[m])
        if g < t:
            best = m
    return best


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--ms", default="1,2,3,4,5,6,7,8,9,16,32,64,128,256,512,2048")
    ap.add_argument("--shapes", default=",".join(SHAPES))
    ap.add_argument("--out", default=None)
    ap.add_argument("--fp16", action="store_true", help="also time F.linear on fp16 weights (hipBLASLt)")
    ap.add_argument("--mfma16", action="store_true",
                    help="int4_gemm builds and reads the MFMA-16 weight copy (ops.MFMA16_CACHE = True); "
                         "default: the public layout")
    args = ap.parse_args()
    ops.MFMA16_CACHE = bool(args.mfma16)
    ms = [int(v) for v in args.ms.split(",")]
    shapes = {s: SHAPES[s] for s in args.shapes.split(",")}
    res = sweep(ms, shapes, fp16=args.fp16)
    out = {"results_us": res, "gemv_max_m": crossover(res, ms), "current_GEMV_MAX_M": ops.GEMV_MAX_M,
           "mfma16_cache": ops.MFMA16_CACHE,
           "device": torch.cuda.get_device_name(0)}
    print(json.dumps({"gemv_max_m": out["gemv_max_m"]}), flush=True)
    if args.out:
        Path(args.out).write_text(json.dumps(out, indent=1))


if __name__ == "__main__":
    main()
