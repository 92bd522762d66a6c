#!/usr/bin/env python3
"""Headline benchmark of the MI355X INT4 weight-only linear path (one GPU).

Metric: "int4_linear M=1 HBM GB/s (% peak) over 7 layers; TFLOPS at M=2048".

Workload: the 7 TinyLlama-1.1B decoder linears (q, k, v,
o, gate, up, down; G=128) at M=1.  Weights W ~ 0.02 N(0,1) fp32 per layer
(seeded) quantized by the package's quantize_weight, x ~ N(0,1) fp16 per
layer: synthetic, resident in HBM.  A *step* computes all 7 linears once;
``value`` = the 7-layer algorithmic bytes (22,779,904 B, formula of
bench/bench_gemm.py:80,98) / time per step, in GB/s.

The 7 problems of a step are independent, so the step is one
``ops.int4_linear_grouped`` call: one GEMV launch over all 7 (each output is
bit-identical to its own ``int4_linear``).  Two other step structures are
timed and reported beside it:
  * decoder: the launches a real decoder layer can make, where q|k|v share x
    and gate|up share x: grouped(q,k,v), o, grouped(gate,up), down;
  * separate: 7 ``ops.int4_linear`` calls, one launch each (the reference's
    per-layer structure).

Protocol
* Infinity-Cache-cold: R copies of the 7-layer weight set (R * 22.8 MB >= 2x
  the 256 MB MALL) are rotated, step i using copy i % R.
* W warm-up steps, then exactly K timed steps, bracketed by
  torch.cuda.synchronize() and timed by a HIP event pair on the launching
  stream behind a GPU spin (the reference's launch guard), so host launch cost
  is excluded.  K <= 512: the K steps are eager launches of the op's C-ABI call
  with each weight copy's problem table built once, queued behind a spin longer
  than their enqueue (a HIP graph launch has ~6 us of fixed cost on ROCm, 5% of
  the step at K = 20), after two untimed runs of that same pattern (the first
  two in a process read slow); larger K: replays of HIP graphs (R steps per graph, as in
  the reference's CUDA-graph decode), all captured before timing.  The graph
  timing of the same K and the host wall clock are reported beside it.
* roofline: the dominant kernel is the grouped GEMV (the whole step, one launch
  per step), so its average duration per launch is the timed region's event
  time / K; achieved = 22,779,904 B / that duration.
* reference_protocol: the same step timed the reference's way
  (kernelforge/bench_utils.py:114-185): 50 eager calls, each behind a GPU spin
  guard and between its own event pair; median / p10 / p90 per call.  It
  includes each call's launch and one event pair, so it sits above the
  graph-replay average.
* ceilings: HBM copy/read peaks measured in the same run with the library's
  dwordx4 kernels on 1 GiB buffers; fp16 MFMA peak with torch.matmul
  (hipBLASLt) at 4096/6144/8192.  Also the bare read of exactly one step's
  bytes in one launch (same rotation and graph protocol): the ceiling a
  one-launch step of this size can reach, launch and ramp included.
* M=2048 (BASELINE config 4's largest point): the MFMA GEMM on every
  TinyLlama shape, 10 launches per HIP graph, HIP events around replays;
  TFLOPS = 2*M*N*K / time, for gate and the 7-layer sum, each beside
  hipBLASLt's dense fp16 GEMM on the same shape (torch F.linear with fp16
  weights, same protocol).
* per-layer, step-structure, Qwen2.5 (config 3) and quantize legs: graph replays
  of several steps, the median of five timed regions, each after an untimed
  run of the same graph.
* cpu_baseline: the reference's FP32 dequant + matmul restated in torch
  (oracle/cpu_baseline.py) on the host cores over a bounded sample, per call
  and matmul-only.
* --headline-only: only the ceilings and the timed step (the command whose
  rocprofv3 kernel trace backs roofline.avg_launch_us).

--gpus N > 1 is refused: this build measures one GPU.
"""

from __future__ import annotations

import argparse
import csv
import json
import os
import shutil
import statistics
import subprocess
import sys
import tempfile
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
QWEN_LAYERS = [("q", 1536, 1536), ("k", 256, 1536), ("v", 256, 1536), ("o", 1536, 1536),
               ("gate", 8960, 1536), ("up", 8960, 1536), ("down", 1536, 8960)]
REFERENCE_QWEN_PCT_OF_COPY = 79.4  # reference's Qwen2.5 7-layer aggregate on its own GPU
MALL_BYTES = 256 << 20
SPEC_HBM_GBPS = 8000.0
SPEC_FP16_TFLOPS = 2500.0
REFERENCE_PCT_OF_COPY = 79.0  # reference's 7-layer aggregate on its own GPU (RTX 4060 Laptop)


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
    ap.add_argument("--profile", choices=["gemv_grouped", "gemm_m2048", "blas_m2048", "copy", "decode", "quantize"],
                    help="only launch one kernel --profile-iters times (for rocprofv3 --pmc runs) and exit")
    ap.add_argument("--profile-iters", type=int, default=20)
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 FETCH_SIZE/WRITE_SIZE passes")
    ap.add_argument("--no-e2e", action="store_true", help="skip the TinyLlama graph-decode leg (config 5)")
    ap.add_argument("--no-quant", action="store_true", help="skip the on-device quantize leg")
    ap.add_argument("--headline-only", action="store_true",
                    help="only the ceilings and the timed grouped step (the command profiles/ traces)")
    ap.add_argument("--power", action="store_true",
                    help="only the board power / clock of the M=2048 gate GEMM run back to back (INT4 and "
                         "hipBLASLt fp16), from amd-smi samples; prints one JSON line")
    ap.add_argument("--power-seconds", type=float, default=3.0)
    return ap.parse_args()


def _pmc_median_kib(counter: str, profile: str, kernel_substr: str, outdir: str) -> float | None:
    """Runs this script under `rocprofv3 --pmc <counter>` in --profile mode; median KiB per dispatch."""
    name = f"{profile}_{counter}"
    cmd = ["rocprofv3", "--pmc", counter, "--output-format", "csv", "-d", outdir, "-o", name, "--",
           sys.executable, "-u", str(Path(__file__).resolve()), "--profile", profile, "--profile-iters", "10"]
    env = dict(os.environ, TMPDIR="/tmp")
    try:
        subprocess.run(cmd, timeout=120, capture_output=True, env=env, cwd="/tmp")
    except (OSError, subprocess.SubprocessError):
        return None
    vals = []
    for f in Path(outdir).rglob(f"{name}*counter_collection.csv"):
        with open(f) as fh:
            for row in csv.DictReader(fh):
                if kernel_substr in row.get("Kernel_Name", "") and row.get("Counter_Name") == counter:
                    vals.append(float(row["Counter_Value"]))
    return statistics.median(vals) if vals else None


def measure_traffic() -> dict | None:
    """HBM bytes per grouped-GEMV launch from FETCH_SIZE and WRITE_SIZE, each calibrated against a
    64 MiB copy (known to read and write 65,536 KiB).  Runs before this process touches the GPU;
    returns None when rocprofv3 is unavailable or a pass fails."""
    if shutil.which("rocprofv3") is None:
        return None
    outdir = tempfile.mkdtemp(prefix="kf_pmc_")
    try:
        cf = _pmc_median_kib("FETCH_SIZE", "copy", "bw_copy_kernel", outdir)
        cw = _pmc_median_kib("WRITE_SIZE", "copy", "bw_copy_kernel", outdir)
        gf = _pmc_median_kib("FETCH_SIZE", "gemv_grouped", "gemv_grouped_kernel", outdir)
        gw = _pmc_median_kib("WRITE_SIZE", "gemv_grouped", "gemv_grouped_kernel", outdir)
    finally:
        shutil.rmtree(outdir, ignore_errors=True)
    if not all(v for v in (cf, cw, gf)) or gw is None:
        return None
    fetch_factor, write_factor = 65536.0 / cf, 65536.0 / cw
    return {"bytes": (gf * fetch_factor + gw * write_factor) * 1024.0, "fetch_kib": gf, "write_kib": gw,
            "fetch_factor": round(fetch_factor, 4), "write_factor": round(write_factor, 4)}


def profile_only(args, torch, lib, kl, ops, kq) -> int:
    """Launches one kernel a fixed number of times, eagerly, for counter collection.

    gemv_grouped: the grouped 7-layer GEMV (22,779,904 algorithmic bytes per launch), rotating
      weight copies so every launch reads its weights from HBM.
    gemm_m2048:  the MFMA GEMM on the gate shape at M=2048.
    blas_m2048:  hipBLASLt's dense fp16 GEMM (torch F.linear) on the same shape, for comparison.
    copy:        kf_bw_copy of 64 MiB (64 MiB read + 64 MiB written per launch), the known-size
      kernel that calibrates FETCH_SIZE / WRITE_SIZE.
    decode:      the INT4 TinyLlama of the e2e leg: 16-token prompt, capture, --profile-iters graph
      replays of the decode step (for a kernel trace of one token).
    quantize:    the on-device quantize + pack of the quantize leg (fp32 gate 5632 x 2048, G=128),
      weights rotated over more than twice the MALL as in that leg.
    """
    stream = torch.cuda.current_stream().cuda_stream
    if args.profile == "copy":
        nbytes = 64 << 20
        a = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(args.profile_iters):
            kl.check(lib.kf_bw_copy(a.data_ptr(), b.data_ptr(), nbytes, 0, stream), "copy")
    elif args.profile == "decode":
        from kernelforge import tinyllama as tl
        import dataclasses

        cfg = dataclasses.replace(tl.TinyLlamaConfig(), max_seq=16 + args.profile_iters + 3)
        dec = tl.GraphDecoder(tl.build_int4_model(cfg, "cuda", seed=0), "cuda")
        gen = torch.Generator(device="cuda").manual_seed(1)
        dec.prefill(torch.randint(0, cfg.vocab, (16,), device="cuda", generator=gen))
        dec.capture()
        dec.decode(args.profile_iters)
    elif args.profile == "gemm_m2048":
        layers = make_layers(torch, kq)
        gate = [ly for ly in layers if ly["name"] == "gate"][0]
        p, s = gate["packed"].cuda(), gate["scales"].cuda()
        x = torch.randn(2048, gate["K"], dtype=torch.float16, device="cuda")
        for _ in range(args.profile_iters):
            ops.int4_gemm(x, p, s, GROUP)
    elif args.profile == "quantize":
        qn, qk = 5632, 2048
        qcopies = max(2, -(-(2 * MALL_BYTES) // (qn * qk * 4)))
        wq = [torch.randn(qn, qk, device="cuda") * 0.02 for _ in range(qcopies)]
        for i in range(args.profile_iters):
            ops.int4_quantize(wq[i % qcopies], GROUP)
    elif args.profile == "blas_m2048":
        x = torch.randn(2048, 2048, dtype=torch.float16, device="cuda")
        w = torch.randn(5632, 2048, dtype=torch.float16, device="cuda")
        for _ in range(args.profile_iters):
            torch.nn.functional.linear(x, w)
    else:
        layers = make_layers(torch, kq)
        set_bytes = sum(ly["packed"].numel() * 4 + ly["scales"].numel() * 2 for ly in layers)
        copies = max(2, -(-(2 * MALL_BYTES) // set_bytes))
        dev = [[(ly["packed"].cuda(), ly["scales"].cuda()) for ly in layers] for _ in range(copies)]
        xs = [ly["x"].cuda() for ly in layers]
        for i in range(args.profile_iters):
            r = i % copies
            ops.int4_linear_grouped(xs, [d[0] for d in dev[r]], [d[1] for d in dev[r]], GROUP)
    torch.cuda.synchronize()
    print(f"profiled {args.profile} x{args.profile_iters}", flush=True)
    return 0


def e2e_decode(torch, prompt_len: int = 16, new_tokens: int = 128) -> dict:
    """random-init TinyLlama architecture, greedy decode with one HIP-graph-captured
    step, tokens/s over `new_tokens` back-to-back replays.  INT4 (q|k|v and gate|up fused), INT4
    with the 7 linears unfused, and the same network with fp16 nn.Linear layers (hipBLASLt)."""
    import dataclasses

    from kernelforge import tinyllama as tl

    dev = torch.device("cuda")
    cfg = dataclasses.replace(tl.TinyLlamaConfig(), max_seq=prompt_len + new_tokens + 1)
    prompt = torch.randint(0, cfg.vocab, (prompt_len,), generator=torch.Generator().manual_seed(7)).to(dev)
    out = {"model": "tinyllama-1.1b-arch random-init", "layers": cfg.layers, "prompt": prompt_len,
           "new_tokens": new_tokens}

    def run(model):
        dec = tl.GraphDecoder(model, dev)
        dec.prefill(prompt)
        dec.capture()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        dec.decode(new_tokens)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        return new_tokens / dt, dec.generated(prompt_len, new_tokens)

    for label, kw in (("int4_fused", {"fuse": True}), ("int4_unfused", {"fuse": False})):
        model = tl.build_int4_model(cfg, dev, seed=0, **kw)
        tps, toks = run(model)
        out[f"{label}_tok_s"] = round(tps, 1)
        out[f"{label}_first_tokens"] = toks[:8].tolist()
        if label == "int4_fused":
            out["mfma16_copies"] = mfma16_copy_report(model)
        del model
        torch.cuda.empty_cache()
    with torch.device(dev):
        fp16 = tl.TinyLlama(cfg)
    fp16.init_random_(0).half().eval()
    out["fp16_tok_s"] = round(run(fp16)[0], 1)
    del fp16
    torch.cuda.empty_cache()
    return out


def hf_llama_decode(torch, prompt_len: int = 16, new_tokens: int = 64) -> dict:
    """The reference's real caller at decode: a transformers LlamaForCausalLM of the TinyLlama
    architecture (config 5's shapes, random init, SDPA attention, fp16), its 7 decoder linears
    per layer swapped by quantize_linears_, decoded the way the reference's harness does
    (bench/e2e_model.py:85-141: StaticCache, one decode step captured in a HIP graph, each replay
    followed by the argmax copy, the position bump and a host sync; tokens/s = 1 / median step).
    Three models: the INT4 modules as quantize_linears_ leaves them, the same after
    group_sibling_linears_ (q|k|v and gate|up as one grouped launch each), and fp16 weights."""
    import transformers
    from transformers import StaticCache

    from kernelforge import modules

    dev = torch.device("cuda")
    cfg = transformers.LlamaConfig(vocab_size=32000, hidden_size=2048, intermediate_size=5632, num_hidden_layers=22,
                                   num_attention_heads=32, num_key_value_heads=4, head_dim=64,
                                   max_position_embeddings=2048, rms_norm_eps=1e-5, rope_theta=10000.0,
                                   tie_word_embeddings=False, attn_implementation="sdpa")
    prompt = torch.randint(0, cfg.vocab_size, (1, prompt_len), generator=torch.Generator().manual_seed(7)).to(dev)
    out = {"model": "transformers LlamaForCausalLM, tinyllama-1.1b-arch random-init, sdpa", "prompt": prompt_len,
           "new_tokens": new_tokens, "protocol": "bench/e2e_model.py graph_decode: median step incl. argmax + sync"}

    def graph_decode(model):
        p = prompt.shape[1]
        cache = StaticCache(config=model.config, max_cache_len=p + new_tokens + 8)
        logits = model(prompt, cache_position=torch.arange(p, device=dev), past_key_values=cache, use_cache=True).logits
        tok = logits[:, -1:].argmax(-1).clone()
        tokens = [tok.item()]
        pos = torch.tensor([p], device=dev)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                model(tok, cache_position=pos, past_key_values=cache, use_cache=True)
        torch.cuda.current_stream().wait_stream(side)
        for layer in cache.layers:
            if hasattr(layer, "cumulative_length"):
                layer.cumulative_length.fill_(p)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            logits = model(tok, cache_position=pos, past_key_values=cache, use_cache=True).logits
        times = []
        for _ in range(new_tokens):
            t = time.perf_counter()
            graph.replay()
            tok.copy_(logits[:, -1:].argmax(-1))
            pos.add_(1)
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t)
            tokens.append(tok.item())
        del graph, cache
        med = statistics.median(times)
        return round(1.0 / med, 1), round(med * 1e3, 4), tokens

    with torch.no_grad():
        torch.manual_seed(0)
        with torch.device(dev):
            model = transformers.LlamaForCausalLM(cfg)
        model = model.half().eval()
        fp16 = graph_decode(model)
        out["fp16_tok_s"], out["fp16_step_ms"] = fp16[0], fp16[1]
        modules.quantize_linears_(model, GROUP)
        plain = graph_decode(model)
        out["int4_tok_s"], out["int4_step_ms"] = plain[0], plain[1]
        out["grouped_siblings"] = modules.group_sibling_linears_(model)
        grouped = graph_decode(model)
        out["int4_grouped_tok_s"], out["int4_grouped_step_ms"] = grouped[0], grouped[1]
        out["grouped_tokens_equal_ungrouped"] = grouped[2] == plain[2]
        out["first_tokens"] = plain[2][:8]
    del model
    torch.cuda.empty_cache()
    return out


def mfma16_copy_report(model) -> dict:
    """Device memory of the MFMA-16 weight copies int4_gemm attached to the model's INT4 weights
    (built on the first skinny-kernel call per weight: here the 16-token prefill), against the
    INT4 weights themselves."""
    from kernelforge import ops

    storages, copies, copy_bytes = {}, 0, 0
    for mod in model.modules():
        packed, scales = getattr(mod, "packed", None), getattr(mod, "scales", None)
        if packed is None or scales is None:
            continue
        for t in (packed, scales):  # a fused module's parts are views of its buffers: count storages
            storages[t.untyped_storage().data_ptr()] = t.untyped_storage().nbytes()
        cached = getattr(packed, ops._MFMA16_ATTR, None)
        if cached is not None:
            copies += 1
            copy_bytes += cached[1].numel() * 4 + cached[2].numel() * 2
    int4 = sum(storages.values())
    return {"weights_with_copy": copies, "copy_bytes": copy_bytes, "int4_weight_bytes": int4,
            "copy_over_int4_weights": round(copy_bytes / int4, 3) if int4 else None,
            "note": "second layout of each weight the skinny kernel has run on (ops.MFMA16_CACHE)"}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _timed_ms(fn) -> float:
    t0 = time.perf_counter()
    fn()
    return (time.perf_counter() - t0) * 1e3


_SPIN_CYCLES_PER_MS = None


def spin_cycles_per_ms(torch) -> float:
    """Cycles of torch.cuda._sleep per millisecond, from one timed 1M-cycle spin (cached)."""
    global _SPIN_CYCLES_PER_MS
    if _SPIN_CYCLES_PER_MS is None:
        torch.cuda._sleep(100_000)
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        torch.cuda._sleep(1_000_000)
        e.record()
        torch.cuda.synchronize()
        _SPIN_CYCLES_PER_MS = 1_000_000 / max(s.elapsed_time(e), 1e-3)
    return _SPIN_CYCLES_PER_MS


class GraphSteps:
    """Runs `count` steps as replays of captured graphs; step i uses weight copy i % copies.

    Graphs are built by prepare(); run() only replays, so a timed run() never captures or
    instantiates a graph (it raises if one is missing)."""

    def __init__(self, torch, step_fn, copies: int):
        self.torch, self.step_fn, self.copies = torch, step_fn, copies
        self.graphs = {}
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # eager warm-up off the capture path
            for r in range(copies):
                step_fn(r)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()

    def _sizes(self, count: int) -> list[int]:
        full, rem = divmod(count, self.copies)
        return [self.copies] * full + ([rem] if rem else [])

    def prepare(self, count: int) -> None:
        """Captures every graph run(count) replays, and replays each new one once: a graph's first
        launch also does one-time work (its kernel arguments are uploaded to the device), which
        must not land in a timed run."""
        for n in set(self._sizes(count)):
            if n not in self.graphs:
                g = self.torch.cuda.CUDAGraph()
                with self.torch.cuda.graph(g):
                    for r in range(n):
                        self.step_fn(r)
                self.graphs[n] = g
                g.replay()
        self.torch.cuda.synchronize()

    def run(self, count: int) -> None:
        sizes = self._sizes(count)
        missing = sorted({n for n in sizes if n not in self.graphs})
        if missing:
            raise RuntimeError(f"GraphSteps.run({count}): graphs of {missing} steps not prepared")
        for n in sizes:
            self.graphs[n].replay()

    def timed(self, count: int, guard_ms: float = 0.2) -> tuple[float, float]:
        """(ms per step from a HIP event pair on the launching stream, wall-clock ms per step),
        both over exactly `count` replayed steps bracketed by synchronize().

        A GPU spin of `guard_ms` runs before the start event (the reference's launch guard,
        kernelforge/bench_utils.py:114-185), so the replays are already queued when the start
        event fires and host launch latency does not count as GPU time.  The wall clock runs
        from the first enqueue to the final synchronize, minus the spin."""
        torch = self.torch
        self.prepare(count)
        cycles = int(guard_ms * spin_cycles_per_ms(torch))
        torch.cuda.synchronize()
        g, s, e = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        t0 = time.perf_counter()
        g.record()
        torch.cuda._sleep(cycles)
        s.record()
        self.run(count)
        e.record()
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3 - g.elapsed_time(s)
        return s.elapsed_time(e) / count, wall_ms / count

    def event_avg_ms(self, count: int) -> float:
        """Average time per step from one HIP event pair on the launching stream (after one
        untimed run of the same count)."""
        self.prepare(count)
        self.run(count)
        return self.timed(count)[0]


BOUND_MAX_STEPS = 512  # longest timed region run as eager launches behind one spin (BoundSteps)
BOUND_REHEARSALS = 2   # untimed runs of that region's pattern before the timed one


class BoundSteps:
    """The headline step as eager launches of kf_int4_gemv_grouped, the C-ABI call
    ops.int4_linear_grouped makes, with each weight copy's problem table built once: step i runs
    the same kernel on the same 7 problems, reading weight copy i % copies and writing outputs
    shared by every call (as graph replays share theirs).

    A timed run queues its `count` launches behind a GPU spin longer than their host enqueue
    time, so the GPU runs them back to back: one HIP graph launch costs ~6 us of fixed time on
    ROCm (a timed region of K graph-replayed steps measured 8.5 us + 5.69 us per step, eager
    launches behind a spin 2.4 us + 5.69 us per step), which at the driver's K = 20 is 5% of
    the step.  Each run checks that the host had queued every launch before the spin ended."""

    def __init__(self, torch, kl, lib, xs, dev, group: int):
        self.torch, self.m, self.group, self.count = torch, xs[0].shape[0], group, len(xs)
        if self.count > kl.GEMV_MAX_GROUP:
            raise ValueError(f"one grouped launch takes at most {kl.GEMV_MAX_GROUP} problems")
        self.ys = [torch.empty(self.m, p.shape[0], dtype=torch.float16, device=xs[0].device) for p, _ in dev[0]]
        self.tables = []
        for weights in dev:
            table = (kl.GemvProblem * self.count)()
            for j, (x, (p, s), y) in enumerate(zip(xs, weights, self.ys)):
                table[j] = kl.GemvProblem(x.data_ptr(), p.data_ptr(), s.data_ptr(), y.data_ptr(), p.shape[0],
                                          x.shape[1])
            self.tables.append(table)
        self.fn, self.kl = lib.kf_int4_gemv_grouped, kl
        self.stream = torch.cuda.current_stream().cuda_stream

    def launch(self, i: int) -> None:
        st = self.fn(self.tables[i % len(self.tables)], self.count, self.m, self.group, self.stream)
        if st:
            self.kl.check(st, "kf_int4_gemv_grouped")

    def enqueue_us(self, n: int = 100) -> float:
        """Host time per launch while the GPU is busy (median of 5 batches of n)."""
        torch = self.torch
        times = []
        for _ in range(5):
            torch.cuda._sleep(int((0.5 + 0.02 * n) * spin_cycles_per_ms(torch)))
            t = time.perf_counter()
            for i in range(n):
                self.launch(i)
            times.append((time.perf_counter() - t) / n * 1e6)
            torch.cuda.synchronize()
        return statistics.median(times)

    def timed(self, count: int) -> dict:
        """ms per step from a HIP event pair on the launching stream around exactly `count` launches,
        between synchronize() calls, and the wall clock over the same launches minus the spin."""
        torch = self.torch
        enq = self.enqueue_us()
        spin_ms = 0.5 + 2.0 * count * enq / 1e3
        torch.cuda.synchronize()
        g, s, e = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        t0 = time.perf_counter()
        g.record()
        torch.cuda._sleep(int(spin_ms * spin_cycles_per_ms(torch)))
        s.record()
        t1 = time.perf_counter()
        for i in range(count):
            self.launch(i)
        queued_ms = (time.perf_counter() - t1) * 1e3
        e.record()
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3 - g.elapsed_time(s)
        return {"ms_per_step": s.elapsed_time(e) / count, "wall_ms_per_step": wall_ms / count,
                "host_enqueue_us": round(enq, 2), "spin_ms": round(g.elapsed_time(s), 3),
                "queued_ms": round(queued_ms, 3), "covered": queued_ms < g.elapsed_time(s)}


def reference_protocol(torch, fn, copies: int, iters: int = 50, warmup: int = 10,
                       min_warmup_ms: float = 100.0) -> dict:
    """The reference's per-call timing (kernelforge/bench_utils.py:114-185), restated: warm up for at
    least `warmup` synchronized calls and `min_warmup_ms`, measure the host enqueue cost, then time
    `iters` eager calls, each behind a GPU spin (torch.cuda._sleep) longer than 5x that cost + 0.5 ms
    and bracketed by its own event pair; median, p10, p90, mean and min per call. Call i uses weight
    copy i % copies, so every timed call reads its weights from HBM."""
    done, t0 = 0, time.perf_counter()
    while done < warmup or (time.perf_counter() - t0) * 1e3 < min_warmup_ms:
        fn(done % copies)
        torch.cuda.synchronize()
        done += 1
    t0 = time.perf_counter()
    for i in range(5):
        fn(i % copies)
    host_ms = (time.perf_counter() - t0) * 1e3 / 5
    torch.cuda.synchronize()
    cycles_per_ms = spin_cycles_per_ms(torch)
    guard_ms = max(1.0, 5.0 * host_ms + 0.5)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    for i in range(iters):
        torch.cuda._sleep(int(guard_ms * cycles_per_ms))
        starts[i].record()
        fn(i % copies)
        ends[i].record()
    torch.cuda.synchronize()
    us = sorted(a.elapsed_time(b) * 1e3 for a, b in zip(starts, ends))

    def pct(p: float) -> float:
        return us[min(len(us) - 1, int(round(p * (len(us) - 1))))]

    return {"median_us": round(statistics.median(us), 3), "p10_us": round(pct(0.10), 3),
            "p90_us": round(pct(0.90), 3), "mean_us": round(statistics.fmean(us), 3), "min_us": round(us[0], 3),
            "iters": iters, "warmup_calls": done, "host_enqueue_us": round(host_ms * 1e3, 1),
            "launch_guard_ms": round(guard_ms, 2)}


def batch_avg_ms(torch, fn, reps: int) -> float:
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps


def measure_hbm(torch, lib, kl) -> dict:
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

        copy()
        read()
        t_copy = min(batch_avg_ms(torch, copy, 1) for _ in range(5))
        t_read = min(batch_avg_ms(torch, read, 1) for _ in range(5))
        best["copy"] = max(best["copy"], 2 * nbytes / (t_copy * 1e-3) / 1e9)
        best["read"] = max(best["read"], nbytes / (t_read * 1e-3) / 1e9)
    del a, b
    torch.cuda.empty_cache()
    return {"hbm_copy_gbps": best["copy"], "hbm_read_gbps": best["read"], "buffer_bytes": nbytes}


def measure_same_size_read(torch, lib, kl, nbytes: int, copies: int = 24) -> dict:
    """The bare-read ceiling for one step: kf_bw_read over exactly `nbytes` in one launch, from
    `copies` disjoint windows rotated so every launch reads from HBM, graph-replayed like the
    step itself.  Best over grid sizes (one 16-byte load per thread, and grid-stride loops).

    Beside it, the same read with the stores a decode GEMV makes (kf_bw_read_store: two fp16 per
    wavefront, as lanes 31 and 63 of a two-row GEMV wavefront store them), and the launch floor:
    a one-workgroup kernel reading 16 bytes, graph-replayed the same way.  A one-launch step that
    writes its outputs cannot be faster than the read with stores."""
    nbytes = nbytes // 16 * 16
    buf = torch.empty(copies * nbytes // 4, dtype=torch.int32, device="cuda").fill_(1)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    one_shot = -(-nbytes // (16 * 256))
    grids = sorted({min(one_shot, 1 << 16), 8 * cus, 16 * cus})
    sink = torch.zeros(16 * max(grids) // 4 + 16, dtype=torch.int32, device="cuda")
    out = {}
    for kind in ("read", "read_store"):
        best = None
        for grid in grids:
            def step(r, grid=grid, kind=kind):
                fn = lib.kf_bw_read if kind == "read" else lib.kf_bw_read_store
                kl.check(fn(buf.data_ptr() + r * nbytes, sink.data_ptr(), nbytes, grid,
                            torch.cuda.current_stream().cuda_stream), kind)
            steps = GraphSteps(torch, step, copies)
            us = statistics.median(steps.event_avg_ms(4 * copies) for _ in range(5)) * 1e3
            if best is None or us < best["us"]:
                best = {"us": round(us, 3), "gbps": round(nbytes / (us * 1e-6) / 1e9, 1), "grid_blocks": grid,
                        "bytes": nbytes}
            del steps
        out[kind] = best

    def floor_step(r):
        kl.check(lib.kf_bw_read(buf.data_ptr() + r * 4096, sink.data_ptr(), 16, 1,
                                torch.cuda.current_stream().cuda_stream), "launch floor")
    steps = GraphSteps(torch, floor_step, copies)
    floor_us = statistics.median(steps.event_avg_ms(4 * copies) for _ in range(5)) * 1e3
    del steps, buf, sink
    torch.cuda.empty_cache()
    best = dict(out["read"])
    best["with_gemv_stores"] = out["read_store"]
    best["launch_floor_us"] = round(floor_us, 3)
    return best


def measure_mfma_peak(torch) -> float:
    best = 0.0
    for s in (4096, 6144, 8192):
        a = torch.randn(s, s, dtype=torch.float16, device="cuda")
        b = torch.randn(s, s, dtype=torch.float16, device="cuda")
        torch.matmul(a, b)
        t = min(batch_avg_ms(torch, lambda: torch.matmul(a, b), 3) for _ in range(3))
        best = max(best, 2 * s ** 3 / (t * 1e-3) / 1e12)
        del a, b
    torch.cuda.empty_cache()
    return best


def make_layers(torch, kq, shapes=TL_LAYERS, seed=1000, group=GROUP):
    """Seeded fp32 weights quantized by the package (the format producer), plus x per layer."""
    layers = []
    for i, (name, n, k) in enumerate(shapes):
        g = torch.Generator().manual_seed(seed + i)
        w = torch.randn(n, k, generator=g) * 0.02
        qw = kq.quantize_weight(w, group)
        x = torch.randn(1, k, generator=g).half()
        layers.append({"name": name, "N": n, "K": k, "packed": qw.packed, "scales": qw.scales, "x": x})
    return layers


def environment(torch, props) -> dict:
    """Software and clock/power state of the box the line was measured on."""
    env = {"device": props.name, "gcn_arch": getattr(props, "gcnArchName", None),
           "cu_count": props.multi_processor_count, "hbm_gib": round(props.total_memory / 2**30, 1),
           "torch": torch.__version__, "torch_hip": torch.version.hip}
    try:
        env["rocm"] = Path("/opt/rocm/.info/version").read_text().strip()
    except OSError:
        env["rocm"] = None
    for key, cmd in (("amd_smi_metric", ["amd-smi", "metric", "-g", "0", "-p", "-c", "--json"]),
                     ("amd_smi_driver", ["amd-smi", "static", "-g", "0", "--driver", "--json"])):
        try:
            out = subprocess.run(cmd, capture_output=True, text=True, timeout=30)
            env[key] = json.loads(out.stdout) if out.returncode == 0 else f"exit {out.returncode}"
        except (OSError, subprocess.SubprocessError, ValueError) as exc:
            env[key] = f"unavailable: {type(exc).__name__}"
    return env


def _board_sample() -> tuple[float, float] | None:
    """(socket power W, mean gfx clock MHz over the XCDs) from one `amd-smi metric` read."""
    try:
        out = subprocess.run(["amd-smi", "metric", "-g", "0", "-p", "-c", "--json"], capture_output=True,
                             text=True, timeout=5)
        d = json.loads(out.stdout)
        g = d[0] if isinstance(d, list) else d["gpu_data"][0]
        clocks = [c["clk"]["value"] for k, c in g["clock"].items()
                  if k.startswith("gfx_") and isinstance(c, dict) and isinstance(c.get("clk"), dict)]
        return float(g["power"]["socket_power"]["value"]), float(statistics.mean(clocks))
    except (OSError, subprocess.SubprocessError, ValueError, KeyError, TypeError, statistics.StatisticsError):
        return None


def power_leg(torch, ops, kq, seconds: float) -> dict:
    """Board power and shader clock while the M=2048 gate GEMM runs back to back.

    The INT4 GEMM (weights of the bench's gate layer, resident) and hipBLASLt's fp16 GEMM on the
    same shape each replay a graph of 20 launches for `seconds`; a thread reads `amd-smi metric`
    every 50 ms, and the medians of the samples after the first 0.5 s of each run are reported
    with the per-launch time (HIP events around all replays) and the rate.  Two rounds, then the
    idle board.  The GEMM's speed is set by the clock the board's power limit allows, which this
    shows."""
    import threading

    samples: list = []
    stop = threading.Event()

    def sampler():
        while not stop.is_set():
            v = _board_sample()
            if v is not None:
                samples.append((time.time(), *v))
            time.sleep(0.05)

    layers = make_layers(torch, kq)
    gate = [ly for ly in layers if ly["name"] == "gate"][0]
    p, s_ = gate["packed"].cuda(), gate["scales"].cuda()
    m, n, k = 2048, gate["N"], gate["K"]
    x = torch.randn(m, k, dtype=torch.float16, device="cuda")
    wf = (torch.randn(n, k, device="cuda") * 0.02).half()

    def graph_of(fn):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                fn()
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(20):
                fn()
        return g

    graphs = {"int4_gemm": graph_of(lambda: ops.int4_gemm(x, p, s_, GROUP)),
              "hipblaslt_fp16": graph_of(lambda: torch.nn.functional.linear(x, wf))}
    th = threading.Thread(target=sampler, daemon=True)
    th.start()
    out: dict = {"shape": [m, n, k], "launches_per_replay": 20, "seconds": seconds, "runs": []}
    try:
        time.sleep(1.5)
        for rnd in range(2):
            for name, g in graphs.items():
                torch.cuda.synchronize()
                t0 = time.time()
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                reps = 0
                while time.time() - t0 < seconds:
                    g.replay()
                    reps += 1
                    if reps % 20 == 0:
                        torch.cuda.synchronize()
                b.record()
                torch.cuda.synchronize()
                t1 = time.time()
                us = a.elapsed_time(b) * 1e3 / (reps * 20)
                sel = [q for q in samples if t0 + 0.5 <= q[0] <= t1]
                out["runs"].append({
                    "kernel": name, "round": rnd, "us_per_launch": round(us, 2),
                    "tflops": round(2.0 * m * n * k / (us * 1e-6) / 1e12, 1),
                    "power_w": statistics.median([q[1] for q in sel]) if sel else None,
                    "gfx_mhz": round(statistics.median([q[2] for q in sel])) if sel else None, "samples": len(sel)})
                log(f"power: {out['runs'][-1]}")
                time.sleep(1.5)
        idle = [q for q in samples if q[0] >= time.time() - 1.0]
        out["idle_power_w"] = statistics.median([q[1] for q in idle]) if idle else None
    finally:
        stop.set()
        th.join(timeout=10)
    return out


def host_enqueue_us(torch, fn, calls: int = 200) -> float:
    """Host time per eager call (launch enqueue, no synchronization), median of 5 batches."""
    for _ in range(20):
        fn()
    torch.cuda.synchronize()
    per = []
    for _ in range(5):
        t0 = time.perf_counter()
        for _ in range(calls):
            fn()
        per.append((time.perf_counter() - t0) * 1e6 / calls)
        torch.cuda.synchronize()
    return round(statistics.median(per), 2)


def cpu_baseline(torch, layers, step_bytes: int, seconds: float) -> dict:
    """The reference's CPU FP32 dequant + matmul (oracle/cpu_baseline.py, torch on the host cores)
    over a bounded sample of the workload: the 7 TinyLlama linears at M=1.  Threads: every core
    in this process's affinity set, capped by OMP_NUM_THREADS where the box sets it (its CPU
    share); both counts are recorded."""
    from oracle import cpu_baseline as cb

    affinity = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    threads = min(affinity, int(omp)) if omp and omp.isdigit() and int(omp) > 0 else affinity
    saved = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        host = [(ly["x"], ly["packed"], ly["scales"]) for ly in layers]
        w_hats = [cb.dequantize_fp32(p, s, GROUP) for _, p, s in host]

        def sample(fn, budget):
            for i, (x, p, s) in enumerate(host):  # warm-up
                fn(i, x, p, s)
            times, t_end = [], time.perf_counter() + budget
            while time.perf_counter() < t_end or len(times) < 5:
                t1 = time.perf_counter()
                for i, (x, p, s) in enumerate(host):
                    fn(i, x, p, s)
                times.append(time.perf_counter() - t1)
            return statistics.median(times), len(times)

        full, n_full = sample(lambda i, x, p, s: cb.linear_fp32(x, p, s, GROUP), 0.7 * seconds)
        mm, n_mm = sample(lambda i, x, p, s: cb.matmul_only(x, w_hats[i]), 0.3 * seconds)
    finally:
        torch.set_num_threads(saved)
    return {"value": round(step_bytes / full / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{n_full} steps of the 7 TinyLlama linears at M=1, FP32 dequant + matmul per call "
                      f"(torch on {threads} threads: unpack, q*s, x.float() @ W_hat.T); "
                      f"median {full * 1e3:.2f} ms/step",
            "us_per_step": round(full * 1e6, 1),
            "matmul_only": {"value": round(step_bytes / mm / 1e9, 3), "unit": "GB/s", "us_per_step": round(mm * 1e6, 1),
                            "steps": n_mm, "note": "x.float() @ W_hat.T on W_hat dequantized once"},
            "affinity_cores": affinity, "os_cpu_count": os.cpu_count(), "omp_num_threads": omp,
            "cpu_model": _cpu_model()}


def main() -> int:
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures a single GPU: --gpus {args.gpus} (WORLD_SIZE={world}) is not supported. "
              "This build has no multi-GPU path; run with --gpus 1.", file=sys.stderr)
        return 2
    full = not args.headline_only
    traffic = None
    if full and not args.profile and not args.power and not args.no_traffic:
        log("rocprofv3 FETCH_SIZE / WRITE_SIZE passes (child processes)")
        traffic = measure_traffic()
        log(f"traffic: {traffic}")

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
    if args.profile:
        return profile_only(args, torch, lib, kl, ops, kq)
    if args.power:
        print(json.dumps({"power_m2048": power_leg(torch, ops, kq, args.power_seconds)}), flush=True)
        return 0

    log("measuring HBM ceilings")
    ceil = measure_hbm(torch, lib, kl)
    log(f"copy {ceil['hbm_copy_gbps']:.0f} GB/s, read {ceil['hbm_read_gbps']:.0f} GB/s")

    log("quantizing TinyLlama-shaped layers")
    layers = make_layers(torch, kq)
    names = [ly["name"] for ly in layers]
    idx = {nm: i for i, nm in enumerate(names)}
    step_bytes = sum(algo_bytes(1, ly["N"], ly["K"]) for ly in layers)
    same_read = measure_same_size_read(torch, lib, kl, step_bytes)
    log(f"bare read of one step's {step_bytes} B in one launch: {same_read['us']} us = {same_read['gbps']} GB/s; "
        f"with a GEMV's stores {same_read['with_gemv_stores']['us']} us; launch floor {same_read['launch_floor_us']} us")
    set_bytes = sum(ly["packed"].numel() * 4 + ly["scales"].numel() * 2 for ly in layers)
    copies = max(2, -(-(2 * MALL_BYTES) // set_bytes))
    dev = [[(ly["packed"].cuda(), ly["scales"].cuda()) for ly in layers] for _ in range(copies)]
    xs = [ly["x"].cuda() for ly in layers]

    def grouped(r, subset):
        ids = [idx[nm] for nm in subset]
        return ops.int4_linear_grouped([xs[i] for i in ids], [dev[r][i][0] for i in ids],
                                       [dev[r][i][1] for i in ids], GROUP)

    def single(r, nm):
        i = idx[nm]
        return ops.int4_linear(xs[i], dev[r][i][0], dev[r][i][1], GROUP)

    def step_grouped(r):
        grouped(r, names)

    def step_decoder(r):
        grouped(r, ["q", "k", "v"])
        single(r, "o")
        grouped(r, ["gate", "up"])
        single(r, "down")

    def step_separate(r):
        for nm in names:
            single(r, nm)

    # --- the timed step (value): one grouped launch over the 7 linears --------------------------
    # W warm-up steps, then exactly K steps between synchronize() calls, timed by a HIP event pair
    # on the launching stream, with the host's wall clock beside it.  Up to BOUND_MAX_STEPS the K
    # steps are eager launches of the op's C-ABI call queued behind a spin (BoundSteps: no graph
    # launch's fixed cost in a short timed region); beyond, replays of graphs all captured before
    # the timed region (GraphSteps: the fixed cost is spread over many steps, and the GPU's
    # command queue need not hold every launch at once).  Both timings are reported.
    log(f"{copies} weight copies ({copies * set_bytes / 2**20:.0f} MiB); warmup {args.warmup} steps")
    main_steps = GraphSteps(torch, step_grouped, copies)
    main_steps.prepare(args.warmup)
    main_steps.prepare(args.steps)
    main_steps.prepare(copies)
    main_steps.run(args.warmup)
    bound = BoundSteps(torch, kl, lib, xs, dev, GROUP)
    # The reference's warm-up rule on top of the W requested steps (kernelforge/bench_utils.py:
    # 114-185: at least 10 calls and 100 ms), in whole passes over the weight copies, so a short
    # run (the driver's --steps 20 --warmup 5) times a warm GPU as a long one does.
    warm_steps, t_warm = args.warmup, time.perf_counter()
    while warm_steps < args.warmup + 10 or time.perf_counter() - t_warm < 0.1:
        main_steps.run(copies)
        for i in range(copies):
            bound.launch(i)
        torch.cuda.synchronize()
        warm_steps += 2 * copies
    graph_ms, graph_wall_ms = main_steps.timed(args.steps)
    bound_timing = None
    if args.steps <= BOUND_MAX_STEPS:
        # Two untimed rehearsals of the timed pattern (spin, then K queued launches): the first
        # two such regions of a process read 0.1-0.3 us per step slow on MI355X, later ones do not.
        for _ in range(BOUND_REHEARSALS):
            bound.timed(args.steps)
            warm_steps += args.steps
        bound_timing = bound.timed(args.steps)
        if not bound_timing["covered"]:  # the host fell behind the spin once: one retry, then graphs
            bound_timing = bound.timed(args.steps)
    if bound_timing and bound_timing["covered"]:
        ms_per_step, wall_ms_per_step, timed_by = bound_timing["ms_per_step"], bound_timing["wall_ms_per_step"], "bound"
    else:
        ms_per_step, wall_ms_per_step, timed_by = graph_ms, graph_wall_ms, "graph"
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"grouped 7-layer step {ms_per_step * 1e3:.3f} us ({timed_by} launches, events; wall clock "
        f"{wall_ms_per_step * 1e3:.3f} us; graph replays {graph_ms * 1e3:.3f} us) -> {value:.0f} GB/s")

    # --- roofline of the dominant kernel (the grouped GEMV: one launch per step) ----------------
    # achieved: the timed region's own event average (one launch per step); a longer event run
    # of 8 x copies steps is reported beside it.
    achieved = value
    long_avg_ms = main_steps.event_avg_ms(8 * copies)
    log(f"grouped GEMV: {ms_per_step * 1e3:.3f} us per launch in the timed region, {long_avg_ms * 1e3:.3f} us over "
        f"{8 * copies} launches")

    ref_proto = structures = per_layer = qwen = host_us = None
    if full:
        # The same step timed the reference's way: one eager call per event pair, behind a spin guard.
        ref_proto = reference_protocol(torch, step_grouped, copies)
        ref_proto["gbps_at_median"] = round(step_bytes / (ref_proto["median_us"] * 1e-6) / 1e9, 1)
        log(f"reference protocol (per-call events): median {ref_proto['median_us']} us, "
            f"p10 {ref_proto['p10_us']}, p90 {ref_proto['p90_us']}")
        host_us = {"int4_linear_gate": host_enqueue_us(torch, lambda: single(0, "gate")),
                   "int4_linear_grouped_7": host_enqueue_us(torch, lambda: step_grouped(0))}
        log(f"host enqueue per eager call: {host_us}")

        # --- the other step structures ------------------------------------------------------------
        structures = {}
        for label, fn, launches in (("decoder_4_launches", step_decoder, 4), ("separate_7_launches", step_separate, 7)):
            gs = GraphSteps(torch, fn, copies)
            ms = statistics.median(gs.event_avg_ms(8 * copies) for _ in range(5))
            structures[label] = {"launches": launches, "us_per_step": round(ms * 1e3, 3),
                                 "gbps": round(step_bytes / (ms * 1e-3) / 1e9, 1),
                                 "pct_of_copy": round(100 * step_bytes / (ms * 1e-3) / 1e9 / ceil["hbm_copy_gbps"], 1)}
            log(f"{label}: {ms * 1e3:.2f} us/step")
        per_layer = {}
        for nm in names:
            i = idx[nm]
            gs = GraphSteps(torch, lambda r, nm=nm: single(r, nm), copies)
            ms = statistics.median(gs.event_avg_ms(8 * copies) for _ in range(5))
            b = algo_bytes(1, layers[i]["N"], layers[i]["K"])
            per_layer[nm] = {"N": layers[i]["N"], "K": layers[i]["K"], "bytes": b, "us": round(ms * 1e3, 3),
                             "gbps": round(b / (ms * 1e-3) / 1e9, 1),
                             "pct_of_copy": round(100 * b / (ms * 1e-3) / 1e9 / ceil["hbm_copy_gbps"], 1)}

        # --- config 3: the Qwen2.5-1.5B decoder linears as one grouped launch --------------------
        qlayers = make_layers(torch, kq, QWEN_LAYERS, seed=2000)
        q_bytes = sum(algo_bytes(1, ly["N"], ly["K"]) for ly in qlayers)
        q_set = sum(ly["packed"].numel() * 4 + ly["scales"].numel() * 2 for ly in qlayers)
        q_copies = max(2, -(-(2 * MALL_BYTES) // q_set))
        q_dev = [[(ly["packed"].cuda(), ly["scales"].cuda()) for ly in qlayers] for _ in range(q_copies)]
        q_xs = [ly["x"].cuda() for ly in qlayers]
        gs = GraphSteps(torch, lambda r: ops.int4_linear_grouped(q_xs, [p for p, _ in q_dev[r]],
                                                                 [s for _, s in q_dev[r]], GROUP), q_copies)
        q_ms = statistics.median(gs.event_avg_ms(8 * q_copies) for _ in range(5))
        q_gbps = q_bytes / (q_ms * 1e-3) / 1e9
        qwen = {"workload": "qwen2.5_1.5b_7_linears_m1_g128", "shapes_NxK": [[n, k] for _, n, k in QWEN_LAYERS],
                "bytes_per_step": q_bytes, "us_per_step": round(q_ms * 1e3, 3), "gbps": round(q_gbps, 1),
                "pct_of_measured_copy": round(100 * q_gbps / ceil["hbm_copy_gbps"], 1),
                "reference_pct_of_copy_on_its_gpu": REFERENCE_QWEN_PCT_OF_COPY, "weight_copies_rotated": q_copies}
        log(f"Qwen2.5 grouped 7-layer step {q_ms * 1e3:.2f} us -> {q_gbps:.0f} GB/s")
        del gs, q_dev

    # --- M=2048: MFMA GEMM on every shape ------------------------------------------------------
    m2048 = None
    if full and not args.no_m2048:
        log("M=2048 GEMM leg")
        mfma_peak = measure_mfma_peak(torch)
        # Beside each INT4 layer: hipBLASLt's dense fp16 GEMM on the same shape (torch F.linear,
        # fp16 weights, same protocol), the library's own rate where the cube peak is out of reach.
        total_flops, total_ms, blas_ms, per = 0.0, 0.0, 0.0, {}
        for i, ly in enumerate(layers):
            xm = torch.randn(2048, ly["K"], dtype=torch.float16, device="cuda")
            p, s = dev[0][i]
            steps = GraphSteps(torch, lambda r, xm=xm, p=p, s=s: ops.int4_gemm(xm, p, s, GROUP), 10)
            t = statistics.median(steps.event_avg_ms(10) for _ in range(5))
            wd = torch.randn(ly["N"], ly["K"], dtype=torch.float16, device="cuda")
            bsteps = GraphSteps(torch, lambda r, xm=xm, wd=wd: torch.nn.functional.linear(xm, wd), 10)
            tb = statistics.median(bsteps.event_avg_ms(10) for _ in range(5))
            fl = 2.0 * 2048 * ly["N"] * ly["K"]
            plan = ops.gemm_plan(2048, ly["N"], ly["K"], GROUP)
            per[ly["name"]] = {"us": round(t * 1e3, 1), "tflops": round(fl / (t * 1e-3) / 1e12, 1),
                               "hipblaslt_fp16_us": round(tb * 1e3, 1),
                               "hipblaslt_fp16_tflops": round(fl / (tb * 1e-3) / 1e12, 1),
                               "int4_over_hipblaslt_fp16": round(tb / t, 3),
                               "plan": {"kernel": plan["kernel"], "splits": plan["splits"], "tile": plan["tile"]}}
            total_flops += fl
            total_ms += t
            blas_ms += tb
            del xm, wd, steps, bsteps
        gate_tf = per["gate"]["tflops"]
        m2048 = {"gate_tflops": gate_tf, "seven_layer_tflops": round(total_flops / (total_ms * 1e-3) / 1e12, 1),
                 "seven_layer_hipblaslt_fp16_tflops": round(total_flops / (blas_ms * 1e-3) / 1e12, 1),
                 "seven_layer_int4_over_hipblaslt_fp16": round(blas_ms / total_ms, 3),
                 "measured_fp16_mfma_peak_tflops": round(mfma_peak, 1),
                 "gate_frac_of_measured_peak": round(gate_tf / mfma_peak, 4),
                 "gate_frac_of_spec_peak": round(gate_tf / SPEC_FP16_TFLOPS, 4), "per_layer": per}
        log(f"M=2048 gate {gate_tf} TFLOPS (hipBLASLt fp16 on the same shape "
            f"{per['gate']['hipblaslt_fp16_tflops']}); hipBLASLt fp16 cube peak {mfma_peak:.0f} TFLOPS")

    # --- on-device quantize + pack of an fp32 gate weight (format producer) --------------------
    quant = None
    if full and not args.no_quant:
        log("quantize leg")
        qn, qk = 5632, 2048
        in_bytes, out_bytes = qn * qk * 4, qn * qk // 2 + 2 * qn * (qk // GROUP)
        qcopies = max(2, -(-(2 * MALL_BYTES) // in_bytes))
        wq = [torch.randn(qn, qk, device="cuda") * 0.02 for _ in range(qcopies)]
        gs = GraphSteps(torch, lambda r: ops.int4_quantize(wq[r], GROUP), qcopies)
        ms = statistics.median(gs.event_avg_ms(4 * qcopies) for _ in range(5))
        gbps = (in_bytes + out_bytes) / (ms * 1e-3) / 1e9
        w_host = wq[0].cpu()
        kq.quantize_weight(w_host, GROUP)
        cpu_ms = statistics.median(_timed_ms(lambda: kq.quantize_weight(w_host, GROUP)) for _ in range(3))
        quant = {"shape_NxK": [qn, qk], "dtype_in": "fp32", "group_size": GROUP, "bytes_per_call": in_bytes + out_bytes,
                 "us": round(ms * 1e3, 2), "gbps": round(gbps, 1),
                 "pct_of_measured_copy": round(100 * gbps / ceil["hbm_copy_gbps"], 1),
                 "cpu_torch_quantize_ms": round(cpu_ms, 2), "cpu_threads": torch.get_num_threads()}
        log(f"quantize {ms * 1e3:.1f} us -> {gbps:.0f} GB/s; torch on the CPU {cpu_ms:.1f} ms")
        del wq, gs

    # --- config 5: end-to-end graph decode ------------------------------------------------------
    e2e = None
    if full and not args.no_e2e:
        log("TinyLlama graph decode leg")
        e2e = e2e_decode(torch)
        log(f"decode tok/s: int4 fused {e2e['int4_fused_tok_s']}, unfused {e2e['int4_unfused_tok_s']}, "
            f"fp16 {e2e['fp16_tok_s']}")
        try:
            log("HF LlamaForCausalLM graph decode leg")
            e2e["hf_llama"] = hf_llama_decode(torch)
            h = e2e["hf_llama"]
            log(f"HF decode tok/s: int4 {h['int4_tok_s']}, grouped {h['int4_grouped_tok_s']}, fp16 {h['fp16_tok_s']}")
        except ImportError as exc:
            e2e["hf_llama"] = f"unavailable: {exc}"

    # --- CPU baseline: the reference's FP32 dequant + matmul on the host cores ------------------
    cpu = None
    if full and not args.no_cpu:
        cpu = cpu_baseline(torch, layers, step_bytes, args.cpu_seconds)
        log(f"CPU baseline {cpu['value']} GB/s ({cpu['us_per_step']} us/step on {cpu['cores']} threads); "
            f"matmul only {cpu['matmul_only']['value']} GB/s")

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": "tinyllama_7_linears_m1_g128", "shapes_NxK": [[n, k] for _, n, k in TL_LAYERS],
                   "group_size": GROUP, "bytes_per_step": step_bytes, "weight_copies_rotated": copies,
                   "step": "one int4_linear_grouped launch (its C-ABI call kf_int4_gemv_grouped) over the 7 "
                           "independent linears",
                   "launched_as": timed_by},
        "timer": {"ms_per_step": "HIP event pair on the launching stream around exactly K steps, between "
                                 "synchronize() calls: K <= %d eager launches of kf_int4_gemv_grouped queued behind "
                                 "a GPU spin longer than their host enqueue (bound), else replays of graphs "
                                 "captured before the timed region (graph)" % BOUND_MAX_STEPS,
                  "launched_as": timed_by,
                  "bound": bound_timing,
                  "graph_ms_per_step": round(graph_ms, 6),
                  "graph_wall_ms_per_step": round(graph_wall_ms, 6),
                  "wall_ms_per_step": round(wall_ms_per_step, 6),
                  "warmup_steps_run": warm_steps,
                  "warmup_rule": "the W requested steps, then whole passes over the weight copies until at "
                                 "least W + 10 steps and 100 ms (the reference's rule); for bound timing also "
                                 f"{BOUND_REHEARSALS} untimed runs of the timed region's pattern"},
        "pct_of_measured_copy": round(100 * value / ceil["hbm_copy_gbps"], 1),
        "pct_of_measured_read": round(100 * value / ceil["hbm_read_gbps"], 1),
        "reference_pct_of_copy_on_its_gpu": REFERENCE_PCT_OF_COPY,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": SPEC_HBM_GBPS, "unit": "GB/s",
                     "frac": round(achieved / SPEC_HBM_GBPS, 4),
                     "traffic": round(traffic["bytes"]) if traffic else None,
                     "traffic_detail": traffic,
                     "kernel": "kf::gemv_grouped_kernel (7 TinyLlama linears; gate at 3 rows per wavefront)",
                     "bytes_per_launch": step_bytes, "avg_launch_us": round(ms_per_step * 1e3, 3),
                     "avg_launch_us_over_8x_copies": round(long_avg_ms * 1e3, 3),
                     "frac_of_measured_copy": round(achieved / ceil["hbm_copy_gbps"], 4),
                     "frac_of_measured_read": round(achieved / ceil["hbm_read_gbps"], 4),
                     "same_size_read": same_read,
                     "frac_of_same_size_read": round(achieved / same_read["gbps"], 4),
                     "frac_of_same_size_read_with_stores": round(achieved / same_read["with_gemv_stores"]["gbps"], 4)},
        "cpu_baseline": cpu,
        "reference_protocol": ref_proto,
        "host_enqueue_us": host_us,
        "ceilings": {k: round(v, 1) if isinstance(v, float) else v for k, v in ceil.items()},
        "step_structures": structures,
        "per_layer_m1": per_layer,
        "qwen_m1": qwen,
        "m2048": m2048,
        "e2e_decode": e2e,
        "quantize": quant,
        "environment": environment(torch, props) if full else None,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
