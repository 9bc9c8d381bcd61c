"""Benchmark of the MI355X Pairformer hot path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--op block] [--n 768]

A "step" is one forward pass of the selected op over one batch of synthetic,
HBM-resident input.  The default op is one full bf16 Pairformer block at N=768,
c_z=128, c_s=384 (the BASELINE metric); the default run then measures every
BASELINE config the same way (configs 1-5: the N=64 fp32-I/O block, pair-bias
attention B=8 N=512, the fused OPM, the four triangle ops at N=768 and one pass
of the 48-block trunk at N=2048) and adds them under ``configs``.  ``--op``
selects a single op at its config shape instead (a diagnostic line).

Printed on one line as JSON: ms per step (K steps between two hipEvents on the
launch stream, synchronised on both sides), the roofline of the dominant
kernel and a CPU baseline (the fp32 oracle timed on a bounded sample, rank 0
only).  The dominant kernel's average duration comes from a second timed
region of the same K steps in which the library's kernel timer brackets every
launch with hipEvents on the kernel's own stream.
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

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_F32_TFLOPS = 157.3  # MI355X dense fp32 MFMA
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E


def _peak(bound: str) -> tuple[float, str, float]:
    """(published peak, unit, divisor of work/s) for a kernel's bound: bf16 MFMA, fp32 MFMA or HBM."""
    if bound == "mfma":
        return PEAK_BF16_TFLOPS, "TFLOP/s", 1e12
    if bound == "mfma_f32":
        return PEAK_F32_TFLOPS, "TFLOP/s", 1e12
    return PEAK_HBM_GBS, "GB/s", 1e9


def _parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--op", default="block")
    ap.add_argument("--n", type=int, default=None, help="override N (tokens)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="default run only: skip the per-config entries (configs 1-5) after the headline")
    ap.add_argument("--kernels", action="store_true", help="also print the per-kernel table to stderr")
    ap.add_argument("--no-kernel-timer", action="store_true",
                    help="time the steps without per-kernel events (no roofline; diagnostic)")
    ap.add_argument("--calibrate-bytes", type=int, default=0,
                    help="first run torch's negation of a tensor of this many bf16 bytes (a PMC calibration "
                         "dispatch that reads and writes exactly that much)")
    return ap.parse_args()


def cpu_baseline(wl) -> dict:
    """The fp32 CPU oracle on a bounded sample of the same workload (rank 0, N=1 only).

    By default 1 warm-up then the median of up to 3 timed calls, stopping
    early once ~30 s of CPU time is spent (the 48-block trunk times one call
    of its scaled sample); ``value`` is scaled to ms per full step.
    """
    import torch

    import oracle  # the checker, timed here as the CPU baseline only

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    fn, fraction, sample = wl.cpu_sample(oracle)
    warm = getattr(wl, "cpu_warmup", 1)
    calls = getattr(wl, "cpu_calls", 3)
    for _ in range(warm):
        fn()
    times = []
    budget = time.perf_counter() + 30.0
    while len(times) < calls:
        t0 = time.perf_counter()
        r = fn()
        # a sample of separately scaled parts returns its own extrapolated seconds (fraction None)
        times.append(r if fraction is None else (time.perf_counter() - t0) / fraction)
        if time.perf_counter() > budget:
            break
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": round(med * 1e3, 1),
        "unit": "ms",
        "cores": threads,
        "kind": "port",
        "sample": f"{sample}; {len(times)} timed call(s) after {warm} warm-up(s), median",
        "cpu_model": _cpu_model(),
    }


def _cpu_model() -> str:
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# The five BASELINE configs measured after the headline line's own workload (the default run): name ->
# (workloads.make op, steps, warm-up steps, CPU-baseline warm-ups, CPU-baseline timed calls).  Config 4 is the
# four triangle ops at N = 768; config 5 one pass of the 48-block trunk at N = 2048, whose CPU baseline is one
# oracle block at N = 512 scaled to the pass by algorithmic flops.
CONFIGS = [
    ("1_block_n64_fp32io", "config1", 20, 3, 1, 3),
    ("2_apb_b8_n512", "apb", 20, 3, 1, 3),
    ("3_opm_s1024_n512", "opm", 20, 3, 1, 3),
    ("4_trimul_out_n768", "trimul_out", 20, 3, 1, 3),
    ("4_trimul_in_n768", "trimul_in", 20, 3, 1, 3),
    ("4_triatt_start_n768", "triatt_start", 20, 3, 1, 3),
    ("4_triatt_end_n768", "triatt_end", 20, 3, 1, 3),
    ("5_trunk48_n2048", "trunk", 2, 1, 0, 1),
]


def measure(wl, steps: int, warmup: int, with_cpu: bool, kernels_to_stderr: bool = False) -> dict:
    """Time ``steps`` steps of a workload (after ``warmup`` untimed ones) between two hipEvents on the launch
    stream, then the same steps with the kernel timer; returns ms per step, the dominant kernel's roofline,
    the per-kernel table and (``with_cpu``) the CPU baseline."""
    import torch

    from bioemu2_amd import workloads
    from bioemu2_amd.profiling import TIMER_TO_KERNEL
    from bioemu2_amd.timing import KernelTimer

    with torch.no_grad():
        for _ in range(warmup):
            wl.step()
        torch.cuda.synchronize()

        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)

        def timed(k: int) -> float:
            torch.cuda.synchronize()
            start.record()
            for _ in range(k):
                wl.step()
            stop.record()
            torch.cuda.synchronize()
            return start.elapsed_time(stop) / k

        # Timed region 1: the K steps alone -> value.
        ms_per_step = timed(steps)
        # Timed region 2: the same K steps with a hipEvent pair around every
        # kernel launch (on the launch stream) -> per-kernel average durations.
        # The events serialise kernel tails, so this region runs a few % slower.
        with KernelTimer() as kt:
            ms_per_step_events = timed(steps)
        kernels = kt.results()

    # Dominant kernel = largest total time in the timed region.
    dom_name, (dom_launches, dom_ms) = max(kernels.items(), key=lambda kv: kv[1][1])
    dom_avg_ms = dom_ms / dom_launches
    bound, amount = wl.kernel_work(dom_name)  # (bound, algorithmic amount per launch)
    peak, unit, div = _peak(bound)
    achieved = amount / (dom_avg_ms * 1e-3) / div
    roofline = {
        "kernel": dom_name,
        "bound": bound,
        "achieved": round(achieved, 2),
        "peak": peak,
        "unit": unit,
        "frac": round(achieved / peak, 4),
        "traffic": workloads.measured_traffic(TIMER_TO_KERNEL.get(dom_name, dom_name), wl.name),
        "avg_ms": round(dom_avg_ms, 5),
        "algorithmic_per_launch": amount,
    }
    per_kernel = {}
    for name, (n, ms) in sorted(kernels.items(), key=lambda kv: -kv[1][1]):
        try:
            b, a = wl.kernel_work(name)
        except KeyError:
            print(f"[kernel] {name}: no algorithmic-work entry; timing only", file=sys.stderr)
            per_kernel[name] = {"launches_per_step": n / steps, "avg_ms": round(ms / n, 5)}
            continue
        avg = ms / n
        pk, _, div = _peak(b)
        rate = a / (avg * 1e-3) / div
        per_kernel[name] = {
            "launches_per_step": n / steps,
            "avg_ms": round(avg, 5),
            "bound": b,
            "work": a,
            "rate": round(rate, 1),
            "frac": round(rate / pk, 4),
        }
    if kernels_to_stderr:
        for k, v in per_kernel.items():
            print(f"[kernel] {k}: {v}", file=sys.stderr)
    return {
        "ms_per_step": ms_per_step,
        "ms_per_step_events": ms_per_step_events,
        "tflops": round(wl.flops / (ms_per_step * 1e-3) / 1e12, 1),
        "roofline": roofline,
        "kernels": per_kernel,
        "cpu_baseline": cpu_baseline(wl) if with_cpu else None,
    }


def measure_configs(dev, with_cpu: bool) -> dict:
    """Every BASELINE config on this GPU, one after another (each workload freed before the next)."""
    import torch

    from bioemu2_amd import workloads

    out = {}
    for key, op, steps, warmup, cpu_warm, cpu_calls in CONFIGS:
        t0 = time.perf_counter()
        wl = workloads.make(op, dev)
        wl.cpu_warmup, wl.cpu_calls = cpu_warm, cpu_calls
        r = measure(wl, steps, warmup, with_cpu)
        out[key] = {
            "metric": wl.metric,
            "ms": round(r["ms_per_step"], 4),
            "tflops": r["tflops"],
            "dtype": getattr(wl, "dtype", "bf16"),
            "steps": steps,
            "warmup": warmup,
            "config": wl.config,
            "roofline": r["roofline"],
            "cpu_baseline": r["cpu_baseline"],
        }
        print(f"[config] {key}: {r['ms_per_step']:.4f} ms, {r['roofline']['kernel']} frac "
              f"{r['roofline']['frac']} ({time.perf_counter() - t0:.1f} s)", file=sys.stderr, flush=True)
        del wl, r
        torch.cuda.empty_cache()
    return out


def main() -> int:
    args = _parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(
            "bench.py measures one MI355X only: this build has no multi-GPU path. Run with --gpus 1.",
            file=sys.stderr,
        )
        return 2

    import torch

    from bioemu2_amd import workloads

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.calibrate_bytes:
        src = torch.ones(args.calibrate_bytes // 2, dtype=torch.bfloat16, device=dev)
        torch.neg(src, out=torch.empty_like(src))
        torch.cuda.synchronize()
        del src

    wl = workloads.make(args.op, dev, n=args.n)
    if args.no_kernel_timer:
        with torch.no_grad():
            for _ in range(args.warmup):
                wl.step()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(args.steps):
                wl.step()
            torch.cuda.synchronize()
            ms = (time.perf_counter() - t0) * 1e3 / args.steps
        print(json.dumps({"metric": wl.metric, "ms_per_step": round(ms, 4), "kernel_timer": False}), flush=True)
        return 0
    r = measure(wl, args.steps, args.warmup, not args.no_cpu_baseline, args.kernels)
    ms_per_step = r["ms_per_step"]
    line = {
        "metric": wl.metric,
        "value": round(ms_per_step, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": getattr(wl, "dtype", "bf16"),
        "data": "synthetic (seeded randn inputs, seeded random-init weights)",
        "config": wl.config,
        "tflops": r["tflops"],
        "ms_per_step_with_kernel_events": round(r["ms_per_step_events"], 4),
        "roofline": r["roofline"],
        "kernels": r["kernels"],
        "cpu_baseline": r["cpu_baseline"],
    }
    if args.op == "block" and args.n is None and not args.no_configs:
        del wl
        torch.cuda.empty_cache()
        line["configs"] = measure_configs(dev, not args.no_cpu_baseline)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
