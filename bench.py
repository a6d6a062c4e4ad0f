#!/usr/bin/env python3
"""Benchmark of the MI355X GEMM core of rustnn (one GPU).

Metric: "ResNet-20 W32 train images/s; implicit-GEMM conv
TFLOP/s and % fp32 MFMA peak".  Until the device-resident ResNet-20 step
exists, the step timed here is BASELINE config 1: the ResNet stage sweep of
fp32 convolutions at batch 128 -- 3x3 32->32 @32x32 s1, 32->64 @32x32 s2,
64->64 @16x16, 64->128 @16x16 s2, 128->128 @8x8, and the 1x1 s2 projections
32->64 @32x32 and 64->128 @16x16 -- each forward + dX + dW.  `value` is the
whole step's algorithmic conv TFLOP/s (2*cout*cin*k*k*oh*ow*N per pass) with
every operand resident in HBM.

Also reported: `roofline` for the dominant kernel (HIP events on the library's
stream around that op, algorithmic FLOP / average duration vs the 157.3 TFLOP/s
fp32 MFMA peak) and `cpu_baseline`: the restated reference CPU path (oracle/,
AVX2 micro-kernel, per-image OpenMP parallelism) on a bounded sample of the
same sweep, timed on this host's cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "ResNet-20 W32 train images/s; implicit-GEMM conv TFLOP/s and % fp32 MFMA peak"
PEAK_FP32_MFMA_TFLOPS = 157.3
N = 128
SWEEP = [  # name, cin, cout, k, stride, pad, h  (BASELINE config 1)
    ("3x3s1_32to32_32", 32, 32, 3, 1, 1, 32),
    ("3x3s2_32to64_32", 32, 64, 3, 2, 1, 32),
    ("3x3s1_64to64_16", 64, 64, 3, 1, 1, 16),
    ("3x3s2_64to128_16", 64, 128, 3, 2, 1, 16),
    ("3x3s1_128to128_8", 128, 128, 3, 1, 1, 8),
    ("1x1s2_32to64_32", 32, 64, 1, 2, 0, 32),
    ("1x1s2_64to128_16", 64, 128, 1, 2, 0, 16),
]
PASSES = ("fwd", "dx", "dw")


def pass_flops(cin, cout, k, s, p, h, n=N):
    oh = (h + 2 * p - k) // s + 1
    return 2.0 * cout * cin * k * k * oh * oh * n


def traffic_from_profiles(kernel_tag):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary
    (profiles/<tag>_pmc.txt), or None when it has not been measured."""
    path = os.path.join(ROOT, "profiles", f"{kernel_tag}_pmc.txt")
    if not os.path.exists(path):
        return None
    vals = {}
    for ln in open(path):
        if ":" in ln and not ln.lstrip().startswith("#"):
            k, v = ln.split(":", 1)
            try:
                vals[k.strip()] = float(v.split()[0])
            except (ValueError, IndexError):
                pass
    try:
        return (vals["FETCH_SIZE_KiB_per_dispatch"] + vals["WRITE_SIZE_KiB_per_dispatch"]) * 1024 * \
            vals.get("copy_kernel_scale", 1.0)
    except KeyError:
        return None


def cpu_baseline(budget_s=12.0):
    """Oracle (restated reference CPU path) on a bounded sample of the sweep:
    the 7 conv shapes x fwd/dX/dW on `sample` images, repeated until the time
    budget is used (at least once).  Returns TFLOP/s and the sample."""
    import numpy as np
    from oracle import pyorc as O
    O.build()
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    threads = max(1, min(threads, 16, os.cpu_count() or 1))
    sample = 8
    layers = []
    for name, cin, cout, k, s, p, h in SWEEP:
        sp = O.ConvSpec.make(cin, cout, k, s, p, h, h)
        r = np.random.default_rng(7)
        x = r.standard_normal(sample * cin * h * h).astype(np.float32)
        w = (r.standard_normal(cout * sp.ckk) * np.sqrt(2.0 / sp.ckk)).astype(np.float32)
        dy = r.standard_normal(sample * cout * sp.hw).astype(np.float32)
        layers.append((sp, x, w, dy))
    flops = sum(3 * pass_flops(c[1], c[2], c[3], c[4], c[5], c[6], sample) for c in SWEEP)

    def one():
        for sp, x, w, dy in layers:
            O.conv2d_forward(sp, sample, x, w)
            O.conv2d_backward_x(sp, sample, dy, w)
            O.conv2d_backward_w(sp, sample, dy, x)

    with O.threads(threads):
        one()  # warm-up (bench.rs:29-30 protocol: one untimed call)
        reps, t0 = 0, time.perf_counter()
        while True:
            one()
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget_s or el / reps * (reps + 1) > 2.5 * budget_s:
                break
    return {"value": round(flops * reps / el / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"config-1 sweep (7 conv shapes x fwd/dX/dW) on {sample} of 128 images, "
                      f"{reps} reps in {el:.1f}s; oracle/ AVX2 restatement, OpenMP {threads} threads"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--op-reps", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on one GPU only (single-GPU tier); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)

    import torch
    import rustnn_amd as R

    torch.cuda.set_device(0)
    ctx = R.default_ctx(0)
    g = torch.Generator(device="cuda").manual_seed(7)
    layers = []
    for name, cin, cout, k, s, p, h in SWEEP:
        sp = R.ConvSpec.make(cin, cout, k, s, p, h, h)
        x = torch.randn(N * cin * h * h, device="cuda", generator=g)
        w = torch.randn(cout * sp.ckk, device="cuda", generator=g) * (2.0 / sp.ckk) ** 0.5
        dy = torch.randn(N * cout * sp.hw, device="cuda", generator=g)
        y = torch.empty(N * cout * sp.hw, device="cuda")
        dx = torch.empty(N * cin * h * h, device="cuda")
        dw = torch.zeros(cout * sp.ckk, device="cuda")
        layers.append(dict(name=name, sp=sp, x=x, w=w, dy=dy, y=y, dx=dx, dw=dw,
                           flops=pass_flops(cin, cout, k, s, p, h)))

    def run_op(L, ps):
        if ps == "fwd":
            R.conv2d_forward(L["sp"], N, L["x"], L["w"], L["y"], ctx=ctx)
        elif ps == "dx":
            R.conv2d_backward_x(L["sp"], N, L["dy"], L["w"], L["dx"], ctx=ctx)
        else:
            R.conv2d_backward_w(L["sp"], N, L["dy"], L["x"], L["dw"], ctx=ctx)

    def step():
        for L in layers:
            for ps in PASSES:
                run_op(L, ps)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # events are recorded on the current stream, which is the library's stream
    assert ctx.stream_ptr() == torch.cuda.current_stream().cuda_stream
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    step_flops = sum(3 * L["flops"] for L in layers)
    value = step_flops / (ms * 1e-3) / 1e12

    # per-op durations (HIP events around each op, op-reps back-to-back)
    per_op = []
    for L in layers:
        for ps in PASSES:
            run_op(L, ps)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(args.op_reps):
                run_op(L, ps)
            b.record()
            torch.cuda.synchronize()
            t = a.elapsed_time(b) / args.op_reps
            per_op.append(dict(op=f"{L['name']}:{ps}", ms=round(t, 5),
                               tflops=round(L["flops"] / (t * 1e-3) / 1e12, 2),
                               frac=round(L["flops"] / (t * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4)))
    dom = max(per_op, key=lambda r: r["ms"])
    dom_layer = next(L for L in layers if dom["op"].startswith(L["name"] + ":"))
    achieved = dom_layer["flops"] / (dom["ms"] * 1e-3) / 1e12
    tag = dom["op"].replace(":", "_")
    roof = {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4),
            "traffic": traffic_from_profiles(tag), "kernel": dom["op"]}

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args.cpu_budget)

    out = {
        "metric": METRIC, "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic (x, dY ~ N(0,1); W Kaiming-normal; seeded on device)",
        "config": {"workload": "config1 ResNet stage conv sweep, batch 128, fwd+dX+dW "
                               "(5 3x3 shapes + 2 1x1 s2 projections)",
                   "batch": N, "flop_per_step": step_flops,
                   "conv_sweep_frac_of_fp32_mfma_peak": round(value / PEAK_FP32_MFMA_TFLOPS, 4),
                   "wall_s_timed": round(wall, 3)},
        "roofline": roof, "cpu_baseline": cpu, "per_op": per_op,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
