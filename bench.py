#!/usr/bin/env python3
"""Benchmark of the MI355X GEMM core of rustnn (one GPU).

Metric: "ResNet-20 W32 train images/s; implicit-GEMM conv
TFLOP/s and % fp32 MFMA peak".

Headline (`value`, images/s): BASELINE config 3, the full ResNet-20 (W=32)
train step at batch 128 on 32x32 synthetic images -- forward, softmax
cross-entropy (smoothing 0.1), backward and the Nesterov SGD step (lr 0.2,
momentum 0.9, wd 5e-4) -- through the device-resident runtime (rnn_resnet_*,
replayed from a hipGraph), every operand resident in HBM.  One "step" is one
train step on one batch; `value` = steps * 128 / timed seconds.

Also reported:
  * `roofline`: the kernel with the largest share of the ResNet step, timed
    on its own with HIP events on the library's stream: its algorithmic FLOP
    per launch / average launch duration vs the 157.3 TFLOP/s fp32 MFMA peak;
    `traffic` from the committed rocprofv3 --pmc summary;
  * `cpu_baseline`: the restated reference CPU path (oracle/, AVX2 micro-kernel,
    OpenMP) running the same ResNet-20 train step on this host's cores for a
    bounded number of steps;
  * `config1_conv_sweep`: BASELINE config 1, the ResNet stage sweep of fp32
    convolutions at batch 128 (3x3 32->32 @32 s1, 32->64 @32 s2, 64->64 @16,
    64->128 @16 s2, 128->128 @8, and the 1x1 s2 projections) each forward + dX
    + dW: algorithmic conv TFLOP/s of the sweep, per-op durations, and the
    oracle's rate on a sample of it;
  * `config2_attention` and `gemmbench` (bench.rs:17-24 shapes).

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
PEAK_HBM_GBS = 8000.0
GEMMBENCH = [  # bench.rs:17-24 (--gemmbench): m, n, k, at, bt
    (16384, 768, 256, False, True, "S3 qkv fwd"),
    (16384, 704, 256, False, True, "S3 swiglu wg"),
    (16384, 256, 768, False, False, "S3 qkv dX"),
    (768, 256, 16384, True, False, "S3 qkv dW"),
    (16384, 256, 352, False, True, "S3 swiglu wd fwd"),
    (4096, 384, 1024, False, True, "merge fwd"),
]


def pass_flops(cin, cout, k, s, p, h, n=N):
    oh = (h + 2 * p - k) // s + 1
    return 2.0 * cout * cin * k * k * oh * oh * n


def traffic_from_profiles(op):
    """HBM bytes per launch of `op` (e.g. "3x3s1_32to32_32:dw") from the committed
    rocprofv3 --pmc summary profiles/conv_sweep_hbm_traffic.md: FETCH_SIZE +
    WRITE_SIZE summed over the op's kernels, scaled by the copy-kernel factor
    recorded there.  None when the op has not been measured."""
    path = os.path.join(ROOT, "profiles", "conv_sweep_hbm_traffic.md")
    if not os.path.exists(path):
        return None
    for ln in open(path):
        cells = [c.strip().strip("`") for c in ln.strip().strip("|").split("|")]
        if len(cells) >= 5 and cells[0] == op:
            try:
                return float(cells[4]) * 1024
            except ValueError:
                return None
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


def time_gpu(fn, reps):
    """Average ms of `fn` over `reps` back-to-back calls (HIP events on the
    current stream, which is the library's stream)."""
    import torch
    fn()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def time_graph(ctx, fn, reps):
    """Average ms of `fn` from replays of a graph holding `reps` calls: the
    library's context records on a side stream, replays run on the current
    stream between HIP events."""
    import torch
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    ctx.set_stream(side)
    g = torch.cuda.CUDAGraph()
    try:
        with torch.cuda.graph(g, stream=side):
            for _ in range(reps):
                fn()
    finally:
        ctx.set_stream(torch.cuda.current_stream())
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(3):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / (3 * reps)


def bench_attention(R, ctx, reps):
    """128 images x 4 heads, T=64 (8x8), dh=32, SelfAttn
    buffer [128, 64, 384] (q/k/v at 0/128/256), tau=1, rel=0, no mask; Q, K, V
    ~N(0,1)/sqrt(32), dO ~N(0,1).  HBM-bound: algorithmic bytes (each tensor
    once) fwd Q,K,V,O + P, bwd Q,K,V,dO,P in + dQ,dK,dV out."""
    import torch
    n, h, dh, t = 128, 4, 32, 64
    c = h * dh
    g = torch.Generator(device="cuda").manual_seed(7)
    qkv = torch.randn(n * t * 3 * c, device="cuda", generator=g) / dh ** 0.5
    dout = torch.randn(n * t * c, device="cuda", generator=g)
    relidx, nrel = R.rel_index(8, 8, 8, 8)
    tau = torch.ones(h, device="cuda")
    rel = torch.zeros(h * nrel, device="cuda")
    core = R.Core(h, dh, t, t, relidx, nrel, False, ctx=ctx)
    p = torch.empty(n * h * t * t, device="cuda")
    o = torch.empty(n * t * c, device="cuda")
    dqkv = torch.zeros_like(qkv)
    dtau = torch.zeros(h, device="cuda")
    drel = torch.zeros(h * nrel, device="cuda")
    fwd = lambda: core.forward(n, qkv, 3 * c, 0, qkv, 3 * c, c, 2 * c, tau, rel, p, o)
    bwd = lambda: core.backward(n, qkv, 3 * c, 0, qkv, 3 * c, c, 2 * c, tau, p, dout, dqkv, dqkv,
                                dtau, drel)
    fwd()
    bwd()
    # A call costs more host time than these kernels take, so back-to-back
    # eager calls would time the host: record `reps` calls into a graph (on
    # a capture stream given to the library's context) and time its replays.
    tf, tb = time_graph(ctx, fwd, reps), time_graph(ctx, bwd, reps)
    mb = n * h * t * dh * 4  # one [n, h, t, dh] tensor, bytes
    pb = n * h * t * t * 4
    fwd_bytes, bwd_bytes = 4 * mb + pb, 7 * mb + pb
    fwd_flop = 2 * 2.0 * n * h * t * t * dh
    bwd_flop = 4 * 2.0 * n * h * t * t * dh
    res = {}
    for name, ms, by, fl in (("fwd", tf, fwd_bytes, fwd_flop), ("bwd", tb, bwd_bytes, bwd_flop)):
        gbs = by / (ms * 1e-3) / 1e9
        res[name] = {"us": round(ms * 1e3, 2), "GB_s": round(gbs, 1),
                     "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
                     "TFLOP_s": round(fl / (ms * 1e-3) / 1e12, 3)}
    res["workload"] = "config2: 512 (image, head) problems, T=64, dh=32, fwd + bwd"
    res["timing"] = "graph replays of back-to-back calls (per call: launch gap included)"
    return res


def bench_gemm(R, ctx, reps):
    """The reference's --gemmbench shapes (bench.rs:17-24) through rnn_matmul."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(7)
    out = []
    for m, n, k, at, bt, tag in GEMMBENCH:
        a = torch.randn(m * k, device="cuda", generator=g)
        b = torch.randn(k * n, device="cuda", generator=g)
        cc = torch.empty(m * n, device="cuda")
        ms = time_gpu(lambda: R.matmul(m, n, k, a, at, b, bt, cc, False, ctx=ctx), reps)
        tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
        out.append({"shape": f"{m}x{n}x{k}", "at": at, "bt": bt, "tag": tag,
                    "us": round(ms * 1e3, 2), "TFLOP_s": round(tf, 2),
                    "frac": round(tf / PEAK_FP32_MFMA_TFLOPS, 4)})
    return out


RESNET = dict(depth_n=3, width=32, nclass=100, batch=128, hw=32, smooth=0.1, lr=0.2, mom=0.9,
              wd=5e-4, seed=7)
# Each conv op of the ResNet-20 step with its multiplicity (config-1 sweep
# names; the stem 3->32 conv runs forward + dW only).
RESNET_OPS = {"3x3s1_32to32_32": 6, "3x3s2_32to64_32": 1, "3x3s1_64to64_16": 5,
              "3x3s2_64to128_16": 1, "3x3s1_128to128_8": 5, "1x1s2_32to64_32": 1,
              "1x1s2_64to128_16": 1}
CIFAR_MEAN = (0.5071, 0.4865, 0.4409)  # data.rs:13-14
CIFAR_STD = (0.2673, 0.2564, 0.2762)


def resnet_inputs_gpu(n, seed):
    """Config 3 inputs: images uniform in [0, 1] normalised per channel
    (data.rs:96-98), labels uniform over 100 classes; drawn on the device."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    u = torch.rand(n, 3, 32, 32, device="cuda", generator=g)
    mean = torch.tensor(CIFAR_MEAN, device="cuda").view(1, 3, 1, 1)
    std = torch.tensor(CIFAR_STD, device="cuda").view(1, 3, 1, 1)
    x = ((u - mean) / std).contiguous()
    labels = torch.randint(0, 100, (n,), device="cuda", generator=g, dtype=torch.int32)
    return x, labels


def cpu_baseline_resnet(budget_s=12.0):
    """The oracle's ResNet-20 train step (restated reference CPU path: AVX2
    micro-kernel convs, f64 BN statistics, OpenMP over images / channels) on
    config-3 batches of 128, one untimed warm-up step, then steps until the
    budget is used.  Returns images/s."""
    import numpy as np
    from oracle import pyorc as O
    from oracle import pymodel as M
    O.build()
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    threads = max(1, min(threads, 16, os.cpu_count() or 1))
    c = RESNET
    rng = O.Rng(2026)
    n = c["batch"]
    u = rng.uniform_vec(n * 3 * 32 * 32).reshape(n, 3, 32, 32)
    x = ((u - np.array(CIFAR_MEAN, np.float32)[None, :, None, None]) /
         np.array(CIFAR_STD, np.float32)[None, :, None, None]).astype(np.float32)
    labels = np.array([rng.below(100) for _ in range(n)], np.uint32)
    net = M.ResNet(c["depth_n"], c["width"], c["nclass"], c["seed"])
    with O.threads(threads):
        net.train_step(x, labels, c["smooth"], c["lr"], c["mom"], c["wd"])  # warm-up
        steps, t0 = 0, time.perf_counter()
        while True:
            net.train_step(x, labels, c["smooth"], c["lr"], c["mom"], c["wd"])
            steps += 1
            el = time.perf_counter() - t0
            if el >= budget_s or el / steps * (steps + 1) > 2.5 * budget_s:
                break
    return {"value": round(steps * n / el, 2), "unit": "images/s", "cores": threads,
            "kind": "port",
            "sample": f"config-3 ResNet-20 W32 train step (fwd + softmax-CE + bwd + SGD) at batch "
                      f"{n}, {steps} steps in {el:.1f}s after 1 warm-up step; oracle/ AVX2 "
                      f"restatement, OpenMP {threads} threads"}


def bench_resnet(R, ctx, steps, warmup):
    """Config 3: the ResNet-20 train step through rnn_resnet_train_step."""
    import torch
    from rustnn_amd.model import ResNet
    c = RESNET
    net = ResNet(c["depth_n"], c["width"], c["nclass"], c["seed"], ctx=ctx)
    # bench.rs:110-140: one batch assembled before the loop, every step on it.
    # The batch goes straight into the network's input slots.
    x, labels = resnet_inputs_gpu(c["batch"], 2026)
    xs, ls = net.inputs(c["batch"], 32, 32)
    xs.copy_(x)
    ls.copy_(labels)
    del x, labels
    step = lambda: net.train_step(None, None, c["smooth"], c["lr"], c["mom"], c["wd"])
    for _ in range(max(warmup, 2)):  # the second call records the graph
        step()
    torch.cuda.synchronize()
    assert ctx.stream_ptr() == torch.cuda.current_stream().cuda_stream
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / steps
    graph, why = net.graph_state()
    loss = torch.zeros(1, device="cuda")  # one more step, reading its loss
    net.train_step(None, None, c["smooth"], c["lr"], c["mom"], c["wd"], loss)
    flop_img = 3 * net.flops(32, 32)  # bench.rs:142: train = 3 x forward
    out = {"ms": ms, "images_s": c["batch"] / (ms * 1e-3), "wall": wall, "graph": graph,
           "graph_note": why, "flop_per_image": flop_img,
           "loss": float(loss.item()), "params": net.num_params()}
    net.close()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--op-reps", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--ops-only", type=int, default=0, metavar="REPS",
                    help="no timing: run a 256 MiB copy, then each sweep op REPS times in sweep "
                         "order (the workload of the rocprofv3 --pmc passes)")
    ap.add_argument("--resnet-only", type=int, default=0, metavar="STEPS",
                    help="no timing: STEPS ResNet-20 train steps (the workload of the "
                         "rocprofv3 kernel trace of the step)")
    ap.add_argument("--attn-only", type=int, default=0, metavar="REPS",
                    help="config 2 only: the attention forward / backward timing with REPS calls "
                         "per graph (the workload of the rocprofv3 kernel trace of attention)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on one GPU only (single-GPU tier); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)

    import torch
    import rustnn_amd as R

    torch.cuda.set_device(0)
    ctx = R.default_ctx(0)

    if args.resnet_only:
        r = bench_resnet(R, ctx, args.resnet_only, 2)
        print(json.dumps({"resnet_only": args.resnet_only, "ms": r["ms"]}))
        return
    if args.attn_only:
        print(json.dumps({"attn_only": bench_attention(R, ctx, args.attn_only)}))
        return

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
        # W in the slab order of the forward / dX kernels (rnn_conv_pack_weights):
        # a train step packs each conv's weights once per update
        wpf, wpx = R.conv_pack_weights(sp, 0, w, ctx=ctx), R.conv_pack_weights(sp, 1, w, ctx=ctx)
        layers.append(dict(name=name, sp=sp, x=x, w=w, dy=dy, y=y, dx=dx, dw=dw, wpf=wpf,
                           wpx=wpx, flops=pass_flops(cin, cout, k, s, p, h)))

    def run_op(L, ps, packed=True):
        if ps == "fwd":
            if packed:
                R.conv2d_forward_packed(L["sp"], N, L["x"], L["w"], L["wpf"], L["y"], ctx=ctx)
            else:
                R.conv2d_forward(L["sp"], N, L["x"], L["w"], L["y"], ctx=ctx)
        elif ps == "dx":
            if packed:
                R.conv2d_backward_x_packed(L["sp"], N, L["dy"], L["w"], L["wpx"], L["dx"],
                                           ctx=ctx)
            else:
                R.conv2d_backward_x(L["sp"], N, L["dy"], L["w"], L["dx"], ctx=ctx)
        elif ps == "pack":
            R.conv_pack_weights(L["sp"], 0, L["w"], L["wpf"], ctx=ctx)
            R.conv_pack_weights(L["sp"], 1, L["w"], L["wpx"], ctx=ctx)
        else:
            R.conv2d_backward_w(L["sp"], N, L["dy"], L["x"], L["dw"], ctx=ctx)

    def sweep_step(packs=True, packed=True):
        for L in layers:
            if packs:
                run_op(L, "pack")
            for ps in PASSES:
                run_op(L, ps, packed)

    def time_sweep(**kw):
        # eager warm-up (sizes the workspaces), then graph replays: the GPU's
        # time for the step, without the Python launch overhead
        for _ in range(args.warmup):
            sweep_step(**kw)
        torch.cuda.synchronize()
        return time_graph(ctx, lambda: sweep_step(**kw), args.steps)

    if args.ops_only:
        # calibration copy of known size first, then the ops in sweep order
        src = torch.empty(64 << 20, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        for L in layers:
            for ps in PASSES:
                for _ in range(args.ops_only):
                    run_op(L, ps)
        torch.cuda.synchronize()
        print(json.dumps({"ops_only": [f"{L['name']}:{ps}" for L in layers for ps in PASSES],
                          "reps": args.ops_only, "copy_bytes": 2 * src.numel() * 4}))
        return

    # ---- headline: config 3, the ResNet-20 train step
    rn = bench_resnet(R, ctx, args.steps, args.warmup)

    # ---- config 1: the conv sweep.  One sweep step = per layer: pack W for
    # the forward and dX kernels, forward, dX, dW (the weights are packed once
    # per update, as the ResNet step does).  Also timed: the same without the
    # packs (the conv kernels alone) and with unpacked weights.
    sweep_ms = time_sweep()
    sweep_ms_nopack = time_sweep(packs=False)
    sweep_ms_unpacked = time_sweep(packs=False, packed=False)
    sweep_flops = sum(3 * L["flops"] for L in layers)
    sweep_tf = sweep_flops / (sweep_ms * 1e-3) / 1e12

    # per-op durations: op-reps back-to-back launches replayed from a graph
    per_op = []
    for L in layers:
        for ps in PASSES + ("pack",):
            run_op(L, ps)
            t = time_graph(ctx, lambda: run_op(L, ps), args.op_reps)
            if ps == "pack":
                per_op.append(dict(op=f"{L['name']}:pack", ms=round(t, 5),
                                   note="packs W for both the forward and dX kernels"))
                continue
            tf = L["flops"] / (t * 1e-3) / 1e12
            per_op.append(dict(op=f"{L['name']}:{ps}", ms=round(t, 5), tflops=round(tf, 2),
                               frac=round(tf / PEAK_FP32_MFMA_TFLOPS, 4),
                               in_resnet_step=RESNET_OPS[L["name"]]))

    def roofline(op_row, flops):
        achieved = flops / (op_row["ms"] * 1e-3) / 1e12
        return {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_FP32_MFMA_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4),
                "traffic": traffic_from_profiles(op_row["op"]), "kernel": op_row["op"],
                "flop_per_launch": flops, "avg_launch_ms": op_row["ms"]}

    lay = {L["name"]: L for L in layers}
    # dominant op of the ResNet step: largest multiplicity x duration
    conv_ops = [r for r in per_op if "tflops" in r]
    dom = max(conv_ops, key=lambda r: r["ms"] * r["in_resnet_step"])
    roof = roofline(dom, lay[dom["op"].split(":")[0]]["flops"])
    roof["share_of_resnet_step"] = round(dom["ms"] * dom["in_resnet_step"] / rn["ms"], 4)
    sdom = max(conv_ops, key=lambda r: r["ms"])
    sweep_roof = roofline(sdom, lay[sdom["op"].split(":")[0]]["flops"])

    attention = bench_attention(R, ctx, args.op_reps)
    gemms = bench_gemm(R, ctx, args.op_reps)

    cpu = sweep_cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_resnet(args.cpu_budget)
        sweep_cpu = cpu_baseline(args.cpu_budget / 2)

    c = RESNET
    model_tf = rn["flop_per_image"] * rn["images_s"] / 1e12
    out = {
        "metric": METRIC, "value": round(rn["images_s"], 1), "unit": "images/s", "n_gpus": 1,
        "steps": args.steps, "warmup": max(args.warmup, 2), "ms_per_step": round(rn["ms"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic (images uniform [0,1] normalised with the CIFAR-100 mean/std, "
                "labels uniform over 100; random Kaiming init; drawn on the device)",
        "config": {"workload": "config3 ResNet-20 W32 train step: forward + softmax-CE "
                               "(smooth 0.1) + backward + Nesterov SGD (lr 0.2, mom 0.9, "
                               "wd 5e-4), batch 128, 32x32x3",
                   "batch": c["batch"], "depth": 6 * c["depth_n"] + 2, "width": c["width"],
                   "classes": c["nclass"], "params": rn["params"],
                   "flop_per_image": rn["flop_per_image"],
                   "model_tflops": round(model_tf, 3),
                   "model_frac_of_fp32_mfma_peak": round(model_tf / PEAK_FP32_MFMA_TFLOPS, 4),
                   "hip_graph": rn["graph"], "wall_s_timed": round(rn["wall"], 3)},
        "roofline": roof, "cpu_baseline": cpu,
        "vs_cpu_baseline": round(rn["images_s"] / cpu["value"], 1) if cpu else None,
        "config1_conv_sweep": {
            "value": round(sweep_tf, 3), "unit": "TFLOP/s", "ms_per_step": round(sweep_ms, 4),
            "frac_of_fp32_mfma_peak": round(sweep_tf / PEAK_FP32_MFMA_TFLOPS, 4),
            "step": "per layer: pack W (forward + dX forms), forward, dX, dW",
            "tflops_without_packs": round(sweep_flops / (sweep_ms_nopack * 1e-3) / 1e12, 3),
            "tflops_unpacked_weights": round(sweep_flops / (sweep_ms_unpacked * 1e-3) / 1e12,
                                             3),
            "flop_per_step": sweep_flops, "roofline": sweep_roof, "cpu_baseline": sweep_cpu,
            "per_op": per_op},
        "config2_attention": attention, "gemmbench": gemms,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
