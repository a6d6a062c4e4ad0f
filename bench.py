#!/usr/bin/env python3
"""Benchmark of the MI355X GEMM core of rustnn (one GPU).

Metric: "ResNet-20 W32 train images/s; implicit-GEMM conv
TFLOP/s and % fp32 MFMA peak".

Headline (`value`, images/s): BASELINE config 3, the full ResNet-20 (W=32)
train step at batch 128 on 32x32 synthetic images -- forward, softmax
cross-entropy (smoothing 0.1), backward and the Nesterov SGD step (lr 0.2,
momentum 0.9, wd 5e-4) -- through the device-resident runtime (rnn_resnet_*,
issued eagerly; the 3x3 stride-1 weight gradients in one grouped launch
after the input-gradient chain, the others on a second stream beside it),
every operand resident in HBM.  One "step"
is one train step on one batch; `value` = steps * 128 / timed seconds.

Also reported:
  * `roofline`: the kernel template with the most launch time per ResNet
    step (`candidates` lists them all): its algorithmic FLOP per launch / its
    average launch duration in the committed rocprofv3 kernel trace
    (profiles/resnet20_step_kernel_stats.md for the step's grouped dW launch,
    profiles/conv_sweep_kernel_stats.md for a sweep op) vs the 157.3 TFLOP/s
    fp32 MFMA peak (`frac`); the same kernel timed live with HIP events on
    the library's stream beside it (`live`); `traffic` from the committed
    rocprofv3 --pmc summary and `traffic_ratio` = that traffic / the kernel's
    algorithmic bytes;
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
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
# The CPU baseline's OpenMP threads stay on their cores (the reference's
# protocol binds its rayon pool by running pinned; OMP_PROC_BIND=close is the
# OpenMP statement of it).  Read when the OpenMP runtime starts, so set first.
os.environ.setdefault("OMP_PROC_BIND", "close")
os.environ.setdefault("OMP_PLACES", "cores")
# The CPUs this process may use, read before an OpenMP runtime binds the main
# thread to one of them.
USABLE_CPUS = sorted(os.sched_getaffinity(0))

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
# Per-op rows also time the dW kernel alone ("dw_kernel": the split-K slabs
# without their reduction), which is how each dW runs inside the ResNet step
# (the step folds the slab sums into its gradient pass).
OP_PASSES = PASSES + ("dw_kernel",)
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


def op_bytes(op):
    """Algorithmic HBM bytes of one launch of a sweep op ("name:pass"), each
    tensor once: fwd x + W + y, dx dY + W + dX, dw / dw_kernel dY + x + dW.
    A 1x1 stride-2 op counts only the x positions its window samples.  None
    for an op outside the sweep."""
    name, _, ps = op.partition(":")
    for nm, cin, cout, k, s, p, h in SWEEP:
        if nm != name:
            continue
        oh = (h + 2 * p - k) // s + 1
        xin = N * cin * (oh * oh if k == 1 else h * h)
        w, yo = cout * cin * k * k, N * cout * oh * oh
        if ps == "fwd":
            return 4 * (xin + w + yo)
        if ps == "dx":
            return 4 * (yo + w + N * cin * h * h)
        if ps in ("dw", "dw_kernel"):
            return 4 * (yo + xin + w)
    return None


def step_profile_avg(template):
    """Average duration (us) of kernel `template` in the committed kernel
    trace of the ResNet step (profiles/resnet20_step_kernel_stats.md), or
    None."""
    path = os.path.join(ROOT, "profiles", "resnet20_step_kernel_stats.md")
    if not os.path.exists(path):
        return None
    for ln in open(path):
        cells = [c.strip().strip("`") for c in ln.strip().strip("|").split("|")]
        if len(cells) >= 4 and cells[0] == template:
            try:
                return float(cells[3])
            except ValueError:
                return None
    return None


def step_profile_traffic(template):
    """HBM bytes per launch of kernel `template` of the ResNet step from the
    committed rocprofv3 --pmc summary profiles/resnet20_dw_group_hbm_traffic.md
    (FETCH_SIZE + WRITE_SIZE, scaled as recorded there), or None."""
    path = os.path.join(ROOT, "profiles", "resnet20_dw_group_hbm_traffic.md")
    if not os.path.exists(path):
        return None
    for ln in open(path):
        cells = [c.strip().strip("`") for c in ln.strip().strip("|").split("|")]
        if len(cells) >= 5 and cells[0] == template:
            try:
                return float(cells[4]) * 1024
            except ValueError:
                return None
    return None


DW_GROUP_TEMPLATE = "conv_dw_group_kernel<3, 1, 0, 2>"


def step_profile_table():
    """[(kernel template, us per step)] of the committed kernel trace of the
    ResNet step (profiles/resnet20_step_kernel_stats.md), most time first."""
    path = os.path.join(ROOT, "profiles", "resnet20_step_kernel_stats.md")
    out = []
    if not os.path.exists(path):
        return out
    for ln in open(path):
        cells = [c.strip().strip("`") for c in ln.strip().strip("|").split("|")]
        if len(cells) >= 5 and cells[0] != "kernel":
            try:
                out.append((cells[0], float(cells[2])))
            except ValueError:
                pass
    return sorted(out, key=lambda t: -t[1])


def template_base(t):
    """A conv_fast_kernel template without its last argument (the store-pass
    statistics flag: the step's forward convs take the batch statistics in
    the store pass, the sweep's forward ops do not), else t."""
    return t.rsplit(",", 1)[0] if t.startswith("conv_fast_kernel<") else t


def profile_kernels(op):
    """The kernel rows of `op` in the committed rocprofv3 kernel-trace summary
    profiles/conv_sweep_kernel_stats.md: [(kernel template, avg us)], the
    op's main kernel first; [] when the op is not in it."""
    path = os.path.join(ROOT, "profiles", "conv_sweep_kernel_stats.md")
    if not os.path.exists(path):
        return []
    out, cur = [], None
    for ln in open(path):
        if not ln.startswith("|") or ln.startswith("|---"):
            continue
        cells = [c.strip() for c in ln.strip().strip("|").split("|")]
        if len(cells) < 3:
            continue
        if cells[0]:
            cur = cells[0].strip("`")
        if cur == op:
            try:
                out.append((cells[1].strip("`").split(" (")[0], float(cells[2])))
            except ValueError:
                pass
    return out


def host_cpu():
    """The host CPU as lscpu reports it, and the CPUs this process may use."""
    info = {}
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
    except (OSError, subprocess.SubprocessError):
        txt = ""
    for ln in txt.splitlines():
        k, _, v = ln.partition(":")
        k, v = k.strip(), v.strip()
        if k in ("Model name", "Socket(s)", "Core(s) per socket", "Thread(s) per core", "CPU(s)"):
            info[k] = v
    info["cpus_usable"] = len(USABLE_CPUS)
    return info


class _PinnedThread:
    """Runs the block on one thread pinned to one usable CPU."""

    def __enter__(self):
        self.old = os.sched_getaffinity(0)
        os.sched_setaffinity(0, {USABLE_CPUS[0]})
        return self

    def __exit__(self, *a):
        os.sched_setaffinity(0, self.old)


def cpu_protocol(samples=3, cooldown_s=1.0):
    """The restated reference CPU path (oracle/: the 6x16 AVX2 micro-kernel,
    KC 256 packing, fused im2col / col2im, per-image parallel convs, 6-row
    panel parallel matmul, split-K matmul_dw, per-image attention) timed on
    this host by the reference's regression protocol: every workload with all the
    usable cores (OpenMP, OMP_PROC_BIND=close) and with one pinned thread;
    `samples` samples each, the best kept (regress.sh:57-76), with a
    cooldown between samples; inputs seeded with the restated Rng (seed 7,
    bench.rs:16).  Workloads: config 0 (forward, dX, dW at batch 128),
    config 1 (the whole sweep, forward + dX + dW of every shape at batch
    128), config 2 (Core forward and backward, 512 problems), the six
    --gemmbench shapes (1 warm-up + 5 reps, bench.rs:29-35) and the config-3
    ResNet-20 train step at batch 128 (one warm-up step, then one timed
    step per sample), on all cores and on the one pinned thread alike."""
    import numpy as np
    from oracle import pyorc as O
    from oracle import pymodel as M
    O.build()
    allt = max(1, len(USABLE_CPUS))
    rng = O.Rng(7)
    convs = []
    for name, cin, cout, k, st, p, h in SWEEP:
        sp = O.ConvSpec.make(cin, cout, k, st, p, h, h)
        x = rng.rand_vec(N * cin * h * h)
        w = rng.rand_vec(cout * sp.ckk) * np.float32(np.sqrt(2.0 / sp.ckk))
        dy = rng.rand_vec(N * cout * sp.hw)
        convs.append((name, sp, x, w, dy, pass_flops(cin, cout, k, st, p, h)))
    # config 2: SelfAttn buffer [128, 64, 384], tau 1, rel 0, no mask
    n2, h2, dh2, t2 = 128, 4, 32, 64
    c2 = h2 * dh2
    relidx, nrel = O.rel_index(8, 8, 8, 8)
    qkv = rng.rand_vec(n2 * t2 * 3 * c2) * np.float32(1 / np.sqrt(dh2))
    dout = rng.rand_vec(n2 * t2 * c2)
    tau, rel = np.ones(h2, np.float32), np.zeros(h2 * nrel, np.float32)
    desc = O.attn_desc(h2, dh2, t2, t2, 3 * c2, 0, 3 * c2, c2, 2 * c2, relidx, nrel, False)
    p_att, _ = O.attn_forward(desc, n2, qkv, qkv, tau, rel)
    z = np.zeros(qkv.size, np.float32)
    gem = []
    for m, n, k, at, bt, tag in GEMMBENCH:
        gem.append((tag, m, n, k, at, bt, rng.rand_vec(m * k), rng.rand_vec(k * n)))
    c = RESNET
    u = rng.uniform_vec(c["batch"] * 3 * 32 * 32).reshape(c["batch"], 3, 32, 32)
    xr = ((u - np.array(CIFAR_MEAN, np.float32)[None, :, None, None]) /
          np.array(CIFAR_STD, np.float32)[None, :, None, None]).astype(np.float32)
    lab = np.array([rng.below(100) for _ in range(c["batch"])], np.uint32)
    net = M.ResNet(c["depth_n"], c["width"], c["nclass"], c["seed"])

    def timed(fn):
        t0 = time.perf_counter()
        fn()
        return time.perf_counter() - t0

    def one_sample(threads):
        r = {}
        cfg0 = convs[0]
        _, sp, x, w, dy, fl = cfg0
        for ps, fn in (("fwd", lambda: O.conv2d_forward(sp, N, x, w)),
                       ("dx", lambda: O.conv2d_backward_x(sp, N, dy, w)),
                       ("dw", lambda: O.conv2d_backward_w(sp, N, dy, x))):
            r["config0_" + ps] = fl / timed(fn) / 1e9
        r["config1_sweep"] = sum(3 * cv[5] for cv in convs) / timed(lambda: [
            (O.conv2d_forward(cv[1], N, cv[2], cv[3]), O.conv2d_backward_x(cv[1], N, cv[4], cv[3]),
             O.conv2d_backward_w(cv[1], N, cv[4], cv[2])) for cv in convs]) / 1e9
        r["config2_fwd"] = 2 * 2.0 * n2 * h2 * t2 * t2 * dh2 / timed(
            lambda: O.attn_forward(desc, n2, qkv, qkv, tau, rel)) / 1e9
        r["config2_bwd"] = 4 * 2.0 * n2 * h2 * t2 * t2 * dh2 / timed(
            lambda: O.attn_backward(desc, n2, qkv, qkv, tau, p_att, dout, z, z,
                                    np.zeros(h2, np.float32),
                                    np.zeros(h2 * nrel, np.float32))) / 1e9
        reps = 5
        for tag, m, n, k, at, bt, a, b in gem:
            O.matmul(m, n, k, a, at, b, bt)  # bench.rs:29-30: one untimed call
            r["gemm " + tag] = 2.0 * m * n * k * reps / timed(
                lambda: [O.matmul(m, n, k, a, at, b, bt) for _ in range(reps)]) / 1e9
        bs = c["batch"]
        step = lambda: net.train_step(xr[:bs], lab[:bs], c["smooth"], c["lr"], c["mom"], c["wd"])
        if threads not in warmed:
            step()
            warmed.add(threads)
        r["config3_step"] = bs / timed(step)
        return r

    out = {}
    warmed = set()
    for label, threads in (("all_cores", allt), ("one_thread", 1)):
        best = {}
        for i in range(samples):
            if i:
                time.sleep(cooldown_s)
            with O.threads(threads):
                if threads == 1:
                    with _PinnedThread():
                        r = one_sample(1)
                else:
                    r = one_sample(threads)
            for k, v in r.items():
                best[k] = max(best.get(k, 0.0), v)
        out[label] = {"threads": threads, **{k: round(v, 2) for k, v in best.items()}}
    out["units"] = {"config0_*, config1_sweep, config2_*, gemm *": "GFLOP/s",
                    "config3_step": "images/s"}
    out["protocol"] = (f"best of {samples} samples, {cooldown_s:g} s cooldown between samples, "
                       "OMP_PROC_BIND=close; one thread pinned with sched_setaffinity; "
                       "gemm shapes 1 warm-up + 5 timed calls (bench.rs:29-35); config-3 step "
                       "at batch 128 after one warm-up step per thread count, one timed step "
                       "per sample")
    out["host"] = host_cpu()
    out["label"] = "restated reference CPU path (oracle/, C + AVX2), not the Rust binary"
    return out


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


MALL_BYTES = 256 << 20  # MI355X Infinity Cache: rotated inputs exceed it


def bench_attention(R, ctx, reps):
    """128 images x 4 heads, T=64 (8x8), dh=32, SelfAttn
    buffer [128, 64, 384] (q/k/v at 0/128/256), tau=1, rel=0, no mask; Q, K, V
    ~N(0,1)/sqrt(32), dO ~N(0,1).  HBM-bound: algorithmic bytes (each tensor
    once) fwd Q,K,V,O + P, bwd Q,K,V,dO,P in + dQ,dK,dV out.  Timed twice:
    the same buffers every call (they stay in the 256 MB Infinity Cache) and
    with every call on its own copy of all its operands, rotating through
    enough copies to exceed that cache, so each call reads HBM."""
    import torch
    n, h, dh, t = 128, 4, 32, 64
    c = h * dh
    g = torch.Generator(device="cuda").manual_seed(7)
    relidx, nrel = R.rel_index(8, 8, 8, 8)
    tau = torch.ones(h, device="cuda")
    rel = torch.zeros(h * nrel, device="cuda")
    core = R.Core(h, dh, t, t, relidx, nrel, False, ctx=ctx)
    mb = n * h * t * dh * 4  # one [n, h, t, dh] tensor, bytes
    pb = n * h * t * t * 4
    ncopy = -(-MALL_BYTES // (7 * mb + pb)) + 1
    sets = []
    for _ in range(ncopy):
        qkv = torch.randn(n * t * 3 * c, device="cuda", generator=g) / dh ** 0.5
        sets.append(dict(qkv=qkv, dout=torch.randn(n * t * c, device="cuda", generator=g),
                         p=torch.empty(n * h * t * t, device="cuda"),
                         o=torch.empty(n * t * c, device="cuda"), dqkv=torch.zeros_like(qkv)))
    dtau = torch.zeros(h, device="cuda")
    drel = torch.zeros(h * nrel, device="cuda")
    state = {"i": 0}

    def fwd(rot):
        b = sets[state["i"] % ncopy] if rot else sets[0]
        state["i"] += 1
        core.forward(n, b["qkv"], 3 * c, 0, b["qkv"], 3 * c, c, 2 * c, tau, rel, b["p"], b["o"])

    def bwd(rot, acc=False):
        # SelfAttn::backward (attn.rs:418-438): dq, dk, dv written into one
        # fused-QKV gradient; acc: the accumulating form (reads dqkv as well)
        b = sets[state["i"] % ncopy] if rot else sets[0]
        state["i"] += 1
        core.backward(n, b["qkv"], 3 * c, 0, b["qkv"], 3 * c, c, 2 * c, tau, b["p"], b["dout"],
                      b["dqkv"], b["dqkv"], dtau, drel, set_dq=not acc, set_dkv=not acc)

    for b in sets:  # every copy gets a P before the backward reads it
        core.forward(n, b["qkv"], 3 * c, 0, b["qkv"], 3 * c, c, 2 * c, tau, rel, b["p"], b["o"])
    bwd(False)
    # A call costs more host time than these kernels take, so back-to-back
    # eager calls would time the host: record the calls into a graph (on a
    # capture stream given to the library's context) and time its replays.
    nrep = max(reps, 2 * ncopy)
    times = {}
    for rot in (False, True):
        times[("fwd", rot)] = time_graph(ctx, lambda: fwd(rot), nrep)
        times[("bwd", rot)] = time_graph(ctx, lambda: bwd(rot), nrep)
    times[("bwd_accumulate", True)] = time_graph(ctx, lambda: bwd(True, acc=True), nrep)
    fwd_bytes, bwd_bytes = 4 * mb + pb, 7 * mb + pb
    fwd_flop = 2 * 2.0 * n * h * t * t * dh
    bwd_flop = 4 * 2.0 * n * h * t * t * dh
    res = {}
    for name, by, fl in (("fwd", fwd_bytes, fwd_flop), ("bwd", bwd_bytes, bwd_flop)):
        for rot in (True, False):
            ms = times[(name, rot)]
            gbs = by / (ms * 1e-3) / 1e9
            res[name + ("" if rot else "_cache_resident")] = {
                "us": round(ms * 1e3, 2), "GB_s": round(gbs, 1),
                "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
                "TFLOP_s": round(fl / (ms * 1e-3) / 1e12, 3), "bytes": by}
    ms = times[("bwd_accumulate", True)]
    acc_bytes = bwd_bytes + 3 * mb  # the old dQ, dK, dV read as well
    res["bwd_accumulate"] = {"us": round(ms * 1e3, 2),
                             "GB_s": round(acc_bytes / (ms * 1e-3) / 1e9, 1),
                             "hbm_frac": round(acc_bytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                             "bytes": acc_bytes}
    res["workload"] = ("config2: 512 (image, head) problems, T=64, dh=32, fwd + bwd (bwd as "
                       "SelfAttn::backward: dq, dk, dv written; bwd_accumulate: added to dqkv)")
    res["timing"] = (f"graph replays of {nrep} back-to-back calls (launch gaps included); "
                     f"fwd / bwd: each call on its own operands, rotating over {ncopy} copies "
                     f"({ncopy * (7 * mb + pb) >> 20} MiB, past the 256 MiB Infinity Cache); "
                     "*_cache_resident: one set of operands")
    return res


def bench_1x1_rotated(R, ctx, layers, run_op, reps):
    """The 1x1 stride-2 shortcut convs are HBM-bound: their passes in GB/s
    against 8 TB/s, each call on its own copy of its operands, rotating over
    enough copies to exceed the 256 MB Infinity Cache.  Algorithmic bytes:
    forward x at the sampled positions + W + y; dX dY + W + dX (written
    whole: the skipped positions get zeros); dW dY + x at the sampled
    positions + the weight-gradient slabs the kernel writes."""
    import torch
    out = []
    for L in layers:
        sp = L["sp"]
        if sp.k != 1 or sp.stride != 2:
            continue
        n_in, n_out = N * sp.cin * sp.h * sp.w, N * sp.cout * sp.oh * sp.ow
        sampled = N * sp.cin * sp.oh * sp.ow
        per_set = 4 * (2 * n_in + 2 * n_out)
        ncopy = -(-MALL_BYTES // per_set) + 1
        sets = []
        for _ in range(ncopy):
            c = dict(L)
            c["x"] = torch.randn(n_in, device="cuda")
            c["dy"] = torch.randn(n_out, device="cuda")
            c["y"] = torch.empty(n_out, device="cuda")
            c["dx"] = torch.empty(n_in, device="cuda")
            sets.append(c)
        wb = 4 * sp.cout * sp.cin
        slab_b = 4 * L["slabs"].numel()
        bytes_of = {"fwd": 4 * (sampled + n_out) + wb, "dx": 4 * (n_out + n_in) + wb,
                    "dw_kernel": 4 * (n_out + sampled) + slab_b}
        for ps, by in bytes_of.items():
            st = {"i": 0}

            def one():
                run_op(sets[st["i"] % ncopy], ps)
                st["i"] += 1
            one()
            ms = time_graph(ctx, one, max(reps, 2 * ncopy))
            gbs = by / (ms * 1e-3) / 1e9
            out.append({"op": f"{L['name']}:{ps}", "us": round(ms * 1e3, 2), "bytes": by,
                        "GB_s": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
                        "copies": ncopy})
    return out


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


# rustvit default configuration (vit.rs:371-387, cli.rs:97-100): Muon with 3
# Newton-Schulz steps, clip 1.0, EMA 0.9998; 100 fine / 20 coarse classes.
VIT = dict(width=32, cmid=96, dim=256, heads=4, depth3=5, dim4=384, heads4=6, depth4=2,
           mem_at=(1, 3), img=32, nclass=100, ncoarse=20, ns=3, clip=1.0, ema=0.9998)


def rustvit_param_specs(R):
    """(len, rows, cols, decay) of every parameter of the default RustViT in
    for_each_param order (vit.rs:690-716, Block vit.rs:234-249): Linear
    weights are [fout x fin] matrices (linear.rs:25-33) and take Muon; conv
    kernels, norms, LayerScale, biases, tau / rel and SeqPool vectors AdamW."""
    c = VIT
    out = []
    conv = lambda cin, cout, k: out.append((cout * cin * k * k, 0, 0, True))  # nn.rs:135
    vec = lambda n, decay=False: out.append((n, 0, 0, decay))

    def bn(ch):
        vec(ch)
        vec(ch)

    def lin(fin, fout, bias=True):
        out.append((fin * fout, fout, fin, True))
        if bias:
            vec(fout)

    def basic(cin, cout, stride):  # model.rs:21-33
        conv(cin, cout, 3)
        bn(cout)
        conv(cout, cout, 3)
        bn(cout)
        if stride != 1 or cin != cout:
            conv(cin, cout, 1)
            bn(cout)

    def block(ch, h, th, mem):  # vit.rs:108-135
        hidden = -(-(4 * ch // 3) // 16) * 16
        nrel = R.rel_index(th, th, th, th)[1]
        bn(ch)                                  # n1
        lin(ch, 3 * ch)                         # attn.qkv
        lin(ch, ch)                             # attn.proj
        vec(h)                                  # attn.tau
        vec(h * nrel)                           # attn.rel
        vec(9 * ch)                             # dw.w
        vec(ch)                                 # dw.b
        vec(ch)                                 # gamma
        vec(ch)                                 # ls1
        if mem:
            lin(ch, ch)                         # cross.wq
            lin(ch, ch)                         # cross.proj
            vec(h)
            vec(h * R.rel_index(th, th, 2 * th, 2 * th)[1])
            vec(ch)                             # lsm
        bn(ch)                                  # n2
        lin(ch, 2 * hidden)                     # mlp.wg
        lin(hidden, ch)                         # mlp.wd
        vec(ch)                                 # ls2

    w, cm, d, d4 = c["width"], c["cmid"], c["dim"], c["dim4"]
    th = c["img"] // 4
    conv(3, w, 3)
    bn(w)
    basic(w, w, 1)
    basic(w, cm, 2)
    conv(cm, 2 * d, 1)                          # memconv
    bn(2 * d)                                   # memln
    conv(cm, d, 3)                              # tokconv
    bn(d)
    for i in range(c["depth3"]):
        block(d, c["heads"], th, i in c["mem_at"])
    bn(4 * d)                                   # mergeln
    lin(4 * d, d4)                              # merge
    for _ in range(c["depth4"]):
        block(d4, c["heads4"], th // 2, False)
    bn(d4)                                      # headln
    vec(d4, True)                               # pool.p
    lin(d4, c["ncoarse"])                       # head.coarse
    lin(d4, c["nclass"])                        # head.resid
    lin(cm, c["nclass"])                        # e1.fc
    lin(cm, d4, False)                          # e1.hint
    vec(d, True)                                # pool2.p
    lin(d, c["nclass"])                         # e2.fc
    lin(d, d4, False)                           # e2.hint
    return out


def bench_rustvit_optim(R, ctx, reps, cpu_budget):
    """The optimiser phase of a rustvit train step (train.rs:371-379) over the
    default model's parameters: clip_ (1.0), Optim::step_all (Muon, 3
    Newton-Schulz steps; AdamW for the rest) and the EMA update.  Gradients are
    N(0,1) in one flat buffer that every step refills (one copy, included).
    Timed from graph replays of `reps` steps (the AdamW bias correction stays
    at the captured step) and, eagerly, with the Python calls included."""
    import numpy as np
    import torch
    from rustnn_amd.optim import Ema, Optim, Param, clip_
    specs = rustvit_param_specs(R)
    total = sum(n for n, _, _, _ in specs)
    g = torch.Generator(device="cuda").manual_seed(11)
    gsrc = torch.randn(total, device="cuda", generator=g)
    gflat = torch.empty_like(gsrc)
    params, off = [], 0
    for n, r, cc, dec in specs:
        p = Param(torch.randn(n, device="cuda", generator=g) * 0.02, dec, r, cc)
        p.g = gflat[off:off + n]
        off += n
        params.append(p)
    opt = Optim(True, VIT["ns"], ctx=ctx)
    ema = Ema(VIT["ema"], ctx=ctx)
    norm = torch.zeros(1, device="cuda")
    lr, wd = 1e-3, 0.05

    def phase():
        gflat.copy_(gsrc)
        clip_(params, VIT["clip"], ctx=ctx, norm=norm)
        opt.step_all(params, lr, wd)
        ema.update(params)

    def step_only():
        gflat.copy_(gsrc)
        opt.step_all(params, lr, wd)

    for _ in range(3):
        phase()
    torch.cuda.synchronize()
    ms_phase = time_graph(ctx, phase, reps)
    ms_step = time_graph(ctx, step_only, reps)
    ms_eager = time_gpu(phase, reps)
    muon = [(n, r, cc) for n, r, cc, _ in specs if r > 0 and min(r, cc) > 1]
    ns_flop = 0
    for _, r, cc in muon:
        m, n = min(r, cc), max(r, cc)
        ns_flop += VIT["ns"] * 2.0 * (m * m * n + m * m * m + m * m * n)
    res = {"workload": "rustvit default (d256x5-384x2, mem at blocks 1,3): clip 1.0 + "
                       "Muon/AdamW step_all + EMA 0.9998 over every parameter",
           "params": total, "tensors": len(specs), "muon_matrices": len(muon),
           "muon_shapes": len({(r, cc) for _, r, cc in muon}),
           "ms_optimizer_phase": round(ms_phase, 4), "ms_step_all": round(ms_step, 4),
           "ms_optimizer_phase_eager": round(ms_eager, 4),
           "ns_tflop_s": round(ns_flop / (ms_step * 1e-3) / 1e12, 3),
           "timing": "graph replays (ms per phase); eager: back-to-back Python calls"}
    if cpu_budget > 0:
        res["cpu_baseline"] = cpu_rustvit_optim(specs, cpu_budget)
        res["vs_cpu_baseline"] = round(res["cpu_baseline"]["ms"] / ms_phase, 1)
    opt.close()
    return res


def cpu_rustvit_optim(specs, budget_s):
    """The oracle's optimiser phase over the same parameter list: clip, then
    Muon over the matrices on an OpenMP loop (the reference's rayon par_iter
    over the parameters, optim.rs:177-196; largest Newton-Schulz first), AdamW,
    the EMA; on host threads."""
    import numpy as np
    from oracle import pyorc as O
    O.build()
    threads = int(os.environ.get("OMP_NUM_THREADS", len(USABLE_CPUS)))
    threads = max(1, min(threads, 16, len(USABLE_CPUS)))
    rng = np.random.default_rng(3)
    ps = [dict(v=(rng.standard_normal(n) * 0.02).astype(np.float32),
               g0=rng.standard_normal(n).astype(np.float32), m=np.zeros(n, np.float32),
               v2=np.zeros(n, np.float32), w=None, r=r, c=cc, d=dec) for n, r, cc, dec in specs]
    for p in ps:
        p["w"] = p["v"].copy()
    lens = [p["v"].size for p in ps]
    muon = [p for p in ps if p["r"] > 0 and min(p["r"], p["c"]) > 1]
    adam = [p for p in ps if not (p["r"] > 0 and min(p["r"], p["c"]) > 1)]
    # Largest Newton-Schulz first (cost ~ min^2 * max), so that the loop's
    # last matrices are small ones; the updates are independent.
    muon.sort(key=lambda p: -min(p["r"], p["c"]) ** 2 * max(p["r"], p["c"]))
    gall = np.concatenate([p["g0"] for p in ps])
    offs = np.cumsum([0] + lens)
    index = {id(p): i for i, p in enumerate(ps)}

    def one(t):
        g = gall.copy()
        O.clip(g, lens, VIT["clip"])
        gs = [g[offs[i]:offs[i + 1]] for i in range(len(ps))]
        O.muon_steps([(p["v"], gs[index[id(p)]], p["m"], p["r"], p["c"], p["d"]) for p in muon],
                     1e-3, 0.05, 0.95, VIT["ns"], threads=threads)
        for p in adam:
            O.adam_step(p["v"], gs[index[id(p)]], p["m"], p["v2"], p["d"], 1e-3, 0.05, t)
        for p in ps:
            O.ema_update(p["w"], p["v"], VIT["ema"], t + 2)

    one(0)
    steps, t0 = 0, time.perf_counter()
    while True:
        one(steps + 1)
        steps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or el / steps * (steps + 1) > 2.5 * budget_s:
            break
    return {"ms": round(el / steps * 1e3, 3), "cores": threads, "kind": "port",
            "sample": f"{steps} optimiser phases in {el:.1f}s after 1 warm-up; Muon matrices "
                      f"on an OpenMP loop over {threads} threads (OMP_PROC_BIND=close, largest "
                      f"first), the rest on one"}


def bench_rustvit_step(R, ctx, steps, warmup, batch=128):
    """the rustvit default train step at batch 128 --
    forward, soft targets with the taxonomy (5 fine classes per superclass,
    fixed seeded assignment), the multi-head loss, backward, clip, Muon /
    AdamW and the EMA (train.rs:340-380).  Inputs uniform [0, 1] normalised,
    labels uniform over 100 classes; all on the device.  Timed eagerly (the
    Python layer issues every launch)."""
    import numpy as np
    import torch
    from rustnn_amd.vit import RustViT, ViTStep
    g = torch.Generator(device="cuda").manual_seed(2026)
    parent_np = np.random.default_rng(7).permutation(np.arange(100) // 5).astype(np.int32)
    parent = torch.from_numpy(parent_np).cuda()
    net = RustViT(None, parent, 20, seed=7, ctx=ctx)
    step = ViTStep(net, parent, 20)
    u = torch.rand(batch, 3, 32, 32, device="cuda", generator=g)
    mean = torch.tensor(CIFAR_MEAN, device="cuda").view(1, 3, 1, 1)
    std = torch.tensor(CIFAR_STD, device="cuda").view(1, 3, 1, 1)
    x = ((u - mean) / std).contiguous()
    labels = torch.randint(0, 100, (batch,), device="cuda", generator=g, dtype=torch.int32)
    coarse = parent[labels.long()].contiguous()
    for i in range(warmup):
        net.drop_seed = 1000 + i
        step(x, labels, coarse)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for i in range(steps):
        net.drop_seed = 2000 + i  # a fresh DropPath draw per step, as the trainer's rng gives
        loss, _ = step(x, labels, coarse)
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / steps
    cfg = net.cfg
    return {"workload": "config4 rustvit default (width 32, cmid 96, d256 x 5 with memory readers "
                        "at 1,3, d384 x 2) train step at batch %d: forward + taxonomy targets + "
                        "multi-head loss + backward + clip + Muon/AdamW + EMA" % batch,
            "batch": batch, "ms_per_step": round(ms, 3), "images_s": round(batch / (ms * 1e-3), 1),
            "wall_ms_per_step": round(wall / steps * 1e3, 3), "loss": float(loss.item()),
            "params": sum(p.v.numel() for p in step.params),
            "reference_published": "102.6 img/s at batch 256 on a Core Ultra 265U CPU "
                                   "(the reference's README.md:426)",
            "timing": "eager, HIP events around the steps; drop_seed changes per step"}


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


def bench_resnet(R, ctx, steps, warmup, time_group=True):
    """Config 3: the ResNet-20 train step through rnn_resnet_train_step
    (and, with time_group, the step's grouped dW launch alone)."""
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
    # The step's grouped weight-gradient launch (every 3x3 stride-1 conv's dW
    # in one persistent kernel) timed alone: graph replays of back-to-back
    # launches over the buffers the last backward left, HIP events on the
    # library's stream.
    gfl = net.dw_group(launch=False)
    if gfl and time_group:
        net.dw_group()
        torch.cuda.synchronize()
        out["dw_group"] = {"flops": gfl, "ms": time_graph(ctx, lambda: net.dw_group(), 10)}
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
    ap.add_argument("--vit-only", type=int, default=0, metavar="STEPS",
                    help="only the config-4 rustvit train step, STEPS timed steps")
    ap.add_argument("--optim-only", type=int, default=0, metavar="REPS",
                    help="only the rustvit optimiser phase, REPS phases per graph")
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
        r = bench_resnet(R, ctx, args.resnet_only, 2, time_group=False)
        print(json.dumps({"resnet_only": args.resnet_only, "ms": r["ms"]}))
        return
    if args.attn_only:
        print(json.dumps({"attn_only": bench_attention(R, ctx, args.attn_only)}))
        return
    if args.vit_only:
        print(json.dumps({"vit_only": bench_rustvit_step(R, ctx, args.vit_only, 2)}))
        return
    if args.optim_only:
        print(json.dumps({"optim_only": bench_rustvit_optim(R, ctx, args.optim_only,
                                                            0 if args.no_cpu else 4.0)}))
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
        slabs = torch.empty(R.conv2d_backward_w_slab_floats(sp, N, ctx=ctx), device="cuda")
        layers.append(dict(name=name, sp=sp, x=x, w=w, dy=dy, y=y, dx=dx, dw=dw, wpf=wpf,
                           wpx=wpx, slabs=slabs, flops=pass_flops(cin, cout, k, s, p, h)))

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
        elif ps == "dw_kernel":
            R.conv2d_backward_w_slabs(L["sp"], N, L["dy"], L["x"], L["slabs"], ctx=ctx)
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
            for ps in OP_PASSES:
                for _ in range(args.ops_only):
                    run_op(L, ps)
        torch.cuda.synchronize()
        print(json.dumps({"ops_only": [f"{L['name']}:{ps}" for L in layers for ps in OP_PASSES],
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
        for ps in OP_PASSES + ("pack",):
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
        # `achieved` / `frac`: the kernel's average duration in the committed
        # rocprofv3 kernel trace (every dispatch serialised and timed alone),
        # so the figure follows from profiles/; the live graph-replay timing
        # of this run (back-to-back launches, which hide part of each
        # dispatch's start-up) sits beside it under `live`.
        live_tf = flops / (op_row["ms"] * 1e-3) / 1e12
        live = {"achieved": round(live_tf, 3), "frac": round(live_tf / PEAK_FP32_MFMA_TFLOPS, 4),
                "avg_launch_ms": op_row["ms"],
                "timing": "graph replays of op-reps back-to-back launches (launch gaps "
                          "included), HIP events on the library's stream"}
        prof = profile_kernels(op_row["op"])
        if prof:
            us = prof[0][1]
            achieved, src = flops / (us * 1e-6) / 1e12, "profiles/conv_sweep_kernel_stats.md"
        else:
            us, achieved, src = op_row["ms"] * 1e3, live_tf, "live (op not in the kernel trace)"
        traffic = traffic_from_profiles(op_row["op"])
        alg = op_bytes(op_row["op"])
        out = {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_FP32_MFMA_TFLOPS,
               "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4),
               "traffic": traffic,
               "traffic_ratio": round(traffic / alg, 3) if traffic and alg else None,
               "algorithmic_bytes": alg, "kernel": op_row["op"],
               "template": prof[0][0] if prof else None,
               "flop_per_launch": flops, "avg_launch_us": us, "source": src, "live": live}
        return out

    lay = {L["name"]: L for L in layers}
    # Dominant kernel of the ResNet step: the kernel template with the most
    # launch time per step.  Candidates: the conv kernel templates of the
    # sweep ops the step launches (forward, dX, and the dW kernel of the
    # shapes without a grouped launch) with their multiplicity in the step,
    # and the step's grouped weight-gradient launch (one per step, timed
    # alone above).  A sweep template's roofline row is its op with the most
    # launch time.
    conv_ops = [r for r in per_op if "tflops" in r]
    grouped = set()
    if rn.get("dw_group"):
        grouped = {L["name"] for L in layers if L["sp"].k == 3 and L["sp"].stride == 1}
    step_kernels = [r for r in conv_ops if not r["op"].endswith(":dw") and
                    not (r["op"].endswith(":dw_kernel") and r["op"].split(":")[0] in grouped)]
    tmpl = {r["op"]: (profile_kernels(r["op"]) or [(r["op"], 0)])[0][0] for r in step_kernels}
    by_t = {}
    for r in step_kernels:
        by_t.setdefault(tmpl[r["op"]], []).append(r)
    # The dominant template is the one with the most kernel time per step in
    # the committed kernel trace of the step itself; without that file, the
    # live timings of each kernel alone times its launches per step decide.
    cands = {t: sum(r["ms"] * r["in_resnet_step"] for r in by_t[t]) for t in by_t}
    if rn.get("dw_group"):
        cands[DW_GROUP_TEMPLATE] = rn["dw_group"]["ms"]
    step_tab = step_profile_table()
    t_dom = None
    if step_tab:
        top = step_tab[0][0]
        if top == DW_GROUP_TEMPLATE and rn.get("dw_group"):
            t_dom = top
        else:
            t_dom = next((t for t in by_t if template_base(t) == template_base(top)), None)
    if t_dom is None:
        t_dom = max(cands, key=lambda t: cands[t])
    candidates = {"step_trace_us_per_step": [{"template": t, "us_per_step": v}
                                             for t, v in step_tab[:8]],
                  "live_ms_per_step": [{"template": t, "ms_per_step": round(v, 5)}
                                       for t, v in sorted(cands.items(), key=lambda kv: -kv[1])]}

    def group_roofline():
        gf, gms = rn["dw_group"]["flops"], rn["dw_group"]["ms"]
        live_tf = gf / (gms * 1e-3) / 1e12
        us = step_profile_avg(DW_GROUP_TEMPLATE)
        if us:
            achieved, src = gf / (us * 1e-6) / 1e12, "profiles/resnet20_step_kernel_stats.md"
        else:
            us, achieved, src = gms * 1e3, live_tf, "live (kernel not in the step trace)"
        members = [(L["name"], RESNET_OPS[L["name"]]) for L in layers if L["name"] in grouped]
        alg = sum(m * op_bytes(f"{nm}:dw_kernel") for nm, m in members)
        traffic = step_profile_traffic(DW_GROUP_TEMPLATE)
        return {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_FP32_MFMA_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4),
                "traffic": traffic,
                "traffic_ratio": round(traffic / alg, 3) if traffic and alg else None,
                "algorithmic_bytes": alg, "kernel": "resnet step: grouped dW of " +
                ", ".join(f"{nm} x{m}" for nm, m in members),
                "template": DW_GROUP_TEMPLATE, "flop_per_launch": gf, "avg_launch_us": us,
                "source": src,
                "live": {"achieved": round(live_tf, 3),
                         "frac": round(live_tf / PEAK_FP32_MFMA_TFLOPS, 4),
                         "avg_launch_ms": round(gms, 5),
                         "timing": "graph replays of 10 back-to-back launches over the last "
                                   "backward's buffers (rnn_dbg_resnet_dw_group), HIP events "
                                   "on the library's stream"},
                "share_of_resnet_step": round(gms / rn["ms"], 4),
                "template_launches_per_step": 1}

    if t_dom == DW_GROUP_TEMPLATE:
        roof = group_roofline()
    else:
        rows_t = by_t[t_dom]
        dom = max(rows_t, key=lambda r: r["ms"] * r["in_resnet_step"])
        roof = roofline(dom, lay[dom["op"].split(":")[0]]["flops"])
        t_ms = sum(r["ms"] * r["in_resnet_step"] for r in rows_t)
        t_fl = sum(lay[r["op"].split(":")[0]]["flops"] * r["in_resnet_step"] for r in rows_t)
        roof["share_of_resnet_step"] = round(t_ms / rn["ms"], 4)
        roof["template_launches_per_step"] = sum(r["in_resnet_step"] for r in rows_t)
        roof["template_ops"] = [r["op"] for r in rows_t]
        roof["template_frac"] = round(t_fl / (t_ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4)
        if template_base(t_dom) != t_dom:
            roof["step_template_note"] = (
                "the step runs this kernel with the batch statistics taken in its store pass "
                "(last template argument 1); the sweep op above runs it without them")
    roof["candidates"] = candidates
    roof["share_note"] = ("launch time of every launch of the template per step / step time "
                          "(live timings of each kernel alone)")
    sdom = max(step_kernels, key=lambda r: r["ms"])
    sweep_roof = roofline(sdom, lay[sdom["op"].split(":")[0]]["flops"])
    ones = bench_1x1_rotated(R, ctx, layers, run_op, args.op_reps)

    attention = bench_attention(R, ctx, args.op_reps)
    gemms = bench_gemm(R, ctx, args.op_reps)
    vit_optim = bench_rustvit_optim(R, ctx, 5, 0 if args.no_cpu else args.cpu_budget / 4)
    vit_step = bench_rustvit_step(R, ctx, 5, 2)

    cpu = sweep_cpu = proto = None
    if not args.no_cpu:
        proto = cpu_protocol()
        a1, a0 = proto["all_cores"], proto["one_thread"]
        cpu = {"value": a1["config3_step"], "unit": "images/s", "cores": a1["threads"],
               "kind": "port",
               "sample": "config-3 ResNet-20 W32 train step (fwd + softmax-CE + bwd + SGD) at "
                         "batch 128 on the same inputs, one step per sample after a warm-up "
                         f"step, best of 3 with cooldown; {proto['label']}, OpenMP "
                         f"{a1['threads']} threads",
               "one_thread_value": a0["config3_step"],
               "host": proto["host"]}
        sweep_cpu = {"value": round(a1["config1_sweep"] / 1e3, 4), "unit": "TFLOP/s",
                     "cores": a1["threads"], "kind": "port",
                     "sample": "config-1 sweep (7 conv shapes x fwd/dX/dW) at batch 128, best of "
                               f"3; {proto['label']}",
                     "one_thread_value": round(a0["config1_sweep"] / 1e3, 4)}

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
        "roofline_dw_group": (group_roofline() if rn.get("dw_group") and
                              t_dom != DW_GROUP_TEMPLATE else None),
        "vs_cpu_baseline": round(rn["images_s"] / cpu["value"], 1) if cpu else None,
        "config1_conv_sweep": {
            "value": round(sweep_tf, 3), "unit": "TFLOP/s", "ms_per_step": round(sweep_ms, 4),
            "frac_of_fp32_mfma_peak": round(sweep_tf / PEAK_FP32_MFMA_TFLOPS, 4),
            "step": "per layer: pack W (forward + dX forms), forward, dX, dW",
            "tflops_without_packs": round(sweep_flops / (sweep_ms_nopack * 1e-3) / 1e12, 3),
            "tflops_unpacked_weights": round(sweep_flops / (sweep_ms_unpacked * 1e-3) / 1e12,
                                             3),
            "flop_per_step": sweep_flops, "roofline": sweep_roof, "cpu_baseline": sweep_cpu,
            "per_op": per_op, "ops_1x1_s2_hbm": ones},
        "config2_attention": attention, "gemmbench": gemms, "rustvit_optimizer": vit_optim,
        "config4_rustvit_step": vit_step, "cpu_reference_path": proto,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
