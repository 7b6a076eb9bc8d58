"""Benchmark of the MI355X TOSA execution path.

Headline workload (one "step" = one run of the graph through the C ABI on
device-resident input): int8 CONV2D [64,28,28,128] x [128,3,3,128] (stride 1,
pad 1) + per-channel DOUBLE_ROUND RESCALE to int8, with the distributions and
zero points of the reference's int8 CONV2D+RESCALE configuration (x U[-128,127]
zx=-3, w U zw=0, bias U[-2^15,2^15], multiplier U[2^30,2^31), shift U[30,40],
output zp 5) at ResNet conv3_x scale, where int8 MFMA (not HBM) bounds it.

The JSON line reports whole-job throughput (TOPS), the fused conv kernel's
roofline (MFMA-bound; average duration from HIP events on the library's
stream) and the CPU oracle timed on the host beside it (the calling thread
pinned to one CPU for the CPU legs; the host's CPU count and model recorded);
`extra` carries the other benchmark configurations, incl. the int8
MobileNetV2-style graph img/s with its own CPU leg (the oracle's graph runner
on a batch of 4, whose logits the GPU must match bit for bit).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
    python bench.py --only NAME [--copy-mib M]   # one workload, for profilers

`--only` runs one workload of WORKLOADS (timing only, no CPU baseline) and
`--copy-mib` appends device-to-device copies of M MiB (torch's copy kernel),
whose FETCH_SIZE / WRITE_SIZE readings calibrate the HBM traffic counters.
The conv kernel's HBM traffic per launch comes from those counter runs and is
read from the `TRAFFIC` line of the committed profile summary.
"""

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_INT8_TOPS = 5000.0     # MI355X dense int8 MFMA, 5.0 POP/s
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16/fp16 MFMA, 2.5 PFLOP/s
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E, 8 TB/s
METRIC = "int8 CONV2D+RESCALE TOPS (% MFMA peak); int8 MobileNetV2-style graph img/s"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=500)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--quick", action="store_true", help="headline workload only")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="bound of the CPU baseline sample")
    p.add_argument("--only", default=None, help="run one workload (a WORKLOADS key) and print its timing")
    p.add_argument("--copy-mib", type=int, default=0, help="with --only: also run device copies of this size")
    p.add_argument("--option", action="append", default=[], metavar="KEY=VALUE",
                   help="with --only: set a library option first (tosa_set_option, e.g. deferred=0)")
    return p.parse_args()


HEADLINE = "conv_rescale_64x28x28x128"
HEADLINE_KERNEL = "conv_i8_rows_kernel"
# name -> (builder name in tosa_amd.workloads, kwargs, count ops, steps override)
WORKLOADS = {
    HEADLINE: ("conv_rescale", dict(n=64, h=28, w=28, cin=128, cout=128), True, None),
    "mobilenet_v2_int8_n64": ("mobilenet_v2", dict(n=64), True, None),
    "cfg1_conv_rescale_1x56x56x64": ("conv_rescale", {}, True, None),
    "conv_rescale_64x14x14x256": ("conv_rescale", dict(n=64, h=14, w=14, cin=256, cout=256), True, None),
    "cfg2_matmul_rescale_8x512x1024x1024": ("matmul_rescale", {}, True, None),
    "cfg3_depthwise_32x112x112x144_s2": ("depthwise", {}, True, None),
    "cfg3_avg_pool_32x7x7x1280": ("avg_pool", {}, False, None),
    "cfg5_bf16_conv3x3_64x28x28x128": ("float_conv", dict(dtype="BF16"), True, None),
    "cfg5_fp16_conv3x3_64x28x28x128": ("float_conv", dict(dtype="FP16"), True, None),
    "cfg5_bf16_conv1x1_64x28x28x128to512": ("float_conv", dict(dtype="BF16", cout=512, k=1), True, None),
    "cfg5_bf16_matmul_16x2048x2048x2048": ("float_matmul", {}, True, 5),
    "i16_conv_rescale_64x28x28x128": ("conv_i16", {}, True, None),
}


def traffic_from_profile(kernel):
    """HBM bytes per launch of `kernel` from the TRAFFIC line of the committed
    counter summary (FETCH_SIZE + WRITE_SIZE, calibrated against a copy)."""
    path = os.path.join(ROOT, "profiles", "conv_i8_rescale_64x28x28x128.md")
    try:
        with open(path) as f:
            for ln in f:
                parts = ln.split()
                if len(parts) == 3 and parts[0] == "TRAFFIC" and parts[1] == kernel:
                    return int(parts[2])
    except OSError:
        pass
    return None


class Runner:
    """An Interpreter with device-resident inputs, running pipelined
    (deferred) on torch's current stream."""

    def __init__(self, T, torch, graph, inputs):
        self.T, self.torch = T, torch
        self.interp = T.Interpreter.from_flatbuffer(graph)
        self.inputs = []
        self.keep = []
        for name, (arr, dt) in inputs.items():
            dev = torch.from_numpy(np.ascontiguousarray(arr).view(np.uint8).reshape(-1).copy()).cuda()
            self.keep.append(dev)
            self.inputs.append(T.Tensor.from_device(name, arr.shape, dt, dev.data_ptr(), arr.nbytes, keep=dev))
        torch.cuda.synchronize()

    def run(self):
        return self.interp.run(self.inputs)

    def sync(self):
        self.T.synchronize()
        self.torch.cuda.synchronize()

    def wall(self, steps, warmup):
        # The warm-up runs exactly as the timed ones do (each run's outputs
        # held until the next run replaces them), so the device pool already
        # holds the blocks the timed runs cycle through.
        out = None
        for _ in range(warmup):
            out = self.run()
        self.sync()
        t0 = time.perf_counter()
        for _ in range(steps):
            out = self.run()
        self.sync()
        t1 = time.perf_counter()
        del out
        return (t1 - t0) / steps

    def gpu_time(self, reps, sleep_cycles):
        """Average GPU time of one run with host overhead hidden: the runs are
        enqueued behind a spin kernel, so they execute back to back between
        the two events, all on the stream the library launches on."""
        torch = self.torch
        s = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(sleep_cycles)
        e0.record(s)
        outs = [self.run() for _ in range(reps)]
        e1.record(s)
        self.sync()
        del outs
        return e0.elapsed_time(e1) / 1e3 / reps


def calibrate_sleep(torch, seconds):
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    cycles = 1_000_000
    s = torch.cuda.current_stream()
    e0.record(s)
    torch.cuda._sleep(cycles)
    e1.record(s)
    torch.cuda.synchronize()
    per = max(e0.elapsed_time(e1) / 1e3, 1e-6) / cycles
    return int(min(seconds / per, 2 ** 31 - 1))


def host_facts():
    """The box's host CPU: logical CPUs, those this process may use, model."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"host_cpus": os.cpu_count(), "host_cpus_allowed": len(os.sched_getaffinity(0)), "host_cpu_model": model}


def pinned(fn):
    """Run `fn` with the calling thread pinned to one CPU (the highest one it
    may use), in-process; the previous mask is restored afterwards. Only this
    thread moves: the GPU runtime's own threads keep their CPUs."""
    before = os.sched_getaffinity(0)
    core = max(before)
    os.sched_setaffinity(0, {core})
    try:
        return fn(), core
    finally:
        os.sched_setaffinity(0, before)


def cpu_baseline(seconds):
    """The oracle (C restatement of the reference loops, 1 thread) on a
    bounded sample of the headline workload: whole images of the batch until
    `seconds` of CPU work; also checks the GPU's image-0 output bit for bit."""
    from oracle import oracle as O
    from tosa_amd import workloads as W
    _, ins, info = W.conv_rescale(n=1, h=28, w=28, cin=128, cout=128)  # image 0 of the batch
    x = ins["x"][0]
    params = _conv_params()
    done, t_total, out0 = 0, 0.0, None
    xs = W.i8(W.rng(1, 0), (64, 28, 28, 128))
    while t_total < seconds and done < 64:
        xi = xs[done:done + 1]
        t0 = time.perf_counter()
        y = _oracle_conv_rescale(O, xi, params)
        t_total += time.perf_counter() - t0
        if done == 0:
            out0 = y
        done += 1
    ops = done * info["ops"]
    del x
    return {"value": ops / t_total / 1e12, "unit": "TOPS", "cores": 1, "kind": "port",
            "sample": f"{done} of 64 images of the headline CONV2D+RESCALE ({done * info['macs']:.3g} MAC) "
                      f"through oracle/tosa_oracle.c (C restatement of the reference loops, 1 thread), "
                      f"{t_total:.1f} s"}, out0


def cpu_mobilenet(n=4):
    """The oracle's graph runner (C restatement of the reference's operators,
    1 thread) on the int8 MobileNetV2-style graph at batch `n`: img/s, which
    per image is the same figure as for the batch of 64, and the logits."""
    from oracle import oracle as O
    from oracle import tosa_reader as fb
    from tosa_amd import workloads as W
    g, ins, _ = W.mobilenet_v2(n=n)
    blk = fb.main_block(g)
    feeds = {k: O.T(dt, list(a.shape), O.decode(dt, a)) for k, (a, dt) in ins.items()}
    t0 = time.perf_counter()
    out = O.run_block(blk, feeds)
    t = time.perf_counter() - t0
    logits = out[blk.outputs[0]].vals
    return {"img_s": n / t, "cores": 1, "kind": "port",
            "sample": f"batch {n} of the same graph through the oracle's graph runner (oracle/oracle.py over "
                      f"oracle/tosa_oracle.c, 1 thread), {t:.1f} s; img/s scales to the batch of 64 as is "
                      f"(images are independent)"}, g, ins, logits


def _conv_params():
    from tosa_amd import workloads as W
    cout, k, cin = 128, 3, 128
    return {"w": W.i8(W.rng(1, 1), (cout, k, k, cin)),
            "bias": W.rng(1, 2).integers(-2 ** 15, 2 ** 15 + 1, size=cout).astype(np.int32),
            "mult": W.rng(1, 3).integers(2 ** 30, 2 ** 31, size=cout).astype(np.int64),
            "shift": W.rng(1, 4).integers(30, 41, size=cout).astype(np.int8)}


def _oracle_conv_rescale(O, x, p):
    acc = O.conv2d(O.T("INT8", x.shape, x), O.T("INT8", p["w"].shape, p["w"]), O.T("INT32", p["bias"].shape, p["bias"]),
                   -3, 0, [1, 1, 1, 1], [1, 1], [1, 1], "INT32", "INT32")
    y = O.rescale(acc, O.T("INT32", [128], p["mult"]), O.T("INT8", [128], p["shift"]), 0, 5, "INT8", True, 3, True,
                  False, False)
    return y.vals.astype(np.int8).reshape(acc.shape)


def run_only(args, torch, T, W, sleep):
    """One workload, `--steps` timed runs after `--warmup`, then optionally
    `--copy-mib` device copies: the command profilers wrap."""
    if args.only not in WORKLOADS:
        print(f"unknown workload {args.only!r}; choose one of {', '.join(WORKLOADS)}", file=sys.stderr)
        sys.exit(2)
    for kv in args.option:
        key, _, val = kv.partition("=")
        T.set_option(key, int(val))
    builder, kw, unit_ops, _ = WORKLOADS[args.only]
    g, i, inf = getattr(W, builder)(**kw)
    r = Runner(T, torch, g, i)
    sec = r.wall(args.steps, args.warmup)
    # At most 50 runs queued behind the spin kernel: each holds its outputs
    # until the events are read, and more would grow the device pool mid-way.
    k = r.gpu_time(max(1, min(args.steps, 50)), sleep)
    line = {"workload": args.only, "options": args.option, "ms_per_step": sec * 1e3, "gpu_ms": k * 1e3,
            "GB_s": inf["bytes"] / k / 1e9}
    if unit_ops:
        line["TOPS"] = inf["ops"] / k / 1e12
    if args.copy_mib:
        n = args.copy_mib << 20
        src = torch.randint(0, 255, (n,), dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(max(1, args.steps)):
            dst.copy_(src)
        torch.cuda.synchronize()
        line["copy_bytes_per_launch"] = {"read": n, "write": n}
    print(json.dumps(line))


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this path shards by batch with "
              f"no exchange step, see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    import torch
    import tosa_amd as T
    from tosa_amd import workloads as W

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    torch.cuda.init()
    # A stream of our own (default priority): the library launches on it and
    # the timing events are recorded on it. (torch's default stream is the
    # NULL stream, which set_stream would read as "library-owned stream".)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    T.set_stream(stream.cuda_stream)
    T.set_option("deferred", 1)
    sleep = calibrate_sleep(torch, 0.02)

    if args.only is not None:
        run_only(args, torch, T, W, sleep)
        return

    # ---- headline: int8 CONV2D + RESCALE at ResNet conv3_x scale ----------
    graph, ins, info = W.conv_rescale(n=64, h=28, w=28, cin=128, cout=128)
    r = Runner(T, torch, graph, ins)
    sec = r.wall(args.steps, args.warmup)
    kern = r.gpu_time(20, sleep)
    value = info["ops"] / sec / 1e12
    achieved = info["ops"] / kern / 1e12
    out_img0 = r.run()["y"].numpy()[0]
    r.sync()

    # CPU legs after every GPU figure of the headline, on one pinned core.
    (cpu, cpu_img0), core = pinned(lambda: cpu_baseline(args.cpu_seconds))
    cpu.update(host_facts())
    cpu["pinned_cpu"] = core
    extra = {"headline_image0_bit_exact_vs_oracle": bool(np.array_equal(out_img0, cpu_img0[0])),
             "headline_kernel_us": kern * 1e6}

    def measure(name):
        builder, kw, unit_ops, steps = WORKLOADS[name]
        g, i, inf = getattr(W, builder)(**kw)
        rr = Runner(T, torch, g, i)
        s = rr.wall(steps or max(5, args.steps // 5), 2)
        k = rr.gpu_time(5, sleep)
        e = {"ms_per_step": s * 1e3, "gpu_ms": k * 1e3}
        if unit_ops:
            e["TOPS"] = inf["ops"] / k / 1e12
        e["GB_s"] = inf["bytes"] / k / 1e9
        extra[name] = e
        return inf, s, k

    if not args.quick:
        inf, s, k = measure("mobilenet_v2_int8_n64")
        extra["mobilenet_v2_int8_n64"].update({"img_s": 64 / s, "img_s_gpu": 64 / k,
                                               "hbm_roofline_frac": inf["bytes"] / k / 1e9 / PEAK_HBM_GBS})
        (mcpu, mg, mins, mlogits), core = pinned(cpu_mobilenet)
        # The same batch-4 graph on the GPU, logits compared bit for bit.
        got = Runner(T, torch, mg, mins).run()
        name = next(iter(got))
        mcpu["gpu_logits_bit_exact"] = bool(np.array_equal(got[name].numpy().reshape(-1).astype(np.int64),
                                                           np.asarray(mlogits).reshape(-1).astype(np.int64)))
        mcpu["pinned_cpu"] = core
        extra["mobilenet_v2_int8_n64"]["cpu_baseline"] = mcpu
        for name in WORKLOADS:
            if name not in (HEADLINE, "mobilenet_v2_int8_n64"):
                measure(name)

    line = {
        "metric": METRIC,
        "value": value,
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": sec * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "int8 CONV2D [64,28,28,128]x[128,3,3,128] s1 p1 + per-channel DOUBLE_ROUND "
                               "RESCALE->int8 (zx=-3, zw=0, output zp 5)",
                   "global_batch": 64, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_INT8_TOPS, "unit": "TOPS",
                     "frac": achieved / PEAK_INT8_TOPS, "traffic": traffic_from_profile(HEADLINE_KERNEL)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
