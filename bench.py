"""Benchmark: ResNet-18-shape 3x3 conv stack, batch 32, fp32,
through the libnhip C ABI on one MI355X, plus the int8 requantized conv
(config 4) as a secondary figure.

Secondary figures in the same line: the int8 conv (config 4) and the
MobileNetV2-shape graph at batch 32 (config 5).

One step = the four ResNet-18 basic-block stages (64@56, 128@28, 256@14,
512@7), each two 3x3 s1 p1 convs with folded-BN bias, ReLU and the residual
add: 8 Winograd F(4,3) convolutions over 32 images whose inputs are already
resident in HBM.

value = direct-equivalent conv TFLOP/s (2*N*K*OH*OW*C*9 per conv, the same
count for Winograd as for direct convolution).  roofline = the dominant
kernel, the Winograd GEMM with the output transform fused (wino_fused: 36
fp32 MFMA GEMMs and the output transform per conv; it runs the three stages
with at least 256 tiles, the 512@7 stage takes the three-kernel path): its
work 2*36*T*C*K per launch (T = N*ceil(OH/4)*ceil(OW/4) tiles) over its
duration, from HIP events stamped by each of its dispatches on the launch
stream over a second run of the same K steps (the events cost ~5% of a
step, so the timed region that gives value runs without them); traffic = its HBM bytes per launch from the
committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
(profiles/wino_fused_traffic.json).  cpu_baseline = the
CPU oracle (restatement of the reference's lowered loops, compiled like the
reference's .so: -O3, no -march, no FP contraction, OpenMP) on a bounded
sample of the same stages.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "ncnn-compiler_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "conv TFLOP/s (% MFMA peak) + images/sec, ResNet-18-shape b32 fp32/int8"
PEAK_FP32_TFLOPS = 157.3
PEAK_INT8_TOPS = 5000.0
BATCH = 32


def stage_stack(nhip, workloads, torch, batch):
    stages = []
    for c, hw in workloads.RESNET18_STAGES:
        x, w1, b1, w2, b2 = workloads.resnet_stage(c, hw, n=batch, seed=0)
        d = nhip.conv_desc(c, c, act=nhip.ACT_RELU, algorithm=nhip.ALGO_WINOGRAD)
        c1, c2 = nhip.Conv2dF32(d, w1, b1), nhip.Conv2dF32(d, w2, b2)
        ws = max(c1.workspace_size(batch, hw, hw), c2.workspace_size(batch, hw, hw))
        stages.append(dict(
            c=c, hw=hw, conv1=c1, conv2=c2,
            x=torch.from_numpy(x).cuda(),
            y=torch.empty((batch, c, hw, hw), device="cuda"),
            out=torch.empty((batch, c, hw, hw), device="cuda"),
            ws=torch.empty(ws, dtype=torch.uint8, device="cuda")))
    return stages


def run_step(stages):
    for s in stages:
        s["conv1"].forward(s["x"], out=s["y"], workspace=s["ws"])
        s["conv2"].forward(s["y"], residual=s["x"], out=s["out"], workspace=s["ws"])


def cpu_baseline(workloads, target_s=12.0):
    """Oracle on a bounded sample: one image per stage through both convs,
    the relu and the residual add, repeated until about target_s elapsed."""
    from oracle import refcpu
    threads = min(16, os.cpu_count() or 1)
    samples = []
    for c, hw in workloads.RESNET18_STAGES:
        x, w1, b1, w2, b2 = workloads.resnet_stage(c, hw, n=1, seed=0)
        samples.append((c, hw, x, w1, b1, w2, b2))
    flops = 0.0
    t0 = time.perf_counter()
    rounds = 0
    while True:
        for c, hw, x, w1, b1, w2, b2 in samples:
            g = refcpu.geom(1, c, hw, hw, c)
            y = refcpu.relu_f32(refcpu.conv2d_f32(g, x, w1, b1, threads=threads))
            refcpu.relu_f32(refcpu.add_f32(refcpu.conv2d_f32(g, y, w2, b2, threads=threads), x))
            flops += 2 * workloads.conv_flops(1, c, c, hw, hw)
        rounds += 1
        if time.perf_counter() - t0 >= target_s:
            break
    dt = time.perf_counter() - t0
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"{rounds} x (1 image through each of the 4 stages: 8 convs + relu + add), "
                      f"{dt:.1f} s, OpenMP {threads} threads; {rounds / dt:.3f} images/s through the stack"}


def int8_secondary(nhip, workloads, torch, steps, warmup):
    cfg = workloads.int8_conv(seed=0, n=BATCH)
    d = nhip.conv_desc(128, 128, act=nhip.ACT_RELU, int8_scale_term=101)
    conv = nhip.Conv2dInt8(d, cfg["w"], cfg["bias"], cfg["ws"], cfg["input_scale"], cfg["output_scale"])
    x = torch.from_numpy(cfg["x"]).cuda()
    out = torch.empty((BATCH, 128, 28, 28), dtype=torch.int8, device="cuda")
    ws = torch.empty(conv.workspace_size(BATCH, 28, 28), dtype=torch.uint8, device="cuda")
    for _ in range(warmup):
        conv.forward(x, out=out, workspace=ws)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        conv.forward(x, out=out, workspace=ws)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    nhip.timer_start("conv_int8")  # the GEMM kernel's duration, in a second instrumented pass
    for _ in range(steps):
        conv.forward(x, out=out, workspace=ws)
    torch.cuda.synchronize()
    launches, kms = nhip.timer_stop()
    ops = workloads.conv_flops(BATCH, 128, 128, 28, 28)
    kavg = kms / max(launches, 1) / 1e3
    return {"workload": "int8 conv 32x128x28x28 3x3 requant(term 101)+relu, fp32 input",
            "ms_per_step": dt * 1e3, "tops": ops / dt / 1e12,
            "images_per_sec": BATCH / dt,
            "gemm_kernel_tops": ops / kavg / 1e12,
            "gemm_kernel_frac_int8_peak": ops / kavg / 1e12 / PEAK_INT8_TOPS}


def mobilenetv2_secondary(nhip, torch, steps, warmup):
    """The graph runs through the native executor (`nhip_graph_run`) from
    its .param/.bin form, as a compiled model would (on torch's default
    stream, so every kernel is launched eagerly: replay of a recorded
    hipGraph applies to calls on other streams and measured the same GPU
    time)."""
    import graphs
    import ncnn_format
    layers = graphs.mobilenetv2_layers(seed=0)
    m = ncnn_format.from_layer_list(layers)
    g = nhip.Graph(m.param_text(), bytes(m.payload))
    x = torch.from_numpy(
        __import__("numpy").random.default_rng(0).uniform(-1, 1, (BATCH, 3, 224, 224)).astype("float32")).cuda()
    out = g.run(x)  # outputs reused by every step
    for _ in range(warmup):
        g.run(x, out=out)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        g.run(x, out=out)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    flops = graphs.graph_flops(layers, BATCH, 224, 224)
    return {"workload": "MobileNetV2-shape graph b32 224x224 fp32 (53 conv/dw layers, GAP, IP 1280->1000), native graph executor",
            "ms_per_step": dt * 1e3, "images_per_sec": BATCH / dt, "tflops": flops / dt / 1e12}


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel`, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (profiles/<kernel>_traffic.json, averaged
    over the stage shapes it runs, copy-calibrated); None if absent."""
    try:
        with open(os.path.join(ROOT, "profiles", f"{kernel}_traffic.json")) as f:
            d = json.load(f)
        return int(d["bytes_per_launch"]) if d.get("kernel") == kernel else None
    except (OSError, ValueError, KeyError):
        return None


def fused_stage(c, hw):
    """The library's default Winograd path choice: the fused GEMM from 256
    tiles up (winograd.hip, direct_selected / fused_selected)."""
    t = -(-hw // 4)
    return BATCH * t * t >= 256


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="first run a plain device copy of this many MiB (hipMemcpy D2D) so that "
                         "rocprofv3 FETCH_SIZE/WRITE_SIZE can be scaled against known bytes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(images would shard across GPUs as independent data-parallel work).", file=sys.stderr)
        sys.exit(2)

    import torch

    import nhip
    import workloads

    torch.cuda.set_device(0)
    nhip.init(0)
    if args.copy_calibration_mib:
        nbytes = args.copy_calibration_mib << 20
        src = torch.ones(nbytes // 4, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            nhip.check(nhip.load().nhip_memcpy_d2d(nhip._ptr(dst), nhip._ptr(src), nbytes, nhip._stream()))
        torch.cuda.synchronize()
        del src, dst
    stages = stage_stack(nhip, workloads, torch, BATCH)
    for _ in range(args.warmup):
        run_step(stages)
    torch.cuda.synchronize()

    variant = os.environ.get("NHIP_WINOGRAD_VARIANT", "")
    fused_convs = [(c, hw) for c, hw in workloads.RESNET18_STAGES
                   if variant == "2" or (variant != "1" and fused_stage(c, hw))]
    kernel = "wino_fused" if fused_convs else "wino_gemm"
    kernel_convs = fused_convs or list(workloads.RESNET18_STAGES)
    # The timed region: exactly K steps, no per-launch instrumentation.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run_step(stages)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    # The same K steps again with HIP events on every launch of the roofline
    # kernel (stamped by its dispatches on the launch stream): its average
    # duration.  The events cost ~5% of a step, so the throughput above is
    # taken without them.
    nhip.timer_start(kernel)
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    for _ in range(args.steps):
        run_step(stages)
    torch.cuda.synchronize()
    t3 = time.perf_counter()
    launches, kernel_ms = nhip.timer_stop()

    ms_per_step = (t1 - t0) * 1e3 / args.steps
    ms_per_step_instrumented = (t3 - t2) * 1e3 / args.steps
    direct_flops = sum(2 * workloads.conv_flops(BATCH, c, c, hw, hw) for c, hw in workloads.RESNET18_STAGES)
    wino_flops = sum(2 * workloads.winograd_flops(BATCH, c, c, hw, hw) for c, hw in workloads.RESNET18_STAGES)
    kernel_flops = sum(2 * workloads.winograd_flops(BATCH, c, c, hw, hw) for c, hw in kernel_convs)
    value = direct_flops / (ms_per_step / 1e3) / 1e12
    # two convs per stage; each runs as one or two batch parts (one kernel launch each)
    per_step = launches // args.steps
    assert launches % args.steps == 0 and per_step in (2 * len(kernel_convs), 4 * len(kernel_convs)), \
        (launches, args.steps, kernel_convs)
    kernel_s_per_step = kernel_ms / args.steps / 1e3
    achieved = kernel_flops / kernel_s_per_step / 1e12
    int8 = int8_secondary(nhip, workloads, torch, args.steps, args.warmup)
    mbv2 = mobilenetv2_secondary(nhip, torch, args.steps, args.warmup)
    result = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (uniform[-1,1] inputs, He-normal weights, seeded)",
        "config": {
            "workload": "resnet18_stage_stack_b32_fp32 (4 stages x 2 Winograd F(4,3) 3x3 s1 p1 convs, "
                        "bias+relu, residual add+relu)",
            "batch": BATCH,
            "images_per_sec": round(BATCH / (ms_per_step / 1e3), 1),
            "frac_fp32_mfma_peak_direct_equivalent": round(value / PEAK_FP32_TFLOPS, 4),
            "winograd_executed_tflops": round(wino_flops / (ms_per_step / 1e3) / 1e12, 3),
            "int8": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in int8.items()},
            "mobilenetv2": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in mbv2.items()},
        },
        "roofline": {
            "bound": "mfma",
            "kernel": ("wino_fused (36 batched fp32 MFMA GEMMs + output transform per conv; stages "
                       + ", ".join(f"{c}@{hw}" for c, hw in kernel_convs) + ")") if kernel == "wino_fused"
                      else "wino_gemm (36 batched fp32 MFMA GEMMs per conv)",
            "achieved": round(achieved, 3),
            "peak": PEAK_FP32_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_FP32_TFLOPS, 4),
            "traffic": measured_traffic(kernel),
            "avg_launch_us": round(kernel_s_per_step / per_step * 1e6, 2),
            "launches_timed": launches,
            "ms_per_step_instrumented": round(ms_per_step_instrumented, 4),
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(workloads)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
