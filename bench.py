"""Benchmark: the ResNet-18-shape 3x3 conv stack, batch 32, fp32 (config 3,
the third entry of BASELINE.json's `configs`) is the headline `value`;
configs 1, 2, 4 and 5 (the other entries, in order) are measured in the
same run and reported under `config`, each with the roofline of its dominant
kernel and a CPU baseline.

One step (config 3) = the four ResNet-18 basic-block stages (64@56, 128@28,
256@14, 512@7), each two 3x3 s1 p1 convs with folded-BN bias, ReLU and the
residual add: 8 Winograd F(4,3) convolutions over 32 images whose inputs are
already resident in HBM.  value = direct-equivalent conv TFLOP/s
(2*N*K*OH*OW*C*9 per conv, the same count for Winograd as for direct
convolution).

Every timed region runs exactly K steps between synchronizations with no
per-launch instrumentation; kernel durations come from a second run of the
same K steps with HIP events that each kernel's own dispatch stamps on its
launch stream (nhip_timer_*).

Secondary figures:
- config 1: one 64->64 3x3 conv on 1x64x56x56 through the layer ABI
  (device buffers), and the same model through the library ncnn-compile
  writes, called on host buffers (the reference's entry: H2D, kernels, D2H);
- config 2: InnerProduct 256x2048 -> 1000 (device buffers);
- config 4: int8 conv 32x128x28x28 -> 128, requantize (term 101) + ReLU,
  fp32 input (quantize pass + int8 MFMA GEMM);
- config 5: the MobileNetV2-shape graph at batch 32 through the native
  executor from its .param/.bin form, and the compiled library on one image
  from host buffers.

roofline: the dominant kernel's algorithmic work per launch over its average
duration.  For config 3 that is the Winograd GEMM with the output transform
fused (wino_fused: executed FLOPs 2*36*T*C*K per launch, T tiles); traffic =
its HBM bytes per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
summary (profiles/wino_fused_traffic.json, copy-calibrated), null when that
summary was taken on another version of the kernel's source.  For config 5
it is the streaming 1x1 kernel (pw_conv_f32) inside the graph, HBM-bound.

cpu_baseline: the CPU oracle (a restatement of the reference's lowered loop
nests, compiled like the reference's .so: -O3, no -march, no FP contraction,
OpenMP over the outer loops) on bounded samples, one image per call as the
reference's entry runs, with all threads of this job's CPU share and with one
thread.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""
import argparse
import ctypes
import json
import os
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "ncnn-compiler_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "conv TFLOP/s (% MFMA peak) + images/sec, ResNet-18-shape b32 fp32/int8"
PEAK_FP32_TFLOPS = 157.3
PEAK_INT8_TOPS = 5000.0
PEAK_HBM_GBS = 8000.0
BATCH = 32
TOOL = os.path.join(ROOT, "ncnn-compiler_amd", "bin", "ncnn-compile")


# ----------------------------------------------------------------- helpers
def timed(torch, fn, steps):
    """Wall time per call of `fn` over exactly `steps` calls, synchronized on
    both sides (seconds)."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def kernel_time(nhip, torch, fn, steps, name, required=True):
    """(launches per call, seconds per launch) of the kernels whose name
    contains `name`, from HIP events on their own dispatches; (0, 0.0) when
    none ran and `required` is false."""
    torch.cuda.synchronize()
    nhip.timer_start(name)
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    launches, ms = nhip.timer_stop()
    if launches == 0:
        if not required:
            return 0, 0.0
        raise RuntimeError(f"no kernel launch named like {name!r} was timed")
    return launches / steps, ms / 1e3 / launches


def dominant(nhip, torch, fn, steps, names):
    """The kernel of `names` with the largest time per call:
    (name, launches per call, seconds per launch)."""
    best = None
    for nm in names:
        per, sec = kernel_time(nhip, torch, fn, steps, nm, required=False)
        if per and (best is None or per * sec > best[1] * best[2]):
            best = (nm, per, sec)
    return best


def roofline(bound, kernel, work_per_launch, sec_per_launch, launches_per_step, traffic=None):
    peak, unit = {"mfma": (PEAK_FP32_TFLOPS, "TFLOP/s"), "mfma_int8": (PEAK_INT8_TOPS, "TOP/s"),
                  "hbm": (PEAK_HBM_GBS, "GB/s")}[bound]
    achieved = work_per_launch / sec_per_launch / (1e9 if bound == "hbm" else 1e12)
    return {"bound": "mfma" if bound.startswith("mfma") else "hbm", "kernel": kernel, "achieved": round(achieved, 3),
            "peak": peak, "unit": unit, "frac": round(achieved / peak, 4), "traffic": traffic,
            "avg_launch_us": round(sec_per_launch * 1e6, 2), "launches_per_step": round(launches_per_step, 2)}


def rounded(d):
    if isinstance(d, dict):
        return {k: rounded(v) for k, v in d.items()}
    return round(d, 4) if isinstance(d, float) else d


def cpu_info():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
    return model, os.cpu_count() or 1, share


def cpu_rate(fn, work, target_s):
    """Repeat fn until about target_s elapsed: (work units per second,
    calls made, seconds)."""
    fn()  # warm
    t0 = time.perf_counter()
    calls = 0
    while True:
        fn()
        calls += 1
        dt = time.perf_counter() - t0
        if dt >= target_s:
            return work * calls / dt, calls, dt


def cpu_pair(fn_threads, work, unit, what, target_s, share):
    """The same sample with all threads of the job's share and with one."""
    out = {}
    for label, threads in (("all", share), ("one", 1)):
        rate, calls, dt = cpu_rate(lambda: fn_threads(threads), work, target_s)
        out[label] = {"value": rate, "unit": unit, "threads": threads,
                      "sample": f"{calls} x {what} in {dt:.1f} s"}
    return out


def compile_model(model, name, workdir, extra=()):
    """The model through ncnn-compile -> ctypes handle of lib<name>.so, or
    None when the tool has not been built."""
    if not os.path.exists(TOOL):
        return None
    p, b = os.path.join(workdir, f"{name}.param"), os.path.join(workdir, f"{name}.bin")
    model.save(p, b)
    r = subprocess.run([TOOL, p, "-o", os.path.join(workdir, name), *extra], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(r.stderr)
    return ctypes.CDLL(os.path.join(workdir, name, f"lib{name}.so"))


def host_entry_latency(entry, args, calls):
    """Seconds per call of a generated entry on host buffers (synchronous:
    H2D, kernels, D2H), after warm calls."""
    for _ in range(5):
        assert entry(*args) == 0
    t0 = time.perf_counter()
    for _ in range(calls):
        entry(*args)
    return (time.perf_counter() - t0) / calls


# ------------------------------------------------------------ config 3
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


def fused_stage(c, hw):
    """The library's default Winograd path choice: the fused GEMM from 128
    tiles up (winograd.hip, fused_selected)."""
    t = -(-hw // 4)
    return BATCH * t * t >= 128


KERNEL_SOURCES = {"wino_fused": "ncnn-compiler_amd/csrc/winograd_fused.hip"}


def source_sha256(kernel):
    import hashlib
    with open(os.path.join(ROOT, KERNEL_SOURCES[kernel]), "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel`, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (profiles/<kernel>_traffic.json, averaged
    over the stage shapes it runs, copy-calibrated); None if absent or if it
    was measured on another version of the kernel's source (the summary
    records the SHA-256 of the source file it was taken with)."""
    try:
        with open(os.path.join(ROOT, "profiles", f"{kernel}_traffic.json")) as f:
            d = json.load(f)
        if d.get("kernel") != kernel or d.get("source_sha256") != source_sha256(kernel):
            return None
        return int(d["bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def cpu_config3(workloads, share, target_s):
    from oracle import refcpu
    samples = []
    for c, hw in workloads.RESNET18_STAGES:
        x, w1, b1, w2, b2 = workloads.resnet_stage(c, hw, n=1, seed=0)
        samples.append((c, hw, x, w1, b1, w2, b2))

    def one_image(threads):
        for c, hw, x, w1, b1, w2, b2 in samples:
            g = refcpu.geom(1, c, hw, hw, c)
            y = refcpu.relu_f32(refcpu.conv2d_f32(g, x, w1, b1, threads=threads))
            refcpu.relu_f32(refcpu.add_f32(refcpu.conv2d_f32(g, y, w2, b2, threads=threads), x))

    flops = sum(2 * workloads.conv_flops(1, c, c, hw, hw) for c, hw in workloads.RESNET18_STAGES)
    return cpu_pair(one_image, flops / 1e12, "TFLOP/s", "(1 image through the 4 stages: 8 convs + relu + add)",
                    target_s, share)


# ------------------------------------------------------------ config 1
def config1(nhip, workloads, torch, steps, warmup, workdir, share, cpu, target_s):
    import ncnn_format
    x, w, b = workloads.conv_single(seed=0)
    d = nhip.conv_desc(64, 64, act=nhip.ACT_RELU)
    conv = nhip.Conv2dF32(d, w, b)
    xd = torch.from_numpy(x).cuda()
    out = torch.empty((1, 64, 56, 56), device="cuda")
    ws = torch.empty(max(conv.workspace_size(1, 56, 56), 256), dtype=torch.uint8, device="cuda")

    def fn():
        conv.forward(xd, out=out, workspace=ws)

    for _ in range(warmup):
        fn()
    n = max(steps * 10, 100)
    dt = timed(torch, fn, n)
    flops = workloads.conv_flops(1, 64, 64, 56, 56)
    # the library's choice for one image (the plan is Winograd, as the
    # automatic choice makes it): the one-kernel implicit GEMM with the
    # reduction split over each workgroup's waves (196 blocks of 32x32, at
    # most one per CU), else the Winograd kernels; the roofline is the
    # dominant kernel's, in the FLOPs it executes
    name, per, sec = dominant(nhip, torch, fn, n, ["conv_kq", "wino_gemm", "wino_fused"])
    kernels = {}
    for k in ("conv_kq", "wino_input_transform", "wino_gemm", "wino_output_transform", "wino_fused"):
        kp, ks = kernel_time(nhip, torch, fn, n, k, required=False)
        if kp:
            kernels[k] = round(kp * ks * 1e6, 2)
    if name == "conv_kq":
        rl = roofline("mfma", "conv_kq (implicit GEMM, 2*C*K*9*OH*OW)", flops / per, sec, per)
    else:
        wflops = workloads.winograd_flops(1, 64, 64, 56, 56)
        rl = roofline("mfma", f"{name} (executed 2*36*T*C*K, T=196 tiles)", wflops / per, sec, per)
    res = {"workload": "conv fp32 1x64x56x56 -> 64, 3x3 s1 p1, bias + ReLU (device buffers)",
           "ms_per_step": dt * 1e3, "tflops_direct_equivalent": flops / dt / 1e12, "images_per_sec": 1 / dt,
           "kernel_us_per_step": kernels, "roofline": rl}
    m = ncnn_format.Model()
    m.input("data", 64, 56, 56)
    m.conv("conv", "data", "output", w, b, act=1)
    lib = compile_model(m, "conv", workdir)
    if lib is not None:
        lib.conv.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        xh = x[0].copy()
        oh = __import__("numpy").empty((64, 56, 56), "float32")
        lat = host_entry_latency(lib.conv, (xh.ctypes.data, oh.ctypes.data), max(steps * 5, 50))
        res["dropin_entry"] = {"what": "generated int conv(const float*, float*) on host buffers, one image "
                                       "(H2D + kernels + D2H, synchronous)",
                               "ms_per_call": lat * 1e3, "images_per_sec": 1 / lat}
    if cpu:
        from oracle import refcpu
        g = refcpu.geom(1, 64, 56, 56, 64)
        res["cpu_baseline"] = cpu_pair(
            lambda t: refcpu.relu_f32(refcpu.conv2d_f32(g, x, w, b, threads=t)), flops / 1e12, "TFLOP/s",
            "(1 image: conv + bias + relu)", target_s, share)
    return res


# ------------------------------------------------------------ config 2
def config2(nhip, workloads, torch, steps, warmup, share, cpu, target_s):
    x, w, b = workloads.innerproduct(seed=0)
    ip = nhip.InnerProductF32(w, b)
    xd = torch.from_numpy(x).cuda()
    out = torch.empty((256, 1000), device="cuda")
    ws = torch.empty(max(ip.workspace_size(256), 256), dtype=torch.uint8, device="cuda")

    def fn():
        ip.forward(xd, out=out, workspace=ws)

    for _ in range(warmup):
        fn()
    n = max(steps * 10, 100)
    dt = timed(torch, fn, n)
    flops = 2.0 * 256 * 1000 * 2048
    # the one-workgroup-per-32x32-block kernel (reduction over the 16 waves
    # of the workgroup, summed in LDS) when it takes the shape, else the tiled
    # GEMM with split-K partials and a reduce launch
    kq, _ = kernel_time(nhip, torch, fn, 2, "innerproduct_f32_kq", required=False)
    per, sec = kernel_time(nhip, torch, fn, n, "innerproduct_f32")
    what = ("innerproduct_f32_kq (one workgroup per 32x32 output block, the 2048-long reduction over its 16 waves)"
            if kq else "innerproduct_f32 (MFMA GEMM fed by direct-to-LDS loads, split-K partials)")
    res = {"workload": "InnerProduct fp32 256x2048 -> 1000 + bias (device buffers)",
           "ms_per_step": dt * 1e3, "tflops": flops / dt / 1e12,
           "roofline": roofline("mfma", what, flops / per, sec, per)}
    if cpu:
        from oracle import refcpu
        res["cpu_baseline"] = cpu_pair(lambda t: refcpu.innerproduct_f32(x, w, b, threads=t), flops / 1e12,
                                       "TFLOP/s", "(256x2048 @ 2048x1000 + bias)", target_s, share)
    return res


# ------------------------------------------------------------ config 4
def config4(nhip, workloads, torch, steps, warmup, share, cpu, target_s):
    cfg = workloads.int8_conv(seed=0, n=BATCH)
    d = nhip.conv_desc(128, 128, act=nhip.ACT_RELU, int8_scale_term=101)
    conv = nhip.Conv2dInt8(d, cfg["w"], cfg["bias"], cfg["ws"], cfg["input_scale"], cfg["output_scale"])
    x = torch.from_numpy(cfg["x"]).cuda()
    out = torch.empty((BATCH, 128, 28, 28), dtype=torch.int8, device="cuda")
    ws = torch.empty(max(conv.workspace_size(BATCH, 28, 28), 256), dtype=torch.uint8, device="cuda")

    def fn():
        conv.forward(x, out=out, workspace=ws)

    for _ in range(warmup):
        fn()
    n = max(steps * 5, 50)
    dt = timed(torch, fn, n)
    ops = workloads.conv_flops(BATCH, 128, 128, 28, 28)
    per, sec = kernel_time(nhip, torch, fn, n, "conv_int8")
    qper, qsec = kernel_time(nhip, torch, fn, n, "quantize", required=False)
    fq, _ = kernel_time(nhip, torch, fn, 2, "conv_int8_rw_fq", required=False)
    what = ("conv_int8_rw_fq (fp32 input quantized into the LDS window, int8 MFMA GEMM, weights in registers, "
            "exact requantize epilogue; one launch)" if fq else
            "conv_int8_rw (int8 MFMA GEMM, weights in registers, exact requantize epilogue)")
    res = {"workload": "int8 conv 32x128x28x28 3x3 requant(term 101)+relu, fp32 input",
           "ms_per_step": dt * 1e3, "tops": ops / dt / 1e12, "images_per_sec": BATCH / dt,
           "roofline": roofline("mfma_int8", what, ops / per, sec, per)}
    if qper:
        # quantize pass: reads the fp32 input once, writes the int8 NHWC image
        qbytes = BATCH * 128 * 28 * 28 * 5
        res["quantize_kernel"] = {"avg_launch_us": round(qsec * 1e6, 2),
                                  "gbs": round(qbytes / qsec / 1e9, 1),
                                  "frac_hbm": round(qbytes / qsec / 1e9 / PEAK_HBM_GBS, 4)}
    if cpu:
        from oracle import refcpu
        g = refcpu.geom(1, 128, 28, 28, 128)
        x1 = cfg["x"][:1]
        res["cpu_baseline"] = cpu_pair(
            lambda t: refcpu.conv2d_int8(g, x1, cfg["w"], cfg["bias"], cfg["ws"], 1.0, 1.0, 101, 1, threads=t),
            ops / BATCH / 1e12, "TOP/s", "(1 image: quantize, int8 conv, requantize, relu)", target_s, share)
    return res


# ------------------------------------------------------------ config 5
def pw_kernel_layers(nhip, torch, layers, batch, name="pw_conv_f32"):
    """The graph's 1x1 layers that run on the streaming 1x1 kernel, with the
    executor's fusion decisions: an expand 1x1 whose depthwise consumer the
    expand + depthwise kernel takes runs as expand_dw_f32 (that depthwise
    then runs with it, not fused into the 1x1 after it); a 1x1 whose
    depthwise producer runs fused into it is a dwpw_fused_f32 launch; every
    other 1x1 goes once through the layer ABI with the launch timer on
    `name`.  Returns (launches, algorithmic HBM bytes) per graph run for the
    streaming kernel and (launches, bytes) for the expand + depthwise
    kernel: each layer reads its input, weights and bias (and residual) once
    and writes its output once (the fused pair: its input and the
    depthwise's output)."""
    shapes = {"data": (3, 224, 224)}
    producer, consumers = {}, {}
    for L in layers:
        consumers.setdefault(L["src"], []).append(L)
    launches, nbytes = 0, 0.0
    ed_launches, ed_bytes = 0, 0.0
    with_expand = set()  # depthwise layers run with their expand
    for L in layers:
        if L["kind"] not in ("conv", "dw"):
            continue
        c, h, w = shapes[L["src"]]
        ker = L.get("kernel", 3)
        pad = L.get("pad", 1)
        oh, ow = (h + 2 * pad - ker) // L["stride"] + 1, (w + 2 * pad - ker) // L["stride"] + 1
        k = L["k"] if L["kind"] == "conv" else L["c"]
        shapes[L["dst"]] = (k, oh, ow)
        producer[L["dst"]] = L
        if L["kind"] != "conv" or ker != 1:
            continue
        pw = nhip.Conv2dF32(nhip.conv_desc(c, k, kernel=(1, 1), pad=(0, 0, 0, 0), act=L["act"],
                                           algorithm=nhip.ALGO_IMPLICIT_GEMM), L["w"], L["b"])
        cons = consumers.get(L["dst"], [])
        if not L.get("residual") and len(cons) == 1 and cons[0]["kind"] == "dw":
            D = cons[0]
            dw = nhip.DwConv2dF32(nhip.conv_desc(k, k, stride=(D["stride"],) * 2, act=D["act"], group=k),
                                  D["w"], D["b"])
            if nhip.conv1x1_dw_supported(pw, dw, batch, h, w):
                with_expand.add(D["dst"])
                dh, dwid = (h - 1) // D["stride"] + 1, (w - 1) // D["stride"] + 1
                ed_launches += 1
                ed_bytes += 4.0 * (batch * c * h * w + L["w"].size + L["b"].size + D["w"].size + D["b"].size
                                   + batch * k * dh * dwid)
                continue
        src = producer.get(L["src"])
        if (src is not None and src["kind"] == "dw" and src["dst"] not in with_expand
                and not L.get("residual") == src["dst"]):
            sc, sh, sw = shapes[src["src"]]
            dw = nhip.DwConv2dF32(nhip.conv_desc(sc, sc, stride=(src["stride"],) * 2, act=src["act"], group=sc),
                                  src["w"], src["b"])
            if nhip.dwconv_pw_supported(dw, pw, batch, sh, sw):
                continue
        x = torch.zeros((batch, c, h, w), device="cuda")
        res = torch.zeros((batch, k, oh, ow), device="cuda") if L.get("residual") else None
        nhip.timer_start(name)
        pw.forward(x, residual=res)
        torch.cuda.synchronize()
        n, _ = nhip.timer_stop()
        if n:
            launches += n
            nbytes += 4.0 * (batch * c * h * w + L["w"].size + L["b"].size + batch * k * oh * ow
                             * (2 if L.get("residual") else 1))
        del x, res
    return (launches, nbytes), (ed_launches, ed_bytes)


def config5(nhip, torch, steps, warmup, workdir, share, cpu, target_s):
    import numpy as np

    import graphs
    import ncnn_format
    layers = graphs.mobilenetv2_layers(seed=0)
    m = ncnn_format.from_layer_list(layers)
    g = nhip.Graph(m.param_text(), bytes(m.payload))
    x = torch.from_numpy(np.random.default_rng(0).uniform(-1, 1, (BATCH, 3, 224, 224)).astype(np.float32)).cuda()
    flops = graphs.graph_flops(layers, BATCH, 224, 224)
    gbytes = graphs.graph_bytes(layers, BATCH, 224, 224)
    res = {"workload": "MobileNetV2-shape graph b32 224x224 fp32 (53 conv/dw layers, GAP, IP 1280->1000), "
                       "native graph executor from the .param/.bin form"}
    # eager launches on torch's default (legacy) stream, and the steady-state
    # path on a side stream where repeated calls replay a recorded hipGraph
    for label, stream in (("eager", None), ("replay", torch.cuda.Stream())):
        out = g.run(x)
        ctx = torch.cuda.stream(stream) if stream is not None else None
        if ctx:
            ctx.__enter__()

        def fn():
            g.run(x, out=out, stream=stream)

        for _ in range(max(warmup, 3)):
            fn()
        dt = timed(torch, fn, steps)
        if ctx:
            ctx.__exit__(None, None, None)
        res[label] = {"ms_per_step": dt * 1e3, "images_per_sec": BATCH / dt, "tflops": flops / dt / 1e12}
    best = min(res["eager"]["ms_per_step"], res["replay"]["ms_per_step"]) / 1e3
    res["ms_per_step"] = best * 1e3
    res["images_per_sec"] = BATCH / best
    res["graph_bytes"] = {"what": "layer-by-layer algorithmic bytes of the whole graph over the best step time",
                          "bytes_per_step": int(gbytes), "achieved_gbs": round(gbytes / best / 1e9, 1),
                          "frac_hbm_peak": round(gbytes / best / 1e9 / PEAK_HBM_GBS, 4)}
    # dominant kernel: the streaming 1x1 kernel (expand / project layers),
    # timed inside the graph (eager: the timer's events need eager launches)
    (pw_launches, pw_bytes), (ed_launches, ed_bytes) = pw_kernel_layers(nhip, torch, layers, BATCH)
    per, sec = kernel_time(nhip, torch, lambda: g.run(x, out=out), steps, "pw_conv_f32")
    assert round(per) == pw_launches, (per, pw_launches)
    res["roofline"] = roofline("hbm", "pw_conv_f32 (streaming 1x1 convolution: the 1x1 layers fused with no "
                                      "depthwise; bytes = each layer's input, weights, output (+ residual) once)",
                               pw_bytes / per, sec, per)
    res["roofline"]["step_share"] = round(per * sec / best, 4)
    # the expand + depthwise kernel (the 28x28, 14x14 and 7x7 blocks), its
    # share of the step and its bytes against HBM (it is bound by MFMA and
    # per-workgroup latency rather than by HBM)
    if ed_launches:
        per_e, sec_e = kernel_time(nhip, torch, lambda: g.run(x, out=out), steps, "expand_dw_f32")
        assert round(per_e) == ed_launches, (per_e, ed_launches)
        res["roofline_expand_dw"] = roofline("hbm", "expand_dw_f32 (1x1 expand + 3x3 depthwise in one kernel; "
                                                    "bytes = the expand's input and weights, the depthwise "
                                                    "output, once)", ed_bytes / per_e, sec_e, per_e)
        res["roofline_expand_dw"]["step_share"] = round(per_e * sec_e / best, 4)
    lib = compile_model(m, "mbv2", workdir)
    if lib is not None:
        lib.mbv2.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        xh = x[0].cpu().numpy().copy()
        oh = np.empty(1000, np.float32)
        lat = host_entry_latency(lib.mbv2, (xh.ctypes.data, oh.ctypes.data), max(steps, 20))
        res["dropin_entry"] = {"what": "generated int mbv2(const float*, float*) on host buffers, one image "
                                       "(H2D + 57 kernels or their replay + D2H, synchronous)",
                               "ms_per_call": lat * 1e3, "images_per_sec": 1 / lat}
    if cpu:
        from oracle import refcpu
        x1 = x[:1].cpu().numpy()

        def one_image(threads):
            blobs = {"data": x1}
            for L in layers:
                src = blobs[L["src"]]
                n, c, h, w = src.shape if src.ndim == 4 else (src.shape[0], src.shape[1], 1, 1)
                if L["kind"] == "conv":
                    p = L["pad"]
                    gg = refcpu.geom(n, c, h, w, L["k"], (L["kernel"],) * 2, (L["stride"],) * 2, (1, 1), (p,) * 4)
                    y = refcpu.conv2d_f32(gg, src, L["w"], L["b"], threads=threads)
                    if L["residual"]:
                        y = refcpu.add_f32(y, blobs[L["residual"]])
                    if L["act"] == 1:
                        y = refcpu.relu_f32(y)
                elif L["kind"] == "dw":
                    gg = refcpu.geom(n, c, h, w, c, (3, 3), (L["stride"],) * 2, (1, 1), (1, 1, 1, 1))
                    y = refcpu.relu_f32(refcpu.dwconv2d_f32(gg, src, L["w"], L["b"], threads=threads))
                elif L["kind"] == "gap":
                    y = refcpu.global_avgpool_f32(src)
                else:
                    y = refcpu.innerproduct_f32(src.reshape(n, -1), L["w"], L["b"], threads=threads)
                blobs[L["dst"]] = y

        res["cpu_baseline"] = cpu_pair(one_image, 1.0, "images/s", "(1 image through the whole graph)",
                                       target_s, share)
    return res


def hbm_kernels(nhip, workloads, torch, steps, warmup):
    """Bandwidth-bound kernels on their own at batch-32 MobileNetV2 shapes
    (the graph fuses these layers, or runs them on small planes where launch
    costs dominate): algorithmic bytes (each input read once, each output
    written once) over the kernel's average launch time from HIP events."""
    import numpy as np
    rng = np.random.default_rng(0)
    rows = []

    def timed_kernel(what, fn, nbytes, name):
        for _ in range(warmup):
            fn()
        per, sec = kernel_time(nhip, torch, fn, steps, name)
        gbs = nbytes / sec / 1e9
        rows.append({"kernel": what, "mb": round(nbytes / 1e6, 1), "avg_launch_us": round(sec * 1e6, 2),
                     "gbs": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4)})

    for shape in [(BATCH, 96, 112, 112), (BATCH, 144, 56, 56)]:
        x = torch.from_numpy(rng.uniform(-1, 1, shape).astype(np.float32)).cuda()
        z = torch.from_numpy(rng.uniform(-1, 1, shape).astype(np.float32)).cuda()
        y = torch.empty_like(x)
        nb = x.numel() * 4
        tag = "x".join(map(str, shape))
        timed_kernel(f"relu_f32 {tag}", lambda: nhip.relu(x, out=y), 2 * nb, "relu_f32")
        timed_kernel(f"add_f32 {tag}", lambda: nhip.add(x, z, out=y), 3 * nb, "add_f32")
        timed_kernel(f"add_f32 + relu {tag}", lambda: nhip.add(x, z, relu_after=True, out=y), 3 * nb, "add_f32")
        c = shape[1]
        for st in (1, 2):
            w = workloads.he_normal(rng, (c, 1, 3, 3), 9)
            b = rng.normal(0, 0.05, c).astype(np.float32)
            d = nhip.DwConv2dF32(nhip.conv_desc(c, c, (3, 3), (st, st), (1, 1), (1, 1, 1, 1), act=nhip.ACT_RELU,
                                                group=c), w, b)
            oh = (shape[2] - 1) // st + 1
            o = torch.empty((shape[0], c, oh, oh), device="cuda")
            timed_kernel(f"dw3x3s{st}_f32 + relu {tag}", lambda: d.forward(x, out=o), nb + o.numel() * 4, "dw3x3")
    return {"what": "achieved HBM bandwidth of the depthwise and elementwise kernels, batch-32 MobileNetV2 "
                    "shapes, fp32; bytes = inputs read once + outputs written once; time = HIP events around "
                    "each launch", "peak_gbs": PEAK_HBM_GBS, "kernels": rows}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=3.0,
                    help="length of each bounded CPU-baseline sample (per config and thread count)")
    ap.add_argument("--only-config3", action="store_true", help="skip the secondary configurations")
    ap.add_argument("--hbm-kernels", action="store_true",
                    help="instead of the bench line: the achieved HBM bandwidth of the depthwise and "
                         "elementwise kernels at batch-32 MobileNetV2 shapes (one JSON line)")
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
    if args.hbm_kernels:
        print(json.dumps(hbm_kernels(nhip, workloads, torch, max(args.steps, 10), args.warmup)), flush=True)
        return
    cpu = not args.no_cpu_baseline
    model, host_cpus, share = cpu_info()

    # ---- config 3: the headline
    stages = stage_stack(nhip, workloads, torch, BATCH)
    for _ in range(args.warmup):
        run_step(stages)
    torch.cuda.synchronize()
    fused_convs = [(c, hw) for c, hw in workloads.RESNET18_STAGES if fused_stage(c, hw)]
    kernel = "wino_fused" if fused_convs else "wino_gemm"
    kernel_convs = fused_convs or list(workloads.RESNET18_STAGES)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run_step(stages)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
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
    per_step = launches // args.steps
    assert launches % args.steps == 0 and per_step in (2 * len(kernel_convs), 4 * len(kernel_convs)), \
        (launches, args.steps, kernel_convs)
    kernel_s_per_step = kernel_ms / args.steps / 1e3
    achieved = kernel_flops / kernel_s_per_step / 1e12

    secondary = {}
    with tempfile.TemporaryDirectory() as workdir:
        if not args.only_config3:
            secondary["config1_conv"] = config1(nhip, workloads, torch, args.steps, args.warmup, workdir, share, cpu,
                                                args.cpu_seconds)
            secondary["config2_innerproduct"] = config2(nhip, workloads, torch, args.steps, args.warmup, share, cpu,
                                                        args.cpu_seconds)
            secondary["config4_int8"] = config4(nhip, workloads, torch, args.steps, args.warmup, share, cpu,
                                                args.cpu_seconds)
            secondary["config5_mobilenetv2"] = config5(nhip, torch, args.steps, args.warmup, workdir, share, cpu,
                                                       args.cpu_seconds)
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
            **rounded(secondary),
        },
        "roofline": {
            "bound": "mfma",
            "kernel": ("wino_fused (36 batched fp32 MFMA GEMMs + output transform per conv, at 64@56 the input "
                       "transform too; stages " + ", ".join(f"{c}@{hw}" for c, hw in kernel_convs) + ")")
                      if kernel == "wino_fused"
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
    if cpu:
        pair = cpu_config3(workloads, share, args.cpu_seconds * 2)
        result["cpu_baseline"] = {
            "value": pair["all"]["value"], "unit": "TFLOP/s", "cores": share, "kind": "port",
            "sample": f"{pair['all']['sample']}, OpenMP {share} threads (this job's CPU share of the host's "
                      f"{host_cpus} logical CPUs, {model}); one image per call as the reference's entry runs",
            "one_thread": pair["one"]["value"],
            "one_thread_sample": pair["one"]["sample"],
            "cpu_model": model, "host_logical_cpus": host_cpus}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
