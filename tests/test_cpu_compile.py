"""The .param/.bin front end, the lowering and ncnn-compile, on the CPU.

nhip_graph_describe runs the parser, weight loader, lowering and shape
inference without touching a device, so everything here runs without a GPU:
I/O shapes, the reference's rejection statuses, and the compiled artifact set
(header text, exported symbols, manifest, host-side shape inference and the
null-pointer status of the generated entry).
"""
import ctypes
import json
import os
import subprocess

import numpy as np
import pytest

import graphs
import ncnn_format
import nhip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TOOL = os.path.join(ROOT, "ncnn-compiler_amd", "bin", "ncnn-compile")
RNG = np.random.default_rng(3)

i64p = ctypes.POINTER(ctypes.c_int64)


def glib():
    L = nhip.load()
    L.nhip_graph_describe.argtypes = [ctypes.c_char_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64, i64p,
                                      ctypes.c_int32, ctypes.POINTER(ctypes.c_void_p)]
    L.nhip_graph_num_io.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32)]
    L.nhip_graph_io_info.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(ctypes.c_int32),
                                     i64p, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_char_p)]
    L.nhip_graph_infer_shapes.argtypes = [ctypes.c_void_p, i64p, i64p, ctypes.POINTER(ctypes.c_int32)]
    L.nhip_graph_destroy.argtypes = [ctypes.c_void_p]
    return L


def describe(model, shapes=None):
    """-> (status, message, inputs, outputs); io entries (name, dims, dtype)."""
    L = glib()
    param = model.param_text().encode()
    binb = bytes(model.payload)
    h = ctypes.c_void_p()
    arr = None
    if shapes is not None:
        flat = [v for s in shapes for v in s]
        arr = (ctypes.c_int64 * len(flat))(*flat)
    st = L.nhip_graph_describe(param, len(param), binb, len(binb), arr, 0 if shapes is None else len(shapes),
                               ctypes.byref(h))
    if st != 0:
        return st, L.nhip_last_error().decode(), None, None
    ni, no = ctypes.c_int32(), ctypes.c_int32()
    L.nhip_graph_num_io(h, ctypes.byref(ni), ctypes.byref(no))
    io = []
    for is_out, count in ((0, ni.value), (1, no.value)):
        lst = []
        for i in range(count):
            rank, dt, name = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_char_p()
            dims = (ctypes.c_int64 * 4)()
            assert L.nhip_graph_io_info(h, is_out, i, ctypes.byref(rank), dims, ctypes.byref(dt), ctypes.byref(name)) == 0
            lst.append((name.value.decode(), list(dims)[:rank.value], dt.value))
        io.append(lst)
    L.nhip_graph_destroy(h)
    return 0, "", io[0], io[1]


def conv_model(c=64, k=64, hw=56, act=1):
    m = ncnn_format.Model()
    m.input("data", c, hw, hw)
    m.conv("conv", "data", "output", RNG.standard_normal((k, c, 3, 3)).astype(np.float32),
           RNG.standard_normal(k).astype(np.float32), act=act)
    return m


def ip_dynamic_model(k=2048, n=1000):
    # reference fixture shape: test/Numerical/fixtures/inner_product_dynamic_m.param
    m = ncnn_format.Model()
    m.input("data", 0, 0, 0)
    m.squeeze("squeeze", "data", "matrix", [0])
    m.innerproduct("ip", "matrix", "output", RNG.standard_normal((n, k)).astype(np.float32),
                   RNG.standard_normal(n).astype(np.float32))
    return m


def resnet_block_model(c=16, hw=8):
    """conv-BN-ReLU-conv-BN + identity -> ReLU, BN unfolded, Split fan-out."""
    m = ncnn_format.Model()
    m.input("data", c, hw, hw)
    m.split("split", "data", ["d0", "d1"])
    for i, (src, dst) in enumerate((("d0", "c1"), ("r1", "c2"))):
        m.conv(f"conv{i}", src, dst + "_raw", RNG.standard_normal((c, c, 3, 3)).astype(np.float32) * 0.1,
               RNG.standard_normal(c).astype(np.float32) * 0.1)
        m.batchnorm(f"bn{i}", dst + "_raw", dst, RNG.uniform(0.5, 1.5, c).astype(np.float32),
                    RNG.normal(0, 0.1, c).astype(np.float32), RNG.uniform(0.5, 2, c).astype(np.float32),
                    RNG.normal(0, 0.1, c).astype(np.float32))
        if i == 0:
            m.relu("relu0", "c1", "r1")
    m.add("add", "c2", "d1", "sum")
    m.relu("relu1", "sum", "output")
    return m


def test_static_conv_io():
    st, msg, ins, outs = describe(conv_model())
    assert st == 0, msg
    assert ins == [("data", [64, 56, 56], 0)]
    assert outs == [("output", [64, 56, 56], 0)]


def test_dynamic_innerproduct_io():
    st, msg, ins, outs = describe(ip_dynamic_model(), shapes=[(1, -1, 2048)])
    assert st == 0, msg
    assert ins == [("data", [1, -1, 2048], 0)]
    assert outs == [("output", [-1, 1000], 0)]


def test_resnet_block_and_mobilenetv2_io():
    st, msg, ins, outs = describe(resnet_block_model())
    assert st == 0, msg
    assert outs == [("output", [16, 8, 8], 0)]
    m = ncnn_format.from_layer_list(graphs.mobilenetv2_layers(seed=0))
    st, msg, ins, outs = describe(m)
    assert st == 0, msg
    assert ins == [("data", [3, 224, 224], 0)] and outs == [("fc", [1000], 0)]


def test_int8_chain_io_types():
    m = ncnn_format.Model()
    m.input("data", 8, 5, 5)
    w = RNG.integers(-127, 128, (4, 8, 3, 3)).astype(np.int8)
    m.conv("q", "data", "q8", w, RNG.standard_normal(4).astype(np.float32),
           int8=dict(term=101, ws=np.full(4, 50.0, np.float32), **{"is": 20.0, "os": 10.0}))
    st, msg, ins, outs = describe(m)
    assert st == 0, msg
    assert outs == [("q8", [4, 5, 5], 1)]


def requantize_model(c=6, hw=5, deq=False, bias=True, act=1):
    """Input (i32 storage: read by Requantize / Dequantize) -> one layer."""
    m = ncnn_format.Model()
    m.input("data", c, hw, hw)
    b = RNG.standard_normal(c).astype(np.float32) if bias else None
    if deq:
        m.dequantize("deq", "data", "out", RNG.uniform(1e-3, 1e-2, c).astype(np.float32), b)
    else:
        m.requantize("rq", "data", "out", RNG.uniform(1e-3, 1e-2, c).astype(np.float32), np.float32(4.0), b, act=act)
    return m


def test_quantization_layers_io_types():
    # Requantize: i32 in, i8 out; Dequantize: i32 in, f32 out
    st, msg, ins, outs = describe(requantize_model())
    assert st == 0, msg
    assert ins == [("data", [6, 5, 5], 2)] and outs == [("out", [6, 5, 5], 1)]
    st, msg, ins, outs = describe(requantize_model(deq=True))
    assert st == 0, msg
    assert ins == [("data", [6, 5, 5], 2)] and outs == [("out", [6, 5, 5], 0)]


def test_quantization_layers_consume_raw_fp32_weights_in_order():
    """test/Unit/malformed_graph_test.cpp:564-597: Quantize (1 scale),
    Dequantize (scale + bias), Requantize (two scales + bias) read six raw
    fp32 words in layer order; the reference's importer then rejects the
    Dequantize, whose operand is the Quantize's i8 output, not i32
    (NCNNOps.cpp:1440-1442), and a truncated payload names the Requantize
    bias."""
    text = ("7767517\n4 4\nInput input 0 1 in\nQuantize quantize 1 1 in quantized 0=1\n"
            "Dequantize dequantize 1 1 quantized restored 0=1 1=1\n"
            "Requantize requantize 1 1 restored out 0=1 1=1 2=1 3=0\n")

    class Raw:
        def __init__(self, payload):
            self.payload = payload

        def param_text(self):
            return text

    ones = np.ones(6, "<f4").tobytes()
    st, msg, _, _ = describe(Raw(ones), shapes=[(1, 1, 1)])
    assert st == 3 and "Dequantize input must be ranked i32" in msg, msg  # weights loaded, import rejected
    st, msg, _, _ = describe(Raw(ones[:-1]), shapes=[(1, 1, 1)])
    assert st == 3 and "truncated" in msg and "Requantize bias" in msg, msg


@pytest.mark.parametrize("case,needle", [
    ("act6", "no activation or ReLU"),
    ("count", "dimension zero"),
    ("negative", "invalid Requantize"),
    ("f32_operand", "int32 operand"),
])
def test_quantization_layer_rejections(case, needle):
    if case == "act6":
        m = requantize_model(act=6)
    elif case == "count":  # 4 scales on 6 channels
        m = ncnn_format.Model()
        m.input("data", 6, 5, 5)
        m.dequantize("deq", "data", "out", np.ones(4, np.float32))
    elif case == "negative":
        m = requantize_model()
        m.lines[-1] = m.lines[-1].replace("2=6", "2=-1")
    else:  # an i32 Input also read by a convolution
        m = requantize_model()
        m.conv("c", "data", "c_out", RNG.standard_normal((2, 6, 3, 3)).astype(np.float32))
    st, msg, _, _ = describe(m)
    assert st != 0 and needle in msg, msg


def test_quantization_model_compiles_with_int32_input(tmp_path):
    out = compile_model(tmp_path, requantize_model(), "rq", ["--emit-manifest"])
    h = (out / "rq.h").read_text()
    assert "int rq(const int32_t *input1, int8_t *output1);" in h
    man = json.loads((out / "rq.json").read_text())
    assert man["inputs"][0]["element_type"] == "i32" and man["outputs"][0]["element_type"] == "i8"


def test_weight_count_beyond_the_payload_allocates_nothing():
    # a .param claiming 1.2e9 weights with an 8-byte .bin fails as truncated
    m = ncnn_format.Model()
    m.input("data", 4, 6, 6)
    m.conv("c", "data", "out", RNG.standard_normal((4, 4, 3, 3)).astype(np.float32))
    m.lines[-1] = m.lines[-1].replace("6=144", "6=1207959552")  # 36 * 2^25 weights, passes the parameter rules
    m.payload = m.payload[:8]
    st, msg, _, _ = describe(m)
    assert st == 3 and "truncated" in msg, msg


@pytest.mark.parametrize("case,status,needle", [
    ("softmax", 7, "Softmax 'prob'"),
    ("magic", 3, "magic"),
    ("truncated", 3, "truncated"),
    ("omitted", 2, "omitted"),
    ("int8_dw_f32_input_relu6", 7, "activation"),
    ("channels", 2, "channels"),
])
def test_rejections(case, status, needle):
    m = conv_model(c=4, k=4, hw=6)
    if case == "softmax":
        m.layer("Softmax", "prob", ["output"], ["prob"])
    if case == "omitted":
        m = ip_dynamic_model()
    if case == "int8_dw_f32_input_relu6":
        m = ncnn_format.Model()
        m.input("data", 4, 6, 6)
        m.conv("dw", "data", "out", RNG.integers(-9, 9, (4, 1, 3, 3)).astype(np.int8), None, depthwise=True,
               act=2, int8=dict(term=1, ws=np.ones(4, np.float32), **{"is": 1.0}))
    if case == "channels":
        m = ncnn_format.Model()
        m.input("data", 3, 6, 6)
        m.conv("c", "data", "out", RNG.standard_normal((4, 5, 3, 3)).astype(np.float32))
    if case == "magic":
        m.lines.insert(0, "")
        text = m.param_text().replace("7767517", "7767518")
        m.param_text = lambda: text
    if case == "truncated":
        m.payload = m.payload[:-8]
    st, msg, _, _ = describe(m)
    assert st == status, msg
    assert needle in msg, msg


def compile_model(tmp_path, model, name, extra=()):
    p = tmp_path / f"{name}.param"
    b = tmp_path / f"{name}.bin"
    model.save(p, b)
    out = tmp_path / "out"
    r = subprocess.run([TOOL, str(p), "-o", str(out), *extra], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return out


def exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True).stdout
    return sorted(line.split()[-1] for line in out.splitlines() if " T " in line)


def test_compile_static_model_artifacts(tmp_path):
    out = compile_model(tmp_path, conv_model(), "conv", ["--emit-manifest"])
    assert sorted(os.listdir(out)) == ["conv.h", "conv.json", "libconv.so"]
    h = (out / "conv.h").read_text()
    for line in ("#define NCNN_STATUS_OUTPUT_CAPACITY_INSUFFICIENT 5", "#define CONV_INPUT_COUNT 1",
                 "#define CONV_INPUT1_RANK 3", "#define CONV_INPUT1_DIM0 INT64_C(64)",
                 "#define CONV_INPUT1_DYNAMIC_DIM_MASK UINT32_C(0x0)", "#define CONV_INPUT1_ELEMENTS UINT64_C(200704)",
                 "#define CONV_OUTPUT1_SHAPE_DEPENDS_ON_DATA 0", "int conv(const float *input1, float *output1);"):
        assert line in h, line
    assert exported(out / "libconv.so") == ["conv"]
    man = json.loads((out / "conv.json").read_text())
    assert man["function"] == "conv"
    assert man["inputs"][0]["shape"] == [64, 56, 56] and man["outputs"][0]["element_type"] == "f32"
    # the generated entry rejects null pointers before any device work
    lib = ctypes.CDLL(str(out / "libconv.so"))
    lib.conv.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    assert lib.conv(None, None) == 1


def test_compile_dynamic_model_shape_inference(tmp_path):
    out = compile_model(tmp_path, ip_dynamic_model(), "ip", ["--input-shape=1x?x2048"])
    h = (out / "ip.h").read_text()
    assert ("int ip(const float *input1, const int64_t input1_shape[IP_INPUT1_RANK], float *output1, "
            "uint64_t output1_capacity);") in h
    assert "int ip_infer_output_shapes(const int64_t input1_shape[IP_INPUT1_RANK], " \
           "int64_t output1_shape[IP_OUTPUT1_RANK]);" in h
    assert "#define IP_INPUT1_DIM1 NCNN_DYNAMIC_DIM" in h and "#define IP_OUTPUT1_DYNAMIC_DIM_MASK UINT32_C(0x1)" in h
    assert exported(out / "libip.so") == ["ip", "ip_infer_output_shapes"]
    lib = ctypes.CDLL(str(out / "libip.so"))
    lib.ip_infer_output_shapes.argtypes = [i64p, i64p]
    ishape = (ctypes.c_int64 * 3)(1, 256, 2048)
    oshape = (ctypes.c_int64 * 2)()
    assert lib.ip_infer_output_shapes(ishape, oshape) == 0
    assert list(oshape) == [256, 1000]
    bad = (ctypes.c_int64 * 3)(1, 256, 2047)
    assert lib.ip_infer_output_shapes(bad, oshape) == 2  # NCNN_STATUS_INVALID_SHAPE


@pytest.mark.parametrize("raw,expect", [("resnet-50", "resnet_50"), ("123model", "ncnn_123model"),
                                        ("main", "ncnn_main"), ("a..b", "a_b")])
def test_model_name_rules(tmp_path, raw, expect):
    out = compile_model(tmp_path, conv_model(c=4, k=4, hw=6), "m", [f"--model-name={raw}"])
    assert (out / f"{expect}.h").exists() and (out / f"lib{expect}.so").exists()


def test_compile_failure_publishes_nothing(tmp_path):
    m = conv_model(c=4, k=4, hw=6)
    m.layer("Softmax", "prob", ["output"], ["prob"])
    p, b = tmp_path / "bad.param", tmp_path / "bad.bin"
    m.save(p, b)
    r = subprocess.run([TOOL, str(p), "-o", str(tmp_path / "out")], capture_output=True, text=True)
    assert r.returncode != 0 and "Softmax 'prob'" in r.stderr
    assert not (tmp_path / "out").exists()


def run_tool(tmp_path, model, name, extra=()):
    p, b = tmp_path / f"{name}.param", tmp_path / f"{name}.bin"
    model.save(p, b)
    return subprocess.run([TOOL, str(p), "-o", str(tmp_path / "out"), *extra], capture_output=True, text=True)


@pytest.mark.parametrize("flag,needle", [
    ("--input-dim-constraint=0:1:min=32", "INPUT:DIM:min=N,multiple=N"),          # multiple missing
    ("--input-dim-constraint=0:1:min=0,multiple=4", "positive"),                  # non-positive
    ("--input-dim-constraint=0:1:min=4,multiple=4,min=8", "INPUT:DIM"),           # repeated field
    ("--input-dim-constraint=1:1:min=4,multiple=4", "input index 1 is out of range"),
    ("--input-dim-constraint=0:5:min=4,multiple=4", "dimension 5 is out of range"),
    ("--input-dim-constraint=0:2:min=4,multiple=4", "is static"),
])
def test_input_dim_constraint_rejections(tmp_path, flag, needle):
    r = run_tool(tmp_path, ip_dynamic_model(), "ip", ["--input-shape=1x?x2048", flag])
    assert r.returncode != 0 and needle in r.stderr, r.stderr
    assert not (tmp_path / "out").exists()


def test_input_dim_constraint_duplicate_rejected(tmp_path):
    c = "--input-dim-constraint=0:1:min=4,multiple=4"
    r = run_tool(tmp_path, ip_dynamic_model(), "ip", ["--input-shape=1x?x2048", c, c])
    assert r.returncode != 0 and "duplicate" in r.stderr


def test_input_dim_constraint_header_manifest_and_checks(tmp_path):
    """docs/ncnn-compile-command-line.md section 2.6: per-dimension minimum
    and divisor macros (tools/ncnn-compile.cpp:1059-1073), the manifest's
    dimension_constraints (:818-830), and status 3 from the entry points
    when an extent breaks them (status 2 first for a non-positive extent)."""
    out = compile_model(tmp_path, ip_dynamic_model(), "ip",
                        ["--input-shape=1x?x2048", "--input-dim-constraint=0:1:min=32,multiple=16",
                         "--emit-manifest"])
    h = (out / "ip.h").read_text()
    assert "#define IP_INPUT1_DIM1_MINIMUM INT64_C(32)" in h
    assert "#define IP_INPUT1_DIM1_MULTIPLE_OF INT64_C(16)" in h
    man = json.loads((out / "ip.json").read_text())
    assert man["inputs"][0]["dimension_constraints"] == [{"dimension": 1, "minimum": 32, "multiple_of": 16}]
    lib = ctypes.CDLL(str(out / "libip.so"))
    lib.ip_infer_output_shapes.argtypes = [i64p, i64p]
    oshape = (ctypes.c_int64 * 2)()
    for m, status in ((48, 0), (32, 0), (16, 3), (40, 3), (0, 2), (-5, 2)):
        ishape = (ctypes.c_int64 * 3)(1, m, 2048)
        assert lib.ip_infer_output_shapes(ishape, oshape) == status, m
    # the model entry checks the same before any device work
    lib.ip.argtypes = [ctypes.c_void_p, i64p, ctypes.c_void_p, ctypes.c_uint64]
    buf = np.zeros(64 * 2048, np.float32)
    ishape = (ctypes.c_int64 * 3)(1, 40, 2048)
    assert lib.ip(buf.ctypes.data, ishape, buf.ctypes.data, 64 * 1000) == 3


def test_artifact_passes_the_extended_audit(tmp_path):
    """The generated library satisfies the reference's audit rules
    (tools/ncnn-compile.cpp:2070-2196) as extended for the GPU runtime:
    exports exactly the entry points, undefined symbols are the reference's
    libc/libm allowlist plus pthread_once and nhip_*, DT_NEEDED is libc /
    libm / libnhip, and no forbidden runtime names appear."""
    for model, extra, name in ((conv_model(c=4, k=4, hw=6), [], "conv"),
                               (ip_dynamic_model(), ["--input-shape=1x?x2048"], "ip")):
        (tmp_path / name).mkdir()
        out = compile_model(tmp_path / name, model, name, extra)
        lib = str(out / f"lib{name}.so")
        und = subprocess.run(["nm", "-D", "--undefined-only", lib], capture_output=True, text=True).stdout.split()
        und = {s.split("@")[0] for s in und if s not in ("U", "w")}
        assert und <= {"memcpy", "memset", "malloc", "free", "pthread_once"} | {s for s in und if s.startswith("nhip_")}
        need = subprocess.run(["readelf", "-d", lib], capture_output=True, text=True).stdout
        needed = {line.split("[")[1].split("]")[0] for line in need.splitlines() if "(NEEDED)" in line}
        assert needed <= {"libc.so.6", "libm.so.6", "libnhip.so"}, needed
        allsyms = subprocess.run(["nm", "-D", lib], capture_output=True, text=True).stdout
        assert not any(f in allsyms for f in ("memrefCopy", "runner_utils", "RunnerUtils", "ncnn_runtime"))


def _gpu_present():
    count = ctypes.c_int32(0)
    return nhip.load().nhip_device_count(ctypes.byref(count)) == 0 and count.value > 0


def test_verify_execution_without_a_gpu_fails_closed(tmp_path):
    """--verify-execution builds the ABI harness and runs it; on a host with
    no GPU the model call fails, so the tool fails and publishes nothing
    (the GPU tests run the passing case)."""
    if _gpu_present():
        pytest.skip("a GPU is present: the passing case is covered by the GPU tests")
    r = run_tool(tmp_path, conv_model(c=4, k=4, hw=6), "conv", ["--verify-execution"])
    assert r.returncode != 0 and "ABI execution verification failed" in r.stderr, r.stderr
    assert not (tmp_path / "out").exists()
