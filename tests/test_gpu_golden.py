"""GPU parity on the reference's own numerical fixtures
(test/Numerical/fixtures/*.param with the payloads and golden vectors of
tests/golden/make_golden.py): the device graph executor (include/nhip_graph.h)
and the library ncnn-compile generates from each fixture are compared with
the golden outputs at the reference test's tolerance (int8, copies and ReLU
bit-exact), as test/Numerical/operators/{supported_ops,int8_ops,dynamic_ops}_test.cpp
compare the compiled CPU library with ncnn."""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import nhip  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden as mg  # noqa: E402
from test_golden import assert_golden, committed_bin, vectors  # noqa: E402

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(HERE)
TOOL = os.path.join(ROOT, "ncnn-compiler_amd", "bin", "ncnn-compile")
CASES = sorted(mg.CASES)
P = ctypes.c_void_p


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nhip.init(0)


def case_graph(case):
    fixture, inputs, _, _, tol, shapes = mg.CASES[case]
    param = open(os.path.join(mg.PARAMS, fixture + ".param")).read()
    return nhip.Graph(param, committed_bin(fixture), shapes), inputs, tol


@pytest.mark.parametrize("case", CASES)
def test_graph_executor_matches_golden(case):
    g, inputs, tol = case_graph(case)
    z = vectors(case)
    outs = g.run_host(*[z["in_" + name] for name, _ in inputs])
    for io, got in zip(g.outputs, outs):
        assert_golden(got, z["out_" + io["name"]], tol, f"{case}:{io['name']}")


@pytest.mark.parametrize("case", ["convolution_asymmetric_stride", "convolution_depthwise_9x9", "binary_add",
                                  "int8_complete_chain", "inner_product_dynamic_m_rows7",
                                  "pooling_global_average_dynamic", "split"])
def test_graph_batch_run_equals_per_image(case):
    # nhip_graph_run on a batch of 3 perturbed copies == three single-image runs
    g, inputs, tol = case_graph(case)
    z = vectors(case)
    batch = {name: np.stack([z["in_" + name] * s for s in (1.0, -0.5, 2.0)]).astype(np.float32)
             for name, _ in inputs}
    outs = g.run(*[torch.from_numpy(batch[name]).cuda() for name, _ in inputs])
    torch.cuda.synchronize()
    for i in range(3):
        ref = g.run_host(*[batch[name][i] for name, _ in inputs])
        for o, r in zip(outs, ref):
            np.testing.assert_array_equal(o[i].cpu().numpy(), r)


def _compile(tmp_path, case):
    fixture, _, _, _, _, shapes = mg.CASES[case]
    out = tmp_path / fixture
    args = [TOOL, os.path.join(mg.PARAMS, fixture + ".param"), "--bin", os.path.join(mg.BINS, fixture + ".bin"),
            "-o", str(out), "--model-name", fixture]
    for s in shapes or []:
        args.append("--input-shape=" + "x".join("?" if d < 0 else str(d) for d in s))
    r = subprocess.run(args, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return ctypes.CDLL(str(out / f"lib{fixture}.so")), fixture


@pytest.mark.parametrize("case", CASES)
def test_compiled_library_matches_golden(tmp_path, case):
    lib, fixture = _compile(tmp_path, case)
    g, inputs, tol = case_graph(case)
    z = vectors(case)
    xs = [np.ascontiguousarray(z["in_" + name]) for name, _ in inputs]
    shapes_out = g.infer_shapes([x.shape for x in xs])
    outs = [np.zeros(s, io["dtype"]) for s, io in zip(shapes_out, g.outputs)]
    args, types = [], []
    keep = []
    for io, x in zip(g.inputs, xs):
        args.append(x.ctypes.data_as(P))
        types.append(P)
        if any(d < 0 for d in io["shape"]):
            arr = (ctypes.c_int64 * 3)(*x.shape)
            keep.append(arr)
            args.append(arr)
            types.append(ctypes.POINTER(ctypes.c_int64))
    for io, o in zip(g.outputs, outs):
        args.append(o.ctypes.data_as(P))
        types.append(P)
        if any(d < 0 for d in io["shape"]):
            args.append(ctypes.c_uint64(o.size))
            types.append(ctypes.c_uint64)
    fn = getattr(lib, fixture)
    fn.argtypes = types
    assert fn(*args) == 0
    for io, got in zip(g.outputs, outs):
        assert_golden(got, z["out_" + io["name"]], tol, f"{case}:{io['name']} (compiled)")
