"""GPU parity of the standalone ncnn quantization layers in a model:
Requantize (ConvertRequantize, NCNNToTosa.cpp:4846-4888) and Dequantize
(ConvertDequantize, :4823-4840) on i32 Input blobs (the reference's integer
storage, ImportInput.cpp:78-80), through the graph executor and through a
library compiled by ncnn-compile, against the oracle bit for bit; and a
Requantize feeding an int8 Convolution that reads its i8 output as is."""
import ctypes
import subprocess

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import ncnn_format  # noqa: E402
import nhip  # noqa: E402
from oracle import refcpu  # noqa: E402

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(44)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nhip.init(0)


def accumulators(n, c, h, w):
    x = RNG.integers(-40000, 40000, (n, c, h, w)).astype(np.int32)
    x.flat[:8] = [0, 1, -1, 125, -125, 2 ** 31 - 1, -2 ** 31, 50]
    return x


def per_channel_or_scalar(c, per_channel, lo, hi):
    return RNG.uniform(lo, hi, c if per_channel else 1).astype(np.float32)


@pytest.mark.parametrize("per_channel_in,per_channel_out,bias,act", [
    (True, False, True, 1), (False, True, False, 0), (True, True, True, 0), (False, False, False, 1),
])
def test_requantize_layer_bit_exact(per_channel_in, per_channel_out, bias, act):
    c, h, w = 7, 9, 11
    isc = per_channel_or_scalar(c, per_channel_in, 1e-4, 3e-3)
    osc = per_channel_or_scalar(c, per_channel_out, 0.5, 4.0)
    b = RNG.standard_normal(c).astype(np.float32) * 3 if bias else None
    m = ncnn_format.Model()
    m.input("data", c, h, w)
    m.requantize("rq", "data", "out", isc, osc, b, act=act)
    g = nhip.Graph(m.param_text(), bytes(m.payload))
    assert g.inputs[0]["dtype"] == np.int32 and g.outputs[0]["dtype"] == np.int8
    x = accumulators(3, c, h, w)
    got = g.run(torch.from_numpy(x).cuda())[0].cpu().numpy()
    for i in range(3):
        exp = refcpu.requantize_i32_i8(x[i], isc, osc, b, act)
        np.testing.assert_array_equal(got[i], exp)
    # the reference entry semantics: one image from host buffers
    np.testing.assert_array_equal(g.run_host(x[1])[0], refcpu.requantize_i32_i8(x[1], isc, osc, b, act))
    g.close()


@pytest.mark.parametrize("bias", [None, "scalar", "channel"])
def test_dequantize_layer_bit_exact(bias):
    c, h, w = 5, 6, 8
    sc = RNG.uniform(1e-4, 1e-2, c).astype(np.float32)
    b = None if bias is None else RNG.standard_normal(1 if bias == "scalar" else c).astype(np.float32)
    m = ncnn_format.Model()
    m.input("data", c, h, w)
    m.dequantize("deq", "data", "out", sc, b)
    g = nhip.Graph(m.param_text(), bytes(m.payload))
    x = accumulators(2, c, h, w)
    got = g.run(torch.from_numpy(x).cuda())[0].cpu().numpy()
    for i in range(2):
        np.testing.assert_array_equal(got[i], refcpu.dequantize_i32_f32(x[i], sc, b))
    g.close()


def test_requantize_feeds_int8_convolution(tmp_path):
    """i32 -> Requantize (ReLU) -> i8 -> int8 Convolution (term 101, ReLU):
    the convolution reads the requantized bytes as is; through the library
    ncnn-compile writes (int32_t input, int8_t output)."""
    c, k, hw = 16, 24, 10
    isc = RNG.uniform(1e-4, 1e-3, c).astype(np.float32)
    osc = np.float32(2.0)
    wq = RNG.integers(-127, 128, (k, c, 3, 3)).astype(np.int8)
    ws = RNG.uniform(20, 60, k).astype(np.float32)
    cb = RNG.standard_normal(k).astype(np.float32)
    m = ncnn_format.Model()
    m.input("data", c, hw, hw)
    m.requantize("rq", "data", "q", isc, osc, None, act=1)
    m.conv("conv", "q", "out", wq, cb, act=1, int8=dict(term=101, ws=ws, **{"is": 1.0, "os": 0.5}))
    x = accumulators(1, c, hw, hw)
    q = refcpu.requantize_i32_i8(x[0], isc, osc, None, 1)
    exp = refcpu.conv2d_int8(refcpu.geom(1, c, hw, hw, k), q[None], wq, cb, ws, 1.0, 0.5, 101, 1)[0]
    p, b = tmp_path / "rqconv.param", tmp_path / "rqconv.bin"
    m.save(p, b)
    tool = nhip.LIB_PATH.replace("libnhip.so", "bin/ncnn-compile")
    r = subprocess.run([tool, str(p), "-o", str(tmp_path / "rqconv")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert "int rqconv(const int32_t *input1, int8_t *output1);" in (tmp_path / "rqconv" / "rqconv.h").read_text()
    lib = ctypes.CDLL(str(tmp_path / "rqconv" / "librqconv.so"))
    lib.rqconv.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    out = np.zeros((k, hw, hw), np.int8)
    xi = np.ascontiguousarray(x[0])
    assert lib.rqconv(xi.ctypes.data_as(ctypes.c_void_p), out.ctypes.data_as(ctypes.c_void_p)) == 0
    np.testing.assert_array_equal(out, exp)
