"""GPU parity: ConvolutionDepthWise, InnerProduct and the elementwise
neighbours against the CPU oracle.

Depthwise runs the reference's exact operation order (zero-init sum over
kh, kw, then + bias, NCNNToTosa.cpp:3376-3503) with no fused multiply-add, so
it is checked bit for bit.  InnerProduct (NCNNToTosa.cpp:5254-5392) is an
MFMA GEMM: max relative error <= 1e-4.  Quantize / requantize / dequantize
are bit-exact; global average pooling is checked to 1e-6 (planes of up to
256 pixels are summed in the oracle's order and match it bit for bit).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import nhip  # noqa: E402
import workloads  # noqa: E402
from numerics import assert_close, max_rel_err  # noqa: E402
from oracle import refcpu  # noqa: E402

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(11)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nhip.init(0)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


DW_CASES = [
    # (n, c, h, w, kernel, stride, dil, pad) - MobileNetV2 depthwise shapes at
    # small batch, plus ragged / general ones
    (2, 32, 112, 112, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1)),
    (2, 96, 112, 112, (3, 3), (2, 2), (1, 1), (1, 1, 1, 1)),
    (2, 144, 56, 56, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1)),
    (2, 144, 56, 56, (3, 3), (2, 2), (1, 1), (1, 1, 1, 1)),
    (2, 192, 28, 28, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1)),
    (2, 384, 14, 14, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1)),
    (2, 576, 14, 14, (3, 3), (2, 2), (1, 1), (1, 1, 1, 1)),
    (2, 960, 7, 7, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1)),
    (3, 5, 9, 13, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1)),
    (1, 6, 17, 11, (5, 5), (2, 1), (2, 1), (3, 1, 0, 2)),
    (2, 4, 6, 7, (2, 3), (1, 2), (1, 1), (0, 0, 1, 1)),
    (1, 3, 301, 5, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1)),
]


@pytest.mark.parametrize("case", DW_CASES, ids=lambda c: "x".join(map(str, c[:4])) + f"s{c[5][0]}")
@pytest.mark.parametrize("act,bias", [(0, True), (1, True), (1, False)])
def test_depthwise_bit_exact(case, act, bias):
    n, c, h, w, ker, st, dl, pad = case
    x = RNG.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = workloads.he_normal(RNG, (c, 1) + ker, ker[0] * ker[1])
    b = RNG.normal(0, 0.05, c).astype(np.float32) if bias else None
    d = nhip.conv_desc(c, c, ker, st, dl, pad, bias=bias, act=act, group=c)
    got = host(nhip.DwConv2dF32(d, wt, b).forward(dev(x)))
    g = refcpu.geom(n, c, h, w, c, ker, st, dl, pad)
    exp = refcpu.dwconv2d_f32(g, x, wt, b)
    if act == 1:
        exp = refcpu.relu_f32(exp)
    np.testing.assert_array_equal(got, exp)


PLANE_CASES = [
    # (n, c, h, w, stride, pad): 3x3 depthwise on planes of at most 1024
    # pixels, the whole-plane LDS kernel - the MobileNetV2 layers at batch 32,
    # blocks that end part-way (channel counts no multiple of the planes per
    # block), odd plane sizes, 1x1 planes, asymmetric padding
    (32, 960, 7, 7, 1, (1, 1, 1, 1)),
    (32, 576, 14, 14, 2, (1, 1, 1, 1)),
    (32, 384, 14, 14, 1, (1, 1, 1, 1)),
    (32, 192, 28, 28, 2, (1, 1, 1, 1)),
    (3, 37, 7, 7, 1, (1, 1, 1, 1)),
    (1, 5, 1, 1, 1, (1, 1, 1, 1)),
    (2, 7, 9, 13, 2, (0, 1, 0, 1)),
    (2, 11, 32, 32, 2, (1, 1, 1, 1)),
    (1, 3, 5, 31, 1, (2, 0, 1, 2)),
]


@pytest.mark.parametrize("case", PLANE_CASES, ids=lambda c: "x".join(map(str, c[:4])) + f"s{c[4]}")
@pytest.mark.parametrize("planes", ["1", "2", "0"])
def test_depthwise_small_planes_bit_exact(case, planes, nhip_env):
    """The streamed whole-plane kernel (NHIP_DW_PLANES=1, default: rows that
    are not 16-byte vectors; =2: every shape it takes) and the window kernel
    (=0) against the oracle, bit for bit, also from a 4-byte-offset input
    view (direct-to-LDS copies from an address that is not 16-byte
    aligned)."""
    nhip_env.setenv("NHIP_DW_PLANES", planes)
    n, c, h, w, st, pad = case
    x = RNG.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = workloads.he_normal(RNG, (c, 1, 3, 3), 9)
    b = RNG.normal(0, 0.05, c).astype(np.float32)
    d = nhip.conv_desc(c, c, (3, 3), (st, st), (1, 1), pad, bias=True, act=1, group=c)
    plan = nhip.DwConv2dF32(d, wt, b)
    got = host(plan.forward(dev(x)))
    g = refcpu.geom(n, c, h, w, c, (3, 3), (st, st), (1, 1), pad)
    exp = refcpu.relu_f32(refcpu.dwconv2d_f32(g, x, wt, b))
    np.testing.assert_array_equal(got, exp)
    buf = torch.empty(x.size + 1, dtype=torch.float32, device="cuda")
    xv = buf[1:].view(x.shape)
    xv.copy_(dev(x))
    np.testing.assert_array_equal(host(plan.forward(xv)), exp)


def test_innerproduct_config2():
    x, w, b = workloads.innerproduct(seed=0)
    ip = nhip.InnerProductF32(w, b)
    got = host(ip.forward(dev(x)))
    exp = refcpu.innerproduct_f32(x, w, b)
    assert_close(got, exp, 1e-4, "ip config2")
    assert max_rel_err(got, exp) <= 1e-4


@pytest.mark.parametrize("m,k,n,act", [
    (1, 1280, 1000, 0),    # MobileNetV2 head
    (1, 33, 5, 1),
    (7, 130, 65, 1),
    (70, 2049, 3, 0),
    (32, 1280, 1000, 0),
    (300, 96, 200, 1),
])
def test_innerproduct_shapes(m, k, n, act):
    x = RNG.uniform(-1, 1, (m, k)).astype(np.float32)
    w = (RNG.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
    b = RNG.normal(0, 0.01, n).astype(np.float32)
    got = host(nhip.InnerProductF32(w, b, act).forward(dev(x)))
    exp = refcpu.innerproduct_f32(x, w, b)
    if act:
        exp = refcpu.relu_f32(exp)
    assert_close(got, exp, 1e-4, f"ip {m}x{k}x{n}")


def test_innerproduct_without_bias_zero_init_then_bias():
    # zero-initialised matmul, bias added after: (1e8 - 1e8) + 1 = 1
    x = np.ones((1, 2), np.float32)
    w = np.array([[1e8, -1e8]], np.float32)
    got = host(nhip.InnerProductF32(w, np.array([1.0], np.float32)).forward(dev(x)))
    assert got[0, 0] == 1.0
    got = host(nhip.InnerProductF32(w).forward(dev(x)))
    assert got[0, 0] == 0.0


@pytest.mark.parametrize("count", [1, 3, 4, 7, 1024, 4099, 65536 * 5 + 2, 1 << 22])
@pytest.mark.parametrize("offset", [0, 1])
def test_relu_and_add_vector_paths_bit_exact(count, offset):
    """ReLU and add on 16-byte vectors (aligned buffers: four vectors in
    flight per thread, the last count % 4 elements on the scalar kernel) and
    on the scalar kernel alone (offset 1: views 4 bytes past an aligned
    base), bit for bit against the oracle, signed zeros and NaN included."""
    x = RNG.uniform(-1, 1, count).astype(np.float32)
    y = RNG.uniform(-1, 1, count).astype(np.float32)
    x[: min(count, 3)] = np.array([-0.0, np.nan, 0.0], np.float32)[: min(count, 3)]
    def view(a):
        buf = torch.empty(a.size + offset, dtype=torch.float32, device="cuda")
        v = buf[offset:]
        v.copy_(torch.from_numpy(a).cuda())
        return v
    got = host(nhip.relu(view(x), out=view(np.zeros_like(x))))
    np.testing.assert_array_equal(got.view(np.uint32), refcpu.relu_f32(x).view(np.uint32))
    for relu_after in (False, True):
        exp = refcpu.add_f32(x, y)
        if relu_after:
            exp = refcpu.relu_f32(exp)
        got = host(nhip.add(view(x), view(y), relu_after=relu_after, out=view(np.zeros_like(x))))
        np.testing.assert_array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_relu_add_and_avgpool():
    x = RNG.uniform(-1, 1, (3, 5, 7, 9)).astype(np.float32)
    y = RNG.uniform(-1, 1, (3, 5, 7, 9)).astype(np.float32)
    np.testing.assert_array_equal(host(nhip.relu(dev(x))), refcpu.relu_f32(x))
    np.testing.assert_array_equal(host(nhip.add(dev(x), dev(y))), refcpu.add_f32(x, y))
    np.testing.assert_array_equal(host(nhip.add(dev(x), dev(y), relu_after=True)),
                                  refcpu.relu_f32(refcpu.add_f32(x, y)))
    xi = RNG.integers(-127, 128, 1000).astype(np.int8)
    np.testing.assert_array_equal(host(nhip.relu(dev(xi))), refcpu.relu_i8(xi))
    p = RNG.uniform(-1, 1, (4, 1280, 7, 7)).astype(np.float32)
    assert_close(host(nhip.global_avgpool(dev(p))), refcpu.global_avgpool_f32(p), 1e-6, "gap")
    q = np.arange(16, dtype=np.float32).reshape(1, 1, 4, 4)
    assert host(nhip.global_avgpool(dev(q)))[0, 0] == 7.5


def test_quantize_requantize_dequantize_bit_exact():
    x = RNG.uniform(-3, 3, (2, 6, 5, 5)).astype(np.float32)
    x.ravel()[:6] = [0.5, -0.5, 2.5, -2.5, 0.49999997, 1e9]
    for scale in (np.float32(41.5), RNG.uniform(10, 60, 6).astype(np.float32)):
        got = host(nhip.quantize(dev(x), scale))
        exp = np.stack([refcpu.quantize_f32_i8(x[i], np.atleast_1d(scale),
                                               channel_size=25) for i in range(2)])
        np.testing.assert_array_equal(got, exp)
    acc = RNG.integers(-20000, 20000, (2, 6, 4, 4)).astype(np.int32)
    isc = RNG.uniform(1e-3, 1e-2, 6).astype(np.float32)
    bias = RNG.normal(0, 1, 6).astype(np.float32)
    for act in (0, 1):
        got = host(nhip.requantize(dev(acc), isc, np.float32(3.0), bias, act))
        exp = np.stack([refcpu.requantize_i32_i8(acc[i], isc, 3.0, bias, act) for i in range(2)])
        np.testing.assert_array_equal(got, exp)
    got = host(nhip.dequantize(dev(acc), isc, bias))
    exp = np.stack([refcpu.dequantize_i32_f32(acc[i], isc, bias) for i in range(2)])
    np.testing.assert_array_equal(got, exp)
