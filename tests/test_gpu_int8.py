"""GPU parity: int8 Convolution with requantize, bit-exact against the CPU
oracle's restatement of NCNNToTosa.cpp:1136-1315 (quantize :322-389,
dequantizeAccumulator :577-637, bias add :1294-1300, requantize :1309-1312,
relu after, ImportConvolution.cpp:236-241), plus the reference's own
known-answer cases (test/Conversion/NCNNToTosa/quantized-contractions.mlir,
test/Numerical/fixtures/generate_int8_bins.py)."""
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import nhip  # noqa: E402
import workloads  # noqa: E402
from oracle import refcpu  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nhip.init(0)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def run(desc, x, w, b, ws, is_, os_):
    conv = nhip.Conv2dInt8(desc, w, b, ws, is_, os_)
    return host(conv.forward(dev(x)))


def oracle(desc, x, w_i8, b, ws, is_, os_):
    n, c, h, wd = x.shape
    g = refcpu.geom(n, c, h, wd, desc.num_output, (desc.kernel_h, desc.kernel_w),
                    (desc.stride_h, desc.stride_w), (desc.dilation_h, desc.dilation_w),
                    (desc.pad_top, desc.pad_bottom, desc.pad_left, desc.pad_right))
    return refcpu.conv2d_int8(g, x, w_i8, b, ws, is_, os_, scale_term=desc.int8_scale_term,
                              activation=desc.activation_type)


def test_config4_batch2_bit_exact():
    cfg = workloads.int8_conv(seed=0, n=2)
    d = nhip.conv_desc(128, 128, act=nhip.ACT_RELU, int8_scale_term=101)
    got = run(d, cfg["x"], cfg["w"], cfg["bias"], cfg["ws"], cfg["input_scale"], cfg["output_scale"])
    exp = oracle(d, cfg["x"], cfg["w"], cfg["bias"], cfg["ws"], cfg["input_scale"], cfg["output_scale"])
    assert got.dtype == np.int8
    np.testing.assert_array_equal(got, exp)
    # the case is not degenerate: many distinct levels, some saturation
    assert len(np.unique(got)) > 64 and (got == 127).any() and (got == 0).any()


def test_config4_full_batch_bit_exact():
    cfg = workloads.int8_conv(seed=0, n=32)
    d = nhip.conv_desc(128, 128, act=nhip.ACT_RELU, int8_scale_term=101)
    got = run(d, cfg["x"], cfg["w"], cfg["bias"], cfg["ws"], 1.0, 1.0)
    exp = oracle(d, cfg["x"], cfg["w"], cfg["bias"], cfg["ws"], 1.0, 1.0)
    for i in range(32):  # every image of the bench's batch, bit for bit
        np.testing.assert_array_equal(got[i:i + 1], exp[i:i + 1], err_msg=f"image {i}")


def test_quantized_contractions_known_answers():
    # quantized-contractions.mlir:3-8: ones weight [3,2,1,1], ws [2,4,8], is 2,
    # bias [1,2,3], term 1: out = 3/(ws*2) + bias = 1.75, 2.375, 3.1875.
    x = np.stack([np.full((3, 3), 1.0), np.full((3, 3), 0.25)]).astype(np.float32)[None]
    w = np.ones((3, 2, 1, 1), np.int8)
    d = nhip.conv_desc(2, 3, (1, 1), pad=(0, 0, 0, 0), int8_scale_term=1)
    got = run(d, x, w, np.array([1, 2, 3], np.float32), np.array([2, 4, 8], np.float32), 2.0, 1.0)
    assert got.dtype == np.float32
    for ch, v in enumerate([1.75, 2.375, 3.1875]):
        np.testing.assert_array_equal(got[0, ch], np.full((3, 3), v, np.float32))
    # requantized_convolution: int8 input 3 and 5, os 4, term 101 -> 8, 4, 2
    xi = np.stack([np.full((3, 3), 3), np.full((3, 3), 5)]).astype(np.int8)[None]
    d = nhip.conv_desc(2, 3, (1, 1), pad=(0, 0, 0, 0), bias=False, int8_scale_term=101)
    got = run(d, xi, w, None, np.array([2, 4, 8], np.float32), 2.0, 4.0)
    np.testing.assert_array_equal(got[0, :, 0, 0], [8, 4, 2])
    got = run(d, -xi, w, None, np.array([2, 4, 8], np.float32), 2.0, 4.0)
    np.testing.assert_array_equal(got[0, :, 0, 0], [-8, -4, -2])


def test_fixture_generator_weights_known_answer():
    # generate_int8_bins.py:20-28 closed-form weights, convolution_int8_term101
    w = np.array([((i * 7 + 3) % 15) - 7 for i in range(6)], np.int8).reshape(3, 2, 1, 1)
    b = np.array([-0.125, 0.0, 0.125], np.float32)
    ws = np.array([5.0, 6.5, 8.0], np.float32)
    x = np.array([0.25, -0.5], np.float32).reshape(1, 2, 1, 1)
    d = nhip.conv_desc(2, 3, (1, 1), pad=(0, 0, 0, 0), int8_scale_term=101)
    got = run(d, x, w, b, ws, 8.0, 6.0)
    np.testing.assert_array_equal(got[0, :, 0, 0], [-4, -2, -1])


CASES = [
    # (n, c, h, w, k, kernel, stride, dil, pad, term, act, weight fp32?, scalar ws?)
    (2, 3, 11, 9, 70, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1), 101, 1, False, False),
    (1, 40, 14, 14, 64, (1, 1), (1, 1), (1, 1), (0, 0, 0, 0), 101, 0, True, False),
    (2, 16, 15, 13, 20, (3, 3), (2, 2), (1, 1), (1, 1, 1, 1), 1, 1, True, True),
    (1, 24, 12, 12, 130, (3, 3), (1, 1), (2, 2), (2, 2, 2, 2), 2, 0, False, True),
    (3, 33, 8, 10, 48, (2, 3), (1, 2), (1, 1), (0, 1, 2, 0), 102, 1, True, False),
    # footprint windows: unused last column, two right halo columns, 6 + 1 output rows
    (2, 32, 16, 16, 40, (3, 3), (2, 2), (1, 1), (0, 0, 0, 0), 101, 1, False, False),
    (1, 64, 8, 12, 64, (3, 3), (1, 1), (1, 1), (1, 2, 1, 2), 1, 0, True, True),
    (2, 96, 7, 20, 32, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1), 102, 1, False, True),
    # 260 output channels: five 64-channel blocks of the footprint kernel
    (1, 32, 9, 14, 260, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1), 101, 1, False, False),
    # 5x5 taps over 64 channels: K stages cross taps, K padding past the 25th
    (1, 64, 9, 11, 24, (5, 5), (1, 1), (1, 1), (2, 2, 2, 2), 101, 1, False, False),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c[:5])) + f"-t{c[9]}")
@pytest.mark.parametrize("footprint", ["1", "0"])
def test_int8_shapes_bit_exact(case, footprint, nhip_env):
    """footprint: the whole-row footprint kernel where the shape allows it
    (NHIP_INT8_FOOTPRINT=1, default) or the im2col-gather kernel (=0)."""
    nhip_env.setenv("NHIP_INT8_FOOTPRINT", footprint)
    n, c, h, w, k, ker, st, dl, pad, term, act, wf32, scalar = case
    rng = np.random.default_rng(hash(case) % (2 ** 32))
    x = rng.uniform(-1.5, 1.5, (n, c, h, w)).astype(np.float32)
    ws = np.float32(rng.uniform(20, 200)) * np.ones(1 if scalar else k, np.float32)
    if not scalar:
        ws = rng.uniform(20, 200, k).astype(np.float32)
    wfloat = rng.uniform(-0.6, 0.6, (k, c) + ker).astype(np.float32)
    # oracle takes the already-quantized int8 weights
    ws_full = np.broadcast_to(ws, (k,)) if ws.size == 1 else ws
    w_i8 = np.stack([refcpu.quantize_f32_i8(wfloat[o], ws_full[o:o + 1]) for o in range(k)])
    b = rng.normal(0, 0.3, k).astype(np.float32)
    is_, os_ = 60.0, 25.0
    d = nhip.conv_desc(c, k, ker, st, dl, pad, act=act, int8_scale_term=term)
    got = run(d, x, wfloat if wf32 else w_i8, b, ws, is_, os_)
    exp = oracle(d, x, w_i8, b, ws, is_, os_)
    assert got.dtype == exp.dtype
    np.testing.assert_array_equal(got, exp)


RW_CASES = [
    # Reductions of exactly 1152 bytes (the register-weight kernel's):
    # (n, c, h, w, k, kernel, stride, dil, pad, term, act, scalar ws?)
    (2, 128, 28, 28, 128, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1), 101, 1, False),  # the benchmarked int8 conv at batch 2
    # 100 of 128 channels, 11 columns (byte stores), fp32 output
    (1, 120, 13, 11, 100, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1), 1, 0, False),
    # two channel blocks, stride 2, asymmetric padding, scalar scale
    (2, 128, 15, 17, 256, (3, 3), (2, 2), (1, 1), (0, 1, 1, 0), 102, 1, True),
    # 250 of 256 channels, dilation 2, 40 columns (3 or 1 rows per workgroup)
    (1, 113, 10, 40, 250, (3, 3), (1, 1), (2, 2), (2, 2, 2, 2), 2, 1, True),
    # a 1x1 convolution over 1152 channels: every k step inside one tap
    (1, 1152, 5, 5, 128, (1, 1), (1, 1), (1, 1), (0, 0, 0, 0), 101, 0, False),
    # 7x7 planes: 49 pixels per workgroup, byte stores of int8 results
    (3, 128, 7, 7, 128, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1), 101, 0, False),
    # 32 columns: four whole 32-pixel blocks per wave
    (1, 128, 9, 32, 128, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1), 1, 1, False),
    # no padding: the window's columns are exactly the image's
    (2, 128, 28, 28, 128, (3, 3), (1, 1), (1, 1), (0, 0, 0, 0), 1, 0, False),
    # 124 of 128 window channels filled (4-channel groups), 16 columns
    (1, 124, 12, 16, 128, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1), 101, 1, True),
]


@pytest.mark.parametrize("case", RW_CASES, ids=lambda c: "x".join(map(str, c[:5])) + f"-t{c[9]}")
@pytest.mark.parametrize("rw", ["1", "1k", "1q", "2", "0"])
def test_int8_register_weight_kernel_bit_exact(case, rw, nhip_env):
    """The register-weight kernel (NHIP_INT8_RW=1, default: four 32-pixel
    blocks per wave, with the input quantized inside its window fill where
    the shape allows (fp32 input, width and channels multiples of 4), then
    eight waves splitting the reduction in two halves; "1k": the fused fill
    on four waves with the whole reduction each (NHIP_INT8_KSPLIT=1); "1q":
    the fusion off, a separate quantize pass first; =2: two blocks per wave)
    against the oracle, bit for bit, and with it off (=0: the footprint
    kernel)."""
    nhip_env.setenv("NHIP_INT8_FUSED_QUANT", "0" if rw == "1q" else "1")
    nhip_env.setenv("NHIP_INT8_KSPLIT", "1" if rw == "1k" else "2")
    rw = rw[0]
    nhip_env.setenv("NHIP_INT8_RW", rw)
    n, c, h, w, k, ker, st, dl, pad, term, act, scalar = case
    rng = np.random.default_rng(hash(case) % (2 ** 32))
    x = rng.uniform(-1.5, 1.5, (n, c, h, w)).astype(np.float32)
    ws = (np.float32(rng.uniform(20, 200)) * np.ones(1, np.float32) if scalar
          else rng.uniform(20, 200, k).astype(np.float32))
    ws_full = np.broadcast_to(ws, (k,)) if ws.size == 1 else ws
    wfloat = rng.uniform(-0.6, 0.6, (k, c) + ker).astype(np.float32)
    w_i8 = np.stack([refcpu.quantize_f32_i8(wfloat[o], ws_full[o:o + 1]) for o in range(k)])
    b = rng.normal(0, 0.3, k).astype(np.float32)
    is_, os_ = 60.0, 25.0 / np.sqrt(c * ker[0] * ker[1] / 128.0)
    d = nhip.conv_desc(c, k, ker, st, dl, pad, act=act, int8_scale_term=term)
    conv = nhip.Conv2dInt8(d, w_i8, b, ws, is_, os_)
    xd = dev(x)
    exp = oracle(d, x, w_i8, b, ws, is_, os_)
    # where the fused window fill takes the shape (4 output rows' window of
    # at most 6 x 256 items of 4 channels x 4 pixels, covering every column)
    oh = (h + pad[0] + pad[1] - dl[0] * (ker[0] - 1) - 1) // st[0] + 1
    ow = (w + pad[2] + pad[3] - dl[1] * (ker[1] - 1) - 1) // st[1] + 1
    rows = min(128 // ow, oh)
    fh = (rows - 1) * st[0] + (ker[0] - 1) * dl[0] + 1
    fw = (ow - 1) * st[1] + (ker[1] - 1) * dl[1] + 1
    fused = (rw == "1" and w % 4 == 0 and c % 4 == 0 and pad[2] + w <= fw
             and (c // 4) * fh * (w // 4) <= 6 * 256 and os.environ["NHIP_INT8_FUSED_QUANT"] == "1")
    for rep in range(2):  # the second call reuses the plan and the workspace
        nhip.timer_start("conv_int8_rw_fq")
        got = host(conv.forward(xd))
        assert nhip.timer_stop()[0] == (1 if fused else 0)
        assert got.dtype == exp.dtype
        np.testing.assert_array_equal(got, exp, err_msg=f"call {rep}")
    if term > 100:  # not degenerate: many levels, not all saturated
        assert len(np.unique(got)) > 32


def test_rounding_ties_and_saturation_on_device():
    # x*is lands exactly on .5 and on the 0.49999997 trap; acc passes through
    # a 1x1 identity so the output requantize sees the same values.
    vals = np.array([0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 0.49999997, -0.49999997,
                     126.5, -126.5, 127.5, -127.5, 1e6, -1e6, 0.0, 3.0], np.float32)
    x = vals.reshape(1, 1, 4, 4)
    w = np.ones((1, 1, 1, 1), np.int8)
    d = nhip.conv_desc(1, 1, (1, 1), pad=(0, 0, 0, 0), bias=False, int8_scale_term=101)
    got = run(d, x, w, None, np.ones(1, np.float32), 1.0, 1.0)
    exp = oracle(d, x, w, None, np.ones(1, np.float32), 1.0, 1.0)
    np.testing.assert_array_equal(got, exp)
    np.testing.assert_array_equal(got.ravel()[:8], [1, -1, 2, -2, 3, -3, 1, -1])
    np.testing.assert_array_equal(got.ravel()[8:14], [127, -127, 127, -127, 127, -127])


def test_zero_weight_scale_selects_zero():
    x = np.ones((1, 2, 3, 3), np.float32)
    w = np.ones((2, 2, 1, 1), np.int8)
    d = nhip.conv_desc(2, 2, (1, 1), pad=(0, 0, 0, 0), int8_scale_term=1)
    got = run(d, x, w, np.array([0.5, 0.25], np.float32), np.array([0.0, 2.0], np.float32), 1.0, 1.0)
    np.testing.assert_array_equal(got[0, 0], np.full((3, 3), 0.5, np.float32))
    np.testing.assert_array_equal(got[0, 1], np.full((3, 3), 2 * 0.5 + 0.25, np.float32))


# ---- int8 ConvolutionDepthWise (NCNNToTosa.cpp:3257-3376) ----
DW_CASES = [
    # (n, c, h, w, kernel, stride, dil, pad, term, act, fp32 weights?, int8 input?)
    (2, 32, 28, 28, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1), 101, 1, False, False),
    (2, 96, 28, 28, (3, 3), (2, 2), (1, 1), (1, 1, 1, 1), 1, 1, True, False),
    (1, 24, 13, 17, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1), 2, 0, False, True),
    (3, 8, 11, 9, (5, 5), (2, 1), (2, 1), (3, 1, 0, 2), 102, 0, True, True),
    (1, 960, 7, 7, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1), 101, 1, False, False),
]


@pytest.mark.parametrize("case", DW_CASES, ids=lambda c: "x".join(map(str, c[:4])) + f"-t{c[8]}")
def test_int8_depthwise_bit_exact(case):
    n, c, h, w, ker, st, dl, pad, term, act, wf32, in_i8 = case
    rng = np.random.default_rng(hash(case) % (2 ** 32))
    x = (rng.integers(-127, 128, (n, c, h, w)).astype(np.int8) if in_i8
         else rng.uniform(-1.5, 1.5, (n, c, h, w)).astype(np.float32))
    scalar = term in (2, 102)
    ws = rng.uniform(20, 200, 1 if scalar else c).astype(np.float32)
    wfloat = rng.uniform(-0.6, 0.6, (c, 1) + ker).astype(np.float32)
    ws_full = np.broadcast_to(ws, (c,))
    w_i8 = np.stack([refcpu.quantize_f32_i8(wfloat[o], ws_full[o:o + 1]) for o in range(c)])
    b = rng.normal(0, 0.3, c).astype(np.float32)
    d = nhip.conv_desc(c, c, ker, st, dl, pad, act=act, int8_scale_term=term, group=c)
    conv = nhip.DwConv2dInt8(d, wfloat if wf32 else w_i8, b, ws, 60.0, 25.0)
    got = host(conv.forward(dev(x)))
    g = refcpu.geom(n, c, h, w, c, ker, st, dl, pad)
    exp = refcpu.dwconv2d_int8(g, x, w_i8, b, ws, 60.0, 25.0, term, act)
    assert got.dtype == exp.dtype
    np.testing.assert_array_equal(got, exp)


def test_int8_depthwise_fixture_known_answer_on_device():
    w = np.array([-4, 1, -5], np.int8).reshape(3, 1, 1, 1)
    b = np.array([-0.1, 0.0, 0.1], np.float32)
    x = np.array([0.5, -0.25, 1.0], np.float32).reshape(1, 3, 1, 1)
    d = nhip.conv_desc(3, 3, (1, 1), pad=(0, 0, 0, 0), int8_scale_term=101, group=3)
    got = host(nhip.DwConv2dInt8(d, w, b, np.array([4.0, 5.0, 6.0], np.float32), 7.0, 5.0).forward(dev(x)))
    np.testing.assert_array_equal(got[0, :, 0, 0], [-3, 0, -4])


# ---- int8 InnerProduct (NCNNToTosa.cpp:5300-5390) ----
@pytest.mark.parametrize("m,k,n,act,wf32,in_i8", [
    (1, 4, 3, 0, False, False), (256, 2048, 1000, 0, False, False), (7, 130, 65, 1, True, False),
    (33, 1280, 1000, 1, False, True), (2, 17, 5, 0, True, True)])
def test_int8_innerproduct_bit_exact(m, k, n, act, wf32, in_i8):
    rng = np.random.default_rng(m * 1000 + k + n)
    x = rng.integers(-127, 128, (m, k)).astype(np.int8) if in_i8 else rng.uniform(-1.5, 1.5, (m, k)).astype(np.float32)
    ws = rng.uniform(20, 200, n).astype(np.float32)
    wfloat = rng.uniform(-0.6, 0.6, (n, k)).astype(np.float32)
    w_i8 = np.stack([refcpu.quantize_f32_i8(wfloat[j], ws[j:j + 1]) for j in range(n)])
    b = rng.normal(0, 0.3, n).astype(np.float32)
    ip = nhip.InnerProductInt8(wfloat if wf32 else w_i8, b, ws, 60.0, act)
    got = host(ip.forward(dev(x)))
    exp = refcpu.innerproduct_int8(x, w_i8, b, ws, 60.0, act)
    np.testing.assert_array_equal(got, exp)


def test_int8_innerproduct_fixture_known_answer_on_device():
    w = np.array([3, -2, 1, 4, -4, 2, 5, -1, 2, 3, -3, 1], np.int8).reshape(3, 4)
    ip = nhip.InnerProductInt8(w, np.array([0.25, -0.5, 0.125], np.float32), np.array([4.0, 6.0, 8.0], np.float32), 9.0)
    got = host(ip.forward(dev(np.array([[1.0, 0.5, -1.0, 0.25]], np.float32))))
    exp = np.array([16 / 36 + 0.25, -73 / 54 - 0.5, 62 / 72 + 0.125], np.float32)
    np.testing.assert_allclose(got[0], exp, rtol=1e-6)
