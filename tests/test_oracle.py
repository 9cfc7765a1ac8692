"""Pins the CPU oracle (oracle/refcpu.c) before anything is checked against it.

Each check is independent of the oracle's own code: a float64 textbook
convolution / matmul, brute-force integer sums, hand-computed known answers
taken from the reference's lit tests and fixture generators, and special cases
that make the plausible mistakes (roundf instead of floor(x+0.5), half-even
rounding, a +-128 clamp, (acc+bias)*s instead of acc*s+bias, dropped bias,
transposed weights, wrong pad side) fail.
"""
import numpy as np
import pytest

from oracle import refcpu


def conv_f64(x, w, b, stride=(1, 1), dil=(1, 1), pad=(1, 1, 1, 1), groups=1):
    """Textbook cross-correlation in float64 (NCHW, OIHW), zero padding."""
    x = x.astype(np.float64)
    w = w.astype(np.float64)
    n, c, h, wd = x.shape
    k, cg, kh, kw = w.shape
    pt, pb, pl, pr = pad
    xp = np.zeros((n, c, h + pt + pb, wd + pl + pr))
    xp[:, :, pt:pt + h, pl:pl + wd] = x
    oh = (h + pt + pb - ((kh - 1) * dil[0] + 1)) // stride[0] + 1
    ow = (wd + pl + pr - ((kw - 1) * dil[1] + 1)) // stride[1] + 1
    out = np.zeros((n, k, oh, ow))
    kpg = k // groups
    for g in range(groups):
        xs = xp[:, g * cg:(g + 1) * cg]
        ws = w[g * kpg:(g + 1) * kpg]
        for i in range(kh):
            for j in range(kw):
                y0, x0 = i * dil[0], j * dil[1]
                patch = xs[:, :, y0:y0 + stride[0] * (oh - 1) + 1:stride[0],
                           x0:x0 + stride[1] * (ow - 1) + 1:stride[1]]
                out[:, g * kpg:(g + 1) * kpg] += np.einsum(
                    "nchw,kc->nkhw", patch, ws[:, :, i, j])
    if b is not None:
        out += b.astype(np.float64)[None, :, None, None]
    return out


def assert_close(actual, expected, rtol, what=""):
    """|a - e| <= rtol*|e| + rtol*rms(e)  (reference comparator form,
    numerical_test_support.cpp:701-770, with atol scaled to the data)."""
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    atol = rtol * max(float(np.sqrt(np.mean(expected ** 2))), 1e-30)
    err = np.abs(actual - expected)
    bad = err > rtol * np.abs(expected) + atol
    assert not bad.any(), (
        f"{what}: {bad.sum()} of {bad.size} outside tolerance; max err "
        f"{err.max():.3e}, max |e| {np.abs(expected).max():.3e}")


RNG = np.random.default_rng(1234)

CONV_CASES = [
    # (n, c, h, w, k, kernel, stride, dilation, pad)  - fixture shapes of
    # test/Numerical/fixtures/convolution*.param plus config shapes
    (1, 1, 4, 4, 2, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1)),
    (2, 3, 7, 6, 5, (3, 3), (2, 2), (1, 1), (1, 1, 1, 1)),
    (1, 4, 9, 8, 3, (3, 3), (1, 1), (2, 2), (2, 2, 2, 2)),
    (1, 2, 6, 7, 3, (2, 3), (1, 2), (1, 1), (0, 1, 2, 0)),
    (2, 8, 5, 5, 4, (1, 1), (1, 1), (1, 1), (0, 0, 0, 0)),
    (1, 3, 11, 11, 8, (3, 3), (2, 2), (1, 1), (1, 1, 1, 1)),
]


@pytest.mark.parametrize("case", CONV_CASES)
def test_conv_f32_matches_float64_textbook(case):
    n, c, h, w, k, ker, st, dl, pad = case
    x = RNG.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = RNG.normal(0, 0.3, (k, c) + ker).astype(np.float32)
    b = RNG.normal(0, 0.1, k).astype(np.float32)
    g = refcpu.geom(n, c, h, w, k, ker, st, dl, pad)
    out = refcpu.conv2d_f32(g, x, wt, b)
    exp = conv_f64(x, wt, b, st, dl, pad)
    assert out.shape == exp.shape
    assert_close(out, exp, 1e-6, "conv")


def test_conv_delta_input_reproduces_kernel():
    # one-hot input at (c, y, x) -> out[k, y-kh+1, x-kw+1] = w[k, c, kh, kw] + b
    c, k = 3, 2
    x = np.zeros((1, c, 5, 5), np.float32)
    x[0, 1, 2, 2] = 1.0
    wt = np.arange(k * c * 9, dtype=np.float32).reshape(k, c, 3, 3)
    b = np.array([0.5, -0.25], np.float32)
    out = refcpu.conv2d_f32(refcpu.geom(1, c, 5, 5, k), x, wt, b)
    for kk in range(k):
        window = out[0, kk, 1:4, 1:4] - b[kk]
        # correlation: out[y, x] picks w[kh, kw] with y + kh - 1 = 2
        np.testing.assert_array_equal(window, wt[kk, 1, ::-1, ::-1])


def test_conv_zero_pad_border_and_bias_only():
    x = np.zeros((1, 2, 4, 4), np.float32)
    wt = RNG.normal(size=(3, 2, 3, 3)).astype(np.float32)
    b = np.array([1.0, -2.0, 0.5], np.float32)
    out = refcpu.conv2d_f32(refcpu.geom(1, 2, 4, 4, 3), x, wt, b)
    np.testing.assert_array_equal(out, np.broadcast_to(b[None, :, None, None], out.shape))


def test_conv_1x1_equals_gemm_and_is_linear():
    n, c, h, w, k = 2, 16, 5, 6, 8
    x = RNG.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = RNG.normal(size=(k, c, 1, 1)).astype(np.float32)
    g = refcpu.geom(n, c, h, w, k, (1, 1), pad=(0, 0, 0, 0))
    out = refcpu.conv2d_f32(g, x, wt)
    gemm = np.einsum("kc,nchw->nkhw", wt[:, :, 0, 0].astype(np.float64), x)
    assert_close(out, gemm, 1e-6, "1x1")
    out2 = refcpu.conv2d_f32(g, 2.0 * x, wt)  # exact power-of-two scaling
    np.testing.assert_array_equal(out2, 2.0 * out)


def test_conv_asymmetric_padding_side():
    # pad only on the left: first output column sees the zero column
    x = np.ones((1, 1, 1, 3), np.float32)
    wt = np.array([[[[1.0, 10.0, 100.0]]]], np.float32)
    g = refcpu.geom(1, 1, 1, 3, 1, (1, 3), pad=(0, 0, 1, 0))
    out = refcpu.conv2d_f32(g, x, wt)
    np.testing.assert_array_equal(out[0, 0, 0], [110.0, 111.0])


def test_bias_added_once_and_order_is_bias_first():
    # bias-initialised accumulation (tosa.conv2d bias init):
    # ((1 + 1e8) + -1e8) = 0 in fp32; a zero-init sum with the bias added
    # last, ((0 + 1e8) + -1e8) + 1, would give 1.
    x = np.array([1.0, 1.0], np.float32).reshape(1, 2, 1, 1)
    wt = np.array([1e8, -1e8], np.float32).reshape(1, 2, 1, 1)
    b = np.array([1.0], np.float32)
    g = refcpu.geom(1, 2, 1, 1, 1, (1, 1), pad=(0, 0, 0, 0))
    out = refcpu.conv2d_f32(g, x, wt, b)
    assert out[0, 0, 0, 0] == 0.0


@pytest.mark.parametrize("mult", [1, 2])
@pytest.mark.parametrize("stride", [1, 2])
def test_depthwise_matches_float64_textbook(mult, stride):
    n, c, h, w = 2, 6, 9, 10
    k = c * mult
    x = RNG.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = RNG.normal(size=(k, 1, 3, 3)).astype(np.float32)
    b = RNG.normal(0, 0.1, k).astype(np.float32)
    g = refcpu.geom(n, c, h, w, k, (3, 3), (stride, stride))
    out = refcpu.dwconv2d_f32(g, x, wt, b)
    # grouped textbook conv: group g owns input channel g, outputs g*mult..
    exp = conv_f64(x, wt, b, (stride, stride), groups=c)
    assert_close(out, exp, 1e-6, "dw")


def test_depthwise_bias_added_after_sum():
    # zero-init then bias add: (1e8 + -1e8) + 1 = 1 (bias-first would give 0)
    wt = np.array([1e8, -1e8], np.float32).reshape(1, 1, 1, 2)
    x = np.ones((1, 1, 1, 2), np.float32)
    b = np.array([1.0], np.float32)
    g = refcpu.geom(1, 1, 1, 2, 1, (1, 2), pad=(0, 0, 0, 0))
    out = refcpu.dwconv2d_f32(g, x, wt, b)
    assert out[0, 0, 0, 0] == 1.0


def test_innerproduct_matches_float64_and_bias_last():
    m, k, n = 7, 33, 5
    x = RNG.uniform(-1, 1, (m, k)).astype(np.float32)
    wt = RNG.normal(size=(n, k)).astype(np.float32)
    b = RNG.normal(size=n).astype(np.float32)
    out = refcpu.innerproduct_f32(x, wt, b)
    exp = x.astype(np.float64) @ wt.T.astype(np.float64) + b
    assert_close(out, exp, 1e-6, "ip")
    # weight is [N][K] (not [K][N]): a transposed read would fail this
    x1 = np.zeros((1, 3), np.float32)
    x1[0, 2] = 1.0
    w1 = np.arange(6, dtype=np.float32).reshape(2, 3)
    np.testing.assert_array_equal(refcpu.innerproduct_f32(x1, w1), [[2.0, 5.0]])
    # zero-init matmul then bias: (1e8 - 1e8) + 1 = 1
    xb = np.ones((1, 2), np.float32)
    wb = np.array([[1e8, -1e8]], np.float32)
    assert refcpu.innerproduct_f32(xb, wb, np.array([1.0], np.float32))[0, 0] == 1.0


# ---- int8 quantization (NCNNToTosa.cpp:322-389) ----

def test_quantize_round_half_away_and_saturate():
    q = refcpu.quantize_one
    assert q(0.5, 1.0) == 1 and q(-0.5, 1.0) == -1
    assert q(2.5, 1.0) == 3 and q(-2.5, 1.0) == -3      # half-even would give 2
    assert q(1.4999999, 1.0) == 1
    assert q(126.5, 1.0) == 127 and q(-126.5, 1.0) == -127
    assert q(127.5, 1.0) == 127 and q(-127.5, 1.0) == -127  # no -128
    assert q(1e10, 1.0) == 127 and q(-1e10, 1.0) == -127
    assert q(0.0, 1.0) == 0 and q(-0.0, 1.0) == 0
    assert q(3.0, 0.5) == 2 and q(-3.0, 0.5) == -2   # 1.5 -> 2, -1.5 -> -2


def test_quantize_floor_x_plus_half_is_not_roundf():
    # 0.49999997f + 0.5f rounds to 1.0f in fp32, so floor(x+0.5) gives 1,
    # while roundf(0.49999997) = 0.  The reference uses floor/ceil.
    x = np.float32(0.49999997)
    assert np.float32(x + np.float32(0.5)) == np.float32(1.0)
    assert refcpu.quantize_one(float(x), 1.0) == 1
    assert refcpu.quantize_one(-float(x), 1.0) == -1


def test_quantize_per_channel_scale():
    x = np.array([[1.0, 2.0], [1.0, 2.0]], np.float32)
    out = refcpu.quantize_f32_i8(x, np.array([10.0, 100.0], np.float32), channel_size=2)
    np.testing.assert_array_equal(out, [[10, 20], [100, 127]])


def test_dequant_reciprocal_zero_weight_scale_selects_zero():
    r = refcpu.dequant_reciprocal(np.array([2.0, 0.0, 8.0], np.float32), 2.0)
    np.testing.assert_array_equal(r, [0.25, 0.0, 0.0625])


def _conv_i8_case(n, c, h, w, k, seed):
    rng = np.random.default_rng(seed)
    x = rng.integers(-127, 128, (n, c, h, w)).astype(np.int8)
    wt = rng.integers(-127, 128, (k, c, 3, 3)).astype(np.int8)
    return x, wt


def test_int8_accumulator_matches_bruteforce_int64():
    x, wt = _conv_i8_case(2, 5, 6, 7, 4, 7)
    g = refcpu.geom(2, 5, 6, 7, 4)
    acc = refcpu.conv2d_i8_acc(g, x, wt)
    exp = np.rint(conv_f64(x.astype(np.float64), wt.astype(np.float64), None)).astype(np.int64)
    np.testing.assert_array_equal(acc, exp)


def test_int8_conv_known_answer_quantized_contractions_case1():
    # test/Conversion/NCNNToTosa/quantized-contractions.mlir:3-8:
    # weight all ones [3,2,1,1], bias [1,2,3], ws [2,4,8], is 2, term 1.
    # x ch0 = 1.0 -> q 2; ch1 = 0.25 -> q round(0.5) = 1; acc = 3.
    # out[c] = 3 * (1/(ws[c]*2)) + bias[c] = 1.75, 2.375, 3.1875 (all exact).
    x = np.stack([np.full((3, 3), 1.0), np.full((3, 3), 0.25)]).astype(np.float32)[None]
    wt = np.ones((3, 2, 1, 1), np.int8)
    g = refcpu.geom(1, 2, 3, 3, 3, (1, 1), pad=(0, 0, 0, 0))
    out = refcpu.conv2d_int8(g, x, wt, np.array([1.0, 2.0, 3.0], np.float32),
                             np.array([2.0, 4.0, 8.0], np.float32), 2.0,
                             scale_term=1, activation=0)
    assert out.dtype == np.float32
    for ch, v in enumerate([1.75, 2.375, 3.1875]):
        np.testing.assert_array_equal(out[0, ch], np.full((3, 3), v, np.float32))
    # (acc + bias) * r would give 1.0, 1.25, 1.125: the order matters.


def test_int8_conv_known_answer_quantized_contractions_case2():
    # quantized-contractions.mlir requantized_convolution: int8 input,
    # weight ones, ws [2,4,8], is 2, os 4, term 101, no bias.
    # acc = 3 + 5 = 8 -> f = 8/(ws*2) = 2, 1, 0.5 -> *4 = 8, 4, 2.
    x = np.stack([np.full((3, 3), 3), np.full((3, 3), 5)]).astype(np.int8)[None]
    wt = np.ones((3, 2, 1, 1), np.int8)
    g = refcpu.geom(1, 2, 3, 3, 3, (1, 1), pad=(0, 0, 0, 0))
    args = (None, np.array([2.0, 4.0, 8.0], np.float32), 2.0, 4.0)
    out = refcpu.conv2d_int8(g, x, wt, *args, scale_term=101, activation=0)
    assert out.dtype == np.int8
    np.testing.assert_array_equal(out[0, :, 0, 0], [8, 4, 2])
    neg = refcpu.conv2d_int8(g, -x, wt, *args, scale_term=101, activation=0)
    np.testing.assert_array_equal(neg[0, :, 0, 0], [-8, -4, -2])
    relu = refcpu.conv2d_int8(g, -x, wt, *args, scale_term=101, activation=1)
    np.testing.assert_array_equal(relu[0, :, 0, 0], [0, 0, 0])


def int8_fixture_conv_weights(inputs, outputs):
    """Closed-form weights of test/Numerical/fixtures/generate_int8_bins.py:20-28."""
    w = np.array([((i * 7 + 3) % 15) - 7 for i in range(inputs * outputs)], np.int8)
    bias = np.array([0.125 * (i - 1) for i in range(outputs)], np.float32)
    ws = np.array([5.0 + i * 1.5 for i in range(outputs)], np.float32)
    return w.reshape(outputs, inputs, 1, 1), bias, ws, 8.0, 6.0


def test_int8_conv_known_answer_fixture_generator_weights():
    # convolution_int8_term101 layer 1: 2->3 1x1, is 8, os 6, weights
    # [[-4,3],[-5,2],[-6,1]], bias [-0.125,0,0.125], ws [5,6.5,8].
    w, b, ws, is_, os_ = int8_fixture_conv_weights(2, 3)
    np.testing.assert_array_equal(w[:, :, 0, 0], [[-4, 3], [-5, 2], [-6, 1]])
    # x = (0.25, -0.5): q = (2, -4): acc = (-20, -18, -16)
    x = np.array([0.25, -0.5], np.float32).reshape(1, 2, 1, 1)
    g = refcpu.geom(1, 2, 1, 1, 3, (1, 1), pad=(0, 0, 0, 0))
    f = refcpu.conv2d_int8(g, x, w, b, ws, is_, scale_term=1, activation=0)[0, :, 0, 0]
    # -20/40 - 0.125 = -0.625 ; -18/52 + 0 ; -16/64 + 0.125 = -0.125
    assert abs(f[0] - (-0.625)) < 1e-7
    assert abs(f[1] - (-18.0 / 52.0)) < 1e-7
    assert abs(f[2] - (-0.125)) < 1e-7
    q = refcpu.conv2d_int8(g, x, w, b, ws, is_, os_, scale_term=101, activation=0)
    # *6: -3.75 -> -4 ; -2.0769 -> -2 ; -0.75 -> -1
    np.testing.assert_array_equal(q[0, :, 0, 0], [-4, -2, -1])


def test_requantize_and_dequantize_known_answers():
    acc = np.array([[10, -10], [3, 7]], np.int32)
    # ch0: 10*0.5+1 = 6 -> *2 = 12 ; -10*0.5+1 = -4 -> relu 0
    # ch1: 3*0.25-1 = -0.25 -> 0 (relu) ; 7*0.25-1 = 0.75 -> *2 = 1.5 -> 2
    out = refcpu.requantize_i32_i8(acc, np.array([0.5, 0.25]), 2.0,
                                   bias=np.array([1.0, -1.0]), activation=1)
    np.testing.assert_array_equal(out, [[12, 0], [0, 2]])
    deq = refcpu.dequantize_i32_f32(acc, np.array([0.5, 0.25]), bias=np.array([1.0, -1.0]))
    np.testing.assert_array_equal(deq, [[6.0, -4.0], [-0.25, 0.75]])


def test_relu_add_avgpool():
    x = np.array([-1.5, 0.0, 2.0], np.float32)
    np.testing.assert_array_equal(refcpu.relu_f32(x), [0.0, 0.0, 2.0])
    np.testing.assert_array_equal(refcpu.relu_i8(np.array([-127, 0, 5], np.int8)), [0, 0, 5])
    np.testing.assert_array_equal(refcpu.add_f32(x, x), 2 * x)
    p = RNG.uniform(-1, 1, (2, 3, 7, 7)).astype(np.float32)
    assert_close(refcpu.global_avgpool_f32(p), p.astype(np.float64).mean(axis=(2, 3)), 1e-6, "gap")
    q = np.arange(16, dtype=np.float32).reshape(1, 1, 4, 4)
    assert refcpu.global_avgpool_f32(q)[0, 0] == 7.5


def test_bn_fold_matches_float64_and_zero_variance_rule():
    k, per = 4, 18
    w = RNG.normal(size=(k, 2, 3, 3)).astype(np.float32)
    b = RNG.normal(size=k).astype(np.float32)
    slope = RNG.uniform(0.5, 2, k).astype(np.float32)
    mean = RNG.normal(size=k).astype(np.float32)
    var = RNG.uniform(0.1, 2, k).astype(np.float32)
    beta = RNG.normal(size=k).astype(np.float32)
    fw, fb = refcpu.bn_fold(w, b, slope, mean, var, beta, 1e-5)
    scale = slope.astype(np.float64) / np.sqrt(var.astype(np.float64) + 1e-5)
    assert_close(fw, w * scale[:, None, None, None], 1e-6, "bnw")
    assert_close(fb, b * scale + (beta - scale * mean), 1e-6, "bnb")
    # var + eps == 0 -> inverse std 1e4 (FoldNCNNBatchNorm.cpp:113-114)
    fw0, fb0 = refcpu.bn_fold(np.ones((1, 1, 1, 1), np.float32), None,
                              np.ones(1), np.zeros(1), np.zeros(1), np.zeros(1), 0.0)
    assert fw0[0, 0, 0, 0] == 10000.0 and fb0[0] == 0.0
    # folded conv equals conv followed by the BN formula
    x = RNG.uniform(-1, 1, (1, 2, 5, 5)).astype(np.float32)
    g = refcpu.geom(1, 2, 5, 5, k)
    plain = conv_f64(x, w, b)
    bn = (plain - mean[None, :, None, None]) * scale[None, :, None, None] + beta[None, :, None, None]
    assert_close(refcpu.conv2d_f32(g, x, fw, fb), bn, 1e-5, "bn-conv")


def test_same_padding_upper_lower():
    # SAME: out = ceil(in/stride); extra pad goes after (upper) or before (lower)
    assert refcpu.same_padding(4, 3, 2, 1, -233) == (0, 1)
    assert refcpu.same_padding(4, 3, 2, 1, -234) == (1, 0)
    assert refcpu.same_padding(5, 3, 2, 1, -233) == (1, 1)
    assert refcpu.same_padding(7, 3, 1, 2, -233) == (2, 2)
    assert refcpu.same_padding(8, 1, 1, 1, -233) == (0, 0)


# ---- int8 depthwise / InnerProduct (NCNNToTosa.cpp:3257-3376, 5300-5390) ----

def test_int8_depthwise_known_answer_fixture_generator():
    # generate_int8_bins.py depthwise(101, 3): weights ((i*5+1)%11)-5 = [-4, 1, -5],
    # bias 0.1*(i-1), ws 4+i, is 7, os 5; 1x1 kernel.
    w = np.array([((i * 5 + 1) % 11) - 5 for i in range(3)], np.int8).reshape(3, 1, 1, 1)
    np.testing.assert_array_equal(w.ravel(), [-4, 1, -5])
    b = np.array([0.1 * (i - 1) for i in range(3)], np.float32)
    ws = np.array([4.0, 5.0, 6.0], np.float32)
    x = np.array([0.5, -0.25, 1.0], np.float32).reshape(1, 3, 1, 1)
    g = refcpu.geom(1, 3, 1, 1, 3, (1, 1), pad=(0, 0, 0, 0))
    f = refcpu.dwconv2d_int8(g, x, w, b, ws, 7.0, scale_term=1, activation=0)[0, :, 0, 0]
    # q = round(3.5)=4, round(-1.75)=-2, 7 ; acc = -16, -2, -35
    # f = -16/28 - 0.1 ; -2/35 + 0 ; -35/42 + 0.1
    np.testing.assert_allclose(f, [-16 / 28 - 0.1, -2 / 35, -35 / 42 + 0.1], rtol=1e-6)
    q = refcpu.dwconv2d_int8(g, x, w, b, ws, 7.0, 5.0, scale_term=101, activation=0)[0, :, 0, 0]
    # *5: -3.357 -> -3 ; -0.2857 -> 0 ; -3.6667 -> -4
    np.testing.assert_array_equal(q, [-3, 0, -4])
    relu = refcpu.dwconv2d_int8(g, x, w, b, ws, 7.0, 5.0, scale_term=101, activation=1)[0, :, 0, 0]
    np.testing.assert_array_equal(relu, [0, 0, 0])
    # scalar weight scale (terms 2 / 102): ws count 1 applies to every channel
    s = refcpu.dwconv2d_int8(g, x, w, b, np.array([4.0], np.float32), 7.0, scale_term=2, activation=0)[0, :, 0, 0]
    np.testing.assert_allclose(s, [-16 / 28 - 0.1, -2 / 28, -35 / 28 + 0.1], rtol=1e-6)


def test_int8_depthwise_accumulator_bruteforce():
    rng = np.random.default_rng(5)
    x = rng.integers(-127, 128, (2, 4, 7, 6)).astype(np.int8)
    w = rng.integers(-127, 128, (4, 1, 3, 3)).astype(np.int8)
    g = refcpu.geom(2, 4, 7, 6, 4, (3, 3), (2, 1))
    # ws = 1, is = 1 and a huge fp32 output keep the accumulator exact in fp32
    out = refcpu.dwconv2d_int8(g, x, w, None, np.ones(4, np.float32), 1.0, scale_term=1, activation=0)
    exp = conv_f64(x.astype(np.float64), w.astype(np.float64), None, (2, 1), groups=4)
    np.testing.assert_array_equal(out, exp.astype(np.float32))


def test_int8_innerproduct_known_answer_fixture_generator():
    # generate_int8_bins.py inner_product(): weights [3,-2,1,4 | -4,2,5,-1 | 2,3,-3,1],
    # bias [0.25,-0.5,0.125], ws [4,6,8], is 9
    w = np.array([3, -2, 1, 4, -4, 2, 5, -1, 2, 3, -3, 1], np.int8).reshape(3, 4)
    b = np.array([0.25, -0.5, 0.125], np.float32)
    ws = np.array([4.0, 6.0, 8.0], np.float32)
    x = np.array([[1.0, 0.5, -1.0, 0.25]], np.float32)
    out = refcpu.innerproduct_int8(x, w, b, ws, 9.0)
    # q = [9, round(4.5)=5, -9, round(2.25)=2]; acc = 27-10-9+8 = 16, -36+10-45-2 = -73, 18+15+27+2 = 62
    np.testing.assert_allclose(out[0], [16 / 36 + 0.25, -73 / 54 - 0.5, 62 / 72 + 0.125], rtol=1e-6)
    relu = refcpu.innerproduct_int8(x, w, b, ws, 9.0, activation=1)
    assert relu[0, 1] == 0.0 and relu[0, 0] == out[0, 0]
    rng = np.random.default_rng(6)
    xi = rng.integers(-127, 128, (5, 33)).astype(np.int8)
    wi = rng.integers(-127, 128, (7, 33)).astype(np.int8)
    acc = refcpu.innerproduct_int8(xi, wi, None, np.ones(7, np.float32), 1.0)
    np.testing.assert_array_equal(acc, (xi.astype(np.int64) @ wi.T.astype(np.int64)).astype(np.float32))
