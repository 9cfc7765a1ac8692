"""GPU parity: a 3x3 ConvolutionDepthWise feeding a 1x1 Convolution run as
one kernel (nhip_dwconv2d_pw_f32_forward, the graph executor's fusion of an
inverted-residual block's depthwise -> project pair).

The fused result must equal the two layers run separately bit for bit (the
depthwise values are formed in the same order, zero + x*w over (kh, kw) +
bias, then the same MFMA reduction), and the CPU oracle restating the
reference's ConvolutionDepthWise (NCNNToTosa.cpp:3376-3503) and Convolution
(NCNNToTosa.cpp:1316-1529) within 1e-4.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import ncnn_format  # noqa: E402
import nhip  # noqa: E402
import workloads  # noqa: E402
from numerics import assert_close  # noqa: E402
from oracle import refcpu  # noqa: E402

pytestmark = pytest.mark.gpu

RTOL = 1e-4
RNG = np.random.default_rng(5)
R, S, N0 = nhip.ACT_RELU, nhip.ACT_SIGMOID, nhip.ACT_NONE


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nhip.init(0)


@pytest.fixture(autouse=True)
def _every_pair(nhip_env):
    """NHIP_DWPW=2: fuse every pair the kernel can run; by default the library
    fuses only the stride-2 pairs with up to 32 output channels, where it
    measured faster than the two layers.  NHIP_CONV_KQ=0 keeps the separate
    1x1 layer on the pointwise GEMM kernel, whose reduction order the fused
    kernel shares (the split-reduction kernel that small 1x1 launches take
    sums in another order and has its own parity test)."""
    nhip_env.setenv("NHIP_DWPW", "2")
    nhip_env.setenv("NHIP_CONV_KQ", "0")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def make(c, k, stride, dw_act, pw_act):
    wd = workloads.he_normal(RNG, (c, 1, 3, 3), 9)
    bd = RNG.normal(0, 0.05, c).astype(np.float32)
    wp = workloads.he_normal(RNG, (k, c, 1, 1), c)
    bp = RNG.normal(0, 0.05, k).astype(np.float32)
    dw = nhip.DwConv2dF32(nhip.conv_desc(c, c, (3, 3), (stride, stride), (1, 1), (1, 1, 1, 1), act=dw_act, group=c),
                          wd, bd)
    pw = nhip.Conv2dF32(nhip.conv_desc(c, k, (1, 1), (1, 1), (1, 1), (0, 0, 0, 0), act=pw_act), wp, bp)
    return dw, pw, (wd, bd, wp, bp)


def oracle(x, stride, dw_act, pw_act, params, residual):
    wd, bd, wp, bp = params
    n, c, h, w = x.shape
    y = refcpu.dwconv2d_f32(refcpu.geom(n, c, h, w, c, (3, 3), (stride, stride), (1, 1), (1, 1, 1, 1)), x, wd, bd)
    if dw_act == R:
        y = refcpu.relu_f32(y)
    _, _, oh, ow = y.shape
    z = refcpu.conv2d_f32(refcpu.geom(n, c, oh, ow, wp.shape[0], (1, 1), (1, 1), (1, 1), (0, 0, 0, 0)), y, wp, bp)
    if residual is not None:
        z = refcpu.add_f32(z, residual)
    if pw_act == R:
        z = refcpu.relu_f32(z)
    elif pw_act == S:
        z = (1.0 / (1.0 + np.exp(-z.astype(np.float64)))).astype(np.float32)
    return z


def check_pair(n, c, h, w, k, stride, dw_act, pw_act, res, env=None, lds=False, images=None):
    """Fused launch against the two layers run separately (bit for bit) and
    the oracle (on `images`, default all).  lds: the LDS-staged kernel is
    expected to take the pair; the separate 1x1 layer then runs the
    streaming kernel's sequential configuration (NHIP_PW_CFG=1,1), whose
    per-output summation order that kernel shares."""
    dw, pw, params = make(c, k, stride, dw_act, pw_act)
    x = RNG.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    oh, ow = (h + 2 - 3) // stride + 1, (w + 2 - 3) // stride + 1
    r = RNG.uniform(-1, 1, (n, k, oh, ow)).astype(np.float32) if res else None
    assert nhip.dwconv_pw_supported(dw, pw, n, h, w)
    xd = dev(x)
    rd = dev(r) if res else None
    nhip.timer_start("dwpw")
    fused = host(nhip.dwconv_pw_forward(dw, pw, xd, residual=rd))
    assert nhip.timer_stop()[0] == 1
    nhip.timer_start("dwpw_lds")
    again = host(nhip.dwconv_pw_forward(dw, pw, xd, residual=rd))
    assert nhip.timer_stop()[0] == (1 if lds else 0)
    np.testing.assert_array_equal(again, fused)
    if lds:
        env.setenv("NHIP_PW_CFG", "1,1")
    separate = host(pw.forward(dw.forward(xd), residual=rd))
    if lds:
        env.delenv("NHIP_PW_CFG")
    np.testing.assert_array_equal(fused, separate)
    sel = slice(None) if images is None else images
    exp = oracle(x[sel], stride, dw_act, pw_act, params, r[sel] if res else None)
    assert_close(fused[sel], exp, RTOL, f"dw+pw {(n, c, h, w, k, stride)}")


CASES = [
    # (n, c, h, w, k, stride, dw_act, pw_act, residual)
    (2, 32, 16, 16, 16, 1, R, N0, False),
    (2, 96, 16, 16, 24, 2, R, N0, False),
    (2, 144, 12, 12, 24, 1, R, N0, True),
    (1, 20, 8, 12, 33, 1, N0, R, True),        # 5 chunks of 4 channels, K = 33
    (3, 48, 8, 8, 40, 2, R, S, False),         # 4-wide output rows
    (2, 64, 28, 28, 32, 1, R, N0, True),
    (1, 30, 4, 4, 7, 1, R, R, False),          # C % 4 != 0, a single output row of 4
    (2, 144, 56, 56, 24, 1, R, N0, True),      # MobileNetV2 block 3 at batch 2
    (2, 96, 112, 112, 24, 2, R, N0, False),    # MobileNetV2 block 2 at batch 2
    (2, 192, 28, 28, 32, 1, R, N0, True),      # MobileNetV2 blocks 5/6
]


@pytest.mark.parametrize("kern", ["lds", "stream"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c[:5])) + f"s{c[5]}" + ("r" if c[8] else ""))
def test_dw_pw_fused_matches_separate_and_oracle(case, kern, nhip_env):
    """Both fused kernels: the LDS-staged one (channels a multiple of 8, at
    most 32 output channels) and the streaming 1x1 kernel's depthwise mode
    (NHIP_DWPW_LDS=0)."""
    n, c, h, w, k = case[:5]
    if kern == "lds" and (c % 8 or k > 32):
        pytest.skip("outside the LDS-staged kernel's shapes (the streaming kernel takes them)")
    # the LDS-staged kernel is the default at stride 2 only; 2 forces it at stride 1 too
    nhip_env.setenv("NHIP_DWPW_LDS", "0" if kern == "stream" else "2")
    check_pair(*case, env=nhip_env, lds=kern == "lds")


LDS_CASES = [
    # (n, c, h, w, k, stride, dw_act, pw_act, residual): bands of 4, 2 and 1
    # output rows, partial last bands, 16-pixel blocks across row ends
    (1, 8, 8, 8, 1, 1, R, N0, False),
    (3, 16, 28, 20, 17, 1, N0, S, True),
    (2, 40, 20, 40, 32, 2, R, R, True),
    (5, 24, 12, 16, 16, 2, R, N0, False),
    (1, 64, 100, 4, 9, 1, R, N0, True),
    (2, 8, 4, 200, 32, 2, N0, N0, False),
    (4, 72, 44, 44, 30, 1, R, N0, True),
]


@pytest.mark.parametrize("case", LDS_CASES, ids=lambda c: "x".join(map(str, c[:5])) + f"s{c[5]}")
def test_dw_pw_lds_shapes(case, nhip_env):
    nhip_env.setenv("NHIP_DWPW_LDS", "2")
    check_pair(*case, env=nhip_env, lds=True)


MBV2_PAIRS = [
    # MobileNetV2 at batch 32: blocks 1 (32@112 s1 -> 16), 2 (96@112 s2 ->
    # 24), 3 (144@56 s1 -> 24 + residual), 4 (144@56 s2 -> 32)
    (32, 32, 112, 112, 16, 1, R, N0, False),
    (32, 96, 112, 112, 24, 2, R, N0, False),
    (32, 144, 56, 56, 24, 1, R, N0, True),
    (32, 144, 56, 56, 32, 2, R, N0, False),
]


@pytest.mark.parametrize("case", MBV2_PAIRS, ids=lambda c: f"{c[1]}at{c[2]}s{c[5]}to{c[4]}")
def test_dw_pw_lds_mobilenetv2_batch32(case, nhip_env):
    """The graph's fused pairs at batch 32 on the LDS-staged kernel (its
    default at stride 2, forced at stride 1): all 32 images bit for bit
    against the two layers, images 0 and 31 against the oracle."""
    nhip_env.setenv("NHIP_DWPW_LDS", "2")
    check_pair(*case, env=nhip_env, lds=True, images=[0, 31])


def test_dw_pw_default_kernel_choice(nhip_env):
    """Default choice: the LDS-staged kernel at stride 2, the streaming 1x1
    kernel's depthwise mode at stride 1."""
    nhip_env.delenv("NHIP_DWPW_LDS", raising=False)
    for stride, lds in ((2, True), (1, False)):
        check_pair(2, 48, 16, 16, 24, stride, R, N0, False, env=nhip_env, lds=lds)


@pytest.mark.parametrize("stride", [1, 2])
@pytest.mark.parametrize("cfg", ["1,1", "2,1", "3,1", "1,4", "2,4", "3,4"])
def test_dw_pw_every_configuration(cfg, stride, nhip_env):
    """Each (KT, WC) forced through NHIP_PW_CFG (stride 2 caps KT at 2), with
    C = 72: five 16-channel groups, split 2, 1, 1, 1 over four waves, the
    last group partial."""
    nhip_env.setenv("NHIP_PW_CFG", cfg)
    nhip_env.setenv("NHIP_DWPW_LDS", "0")
    check_pair(2, 72, 12, 16, 70, stride, R, N0, True)


def test_dw_pw_unsupported_shapes():
    """Rows that are not float4-aligned, a 5x5 depthwise, a 1x1 with stride:
    no fused kernel; forward says so with status 7 (unsupported)."""
    dw, pw, _ = make(16, 8, 1, R, N0)
    assert not nhip.dwconv_pw_supported(dw, pw, 1, 7, 7)
    with pytest.raises(nhip.NhipError) as e:
        nhip.dwconv_pw_forward(dw, pw, dev(RNG.uniform(-1, 1, (1, 16, 7, 7)).astype(np.float32)))
    assert e.value.status == 7
    wd = workloads.he_normal(RNG, (16, 1, 5, 5), 25)
    dw5 = nhip.DwConv2dF32(nhip.conv_desc(16, 16, (5, 5), (1, 1), (1, 1), (2, 2, 2, 2), bias=False, group=16), wd)
    assert not nhip.dwconv_pw_supported(dw5, pw, 1, 8, 8)
    wp = workloads.he_normal(RNG, (8, 16, 1, 1), 16)
    pw2 = nhip.Conv2dF32(nhip.conv_desc(16, 8, (1, 1), (2, 2), (1, 1), (0, 0, 0, 0), bias=False), wp)
    assert not nhip.dwconv_pw_supported(dw, pw2, 1, 8, 8)


def test_graph_executor_fuses_depthwise_into_project(nhip_env):
    """A graph with two dw -> 1x1 pairs (the first feeding a residual add)
    runs each pair as one launch, bit-identical to NHIP_DWPW=0; by default
    only the stride-2 pair with 24 output channels is fused, and only while
    its launch has at least 24576 output pixels (6 images of 64x64 do, one
    image does not)."""
    m = ncnn_format.Model()
    c, k = 48, 48
    m.input("data", c, 128, 128)
    wd = workloads.he_normal(RNG, (c, 1, 3, 3), 9)
    m.conv("dw1", "data", "d1", wd, RNG.normal(0, .05, c).astype(np.float32), act=1, depthwise=True)
    wp = workloads.he_normal(RNG, (k, c, 1, 1), c)
    m.conv("pw1", "d1", "p1", wp, RNG.normal(0, .05, k).astype(np.float32), pad=0)
    m.add("add1", "p1", "data", "y1")
    wd2 = workloads.he_normal(RNG, (k, 1, 3, 3), 9)
    m.conv("dw2", "y1", "d2", wd2, RNG.normal(0, .05, k).astype(np.float32), stride=2, act=1, depthwise=True)
    wp2 = workloads.he_normal(RNG, (24, k, 1, 1), k)
    m.conv("pw2", "d2", "out", wp2, RNG.normal(0, .05, 24).astype(np.float32), pad=0)
    g = nhip.Graph(m.param_text(), bytes(m.payload))
    x = dev(RNG.uniform(-1, 1, (6, c, 128, 128)).astype(np.float32))
    nhip.timer_start("dwpw")
    fused = host(g.run(x)[0])
    assert nhip.timer_stop()[0] == 2
    nhip_env.setenv("NHIP_DWPW", "0")
    nhip.timer_start("dwpw")
    separate = host(g.run(x)[0])
    assert nhip.timer_stop()[0] == 0
    np.testing.assert_array_equal(fused, separate)
    nhip_env.delenv("NHIP_DWPW")
    nhip.timer_start("dwpw")
    default = host(g.run(x)[0])
    assert nhip.timer_stop()[0] == 1
    np.testing.assert_array_equal(default, separate)
    nhip.timer_start("dwpw")
    one = host(g.run(x[:1].contiguous())[0])
    assert nhip.timer_stop()[0] == 0
    np.testing.assert_array_equal(one, separate[:1])
