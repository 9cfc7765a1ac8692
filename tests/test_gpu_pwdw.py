"""GPU parity: a 1x1 Convolution feeding a 3x3 ConvolutionDepthWise run as one
kernel (nhip_conv1x1_dw_f32_forward, the graph executor's fusion of an
inverted-residual block's expand -> depthwise pair on planes of at most 256
pixels).

The fused result is checked against the two layers run separately and
against the CPU oracle restating the reference's Convolution
(NCNNToTosa.cpp:1316-1529) and ConvolutionDepthWise (:3074-3503), within
1e-4 (the 1x1 sum is formed in another order than the separate 1x1 kernels';
the depthwise sum in the reference's order).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import nhip  # noqa: E402
import workloads  # noqa: E402
from numerics import assert_close, max_rel_err  # noqa: E402
from oracle import refcpu  # noqa: E402

pytestmark = pytest.mark.gpu

RTOL = 1e-4
R, N0 = nhip.ACT_RELU, nhip.ACT_NONE


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nhip.init(0)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


CASES = [
    # (n, c, h, w, k, stride, act1, actd)
    (2, 64, 14, 14, 384, 1, R, R),     # MobileNetV2 blocks 8-11 (expand 64 -> 384)
    (2, 96, 14, 14, 576, 2, R, R),     # block 14 (stride 2 to 7x7)
    (3, 160, 7, 7, 960, 1, R, R),      # blocks 15-17
    (2, 96, 14, 14, 576, 1, R, R),     # blocks 12-13
    (1, 32, 10, 10, 70, 2, N0, R),     # 70 channels: a partial 64-channel slice
    (2, 64, 12, 9, 100, 1, R, N0),     # 108 pixels: 7 tiles rounded up to 8
    (1, 96, 16, 16, 64, 2, R, R),      # 256 pixels, one slice
    (1, 96, 5, 3, 130, 1, N0, N0),     # 15 pixels: one tile of a plane
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c[:5])) + f"s{c[5]}")
def test_expand_dw_fused_matches_separate_and_oracle(case, nhip_env):
    nhip_env.setenv("NHIP_PWDW", "2")  # every plane size the kernel takes (default: up to 196 pixels)
    n, c, h, w, k, st, act1, actd = case
    rng = np.random.default_rng(hash(case) % (2 ** 32))
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    w1 = workloads.he_normal(rng, (k, c, 1, 1), c)
    b1 = rng.normal(0, 0.05, k).astype(np.float32)
    wd = workloads.he_normal(rng, (k, 1, 3, 3), 9)
    bd = rng.normal(0, 0.05, k).astype(np.float32)
    pw = nhip.Conv2dF32(nhip.conv_desc(c, k, (1, 1), (1, 1), (1, 1), (0, 0, 0, 0), act=act1,
                                       algorithm=nhip.ALGO_IMPLICIT_GEMM), w1, b1)
    dw = nhip.DwConv2dF32(nhip.conv_desc(k, k, (3, 3), (st, st), (1, 1), (1, 1, 1, 1), act=actd, group=k), wd, bd)
    assert nhip.conv1x1_dw_supported(pw, dw, n, h, w)
    xd = dev(x)
    nhip.timer_start("expand_dw")
    fused = host(nhip.conv1x1_dw_forward(pw, dw, xd))
    assert nhip.timer_stop()[0] == 1
    separate = host(dw.forward(pw.forward(xd)))
    assert_close(fused, separate, RTOL, f"fused vs separate {case}")
    # oracle: the reference's two layers
    e = refcpu.conv2d_f32(refcpu.geom(n, c, h, w, k, (1, 1), (1, 1), (1, 1), (0, 0, 0, 0)), x, w1, b1)
    if act1 == R:
        e = refcpu.relu_f32(e)
    y = refcpu.dwconv2d_f32(refcpu.geom(n, k, h, w, k, (3, 3), (st, st), (1, 1), (1, 1, 1, 1)), e, wd, bd)
    if actd == R:
        y = refcpu.relu_f32(y)
    assert_close(fused, y, RTOL, f"fused vs oracle {case}")
    assert max_rel_err(fused, y) <= RTOL


def test_expand_dw_not_taken_for_unsupported_pairs(nhip_env):
    """Planes over 256 pixels, other channel counts and a 5x5 depthwise have
    no fused kernel; the default also leaves planes over 196 pixels alone."""
    rng = np.random.default_rng(3)

    def plans(c, k, kernel=3):
        pw = nhip.Conv2dF32(nhip.conv_desc(c, k, (1, 1), (1, 1), (1, 1), (0, 0, 0, 0), act=R,
                                           algorithm=nhip.ALGO_IMPLICIT_GEMM),
                            workloads.he_normal(rng, (k, c, 1, 1), c), np.zeros(k, np.float32))
        pad = kernel // 2
        dw = nhip.DwConv2dF32(nhip.conv_desc(k, k, (kernel, kernel), (1, 1), (1, 1), (pad,) * 4, act=R, group=k),
                              workloads.he_normal(rng, (k, 1, kernel, kernel), kernel * kernel),
                              np.zeros(k, np.float32))
        return pw, dw

    pw, dw = plans(64, 128)
    assert nhip.conv1x1_dw_supported(pw, dw, 2, 14, 14)
    assert not nhip.conv1x1_dw_supported(pw, dw, 2, 16, 16)   # 256 pixels: only with NHIP_PWDW=2
    assert not nhip.conv1x1_dw_supported(pw, dw, 2, 28, 28)
    nhip_env.setenv("NHIP_PWDW", "2")
    assert nhip.conv1x1_dw_supported(pw, dw, 2, 16, 16)
    assert not nhip.conv1x1_dw_supported(pw, dw, 2, 17, 16)
    pw160, dw160 = plans(160, 64)
    assert not nhip.conv1x1_dw_supported(pw160, dw160, 1, 16, 16)  # 166 KB of LDS
    assert nhip.conv1x1_dw_supported(pw160, dw160, 1, 14, 14)
    pw2, dw2 = plans(48, 96)
    assert not nhip.conv1x1_dw_supported(pw2, dw2, 2, 14, 14)
    pw3, dw3 = plans(64, 64, kernel=5)
    assert not nhip.conv1x1_dw_supported(pw3, dw3, 2, 14, 14)
    nhip_env.setenv("NHIP_PWDW", "0")
    assert not nhip.conv1x1_dw_supported(pw, dw, 2, 14, 14)
