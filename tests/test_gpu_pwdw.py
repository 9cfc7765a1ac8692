"""GPU parity: a 1x1 Convolution feeding a 3x3 ConvolutionDepthWise run as one
kernel (nhip_conv1x1_dw_f32_forward, the graph executor's fusion of an
inverted-residual block's expand -> depthwise pair: whole planes, or row
strips with a one-row halo).

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
    # row strips (planes the LDS cannot hold whole, or cut for more workgroups)
    (2, 16, 28, 28, 96, 2, R, R),      # MobileNetV2 block 2's channels (16 -> 96, stride 2)
    (2, 24, 20, 20, 144, 1, R, R),     # blocks 3 (24 -> 144; channels padded to 32)
    (1, 24, 17, 13, 48, 2, R, N0),     # odd plane, stride 2
    (2, 32, 28, 28, 192, 1, R, R),     # blocks 5-6 (32 -> 192 at 28x28)
    (1, 32, 28, 28, 64, 2, N0, R),     # block 7's stride 2
    (1, 160, 16, 16, 64, 2, R, R),     # too large for a whole plane: strips of 64-wide slices
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c[:5])) + f"s{c[5]}")
def test_expand_dw_fused_matches_separate_and_oracle(case, nhip_env):
    nhip_env.setenv("NHIP_PWDW", "2")  # every plane the kernel takes (default: up to 784 pixels)
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


# forced (slice width, rows per strip): every strip shape, first / middle /
# last strips, strips shorter than the kernel's 7-row depthwise runs
FORCED = [
    ("32,1", (1, 16, 12, 12, 40, 2)),
    ("32,2", (1, 16, 20, 16, 32, 2)),
    ("32,3", (1, 24, 13, 12, 32, 1)),
    ("32,5", (1, 32, 14, 8, 32, 2)),
    ("64,3", (1, 64, 14, 14, 96, 1)),
    ("64,2", (1, 96, 14, 14, 64, 2)),
    ("32,9", (1, 24, 17, 12, 40, 1)),
]


def _layers(rng, c, k, st, act1, actd):
    w1 = workloads.he_normal(rng, (k, c, 1, 1), c)
    b1 = rng.normal(0, 0.05, k).astype(np.float32)
    wd = workloads.he_normal(rng, (k, 1, 3, 3), 9)
    bd = rng.normal(0, 0.05, k).astype(np.float32)
    pw = nhip.Conv2dF32(nhip.conv_desc(c, k, (1, 1), (1, 1), (1, 1), (0, 0, 0, 0), act=act1,
                                       algorithm=nhip.ALGO_IMPLICIT_GEMM), w1, b1)
    dw = nhip.DwConv2dF32(nhip.conv_desc(k, k, (3, 3), (st, st), (1, 1), (1, 1, 1, 1), act=actd, group=k), wd, bd)
    return pw, dw


@pytest.mark.parametrize("cfg,case", FORCED, ids=[f[0].replace(",", "x") for f in FORCED])
def test_expand_dw_forced_strip_configs(cfg, case, nhip_env):
    nhip_env.setenv("NHIP_PWDW", "2")
    nhip_env.setenv("NHIP_PWDW_CFG", cfg)
    n, c, h, w, k, st = case
    rng = np.random.default_rng(7)
    pw, dw = _layers(rng, c, k, st, R, R)
    assert nhip.conv1x1_dw_supported(pw, dw, n, h, w)
    xd = dev(rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32))
    fused = host(nhip.conv1x1_dw_forward(pw, dw, xd))
    separate = host(dw.forward(pw.forward(xd)))
    assert_close(fused, separate, RTOL, f"forced {cfg} {case}")


@pytest.mark.parametrize("h,w", [(14, 14), (7, 7), (20, 20)])
def test_expand_dw_misaligned_input(h, w, nhip_env):
    """An input that is not 16-byte aligned takes the 4-byte copies (whole
    plane and strips)."""
    nhip_env.setenv("NHIP_PWDW", "2")
    rng = np.random.default_rng(11)
    c, k = 32, 64
    pw, dw = _layers(rng, c, k, 1, R, R)
    x = rng.uniform(-1, 1, (2, c, h, w)).astype(np.float32)
    buf = torch.zeros(x.size + 1, dtype=torch.float32, device="cuda")
    xd = buf[1:].view(2, c, h, w)
    xd.copy_(torch.from_numpy(x).cuda())
    assert xd.data_ptr() % 16 != 0
    fused = host(nhip.conv1x1_dw_forward(pw, dw, xd))
    separate = host(dw.forward(pw.forward(dev(x))))
    assert_close(fused, separate, RTOL, f"misaligned {h}x{w}")


def test_expand_dw_not_taken_for_unsupported_pairs(nhip_env):
    """Other channel counts and a 5x5 depthwise have no fused kernel; the
    default leaves planes over 784 pixels alone."""
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
    assert nhip.conv1x1_dw_supported(pw, dw, 2, 28, 28)
    assert not nhip.conv1x1_dw_supported(pw, dw, 2, 29, 28)   # over 784 pixels: only with NHIP_PWDW=2
    assert not nhip.conv1x1_dw_supported(pw, dw, 2, 56, 56)
    nhip_env.setenv("NHIP_PWDW", "2")
    assert nhip.conv1x1_dw_supported(pw, dw, 2, 56, 56)       # row strips
    pw2, dw2 = plans(48, 96)
    assert not nhip.conv1x1_dw_supported(pw2, dw2, 2, 14, 14)
    pw3, dw3 = plans(64, 64, kernel=5)
    assert not nhip.conv1x1_dw_supported(pw3, dw3, 2, 14, 14)
    nhip_env.setenv("NHIP_PWDW", "0")
    assert not nhip.conv1x1_dw_supported(pw, dw, 2, 14, 14)


def test_expand_dw_random_shapes(nhip_env):
    """40 seeded random pairs (channels, planes of 1-30 rows and columns,
    stride, activations, batch) with every plane the kernel takes: the fused
    result within 1e-4 of the two layers."""
    nhip_env.setenv("NHIP_PWDW", "2")
    rng = np.random.default_rng(2024)
    taken = 0
    for _ in range(40):
        c = int(rng.choice([16, 24, 32, 64, 96, 160]))
        k = int(rng.integers(2, 100)) * 4
        h, w = int(rng.integers(1, 31)), int(rng.integers(1, 31))
        st = int(rng.integers(1, 3))
        n = int(rng.integers(1, 4))
        a1, ad = (R if rng.random() < 0.7 else N0), (R if rng.random() < 0.7 else N0)
        pw, dw = _layers(rng, c, k, st, a1, ad)
        if not nhip.conv1x1_dw_supported(pw, dw, n, h, w):
            continue
        taken += 1
        xd = dev(rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32))
        fused = host(nhip.conv1x1_dw_forward(pw, dw, xd))
        separate = host(dw.forward(pw.forward(xd)))
        assert_close(fused, separate, RTOL, f"random pair c{c} k{k} {h}x{w} s{st} n{n}")
    assert taken >= 30
