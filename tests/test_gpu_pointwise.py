"""GPU parity: the streaming 1x1 convolution kernel (pointwise.hip) against
the CPU oracle restating the reference's Convolution lowering
(NCNNToTosa.cpp:1316-1529, kernel 1x1 stride 1 pad 0, + the importer's
separate relu and the BinaryOp add), max relative error <= 1e-4.

The cases cover every kernel configuration (16..48 output channels per
slice, one or several slices, the channels of a tile split over one or four
waves, float4-aligned and unaligned pixel rows), channel counts that are not
multiples of 4 or 16, pixel tiles that cross image boundaries and end past
the last pixel, the persistent loop (a workgroup walking many tiles, its
prefetch crossing tile boundaries) and all three activations with and
without a residual.
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


def oracle(x, w, b, act, residual):
    n, c, h, wd = x.shape
    g = refcpu.geom(n, c, h, wd, w.shape[0], (1, 1), (1, 1), (1, 1), (0, 0, 0, 0))
    y = refcpu.conv2d_f32(g, x, w, b)
    if residual is not None:
        y = refcpu.add_f32(y, residual)
    if act == nhip.ACT_RELU:
        y = refcpu.relu_f32(y)
    elif act == nhip.ACT_SIGMOID:
        y = (1.0 / (1.0 + np.exp(-y.astype(np.float64)))).astype(np.float32)
    return y


def run(n, c, h, w, k, res, act, bias=True):
    x = RNG.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = workloads.he_normal(RNG, (k, c, 1, 1), c)
    b = RNG.normal(0, 0.05, k).astype(np.float32) if bias else None
    r = RNG.uniform(-1, 1, (n, k, h, w)).astype(np.float32) if res else None
    d = nhip.conv_desc(c, k, (1, 1), (1, 1), (1, 1), (0, 0, 0, 0), bias=bias, act=act)
    conv = nhip.Conv2dF32(d, wt, b)
    assert conv.workspace_size(n, h, w) == 0
    nhip.timer_start("pw_conv")
    got = host(conv.forward(dev(x), residual=dev(r) if res else None))
    launches, _ = nhip.timer_stop()
    assert launches == 1, "the layer did not take the pointwise kernel"
    exp = oracle(x, wt, b, act, r)
    assert_close(got, exp, RTOL, f"pointwise {(n, c, h, w, k, res, act)}")
    assert max_rel_err(got, exp) <= RTOL
    return got


CASES = [
    # (n, c, h, w, k, residual, act)
    (2, 16, 12, 12, 96, False, nhip.ACT_RELU),      # 2 slices of KT 3, last tile partly past the end
    (3, 24, 8, 8, 144, False, nhip.ACT_RELU),       # 3 slices of KT 3
    (2, 32, 6, 6, 192, False, nhip.ACT_SIGMOID),    # 4 slices
    (1, 64, 14, 14, 384, False, nhip.ACT_RELU),     # 8 slices
    (2, 144, 10, 10, 24, True, nhip.ACT_NONE),      # 9 channel chunks, residual
    (2, 40, 6, 6, 100, True, nhip.ACT_RELU),        # residual, K = 100: KT 3 with a partial slice
    (2, 40, 6, 6, 90, True, nhip.ACT_SIGMOID),      # residual, sigmoid
    (1, 5, 4, 4, 3, False, nhip.ACT_NONE),          # C and K below one block
    (5, 7, 2, 2, 20, True, nhip.ACT_RELU),          # 4-pixel images: a lane vector per image
    (1, 17, 20, 20, 33, False, nhip.ACT_NONE),      # C % 4 != 0, K = 33
    (2, 96, 14, 14, 24, False, nhip.ACT_NONE),      # MobileNetV2 project shape
    (2, 16, 28, 28, 96, False, nhip.ACT_RELU),      # MobileNetV2 expand shape
    (36, 8, 64, 64, 16, True, nhip.ACT_RELU),       # 576 tiles: more than the default grid
    (32, 16, 28, 28, 64, False, nhip.ACT_RELU),     # 25088 pixels: picked without the override
    (2, 72, 7, 7, 40, True, nhip.ACT_RELU),         # 7x7: unaligned rows, channels over 4 waves
    (3, 100, 5, 5, 20, False, nhip.ACT_SIGMOID),    # 5x5
    (4, 576, 7, 7, 160, False, nhip.ACT_NONE, "1,4"),  # MobileNetV2 576 -> 160 at 7x7 (forced)
    (2, 384, 14, 14, 64, True, nhip.ACT_NONE),      # MobileNetV2 384 -> 64 (+ residual) at 14x14
    (1, 960, 7, 7, 320, False, nhip.ACT_NONE, "2,4"),  # a 960-channel weight slice in LDS (forced)
    (32, 576, 14, 14, 96, True, nhip.ACT_NONE),     # MobileNetV2 576 -> 96 + residual at batch 32 (six slices)
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c[:5])) + ("r" if c[5] else "") + f"a{c[6]}")
def test_pointwise_matches_oracle(case, nhip_env):
    """Cases with an eighth entry force that configuration (NHIP_PW_CFG):
    the library leaves those shapes to the implicit GEMM by default.
    NHIP_CONV_KQ=0: the one-block-per-CU kernel, tried first, would take
    some of these shapes (64 -> 384 at 14x14, 576 -> 160 at 7x7)."""
    nhip_env.setenv("NHIP_CONV_KQ", "0")
    if len(case) > 7:
        nhip_env.setenv("NHIP_PW_CFG", case[7])
    run(*case[:7])


@pytest.mark.parametrize("wgs", ["1", "3", "8"])
@pytest.mark.parametrize("case", [(3, 20, 12, 12, 40, True, nhip.ACT_RELU),
                                  (2, 48, 10, 10, 96, False, nhip.ACT_NONE),
                                  (2, 16, 8, 8, 200, False, nhip.ACT_RELU)],
                         ids=["res", "kt6", "slices"])
def test_pointwise_persistent_walk(case, wgs, nhip_env):
    """A few workgroups walking every tile: the chunk prefetch crosses tile
    boundaries, and the results equal the one-tile-per-workgroup launch bit
    for bit (the per-pixel arithmetic does not depend on the walk)."""
    n, c, h, w, k, res, act = case
    x = dev(RNG.uniform(-1, 1, (n, c, h, w)).astype(np.float32))
    wt = workloads.he_normal(RNG, (k, c, 1, 1), c)
    b = RNG.normal(0, 0.05, k).astype(np.float32)
    r = dev(RNG.uniform(-1, 1, (n, k, h, w)).astype(np.float32)) if res else None
    conv = nhip.Conv2dF32(nhip.conv_desc(c, k, (1, 1), (1, 1), (1, 1), (0, 0, 0, 0), act=act), wt, b)
    wide = host(conv.forward(x, residual=r))
    nhip_env.setenv("NHIP_PW_WGS", wgs)
    narrow = host(conv.forward(x, residual=r))
    np.testing.assert_array_equal(narrow, wide)
    exp = oracle(host(x), wt, b, act, host(r) if res else None)
    assert_close(narrow, exp, RTOL, f"walk {case} wgs={wgs}")


CFGS = ["1,1", "2,1", "3,1", "1,4", "2,4", "3,4"]


@pytest.mark.parametrize("res", [False, True], ids=["plain", "res"])
@pytest.mark.parametrize("cfg", CFGS)
@pytest.mark.parametrize("hw", [(6, 8), (5, 5)], ids=["aligned", "unaligned"])
def test_pointwise_every_instantiation(cfg, res, hw, nhip_env):
    """Each kernel forced through NHIP_PW_CFG="kt,wc" (16*kt output channels
    per slice, the channels of a tile over wc waves; unaligned rows always
    take wc = 4), with K = 70 (several slices, a partial last block) and
    C = 72 (five chunks: the four waves get 2, 1, 1, 1)."""
    if hw == (5, 5) and cfg.endswith(",1"):
        pytest.skip("unaligned pixel rows have no one-wave split")
    nhip_env.setenv("NHIP_PW_CFG", cfg)
    run(3, 72, hw[0], hw[1], 70, res, nhip.ACT_RELU)


def test_pointwise_no_bias_and_batch_independence():
    n, c, h, w, k = 4, 24, 8, 8, 48
    x = RNG.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = workloads.he_normal(RNG, (k, c, 1, 1), c)
    conv = nhip.Conv2dF32(nhip.conv_desc(c, k, (1, 1), (1, 1), (1, 1), (0, 0, 0, 0), bias=False), wt)
    whole = host(conv.forward(dev(x)))
    assert_close(whole, oracle(x, wt, None, nhip.ACT_NONE, None), RTOL, "no bias")
    for i in range(n):
        np.testing.assert_array_equal(host(conv.forward(dev(x[i:i + 1]))), whole[i:i + 1])


def test_pointwise_off_switch_and_ineligible_shapes(nhip_env):
    """NHIP_POINTWISE=0 routes 1x1 layers to the implicit GEMM (the tuning
    comparison); both agree within the budget.  Shapes the kernel does not
    take go to the implicit GEMM: stride 2, and unaligned pixel rows with
    fewer than four channel chunks (one per wave)."""
    n, c, h, w, k = 2, 32, 8, 8, 64
    x = RNG.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = workloads.he_normal(RNG, (k, c, 1, 1), c)
    d = nhip.conv_desc(c, k, (1, 1), (1, 1), (1, 1), (0, 0, 0, 0), bias=False)
    nhip.timer_start("pw_conv")
    a = host(nhip.Conv2dF32(d, wt).forward(dev(x)))
    assert nhip.timer_stop()[0] == 1
    nhip_env.setenv("NHIP_POINTWISE", "0")
    nhip.timer_start("pw_conv")
    b = host(nhip.Conv2dF32(d, wt).forward(dev(x)))
    assert nhip.timer_stop()[0] == 0
    assert_close(a, b, RTOL, "pointwise vs implicit GEMM")
    nhip_env.delenv("NHIP_POINTWISE")
    for c, hw, stride in ((32, 8, 2), (48, 7, 1)):
        x = dev(RNG.uniform(-1, 1, (n, c, hw, hw)).astype(np.float32))
        wt = workloads.he_normal(RNG, (k, c, 1, 1), c)
        d = nhip.conv_desc(c, k, (1, 1), (stride, stride), (1, 1), (0, 0, 0, 0), bias=False)
        nhip.timer_start("pw_conv")
        nhip.Conv2dF32(d, wt).forward(x)
        assert nhip.timer_stop()[0] == 0
