"""GPU parity of the short-reduction fp32 convolution (csrc/conv_smallk.hip:
C*kh*kw <= 32 and at most 32 output channels, the MobileNetV2 stem) against
the CPU oracle (ConvertConvolution fp32, NCNNToTosa.cpp:1316-1529), within
the implicit-GEMM budget of max relative error 1e-4, with the kernel forced
on (NHIP_CONV_SMALLK=2: every shape it supports; by default it takes
launches of at least four 32-pixel blocks per CU) and off (=0: the implicit
GEMM).  Shapes cover
the stem at batch 2 and at the bench's batch 32 (every image), reductions
of 1 to 32, strides, dilation, asymmetric padding, 1x1 stride 2, output
channel counts that are not a multiple of 4, a residual, sigmoid, and
pixel counts that end part-way through a 32-pixel block."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import nhip  # noqa: E402
import workloads  # noqa: E402
from numerics import assert_close, max_rel_err  # noqa: E402
from oracle import refcpu  # noqa: E402

pytestmark = pytest.mark.gpu
IGEMM_RTOL = 1e-4
RNG = np.random.default_rng(29)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nhip.init(0)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def oracle(x, w, b, stride, dil, pad, act, residual=None):
    n, c, h, wd = x.shape
    g = refcpu.geom(n, c, h, wd, w.shape[0], w.shape[2:], stride, dil, pad)
    y = refcpu.conv2d_f32(g, x, w, b)
    if residual is not None:
        y = refcpu.add_f32(y, residual)
    if act == nhip.ACT_RELU:
        y = refcpu.relu_f32(y)
    elif act == nhip.ACT_SIGMOID:
        y = (1.0 / (1.0 + np.exp(-y.astype(np.float64)))).astype(np.float32)
    return y


CASES = [
    # (n, c, h, w, k, kernel, stride, dilation, pad(t,b,l,r), act, residual)
    (2, 3, 224, 224, 32, (3, 3), (2, 2), (1, 1), (1, 1, 1, 1), 1, False),  # the stem
    (3, 1, 7, 9, 5, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1), 0, False),
    (1, 1, 12, 11, 32, (5, 5), (1, 1), (1, 1), (2, 2, 2, 2), 1, True),     # reduction 25
    (2, 2, 10, 13, 7, (4, 4), (2, 1), (1, 1), (1, 2, 0, 3), 4, False),     # reduction 32, sigmoid
    (1, 3, 17, 15, 17, (3, 3), (1, 2), (2, 2), (2, 1, 2, 0), 1, False),    # dilation 2
    (2, 32, 9, 9, 30, (1, 1), (2, 2), (1, 1), (0, 0, 0, 0), 0, True),      # 1x1 stride 2
    (1, 5, 3, 3, 1, (2, 2), (1, 1), (1, 1), (0, 0, 0, 0), 1, False),       # 4 pixels, one channel
    (4, 16, 6, 5, 24, (1, 2), (1, 1), (1, 1), (0, 0, 1, 0), 1, False),     # reduction 32 from 16 channels
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c[:5])) + f"k{c[5][0]}{c[5][1]}")
@pytest.mark.parametrize("smallk", ["2", "0"])
def test_short_reduction_conv(case, smallk, nhip_env):
    nhip_env.setenv("NHIP_CONV_SMALLK", smallk)
    n, c, h, w, k, ker, st, dl, pad, act, with_res = case
    x = RNG.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = workloads.he_normal(RNG, (k, c) + ker, c * ker[0] * ker[1])
    b = RNG.normal(0, 0.05, k).astype(np.float32)
    oh = (h + pad[0] + pad[1] - dl[0] * (ker[0] - 1) - 1) // st[0] + 1
    ow = (w + pad[2] + pad[3] - dl[1] * (ker[1] - 1) - 1) // st[1] + 1
    res = RNG.uniform(-1, 1, (n, k, oh, ow)).astype(np.float32) if with_res else None
    d = nhip.conv_desc(c, k, ker, st, dl, pad, bias=True, act=act, algorithm=nhip.ALGO_IMPLICIT_GEMM)
    plan = nhip.Conv2dF32(d, wt, b)
    got = host(plan.forward(torch.from_numpy(x).cuda(),
                            residual=None if res is None else torch.from_numpy(res).cuda()))
    exp = oracle(x, wt, b, st, dl, pad, act, res)
    assert got.shape == exp.shape
    assert_close(got, exp, IGEMM_RTOL, f"short-reduction conv {case} smallk={smallk}")
    assert max_rel_err(got, exp) <= IGEMM_RTOL


def test_stem_full_batch(nhip_env):
    """The MobileNetV2 stem at the bench's batch 32 on the default path (the
    short-reduction kernel): every image against the oracle, into a reused
    output buffer (two passes)."""
    nhip_env.delenv("NHIP_CONV_SMALLK", raising=False)
    x = RNG.uniform(-1, 1, (32, 3, 224, 224)).astype(np.float32)
    wt = workloads.he_normal(RNG, (32, 3, 3, 3), 27)
    b = RNG.normal(0, 0.05, 32).astype(np.float32)
    d = nhip.conv_desc(3, 32, (3, 3), (2, 2), (1, 1), (1, 1, 1, 1), bias=True, act=nhip.ACT_RELU,
                       algorithm=nhip.ALGO_IMPLICIT_GEMM)
    plan = nhip.Conv2dF32(d, wt, b)
    xd = torch.from_numpy(x).cuda()
    out = torch.empty((32, 32, 112, 112), dtype=torch.float32, device="cuda")
    exp = oracle(x, wt, b, (2, 2), (1, 1), (1, 1, 1, 1), nhip.ACT_RELU)
    for rep in range(2):
        out.fill_(float("nan"))
        plan.forward(xd, out=out)
        got = host(out)
        for i in range(32):
            assert_close(got[i:i + 1], exp[i:i + 1], IGEMM_RTOL, f"stem image {i} pass {rep}")
