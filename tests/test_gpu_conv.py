"""GPU parity: fp32 Convolution through the C ABI (implicit GEMM and
Winograd F(4,3)) against the CPU oracle restating the reference's lowering
(NCNNToTosa.cpp:1316-1529 + the importer's separate relu and the BinaryOp add).

Budgets from the north star: max relative error <= 1e-4 for implicit GEMM,
<= 1e-3 for Winograd (checked elementwise with a data-scaled absolute term,
and normwise).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import nhip  # noqa: E402
import workloads  # noqa: E402
from numerics import assert_close, max_rel_err  # noqa: E402
from oracle import refcpu  # noqa: E402

pytestmark = pytest.mark.gpu

IGEMM_RTOL = 1e-4
WINO_RTOL = 1e-3


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nhip.init(0)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def oracle_conv(x, w, b, stride, dil, pad, act=0, residual=None):
    n, c, h, wd = x.shape
    k = w.shape[0]
    g = refcpu.geom(n, c, h, wd, k, w.shape[2:], stride, dil, pad)
    y = refcpu.conv2d_f32(g, x, w, b)
    if residual is not None:
        y = refcpu.add_f32(y, residual)
    if act == nhip.ACT_RELU:
        y = refcpu.relu_f32(y)
    elif act == nhip.ACT_SIGMOID:
        y = (1.0 / (1.0 + np.exp(-y.astype(np.float64)))).astype(np.float32)
    return y


RNG = np.random.default_rng(7)

GENERAL_CASES = [
    # (n, c, h, w, k, kernel, stride, dilation, pad(t,b,l,r))
    (1, 1, 4, 4, 2, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1)),
    (2, 3, 7, 6, 5, (3, 3), (2, 2), (1, 1), (1, 1, 1, 1)),
    (1, 4, 9, 8, 3, (3, 3), (1, 1), (2, 2), (2, 2, 2, 2)),
    (1, 2, 6, 7, 3, (2, 3), (1, 2), (1, 1), (0, 1, 2, 0)),
    (2, 8, 5, 5, 4, (1, 1), (1, 1), (1, 1), (0, 0, 0, 0)),
    (1, 3, 11, 11, 8, (3, 3), (2, 2), (1, 1), (1, 1, 1, 1)),
    (3, 70, 13, 9, 130, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1)),
    (2, 3, 32, 30, 32, (3, 3), (2, 2), (1, 1), (1, 1, 1, 1)),   # MobileNetV2 stem shape
    (2, 96, 14, 14, 24, (1, 1), (1, 1), (1, 1), (0, 0, 0, 0)),  # 1x1 project
    (1, 320, 7, 7, 1280, (1, 1), (1, 1), (1, 1), (0, 0, 0, 0)),  # 1x1 head
    (1, 5, 10, 12, 6, (5, 5), (3, 2), (1, 2), (2, 1, 0, 3)),
]


@pytest.mark.parametrize("case", GENERAL_CASES, ids=lambda c: "x".join(map(str, c[:5])))
@pytest.mark.parametrize("act", [nhip.ACT_NONE, nhip.ACT_RELU])
def test_implicit_gemm_matches_oracle(case, act):
    n, c, h, w, k, ker, st, dl, pad = case
    x = RNG.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = workloads.he_normal(RNG, (k, c) + ker, c * ker[0] * ker[1])
    b = RNG.normal(0, 0.05, k).astype(np.float32)
    d = nhip.conv_desc(c, k, ker, st, dl, pad, bias=True, act=act, algorithm=nhip.ALGO_IMPLICIT_GEMM)
    conv = nhip.Conv2dF32(d, wt, b)
    got = host(conv.forward(dev(x)))
    exp = oracle_conv(x, wt, b, st, dl, pad, act)
    assert_close(got, exp, IGEMM_RTOL, f"igemm {case}")
    assert max_rel_err(got, exp) <= IGEMM_RTOL


def test_implicit_gemm_no_bias_sigmoid_and_residual():
    n, c, h, w, k = 2, 24, 9, 11, 40
    x = RNG.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = workloads.he_normal(RNG, (k, c, 3, 3), c * 9)
    r = RNG.uniform(-1, 1, (n, k, h, w)).astype(np.float32)
    d = nhip.conv_desc(c, k, bias=False, act=nhip.ACT_SIGMOID, algorithm=nhip.ALGO_IMPLICIT_GEMM)
    got = host(nhip.Conv2dF32(d, wt).forward(dev(x)))
    exp = oracle_conv(x, wt, None, (1, 1), (1, 1), (1, 1, 1, 1), nhip.ACT_SIGMOID)
    assert_close(got, exp, IGEMM_RTOL, "sigmoid")
    d = nhip.conv_desc(c, k, bias=False, act=nhip.ACT_RELU, algorithm=nhip.ALGO_IMPLICIT_GEMM)
    got = host(nhip.Conv2dF32(d, wt).forward(dev(x), residual=dev(r)))
    exp = oracle_conv(x, wt, None, (1, 1), (1, 1), (1, 1, 1, 1), nhip.ACT_RELU, residual=r)
    assert_close(got, exp, IGEMM_RTOL, "residual")


KQ_CASES = [
    # (n, c, h, w, k, stride, dilation, pad(t,b,l,r), residual, act)
    (1, 64, 56, 56, 64, (1, 1), (1, 1), (1, 1, 1, 1), False, 1),   # the benchmarked single conv
    (1, 32, 13, 11, 40, (1, 1), (1, 1), (1, 1, 1, 1), True, 0),    # 40 of 64 channels, 143 pixels
    (2, 32, 9, 17, 70, (2, 1), (1, 1), (0, 2, 1, 1), False, 1),    # stride 2 x 1, asymmetric padding, 2 images
    (1, 64, 12, 10, 32, (1, 1), (2, 2), (2, 2, 2, 2), True, 1),    # dilation 2
    (3, 32, 5, 5, 96, (2, 2), (1, 1), (1, 1, 1, 1), False, 0),     # blocks spanning images
]


@pytest.mark.parametrize("case", KQ_CASES, ids=lambda c: "x".join(map(str, c[:5])))
@pytest.mark.parametrize("kq", ["2", "0"])
def test_conv_kq_matches_oracle(case, kq, nhip_env):
    """The one-block-per-32x32 kernel with the reduction split over its
    waves (NHIP_CONV_KQ=2: every shape it takes; by default launches of at
    most two blocks per CU) and the tiled implicit GEMM (=0)."""
    nhip_env.setenv("NHIP_CONV_KQ", kq)
    n, c, h, w, k, st, dl, pad, with_res, act = case
    rng = np.random.default_rng(hash(case) % (2 ** 32))
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = workloads.he_normal(rng, (k, c, 3, 3), c * 9)
    b = rng.normal(0, 0.05, k).astype(np.float32)
    oh = (h + pad[0] + pad[1] - dl[0] * 2 - 1) // st[0] + 1
    ow = (w + pad[2] + pad[3] - dl[1] * 2 - 1) // st[1] + 1
    res = rng.uniform(-1, 1, (n, k, oh, ow)).astype(np.float32) if with_res else None
    d = nhip.conv_desc(c, k, (3, 3), st, dl, pad, bias=True, act=act, algorithm=nhip.ALGO_IMPLICIT_GEMM)
    plan = nhip.Conv2dF32(d, wt, b)
    exp = oracle_conv(x, wt, b, st, dl, pad, act, residual=res)
    out = torch.full(exp.shape, float("nan"), dtype=torch.float32, device="cuda")
    for rep in range(2):  # into the same output twice
        nhip.timer_start("conv_kq")
        got = host(plan.forward(dev(x), residual=None if res is None else dev(res), out=out))
        assert nhip.timer_stop()[0] == (1 if kq == "2" else 0)
        assert_close(got, exp, IGEMM_RTOL, f"conv kq={kq} {case} call {rep}")
        assert max_rel_err(got, exp) <= IGEMM_RTOL


KQ1_CASES = [
    # (n, c, h, w, k, stride, pad(t,b,l,r), residual, act): 1x1, C = 8*ch or 960
    (32, 960, 7, 7, 160, (1, 1), (0, 0, 0, 0), True, 0),   # MobileNetV2's 960 -> 160 + residual
    (1, 64, 5, 9, 40, (1, 1), (0, 0, 0, 0), False, 1),
    (2, 96, 14, 14, 70, (1, 1), (0, 0, 0, 0), True, 0),
    (3, 320, 6, 5, 33, (1, 1), (0, 0, 0, 0), False, 1),
    (1, 576, 7, 7, 96, (1, 1), (0, 0, 0, 0), True, 0),
    (2, 384, 3, 11, 64, (1, 1), (0, 0, 0, 0), False, 0),
    (1, 160, 7, 7, 16, (1, 1), (0, 0, 0, 0), False, 1),
    (2, 64, 9, 9, 32, (2, 2), (1, 0, 1, 0), False, 1),     # stride 2, padding
]


@pytest.mark.parametrize("case", KQ1_CASES, ids=lambda c: "x".join(map(str, c[:5])))
@pytest.mark.parametrize("kq", ["2", "0"])
def test_conv_kq_1x1_matches_oracle(case, kq, nhip_env):
    """1x1 convolutions on the split-reduction kernel (NHIP_CONV_KQ=2:
    every shape it takes, with the streaming pointwise kernel, which is
    picked first, switched off; by default at most one 32x32 block per CU)
    and off (=0: the pointwise, direct-to-LDS or tiled kernels)."""
    nhip_env.setenv("NHIP_CONV_KQ", kq)
    if kq == "2":
        nhip_env.setenv("NHIP_POINTWISE", "0")
    n, c, h, w, k, st, pad, with_res, act = case
    rng = np.random.default_rng(hash(case) % (2 ** 32))
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = workloads.he_normal(rng, (k, c, 1, 1), c)
    b = rng.normal(0, 0.05, k).astype(np.float32)
    oh = (h + pad[0] + pad[1] - 1) // st[0] + 1
    ow = (w + pad[2] + pad[3] - 1) // st[1] + 1
    res = rng.uniform(-1, 1, (n, k, oh, ow)).astype(np.float32) if with_res else None
    d = nhip.conv_desc(c, k, (1, 1), st, (1, 1), pad, bias=True, act=act, algorithm=nhip.ALGO_IMPLICIT_GEMM)
    plan = nhip.Conv2dF32(d, wt, b)
    exp = oracle_conv(x, wt, b, st, (1, 1), pad, act, residual=res)
    nhip.timer_start("conv_kq")
    got = host(plan.forward(dev(x), residual=None if res is None else dev(res)))
    assert nhip.timer_stop()[0] == (1 if kq == "2" else 0)
    assert_close(got, exp, IGEMM_RTOL, f"1x1 kq={kq} {case}")
    assert max_rel_err(got, exp) <= IGEMM_RTOL


TWIN_CASES = [
    # (n, c, h, w, k, residual): Winograd plans of 256+ input channels, launches of <= 32 tiles
    (1, 512, 7, 7, 512, True),     # one image of ResNet-18's last stage (4 tiles)
    (2, 256, 14, 14, 256, False),  # two images of the 256@14 stage (32 tiles)
    (1, 256, 5, 9, 130, True),     # ragged extents, 130 output channels
]


@pytest.mark.parametrize("case", TWIN_CASES, ids=lambda c: "x".join(map(str, c[:5])))
@pytest.mark.parametrize("twin", ["1", "0"])
def test_winograd_plan_small_launch_twin(case, twin, nhip_env):
    """A Winograd plan of 256+ input channels runs launches of at most 32
    tiles on its implicit-GEMM twin (NHIP_WINO_TWIN=1, the default: no
    Winograd kernel launched, the implicit GEMM's 1e-4 budget) and on the
    Winograd kernels with the route off (=0, the Winograd budget)."""
    nhip_env.delenv("NHIP_WINOGRAD_VARIANT", raising=False)
    nhip_env.setenv("NHIP_WINO_TWIN", twin)
    n, c, h, w, k, with_res = case
    rng = np.random.default_rng(hash(case) % (2 ** 32))
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = workloads.he_normal(rng, (k, c, 3, 3), c * 9)
    b = rng.normal(0, 0.05, k).astype(np.float32)
    res = rng.uniform(-1, 1, (n, k, h, w)).astype(np.float32) if with_res else None
    plan = nhip.Conv2dF32(nhip.conv_desc(c, k, act=1, algorithm=nhip.ALGO_WINOGRAD), wt, b)
    exp = oracle_conv(x, wt, b, (1, 1), (1, 1), (1, 1, 1, 1), act=1, residual=res)
    nhip.timer_start("wino")
    got = host(plan.forward(dev(x), residual=None if res is None else dev(res)))
    launches = nhip.timer_stop()[0]
    assert (launches == 0) == (twin == "1")
    tol = IGEMM_RTOL if twin == "1" else WINO_RTOL
    assert_close(got, exp, tol, f"twin={twin} {case}")
    assert max_rel_err(got, exp) <= tol


WINO_CASES = [
    # (n, c, h, w, k, pad)
    (1, 16, 4, 4, 16, (1, 1, 1, 1)),
    (2, 20, 13, 10, 24, (1, 1, 1, 1)),      # ragged tiles, C not a multiple of 16
    (2, 32, 9, 9, 48, (0, 0, 0, 0)),        # valid conv
    (1, 17, 8, 12, 70, (2, 0, 1, 2)),       # asymmetric padding
    (3, 64, 7, 7, 64, (1, 1, 1, 1)),
    (1, 130, 6, 5, 200, (1, 1, 1, 1)),
    (2, 16, 40, 40, 24, (1, 1, 1, 1)),      # 10 x 10 tiles: 32-tile blocks start mid-row and span images
    (1, 8, 30, 30, 16, (1, 1, 1, 1)),       # the same with rows that are not float4-aligned
    (1, 8, 5, 135, 12, (1, 1, 1, 1)),       # 34 tiles per row: a block inside one tile row
    (2, 4, 4, 132, 8, (1, 1, 1, 1)),        # the same with float4 rows
    (3, 8, 10, 16, 16, (1, 1, 1, 1)),       # float4 rows, last tile row clipped (OH % 4 = 2), blocks span images
    (5, 8, 11, 9, 24, (1, 1, 1, 1)),        # clipped rows and columns, 9 tiles per image
]


@pytest.fixture(params=["auto", "1", "2", "2split", "2ks"])
def wino_variant(request, nhip_env):
    """Winograd implementations: the default per-shape choice (auto), the
    three-kernel path (1), the GEMM with the output transform fused (2) with
    each workgroup's halves taking alternate input-channel chunks of one
    32-channel block, the same with the input channels split over two
    workgroups per block and the parts summed by the reduce kernel
    (2split), and the halves owning two 32-channel blocks (2ks)."""
    nhip_env.delenv("NHIP_WINO_SPLITS", raising=False)
    nhip_env.setenv("NHIP_WINO_KS", "1" if request.param == "2ks" else "0")
    if request.param == "auto":
        nhip_env.delenv("NHIP_WINOGRAD_VARIANT", raising=False)
        nhip_env.delenv("NHIP_WINO_KS", raising=False)
    else:
        nhip_env.setenv("NHIP_WINOGRAD_VARIANT", request.param[0])
        if request.param == "2split":
            nhip_env.setenv("NHIP_WINO_SPLITS", "2")
    return request.param


@pytest.mark.parametrize("case", WINO_CASES, ids=lambda c: "x".join(map(str, c[:5])))
def test_winograd_matches_oracle(case, wino_variant):
    n, c, h, w, k, pad = case
    x = RNG.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = workloads.he_normal(RNG, (k, c, 3, 3), c * 9)
    b = RNG.normal(0, 0.05, k).astype(np.float32)
    d = nhip.conv_desc(c, k, pad=pad, act=nhip.ACT_RELU, algorithm=nhip.ALGO_WINOGRAD)
    got = host(nhip.Conv2dF32(d, wt, b).forward(dev(x)))
    exp = oracle_conv(x, wt, b, (1, 1), (1, 1), pad, nhip.ACT_RELU)
    assert_close(got, exp, WINO_RTOL, f"winograd {case}")
    assert max_rel_err(got, exp) <= WINO_RTOL


def _random_wino_cases(count, seed):
    """Seeded random shapes for the fused GEMM's write-out: tile blocks that
    start mid-row and span images, rows and columns clipped by OH, OW % 4,
    float4 and single-pixel units, channel splits (few blocks), residual."""
    r = np.random.default_rng(seed)
    cases = []
    for _ in range(count):
        n = int(r.integers(1, 5))
        h, w = int(r.integers(3, 42)), int(r.integers(3, 42))
        c = int(r.choice([3, 8, 16, 24, 40, 64]))
        k = int(r.choice([8, 16, 32, 40, 72]))
        pad = tuple(int(v) for v in r.integers(0, 3, 4))
        if h + pad[0] + pad[1] < 3 or w + pad[2] + pad[3] < 3:
            pad = (1, 1, 1, 1)
        cases.append((n, c, h, w, k, pad, bool(r.integers(0, 2))))
    return cases


@pytest.mark.parametrize("mode", ["1", "4", "ks"])
@pytest.mark.parametrize("case", _random_wino_cases(16, 7), ids=lambda c: "x".join(map(str, c[:5])))
def test_winograd_fused_random_shapes(case, mode, nhip_env):
    """Modes: one part; up to four input-channel splits summed by the
    reduce kernel (4); workgroups of two 32-channel blocks (ks)."""
    nhip_env.setenv("NHIP_WINOGRAD_VARIANT", "2")  # the fused GEMM whatever the tile count
    nhip_env.setenv("NHIP_WINO_SPLITS", mode[0] if mode != "ks" else "1")
    nhip_env.setenv("NHIP_WINO_KS", "1" if mode == "ks" else "0")
    n, c, h, w, k, pad, with_res = case
    rng = np.random.default_rng(hash(case) % (2 ** 32))
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = workloads.he_normal(rng, (k, c, 3, 3), c * 9)
    b = rng.normal(0, 0.05, k).astype(np.float32)
    oh, ow = h + pad[0] + pad[1] - 2, w + pad[2] + pad[3] - 2
    res = rng.uniform(-1, 1, (n, k, oh, ow)).astype(np.float32) if with_res else None
    d = nhip.conv_desc(c, k, pad=pad, act=nhip.ACT_RELU, algorithm=nhip.ALGO_WINOGRAD)
    got = host(nhip.Conv2dF32(d, wt, b).forward(dev(x), residual=dev(res) if with_res else None))
    exp = oracle_conv(x, wt, b, (1, 1), (1, 1), pad, nhip.ACT_RELU, residual=res)
    assert_close(got, exp, WINO_RTOL, f"winograd fused {case}")


XT_CASES = [
    # (n, c, h, w, k, pad): launches of paired 32-channel blocks, where the
    # input transform runs inside the GEMM by default: rows not float4-aligned,
    # left padding 0 and 2, channels not a multiple of 8, an odd number of
    # 32-channel blocks (the last pair half empty), tiles not a multiple of 32
    (32, 64, 56, 56, 64, (1, 1, 1, 1)),
    (9, 24, 30, 22, 72, (1, 1, 1, 1)),
    (7, 19, 26, 27, 40, (2, 0, 0, 2)),
    (5, 40, 33, 36, 96, (0, 2, 2, 1)),
]


@pytest.mark.parametrize("case", XT_CASES, ids=lambda c: "x".join(map(str, c[:5])))
def test_winograd_in_kernel_transform(case, nhip_env):
    """The fused GEMM forming V from the input itself (no transform launch,
    no V workspace) against the oracle, and against the separate transform
    (NHIP_WINO_XT=0) within the Winograd budget."""
    n, c, h, w, k, pad = case
    nhip_env.setenv("NHIP_WINOGRAD_VARIANT", "2")
    nhip_env.setenv("NHIP_WINO_KS", "1")
    nhip_env.setenv("NHIP_WINO_SPLITS", "1")
    rng = np.random.default_rng(c * 100 + k)
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = workloads.he_normal(rng, (k, c, 3, 3), c * 9)
    b = rng.normal(0, 0.05, k).astype(np.float32)
    oh, ow = h + pad[0] + pad[1] - 2, w + pad[2] + pad[3] - 2
    res = rng.uniform(-1, 1, (n, k, oh, ow)).astype(np.float32)
    conv = nhip.Conv2dF32(nhip.conv_desc(c, k, pad=pad, act=nhip.ACT_RELU, algorithm=nhip.ALGO_WINOGRAD), wt, b)
    assert conv.workspace_size(n, h, w) == 0  # no V
    nhip.timer_start("wino_input")
    got = host(conv.forward(dev(x), residual=dev(res)))
    assert nhip.timer_stop()[0] == 0
    nhip_env.setenv("NHIP_WINO_XT", "0")
    assert conv.workspace_size(n, h, w) > 0
    sep = host(conv.forward(dev(x), residual=dev(res)))
    exp = oracle_conv(x, wt, b, (1, 1), (1, 1), pad, nhip.ACT_RELU, residual=res)
    assert_close(got, exp, WINO_RTOL, f"winograd in-kernel transform {case}")
    assert_close(got, sep, WINO_RTOL, f"winograd in-kernel transform against the transform launch {case}")


@pytest.mark.parametrize("act", [nhip.ACT_NONE, nhip.ACT_SIGMOID])
@pytest.mark.parametrize("bias", [True, False])
def test_winograd_in_kernel_transform_epilogues(act, bias, nhip_env):
    """The in-kernel transform's other epilogue instances: no activation and
    sigmoid, with and without bias, no residual; a batch whose tiles end
    inside a 32-tile block."""
    n, c, h, w, k = 3, 32, 20, 24, 64
    nhip_env.setenv("NHIP_WINOGRAD_VARIANT", "2")
    nhip_env.setenv("NHIP_WINO_KS", "1")
    nhip_env.setenv("NHIP_WINO_SPLITS", "1")
    rng = np.random.default_rng(7 + act)
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = workloads.he_normal(rng, (k, c, 3, 3), c * 9)
    b = rng.normal(0, 0.05, k).astype(np.float32) if bias else None
    d = nhip.conv_desc(c, k, bias=bias, act=act, algorithm=nhip.ALGO_WINOGRAD)
    conv = nhip.Conv2dF32(d, wt, b) if bias else nhip.Conv2dF32(d, wt)
    assert conv.workspace_size(n, h, w) == 0  # the in-kernel transform
    nhip.timer_start("wino_input")
    got = host(conv.forward(dev(x)))
    assert nhip.timer_stop()[0] == 0
    exp = oracle_conv(x, wt, b, (1, 1), (1, 1), (1, 1, 1, 1), act)
    assert_close(got, exp, WINO_RTOL, f"winograd in-kernel transform act {act} bias {bias}")


@pytest.mark.parametrize("algo", [nhip.ALGO_IMPLICIT_GEMM, nhip.ALGO_WINOGRAD])
def test_config1_single_conv(algo):
    x, wt, b = workloads.conv_single(seed=0)
    d = nhip.conv_desc(64, 64, act=nhip.ACT_RELU, algorithm=algo)
    got = host(nhip.Conv2dF32(d, wt, b).forward(dev(x)))
    exp = oracle_conv(x, wt, b, (1, 1), (1, 1), (1, 1, 1, 1), nhip.ACT_RELU)
    rtol = WINO_RTOL if algo == nhip.ALGO_WINOGRAD else IGEMM_RTOL
    assert_close(got, exp, rtol, f"config1 algo {algo}")


def run_stage(c, hw, n, algo, x, w1, b1, w2, b2):
    """ResNet basic block: relu(conv1) -> relu(conv2 + x)."""
    d1 = nhip.conv_desc(c, c, act=nhip.ACT_RELU, algorithm=algo)
    d2 = nhip.conv_desc(c, c, act=nhip.ACT_RELU, algorithm=algo)
    c1, c2 = nhip.Conv2dF32(d1, w1, b1), nhip.Conv2dF32(d2, w2, b2)
    xd = dev(x)
    y = c1.forward(xd)
    return host(c2.forward(y, residual=xd))


def oracle_stage(x, w1, b1, w2, b2):
    p = (1, 1, 1, 1)
    y = oracle_conv(x, w1, b1, (1, 1), (1, 1), p, nhip.ACT_RELU)
    return oracle_conv(y, w2, b2, (1, 1), (1, 1), p, nhip.ACT_RELU, residual=x)


@pytest.mark.parametrize("stage", workloads.RESNET18_STAGES, ids=lambda s: f"{s[0]}x{s[1]}")
@pytest.mark.parametrize("algo", [nhip.ALGO_IMPLICIT_GEMM, nhip.ALGO_WINOGRAD])
def test_resnet_stage_n2_matches_oracle(stage, algo, wino_variant):
    if algo == nhip.ALGO_IMPLICIT_GEMM and wino_variant != "auto":
        pytest.skip("variant applies to Winograd only")
    c, hw = stage
    x, w1, b1, w2, b2 = workloads.resnet_stage(c, hw, n=2, seed=0)
    got = run_stage(c, hw, 2, algo, x, w1, b1, w2, b2)
    exp = oracle_stage(x, w1, b1, w2, b2)
    rtol = WINO_RTOL if algo == nhip.ALGO_WINOGRAD else IGEMM_RTOL
    assert_close(got, exp, rtol, f"stage {stage} algo {algo}")


@pytest.mark.parametrize("stage", workloads.RESNET18_STAGES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_resnet_stage_full_batch(stage, nhip_env):
    """Batch 32, the bench's exact plans (default per-shape Winograd choice,
    workspace passed the way bench.py passes it): every one of the 32 images
    is checked against the oracle, for Winograd and the implicit GEMM."""
    nhip_env.delenv("NHIP_WINOGRAD_VARIANT", raising=False)
    c, hw = stage
    x, w1, b1, w2, b2 = workloads.resnet_stage(c, hw, n=32, seed=0)
    exp = oracle_stage(x, w1, b1, w2, b2)
    d = nhip.conv_desc(c, c, act=nhip.ACT_RELU, algorithm=nhip.ALGO_WINOGRAD)
    c1, c2 = nhip.Conv2dF32(d, w1, b1), nhip.Conv2dF32(d, w2, b2)
    ws = torch.empty(max(c1.workspace_size(32, hw, hw), c2.workspace_size(32, hw, hw)),
                     dtype=torch.uint8, device="cuda")
    xd = dev(x)
    y = torch.empty_like(xd)
    out = torch.empty_like(xd)
    for rep in range(2):  # the second pass reuses the workspace and outputs, as bench steps do
        c1.forward(xd, out=y, workspace=ws)
        c2.forward(y, residual=xd, out=out, workspace=ws)
        wino = host(out)
        for i in range(32):
            assert_close(wino[i:i + 1], exp[i:i + 1], WINO_RTOL, f"wino image {i} pass {rep}")
        assert max_rel_err(wino, exp) <= WINO_RTOL
    igemm = run_stage(c, hw, 32, nhip.ALGO_IMPLICIT_GEMM, x, w1, b1, w2, b2)
    for i in range(32):
        assert_close(igemm[i:i + 1], exp[i:i + 1], IGEMM_RTOL, f"igemm image {i}")


@pytest.mark.parametrize("variant", ["2", "1", "2split"])
def test_batch_is_independent_images(variant, nhip_env):  # 1 = three-kernel path, 2 = fused (2split: channel splits)
    """The [N,C,H,W] batch equals N single-image calls (the reference ABI),
    bit for bit for a fixed kernel variant."""
    nhip_env.setenv("NHIP_WINOGRAD_VARIANT", variant[0])
    if variant == "2split":
        nhip_env.setenv("NHIP_WINO_SPLITS", "2")
    else:
        nhip_env.delenv("NHIP_WINO_SPLITS", raising=False)
    c, k = 32, 32
    x = RNG.uniform(-1, 1, (4, c, 10, 10)).astype(np.float32)
    wt = workloads.he_normal(RNG, (k, c, 3, 3), c * 9)
    for algo in (nhip.ALGO_IMPLICIT_GEMM, nhip.ALGO_WINOGRAD):
        conv = nhip.Conv2dF32(nhip.conv_desc(c, k, bias=False, algorithm=algo), wt)
        whole = host(conv.forward(dev(x)))
        for i in range(4):
            one = host(conv.forward(dev(x[i:i + 1])))
            np.testing.assert_array_equal(one, whole[i:i + 1])


def test_empty_batch_and_workspace_errors(nhip_env):
    nhip_env.delenv("NHIP_WINOGRAD_VARIANT", raising=False)  # default path needs a workspace
    c, k = 16, 16
    wt = workloads.he_normal(RNG, (k, c, 3, 3), c * 9)
    conv = nhip.Conv2dF32(nhip.conv_desc(c, k, bias=False, algorithm=nhip.ALGO_WINOGRAD), wt)
    x = torch.empty((0, c, 8, 8), device="cuda")
    assert conv.forward(x).shape == (0, k, 8, 8)
    x = dev(RNG.uniform(-1, 1, (1, c, 8, 8)).astype(np.float32))
    need = conv.workspace_size(1, 8, 8)
    assert need > 0
    small = torch.empty(need - 1, dtype=torch.uint8, device="cuda")
    with pytest.raises(nhip.NhipError) as e:
        conv.forward(x, workspace=small)
    assert e.value.status == 5


def test_kernel_timer_counts_launches():
    c, k = 16, 16
    wt = workloads.he_normal(RNG, (k, c, 3, 3), c * 9)
    conv = nhip.Conv2dF32(nhip.conv_desc(c, k, bias=False, algorithm=nhip.ALGO_WINOGRAD), wt)
    # one image: a single Winograd part, one GEMM launch per forward
    x = dev(RNG.uniform(-1, 1, (1, c, 8, 8)).astype(np.float32))
    nhip.timer_start("wino_gemm")
    for _ in range(3):
        conv.forward(x)
    n, ms = nhip.timer_stop()
    assert n == 3 and ms > 0.0
