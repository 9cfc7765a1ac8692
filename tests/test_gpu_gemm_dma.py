"""GPU parity of the direct-to-LDS fp32 GEMM (csrc/gemm_dma.hip) on its two
contractions, against the CPU oracle: InnerProduct (ConvertInnerProduct,
NCNNToTosa.cpp:5254-5392) and the 1x1 stride-1 convolution over NCHW
(ConvertConvolution fp32, :1316-1529), within the implicit-GEMM budget of
max relative error 1e-4.  Every case runs with the kernel on (NHIP_GEMM_DMA=1,
the default; 64- and 128-row tiles) and off (the register-prefetch kernels).  Shapes cover rows, columns and reductions that are not
multiples of the 64 x 64 tile and 32-wide stage, split K, residual add,
pixel columns that cross image boundaries and a misaligned input view."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import nhip  # noqa: E402
from numerics import assert_close, max_rel_err  # noqa: E402
from oracle import refcpu  # noqa: E402

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(71)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nhip.init(0)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def set_dma(env, mode):
    """mode "1": the kernel with 64-row tiles (for every supported shape),
    "128": 128-row tiles where M allows, "0": off."""
    env.setenv("NHIP_GEMM_DMA", "0" if mode == "0" else "2")
    env.setenv("NHIP_GEMM_DMA_BM", "128" if mode == "128" else "64")


@pytest.mark.parametrize("m,k,n,act", [
    (256, 2048, 1000, 0),   # the benchmarked InnerProduct
    (32, 1280, 1000, 0),    # MobileNetV2 head at batch 32 (split K)
    (1, 1280, 1000, 1),
    (7, 132, 65, 1),        # k not a multiple of 32, n past one tile
    (70, 2052, 3, 0),       # two row tiles, long reduction, 3 outputs
    (130, 36, 200, 1),      # three row tiles, one stage
    (300, 1000, 130, 1),    # reduction not a multiple of 256, ragged blocks
])
@pytest.mark.parametrize("dma", ["kq", "1", "128", "0"])
def test_innerproduct(m, k, n, act, dma, nhip_env):
    """Mode "kq" forces the one-workgroup-per-block kernel (csrc/ip_kq.hip,
    reductions up to 2048; longer ones fall back to the tiled GEMMs); the
    other modes switch it off."""
    nhip_env.setenv("NHIP_IP_KQ", "1" if dma == "kq" else "0")
    set_dma(nhip_env, "1" if dma == "kq" else dma)
    x = RNG.uniform(-1, 1, (m, k)).astype(np.float32)
    w = (RNG.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
    b = RNG.normal(0, 0.01, n).astype(np.float32)
    ip = nhip.InnerProductF32(w, b, act)
    got = host(ip.forward(torch.from_numpy(x).cuda()))
    exp = refcpu.innerproduct_f32(x, w, b)
    if act:
        exp = refcpu.relu_f32(exp)
    assert_close(got, exp, 1e-4, f"ip {m}x{k}x{n} dma={dma}")
    assert max_rel_err(got, exp) <= 1e-4
    # a 4-byte-offset input (not 16-byte aligned) takes the other kernel
    buf = torch.empty(x.size + 1, dtype=torch.float32, device="cuda")
    xv = buf[1:].view(x.shape)
    xv.copy_(torch.from_numpy(x).cuda())
    assert_close(host(ip.forward(xv)), exp, 1e-4, f"ip {m}x{k}x{n} misaligned")


@pytest.mark.parametrize("n,c,k,h,w,res", [
    (32, 160, 960, 7, 7, False),    # MobileNetV2 expand at 7x7
    (32, 960, 160, 7, 7, True),     # project with residual (split K)
    (32, 320, 1280, 7, 7, False),   # head 1x1
    (4, 576, 160, 7, 7, False),
    (2, 37, 70, 5, 9, True),        # channels not a multiple of 4 or 32
    (3, 512, 33, 3, 3, False),      # 9-pixel planes, split K, 33 outputs
    (1, 8, 5, 1, 1, False),
    (5, 64, 96, 14, 14, True),
])
@pytest.mark.parametrize("dma", ["1", "128", "0"])
def test_pointwise_conv(n, c, k, h, w, res, dma, nhip_env):
    set_dma(nhip_env, dma)
    nhip_env.setenv("NHIP_POINTWISE", "0")  # not the pointwise streaming kernel
    x = RNG.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = (RNG.standard_normal((k, c, 1, 1)) * np.sqrt(2.0 / c)).astype(np.float32)
    b = RNG.normal(0, 0.01, k).astype(np.float32)
    r = RNG.uniform(-1, 1, (n, k, h, w)).astype(np.float32) if res else None
    d = nhip.conv_desc(c, k, (1, 1), (1, 1), (1, 1), (0, 0, 0, 0), bias=True, act=1)
    plan = nhip.Conv2dF32(d, wt, b)
    got = host(plan.forward(torch.from_numpy(x).cuda(),
                            residual=None if r is None else torch.from_numpy(r).cuda()))
    exp = refcpu.conv2d_f32(refcpu.geom(n, c, h, w, k, (1, 1), (1, 1), (1, 1), (0, 0, 0, 0)), x, wt, b)
    if r is not None:
        exp = refcpu.add_f32(exp, r)
    exp = refcpu.relu_f32(exp)
    assert_close(got, exp, 1e-4, f"1x1 {(n, c, k, h, w)} dma={dma}")
    assert max_rel_err(got, exp) <= 1e-4
