"""GPU parity of global average pooling fused with the InnerProduct that
reads it (nhip_global_avgpool_innerproduct_f32_forward; the head of
MobileNet-style graphs): against the oracle's global average pooling
(ConvertPooling, NCNNToTosa.cpp:1880-1990) followed by its InnerProduct
(ConvertInnerProduct, :5254-5392), within the InnerProduct budget 1e-4,
and through the graph executor, which fuses Pooling -> InnerProduct when
NHIP_GAP_IP=1."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import ncnn_format  # noqa: E402
import nhip  # noqa: E402
from numerics import assert_close, max_rel_err  # noqa: E402
from oracle import refcpu  # noqa: E402

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(31)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nhip.init(0)


def oracle(x, w, b, act):
    y = refcpu.innerproduct_f32(refcpu.global_avgpool_f32(x), w, b)
    return refcpu.relu_f32(y) if act else y


@pytest.mark.parametrize("n,c,h,w,k,act", [
    (32, 1280, 7, 7, 1000, 0),    # the MobileNetV2 head at batch 32
    (1, 1280, 7, 7, 1000, 1),
    (5, 37, 3, 5, 70, 1),         # channels not a multiple of 4, few outputs, ragged images
    (17, 512, 1, 1, 300, 0),      # 1x1 planes, 17 images (two row groups)
    (3, 4096, 2, 2, 513, 0),      # long reduction: many splits
    (3, 100, 40, 40, 30, 1),      # 1600-pixel planes: 16 channels per slice, one image per pass
    (2, 24, 80, 80, 50, 0),       # 6400 pixels, the largest plane: 4 channels per slice
    (40, 64, 7, 7, 10, 0),        # three row groups, the last one partial
])
def test_gap_innerproduct_matches_oracle(n, c, h, w, k, act):
    x = RNG.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = (RNG.standard_normal((k, c)) / np.sqrt(c)).astype(np.float32)
    b = (RNG.standard_normal(k) * 0.01).astype(np.float32)
    ip = nhip.InnerProductF32(wt, b, activation=act)
    got = ip.forward_pooled(torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    exp = oracle(x, wt, b, act)
    assert_close(got, exp, 1e-4, f"gap+ip {(n, c, h, w, k)}")
    assert max_rel_err(got, exp) <= 1e-4
    # the same as the two standalone device ops
    sep = ip.forward(nhip.global_avgpool(torch.from_numpy(x).cuda()).reshape(n, c))
    torch.cuda.synchronize()
    assert_close(got, sep.cpu().numpy(), 1e-5, "fused vs separate")


def test_gap_innerproduct_pools_bit_exact():
    """The fused kernel's means are the oracle's bit for bit: with a single
    output of weight 1 over one channel the InnerProduct is the mean itself
    (one MFMA product 1 * mean, plus bias 0)."""
    x = RNG.uniform(-1, 1, (33, 1, 7, 7)).astype(np.float32)
    ip = nhip.InnerProductF32(np.ones((1, 1), np.float32), np.zeros(1, np.float32))
    got = ip.forward_pooled(torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), refcpu.global_avgpool_f32(x))
    np.testing.assert_array_equal(nhip.global_avgpool(torch.from_numpy(x).cuda()).cpu().numpy(),
                                  refcpu.global_avgpool_f32(x))


def test_gap_innerproduct_rejects_large_planes():
    ip = nhip.InnerProductF32(np.ones((10, 8), np.float32))
    for call in (lambda: ip.gap_workspace_size(2, 81, 80),
                 lambda: ip.forward_pooled(torch.zeros((2, 8, 81, 80), device="cuda"))):
        with pytest.raises(nhip.NhipError) as e:
            call()
        assert e.value.status == 3  # NHIP_STATUS_CONSTRAINT_VIOLATION


def test_gap_innerproduct_rejects_mismatched_channels():
    ip = nhip.InnerProductF32(np.ones((10, 8), np.float32))
    with pytest.raises(nhip.NhipError) as e:
        ip.forward_pooled(torch.zeros((2, 9, 3, 3), device="cuda"))
    assert e.value.status == 2


@pytest.mark.parametrize("flatten", [False, True])
def test_graph_fuses_pooling_into_innerproduct(flatten, nhip_env):
    """Convolution -> Pooling (global average) [-> Flatten] -> InnerProduct:
    fused (NHIP_GAP_IP=1) and unfused (=0, the default) runs both match the
    oracle chain."""
    c, k, hw, n = 48, 200, 9, 6
    wc = (RNG.standard_normal((c, 16, 3, 3)) * 0.1).astype(np.float32)
    bc = RNG.standard_normal(c).astype(np.float32) * 0.01
    wi = (RNG.standard_normal((k, c)) / np.sqrt(c)).astype(np.float32)
    bi = RNG.standard_normal(k).astype(np.float32) * 0.01
    m = ncnn_format.Model()
    m.input("data", 16, hw, hw)
    m.conv("conv", "data", "feat", wc, bc, act=1)
    m.global_avgpool("pool", "feat", "pooled")
    src = "pooled"
    if flatten:
        m.layer("Flatten", "flat", ["pooled"], ["flat"])
        src = "flat"
    m.innerproduct("fc", src, "logits", wi, bi)
    x = RNG.uniform(-1, 1, (n, 16, hw, hw)).astype(np.float32)
    feat = refcpu.relu_f32(refcpu.conv2d_f32(refcpu.geom(n, 16, hw, hw, c), x, wc, bc))
    exp = oracle(feat, wi, bi, 0)
    for setting in ("1", "0"):
        nhip_env.setenv("NHIP_GAP_IP", setting)
        g = nhip.Graph(m.param_text(), bytes(m.payload))
        got = g.run(torch.from_numpy(x).cuda())[0]
        torch.cuda.synchronize()
        got = got.cpu().numpy().reshape(n, k)
        assert_close(got, exp, 1e-4, f"graph gap+ip fused={setting}")
        g.close()


def test_graph_large_planes_run_unfused(nhip_env):
    """Pooling over 81x81 planes (beyond the fused kernel) -> InnerProduct:
    the graph runs the two ops and matches the oracle."""
    c, k, hw, n = 8, 20, 81, 2
    wi = (RNG.standard_normal((k, c)) / np.sqrt(c)).astype(np.float32)
    bi = RNG.standard_normal(k).astype(np.float32) * 0.01
    m = ncnn_format.Model()
    m.input("data", c, hw, hw)
    m.global_avgpool("pool", "data", "pooled")
    m.innerproduct("fc", "pooled", "logits", wi, bi)
    x = RNG.uniform(-1, 1, (n, c, hw, hw)).astype(np.float32)
    g = nhip.Graph(m.param_text(), bytes(m.payload))
    got = g.run(torch.from_numpy(x).cuda())[0]
    torch.cuda.synchronize()
    assert_close(got.cpu().numpy().reshape(n, k), oracle(x, wi, bi, 0), 1e-4, "graph gap+ip, 81x81 planes")
    g.close()
