"""GPU parity at graph level: the MobileNetV2-shape graph
run through libnhip against the same layer list run through the CPU oracle,
layer by layer in the reference's op order (conv + bias, add, relu; depthwise
zero-init + bias; global average pool; InnerProduct zero-init + bias)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import graphs  # noqa: E402
import nhip  # noqa: E402
from numerics import assert_close, max_rel_err  # noqa: E402
from oracle import refcpu  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nhip.init(0)


def oracle_forward(layers, x):
    blobs = {"data": x}
    for L in layers:
        src = blobs[L["src"]]
        n, c, h, w = src.shape if src.ndim == 4 else (src.shape[0], src.shape[1], 1, 1)
        if L["kind"] == "conv":
            p = L["pad"]
            g = refcpu.geom(n, c, h, w, L["k"], (L["kernel"],) * 2, (L["stride"],) * 2, (1, 1), (p, p, p, p))
            y = refcpu.conv2d_f32(g, src, L["w"], L["b"])
            if L["residual"]:
                y = refcpu.add_f32(y, blobs[L["residual"]])
            if L["act"] == 1:
                y = refcpu.relu_f32(y)
        elif L["kind"] == "dw":
            g = refcpu.geom(n, c, h, w, c, (3, 3), (L["stride"],) * 2, (1, 1), (1, 1, 1, 1))
            y = refcpu.relu_f32(refcpu.dwconv2d_f32(g, src, L["w"], L["b"]))
        elif L["kind"] == "gap":
            y = refcpu.global_avgpool_f32(src)
        elif L["kind"] == "ip":
            y = refcpu.innerproduct_f32(src.reshape(n, -1), L["w"], L["b"])
        blobs[L["dst"]] = y
    return blobs


@pytest.mark.parametrize("n", [2, 32])
def test_mobilenetv2_matches_oracle(n):
    layers = graphs.mobilenetv2_layers(seed=0)
    assert sum(1 for L in layers if L["kind"] == "dw") == 17
    x = np.random.default_rng(0).uniform(-1, 1, (n, 3, 224, 224)).astype(np.float32)
    g = graphs.DeviceGraph(layers)
    got = g.forward(torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    exp = oracle_forward(layers, x)
    assert got.shape == (n, 1000)
    # Every layer is within 1e-4 (implicit GEMM, InnerProduct) or exact
    # (depthwise); 50+ layers in sequence stay within 1e-4 of the oracle.
    assert_close(got, exp["fc"], 1e-4, "mobilenetv2 logits")
    assert max_rel_err(got, exp["fc"]) <= 1e-4
    # same top-1 class per image as the oracle
    np.testing.assert_array_equal(got.argmax(1), exp["fc"].argmax(1))
