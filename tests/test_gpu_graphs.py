"""GPU parity at graph level: the MobileNetV2-shape graph (the benchmarked one)
run through libnhip against the same layer list run through the CPU oracle,
layer by layer in the reference's op order (conv + bias, add, relu; depthwise
zero-init + bias; global average pool; InnerProduct zero-init + bias)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import graphs  # noqa: E402
import ncnn_format  # noqa: E402
import nhip  # noqa: E402
from numerics import assert_close, max_rel_err  # noqa: E402
from oracle_graphs import oracle_forward  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nhip.init(0)


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


@pytest.mark.parametrize("n", [2, 32])
def test_native_executor_mobilenetv2_matches_oracle(n):
    """The path bench.py times: the graph from its .param/.bin form through
    the native executor (nhip_graph_run) with its default lowering
    (depthwise->1x1 fusion, pointwise kernel choice by batch size).  On a
    non-default stream the second identical call is recorded into a hipGraph
    and the third replays it; each result is checked against the oracle."""
    layers = graphs.mobilenetv2_layers(seed=0)
    m = ncnn_format.from_layer_list(layers)
    g = nhip.Graph(m.param_text(), bytes(m.payload))
    x = np.random.default_rng(0).uniform(-1, 1, (n, 3, 224, 224)).astype(np.float32)
    exp = oracle_forward(layers, x)["fc"]
    xd = torch.from_numpy(x).cuda()

    def check(got, what):
        torch.cuda.synchronize()
        got = got.cpu().numpy().reshape(n, -1)
        assert_close(got, exp, 1e-4, f"native mobilenetv2 n={n} {what}")
        assert max_rel_err(got, exp) <= 1e-4, what
        np.testing.assert_array_equal(got.argmax(1), exp.argmax(1))

    check(g.run(xd)[0], "default stream")
    out = [torch.empty((n, 1000), device="cuda").fill_(float("nan"))]
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for what in ("eager", "record", "replay", "replay 2"):
            out[0].fill_(float("nan"))
            g.run(xd, out=out, stream=s)
            s.synchronize()
            check(out[0], what)
    g.close()


@pytest.mark.parametrize("mode", ["1", "2"])
@pytest.mark.parametrize("side", [160, 96])
def test_native_executor_mobilenetv2_other_resolutions(nhip_env, side, mode):
    """The MobileNetV2-shape graph declared at 160x160 (planes 80/40/20/10/5)
    and 96x96 (48/24/12/6/3) through the native executor: the expand ->
    depthwise pairs run fused as whole planes (up to 784 pixels, the default
    NHIP_PWDW=1) or also as row strips (NHIP_PWDW=2, the 80x80, 40x40 and
    48x48 planes), at plane sizes the 224x224 graph never produces.  Logits
    within 1e-4 of the oracle, same top-1 class."""
    nhip_env.setenv("NHIP_PWDW", mode)
    layers = graphs.mobilenetv2_layers(seed=1)
    m = ncnn_format.from_layer_list(layers, input_shape=(3, side, side))
    g = nhip.Graph(m.param_text(), bytes(m.payload))
    n = 3
    x = np.random.default_rng(side).uniform(-1, 1, (n, 3, side, side)).astype(np.float32)
    exp = oracle_forward(layers, x)["fc"]
    got = g.run(torch.from_numpy(x).cuda())[0]
    torch.cuda.synchronize()
    got = got.cpu().numpy().reshape(n, -1)
    g.close()
    assert got.shape == (n, 1000)
    assert_close(got, exp, 1e-4, f"native mobilenetv2 {side}x{side} NHIP_PWDW={mode}")
    assert max_rel_err(got, exp) <= 1e-4
    np.testing.assert_array_equal(got.argmax(1), exp.argmax(1))
