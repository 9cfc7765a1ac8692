"""GPU: the graph executor's hipGraph replay (nhip_graph_run records the
call plan on the second call with the same buffers and replays it after;
replay needs a non-default stream, which every test here runs on) gives the
eager executor's results bit for bit: on every replay, with the program's
own device work and synchronizations between replays, after the input
changes in place, on another stream, when a tuning setting changes (which
must re-record, not replay a stale plan), with fresh output tensors, and
after a larger batch has reallocated the executor's buffers."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import graphs  # noqa: E402
import ncnn_format  # noqa: E402
import nhip  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    nhip.init(0)


@pytest.fixture(autouse=True)
def _side_stream():
    """Replay needs a capturable stream: torch's default stream is the legacy
    null stream (handle 0), on which the executor always runs eagerly."""
    s = torch.cuda.Stream()
    assert s.cuda_stream != 0
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        yield
    torch.cuda.synchronize()


def mobilenet_graph():
    m = ncnn_format.from_layer_list(graphs.mobilenetv2_layers(seed=0))
    return nhip.Graph(m.param_text(), bytes(m.payload))


def eager(g, x, nhip_env):
    nhip_env.setenv("NHIP_GRAPH_REPLAY", "0")
    out = g.run(x)[0].clone()
    torch.cuda.synchronize()
    nhip_env.delenv("NHIP_GRAPH_REPLAY")
    return out


def test_replay_matches_eager_on_every_call(nhip_env):
    nhip_env.delenv("NHIP_GRAPH_REPLAY", raising=False)
    g = mobilenet_graph()
    rng = np.random.default_rng(1)
    x = torch.from_numpy(rng.uniform(-1, 1, (2, 3, 224, 224)).astype(np.float32)).cuda()
    ref = eager(g, x, nhip_env)
    out = [torch.empty_like(ref)]
    for call in range(6):  # call 0: eager, 1: eager + recorded, 2..5: replays
        out[0].fill_(float("nan"))
        torch.cuda.synchronize()
        g.run(x, out=out)
        torch.cuda.synchronize()
        assert torch.equal(out[0], ref), f"call {call} differs from the eager run"
        scratch = torch.randn(1 << 20, device="cuda") * 2  # unrelated eager work between replays
        torch.cuda.synchronize()
        del scratch
    # new input values in the same buffer: the replay reads them
    x.copy_(torch.from_numpy(rng.uniform(-1, 1, (2, 3, 224, 224)).astype(np.float32)))
    ref2 = eager(g, x, nhip_env)
    assert not torch.equal(ref2, ref)
    for _ in range(3):
        g.run(x, out=out)
        torch.cuda.synchronize()
        assert torch.equal(out[0], ref2)
    # on another stream: the recorded plan is launched there
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            out[0].zero_()
            g.run(x, out=out)
    torch.cuda.synchronize()
    assert torch.equal(out[0], ref2)


def test_default_stream_runs_eagerly_and_correct(nhip_env):
    nhip_env.delenv("NHIP_GRAPH_REPLAY", raising=False)
    g = mobilenet_graph()
    x = torch.from_numpy(np.random.default_rng(5).uniform(-1, 1, (2, 3, 224, 224)).astype(np.float32)).cuda()
    ref = eager(g, x, nhip_env)
    out = [torch.empty_like(ref)]
    torch.cuda.synchronize()
    with torch.cuda.stream(torch.cuda.default_stream()):
        for _ in range(3):
            g.run(x, out=out)
    torch.cuda.synchronize()
    assert torch.equal(out[0], ref)


def test_setting_change_rerecords(nhip_env):
    """NHIP_DWPW picks fused or separate depthwise -> 1x1 kernels: after a
    recorded plan exists, changing it must give that setting's eager result."""
    nhip_env.delenv("NHIP_GRAPH_REPLAY", raising=False)
    g = mobilenet_graph()
    x = torch.from_numpy(np.random.default_rng(2).uniform(-1, 1, (2, 3, 224, 224)).astype(np.float32)).cuda()
    out = [torch.empty((2, 1000), device="cuda")]
    for setting in ("1", "0", "2", "1"):
        nhip_env.setenv("NHIP_DWPW", setting)
        ref = eager(g, x, nhip_env)
        for _ in range(3):
            g.run(x, out=out)
            torch.cuda.synchronize()
            assert torch.equal(out[0], ref), f"NHIP_DWPW={setting}"


def test_changing_outputs_stay_eager_and_correct(nhip_env):
    """Fresh output tensors on every call (no out=) never reuse a recorded
    plan with stale pointers."""
    nhip_env.delenv("NHIP_GRAPH_REPLAY", raising=False)
    g = mobilenet_graph()
    x = torch.from_numpy(np.random.default_rng(3).uniform(-1, 1, (2, 3, 224, 224)).astype(np.float32)).cuda()
    ref = eager(g, x, nhip_env)
    keep = [g.run(x)[0] for _ in range(4)]  # kept alive: every call has new output pointers
    torch.cuda.synchronize()
    for o in keep:
        assert torch.equal(o, ref)


def test_outputs_written_in_place_or_copied_agree(nhip_env):
    """An aligned output buffer receives the last layer's result directly (no
    copy after it); a view 4 bytes past an aligned base, and an output that
    overlaps the input, are written by a copy after the last layer instead.
    Each equals the eager result, recorded and replayed as well."""
    nhip_env.delenv("NHIP_GRAPH_REPLAY", raising=False)
    g = mobilenet_graph()
    x = torch.from_numpy(np.random.default_rng(5).uniform(-1, 1, (2, 3, 224, 224)).astype(np.float32)).cuda()
    ref = eager(g, x, nhip_env)
    aligned = torch.empty_like(ref)
    assert aligned.data_ptr() % 256 == 0
    base = torch.empty(ref.numel() + 1, device="cuda")
    misaligned = base[1:].view(ref.shape)
    for out in (aligned, misaligned):
        for call in range(4):  # eager, eager + recorded, replays
            out.fill_(float("nan"))
            g.run(x, out=[out])
            torch.cuda.synchronize()
            assert torch.equal(out, ref), f"call {call}, output at {out.data_ptr() % 256} mod 256"
    # the output over the first bytes of the input: the input must survive
    # until the last layer, so the result arrives by the final copy
    xin = x.clone()
    over = xin.view(-1)[: ref.numel()].view(ref.shape)
    g.run(xin, out=[over])
    torch.cuda.synchronize()
    assert torch.equal(over, ref)


def test_buffers_grown_by_a_larger_batch_invalidate_the_recorded_plan(nhip_env):
    """A recorded plan uses the executor's blob buffers; a call with a larger
    batch reallocates them, and the next call with the recorded key must not
    replay the plan over the freed buffers."""
    nhip_env.delenv("NHIP_GRAPH_REPLAY", raising=False)
    g = mobilenet_graph()
    rng = np.random.default_rng(4)
    xa = torch.from_numpy(rng.uniform(-1, 1, (2, 3, 224, 224)).astype(np.float32)).cuda()
    xb = torch.from_numpy(rng.uniform(-1, 1, (4, 3, 224, 224)).astype(np.float32)).cuda()
    ref_a = eager(g, xa, nhip_env)
    ref_b = eager(g, xb, nhip_env)  # the executor's buffers now hold batch 4
    g2 = mobilenet_graph()
    out_a, out_b = [torch.empty_like(ref_a)], [torch.empty_like(ref_b)]
    for _ in range(3):  # records and replays batch 2
        g2.run(xa, out=out_a)
    torch.cuda.synchronize()
    assert torch.equal(out_a[0], ref_a)
    for _ in range(2):  # grows every buffer
        g2.run(xb, out=out_b)
    torch.cuda.synchronize()
    assert torch.equal(out_b[0], ref_b)
    for _ in range(3):  # the batch-2 key again: buffers changed since it was recorded
        out_a[0].zero_()
        g2.run(xa, out=out_a)
        torch.cuda.synchronize()
        assert torch.equal(out_a[0], ref_a)


def test_calls_inside_a_callers_capture_run_eagerly_into_it(nhip_env):
    """A caller capturing its own stream (torch.cuda.graph): the executor
    sees the capture, records nothing of its own and launches eagerly into
    the caller's graph; no error is left behind for later calls, and every
    replay of the caller's graph gives the eager result."""
    nhip_env.delenv("NHIP_GRAPH_REPLAY", raising=False)
    g = mobilenet_graph()
    rng = np.random.default_rng(5)
    x = torch.from_numpy(rng.uniform(-1, 1, (2, 3, 224, 224)).astype(np.float32)).cuda()
    ref = eager(g, x, nhip_env)
    out = [torch.empty_like(ref)]
    s = torch.cuda.current_stream()
    g.run(x, out=out, stream=s)  # sizes every buffer before the capture
    torch.cuda.synchronize()
    cg = torch.cuda.CUDAGraph()
    with torch.cuda.graph(cg, stream=s):
        for _ in range(2):  # twice: the second would record if the capture went unseen
            g.run(x, out=out, stream=s)
    torch.cuda.synchronize()
    for rep in range(4):
        out[0].fill_(float("nan"))
        torch.cuda.synchronize()
        _ = torch.ones(1 << 20, device="cuda").sum()  # the program's own eager work between replays
        cg.replay()
        torch.cuda.synchronize()
        assert torch.equal(out[0], ref), f"replay {rep} of the caller's graph"
    # the next call of the library succeeds and is still correct
    out[0].fill_(float("nan"))
    g.run(x, out=out, stream=s)
    torch.cuda.synchronize()
    assert torch.equal(out[0], ref)
    del cg
    g.close()


def test_larger_call_after_a_callers_capture_keeps_its_buffers(nhip_env):
    """After a caller's capture at batch 2, a call at batch 4 grows the
    executor's buffers; the buffers the caller's graph was captured with stay
    allocated, so replaying it still gives the batch-2 result."""
    nhip_env.delenv("NHIP_GRAPH_REPLAY", raising=False)
    g = mobilenet_graph()
    rng = np.random.default_rng(6)
    xa = torch.from_numpy(rng.uniform(-1, 1, (2, 3, 224, 224)).astype(np.float32)).cuda()
    xb = torch.from_numpy(rng.uniform(-1, 1, (4, 3, 224, 224)).astype(np.float32)).cuda()
    ref_a = eager(g, xa, nhip_env)
    g.close()
    g = mobilenet_graph()
    out_a = [torch.empty_like(ref_a)]
    s = torch.cuda.current_stream()
    g.run(xa, out=out_a, stream=s)  # sizes the buffers for batch 2
    torch.cuda.synchronize()
    cg = torch.cuda.CUDAGraph()
    with torch.cuda.graph(cg, stream=s):
        g.run(xa, out=out_a, stream=s)
    torch.cuda.synchronize()
    out_b = g.run(xb, stream=s)  # grows every buffer past the captured ones
    torch.cuda.synchronize()
    ref_b = eager(mobilenet_graph(), xb, nhip_env)
    assert torch.equal(out_b[0], ref_b)
    for rep in range(3):
        out_a[0].fill_(float("nan"))
        scratch = torch.randn(1 << 22, device="cuda")  # allocations that could reuse freed memory
        torch.cuda.synchronize()
        cg.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_a[0], ref_a), f"replay {rep} after the larger call"
        del scratch
    del cg
    g.close()


def test_capture_that_would_grow_buffers_fails_cleanly(nhip_env):
    """A call inside a caller's capture on a graph whose buffers are too small
    for it fails with status 3 and launches nothing; the capture stays valid
    and the next call outside it runs normally."""
    nhip_env.delenv("NHIP_GRAPH_REPLAY", raising=False)
    g = mobilenet_graph()
    x = torch.from_numpy(np.random.default_rng(7).uniform(-1, 1, (2, 3, 224, 224)).astype(np.float32)).cuda()
    ref = eager(mobilenet_graph(), x, nhip_env)
    out = [torch.empty_like(ref)]
    s = torch.cuda.current_stream()
    cg = torch.cuda.CUDAGraph()
    with torch.cuda.graph(cg, stream=s):
        out[0].zero_()
        with pytest.raises(nhip.NhipError) as err:
            g.run(x, out=out, stream=s)  # never run before: every buffer would have to grow
    assert err.value.status == 3
    torch.cuda.synchronize()
    cg.replay()
    torch.cuda.synchronize()
    assert torch.count_nonzero(out[0]) == 0
    g.run(x, out=out, stream=s)
    torch.cuda.synchronize()
    assert torch.equal(out[0], ref)
    del cg
    g.close()


def test_run_leaves_the_callers_current_device():
    g = mobilenet_graph()
    x = torch.zeros((1, 3, 224, 224), device="cuda")
    before = torch.cuda.current_device()
    g.run(x)
    assert torch.cuda.current_device() == before
    g.close()
