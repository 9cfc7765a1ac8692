"""The reference's own numerical fixtures (test/Numerical/fixtures/*.param, in
tests/golden/params/) with the golden vectors of tests/golden/make_golden.py,
on the CPU:

- the committed .bin payloads are exactly what the generator rules produce
  (generate_bins.py / generate_int8_bins.py restated), and the committed
  vectors are reproducible;
- the oracle (oracle/refcpu.c) run over each fixture agrees with the
  independent numpy evaluator at the reference test's tolerance (int8 and
  copies bit-exact), which pins the oracle on the reference's fixtures;
- the device library's front end (nhip_graph_describe: parser, weight loader,
  lowering, shape inference; no device work) accepts every fixture and
  reports the golden input/output shapes and element types.
"""
import os
import sys

import numpy as np
import pytest

import golden_oracle
import nhip

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden as mg  # noqa: E402

CASES = sorted(mg.CASES)


def vectors(case):
    with np.load(os.path.join(mg.VECTORS, case + ".npz")) as z:
        return {k: z[k] for k in z.files}


def committed_bin(fixture):
    with open(os.path.join(mg.BINS, fixture + ".bin"), "rb") as f:
        return f.read()


def assert_golden(got, exp, tol, what):
    exp32 = exp.astype(got.dtype) if got.dtype == np.int8 else exp
    assert got.shape == exp.shape, (what, got.shape, exp.shape)
    if tol == 0.0 or got.dtype == np.int8:
        np.testing.assert_array_equal(got, exp32.astype(got.dtype), err_msg=what)
    else:
        # compare_values(actual, expected, abs, rel) of the reference tests
        err = np.abs(got.astype(np.float64) - exp)
        bound = tol + tol * np.abs(exp)
        assert (err <= bound).all(), f"{what}: max err {err.max():.3g}"


@pytest.mark.parametrize("fixture", sorted({c[0] for c in mg.CASES.values()}))
def test_committed_bin_matches_generator_rules(fixture):
    assert committed_bin(fixture) == mg.payload(fixture)


def test_generator_rules_known_bytes():
    # generate_int8_bins.py:9-16: int8 tag, payload padded to 4 bytes
    b = mg.int8_depthwise(101, 3)
    assert b[:4] == (0x000D4B38).to_bytes(4, "little")
    assert list(np.frombuffer(b[4:7], np.int8)) == [-4, 1, -5]  # ((i*5+1)%11)-5
    assert b[7] == 0 and len(b) == 8 + 4 * (3 + 3 + 1 + 1)
    # generate_bins.py:76-83: flag 0, weights then bias
    c = mg.fp32_payload("convolution")
    assert c[:4] == b"\0\0\0\0" and len(c) == 4 + 4 * 20
    assert np.frombuffer(c, "<f4", 2, 4 + 72).tolist() == [0.125, -0.25]


@pytest.mark.parametrize("case", CASES)
def test_vectors_reproducible(case):
    xs, outs = mg.expected_for(case)
    z = vectors(case)
    for k, v in xs.items():
        np.testing.assert_array_equal(z["in_" + k], v)
    for k, v in outs.items():
        np.testing.assert_array_equal(z["out_" + k], v.astype(np.float64) if v.dtype != np.int8 else v)


@pytest.mark.parametrize("case", CASES)
def test_oracle_matches_golden(case):
    fixture, inputs, _, _, tol, _ = mg.CASES[case]
    layers = mg.load_fixture(fixture, committed_bin(fixture))
    z = vectors(case)
    blobs = golden_oracle.run(layers, {name: z["in_" + name] for name, _ in inputs})
    for key in z:
        if key.startswith("out_"):
            assert_golden(np.asarray(blobs[key[4:]]), z[key], tol, f"{case}:{key}")


def test_int8_fixture_golden_hand_value():
    # convolution_int8_term1, output channel 0 at pixel 0 by hand: weights
    # ((i*7+3)%15)-7 -> w[0] = (-4, 3); is = 8, ws[0] = 5, bias[0] = -0.125
    z = vectors("convolution_int8_term1")
    x = z["in_data"][:, 0, 0]
    q = [int(mg.quantize(np.float32(v), np.float32(8.0))) for v in x]
    acc = -4 * q[0] + 3 * q[1]
    r = np.float32(1.0) / np.float32(40.0)
    exp = np.float32(np.float32(acc) * r) + np.float32(-0.125)
    assert z["out_output"][0, 0, 0] == exp


@pytest.mark.parametrize("case", CASES)
def test_front_end_accepts_fixture_and_reports_golden_io(case):
    fixture, inputs, _, _, _, shapes = mg.CASES[case]
    param = open(os.path.join(mg.PARAMS, fixture + ".param")).read()
    g = nhip.Graph(param, committed_bin(fixture), shapes, describe_only=True)
    z = vectors(case)
    assert [io["name"] for io in g.inputs] == [name for name, _ in inputs]
    concrete = [shape for _, shape in inputs]
    outs = g.infer_shapes(concrete)
    expected = {k[4:]: v for k, v in z.items() if k.startswith("out_")}
    assert sorted(io["name"] for io in g.outputs) == sorted(expected)
    for io, shape in zip(g.outputs, outs):
        assert shape == expected[io["name"]].shape, (io["name"], shape)
        assert io["dtype"] == np.float32
    with pytest.raises(nhip.NhipError) as e:
        g.run_host(*[z["in_" + name] for name, _ in inputs])
    assert e.value.status == 3
