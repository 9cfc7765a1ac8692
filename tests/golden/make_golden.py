"""Writes the golden vectors under tests/golden/ for the reference's own
numerical fixtures (test/Numerical/fixtures/*.param, copied verbatim into
tests/golden/params/ as data).

For each case:
  bins/<fixture>.bin   the weight payload, built by the rules of the
                       reference's generators (generate_bins.py:7-83 for fp32 /
                       fp16 fixtures, generate_int8_bins.py:9-72 for int8) —
                       restated here, the reference scripts are not run;
  vectors/<case>.npz   inputs (CHW float32, seeded) and expected outputs.

Expected outputs come from an evaluator written here in numpy, independent of
the C oracle (oracle/refcpu.c) and of the device library:
  - fp32 layers in float64 (textbook direct convolution / matmul / mean), so
    the tests compare at the reference's tolerances (1e-5 .. 1e-6, 0 for
    copies and relu);
  - int8 layers with integer accumulation in int64 and the reference's
    fp32 epilogue sequence applied op by op in numpy float32 (IEEE single, no
    contraction): quantize s = x*scale, floor(s+0.5) / ceil(s-0.5), clamp +-127
    (NCNNToTosa.cpp:322-389); r = ws*is, 1/r, 0 where ws == 0 (:577-637);
    (float)acc * r, + bias (:1294-1300); requantize by the top scale when the
    term is > 100 (:1309-1312); ReLU after (ImportConvolution.cpp:236-241).

The reference's tests draw inputs with std::mt19937 + std::*_distribution
(numerical_test_support.cpp:503-521), which is implementation-defined; these
vectors use numpy's PCG64 seeded with the reference test's seed, same
distribution and range (normal(0,1) for the fp32 operator tests, uniform
[-1.5,1.5] for the int8 tests, int8_ops_test.cpp:30).

Run:  python tests/golden/make_golden.py   (rewrites bins/ and vectors/)
"""
from __future__ import annotations

import os
import random
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import fixture_io as fio  # noqa: E402

PARAMS = os.path.join(HERE, "params")
BINS = os.path.join(HERE, "bins")
VECTORS = os.path.join(HERE, "vectors")

# case -> (fixture, [(input blob, CHW shape)], seed, distribution, tolerance,
#          compile-time input shapes or None).  Shapes, seeds and tolerances
# are those of test/Numerical/operators/{supported_ops,int8_ops,dynamic_ops}_test.cpp.
N = "normal"
U15 = ("uniform", -1.5, 1.5)
CASES = {
    "convolution": ("convolution", [("data", (1, 4, 4))], 0x434F4E56, N, 1e-5, None),
    "convolution_no_bias": ("convolution_no_bias", [("data", (1, 4, 4))], 0x434E4249, N, 1e-5, None),
    "convolution_dilated": ("convolution_dilated", [("data", (1, 7, 7))], 0x4344494C, N, 1e-5, None),
    "convolution_asymmetric": ("convolution_asymmetric", [("data", (1, 4, 4))], 0x43415359, N, 1e-5, None),
    "convolution_asymmetric_stride": ("convolution_asymmetric_stride", [("data", (1, 9, 8))], 0x43415354, N,
                                      1e-5, None),
    "convolution_same_upper": ("convolution_same_upper", [("data", (1, 5, 5))], 0x43535550, N, 1e-5, None),
    "convolution_same_lower": ("convolution_same_lower", [("data", (1, 5, 5))], 0x43534C4F, N, 1e-5, None),
    "convolution_fp16_storage": ("convolution_fp16_storage", [("data", (1, 4, 4))], 0x46313643, N, 1e-5, None),
    "convolution_depthwise": ("convolution_depthwise", [("data", (2, 5, 5))], 0x44574356, N, 1e-5, None),
    "convolution_depthwise_fp16_storage": ("convolution_depthwise_fp16_storage", [("data", (2, 5, 5))],
                                           0x46313644, N, 1e-5, None),
    "convolution_depthwise_7x7": ("convolution_depthwise_7x7", [("data", (96, 4, 5))], 0x44573737, N, 1e-5, None),
    "convolution_depthwise_9x9": ("convolution_depthwise_9x9", [("data", (256, 4, 5))], 0x44573939, N, 1e-5,
                                  None),
    "convolution_depthwise_asymmetric": ("convolution_depthwise_asymmetric", [("data", (2, 11, 9))], 0x44574153,
                                         N, 1e-5, None),
    "convolution_depthwise_same_upper": ("convolution_depthwise_same_upper", [("data", (2, 4, 5))], 0x44535550,
                                         N, 1e-5, None),
    "convolution_depthwise_same_lower": ("convolution_depthwise_same_lower", [("data", (2, 4, 5))], 0x44534C4F,
                                         N, 1e-5, None),
    "inner_product": ("inner_product", [("data", (1, 1, 8))], 0x49505054, N, 1e-6, None),
    "inner_product_dynamic_m_rows3": ("inner_product_dynamic_m", [("data", (1, 3, 4))], 0x1AAE2, N, 1e-5,
                                      [(1, -1, 4)]),
    "inner_product_dynamic_m_rows7": ("inner_product_dynamic_m", [("data", (1, 7, 4))], 0x1AAE2, N, 1e-5,
                                      [(1, -1, 4)]),
    "inner_product_fused_relu": ("inner_product_fused_relu", [("data", (2, 1, 3))], 0x49504652, N, 1e-6, None),
    "binary_add": ("binary_add", [("first", (2, 3, 4)), ("second", (2, 3, 4))], 0x42414431, N, 0.0, None),
    "relu": ("relu", [("data", (3, 4, 5))], 0x52454C55, N, 0.0, None),
    "dropout": ("dropout", [("data", (3, 4, 5))], 0x44524F50, N, 0.0, None),
    "split": ("split", [("data", (3, 4, 5))], 0x53504C54, N, 0.0, None),
    "pooling_global_average": ("pooling_global_average", [("data", (2, 5, 5))], 0x50474156, N, 1e-6, None),
    "pooling_global_average_ignored_params": ("pooling_global_average_ignored_params", [("data", (2, 4, 5))],
                                              0x50474941, N, 1e-6, None),
    "pooling_global_average_dynamic": ("pooling_global_average_dynamic", [("data", (3, 6, 5))], 0x610BA1,
                                       ("uniform", -2.0, 2.0), 1e-6, [(3, -1, -1)]),
    "convolution_int8_term1": ("convolution_int8_term1", [("data", (2, 3, 4))], 0xC001, U15, 0.0, [(2, 3, 4)]),
    "convolution_int8_term2": ("convolution_int8_term2", [("data", (2, 3, 4))], 0xC002, U15, 0.0, [(2, 3, 4)]),
    "convolution_int8_term101": ("convolution_int8_term101", [("data", (2, 3, 4))], 0xC101, U15, 0.0,
                                 [(2, 3, 4)]),
    "convolution_int8_term102": ("convolution_int8_term102", [("data", (2, 3, 4))], 0xC102, U15, 0.0,
                                 [(2, 3, 4)]),
    "depthwise_int8_term1": ("depthwise_int8_term1", [("data", (3, 3, 4))], 0xD001, U15, 0.0, [(3, 3, 4)]),
    "depthwise_int8_term2": ("depthwise_int8_term2", [("data", (3, 3, 4))], 0xD002, U15, 0.0, [(3, 3, 4)]),
    "depthwise_int8_term101": ("depthwise_int8_term101", [("data", (3, 3, 4))], 0xD101, U15, 0.0, [(3, 3, 4)]),
    "depthwise_int8_term102": ("depthwise_int8_term102", [("data", (3, 3, 4))], 0xD102, U15, 0.0, [(3, 3, 4)]),
    "inner_product_int8_term1": ("inner_product_int8_term1", [("data", (1, 1, 4))], 0x1F01, U15, 0.0,
                                 [(1, 1, 4)]),
    "inner_product_int8_term2": ("inner_product_int8_term2", [("data", (1, 1, 4))], 0x1F02, U15, 0.0,
                                 [(1, 1, 4)]),
    "int8_complete_chain": ("int8_complete_chain", [("data", (2, 3, 4))], 0x8C11, U15, 0.0, [(2, 3, 4)]),
}


# ---------------------------------------------------------------- payloads
# generate_bins.py:9-31 (kernel_count, bias_count)
FP32_SIZES = {
    "convolution": (18, 2), "convolution_no_bias": (18, 0), "convolution_dilated": (8, 2),
    "convolution_asymmetric": (12, 0), "convolution_asymmetric_stride": (12, 0),
    "convolution_same_upper": (18, 0), "convolution_same_lower": (18, 0),
    "convolution_fp16_storage": (18, 2), "convolution_depthwise": (18, 2),
    "convolution_depthwise_fp16_storage": (18, 2), "convolution_depthwise_7x7": (4704, 96),
    "convolution_depthwise_9x9": (20736, 256), "convolution_depthwise_asymmetric": (12, 2),
    "convolution_depthwise_same_upper": (18, 0), "convolution_depthwise_same_lower": (18, 0),
    "inner_product": (24, 3), "inner_product_dynamic_m": (12, 3), "inner_product_fused_relu": (24, 4),
}
# generate_bins.py:76-82 (the hand-written convolution weights)
CONV_CONSTANTS = [0.25, -0.5, 0.75, -1.0, 0.5, 0.125, 0.375, -0.25, 1.0,
                  -0.125, 0.625, -0.75, 0.5, 0.25, -0.375, 0.875, -0.625, 0.125]


def fp32_payload(fixture: str) -> bytes:
    """generate_bins.py:45-83 for the fixtures of this path."""
    if fixture not in FP32_SIZES:
        return b""
    kc, bc = FP32_SIZES[fixture]
    if fixture.endswith("fp16_storage"):
        rng = random.Random(0x46313657)
        w = [rng.uniform(-0.25, 0.25) for _ in range(kc)]
        b = [rng.uniform(-0.1, 0.1) for _ in range(bc)]
        return fio.tagged_f16(w) + fio.raw_f32(b)
    if fixture in ("convolution_depthwise_7x7", "convolution_depthwise_9x9"):
        rng = random.Random(0x44573758 if fixture.endswith("7x7") else 0x44573958)
        w = [rng.uniform(-0.025, 0.025) for _ in range(kc)]
        b = [rng.uniform(-0.01, 0.01) for _ in range(bc)]
    elif fixture.startswith("convolution_depthwise") or fixture.startswith("inner_product"):
        rng = random.Random(0x4E434E4E if fixture.startswith("convolution_depthwise") else 0x49505052)
        w = [rng.uniform(-0.25, 0.25) for _ in range(kc)]
        b = [rng.uniform(-0.1, 0.1) for _ in range(bc)]
    else:
        w = CONV_CONSTANTS[:kc]
        b = [0.125, -0.25][:bc]
    return fio.tagged_f32(w) + fio.raw_f32(b)


def int8_conv(term, cin, cout):
    """generate_int8_bins.py:19-29."""
    data = fio.tagged_i8([((i * 7 + 3) % 15) - 7 for i in range(cin * cout)])
    data += fio.raw_f32([0.125 * (i - 1) for i in range(cout)])
    data += fio.raw_f32([5.0 + i * 1.5 for i in range(cout)])
    data += fio.raw_f32([8.0])
    if term > 100:
        data += fio.raw_f32([6.0])
    return data


def int8_depthwise(term, channels):
    """generate_int8_bins.py:32-42."""
    data = fio.tagged_i8([((i * 5 + 1) % 11) - 5 for i in range(channels)])
    data += fio.raw_f32([0.1 * (i - 1) for i in range(channels)])
    data += fio.raw_f32([4.0 + i for i in range(channels if term in (1, 101) else 1)])
    data += fio.raw_f32([7.0])
    if term > 100:
        data += fio.raw_f32([5.0])
    return data


def int8_inner_product():
    """generate_int8_bins.py:45-52."""
    return (fio.tagged_i8([3, -2, 1, 4, -4, 2, 5, -1, 2, 3, -3, 1]) + fio.raw_f32([0.25, -0.5, 0.125])
            + fio.raw_f32([4.0, 6.0, 8.0]) + fio.raw_f32([9.0]))


def int8_payload(fixture: str) -> bytes:
    """generate_int8_bins.py:65-83."""
    if fixture in ("convolution_int8_term1", "convolution_int8_term2"):
        return int8_conv(1 if fixture.endswith("term1") else 2, 2, 3)
    if fixture in ("convolution_int8_term101", "convolution_int8_term102"):
        return int8_conv(101 if fixture.endswith("101") else 102, 2, 3) + int8_conv(1, 3, 2)
    if fixture in ("depthwise_int8_term1", "depthwise_int8_term2"):
        return int8_depthwise(1 if fixture.endswith("term1") else 2, 3)
    if fixture in ("depthwise_int8_term101", "depthwise_int8_term102"):
        return int8_depthwise(101 if fixture.endswith("101") else 102, 3) + int8_depthwise(1, 3)
    if fixture.startswith("inner_product_int8"):
        return int8_inner_product()
    if fixture == "int8_complete_chain":
        return int8_conv(101, 2, 3) + int8_depthwise(101, 3) + int8_conv(1, 3, 2)
    raise KeyError(fixture)


def payload(fixture: str) -> bytes:
    if "int8" in fixture:
        return int8_payload(fixture)
    return fp32_payload(fixture)


# -------------------------------------------------------------- evaluator
def conv_params(p, ih, iw):
    kw = p[1]
    kh = p.get(11, kw)
    dw = p.get(2, 1)
    dh = p.get(12, dw)
    sw = p.get(3, 1)
    sh = p.get(13, sw)
    pl = p.get(4, 0)
    pr = p.get(15, pl)
    pt = p.get(14, pl)
    pb = p.get(16, pt)
    if pl in (-233, -234):
        # SAME_UPPER / SAME_LOWER (NormalizeNCNN.cpp:31-51)
        def same(n, k, s, d):
            extent = d * (k - 1) + 1
            out = 1 + (n - 1) // s
            total = max((out - 1) * s + extent - n, 0)
            before = total // 2 + (total % 2 if pl == -234 else 0)
            return before, total - before
        pt, pb = same(ih, kh, sh, dh)
        pl, pr = same(iw, kw, sw, dw)
    return kh, kw, dh, dw, sh, sw, pt, pb, pl, pr


def direct_conv_f64(x, w, b, group, p):
    """Textbook grouped convolution in float64. x [C,H,W], w [K, C/g, kh, kw]."""
    c, ih, iw = x.shape
    k = w.shape[0]
    kh, kw, dh, dw, sh, sw, pt, pb, pl, pr = conv_params(p, ih, iw)
    xp = np.zeros((c, ih + pt + pb, iw + pl + pr))
    xp[:, pt:pt + ih, pl:pl + iw] = x
    oh = (ih + pt + pb - (dh * (kh - 1) + 1)) // sh + 1
    ow = (iw + pl + pr - (dw * (kw - 1) + 1)) // sw + 1
    cg, kg = c // group, k // group
    out = np.zeros((k, oh, ow))
    for o in range(k):
        g = o // kg
        for ci in range(cg):
            for u in range(kh):
                for v in range(kw):
                    out[o] += w[o, ci, u, v] * xp[g * cg + ci, u * dh:u * dh + sh * (oh - 1) + 1:sh,
                                                  v * dw:v * dw + sw * (ow - 1) + 1:sw]
        if b is not None:
            out[o] += b[o]
    return out


def int_conv(xq, wq, group, p):
    """Exact integer convolution (int64) of int8 tensors."""
    return np.rint(direct_conv_f64(xq.astype(np.float64), wq.astype(np.float64), None, group, p)).astype(np.int64)


def quantize(x, scale):
    """NCNNToTosa.cpp:322-389 in float32: per element (scalar scale) or per dim-0 channel."""
    x = np.asarray(x, np.float32)
    scale = np.asarray(scale, np.float32)
    s = x * (scale.reshape((-1,) + (1,) * (x.ndim - 1)) if scale.size > 1 else scale.reshape(()))
    s = s.astype(np.float32)
    r = np.where(s >= 0, np.floor((s + np.float32(0.5)).astype(np.float32)),
                 np.ceil((s - np.float32(0.5)).astype(np.float32)))
    return np.clip(r, -127, 127).astype(np.int8)


def int8_epilogue(acc, bias, ws, is_, term, act, os_):
    """acc [K,...] int64 -> float32 or int8 (term > 100)."""
    k = acc.shape[0]
    ws = np.broadcast_to(np.asarray(ws, np.float32), (k,))
    c = (ws * np.float32(is_)).astype(np.float32)
    with np.errstate(divide="ignore"):
        r = (np.float32(1.0) / c).astype(np.float32)
    r = np.where(ws == 0, np.float32(0), r).astype(np.float32)
    shape = (k,) + (1,) * (acc.ndim - 1)
    f = (acc.astype(np.int32).astype(np.float32) * r.reshape(shape)).astype(np.float32)
    if bias is not None:
        f = (f + np.asarray(bias, np.float32).reshape(shape)).astype(np.float32)
    if term > 100:
        q = quantize(f, np.float32(os_))
        return np.maximum(q, 0).astype(np.int8) if act == 1 else q
    return np.maximum(f, np.float32(0)) if act == 1 else f


def evaluate(layers, inputs):
    """inputs: {blob: CHW float32} -> {blob: array}."""
    blobs = dict(inputs)
    for L in layers:
        ty, p, W = L["type"], L["params"], L.get("weights")
        bt = L["bottoms"]
        if ty == "Input":
            continue
        x = blobs[bt[0]] if bt else None
        if ty in ("Convolution", "ConvolutionDepthWise"):
            k = p[0]
            kw = p[1]
            kh = p.get(11, kw)
            group = p.get(7, 1) if ty == "ConvolutionDepthWise" else 1
            c = x.shape[0]
            w = W["weight"].reshape(k, -1, kh, kw)
            term = p.get(8, 0)
            if term == 0:
                y = direct_conv_f64(x.astype(np.float64), w.astype(np.float64), W.get("bias"), group, p)
                if p.get(9, 0) == 1:
                    y = np.maximum(y, 0)
            else:
                ws = W["weight_scale"]
                if W["weight_dtype"] == "f32":
                    w = np.stack([quantize(w[o], ws[o] if ws.size > 1 else ws[0]) for o in range(k)])
                xq = x if x.dtype == np.int8 else quantize(x, np.float32(W["bottom_scale"]))
                acc = int_conv(xq, w, group, p)
                y = int8_epilogue(acc, W.get("bias"), ws, W["bottom_scale"], term, p.get(9, 0),
                                  W.get("top_scale", 1.0))
            assert c % group == 0
        elif ty == "InnerProduct":
            n = p[0]
            w = W["weight"].reshape(n, -1)
            # a rank-2 blob is [M, K] (dynamic-M, NCNNToTosa.cpp:5290-5304);
            # anything else is flattened to one row of K
            flat = x if x.ndim == 2 else x.reshape(1, -1)
            if p.get(8, 0):
                ws = W["weight_scale"]
                xq = flat if flat.dtype == np.int8 else quantize(flat, np.float32(W["bottom_scale"]))
                acc = xq.astype(np.int64) @ w.astype(np.int64).T
                y = int8_epilogue(acc.T, W.get("bias"), ws, W["bottom_scale"], 1, p.get(9, 0), 1.0).T
            else:
                y = flat.astype(np.float64) @ w.astype(np.float64).T
                if "bias" in W:
                    y = y + W["bias"]
                if p.get(9, 0) == 1:
                    y = np.maximum(y, 0)
            y = y if x.ndim == 2 else y.reshape(-1)
        elif ty == "ReLU":
            y = np.maximum(x, 0).astype(x.dtype)
        elif ty in ("Dropout", "Noop"):
            y = x
        elif ty == "Split":
            for t in L["tops"]:
                blobs[t] = x
            continue
        elif ty == "BinaryOp":
            assert p.get(0, 0) == 0
            y = x.astype(np.float64) + blobs[bt[1]].astype(np.float64)
        elif ty == "Pooling":
            assert p.get(0, 0) == 1 and p.get(4, 0) == 1
            y = x.astype(np.float64).reshape(x.shape[0], -1).mean(axis=1)
        elif ty == "Reshape":
            y = x.reshape(p[0])
        elif ty == "Squeeze":
            axes = p.get(3, [])
            y = np.squeeze(x, axis=tuple(axes)) if axes else np.squeeze(x)
        else:
            raise NotImplementedError(ty)
        blobs[L["tops"][0]] = y
    return blobs


def graph_outputs(layers):
    consumed = {b for L in layers for b in L["bottoms"]}
    return [t for L in layers for t in L["tops"] if t not in consumed]


def make_inputs(inputs, seed, dist):
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in inputs:
        if dist == N:
            out[name] = rng.standard_normal(shape).astype(np.float32)
        else:
            _, lo, hi = dist
            out[name] = rng.uniform(lo, hi, shape).astype(np.float32)
    return out


def load_fixture(fixture, bin_bytes=None):
    layers = fio.parse_param(open(os.path.join(PARAMS, fixture + ".param")).read())
    if bin_bytes is None:
        bin_bytes = payload(fixture)
    used = fio.load_weights(layers, bin_bytes)
    assert used == len(bin_bytes), (fixture, used, len(bin_bytes))
    return layers


def expected_for(case):
    fixture, inputs, seed, dist, _, _ = CASES[case]
    layers = load_fixture(fixture)
    xs = make_inputs(inputs, seed, dist)
    blobs = evaluate(layers, {k: v for k, v in xs.items()})
    outs = graph_outputs(layers)
    return xs, {o: blobs[o] for o in outs}


def main():
    os.makedirs(BINS, exist_ok=True)
    os.makedirs(VECTORS, exist_ok=True)
    for fixture in sorted({c[0] for c in CASES.values()}):
        with open(os.path.join(BINS, fixture + ".bin"), "wb") as f:
            f.write(payload(fixture))
    for case in CASES:
        xs, outs = expected_for(case)
        arrays = {f"in_{k}": v for k, v in xs.items()}
        for k, v in outs.items():
            arrays[f"out_{k}"] = v if v.dtype == np.int8 else v.astype(np.float64)
        np.savez(os.path.join(VECTORS, case + ".npz"), **arrays)
    print(f"wrote {len(CASES)} cases")


if __name__ == "__main__":
    main()
