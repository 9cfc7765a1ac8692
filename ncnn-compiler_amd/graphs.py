"""Graph-level workloads built from libnhip layers.

A graph is a list of layer records (plain data: kind, ncnn parameters,
weights, input/output blob names), so the same list drives the device
runner here and the oracle chain in the tests.  Blob names follow ncnn's
.param convention: every layer consumes and produces named blobs.

MobileNetV2 (the benchmarked graph): width 1.0, 224x224 input, the standard
(t, c, n, s) table, BN folded into the convolution biases, ReLU after the
stem, every expand and every depthwise conv (the reference's Convolution and
ConvolutionDepthWise importers accept no ReLU6, ImportConvolution.cpp:63-72,
ImportOps.cpp:869-875), residual add where stride 1 and channels match,
1x1 conv to 1280, global average pooling and InnerProduct 1280->1000.
"""
from __future__ import annotations

import numpy as np

import nhip
import workloads

MBV2_SETTINGS = ((1, 16, 1, 1), (6, 24, 2, 2), (6, 32, 3, 2), (6, 64, 4, 2),
                 (6, 96, 3, 1), (6, 160, 3, 2), (6, 320, 1, 1))


def _bias(rng, k):
    return (rng.standard_normal(k) * 0.01).astype(np.float32)


def mobilenetv2_layers(seed=0, num_classes=1000):
    """Layer records of the MobileNetV2-shape graph with seeded He-init weights."""
    rng = np.random.default_rng([seed, 5])
    layers = []

    def conv(name, src, c, k, kernel, stride, pad, act, residual=None):
        w = workloads.he_normal(rng, (k, c, kernel, kernel), c * kernel * kernel)
        layers.append(dict(kind="conv", name=name, src=src, dst=name, c=c, k=k, kernel=kernel,
                           stride=stride, pad=pad, act=act, residual=residual, w=w, b=_bias(rng, k)))
        return name

    def dw(name, src, c, stride):
        w = workloads.he_normal(rng, (c, 1, 3, 3), 9)
        layers.append(dict(kind="dw", name=name, src=src, dst=name, c=c, stride=stride, act=1,
                           w=w, b=_bias(rng, c)))
        return name

    x = conv("stem", "data", 3, 32, 3, 2, 1, 1)
    cin = 32
    idx = 0
    for t, c, n, s in MBV2_SETTINGS:
        for i in range(n):
            stride = s if i == 0 else 1
            hidden = cin * t
            blk = f"b{idx}"
            h = x
            if t != 1:
                h = conv(f"{blk}_expand", h, cin, hidden, 1, 1, 0, 1)
            h = dw(f"{blk}_dw", h, hidden, stride)
            res = x if (stride == 1 and cin == c) else None
            x = conv(f"{blk}_project", h, hidden, c, 1, 1, 0, 0, residual=res)
            cin = c
            idx += 1
    x = conv("head", x, cin, 1280, 1, 1, 0, 1)
    layers.append(dict(kind="gap", name="pool", src=x, dst="pool"))
    w = (rng.standard_normal((num_classes, 1280)) / np.sqrt(1280)).astype(np.float32)
    layers.append(dict(kind="ip", name="fc", src="pool", dst="fc", w=w, b=_bias(rng, num_classes)))
    return layers


def graph_flops(layers, n, h, w):
    """Direct-equivalent FLOPs of the conv / depthwise / InnerProduct layers."""
    shapes = {"data": (3, h, w)}
    total = 0.0
    for L in layers:
        c, hh, ww = shapes[L["src"]]
        if L["kind"] in ("conv", "dw"):
            k = L["k"] if L["kind"] == "conv" else L["c"]
            ker = L.get("kernel", 3)
            pad = L.get("pad", 1)
            oh = (hh + 2 * pad - ker) // L["stride"] + 1
            ow = (ww + 2 * pad - ker) // L["stride"] + 1
            per = (c if L["kind"] == "conv" else 1) * ker * ker
            total += 2.0 * n * k * oh * ow * per
            shapes[L["dst"]] = (k, oh, ow)
        elif L["kind"] == "gap":
            shapes[L["dst"]] = (c, 1, 1)
        elif L["kind"] == "ip":
            total += 2.0 * n * L["w"].shape[0] * L["w"].shape[1]
            shapes[L["dst"]] = (L["w"].shape[0], 1, 1)
    return total


def graph_bytes(layers, n, h, w):
    """Algorithmic HBM bytes of the graph run layer by layer (fp32): every
    layer reads its input(s) and weights once and writes its output once (a
    residual operand is read once more)."""
    shapes = {"data": (3, h, w)}
    total = 0.0
    for L in layers:
        c, hh, ww = shapes[L["src"]]
        inp = n * c * hh * ww
        if L["kind"] in ("conv", "dw"):
            k = L["k"] if L["kind"] == "conv" else L["c"]
            ker = L.get("kernel", 3)
            pad = L.get("pad", 1)
            oh = (hh + 2 * pad - ker) // L["stride"] + 1
            ow = (ww + 2 * pad - ker) // L["stride"] + 1
            out = n * k * oh * ow
            wts = L["w"].size + L["b"].size
            total += 4.0 * (inp + wts + out + (out if L.get("residual") else 0))
            shapes[L["dst"]] = (k, oh, ow)
        elif L["kind"] == "gap":
            total += 4.0 * (inp + n * c)
            shapes[L["dst"]] = (c, 1, 1)
        elif L["kind"] == "ip":
            total += 4.0 * (n * L["w"].shape[1] + L["w"].size + L["b"].size + n * L["w"].shape[0])
            shapes[L["dst"]] = (L["w"].shape[0], 1, 1)
    return total


class DeviceGraph:
    """Runs a layer list on the GPU through the libnhip C ABI.

    Plans (prepacked weights) are created once; activations live in device
    memory allocated per distinct (blob, batch) and reused across calls.
    """

    def __init__(self, layers):
        import torch
        self.torch = torch
        self.layers = layers
        self.plans = {}
        for L in layers:
            if L["kind"] == "conv":
                p = L["pad"]
                d = nhip.conv_desc(L["c"], L["k"], (L["kernel"],) * 2, (L["stride"],) * 2, (1, 1),
                                   (p, p, p, p), bias=True, act=L["act"])
                self.plans[L["name"]] = nhip.Conv2dF32(d, L["w"], L["b"])
            elif L["kind"] == "dw":
                d = nhip.conv_desc(L["c"], L["c"], (3, 3), (L["stride"],) * 2, (1, 1), (1, 1, 1, 1),
                                   bias=True, act=L["act"], group=L["c"])
                self.plans[L["name"]] = nhip.DwConv2dF32(d, L["w"], L["b"])
            elif L["kind"] == "ip":
                self.plans[L["name"]] = nhip.InnerProductF32(L["w"], L["b"])
        self._buffers = {}
        self._ws = None

    def _buf(self, name, shape):
        key = (name, tuple(shape))
        t = self._buffers.get(key)
        if t is None:
            t = self.torch.empty(shape, dtype=self.torch.float32, device="cuda")
            self._buffers[key] = t
        return t

    def _workspace(self, nbytes):
        if nbytes == 0:
            return None
        if self._ws is None or self._ws.numel() < nbytes:
            self._ws = self.torch.empty(nbytes, dtype=self.torch.uint8, device="cuda")
        return self._ws

    def forward(self, x):
        """x: [N,3,H,W] fp32 device tensor -> logits [N, classes]."""
        blobs = {"data": x}
        n = x.shape[0]
        for L in self.layers:
            src = blobs[L["src"]]
            plan = self.plans.get(L["name"])
            if L["kind"] == "conv":
                _, _, h, w = src.shape
                oh, ow = nhip.output_shape(plan.desc, h, w)
                out = self._buf(L["dst"], (n, L["k"], oh, ow))
                res = blobs[L["residual"]] if L["residual"] else None
                ws = self._workspace(plan.workspace_size(n, h, w))
                plan.forward(src, residual=res, out=out, workspace=ws)
            elif L["kind"] == "dw":
                _, c, h, w = src.shape
                oh, ow = nhip.output_shape(plan.desc, h, w)
                out = self._buf(L["dst"], (n, c, oh, ow))
                plan.forward(src, out=out)
            elif L["kind"] == "gap":
                out = nhip.global_avgpool(src)
            elif L["kind"] == "ip":
                ws = self._workspace(plan.workspace_size(n))
                out = plan.forward(src.reshape(n, -1), workspace=ws)
            blobs[L["dst"]] = out
        return blobs[self.layers[-1]["dst"]]
