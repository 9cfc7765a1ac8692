"""Writer for ncnn .param/.bin model files (the format lib/Graph/graph.cpp and
lib/Graph/parser.cpp of the reference read).

.param: magic 7767517, "layer_count blob_count", then one line per layer
"Type name nbottom ntop bottoms... tops... id=value ...", arrays as
"-(23300+id)=count,v1,...".  .bin: per layer, in layer order, the weights the
layer's loader expects (graph.cpp:1381-1678,1960-2030): tagged payloads (u32
flag, 0 = fp32, 0x000D4B38 = int8 padded to 4 bytes, 0x01306B47 = fp16) for
convolution / InnerProduct weights, raw fp32 for everything else.
"""
from __future__ import annotations

import struct

import numpy as np

FLAG_F32 = 0
FLAG_F16 = 0x01306B47
FLAG_I8 = 0x000D4B38


def _fmt(v):
    if isinstance(v, (list, tuple, np.ndarray)):
        vals = list(v)
        return f"{len(vals)}," + ",".join(_fmt(x) for x in vals)
    if isinstance(v, (float, np.floating)):
        return repr(float(v)) if not float(v).is_integer() else f"{float(v):.1f}"
    return str(int(v))


class Model:
    """Builds an ncnn model layer by layer; save() writes .param and .bin."""

    def __init__(self):
        self.lines = []
        self.blobs = set()
        self.payload = bytearray()

    def _layer(self, typ, name, bottoms, tops, params=None):
        parts = [typ, name, str(len(bottoms)), str(len(tops)), *bottoms, *tops]
        for k, v in (params or {}).items():
            if isinstance(v, (list, tuple, np.ndarray)):
                parts.append(f"{-23300 - k}={_fmt(v)}")
            else:
                parts.append(f"{k}={_fmt(v)}")
        self.lines.append(" ".join(parts))
        self.blobs.update(tops)
        self.blobs.update(bottoms)

    def _tagged(self, arr):
        arr = np.ascontiguousarray(arr)
        if arr.dtype == np.int8:
            data = arr.tobytes()
            self.payload += struct.pack("<I", FLAG_I8) + data + b"\0" * (-len(data) % 4)
        elif arr.dtype == np.float16:
            data = arr.tobytes()
            self.payload += struct.pack("<I", FLAG_F16) + data + b"\0" * (-len(data) % 4)
        else:
            self.payload += struct.pack("<I", FLAG_F32) + arr.astype("<f4").tobytes()

    def _raw(self, arr):
        self.payload += np.ascontiguousarray(arr, dtype="<f4").tobytes()

    # ---------------------------------------------------------------- layers
    def input(self, name, c, h, w):
        """Input blob [c,h,w]; pass 0, 0, 0 to omit the dims (--input-shape)."""
        self._layer("Input", name, [], [name], {0: w, 1: h, 2: c} if c else {})

    def conv(self, name, bottom, top, weight, bias=None, stride=1, pad=1, dilation=1, act=0,
             int8=None, depthwise=False):
        """weight [K][C][kh][kw] (fp32, fp16 or int8).  int8 = dict(term, ws,
        is, os) adds int8_scale_term and its scales.  pad: int or
        (top, bottom, left, right)."""
        k, c, kh, kw = weight.shape
        pt, pb, pl, pr = (pad,) * 4 if np.isscalar(pad) else pad
        sh, sw = (stride, stride) if np.isscalar(stride) else stride
        dh, dw = (dilation, dilation) if np.isscalar(dilation) else dilation
        p = {0: k, 1: kw, 11: kh, 2: dw, 12: dh, 3: sw, 13: sh, 4: pl, 15: pr, 14: pt, 16: pb,
             5: 1 if bias is not None else 0, 6: int(weight.size)}
        if int8:
            p[8] = int8["term"]
        if act:
            p[9] = act
        if depthwise:
            p[7] = k
        self._layer("ConvolutionDepthWise" if depthwise else "Convolution", name, [bottom], [top], p)
        self._tagged(weight)
        if bias is not None:
            self._raw(bias)
        if int8:
            self._raw(np.atleast_1d(int8["ws"]))
            self._raw(np.atleast_1d(np.float32(int8["is"])))
            if int8["term"] > 100:
                self._raw(np.atleast_1d(np.float32(int8["os"])))

    def innerproduct(self, name, bottom, top, weight, bias=None, act=0):
        n, k = weight.shape
        p = {0: n, 1: 1 if bias is not None else 0, 2: int(weight.size)}
        if act:
            p[9] = act
        self._layer("InnerProduct", name, [bottom], [top], p)
        self._tagged(weight)
        if bias is not None:
            self._raw(bias)

    def batchnorm(self, name, bottom, top, slope, mean, var, beta, eps=1e-5):
        self._layer("BatchNorm", name, [bottom], [top], {0: len(slope), 1: float(eps)})
        for a in (slope, mean, var, beta):
            self._raw(a)

    def relu(self, name, bottom, top):
        self._layer("ReLU", name, [bottom], [top])

    def split(self, name, bottom, tops):
        self._layer("Split", name, [bottom], list(tops))

    def add(self, name, a, b, top, eltwise=False):
        if eltwise:
            self._layer("Eltwise", name, [a, b], [top], {0: 1})
        else:
            self._layer("BinaryOp", name, [a, b], [top], {0: 0})

    def global_avgpool(self, name, bottom, top):
        self._layer("Pooling", name, [bottom], [top], {0: 1, 4: 1})

    def reshape(self, name, bottom, top, w):
        self._layer("Reshape", name, [bottom], [top], {0: w})

    def squeeze(self, name, bottom, top, axes):
        self._layer("Squeeze", name, [bottom], [top], {3: list(axes)})

    def quantize(self, name, bottom, top, scale):
        scale = np.atleast_1d(np.asarray(scale, np.float32))
        self._layer("Quantize", name, [bottom], [top], {0: scale.size})
        self._raw(scale)

    def dequantize(self, name, bottom, top, scale, bias=None):
        """Dequantize (graph.cpp:1975-1996): scale [, bias], raw fp32."""
        scale = np.atleast_1d(np.asarray(scale, np.float32))
        p = {0: scale.size}
        if bias is not None:
            bias = np.atleast_1d(np.asarray(bias, np.float32))
            p[1] = bias.size
        self._layer("Dequantize", name, [bottom], [top], p)
        self._raw(scale)
        if bias is not None:
            self._raw(bias)

    def requantize(self, name, bottom, top, in_scale, out_scale, bias=None, act=0):
        """Requantize (graph.cpp:1998-2022): input scale, output scale
        [, bias], raw fp32; activation_type 0 or 1."""
        in_scale = np.atleast_1d(np.asarray(in_scale, np.float32))
        out_scale = np.atleast_1d(np.asarray(out_scale, np.float32))
        p = {0: in_scale.size, 1: out_scale.size}
        if bias is not None:
            bias = np.atleast_1d(np.asarray(bias, np.float32))
            p[2] = bias.size
        if act:
            p[3] = act
        self._layer("Requantize", name, [bottom], [top], p)
        self._raw(in_scale)
        self._raw(out_scale)
        if bias is not None:
            self._raw(bias)

    def layer(self, typ, name, bottoms, tops, params=None):
        """Any other layer type (no weights)."""
        self._layer(typ, name, bottoms, tops, params)

    # ----------------------------------------------------------------- output
    def param_text(self):
        return "7767517\n%d %d\n" % (len(self.lines), len(self.blobs)) + "\n".join(self.lines) + "\n"

    def save(self, param_path, bin_path):
        with open(param_path, "w") as f:
            f.write(self.param_text())
        with open(bin_path, "wb") as f:
            f.write(bytes(self.payload))


def from_layer_list(layers, input_shape=(3, 224, 224)):
    """An ncnn model of a graphs.py layer list (conv / dw / gap / ip records).
    A residual conv becomes Convolution + BinaryOp add; a blob read by more
    than one layer is fanned out through a Split layer, as ncnn models do."""
    steps = []  # (record, bottoms, top)
    for L in layers:
        if L["kind"] == "conv" and L["residual"]:
            if L["act"]:
                raise ValueError("an activation after a residual add needs its own ReLU layer")
            steps.append((dict(L, residual=None), [L["src"]], L["dst"] + "_pre"))
            steps.append((dict(kind="add", name=L["name"] + "_add"), [L["dst"] + "_pre", L["residual"]], L["dst"]))
        else:
            steps.append((L, [L["src"]], L["dst"]))
    uses = {}
    for _, bottoms, _ in steps:
        for b in bottoms:
            uses[b] = uses.get(b, 0) + 1
    taken = {}

    def ref(blob):
        if uses.get(blob, 0) <= 1:
            return blob
        k = taken.get(blob, 0)
        taken[blob] = k + 1
        return f"{blob}_split{k}"

    m = Model()
    c, h, w = input_shape
    m.input("data", c, h, w)

    def fan_out(blob):
        if uses.get(blob, 0) > 1:
            m.split(blob + "_split", blob, [f"{blob}_split{k}" for k in range(uses[blob])])

    fan_out("data")
    for L, bottoms, top in steps:
        bs = [ref(b) for b in bottoms]
        if L["kind"] == "conv":
            m.conv(L["name"], bs[0], top, L["w"], L["b"], stride=L["stride"], pad=L["pad"], act=L["act"])
        elif L["kind"] == "dw":
            m.conv(L["name"], bs[0], top, L["w"], L["b"], stride=L["stride"], pad=1, act=L["act"], depthwise=True)
        elif L["kind"] == "add":
            m.add(L["name"], bs[0], bs[1], top)
        elif L["kind"] == "gap":
            m.global_avgpool(L["name"], bs[0], top)
        elif L["kind"] == "ip":
            m.innerproduct(L["name"], bs[0], top, L["w"], L["b"])
        fan_out(top)
    return m
