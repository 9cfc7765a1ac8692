"""Reading and writing the reference's numerical fixtures (test helper).

`.param` text: the ncnn format of lib/Graph/parser.cpp and docs/ncnn-ir-format.md
(magic 7767517, "layers blobs", then one layer per line:
`type name n_bottom n_top bottoms... tops... key=value...`; a key -233xx is an
array "count,v1,...", an integer unless a value holds '.', 'e' or 'E').

`.bin` payloads: a tagged weight is a u32 flag (0 or 0x0002C056 = fp32,
0x01306B47 = fp16, 0x000D4B38 = int8) followed by the data, fp16/int8 padded to
4 bytes; a raw weight (bias, scales) is fp32 with no flag
(lib/Graph/graph.cpp:1260-1327).  Per-layer order follows the loaders of
graph.cpp:1381-1678: Convolution/ConvolutionDepthWise = weight (tagged), bias
[num_output] if 5=1, and when 8 (int8_scale_term) != 0 the weight scales
([num_output] for Convolution; [group] for depthwise terms 1/101 else [1]), the
bottom scale [1], and the top scale [1] when the term is > 100; InnerProduct =
weight (tagged), bias if 1=1, and for 8 != 0 weight scales [num_output] and
the bottom scale [1].
"""
from __future__ import annotations

import struct

import numpy as np

FLAG_F32 = (0, 0x0002C056)
FLAG_F16 = 0x01306B47
FLAG_I8 = 0x000D4B38


def _value(text):
    if any(ch in text for ch in ".eE"):
        return float(text)
    return int(text)


def parse_param(text: str):
    """-> list of dicts {type, name, bottoms, tops, params}."""
    lines = [ln.split() for ln in text.splitlines() if ln.strip()]
    assert lines[0] == ["7767517"], "bad magic"
    layers = []
    for tok in lines[2:]:
        ty, name, nb, nt = tok[0], tok[1], int(tok[2]), int(tok[3])
        bottoms = tok[4:4 + nb]
        tops = tok[4 + nb:4 + nb + nt]
        params = {}
        for kv in tok[4 + nb + nt:]:
            k, v = kv.split("=", 1)
            k = int(k)
            if k <= -23300:
                vals = v.split(",")
                params[-k - 23300] = [_value(x) for x in vals[1:1 + int(vals[0])]]
            else:
                params[k] = _value(v)
        layers.append(dict(type=ty, name=name, bottoms=bottoms, tops=tops, params=params))
    return layers


class Cursor:
    def __init__(self, data: bytes):
        self.data, self.pos = data, 0

    def raw_f32(self, count):
        out = np.frombuffer(self.data, "<f4", count, self.pos).astype(np.float32)
        self.pos += 4 * count
        return out

    def tagged(self, count):
        """-> (array, dtype name); fp16 is promoted to fp32 exactly."""
        flag = struct.unpack_from("<I", self.data, self.pos)[0]
        self.pos += 4
        if flag in FLAG_F32:
            return self.raw_f32(count), "f32"
        if flag == FLAG_F16:
            out = np.frombuffer(self.data, "<f2", count, self.pos).astype(np.float32)
            self.pos += (2 * count + 3) // 4 * 4
            return out, "f32"
        if flag == FLAG_I8:
            out = np.frombuffer(self.data, np.int8, count, self.pos).copy()
            self.pos += (count + 3) // 4 * 4
            return out, "i8"
        raise ValueError(f"unknown weight flag {flag:#x}")


def load_weights(layers, data: bytes):
    """Attach 'weights' (dict) to each weighted layer; returns bytes consumed."""
    cur = Cursor(data)
    for L in layers:
        p, ty = L["params"], L["type"]
        if ty in ("Convolution", "ConvolutionDepthWise"):
            k, term = p.get(0, 0), p.get(8, 0)
            w, wdt = cur.tagged(p[6])
            W = dict(weight=w, weight_dtype=wdt)
            if p.get(5, 0):
                W["bias"] = cur.raw_f32(k)
            if term:
                if ty == "Convolution":
                    n_ws = k
                else:
                    n_ws = p.get(7, 1) if term in (1, 101) else 1
                W["weight_scale"] = cur.raw_f32(n_ws)
                W["bottom_scale"] = float(cur.raw_f32(1)[0])
            if term > 100:
                W["top_scale"] = float(cur.raw_f32(1)[0])
            L["weights"] = W
        elif ty == "InnerProduct":
            n = p.get(0, 0)
            w, wdt = cur.tagged(p[2])
            W = dict(weight=w, weight_dtype=wdt)
            if p.get(1, 0):
                W["bias"] = cur.raw_f32(n)
            if p.get(8, 0):
                W["weight_scale"] = cur.raw_f32(n)
                W["bottom_scale"] = float(cur.raw_f32(1)[0])
            L["weights"] = W
    return cur.pos


def tagged_f32(values):
    return struct.pack("<I", 0) + struct.pack(f"<{len(values)}f", *values)


def tagged_f16(values):
    body = struct.pack(f"<{len(values)}e", *values)
    return struct.pack("<I", FLAG_F16) + body + bytes((-len(body)) % 4)


def tagged_i8(values):
    body = struct.pack(f"<{len(values)}b", *values)
    return struct.pack("<I", FLAG_I8) + body + bytes((-len(body)) % 4)


def raw_f32(values):
    return struct.pack(f"<{len(values)}f", *values)
