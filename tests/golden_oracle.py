"""Runs a parsed reference fixture (tests/golden/fixture_io.py layers) through
the CPU oracle, layer by layer (test helper, not collected).  Each layer maps
onto the oracle function restating the reference lowering it names."""
import numpy as np

from oracle import refcpu


def _pads(p, ih, iw, kh, kw, sh, sw, dh, dw):
    pl = p.get(4, 0)
    pr = p.get(15, pl)
    pt = p.get(14, pl)
    pb = p.get(16, pt)
    if pl in (-233, -234):
        pt, pb = refcpu.same_padding(ih, kh, sh, dh, pl)
        pl, pr = refcpu.same_padding(iw, kw, sw, dw, pl)
    return pt, pb, pl, pr


def _geom(p, x, k):
    c, ih, iw = x.shape
    kw = p[1]
    kh = p.get(11, kw)
    dw = p.get(2, 1)
    dh = p.get(12, dw)
    sw = p.get(3, 1)
    sh = p.get(13, sw)
    pads = _pads(p, ih, iw, kh, kw, sh, sw, dh, dw)
    return refcpu.geom(1, c, ih, iw, k, (kh, kw), (sh, sw), (dh, dw), pads), kh, kw


def run(layers, inputs):
    blobs = dict(inputs)
    for L in layers:
        ty, p, W, bt = L["type"], L["params"], L.get("weights"), L["bottoms"]
        if ty == "Input":
            continue
        x = blobs[bt[0]]
        act = p.get(9, 0)
        if ty in ("Convolution", "ConvolutionDepthWise"):
            k = p[0]
            g, kh, kw = _geom(p, x, k)
            term = p.get(8, 0)
            dw = ty == "ConvolutionDepthWise"
            w = W["weight"].reshape(k, -1, kh, kw)
            if term == 0:
                fn = refcpu.dwconv2d_f32 if dw else refcpu.conv2d_f32
                y = fn(g, x[None], w, W.get("bias"))[0]
                if act == 1:
                    y = refcpu.relu_f32(y)
            else:
                ws = W["weight_scale"]
                if W["weight_dtype"] == "f32":
                    wsf = np.broadcast_to(ws, (k,))
                    w = np.stack([refcpu.quantize_f32_i8(w[o], wsf[o:o + 1]) for o in range(k)])
                fn = refcpu.dwconv2d_int8 if dw else refcpu.conv2d_int8
                y = fn(g, x[None], w, W.get("bias"), ws, W["bottom_scale"], W.get("top_scale", 1.0), term, act)[0]
        elif ty == "InnerProduct":
            n = p[0]
            w = W["weight"].reshape(n, -1)
            x2 = x if x.ndim == 2 else x.reshape(1, -1)
            if p.get(8, 0):
                y = refcpu.innerproduct_int8(x2, w, W.get("bias"), W["weight_scale"], W["bottom_scale"], act)
            else:
                y = refcpu.innerproduct_f32(x2, w, W.get("bias"))
                if act == 1:
                    y = refcpu.relu_f32(y)
            y = y if x.ndim == 2 else y.reshape(-1)
        elif ty == "ReLU":
            y = refcpu.relu_i8(x) if x.dtype == np.int8 else refcpu.relu_f32(x)
        elif ty in ("Dropout", "Noop"):
            y = x
        elif ty == "Split":
            for t in L["tops"]:
                blobs[t] = x
            continue
        elif ty == "BinaryOp":
            y = refcpu.add_f32(x, blobs[bt[1]])
        elif ty == "Pooling":
            y = refcpu.global_avgpool_f32(x[None])[0]
        elif ty == "Reshape":
            y = x.reshape(p[0])
        elif ty == "Squeeze":
            y = np.squeeze(x, axis=tuple(p.get(3, [])))
        else:
            raise NotImplementedError(ty)
        blobs[L["tops"][0]] = y
    return blobs
