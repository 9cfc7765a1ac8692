"""Oracle execution of graphs.py layer lists (test helper, not collected)."""
from oracle import refcpu


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
