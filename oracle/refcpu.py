"""ctypes binding of oracle/librefcpu.so (the CPU restatement of the reference).

TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker / timed CPU baseline, never by the
product.  Every function takes and returns numpy arrays; batches are [N,C,H,W]
stacks of independent ncnn [C,H,W] blobs.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "librefcpu.so")
_lib = None


class ConvGeom(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int32) for name in (
        "n", "c", "h", "w", "k", "kernel_h", "kernel_w", "stride_h", "stride_w",
        "dilation_h", "dilation_w", "pad_top", "pad_bottom", "pad_left",
        "pad_right")]


def build() -> None:
    """Compile librefcpu.so with its Makefile (gcc, no GPU needed)."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "librefcpu.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.ref_quantize_one.restype = ctypes.c_int8
        _lib.ref_quantize_one.argtypes = [ctypes.c_float, ctypes.c_float]
        _lib.ref_conv_out_h.argtypes = [ctypes.POINTER(ConvGeom)]
        _lib.ref_conv_out_w.argtypes = [ctypes.POINTER(ConvGeom)]
        _lib.ref_bn_fold.restype = ctypes.c_int
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def geom(n, c, h, w, k, kernel=(3, 3), stride=(1, 1), dilation=(1, 1),
         pad=(1, 1, 1, 1)):
    """pad = (top, bottom, left, right)."""
    return ConvGeom(n, c, h, w, k, kernel[0], kernel[1], stride[0], stride[1],
                    dilation[0], dilation[1], pad[0], pad[1], pad[2], pad[3])


def out_hw(g: ConvGeom):
    L = lib()
    return L.ref_conv_out_h(ctypes.byref(g)), L.ref_conv_out_w(ctypes.byref(g))


def conv2d_f32(g: ConvGeom, x, w, b=None, threads=0):
    x, w, b = _f32(x), _f32(w), _f32(b)
    oh, ow = out_hw(g)
    out = np.empty((g.n, g.k, oh, ow), np.float32)
    lib().ref_conv2d_f32(ctypes.byref(g), _p(x), _p(w), _p(b), _p(out),
                         ctypes.c_int(threads))
    return out


def dwconv2d_f32(g: ConvGeom, x, w, b=None, threads=0):
    x, w, b = _f32(x), _f32(w), _f32(b)
    oh, ow = out_hw(g)
    out = np.empty((g.n, g.k, oh, ow), np.float32)
    lib().ref_dwconv2d_f32(ctypes.byref(g), _p(x), _p(w), _p(b), _p(out),
                           ctypes.c_int(threads))
    return out


def innerproduct_f32(x, w, b=None, threads=0):
    x, w, b = _f32(x), _f32(w), _f32(b)
    m, k = x.shape
    n = w.shape[0]
    out = np.empty((m, n), np.float32)
    lib().ref_innerproduct_f32(ctypes.c_int32(m), ctypes.c_int32(k),
                               ctypes.c_int32(n), _p(x), _p(w), _p(b), _p(out),
                               ctypes.c_int(threads))
    return out


def quantize_one(x: float, scale: float) -> int:
    return int(lib().ref_quantize_one(ctypes.c_float(x), ctypes.c_float(scale)))


def quantize_f32_i8(x, scale, channel_size=None):
    x = _f32(x)
    scale = _f32(np.atleast_1d(scale))
    out = np.empty(x.shape, np.int8)
    cs = 1 if channel_size is None else channel_size
    lib().ref_quantize_f32_i8(ctypes.c_int64(x.size), _p(x), _p(scale),
                              ctypes.c_int32(scale.size), ctypes.c_int64(cs),
                              _p(out))
    return out


def dequant_reciprocal(weight_scale, input_scale):
    ws = _f32(np.atleast_1d(weight_scale))
    out = np.empty(ws.shape, np.float32)
    lib().ref_dequant_reciprocal(ctypes.c_int32(ws.size), _p(ws),
                                 ctypes.c_float(input_scale), _p(out))
    return out


def conv2d_int8(g: ConvGeom, x, w_i8, b, weight_scale, input_scale,
                output_scale=1.0, scale_term=101, activation=1, threads=0):
    """x: float32 (quantized by input_scale) or int8 (used as is)."""
    is_i8 = x.dtype == np.int8
    x = np.ascontiguousarray(x) if is_i8 else _f32(x)
    w_i8 = np.ascontiguousarray(w_i8, dtype=np.int8)
    b = _f32(b)
    ws = _f32(np.atleast_1d(weight_scale))
    oh, ow = out_hw(g)
    dt = np.int8 if scale_term > 100 else np.float32
    out = np.empty((g.n, g.k, oh, ow), dt)
    lib().ref_conv2d_int8(ctypes.byref(g), _p(x), ctypes.c_int32(int(is_i8)),
                          _p(w_i8), _p(b), _p(ws), ctypes.c_int32(ws.size),
                          ctypes.c_float(input_scale),
                          ctypes.c_float(output_scale),
                          ctypes.c_int32(scale_term), ctypes.c_int32(activation),
                          _p(out), ctypes.c_int(threads))
    return out


def dwconv2d_int8(g: ConvGeom, x, w_i8, b, weight_scale, input_scale,
                  output_scale=1.0, scale_term=101, activation=1, threads=0):
    """x: float32 (quantized by input_scale) or int8; w_i8 [C][1][kh][kw]."""
    is_i8 = x.dtype == np.int8
    x = np.ascontiguousarray(x) if is_i8 else _f32(x)
    w_i8 = np.ascontiguousarray(w_i8, dtype=np.int8)
    ws = _f32(np.atleast_1d(weight_scale))
    oh, ow = out_hw(g)
    out = np.empty((g.n, g.k, oh, ow), np.int8 if scale_term > 100 else np.float32)
    lib().ref_dwconv2d_int8(ctypes.byref(g), _p(x), ctypes.c_int32(int(is_i8)), _p(w_i8), _p(_f32(b)), _p(ws),
                            ctypes.c_int32(ws.size), ctypes.c_float(input_scale), ctypes.c_float(output_scale),
                            ctypes.c_int32(scale_term), ctypes.c_int32(activation), _p(out), ctypes.c_int(threads))
    return out


def innerproduct_int8(x, w_i8, b, weight_scale, input_scale, activation=0, threads=0):
    """x [M][K] float32 or int8, w_i8 [N][K] -> float32 [M][N]."""
    is_i8 = x.dtype == np.int8
    x = np.ascontiguousarray(x) if is_i8 else _f32(x)
    w_i8 = np.ascontiguousarray(w_i8, dtype=np.int8)
    m, k = x.shape
    n = w_i8.shape[0]
    ws = _f32(np.broadcast_to(np.atleast_1d(weight_scale), (n,)))
    out = np.empty((m, n), np.float32)
    lib().ref_innerproduct_int8(ctypes.c_int32(m), ctypes.c_int32(k), ctypes.c_int32(n), _p(x),
                                ctypes.c_int32(int(is_i8)), _p(w_i8), _p(_f32(b)), _p(ws),
                                ctypes.c_float(input_scale), ctypes.c_int32(activation), _p(out),
                                ctypes.c_int(threads))
    return out


def conv2d_i8_acc(g: ConvGeom, x_i8, w_i8, threads=0):
    x_i8 = np.ascontiguousarray(x_i8, dtype=np.int8)
    w_i8 = np.ascontiguousarray(w_i8, dtype=np.int8)
    oh, ow = out_hw(g)
    out = np.empty((g.n, g.k, oh, ow), np.int64)
    lib().ref_conv2d_i8_acc(ctypes.byref(g), _p(x_i8), _p(w_i8), _p(out),
                            ctypes.c_int(threads))
    return out


def _scale_args(v):
    v = _f32(np.atleast_1d(v))
    return v, ctypes.c_int32(v.size)


def requantize_i32_i8(x_i32, in_scale, out_scale, bias=None, activation=0):
    """x_i32: [C, ...] (channel = dim 0)."""
    x = np.ascontiguousarray(x_i32, dtype=np.int32)
    c = x.shape[0]
    cs = x.size // c
    isc, isn = _scale_args(in_scale)
    osc, osn = _scale_args(out_scale)
    if bias is None:
        bp, bn = None, ctypes.c_int32(0)
    else:
        bp, bn = _scale_args(bias)
    out = np.empty(x.shape, np.int8)
    lib().ref_requantize_i32_i8(ctypes.c_int32(c), ctypes.c_int64(cs), _p(x),
                                _p(isc), isn, _p(osc), osn, _p(bp), bn,
                                ctypes.c_int32(activation), _p(out))
    return out


def dequantize_i32_f32(x_i32, scale, bias=None):
    x = np.ascontiguousarray(x_i32, dtype=np.int32)
    c = x.shape[0]
    cs = x.size // c
    sc, sn = _scale_args(scale)
    if bias is None:
        bp, bn = None, ctypes.c_int32(0)
    else:
        bp, bn = _scale_args(bias)
    out = np.empty(x.shape, np.float32)
    lib().ref_dequantize_i32_f32(ctypes.c_int32(c), ctypes.c_int64(cs), _p(x),
                                 _p(sc), sn, _p(bp), bn, _p(out))
    return out


def relu_f32(x):
    x = _f32(x)
    out = np.empty_like(x)
    lib().ref_relu_f32(ctypes.c_int64(x.size), _p(x), _p(out))
    return out


def relu_i8(x):
    x = np.ascontiguousarray(x, dtype=np.int8)
    out = np.empty_like(x)
    lib().ref_relu_i8(ctypes.c_int64(x.size), _p(x), _p(out))
    return out


def add_f32(a, b):
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    lib().ref_add_f32(ctypes.c_int64(a.size), _p(a), _p(b), _p(out))
    return out


def global_avgpool_f32(x):
    x = _f32(x)
    n, c, h, w = x.shape
    out = np.empty((n, c), np.float32)
    lib().ref_global_avgpool_f32(ctypes.c_int32(n), ctypes.c_int32(c),
                                 ctypes.c_int32(h), ctypes.c_int32(w), _p(x),
                                 _p(out))
    return out


def bn_fold(weight, bias, slope, mean, variance, bn_bias, epsilon):
    """Returns (folded_weight, folded_bias) or None when folding is refused."""
    w = np.array(weight, dtype=np.float32, copy=True, order="C")
    k = w.shape[0]
    per = w.size // k
    b = _f32(bias)
    out_b = np.empty(k, np.float32)
    ok = lib().ref_bn_fold(ctypes.c_int32(k), ctypes.c_int64(per), _p(w), _p(b),
                           _p(_f32(slope)), _p(_f32(mean)), _p(_f32(variance)),
                           _p(_f32(bn_bias)), ctypes.c_float(epsilon), _p(out_b))
    return (w, out_b) if ok else None


def same_padding(inp, kernel, stride, dilation, pad_type):
    b = ctypes.c_int32()
    a = ctypes.c_int32()
    lib().ref_same_padding(ctypes.c_int32(inp), ctypes.c_int32(kernel),
                           ctypes.c_int32(stride), ctypes.c_int32(dilation),
                           ctypes.c_int32(pad_type), ctypes.byref(b),
                           ctypes.byref(a))
    return b.value, a.value
