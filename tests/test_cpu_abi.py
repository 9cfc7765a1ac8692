"""C-ABI checks that need no GPU: libnhip.so loads, exports every function
include/nhip.h declares, and rejects invalid parameters with the reference's
status codes before any device work (tools/ncnn-compile.cpp:955-960 codes;
parameter rules of lib/Graph/graph.cpp:219-301 and the importers)."""
import ctypes
import os
import re

import pytest

import nhip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions(header="nhip.h"):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nhip_\w+)\s*\(", text)))


def test_header_declares_exactly_the_binding_exports():
    assert header_functions() == sorted(nhip.EXPORTS)
    assert header_functions("nhip_graph.h") == sorted(nhip.GRAPH_EXPORTS)


def test_library_exports_every_header_symbol():
    lib = nhip.load()
    for name in header_functions() + header_functions("nhip_graph.h"):
        assert hasattr(lib, name), name
    # and nothing reference-reserved (tools/ncnn-compile.cpp:2189-2196)
    syms = os.popen(f"nm -D --defined-only {nhip.LIB_PATH}").read()
    assert "ncnn_runtime" not in syms


def test_status_codes_match_reference_header():
    text = open(os.path.join(ROOT, "include", "nhip.h")).read()
    codes = dict(re.findall(r"#define NHIP_STATUS_(\w+) (\d+)", text))
    # generated header of the reference: tools/ncnn-compile.cpp:955-960
    assert codes["SUCCESS"] == "0" and codes["NULL_POINTER"] == "1"
    assert codes["INVALID_SHAPE"] == "2" and codes["CONSTRAINT_VIOLATION"] == "3"
    assert codes["SHAPE_ARITHMETIC_OVERFLOW"] == "4"
    assert codes["OUTPUT_CAPACITY_INSUFFICIENT"] == "5"


def _status(fn, *args):
    return fn(*args)


@pytest.mark.parametrize("field,value,status", [
    ("kernel_w", 0, 2), ("stride_h", 0, 2), ("dilation_w", -1, 2),
    ("pad_left", -233, 3), ("bias_term", 2, 3), ("int8_scale_term", 3, 3),
    ("activation_type", 2, 7), ("num_output", 0, 2),
])
def test_conv_create_rejects_invalid_params(field, value, status):
    lib = nhip.load()
    d = nhip.conv_desc(4, 4)
    setattr(d, field, value)
    h = ctypes.c_void_p()
    w = (ctypes.c_float * 256)()
    b = (ctypes.c_float * 16)()
    st = lib.nhip_conv2d_f32_create(ctypes.byref(d), ctypes.cast(w, ctypes.c_void_p),
                                    ctypes.cast(b, ctypes.c_void_p), ctypes.byref(h))
    assert st == status, lib.nhip_last_error()
    assert not h.value
    assert lib.nhip_last_error()


def test_null_pointers_return_status_1():
    lib = nhip.load()
    d = nhip.conv_desc(4, 4)
    h = ctypes.c_void_p()
    assert lib.nhip_conv2d_f32_create(ctypes.byref(d), None, None, ctypes.byref(h)) == 1
    assert lib.nhip_conv2d_f32_create(None, None, None, ctypes.byref(h)) == 1
    assert lib.nhip_conv2d_f32_forward(None, None, None, None, 1, 4, 4, None, 0, None) == 1
    assert lib.nhip_innerproduct_f32_forward(None, None, None, 1, None, 0, None) == 1
    assert lib.nhip_relu_f32(None, None, 4, None) == 1


def test_depthwise_requires_group_equal_channels():
    lib = nhip.load()
    d = nhip.conv_desc(8, 8, group=4, bias=False)
    h = ctypes.c_void_p()
    w = (ctypes.c_float * 72)()
    st = lib.nhip_dwconv2d_f32_create(ctypes.byref(d), ctypes.cast(w, ctypes.c_void_p), None, ctypes.byref(h))
    assert st == 3
    assert b"group" in lib.nhip_last_error()


def test_winograd_rejects_non_3x3_s1():
    lib = nhip.load()
    d = nhip.conv_desc(16, 16, stride=(2, 2), bias=False, algorithm=nhip.ALGO_WINOGRAD)
    h = ctypes.c_void_p()
    w = (ctypes.c_float * (16 * 16 * 9))()
    assert lib.nhip_conv2d_f32_create(ctypes.byref(d), ctypes.cast(w, ctypes.c_void_p), None,
                                      ctypes.byref(h)) == 7


@pytest.mark.parametrize("case", [
    # (c, k, kernel, stride, dilation, pad, h, w)
    (3, 8, (3, 3), (1, 1), (1, 1), (1, 1, 1, 1), 7, 6),
    (3, 8, (3, 3), (2, 2), (1, 1), (1, 1, 1, 1), 224, 224),
    (3, 8, (2, 3), (1, 2), (2, 1), (0, 1, 2, 0), 9, 8),
    (3, 8, (1, 1), (1, 1), (1, 1), (0, 0, 0, 0), 7, 7),
])
def test_output_shape_matches_oracle(case):
    from oracle import refcpu
    c, k, ker, st, dl, pad, h, w = case
    d = nhip.conv_desc(c, k, ker, st, dl, pad)
    g = refcpu.geom(1, c, h, w, k, ker, st, dl, pad)
    assert nhip.output_shape(d, h, w) == refcpu.out_hw(g)


def test_output_shape_rejects_input_smaller_than_kernel():
    d = nhip.conv_desc(3, 3, kernel=(5, 5), pad=(0, 0, 0, 0))
    with pytest.raises(nhip.NhipError) as e:
        nhip.output_shape(d, 3, 3)
    assert e.value.status == 2


def test_timer_without_launches():
    nhip.timer_start("none")
    assert nhip.timer_stop() == (0, 0.0)
