"""ctypes binding of libnhip.so, the gfx950 runtime for the ncnn Convolution /
ConvolutionDepthWise / InnerProduct / int8 Convolution hot path.

Every compute call goes through the C ABI declared in include/nhip.h; torch is
used only as the device allocator and for the current HIP stream.  There is
no CPU fallback: if libnhip.so is missing or no GPU is visible, the calls
raise.

Layer objects mirror the reference's ncnn layer parameters
(include/ncnn-mlir/Graph/graph.hpp:73-150) and its lowering semantics
(lib/Conversion/NCNNToTosa/NCNNToTosa.cpp); batches are [N,C,H,W] stacks of the
reference's single-image [C,H,W] blobs.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libnhip.so")

STATUS_NAMES = {
    0: "SUCCESS", 1: "NULL_POINTER", 2: "INVALID_SHAPE",
    3: "CONSTRAINT_VIOLATION", 4: "SHAPE_ARITHMETIC_OVERFLOW",
    5: "OUTPUT_CAPACITY_INSUFFICIENT", 6: "DEVICE_ERROR", 7: "UNSUPPORTED",
}

ALGO_AUTO, ALGO_IMPLICIT_GEMM, ALGO_WINOGRAD = 0, 1, 2
ACT_NONE, ACT_RELU, ACT_SIGMOID = 0, 1, 4

# Every symbol include/nhip.h declares (checked by the CPU test suite).
EXPORTS = (
    "nhip_init", "nhip_device_count", "nhip_last_error", "nhip_malloc",
    "nhip_free", "nhip_memcpy_h2d", "nhip_memcpy_d2h", "nhip_memcpy_d2d",
    "nhip_stream_sync", "nhip_reload_settings", "nhip_timer_start", "nhip_timer_stop",
    "nhip_conv_output_shape", "nhip_conv2d_f32_create",
    "nhip_conv2d_workspace_size", "nhip_conv2d_f32_forward", "nhip_conv2d_f32_forward_noalloc",
    "nhip_conv2d_int8_create", "nhip_conv2d_int8_forward",
    "nhip_dwconv2d_f32_create", "nhip_dwconv2d_f32_forward",
    "nhip_dwconv2d_pw_f32_supported", "nhip_dwconv2d_pw_f32_forward",
    "nhip_conv1x1_dw_f32_supported", "nhip_conv1x1_dw_f32_forward",
    "nhip_dwconv2d_int8_create", "nhip_dwconv2d_int8_forward",
    "nhip_conv_destroy", "nhip_innerproduct_f32_create",
    "nhip_innerproduct_int8_create", "nhip_innerproduct_int8_forward",
    "nhip_innerproduct_workspace_size", "nhip_innerproduct_f32_forward",
    "nhip_innerproduct_destroy", "nhip_global_avgpool_innerproduct_f32_workspace_size",
    "nhip_global_avgpool_innerproduct_f32_forward", "nhip_relu_f32", "nhip_relu_i8",
    "nhip_add_f32", "nhip_global_avgpool_f32", "nhip_quantize_f32_i8",
    "nhip_requantize_i32_i8", "nhip_dequantize_i32_f32",
)

# Every symbol include/nhip_graph.h declares.
GRAPH_EXPORTS = (
    "nhip_graph_load", "nhip_graph_describe", "nhip_graph_num_io",
    "nhip_graph_io_info", "nhip_graph_infer_shapes", "nhip_graph_run",
    "nhip_graph_run_host", "nhip_graph_destroy",
)
DTYPE_F32, DTYPE_I8, DTYPE_I32 = 0, 1, 2
_NP_DTYPE = {DTYPE_F32: np.float32, DTYPE_I8: np.int8, DTYPE_I32: np.int32}


class NhipError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"nhip status {status} ({STATUS_NAMES.get(status, '?')}): {message}")
        self.status = status


class ConvDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "input_channels", "num_output", "kernel_w", "kernel_h", "dilation_w",
        "dilation_h", "stride_w", "stride_h", "pad_left", "pad_right",
        "pad_top", "pad_bottom", "bias_term", "int8_scale_term",
        "activation_type", "group", "algorithm")]


_lib = None
_P = ctypes.c_void_p


def load():
    """Load libnhip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build()")
    # torch ships its own libamdhip64.so.7; load it first so that torch and
    # libnhip share that one HIP runtime (same SONAME, resolved once).
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    L = ctypes.CDLL(LIB_PATH)
    i32, i64, u64, f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float
    D = ctypes.POINTER(ConvDesc)
    sig = {
        "nhip_init": [i32],
        "nhip_device_count": [ctypes.POINTER(i32)],
        "nhip_malloc": [ctypes.POINTER(_P), u64],
        "nhip_free": [_P],
        "nhip_memcpy_h2d": [_P, _P, u64, _P],
        "nhip_memcpy_d2h": [_P, _P, u64, _P],
        "nhip_memcpy_d2d": [_P, _P, u64, _P],
        "nhip_stream_sync": [_P],
        "nhip_reload_settings": [],
        "nhip_timer_start": [ctypes.c_char_p],
        "nhip_timer_stop": [ctypes.POINTER(u64), ctypes.POINTER(ctypes.c_double)],
        "nhip_conv_output_shape": [D, i32, i32, ctypes.POINTER(i32), ctypes.POINTER(i32)],
        "nhip_conv2d_f32_create": [D, _P, _P, ctypes.POINTER(_P)],
        "nhip_conv2d_workspace_size": [_P, i32, i32, i32, ctypes.POINTER(u64)],
        "nhip_conv2d_f32_forward": [_P, _P, _P, _P, i32, i32, i32, _P, u64, _P],
        "nhip_conv2d_f32_forward_noalloc": [_P, _P, _P, _P, i32, i32, i32, _P],
        "nhip_conv2d_int8_create": [D, _P, i32, _P, _P, i32, f32, f32, ctypes.POINTER(_P)],
        "nhip_conv2d_int8_forward": [_P, _P, i32, _P, i32, i32, i32, _P, u64, _P],
        "nhip_dwconv2d_f32_create": [D, _P, _P, ctypes.POINTER(_P)],
        "nhip_dwconv2d_f32_forward": [_P, _P, _P, i32, i32, i32, _P],
        "nhip_dwconv2d_pw_f32_supported": [_P, _P, i32, i32, i32, ctypes.POINTER(i32)],
        "nhip_dwconv2d_pw_f32_forward": [_P, _P, _P, _P, _P, i32, i32, i32, _P],
        "nhip_conv1x1_dw_f32_supported": [_P, _P, i32, i32, i32, ctypes.POINTER(i32)],
        "nhip_conv1x1_dw_f32_forward": [_P, _P, _P, _P, i32, i32, i32, _P],
        "nhip_dwconv2d_int8_create": [D, _P, i32, _P, _P, i32, f32, f32, ctypes.POINTER(_P)],
        "nhip_dwconv2d_int8_forward": [_P, _P, i32, _P, i32, i32, i32, _P],
        "nhip_innerproduct_int8_create": [i32, i32, _P, i32, _P, _P, f32, i32, ctypes.POINTER(_P)],
        "nhip_innerproduct_int8_forward": [_P, _P, i32, _P, i32, _P, u64, _P],
        "nhip_conv_destroy": [_P],
        "nhip_innerproduct_f32_create": [i32, i32, _P, _P, i32, ctypes.POINTER(_P)],
        "nhip_innerproduct_workspace_size": [_P, i32, ctypes.POINTER(u64)],
        "nhip_innerproduct_f32_forward": [_P, _P, _P, i32, _P, u64, _P],
        "nhip_innerproduct_destroy": [_P],
        "nhip_global_avgpool_innerproduct_f32_workspace_size": [_P, i32, i32, i32, ctypes.POINTER(u64)],
        "nhip_global_avgpool_innerproduct_f32_forward": [_P, _P, _P, i32, i32, i32, i32, _P, u64, _P],
        "nhip_relu_f32": [_P, _P, i64, _P],
        "nhip_relu_i8": [_P, _P, i64, _P],
        "nhip_add_f32": [_P, _P, _P, i64, i32, _P],
        "nhip_global_avgpool_f32": [_P, _P, i32, i32, i32, i32, _P],
        "nhip_quantize_f32_i8": [_P, _P, i32, i32, i64, _P, i32, _P],
        "nhip_requantize_i32_i8": [_P, _P, i32, i32, i64, _P, i32, _P, i32, _P, i32, i32, _P],
        "nhip_dequantize_i32_f32": [_P, _P, i32, i32, i64, _P, i32, _P, i32, _P],
    }
    i64p, i32p, vpp = ctypes.POINTER(i64), ctypes.POINTER(i32), ctypes.POINTER(_P)
    sig.update({
        "nhip_graph_load": [ctypes.c_char_p, u64, _P, u64, i64p, i32, vpp],
        "nhip_graph_describe": [ctypes.c_char_p, u64, _P, u64, i64p, i32, vpp],
        "nhip_graph_num_io": [_P, i32p, i32p],
        "nhip_graph_io_info": [_P, i32, i32, i32p, i64p, i32p, ctypes.POINTER(ctypes.c_char_p)],
        "nhip_graph_infer_shapes": [_P, i64p, i64p, i32p],
        "nhip_graph_run": [_P, i32, i64p, vpp, vpp, _P],
        "nhip_graph_run_host": [_P, i64p, vpp, vpp, ctypes.POINTER(u64)],
        "nhip_graph_destroy": [_P],
    })
    for name, args in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    L.nhip_last_error.argtypes = []
    L.nhip_last_error.restype = ctypes.c_char_p
    _lib = L
    return L


def check(status: int) -> None:
    if status != 0:
        raise NhipError(status, load().nhip_last_error().decode(errors="replace"))


# ---------------------------------------------------------------- device glue
def _torch():
    import torch
    return torch


def init(device: int = 0) -> None:
    check(load().nhip_init(device))


def reload_settings() -> None:
    """Re-read the NHIP_* tuning / test switches from the environment (the
    library reads them once, at first use)."""
    check(load().nhip_reload_settings())


def timer_start(kernel_filter: str = "") -> None:
    """Bracket every matching kernel launch with HIP events on its stream."""
    check(load().nhip_timer_start(kernel_filter.encode()))


def timer_stop():
    """-> (launches, total_ms) of the launches timed since timer_start."""
    n, ms = ctypes.c_uint64(), ctypes.c_double()
    check(load().nhip_timer_stop(ctypes.byref(n), ctypes.byref(ms)))
    return n.value, ms.value


def _ptr(t):
    return None if t is None else _P(t.data_ptr())


def _torch_dtype(np_dtype):
    torch = _torch()
    return {np.int8: torch.int8, np.int32: torch.int32}.get(np_dtype, torch.float32)


def _stream(stream=None):
    torch = _torch()
    s = torch.cuda.current_stream() if stream is None else stream
    return _P(s.cuda_stream)


def _dev(t, dtype):
    """Device tensor check (no host fallback)."""
    torch = _torch()
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError("nhip expects a CUDA (HIP) device tensor")
    if t.dtype != dtype:
        raise TypeError(f"expected {dtype}, got {t.dtype}")
    return t.contiguous()


def _workspace(nbytes: int, device):
    torch = _torch()
    if nbytes == 0:
        return None, 0
    return torch.empty(int(nbytes), dtype=torch.uint8, device=device), int(nbytes)


def conv_desc(c, k, kernel=(3, 3), stride=(1, 1), dilation=(1, 1),
              pad=(1, 1, 1, 1), bias=True, act=ACT_NONE, int8_scale_term=0,
              group=1, algorithm=ALGO_AUTO) -> ConvDesc:
    """kernel/stride/dilation are (h, w); pad is (top, bottom, left, right)."""
    d = ConvDesc()
    d.input_channels, d.num_output = c, k
    d.kernel_h, d.kernel_w = kernel
    d.stride_h, d.stride_w = stride
    d.dilation_h, d.dilation_w = dilation
    d.pad_top, d.pad_bottom, d.pad_left, d.pad_right = pad
    d.bias_term = 1 if bias else 0
    d.int8_scale_term = int8_scale_term
    d.activation_type = act
    d.group = group
    d.algorithm = algorithm
    return d


def output_shape(desc: ConvDesc, h: int, w: int):
    oh, ow = ctypes.c_int32(), ctypes.c_int32()
    check(load().nhip_conv_output_shape(ctypes.byref(desc), h, w, ctypes.byref(oh), ctypes.byref(ow)))
    return oh.value, ow.value


def _np_ptr(a):
    return None if a is None else a.ctypes.data_as(_P)


class _Plan:
    _destroy = "nhip_conv_destroy"

    def __init__(self):
        self.handle = _P()

    def close(self):
        if self.handle:
            getattr(load(), self._destroy)(self.handle)
            self.handle = _P()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Conv2dF32(_Plan):
    """ncnn Convolution, fp32 (reference ConvertConvolution fp32 path)."""

    def __init__(self, desc: ConvDesc, weight, bias=None):
        super().__init__()
        self.desc = desc
        self._w = np.ascontiguousarray(weight, dtype=np.float32)
        self._b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        expect = desc.num_output * desc.input_channels * desc.kernel_h * desc.kernel_w
        if self._w.size != expect:
            raise ValueError(f"weight has {self._w.size} elements, expected {expect}")
        check(load().nhip_conv2d_f32_create(ctypes.byref(desc), _np_ptr(self._w), _np_ptr(self._b),
                                            ctypes.byref(self.handle)))

    def workspace_size(self, n, h, w) -> int:
        b = ctypes.c_uint64()
        check(load().nhip_conv2d_workspace_size(self.handle, n, h, w, ctypes.byref(b)))
        return b.value

    def forward(self, x, residual=None, out=None, workspace=None, stream=None):
        torch = _torch()
        x = _dev(x, torch.float32)
        n, c, h, w = x.shape
        oh, ow = output_shape(self.desc, h, w)
        if out is None:
            out = torch.empty((n, self.desc.num_output, oh, ow), dtype=torch.float32, device=x.device)
        if residual is not None:
            residual = _dev(residual, torch.float32)
        if workspace is None:
            workspace, nbytes = _workspace(self.workspace_size(n, h, w), x.device)
        else:
            nbytes = workspace.numel()
        check(load().nhip_conv2d_f32_forward(self.handle, _ptr(x), _ptr(residual), _ptr(out), n, h, w,
                                             _ptr(workspace), nbytes, _stream(stream)))
        return out


class Conv2dInt8(_Plan):
    """ncnn Convolution with int8_scale_term (reference int8 path)."""

    def __init__(self, desc: ConvDesc, weight, bias, weight_scale, input_scale, output_scale=1.0):
        super().__init__()
        self.desc = desc
        w = np.ascontiguousarray(weight)
        self._w = w if w.dtype == np.int8 else np.ascontiguousarray(w, dtype=np.float32)
        self._b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        self._ws = np.ascontiguousarray(np.atleast_1d(weight_scale), dtype=np.float32)
        check(load().nhip_conv2d_int8_create(
            ctypes.byref(desc), _np_ptr(self._w), 1 if self._w.dtype == np.int8 else 0,
            _np_ptr(self._b), _np_ptr(self._ws), self._ws.size, ctypes.c_float(input_scale),
            ctypes.c_float(output_scale), ctypes.byref(self.handle)))

    def workspace_size(self, n, h, w) -> int:
        b = ctypes.c_uint64()
        check(load().nhip_conv2d_workspace_size(self.handle, n, h, w, ctypes.byref(b)))
        return b.value

    def forward(self, x, out=None, workspace=None, stream=None):
        torch = _torch()
        if not x.is_cuda or x.dtype not in (torch.float32, torch.int8):
            raise TypeError("int8 conv input must be a float32 or int8 device tensor")
        x = x.contiguous()
        n, c, h, w = x.shape
        oh, ow = output_shape(self.desc, h, w)
        odt = torch.int8 if self.desc.int8_scale_term > 100 else torch.float32
        if out is None:
            out = torch.empty((n, self.desc.num_output, oh, ow), dtype=odt, device=x.device)
        if workspace is None:
            workspace, nbytes = _workspace(self.workspace_size(n, h, w), x.device)
        else:
            nbytes = workspace.numel()
        check(load().nhip_conv2d_int8_forward(self.handle, _ptr(x), 1 if x.dtype == torch.int8 else 0,
                                              _ptr(out), n, h, w, _ptr(workspace), nbytes,
                                              _stream(stream)))
        return out


class DwConv2dF32(_Plan):
    """ncnn ConvolutionDepthWise, fp32."""

    def __init__(self, desc: ConvDesc, weight, bias=None):
        super().__init__()
        self.desc = desc
        self._w = np.ascontiguousarray(weight, dtype=np.float32)
        self._b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        check(load().nhip_dwconv2d_f32_create(ctypes.byref(desc), _np_ptr(self._w), _np_ptr(self._b),
                                              ctypes.byref(self.handle)))

    def forward(self, x, out=None, stream=None):
        torch = _torch()
        x = _dev(x, torch.float32)
        n, c, h, w = x.shape
        oh, ow = output_shape(self.desc, h, w)
        if out is None:
            out = torch.empty((n, self.desc.num_output, oh, ow), dtype=torch.float32, device=x.device)
        check(load().nhip_dwconv2d_f32_forward(self.handle, _ptr(x), _ptr(out), n, h, w, _stream(stream)))
        return out


def dwconv_pw_supported(dw: "DwConv2dF32", pw: "Conv2dF32", n: int, h: int, w: int) -> bool:
    """Whether a depthwise plan feeding a 1x1 convolution plan has the fused
    kernel for n images of h x w (nhip_dwconv2d_pw_f32_supported)."""
    sup = ctypes.c_int32()
    check(load().nhip_dwconv2d_pw_f32_supported(dw.handle, pw.handle, n, h, w, ctypes.byref(sup)))
    return bool(sup.value)


def dwconv_pw_forward(dw: "DwConv2dF32", pw: "Conv2dF32", x, residual=None, out=None, stream=None):
    """pw(dw(x)) (+ residual) in one pass without the depthwise output in
    memory (nhip_dwconv2d_pw_f32_forward; the graph executor's fusion)."""
    torch = _torch()
    x = _dev(x, torch.float32)
    n, c, h, w = x.shape
    oh, ow = output_shape(dw.desc, h, w)
    if out is None:
        out = torch.empty((n, pw.desc.num_output, oh, ow), dtype=torch.float32, device=x.device)
    res = None if residual is None else _dev(residual, torch.float32)
    check(load().nhip_dwconv2d_pw_f32_forward(dw.handle, pw.handle, _ptr(x), _ptr(res), _ptr(out), n, h, w,
                                               _stream(stream)))
    return out


def conv1x1_dw_supported(pw: "Conv2dF32", dw: "DwConv2dF32", n: int, h: int, w: int) -> bool:
    """Whether a 1x1 convolution plan feeding a depthwise plan has the fused
    kernel for n images of h x w (nhip_conv1x1_dw_f32_supported)."""
    sup = ctypes.c_int32()
    check(load().nhip_conv1x1_dw_f32_supported(pw.handle, dw.handle, n, h, w, ctypes.byref(sup)))
    return bool(sup.value)


def conv1x1_dw_forward(pw: "Conv2dF32", dw: "DwConv2dF32", x, out=None, stream=None):
    """dw(pw(x)) in one pass without the 1x1 output in memory
    (nhip_conv1x1_dw_f32_forward; the graph executor's fusion)."""
    torch = _torch()
    x = _dev(x, torch.float32)
    n, c, h, w = x.shape
    oh, ow = output_shape(dw.desc, h, w)
    if out is None:
        out = torch.empty((n, dw.desc.num_output, oh, ow), dtype=torch.float32, device=x.device)
    check(load().nhip_conv1x1_dw_f32_forward(pw.handle, dw.handle, _ptr(x), _ptr(out), n, h, w, _stream(stream)))
    return out


class DwConv2dInt8(_Plan):
    """ncnn ConvolutionDepthWise with int8_scale_term."""

    def __init__(self, desc: ConvDesc, weight, bias, weight_scale, input_scale, output_scale=1.0):
        super().__init__()
        self.desc = desc
        w = np.ascontiguousarray(weight)
        self._w = w if w.dtype == np.int8 else np.ascontiguousarray(w, dtype=np.float32)
        self._b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        self._ws = np.ascontiguousarray(np.atleast_1d(weight_scale), dtype=np.float32)
        check(load().nhip_dwconv2d_int8_create(
            ctypes.byref(desc), _np_ptr(self._w), 1 if self._w.dtype == np.int8 else 0, _np_ptr(self._b),
            _np_ptr(self._ws), self._ws.size, ctypes.c_float(input_scale), ctypes.c_float(output_scale),
            ctypes.byref(self.handle)))

    def forward(self, x, out=None, stream=None):
        torch = _torch()
        if not x.is_cuda or x.dtype not in (torch.float32, torch.int8):
            raise TypeError("int8 depthwise input must be a float32 or int8 device tensor")
        x = x.contiguous()
        n, c, h, w = x.shape
        oh, ow = output_shape(self.desc, h, w)
        odt = torch.int8 if self.desc.int8_scale_term > 100 else torch.float32
        if out is None:
            out = torch.empty((n, c, oh, ow), dtype=odt, device=x.device)
        check(load().nhip_dwconv2d_int8_forward(self.handle, _ptr(x), 1 if x.dtype == torch.int8 else 0, _ptr(out),
                                                n, h, w, _stream(stream)))
        return out


class InnerProductInt8(_Plan):
    """ncnn InnerProduct with int8_scale_term (fp32 output)."""
    _destroy = "nhip_innerproduct_destroy"

    def __init__(self, weight, bias, weight_scale, input_scale, activation=ACT_NONE):
        super().__init__()
        w = np.ascontiguousarray(weight)
        self._w = w if w.dtype == np.int8 else np.ascontiguousarray(w, dtype=np.float32)
        self.num_output, self.num_input = self._w.shape
        self._b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        self._ws = np.ascontiguousarray(np.broadcast_to(np.atleast_1d(weight_scale), (self.num_output,)),
                                        dtype=np.float32)
        check(load().nhip_innerproduct_int8_create(
            self.num_output, self.num_input, _np_ptr(self._w), 1 if self._w.dtype == np.int8 else 0,
            _np_ptr(self._b), _np_ptr(self._ws), ctypes.c_float(input_scale), activation,
            ctypes.byref(self.handle)))

    def workspace_size(self, m) -> int:
        b = ctypes.c_uint64()
        check(load().nhip_innerproduct_workspace_size(self.handle, m, ctypes.byref(b)))
        return b.value

    def forward(self, x, out=None, workspace=None, stream=None):
        torch = _torch()
        if not x.is_cuda or x.dtype not in (torch.float32, torch.int8):
            raise TypeError("int8 InnerProduct input must be a float32 or int8 device tensor")
        x = x.contiguous()
        m = x.shape[0]
        if out is None:
            out = torch.empty((m, self.num_output), dtype=torch.float32, device=x.device)
        if workspace is None:
            workspace, nbytes = _workspace(self.workspace_size(m), x.device)
        else:
            nbytes = workspace.numel()
        check(load().nhip_innerproduct_int8_forward(self.handle, _ptr(x), 1 if x.dtype == torch.int8 else 0,
                                                    _ptr(out), m, _ptr(workspace), nbytes, _stream(stream)))
        return out


class InnerProductF32(_Plan):
    """ncnn InnerProduct, fp32 packed matmul."""
    _destroy = "nhip_innerproduct_destroy"

    def __init__(self, weight, bias=None, activation=ACT_NONE):
        super().__init__()
        self._w = np.ascontiguousarray(weight, dtype=np.float32)
        self.num_output, self.num_input = self._w.shape
        self._b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        check(load().nhip_innerproduct_f32_create(self.num_output, self.num_input, _np_ptr(self._w),
                                                  _np_ptr(self._b), activation, ctypes.byref(self.handle)))

    def workspace_size(self, m) -> int:
        b = ctypes.c_uint64()
        check(load().nhip_innerproduct_workspace_size(self.handle, m, ctypes.byref(b)))
        return b.value

    def forward(self, x, out=None, workspace=None, stream=None):
        torch = _torch()
        x = _dev(x, torch.float32)
        m = x.shape[0]
        if out is None:
            out = torch.empty((m, self.num_output), dtype=torch.float32, device=x.device)
        if workspace is None:
            workspace, nbytes = _workspace(self.workspace_size(m), x.device)
        else:
            nbytes = workspace.numel()
        check(load().nhip_innerproduct_f32_forward(self.handle, _ptr(x), _ptr(out), m, _ptr(workspace),
                                                   nbytes, _stream(stream)))
        return out

    def gap_workspace_size(self, n, h, w) -> int:
        b = ctypes.c_uint64()
        check(load().nhip_global_avgpool_innerproduct_f32_workspace_size(self.handle, n, h, w, ctypes.byref(b)))
        return b.value

    def forward_pooled(self, x, out=None, workspace=None, stream=None):
        """Global average pooling of x [n, C, H, W] fused with this
        InnerProduct (C = num_input) -> [n, num_output]."""
        torch = _torch()
        x = _dev(x, torch.float32)
        n, c, h, w = x.shape
        if out is None:
            out = torch.empty((n, self.num_output), dtype=torch.float32, device=x.device)
        if workspace is None:
            workspace, nbytes = _workspace(self.gap_workspace_size(n, h, w), x.device)
        else:
            nbytes = workspace.numel()
        check(load().nhip_global_avgpool_innerproduct_f32_forward(self.handle, _ptr(x), _ptr(out), n, c, h, w,
                                                                  _ptr(workspace), nbytes, _stream(stream)))
        return out


# ---------------------------------------------------------------- elementwise
def relu(x, out=None, stream=None):
    torch = _torch()
    if out is None:
        out = torch.empty_like(x)
    if x.dtype == torch.int8:
        check(load().nhip_relu_i8(_ptr(x), _ptr(out), x.numel(), _stream(stream)))
    else:
        x = _dev(x, torch.float32)
        check(load().nhip_relu_f32(_ptr(x), _ptr(out), x.numel(), _stream(stream)))
    return out


def add(a, b, relu_after=False, out=None, stream=None):
    torch = _torch()
    a, b = _dev(a, torch.float32), _dev(b, torch.float32)
    if a.shape != b.shape:
        raise ValueError("add: shapes differ")
    if out is None:
        out = torch.empty_like(a)
    check(load().nhip_add_f32(_ptr(a), _ptr(b), _ptr(out), a.numel(), 1 if relu_after else 0, _stream(stream)))
    return out


def global_avgpool(x, stream=None):
    torch = _torch()
    x = _dev(x, torch.float32)
    n, c, h, w = x.shape
    out = torch.empty((n, c), dtype=torch.float32, device=x.device)
    check(load().nhip_global_avgpool_f32(_ptr(x), _ptr(out), n, c, h, w, _stream(stream)))
    return out


def quantize(x, scale, stream=None):
    """x [N,C,...] fp32 -> int8; scale: 1 or C values (per channel dim 1)."""
    torch = _torch()
    x = _dev(x, torch.float32)
    n, c = x.shape[0], x.shape[1]
    plane = x[0, 0].numel()
    s = torch.as_tensor(np.atleast_1d(np.asarray(scale, np.float32)), device=x.device)
    out = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    check(load().nhip_quantize_f32_i8(_ptr(x), _ptr(out), n, c, plane, _ptr(s), s.numel(), _stream(stream)))
    return out


def requantize(x, in_scale, out_scale, bias=None, activation=ACT_NONE, stream=None):
    torch = _torch()
    x = _dev(x, torch.int32)
    n, c = x.shape[0], x.shape[1]
    plane = x[0, 0].numel()
    dev = x.device
    isc = torch.as_tensor(np.atleast_1d(np.asarray(in_scale, np.float32)), device=dev)
    osc = torch.as_tensor(np.atleast_1d(np.asarray(out_scale, np.float32)), device=dev)
    b = None if bias is None else torch.as_tensor(np.atleast_1d(np.asarray(bias, np.float32)), device=dev)
    out = torch.empty(x.shape, dtype=torch.int8, device=dev)
    check(load().nhip_requantize_i32_i8(_ptr(x), _ptr(out), n, c, plane, _ptr(isc), isc.numel(), _ptr(osc),
                                        osc.numel(), _ptr(b), 0 if b is None else b.numel(), activation,
                                        _stream(stream)))
    return out


def dequantize(x, scale, bias=None, stream=None):
    torch = _torch()
    x = _dev(x, torch.int32)
    n, c = x.shape[0], x.shape[1]
    plane = x[0, 0].numel()
    dev = x.device
    s = torch.as_tensor(np.atleast_1d(np.asarray(scale, np.float32)), device=dev)
    b = None if bias is None else torch.as_tensor(np.atleast_1d(np.asarray(bias, np.float32)), device=dev)
    out = torch.empty(x.shape, dtype=torch.float32, device=dev)
    check(load().nhip_dequantize_i32_f32(_ptr(x), _ptr(out), n, c, plane, _ptr(s), s.numel(), _ptr(b),
                                         0 if b is None else b.numel(), _stream(stream)))
    return out


class Graph:
    """An ncnn model (.param text + .bin payload) lowered onto libnhip
    (include/nhip_graph.h), the device counterpart of the reference's
    compiled model: Graph::load (lib/Graph/graph.cpp:2129-2333) + the
    generated entry (tools/ncnn-compile.cpp:915-932).

    input_shapes: None, or one CHW triple per Input layer (-1 = given at run
    time, the reference's "?" of --input-shape).  describe_only=True parses,
    validates and lowers without any device work (what a compiler on a host
    without a GPU needs); running such a graph is a constraint violation.
    """

    def __init__(self, param_text, bin_bytes=b"", input_shapes=None, describe_only=False):
        L = load()
        param = param_text.encode() if isinstance(param_text, str) else bytes(param_text)
        self._bin = bytes(bin_bytes)
        arr, count = None, 0
        if input_shapes is not None:
            flat = [int(v) for s in input_shapes for v in s]
            arr = (ctypes.c_int64 * max(len(flat), 1))(*flat)
            count = len(input_shapes)
        self.handle = _P()
        fn = L.nhip_graph_describe if describe_only else L.nhip_graph_load
        check(fn(param, len(param), self._bin or None, len(self._bin), arr, count, ctypes.byref(self.handle)))
        ni, no = ctypes.c_int32(), ctypes.c_int32()
        check(L.nhip_graph_num_io(self.handle, ctypes.byref(ni), ctypes.byref(no)))
        self.inputs = [self._io(0, i) for i in range(ni.value)]
        self.outputs = [self._io(1, i) for i in range(no.value)]

    def _io(self, is_output, index):
        rank, dtype, name = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_char_p()
        dims = (ctypes.c_int64 * 4)()
        check(load().nhip_graph_io_info(self.handle, is_output, index, ctypes.byref(rank), dims,
                                        ctypes.byref(dtype), ctypes.byref(name)))
        return dict(name=name.value.decode(), shape=tuple(dims[:rank.value]),
                    dtype=_NP_DTYPE[dtype.value])

    @staticmethod
    def _shape_arg(shapes):
        if shapes is None:
            return None
        flat = [int(v) for s in shapes for v in s]
        return (ctypes.c_int64 * len(flat))(*flat)

    def infer_shapes(self, input_shapes=None):
        """-> list of output shapes for concrete CHW input shapes."""
        n = len(self.outputs)
        out = (ctypes.c_int64 * (4 * n))()
        ranks = (ctypes.c_int32 * n)()
        check(load().nhip_graph_infer_shapes(self.handle, self._shape_arg(input_shapes), out, ranks))
        return [tuple(out[4 * j:4 * j + ranks[j]]) for j in range(n)]

    def run_host(self, *arrays, capacity=None):
        """The reference entry semantics: one image per input (host numpy
        arrays), returns the list of outputs as numpy arrays."""
        xs = [np.ascontiguousarray(a, dtype=io["dtype"]) for a, io in zip(arrays, self.inputs)]
        if len(xs) != len(self.inputs):
            raise ValueError(f"expected {len(self.inputs)} inputs")
        shapes = [a.shape if a.ndim == 3 else (1,) * (3 - a.ndim) + a.shape for a in xs]
        dyn = any(d < 0 for io in self.inputs for d in io["shape"])
        arg = self._shape_arg(shapes) if dyn else None
        oshapes = self.infer_shapes(shapes if dyn else None)
        outs = [np.empty(s, io["dtype"]) for s, io in zip(oshapes, self.outputs)]
        ins = (_P * len(xs))(*[a.ctypes.data for a in xs])
        ops = (_P * len(outs))(*[o.ctypes.data for o in outs])
        cap = None
        if capacity is not None:
            cap = (ctypes.c_uint64 * len(outs))(*capacity)
        check(load().nhip_graph_run_host(self.handle, arg, ins, ops, cap))
        return outs

    def run(self, *tensors, stream=None, out=None):
        """Batch execution: each input a [N, ...] device tensor of N blobs;
        returns device tensors [N, ...] per output (written into `out`, a
        list of preallocated tensors, when given).  On a non-default stream,
        repeated calls with the same inputs and outputs replay a recorded
        hipGraph of the call plan (nhip_graph_run), so steady loops should
        pass `out`."""
        torch = _torch()
        if len(tensors) != len(self.inputs):
            raise ValueError(f"expected {len(self.inputs)} inputs")
        n = int(tensors[0].shape[0])
        xs = [_dev(t, _torch_dtype(io["dtype"]))
              for t, io in zip(tensors, self.inputs)]
        shapes = [tuple(t.shape[1:]) if t.dim() == 4 else (1,) * (4 - t.dim()) + tuple(t.shape[1:])
                  for t in xs]
        dyn = any(d < 0 for io in self.inputs for d in io["shape"])
        oshapes = self.infer_shapes(shapes if dyn else None)
        if out is None:
            outs = [torch.empty((n,) + s, dtype=_torch_dtype(io["dtype"]),
                                device=xs[0].device) for s, io in zip(oshapes, self.outputs)]
        else:
            outs = list(out)
            for o, s, io in zip(outs, oshapes, self.outputs):
                want = _torch_dtype(io["dtype"])
                if tuple(o.shape) != (n,) + tuple(s) or o.dtype != want or not o.is_contiguous() or not o.is_cuda:
                    raise ValueError(f"out tensor must be a contiguous {want} device tensor of shape {(n,) + tuple(s)}")
        ins = (_P * len(xs))(*[t.data_ptr() for t in xs])
        ops = (_P * len(outs))(*[o.data_ptr() for o in outs])
        check(load().nhip_graph_run(self.handle, n, self._shape_arg(shapes) if dyn else None, ins, ops,
                                    _stream(stream)))
        return outs

    def close(self):
        if self.handle:
            load().nhip_graph_destroy(self.handle)
            self.handle = _P()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
