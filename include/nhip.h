/*
 * nhip.h — C ABI of the MI355X (gfx950) runtime that executes the ncnn
 * Convolution / ConvolutionDepthWise / InnerProduct / int8 Convolution hot
 * path.  Everything here is plain C: opaque handles, device pointers and
 * sizes.  No torch, no HIP types in the signatures (streams are `void*`
 * holding a hipStream_t; NULL is the default stream).
 *
 * Replaces, in the reference (hqu-little-boy/ncnn-compiler):
 *   - the CPU loop nests that lib/Pipelines/NCNNPipelines.cpp:88-130 generates
 *     for the Linalg ops produced by lib/Conversion/NCNNToTosa/NCNNToTosa.cpp
 *     (ConvertConvolution :1107-1530, ConvertDepthwiseConvolution :3074-3503,
 *     ConvertInnerProduct :5254-5392, quantize/dequantize :234-637,
 *     ConvertRequantize :4846-4888, ConvertRelu :1532-1578,
 *     ConvertBinary :5111-5223, ConvertPooling global average :1580-1995);
 *   - weights as .rodata constants of the generated .so
 *     (lib/Conversion/NCNNToFunc/NCNNToFunc.cpp:915-925): here they are
 *     prepacked once into device memory by the *_create calls.
 *
 * Tensors are batches of independent ncnn blobs.  An ncnn blob is [C,H,W]
 * contiguous (lib/Importer/ImportInput.cpp:22-45); a batch of N of them is
 * [N,C,H,W] contiguous, exactly N back-to-back single-image buffers of the
 * reference's generated entry point (tools/ncnn-compile.cpp:915-932).
 *
 * Status codes 0..5 keep the values of the generated header's NCNN_STATUS_*
 * (tools/ncnn-compile.cpp:955-960); 6 and 7 are new for device execution.
 *
 * Threading: handles are immutable after *_create, so forward calls on one
 * handle may run concurrently from several threads as long as each call uses
 * its own output and workspace buffers.  The last error message is
 * thread-local.
 */
#ifndef NHIP_H
#define NHIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NHIP_STATUS_SUCCESS 0
#define NHIP_STATUS_NULL_POINTER 1
#define NHIP_STATUS_INVALID_SHAPE 2
#define NHIP_STATUS_CONSTRAINT_VIOLATION 3
#define NHIP_STATUS_SHAPE_ARITHMETIC_OVERFLOW 4
#define NHIP_STATUS_OUTPUT_CAPACITY_INSUFFICIENT 5
#define NHIP_STATUS_DEVICE_ERROR 6 /* a HIP runtime call or launch failed */
#define NHIP_STATUS_UNSUPPORTED 7  /* parameters the reference importer rejects */

/* Convolution algorithms (fp32).  AUTO picks Winograd F(4,3) for 3x3,
 * stride 1, dilation 1, and implicit GEMM for everything else. */
#define NHIP_CONV_ALGO_AUTO 0
#define NHIP_CONV_ALGO_IMPLICIT_GEMM 1
#define NHIP_CONV_ALGO_WINOGRAD 2

/* ncnn activation_type values accepted by the Convolution importer
 * (lib/Importer/ImportConvolution.cpp:63-72, split out at :236-248). */
#define NHIP_ACT_NONE 0
#define NHIP_ACT_RELU 1
#define NHIP_ACT_SIGMOID 4

/* ---------------------------------------------------------------------------
 * Device, memory, stream.  The reference has no device (everything runs in
 * the caller's thread on host memory, tools/ncnn-compile.cpp:955-960 codes);
 * these are the runtime's own plumbing.
 * ------------------------------------------------------------------------- */
int nhip_init(int32_t device);
int nhip_device_count(int32_t* count);
/* Thread-local description of the last non-zero status returned on this
 * thread ("" when none).  Valid until the next nhip_* call on the thread. */
const char* nhip_last_error(void);
int nhip_malloc(void** ptr, uint64_t bytes);
int nhip_free(void* ptr);
int nhip_memcpy_h2d(void* dst, const void* src, uint64_t bytes, void* stream);
int nhip_memcpy_d2h(void* dst, const void* src, uint64_t bytes, void* stream);
int nhip_memcpy_d2d(void* dst, const void* src, uint64_t bytes, void* stream);
int nhip_stream_sync(void* stream);

/* NHIP_* environment switches (kernel-choice tuning and test overrides; no
 * counterpart in the reference).  The library reads them once, at first use,
 * into an immutable snapshot; this call re-reads the environment and
 * publishes a new snapshot (launches already in progress keep the old one).
 * The graph executor records a new hipGraph after a reload. */
int nhip_reload_settings(void);

/* Kernel timer (observability; the reference has no timing code at all).
 * While started, every kernel launch of this library whose name contains
 * `kernel_filter` (NULL or "" = all) is bracketed by a pair of HIP events
 * recorded on the launch's own stream.  nhip_timer_stop synchronizes on those
 * events and returns the number of timed launches and their summed duration.
 * Process-wide; not meant to be used from several threads at once. */
int nhip_timer_start(const char* kernel_filter);
int nhip_timer_stop(uint64_t* launches, double* total_ms);

/* ---------------------------------------------------------------------------
 * Convolution parameters: the fields of ncnn_graph::ConvolutionParams /
 * ConvolutionDepthWiseParams (include/ncnn-mlir/Graph/graph.hpp:73-114, param
 * ids decoded in lib/Graph/graph.cpp:219-301) after normalize-ncnn has made the
 * padding explicit (lib/Transforms/NormalizeNCNN/NormalizeNCNN.cpp:31-66).
 * ------------------------------------------------------------------------- */
typedef struct nhip_conv_desc {
  int32_t input_channels;  /* C of the [C,H,W] input blob */
  int32_t num_output;      /* param 0 */
  int32_t kernel_w;        /* param 1 */
  int32_t kernel_h;        /* param 11 */
  int32_t dilation_w;      /* param 2 */
  int32_t dilation_h;      /* param 12 */
  int32_t stride_w;        /* param 3 */
  int32_t stride_h;        /* param 13 */
  int32_t pad_left;        /* param 4 */
  int32_t pad_right;       /* param 15 */
  int32_t pad_top;         /* param 14 */
  int32_t pad_bottom;      /* param 16 */
  int32_t bias_term;       /* param 5 */
  int32_t int8_scale_term; /* param 8: 0 (fp32), 1/2, 101/102 (int8 out) */
  int32_t activation_type; /* param 9 */
  int32_t group;           /* param 7 (depthwise only; 1 for Convolution) */
  int32_t algorithm;       /* NHIP_CONV_ALGO_* (fp32 Convolution only) */
} nhip_conv_desc;

typedef struct nhip_conv_plan* nhip_conv_t;
typedef struct nhip_ip_plan* nhip_ip_t;

/* Output extent, NCNNOps.cpp:44 computeConvResult:
 * (in + pad_a + pad_b - ((k-1)*d+1)) / s + 1.  Returns INVALID_SHAPE if <= 0. */
int nhip_conv_output_shape(const nhip_conv_desc* desc, int32_t h, int32_t w,
                           int32_t* out_h, int32_t* out_w);

/* a1 — fp32 Convolution (NCNNToTosa.cpp:1316-1529) with the importer's fused
 * activation (ImportConvolution.cpp:236-248).  weight: host fp32
 * [num_output][C][kernel_h][kernel_w] (the ncnn .bin order,
 * lib/Graph/graph.cpp:1381-1478); bias: host fp32 [num_output] or NULL. */
int nhip_conv2d_f32_create(const nhip_conv_desc* desc, const float* weight,
                           const float* bias, nhip_conv_t* plan);
/* Device scratch bytes a forward call of this batch/shape needs (0 if none). */
int nhip_conv2d_workspace_size(nhip_conv_t plan, int32_t n, int32_t h,
                               int32_t w, uint64_t* bytes);
/* out[n] = act(conv(in[n]) + bias (+ residual[n])).  `residual` (may be NULL)
 * is the second operand of a following ncnn BinaryOp add / Eltwise SUM
 * (NCNNToTosa.cpp:5111-5223); with it the activation applies after the add,
 * which is the order conv -> add -> relu of a ResNet basic block.
 * input [n,C,h,w], output/residual [n,num_output,oh,ow], device pointers. */
int nhip_conv2d_f32_forward(nhip_conv_t plan, const float* input,
                            const float* residual, float* output, int32_t n,
                            int32_t h, int32_t w, void* workspace,
                            uint64_t workspace_bytes, void* stream);
/* No counterpart in the reference: nhip_conv2d_f32_forward for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same kernels and results; the
 * scratch is a static 64 MiB device array per GPU (held until the process
 * ends) instead of a workspace argument, and the call allocates nothing.  A
 * batch needing more scratch than that (nhip_conv2d_workspace_size) returns
 * NHIP_STATUS_OUTPUT_CAPACITY_INSUFFICIENT.  Every call on a GPU shares that
 * GPU's array: calls that overlap on one GPU (other threads, other streams)
 * race. */
int nhip_conv2d_f32_forward_noalloc(nhip_conv_t plan, const float* input,
                                    const float* residual, float* output,
                                    int32_t n, int32_t h, int32_t w,
                                    void* stream);

/* a2 — int8 Convolution (NCNNToTosa.cpp:1136-1315).  weight: host
 * [num_output][C][kh][kw], int8 when weight_is_i8 (used as stored), else fp32
 * quantized per output channel with weight_scale (quantizeConstantToI8,
 * NCNNToTosa.cpp:234-301).  weight_scale: num_output floats, or 1 (scalar,
 * broadcast as in quantizeConstantToI8's scalarScale); input_scale and
 * output_scale (used when int8_scale_term > 100) are scalars
 * (ImportConvolution.cpp:93-121).  bias: fp32 or NULL. */
int nhip_conv2d_int8_create(const nhip_conv_desc* desc, const void* weight,
                            int32_t weight_is_i8, const float* bias,
                            const float* weight_scale,
                            int32_t weight_scale_count, float input_scale,
                            float output_scale, nhip_conv_t* plan);
/* input: fp32 (quantized by input_scale) or int8 when input_is_i8 (used as
 * is, NCNNToTosa.cpp:328-330); output int8 when int8_scale_term > 100, else
 * fp32.  Needs nhip_conv2d_workspace_size bytes of workspace. */
int nhip_conv2d_int8_forward(nhip_conv_t plan, const void* input,
                             int32_t input_is_i8, void* output, int32_t n,
                             int32_t h, int32_t w, void* workspace,
                             uint64_t workspace_bytes, void* stream);

/* a3 — fp32 ConvolutionDepthWise (NCNNToTosa.cpp:3376-3503), group == C
 * (ImportOps.cpp:902-907), activation 0 or 1 (ImportOps.cpp:869-875).
 * weight: host [num_output][1][kh][kw]; bias fp32 or NULL. */
int nhip_dwconv2d_f32_create(const nhip_conv_desc* desc, const float* weight,
                             const float* bias, nhip_conv_t* plan);
int nhip_dwconv2d_f32_forward(nhip_conv_t plan, const float* input,
                              float* output, int32_t n, int32_t h, int32_t w,
                              void* stream);

/* No counterpart in the reference (it lowers every layer on its own): an fp32
 * 3x3 ConvolutionDepthWise (stride 1 or 2, padding 1, its bias and
 * activation) whose output only feeds a 1x1 stride-1 fp32 Convolution, run
 * as one kernel without writing the depthwise output — the depthwise ->
 * project pair of an inverted-residual block, fused by the graph executor.
 * Results are those of nhip_dwconv2d_f32_forward followed by
 * nhip_conv2d_f32_forward (the depthwise values are computed in the same
 * order).  _supported sets *supported to 1 when the pair and the input
 * extent qualify (3x3, padding 1, W and the output width multiples of 4);
 * _forward then takes input [n,C,h,w] of dw, residual/output of pw's shape
 * (residual may be NULL), device pointers, no workspace. */
int nhip_dwconv2d_pw_f32_supported(nhip_conv_t dw, nhip_conv_t pw, int32_t n,
                                   int32_t h, int32_t w, int32_t* supported);
int nhip_dwconv2d_pw_f32_forward(nhip_conv_t dw, nhip_conv_t pw,
                                 const float* input, const float* residual,
                                 float* output, int32_t n, int32_t h, int32_t w,
                                 void* stream);

/* No counterpart in the reference (it lowers every layer on its own): an fp32
 * 1x1 stride-1 unpadded Convolution (ConvertConvolution,
 * NCNNToTosa.cpp:1316-1529; implicit-GEMM plan, 16, 24, 32, 64, 96 or 160
 * input channels) whose output only feeds a 3x3 fp32 ConvolutionDepthWise
 * over its channels (ConvertDepthwiseConvolution, :3074-3503; stride 1 or 2,
 * padding 1), run as one kernel without writing the 1x1 output (whole planes
 * or row strips with a one-row halo) — the expand -> depthwise pair of an
 * inverted-residual block, fused by the graph executor.  Results equal
 * nhip_conv2d_f32_forward followed by nhip_dwconv2d_f32_forward within
 * rounding (the 1x1 sum is formed in another order; the depthwise sum in the
 * reference's).  _supported sets *supported to 1 when the pair and the input
 * extent qualify (planes of at most 784 pixels by default, any plane the LDS
 * takes with NHIP_PWDW=2); _forward then takes input [n,C,h,w] of pw and
 * output of dw's shape, device pointers, no workspace. */
int nhip_conv1x1_dw_f32_supported(nhip_conv_t pw, nhip_conv_t dw, int32_t n,
                                  int32_t h, int32_t w, int32_t* supported);
int nhip_conv1x1_dw_f32_forward(nhip_conv_t pw, nhip_conv_t dw,
                                const float* input, float* output, int32_t n,
                                int32_t h, int32_t w, void* stream);

/* a3 int8 — ConvolutionDepthWise with int8_scale_term (NCNNToTosa.cpp:
 * 3257-3376).  weight: host [C][1][kh][kw], int8 when weight_is_i8 else fp32
 * quantized per channel with weight_scale; weight_scale has C entries
 * (terms 1/101) or 1 (terms 2/102, graph.cpp:1545-1548); input_scale and
 * output_scale (term > 100) are scalars; bias fp32 or NULL.  Activation 0/1. */
int nhip_dwconv2d_int8_create(const nhip_conv_desc* desc, const void* weight,
                              int32_t weight_is_i8, const float* bias,
                              const float* weight_scale,
                              int32_t weight_scale_count, float input_scale,
                              float output_scale, nhip_conv_t* plan);
/* input fp32 (quantized by input_scale) or int8 (input_is_i8); output int8
 * when int8_scale_term > 100, else fp32.  No workspace. */
int nhip_dwconv2d_int8_forward(nhip_conv_t plan, const void* input,
                               int32_t input_is_i8, void* output, int32_t n,
                               int32_t h, int32_t w, void* stream);

int nhip_conv_destroy(nhip_conv_t plan);

/* a4 — fp32 InnerProduct (NCNNToTosa.cpp:5254-5392):
 * out[m][j] = act((sum_k in[m][k] * W[j][k]) + bias[j]).  weight: host
 * [num_output][num_input] (lib/Graph/graph.cpp:1638-1678); bias or NULL;
 * activation 0 or 1 (ImportOps.cpp:741-847 splits it into ncnn.relu). */
int nhip_innerproduct_f32_create(int32_t num_output, int32_t num_input,
                                 const float* weight, const float* bias,
                                 int32_t activation_type, nhip_ip_t* plan);
int nhip_innerproduct_workspace_size(nhip_ip_t plan, int32_t m,
                                     uint64_t* bytes);
/* input [m][num_input], output [m][num_output], device pointers.  m is the
 * dynamic M of the Squeeze -> [?,K] path (NCNNOps.cpp:1270-1280). */
int nhip_innerproduct_f32_forward(nhip_ip_t plan, const float* input,
                                  float* output, int32_t m, void* workspace,
                                  uint64_t workspace_bytes, void* stream);
/* a10 + a4 — global average pooling feeding an fp32 InnerProduct, fused
 * (ConvertPooling global average NCNNToTosa.cpp:1880-1990, then
 * ConvertInnerProduct :5254-5392): output[n][num_output] = InnerProduct of
 * the per-channel means of input [n][C][h][w], C = num_input.  Each mean is
 * the plane summed in order and divided by h*w, as the reference and
 * nhip_global_avgpool_f32 compute it.  Planes of at most 6400 pixels
 * (h*w larger: NHIP_STATUS_CONSTRAINT_VIOLATION; run the two ops).  Needs
 * the workspace this reports for the same n, h, w. */
int nhip_global_avgpool_innerproduct_f32_workspace_size(nhip_ip_t plan,
                                                        int32_t n, int32_t h,
                                                        int32_t w,
                                                        uint64_t* bytes);
int nhip_global_avgpool_innerproduct_f32_forward(nhip_ip_t plan,
                                                 const float* input,
                                                 float* output, int32_t n,
                                                 int32_t c, int32_t h,
                                                 int32_t w, void* workspace,
                                                 uint64_t workspace_bytes,
                                                 void* stream);
/* a4 int8 — InnerProduct with int8_scale_term (NCNNToTosa.cpp:5300-5390):
 * out = act((float)(sum_k q(x)*q(W)) * r[j] + bias[j]), fp32 output.
 * weight: host [num_output][num_input], int8 when weight_is_i8 else fp32
 * quantized per output row; weight_scale: num_output entries (graph.cpp:
 * 1638-1678); input_scale scalar.  Forward: input [m][num_input] fp32 (or
 * int8 when input_is_i8), output [m][num_output] fp32, workspace from
 * nhip_innerproduct_workspace_size. */
int nhip_innerproduct_int8_create(int32_t num_output, int32_t num_input,
                                  const void* weight, int32_t weight_is_i8,
                                  const float* bias, const float* weight_scale,
                                  float input_scale, int32_t activation_type,
                                  nhip_ip_t* plan);
int nhip_innerproduct_int8_forward(nhip_ip_t plan, const void* input,
                                   int32_t input_is_i8, float* output,
                                   int32_t m, void* workspace,
                                   uint64_t workspace_bytes, void* stream);
int nhip_innerproduct_destroy(nhip_ip_t plan);

/* ---------------------------------------------------------------------------
 * Elementwise neighbours of the hot path (device pointers, `count` elements).
 * ------------------------------------------------------------------------- */
/* a8 — ConvertRelu slope 0 (NCNNToTosa.cpp:1532-1578). */
int nhip_relu_f32(const float* input, float* output, int64_t count,
                  void* stream);
int nhip_relu_i8(const int8_t* input, int8_t* output, int64_t count,
                 void* stream);
/* a9 — ConvertBinary add (NCNNToTosa.cpp:5111-5223), optional following relu. */
int nhip_add_f32(const float* a, const float* b, float* output, int64_t count,
                 int32_t relu, void* stream);
/* a10 — Pooling global average (NCNNToTosa.cpp:1880-1990): [n,c,h,w]->[n,c]. */
int nhip_global_avgpool_f32(const float* input, float* output, int32_t n,
                            int32_t c, int32_t h, int32_t w, void* stream);
/* a5 — quantizeSignedI8 (NCNNToTosa.cpp:322-389) over [n, c, plane]:
 * scale_count 1 (scalar) or c (per channel).  `scale` is a device array. */
int nhip_quantize_f32_i8(const float* input, int8_t* output, int32_t n,
                         int32_t c, int64_t plane, const float* scale,
                         int32_t scale_count, void* stream);
/* a7 — ConvertRequantize (NCNNToTosa.cpp:4846-4888) over [n, c, plane]:
 * dequantize (in_scale, bias), optional relu, quantize (out_scale).
 * Device arrays with 1 or c entries; bias may be NULL. */
int nhip_requantize_i32_i8(const int32_t* input, int8_t* output, int32_t n,
                           int32_t c, int64_t plane, const float* in_scale,
                           int32_t in_scale_count, const float* out_scale,
                           int32_t out_scale_count, const float* bias,
                           int32_t bias_count, int32_t activation,
                           void* stream);
/* ConvertDequantize (NCNNToTosa.cpp:4823-4840) over [n, c, plane]; device
 * scale/bias arrays with 1 or c entries, bias may be NULL. */
int nhip_dequantize_i32_f32(const int32_t* input, float* output, int32_t n,
                            int32_t c, int64_t plane, const float* scale,
                            int32_t scale_count, const float* bias,
                            int32_t bias_count, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NHIP_H */
