/*
 * nhip_graph.h — ncnn model execution on libnhip: the `.param/.bin` parser,
 * the lowering of the parsed graph to a call plan of nhip_* kernels, and the
 * executor.  Plain C ABI (opaque handle, pointers, sizes).
 *
 * Replaces, in the reference (hqu-little-boy/ncnn-compiler):
 *   - lib/Graph/{graph,parser}.cpp (Graph::load graph.cpp:2129-2333, the
 *     tagged weight loader graph.cpp:1260-1327 and the per-layer loaders
 *     graph.cpp:1381-1678,1960-2030) for the layer types below;
 *   - the pipeline that lowers them to CPU loops
 *     (lib/Conversion/NCNNToTosa/NCNNToTosa.cpp, lib/Pipelines/NCNNPipelines.cpp)
 *     with fold-ncnn-batchnorm (lib/Transforms/FoldNCNNBatchNorm.cpp:56-177);
 *   - the body of the generated entry point `int <model>(inputs..., outputs...)`
 *     (tools/ncnn-compile.cpp:915-932; GenerateCAPI.cpp:1460-1590): a
 *     generated library calls nhip_graph_run_host with the caller's buffers.
 *
 * Layer types: Input, Convolution and ConvolutionDepthWise (fp32, int8 terms
 * 1/2/101/102), InnerProduct (fp32, int8 terms 1/2), ReLU (slope 0),
 * BatchNorm (folded into the producing fp32 convolution), BinaryOp add and
 * Eltwise sum of equal shapes, Pooling global average, Quantize, Dequantize
 * and Requantize (on i32 Input blobs, the reference's integer storage),
 * Split, Reshape/Flatten/Squeeze, Dropout/Noop.  Anything else is rejected with
 * NHIP_STATUS_UNSUPPORTED and a message naming the layer.
 *
 * Shapes: an ncnn blob is [C,H,W] (rank 3) or a rank 1/2 view of it.  An
 * Input's extents come from its .param dims or from `input_shapes`; -1 marks
 * an extent given at run time (the reference's "?" of --input-shape).
 */
#ifndef NHIP_GRAPH_H
#define NHIP_GRAPH_H

#include <stdint.h>

#include "nhip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define NHIP_DTYPE_F32 0
#define NHIP_DTYPE_I8 1
#define NHIP_DTYPE_I32 2 /* Input blobs read by Dequantize / Requantize / Embed */

typedef struct nhip_graph* nhip_graph_t;

/* Parse and lower a model held in memory.  input_shapes: NULL, or
 * input_shape_count rank-3 CHW shapes (3 int64 each, -1 = dynamic), one per
 * Input layer in source order, overriding the .param dims (the reference's
 * --input-shape, docs/ncnn-compile-command-line.md section 2.5).  Weights are
 * uploaded to the calling thread's current device, which the graph keeps.
 * On error *graph is NULL and
 * nhip_last_error() names the layer. */
int nhip_graph_load(const char* param_text, uint64_t param_len, const void* bin,
                    uint64_t bin_len, const int64_t* input_shapes,
                    int32_t input_shape_count, nhip_graph_t* graph);

/* Same parsing, validation, lowering and shape rules as nhip_graph_load, but
 * no device work at all (no plans, no uploads): the handle answers
 * nhip_graph_num_io / io_info / infer_shapes and is what a compiler running
 * on a host without a GPU uses.  nhip_graph_run* on it return
 * NHIP_STATUS_CONSTRAINT_VIOLATION. */
int nhip_graph_describe(const char* param_text, uint64_t param_len,
                        const void* bin, uint64_t bin_len,
                        const int64_t* input_shapes, int32_t input_shape_count,
                        nhip_graph_t* graph);

int nhip_graph_num_io(nhip_graph_t graph, int32_t* inputs, int32_t* outputs);

/* Declared shape of input/output `index` (rank 1..4, extents, -1 where
 * dynamic), element type NHIP_DTYPE_* and blob name. */
int nhip_graph_io_info(nhip_graph_t graph, int32_t is_output, int32_t index,
                       int32_t* rank, int64_t dims[4], int32_t* dtype,
                       const char** name);

/* Output shapes for concrete input shapes (3 extents per input, NULL when
 * no input is dynamic): 4 slots per output in output_shapes, ranks in
 * output_ranks.  Checks the same shape rules as a run. */
int nhip_graph_infer_shapes(nhip_graph_t graph, const int64_t* input_shapes,
                            int64_t* output_shapes, int32_t* output_ranks);

/* Batch execution on device memory: n images per input, inputs[i] and
 * outputs[j] are device pointers of n back-to-back blobs.  input_shapes as in
 * nhip_graph_infer_shapes.  An output buffer that is 256-byte aligned and
 * overlaps no input is written by the layer that computes it (no copy at the
 * end); other outputs are copied there after the last layer.  Calls on one
 * graph are serialised (it owns the
 * intermediate buffers).  Kernels run on the device the graph was loaded
 * on; the calling thread's current device is restored afterwards.  On a
 * non-default stream, a call repeating the previous call's batch, shapes,
 * buffers and stream is recorded into a hipGraph, and later such calls
 * replay it.
 * A call on a stream the caller is capturing launches into the caller's
 * graph.  Such a capture is only valid when the batch and shapes do not
 * exceed those of a call already run on this graph: the executor's
 * intermediate buffers cannot grow inside a capture, and the call then
 * fails with NHIP_STATUS_CONSTRAINT_VIOLATION (launching nothing).  After a
 * caller's capture, buffers superseded by a later, larger call are kept
 * until nhip_graph_destroy, so the caller's graph stays replayable for the
 * graph's lifetime. */
int nhip_graph_run(nhip_graph_t graph, int32_t n, const int64_t* input_shapes,
                   const void* const* inputs, void* const* outputs,
                   void* stream);

/* The reference entry semantics: one image, host buffers, synchronous.
 * output_capacity (elements per output, NULL = not checked) returns
 * NHIP_STATUS_OUTPUT_CAPACITY_INSUFFICIENT when too small.  Runs on the
 * graph's own stream on the device the graph was loaded on (the calling
 * thread's current device is left as it was), staging the copies through
 * pinned host buffers; repeated calls replay one recorded hipGraph of the
 * plan.  Serialised per graph, so concurrent callers are safe. */
int nhip_graph_run_host(nhip_graph_t graph, const int64_t* input_shapes,
                        const void* const* inputs, void* const* outputs,
                        const uint64_t* output_capacity);

int nhip_graph_destroy(nhip_graph_t graph);

#ifdef __cplusplus
}
#endif

#endif /* NHIP_GRAPH_H */
