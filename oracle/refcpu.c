/*
 * refcpu.c — CPU restatement of the reference lowering (see refcpu.h).
 *
 * TEST INFRASTRUCTURE ONLY: a checker and the timed CPU baseline, never part
 * of the product path.  Built with -O3 -ffp-contract=off -fopenmp and no
 * -march, mirroring the reference's default clang -O3 build of its .so
 * (tools/ncnn-compile.cpp:1910-1935) and its OpenMP lowering of the parallel
 * loop dimensions (lib/Pipelines/NCNNPipelines.cpp:88-97).
 *
 * Layout note: the reference keeps rank-3 blobs as NHWC [1,H,W,C] internally
 * (NCNNToTosa.cpp:48-52, 939-965) but the results do not depend on the storage
 * layout, only on the per-element operation order restated here.
 */
#include "refcpu.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

static int pick_threads(int threads) {
  return threads > 0 ? threads : omp_get_max_threads();
}

/* NCNNOps.cpp:44 computeConvResult: out = (in + pt + pb - ((k-1)d+1))/s + 1.
 * The trailing-pad adjustment of NCNNToTosa.cpp:1434-1465 only enlarges the
 * computed region at the bottom/right, which the tosa.slice at :1499-1522 then
 * drops, so the visible output is exactly this extent. */
int ref_conv_out_h(const ref_conv_geom* g) {
  int eff = (g->kernel_h - 1) * g->dilation_h + 1;
  return (g->h + g->pad_top + g->pad_bottom - eff) / g->stride_h + 1;
}

int ref_conv_out_w(const ref_conv_geom* g) {
  int eff = (g->kernel_w - 1) * g->dilation_w + 1;
  return (g->w + g->pad_left + g->pad_right - eff) / g->stride_w + 1;
}

/* Zero-padded read (tosa.pad / tensor.pad with a zero pad constant). */
static inline float padded_f32(const float* plane, int h, int w, int y, int x) {
  if (y < 0 || y >= h || x < 0 || x >= w) return 0.0f;
  return plane[(int64_t)y * w + x];
}

/* a1 — NCNNToTosa.cpp:1316-1529 (fp32 path of ConvertConvolution).
 * tosa.conv2d with a bias operand lowers (upstream TOSA->Linalg) to a
 * bias-broadcast init followed by linalg.conv_2d_nhwc_hwcf, whose reduction
 * iterators are (kh, kw, c) innermost-last: acc = bias; acc += x*w in that
 * order, each mul and add rounded separately. */
void ref_conv2d_f32(const ref_conv_geom* g, const float* input,
                    const float* weight, const float* bias, float* output,
                    int threads) {
  const int oh_n = ref_conv_out_h(g), ow_n = ref_conv_out_w(g);
  const int C = g->c, H = g->h, W = g->w, K = g->k;
  const int KH = g->kernel_h, KW = g->kernel_w;
  const int64_t in_img = (int64_t)C * H * W;
  const int64_t out_img = (int64_t)K * oh_n * ow_n;
#pragma omp parallel for collapse(3) num_threads(pick_threads(threads)) schedule(static)
  for (int n = 0; n < g->n; ++n) {
    for (int oh = 0; oh < oh_n; ++oh) {
      for (int ow = 0; ow < ow_n; ++ow) {
        const float* img = input + n * in_img;
        for (int f = 0; f < K; ++f) {
          float acc = bias ? bias[f] : 0.0f;
          const float* wf = weight + (int64_t)f * C * KH * KW;
          for (int kh = 0; kh < KH; ++kh) {
            const int y = oh * g->stride_h - g->pad_top + kh * g->dilation_h;
            for (int kw = 0; kw < KW; ++kw) {
              const int x = ow * g->stride_w - g->pad_left + kw * g->dilation_w;
              for (int c = 0; c < C; ++c) {
                float prod = padded_f32(img + (int64_t)c * H * W, H, W, y, x) *
                             wf[((int64_t)c * KH + kh) * KW + kw];
                acc = acc + prod;
              }
            }
          }
          output[n * out_img + ((int64_t)f * oh_n + oh) * ow_n + ow] = acc;
        }
      }
    }
  }
}

/* a3 — NCNNToTosa.cpp:3376-3503.  tosa.depthwise_conv2d lowers to a
 * zero-filled linalg.depthwise_conv_2d_nhwc_hwcm (reduction kh, kw) followed
 * by a separate bias-add generic.  group == C; output channel o reads input
 * channel o / multiplier (weights reshaped [C,M,kh,kw] -> HWCM, :3164-3180). */
void ref_dwconv2d_f32(const ref_conv_geom* g, const float* input,
                      const float* weight, const float* bias, float* output,
                      int threads) {
  const int oh_n = ref_conv_out_h(g), ow_n = ref_conv_out_w(g);
  const int C = g->c, H = g->h, W = g->w, K = g->k;
  const int mult = K / C;
  const int KH = g->kernel_h, KW = g->kernel_w;
  const int64_t in_img = (int64_t)C * H * W;
  const int64_t out_img = (int64_t)K * oh_n * ow_n;
#pragma omp parallel for collapse(3) num_threads(pick_threads(threads)) schedule(static)
  for (int n = 0; n < g->n; ++n) {
    for (int o = 0; o < K; ++o) {
      for (int oh = 0; oh < oh_n; ++oh) {
        const float* plane = input + n * in_img + (int64_t)(o / mult) * H * W;
        const float* wo = weight + (int64_t)o * KH * KW;
        for (int ow = 0; ow < ow_n; ++ow) {
          float acc = 0.0f;
          for (int kh = 0; kh < KH; ++kh) {
            const int y = oh * g->stride_h - g->pad_top + kh * g->dilation_h;
            for (int kw = 0; kw < KW; ++kw) {
              const int x = ow * g->stride_w - g->pad_left + kw * g->dilation_w;
              float prod = padded_f32(plane, H, W, y, x) * wo[kh * KW + kw];
              acc = acc + prod;
            }
          }
          if (bias) acc = acc + bias[o];
          output[n * out_img + ((int64_t)o * oh_n + oh) * ow_n + ow] = acc;
        }
      }
    }
  }
}

/* a4 — NCNNToTosa.cpp:5254-5392.  tosa.matmul [1,M,K]x[1,K,N] lowers to a
 * zero-filled linalg.batch_matmul (reduction k ascending); the bias is a
 * separate tosa.add afterwards (:5371-5381).  Weight [N][K] is transposed to
 * [K][N] at compile time (:5339-5350), which changes no arithmetic. */
void ref_innerproduct_f32(int32_t m, int32_t k, int32_t n, const float* input,
                          const float* weight, const float* bias,
                          float* output, int threads) {
#pragma omp parallel for collapse(2) num_threads(pick_threads(threads)) schedule(static)
  for (int i = 0; i < m; ++i) {
    for (int j = 0; j < n; ++j) {
      const float* x = input + (int64_t)i * k;
      const float* wj = weight + (int64_t)j * k;
      float acc = 0.0f;
      for (int t = 0; t < k; ++t) {
        float prod = x[t] * wj[t];
        acc = acc + prod;
      }
      if (bias) acc = acc + bias[j];
      output[(int64_t)i * n + j] = acc;
    }
  }
}

/* a5 — quantizeSignedI8, NCNNToTosa.cpp:322-389 (runtime generic) and its
 * constant-folding twin quantizeConstantToI8 :234-301:
 *   s = x*scale; r = s >= 0 ? floor(s+0.5) : ceil(s-0.5);
 *   clamp(r, -127, 127) (minimumf then maximumf); fptosi.
 * A NaN product is poison in the reference; it maps to 0 here. */
int8_t ref_quantize_one(float x, float scale) {
  float s = x * scale;
  if (s != s) return 0;
  float r = (s >= 0.0f) ? floorf(s + 0.5f) : ceilf(s - 0.5f);
  if (r > 127.0f) r = 127.0f;
  if (r < -127.0f) r = -127.0f;
  return (int8_t)(int)r;
}

void ref_quantize_f32_i8(int64_t count, const float* input, const float* scale,
                         int32_t scale_count, int64_t channel_size,
                         int8_t* output) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < count; ++i) {
    int64_t si = scale_count == 1 ? 0 : i / channel_size;
    output[i] = ref_quantize_one(input[i], scale[si]);
  }
}

/* a6 — dequantizeAccumulator, NCNNToTosa.cpp:577-637: combined = ws*is
 * (tosa.mul), reciprocal = 1/combined (tosa.reciprocal -> arith.divf),
 * select(ws == 0, 0, reciprocal). */
void ref_dequant_reciprocal(int32_t count, const float* weight_scale,
                            float input_scale, float* reciprocal) {
  for (int i = 0; i < count; ++i) {
    float combined = weight_scale[i] * input_scale;
    float r = 1.0f / combined;
    reciprocal[i] = weight_scale[i] == 0.0f ? 0.0f : r;
  }
}

void ref_conv2d_i8_acc(const ref_conv_geom* g, const int8_t* input,
                       const int8_t* weight, int64_t* acc, int threads) {
  const int oh_n = ref_conv_out_h(g), ow_n = ref_conv_out_w(g);
  const int C = g->c, H = g->h, W = g->w, K = g->k;
  const int KH = g->kernel_h, KW = g->kernel_w;
  const int64_t in_img = (int64_t)C * H * W;
  const int64_t out_img = (int64_t)K * oh_n * ow_n;
#pragma omp parallel for collapse(3) num_threads(pick_threads(threads)) schedule(static)
  for (int n = 0; n < g->n; ++n) {
    for (int f = 0; f < K; ++f) {
      for (int oh = 0; oh < oh_n; ++oh) {
        const int8_t* img = input + n * in_img;
        const int8_t* wf = weight + (int64_t)f * C * KH * KW;
        for (int ow = 0; ow < ow_n; ++ow) {
          int64_t s = 0;
          for (int kh = 0; kh < KH; ++kh) {
            const int y = oh * g->stride_h - g->pad_top + kh * g->dilation_h;
            if (y < 0 || y >= H) continue;
            for (int kw = 0; kw < KW; ++kw) {
              const int x = ow * g->stride_w - g->pad_left + kw * g->dilation_w;
              if (x < 0 || x >= W) continue;
              for (int c = 0; c < C; ++c) {
                s += (int64_t)img[((int64_t)c * H + y) * W + x] *
                     (int64_t)wf[((int64_t)c * KH + kh) * KW + kw];
              }
            }
          }
          acc[n * out_img + ((int64_t)f * oh_n + oh) * ow_n + ow] = s;
        }
      }
    }
  }
}

/* a2 — NCNNToTosa.cpp:1136-1315 (int8 path of ConvertConvolution):
 *   q_in = quantizeSignedI8(x, is)          (no-op for int8 input, :328-330)
 *   acc  = tosa.conv2d i8 x i8 -> i32, zero points 0, zero i32 bias
 *   f    = (float)acc * r[c]                (dequantizeAccumulator, :577-637)
 *   f    = f + bias[c]                      (tosa.add, :1294-1300)
 *   term > 100: out = quantizeSignedI8(f, os)  (:1309-1312)
 * then the importer's separate ncnn.relu (ImportConvolution.cpp:236-241) as
 * tosa.clamp [0, +inf] on fp32 or [0, 127] on int8 (:1532-1560). */
void ref_conv2d_int8(const ref_conv_geom* g, const void* input,
                     int32_t input_is_i8, const int8_t* weight,
                     const float* bias, const float* weight_scale,
                     int32_t weight_scale_count, float input_scale,
                     float output_scale, int32_t scale_term,
                     int32_t activation, void* output, int threads) {
  const int oh_n = ref_conv_out_h(g), ow_n = ref_conv_out_w(g);
  const int64_t in_count = (int64_t)g->n * g->c * g->h * g->w;
  const int64_t out_img = (int64_t)g->k * oh_n * ow_n;
  const int64_t out_count = (int64_t)g->n * out_img;
  int8_t* q = (int8_t*)malloc((size_t)in_count);
  int64_t* acc = (int64_t*)malloc((size_t)out_count * sizeof(int64_t));
  float* recip = (float*)malloc((size_t)g->k * sizeof(float));
  if (input_is_i8) {
    memcpy(q, input, (size_t)in_count);
  } else {
    ref_quantize_f32_i8(in_count, (const float*)input, &input_scale, 1, 1, q);
  }
  ref_conv2d_i8_acc(g, q, weight, acc, threads);
  for (int c = 0; c < g->k; ++c) {
    float ws = weight_scale[weight_scale_count == 1 ? 0 : c];
    ref_dequant_reciprocal(1, &ws, input_scale, &recip[c]);
  }
  const int64_t plane = (int64_t)oh_n * ow_n;
#pragma omp parallel for schedule(static) num_threads(pick_threads(threads))
  for (int64_t i = 0; i < out_count; ++i) {
    const int c = (int)((i % out_img) / plane);
    /* sitofp of the i32 accumulator (the i32 conv result is exact here). */
    float f = (float)(int32_t)acc[i];
    f = f * recip[c];
    if (bias) f = f + bias[c];
    if (scale_term > 100) {
      int8_t v = ref_quantize_one(f, output_scale);
      if (activation == 1 && v < 0) v = 0;
      ((int8_t*)output)[i] = v;
    } else {
      if (activation == 1) f = f < 0.0f ? 0.0f : f;
      ((float*)output)[i] = f;
    }
  }
  free(q);
  free(acc);
  free(recip);
}

/* a7 — ConvertRequantize, NCNNToTosa.cpp:4846-4888, via dequantizeNcnn
 * :411-460 ((float)x * scale, then + bias) and quantizeSignedI8. */
void ref_requantize_i32_i8(int32_t c, int64_t channel_size, const int32_t* input,
                           const float* in_scale, int32_t in_scale_count,
                           const float* out_scale, int32_t out_scale_count,
                           const float* bias, int32_t bias_count,
                           int32_t activation, int8_t* output) {
  const int64_t count = (int64_t)c * channel_size;
  for (int64_t i = 0; i < count; ++i) {
    const int64_t ch = i / channel_size;
    float f = (float)input[i] * in_scale[in_scale_count == 1 ? 0 : ch];
    if (bias) f = f + bias[bias_count == 1 ? 0 : ch];
    if (activation == 1) f = f < 0.0f ? 0.0f : f;
    output[i] = ref_quantize_one(f, out_scale[out_scale_count == 1 ? 0 : ch]);
  }
}

/* ConvertDequantize, NCNNToTosa.cpp:4823-4840 -> dequantizeNcnn :411-460. */
void ref_dequantize_i32_f32(int32_t c, int64_t channel_size, const int32_t* input,
                            const float* scale, int32_t scale_count,
                            const float* bias, int32_t bias_count, float* output) {
  const int64_t count = (int64_t)c * channel_size;
  for (int64_t i = 0; i < count; ++i) {
    const int64_t ch = i / channel_size;
    float f = (float)input[i] * scale[scale_count == 1 ? 0 : ch];
    if (bias) f = f + bias[bias_count == 1 ? 0 : ch];
    output[i] = f;
  }
}

/* a8 — ConvertRelu, NCNNToTosa.cpp:1532-1578 (slope 0 -> tosa.clamp). */
void ref_relu_f32(int64_t count, const float* input, float* output) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < count; ++i) {
    float v = input[i];
    output[i] = v < 0.0f ? 0.0f : v;
  }
}

void ref_relu_i8(int64_t count, const int8_t* input, int8_t* output) {
  for (int64_t i = 0; i < count; ++i) output[i] = input[i] < 0 ? 0 : input[i];
}

/* a9 — ConvertBinary op 0, NCNNToTosa.cpp:5111-5223 (tosa.add). */
void ref_add_f32(int64_t count, const float* a, const float* b, float* output) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < count; ++i) output[i] = a[i] + b[i];
}

/* a10 — ConvertPooling global average, NCNNToTosa.cpp:1880-1990:
 * tosa.avg_pool2d over the whole plane = pooling sum (h outer, w inner)
 * followed by a division by the element count. */
void ref_global_avgpool_f32(int32_t n, int32_t c, int32_t h, int32_t w,
                            const float* input, float* output) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int i = 0; i < n; ++i) {
    for (int ch = 0; ch < c; ++ch) {
      const float* p = input + ((int64_t)i * c + ch) * h * w;
      float s = 0.0f;
      for (int y = 0; y < h; ++y)
        for (int x = 0; x < w; ++x) s = s + p[y * w + x];
      output[(int64_t)i * c + ch] = s / (float)(h * w);
    }
  }
}

/* a11 — foldBatchNormIntoConvolution, FoldNCNNBatchNorm.cpp:56-177:
 *   v = var + eps; k = v == 0 ? 1e4 : pow(v, -0.5); scale = slope*k;
 *   offset = beta - scale*mean; W' = W*scale[o]; b' = b*scale + offset.
 * Returns 0 when folding is refused (non-finite k or bias). */
int ref_bn_fold(int32_t k, int64_t per_out, float* weight, const float* bias,
                const float* slope, const float* mean, const float* variance,
                const float* bn_bias, float epsilon, float* bias_out) {
  for (int o = 0; o < k; ++o) {
    const float v = variance[o] + epsilon;
    const float inv = v == 0.0f ? 10000.0f : powf(v, -0.5f);
    if (!isfinite(inv)) return 0;
    if (bias && !isfinite(bias[o])) return 0;
  }
  for (int o = 0; o < k; ++o) {
    const float v = variance[o] + epsilon;
    const float inv = v == 0.0f ? 10000.0f : powf(v, -0.5f);
    const float scale = slope[o] * inv;
    const float sm = scale * mean[o];
    const float offset = bn_bias[o] - sm;
    for (int64_t i = 0; i < per_out; ++i)
      weight[o * per_out + i] = weight[o * per_out + i] * scale;
    if (bias) {
      const float bs = bias[o] * scale;
      bias_out[o] = bs + offset;
    } else {
      bias_out[o] = offset;
    }
  }
  return 1;
}

/* a12 — computeSamePadding, NormalizeNCNN.cpp:31-50. */
void ref_same_padding(int32_t input, int32_t kernel, int32_t stride,
                      int32_t dilation, int32_t type, int32_t* before,
                      int32_t* after) {
  const int64_t extent = (int64_t)dilation * (kernel - 1) + 1;
  const int64_t out = 1 + (input - 1) / stride;
  const int64_t required = (out - 1) * stride + extent;
  const int64_t total = required > input ? required - input : 0;
  const int same_lower = type == -234;
  const int64_t b = same_lower ? total / 2 + total % 2 : total / 2;
  *before = (int32_t)b;
  *after = (int32_t)(total - b);
}

/* Shared int8 epilogue: (float)acc * r, + bias, then either requantize by
 * os (term > 100) with relu on int8, or relu on fp32 (NCNNToTosa.cpp:577-637,
 * :1292-1312, ConvertRelu :1532-1578). */
static void int8_epilogue(int64_t acc, float r, const float* bias, int c,
                          float os, int32_t term, int32_t act, void* out,
                          int64_t i) {
  float f = (float)(int32_t)acc;
  f = f * r;
  if (bias) f = f + bias[c];
  if (term > 100) {
    int8_t v = ref_quantize_one(f, os);
    if (act == 1 && v < 0) v = 0;
    ((int8_t*)out)[i] = v;
  } else {
    if (act == 1) f = f < 0.0f ? 0.0f : f;
    ((float*)out)[i] = f;
  }
}

void ref_dwconv2d_int8(const ref_conv_geom* g, const void* input,
                       int32_t input_is_i8, const int8_t* weight,
                       const float* bias, const float* weight_scale,
                       int32_t weight_scale_count, float input_scale,
                       float output_scale, int32_t scale_term,
                       int32_t activation, void* output, int threads) {
  const int oh_n = ref_conv_out_h(g), ow_n = ref_conv_out_w(g);
  const int C = g->c, H = g->h, W = g->w, KH = g->kernel_h, KW = g->kernel_w;
  const int64_t in_count = (int64_t)g->n * C * H * W;
  int8_t* q = (int8_t*)malloc((size_t)in_count);
  float* recip = (float*)malloc((size_t)C * sizeof(float));
  if (input_is_i8) {
    memcpy(q, input, (size_t)in_count);
  } else {
    ref_quantize_f32_i8(in_count, (const float*)input, &input_scale, 1, 1, q);
  }
  for (int c = 0; c < C; ++c) {
    float ws = weight_scale[weight_scale_count == 1 ? 0 : c];
    ref_dequant_reciprocal(1, &ws, input_scale, &recip[c]);
  }
#pragma omp parallel for collapse(2) num_threads(pick_threads(threads)) schedule(static)
  for (int n = 0; n < g->n; ++n) {
    for (int c = 0; c < C; ++c) {
      const int8_t* plane = q + ((int64_t)n * C + c) * H * W;
      const int8_t* wc = weight + (int64_t)c * KH * KW;
      for (int oh = 0; oh < oh_n; ++oh) {
        for (int ow = 0; ow < ow_n; ++ow) {
          int64_t s = 0;
          for (int kh = 0; kh < KH; ++kh) {
            const int y = oh * g->stride_h - g->pad_top + kh * g->dilation_h;
            if (y < 0 || y >= H) continue;
            for (int kw = 0; kw < KW; ++kw) {
              const int x = ow * g->stride_w - g->pad_left + kw * g->dilation_w;
              if (x < 0 || x >= W) continue;
              s += (int64_t)plane[(int64_t)y * W + x] * (int64_t)wc[kh * KW + kw];
            }
          }
          const int64_t i = (((int64_t)n * C + c) * oh_n + oh) * ow_n + ow;
          int8_epilogue(s, recip[c], bias, c, output_scale, scale_term, activation, output, i);
        }
      }
    }
  }
  free(q);
  free(recip);
}

void ref_innerproduct_int8(int32_t m, int32_t k, int32_t n, const void* input,
                           int32_t input_is_i8, const int8_t* weight,
                           const float* bias, const float* weight_scale,
                           float input_scale, int32_t activation,
                           float* output, int threads) {
  const int64_t in_count = (int64_t)m * k;
  int8_t* q = (int8_t*)malloc((size_t)in_count);
  float* recip = (float*)malloc((size_t)n * sizeof(float));
  if (input_is_i8) {
    memcpy(q, input, (size_t)in_count);
  } else {
    ref_quantize_f32_i8(in_count, (const float*)input, &input_scale, 1, 1, q);
  }
  ref_dequant_reciprocal(n, weight_scale, input_scale, recip);
#pragma omp parallel for collapse(2) num_threads(pick_threads(threads)) schedule(static)
  for (int i = 0; i < m; ++i) {
    for (int j = 0; j < n; ++j) {
      int64_t s = 0;
      for (int t = 0; t < k; ++t)
        s += (int64_t)q[(int64_t)i * k + t] * (int64_t)weight[(int64_t)j * k + t];
      int8_epilogue(s, recip[j], bias, j, 1.0f, 1, activation, output, (int64_t)i * n + j);
    }
  }
  free(q);
  free(recip);
}
