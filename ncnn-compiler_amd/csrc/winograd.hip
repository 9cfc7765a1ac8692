// Winograd F(4x4, 3x3) for 3x3, stride 1, dilation 1 Convolution.
//
// The reference has no Winograd: its 3x3 conv is the plain
// linalg.conv_2d_nhwc_hwcf loop nest (NCNNToTosa.cpp:1485-1498,
// NCNNPipelines.cpp:54-56).  This is the build's own algorithm choice with the
// reference's result (bias + sum x*w, then activation), checked to a 1e-3
// relative budget.
//
// Transform matrices: interpolation points 0, 1, -1, 2, -2 and infinity
// (Lavin & Gray, "Fast Algorithms for Convolutional Neural Networks", 2016):
//   Y = A^T [ (G g G^T) .* (B^T d B) ] A
// with 6x6 input tiles d overlapping by 2, 4x4 output tiles Y.
//
// Three kernels, all launched on the caller's stream:
//   1. input transform  x[N,C,H,W] -> V[36][c_pad][t_pad]  (HBM bound)
//   2. 36 batched MFMA GEMMs M[xi] = U[xi] (m_pad x c_pad) * V[xi]
//   3. output transform M -> out[N,K,OH,OW] with bias, residual add and the
//      activation fused (HBM bound).
// The weight transform U = G g G^T is done once on the host at plan creation.
#include <cstdlib>
#include <type_traits>
#include <vector>

#include "nhip_internal.h"

namespace nhip {
// winograd_fused.hip: the batched GEMM with the output transform fused.
int launch_wino_gemm_out(const nhip_conv_plan* p, const float* V, int t_pad, const float* residual, float* out,
                         int n, int oh, int ow, float* parts, hipStream_t s);
uint64_t wino_gemm_out_parts_bytes(const nhip_conv_plan* p, int n, int oh, int ow);
bool wino_xt_selected(const nhip_conv_plan* p, int n, int h, int w, int oh, int ow);
int launch_wino_gemm_xt(const nhip_conv_plan* p, const float* in, const float* residual, float* out, int n, int h,
                        int w, int oh, int ow, hipStream_t s);

// Path selection: input transform + GEMM with the output transform fused
// (winograd_fused.hip), or the three-kernel path (M through HBM).
// NHIP_WINOGRAD_VARIANT = 1 forces the three-kernel path, 2 the fused GEMM
// (where its limits allow); unset or 0 chooses by shape: the fused GEMM from
// 128 tiles up (four 32-tile blocks; below that the three-kernel path).
static int variant_requested() {
  return setting_int("NHIP_WINOGRAD_VARIANT", 0);
}

static bool fused_selected(const nhip_conv_plan* p, int n, int oh, int ow) {
  // The fused GEMM's limit: V (32-bit buffer offsets) below 2 GiB.
  const int64_t t_pad = round_up((int64_t)n * ceil_div(oh, 4) * ceil_div(ow, 4), 128);
  if ((int64_t)36 * p->c_pad * t_pad * (int64_t)sizeof(float) >= (int64_t(1) << 31)) return false;
  const int v = variant_requested();
  if (v == 1) return false;
  if (v == 2) return true;
  return (int64_t)n * ceil_div(oh, 4) * ceil_div(ow, 4) >= 128;
}

namespace {

struct WinoShape {
  int n, c, h, w, oh, ow, th, tw, t, t_pad, c_pad, m_pad;
};

WinoShape wino_shape(const nhip_conv_plan* p, int n, int h, int w, int oh, int ow) {
  WinoShape s;
  s.n = n;
  s.c = p->g.c;
  s.h = h;
  s.w = w;
  s.oh = oh;
  s.ow = ow;
  s.th = (int)ceil_div(oh, 4);
  s.tw = (int)ceil_div(ow, 4);
  s.t = n * s.th * s.tw;
  s.t_pad = (int)round_up(s.t, 128);
  s.c_pad = p->c_pad;
  s.m_pad = p->m_pad;
  return s;
}

// Row i of B^T d for one column (d0..d5 = column j of the patch), the
// interpolation-point rows of B^T for F(4x4, 3x3).
template <int I>
__device__ __forceinline__ float bt_row(float d0, float d1, float d2, float d3, float d4, float d5) {
  if constexpr (I == 0) return 4.f * d0 - 5.f * d2 + d4;
  if constexpr (I == 1) return -4.f * (d1 + d2) + d3 + d4;
  if constexpr (I == 2) return 4.f * (d1 - d2) - d3 + d4;
  if constexpr (I == 3) return -2.f * (d1 - d3) - d2 + d4;
  if constexpr (I == 4) return 2.f * (d1 - d3) - d2 + d4;
  return 4.f * d1 - 5.f * d3 + d5;
}

// V = B^T d B for one (channel, tile), stored V[6i + j] at vout + (6i + j) *
// plane_stride.  Loads of rows outside the image (or of a padding tile or
// channel, ok = false) return 0.
template <bool VEC>
__device__ __forceinline__ void wino_in_patch(__amdgpu_buffer_rsrc_t rs, bool ok, int plane, int H, int W, int y0,
                                              int x0, float* __restrict__ vout, int64_t plane_stride) {
  float d[6][6];
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    const int y = y0 + i;
    const bool yok = ok && (unsigned)y < (unsigned)H;
    if constexpr (VEC) {
      const uint32_t rb = (uint32_t)((plane + y) * W * (int)sizeof(float));
      d[i][0] = buf_load_f32(rs, (yok && x0 >= 0) ? rb + (uint32_t)(x0 * 4) : kBufOOB);
      const int4 m = buf_load_b128(rs, (yok && x0 + 1 < W) ? rb + (uint32_t)((x0 + 1) * 4) : kBufOOB);
      d[i][1] = __builtin_bit_cast(float, m.x);
      d[i][2] = __builtin_bit_cast(float, m.y);
      d[i][3] = __builtin_bit_cast(float, m.z);
      d[i][4] = __builtin_bit_cast(float, m.w);
      d[i][5] = buf_load_f32(rs, (yok && x0 + 5 < W) ? rb + (uint32_t)((x0 + 5) * 4) : kBufOOB);
    } else {
#pragma unroll
      for (int j = 0; j < 6; ++j) {
        const int xx = x0 + j;
        const uint32_t off =
            (yok && (unsigned)xx < (unsigned)W) ? (uint32_t)(((plane + y) * W + xx) * (int)sizeof(float)) : kBufOOB;
        d[i][j] = buf_load_f32(rs, off);
      }
    }
  }
  auto row = [&](auto ic) {
    constexpr int i = decltype(ic)::value;
    float tr[6];  // row i of B^T d
#pragma unroll
    for (int j = 0; j < 6; ++j) tr[j] = bt_row<i>(d[0][j], d[1][j], d[2][j], d[3][j], d[4][j], d[5][j]);
    // (B^T d)[i] B: the same six combinations along the row
    vout[(6 * i + 0) * plane_stride] = bt_row<0>(tr[0], tr[1], tr[2], tr[3], tr[4], tr[5]);
    vout[(6 * i + 1) * plane_stride] = bt_row<1>(tr[0], tr[1], tr[2], tr[3], tr[4], tr[5]);
    vout[(6 * i + 2) * plane_stride] = bt_row<2>(tr[0], tr[1], tr[2], tr[3], tr[4], tr[5]);
    vout[(6 * i + 3) * plane_stride] = bt_row<3>(tr[0], tr[1], tr[2], tr[3], tr[4], tr[5]);
    vout[(6 * i + 4) * plane_stride] = bt_row<4>(tr[0], tr[1], tr[2], tr[3], tr[4], tr[5]);
    vout[(6 * i + 5) * plane_stride] = bt_row<5>(tr[0], tr[1], tr[2], tr[3], tr[4], tr[5]);
  };
  row(std::integral_constant<int, 0>{});
  row(std::integral_constant<int, 1>{});
  row(std::integral_constant<int, 2>{});
  row(std::integral_constant<int, 3>{});
  row(std::integral_constant<int, 4>{});
  row(std::integral_constant<int, 5>{});
}

// Thread (c, t): the 6x6 transform of the zero-padded patch of channel c,
// tile t.  Layouts:
//   QUADS  V[xi][c_pad/4][t_pad][4] (the fused GEMM's 4-channel groups); the
//          four channels of a group are neighbouring lanes, so a wave's
//          stores for one point cover 256 contiguous bytes;
//   else   V[xi][c_pad][t_pad].
// VEC (left padding 1, W % 4 == 0, 16-byte aligned input): columns 1..4 of a
// patch row are the aligned run x = 4*tx .. +3, wholly inside the row or
// wholly past its end, loaded as one 16-byte vector.
template <bool QUADS, bool VEC>
__global__ __launch_bounds__(256) void wino_input_transform(
    const float* __restrict__ x, uint32_t x_bytes, float* __restrict__ V, int C, int H, int W,
    int th, int tw, int T, int t_pad, int c_pad, int pt, int pl) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_block = (int64_t)c_pad * t_pad;
  if (idx >= per_block) return;
  const int64_t rem = idx;
  int c, t;
  float* vout;
  if constexpr (QUADS) {
    const int e = (int)(rem & 3);
    const int64_t q = rem >> 2;
    const int cq = (int)(q / t_pad);
    t = (int)(q - (int64_t)cq * t_pad);
    c = 4 * cq + e;
    vout = V + ((int64_t)cq * t_pad + t) * 4 + e;
  } else {
    c = (int)(rem / t_pad);
    t = (int)(rem - (int64_t)c * t_pad);
    vout = V + (int64_t)c * t_pad + t;
  }
  const int64_t plane_stride = per_block;
  const int per_img = th * tw;
  const bool t_ok = t < T;
  const int tt = t_ok ? t : 0;
  const int img = tt / per_img;
  const int r = tt - img * per_img;
  const int ty = r / tw, tx = r - (r / tw) * tw;
  const int y0 = ty * 4 - pt, x0 = tx * 4 - pl;
  const bool ok = t_ok && c < C;  // padding tiles / channels transform a zero patch
  const int plane = (img * C + (ok ? c : 0)) * H;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(x, x_bytes);  // whole input, < 2^31 bytes
  wino_in_patch<VEC>(rs, ok, plane, H, W, y0, x0, vout, plane_stride);
}

// Thread (k, t): 36 GEMM outputs (the sum of S K-partial buffers) -> 4x4
// output tile, + bias (+ residual), act.
template <int S>
__global__ __launch_bounds__(256) void wino_output_transform(
    const float* __restrict__ M, int64_t split_stride, const float* __restrict__ bias,
    const float* __restrict__ residual, float* __restrict__ out, int K, int OH,
    int OW, int th, int tw, int T, int t_pad, int m_pad, int act) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)K * T) return;
  const int k = (int)(idx / T);
  const int t = (int)(idx - (int64_t)k * T);
  const int64_t plane_stride = (int64_t)m_pad * t_pad;
  const float* min = M + (int64_t)k * t_pad + t;
  float m[6][6];
#pragma unroll
  for (int i = 0; i < 6; ++i)
#pragma unroll
    for (int j = 0; j < 6; ++j) {
      float v = min[(i * 6 + j) * plane_stride];
#pragma unroll
      for (int sp = 1; sp < S; ++sp) v += min[sp * split_stride + (i * 6 + j) * plane_stride];
      m[i][j] = v;
    }
  // tmp = A^T m (4x6)
  float tmp[4][6];
#pragma unroll
  for (int j = 0; j < 6; ++j) {
    const float m0 = m[0][j], m1 = m[1][j], m2 = m[2][j], m3 = m[3][j], m4 = m[4][j], m5 = m[5][j];
    const float s12 = m1 + m2, d12 = m1 - m2, s34 = m3 + m4, d34 = m3 - m4;
    tmp[0][j] = m0 + s12 + s34;
    tmp[1][j] = d12 + 2.f * d34;
    tmp[2][j] = s12 + 4.f * s34;
    tmp[3][j] = d12 + 8.f * d34 + m5;
  }
  const int per_img = th * tw;
  const int img = t / per_img;
  const int r = t - img * per_img;
  const int ty = r / tw, tx = r - (r / tw) * tw;
  const float b = bias[k];
  const int64_t plane = ((int64_t)img * K + k) * OH * OW;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float m0 = tmp[i][0], m1 = tmp[i][1], m2 = tmp[i][2], m3 = tmp[i][3], m4 = tmp[i][4], m5 = tmp[i][5];
    const float s12 = m1 + m2, d12 = m1 - m2, s34 = m3 + m4, d34 = m3 - m4;
    float y[4];
    y[0] = m0 + s12 + s34;
    y[1] = d12 + 2.f * d34;
    y[2] = s12 + 4.f * s34;
    y[3] = d12 + 8.f * d34 + m5;
    const int oy = ty * 4 + i;
    if (oy >= OH) break;
    const int64_t row = plane + (int64_t)oy * OW + tx * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (tx * 4 + j < OW) {
        float v = y[j] + b;
        if (residual) v += residual[row + j];
        if (act == NHIP_ACT_RELU) v = v < 0.f ? 0.f : v;
        else if (act == NHIP_ACT_SIGMOID) v = 1.0f / (1.0f + __expf(-v));
        out[row + j] = v;
      }
    }
  }
}

}  // namespace

// U[xi][k][c] = (G g_kc G^T)[xi], computed in double, stored fp32 with zero
// padding to [36][m_pad][c_pad], and again in 4-channel groups for the fused
// kernel as [36][c_pad/4][m_pad][4].
int winograd_prepack_weights(nhip_conv_plan* p, const float* weight) {
  static const double G[6][3] = {
      {1.0 / 4, 0, 0},
      {-1.0 / 6, -1.0 / 6, -1.0 / 6},
      {-1.0 / 6, 1.0 / 6, -1.0 / 6},
      {1.0 / 24, 1.0 / 12, 1.0 / 6},
      {1.0 / 24, -1.0 / 12, 1.0 / 6},
      {0, 0, 1}};
  const int K = p->g.k, C = p->g.c;
  std::vector<float> U((size_t)36 * p->m_pad * p->c_pad, 0.f);
  for (int k = 0; k < K; ++k)
    for (int c = 0; c < C; ++c) {
      const float* g = weight + ((size_t)k * C + c) * 9;
      double tmp[6][3];
      for (int i = 0; i < 6; ++i)
        for (int j = 0; j < 3; ++j)
          tmp[i][j] = G[i][0] * g[0 * 3 + j] + G[i][1] * g[1 * 3 + j] + G[i][2] * g[2 * 3 + j];
      for (int i = 0; i < 6; ++i)
        for (int j = 0; j < 6; ++j) {
          const double u = tmp[i][0] * G[j][0] + tmp[i][1] * G[j][1] + tmp[i][2] * G[j][2];
          U[((size_t)(i * 6 + j) * p->m_pad + k) * p->c_pad + c] = (float)u;
        }
    }
  std::vector<float> Uf(U.size());
  for (int xi = 0; xi < 36; ++xi)
    for (int k = 0; k < p->m_pad; ++k)
      for (int c = 0; c < p->c_pad; ++c)
        Uf[(((size_t)xi * (p->c_pad / 4) + c / 4) * p->m_pad + k) * 4 + c % 4] =
            U[((size_t)xi * p->m_pad + k) * p->c_pad + c];
  NHIP_TRY(check_hip(hipMalloc(&p->weight_fused, Uf.size() * sizeof(float)), "hipMalloc(winograd U, 4-channel groups)"));
  NHIP_TRY(check_hip(hipMemcpy(p->weight_fused, Uf.data(), Uf.size() * sizeof(float), hipMemcpyHostToDevice),
                     "hipMemcpy(winograd U, 4-channel groups)"));
  NHIP_TRY(check_hip(hipMalloc(&p->weight, U.size() * sizeof(float)), "hipMalloc(winograd U)"));
  return check_hip(hipMemcpy(p->weight, U.data(), U.size() * sizeof(float), hipMemcpyHostToDevice),
                   "hipMemcpy(winograd U)");
}

// Launches of at most 32 tiles on a plan with an implicit-GEMM twin take the
// twin: the Winograd GEMM pads the tiles to 128, and a single image of
// 512@7 (4 tiles) took 46.6 us on it against 23.3 us on the implicit GEMM,
// 256@14 22.8 against 17.0 us at one image (16 tiles) and 23.3 against 21.8
// at two (32 tiles), where from 64 tiles on Winograd wins (23.9 against
// 29.4).  Not when a Winograd variant is forced (NHIP_WINOGRAD_VARIANT);
// NHIP_WINO_TWIN=0 switches the route off.
static bool twin_selected(const nhip_conv_plan* p, int n, int oh, int ow) {
  if (p->igemm_twin == nullptr || variant_requested() != 0 || setting_int("NHIP_WINO_TWIN", 1) == 0) return false;
  return (int64_t)n * ceil_div(oh, 4) * ceil_div(ow, 4) <= 32;
}

uint64_t conv_winograd_f32_workspace(const nhip_conv_plan* p, int n, int oh, int ow) {
  if (twin_selected(p, n, oh, ow)) return conv_igemm_f32_workspace(p->igemm_twin, n, oh, ow);
  const int th = (int)ceil_div(oh, 4), tw = (int)ceil_div(ow, 4);
  const int64_t t_pad = round_up((int64_t)n * th * tw, 128);
  if (fused_selected(p, n, oh, ow) && wino_xt_selected(p, n, oh + 2 - p->g.pt - p->g.pb, ow + 2 - p->g.pl - p->g.pr, oh, ow))
    return 0;  // the input transform inside the GEMM: no V
  if (fused_selected(p, n, oh, ow))  // V, then the GEMM's partial sums
    return (uint64_t)36 * t_pad * p->c_pad * sizeof(float) + wino_gemm_out_parts_bytes(p, n, oh, ow);
  const WinoGemmCfg cfg = wino_gemm_config(p->m_pad, p->c_pad, (int)t_pad);
  return (uint64_t)36 * t_pad * (p->c_pad + (int64_t)cfg.splits * p->m_pad) * sizeof(float);
}

int launch_conv_winograd_f32(const nhip_conv_plan* p, const float* in,
                             const float* residual, float* out, int n, int h,
                             int w, int oh, int ow, void* ws, uint64_t ws_bytes,
                             hipStream_t s) {
  const WinoShape ws_ = wino_shape(p, n, h, w, oh, ow);
  const uint64_t need = conv_winograd_f32_workspace(p, n, oh, ow);
  if (need > 0 && (ws == nullptr || ws_bytes < need))
    return fail(NHIP_STATUS_OUTPUT_CAPACITY_INSUFFICIENT,
                "winograd conv: workspace of " + std::to_string(need) + " bytes required");
  // Launches of at most two 32x32 blocks per CU: the one-kernel implicit
  // GEMM on the plan's row-major weights (unless a Winograd variant is
  // forced with NHIP_WINOGRAD_VARIANT)
  if (variant_requested() == 0 && kq_supported(p, n, h, w, oh, ow))
    return launch_conv_kq(p, in, residual, out, n, h, w, oh, ow, s);
  if (twin_selected(p, n, oh, ow))
    return launch_conv_igemm_f32(p->igemm_twin, in, residual, out, n, h, w, oh, ow, ws, ws_bytes, s);
  const bool fused = fused_selected(p, n, oh, ow);
  if (fused && wino_xt_selected(p, n, h, w, oh, ow))
    return launch_wino_gemm_xt(p, in, residual, out, n, h, w, oh, ow, s);
  float* V = static_cast<float*>(ws);
  float* M = V + (int64_t)36 * ws_.c_pad * ws_.t_pad;
  {
    const uint32_t x_bytes = (uint32_t)((size_t)n * ws_.c * h * w * sizeof(float));
    const int64_t units = (int64_t)ws_.c_pad * ws_.t_pad;
    const dim3 grid((unsigned)ceil_div(units, 256));
    const bool vec = p->g.pl == 1 && w % 4 == 0 && (reinterpret_cast<uintptr_t>(in) & 15) == 0;
#define NHIP_WINO_IN(P_, V_)                                                                                  \
  NHIP_LAUNCH("wino_input_transform", (wino_input_transform<P_, V_>), grid, dim3(256), 0, s, in, x_bytes, V, \
              ws_.c, h, w, ws_.th, ws_.tw, ws_.t, ws_.t_pad, ws_.c_pad, p->g.pt, p->g.pl)
    if (fused && vec) NHIP_WINO_IN(true, true);
    else if (fused) NHIP_WINO_IN(true, false);
    else if (vec) NHIP_WINO_IN(false, true);
    else NHIP_WINO_IN(false, false);
#undef NHIP_WINO_IN
    NHIP_TRY(check_launch("wino_input_transform"));
  }
  if (fused) return launch_wino_gemm_out(p, V, ws_.t_pad, residual, out, n, oh, ow, M, s);
  const WinoGemmCfg cfg = wino_gemm_config(ws_.m_pad, ws_.c_pad, ws_.t_pad);
  NHIP_TRY(launch_wino_gemm(p->weight, V, M, ws_.m_pad, ws_.c_pad, ws_.t_pad, cfg, s));
  {
    const int64_t total = (int64_t)p->g.k * ws_.t;
    const int64_t split_stride = (int64_t)36 * ws_.m_pad * ws_.t_pad;
    const dim3 grid((unsigned)ceil_div(total, 256));
#define NHIP_WINO_OUT(S_)                                                                                    \
  case S_:                                                                                                   \
    NHIP_LAUNCH("wino_output_transform", wino_output_transform<S_>, grid, dim3(256), 0, s, M, split_stride, \
                p->bias, residual, out, p->g.k, oh, ow, ws_.th, ws_.tw, ws_.t, ws_.t_pad, ws_.m_pad, p->g.act); \
    break;
    switch (cfg.splits) {
      NHIP_WINO_OUT(1)
      NHIP_WINO_OUT(2)
      NHIP_WINO_OUT(4)
      default:
        return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "winograd conv: unsupported split count");
    }
#undef NHIP_WINO_OUT
    NHIP_TRY(check_launch("wino_output_transform"));
  }
  return ok();
}

}  // namespace nhip
