// An inverted-residual block's 1x1 expand convolution and the 3x3 depthwise
// convolution that reads it, in one kernel, for small planes (at most 256
// pixels: MobileNetV2's 14x14 and 7x7 blocks).  Same operations as the two
// layers (reference ConvertConvolution, NCNNToTosa.cpp:1316-1529, and
// ConvertDepthwiseConvolution, :3074-3503):
//
//   e[k][p]      = act1(sum_c W1[k][c] x[c][p] + b1[k])
//   y[k][oy][ox] = actd(sum_{kh,kw} e_pad[k][oy*s + kh][ox*s + kw] * wd[k][kh][kw] + bd[k])
//
// with e zero-padded by one pixel (padding 1), stride s = 1 or 2.
//
// A workgroup owns one image and a slice of 64 expanded channels, so the
// whole plane of every channel it expands is its own: the depthwise halo is
// in the workgroup and nothing is computed twice, and the expanded tensor
// never reaches memory (at 14x14, batch 32, 96 -> 576 channels: 14.5 MB
// written and read back by the two separate layers).
//   1. The image's input planes [C][HW], one contiguous block in NCHW, are
//      copied into LDS as they lie (16-byte loads, eight in flight per
//      thread), then 16 x PT zeros past the last plane; the 64 x 9 depthwise
//      weights and biases beside them.  An MFMA column past HW reads the next
//      plane's first pixels (or the zeros), and lands in a pixel that is not
//      stored.
//   2. Eight waves: wave w owns expanded channels 16 (w % 4) .. + 15 of the
//      slice and half of the plane's 16-pixel tiles (w / 4 picks which):
//      v_mfma_f32_16x16x4_f32, A = W1 (the wave's C/4 k-steps preloaded into
//      registers from the plan's row-major weights, 16-byte loads), B = x
//      from LDS.
//      Register r of lane l of tile t is channel 4 (l / 16) + r of the
//      wave's group, pixel 16 t + l % 16.  Two waves per SIMD keep one
//      wave's LDS and memory latency behind the other's work in every
//      phase.
//   3. After a barrier the input's LDS holds the expanded planes instead,
//      each (H + 2) x (W + 2) with a zero border: e + b1, act1.
//   4. Every thread takes column strips of 7 outputs (channel, rows, column)
//      and forms each depthwise sum in the reference's order (zero, += e * w
//      over kh then kw, + bias, activation; separately rounded, no fused
//      multiply-add), sliding the 3 x 3 window down the strip in registers.
// The expand's MFMA summation order differs from the 1x1 kernels', so the
// result matches the two separate layers within rounding, not bit for bit.
#include "nhip_internal.h"

namespace nhip {
namespace {

constexpr int kThreads = 512;
constexpr int kSlice = 64;  // expanded channels per workgroup (4 channel groups x 16)
constexpr int kMaxC = 256;  // input channels: C/4 A registers per lane

struct EdArgs {
  const float* x;   // [N][C][H][W]
  const float* w1;  // [m_pad][ldw1], k = c (1x1)
  const float* w1q; // the same weights as [rows/32][C/4][32][4], or null
  const float* b1;  // [m_pad] (zero past K)
  const float* wd;  // [K][9]
  const float* bd;  // [K]
  float* y;         // [N][K][OH][OW]
  int C, K, H, W, OH, OW, s, ldw1, act1, actd;
  int vec;          // x is 16-byte aligned: the block is copied in float4s
};

constexpr int kInFlight = 8;  // loads per thread issued before their LDS writes

// LDS floats from one expanded plane to the next: (H + 2) (W + 2) rounded up
// to 4 more than a multiple of 16
__host__ __device__ __forceinline__ int plane_stride(int h, int w) { return ((h + 2) * (w + 2) + 15) / 16 * 16 + 4; }

__device__ __forceinline__ float act_of(float v, int act) { return (act == NHIP_ACT_RELU && v < 0.f) ? 0.f : v; }

constexpr int kStrip = 7;  // depthwise outputs per lane task: a column strip of 7 rows

// The depthwise layer over the slice's padded planes (es: channel c at
// c * PS, rows of PW floats, zero border).  A task is (channel, strip of
// kStrip output rows, output column); consecutive threads take consecutive
// columns, so each output row of a strip is one coalesced run.  The 3 x 3
// window slides down the strip in registers: S new rows of 3 values per
// output instead of 9.  Every output is the reference's sum: zero, += e * w
// over (kh, kw) in order, + bias, activation, each step separately rounded.
// Rows past OH (the last strip's) are formed from clamped rows and not stored.
template <int S>
__device__ __forceinline__ void depthwise_strips(const float* es, const float* wds, const float* bds, float* yo,
                                                 int nch, int H, int PW, int PS, int OH, int OW, int actd, int tid) {
  const int nrb = (OH + kStrip - 1) / kStrip;
  const int T = nrb * OW;  // tasks per channel
  // e / T and r / OW as (x + 1/2) / d in fp32: exact, the quotients are below
  // 256 and at least 1/(2d) >= 1/512 from an integer
  const float inv_t = 1.f / (float)T, inv_ow = 1.f / (float)OW;
  const int OHW = OH * OW;
  for (int e = tid; e < nch * T; e += kThreads) {
    // (24-bit multiplies: every product here is below 2^23)
    const int c = (int)(((float)e + 0.5f) * inv_t);
    const int rem = e - __mul24(c, T);
    const int rb = (int)(((float)rem + 0.5f) * inv_ow);
    const int ox = rem - __mul24(rb, OW);
    const float* ec = es + __mul24(c, PS) + ox * S;
    float w[9];
#pragma unroll
    for (int t = 0; t < 9; ++t) w[t] = wds[__mul24(c, 9) + t];
    const float bias = bds[c];
    const int oy0 = rb * kStrip;
    float* yc = yo + __mul24(c, OHW) + ox;
    auto row = [&](int r, float* v) {
      const float* q = ec + __mul24(min(r, H + 1), PW);
      v[0] = q[0];
      v[1] = q[1];
      v[2] = q[2];
    };
    float r0[3], r1[3], r2[3];
    int iy = oy0 * S;
    row(iy, r0);
    row(iy + 1, r1);
#pragma unroll
    for (int i = 0; i < kStrip; ++i) {
      row(iy + 2, r2);
      float sum = 0.f;
#pragma unroll
      for (int kw = 0; kw < 3; ++kw) sum = __fadd_rn(sum, __fmul_rn(r0[kw], w[kw]));
#pragma unroll
      for (int kw = 0; kw < 3; ++kw) sum = __fadd_rn(sum, __fmul_rn(r1[kw], w[3 + kw]));
#pragma unroll
      for (int kw = 0; kw < 3; ++kw) sum = __fadd_rn(sum, __fmul_rn(r2[kw], w[6 + kw]));
      sum = __fadd_rn(sum, bias);
      if (oy0 + i < OH) yc[__mul24(oy0 + i, OW)] = act_of(sum, actd);
#pragma unroll
      for (int kw = 0; kw < 3; ++kw) {
        if (S == 1) {
          r0[kw] = r1[kw];
          r1[kw] = r2[kw];
        } else {
          r0[kw] = r2[kw];
        }
      }
      if (S == 2) row(iy + 3, r1);
      iy += S;
    }
  }
}

// PT = 16-pixel tiles of a plane (ceil(H*W / 16)); NK = C / 4 k-steps.
template <int PT, int NK>
__global__ __launch_bounds__(kThreads) void expand_dw_kernel(EdArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int k0 = blockIdx.x * kSlice, img = blockIdx.y;
  const int HW = a.H * a.W, OHW = a.OH * a.OW;
  const int PW = a.W + 2;  // padded expanded plane: (H + 2) x PW
  const int PS = plane_stride(a.H, a.W);
  // LDS: [input planes, later expanded planes][64 x 9 depthwise weights][64 biases]
  const int tot = NK * 4 * HW;  // floats of the image's input block
  const int region = max(tot + 16 * PT, kSlice * PS);
  float* xs = lds;
  float* wds = lds + region;
  float* bds = wds + kSlice * 9;
  const int grp = wave & 3, half = wave >> 2;
  const int chw = 16 * grp + 4 * (lane >> 4);  // slice channel of MFMA register 0

  // ---- 1. every global read of the phase is issued before the first LDS
  // write waits for one: the A operand, the 1x1 bias, the depthwise
  // parameters, then the input block.
  // k-step j of lane group g = l / 16 reduces input channel
  // 16 (j / 4) + 4 g + j % 4, so the A operand of steps 4q .. 4q + 3 is one
  // float4, W1[k0 + 16 grp + l%16][16 q + 4 g ..+ 3], and four lanes read 64
  // contiguous bytes of a weight row (rows are 16-float aligned; rows past K
  // are the plan's zero padding up to m_pad)
  // (grouped layout: lane group g's float4 of step q is group 4q + g of the
  // row's 32-row block, so 16 lanes read 256 contiguous bytes)
  float av[NK];
  {
    const int row = k0 + 16 * grp + (lane & 15);
    const float4* wr;
    int step;  // float4s from group q to group q + 1 of the lane
    if (a.w1q) {
      wr = reinterpret_cast<const float4*>(a.w1q) + ((int64_t)(row >> 5) * NK + (lane >> 4)) * 32 + (row & 31);
      step = 4 * 32;
    } else {
      wr = reinterpret_cast<const float4*>(a.w1 + (int64_t)row * a.ldw1) + (lane >> 4);
      step = 4;
    }
#pragma unroll
    for (int q = 0; q < NK / 4; ++q) {
      const float4 v = wr[q * step];
      av[4 * q] = v.x;
      av[4 * q + 1] = v.y;
      av[4 * q + 2] = v.z;
      av[4 * q + 3] = v.w;
    }
  }
  float bv[4];  // the 1x1 layer's bias for the lane's 4 channels
#pragma unroll
  for (int r = 0; r < 4; ++r) bv[r] = a.b1[k0 + chw + r];
  static_assert(kSlice * 9 <= 2 * kThreads && kSlice <= kThreads, "depthwise parameters: two per thread");
  const int nch = min(kSlice, a.K - k0);
  const int e1 = tid + kThreads;
  const float wd0 = tid < nch * 9 ? a.wd[(int64_t)k0 * 9 + tid] : 0.f;
  const float wd1 = e1 < nch * 9 ? a.wd[(int64_t)k0 * 9 + e1] : 0.f;
  const float bd0 = tid < nch ? a.bd[k0 + tid] : 0.f;
  const float* xi = a.x + (int64_t)img * a.C * HW;
  if (a.vec) {
    // C is a multiple of 4, so the block is whole float4s
    const float4* src = reinterpret_cast<const float4*>(xi);
    const int n4 = tot >> 2;
    for (int base = tid; base < n4; base += kThreads * kInFlight) {
      float4 v[kInFlight];
      // every load issued (index clamped to the block), only in-range ones stored
#pragma unroll
      for (int i = 0; i < kInFlight; ++i) v[i] = src[min(base + i * kThreads, n4 - 1)];
#pragma unroll
      for (int i = 0; i < kInFlight; ++i)
        if (base + i * kThreads < n4) reinterpret_cast<float4*>(xs)[base + i * kThreads] = v[i];
    }
  } else {
    for (int base = tid; base < tot; base += kThreads * kInFlight) {
      float v[kInFlight];
#pragma unroll
      for (int i = 0; i < kInFlight; ++i) v[i] = xi[min(base + i * kThreads, tot - 1)];
#pragma unroll
      for (int i = 0; i < kInFlight; ++i)
        if (base + i * kThreads < tot) xs[base + i * kThreads] = v[i];
    }
  }
  if (tid < 16 * PT) xs[tot + tid] = 0.f;
  wds[tid] = wd0;
  if (e1 < kSlice * 9) wds[e1] = wd1;
  if (tid < kSlice) bds[tid] = bd0;
  // tiles of a half: half * TH .. half * TH + TH - 1; for odd PT the last one
  // is past the plane (its reads stay in the LDS allocation, its pixels are
  // not stored)
  constexpr int TH = (PT + 1) / 2;
  __syncthreads();

  // ---- 2. expand: the wave's 16 channels x its half of the pixel tiles
  v4f acc[TH];
#pragma unroll
  for (int t = 0; t < TH; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  const int t0 = half * TH;
  const float* xb = xs + 4 * (lane >> 4) * HW + (lane & 15) + 16 * t0;
  // step j + 1's B values are read while step j's MFMAs run
  float bv_cur[TH], bv_next[TH];
#pragma unroll
  for (int t = 0; t < TH; ++t) bv_cur[t] = xb[16 * t];
#pragma unroll  // whole: av[j] stays in registers
  for (int j = 0; j < NK; ++j) {
    if (j + 1 < NK) {
      const float* xr = xb + (16 * ((j + 1) >> 2) + ((j + 1) & 3)) * HW;
#pragma unroll
      for (int t = 0; t < TH; ++t) bv_next[t] = xr[16 * t];
    }
#pragma unroll
    for (int t = 0; t < TH; ++t) acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j], bv_cur[t], acc[t], 0, 0, 0);
    // scheduling order: the next step's LDS reads, then this step's MFMAs
    // (left alone, the compiler reads each value right before its MFMA and
    // waits for it there)
    __builtin_amdgcn_sched_group_barrier(0x100, TH, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, TH, 0);
#pragma unroll
    for (int t = 0; t < TH; ++t) bv_cur[t] = bv_next[t];
  }
  __syncthreads();  // every wave done with the input planes

  // ---- 3. expanded planes, PS floats apart (the four register rows of an
  // MFMA result, 4 planes apart, fall on different LDS banks): zeros first,
  // then the interiors, bias + act1.  Planes past K come out zero (zero
  // weight rows and bias) and are never read.
  float* es = xs;
  for (int e = tid; e < kSlice * PS / 4; e += kThreads) reinterpret_cast<float4*>(es)[e] = float4{0.f, 0.f, 0.f, 0.f};
  __syncthreads();
  {
    // p / W as (p + 1/2) / W in fp32, exact for p < 256: the quotient is at
    // least 1/(2W) >= 1/512 from an integer, the rounding error below 2^-15
    const float inv_w = 1.f / (float)a.W;
    const bool relu = a.act1 == NHIP_ACT_RELU;
    float* eb = es + __mul24(chw, PS) + PW + 1;  // interior origin of the lane's first plane
#pragma unroll
    for (int t = 0; t < TH; ++t) {
      const int p = 16 * (t0 + t) + (lane & 15);
      if (p < HW) {
        const int py = (int)(((float)p + 0.5f) * inv_w), px = p - __mul24(py, a.W);
        float* ep = eb + __mul24(py, PW) + px;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // the 1x1 layer's epilogue: sum + bias, then the activation
          const float v = __fadd_rn(acc[t][r], bv[r]);
          ep[r * PS] = (relu && v < 0.f) ? 0.f : v;
        }
      }
    }
  }
  __syncthreads();

  // ---- 4. depthwise 3x3 in the reference's order, in column strips
  float* yo = a.y + ((int64_t)img * a.K + k0) * OHW;
  if (a.s == 1)
    depthwise_strips<1>(es, wds, bds, yo, nch, a.H, PW, PS, a.OH, a.OW, a.actd, tid);
  else
    depthwise_strips<2>(es, wds, bds, yo, nch, a.H, PW, PS, a.OH, a.OW, a.actd, tid);
}

int lds_bytes(int C, int PT, int H, int W) {
  const int region = std::max(C * H * W + 16 * PT, kSlice * plane_stride(H, W));
  return (region + kSlice * 9 + kSlice) * (int)sizeof(float);
}

template <int PT, int NK>
int launch_one(const EdArgs& a, int n, hipStream_t s) {
  const int lds = lds_bytes(a.C, PT, a.H, a.W);
  NHIP_TRY(ensure_dynamic_lds(reinterpret_cast<const void*>(&expand_dw_kernel<PT, NK>), lds));
  NHIP_LAUNCH("expand_dw_f32", (expand_dw_kernel<PT, NK>), dim3((unsigned)ceil_div(a.K, kSlice), (unsigned)n),
              dim3(kThreads), lds, s, a);
  return check_launch("expand_dw_f32");
}

template <int PT>
int launch_pt(const EdArgs& a, int n, hipStream_t s) {
  switch (a.C / 4) {
    case 8: return launch_one<PT, 8>(a, n, s);
    case 16: return launch_one<PT, 16>(a, n, s);
    case 24: return launch_one<PT, 24>(a, n, s);
    case 40: return launch_one<PT, 40>(a, n, s);
    default: return fail(NHIP_STATUS_UNSUPPORTED, "expand + depthwise: input channels outside the kernel's range");
  }
}

}  // namespace

// Whether the fused kernel takes the pair: an fp32 1x1 stride-1 unpadded
// convolution on the implicit-GEMM plan (32, 64, 96 or 160 input channels;
// the 1x1 layers of MobileNetV2's 14x14 and 7x7 blocks) feeding a 3x3
// depthwise convolution (stride 1 or 2, padding 1, dilation 1) over its
// channels, activations none or ReLU, planes of at most 256 pixels.
// NHIP_PWDW=0 never; by default planes of at most 196 pixels (14x14), the
// shapes measured.
bool pwdw_supported(const nhip_conv_plan* pw, const nhip_conv_plan* dw, int n, int h, int w) {
  if (!pw || !dw || pw->kind != PlanKind::ConvF32 || dw->kind != PlanKind::DwConvF32) return false;
  const int mode = setting_int("NHIP_PWDW", 1);
  if (mode == 0) return false;
  const ConvGeom& p = pw->g;
  const ConvGeom& d = dw->g;
  if (pw->algorithm != NHIP_CONV_ALGO_IMPLICIT_GEMM || p.kh != 1 || p.kw != 1 || p.sh != 1 || p.sw != 1 || p.pt ||
      p.pb || p.pl || p.pr || pw->kred != p.c)
    return false;
  if (!(p.c == 32 || p.c == 64 || p.c == 96 || p.c == 160) || p.c > kMaxC || pw->kred_pad % 4) return false;
  if (d.c != p.k || d.k != p.k || d.kh != 3 || d.kw != 3 || d.dh != 1 || d.dw != 1 || d.sh != d.sw ||
      (d.sh != 1 && d.sh != 2) || d.pt != 1 || d.pb != 1 || d.pl != 1 || d.pr != 1)
    return false;
  if ((p.act != NHIP_ACT_NONE && p.act != NHIP_ACT_RELU) || (d.act != NHIP_ACT_NONE && d.act != NHIP_ACT_RELU))
    return false;
  if (h * w > (mode == 2 ? 256 : 196)) return false;
  int pt = (int)ceil_div(h * w, 16);
  for (int c : {2, 4, 8, 13, 16})
    if (pt <= c) {
      pt = c;
      break;
    }
  if (lds_bytes(p.c, pt, h, w) > 160 * 1024) return false;
  const int oh = (h - 1) / d.sh + 1, ow = (w - 1) / d.sw + 1;
  return (int64_t)n * p.c * h * w < INT32_MAX && (int64_t)n * p.k * oh * ow < INT32_MAX && n <= 65535;
}

int launch_pwdw_f32(const nhip_conv_plan* pw, const nhip_conv_plan* dw, const float* in, float* out, int n, int h,
                    int w, hipStream_t s) {
  if (!pwdw_supported(pw, dw, n, h, w))
    return fail(NHIP_STATUS_UNSUPPORTED, "expand + depthwise: this pair or shape has no fused kernel");
  if (n == 0) return ok();
  EdArgs a{};
  a.x = in;
  a.w1 = pw->weight;
  // the grouped copy when its rows (K rounded up to 32) cover every 64-row slice
  a.w1q = pw->weight_kq != nullptr && pw->kq_vw == 4 && round_up(pw->g.k, 32) == round_up(pw->g.k, 64)
              ? pw->weight_kq
              : nullptr;
  a.b1 = pw->bias;
  a.wd = dw->weight;
  a.bd = dw->bias;
  a.y = out;
  a.C = pw->g.c;
  a.K = pw->g.k;
  a.H = h;
  a.W = w;
  a.s = dw->g.sh;
  a.OH = (h - 1) / a.s + 1;
  a.OW = (w - 1) / a.s + 1;
  a.ldw1 = pw->kred_pad;
  a.act1 = pw->g.act;
  a.actd = dw->g.act;
  // 16-pixel tiles, rounded up to an instantiated count (the tiles past the
  // plane hold zero pixels)
  int pt = (int)ceil_div(h * w, 16);
  for (int c : {2, 4, 8, 13, 16})
    if (pt <= c) {
      pt = c;
      break;
    }
  a.vec = (reinterpret_cast<uintptr_t>(in) & 15) == 0;
  switch (pt) {
    case 2: return launch_pt<2>(a, n, s);
    case 4: return launch_pt<4>(a, n, s);
    case 8: return launch_pt<8>(a, n, s);
    case 13: return launch_pt<13>(a, n, s);
    case 16: return launch_pt<16>(a, n, s);
    default: return fail(NHIP_STATUS_UNSUPPORTED, "expand + depthwise: plane size outside the kernel's range");
  }
}

}  // namespace nhip
