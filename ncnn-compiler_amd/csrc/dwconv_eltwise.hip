// Bandwidth-bound kernels of the hot path:
//   - fp32 ConvolutionDepthWise (NCNNToTosa.cpp:3376-3503): zero-init
//     depthwise sum over (kh, kw), then the bias add, then the importer's
//     separate relu (ImportOps.cpp:1004-1010);
//   - relu, add, global average pooling, quantize / requantize / dequantize.
//
// This file is compiled with -ffp-contract=off: the quantize family must
// round every fp32 step separately to match the reference bit for bit.
#include <algorithm>

#include "lds_dma.h"
#include "nhip_internal.h"

namespace nhip {
namespace {

// ---------------------------------------------------------------------------
// Depthwise.  A workgroup owns `ppb` planes (image x channel) and a band of
// `ob` output rows of each.  The input rows the band needs are staged in LDS
// once (coalesced along x, zero halo), every output then reads its
// kh x kw window from LDS.  HBM traffic is one read of the input and one
// write of the output.
struct DwArgs {
  const float* x;
  float* y;
  const float* w;     // [C][kh*kw]
  const float* bias;  // [C] (zeros when absent)
  int C, H, W, OH, OW;
  int kh, kw, sh, sw, dh, dw, pt, pl;
  int planes;         // n*C
  int ppb, ob, bands; // planes per block, output rows per band, bands per plane
  int ir, lw;         // LDS rows / row width per plane
  int act;
};

__global__ __launch_bounds__(256) void dwconv_f32_kernel(DwArgs a) {
  extern __shared__ float lds[];
  const int band = blockIdx.x % a.bands;
  const int pgrp = blockIdx.x / a.bands;
  const int plane0 = pgrp * a.ppb;
  const int oy0 = band * a.ob;
  const int iy0 = oy0 * a.sh - a.pt;
  const int ix0 = -a.pl;
  const int per_plane = a.ir * a.lw;
  const int total_in = a.ppb * per_plane;
  for (int e = threadIdx.x; e < total_in; e += blockDim.x) {
    const int pi = e / per_plane;
    const int r = e - pi * per_plane;
    const int ry = r / a.lw, rx = r - (r / a.lw) * a.lw;
    const int plane = plane0 + pi;
    const int y = iy0 + ry, x = ix0 + rx;
    float v = 0.f;
    if (plane < a.planes && (unsigned)y < (unsigned)a.H && (unsigned)x < (unsigned)a.W)
      v = a.x[(int64_t)plane * a.H * a.W + (int64_t)y * a.W + x];
    lds[e] = v;
  }
  __syncthreads();
  const int rows = min(a.ob, a.OH - oy0);
  const int per_out = rows * a.OW;
  const int total_out = a.ppb * per_out;
  for (int e = threadIdx.x; e < total_out; e += blockDim.x) {
    const int pi = e / per_out;
    const int r = e - pi * per_out;
    const int oy = r / a.OW, ox = r - (r / a.OW) * a.OW;
    const int plane = plane0 + pi;
    if (plane >= a.planes) break;
    const int c = plane % a.C;
    const float* wc = a.w + (int64_t)c * a.kh * a.kw;
    const float* src = lds + pi * per_plane + (oy * a.sh) * a.lw + ox * a.sw;
    float acc = 0.f;
    for (int i = 0; i < a.kh; ++i)
      for (int j = 0; j < a.kw; ++j)
        acc += src[i * a.dh * a.lw + j * a.dw] * wc[i * a.kw + j];
    acc = acc + a.bias[c];
    if (a.act == NHIP_ACT_RELU) acc = acc < 0.f ? 0.f : acc;
    a.y[(int64_t)plane * a.OH * a.OW + (int64_t)(oy0 + oy) * a.OW + ox] = acc;
  }
}

// Same 3x3 stride-1 case with the window unrolled and each thread producing
// four consecutive outputs of a row (one 3x6 LDS window).
__global__ __launch_bounds__(256) void dwconv3x3s1_f32_kernel(DwArgs a) {
  extern __shared__ float lds[];
  const int band = blockIdx.x % a.bands;
  const int pgrp = blockIdx.x / a.bands;
  const int plane0 = pgrp * a.ppb;
  const int oy0 = band * a.ob;
  const int iy0 = oy0 - a.pt;
  const int ix0 = -a.pl;
  const int per_plane = a.ir * a.lw;
  const int total_in = a.ppb * per_plane;
  for (int e = threadIdx.x; e < total_in; e += blockDim.x) {
    const int pi = e / per_plane;
    const int r = e - pi * per_plane;
    const int ry = r / a.lw, rx = r - (r / a.lw) * a.lw;
    const int plane = plane0 + pi;
    const int y = iy0 + ry, x = ix0 + rx;
    float v = 0.f;
    if (plane < a.planes && (unsigned)y < (unsigned)a.H && (unsigned)x < (unsigned)a.W)
      v = a.x[(int64_t)plane * a.H * a.W + (int64_t)y * a.W + x];
    lds[e] = v;
  }
  __syncthreads();
  const int rows = min(a.ob, a.OH - oy0);
  const int quads = (a.OW + 3) / 4;
  const int per_out = rows * quads;
  const int total_out = a.ppb * per_out;
  for (int e = threadIdx.x; e < total_out; e += blockDim.x) {
    const int pi = e / per_out;
    const int r = e - pi * per_out;
    const int oy = r / quads, ox = (r - (r / quads) * quads) * 4;
    const int plane = plane0 + pi;
    if (plane >= a.planes) break;
    const int c = plane % a.C;
    const float* wc = a.w + (int64_t)c * 9;
    float wr[9];
#pragma unroll
    for (int t = 0; t < 9; ++t) wr[t] = wc[t];
    const float* src = lds + pi * per_plane + oy * a.lw + ox;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      float row[6];
#pragma unroll
      for (int t = 0; t < 6; ++t) row[t] = (ox + t < a.lw) ? src[i * a.lw + t] : 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int j = 0; j < 3; ++j) acc[q] += row[q + j] * wr[i * 3 + j];
    }
    const float b = a.bias[c];
    float* dst = a.y + (int64_t)plane * a.OH * a.OW + (int64_t)(oy0 + oy) * a.OW + ox;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (ox + q < a.OW) {
        float v = acc[q] + b;
        if (a.act == NHIP_ACT_RELU) v = v < 0.f ? 0.f : v;
        dst[q] = v;
      }
    }
  }
}

// 3x3 depthwise, stride S (1 or 2), dilation 1, straight from global memory:
// thread = 4 consecutive outputs of R rows of one plane.  Its input window
// ((R-1)*S+3 rows x 3S+3 columns) comes in through raw buffer loads, the zero
// halo through out-of-range offsets (no load waits on a branch); the overlap
// between neighbouring windows is served by the caches.  VEC (W and OW
// multiples of 4): each window row is one or two aligned 16-byte loads plus
// halo words and the four outputs leave as one 16-byte store.  Summation
// order of the CPU loop nest: acc = 0, += x*w over (kh, kw), then + bias.
template <int S, int R, bool VEC>
__global__ __launch_bounds__(256) void dw3x3_f32_kernel(DwArgs a, uint32_t x_bytes) {
  constexpr int IR = (R - 1) * S + 3;  // input rows per thread
  constexpr int IC = 3 * S + 3;        // input columns for 4 outputs
  const int quads = (a.OW + 3) >> 2;
  const int rblocks = (a.OH + R - 1) / R;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int q = (int)(idx % quads);
  const int64_t t2 = idx / quads;
  const int rb = (int)(t2 % rblocks);
  const int plane = (int)(t2 / rblocks);
  if (plane >= a.planes) return;
  const int c = plane % a.C;
  float w[9];
#pragma unroll
  for (int t = 0; t < 9; ++t) w[t] = a.w[c * 9 + t];
  const float b = a.bias[c];
  const int ox0 = q * 4, oy0 = rb * R;
  const int x0 = ox0 * S - a.pl, y0 = oy0 * S - a.pt;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.x, x_bytes);
  const int base = plane * a.H * a.W;  // < 2^31 elements (checked on the host)
  float in[IR][IC];
#pragma unroll
  for (int i = 0; i < IR; ++i) {
    const int y = y0 + i;
    const bool yok = (unsigned)y < (unsigned)a.H;
    if constexpr (VEC) {
      // columns x0 .. x0+IC-1 = (4qS - 1) .. : word x0, then aligned vectors from x0+1
      const int row = base + y * a.W;
      const bool lok = yok && x0 >= 0;
      in[i][0] = buf_load_f32(rs, lok ? (uint32_t)((row + x0) * 4) : kBufOOB);
#pragma unroll
      for (int v = 0; v < S; ++v) {
        const v4f t = __builtin_bit_cast(v4f, buf_load_b128(rs, yok ? (uint32_t)((row + x0 + 1 + 4 * v) * 4) : kBufOOB));
        in[i][1 + 4 * v] = t.x;
        in[i][2 + 4 * v] = t.y;
        in[i][3 + 4 * v] = t.z;
        in[i][4 + 4 * v] = t.w;
      }
      if constexpr (S == 1) {
        const bool rok = yok && x0 + 5 < a.W;
        in[i][5] = buf_load_f32(rs, rok ? (uint32_t)((row + x0 + 5) * 4) : kBufOOB);
      }
    } else {
#pragma unroll
      for (int j = 0; j < IC; ++j) {
        const int x = x0 + j;
        const bool ok = yok && (unsigned)x < (unsigned)a.W;
        in[i][j] = buf_load_f32(rs, ok ? (uint32_t)((base + y * a.W + x) * (int)sizeof(float)) : kBufOOB);
      }
    }
  }
  float* yp = a.y + (int64_t)plane * a.OH * a.OW;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int oy = oy0 + r;
    if (oy >= a.OH) break;
    float o[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) acc = acc + in[r * S + i][u * S + j] * w[i * 3 + j];
      acc = acc + b;
      if (a.act == NHIP_ACT_RELU) acc = acc < 0.f ? 0.f : acc;
      o[u] = acc;
    }
    if constexpr (VEC) {
      *reinterpret_cast<v4f*>(yp + oy * a.OW + ox0) = v4f{o[0], o[1], o[2], o[3]};
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (ox0 + u < a.OW) yp[oy * a.OW + ox0 + u] = o[u];
    }
  }
}

// 3x3 depthwise, stride S (1 or 2), dilation 1, any padding, for planes of
// at most kDwPlaneMax pixels, streamed: the (image, channel) planes are cut
// into chunks of `ppb` whole planes, in NCHW one contiguous block of the
// input and one of the output each.  A persistent workgroup walks the
// chunks blockIdx.x, + gridDim.x, ...; while it computes chunk k, chunk
// k + 1 is on its way into the other of two LDS slots through direct-to-LDS
// copies (1 KB per wave copy, no registers), so the HBM reads of one chunk
// overlap the arithmetic and the stores of the previous one.  Stride 1: a
// lane takes one output row (at most kDwRowMax outputs), its three input
// rows go from LDS into registers in one go (the zero halo decided once per
// column) and the row's outputs are formed from registers.  Stride 2: lanes
// take consecutive outputs (consecutive LDS words), each read from LDS.
// (Measured at batch 32: row lanes 8.2 against 11.1 us at 384@14, 11.0
// against 14.6 at 576@14; output lanes 7.7 against 13.0 at 576@14 stride 2,
// 9.5 against 15.2 at 192@28 stride 2.)  The results are staged in LDS and
// leave as 16-byte stores.  The host picks ppb so that every output block
// starts on a 16-byte boundary.  Summation order of the CPU loop nest:
// acc = 0, += x*w over (kh, kw), then + bias.
constexpr int kDwPlaneMax = 1024;
constexpr int kDwRowMax = 16;

struct DwStream {
  uint32_t x_bytes;
  int chunks;      // ceil(planes / ppb)
  int slot;        // floats per input slot (whole 4 KB: 4 waves x 1 KB copies)
  int copies;      // 1 KB copies per wave and chunk
  FastDiv oh_div, ohw_div, ow_div;
};

template <int S>
__global__ __launch_bounds__(256) void dw3x3_stream_kernel(DwArgs a, DwStream st) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int hw = a.H * a.W, ohw = a.OH * a.OW;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  float* yout = lds + 2 * st.slot;  // [ppb][ohw]
  float* wl = yout + a.ppb * ohw;   // [ppb][10]: the plane's 9 weights, then its bias
  const uint32_t lds0 = (uint32_t)(uintptr_t)lds;
  const v4i rs = dma::raw_rsrc(a.x, st.x_bytes);
  // chunk c into slot: wave w copies bytes [1 KB (w + 4 i), + 1 KB) of the chunk
  auto issue = [&](int c, int slot) {
    const uint32_t src = (uint32_t)((int64_t)c * a.ppb * hw * 4);
    const uint32_t end = (uint32_t)min((int64_t)(c + 1) * a.ppb * hw * 4, (int64_t)st.x_bytes);
    for (int i = 0; i < st.copies; ++i) {
      const uint32_t off = (uint32_t)((wave + 4 * i) * 1024 + lane * 16);
      dma::copy16(lds0 + (uint32_t)(slot * st.slot * 4) + (uint32_t)((wave + 4 * i) * 1024),
                  src + off < end ? src + off : kBufOOB, rs, 0);
    }
  };
  // the chunk's per-plane weights and bias (ppb * 10 <= 4 * 256 values),
  // requested together with its copy and written to LDS after the wait
  float wv[4];
  auto fetch_w = [&](int c) {
    const int p0 = c * a.ppb, np = min(a.ppb, a.planes - p0);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int e = tid + 256 * u;
      const int pi = e / 10, t = e - pi * 10;
      const int ch = (p0 + min(pi, np - 1)) % a.C;
      wv[u] = e < np * 10 ? (t < 9 ? a.w[ch * 9 + t] : a.bias[ch]) : 0.f;
    }
  };
  int k = 0;
  if ((int)blockIdx.x < st.chunks) {
    issue(blockIdx.x, 0);
    fetch_w(blockIdx.x);
  }
  for (int c = blockIdx.x; c < st.chunks; c += gridDim.x, ++k) {
    const int p0 = c * a.ppb, np = min(a.ppb, a.planes - p0);
    dma::wait_vmcnt<0>();  // chunk c and its weights have landed (and earlier stores are done)
    __syncthreads();       // ... for every wave; slot (k + 1) % 2 and the staging are free
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (tid + 256 * u < np * 10) wl[tid + 256 * u] = wv[u];
    if (c + (int)gridDim.x < st.chunks) {
      issue(c + gridDim.x, (k + 1) & 1);
      fetch_w(c + gridDim.x);
    }
    __syncthreads();
    const float* xin = lds + (k & 1) * st.slot;
    const int nout = np * ohw, rows = np * a.OH;
    if constexpr (S == 2) {
      for (int o = tid; o < nout; o += 256) {
        const int pi = fdiv(o, st.ohw_div);
        const int r = o - pi * ohw;
        const int oy = fdiv(r, st.ow_div);
        const int ox = r - oy * a.OW;
        const float* src = xin + pi * hw;
        const float* wp = wl + pi * 10;
        const int y0 = oy * S - a.pt, x0 = ox * S - a.pl;
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
#pragma unroll
          for (int j = 0; j < 3; ++j) {
            const int y = y0 + i, x = x0 + j;
            const bool ok = (unsigned)y < (unsigned)a.H && (unsigned)x < (unsigned)a.W;
            const float v = ok ? src[ok ? y * a.W + x : 0] : 0.f;
            acc = acc + v * wp[i * 3 + j];
          }
        }
        acc = acc + wp[9];
        if (a.act == NHIP_ACT_RELU) acc = acc < 0.f ? 0.f : acc;
        yout[o] = acc;
      }
    }
    constexpr int IC = (kDwRowMax - 1) * S + 3;  // input columns of a row of outputs
    for (int rr = tid; rr < rows && S == 1; rr += 256) {
      const int pi = fdiv(rr, st.oh_div), oy = rr - pi * a.OH;
      const float* src = xin + pi * hw;
      const float* wp = wl + pi * 10;
      float win[3][IC];
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        const int y = oy * S - a.pt + i;
        const bool yok = (unsigned)y < (unsigned)a.H;
#pragma unroll
        for (int c = 0; c < IC; ++c) {
          const int x = c - a.pl;
          const bool ok = yok && (unsigned)x < (unsigned)a.W && c < (a.OW - 1) * S + 3;
          win[i][c] = ok ? src[ok ? y * a.W + x : 0] : 0.f;
        }
      }
      float wr[10];
#pragma unroll
      for (int t = 0; t < 10; ++t) wr[t] = wp[t];
      float* dst = yout + rr * a.OW;
#pragma unroll
      for (int ox = 0; ox < kDwRowMax; ++ox) {
        if (ox < a.OW) {
          float acc = 0.f;
#pragma unroll
          for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = 0; j < 3; ++j) acc = acc + win[i][ox * S + j] * wr[i * 3 + j];
          acc = acc + wr[9];
          if (a.act == NHIP_ACT_RELU) acc = acc < 0.f ? 0.f : acc;
          dst[ox] = acc;
        }
      }
    }
    __syncthreads();
    float* ys = a.y + (int64_t)p0 * ohw;
    const int nout4 = nout >> 2;
    for (int v = tid; v < nout4; v += 256)
      reinterpret_cast<v4f*>(ys)[v] = reinterpret_cast<const v4f*>(yout)[v];
    for (int e = (nout4 << 2) + tid; e < nout; e += 256) ys[e] = yout[e];
  }
}

// ---------------------------------------------------------------------------

// int8 ConvolutionDepthWise (NCNNToTosa.cpp:3257-3376): the input band is
// quantized (fp32 input) or copied (int8 input) into LDS as int8, the window
// sum is exact int32, and the epilogue is the int8 convolution's:
// (float)acc * r[c], + bias[c], requantize when term > 100, relu last.
struct DwI8Args {
  const void* x;
  void* y;
  const int8_t* w;      // [C][kh*kw]
  const float* bias;    // [C]
  const float* recip;   // [C]: ws==0 ? 0 : 1/(ws*is)
  float is, os;
  int term, act, in_i8;
  int C, H, W, OH, OW;
  int kh, kw, sh, sw, dh, dw, pt, pl;
  int planes, ppb, ob, bands, ir, lw;
};

__global__ __launch_bounds__(256) void dwconv_int8_kernel(DwI8Args a) {
  extern __shared__ int8_t lds8[];
  const int band = blockIdx.x % a.bands;
  const int pgrp = blockIdx.x / a.bands;
  const int plane0 = pgrp * a.ppb;
  const int oy0 = band * a.ob;
  const int iy0 = oy0 * a.sh - a.pt;
  const int ix0 = -a.pl;
  const int per_plane = a.ir * a.lw;
  const int total_in = a.ppb * per_plane;
  for (int e = threadIdx.x; e < total_in; e += blockDim.x) {
    const int pi = e / per_plane;
    const int r = e - pi * per_plane;
    const int ry = r / a.lw, rx = r - (r / a.lw) * a.lw;
    const int plane = plane0 + pi;
    const int y = iy0 + ry, x = ix0 + rx;
    int8_t v = 0;
    if (plane < a.planes && (unsigned)y < (unsigned)a.H && (unsigned)x < (unsigned)a.W) {
      const int64_t off = (int64_t)plane * a.H * a.W + (int64_t)y * a.W + x;
      v = a.in_i8 ? static_cast<const int8_t*>(a.x)[off] : quantize_i8(static_cast<const float*>(a.x)[off], a.is);
    }
    lds8[e] = v;
  }
  __syncthreads();
  const int rows = min(a.ob, a.OH - oy0);
  const int per_out = rows * a.OW;
  const int total_out = a.ppb * per_out;
  for (int e = threadIdx.x; e < total_out; e += blockDim.x) {
    const int pi = e / per_out;
    const int r = e - pi * per_out;
    const int oy = r / a.OW, ox = r - (r / a.OW) * a.OW;
    const int plane = plane0 + pi;
    if (plane >= a.planes) break;
    const int c = plane % a.C;
    const int8_t* wc = a.w + (int64_t)c * a.kh * a.kw;
    const int8_t* src = lds8 + pi * per_plane + (oy * a.sh) * a.lw + ox * a.sw;
    int acc = 0;
    for (int i = 0; i < a.kh; ++i)
      for (int j = 0; j < a.kw; ++j) acc += (int)src[i * a.dh * a.lw + j * a.dw] * (int)wc[i * a.kw + j];
    const int64_t o = (int64_t)plane * a.OH * a.OW + (int64_t)(oy0 + oy) * a.OW + ox;
    float f = (float)acc;
    f = f * a.recip[c];
    f = f + a.bias[c];
    if (a.term > 100) {
      static_cast<int8_t*>(a.y)[o] = quantize_i8(f, a.os, a.act == NHIP_ACT_RELU ? 0 : -127);
    } else {
      if (a.act == NHIP_ACT_RELU) f = f < 0.f ? 0.f : f;
      static_cast<float*>(a.y)[o] = f;
    }
  }
}

__global__ void relu_f32_kernel(const float* x, float* y, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float v = x[i];
    y[i] = v < 0.f ? 0.f : v;
  }
}

__global__ void relu_i8_kernel(const int8_t* x, int8_t* y, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int8_t v = x[i];
    y[i] = v < 0 ? 0 : v;
  }
}

__global__ void add_f32_kernel(const float* a, const float* b, float* y, int64_t n, int relu) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    float v = a[i] + b[i];
    if (relu) v = v < 0.f ? 0.f : v;
    y[i] = v;
  }
}

// The same two operations on 16-byte vectors (inputs and output 16-byte
// aligned).  A workgroup takes one contiguous chunk of 4 x 256 vectors (16
// KB) per step, each thread four of them, 4 KB apart, all four loads in
// flight before the stores (the scalar loop above has one 4-byte load per
// lane outstanding, which left a 154 MB ReLU at 56% of HBM; four vectors per
// thread spread a whole grid stride apart lost DRAM page locality on streams
// larger than the infinity cache).  Element for element the expressions of
// the scalar kernels, so the results are identical; OP 0 ReLU, 1 add, 2 add
// then ReLU.  n4 = whole vectors; the last n % 4 elements go to the scalar
// kernels.
template <int OP>
__global__ __launch_bounds__(256) void eltwise_v4_kernel(const v4f* __restrict__ a, const v4f* __restrict__ b,
                                                         v4f* __restrict__ y, int64_t n4) {
  constexpr int kPer = 4;
  auto op = [](v4f u, v4f w) {
    v4f r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float v = OP == 0 ? u[e] : u[e] + w[e];
      if (OP != 1) v = v < 0.f ? 0.f : v;
      r[e] = v;
    }
    return r;
  };
  const int64_t chunk = (int64_t)kPer * blockDim.x;
  for (int64_t base = (int64_t)blockIdx.x * chunk; base < n4; base += (int64_t)gridDim.x * chunk) {
    if (base + chunk <= n4) {
      v4f ua[kPer], ub[kPer];
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        ua[u] = a[base + u * blockDim.x + threadIdx.x];
        if (OP != 0) ub[u] = b[base + u * blockDim.x + threadIdx.x];
      }
#pragma unroll
      for (int u = 0; u < kPer; ++u) y[base + u * blockDim.x + threadIdx.x] = op(ua[u], OP != 0 ? ub[u] : ua[u]);
    } else {
      for (int u = 0; u < kPer; ++u) {
        const int64_t i = base + u * blockDim.x + threadIdx.x;
        if (i < n4) y[i] = op(a[i], OP != 0 ? b[i] : a[i]);
      }
    }
  }
}

// One wave per (image, channel) plane: sum, then divide by h*w.
__global__ __launch_bounds__(256) void gap_f32_kernel(const float* x, float* y, int64_t planes, int hw) {
  const int64_t plane = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (plane >= planes) return;
  const float* p = x + plane * hw;
  float s = 0.f;
  for (int i = lane; i < hw; i += 64) s += p[i];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if (lane == 0) y[plane] = s / (float)hw;
}

// Global average pooling for planes of at most kGapPlaneMax pixels: a
// workgroup takes `ppb` whole planes, one contiguous block of the input,
// brings it into LDS with 16-byte loads (four in flight per lane) and one
// lane sums each plane in element order, the CPU loop's order: s = 0,
// s += x[e] for e = 0 .. h*w-1, mean = s / (h*w).
constexpr int kGapPlaneMax = 256;

__global__ __launch_bounds__(256) void gap_planes_kernel(const float* x, float* y, int64_t planes, int hw,
                                                         int ppb) {
  extern __shared__ float lds[];
  const int64_t p0 = (int64_t)blockIdx.x * ppb;
  const int np = (int)min((int64_t)ppb, planes - p0);
  const float* xs = x + p0 * hw;
  const int nin = np * hw, nin4 = nin >> 2;
  for (int v0 = threadIdx.x; v0 < nin4; v0 += 1024) {
    v4f t[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (v0 + 256 * u < nin4) __builtin_memcpy(&t[u], xs + 4 * (v0 + 256 * u), 16);  // 4-byte aligned source
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (v0 + 256 * u < nin4) reinterpret_cast<v4f*>(lds)[v0 + 256 * u] = t[u];
  }
  for (int e = (nin4 << 2) + threadIdx.x; e < nin; e += 256) lds[e] = xs[e];
  __syncthreads();
  for (int pi = threadIdx.x; pi < np; pi += 256) {
    const float* src = lds + pi * hw;
    float s = 0.f;
    for (int e = 0; e < hw; ++e) s = s + src[e];
    y[p0 + pi] = s / (float)hw;
  }
}

__global__ void quantize_f32_i8_kernel(const float* x, int8_t* y, int64_t n, int c,
                                       int64_t plane, const float* scale, int scale_count) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int ch = (int)((i / plane) % c);
    y[i] = quantize_i8(x[i], scale[scale_count == 1 ? 0 : ch]);
  }
}

__global__ void requantize_kernel(const int32_t* x, int8_t* y, int64_t n, int c, int64_t plane,
                                  const float* isc, int isn, const float* osc, int osn,
                                  const float* bias, int bn, int act) {
#pragma clang fp contract(off)
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int ch = (int)((i / plane) % c);
    float f = (float)x[i] * isc[isn == 1 ? 0 : ch];
    if (bias) f = f + bias[bn == 1 ? 0 : ch];
    if (act == NHIP_ACT_RELU) f = f < 0.f ? 0.f : f;
    y[i] = quantize_i8(f, osc[osn == 1 ? 0 : ch]);
  }
}

__global__ void dequantize_kernel(const int32_t* x, float* y, int64_t n, int c, int64_t plane,
                                  const float* sc, int sn, const float* bias, int bn) {
#pragma clang fp contract(off)
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int ch = (int)((i / plane) % c);
    float f = (float)x[i] * sc[sn == 1 ? 0 : ch];
    if (bias) f = f + bias[bn == 1 ? 0 : ch];
    y[i] = f;
  }
}

unsigned grid_for(int64_t n) {
  const int64_t blocks = ceil_div(n, 256);
  const int64_t cap = 64LL * cu_count();
  return (unsigned)(blocks < cap ? (blocks > 0 ? blocks : 1) : cap);
}

// The vector kernels: one 16 KB chunk per workgroup per step, at most 16
// workgroups per CU walking the rest.
unsigned grid_v4(int64_t n4) {
  const int64_t blocks = ceil_div(n4, 4 * 256);
  const int64_t cap = 16LL * cu_count();
  return (unsigned)(blocks < cap ? (blocks > 0 ? blocks : 1) : cap);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

// Band sizing shared by both depthwise kernels: about 1024 outputs per
// workgroup, LDS staging within 32 KB (elem = bytes per staged element).
static int dw_bands(int planes, int oh, int ow, int kh, int kw, int sh, int dh, int sw, int dw, int elem,
                    int* ppb, int* ob, int* ir, int* lw, int* bands, int64_t* lds) {
  *lw = (ow - 1) * sw + (kw - 1) * dw + 1;
  const int plane_out = oh * ow;
  if (plane_out >= 512) {
    *ppb = 1;
    *ob = std::max(1, std::min(oh, 1024 / ow));
  } else {
    *ppb = std::max(1, 1024 / plane_out);
    *ob = oh;
  }
  *ir = (*ob - 1) * sh + (kh - 1) * dh + 1;
  while (*ppb > 1 && (int64_t)*ppb * *ir * *lw * elem > 32768) *ppb /= 2;
  while (*ob > 1 && (int64_t)*ppb * *ir * *lw * elem > 32768) {
    *ob = (*ob + 1) / 2;
    *ir = (*ob - 1) * sh + (kh - 1) * dh + 1;
  }
  *lds = (int64_t)*ppb * *ir * *lw * elem;
  if (*lds > 65536) return fail(NHIP_STATUS_UNSUPPORTED, "depthwise: input rows too wide for LDS staging");
  *bands = (int)ceil_div(oh, *ob);
  (void)planes;
  return ok();
}

int launch_dwconv_int8(const nhip_conv_plan* p, const void* in, int in_is_i8, void* out, int n, int h, int w,
                       int oh, int ow, hipStream_t s) {
  DwI8Args a{};
  a.x = in;
  a.y = out;
  a.w = p->weight_i8;
  a.bias = p->bias;
  a.recip = p->recip;
  a.is = p->input_scale;
  a.os = p->output_scale;
  a.term = p->scale_term;
  a.act = p->g.act;
  a.in_i8 = in_is_i8;
  a.C = p->g.c;
  a.H = h;
  a.W = w;
  a.OH = oh;
  a.OW = ow;
  a.kh = p->g.kh;
  a.kw = p->g.kw;
  a.sh = p->g.sh;
  a.sw = p->g.sw;
  a.dh = p->g.dh;
  a.dw = p->g.dw;
  a.pt = p->g.pt;
  a.pl = p->g.pl;
  a.planes = n * p->g.c;
  int64_t lds = 0;
  NHIP_TRY(dw_bands(a.planes, oh, ow, a.kh, a.kw, a.sh, a.dh, a.sw, a.dw, 1, &a.ppb, &a.ob, &a.ir, &a.lw, &a.bands,
                    &lds));
  const int64_t blocks = ceil_div(a.planes, a.ppb) * a.bands;
  NHIP_LAUNCH("dwconv_int8", dwconv_int8_kernel, dim3((unsigned)blocks), dim3(256), (size_t)lds, s, a);
  return check_launch("dwconv_int8");
}

int launch_dwconv_f32(const nhip_conv_plan* p, const float* in, float* out,
                      int n, int h, int w, int oh, int ow, hipStream_t s) {
  DwArgs a{};
  a.x = in;
  a.y = out;
  a.w = p->weight;
  a.bias = p->bias;
  a.C = p->g.c;
  a.H = h;
  a.W = w;
  a.OH = oh;
  a.OW = ow;
  a.kh = p->g.kh;
  a.kw = p->g.kw;
  a.sh = p->g.sh;
  a.sw = p->g.sw;
  a.dh = p->g.dh;
  a.dw = p->g.dw;
  a.pt = p->g.pt;
  a.pl = p->g.pl;
  a.planes = n * p->g.c;
  a.act = p->g.act;
  const bool k3 = a.kh == 3 && a.kw == 3 && a.dh == 1 && a.dw == 1 && a.sh == a.sw && (a.sh == 1 || a.sh == 2);
  const uint64_t x_bytes = (uint64_t)a.planes * h * w * sizeof(float);
  const int hw = h * w, ohw = oh * ow;
  // VEC: rows the window kernel reads and writes as 16-byte vectors (it
  // assumes the left pad of 1)
  const bool vec = w % 4 == 0 && ow % 4 == 0 && a.pl == 1;
  // Small planes whose rows are not vector-aligned (7x7, 14x14, stride 2 to
  // 14 or 7): the streamed whole-plane kernel, when y is 16-byte aligned.
  // NHIP_DW_PLANES=0 switches it off (tuning and tests), =2 takes it for
  // vector-aligned rows too.
  const int planes_mode = setting_int("NHIP_DW_PLANES", 1);
  if (k3 && (!vec || planes_mode == 2) && planes_mode != 0 && hw <= kDwPlaneMax && ow <= kDwRowMax &&
      x_bytes < (1ull << 31) && (reinterpret_cast<uintptr_t>(out) & 15) == 0) {
    // at most one output row per lane and 16 KB of input per chunk, ppb *
    // ohw a multiple of 4 (every output block 16-byte aligned); ppb * 10
    // weights fit the four per lane staged with the copy
    const int step = ohw % 4 == 0 ? 1 : (ohw % 2 == 0 ? 2 : 4);
    const int want = std::max(1, a.sh == 1 ? std::min({256 / oh, 4096 / hw, 100}) : std::min(2048 / hw, 100));
    a.ppb = std::max(step, want / step * step);
    DwStream st{};
    st.x_bytes = (uint32_t)x_bytes;
    st.chunks = (int)ceil_div(a.planes, a.ppb);
    st.copies = (int)ceil_div((int64_t)a.ppb * hw * 4, 4096);
    st.slot = st.copies * 1024;  // floats: 4 waves x copies x 1 KB
    st.oh_div = fast_div(oh);
    st.ohw_div = fast_div(ohw);
    st.ow_div = fast_div(ow);
    const size_t lds = ((size_t)2 * st.slot + (size_t)a.ppb * (ohw + 10)) * sizeof(float);
    // persistent grid: NHIP_DW_WGS_PER_CU (default 4) workgroups per CU
    const int per_cu = std::max(1, setting_int("NHIP_DW_WGS_PER_CU", 4));
    const dim3 grid((unsigned)std::min<int64_t>(st.chunks, (int64_t)per_cu * cu_count()));
    if (a.sh == 1)
      NHIP_LAUNCH("dw3x3_planes_f32", (dw3x3_stream_kernel<1>), grid, dim3(256), lds, s, a, st);
    else
      NHIP_LAUNCH("dw3x3_planes_f32", (dw3x3_stream_kernel<2>), grid, dim3(256), lds, s, a, st);
    return check_launch("dw3x3_planes_f32");
  }
  if (k3 && x_bytes < (1ull << 31)) {
    // output rows per thread: 8 at stride 1 (10 input rows for 8 output
    // rows), 1 at stride 2 (measured at batch 32: 96@112 s1 4.9-5.0 TB/s
    // against 4.6-4.9 with 4 rows, 144@56 s1 5.8-5.9 against 5.6; s2 6.5
    // and 5.3-5.5 against 6.4 and 5.1 with 2 rows)
    const int R = a.sh == 1 ? 8 : 1;
    const int64_t threads = (int64_t)a.planes * ceil_div(oh, R) * ((ow + 3) / 4);
    const dim3 grid((unsigned)ceil_div(threads, 256));
#define NHIP_DW3(S_, R_, V_)                                                                            \
  if (a.sh == S_ && vec == V_) {                                                                        \
    NHIP_LAUNCH("dw3x3s" #S_ "_f32", (dw3x3_f32_kernel<S_, R_, V_>), grid, dim3(256), 0, s, a, (uint32_t)x_bytes); \
    return check_launch("dw3x3_f32");                                                                   \
  }
    NHIP_DW3(1, 8, true)
    NHIP_DW3(1, 8, false)
    NHIP_DW3(2, 1, true)
    NHIP_DW3(2, 1, false)
#undef NHIP_DW3
  }
  int64_t lds = 0;
  NHIP_TRY(dw_bands(a.planes, oh, ow, a.kh, a.kw, a.sh, a.dh, a.sw, a.dw, 4, &a.ppb, &a.ob, &a.ir, &a.lw, &a.bands,
                    &lds));
  const int64_t blocks = ceil_div(a.planes, a.ppb) * a.bands;
  const bool fast = a.kh == 3 && a.kw == 3 && a.sh == 1 && a.sw == 1 && a.dh == 1 && a.dw == 1;
  if (fast) {
    NHIP_LAUNCH("dwconv3x3s1_f32", dwconv3x3s1_f32_kernel, dim3((unsigned)blocks), dim3(256), (size_t)lds, s, a);
    return check_launch("dwconv3x3s1_f32");
  }
  NHIP_LAUNCH("dwconv_f32", dwconv_f32_kernel, dim3((unsigned)blocks), dim3(256), (size_t)lds, s, a);
  return check_launch("dwconv_f32");
}

}  // namespace nhip

using namespace nhip;

extern "C" {

int nhip_relu_f32(const float* input, float* output, int64_t count, void* stream) {
  if (!input || !output) return fail(NHIP_STATUS_NULL_POINTER, "relu: null pointer");
  if (count < 0) return fail(NHIP_STATUS_INVALID_SHAPE, "relu: negative count");
  if (count == 0) return ok();
  if (aligned16(input) && aligned16(output) && count >= 4) {
    const int64_t n4 = count / 4;
    NHIP_LAUNCH("relu_f32", eltwise_v4_kernel<0>, dim3(grid_v4(n4)), dim3(256), 0, as_stream(stream),
                reinterpret_cast<const v4f*>(input), nullptr, reinterpret_cast<v4f*>(output), n4);
    NHIP_TRY(check_launch("relu_f32"));
    if (count % 4 == 0) return ok();
    input += 4 * n4;
    output += 4 * n4;
    count -= 4 * n4;
  }
  NHIP_LAUNCH("relu_f32", relu_f32_kernel, dim3(grid_for(count)), dim3(256), 0, as_stream(stream), input,
                     output, count);
  return check_launch("relu_f32");
}

int nhip_relu_i8(const int8_t* input, int8_t* output, int64_t count, void* stream) {
  if (!input || !output) return fail(NHIP_STATUS_NULL_POINTER, "relu_i8: null pointer");
  if (count < 0) return fail(NHIP_STATUS_INVALID_SHAPE, "relu_i8: negative count");
  if (count == 0) return ok();
  NHIP_LAUNCH("relu_i8", relu_i8_kernel, dim3(grid_for(count)), dim3(256), 0, as_stream(stream), input,
                     output, count);
  return check_launch("relu_i8");
}

int nhip_add_f32(const float* a, const float* b, float* output, int64_t count, int32_t relu,
                 void* stream) {
  if (!a || !b || !output) return fail(NHIP_STATUS_NULL_POINTER, "add: null pointer");
  if (count < 0) return fail(NHIP_STATUS_INVALID_SHAPE, "add: negative count");
  if (count == 0) return ok();
  if (aligned16(a) && aligned16(b) && aligned16(output) && count >= 4) {
    const int64_t n4 = count / 4;
    const auto* a4 = reinterpret_cast<const v4f*>(a);
    const auto* b4 = reinterpret_cast<const v4f*>(b);
    auto* y4 = reinterpret_cast<v4f*>(output);
    if (relu)
      NHIP_LAUNCH("add_f32", eltwise_v4_kernel<2>, dim3(grid_v4(n4)), dim3(256), 0, as_stream(stream), a4, b4, y4, n4);
    else
      NHIP_LAUNCH("add_f32", eltwise_v4_kernel<1>, dim3(grid_v4(n4)), dim3(256), 0, as_stream(stream), a4, b4, y4, n4);
    NHIP_TRY(check_launch("add_f32"));
    if (count % 4 == 0) return ok();
    a += 4 * n4;
    b += 4 * n4;
    output += 4 * n4;
    count -= 4 * n4;
  }
  NHIP_LAUNCH("add_f32", add_f32_kernel, dim3(grid_for(count)), dim3(256), 0, as_stream(stream), a, b,
                     output, count, relu ? 1 : 0);
  return check_launch("add_f32");
}

int nhip_global_avgpool_f32(const float* input, float* output, int32_t n, int32_t c, int32_t h,
                            int32_t w, void* stream) {
  if (!input || !output) return fail(NHIP_STATUS_NULL_POINTER, "global_avgpool: null pointer");
  if (n < 0 || c <= 0 || h <= 0 || w <= 0)
    return fail(NHIP_STATUS_INVALID_SHAPE, "global_avgpool: invalid shape");
  if (n == 0) return ok();
  const int64_t planes = (int64_t)n * c;
  const int hw = h * w;
  if ((int64_t)h * w <= kGapPlaneMax) {
    const int ppb = std::max(1, 4096 / hw);  // 16 KB of input per workgroup
    NHIP_LAUNCH("global_avgpool_f32", gap_planes_kernel, dim3((unsigned)ceil_div(planes, ppb)), dim3(256),
                (size_t)ppb * hw * sizeof(float), as_stream(stream), input, output, planes, hw, ppb);
    return check_launch("global_avgpool_f32");
  }
  NHIP_LAUNCH("global_avgpool_f32", gap_f32_kernel, dim3((unsigned)ceil_div(planes, 4)), dim3(256), 0,
                     as_stream(stream), input, output, planes, hw);
  return check_launch("global_avgpool_f32");
}

int nhip_quantize_f32_i8(const float* input, int8_t* output, int32_t n, int32_t c, int64_t plane,
                         const float* scale, int32_t scale_count, void* stream) {
  if (!input || !output || !scale) return fail(NHIP_STATUS_NULL_POINTER, "quantize: null pointer");
  if (n < 0 || c <= 0 || plane <= 0 || (scale_count != 1 && scale_count != c))
    return fail(NHIP_STATUS_INVALID_SHAPE, "quantize: invalid shape or scale count");
  const int64_t count = (int64_t)n * c * plane;
  if (count == 0) return ok();
  NHIP_LAUNCH("quantize_f32_i8", quantize_f32_i8_kernel, dim3(grid_for(count)), dim3(256), 0, as_stream(stream),
                     input, output, count, c, plane, scale, scale_count);
  return check_launch("quantize_f32_i8");
}

int nhip_requantize_i32_i8(const int32_t* input, int8_t* output, int32_t n, int32_t c,
                           int64_t plane, const float* in_scale, int32_t in_scale_count,
                           const float* out_scale, int32_t out_scale_count, const float* bias,
                           int32_t bias_count, int32_t activation, void* stream) {
  if (!input || !output || !in_scale || !out_scale)
    return fail(NHIP_STATUS_NULL_POINTER, "requantize: null pointer");
  if (n < 0 || c <= 0 || plane <= 0 || (in_scale_count != 1 && in_scale_count != c) ||
      (out_scale_count != 1 && out_scale_count != c) ||
      (bias && bias_count != 1 && bias_count != c))
    return fail(NHIP_STATUS_INVALID_SHAPE, "requantize: invalid shape or scale count");
  const int64_t count = (int64_t)n * c * plane;
  if (count == 0) return ok();
  NHIP_LAUNCH("requantize_i32_i8", requantize_kernel, dim3(grid_for(count)), dim3(256), 0, as_stream(stream),
                     input, output, count, c, plane, in_scale, in_scale_count, out_scale,
                     out_scale_count, bias, bias_count, activation);
  return check_launch("requantize_i32_i8");
}

int nhip_dequantize_i32_f32(const int32_t* input, float* output, int32_t n, int32_t c,
                            int64_t plane, const float* scale, int32_t scale_count,
                            const float* bias, int32_t bias_count, void* stream) {
  if (!input || !output || !scale) return fail(NHIP_STATUS_NULL_POINTER, "dequantize: null pointer");
  if (n < 0 || c <= 0 || plane <= 0 || (scale_count != 1 && scale_count != c) ||
      (bias && bias_count != 1 && bias_count != c))
    return fail(NHIP_STATUS_INVALID_SHAPE, "dequantize: invalid shape or scale count");
  const int64_t count = (int64_t)n * c * plane;
  if (count == 0) return ok();
  NHIP_LAUNCH("dequantize_i32_f32", dequantize_kernel, dim3(grid_for(count)), dim3(256), 0, as_stream(stream),
                     input, output, count, c, plane, scale, scale_count, bias, bias_count);
  return check_launch("dequantize_i32_f32");
}

}  // extern "C"
