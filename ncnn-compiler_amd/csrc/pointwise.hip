// 1x1 stride-1 unpadded fp32 convolution on NCHW (the expand / project
// layers of inverted-residual networks):
//   out[n][k][p] = act(sum_c W[k][c] x[n][c][p] + b[k] (+ res[n][k][p]))
// (ncnn Convolution with kernel 1, lowered by the reference through
// tosa.conv2d -> linalg.conv_2d_nhwc_hwcf: NCNNToTosa.cpp:1107-1530).
//
// These layers move far more bytes than they compute (16 -> 96 channels at
// 112x112 is 1.2 GFLOP against 180 MB), so the kernel streams x once per
// output-channel slice and writes out once:
//   * a workgroup (4 waves) holds the weights of its slice of 16*KT output
//     channels in LDS for its whole life and walks pixel tiles (persistent
//     grid when the tiles outnumber what fits on the GPU);
//   * input channels stream in chunks of 16 (four v_mfma_f32_16x16x4_f32
//     k-steps) straight from HBM into MFMA B fragments (no LDS staging),
//     through a ring of NB register buffers, NB - 1 chunks in flight ahead
//     of the one being multiplied, across tile boundaries;
//   * lane l holds pixels 4*(l%16) .. +3 and feeds pixel 4*(l%16) + v to MFMA
//     v of a k-step, so register r of the four accumulators of a channel
//     block holds four consecutive pixels of one output channel: the result
//     leaves as 16-byte stores, 16 lanes covering 256 contiguous bytes.
// Two work splits inside a workgroup (WC):
//   WC = 1  each wave owns 64 pixels of a 256-pixel tile and all channels
//           (long pixel rows: the 112/56/28 layers);
//   WC = 4  the four waves share one 64-pixel tile and take every fourth
//           chunk of the channels, their partial sums added through LDS in
//           a fixed order (few pixels, long reductions: 14x14 and 7x7).
// SCALAR (H*W % 4 != 0, e.g. 7x7): no 16-byte vectors; lane l holds pixels
// l%16 + 16*v instead, loaded and stored one float at a time, 16 lanes
// covering 64 contiguous bytes per instruction.
// DW = 1 or 2: the 1x1 convolution's input is computed on the fly as a 3x3
// depthwise convolution (stride DW, padding 1, ncnn ConvolutionDepthWise,
// NCNNToTosa.cpp:3376-3503) of x, the inverted-residual block's
// depthwise -> project pair in one pass: channels stream 4 per chunk, each
// lane loads its channel's 3 x (4*DW + 2) input window (16-byte loads for
// the centre, the zero padding through out-of-range offsets) and forms its
// four depthwise outputs in the reference's order (zero, += x*w over
// (kh, kw), + bias, activation; no fused multiply-add), which are then the
// MFMA B operand.  The depthwise output never goes to memory.
#include <cstdio>
#include <cstdlib>

#include "nhip_internal.h"

namespace nhip {
namespace {

constexpr int kThreads = 256;   // 4 waves
constexpr int kChunk = 16;      // input channels per chunk (4 MFMA k-steps)
constexpr int kXcds = 8;
constexpr int kMaxLds = 144 * 1024;
constexpr int kRedFloats = 4 * 4 * 4 * 64;  // WC = 4 reduction area: [src wave][v][r][lane]

struct PwArgs {
  const float* x;        // [N][C][P]
  const float* w;        // [m_pad][ldw]
  const float* bias;     // [m_pad]
  const float* res;      // [N][K][P] or null
  float* out;            // [N][K][P]
  int C, K, P, ldw, c4;  // c4 = C rounded up to 4
  int np;                // N * P pixels (< 2^29: x is < 2^31 bytes)
  int ntiles, nch;       // pixel tiles, 16-channel groups (nch >= WC)
  uint32_t x_bytes, out_bytes;
  // DW: x is the depthwise input [N][C][H][W]; P = OH*OW of the output
  const float* dw_w;     // [C][9]
  const float* dw_b;     // [C]
  int H, W, OW, dw_act;
};

template <int ACT>
__device__ __forceinline__ float activate(float v) {
  if constexpr (ACT == NHIP_ACT_RELU) return v < 0.f ? 0.f : v;
  if constexpr (ACT == NHIP_ACT_SIGMOID) return 1.0f / (1.0f + __expf(-v));
  return v;
}

__device__ __forceinline__ v4f load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// Per-lane pixel geometry of a tile: byte offsets of (n, channel 0, p) in x
// and in out / the residual for the lane's four pixels (one offset when they
// are consecutive in one image); out of range past the last pixel.  DW: xo
// are the three input rows of the depthwise window (byte offset of (n, 0,
// row, DW*ox), out of range for rows outside the image) and lok / rok say
// whether the window's left / right halo column lies inside the image; eo
// is the lane's share of the halo loads (see XChunk), out of range if none.
template <bool SCALAR, int DW>
struct Geo {
  uint32_t xo[DW ? 3 : (SCALAR ? 4 : 1)], oo[SCALAR ? 4 : 1];
  uint32_t eo;
  bool lok, rok;
};

// One chunk of input in registers: four 16-byte pixel vectors (one per
// k-step of 4 channels), or the lane's depthwise window rows for one k-step:
// the 16-byte centre vectors (columns DW*ox .. DW*ox + 3, and + 4 .. + 7 at
// stride 2) of rows 0..2, and one halo value e.  A row of 16 lanes (one
// channel) covers 64 consecutive output pixels, so a lane's halo columns are
// the end columns of its neighbours' centre vectors, moved across by DPP;
// only the two ends of the lane row load them: lanes 0, 1, 2 the left halo of
// rows 0, 1, 2 of lane 0's window, and at stride 1 lanes 13, 14, 15 the right
// halo of rows 0, 1, 2 of lane 15's.  Four loads per k-step at stride 1
// (nine with a load per halo column), seven at stride 2.
template <int DW>
struct XChunk {
  v4f x[4];
};
template <>
struct XChunk<1> {
  v4f m[3];
  float e;
};
template <>
struct XChunk<2> {
  v4f m[3], m2[3];
  float e;
};

// v of lane l - N (SHR) or l + N (SHL) within the lane's row of 16 (DPP
// row_shr / row_shl; 0 past the row's end).
template <int N>
__device__ __forceinline__ float row_shr(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x110 + N, 0xf, 0xf, true));
}
template <int N>
__device__ __forceinline__ float row_shl(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x100 + N, 0xf, 0xf, true));
}

// LDS: W[k0 + 16t + j][c] at (c*16 + j)*KT + t + c/4 (c < c4, j < 16,
// t < KT): the A fragments of one k-step (KT floats per lane, lane
// l = (c%4)*16 + j) are one contiguous 64*KT-float run, and the float of
// padding per four channels spreads the staging writes (consecutive threads
// take consecutive groups of four channels) over the banks; then
// bias[k0 .. k0 + 16*KT); then, for WC = 4, the reduction area.
// RES: add the residual.  Its loads for a tile go out right after the X
// loads of the wave's last chunk of the tile when the wave has at least NB
// chunks per tile (one tile's residual pending at a time), otherwise just
// before the prefetch issued beside that chunk's MFMAs; either way waiting
// for them never waits for later prefetches (vmcnt retires in issue order).
// Loads and stores are raw buffer operations on 32-bit offsets: positions
// past the last pixel or channel carry an offset past the buffer's size, so
// they neither branch nor touch memory.
template <int KT, int ACT, bool RES, int WC, bool SCALAR, int DW>
__global__ __launch_bounds__(kThreads, 2) void pw_conv_kernel(PwArgs a) {
  static_assert(WC == 1 || WC == 4, "channel split over 1 or 4 waves");
  static_assert(!SCALAR || WC == 4, "unaligned pixel rows use the 64-pixel tiles");
  static_assert(!(SCALAR && DW), "the depthwise input needs float4-aligned rows");
  constexpr int CCH = DW ? 4 : kChunk;  // channels per chunk
  constexpr int SPC = CCH / 4;          // MFMA k-steps per chunk
  constexpr int NB = (WC == 1 && !DW) ? 2 : 4;  // chunk buffers
  constexpr int TP = 256 / WC;          // pixels per tile
  constexpr int KS = 16 * KT;           // output channels per slice
  constexpr int RR = WC == 1 ? 4 : 1;   // accumulator rows a wave finalizes
  extern __shared__ __attribute__((aligned(16))) float ws[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int k0 = blockIdx.y * KS;
  float* bs = ws + a.c4 * KS + a.c4 / 4;
  float* dws = bs + KS;                          // DW: [c][12] weights, bias
  float* red = dws + (DW ? a.c4 * 12 : 0);

  // ---- weights and bias of the slice into LDS -----------------------------
  // 16-byte loads along c (weight rows are 16-float aligned and zero past C),
  // eight in flight per thread before their LDS stores: a 960-channel slice
  // is then two round trips to memory, not sixty.
  {
    const int q4 = a.c4 / 4, total = KS * q4;
    for (int e0 = 0; e0 < total; e0 += 8 * kThreads) {
      v4f v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int e = e0 + u * kThreads + tid;
        const int kl = e / q4, k = k0 + kl;
        v[u] = (e < total && k < a.K)
                   ? *reinterpret_cast<const v4f*>(a.w + (int64_t)k * a.ldw + 4 * (e - kl * q4))
                   : v4f{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int e = e0 + u * kThreads + tid;
        if (e < total) {
          const int kl = e / q4, c = 4 * (e - kl * q4);
#pragma unroll
          for (int i = 0; i < 4; ++i) ws[((c + i) * 16 + (kl & 15)) * KT + (kl >> 4) + (c >> 2)] = v[u][i];
        }
      }
    }
  }
  for (int e = tid; e < KS; e += kThreads) bs[e] = (k0 + e < a.K) ? a.bias[k0 + e] : 0.f;
  if constexpr (DW != 0)
    for (int e = tid; e < a.c4 * 12; e += kThreads) {
      const int c = e / 12, t = e - c * 12;
      dws[e] = c >= a.C ? 0.f : t < 9 ? a.dw_w[c * 9 + t] : t == 9 ? a.dw_b[c] : 0.f;
    }
  __syncthreads();

  // XCD-contiguous renumbering of the pixel tiles: consecutive tiles stay on
  // one XCD, and (gridDim.x being a multiple of 8) so do the slices of a
  // tile, which read the same x.
  int first;
  {
    const int nb = gridDim.x;
    const int x = blockIdx.x % kXcds, q = blockIdx.x / kXcds;
    first = x * (nb / kXcds) + min(x, nb % kXcds) + q;
  }
  if (first >= a.ntiles) return;  // uniform over the workgroup
  const int my_tiles = (a.ntiles - 1 - first) / gridDim.x + 1;

  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t orr = make_rsrc(a.out, a.out_bytes);
  const __amdgpu_buffer_rsrc_t resr = make_rsrc(a.res, RES ? a.out_bytes : 0u);
  const int jl = lane & 15, cl = lane >> 4;
  // The channels of a tile come in 16-channel groups; with WC = 4 wave w
  // takes groups w, w+4, ... (the same split, and so the same summation
  // order, with or without the depthwise input).  A chunk is one group, or
  // with DW a quarter of one.
  const int wave_c = WC == 1 ? 0 : wave;                       // first group of this wave
  const int nchw = (a.nch - wave_c + WC - 1) / WC * (16 / CCH);  // chunks per tile (>= 1)
  auto chunk_c0 = [&](int j) {  // first channel of chunk j of this wave
    return DW ? (wave_c + WC * (j >> 2)) * kChunk + (j & 3) * CCH : (wave_c + WC * j) * kChunk;
  };
  const uint32_t cstride = (uint32_t)a.P * 4u;      // bytes between channel planes
  const uint32_t xcstride = DW ? (uint32_t)(a.H * a.W) * 4u : cstride;  // ... of x
  const float inv_p = 1.0f / (float)a.P;

  auto geo = [&](int tile) {
    const int q0 = tile * TP;  // uniform
    const int n0 = q0 / a.P, p0 = q0 - n0 * a.P;
    // the lane's pixels: 4*jl + v (one 16-byte vector), or, one float at a
    // time, jl + 16*v (each load and store instruction then covers 16
    // consecutive pixels of a channel row)
    const int u0 = p0 + (WC == 1 ? wave * 64 : 0) + (SCALAR ? jl : 4 * jl);
    Geo<SCALAR, DW> g;
#pragma unroll
    for (int v = 0; v < (SCALAR ? 4 : 1); ++v) {
      const int u = u0 + 16 * v;  // pixel of image n0 + dn at position p
      int dn = (int)((float)u * inv_p);
      int p = u - dn * a.P;
      if (p < 0) { --dn; p += a.P; }
      if (p >= a.P) { ++dn; p -= a.P; }
      const int n = n0 + dn;
      const bool ok = q0 + (u - p0) < a.np;
      if constexpr (DW != 0) {
        // output (oy, ox .. ox+3), OW % 4 == 0; window rows DW*oy - 1 .. +1,
        // columns DW*ox - 1 .. DW*(ox+3) + 1
        const int oy = p / a.OW, ox = p - oy * a.OW;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
          const int iy = DW * oy - 1 + i;
          g.xo[i] = (ok && (unsigned)iy < (unsigned)a.H) ? (uint32_t)((n * a.C * a.H + iy) * a.W + DW * ox) * 4u
                                                         : kBufOOB;
        }
        g.lok = ox > 0;
        g.rok = DW * ox + 4 < a.W;
      } else {
        g.xo[v] = ok ? (uint32_t)(n * a.C * a.P + p) * 4u : kBufOOB;
      }
      g.oo[v] = ok ? (uint32_t)(n * a.K * a.P + p) * 4u : kBufOOB;
    }
    g.eo = kBufOOB;
    if constexpr (DW != 0) {
      // the lane's halo load: the left halo of row jl of lane 0's window
      // (jl <= 2) or, stride 1, the right halo of row jl - 13 of lane 15's
      // (jl >= 13)
      const int side = jl <= 2 ? 0 : (DW == 1 && jl >= 13) ? 1 : -1;
      if (side >= 0) {
        const int u = p0 + (WC == 1 ? wave * 64 : 0) + 60 * side;  // lane 0's or lane 15's first pixel
        int dn = (int)((float)u * inv_p);
        int p = u - dn * a.P;
        if (p < 0) { --dn; p += a.P; }
        if (p >= a.P) { ++dn; p -= a.P; }
        const int n = n0 + dn;
        const bool ok = q0 + (u - p0) < a.np;
        const int oy = p / a.OW, ox = p - oy * a.OW;
        const int iy = DW * oy - 1 + (side ? jl - 13 : jl);
        const int ix = side ? ox + 4 : DW * ox - 1;
        if (ok && (unsigned)iy < (unsigned)a.H && (unsigned)ix < (unsigned)a.W)
          g.eo = (uint32_t)((n * a.C * a.H + iy) * a.W + ix) * 4u;
      }
    }
    return g;
  };
  auto load_px = [&](__amdgpu_buffer_rsrc_t r, const uint32_t* base, uint32_t add, bool on) {
    if constexpr (SCALAR) {
      v4f v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = buf_load_f32(r, (on && base[e] != kBufOOB) ? base[e] + add : kBufOOB);
      return v;
    } else {
      return load4(r, (on && base[0] != kBufOOB) ? base[0] + add : kBufOOB);
    }
  };

  // chunk j of this wave's share of a tile: channels (wave_c + WC*j)*CCH ..
  auto issue = [&](XChunk<DW>& xb, const Geo<SCALAR, DW>& g, int j, bool live) {
    if constexpr (DW == 0) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int c = chunk_c0(j) + 4 * s + cl;
        xb.x[s] = load_px(xr, g.xo, (uint32_t)c * cstride, live && c < a.C);
      }
    } else {
      const int c = chunk_c0(j) + cl;
      const bool on = live && c < a.C;
      const uint32_t add = (uint32_t)c * xcstride;
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        const bool row = on && g.xo[i] != kBufOOB;
        const uint32_t b = g.xo[i] + add;
        xb.m[i] = load4(xr, row ? b : kBufOOB);
        if constexpr (DW == 2) xb.m2[i] = load4(xr, row ? b + 16u : kBufOOB);
      }
      xb.e = buf_load_f32(xr, (on && g.eo != kBufOOB) ? g.eo + add : kBufOOB);
    }
  };

  v4f acc[KT][4];
#pragma unroll
  for (int t = 0; t < KT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[t][v] = v4f{0.f, 0.f, 0.f, 0.f};

  // depthwise outputs of the lane's channel at its four pixels (lok / rok:
  // the halo columns of the computed tile's window lie inside the image)
  auto depthwise = [&](const XChunk<DW>& xb, int c, bool lok, bool rok) {
    v4f d = {0.f, 0.f, 0.f, 0.f};
    if constexpr (DW != 0) {
#pragma clang fp contract(off)
      const float* wq = dws + c * 12;
      float w[10];
#pragma unroll
      for (int t = 0; t < 10; ++t) w[t] = wq[t];
      // halo columns: the neighbour lane's end column, or at the ends of the
      // lane row the halo loads of lanes 0..2 / 13..15 (all lanes run the
      // moves: the loop is not divergent here)
      float hl[3], hr[3];
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        float last;  // the lane's last window column of row i
        if constexpr (DW == 1) last = xb.m[i][3];
        else last = xb.m2[i][3];
        const float from_left = row_shr<1>(last);
        const float edge_l = i == 0 ? xb.e : i == 1 ? row_shl<1>(xb.e) : row_shl<2>(xb.e);
        hl[i] = lok ? (jl == 0 ? edge_l : from_left) : 0.f;
        if constexpr (DW == 1) {
          const float from_right = row_shl<1>(xb.m[i][0]);
          const float edge_r = i == 2 ? xb.e : i == 1 ? row_shr<1>(xb.e) : row_shr<2>(xb.e);
          hr[i] = rok ? (jl == 15 ? edge_r : from_right) : 0.f;
        }
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
          // window row i: columns DW*ox - 1 + (0 .. 4*DW + 1)
          float row[4 * DW + 2];
          row[0] = hl[i];
#pragma unroll
          for (int e = 0; e < 4; ++e) row[1 + e] = xb.m[i][e];
          if constexpr (DW == 1) row[5] = hr[i];
          else
#pragma unroll
            for (int e = 0; e < 4; ++e) row[5 + e] = xb.m2[i][e];
#pragma unroll
          for (int jj = 0; jj < 3; ++jj) acc = acc + row[DW * v + jj] * w[i * 3 + jj];
        }
        acc = acc + w[9];
        if (a.dw_act == NHIP_ACT_RELU) acc = acc < 0.f ? 0.f : acc;
        d[v] = acc;
      }
    }
    return d;
  };

  auto compute = [&](const XChunk<DW>& xb, int j, const Geo<SCALAR, DW>& g) {
#pragma unroll
    for (int s = 0; s < SPC; ++s) {
      const int cs = chunk_c0(j) + 4 * s;  // first channel of the k-step
      if (cs >= a.c4) break;
      v4f bx;
      if constexpr (DW == 0) bx = xb.x[s];
      else bx = depthwise(xb, cs + cl, g.lok, g.rok);
      float av[KT];
      const float* wp = ws + ((cs >> 2) * 64 + lane) * KT + (cs >> 2);
#pragma unroll
      for (int t = 0; t < KT; ++t) av[t] = wp[t];
#pragma unroll
      for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[t][v] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[t], bx[v], acc[t][v], 0, 0, 0);
    }
  };

  // Row q of the rows this wave finalizes in a channel block: all four
  // (WC = 1) or row `wave` (WC = 4); output channel k0 + 16t + 4cl + row.
  auto row_of = [&](int q) { return WC == 1 ? q : wave; };
  auto krow = [&](int t, int q) { return k0 + 16 * t + 4 * cl + row_of(q); };

  v4f rv[RES ? KT : 1][RES ? RR : 1];
  auto issue_res = [&](const Geo<SCALAR, DW>& g) {
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
      for (int q = 0; q < RR; ++q) {
        const int k = krow(t, q);
        rv[RES ? t : 0][RES ? q : 0] = load_px(resr, g.oo, (uint32_t)k * cstride, k < a.K);
      }
  };

  auto finish = [&](v4f y, int t, int q, const Geo<SCALAR, DW>& g) {
    const int k = krow(t, q);
    const float b = bs[k - k0];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float o = y[v] + b;
      if constexpr (RES) o += rv[t][q][v];
      y[v] = activate<ACT>(o);
    }
    const bool on = k < a.K;
    if constexpr (SCALAR) {
      // one element at a time through a scalar: a bit cast of a vector
      // element subscript reads element 0 whatever the index
#pragma unroll
      for (int e = 0; e < 4; ++e)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(static_cast<float>(y[e])), orr,
                                              (on && g.oo[e] != kBufOOB) ? g.oo[e] + (uint32_t)k * cstride : kBufOOB,
                                              0, 0);
    } else {
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, y), orr,
                                             (on && g.oo[0] != kBufOOB) ? g.oo[0] + (uint32_t)k * cstride : kBufOOB,
                                             0, 0);
    }
  };

  auto epilogue = [&](const Geo<SCALAR, DW>& g) {
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      if constexpr (WC == 1) {
#pragma unroll
        for (int r = 0; r < 4; ++r) finish(v4f{acc[t][0][r], acc[t][1][r], acc[t][2][r], acc[t][3][r]}, t, r, g);
      } else {
        // partial sums of the four waves through red[src][v][r][lane],
        // added in source order
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
          for (int r = 0; r < 4; ++r) red[((wave * 4 + v) * 4 + r) * 64 + lane] = acc[t][v][r];
        __syncthreads();
        v4f y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int src = 0; src < 4; ++src)
#pragma unroll
          for (int v = 0; v < 4; ++v) y[v] += red[((src * 4 + v) * 4 + wave) * 64 + lane];
        __syncthreads();  // the area is free for the next block
        finish(y, t, 0, g);
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[t][v] = v4f{0.f, 0.f, 0.f, 0.f};
    }
  };

  // Chunk stream: chunk (i, j) = this wave's chunk j of its workgroup's tile
  // i.  The issue side (ii, ij, gi) runs NB - 1 chunks ahead of the compute
  // side (i, j, gc); issues past the last tile load nothing.  Every wave
  // walks the same tiles, so the WC = 4 reduction barriers line up.
  const bool res_early = RES && nchw >= NB;
  int ii = 0, ij = 0;
  Geo<SCALAR, DW> gi = geo(first);
  auto issue_next = [&](XChunk<DW>& buf) {
    const bool live = ii < my_tiles;
    issue(buf, gi, ij, live);
    if constexpr (RES)
      if (res_early && live && ij == nchw - 1) issue_res(gi);
    if (++ij == nchw) {
      ij = 0;
      ++ii;
      gi = geo(first + ii * (int)gridDim.x);
    }
  };
  int i = 0, j = 0;
  Geo<SCALAR, DW> gc = gi;

  XChunk<DW> xb[NB];
#pragma unroll
  for (int b = 0; b + 1 < NB; ++b) issue_next(xb[b]);
  bool done = false;
  while (!done) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const bool last = j == nchw - 1;
      if constexpr (RES)
        if (!res_early && last) issue_res(gc);
      issue_next(xb[(b + NB - 1) % NB]);
      compute(xb[b], j, gc);
      if (last) {
        epilogue(gc);
        ++i;
        j = 0;
        if (i >= my_tiles) {
          done = true;
          break;
        }
        gc = geo(first + i * (int)gridDim.x);
      } else {
        ++j;
      }
    }
  }
}

struct PwCfg {
  int kt, wc;
  bool scalar;
  int slices;
  int dw;  // depthwise input stride (0: plain 1x1)
};

size_t pw_lds(int c, const PwCfg& k) {
  const size_t c4 = (size_t)round_up(c, 4);
  return ((c4 + 1) * 16 * k.kt + c4 / 4 + (k.dw ? c4 * 12 : 0) + (k.wc == 4 ? kRedFloats : 0)) * sizeof(float);
}

// Grid: one workgroup per (tile, slice) when they all fit on the GPU at
// once, otherwise as many as fit, each walking an equal share of the tiles;
// gridDim.y = slices.  The occupancy figure is cached per device, kernel and
// LDS size by the runtime.
template <class Kernel>
dim3 pw_grid(Kernel kernel, const PwArgs& a, int slices, size_t lds) {
  const int resident = resident_blocks(reinterpret_cast<const void*>(kernel), kThreads, lds);
  const int64_t fit = (int64_t)resident * cu_count();
  int64_t gx = a.ntiles;
  if (gx * slices > fit) {
    const int64_t per = std::max<int64_t>(1, fit / slices);
    gx = ceil_div(a.ntiles, ceil_div(a.ntiles, per));
  }
  // Tuning / test override NHIP_PW_WGS=n: at most n workgroups per slice
  // (each then walks more tiles).
  if (const int v = setting_int("NHIP_PW_WGS", 0); v > 0) gx = std::min<int64_t>(gx, v);
  // a multiple of 8, so that blockIdx.x % 8 is the XCD (workgroups past the
  // last tile exit at once)
  return dim3((unsigned)round_up(gx, kXcds), (unsigned)slices);
}

template <int KT, int ACT, bool RES, int WC, bool SCALAR, int DW>
int launch_one(const PwArgs& a, int slices, size_t lds, hipStream_t s) {
  const auto kernel = pw_conv_kernel<KT, ACT, RES, WC, SCALAR, DW>;
  NHIP_TRY(ensure_dynamic_lds(reinterpret_cast<const void*>(kernel), kMaxLds));
  NHIP_LAUNCH(DW ? "dwpw_fused_f32" : "pw_conv_f32", kernel, pw_grid(kernel, a, slices, lds), dim3(kThreads), lds,
              s, a);
  return check_launch("pw_conv_f32");
}

template <int KT, int WC, bool SCALAR, int DW>
int launch_act(const PwArgs& a, int act, bool res, int slices, size_t lds, hipStream_t s) {
  if (res) {
    if (act == NHIP_ACT_RELU) return launch_one<KT, NHIP_ACT_RELU, true, WC, SCALAR, DW>(a, slices, lds, s);
    if (act == NHIP_ACT_SIGMOID) return launch_one<KT, NHIP_ACT_SIGMOID, true, WC, SCALAR, DW>(a, slices, lds, s);
    return launch_one<KT, NHIP_ACT_NONE, true, WC, SCALAR, DW>(a, slices, lds, s);
  }
  if (act == NHIP_ACT_RELU) return launch_one<KT, NHIP_ACT_RELU, false, WC, SCALAR, DW>(a, slices, lds, s);
  if (act == NHIP_ACT_SIGMOID) return launch_one<KT, NHIP_ACT_SIGMOID, false, WC, SCALAR, DW>(a, slices, lds, s);
  return launch_one<KT, NHIP_ACT_NONE, false, WC, SCALAR, DW>(a, slices, lds, s);
}

template <int WC, bool SCALAR, int DW>
int launch_kt(const PwArgs& a, const PwCfg& c, int act, bool res, size_t lds, hipStream_t s) {
  switch (c.kt) {
    case 1: return launch_act<1, WC, SCALAR, DW>(a, act, res, c.slices, lds, s);
    case 2: return launch_act<2, WC, SCALAR, DW>(a, act, res, c.slices, lds, s);
    case 3:
      if constexpr (DW != 2) return launch_act<3, WC, SCALAR, DW>(a, act, res, c.slices, lds, s);
      break;
  }
  return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "pointwise conv: no kernel for the configuration");
}

// Work split and slicing for n images of P pixels:
//   * WC = 4 when the image rows are not float4-aligned (P % 4 != 0), or
//     when 256-pixel tiles give fewer work items than two per CU for a long
//     reduction (8+ chunks): the channel chain of one wave is then the
//     critical path, and four waves splitting it shorten it fourfold;
//   * output channels per slice 16*KT with KT = 1..3 (larger KT measured
//     slower on every MobileNetV2 layer: each slice's re-read of x comes
//     from L2, and the kernel's code stays small), the largest that still
//     gives two (tile, slice) work items per CU, fits the LDS and leaves no
//     slice mostly padding.
// NHIP_PW_CFG="kt,wc" forces a configuration (tuning and tests).
bool pw_config(const nhip_conv_plan* p, int64_t np, int P, int dw, PwCfg* out) {
  const int kb = (int)ceil_div(p->g.k, 16);
  const int nch = (int)ceil_div(round_up(p->g.c, 4), kChunk);  // 16-channel groups
  const int64_t target = 2LL * cu_count();
  PwCfg c{1, 1, P % 4 != 0, 1, dw};
  if (dw && c.scalar) return false;
  if (c.scalar) c.wc = 4;
  else if (nch >= 8 && ceil_div(np, 256) * kb < target) c.wc = 4;
  const int64_t tiles = ceil_div(np, 256 / c.wc);
  // With a depthwise input every slice recomputes the depthwise values: take
  // the widest slice there (KT <= 2 at stride 2, whose window with 48 output
  // channels and a residual would not fit the registers).
  const int kt_max = std::min(dw == 2 ? 2 : 3, kb);
  for (int t = kt_max; t >= 1; --t) {
    if (dw) {
      c.kt = t;
      break;
    }
    const int slices = (int)ceil_div(kb, t);
    if (t > 1 && slices * t - kb >= (t + 1) / 2) continue;  // a slice mostly padding
    if (pw_lds(p->g.c, PwCfg{t, c.wc, c.scalar, slices, dw}) > (size_t)kMaxLds) continue;
    // (long reductions split over the four waves, 512+ channels: the widest
    // slice whatever the item count; 576 -> 96 at 14x14, batch 32: 19.8 us
    // with 48-channel slices against 22.9 with 16)
    if (tiles * slices >= target || t == 1 || (c.wc == 4 && p->g.c >= 512)) {
      c.kt = t;
      break;
    }
  }
  if (const char* env = setting("NHIP_PW_CFG")) {
    int kt = 0, wc = 0;
    if (std::sscanf(env, "%d,%d", &kt, &wc) == 2 && kt >= 1 && kt <= 3 && (wc == 4 || (wc == 1 && !c.scalar))) {
      c.kt = std::min(kt, dw == 2 ? 2 : 3);
      c.wc = wc;
    }
  }
  c.slices = (int)ceil_div(kb, c.kt);
  if (c.wc == 4 && nch < 4) return false;  // every wave needs a chunk
  if (pw_lds(p->g.c, c) > (size_t)kMaxLds) return false;
  *out = c;
  return true;
}

}  // namespace

bool pointwise_selected(const nhip_conv_plan* p, int n, int h, int w) {
  const ConvGeom& g = p->g;
  if (g.kh != 1 || g.kw != 1 || g.sh != 1 || g.sw != 1 || g.pt || g.pb || g.pl || g.pr) return false;
  if (const char* env = setting("NHIP_POINTWISE"))
    if (env[0] == '0') return false;
  PwCfg c;
  const int64_t np = (int64_t)n * h * w;
  if (!pw_config(p, np, h * w, 0, &c)) return false;
  // x and out are addressed by 32-bit buffer offsets
  const int64_t xb = np * g.c * 4, ob = np * g.k * 4;
  if (xb >= (int64_t(1) << 31) || ob >= (int64_t(1) << 31)) return false;
  // Every tile's workgroups read the whole weight matrix once: when that
  // exceeds twice the activation traffic (few pixels, many channels: the
  // 7x7 layers of MobileNetV2), the implicit GEMM, which streams the weights
  // through its K loop, measured faster.
  const int64_t w_traffic = ceil_div(np, 256 / c.wc) * (int64_t)g.c * g.k * 4;
  const bool forced = setting("NHIP_PW_CFG") != nullptr;
  return forced || w_traffic <= 2 * (xb + ob);
}

namespace {

int launch_pw(const nhip_conv_plan* p, const PwCfg& c, PwArgs& a, int n, const float* residual, hipStream_t s) {
  a.w = p->weight;
  a.bias = p->bias;
  a.res = residual;
  a.C = p->g.c;
  a.K = p->g.k;
  a.ldw = p->kred_pad;
  a.c4 = (int)round_up(a.C, 4);
  a.np = n * a.P;
  a.ntiles = (int)ceil_div(a.np, 256 / c.wc);
  a.nch = (int)ceil_div(a.c4, kChunk);
  a.out_bytes = (uint32_t)((int64_t)n * a.K * a.P * 4);
  const size_t lds = pw_lds(a.C, c);
  const int act = p->g.act;
  const bool res = residual != nullptr;
  if (c.dw == 1) return c.wc == 1 ? launch_kt<1, false, 1>(a, c, act, res, lds, s) : launch_kt<4, false, 1>(a, c, act, res, lds, s);
  if (c.dw == 2) return c.wc == 1 ? launch_kt<1, false, 2>(a, c, act, res, lds, s) : launch_kt<4, false, 2>(a, c, act, res, lds, s);
  if (c.wc == 1) return launch_kt<1, false, 0>(a, c, act, res, lds, s);
  if (!c.scalar) return launch_kt<4, false, 0>(a, c, act, res, lds, s);
  return launch_kt<4, true, 0>(a, c, act, res, lds, s);
}

// The depthwise plan's shape rules for the fused kernel: 3x3, stride 1 or 2
// (both axes), padding 1 on every side, dilation 1, and float4-aligned input
// and output rows (W and OW multiples of 4, so a lane's four outputs and
// their window centres are 16-byte vectors of one row).
bool dw_shape_ok(const nhip_conv_plan* dw, int h, int w, int* oh, int* ow) {
  const ConvGeom& g = dw->g;
  if (dw->kind != PlanKind::DwConvF32 || g.kh != 3 || g.kw != 3 || g.dh != 1 || g.dw != 1 || g.sh != g.sw ||
      (g.sh != 1 && g.sh != 2) || g.pt != 1 || g.pb != 1 || g.pl != 1 || g.pr != 1)
    return false;
  // the fused kernels apply no depthwise activation other than ReLU
  if (g.act != NHIP_ACT_NONE && g.act != NHIP_ACT_RELU) return false;
  *oh = (h + 2 - 3) / g.sh + 1;
  *ow = (w + 2 - 3) / g.sw + 1;
  return w % 4 == 0 && *ow % 4 == 0 && *oh > 0;
}

}  // namespace

int launch_conv_pointwise_f32(const nhip_conv_plan* p, const float* in, const float* residual, float* out, int n,
                              int h, int w, hipStream_t s) {
  PwCfg c;
  if (!pw_config(p, (int64_t)n * h * w, h * w, 0, &c))
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "pointwise conv: unsupported shape");
  PwArgs a{};
  a.x = in;
  a.out = out;
  a.P = h * w;
  a.x_bytes = (uint32_t)((int64_t)n * p->g.c * a.P * 4);
  return launch_pw(p, c, a, n, residual, s);
}

bool dwpw_supported(const nhip_conv_plan* dw, const nhip_conv_plan* pw, int n, int h, int w) {
  bool every = false;  // NHIP_DWPW=2: every pair the kernel can run (tests)
  if (const char* env = setting("NHIP_DWPW")) {
    if (env[0] == '0') return false;
    every = env[0] == '2';
  }
  int oh = 0, ow = 0;
  if (!dw_shape_ok(dw, h, w, &oh, &ow)) return false;
  // Measured on the MobileNetV2 pairs (batch 32): every output-channel
  // slice recomputes the depthwise values, which pays when the 1x1 conv's
  // channels fit one slice (K <= 32): stride 2 (96@112 -> 24 in 32.4 us
  // against ~57 us for the two layers, 144@56 -> 32 in 21.3 against ~25)
  // and stride 1 from 28 output columns (32@112 -> 16 in 26.1 against 35.4
  // us, 144@56 -> 24 with residual 36.9 against 40.6, 192@28 -> 32 with
  // residual 20.5 against 23.4).  With few pixels the fused kernel's
  // workgroups are too few to cover its per-chunk latency: the whole graph
  // ran 0.336 ms unfused against 0.381 fused at batch 1, 0.413 against
  // 0.428 at batch 8, even at 16 and 0.79 against 0.81 at 32, so pairs are
  // fused from 24576 output pixels (a batch-32 28x28 plane set).
  if (!every && (pw->g.k > 32 || (dw->g.sh != 2 && !(dw->g.sh == 1 && ow >= 28)) ||
                 (int64_t)n * oh * ow < 24576))
    return false;
  const ConvGeom& g = pw->g;
  if (pw->kind != PlanKind::ConvF32 || g.c != dw->g.c || g.kh != 1 || g.kw != 1 || g.sh != 1 || g.sw != 1 || g.pt ||
      g.pb || g.pl || g.pr || pw->algorithm != NHIP_CONV_ALGO_IMPLICIT_GEMM)
    return false;
  if (dwpw_lds_supported(dw, pw, n, h, w, oh, ow)) return true;
  PwCfg c;
  const int64_t np = (int64_t)n * oh * ow;
  if (!pw_config(pw, np, oh * ow, dw->g.sh, &c)) return false;
  const int64_t xb = (int64_t)n * g.c * h * w * 4, ob = np * g.k * 4;
  return xb < (int64_t(1) << 31) && ob < (int64_t(1) << 31);
}

int launch_dwpw_f32(const nhip_conv_plan* dw, const nhip_conv_plan* pw, const float* in, const float* residual,
                    float* out, int n, int h, int w, hipStream_t s) {
  int oh = 0, ow = 0;
  PwCfg c;
  if (dw_shape_ok(dw, h, w, &oh, &ow) && dwpw_lds_supported(dw, pw, n, h, w, oh, ow))
    return launch_dwpw_lds_f32(dw, pw, in, residual, out, n, h, w, oh, ow, s);
  if (!dw_shape_ok(dw, h, w, &oh, &ow) || !pw_config(pw, (int64_t)n * oh * ow, oh * ow, dw->g.sh, &c))
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "depthwise + pointwise: unsupported shape");
  PwArgs a{};
  a.x = in;
  a.out = out;
  a.P = oh * ow;
  a.x_bytes = (uint32_t)((int64_t)n * pw->g.c * h * w * 4);
  a.dw_w = dw->weight;
  a.dw_b = dw->bias;
  a.H = h;
  a.W = w;
  a.OW = ow;
  a.dw_act = dw->g.act;
  return launch_pw(pw, c, a, n, residual, s);
}

}  // namespace nhip
