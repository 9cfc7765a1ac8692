// int8 Convolution with requantize (reference ConvertConvolution int8 path,
// NCNNToTosa.cpp:1136-1315), bit-exact with the reference's arithmetic:
//
//   q   = quantizeSignedI8(x, is)     s = x*is; s>=0 ? floor(s+.5) : ceil(s-.5);
//                                     clamp [-127, 127]        (:322-389)
//   acc = sum_{kh,kw,c} q * w_i8      int32, zero points 0     (:1160-1167,1277-1290)
//   f   = (float)acc * r[k]           r = ws==0 ? 0 : 1/(ws*is) (:577-637)
//   f   = f + bias[k]                 (:1294-1300)
//   term > 100: out = quantizeSignedI8(f, os)                  (:1309-1312)
//   activation 1: relu on the result (ImportConvolution.cpp:236-241)
//
// Every fp32 step is a separately rounded operation: this file is compiled
// with -ffp-contract=off and the epilogue helpers also carry the clang
// contract(off) pragma, so no multiply-add is fused.  The integer
// accumulation is exact in any order, which is what lets the reduction run
// on v_mfma_i32_32x32x32_i8 in a different order from the CPU loop nest.
//
// Layout: the GEMM gathers 16-byte channel vectors per (pixel, kh, kw),
// reduction order (kh, kw, c) — the OHWI order the reference itself
// transposes the weights to (NCNNToTosa.cpp:1168-1176) — from an NHWC int8
// image with channels padded to 16.  The register-weight kernel builds that
// layout for its own input window in LDS, quantizing fp32 input on the way
// (NHIP_INT8_FUSED_QUANT=0 turns this off); the other kernels read a scratch
// image that a separate pass quantizes (one pass over HBM).
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "nhip_internal.h"

namespace nhip {
namespace {

constexpr int kThreads = 256;

// x [N][C][HW] (fp32 or int8) -> y [N][HW][c_pad] int8, zero channel padding.
// Workgroup = 64 pixels x one 64-channel slab of one image (grid x: pixel
// blocks, y: slabs, z: images); thread (pixel, q) quantizes channels 16q ..
// 16q + 15 of the slab at its pixel (each load instruction: 64 consecutive
// pixels of one channel) and writes them as one 16-byte NHWC vector, with
// no LDS transpose; the four 16-byte pieces of a pixel's 64 bytes come from
// the four waves of the workgroup.
__global__ __launch_bounds__(kThreads) void quantize_nchw_to_nhwc(
    const void* __restrict__ x, int in_is_i8, int8_t* __restrict__ y, int C,
    int HW, int c_pad, float scale) {
  const int img = blockIdx.z;
  const int p = blockIdx.x * 64 + (threadIdx.x & 63);
  const int cw = blockIdx.y * 64 + (threadIdx.x >> 6) * 16;
  if (p >= HW || cw >= c_pad) return;
  const float* xf = static_cast<const float*>(x) + (int64_t)img * C * HW;
  const int8_t* xi = static_cast<const int8_t*>(x) + (int64_t)img * C * HW;
  int v[16];
  if (in_is_i8) {
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = cw + u < C ? xi[(int64_t)(cw + u) * HW + p] : 0;
  } else {
    float f[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) f[u] = cw + u < C ? xf[(int64_t)(cw + u) * HW + p] : 0.0f;
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = quantize_q(f[u], scale);
  }
  int4 out;
  int* o = reinterpret_cast<int*>(&out);
#pragma unroll
  for (int q = 0; q < 4; ++q) o[q] = (int)pack_i8x4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
  *reinterpret_cast<int4*>(y + ((int64_t)img * HW + p) * c_pad + cw) = out;
}

struct Int8Args {
  const int8_t* w;     // [m_pad][kred_pad]; register-weight kernel: fragment order (weight_i8_frag)
  int kred_pad;
  int m;               // num_output
  const int8_t* x;     // NHWC [N][H][W][c_pad]
  uint32_t x_bytes;    // size of x (< 2^31)
  int H, W, c_pad, OW, OHW, sh, sw, pt, pl;
  int npix;            // N*OH*OW
  const int* ktab;     // per 16-byte k chunk: c0<<16 | dy<<8 | dx (sentinel past kred)
  const float* recip;  // [m_pad]
  const float* bias;   // [m_pad]
  float os;
  int term, act;
  void* out;           // int8 or fp32 NCHW
  // footprint kernel only
  int OH, R;           // output rows per workgroup
  int FH, FW, FS;      // input footprint rows / columns / LDS bytes per pixel
  int fp_bytes;        // LDS bytes of the footprint (multiple of 16)
  int rb_off;             // LDS byte offset of the footprint kernel's reciprocals and biases
  FastDiv cpp_div, fw_div;  // footprint copy: 16-byte channel chunks per pixel, window width
  // register-weight kernel only
  uint32_t out_bytes;     // size of out (< 2^31)
  int kred, KW, dh, dw;   // unpadded reduction bytes, kernel width, dilations
  int vec;                // output stores: 0 single elements, 1 four pixels, 2 sixteen int8 pixels
  // register-weight kernel with the quantization fused into its window fill
  const float* xf;        // fp32 NCHW input [N][C][H][W] (W % 4 == 0, 16-byte aligned)
  uint32_t xf_bytes;      // size of xf (< 2^31)
  int C;                  // input channels (% 4 == 0)
  float in_scale;         // quantizeSignedI8 scale of the input
  FastDiv xg_div, c4_div;  // window items: W/4 column groups, C/4 channel groups
};

// D[i = out channel][j = pixel] over the (kh, kw, c) reduction.
// One workgroup = 4 waves (2x2), each a (BM/2) x (BN/2) tile of 32x32 blocks
// with v_mfma_i32_32x32x32_i8.  K advances BK bytes per stage through two LDS
// buffers; global loads run two stages ahead (stage k multiplies while stage
// k+1 waits in registers and stage k+2 is in flight), and the loop body is
// straight-line so the accumulators stay in one register range.
template <int BM, int BN, int BK>
__global__ __launch_bounds__(kThreads) void conv_int8_kernel(Int8Args g) {
  constexpr int TM = BM / 64, TN = BN / 64;
  constexpr int ROW = BK + 16;              // LDS row stride (bytes): conflict-free b128 reads
  constexpr int CH = BK / 16;               // 16-byte chunks per row per stage
  constexpr int A_LD = BM * CH / kThreads;  // 16-byte loads per thread per stage
  constexpr int B_LD = BN * CH / kThreads;
  static_assert(A_LD >= 1 && B_LD >= 1, "tile too small for the workgroup");
  constexpr int ES = BN + 16;  // LDS row stride of the staged epilogue tile (elements)
  constexpr int OPER = 2 * (BM + BN) * ROW;
  constexpr int EPI = BM * ES * 4;
  __shared__ __attribute__((aligned(16))) int8_t smem[OPER > EPI ? OPER : EPI];
  // operand buffers: A[buf] = smem + buf*BM*ROW, B[buf] = smem + 2*BM*ROW + buf*BN*ROW
  auto As = [&](int buf) { return smem + buf * BM * ROW; };
  auto Bs = [&](int buf) { return smem + 2 * BM * ROW + buf * BN * ROW; };
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 31, lh = lane >> 5;
  const int j0 = blockIdx.x * BN, i0 = blockIdx.y * BM;

  // B gather: load u of a thread covers pixel jj[u] = (tid + u*256) / CH and
  // 16-byte chunk tid % CH of the stage, so CH consecutive lanes read one
  // pixel's contiguous channel run (one cache line per CH lanes, not one per
  // lane).  The pixel geometry of each load is fixed for the whole K loop.
  const int chl = tid % CH;
  int iy0[B_LD], ix0[B_LD], ipix0[B_LD];
  bool pok[B_LD];
#pragma unroll
  for (int u = 0; u < B_LD; ++u) {
    const int p = j0 + (tid + u * kThreads) / CH;
    pok[u] = p < g.npix;
    const int pp = pok[u] ? p : 0;
    const int img = pp / g.OHW;
    const int rem = pp - img * g.OHW;
    const int oh = rem / g.OW, ow = rem - oh * g.OW;
    iy0[u] = oh * g.sh - g.pt;
    ix0[u] = ow * g.sw - g.pl;
    ipix0[u] = img * g.H;
  }
  // the whole NHWC scratch image is one wave-uniform buffer resource
  const __amdgpu_buffer_rsrc_t img_rs = make_rsrc(g.x, g.x_bytes);

  struct Stage {
    v4i a[A_LD];
    v4i b[B_LD];
  };
  auto gload = [&](Stage& st, int kt) {
#pragma unroll
    for (int u = 0; u < A_LD; ++u) {
      const int q = tid + u * kThreads;
      const int row = q / CH, ch = q % CH;
      st.a[u] = *reinterpret_cast<const v4i*>(g.w + (int64_t)(i0 + row) * g.kred_pad + kt * BK + ch * 16);
    }
    const int t = g.ktab[kt * CH + chl];
    const int c0 = t >> 16, dy = (t >> 8) & 255, dx = t & 255;
#pragma unroll
    for (int u = 0; u < B_LD; ++u) {
      const int y = iy0[u] + dy, x = ix0[u] + dx;
      const bool in = pok[u] && c0 < g.c_pad && (unsigned)y < (unsigned)g.H && (unsigned)x < (unsigned)g.W;
      st.b[u] = __builtin_bit_cast(
          v4i, buf_load_b128(img_rs, in ? (uint32_t)(((ipix0[u] + y) * g.W + x) * g.c_pad + c0) : kBufOOB));
    }
  };
  auto lstore = [&](const Stage& st, int buf) {
#pragma unroll
    for (int u = 0; u < A_LD; ++u) {
      const int q = tid + u * kThreads;
      const int row = q / CH, ch = q % CH;
      *reinterpret_cast<v4i*>(As(buf) + row * ROW + ch * 16) = st.a[u];
    }
#pragma unroll
    for (int u = 0; u < B_LD; ++u)
      *reinterpret_cast<v4i*>(Bs(buf) + ((tid + u * kThreads) / CH) * ROW + chl * 16) = st.b[u];
  };

  v16i acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0;

  auto compute = [&](int buf) {
#pragma unroll
    for (int s = 0; s < BK / 32; ++s) {
      v4i af[TM], bf[TN];
#pragma unroll
      for (int a = 0; a < TM; ++a)
        af[a] = *reinterpret_cast<const v4i*>(As(buf) + (wm * (BM / 2) + a * 32 + li) * ROW + s * 32 + lh * 16);
#pragma unroll
      for (int b = 0; b < TN; ++b)
        bf[b] = *reinterpret_cast<const v4i*>(Bs(buf) + (wn * (BN / 2) + b * 32 + li) * ROW + s * 32 + lh * 16);
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[a], bf[b], acc[a][b], 0, 0, 0);
    }
  };

  const int n = g.kred_pad / BK;
  {
    Stage s0, s1;
    gload(s0, 0);
    if (n > 1) gload(s1, 1);
    lstore(s0, 0);
    __syncthreads();
    int i = 0;
    for (; i + 1 < n; i += 2) {
      if (i + 2 < n) gload(s0, i + 2);
      compute(0);
      lstore(s1, 1);
      __syncthreads();
      if (i + 3 < n) gload(s1, i + 3);
      compute(1);
      if (i + 2 < n) lstore(s0, 0);
      __syncthreads();
    }
    if (i < n) compute(0);
  }

  // Epilogue.  Register r of lane l holds row (r%4)+8*(r/4)+4*(l/32), column
  // l%32.  The exact fp32 sequence runs per element, the results are staged
  // in LDS as [i][j] (over the operand buffers, free after the barrier),
  // and each thread then writes 16 consecutive pixels of one output channel
  // with one vector store (bytes or floats), falling back to element stores
  // where the run crosses an image or the tile edge or is misaligned.
  __syncthreads();
  const bool q8 = g.term > 100, relu = g.act == NHIP_ACT_RELU;
  const int qlo = relu ? 0 : -127;  // requantized ReLU: the saturation's lower bound
  float* tf = reinterpret_cast<float*>(smem);
  int8_t* tq = smem;
  // One wave-uniform branch on the output kind; the per-value arithmetic
  // is branch-free.
  auto dequant = [&](int a, int b, int r, int il) {  // il: row of the tile
#pragma clang fp contract(off)
    float f = (float)acc[a][b][r];
    f = f * g.recip[i0 + il];
    return f + g.bias[i0 + il];
  };
#define NHIP_I8_EPI(STORE)                                                                 \
  for (int b = 0; b < TN; ++b) {                                                          \
    const int jl = wn * (BN / 2) + b * 32 + li;                                           \
    _Pragma("unroll") for (int a = 0; a < TM; ++a) _Pragma("unroll") for (int r = 0; r < 16; ++r) { \
      const int il = wm * (BM / 2) + a * 32 + (r & 3) + 8 * (r >> 2) + 4 * lh;            \
      const float f = dequant(a, b, r, il);                                              \
      STORE;                                                                              \
    }                                                                                     \
  }
  if (q8) {
#pragma unroll
    NHIP_I8_EPI({
      tq[il * ES + jl] = quantize_i8(f, g.os, qlo);
    })
  } else {
#pragma unroll
    NHIP_I8_EPI(tf[il * ES + jl] = (relu && f < 0.0f) ? 0.0f : f)
  }
  __syncthreads();
  constexpr int RUNS = BN / 16;  // 16-pixel runs per row
  for (int q = tid; q < BM * RUNS; q += kThreads) {
    const int il = q / RUNS, jl = (q % RUNS) * 16;
    const int i = i0 + il, j = j0 + jl;
    if (i >= g.m || j >= g.npix) continue;
    const int im = j / g.OHW, rm = j - im * g.OHW;
    const int64_t o = ((int64_t)im * g.m + i) * g.OHW + rm;
    const bool whole = j + 16 <= g.npix && rm + 16 <= g.OHW && (o & 15) == 0;
    if (q8) {
      int8_t* dst = static_cast<int8_t*>(g.out);
      if (whole) {
        *reinterpret_cast<v4i*>(dst + o) = *reinterpret_cast<const v4i*>(&tq[il * ES + jl]);
      } else {
        for (int e = 0; e < 16 && j + e < g.npix; ++e) {
          const int je = j + e, ie = je / g.OHW;
          dst[((int64_t)ie * g.m + i) * g.OHW + (je - ie * g.OHW)] = tq[il * ES + jl + e];
        }
      }
    } else {
      float* dst = static_cast<float*>(g.out);
      if (whole) {
#pragma unroll
        for (int e = 0; e < 16; e += 4)
          *reinterpret_cast<v4f*>(dst + o + e) = *reinterpret_cast<const v4f*>(&tf[il * ES + jl + e]);
      } else {
        for (int e = 0; e < 16 && j + e < g.npix; ++e) {
          const int je = j + e, ie = je / g.OHW;
          dst[((int64_t)ie * g.m + i) * g.OHW + (je - ie * g.OHW)] = tf[il * ES + jl + e];
        }
      }
    }
  }
}

// Footprint variant.  A workgroup owns R whole output rows of one image (at
// most 128 pixels, padded to 128 MFMA columns) and BM output channels.  The
// input rows those outputs read (a (R-1)*sh+(kh-1)*dh+1 by
// (OW-1)*sw+(kw-1)*dw+1 window of the NHWC int8 scratch image, zero halo) are
// copied into LDS once, with coalesced 16-byte loads; every tap's B fragment
// is then read straight from that window, so only the weights stream through
// the two-stage K pipeline (they are shared by all workgroups and stay in
// L2).  Same MFMA mapping, accumulation and epilogue as conv_int8_kernel.
template <int BM, int BK>
__global__ __launch_bounds__(kThreads) void conv_int8_fp_kernel(Int8Args g) {
  constexpr int BN = 128;
  constexpr int TM = BM / 64, TN = BN / 64;
  constexpr int ROW = BK + 16;
  constexpr int CH = BK / 16;
  constexpr int A_LD = BM * CH / kThreads;
  constexpr int ES = BN + 16;
  extern __shared__ __attribute__((aligned(16))) int8_t dsm[];
  int8_t* foot = dsm;
  auto As = [&](int buf) { return dsm + g.fp_bytes + buf * BM * ROW; };
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 31, lh = lane >> 5;
  const int rgs = (g.OH + g.R - 1) / g.R;
  const int img = blockIdx.x / rgs, oy0 = (blockIdx.x % rgs) * g.R;
  const int i0 = blockIdx.y * BM;
  const int npx = min(g.R, g.OH - oy0) * g.OW;  // valid pixels of this workgroup

  struct Stage {
    v4i a[A_LD];
  };
  auto gload = [&](Stage& st, int kt) {
#pragma unroll
    for (int u = 0; u < A_LD; ++u) {
      const int q = tid + u * kThreads;
      const int row = q / CH, ch = q % CH;
      st.a[u] = *reinterpret_cast<const v4i*>(g.w + (int64_t)(i0 + row) * g.kred_pad + kt * BK + ch * 16);
    }
  };
  auto lstore = [&](const Stage& st, int buf) {
#pragma unroll
    for (int u = 0; u < A_LD; ++u) {
      const int q = tid + u * kThreads;
      const int row = q / CH, ch = q % CH;
      *reinterpret_cast<v4i*>(As(buf) + row * ROW + ch * 16) = st.a[u];
    }
  };

  // The first two weight stages, the footprint and this workgroup's
  // reciprocals and biases are all requested before anything waits, so
  // their latencies overlap instead of adding up.
  const int n = g.kred_pad / BK;
  Stage s0, s1;
  gload(s0, 0);
  if (n > 1) gload(s1, 1);
  float* rb = reinterpret_cast<float*>(dsm + g.rb_off);  // [BM] reciprocals, then [BM] biases
  if (tid < BM) {
    rb[tid] = g.recip[i0 + tid];
    rb[BM + tid] = g.bias[i0 + tid];
  }

  // ---- footprint -> LDS, eight 16-byte loads in flight per thread
  {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(g.x, g.x_bytes);
    const int cpp = g.c_pad / 16;
    const int total = g.FH * g.FW * cpp;
    const int iy_base = oy0 * g.sh - g.pt;
    for (int base = 0; base < total; base += 8 * kThreads) {
      v4i v[8];
      int dst[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int e = base + q * kThreads + tid;
        const int pix = fdiv(e, g.cpp_div), ch = e - pix * cpp;
        const int fy = fdiv(pix, g.fw_div), fx = pix - fy * g.FW;
        const int iy = iy_base + fy, ix = fx - g.pl;
        const bool in = e < total && (unsigned)iy < (unsigned)g.H && (unsigned)ix < (unsigned)g.W;
        v[q] = __builtin_bit_cast(
            v4i, buf_load_b128(rs, in ? (uint32_t)(((img * g.H + iy) * g.W + ix) * g.c_pad + ch * 16) : kBufOOB));
        dst[q] = e < total ? pix * g.FS + ch * 16 : -1;
      }
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (dst[q] >= 0) *reinterpret_cast<v4i*>(foot + dst[q]) = v[q];
    }
  }

  // per-lane window origin (bytes) of each of the wave's pixel columns
  int fbase[TN];
#pragma unroll
  for (int b = 0; b < TN; ++b) {
    const int pc = min(wn * (BN / 2) + b * 32 + li, npx - 1);
    const int py = pc / g.OW, px = pc - py * g.OW;
    fbase[b] = (py * g.sh * g.FW + px * g.sw) * g.FS;
  }

  v16i acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0;

  auto compute = [&](int buf, int kt) {
#pragma unroll
    for (int s = 0; s < BK / 32; ++s) {
      const int t = g.ktab[kt * CH + s * 2 + lh];  // this lane's 16-byte k chunk
      int c0 = t >> 16;
      const int dy = (t >> 8) & 255, dx = t & 255;
      if (c0 >= g.c_pad) c0 = 0;  // K padding: the weights there are zero
      const int koff = (dy * g.FW + dx) * g.FS + c0;
      v4i af[TM], bf[TN];
#pragma unroll
      for (int a = 0; a < TM; ++a)
        af[a] = *reinterpret_cast<const v4i*>(As(buf) + (wm * (BM / 2) + a * 32 + li) * ROW + s * 32 + lh * 16);
#pragma unroll
      for (int b = 0; b < TN; ++b) bf[b] = *reinterpret_cast<const v4i*>(foot + fbase[b] + koff);
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[a], bf[b], acc[a][b], 0, 0, 0);
    }
  };

  {
    lstore(s0, 0);
    __syncthreads();  // footprint, first A stage, reciprocals and biases visible
    int i = 0;
    for (; i + 1 < n; i += 2) {
      if (i + 2 < n) gload(s0, i + 2);
      compute(0, i);
      lstore(s1, 1);
      __syncthreads();
      if (i + 3 < n) gload(s1, i + 3);
      compute(1, i + 1);
      if (i + 2 < n) lstore(s0, 0);
      __syncthreads();
    }
    if (i < n) compute(0, i);
  }

  // ---- epilogue (as conv_int8_kernel), staged in LDS over the footprint
  __syncthreads();
  const bool q8 = g.term > 100, relu = g.act == NHIP_ACT_RELU;
  const int qlo = relu ? 0 : -127;  // requantized ReLU: the saturation's lower bound
  float* tf = reinterpret_cast<float*>(dsm);
  int8_t* tq = dsm;
  auto dequant = [&](int a, int b, int r, int il) {
#pragma clang fp contract(off)
    float f = (float)acc[a][b][r];
    f = f * rb[il];
    return f + rb[BM + il];
  };
  if (q8) {
#pragma unroll
    NHIP_I8_EPI({
      tq[il * ES + jl] = quantize_i8(f, g.os, qlo);
    })
  } else {
#pragma unroll
    NHIP_I8_EPI(tf[il * ES + jl] = (relu && f < 0.0f) ? 0.0f : f)
  }
#undef NHIP_I8_EPI
  __syncthreads();
  constexpr int RUNS = BN / 16;
  for (int q = tid; q < BM * RUNS; q += kThreads) {
    const int il = q / RUNS, jl = (q % RUNS) * 16;
    const int i = i0 + il;
    if (i >= g.m || jl >= npx) continue;
    const int64_t o = ((int64_t)img * g.m + i) * g.OHW + (int64_t)oy0 * g.OW + jl;
    const bool whole = jl + 16 <= npx && (o & 15) == 0;
    if (q8) {
      int8_t* dst = static_cast<int8_t*>(g.out);
      if (whole) {
        *reinterpret_cast<v4i*>(dst + o) = *reinterpret_cast<const v4i*>(&tq[il * ES + jl]);
      } else {
        for (int e = 0; e < 16 && jl + e < npx; ++e) dst[o + e] = tq[il * ES + jl + e];
      }
    } else {
      float* dst = static_cast<float*>(g.out);
      if (whole) {
#pragma unroll
        for (int e = 0; e < 16; e += 4)
          *reinterpret_cast<v4f*>(dst + o + e) = *reinterpret_cast<const v4f*>(&tf[il * ES + jl + e]);
      } else {
        for (int e = 0; e < 16 && jl + e < npx; ++e) dst[o + e] = tf[il * ES + jl + e];
      }
    }
  }
}

// Register-weight variant.  Each wave keeps its 32 output channels' whole
// reduction (KS 32-byte k steps, 16 bytes per lane and step) in registers,
// loaded once at the start in k order from the fragment-order copy of the
// weights (each step one contiguous 1 KB load per wave, where the row-major
// weights would touch 32 cache lines), so no weight passes through LDS and
// the K loop has no barrier: the MFMAs of step s wait only for step s's
// weights.  The workgroup (4 waves, 128 channels) shares one footprint
// window of R whole output rows (at most 32*TN pixels) in LDS, as in
// conv_int8_fp_kernel.  The MFMA operands are swapped against the other
// kernels (A = pixels, B = weights), so the 32x32 result block is
// D[pixel][channel]: lane (c, h) holds channel c and, in registers 4g..4g+3,
// the four consecutive pixels 8g+4h .. 8g+4h+3.  The epilogue stores from
// registers with no LDS staging: two lane-half swaps give each lane 16
// consecutive int8 results of its channel (one 16-byte store), or four fp32
// results go out as one 16-byte vector.  Same arithmetic as the other
// kernels; the integer sums are exact in any order.
//
// FQ: the input arrives as fp32 NCHW and the window is filled by quantizing
// it on the way into LDS (no NHWC int8 image, no separate launch).  Window
// item i = (row fy, channel group c4 of 4, column group x4 of 4 pixels),
// x4 fastest, so 7 consecutive threads read one 112-byte channel row: four
// 16-byte loads (channels 4c4 .. 4c4 + 3), sixteen quantizations, and one
// 4-byte LDS word (4 channels) per pixel.  Rows outside the image and the
// window's columns outside it (the padding) are zero.  The items come in two
// batches of at most 3 per thread, the first in flight with the weights.
//
// KP = 2: eight waves, wave w holding channel block w % 4 and half w / 4 of
// the reduction (18 k steps, 72 weight registers), so that two waves share
// each SIMD and one's LDS reads and MFMA latency hide behind the other's
// MFMAs.  After the K loop each wave hands its partner (same channels, other
// half) the partial blocks the partner finishes through LDS (the window is
// free by then) and takes the ones it finishes: blocks b with b % 2 == half.
// Integer sums, so the result is the same in any order.
template <int KS, int TN, bool FQ = false, int KP = 1>
__global__ __launch_bounds__(kThreads * KP) void conv_int8_rw_kernel(Int8Args g) {
  constexpr int NT = kThreads * KP;  // threads of the workgroup
  constexpr int KSP = KS / KP;       // k steps per wave
  static_assert(KS % KP == 0 && TN % KP == 0, "whole k steps and pixel blocks per half");
  extern __shared__ __attribute__((aligned(16))) int8_t dsm[];
  int8_t* foot = dsm;
  int* koff_tab = reinterpret_cast<int*>(dsm + g.fp_bytes);  // [KS][2] LDS byte offsets of each k chunk
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cw = wave & 3, kp = KP == 1 ? 0 : __builtin_amdgcn_readfirstlane(wave >> 2);
  const int li = lane & 31, lh = lane >> 5;
  const int rgs = (g.OH + g.R - 1) / g.R;
  const int img = blockIdx.x / rgs, oy0 = (blockIdx.x % rgs) * g.R;
  const int ch0 = blockIdx.y * 128 + cw * 32;
  const int npx = min(g.R, g.OH - oy0) * g.OW;

  // ---- footprint loads first (at most 8 per thread, checked on the host),
  // then the weights in k order, then the epilogue scalars; nothing waits yet
  const int cpp = g.c_pad / 16;
  const int iy_base = oy0 * g.sh - g.pt;
  v4i fv[FQ ? 1 : 8];
  int fdst[FQ ? 1 : 8];
  // FQ items: 16 fp32 values (4 channels x 4 pixels) and the LDS byte
  // offset of the first pixel's 4-channel word (-1: none, -2: zero row)
  constexpr int kQB = 3;
  v4f qv[FQ ? kQB : 1][4];
  int qdst[FQ ? kQB : 1];
  const int c4n = g.C / 4, xgn = g.W / 4;
  const int items = FQ ? c4n * g.FH * xgn : 0;
  auto fq_load = [&](int batch) {
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(g.xf, g.xf_bytes);
#pragma unroll
    for (int q = 0; q < kQB; ++q) {
      const int i = (batch * kQB + q) * NT + tid;
      const int rest = fdiv(i, g.xg_div), x4 = i - rest * xgn;
      const int fy = fdiv(rest, g.c4_div), c4 = rest - fy * c4n;
      const int iy = iy_base + fy;
      const bool row_in = (unsigned)iy < (unsigned)g.H;
      qdst[q] = i < items ? (row_in ? (fy * g.FW + 4 * x4 + g.pl) * g.FS + 4 * c4 : -2) : -1;
      const uint32_t off = ((uint32_t)((img * g.C + 4 * c4) * g.H + iy) * g.W + 4 * x4) * 4;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        qv[q][j] = __builtin_bit_cast(
            v4f, buf_load_b128(xr, i < items && row_in ? off + (uint32_t)(j * g.H * g.W * 4) : kBufOOB));
    }
  };
  auto fq_store = [&](int batch) {
#pragma unroll
    for (int q = 0; q < kQB; ++q) {
      if (qdst[q] == -1) continue;
      int w4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        w4[e] = (int)pack_i8x4(quantize_q(qv[q][0][e], g.in_scale), quantize_q(qv[q][1][e], g.in_scale),
                               quantize_q(qv[q][2][e], g.in_scale), quantize_q(qv[q][3][e], g.in_scale));
      if (qdst[q] == -2) {
        // a row outside the image: its item's pixels and channels are zero
        const int i = (batch * kQB + q) * NT + tid;
        const int rest = fdiv(i, g.xg_div), x4 = i - rest * xgn;
        const int fy = fdiv(rest, g.c4_div), c4 = rest - fy * c4n;
        const int d0 = (fy * g.FW + 4 * x4 + g.pl) * g.FS + 4 * c4;
#pragma unroll
        for (int e = 0; e < 4; ++e) *reinterpret_cast<int*>(foot + d0 + e * g.FS) = 0;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) *reinterpret_cast<int*>(foot + qdst[q] + e * g.FS) = w4[e];
      }
    }
  };
  if constexpr (FQ) {
    fq_load(0);
  } else {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(g.x, g.x_bytes);
    const int total = g.FH * g.FW * cpp;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int e = q * NT + tid;
      const int pix = fdiv(e, g.cpp_div), ch = e - pix * cpp;
      const int fy = fdiv(pix, g.fw_div), fx = pix - fy * g.FW;
      const int iy = iy_base + fy, ix = fx - g.pl;
      const bool in = e < total && (unsigned)iy < (unsigned)g.H && (unsigned)ix < (unsigned)g.W;
      fv[q] = __builtin_bit_cast(
          v4i, buf_load_b128(rs, in ? (uint32_t)(((img * g.H + iy) * g.W + ix) * g.c_pad + ch * 16) : kBufOOB));
      // 24-bit products (window < 2^24 bytes) keep this 32-bit: a 64-bit
      // multiply-add here pairs a register with a weight load's destination
      // and forces an early wait for it
      fdst[q] = e < total ? (int)__umul24(pix, g.FS) + ch * 16 : -1;
    }
  }
  v4i wr[KSP];
  {
    // fragment order: this wave's k step s is 1 KB at ((ch0/32)*KS + s) KB
    const int8_t* wp = g.w + ((int64_t)(ch0 / 32) * KS + kp * KSP) * 1024 + lane * 16;
#pragma unroll
    for (int s = 0; s < KSP; ++s) wr[s] = *reinterpret_cast<const v4i*>(wp + s * 1024);
  }
  const float rc = g.recip[ch0 + li], bs = g.bias[ch0 + li];
  // k chunk q (16 bytes at reduction index 16q, order (kh, kw, c)) -> its
  // byte offset in the window; computed, not loaded, so that nothing here
  // waits for the loads in flight
  if (tid < 2 * KS) {
    const int kidx = tid * 16, r = kidx / g.c_pad, c0 = kidx - r * g.c_pad;
    const int kh = r / g.KW, kw = r - kh * g.KW;
    // K padding (past kred): the weights there are zero, any window byte will do
    koff_tab[tid] = kidx < g.kred ? (kh * g.dh * g.FW + kw * g.dw) * g.FS + c0 : 0;
  }
  if constexpr (FQ) {
    // the window's columns outside the image (left and right padding): zero
    const int nh = g.FW - g.W, hz = g.FH * nh * cpp;
    for (int e = tid; e < hz; e += NT) {
      const int pos = e / cpp, ch = e - pos * cpp;
      const int fy = pos / nh, h = pos - fy * nh;
      const int fx = h < g.pl ? h : g.W + h;
      *reinterpret_cast<v4i*>(foot + (fy * g.FW + fx) * g.FS + ch * 16) = v4i{0, 0, 0, 0};
    }
    fq_store(0);
    // the second batch only where the window has more items than the first
    // covers (not at 128 channels x 6 rows x 28 columns: 1344 items, 1536
    // slots); run unconditionally, its stores wait for every load in flight,
    // the weights included, before the barrier
    if (items > kQB * NT) {
      fq_load(1);
      fq_store(1);
    }
  } else {
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (fdst[q] >= 0) *reinterpret_cast<v4i*>(foot + fdst[q]) = fv[q];
  }

  // per-lane window origin (bytes) of each of the wave's pixel rows of D
  int fbase[TN];
#pragma unroll
  for (int b = 0; b < TN; ++b) {
    const int pc = min(b * 32 + li, npx - 1);
    const int py = pc / g.OW, px = pc - py * g.OW;
    fbase[b] = (py * g.sh * g.FW + px * g.sw) * g.FS;
  }
  __syncthreads();  // footprint and k offsets visible

  v16i acc[TN];
#pragma unroll
  for (int b = 0; b < TN; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[b][r] = 0;
#pragma unroll
  for (int s = 0; s < KSP; ++s) {
    const int koff = koff_tab[(kp * KSP + s) * 2 + lh];
    v4i xf[TN];
#pragma unroll
    for (int b = 0; b < TN; ++b) xf[b] = *reinterpret_cast<const v4i*>(foot + fbase[b] + koff);
#pragma unroll
    for (int b = 0; b < TN; ++b) acc[b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xf[b], wr[s], acc[b], 0, 0, 0);
  }
  if constexpr (KP == 2) {
    // exchange through LDS, 16-byte records [channel block][pixel block]
    // [register quad][lane] (64 KB for TN = 4): every wave done with the
    // window first
    v4i* xch = reinterpret_cast<v4i*>(dsm);
    __syncthreads();
#pragma unroll
    for (int b = 0; b < TN; ++b)
      if (b % 2 != kp)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          xch[((cw * TN + b) * 4 + r4) * 64 + lane] =
              v4i{acc[b][4 * r4], acc[b][4 * r4 + 1], acc[b][4 * r4 + 2], acc[b][4 * r4 + 3]};
    __syncthreads();
#pragma unroll
    for (int b = 0; b < TN; ++b)
      if (b % 2 == kp)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const v4i v = xch[((cw * TN + b) * 4 + r4) * 64 + lane];
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[b][4 * r4 + e] += v[e];
        }
  }

  // ---- epilogue from registers: channel ch0 + li, pixels 8g + 4lh + q
  const bool q8 = g.term > 100, relu = g.act == NHIP_ACT_RELU;
  const int qlo = relu ? 0 : -127;  // requantized ReLU: the saturation's lower bound
  const int ch = ch0 + li;
  const bool chan_ok = ch < g.m;
  const int es = q8 ? 1 : 4;
  const uint32_t base = (uint32_t)((((int64_t)img * g.m + ch) * g.OHW + (int64_t)oy0 * g.OW) * es);
  const __amdgpu_buffer_rsrc_t orr = make_rsrc(g.out, g.out_bytes);
  auto dequant = [&](int b, int r) {
#pragma clang fp contract(off)
    float v = (float)acc[b][r];
    v = v * rc;
    return v + bs;
  };
#pragma unroll
  for (int b = 0; b < TN; ++b) {
    if (KP == 2 && b % 2 != kp) continue;  // the partner's block
    if (q8) {
      uint32_t wd[4];  // pixels 8g + 4lh .. + 3 as bytes
#pragma unroll
      for (int gi = 0; gi < 4; ++gi)
        wd[gi] = pack_i8x4(quantize_q(dequant(b, 4 * gi), g.os, qlo), quantize_q(dequant(b, 4 * gi + 1), g.os, qlo),
                           quantize_q(dequant(b, 4 * gi + 2), g.os, qlo), quantize_q(dequant(b, 4 * gi + 3), g.os, qlo));
      if (g.vec == 2) {
        // swap words between lane halves so that lane (c, h) holds pixels
        // 16h .. 16h + 15 of the block: one 16-byte store per lane
        const auto s02 = __builtin_amdgcn_permlane32_swap(wd[0], wd[2], false, false);
        const auto s13 = __builtin_amdgcn_permlane32_swap(wd[1], wd[3], false, false);
        const v4i y{(int)s02[0], (int)s02[1], (int)s13[0], (int)s13[1]};
        const int p0 = b * 32 + 16 * lh;
        __builtin_amdgcn_raw_buffer_store_b128(y, orr, chan_ok && p0 < npx ? base + p0 : kBufOOB, 0, 0);
      } else if (g.vec == 1) {
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const int p0 = b * 32 + 8 * gi + 4 * lh;
          __builtin_amdgcn_raw_buffer_store_b32((int)wd[gi], orr, chan_ok && p0 < npx ? base + p0 : kBufOOB, 0, 0);
        }
      } else {
#pragma unroll
        for (int gi = 0; gi < 4; ++gi)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int p = b * 32 + 8 * gi + 4 * lh + q;
            __builtin_amdgcn_raw_buffer_store_b8((char)(wd[gi] >> (8 * q)), orr,
                                                 chan_ok && p < npx ? base + p : kBufOOB, 0, 0);
          }
      }
    } else {
#pragma unroll
      for (int gi = 0; gi < 4; ++gi) {
        const int p0 = b * 32 + 8 * gi + 4 * lh;
        float f[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          f[q] = dequant(b, 4 * gi + q);
          f[q] = (relu && f[q] < 0.0f) ? 0.0f : f[q];
        }
        if (g.vec >= 1) {
          const v4i y{__float_as_int(f[0]), __float_as_int(f[1]), __float_as_int(f[2]), __float_as_int(f[3])};
          __builtin_amdgcn_raw_buffer_store_b128(y, orr, chan_ok && p0 < npx ? base + 4 * p0 : kBufOOB, 0, 0);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(f[q]), orr,
                                                  chan_ok && p0 + q < npx ? base + 4 * (p0 + q) : kBufOOB, 0, 0);
        }
      }
    }
  }
}

}  // namespace

uint64_t conv_int8_workspace(const nhip_conv_plan* p, int n, int h, int w) {
  return (uint64_t)n * h * w * p->c_pad;
}

int launch_conv_int8(const nhip_conv_plan* p, const void* in, int in_is_i8,
                     void* out, int n, int h, int w, int oh, int ow, void* ws,
                     uint64_t ws_bytes, hipStream_t s) {
  const uint64_t need = conv_int8_workspace(p, n, h, w);
  if (ws == nullptr || ws_bytes < need)
    return fail(NHIP_STATUS_OUTPUT_CAPACITY_INSUFFICIENT,
                "int8 conv: workspace of " + std::to_string(need) + " bytes required");
  int8_t* xq = static_cast<int8_t*>(ws);
  auto quantize = [&]() {
    NHIP_LAUNCH("quantize_nchw_to_nhwc", quantize_nchw_to_nhwc,
                dim3((unsigned)ceil_div((int64_t)h * w, 64), (unsigned)ceil_div(p->c_pad, 64), n), dim3(kThreads), 0, s,
                in, in_is_i8, xq, p->g.c, h * w, p->c_pad, p->input_scale);
    return check_launch("quantize_nchw_to_nhwc");
  };

  Int8Args g{};
  g.w = p->weight_i8;
  g.kred_pad = p->kred_pad;
  g.m = p->g.k;
  g.x = xq;
  g.x_bytes = (uint32_t)need;
  g.H = h;
  g.W = w;
  g.c_pad = p->c_pad;
  g.OW = ow;
  g.OHW = oh * ow;
  g.sh = p->g.sh;
  g.sw = p->g.sw;
  g.pt = p->g.pt;
  g.pl = p->g.pl;
  g.npix = n * oh * ow;
  g.ktab = p->ktab;
  g.recip = p->recip;
  g.bias = p->bias;
  g.os = p->output_scale;
  g.term = p->scale_term;
  g.act = p->g.act;
  g.out = out;
  const int64_t out_bytes = (int64_t)n * p->g.k * oh * ow * (p->scale_term > 100 ? 1 : 4);
  g.out_bytes = (uint32_t)std::min<int64_t>(out_bytes, INT32_MAX);
  // Register-weight kernel: a reduction of 36 k steps (1152 bytes: 128
  // channels at 3x3), whole 128-channel blocks and a footprint window of at
  // most 2048 16-byte chunks.  NHIP_INT8_RW=0 turns it off, =2 takes two
  // 32-pixel blocks per wave instead of four (tuning and comparison
  // switches).
  {
    const int mode = setting_int("NHIP_INT8_RW", 1);
    const int tn = mode == 2 ? 2 : 4;
    const int R = ow > 0 ? std::min(32 * tn / ow, oh) : 0;
    constexpr int KS = kRwKred / 32;
    if (mode != 0 && R >= 1 && p->weight_i8_frag != nullptr && p->m_pad % 128 == 0 && p->kred_pad == kRwKred &&
        out_bytes < INT32_MAX) {
      Int8Args r = g;
      r.w = p->weight_i8_frag;
      r.OH = oh;
      r.R = R;
      r.FH = (R - 1) * p->g.sh + (p->g.kh - 1) * p->g.dh + 1;
      r.FW = (ow - 1) * p->g.sw + (p->g.kw - 1) * p->g.dw + 1;
      r.FS = p->c_pad + 16;
      r.fp_bytes = (int)round_up((int64_t)r.FH * r.FW * r.FS, 16);
      r.cpp_div = fast_div((uint32_t)(p->c_pad / 16));
      r.fw_div = fast_div((uint32_t)r.FW);
      r.kred = p->kred;
      r.KW = p->g.kw;
      r.dh = p->g.dh;
      r.dw = p->g.dw;
      // Store mode: whole 16-pixel int8 runs (16-byte aligned and all valid
      // or all past the workgroup's pixels) when OHW and R*OW are multiples
      // of 16; whole 4-pixel groups when they are multiples of 4; else
      // single elements.
      {
        const uintptr_t oa = reinterpret_cast<uintptr_t>(out);
        const bool q8 = p->scale_term > 100;
        const int64_t run = (int64_t)R * ow, ohw = (int64_t)oh * ow;
        if (q8 && ohw % 16 == 0 && run % 16 == 0 && oa % 16 == 0)
          r.vec = 2;
        else if (ohw % 4 == 0 && run % 4 == 0 && oa % (q8 ? 4 : 16) == 0)
          r.vec = 1;
        else
          r.vec = 0;
      }
      const int64_t chunks = (int64_t)r.FH * r.FW * (p->c_pad / 16);
      const int64_t lds = r.fp_bytes + 2 * KS * 4;
      // Quantization fused into the window fill: fp32 input with whole
      // 4-pixel column groups and 4-channel groups (16-byte loads), the
      // window covering every input column, at most 6 items per thread
      const int64_t fq_items = (int64_t)(p->g.c / 4) * r.FH * (w / 4);
      const bool fq = !in_is_i8 && setting_int("NHIP_INT8_FUSED_QUANT", 1) != 0 && tn == 4 && w % 4 == 0 &&
                      p->g.c % 4 == 0 && (reinterpret_cast<uintptr_t>(in) & 15) == 0 && p->g.pl + w <= r.FW &&
                      fq_items <= 6 * kThreads && (int64_t)n * p->g.c * h * w * 4 < INT32_MAX;
      if (chunks <= 8 * kThreads && lds <= 64 * 1024) {
        const dim3 grid((unsigned)(n * ceil_div(oh, R)), (unsigned)(p->m_pad / 128));
        if (fq) {
          r.xf = static_cast<const float*>(in);
          r.xf_bytes = (uint32_t)((int64_t)n * p->g.c * h * w * 4);
          r.C = p->g.c;
          r.in_scale = p->input_scale;
          r.xg_div = fast_div((uint32_t)(w / 4));
          r.c4_div = fast_div((uint32_t)(p->g.c / 4));
          // NHIP_INT8_KSPLIT=1: four waves, each with the whole reduction
          if (setting_int("NHIP_INT8_KSPLIT", 2) == 2) {
            const auto kernel = conv_int8_rw_kernel<KS, 4, true, 2>;
            const int lds2 = (int)std::max<int64_t>(lds, 4 * 4 * 16 * 64 * 4);  // + the exchange
            NHIP_TRY(ensure_dynamic_lds(reinterpret_cast<const void*>(kernel), lds2));
            NHIP_LAUNCH("conv_int8_rw_fq", kernel, grid, dim3(2 * kThreads), (unsigned)lds2, s, r);
            return check_launch("conv_int8_rw_fq");
          }
          NHIP_LAUNCH("conv_int8_rw_fq", (conv_int8_rw_kernel<KS, 4, true>), grid, dim3(kThreads), (unsigned)lds, s, r);
          return check_launch("conv_int8_rw_fq");
        }
        NHIP_TRY(quantize());
        if (tn == 4) {
          NHIP_LAUNCH("conv_int8_rw", (conv_int8_rw_kernel<KS, 4>), grid, dim3(kThreads), (unsigned)lds, s, r);
        } else {
          NHIP_LAUNCH("conv_int8_rw", (conv_int8_rw_kernel<KS, 2>), grid, dim3(kThreads), (unsigned)lds, s, r);
        }
        return check_launch("conv_int8_rw");
      }
    }
  }
  // The other kernels read the NHWC int8 image.
  NHIP_TRY(quantize());
  // Footprint kernel when a workgroup's input window fits in LDS (whole rows
  // of at most 128 output pixels); NHIP_INT8_FOOTPRINT=0 turns it off (a
  // tuning and comparison switch).
  {
    const bool allowed = setting_int("NHIP_INT8_FOOTPRINT", 1) != 0;
    const int R = ow > 0 ? 128 / ow : 0;
    const int max_dy = (p->g.kh - 1) * p->g.dh, max_dx = (p->g.kw - 1) * p->g.dw;
    if (allowed && R >= 1 && p->kred_pad % 128 == 0) {
      g.OH = oh;
      g.R = std::min(R, oh);
      g.FH = (g.R - 1) * p->g.sh + max_dy + 1;
      g.FW = (ow - 1) * p->g.sw + max_dx + 1;
      g.FS = p->c_pad + 16;
      g.fp_bytes = (int)round_up((int64_t)g.FH * g.FW * g.FS, 16);
      g.cpp_div = fast_div((uint32_t)(p->c_pad / 16));
      g.fw_div = fast_div((uint32_t)g.FW);
      // 64 output channels per workgroup (a 128-channel block's epilogue
      // staging alone would take 72 KB and leave one workgroup per CU)
      const int bm = 64;
      // K stage: the widest of 384 / 192 / 128 bytes that divides the
      // reduction (fewer stages: fewer global-load round trips and barriers
      // per workgroup; 32x128x28x28 -> 128 channels: 3 stages of 384 bytes, 16.3 against 17.2 us
      // with 128-byte stages); NHIP_INT8_FP_BK overrides (tuning switch,
      // ignored when invalid).
      // operands (footprint + two weight stages) or the epilogue's staging,
      // then bm reciprocals and bm biases past both
      auto rb_at = [&](int bk) {
        const int64_t oper = (int64_t)g.fp_bytes + 2LL * bm * (bk + 16);
        const int64_t epi = (int64_t)bm * (128 + 16) * 4;
        return round_up(std::max(oper, epi), 16);
      };
      auto lds_for = [&](int bk) { return rb_at(bk) + 2LL * bm * 4; };
      // Eligible when the window fits beside 128-byte stages in 64 KB; wider
      // stages may take up to 80 KB (still two workgroups per CU).
      constexpr int64_t kMaxLds = 80 * 1024;
      int bk = 128;
      for (int c : {384, 192})
        if (p->kred_pad % c == 0 && lds_for(c) <= kMaxLds) {
          bk = c;
          break;
        }
      if (setting("NHIP_INT8_FP_BK")) {
        const int c = setting_int("NHIP_INT8_FP_BK", 0);
        if ((c == 128 || c == 192 || c == 384) && p->kred_pad % c == 0 && lds_for(c) <= kMaxLds) bk = c;
      }
      const int64_t lds = lds_for(bk);
      g.rb_off = (int)rb_at(bk);
      if (lds_for(128) <= 64 * 1024) {
        const dim3 grid((unsigned)(n * ceil_div(oh, g.R)), (unsigned)(p->m_pad / bm));
#define NHIP_FP_CASE(BM_, BK_)                                                                                   \
  if (bm == BM_ && bk == BK_) {                                                                                 \
    const auto kernel = conv_int8_fp_kernel<BM_, BK_>;                                                          \
    NHIP_TRY(ensure_dynamic_lds(reinterpret_cast<const void*>(kernel), (int)kMaxLds));                          \
    NHIP_LAUNCH("conv_int8_fp", kernel, grid, dim3(kThreads), (unsigned)lds, s, g);                              \
    return check_launch("conv_int8_fp");                                                                        \
  }
        NHIP_FP_CASE(64, 128)
        NHIP_FP_CASE(64, 192)
        NHIP_FP_CASE(64, 384)
#undef NHIP_FP_CASE
      }
    }
  }
  // Tile shape: NHIP_INT8_TILE="bm,bn,bk" overrides (tuning switch, ignored
  // when not valid for the plan).
  int bm = p->m_pad % 128 == 0 ? 128 : 64, bn = 64, bk = 128;
  if (const char* env = setting("NHIP_INT8_TILE")) {
    int a = 0, b = 0, c = 0;
    if (std::sscanf(env, "%d,%d,%d", &a, &b, &c) == 3 && (a == 64 || a == 128) && (b == 64 || b == 128) &&
        (c == 128 || c == 256) && p->m_pad % a == 0 && p->kred_pad % c == 0) {
      bm = a;
      bn = b;
      bk = c;
    }
  }
  const dim3 grid((unsigned)ceil_div(g.npix, bn), (unsigned)(p->m_pad / bm));
#define NHIP_INT8_CASE(BM_, BN_, BK_)                                                                     \
  if (bm == BM_ && bn == BN_ && bk == BK_) {                                                              \
    NHIP_LAUNCH("conv_int8<" #BM_ "," #BN_ "," #BK_ ">", (conv_int8_kernel<BM_, BN_, BK_>), grid, dim3(kThreads), \
                0, s, g);                                                                                 \
    return check_launch("conv_int8");                                                                     \
  }
  NHIP_INT8_CASE(64, 64, 128)
  NHIP_INT8_CASE(128, 64, 128)
  NHIP_INT8_CASE(64, 128, 128)
  NHIP_INT8_CASE(128, 128, 128)
  NHIP_INT8_CASE(64, 64, 256)
  NHIP_INT8_CASE(128, 64, 256)
  NHIP_INT8_CASE(64, 128, 256)
#undef NHIP_INT8_CASE
  return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "int8 conv: bad tile config");
}

}  // namespace nhip
