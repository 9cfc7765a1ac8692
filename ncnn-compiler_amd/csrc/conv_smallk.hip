// fp32 convolution with a short reduction and few output channels
// (C*kh*kw <= 32, K <= 32): the stem of MobileNetV2-style networks, 3 -> 32
// channels, 3x3, stride 2 (ncnn Convolution, lowered by the reference
// through tosa.conv2d: NCNNToTosa.cpp:1316-1529).
//
// Such a layer moves far more bytes than it computes (the 224x224 stem at
// batch 32 writes 51 MB for 0.7 GFLOP), and its GEMM is one MFMA block high:
// M = 32 output channels, K = the whole reduction.  A wave takes 32 output
// pixels at a time as one v_mfma_f32_32x32x2_f32 block: A = the weights (the
// lane's 8 or 16 values, loaded once), B = the input taps gathered straight
// from memory (lane (n, h) loads tap 2s + h of pixel n for step s; padding
// and positions past the image read zero through out-of-range buffer
// offsets), and the next block's gathers are in flight while the current
// block multiplies and is written.  Register r of lane l holds output
// channel 8(r/4) + 4(l/32) + r%4 of pixel l%32, so each store instruction
// writes two 128-byte runs of one channel plane.
#include <algorithm>

#include "nhip_internal.h"

namespace nhip {
namespace {

constexpr int kThreads = 256;

struct SmallkArgs {
  const float* w;         // [m_pad][kred_pad], k = (c, kh, kw); zero past the reduction and past K
  const int* ktab;        // reduction index -> c << 16 | dy << 8 | dx (c = 0x7fff past the reduction)
  const float* bias;      // [m_pad], m_pad >= 64, zero past K
  const float* residual;  // [N][K][OH][OW] when RES
  const float* x;         // [N][C][H][W]
  uint32_t x_bytes;       // < 2^31
  float* out;             // [N][K][OH][OW]
  uint32_t out_bytes;     // < 2^31
  int K, C, H, W, OW, OHW, sh, sw, pt, pl, ldw;
  int ymax, xmax;         // (kh - 1)*dh, (kw - 1)*dw: the window's last row and column
  FastDiv ohw_div, ow_div;
  int npix;               // N*OH*OW
  int nblk;               // 32-pixel blocks
};

template <int ACT>
__device__ __forceinline__ float smallk_act(float v) {
  if constexpr (ACT == NHIP_ACT_RELU) return v < 0.f ? 0.f : v;
  if constexpr (ACT == NHIP_ACT_SIGMOID) return 1.0f / (1.0f + __expf(-v));
  return v;
}

template <int STEPS, int ACT, bool RES>  // STEPS: MFMA k-steps, the padded reduction / 2
__global__ __launch_bounds__(kThreads) void conv_smallk_kernel(SmallkArgs a) {
  const int lane = threadIdx.x & 63, li = lane & 31, lh = lane >> 5;
  const int gw = __builtin_amdgcn_readfirstlane((int)((blockIdx.x * kThreads + threadIdx.x) >> 6));  // global wave
  const int nw = (int)(gridDim.x * (kThreads / 64));
  if (gw >= a.nblk) return;  // uniform over the wave; no barrier below

  // A operand of step s: W[k = l%32][2s + l/32]; the lane's tap 2s + l/32
  // as an element offset from the window's corner (c*H + dy)*W + dx and its
  // row / column offsets; a tap past the reduction gets the offset 2^29
  // (corner + 2^29 is past the input, < 2^29 elements, without wrapping 32
  // bits as a byte offset) and the row offset 2^30 (it always fails the row
  // check), so it reads zero either way; the bias of the lane's 16 output
  // channels (m_pad >= 64 entries)
  float wa[STEPS], bias[16];
  int toff[STEPS], tdy[STEPS], tdx[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    wa[s] = a.w[li * a.ldw + 2 * s + lh];
    const int t = a.ktab[2 * s + lh];
    const int c = t >> 16, dy = (t >> 8) & 255, dx = t & 255;
    const bool live = c < a.C;
    toff[s] = live ? (c * a.H + dy) * a.W + dx : (1 << 29);
    tdy[s] = live ? dy : (1 << 30);
    tdx[s] = dx;
    // opaque to the optimizer: otherwise it folds the offset back into the
    // per-block address arithmetic, two integer multiplies per tap
    asm volatile("" : "+v"(toff[s]), "+v"(tdy[s]), "+v"(tdx[s]));
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) bias[r] = a.bias[8 * (r >> 2) + 4 * lh + (r & 3)];
  const uint32_t plane_bytes = (uint32_t)a.OHW * 4u;
  const uint32_t lane_off = (uint32_t)(4 * lh) * plane_bytes;  // channel 4(l/32)
  const int k_left = a.K - 4 * lh;                             // channels m < K: 8(r/4) + r%4 < k_left
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t orr = make_rsrc(a.out, a.out_bytes);
  const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.residual, RES ? a.out_bytes : 0u);

  // pixel l%32 of a block: image and position in the image's plane
  struct Px {
    int img, q;
    bool ok;
  };
  auto locate = [&](int blk) {
    Px px;
    const int pix = blk * 32 + li;
    px.ok = pix < a.npix;
    const int pp = px.ok ? pix : 0;
    px.img = fdiv(pp, a.ohw_div);
    px.q = pp - px.img * a.OHW;
    return px;
  };
  // the lane's taps of its pixel (zero for padding and past the pixels);
  // when every pixel of the block has its whole window inside the image (all
  // but the border blocks) the taps need no bounds check
  auto gather = [&](const Px& px, float (&v)[STEPS]) {
    const int oy = fdiv(px.q, a.ow_div), ox = px.q - oy * a.OW;
    const int iy0 = oy * a.sh - a.pt, ix0 = ox * a.sw - a.pl;
    const int corner = (px.img * a.C * a.H + iy0) * a.W + ix0;  // element (img, 0, iy0, ix0)
    const bool interior = px.ok && iy0 >= 0 && iy0 + a.ymax < a.H && ix0 >= 0 && ix0 + a.xmax < a.W;
    if (__all(interior)) {
#pragma unroll
      for (int s = 0; s < STEPS; ++s) v[s] = buf_load_f32(xr, (uint32_t)(corner + toff[s]) * 4u);
    } else {
      const int ylim = px.ok ? a.H : 0;  // no row passes past the pixels
#pragma unroll
      for (int s = 0; s < STEPS; ++s) {
        const bool in = (unsigned)(iy0 + tdy[s]) < (unsigned)ylim && (unsigned)(ix0 + tdx[s]) < (unsigned)a.W;
        v[s] = buf_load_f32(xr, in ? (uint32_t)(corner + toff[s]) * 4u : kBufOOB);
      }
    }
  };
  // out = act(sum + bias (+ residual)); channels past K and pixels past the
  // last one get out-of-range offsets (their loads read zero, their stores
  // are dropped), so the epilogue has no branch
  auto finish = [&](int blk, const Px& px, const float (&v)[STEPS]) {
    v16f acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(wa[s], v[s], acc, 0, 0, 0);
    // channel m = 8(r/4) + r%4 + 4(l/32): the lane's part of the offset and
    // of the channel bound are per lane, the register's part a multiple of
    // the plane size
    const uint32_t base = (uint32_t)((px.img * a.K) * a.OHW + px.q) * 4u + lane_off;
    if (a.K == 32 && (blk + 1) * 32 <= a.npix) {
      // every channel and pixel present: the register's part of the offset
      // goes in the instructions' scalar offset
      float res[16];
#pragma unroll
      for (int r = 0; r < 16; ++r)
        res[r] = RES ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                           rr, base, (8 * (r >> 2) + (r & 3)) * plane_bytes, 0))
                     : 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float y = acc[r] + bias[r];
        if constexpr (RES) y += res[r];
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(smallk_act<ACT>(y)), orr, base,
                                              (8 * (r >> 2) + (r & 3)) * plane_bytes, 0);
      }
      return;
    }
    const int mlim = px.ok ? k_left : 0;
    uint32_t off[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int mr = 8 * (r >> 2) + (r & 3);
      off[r] = mr < mlim ? base + (uint32_t)mr * plane_bytes : kBufOOB;
    }
    float res[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) res[r] = RES ? buf_load_f32(rr, off[r]) : 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float y = acc[r] + bias[r];
      if constexpr (RES) y += res[r];
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(smallk_act<ACT>(y)), orr, off[r], 0, 0);
    }
  };

  // Blocks gw, gw + nw, ...: two register buffers, the next block's gathers
  // issued before the current block's MFMAs and stores.
  float b0[STEPS], b1[STEPS];
  int blk = gw;
  Px p0 = locate(blk), p1;
  gather(p0, b0);
  while (true) {
    p1 = locate(blk + nw);
    gather(p1, b1);
    finish(blk, p0, b0);
    blk += nw;
    if (blk >= a.nblk) break;
    p0 = locate(blk + nw);
    gather(p0, b0);
    finish(blk, p1, b1);
    blk += nw;
    if (blk >= a.nblk) break;
  }
}

template <int STEPS>
void launch_steps(const SmallkArgs& a, int act, dim3 grid, hipStream_t s) {
  const bool res = a.residual != nullptr;
#define NHIP_SMALLK(ACT_, RES_) \
  NHIP_LAUNCH("conv_smallk_f32", (conv_smallk_kernel<STEPS, ACT_, RES_>), grid, dim3(kThreads), 0, s, a)
  if (act == NHIP_ACT_RELU) {
    if (res) NHIP_SMALLK(NHIP_ACT_RELU, true); else NHIP_SMALLK(NHIP_ACT_RELU, false);
  } else if (act == NHIP_ACT_SIGMOID) {
    if (res) NHIP_SMALLK(NHIP_ACT_SIGMOID, true); else NHIP_SMALLK(NHIP_ACT_SIGMOID, false);
  } else {
    if (res) NHIP_SMALLK(NHIP_ACT_NONE, true); else NHIP_SMALLK(NHIP_ACT_NONE, false);
  }
#undef NHIP_SMALLK
}

}  // namespace

// Shapes taken: a plain (groups 1) fp32 convolution on the implicit-GEMM
// plan whose reduction is at most 32 long with at most 32 output channels,
// except 1x1 stride-1 unpadded ones (the pointwise kernels' shapes), and
// 32-bit buffer offsets; by default only from four 32-pixel blocks per CU
// (measured on the 224x224 stem: 26.4 against 35.7 us at batch 32, 11.1
// against 13.1 at batch 8, equal at batch 2, 9.7 against 8.6 us for one
// image, where the implicit GEMM's smaller tiles spread better).
// NHIP_CONV_SMALLK=0 turns it off, =2 takes it for every shape it supports
// (tests).
bool smallk_supported(const nhip_conv_plan* p, int n, int h, int w, int oh, int ow) {
  const ConvGeom& g = p->g;
  if (p->kind != PlanKind::ConvF32 || p->algorithm != NHIP_CONV_ALGO_IMPLICIT_GEMM) return false;
  const int mode = setting_int("NHIP_CONV_SMALLK", 1);
  if (mode == 0) return false;
  if (p->kred > 32 || p->kred_pad > 32 || g.k > 32) return false;
  if (g.kh == 1 && g.kw == 1 && g.sh == 1 && g.sw == 1 && !g.pt && !g.pb && !g.pl && !g.pr) return false;
  const int64_t xb = (int64_t)n * g.c * h * w * 4, ob = (int64_t)n * g.k * oh * ow * 4;
  if (!(xb < (int64_t(1) << 31) && ob < (int64_t(1) << 31) && oh > 0 && ow > 0)) return false;
  return mode == 2 || ceil_div((int64_t)n * oh * ow, 32) >= 4LL * cu_count();
}

int launch_conv_smallk(const nhip_conv_plan* p, const float* in, const float* residual, float* out, int n, int h,
                       int w, int oh, int ow, hipStream_t s) {
  if (!smallk_supported(p, n, h, w, oh, ow))
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "short-reduction conv: unsupported shape");
  SmallkArgs a{};
  a.w = p->weight;
  a.ktab = p->ktab;
  a.bias = p->bias;
  a.residual = residual;
  a.x = in;
  a.x_bytes = (uint32_t)((int64_t)n * p->g.c * h * w * 4);
  a.out = out;
  a.out_bytes = (uint32_t)((int64_t)n * p->g.k * oh * ow * 4);
  a.K = p->g.k;
  a.C = p->g.c;
  a.H = h;
  a.W = w;
  a.OW = ow;
  a.OHW = oh * ow;
  a.ohw_div = fast_div((uint32_t)a.OHW);
  a.ow_div = fast_div((uint32_t)ow);
  a.ymax = (p->g.kh - 1) * p->g.dh;
  a.xmax = (p->g.kw - 1) * p->g.dw;
  a.sh = p->g.sh;
  a.sw = p->g.sw;
  a.pt = p->g.pt;
  a.pl = p->g.pl;
  a.ldw = p->kred_pad;
  a.npix = n * oh * ow;
  a.nblk = (int)ceil_div(a.npix, 32);
  if (a.npix == 0) return ok();
  // Two waves per SIMD (grid-stride over the blocks) where each still gets
  // two blocks or more, else one; fewer only when there are fewer blocks.
  // The 224x224 stem at batch 32 (12544 blocks) in the MobileNetV2 graph:
  // 2048 waves 27.6-28.0 us, 1024 31.0-31.3 us, 3072 35.9-36.3 us (four or
  // five blocks a wave); standalone, 1024 waves took 23.2 us, 1568 (two on
  // half of the SIMDs) 26.0 us, 768 29.7 us.  Two-block-deep and
  // three-block-deep gather rings were 1.2 and 2.3 us slower than the
  // one-block-ahead pair of buffers kept here.
  const int per_cu = a.nblk >= 16LL * cu_count() ? 8 : 4;
  const int64_t waves = std::min<int64_t>(a.nblk, (int64_t)per_cu * cu_count());
  const dim3 grid((unsigned)ceil_div(waves, kThreads / 64));
  if (p->kred_pad <= 16) launch_steps<8>(a, p->g.act, grid, s);
  else launch_steps<16>(a, p->g.act, grid, s);
  return check_launch("conv_smallk_f32");
}

}  // namespace nhip
