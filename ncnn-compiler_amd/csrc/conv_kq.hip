// fp32 3x3 convolution for launches with few output pixels (a single image:
// the 1x64x56x56 layer is 231 MFLOP, 2 us of MFMA issue spread over the
// GPU), one kernel instead of the Winograd path's three launches or the
// tiled implicit GEMM's 49 workgroups.  Same operation as the implicit GEMM
// (reference ConvertConvolution, NCNNToTosa.cpp:1316-1529).
//
// A workgroup owns one 32x32 block of (output channel, output pixel) and
// splits the reduction over its four waves: k = c*9 + kh*3 + kw (the plan's
// weight order), lane half h of wave w takes input channels
// (2w + h)*CH .. + CH - 1 with all nine taps (C = 8*CH), so every k step
// of a lane is one (channel, tap) pair known at compile time.  Each lane
// loads its 9*CH weights (one contiguous row segment, 16-byte loads) and
// its pixel's 9*CH input values (zero padding through out-of-range buffer
// offsets; the channel plane offset is wave-uniform) into registers before
// the first v_mfma_f32_32x32x2_f32, so a wave waits once; the four partial
// blocks are summed through LDS in wave order (deterministic), then bias,
// residual and activation.
#include <algorithm>

#include "nhip_internal.h"

namespace nhip {
namespace {

constexpr int kThreads = 256;

struct KqArgs {
  const float* w;       // [m_pad][ldw], k = c*9 + kh*3 + kw
  const float* bias;    // [m_pad]
  const float* x;       // [N][C][H][W]
  const float* res;     // [N][K][OH][OW] or null
  float* out;           // [N][K][OH][OW]
  uint32_t x_bytes, out_bytes;  // (< 2^31)
  int ldw, C, K, H, W, OW, OHW, npix, nmb;
  int sh, sw, pt, pl, dh, dw, act;
};

template <int CH>
__global__ __launch_bounds__(kThreads) void conv_kq_kernel(KqArgs g) {
  __shared__ float red[3][16][64];  // partial blocks of waves 1..3
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 31, lh = lane >> 5;
  const int mb = blockIdx.x % g.nmb, pb = blockIdx.x / g.nmb;

  // this lane's pixel (B column li) and its nine tap offsets in the image
  // of channel (2*wave + lh)*CH; out of range for taps in the padding
  const int pix = pb * 32 + li;
  const bool pok = pix < g.npix;
  const int pp = pok ? pix : 0;
  const int img = pp / g.OHW, rem = pp - img * g.OHW;
  const int oy = rem / g.OW, ox = rem - oy * g.OW;
  const int plane = g.H * g.W;
  uint32_t toff[9];
#pragma unroll
  for (int t = 0; t < 9; ++t) {
    const int iy = oy * g.sh - g.pt + (t / 3) * g.dh, ix = ox * g.sw - g.pl + (t % 3) * g.dw;
    const bool ok = pok && (unsigned)iy < (unsigned)g.H && (unsigned)ix < (unsigned)g.W;
    toff[t] = ok ? (uint32_t)((((int64_t)img * g.C + lh * CH) * plane + iy * g.W + ix) * 4) : kBufOOB;
  }

  // weights: row 32*mb + li, k = 9*((2w + h)*CH) .. + 9*CH - 1, contiguous
  constexpr int KS = 9 * CH;
  static_assert(KS % 4 == 0, "a lane's weight segment is whole, 16-byte aligned float4s");
  v4f a[KS / 4];
  {
    const float* ap = g.w + (int64_t)(mb * 32 + li) * g.ldw + (2 * wave + lh) * KS;
#pragma unroll
    for (int q = 0; q < KS / 4; ++q) a[q] = *reinterpret_cast<const v4f*>(ap + 4 * q);
  }
  float b[KS];
  {
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(g.x, g.x_bytes);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int soff = ((2 * wave * CH + c) * plane) * 4;  // wave-uniform channel plane
#pragma unroll
      for (int t = 0; t < 9; ++t)
        b[c * 9 + t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xr, toff[t], soff, 0));
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // every load issued before the first MFMA
  v16f acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
  for (int s = 0; s < KS; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s / 4][s % 4], b[s], acc, 0, 0, 0);

  if (wave > 0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) red[wave - 1][r][lane] = acc[r];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < 3; ++w)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] += red[w][r][lane];
  // D[channel][pixel]: register r of lane (li, lh) is channel
  // 32mb + (r&3) + 8(r>>2) + 4lh at pixel 32pb + li
  const __amdgpu_buffer_rsrc_t orr = make_rsrc(g.out, g.out_bytes);
  const __amdgpu_buffer_rsrc_t rr = make_rsrc(g.res, g.res ? g.out_bytes : 0);
  uint32_t off[16];
  float rv[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int o = mb * 32 + (r & 3) + 8 * (r >> 2) + 4 * lh;
    off[r] = pok && o < g.K ? (uint32_t)((((int64_t)img * g.K + o) * g.OHW + rem) * 4) : kBufOOB;
    rv[r] = g.res ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rr, off[r], 0, 0)) : 0.f;
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int o = mb * 32 + (r & 3) + 8 * (r >> 2) + 4 * lh;
    float v = acc[r] + g.bias[o];
    if (g.res) v = v + rv[r];
    if (g.act == NHIP_ACT_RELU) v = v < 0.f ? 0.f : v;
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(v), orr, off[r], 0, 0);
  }
}

}  // namespace

// The row-major weights and their row stride: the implicit-GEMM plan's own,
// or a Winograd plan's extra copy (32 or 64 input channels).
bool kq_weights(const nhip_conv_plan* p, const float** w, int* ld) {
  if (p->algorithm == NHIP_CONV_ALGO_IMPLICIT_GEMM) {
    *w = p->weight;
    *ld = p->kred_pad;
  } else {
    *w = p->weight_rows;
    *ld = p->rows_ld;
  }
  return *w != nullptr && *ld % 4 == 0;
}

// Whether the kernel takes the launch: a 3x3 fp32 convolution with 32 or 64
// input channels (a lane's 9*C/8 weights then are whole 16-byte vectors),
// activation none or ReLU, and few blocks: at most two 32x32 blocks per CU
// on an implicit-GEMM plan (larger launches fill the GPU with the tiled
// kernels), at most one on a Winograd plan (config 1, 1x64x56x56: 9.7 us
// against 13.6 us for the Winograd path and 14.6 us for the tiled implicit
// GEMM).  NHIP_CONV_KQ=0 never, =2 whenever it can.
bool kq_supported(const nhip_conv_plan* p, int n, int h, int w, int oh, int ow) {
  const int mode = setting_int("NHIP_CONV_KQ", 1);
  if (mode == 0) return false;
  const ConvGeom& g = p->g;
  const float* wr = nullptr;
  int ld = 0;
  if (p->kind != PlanKind::ConvF32 || !kq_weights(p, &wr, &ld) || g.kh != 3 || g.kw != 3 ||
      (g.c != 32 && g.c != 64) || (g.act != NHIP_ACT_NONE && g.act != NHIP_ACT_RELU))
    return false;
  const int64_t npix = (int64_t)n * oh * ow;
  const int64_t blocks = ceil_div(p->g.k, 32) * ceil_div(npix, 32);
  const int per_cu = p->algorithm == NHIP_CONV_ALGO_IMPLICIT_GEMM ? 2 : 1;
  if (mode != 2 && blocks > per_cu * (int64_t)cu_count()) return false;
  return (int64_t)n * g.c * h * w * 4 < INT32_MAX && npix * g.k * 4 < INT32_MAX;
}

int launch_conv_kq(const nhip_conv_plan* p, const float* in, const float* residual, float* out, int n, int h, int w,
                   int oh, int ow, hipStream_t s) {
  KqArgs a{};
  if (!kq_weights(p, &a.w, &a.ldw)) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "conv_kq: no row-major weights");
  a.bias = p->bias;
  a.x = in;
  a.res = residual;
  a.out = out;
  a.x_bytes = (uint32_t)((int64_t)n * p->g.c * h * w * 4);
  a.out_bytes = (uint32_t)((int64_t)n * oh * ow * p->g.k * 4);
  a.C = p->g.c;
  a.K = p->g.k;
  a.H = h;
  a.W = w;
  a.OW = ow;
  a.OHW = oh * ow;
  a.npix = n * oh * ow;
  a.nmb = (int)ceil_div(p->g.k, 32);
  a.sh = p->g.sh;
  a.sw = p->g.sw;
  a.pt = p->g.pt;
  a.pl = p->g.pl;
  a.dh = p->g.dh;
  a.dw = p->g.dw;
  a.act = p->g.act;
  const dim3 grid((unsigned)(a.nmb * ceil_div(a.npix, 32)));
  if (p->g.c == 32)
    NHIP_LAUNCH("conv_kq", conv_kq_kernel<4>, grid, dim3(kThreads), 0, s, a);
  else
    NHIP_LAUNCH("conv_kq", conv_kq_kernel<8>, grid, dim3(kThreads), 0, s, a);
  return check_launch("conv_kq");
}

}  // namespace nhip
