// fp32 convolution for launches with few output blocks, one kernel with the
// reduction split over each workgroup's waves.  3x3 (32 or 64 input
// channels): a single image (the 1x64x56x56 layer is 231 MFLOP, 2 us of
// MFMA issue spread over the GPU) instead of the Winograd path's three
// launches or the tiled implicit GEMM's 49 workgroups.  1x1: layers with at
// most one 32x32 block per CU (MobileNetV2's 960 -> 160 at 7x7, batch 32),
// instead of a split-K GEMM and its reduce launch.  Same operation as the
// implicit GEMM (reference ConvertConvolution, NCNNToTosa.cpp:1316-1529).
//
// A workgroup owns one 32x32 block of (output channel, output pixel) and
// splits the reduction over its WAVES waves (8 for 3x3): k = c*TAPS +
// kh*3 + kw, lane half h of wave w takes input channels (2w + h)*CH .. +
// CH - 1 with all their taps (C = 2*WAVES*CH), so every k step of a lane is
// one (channel, tap) pair known at compile time.  Each lane loads its
// TAPS*CH weights and its pixel's TAPS*CH input values (zero padding through
// out-of-range buffer offsets; the channel plane offset is wave-uniform)
// into registers before the first v_mfma_f32_32x32x2_f32, so a wave waits
// once.  The weights come from the plan's copy in groups of 2 (3x3) or 4
// (1x1) reduction indices, [K/32][k/VW][32][VW]: a wave's load reads the 32
// output channels of two groups from 2 x 32 x VW contiguous floats (from
// row-major weights each lane read its own row, 64 cache lines a load).
// The partial blocks are summed through LDS in wave order (deterministic)
// by all threads, then bias, residual and activation.
#include <algorithm>

#include "nhip_internal.h"

namespace nhip {
namespace {

struct KqArgs {
  const float* w;       // [m_pad/32][kgroups][32][VW], k = c*TAPS + tap
  const float* bias;    // [m_pad]
  const float* x;       // [N][C][H][W]
  const float* res;     // [N][K][OH][OW] or null
  float* out;           // [N][K][OH][OW]
  uint32_t x_bytes, out_bytes;  // (< 2^31)
  int kgroups, C, K, H, W, OW, OHW, npix, nmb;
  int sh, sw, pt, pl, dh, dw, act;
};

typedef float v2f __attribute__((ext_vector_type(2)));

// Reduction indices per weight group: 2 for 3x3 (a lane's 9*CH weights are
// whole float2s), 4 for 1x1 (its channel counts are multiples of 4).
constexpr int kq_group(int taps) { return taps == 9 ? 2 : 4; }

template <int CH, int TAPS, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void conv_kq_kernel(KqArgs g) {
  extern __shared__ float red[];  // [WAVES][16][64]: every wave's partial block
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 31, lh = lane >> 5;
  const int mb = blockIdx.x % g.nmb, pb = blockIdx.x / g.nmb;

  // this lane's pixel (B column li) and its tap offsets (3x3 or one) in
  // the image of channel (2*wave + lh)*CH; out of range in the padding
  const int plane = g.H * g.W;
  uint32_t toff[TAPS];
  {
    const int pix = pb * 32 + li;
    const bool pok = pix < g.npix;
    const int pp = pok ? pix : 0;
    const int img = pp / g.OHW, rem = pp - img * g.OHW;
    const int oy = rem / g.OW, ox = rem - oy * g.OW;
#pragma unroll
    for (int t = 0; t < TAPS; ++t) {
      const int iy = oy * g.sh - g.pt + (t / 3) * g.dh, ix = ox * g.sw - g.pl + (t % 3) * g.dw;
      const bool ok = pok && (unsigned)iy < (unsigned)g.H && (unsigned)ix < (unsigned)g.W;
      toff[t] = ok ? (uint32_t)((((int64_t)img * g.C + lh * CH) * plane + iy * g.W + ix) * 4) : kBufOOB;
    }
  }

  // weights: row 32*mb + li, k = TAPS*((2w + h)*CH) .. + TAPS*CH - 1, in
  // groups of VW (the plan's layout): one load of a wave reads the 32 rows
  // of two groups, 2 x 32 x VW contiguous floats
  constexpr int KS = TAPS * CH;
  constexpr int VW = kq_group(TAPS);
  static_assert(KS % VW == 0, "a lane's weight segment is whole groups");
  float a[KS];
  {
    const float* ap = g.w + ((int64_t)mb * g.kgroups + (2 * wave + lh) * (KS / VW)) * 32 * VW + li * VW;
#pragma unroll
    for (int q = 0; q < KS / VW; ++q) {
      if constexpr (VW == 4) {
        const v4f v = *reinterpret_cast<const v4f*>(ap + q * 32 * VW);
#pragma unroll
        for (int e = 0; e < 4; ++e) a[4 * q + e] = v[e];
      } else {
        const v2f v = *reinterpret_cast<const v2f*>(ap + q * 32 * VW);
        a[2 * q] = v[0];
        a[2 * q + 1] = v[1];
      }
    }
  }
  float b[KS];
  {
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(g.x, g.x_bytes);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int soff = ((2 * wave * CH + c) * plane) * 4;  // wave-uniform channel plane
#pragma unroll
      for (int t = 0; t < TAPS; ++t)
        b[c * TAPS + t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xr, toff[t], soff, 0));
    }
  }
  // This thread's epilogue entries e = tid + 64*WAVES*j of the 32x32 block
  // (channel o, pixel pix): output offset, bias and residual.  1x1 requests
  // them now, behind the operands, so that their latency passes under the
  // MFMAs and the reduction instead of one round trip per entry after it
  // (MobileNetV2 batch 32 0.665 -> 0.661 ms); 3x3 after the reduction (early,
  // behind its 36-step operand set and with the index divisions ahead of the
  // first MFMA, the 1x64x56x56 layer measured 7.3-7.7 us against 6.6-6.8).
  constexpr int NE = 1024 / (64 * WAVES);
  static_assert(NE * 64 * WAVES == 1024, "the block's 1024 entries split evenly over the threads");
  constexpr bool kEarly = TAPS == 1;
  uint32_t eoff[NE];
  float ebias[NE], eres[NE];
  if constexpr (kEarly) {
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(g.res, g.res ? g.out_bytes : 0);
    const __amdgpu_buffer_rsrc_t br = make_rsrc(g.bias, (uint32_t)(g.nmb * 32 * sizeof(float)));
#pragma unroll
    for (int j = 0; j < NE; ++j) {
      const int e = tid + 64 * WAVES * j;
      const int r = e >> 6, l = e & 63;
      const int pix = pb * 32 + (l & 31);
      const int o = mb * 32 + (r & 3) + 8 * (r >> 2) + 4 * (l >> 5);
      const bool ok = pix < g.npix && o < g.K;
      const int pp = ok ? pix : 0;
      const int img = pp / g.OHW, rem = pp - img * g.OHW;
      eoff[j] = ok ? (uint32_t)((((int64_t)img * g.K + o) * g.OHW + rem) * 4) : kBufOOB;
      ebias[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(br, (uint32_t)(o * 4), 0, 0));
      eres[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rr, eoff[j], 0, 0));
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // every load issued before the first MFMA
  v16f acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
  for (int s = 0; s < KS; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b[s], acc, 0, 0, 0);

#pragma unroll
  for (int r = 0; r < 16; ++r) red[(wave * 16 + r) * 64 + lane] = acc[r];
  __syncthreads();
  // entry (r, l) of the block, r = e / 64, l = e % 64: the partials summed in
  // wave order (deterministic); D[channel][pixel]: register r of lane
  // (li, lh) is channel 32mb + (r&3) + 8(r>>2) + 4lh at pixel 32pb + li
  const __amdgpu_buffer_rsrc_t orr = make_rsrc(g.out, g.out_bytes);
  const __amdgpu_buffer_rsrc_t rr = make_rsrc(g.res, g.res ? g.out_bytes : 0);
#pragma unroll
  for (int j = 0; j < NE; ++j) {
    const int e = tid + 64 * WAVES * j;
    const int r = e >> 6, l = e & 63;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) v += red[(w * 16 + r) * 64 + l];
    if constexpr (kEarly) {
      v = v + ebias[j];
      if (g.res) v = v + eres[j];
      if (g.act == NHIP_ACT_RELU) v = v < 0.f ? 0.f : v;
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(v), orr, eoff[j], 0, 0);
    } else {
      const int pix = pb * 32 + (l & 31);
      const int o = mb * 32 + (r & 3) + 8 * (r >> 2) + 4 * (l >> 5);
      if (pix < g.npix && o < g.K) {
        const int img = pix / g.OHW, rem = pix - img * g.OHW;
        const uint32_t off = (uint32_t)((((int64_t)img * g.K + o) * g.OHW + rem) * 4);
        v = v + g.bias[o];
        if (g.res) v = v + __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rr, off, 0, 0));
        if (g.act == NHIP_ACT_RELU) v = v < 0.f ? 0.f : v;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(v), orr, off, 0, 0);
      }
    }
  }
}

template <int CH, int TAPS, int WAVES>
int launch_kq(const KqArgs& a, dim3 grid, hipStream_t s) {
  constexpr int lds = WAVES * 16 * 64 * 4;
  NHIP_TRY(ensure_dynamic_lds(reinterpret_cast<const void*>(&conv_kq_kernel<CH, TAPS, WAVES>), lds));
  NHIP_LAUNCH("conv_kq", (conv_kq_kernel<CH, TAPS, WAVES>), grid, dim3(64 * WAVES), lds, s, a);
  return check_launch("conv_kq");
}

}  // namespace

// The grouped weights (made with the plan when the kernel can take it).
bool kq_weights(const nhip_conv_plan* p, const float** w) {
  *w = p->weight_kq;
  return *w != nullptr && p->kq_vw == kq_group(p->g.kh * p->g.kw);
}

// Instances: (channels per lane half, waves) for a 1x1 convolution with C
// input channels, C = 2*waves*CH (MobileNetV2's 7x7 and 14x14 layers);
// {0, 0} when none.
struct KqShape {
  int ch, waves;
};
KqShape kq_1x1_shape(int c) {
  for (int ch : {8, 12, 20, 40, 48, 72})
    if (c == 8 * ch) return {ch, 4};
  if (c == 960) return {60, 8};
  return {0, 0};
}

int conv_kq_prepack(nhip_conv_plan* p, const float* weight, int c, int k, int kh, int kw) {
  const bool k3 = kh == 3 && kw == 3 && (c == 32 || c == 64);
  const bool k1 = kh == 1 && kw == 1 && kq_1x1_shape(c).ch != 0;
  if (!k3 && !k1) return ok();
  const int taps = kh * kw, kt = c * taps, vw = kq_group(taps);
  const int mp = (int)round_up(k, 32);
  std::vector<float> wg((size_t)mp * kt, 0.f);
  for (int o = 0; o < k; ++o)
    for (int j = 0; j < kt; ++j)
      wg[(((size_t)(o / 32) * (kt / vw) + j / vw) * 32 + o % 32) * vw + j % vw] = weight[(size_t)o * kt + j];
  p->kq_vw = vw;
  NHIP_TRY(check_hip(hipMalloc(&p->weight_kq, wg.size() * sizeof(float)), "hipMalloc(conv grouped weight)"));
  return check_hip(hipMemcpy(p->weight_kq, wg.data(), wg.size() * sizeof(float), hipMemcpyHostToDevice),
                   "hipMemcpy(conv grouped weight)");
}

// Whether the kernel takes the launch: a 3x3 convolution with 32 or 64 input
// channels (a lane's 9*C/16 weights then are whole float2 groups) or a 1x1
// one with an instantiated channel count, activation none or ReLU, and few
// blocks.  3x3: at most two 32x32 blocks per CU, on either plan (one image
// of 64x56x56, 64 output channels, 196 blocks: 7.1 us in a kernel trace,
// 7.6 us with 4 waves a block, 8.0 with 16; 9.7 us before the grouped
// weights, against 13.6 us for the Winograd path and 14.6 us for the tiled
// implicit GEMM; two such images, 392 blocks, 15.0 against 21.1 us on
// Winograd; at 784 blocks Winograd wins with 64 channels, 25.6 against 26.5
// us).  1x1: at
// most one per CU, two for reductions of 768+ channels, taken before the
// pointwise kernel (MobileNetV2 at batch 32, 7x7: 576 -> 160 9.1 against
// 16.1 us, 960 -> 160 + residual 13.3 against 13.2, 960 -> 320 18.9
// against 21.3; at 14x14, 392 blocks, 384 -> 64 + residual 13.0 against
// 11.4 us on the pointwise kernel) and at least one per eight CUs
// (MobileNetV2 at batch 1 puts its 7x7 and 14x14 projections, 10 to 21
// blocks, on this kernel 11 us slower over the graph, its expansions, 60 to
// 126 blocks, 5 us faster).  NHIP_CONV_KQ=0 never, =2 whenever it can.
bool kq_supported(const nhip_conv_plan* p, int n, int h, int w, int oh, int ow) {
  const int mode = setting_int("NHIP_CONV_KQ", 1);
  if (mode == 0) return false;
  const ConvGeom& g = p->g;
  const float* wr = nullptr;
  if (p->kind != PlanKind::ConvF32 || !kq_weights(p, &wr) || (g.act != NHIP_ACT_NONE && g.act != NHIP_ACT_RELU))
    return false;
  const bool k3 = g.kh == 3 && g.kw == 3 && (g.c == 32 || g.c == 64);
  const bool k1 = g.kh == 1 && g.kw == 1 && kq_1x1_shape(g.c).ch != 0;
  if (!k3 && !k1) return false;
  const int64_t npix = (int64_t)n * oh * ow;
  const int64_t blocks = ceil_div(p->g.k, 32) * ceil_div(npix, 32);
  // (1x1 with reductions of 768+ channels: up to two blocks per CU; the
  // long reduction amortizes each block's fixed cost)
  const int per_cu = k3 || g.c >= 768 ? 2 : 1;
  if (mode != 2 && (blocks > per_cu * (int64_t)cu_count() || (k1 && blocks < cu_count() / 8))) return false;
  return (int64_t)n * g.c * h * w * 4 < INT32_MAX && npix * g.k * 4 < INT32_MAX;
}

int launch_conv_kq(const nhip_conv_plan* p, const float* in, const float* residual, float* out, int n, int h, int w,
                   int oh, int ow, hipStream_t s) {
  KqArgs a{};
  if (!kq_weights(p, &a.w)) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "conv_kq: no grouped weights");
  a.kgroups = p->g.c * p->g.kh * p->g.kw / p->kq_vw;
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
  if (p->g.kh == 3) return p->g.c == 32 ? launch_kq<2, 9, 8>(a, grid, s) : launch_kq<4, 9, 8>(a, grid, s);
  const KqShape k = kq_1x1_shape(p->g.c);
#define NHIP_KQ1(CH_, W_)                                        \
  if (k.ch == CH_ && k.waves == W_) return launch_kq<CH_, 1, W_>(a, grid, s);
  NHIP_KQ1(8, 4)
  NHIP_KQ1(12, 4)
  NHIP_KQ1(20, 4)
  NHIP_KQ1(40, 4)
  NHIP_KQ1(48, 4)
  NHIP_KQ1(72, 4)
  NHIP_KQ1(60, 8)
#undef NHIP_KQ1
  return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "conv_kq: unsupported shape");
}

}  // namespace nhip
