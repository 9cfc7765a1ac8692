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
// Layout: the fp32/int8 NCHW input is first quantized into an NHWC int8
// scratch image with channels padded to 16 (one pass over HBM).  The GEMM
// then gathers 16-byte channel vectors per (pixel, kh, kw), reduction order
// (kh, kw, c) — the OHWI order the reference itself transposes the weights
// to (NCNNToTosa.cpp:1168-1176).
#include <cmath>
#include <vector>

#include "nhip_internal.h"

namespace nhip {
namespace {

constexpr int kThreads = 256;
constexpr int kBK = 64;       // bytes of k per LDS stage = 2 MFMA steps
constexpr int kRow = kBK + 16;  // LDS row stride (bytes), keeps b128 reads conflict-free

__device__ __forceinline__ int8_t quantize_i8(float x, float scale) {
#pragma clang fp contract(off)
  const float s = x * scale;
  if (s != s) return 0;
  float r = (s >= 0.0f) ? floorf(s + 0.5f) : ceilf(s - 0.5f);
  r = fminf(r, 127.0f);
  r = fmaxf(r, -127.0f);
  return (int8_t)(int)r;
}

// x [N][C][HW] (fp32 or int8) -> y [N][HW][c_pad] int8, zero channel padding.
// Block: 64 pixels of one image; loops over 64-channel slabs through LDS.
__global__ __launch_bounds__(kThreads) void quantize_nchw_to_nhwc(
    const void* __restrict__ x, int in_is_i8, int8_t* __restrict__ y, int C,
    int HW, int c_pad, float scale) {
  __shared__ __attribute__((aligned(16))) int8_t tile[64 * kRow];
  const int img = blockIdx.y;
  const int p0 = blockIdx.x * 64;
  const int tid = threadIdx.x;
  const int px = tid & 63, cc = tid >> 6;
  const int p = p0 + px;
  const float* xf = static_cast<const float*>(x) + (int64_t)img * C * HW;
  const int8_t* xi = static_cast<const int8_t*>(x) + (int64_t)img * C * HW;
  for (int c0 = 0; c0 < c_pad; c0 += 64) {
#pragma unroll 4
    for (int u = 0; u < 16; ++u) {
      const int cl = cc + 4 * u;
      const int c = c0 + cl;
      int8_t v = 0;
      if (c < C && p < HW) {
        const int64_t off = (int64_t)c * HW + p;
        v = in_is_i8 ? xi[off] : quantize_i8(xf[off], scale);
      }
      tile[px * kRow + cl] = v;
    }
    __syncthreads();
    const int wp = tid >> 2, chunk = tid & 3;
    const int pw = p0 + wp;
    const int cw = c0 + chunk * 16;
    if (pw < HW && cw < c_pad)
      *reinterpret_cast<int4*>(y + ((int64_t)img * HW + pw) * c_pad + cw) =
          *reinterpret_cast<const int4*>(&tile[wp * kRow + chunk * 16]);
    __syncthreads();
  }
}

struct Int8Args {
  const int8_t* w;     // [m_pad][kred_pad]
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
};

// D[i = out channel][j = pixel] over the (kh, kw, c) reduction.
template <int BM, int BN>
__global__ __launch_bounds__(kThreads) void conv_int8_kernel(Int8Args g) {
  constexpr int TM = BM / 64, TN = BN / 64;
  __shared__ __attribute__((aligned(16))) int8_t As[2][BM * kRow];
  __shared__ __attribute__((aligned(16))) int8_t Bs[2][BN * kRow];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 31, lh = lane >> 5;
  const int j0 = blockIdx.x * BN, i0 = blockIdx.y * BM;

  // A: BM rows x 4 chunks of 16B.
  constexpr int A_LD = BM * 4 / kThreads;
  int4 ra[A_LD];
  // B: BN pixels x 4 chunks; CPT chunks per thread.
  constexpr int CPT = 4 * BN / kThreads;
  int4 rb[CPT];
  const int jj = tid % BN;
  const int kg = __builtin_amdgcn_readfirstlane(tid / BN);
  const int p = j0 + jj;
  const bool pix_ok = p < g.npix;
  const int pp = pix_ok ? p : 0;
  const int img = pp / g.OHW;
  const int rem = pp - img * g.OHW;
  const int oh = rem / g.OW, ow = rem - (rem / g.OW) * g.OW;
  const int iy0 = oh * g.sh - g.pt, ix0 = ow * g.sw - g.pl;
  // the whole NHWC scratch image is one wave-uniform buffer resource
  const __amdgpu_buffer_rsrc_t img_rs = make_rsrc(g.x, g.x_bytes);
  const int img_pix0 = img * g.H;

  auto load = [&](int kt) {
#pragma unroll
    for (int u = 0; u < A_LD; ++u) {
      const int q = tid + u * kThreads;
      const int row = q >> 2, ch = q & 3;
      ra[u] = *reinterpret_cast<const int4*>(g.w + (int64_t)(i0 + row) * g.kred_pad + kt * kBK + ch * 16);
    }
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int chunk = kt * 4 + kg * CPT + u;
      const int t = g.ktab[chunk];  // wave-uniform
      const int c0 = t >> 16, dy = (t >> 8) & 255, dx = t & 255;
      const int y = iy0 + dy, x = ix0 + dx;
      const bool in = pix_ok && c0 < g.c_pad && (unsigned)y < (unsigned)g.H && (unsigned)x < (unsigned)g.W;
      rb[u] = buf_load_b128(img_rs, in ? (uint32_t)(((img_pix0 + y) * g.W + x) * g.c_pad + c0) : kBufOOB);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int u = 0; u < A_LD; ++u) {
      const int q = tid + u * kThreads;
      const int row = q >> 2, ch = q & 3;
      *reinterpret_cast<int4*>(&As[buf][row * kRow + ch * 16]) = ra[u];
    }
#pragma unroll
    for (int u = 0; u < CPT; ++u)
      *reinterpret_cast<int4*>(&Bs[buf][jj * kRow + (kg * CPT + u) * 16]) = rb[u];
  };

  v16i acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0;

  const int nk = g.kred_pad / kBK;
  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) load(kt + 1);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      v4i af[TM], bf[TN];
#pragma unroll
      for (int a = 0; a < TM; ++a)
        af[a] = *reinterpret_cast<const v4i*>(&As[buf][(wm * (BM / 2) + a * 32 + li) * kRow + s * 32 + lh * 16]);
#pragma unroll
      for (int b = 0; b < TN; ++b)
        bf[b] = *reinterpret_cast<const v4i*>(&Bs[buf][(wn * (BN / 2) + b * 32 + li) * kRow + s * 32 + lh * 16]);
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[a], bf[b], acc[a][b], 0, 0, 0);
    }
    if (more) store(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: register r of lane l holds row (r%4)+8*(r/4)+4*(l/32), column l%32.
#pragma unroll
  for (int b = 0; b < TN; ++b) {
    const int j = j0 + wn * (BN / 2) + b * 32 + li;
    if (j >= g.npix) continue;
    const int im = j / g.OHW;
    const int rm = j - im * g.OHW;
    const int64_t obase = (int64_t)im * g.m * g.OHW + rm;
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = i0 + wm * (BM / 2) + a * 32 + (r & 3) + 8 * (r >> 2) + 4 * lh;
        if (i >= g.m) continue;
        const int64_t o = obase + (int64_t)i * g.OHW;
        float f;
        {
#pragma clang fp contract(off)
          f = (float)acc[a][b][r];
          f = f * g.recip[i];
          f = f + g.bias[i];
        }
        if (g.term > 100) {
          int8_t q = quantize_i8(f, g.os);
          if (g.act == NHIP_ACT_RELU && q < 0) q = 0;
          static_cast<int8_t*>(g.out)[o] = q;
        } else {
          if (g.act == NHIP_ACT_RELU) f = f < 0.0f ? 0.0f : f;
          static_cast<float*>(g.out)[o] = f;
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
  NHIP_LAUNCH("quantize_nchw_to_nhwc", quantize_nchw_to_nhwc, dim3((unsigned)ceil_div((int64_t)h * w, 64), n), dim3(kThreads),
                     0, s, in, in_is_i8, xq, p->g.c, h * w, p->c_pad, p->input_scale);
  NHIP_TRY(check_launch("quantize_nchw_to_nhwc"));

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
  const int64_t target = 2LL * cu_count();
  const int mt128 = (int)ceil_div(p->g.k, 128), mt64 = (int)ceil_div(p->g.k, 64);
  const int nt128 = (int)ceil_div(g.npix, 128), nt64 = (int)ceil_div(g.npix, 64);
  if (p->m_pad % 128 == 0 && (int64_t)mt128 * nt128 >= target) {
    NHIP_LAUNCH("conv_int8<128,128>", (conv_int8_kernel<128, 128>), dim3(nt128, mt128), dim3(kThreads), 0, s, g);
    return check_launch("conv_int8<128,128>");
  }
  if ((int64_t)mt64 * nt128 >= target) {
    NHIP_LAUNCH("conv_int8<64,128>", (conv_int8_kernel<64, 128>), dim3(nt128, mt64), dim3(kThreads), 0, s, g);
    return check_launch("conv_int8<64,128>");
  }
  NHIP_LAUNCH("conv_int8<64,64>", (conv_int8_kernel<64, 64>), dim3(nt64, mt64), dim3(kThreads), 0, s, g);
  return check_launch("conv_int8<64,64>");
}

}  // namespace nhip
