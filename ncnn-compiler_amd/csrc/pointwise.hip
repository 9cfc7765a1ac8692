// 1x1 stride-1 unpadded fp32 convolution on NCHW (the expand / project
// layers of inverted-residual networks):
//   out[n][k][p] = act(sum_c W[k][c] x[n][c][p] + b[k] (+ res[n][k][p]))
// (ncnn Convolution with kernel 1, lowered by the reference through
// tosa.conv2d -> linalg.conv_2d_nhwc_hwcf: NCNNToTosa.cpp:1107-1530).
//
// These layers move far more bytes than they compute (16 -> 96 channels at
// 112x112 is 1.2 GFLOP against 180 MB), so the kernel is built to stream x
// once per output-channel slice and write out once at HBM speed:
//   * a workgroup (4 waves) holds the weights of its slice of 16*KT output
//     channels in LDS for its whole life and walks 256-pixel tiles
//     (persistent grid);
//   * a wave owns 64 consecutive pixels x the slice, so every element of x
//     is loaded by exactly one wave per slice, straight into MFMA B
//     fragments (no LDS staging);
//   * input channels stream in chunks of 16 (four v_mfma_f32_16x16x4_f32
//     k-steps) through a ring of NB register buffers, NB - 1 chunks in
//     flight ahead of the one being multiplied, across tile boundaries;
//   * lane l loads pixels 4*(l%16) .. +3 and feeds pixel 4*(l%16) + v to
//     MFMA v of a k-step, so register r of the four accumulators of a
//     channel block holds four consecutive pixels of one output channel: the
//     result leaves as 16-byte stores, 16 lanes covering 256 contiguous bytes
//     of an output row.
#include <cstdio>
#include <cstdlib>

#include "nhip_internal.h"

namespace nhip {
namespace {

constexpr int kThreads = 256;   // 4 waves
constexpr int kChunk = 16;      // input channels per chunk (4 MFMA k-steps)
constexpr int kTilePix = 256;   // pixels per workgroup tile (4 waves x 64)
constexpr int kXcds = 8;
constexpr int kMaxLds = 64 * 1024;

struct PwArgs {
  const float* x;        // [N][C][P]
  const float* w;        // [m_pad][ldw]
  const float* bias;     // [m_pad]
  const float* res;      // [N][K][P] or null
  float* out;            // [N][K][P]
  int C, K, P, ldw, c4;  // c4 = C rounded up to 4
  int np;                // N * P pixels (< 2^29: x is < 2^31 bytes)
  int ntiles, nch;       // pixel tiles, channel chunks
  uint32_t x_bytes, out_bytes;
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

// LDS: Ws[c][j][t] = W[k0 + 16t + j][c] (c < c4, j < 16, t < KT), so the A
// fragments of one k-step (KT floats per lane, lane l = (c%4)*16 + j) are
// one contiguous 64*KT-float run; then bias[k0 .. k0 + 16*KT).
// RES: add the residual.  Its loads for a tile go out right after the X
// loads of the tile's last chunk when the tile has at least NB chunks (one
// tile's residual pending at a time), otherwise just before the prefetch
// issued beside that chunk's MFMAs; either way waiting for them never waits
// for later prefetches (vmcnt retires in issue order).
// Stores and loads are raw buffer operations on 32-bit offsets: positions
// past the last pixel or channel carry an offset past the buffer's size, so
// they neither branch nor touch memory.
template <int KT, int NB, int ACT, bool RES>
__global__ __launch_bounds__(kThreads, 2) void pw_conv_kernel(PwArgs a) {
  extern __shared__ __attribute__((aligned(16))) float ws[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int KS = 16 * KT;  // output channels per slice
  const int k0 = blockIdx.y * KS;
  float* bs = ws + a.c4 * KS;

  // ---- weights and bias of the slice into LDS (coalesced over c) ----------
  for (int e = tid; e < KS * a.c4; e += kThreads) {
    const int kl = e / a.c4, c = e - kl * a.c4;
    const int k = k0 + kl;
    const float v = (c < a.C && k < a.K) ? a.w[(int64_t)k * a.ldw + c] : 0.f;
    ws[(c * 16 + (kl & 15)) * KT + (kl >> 4)] = v;
  }
  for (int e = tid; e < KS; e += kThreads) bs[e] = (k0 + e < a.K) ? a.bias[k0 + e] : 0.f;
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
  if (first >= a.ntiles) return;
  const int my_tiles = (a.ntiles - 1 - first) / gridDim.x + 1;

  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t orr = make_rsrc(a.out, a.out_bytes);
  const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.res, RES ? a.out_bytes : 0u);
  const int jl = lane & 15, cl = lane >> 4;
  const uint32_t cstride = (uint32_t)a.P * 4u;  // bytes between channel planes
  const float inv_p = 1.0f / (float)a.P;

  // Lane geometry of a tile: pixel q = tile*256 + wave*64 + 4*jl of image n
  // at position p; xo = byte offset of (n, c = 0, p) in x, oo = byte offset
  // of (n, k = 0, p) in out (and the residual); q past the end: both out of
  // range.  P % 4 == 0, so the lane's four pixels lie in one image.
  struct Geo {
    uint32_t xo, oo;
  };
  auto geo = [&](int tile) {
    const int q0 = tile * kTilePix;  // uniform
    const int n0 = q0 / a.P, p0 = q0 - n0 * a.P;
    const int u = p0 + wave * 64 + 4 * jl;
    int dn = (int)((float)u * inv_p);
    int p = u - dn * a.P;
    if (p < 0) { --dn; p += a.P; }
    if (p >= a.P) { ++dn; p -= a.P; }
    const int n = n0 + dn;
    const bool ok = q0 + (u - p0) < a.np;
    Geo g;
    g.xo = ok ? (uint32_t)(n * a.C * a.P + p) * 4u : kBufOOB;
    g.oo = ok ? (uint32_t)(n * a.K * a.P + p) * 4u : kBufOOB;
    return g;
  };

  auto issue = [&](v4f (&xb)[4], const Geo& g, int cc, bool live) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int c = cc * kChunk + 4 * s + cl;
      xb[s] = load4(xr, (live && c < a.C && g.xo != kBufOOB) ? g.xo + (uint32_t)c * cstride : kBufOOB);
    }
  };

  v4f acc[KT][4];
#pragma unroll
  for (int t = 0; t < KT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[t][v] = v4f{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const v4f (&xb)[4], int cc) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int cs = cc * kChunk + 4 * s;  // first channel of the k-step
      if (cs >= a.c4) break;
      float av[KT];
      const float* wp = ws + ((cs >> 2) * 64 + lane) * KT;
#pragma unroll
      for (int t = 0; t < KT; ++t) av[t] = wp[t];
#pragma unroll
      for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[t][v] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[t], xb[s][v], acc[t][v], 0, 0, 0);
    }
  };

  // offset of output channel k0 + 16t + 4cl + r at the lane's pixels
  auto out_off = [&](const Geo& g, int t, int r) {
    const int k = k0 + 16 * t + 4 * cl + r;
    return (k < a.K && g.oo != kBufOOB) ? g.oo + (uint32_t)k * cstride : kBufOOB;
  };

  v4f rv[RES ? KT : 1][4];
  auto issue_res = [&](const Geo& g) {
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) rv[RES ? t : 0][r] = load4(rr, out_off(g, t, r));
  };

  auto epilogue = [&](const Geo& g) {
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      const v4f b4 = *reinterpret_cast<const v4f*>(bs + 16 * t + 4 * cl);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        v4f y;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          float o = acc[t][v][r] + b4[r];
          if constexpr (RES) o += rv[t][r][v];
          y[v] = activate<ACT>(o);
        }
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, y), orr, out_off(g, t, r), 0, 0);
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[t][v] = v4f{0.f, 0.f, 0.f, 0.f};
    }
  };

  // Chunk stream: chunk (i, cc) = channel chunk cc of this workgroup's tile
  // i.  The issue side (ii, icc, gi) runs NB - 1 chunks ahead of the compute
  // side (i, cc, gc); issues past the last tile load nothing.
  const bool res_early = RES && a.nch >= NB;
  int ii = 0, icc = 0;
  Geo gi = geo(first);
  auto issue_next = [&](v4f (&buf)[4]) {
    const bool live = ii < my_tiles;
    issue(buf, gi, icc, live);
    if constexpr (RES)
      if (res_early && live && icc == a.nch - 1) issue_res(gi);
    if (++icc == a.nch) {
      icc = 0;
      ++ii;
      gi = geo(first + ii * (int)gridDim.x);
    }
  };
  int i = 0, cc = 0;
  Geo gc = gi;

  v4f xb[NB][4];
#pragma unroll
  for (int b = 0; b + 1 < NB; ++b) issue_next(xb[b]);
  bool done = false;
  while (!done) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const bool last = cc == a.nch - 1;
      if constexpr (RES)
        if (!res_early && last) issue_res(gc);
      issue_next(xb[(b + NB - 1) % NB]);
      compute(xb[b], cc);
      if (last) {
        epilogue(gc);
        ++i;
        cc = 0;
        if (i >= my_tiles) {
          done = true;
          break;
        }
        gc = geo(first + i * (int)gridDim.x);
      } else {
        ++cc;
      }
    }
  }
}

// Workgroups of `kernel` resident per CU with `lds` bytes of LDS each (the
// runtime's occupancy calculation, cached for the last LDS size asked).
template <class Kernel>
int resident_per_cu(Kernel kernel, size_t lds) {
  static size_t last_lds = ~size_t(0);
  static int last = 1;
  if (lds != last_lds) {
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, kThreads, lds) != hipSuccess || occ < 1) occ = 1;
    last = occ;
    last_lds = lds;
  }
  return last;
}

// Grid: one workgroup per (tile, slice) when they all fit on the GPU at
// once, otherwise as many as fit, each walking an equal share of the tiles;
// gridDim.y = slices.
template <class Kernel>
dim3 pw_grid(Kernel kernel, const PwArgs& a, int slices, size_t lds) {
  const int64_t fit = (int64_t)resident_per_cu(kernel, lds) * cu_count();
  int64_t gx = a.ntiles;
  if (gx * slices > fit) {
    const int64_t per = std::max<int64_t>(1, fit / slices);
    gx = ceil_div(a.ntiles, ceil_div(a.ntiles, per));
  }
  // Tuning / test override NHIP_PW_WGS=n: at most n workgroups per slice
  // (each then walks more tiles).
  if (const char* env = std::getenv("NHIP_PW_WGS"))
    if (const int v = std::atoi(env); v > 0) gx = std::min<int64_t>(gx, v);
  // a multiple of 8, so that blockIdx.x % 8 is the XCD (workgroups past the
  // last tile exit at once)
  return dim3((unsigned)round_up(gx, kXcds), (unsigned)slices);
}

template <int KT, int NB, int ACT, bool RES>
int launch_one(const PwArgs& a, int slices, size_t lds, hipStream_t s) {
  const auto kernel = pw_conv_kernel<KT, NB, ACT, RES>;
  NHIP_LAUNCH("pw_conv_f32", kernel, pw_grid(kernel, a, slices, lds), dim3(kThreads), lds, s, a);
  return check_launch("pw_conv_f32");
}

template <int KT, int NB, bool RES>
int launch_act(const PwArgs& a, int act, int slices, size_t lds, hipStream_t s) {
  if (act == NHIP_ACT_RELU) return launch_one<KT, NB, NHIP_ACT_RELU, RES>(a, slices, lds, s);
  if (act == NHIP_ACT_SIGMOID) return launch_one<KT, NB, NHIP_ACT_SIGMOID, RES>(a, slices, lds, s);
  return launch_one<KT, NB, NHIP_ACT_NONE, RES>(a, slices, lds, s);
}

struct PwCfg {
  int kt, nb, slices;
};

// Instantiated (KT, NB) pairs, with and without a residual (whose registers
// are live beside the accumulators).
constexpr PwCfg kPlain[] = {{1, 2, 1}, {1, 4, 1}, {2, 2, 1}, {2, 4, 1}, {3, 2, 1}, {3, 4, 1}, {4, 2, 1}, {6, 2, 1}};
constexpr PwCfg kResid[] = {{1, 2, 1}, {1, 4, 1}, {2, 2, 1}, {2, 4, 1}, {3, 2, 1}, {4, 2, 1}};

bool lds_ok(int c, int kt) { return (int64_t)(round_up(c, 4) + 1) * 16 * kt * (int64_t)sizeof(float) <= kMaxLds; }

// Output channels per slice: KT = 1..3 (the fastest measured on the
// MobileNetV2 layers: the kernel's code stays small and each slice's
// re-read of x comes from L2), the largest that still gives two (tile,
// slice) work items per CU and leaves no slice mostly padding; NB = 2.
bool pw_config(const nhip_conv_plan* p, int64_t np, bool res, PwCfg* out) {
  const int kb = (int)ceil_div(p->g.k, 16);
  const int64_t tiles = ceil_div(np, kTilePix);
  int kt = 1;
  for (int t = std::min(3, kb); t >= 1; --t) {
    const int slices = (int)ceil_div(kb, t);
    if (slices * t - kb >= (t + 1) / 2 && t > 1) continue;  // a slice mostly padding
    if (tiles * slices >= 2LL * cu_count()) {
      kt = t;
      break;
    }
  }
  int nb = 2;
  if (const char* env = std::getenv("NHIP_PW_CFG")) {  // tuning override "kt,nb"
    int ekt = 0, enb = 0;
    if (std::sscanf(env, "%d,%d", &ekt, &enb) == 2) {
      const PwCfg* tab = res ? kResid : kPlain;
      const int nt = res ? (int)(sizeof(kResid) / sizeof(PwCfg)) : (int)(sizeof(kPlain) / sizeof(PwCfg));
      for (int j = 0; j < nt; ++j)
        if (tab[j].kt == ekt && tab[j].nb == enb) kt = ekt, nb = enb;
    }
  }
  if (!lds_ok(p->g.c, kt)) return false;
  *out = {kt, nb, (int)ceil_div(kb, kt)};
  return true;
}

}  // namespace

bool pointwise_selected(const nhip_conv_plan* p, int n, int h, int w) {
  const ConvGeom& g = p->g;
  if (g.kh != 1 || g.kw != 1 || g.sh != 1 || g.sw != 1 || g.pt || g.pb || g.pl || g.pr) return false;
  if ((h * w) % 4 != 0) return false;
  bool forced = false;
  if (const char* env = std::getenv("NHIP_POINTWISE")) {
    if (env[0] == '0') return false;
    forced = env[0] == '2';  // every eligible shape (tests)
  }
  // Few pixels and long reductions: the chunk chain of one wave is the
  // critical path, and the implicit GEMM's split-K keeps more CUs busy
  // (measured on the MobileNetV2 layers: 384 -> 64 and 576 -> 96 at 14x14).
  if (!forced && (int64_t)n * h * w < 16384 && g.c > 192) return false;
  PwCfg c;
  if (!pw_config(p, (int64_t)n * h * w, false, &c) || !pw_config(p, (int64_t)n * h * w, true, &c)) return false;
  // x and out are addressed by 32-bit buffer offsets
  const int64_t xb = (int64_t)n * g.c * h * w * 4, ob = (int64_t)n * g.k * h * w * 4;
  return xb < (int64_t(1) << 31) && ob < (int64_t(1) << 31);
}

int launch_conv_pointwise_f32(const nhip_conv_plan* p, const float* in, const float* residual, float* out, int n,
                              int h, int w, hipStream_t s) {
  PwCfg c;
  if ((h * w) % 4 != 0 || !pw_config(p, (int64_t)n * h * w, residual != nullptr, &c))
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "pointwise conv: unsupported shape");
  PwArgs a{};
  a.x = in;
  a.w = p->weight;
  a.bias = p->bias;
  a.res = residual;
  a.out = out;
  a.C = p->g.c;
  a.K = p->g.k;
  a.P = h * w;
  a.ldw = p->kred_pad;
  a.c4 = (int)round_up(a.C, 4);
  a.np = n * a.P;
  a.ntiles = (int)ceil_div(a.np, kTilePix);
  a.nch = (int)ceil_div(a.c4, kChunk);
  a.x_bytes = (uint32_t)((int64_t)n * a.C * a.P * 4);
  a.out_bytes = (uint32_t)((int64_t)n * a.K * a.P * 4);
  const size_t lds = (size_t)(a.c4 + 1) * 16 * c.kt * sizeof(float);
  const int act = p->g.act;
  if (residual) {
    switch (c.kt * 10 + c.nb) {
      case 12: return launch_act<1, 2, true>(a, act, c.slices, lds, s);
      case 14: return launch_act<1, 4, true>(a, act, c.slices, lds, s);
      case 22: return launch_act<2, 2, true>(a, act, c.slices, lds, s);
      case 24: return launch_act<2, 4, true>(a, act, c.slices, lds, s);
      case 32: return launch_act<3, 2, true>(a, act, c.slices, lds, s);
      case 42: return launch_act<4, 2, true>(a, act, c.slices, lds, s);
    }
  } else {
    switch (c.kt * 10 + c.nb) {
      case 12: return launch_act<1, 2, false>(a, act, c.slices, lds, s);
      case 14: return launch_act<1, 4, false>(a, act, c.slices, lds, s);
      case 22: return launch_act<2, 2, false>(a, act, c.slices, lds, s);
      case 24: return launch_act<2, 4, false>(a, act, c.slices, lds, s);
      case 32: return launch_act<3, 2, false>(a, act, c.slices, lds, s);
      case 34: return launch_act<3, 4, false>(a, act, c.slices, lds, s);
      case 42: return launch_act<4, 2, false>(a, act, c.slices, lds, s);
      case 62: return launch_act<6, 2, false>(a, act, c.slices, lds, s);
    }
  }
  return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "pointwise conv: no kernel for the configuration");
}

}  // namespace nhip
