// Fused Winograd F(4x4, 3x3): input transform, the 36 point-wise products and
// the output transform in one kernel, so the transformed input V and the
// products M never leave the CU (the unfused path in winograd.hip writes and
// re-reads both through HBM).
//
// Work decomposition.  A wave owns a 16 (output channel) x 16 (tile) block for
// all 36 transform points xi and accumulates it with v_mfma_f32_16x16x4_f32:
// 36 x 4 accumulator registers per lane.  In the 16x16 MFMA result layout
// register r of lane l holds (row 4*(l/16)+r, column l%16) for every xi, so a
// lane owns all 36 values of four (k, t) pairs and the output transform
// A^T M A runs in registers.
//
// A workgroup is 4 waves arranged WK x WT x WC: WK*16 output channels, WT*16
// tiles, and the channel reduction split WC ways across waves (reduced
// through LDS at the end) for layers with few tiles.  Per chunk of CB input
// channels the workgroup
//   1. loads the 6x6 input patches of its tiles and transforms them
//      (V = B^T d B) into LDS, one (tile, channel) pair per thread;
//   2. copies U[xi][k][c] (transformed weights, prepacked on the host) into LDS;
//   3. runs 36 * CB/(4*WC) MFMAs per wave.
// Two workgroups fit per CU (73.7 KB LDS each), so one's load/transform
// phase overlaps the other's MFMA phase.
#include <cstdlib>
#include <cstring>

#include "nhip_internal.h"

namespace nhip {
namespace {

constexpr int kThreads = 256;

struct FusedArgs {
  const float* x;       // [N][C][H][W]
  const float* U;       // [36][m_pad][c_pad]
  const float* bias;    // [m_pad]
  const float* residual;
  float* out;           // [N][K][OH][OW]
  int C, H, W, K, OH, OW, th, tw, T, m_pad, c_pad, pt, pl, act;
  uint32_t x_bytes;     // size of x (< 2^31)
};

// LDS layout of one chunk, for both V (rows = tiles) and U (rows = output
// channels): [xi][c / S][row][S].  An MFMA operand read by a wave is then
// rows 0..15 x 4 lane groups of S consecutive floats, and each half-wave
// reads one contiguous 256-byte span: no bank conflicts.
template <int WK, int WT, int WC, int S>
struct FusedCfg {
  static constexpr int KB = 16 * WK;          // output channels per workgroup
  static constexpr int TB = 16 * WT;          // tiles per workgroup
  static constexpr int CB = 4 * S * WC;       // input channels per chunk
  static constexpr int V_ELEMS = 36 * TB * CB;
  static constexpr int U_ELEMS = 36 * KB * CB;
  static_assert(WK * WT * WC == 4, "4 waves per workgroup");
  static_assert(TB * CB == kThreads, "one (tile, channel) pair per thread and chunk");
};

template <int ROWS, int CB, int S>
__device__ __forceinline__ int lds_index(int xi, int c, int row) {
  return ((xi * (CB / S) + c / S) * ROWS + row) * S + (c % S);
}

// V = B^T d B; each transformed row is handed to `store(xi, value)` as soon
// as it is computed, so the 36 outputs never need to be live together.
template <class Store>
__device__ __forceinline__ void input_transform(float d[6][6], Store store) {
#pragma unroll
  for (int j = 0; j < 6; ++j) {  // columns: d <- B^T d, in place
    const float d0 = d[0][j], d1 = d[1][j], d2 = d[2][j], d3 = d[3][j], d4 = d[4][j], d5 = d[5][j];
    d[0][j] = 4.f * d0 - 5.f * d2 + d4;
    d[1][j] = -4.f * (d1 + d2) + d3 + d4;
    d[2][j] = 4.f * (d1 - d2) - d3 + d4;
    d[3][j] = -2.f * (d1 - d3) - d2 + d4;
    d[4][j] = 2.f * (d1 - d3) - d2 + d4;
    d[5][j] = 4.f * d1 - 5.f * d3 + d5;
  }
#pragma unroll
  for (int i = 0; i < 6; ++i) {  // rows: (B^T d) B
    const float d0 = d[i][0], d1 = d[i][1], d2 = d[i][2], d3 = d[i][3], d4 = d[i][4], d5 = d[i][5];
    store(i * 6 + 0, 4.f * d0 - 5.f * d2 + d4);
    store(i * 6 + 1, -4.f * (d1 + d2) + d3 + d4);
    store(i * 6 + 2, 4.f * (d1 - d2) - d3 + d4);
    store(i * 6 + 3, -2.f * (d1 - d3) - d2 + d4);
    store(i * 6 + 4, 2.f * (d1 - d3) - d2 + d4);
    store(i * 6 + 5, 4.f * d1 - 5.f * d3 + d5);
  }
}

template <int WK, int WT, int WC, int S>
__global__ __launch_bounds__(kThreads, 2) void wino_fused_kernel(FusedArgs a) {
  using Cfg = FusedCfg<WK, WT, WC, S>;
  constexpr int KB = Cfg::KB, TB = Cfg::TB, CB = Cfg::CB;
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float* Vs = lds;                    // [36][CB/S][TB][S]
  float* Us = lds + Cfg::V_ELEMS;     // [36][CB/S][KB][S]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wc = wave % WC, wt = (wave / WC) % WT, wk = wave / (WC * WT);
  const int li = lane & 15, lg = lane >> 4;
  const int t0 = blockIdx.x * TB, k0 = blockIdx.y * KB;

  // This thread's (tile, channel) pair for the input transform: consecutive
  // lanes take consecutive tiles (coalesced patch rows, conflict-free V writes).
  const int pt_local = tid % TB, pc_local = tid / TB;
  const int t = t0 + pt_local;
  const bool t_ok = t < a.T;
  int y0 = 0, x0 = 0, im = 0;
  {
    const int per_img = a.th * a.tw;
    const int tt = t_ok ? t : 0;
    im = tt / per_img;
    const int r = tt - im * per_img;
    const int ty = r / a.tw, tx = r - (r / a.tw) * a.tw;
    y0 = ty * 4 - a.pt;
    x0 = tx * 4 - a.pl;
  }
  // The whole input is one (wave-uniform) buffer resource, < 2^31 bytes;
  // padding and out-of-range tiles or channels read as 0 via kBufOOB.
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.x, a.x_bytes);
  float d[6][6];
  auto load_patch = [&](int c0) {
    const int c = c0 + pc_local;
    const bool ok = t_ok && c < a.C;
    const int plane = (im * a.C + c) * a.H;
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      const int y = y0 + i;
      const bool yok = ok && (unsigned)y < (unsigned)a.H;
#pragma unroll
      for (int j = 0; j < 6; ++j) {
        const int x = x0 + j;
        const uint32_t off = (yok && (unsigned)x < (unsigned)a.W)
                                 ? (uint32_t)(((plane + y) * a.W + x) * (int)sizeof(float))
                                 : kBufOOB;
        d[i][j] = buf_load_f32(rs, off);
      }
    }
  };

  v4f acc[36];
#pragma unroll
  for (int xi = 0; xi < 36; ++xi) acc[xi] = v4f{0.f, 0.f, 0.f, 0.f};

  const int nchunks = a.c_pad / CB;
  for (int ch = 0; ch < nchunks; ++ch) {
    const int c0 = ch * CB;
    // 36 independent buffer loads in flight at once; the other workgroup on
    // the CU runs its MFMAs meanwhile.
    load_patch(c0);
    __syncthreads();  // previous chunk's MFMA reads of Vs/Us are done
    {
      // 1. input patch -> V
      float* vrow = Vs + lds_index<TB, CB, S>(0, pc_local, pt_local);
      input_transform(d, [&](int xi, float v) { vrow[xi * TB * CB] = v; });
    }
    {
      // 2. U[xi][k0..k0+KB)[c0..c0+CB) -> LDS, float2 granules
      constexpr int PAIRS = 36 * KB * CB / 2;
      static_assert(PAIRS % kThreads == 0, "whole float2 granules per thread");
#pragma unroll
      for (int it = 0; it < PAIRS / kThreads; ++it) {
        const int q = tid + it * kThreads;
        const int xi = q / (KB * CB / 2);
        const int rem = q - xi * (KB * CB / 2);
        const int kk = rem / (CB / 2), c2 = (rem - (rem / (CB / 2)) * (CB / 2)) * 2;
        const float2 u = *reinterpret_cast<const float2*>(
            a.U + ((int64_t)xi * a.m_pad + k0 + kk) * a.c_pad + c0 + c2);
        Us[lds_index<KB, CB, S>(xi, c2, kk)] = u.x;
        Us[lds_index<KB, CB, S>(xi, c2 + 1, kk)] = u.y;
      }
    }
    __syncthreads();
    // 3. MFMAs: lane group lg supplies channel wc*4S + S*lg + s at step s.
    const int cw = wc * 4 * S + S * lg;
    const float* ua = Us + lds_index<KB, CB, S>(0, cw, wk * 16 + li);
    const float* vb = Vs + lds_index<TB, CB, S>(0, cw, wt * 16 + li);
#pragma unroll
    for (int xi = 0; xi < 36; ++xi) {
      if constexpr (S == 2) {
        const float2 av = *reinterpret_cast<const float2*>(ua + xi * KB * CB);
        const float2 bv = *reinterpret_cast<const float2*>(vb + xi * TB * CB);
        acc[xi] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.x, bv.x, acc[xi], 0, 0, 0);
        acc[xi] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.y, bv.y, acc[xi], 0, 0, 0);
      } else {
        acc[xi] = __builtin_amdgcn_mfma_f32_16x16x4f32(ua[xi * KB * CB], vb[xi * TB * CB], acc[xi], 0, 0, 0);
      }
    }
  }

  // Reduce the WC channel splits through LDS, 12 transform points at a time.
  if constexpr (WC > 1) {
    constexpr int XS = 12;
#pragma unroll
    for (int xs = 0; xs < 36; xs += XS) {
#pragma unroll
      for (int half = WC / 2; half >= 1; half /= 2) {
        __syncthreads();
        const int group = wk * WT + wt;
        if (wc >= half && wc < 2 * half) {
          float* slot = lds + (size_t)((group * half + (wc - half)) * XS * 4) * 64;
#pragma unroll
          for (int xi = 0; xi < XS; ++xi)
#pragma unroll
            for (int r = 0; r < 4; ++r) slot[(xi * 4 + r) * 64 + lane] = acc[xs + xi][r];
        }
        __syncthreads();
        if (wc < half) {
          const float* slot = lds + (size_t)((group * half + wc) * XS * 4) * 64;
#pragma unroll
          for (int xi = 0; xi < XS; ++xi)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[xs + xi][r] += slot[(xi * 4 + r) * 64 + lane];
        }
      }
    }
    if (wc != 0) return;
  }

  // Output transform Y = A^T M A, + bias (+ residual), activation.
  const int tt = t0 + wt * 16 + li;
  if (tt >= a.T) return;
  const int per_img = a.th * a.tw;
  const int oim = tt / per_img;
  const int rr = tt - oim * per_img;
  const int ty = rr / a.tw, tx = rr - (rr / a.tw) * a.tw;
  const bool vec4 = (a.OW % 4 == 0);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int k = k0 + wk * 16 + 4 * lg + r;
    if (k >= a.K) continue;
    float tmp[4][6];
#pragma unroll
    for (int j = 0; j < 6; ++j) {
      const float m0 = acc[0 * 6 + j][r], m1 = acc[1 * 6 + j][r], m2 = acc[2 * 6 + j][r];
      const float m3 = acc[3 * 6 + j][r], m4 = acc[4 * 6 + j][r], m5 = acc[5 * 6 + j][r];
      const float s12 = m1 + m2, d12 = m1 - m2, s34 = m3 + m4, d34 = m3 - m4;
      tmp[0][j] = m0 + s12 + s34;
      tmp[1][j] = d12 + 2.f * d34;
      tmp[2][j] = s12 + 4.f * s34;
      tmp[3][j] = d12 + 8.f * d34 + m5;
    }
    const float b = a.bias[k];
    const int64_t plane = ((int64_t)oim * a.K + k) * a.OH * a.OW;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int oy = ty * 4 + i;
      if (oy >= a.OH) break;
      const float m0 = tmp[i][0], m1 = tmp[i][1], m2 = tmp[i][2], m3 = tmp[i][3], m4 = tmp[i][4], m5 = tmp[i][5];
      const float s12 = m1 + m2, d12 = m1 - m2, s34 = m3 + m4, d34 = m3 - m4;
      float y[4];
      y[0] = m0 + s12 + s34;
      y[1] = d12 + 2.f * d34;
      y[2] = s12 + 4.f * s34;
      y[3] = d12 + 8.f * d34 + m5;
      const int64_t row = plane + (int64_t)oy * a.OW + tx * 4;
      if (vec4) {
        float4 res = make_float4(0.f, 0.f, 0.f, 0.f);
        if (a.residual) res = *reinterpret_cast<const float4*>(a.residual + row);
        float o[4] = {y[0] + b + res.x, y[1] + b + res.y, y[2] + b + res.z, y[3] + b + res.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (a.act == NHIP_ACT_RELU) o[j] = o[j] < 0.f ? 0.f : o[j];
          else if (a.act == NHIP_ACT_SIGMOID) o[j] = __frcp_rn(1.0f + __expf(-o[j]));
        }
        *reinterpret_cast<float4*>(a.out + row) = make_float4(o[0], o[1], o[2], o[3]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (tx * 4 + j < a.OW) {
            float v = y[j] + b;
            if (a.residual) v += a.residual[row + j];
            if (a.act == NHIP_ACT_RELU) v = v < 0.f ? 0.f : v;
            else if (a.act == NHIP_ACT_SIGMOID) v = __frcp_rn(1.0f + __expf(-v));
            a.out[row + j] = v;
          }
        }
      }
    }
  }
}

template <int WK, int WT, int WC, int S>
int launch_cfg(const FusedArgs& a, hipStream_t s, const char* name) {
  using Cfg = FusedCfg<WK, WT, WC, S>;
  const size_t lds = (size_t)(Cfg::V_ELEMS + Cfg::U_ELEMS) * sizeof(float);
  const dim3 grid((unsigned)ceil_div(a.T, Cfg::TB), (unsigned)ceil_div(a.K, Cfg::KB));
  static bool attr_set = false;  // dynamic LDS above 64 KB needs the attribute
  if (!attr_set) {
    NHIP_TRY(check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(&wino_fused_kernel<WK, WT, WC, S>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                       "hipFuncSetAttribute(wino_fused)"));
    attr_set = true;
  }
  NHIP_LAUNCH(name, (wino_fused_kernel<WK, WT, WC, S>), grid, dim3(kThreads), lds, s, a);
  return check_launch(name);
}

}  // namespace

// Workgroup shape: 2x2x1 (32 channels x 32 tiles per workgroup, full channel
// reduction per wave) when that alone gives at least one workgroup per CU;
// otherwise 1x1x4 (16 x 16 per workgroup, channel reduction split over the
// four waves).  NHIP_WINOGRAD_VARIANT=221|114 forces one.
int launch_conv_winograd_fused(const nhip_conv_plan* p, const float* in, const float* residual,
                               float* out, int n, int h, int w, int oh, int ow, hipStream_t s) {
  FusedArgs a{};
  a.x = in;
  a.x_bytes = (uint32_t)((size_t)n * p->g.c * h * w * sizeof(float));
  a.U = p->weight;
  a.bias = p->bias;
  a.residual = residual;
  a.out = out;
  a.C = p->g.c;
  a.H = h;
  a.W = w;
  a.K = p->g.k;
  a.OH = oh;
  a.OW = ow;
  a.th = (int)ceil_div(oh, 4);
  a.tw = (int)ceil_div(ow, 4);
  a.T = n * a.th * a.tw;
  a.m_pad = p->m_pad;
  a.c_pad = p->c_pad;
  a.pt = p->g.pt;
  a.pl = p->g.pl;
  a.act = p->g.act;
  if ((reinterpret_cast<uintptr_t>(out) & 15) || (residual && (reinterpret_cast<uintptr_t>(residual) & 15)))
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "winograd: output/residual must be 16-byte aligned");
  int variant = 0;
  if (const char* env = std::getenv("NHIP_WINOGRAD_VARIANT")) variant = std::atoi(env);
  if (variant != 221 && variant != 114) {
    const int64_t blocks221 = ceil_div(a.T, 32) * ceil_div(a.K, 32);
    variant = blocks221 >= cu_count() ? 221 : 114;
  }
  if (variant == 221) return launch_cfg<2, 2, 1, 2>(a, s, "wino_fused<2,2,1>");
  return launch_cfg<1, 1, 4, 1>(a, s, "wino_fused<1,1,4>");
}

}  // namespace nhip
