// An inverted-residual block's 1x1 expand convolution and the 3x3 depthwise
// convolution that reads it, in one kernel.  Same operations as the two
// layers (reference ConvertConvolution, NCNNToTosa.cpp:1316-1529, and
// ConvertDepthwiseConvolution, :3074-3503):
//
//   e[k][p]      = act1(sum_c W1[k][c] x[c][p] + b1[k])
//   y[k][oy][ox] = actd(sum_{kh,kw} e_pad[k][oy*s + kh][ox*s + kw] * wd[k][kh][kw] + bd[k])
//
// with e zero-padded by one pixel (padding 1), stride s = 1 or 2.
//
// A workgroup owns one image, a slice of SL = 32 or 64 expanded channels and
// a strip of R output rows (the whole plane where it fits: MobileNetV2's
// 14x14 and 7x7 blocks), so the expanded values its depthwise outputs read
// are all its own: the strip's input rows plus a one-row halo are expanded
// (the halo rows twice, by the two strips that need them) and the expanded
// tensor never reaches memory (at 56x56, batch 32, 24 -> 144 channels: 58 MB
// written and read back by the two separate layers).
//   1. The strip's input rows of every channel come into LDS as they lie
//      (16-byte loads, eight in flight per thread; the whole plane as one
//      contiguous block), zero channels up to a multiple of 16, and zeros
//      past the block; the depthwise weights and biases beside them.  An
//      MFMA column past the strip reads the next channel's first pixels (or
//      the zeros), and lands in a pixel that is not stored.
//   2. Eight waves: wave w owns expanded channels 16 (w % G) .. + 15 of the
//      slice (G = SL / 16 channel groups) and every (8 / G)-th run of TQ
//      16-pixel tiles: v_mfma_f32_16x16x4_f32, A = W1 (the wave's k-steps
//      preloaded into registers with 16-byte loads), B = x from LDS, the
//      next k-step's B values read while the current step's MFMAs run.
//      Register r of lane l of tile t is channel 4 (l / 16) + r of the
//      wave's group, pixel 16 t + l % 16.  Two waves per SIMD keep one
//      wave's LDS and memory latency behind the other's work in every
//      phase.
//   3. After a barrier the input's LDS holds the expanded planes instead,
//      (rows of the strip's window) x (W + 2), zero outside the image: e + b1,
//      act1.
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
constexpr int kWaves = kThreads / 64;
constexpr int kMaxSlice = 64;  // expanded channels per workgroup, at most
constexpr int kInFlight = 8;   // loads per thread issued before their LDS writes
constexpr int kStrip = 7;      // depthwise outputs per lane task: a column strip of 7 rows

struct EdArgs {
  const float* x;   // [N][C][H][W]
  const float* w1;  // [m_pad][ldw1], k = c (1x1)
  const float* w1q; // the same weights as [rows/32][C/4][32][4], or null
  const float* b1;  // [m_pad] (zero past K)
  const float* wd;  // [K][9]
  const float* bd;  // [K]
  float* y;         // [N][K][OH][OW]
  int C, K, H, W, OH, OW, s, ldw1, act1, actd;
  int R;            // output rows per strip (gridDim.z strips)
  int vec;          // x is 16-byte aligned
};

// LDS floats from one expanded plane to the next: rows x (W + 2) rounded up
// to 4 more than a multiple of 16
__host__ __device__ __forceinline__ int plane_stride(int rows, int w) { return (rows * (w + 2) + 15) / 16 * 16 + 4; }

__device__ __forceinline__ float act_of(float v, int act) { return (act == NHIP_ACT_RELU && v < 0.f) ? 0.f : v; }

// x / d for x >= 0 as (x + 1/2) * (1/d) in fp32: exact while quotient * d <
// 2^21 (every use here; the LDS bounds the operands): (x + 1/2) / d is at
// least 1/(2d) from an integer, the computed value within q * 2^-22 of it.
__device__ __forceinline__ int div_small(int x, float inv_d) { return (int)(((float)x + 0.5f) * inv_d); }

// The depthwise layer over the slice's padded planes (es: channel c at
// c * PS, `rows` rows of PW floats, zero outside the image), for the strip's
// `roh` output rows; yo is the strip's first output row of channel 0, OHW
// the output's channel stride.  A task is (channel, run of kStrip output
// rows, output column); consecutive threads take consecutive columns, so
// each output row of a run is one coalesced store.  The 3 x 3 window slides
// down the run in registers: S new rows of 3 values per output instead of 9.
// Every output is the reference's sum: zero, += e * w over (kh, kw) in order,
// + bias, activation, each step separately rounded.  Rows past roh (the last
// run's) are formed from clamped rows and not stored.
template <int S>
__device__ __forceinline__ void depthwise_strips(const float* es, const float* wds, const float* bds, float* yo,
                                                 int nch, int rows, int PW, int PS, int roh, int OW, int OHW,
                                                 int actd, int tid) {
  const int nrb = (roh + kStrip - 1) / kStrip;
  const int T = nrb * OW;  // tasks per channel
  const float inv_t = 1.f / (float)T, inv_ow = 1.f / (float)OW;
  for (int e = tid; e < nch * T; e += kThreads) {
    // (24-bit multiplies: every product here is below 2^23)
    const int c = div_small(e, inv_t);
    const int rem = e - __mul24(c, T);
    const int rb = div_small(rem, inv_ow);
    const int ox = rem - __mul24(rb, OW);
    const float* ec = es + __mul24(c, PS) + ox * S;
    float w[9];
#pragma unroll
    for (int t = 0; t < 9; ++t) w[t] = wds[__mul24(c, 9) + t];
    const float bias = bds[c];
    const int oy0 = rb * kStrip;
    float* yc = yo + __mul24(c, OHW) + ox;
    auto row = [&](int r, float* v) {
      const float* q = ec + __mul24(min(r, rows - 1), PW);
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
      if (oy0 + i < roh) yc[__mul24(oy0 + i, OW)] = act_of(sum, actd);
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

// Strip geometry of workgroup z: output rows oy0 .. oy0 + roh - 1 read
// expanded rows iy_lo .. iy_lo + rows - 1 (iy_lo = oy0 * s - 1), of which
// the image holds iy_a .. iy_a + rows_in - 1.
struct Strip {
  int oy0, roh, iy_lo, rows, iy_a, rows_in;
};
__host__ __device__ __forceinline__ Strip strip_of(int z, int R, int OH, int H, int s) {
  Strip t;
  t.oy0 = z * R;
  t.roh = min(R, OH - t.oy0);
  t.iy_lo = t.oy0 * s - 1;
  t.rows = (t.roh - 1) * s + 3;
  t.iy_a = max(t.iy_lo, 0);
  t.rows_in = min(t.iy_lo + t.rows - 1, H - 1) - t.iy_a + 1;
  return t;
}

// TQ = 16-pixel tiles per wave; NK = C_pad / 4 k-steps (C_pad: C rounded up
// to 16); SL = expanded channels per workgroup.
template <int TQ, int NK, int SL>
__global__ __launch_bounds__(kThreads) void expand_dw_kernel(EdArgs a) {
  constexpr int G = SL / 16, WPG = kWaves / G;  // channel groups, waves per group
  constexpr int CP = NK * 4;
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int k0 = blockIdx.x * SL, img = blockIdx.y;
  const Strip st = strip_of(blockIdx.z, a.R, a.OH, a.H, a.s);
  const int HW = a.H * a.W, OHW = a.OH * a.OW;
  const int HWs = st.rows_in * a.W;  // pixels of the strip's input block, per channel
  const int PW = a.W + 2;            // padded expanded rows
  const int PS = plane_stride(st.rows, a.W);
  // LDS: [input block, later expanded planes][SL x 9 depthwise weights][SL biases]
  const int tot = CP * HWs;
  constexpr int kSlack = 16 * WPG * TQ;  // zeros past the block
  const int region = max(tot + kSlack, SL * PS);
  float* xs = lds;
  float* wds = lds + region;
  float* bds = wds + SL * 9;
  const int grp = wave % G, part = wave / G;
  const int chw = 16 * grp + 4 * (lane >> 4);  // slice channel of MFMA register 0

  // ---- 1. every global read of the phase is issued before the first LDS
  // write waits for one: the A operand, the 1x1 bias, the depthwise
  // parameters, then the input block.
  // k-step j of lane group g = l / 16 reduces input channel
  // 16 (j / 4) + 4 g + j % 4, so the A operand of steps 4q .. 4q + 3 is one
  // float4, W1[k0 + 16 grp + l%16][16 q + 4 g ..+ 3], and four lanes read 64
  // contiguous bytes of a weight row (rows are 16-float aligned and zero
  // past C; rows past K are the plan's zero padding up to m_pad).  Grouped
  // layout: lane group g's float4 of step q is group 4q + g of the row's
  // 32-row block, so 16 lanes read 256 contiguous bytes.
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
  static_assert(kMaxSlice * 9 <= 2 * kThreads && kMaxSlice <= kThreads, "depthwise parameters: two per thread");
  const int nch = min(SL, a.K - k0);
  const int e1 = tid + kThreads;
  const float wd0 = tid < nch * 9 ? a.wd[(int64_t)k0 * 9 + tid] : 0.f;
  const float wd1 = e1 < nch * 9 ? a.wd[(int64_t)k0 * 9 + e1] : 0.f;
  const float bd0 = tid < nch ? a.bd[k0 + tid] : 0.f;
  const float* xi = a.x + (int64_t)img * a.C * HW + (int64_t)st.iy_a * a.W;
  const int treal = a.C * HWs;  // input values; channels C .. CP - 1 are zeros
  if (st.rows_in == a.H) {
    // the whole plane: the image's channels are one contiguous block
    if (a.vec && treal % 4 == 0) {
      const float4* src = reinterpret_cast<const float4*>(xi);
      const int n4 = treal >> 2;
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
      for (int base = tid; base < treal; base += kThreads * kInFlight) {
        float v[kInFlight];
#pragma unroll
        for (int i = 0; i < kInFlight; ++i) v[i] = xi[min(base + i * kThreads, treal - 1)];
#pragma unroll
        for (int i = 0; i < kInFlight; ++i)
          if (base + i * kThreads < treal) xs[base + i * kThreads] = v[i];
      }
    }
  } else {
    // a strip: rows iy_a .. of each channel, HWs contiguous values per
    // channel; element e is (c, e - c * n)
    if (a.vec && a.W % 4 == 0) {
      const int n = HWs / 4, tn = a.C * n;
      const float inv_n = 1.f / (float)n;
      for (int base = tid; base < tn; base += kThreads * kInFlight) {
        float4 v[kInFlight];
#pragma unroll
        for (int i = 0; i < kInFlight; ++i) {
          const int e = min(base + i * kThreads, tn - 1);
          const int c = div_small(e, inv_n);
          v[i] = reinterpret_cast<const float4*>(xi + (int64_t)c * HW)[e - c * n];
        }
#pragma unroll
        for (int i = 0; i < kInFlight; ++i)
          if (base + i * kThreads < tn) reinterpret_cast<float4*>(xs)[base + i * kThreads] = v[i];
      }
    } else {
      const int n = HWs, tn = a.C * n;
      const float inv_n = 1.f / (float)n;
      for (int base = tid; base < tn; base += kThreads * kInFlight) {
        float v[kInFlight];
#pragma unroll
        for (int i = 0; i < kInFlight; ++i) {
          const int e = min(base + i * kThreads, tn - 1);
          const int c = div_small(e, inv_n);
          v[i] = xi[(int64_t)c * HW + (e - c * n)];
        }
#pragma unroll
        for (int i = 0; i < kInFlight; ++i)
          if (base + i * kThreads < tn) xs[base + i * kThreads] = v[i];
      }
    }
  }
  for (int i = treal + tid; i < tot + kSlack; i += kThreads) xs[i] = 0.f;
  if (tid < SL * 9) wds[tid] = wd0;
  if (e1 < SL * 9) wds[e1] = wd1;
  if (tid < SL) bds[tid] = bd0;
  __syncthreads();

  // ---- 2. expand: the wave's 16 channels x its tiles part * TQ .. + TQ - 1
  // (tiles past the strip compute values that are not stored; their reads
  // stay inside the block and the zeros after it)
  v4f acc[TQ];
#pragma unroll
  for (int t = 0; t < TQ; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  const int t0 = part * TQ;
  const float* xb = xs + 4 * (lane >> 4) * HWs + (lane & 15) + 16 * t0;
  // step j + 1's B values are read while step j's MFMAs run
  float bv_cur[TQ], bv_next[TQ];
#pragma unroll
  for (int t = 0; t < TQ; ++t) bv_cur[t] = xb[16 * t];
#pragma unroll  // whole: av[j] stays in registers
  for (int j = 0; j < NK; ++j) {
    if (j + 1 < NK) {
      const float* xr = xb + (16 * ((j + 1) >> 2) + ((j + 1) & 3)) * HWs;
#pragma unroll
      for (int t = 0; t < TQ; ++t) bv_next[t] = xr[16 * t];
    }
#pragma unroll
    for (int t = 0; t < TQ; ++t) acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j], bv_cur[t], acc[t], 0, 0, 0);
    // scheduling order: the next step's LDS reads, then this step's MFMAs
    // (left alone, the compiler reads each value right before its MFMA and
    // waits for it there)
    __builtin_amdgcn_sched_group_barrier(0x100, TQ, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, TQ, 0);
#pragma unroll
    for (int t = 0; t < TQ; ++t) bv_cur[t] = bv_next[t];
  }
  __syncthreads();  // every wave done with the input block

  // ---- 3. expanded planes, PS floats apart (the four register rows of an
  // MFMA result, 4 planes apart, fall on different LDS banks): zeros first,
  // then the rows inside the image, bias + act1.  Planes past K come out
  // zero (zero weight rows and bias) and are never read.
  float* es = xs;
  for (int e = tid; e < SL * PS / 4; e += kThreads) reinterpret_cast<float4*>(es)[e] = float4{0.f, 0.f, 0.f, 0.f};
  __syncthreads();
  {
    const float inv_w = 1.f / (float)a.W;
    const bool relu = a.act1 == NHIP_ACT_RELU;
    // origin of the lane's first plane: window row of input row iy_a, column 1
    float* eb = es + __mul24(chw, PS) + (st.iy_a - st.iy_lo) * PW + 1;
#pragma unroll
    for (int t = 0; t < TQ; ++t) {
      const int p = 16 * (t0 + t) + (lane & 15);
      if (p < HWs) {
        const int py = div_small(p, inv_w), px = p - __mul24(py, a.W);
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

  // ---- 4. depthwise 3x3 in the reference's order, in column runs
  float* yo = a.y + ((int64_t)img * a.K + k0) * OHW + (int64_t)st.oy0 * a.OW;
  if (a.s == 1)
    depthwise_strips<1>(es, wds, bds, yo, nch, st.rows, PW, PS, st.roh, a.OW, OHW, a.actd, tid);
  else
    depthwise_strips<2>(es, wds, bds, yo, nch, st.rows, PW, PS, st.roh, a.OW, OHW, a.actd, tid);
}

// A launch configuration: SL expanded channels and R output rows per
// workgroup, TQ tiles per wave.
struct EdCfg {
  int sl = 0, r = 0, tq = 0;
};

// Instantiated tile counts per wave, by slice width.
constexpr int kTq64[] = {1, 2, 4, 7, 8};
constexpr int kTq32[] = {4, 7, 8, 9};

int lds_floats(int cp, int w, int rows, int rows_in, int sl, int tq) {
  const int wpg = kWaves / (sl / 16);
  return std::max(cp * rows_in * w + 16 * wpg * tq, sl * plane_stride(rows, w)) + sl * 10;
}

// The configuration for an expand (c input channels, k outputs) + depthwise
// (stride s) pair on h x w planes, or false.  Whole planes take the 64-wide
// slice when it fits the LDS (one or two workgroups per CU: the 14x14 and
// 7x7 shapes measured); other planes are cut into strips, the candidate
// (slice, rows) that fits two workgroups per CU chosen for the least
// expand work counted with its halo rows and slice padding, scaled up when
// a 32-image batch would give fewer than two workgroups per CU (the choice
// does not depend on the batch), strip heights that are whole 7-row
// depthwise runs first (at 28x28: 7-row strips of 32 channels, 15.3 us at
// stride 1 against 17.2 for 14-row strips and 19.3 for 5-row ones; 12.0 us
// at stride 2, the fastest 11.5).  NHIP_PWDW_CFG="sl,r" forces one.
bool ed_config(int c, int k, int h, int w, int s, EdCfg* out) {
  const int cp = (int)round_up(c, 16);
  const int oh = (h - 1) / s + 1;
  const int nk = cp / 4;
  int fsl = 0, fr = 0;
  if (const char* env = setting("NHIP_PWDW_CFG")) std::sscanf(env, "%d,%d", &fsl, &fr);
  double best = 0;
  bool found = false;
  // first pass: strips of whole 7-row depthwise runs (or the whole plane);
  // second pass, if none fits: any strip height
  for (int pass = 0; pass < 2 && !found; ++pass)
  for (int sl : {64, 32}) {
    if (fsl && sl != fsl) continue;
    const bool nk_ok = sl == 64 ? (nk == 8 || nk == 16 || nk == 24 || nk == 40) : (nk == 4 || nk == 8 || nk == 16);
    if (!nk_ok) continue;
    for (int r = oh; r >= 1; --r) {
      if (fr && r != fr) continue;
      if (pass == 0 && !fr && r != oh && r % kStrip != 0) continue;
      const int rows = (r - 1) * s + 3;
      const int rows_in = std::min(rows, h);
      const int pt = (int)ceil_div(rows_in * w, 16);
      const int wpg = kWaves / (sl / 16);
      const int need = (int)ceil_div(pt, wpg);
      int tq = 0;
      if (sl == 64) {
        for (int v : kTq64)
          if (v >= need) {
            tq = v;
            break;
          }
      } else {
        for (int v : kTq32)
          if (v >= need) {
            tq = v;
            break;
          }
      }
      if (!tq) continue;
      const int64_t bytes = (int64_t)lds_floats(cp, w, rows, rows_in, sl, tq) * 4;
      const bool whole = r == oh;
      if (bytes > (whole ? 160 * 1024 : 80 * 1024)) continue;
      const int strips = (int)ceil_div(oh, r);
      const int64_t wgs = ceil_div(k, sl) * (int64_t)strips * 32;
      double cost = (double)ceil_div(k, sl) * sl * strips * rows * std::max(1.0, 512.0 / (double)wgs);
      // the whole plane where it fits, in 64-wide slices, or 32-wide ones
      // for 64 input channels (measured at 14x14, batch 32: 64 -> 384 13.1
      // us with 32-wide slices against 13.8; 96 -> 576 24.4 against 23.2 us
      // at stride 1 and 19.9 against 18.7 at stride 2)
      if (whole && !fsl && sl == (nk == 16 ? 32 : 64)) cost = 0;
      if (!found || cost < best) {
        found = true;
        best = cost;
        *out = EdCfg{sl, r, tq};
      }
    }
  }
  return found;
}

template <int TQ, int NK, int SL>
int launch_one(const EdArgs& a, int n, int strips, int lds, hipStream_t s) {
  NHIP_TRY(ensure_dynamic_lds(reinterpret_cast<const void*>(&expand_dw_kernel<TQ, NK, SL>), lds));
  NHIP_LAUNCH("expand_dw_f32", (expand_dw_kernel<TQ, NK, SL>),
              dim3((unsigned)ceil_div(a.K, SL), (unsigned)n, (unsigned)strips), dim3(kThreads), lds, s, a);
  return check_launch("expand_dw_f32");
}

template <int SL, int NK>
int launch_tq(const EdArgs& a, int tq, int n, int strips, int lds, hipStream_t s) {
  if constexpr (SL == 64) {
    switch (tq) {
      case 1: return launch_one<1, NK, 64>(a, n, strips, lds, s);
      case 2: return launch_one<2, NK, 64>(a, n, strips, lds, s);
      case 4: return launch_one<4, NK, 64>(a, n, strips, lds, s);
      case 7: return launch_one<7, NK, 64>(a, n, strips, lds, s);
      case 8: return launch_one<8, NK, 64>(a, n, strips, lds, s);
    }
  } else {
    switch (tq) {
      case 4: return launch_one<4, NK, 32>(a, n, strips, lds, s);
      case 7: return launch_one<7, NK, 32>(a, n, strips, lds, s);
      case 8: return launch_one<8, NK, 32>(a, n, strips, lds, s);
      case 9: return launch_one<9, NK, 32>(a, n, strips, lds, s);
    }
  }
  return fail(NHIP_STATUS_UNSUPPORTED, "expand + depthwise: no kernel for the tile count");
}

}  // namespace

// Whether the fused kernel takes the pair: an fp32 1x1 stride-1 unpadded
// convolution on the implicit-GEMM plan (16, 24, 32, 64, 96 or 160 input
// channels: the expand layers of MobileNetV2) feeding a 3x3 depthwise
// convolution (stride 1 or 2, padding 1, dilation 1) over its channels,
// activations none or ReLU, with a configuration that fits the LDS.
// NHIP_PWDW=0 never; 2 every such pair; by default planes of at most 784
// pixels.  Measured at batch 32 against the expand followed by the
// depthwise -> 1x1 pair (or the three layers), expand + depthwise and then
// the 1x1: 26.1 against 33.6 us at 14x14 (64 -> 384 -> 64), 28.4 against
// 30.2 at 28x28 (32 -> 192 -> 32), 24.2 against 34.3 at 28x28 stride 2; at
// 56x56 61.1 against 53.6 and at 112x112 77.5 against 67.9 (many strips,
// each workgroup's phases serial: per-workgroup latency dominates).
bool pwdw_supported(const nhip_conv_plan* pw, const nhip_conv_plan* dw, int n, int h, int w) {
  if (!pw || !dw || pw->kind != PlanKind::ConvF32 || dw->kind != PlanKind::DwConvF32) return false;
  const int mode = setting_int("NHIP_PWDW", 1);
  if (mode == 0) return false;
  const ConvGeom& p = pw->g;
  const ConvGeom& d = dw->g;
  if (pw->algorithm != NHIP_CONV_ALGO_IMPLICIT_GEMM || p.kh != 1 || p.kw != 1 || p.sh != 1 || p.sw != 1 || p.pt ||
      p.pb || p.pl || p.pr || pw->kred != p.c)
    return false;
  if (!(p.c == 16 || p.c == 24 || p.c == 32 || p.c == 64 || p.c == 96 || p.c == 160)) return false;
  // the row-major weights' rows hold C rounded up to 16 (zero past C)
  if (pw->kred_pad < (int)round_up(p.c, 16) || pw->kred_pad % 4) return false;
  if (d.c != p.k || d.k != p.k || d.kh != 3 || d.kw != 3 || d.dh != 1 || d.dw != 1 || d.sh != d.sw ||
      (d.sh != 1 && d.sh != 2) || d.pt != 1 || d.pb != 1 || d.pl != 1 || d.pr != 1)
    return false;
  if ((p.act != NHIP_ACT_NONE && p.act != NHIP_ACT_RELU) || (d.act != NHIP_ACT_NONE && d.act != NHIP_ACT_RELU))
    return false;
  if (mode != 2 && h * w > 784) return false;
  if (h < 1 || w < 1 || w > 4096 || h > 4096) return false;
  EdCfg c;
  if (!ed_config(p.c, p.k, h, w, d.sh, &c)) return false;
  const int oh = (h - 1) / d.sh + 1, ow = (w - 1) / d.sw + 1;
  return (int64_t)n * p.c * h * w < INT32_MAX && (int64_t)n * p.k * oh * ow < INT32_MAX && n <= 65535 &&
         ceil_div(oh, c.r) <= 65535;
}

int launch_pwdw_f32(const nhip_conv_plan* pw, const nhip_conv_plan* dw, const float* in, float* out, int n, int h,
                    int w, hipStream_t s) {
  if (!pwdw_supported(pw, dw, n, h, w))
    return fail(NHIP_STATUS_UNSUPPORTED, "expand + depthwise: this pair or shape has no fused kernel");
  if (n == 0) return ok();
  EdArgs a{};
  a.x = in;
  a.w1 = pw->weight;
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
  a.vec = (reinterpret_cast<uintptr_t>(in) & 15) == 0;
  EdCfg c;
  if (!ed_config(a.C, a.K, h, w, a.s, &c)) return fail(NHIP_STATUS_UNSUPPORTED, "expand + depthwise: no configuration");
  a.R = c.r;
  // the grouped copy when its rows (K rounded up to 32) cover every slice and
  // its channel groups are the kernel's (C a multiple of 16)
  a.w1q = pw->weight_kq != nullptr && pw->kq_vw == 4 && a.C % 16 == 0 &&
                  round_up(pw->g.k, 32) == round_up(pw->g.k, c.sl)
              ? pw->weight_kq
              : nullptr;
  const int cp = (int)round_up(a.C, 16);
  const int rows = (c.r - 1) * a.s + 3;
  const int lds = lds_floats(cp, w, rows, std::min(rows, h), c.sl, c.tq) * (int)sizeof(float);
  const int strips = (int)ceil_div(a.OH, c.r);
  const int nk = cp / 4;
  if (c.sl == 64) {
    switch (nk) {
      case 8: return launch_tq<64, 8>(a, c.tq, n, strips, lds, s);
      case 16: return launch_tq<64, 16>(a, c.tq, n, strips, lds, s);
      case 24: return launch_tq<64, 24>(a, c.tq, n, strips, lds, s);
      case 40: return launch_tq<64, 40>(a, c.tq, n, strips, lds, s);
    }
  } else {
    switch (nk) {
      case 4: return launch_tq<32, 4>(a, c.tq, n, strips, lds, s);
      case 8: return launch_tq<32, 8>(a, c.tq, n, strips, lds, s);
      case 16: return launch_tq<32, 16>(a, c.tq, n, strips, lds, s);
    }
  }
  return fail(NHIP_STATUS_UNSUPPORTED, "expand + depthwise: input channels outside the kernel's range");
}

}  // namespace nhip
