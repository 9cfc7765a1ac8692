// Winograd F(4x4, 3x3) batched GEMM with the output transform fused: the
// 36 point-wise products M[xi] = U[xi] V[xi] and Y = A^T M A in one kernel,
// so M never leaves the CU (the three-kernel path in winograd.hip writes and
// re-reads M through HBM).  V comes from wino_input_transform<true>
// (winograd.hip) in the channel-pair layout [36][c_pad/2][t_pad][2].
//
// The input transform stays a separate, HBM-bound kernel on purpose: on
// gfx950 the fp32 MFMA and fp32 VALU work of the waves on one SIMD do not
// overlap (measured: time(MFMA + VALU) ~ time(MFMA) + time(VALU)), so
// transforming patches inside the GEMM costs MFMA time, at 32 output
// channels per workgroup about 0.7 x the MFMA work of a chunk.
//
// Work decomposition.  A workgroup owns 32 tiles x 32 output channels for
// all 36 transform points xi and runs 8 waves in two roles:
//   * 4 load waves copy, for a chunk of 8 input channels, the V slice
//     (36 x 8 x 32 floats) and the U slice (36 x 32 x 8, transformed
//     weights prepacked on the host) from HBM into LDS, prefetching two
//     chunks ahead in registers;
//   * 4 MFMA waves, a 2 x 2 grid of 16 (channel) x 16 (tile) blocks, each
//     accumulate their block for all 36 xi with v_mfma_f32_16x16x4_f32
//     (36 x 4 accumulator registers per lane).
// LDS holds two chunk slots (2 x 72 KB): while the MFMA waves consume chunk
// i from one slot, the load waves fill the other with chunk i + 1; one
// workgroup barrier per chunk hands the slots over.
//
// In the 16x16 MFMA result layout register r of lane l holds (row
// 4*(l/16)+r, column l%16) for every xi, so an MFMA lane owns all 36 values
// of four (k, t) pairs and the output transform A^T M A runs in registers.
//
// Layers with few tiles split the input channels over `splits` workgroups
// (grid), each writing its partial output transform (linear in M) to a
// workspace; wino_fused_reduce sums the parts and applies bias, residual and
// activation.
#include <cstdlib>
#include <cstring>

#include "nhip_internal.h"

namespace nhip {
namespace {

constexpr int kThreads = 512;                 // 4 MFMA waves + 4 load waves
constexpr int kTB = 32;                       // tiles per workgroup
constexpr int kKB = 32;                       // output channels per workgroup
constexpr int kCB = 8;                        // input channels per chunk
constexpr int kVElems = 36 * kTB * kCB;       // V chunk [36][kCB/2][kTB][2]
constexpr int kUElems = 36 * kKB * kCB;       // U chunk [36][kCB/2][kKB][2]
constexpr int kSlotElems = kVElems + kUElems;
constexpr int kLdsBytes = 2 * kSlotElems * (int)sizeof(float);  // 147456
constexpr int kProducers = 256;               // load threads
constexpr int kULoads = kUElems / 4 / kProducers;  // 16-byte U loads per thread and chunk
constexpr int kVLoads = kVElems / 4 / kProducers;  // 16-byte V loads per thread and chunk
constexpr int kXcds = 8;                      // MI355X: workgroup L runs on XCD L % 8
static_assert(kLdsBytes >= kKB * kTB * 16 * (int)sizeof(float), "the staged output tiles fit in the chunk slots");
static_assert(kUElems % (4 * kProducers) == 0 && kVElems % (4 * kProducers) == 0,
              "whole 16-byte loads per thread");
static_assert(kTB == 32 && kKB == 32 && kCB == 8, "the load mappings below assume 32 x 32 x 8");

typedef float v2f __attribute__((ext_vector_type(2)));

struct FusedArgs {
  const float* x;       // direct variant: the input [N][C][H][W] (<= 1 GiB)
  const float* V;       // otherwise: [36][c_pad/2][t_pad][2]
  const float* U;       // [c_pad/8][36][4][m_pad][2]
  const float* bias;    // [m_pad]
  const float* residual;
  float* out;           // [N][K][OH][OW]; with splits > 1 the parts [splits][N][K][OH][OW]
  int K, OH, OW, th, tw, T, t_pad, m_pad, c_pad;
  int nt, nk, splits, per;  // tile blocks, channel blocks, channel splits, chunks per split
  // Tile blocks (mode = 0, 1, 2):
  //   0  whole images, R = (32 / tw) / th * th tile rows (th <= 32 / tw): a
  //      block's outputs for one image are one contiguous run over its 32
  //      channels;
  //   1  up to R = 32 / tw tile rows of one image (th > 32 / tw), blocks
  //      restarting at each image (bpi per image): one contiguous run per
  //      channel;
  //   2  32-tile pieces of a tile row (tw > 32), bpr per row.
  // G = N * th tile rows.
  int mode, R, bpi, bpr, G;
  int C, H, W, pt, pl;  // direct variant: input geometry
  uint32_t x_bytes;     // size of x
  uint32_t v_bytes;     // size of V (< 2^31)
  uint32_t u_bytes;     // size of U (< 2^31)
};

template <int ACT>
__device__ __forceinline__ float activate(float v) {
  if constexpr (ACT == NHIP_ACT_RELU) return v < 0.f ? 0.f : v;
  if constexpr (ACT == NHIP_ACT_SIGMOID) return __frcp_rn(1.0f + __expf(-v));
  return v;
}

// The load waves: copy the V and U slices of chunks ch_begin ..
// ch_begin + n - 1 into LDS, chunk i into slot i & 1 in iteration i, one
// workgroup barrier per iteration (n + 1 in all).  Both operands sit in LDS
// as [xi][channel pair][row][2], so the MFMA lanes' 8-byte reads of 16
// consecutive rows hit 32 distinct banks; in HBM both are stored so that a
// chunk's slice for one (xi, channel pair) is one contiguous 256-byte run
// (32 rows x 2 channels).  Element e4 = it*256 + p (16-byte units) of a slice
// is xi = e4 / 64, pair (e4 % 64) / 16, rows 2*(e4 % 16) and +1, and lands at
// slot + e4*4.  Consecutive it are 4 transform points apart: a wave-uniform
// byte stride, passed as the scalar offset (which the range check excludes;
// an offset of 2^31 >= the buffer size reads as 0).
__device__ __forceinline__ void load_role(const FusedArgs& a, float* lds, int p, int t0, int k0, int ch_begin,
                                          int n) {
  const __amdgpu_buffer_rsrc_t vr = make_rsrc(a.V, a.v_bytes);
  const __amdgpu_buffer_rsrc_t ur = make_rsrc(a.U, a.u_bytes);
  const int xi0 = p >> 6, cp = (p & 63) >> 4, r2 = 2 * (p & 15);
  // V[xi][c/2][t][2]: pair planes of t_pad x 2 floats, xi planes of c_pad/2 pairs
  const uint32_t v_lane = (uint32_t)(((xi0 * (a.c_pad / 2) + cp) * a.t_pad + t0 + r2) * 2 * 4);
  const uint32_t v_it = (uint32_t)(4 * (a.c_pad / 2) * a.t_pad * 2 * 4);
  const uint32_t v_ch = (uint32_t)(4 * a.t_pad * 2 * 4);
  // U[c/8][xi][pair][k][2]
  const uint32_t u_lane = (uint32_t)((((xi0 * 4 + cp) * a.m_pad + k0 + r2) * 2) * 4);
  const uint32_t u_it = (uint32_t)(4 * 4 * a.m_pad * 2 * 4);
  const uint32_t u_ch = (uint32_t)(36 * 4 * a.m_pad * 2 * 4);

  // Two chunks in flight.  Loads are issued unconditionally (past this
  // workgroup's last chunk they are pointed out of range and return 0): a
  // conditional load would make the compiler copy the loaded registers at
  // the join, which waits for the loads there and defeats the prefetch.
  v4f vA[kVLoads], vB[kVLoads], uA[kULoads], uB[kULoads];
  auto load = [&](int ch, bool live, v4f (&v)[kVLoads], v4f (&u)[kULoads]) {
    const uint32_t vo = live ? v_lane + (uint32_t)ch * v_ch : 0x80000000u;
    const uint32_t uo = live ? u_lane + (uint32_t)ch * u_ch : 0x80000000u;
#pragma unroll
    for (int it = 0; it < kVLoads; ++it)
      v[it] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(vr, vo, it * v_it, 0));
#pragma unroll
    for (int it = 0; it < kULoads; ++it)
      u[it] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(ur, uo, it * u_it, 0));
  };
  auto fill = [&](int slot_idx, v4f (&v)[kVLoads], v4f (&u)[kULoads]) {
    float* slot = lds + slot_idx * kSlotElems;
#pragma unroll
    for (int it = 0; it < kVLoads; ++it) *reinterpret_cast<v4f*>(slot + (it * kProducers + p) * 4) = v[it];
#pragma unroll
    for (int it = 0; it < kULoads; ++it)
      *reinterpret_cast<v4f*>(slot + kVElems + (it * kProducers + p) * 4) = u[it];
  };

  load(ch_begin, n > 0, vA, uA);
  load(ch_begin + 1, n > 1, vB, uB);
  // Iteration i: chunk i (if any) into slot i & 1, then the barrier.
  for (int i = 0; i <= n; i += 2) {
    if (i < n) fill(0, vA, uA);
    load(ch_begin + i + 2, i + 2 < n, vA, uA);
    __syncthreads();  // slot 0 full; slot 1 consumed
    if (i + 1 < n) fill(1, vB, uB);
    load(ch_begin + i + 3, i + 3 < n, vB, uB);
    if (i + 1 <= n) __syncthreads();  // slot 1 full; slot 0 consumed
  }
}

// A workgroup's share of the work: tile block tb (mode 0/1/2 above), output
// channels k0 .. k0 + 31, and chunks ch_begin .. ch_begin + n - 1 of channel
// split cs (chunks of `cb` input channels).
struct Block {
  int tb, kb, cs, k0, g0, nrows, tx_a, t0, ntiles, ch_begin, n;
};

__device__ __forceinline__ Block block_of(const FusedArgs& a, int cb) {
  Block b;
  // XCD-contiguous renumbering: each XCD gets a contiguous range of logical
  // blocks, ordered (tile block, split, channel block) with the channel
  // block fastest, so the workgroups that read the same V slices share an L2.
  {
    const int total = a.nt * a.nk * a.splits;
    const int L = blockIdx.x;
    const int x = L % kXcds, q = L / kXcds;
    const int logical = x * (total / kXcds) + min(x, total % kXcds) + q;
    b.kb = logical % a.nk;
    const int rest = logical / a.nk;
    b.cs = rest % a.splits;
    b.tb = rest / a.splits;
  }
  b.k0 = b.kb * kKB;
  if (a.mode == 0) {
    b.g0 = b.tb * a.R;
    b.nrows = min(a.R, a.G - b.g0);
    b.tx_a = 0;
  } else if (a.mode == 1) {
    const int im = b.tb / a.bpi, ty0 = (b.tb - im * a.bpi) * a.R;
    b.g0 = im * a.th + ty0;
    b.nrows = min(a.R, a.th - ty0);
    b.tx_a = 0;
  } else {
    b.g0 = b.tb / a.bpr;
    b.nrows = 1;
    b.tx_a = (b.tb - b.g0 * a.bpr) * kTB;
  }
  b.t0 = b.g0 * a.tw + b.tx_a;
  b.ntiles = a.mode == 2 ? min(kTB, a.tw - b.tx_a) : b.nrows * a.tw;
  const int nch = a.c_pad / cb;
  b.ch_begin = b.cs * a.per;
  b.n = max(0, min(nch, b.ch_begin + a.per) - b.ch_begin);
  return b;
}

// Output tiles staged in LDS: Ys[k][tile][16] (64 KB for 32 x 32), the four
// 4-float rows of a tile rotated by the tile index so that the MFMA lanes'
// 16-byte writes of consecutive tiles spread over the banks.
__device__ __forceinline__ int ys_off(int kk, int tl, int i) {
  return (kk * kTB + tl) * 16 + ((i ^ tl) & 3) * 4;
}

// Y = A^T M A for the lane's four (k, tile) pairs of the 16x16 MFMA layout
// (wave (wk, wt), lane (li, q)), into Ys.
__device__ __forceinline__ void y_to_lds(const v4f (&acc)[36], float* lds, int wk, int wt, int li, int q) {
  const int tl = wt * 16 + li;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
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
    const int kk = wk * 16 + 4 * q + r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float m0 = tmp[i][0], m1 = tmp[i][1], m2 = tmp[i][2], m3 = tmp[i][3], m4 = tmp[i][4], m5 = tmp[i][5];
      const float s12 = m1 + m2, d12 = m1 - m2, s34 = m3 + m4, d34 = m3 - m4;
      *reinterpret_cast<v4f*>(lds + ys_off(kk, tl, i)) =
          v4f{m0 + s12 + s34, d12 + 2.f * d34, s12 + 4.f * s34, d12 + 8.f * d34 + m5};
    }
  }
}

// Write-out of the staged tiles by NW waves, wave w taking channels w + NW*j.
// Outputs are written in memory order.  All residual loads of a group of
// four channels are issued before its first store: vmcnt counts loads and
// stores in issue order, so a load issued after a store would make its wait
// include the store.  FINAL: act(Y + bias (+ residual)); otherwise the raw
// part of channel split b.cs for wino_fused_reduce.
template <int NW, int ACT, bool FINAL>
__device__ __forceinline__ void write_out(const FusedArgs& a, const Block& bk, const float* lds, int lane,
                                          int wave) {
  constexpr int JW = kKB / NW;  // channels per wave
  float* dst = a.out + (FINAL ? 0 : (int64_t)bk.cs * (a.G / a.th) * a.K * a.OH * a.OW);
  const int OHW = a.OH * a.OW;
  const int k0 = bk.k0;
  if (a.mode == 0) {
    // Whole images: per (image, channel) plane P = OH*OW <= 16 * 32 floats; a
    // lane's pixels p = lane + 64m (m < 8) and their (tile, row, column)
    // within the image are computed once, packed as tile*16 + row*4 + column.
    int tij[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int pix = lane + 64 * m;
      const int oy = pix / a.OW, ox = pix - (pix / a.OW) * a.OW;
      tij[m] = pix < OHW ? ((oy >> 2) * a.tw + (ox >> 2)) * 16 + (oy & 3) * 4 + (ox & 3) : -1;
    }
    const int nimg = bk.nrows / a.th;
    const int im0 = bk.g0 / a.th;
    const int img_tiles = a.th * a.tw;
    for (int il = 0; il < nimg; ++il) {
      for (int j = 0; j < JW; ++j) {
        const int kk = wave + NW * j, k = k0 + kk;
        if (k >= a.K) break;
        const float b = FINAL ? a.bias[k] : 0.f;
        const int64_t base = ((int64_t)(im0 + il) * a.K + k) * OHW;
        float res[8];
#pragma unroll
        for (int m = 0; m < 8; ++m)
          res[m] = (FINAL && a.residual && tij[m] >= 0) ? a.residual[base + lane + 64 * m] : 0.f;
#pragma unroll
        for (int m = 0; m < 8; ++m)
          if (tij[m] >= 0) {
            const int tl = il * img_tiles + (tij[m] >> 4);
            const float y = lds[ys_off(kk, tl, (tij[m] >> 2) & 3) + (tij[m] & 3)];
            dst[base + lane + 64 * m] = activate<ACT>(y + b + res[m]);
          }
      }
    }
    return;
  }
  if (a.mode == 1) {
    // One contiguous run of count = orows x OW floats per channel; a group
    // of 4 channels holds <= 4 x 512 floats, i.e. <= 8 float4 (32 float)
    // slots per lane, E = lane*VW + 64*VW*u over the group's runs.
    const int im = bk.g0 / a.th, ty0 = bk.g0 - im * a.th;
    const int orows = min(4 * bk.nrows, a.OH - 4 * ty0);
    const int count = orows * a.OW;
    const int64_t row0 = (int64_t)4 * ty0 * a.OW;
#pragma unroll
    for (int jg = 0; jg < JW; jg += 4) {
      // channels kk = wave + NW*(jg + j), j < 4
      int nk_g = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) nk_g += (k0 + wave + NW * (jg + j) < a.K) ? 1 : 0;
      float bias4[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = k0 + wave + NW * (jg + j);
        bias4[j] = (FINAL && k < a.K) ? a.bias[k] : 0.f;
      }
      auto slot = [&](int E, int& j, int64_t& o, int& yo) {
        j = E / count;
        const int e = E - j * count;
        const int i = e / a.OW, x = e - i * a.OW;
        const int kk = wave + NW * (jg + j);
        o = ((int64_t)im * a.K + k0 + kk) * OHW + row0 + e;
        yo = ys_off(kk, (i >> 2) * a.tw + (x >> 2), i & 3) + (x & 3);
      };
      if (a.OW % 4 == 0) {
        v4f res[8];
        int64_t o[8];
        int yo[8], jj[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int E = lane * 4 + 256 * u;
          res[u] = v4f{0.f, 0.f, 0.f, 0.f};
          jj[u] = -1;
          if (E < nk_g * count) {
            slot(E, jj[u], o[u], yo[u]);
            if (FINAL && a.residual) res[u] = *reinterpret_cast<const v4f*>(a.residual + o[u]);
          }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (jj[u] < 0) continue;
          const v4f y = *reinterpret_cast<const v4f*>(lds + yo[u]);
          const float b = jj[u] == 0 ? bias4[0] : jj[u] == 1 ? bias4[1] : jj[u] == 2 ? bias4[2] : bias4[3];
          v4f v;
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) v[q4] = activate<ACT>(y[q4] + b + res[u][q4]);
          *reinterpret_cast<v4f*>(dst + o[u]) = v;
        }
      } else {
        float res[32];
        int64_t o[32];
        int yo[32], jj[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) {
          const int E = lane + 64 * u;
          res[u] = 0.f;
          jj[u] = -1;
          if (E < nk_g * count) {
            slot(E, jj[u], o[u], yo[u]);
            if (FINAL && a.residual) res[u] = a.residual[o[u]];
          }
        }
#pragma unroll
        for (int u = 0; u < 32; ++u) {
          if (jj[u] < 0) continue;
          const float b = jj[u] == 0 ? bias4[0] : jj[u] == 1 ? bias4[1] : jj[u] == 2 ? bias4[2] : bias4[3];
          dst[o[u]] = activate<ACT>(lds[yo[u]] + b + res[u]);
        }
      }
    }
    return;
  }
  // mode 2: a cut tile row, written one pixel row at a time per channel.
  const int im = bk.g0 / a.th, ty = bk.g0 - im * a.th;
  const int rows = min(4, a.OH - 4 * ty);
  const int x_base = 4 * bk.tx_a;
  const int cols = min(4 * bk.ntiles, a.OW - x_base);
  for (int j = 0; j < JW; ++j) {
    const int kk = wave + NW * j, k = k0 + kk;
    if (k >= a.K) break;
    const float b = FINAL ? a.bias[k] : 0.f;
    for (int i = 0; i < rows; ++i) {
      const int64_t base = (((int64_t)im * a.K + k) * a.OH + 4 * ty + i) * a.OW + x_base;
      for (int x = lane; x < cols; x += 64) {
        const float r = (FINAL && a.residual) ? a.residual[base + x] : 0.f;
        dst[base + x] = activate<ACT>(lds[ys_off(kk, x >> 2, i) + (x & 3)] + b + r);
      }
    }
  }
}

// Input transform V = B^T d B of one 6x6 patch; each value is handed to
// `store(xi, value)` as soon as it is computed.
template <class Store>
__device__ __forceinline__ void input_transform(float (&d)[36], Store store) {
#pragma unroll
  for (int j = 0; j < 6; ++j) {  // columns: d <- B^T d, in place
    const float d0 = d[0 * 6 + j], d1 = d[1 * 6 + j], d2 = d[2 * 6 + j];
    const float d3 = d[3 * 6 + j], d4 = d[4 * 6 + j], d5 = d[5 * 6 + j];
    d[0 * 6 + j] = 4.f * d0 - 5.f * d2 + d4;
    d[1 * 6 + j] = -4.f * (d1 + d2) + d3 + d4;
    d[2 * 6 + j] = 4.f * (d1 - d2) - d3 + d4;
    d[3 * 6 + j] = -2.f * (d1 - d3) - d2 + d4;
    d[4 * 6 + j] = 2.f * (d1 - d3) - d2 + d4;
    d[5 * 6 + j] = 4.f * d1 - 5.f * d3 + d5;
  }
#pragma unroll
  for (int i = 0; i < 6; ++i) {  // rows: (B^T d) B
    const float d0 = d[i * 6 + 0], d1 = d[i * 6 + 1], d2 = d[i * 6 + 2];
    const float d3 = d[i * 6 + 3], d4 = d[i * 6 + 4], d5 = d[i * 6 + 5];
    store(i * 6 + 0, 4.f * d0 - 5.f * d2 + d4);
    store(i * 6 + 1, -4.f * (d1 + d2) + d3 + d4);
    store(i * 6 + 2, 4.f * (d1 - d2) - d3 + d4);
    store(i * 6 + 3, -2.f * (d1 - d3) - d2 + d4);
    store(i * 6 + 4, 2.f * (d1 - d3) - d2 + d4);
    store(i * 6 + 5, 4.f * d1 - 5.f * d3 + d5);
  }
}

// The transform waves of the direct variant (no V in HBM): for chunks
// ch_begin .. ch_begin + n - 1 they load the 6x6 input patches of the
// block's tiles (thread p = tile p % 32, channel p / 32 of the chunk),
// transform them into the chunk's V slot ([xi][channel pair][tile][2]) and
// copy the U slice as load_role does; same slots, same n + 1 barriers.
// Patch offsets are plane + row + column (bytes), each term exact or kOOB1
// (a channel or tile past the end, a row or column outside the image): one
// invalid term puts the sum at or past 2^30 >= the input size, so the raw
// buffer load returns 0; three stay below 2^32.  Every load has its own
// offset register, so the compiler does not merge neighbouring loads into
// vectors (a vector that straddles the end of the input would come back
// zero as a whole).  VEC (left padding 1, W % 4 == 0): columns 1..4 of a
// patch row are the 16-byte aligned run x = 4*tx .. +3, wholly inside the row
// or wholly past its end, loaded as one vector.
constexpr uint32_t kOOB1 = 0x40000000u;

template <bool VEC>
__device__ __forceinline__ void transform_role(const FusedArgs& a, float* lds, int p, const Block& bk) {
  const int t_l = p % kTB, c_l = p / kTB;
  const bool t_ok = t_l < bk.ntiles;
  int g, tx;
  if (a.mode == 2) {
    g = bk.g0;
    tx = bk.tx_a + t_l;
  } else {
    g = bk.g0 + t_l / a.tw;
    tx = t_l - (t_l / a.tw) * a.tw;
  }
  const int im = t_ok ? g / a.th : 0, ty = t_ok ? g - im * a.th : 0;
  const int y0 = ty * 4 - a.pt, x0 = tx * 4 - a.pl;
  uint32_t rowoff[6], coloff[6];
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    const int y = y0 + i, x = x0 + i;
    rowoff[i] = (unsigned)y < (unsigned)a.H ? (uint32_t)(y * a.W) * 4u : kOOB1;
    coloff[i] = (unsigned)x < (unsigned)a.W ? (uint32_t)x * 4u : kOOB1;
  }
  const uint32_t plane_bytes = (uint32_t)(a.H * a.W) * 4u;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t ur = make_rsrc(a.U, a.u_bytes);
  // U slice addressing as in load_role
  const int xi0 = p >> 6, cp = (p & 63) >> 4, r2 = 2 * (p & 15);
  const uint32_t u_lane = (uint32_t)((((xi0 * 4 + cp) * a.m_pad + bk.k0 + r2) * 2) * 4);
  const uint32_t u_it = (uint32_t)(4 * 4 * a.m_pad * 2 * 4);
  const uint32_t u_ch = (uint32_t)(36 * 4 * a.m_pad * 2 * 4);

  // Two chunks in flight, loads issued unconditionally (see load_role).
  float dA[36], dB[36];
  v4f uA[kULoads], uB[kULoads];
  auto load = [&](int ch, bool live, float (&d)[36], v4f (&u)[kULoads]) {
    const int c = ch * kCB + c_l;
    const uint32_t pb = (live && t_ok && c < a.C) ? (uint32_t)(im * a.C + c) * plane_bytes : kOOB1;
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      const uint32_t rb = pb + rowoff[i];
      if constexpr (VEC) {
        d[i * 6 + 0] = buf_load_f32(xr, rb + coloff[0]);
        const v4f m = __builtin_bit_cast(v4f, buf_load_b128(xr, rb + coloff[1]));
        d[i * 6 + 1] = m[0];
        d[i * 6 + 2] = m[1];
        d[i * 6 + 3] = m[2];
        d[i * 6 + 4] = m[3];
        d[i * 6 + 5] = buf_load_f32(xr, rb + coloff[5]);
      } else {
#pragma unroll
        for (int j = 0; j < 6; ++j) d[i * 6 + j] = buf_load_f32(xr, rb + coloff[j]);
      }
    }
    const uint32_t uo = live ? u_lane + (uint32_t)ch * u_ch : 0x80000000u;
#pragma unroll
    for (int it = 0; it < kULoads; ++it)
      u[it] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(ur, uo, it * u_it, 0));
  };
  const int v_off = ((c_l >> 1) * kTB + t_l) * 2 + (c_l & 1);
  auto fill = [&](int slot_idx, float (&d)[36], v4f (&u)[kULoads]) {
    float* slot = lds + slot_idx * kSlotElems;
    float* vw = slot + v_off;
    input_transform(d, [&](int xi, float v) { vw[xi * kTB * kCB] = v; });
#pragma unroll
    for (int it = 0; it < kULoads; ++it)
      *reinterpret_cast<v4f*>(slot + kVElems + (it * kProducers + p) * 4) = u[it];
  };

  const int n = bk.n, ch_begin = bk.ch_begin;
  load(ch_begin, n > 0, dA, uA);
  load(ch_begin + 1, n > 1, dB, uB);
  for (int i = 0; i <= n; i += 2) {
    if (i < n) fill(0, dA, uA);
    load(ch_begin + i + 2, i + 2 < n, dA, uA);
    __syncthreads();  // slot 0 full; slot 1 consumed
    if (i + 1 < n) fill(1, dB, uB);
    load(ch_begin + i + 3, i + 3 < n, dB, uB);
    if (i + 1 <= n) __syncthreads();  // slot 1 full; slot 0 consumed
  }
}

// The transform waves, staged form (tile blocks of up to R tile rows of one
// image (mode 1), left padding 1, W % 4 == 0): wave w stages the input rows
// its two channels of the chunk need, (4 * nrows + 2) rows x W columns each,
// from row 4 * ty0 - pt, through
// LDS with 16-byte loads, then reads each thread's 6x6 patch from there.
// The rows live in the wave's own quarter of the chunk slot's U region
// ([channel][row][x + 4], row stride W + 8, halo columns zero), which the
// wave overwrites with its share of the U slice only after its patch reads:
// a wave's LDS operations complete in order, so no barrier is needed.
// Its U share is the contiguous quarter e4 = w*576 + it*64 + lane.
__device__ __forceinline__ void transform_role_staged(const FusedArgs& a, float* lds, int p, const Block& bk) {
  const int lane = p & 63, w = p >> 6;
  const int t_l = p % kTB, c_l = p / kTB;  // c_l = 2w + lane / 32
  const bool t_ok = t_l < bk.ntiles;
  const int im = bk.g0 / a.th, ty0 = bk.g0 - im * a.th;
  const int rows = 4 * bk.nrows + 2;
  const int RS = a.W + 8;
  const int quads = a.W >> 2;
  const int per_ch = rows * quads;           // 16-byte row pieces per channel
  const int n_rows_ld = 2 * per_ch;          // per wave and chunk (<= 5 * 64, checked on the host)
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t ur = make_rsrc(a.U, a.u_bytes);
  // row piece e (lane + 64u) of the wave: channel e / per_ch, row, quad
  uint32_t roff[5];
  int rlds[5], rch[5];
#pragma unroll
  for (int u = 0; u < 5; ++u) {
    const int e = lane + 64 * u;
    const int ch = e / per_ch, rem = e - ch * per_ch;
    const int r = rem / quads, xq = rem - r * quads;
    const int y = 4 * ty0 - a.pt + r;
    const bool ok = e < n_rows_ld && (unsigned)y < (unsigned)a.H;
    roff[u] = ok ? (uint32_t)(((im * a.C + 2 * w + ch) * a.H + y) * a.W + 4 * xq) * 4u : 0x80000000u;
    rlds[u] = e < n_rows_ld ? (ch * rows + r) * RS + 4 + 4 * xq : -1;
    rch[u] = 2 * w + ch;  // channel within the chunk
  }
  const uint32_t plane_bytes = (uint32_t)(a.H * a.W) * 4u;
  // U share: e4 = w*576 + it*64 + lane -> xi = 9w + it, pair lane/16, rows 2*(lane%16)
  const uint32_t u_lane = (uint32_t)((((9 * w * 4) + (lane >> 4)) * a.m_pad + bk.k0 + 2 * (lane & 15)) * 2 * 4);
  const uint32_t u_it = (uint32_t)(4 * a.m_pad * 2 * 4);
  const uint32_t u_ch = (uint32_t)(36 * 4 * a.m_pad * 2 * 4);
  // patch of this thread: tile (ty, tx) of the block, rows 4*(ty - ty0) .. +5 of its channel's rows
  const int tyl = t_l / a.tw, tx = t_l - tyl * a.tw;
  const int pbase = ((lane >> 5) * rows + 4 * tyl) * RS + 3 + 4 * tx;  // x = 4tx - 1 at offset 4tx + 3

  v4f rA[5], rB[5], uA[kULoads], uB[kULoads];
  auto load = [&](int ch, bool live, v4f (&r)[5], v4f (&u)[kULoads]) {
    const uint32_t cb = (uint32_t)(ch * kCB) * plane_bytes;  // chunk's channel offset
#pragma unroll
    for (int q = 0; q < 5; ++q)
      r[q] = __builtin_bit_cast(v4f, buf_load_b128(xr, (live && ch * kCB + rch[q] < a.C) ? roff[q] + cb : 0x80000000u));
    const uint32_t uo = live ? u_lane + (uint32_t)ch * u_ch : 0x80000000u;
#pragma unroll
    for (int it = 0; it < kULoads; ++it)
      u[it] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(ur, uo, it * u_it, 0));
  };
  const int v_off = ((c_l >> 1) * kTB + t_l) * 2 + (c_l & 1);
  auto fill = [&](int slot_idx, v4f (&r)[5], v4f (&u)[kULoads]) {
    float* slot = lds + slot_idx * kSlotElems;
    float* raw = slot + kVElems + w * (kUElems / 4);
#pragma unroll
    for (int q = 0; q < 5; ++q)
      if (rlds[q] >= 0) *reinterpret_cast<v4f*>(raw + rlds[q]) = r[q];
    // halo columns x = -1 and x = W of the wave's rows
    for (int e = lane; e < 2 * rows; e += 64) {
      raw[e * RS + 3] = 0.f;
      raw[e * RS + a.W + 4] = 0.f;
    }
    float d[36];
    const float* pr = raw + pbase;
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      d[i * 6 + 0] = pr[i * RS];
      const v4f m = *reinterpret_cast<const v4f*>(pr + i * RS + 1);
      d[i * 6 + 1] = m[0];
      d[i * 6 + 2] = m[1];
      d[i * 6 + 3] = m[2];
      d[i * 6 + 4] = m[3];
      d[i * 6 + 5] = pr[i * RS + 5];
    }
    if (!t_ok) {
#pragma unroll
      for (int e = 0; e < 36; ++e) d[e] = 0.f;
    }
    float* vw = slot + v_off;
    input_transform(d, [&](int xi, float v) { vw[xi * kTB * kCB] = v; });
    float* us = slot + kVElems + w * (kUElems / 4) + lane * 4;
#pragma unroll
    for (int it = 0; it < kULoads; ++it) *reinterpret_cast<v4f*>(us + it * 256) = u[it];
  };

  const int n = bk.n, ch_begin = bk.ch_begin;
  load(ch_begin, n > 0, rA, uA);
  load(ch_begin + 1, n > 1, rB, uB);
  for (int i = 0; i <= n; i += 2) {
    if (i < n) fill(0, rA, uA);
    load(ch_begin + i + 2, i + 2 < n, rA, uA);
    __syncthreads();  // slot 0 full; slot 1 consumed
    if (i + 1 < n) fill(1, rB, uB);
    load(ch_begin + i + 3, i + 3 < n, rB, uB);
    if (i + 1 <= n) __syncthreads();  // slot 1 full; slot 0 consumed
  }
}

// 8 waves, 4 load (XFORM: transform) + 4 MFMA, chunks of 8 channels in
// 2 x 72 KB of LDS (one workgroup per CU).  FINAL: write act(Y + bias
// (+ residual)) with activation ACT; otherwise the raw part of channel split
// cs.  XFORM: the direct variant, V computed from the input in the kernel
// (VEC: the staged form, transform_role_staged).
template <int ACT, bool FINAL, bool XFORM, bool VEC>
__global__ __launch_bounds__(kThreads, 1) void wino_fused_kernel(FusedArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const Block bk = block_of(a, kCB);

  if (wave >= 4) {
    if constexpr (XFORM && VEC)
      transform_role_staged(a, lds, tid - 4 * 64, bk);
    else if constexpr (XFORM)
      transform_role<false>(a, lds, tid - 4 * 64, bk);
    else
      load_role(a, lds, tid - 4 * 64, bk.t0, bk.k0, bk.ch_begin, bk.n);
  } else {
    // ---- MFMA waves ----------------------------------------------------------
    const int li = lane & 15, q = lane >> 4;
    const int wk = wave & 1, wt = wave >> 1;
    // Lane (li, q) supplies reduction index q at MFMA step s as channel
    // 2q + s of the chunk, for both operands: A = U[k = wk*16 + li],
    // B = V[t = wt*16 + li].
    const int ua_off = kVElems + (q * kKB + wk * 16 + li) * 2;
    const int vb_off = (q * kTB + wt * 16 + li) * 2;

    v4f acc[36];
#pragma unroll
    for (int xi = 0; xi < 36; ++xi) acc[xi] = v4f{0.f, 0.f, 0.f, 0.f};

    // Operands are read in groups of kG transform points, one group ahead
    // of the MFMAs that use them; a scheduling fence per group keeps the
    // compiler from hoisting all 72 reads (which would not fit in registers
    // beside the 144 accumulators).  The chunk barrier sits before the last
    // group's MFMAs: by then every read of the chunk's slot has completed, so
    // the barrier can release the slot, and the next chunk's first group is
    // read while the last MFMAs run.  kGroups is even, so a chunk's first
    // group always lands in register buffer 0.
    constexpr int kG = 6, kGroups = 36 / kG;
    static_assert(kGroups % 2 == 0, "static register buffer parity across chunks");
    v2f av[2][kG], bv[2][kG];
    auto read_group = [&](const float* slot, int g, int buf) {
#pragma unroll
      for (int j = 0; j < kG; ++j) {
        av[buf][j] = *reinterpret_cast<const v2f*>(slot + ua_off + (g * kG + j) * kKB * kCB);
        bv[buf][j] = *reinterpret_cast<const v2f*>(slot + vb_off + (g * kG + j) * kTB * kCB);
      }
    };
    __syncthreads();  // barrier 0: chunk 0 in slot 0
    read_group(lds, 0, 0);
    for (int i = 1; i <= bk.n; ++i) {  // consume chunk i - 1; barrier i inside
      const float* slot = lds + ((i - 1) & 1) * kSlotElems;
      const float* next = lds + (i & 1) * kSlotElems;
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int g = 0; g < kGroups; ++g) {
        if (g + 1 < kGroups) {
          read_group(slot, g + 1, (g + 1) & 1);
        } else {
          __syncthreads();  // barrier i: chunk i - 1 read, chunk i in the other slot
          if (i < bk.n) read_group(next, 0, 0);
        }
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int j = 0; j < kG; ++j)
            acc[g * kG + j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[g & 1][j][s], bv[g & 1][j][s],
                                                                  acc[g * kG + j], 0, 0, 0);
        // order within the group: the next group's LDS reads, then this
        // group's MFMAs
        __builtin_amdgcn_sched_group_barrier(0x100, kG, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * kG, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // n + 1 barriers in all, as the load waves
    // both slots are free: every wave has passed the last chunk's barrier
    y_to_lds(acc, lds, wk, wt, li, q);
  }
  __syncthreads();
  write_out<8, ACT, FINAL>(a, bk, lds, lane, wave);
}

// out = act(sum_s part[s] + bias[k] (+ residual)), parts [splits][N][K][OH][OW];
// VEC = 4 when OH*OW % 4 == 0 (a float4 never crosses a channel plane).
template <int VEC, int ACT>
__global__ void wino_fused_reduce(const float* __restrict__ part, int splits, int64_t total, int ohw, int K,
                                  const float* __restrict__ bias, const float* __restrict__ residual,
                                  float* __restrict__ out) {
  const int64_t idx = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * VEC;
  if (idx >= total) return;
  const float b = bias[(int)((idx / ohw) % K)];
  if constexpr (VEC == 4) {
    v4f s = *reinterpret_cast<const v4f*>(part + idx);
    for (int z = 1; z < splits; ++z) s += *reinterpret_cast<const v4f*>(part + (int64_t)z * total + idx);
    v4f r = v4f{0.f, 0.f, 0.f, 0.f};
    if (residual) r = *reinterpret_cast<const v4f*>(residual + idx);
    v4f o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = activate<ACT>(s[j] + b + r[j]);
    *reinterpret_cast<v4f*>(out + idx) = o;
  } else {
    float s = part[idx];
    for (int z = 1; z < splits; ++z) s += part[(int64_t)z * total + idx];
    float v = s + b;
    if (residual) v += residual[idx];
    out[idx] = activate<ACT>(v);
  }
}

template <int ACT, bool FINAL, bool XFORM, bool VEC>
int launch_kernel(const FusedArgs& a, int64_t blocks, hipStream_t s) {
  static bool attr_set = false;  // dynamic LDS above 64 KB needs the attribute
  if (!attr_set) {
    NHIP_TRY(check_hip(
        hipFuncSetAttribute(reinterpret_cast<const void*>(&wino_fused_kernel<ACT, FINAL, XFORM, VEC>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes),
        "hipFuncSetAttribute(wino_fused)"));
    attr_set = true;
  }
  NHIP_LAUNCH("wino_fused", (wino_fused_kernel<ACT, FINAL, XFORM, VEC>), dim3((unsigned)blocks), dim3(kThreads),
              kLdsBytes, s, a);
  return check_launch("wino_fused");
}

template <int ACT, bool FINAL>
int launch_kernel(const FusedArgs& a, int64_t blocks, bool xform, bool vec, hipStream_t s) {
  if (!xform) return launch_kernel<ACT, FINAL, false, false>(a, blocks, s);
  return vec ? launch_kernel<ACT, FINAL, true, true>(a, blocks, s) : launch_kernel<ACT, FINAL, true, false>(a, blocks, s);
}

template <int VEC, int ACT>
int launch_reduce(const float* parts, int splits, int64_t total, int ohw, int K, const float* bias,
                  const float* residual, float* out, hipStream_t s) {
  NHIP_LAUNCH("wino_split_reduce", (wino_fused_reduce<VEC, ACT>), dim3((unsigned)ceil_div(total / VEC, 256)),
              dim3(256), 0, s, parts, splits, total, ohw, K, bias, residual, out);
  return check_launch("wino_split_reduce");
}

struct FusedShape {
  int th, tw, G, mode, R, bpi, bpr, nt, nk, nch, splits, per;
};

// Tile blocks (whole tile rows, or 32-tile pieces of wider rows); channel
// splits: the fewest that minimise (rounds of one workgroup per CU) x
// (chunks per workgroup), each split keeping at least 4 chunks.
FusedShape fused_shape(const nhip_conv_plan* p, int n, int oh, int ow) {
  FusedShape f;
  f.th = (int)ceil_div(oh, 4);
  f.tw = (int)ceil_div(ow, 4);
  f.G = n * f.th;
  f.bpi = f.bpr = 0;
  if (f.tw <= kTB && f.th <= kTB / f.tw) {
    f.mode = 0;
    f.R = kTB / f.tw / f.th * f.th;
    f.nt = (int)ceil_div(f.G, f.R);
  } else if (f.tw <= kTB) {
    f.mode = 1;
    f.R = kTB / f.tw;
    f.bpi = (int)ceil_div(f.th, f.R);
    f.nt = n * f.bpi;
  } else {
    f.mode = 2;
    f.R = 1;
    f.bpr = (int)ceil_div(f.tw, kTB);
    f.nt = f.G * f.bpr;
  }
  f.nk = (int)ceil_div(p->g.k, kKB);
  f.nch = p->c_pad / kCB;
  const int64_t cus = cu_count();
  const int64_t blocks = (int64_t)f.nt * f.nk;
  f.splits = 1;
  int64_t best = ceil_div(blocks, cus) * f.nch;
  for (int s = 2; s <= 8 && ceil_div(f.nch, s) >= 4; s *= 2) {
    const int64_t cost = ceil_div(blocks * s, cus) * ceil_div(f.nch, s);
    if (cost < best) {
      best = cost;
      f.splits = s;
    }
  }
  f.per = (int)ceil_div(f.nch, f.splits);
  return f;
}

}  // namespace

uint64_t wino_gemm_out_parts_bytes(const nhip_conv_plan* p, int n, int oh, int ow) {
  const FusedShape f = fused_shape(p, n, oh, ow);
  return f.splits > 1 ? (uint64_t)f.splits * n * p->g.k * oh * ow * sizeof(float) : 0;
}

namespace {

// Shared by both entries: a = the operand sources already set (V or x).
int launch_fused(const nhip_conv_plan* p, FusedArgs& a, const FusedShape& f, bool xform, bool vec,
                 const float* residual, float* out, int n, int oh, int ow, float* parts, hipStream_t s) {
  if ((reinterpret_cast<uintptr_t>(out) & 15) || (residual && (reinterpret_cast<uintptr_t>(residual) & 15)) ||
      (reinterpret_cast<uintptr_t>(parts) & 15))
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "winograd: buffers must be 16-byte aligned");
  if (f.splits > 1 && parts == nullptr)
    return fail(NHIP_STATUS_NULL_POINTER, "winograd GEMM: partial-sum workspace missing");
  const size_t u_bytes = (size_t)36 * p->m_pad * p->c_pad * sizeof(float);
  if (u_bytes >= (size_t(1) << 31))
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "winograd GEMM: transformed weights above 2 GiB");
  if (p->c_pad % kCB != 0 || p->m_pad % kKB != 0)
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "winograd GEMM: padding mismatch");
  a.U = p->weight_fused;
  a.u_bytes = (uint32_t)u_bytes;
  a.bias = p->bias;
  a.residual = residual;
  a.out = f.splits > 1 ? parts : out;
  a.K = p->g.k;
  a.OH = oh;
  a.OW = ow;
  a.th = f.th;
  a.tw = f.tw;
  a.T = n * f.th * f.tw;
  a.mode = f.mode;
  a.R = f.R;
  a.bpi = f.bpi;
  a.bpr = f.bpr;
  a.G = f.G;
  a.m_pad = p->m_pad;
  a.c_pad = p->c_pad;
  a.nt = f.nt;
  a.nk = f.nk;
  a.splits = f.splits;
  a.per = f.per;
  const int64_t blocks = (int64_t)f.nt * f.nk * f.splits;
  if (f.splits == 1) {
    switch (p->g.act) {
      case NHIP_ACT_NONE: return launch_kernel<NHIP_ACT_NONE, true>(a, blocks, xform, vec, s);
      case NHIP_ACT_RELU: return launch_kernel<NHIP_ACT_RELU, true>(a, blocks, xform, vec, s);
      case NHIP_ACT_SIGMOID: return launch_kernel<NHIP_ACT_SIGMOID, true>(a, blocks, xform, vec, s);
      default: return fail(NHIP_STATUS_UNSUPPORTED, "winograd GEMM: unsupported activation");
    }
  }
  NHIP_TRY((launch_kernel<NHIP_ACT_NONE, false>(a, blocks, xform, vec, s)));
  const int64_t total = (int64_t)n * p->g.k * oh * ow;
  const int ohw = oh * ow;
#define NHIP_REDUCE(V_)                                                                                       \
  switch (p->g.act) {                                                                                         \
    case NHIP_ACT_RELU: return launch_reduce<V_, NHIP_ACT_RELU>(parts, f.splits, total, ohw, p->g.k, p->bias, \
                                                                residual, out, s);                            \
    case NHIP_ACT_SIGMOID:                                                                                    \
      return launch_reduce<V_, NHIP_ACT_SIGMOID>(parts, f.splits, total, ohw, p->g.k, p->bias, residual, out, s); \
    default: return launch_reduce<V_, NHIP_ACT_NONE>(parts, f.splits, total, ohw, p->g.k, p->bias, residual, out, s); \
  }
  if (ohw % 4 == 0) {
    NHIP_REDUCE(4)
  } else {
    NHIP_REDUCE(1)
  }
#undef NHIP_REDUCE
}

}  // namespace

int launch_wino_gemm_out(const nhip_conv_plan* p, const float* V, int t_pad, const float* residual, float* out,
                         int n, int oh, int ow, float* parts, hipStream_t s) {
  const size_t v_bytes = (size_t)36 * p->c_pad * t_pad * sizeof(float);
  if (v_bytes >= (size_t(1) << 31))
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "winograd GEMM: transformed input above 2 GiB");
  if (t_pad % kTB != 0 || (reinterpret_cast<uintptr_t>(V) & 15))
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "winograd GEMM: V padding or alignment");
  FusedArgs a{};
  a.V = V;
  a.v_bytes = (uint32_t)v_bytes;
  a.t_pad = t_pad;
  return launch_fused(p, a, fused_shape(p, n, oh, ow), false, false, residual, out, n, oh, ow, parts, s);
}

// The direct variant's staged input rows apply (by shape; the input must also
// be 16-byte aligned at launch, else the direct kernel gathers patches).
bool wino_direct_staged_shape(const nhip_conv_plan* p, int n, int h, int w, int oh, int ow) {
  const FusedShape f = fused_shape(p, n, oh, ow);
  const int rows = 4 * f.R + 2;
  return f.mode == 1 && p->g.pl == 1 && w % 4 == 0 && 2 * rows * (w / 4) <= 5 * 64 &&
         2 * rows * (w + 8) <= kUElems / 4 && (int64_t)n * p->g.c * h * w * 4 < (int64_t(1) << 30);
}

int launch_wino_fused_direct(const nhip_conv_plan* p, const float* in, int h, int w, const float* residual,
                             float* out, int n, int oh, int ow, float* parts, hipStream_t s) {
  const size_t x_bytes = (size_t)n * p->g.c * h * w * sizeof(float);
  if (x_bytes > (size_t(1) << 30))
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "winograd direct: input above 1 GiB");
  FusedArgs a{};
  a.x = in;
  a.x_bytes = (uint32_t)x_bytes;
  a.C = p->g.c;
  a.H = h;
  a.W = w;
  a.pt = p->g.pt;
  a.pl = p->g.pl;
  // staged rows: tile rows of one image (mode 1), left padding 1, 16-byte
  // rows, and a wave's two channels of rows (<= 5 x 64 pieces, and within
  // its quarter of the U region) per chunk
  const bool staged = wino_direct_staged_shape(p, n, h, w, oh, ow) && (reinterpret_cast<uintptr_t>(in) & 15) == 0;
  return launch_fused(p, a, fused_shape(p, n, oh, ow), true, staged, residual, out, n, oh, ow, parts, s);
}

}  // namespace nhip
