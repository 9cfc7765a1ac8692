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

#include "lds_dma.h"
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
  const float* V;       // [36][c_pad/2][t_pad][2]
  const float* U;       // [c_pad/8][36][4][m_pad][2]
  const float* bias;    // [m_pad]
  const float* residual;
  float* out;           // [N][K][OH][OW]; with splits > 1 the parts [splits][N][K][OH][OW]
  int K, OH, OW, th, tw, T, t_pad, m_pad, c_pad;
  int nt, nk, splits, per;  // tile blocks, channel blocks, channel splits, chunks per split
  int64_t part_stride;      // N*K*OH*OW (< 2^31): elements per channel-split part
  uint32_t v_bytes;         // size of V (< 2^31)
  uint32_t u_bytes;         // size of U (< 2^31)
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

// A workgroup's share of the work: tiles t0 .. t0 + ntiles - 1 (32
// consecutive tiles in (image, tile row, tile column) order, so every tile
// slot of the MFMA block carries a real tile except in the last block),
// output channels k0 .. k0 + 31, and chunks ch_begin .. ch_begin + n - 1 of
// channel split cs (chunks of `cb` input channels).
struct Block {
  int kb, cs, k0, t0, ntiles, ch_begin, n;
};

__device__ __forceinline__ Block block_of(const FusedArgs& a, int cb) {
  Block b;
  int tb;
  // XCD-contiguous renumbering: each XCD gets a contiguous range of logical
  // blocks, ordered (split, tile block, channel block) with the channel
  // block fastest, so the workgroups that read the same V slices share an L2
  // and, with channel splits, an XCD fetches only its split's half of U.
  {
    const int total = a.nt * a.nk * a.splits;
    const int L = blockIdx.x;
    const int x = L % kXcds, q = L / kXcds;
    const int logical = x * (total / kXcds) + min(x, total % kXcds) + q;
    b.kb = logical % a.nk;
    const int rest = logical / a.nk;
    tb = rest % a.nt;
    b.cs = rest / a.nt;
  }
  b.k0 = b.kb * kKB;
  b.t0 = tb * kTB;
  b.ntiles = min(kTB, a.T - b.t0);
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

// The block's output, in memory order, as units of VW consecutive pixels
// (VW = 4 when OW % 4 == 0: a tile row of a full-width tile; else single
// pixels).  The block's tiles form segments of one tile row each (the first
// and last may be partial rows); a segment covers rows 4ty .. 4ty + rows - 1
// (rows <= 4, clipped at OH) and, per row, one run of L pixels (clipped at
// OW where the segment reaches the row's end).  Runs of consecutive
// segments of one image are adjacent in memory, so consecutive units are
// consecutive addresses within a channel plane.  For unit e of the lane the
// table gives the output offset without the channel term (image plane + row
// + column, -1 past the block's units) and its place in the staged tiles Ys
// without the channel term.
template <int VW, int NU>
__device__ __forceinline__ void unit_table(const FusedArgs& a, const Block& bk, int lane, int (&go)[NU],
                                           int (&yo)[NU]) {
  const int OHW = a.OH * a.OW;
  const int per_img = a.th * a.tw;
#pragma unroll
  for (int m = 0; m < NU; ++m) go[m] = -1, yo[m] = 0;
  if (VW == 1 && bk.t0 % per_img == 0 && bk.ntiles % per_img == 0) {
    // whole images: unit e is pixel e % OHW of image t0 / per_img + e / OHW
    const int img0 = bk.t0 / per_img, cnt = bk.ntiles / per_img * OHW;
#pragma unroll
    for (int m = 0; m < NU; ++m) {
      const int e = lane + 64 * m;
      if (e < cnt) {
        const int ir = e / OHW, px = e - ir * OHW;
        const int oy = px / a.OW, ox = px - oy * a.OW;
        const int tl = ir * per_img + (oy >> 2) * a.tw + (ox >> 2), i = oy & 3;
        go[m] = (img0 + ir) * a.K * OHW + px;
        yo[m] = tl * 16 + ((i ^ tl) & 3) * 4 + (ox & 3);
      }
    }
    return;
  }
  int seg_t = bk.t0, first = 0;  // first unit of the segment
  while (seg_t < bk.t0 + bk.ntiles) {
    const int img = seg_t / per_img, rr = seg_t - img * per_img;
    const int ty = rr / a.tw, tx0 = rr - ty * a.tw;
    const int len = min(a.tw - tx0, bk.t0 + bk.ntiles - seg_t);
    const int rows = min(4, a.OH - 4 * ty);
    const int L = VW == 4 ? len : (tx0 + len == a.tw ? a.OW - 4 * tx0 : 4 * len);  // units per row
    const int cnt = rows * L;
    const int tl0 = seg_t - bk.t0;
    const int base = img * a.K * OHW + 4 * ty * a.OW + 4 * tx0;
#pragma unroll
    for (int m = 0; m < NU; ++m) {
      const int u = lane + 64 * m - first;
      if (u >= 0 && u < cnt) {
        const int i = (u >= L) + (u >= 2 * L) + (u >= 3 * L), x = u - i * L;  // row, unit within the row
        const int tt = VW == 4 ? x : x >> 2, j = VW == 4 ? 0 : x & 3;
        const int tl = tl0 + tt;
        go[m] = base + i * a.OW + (VW == 4 ? 4 * x : x);
        yo[m] = tl * 16 + ((i ^ tl) & 3) * 4 + j;
      }
    }
    first += cnt;
    seg_t += len;
  }
}

// Write-out of the staged tiles by NW waves, wave w taking channels w + NW*j,
// each unit of the block's output (unit_table) once per channel.  All
// residual loads of a channel are issued before its first store: vmcnt
// counts loads and stores in issue order, so a load issued after a store
// would make its wait include the store.  FINAL: act(Y + bias (+ residual));
// otherwise the raw part of channel split b.cs for wino_fused_reduce.
template <int NW, int ACT, bool FINAL>
__device__ __forceinline__ void write_out(const FusedArgs& a, const Block& bk, const float* lds, int lane,
                                          int wave) {
  constexpr int JW = kKB / NW;  // channels per wave
  float* dst = a.out + (FINAL ? 0 : (int64_t)bk.cs * a.part_stride);
  const int OHW = a.OH * a.OW;
  if (a.OW % 4 == 0) {
    constexpr int NU = kTB * 4 / 64;  // <= 32 tiles x 4 rows float4 units per channel
    int go[NU], yo[NU];
    unit_table<4, NU>(a, bk, lane, go, yo);
    for (int j = 0; j < JW; ++j) {
      const int kk = wave + NW * j, k = bk.k0 + kk;
      if (k >= a.K) break;
      const float b = FINAL ? a.bias[k] : 0.f;
      v4f res[NU];
#pragma unroll
      for (int m = 0; m < NU; ++m)
        res[m] = (FINAL && a.residual && go[m] >= 0) ? *reinterpret_cast<const v4f*>(a.residual + go[m] + k * OHW)
                                                      : v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < NU; ++m)
        if (go[m] >= 0) {
          const v4f y = *reinterpret_cast<const v4f*>(lds + kk * (kTB * 16) + yo[m]);
          v4f v;
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) v[q4] = activate<ACT>(y[q4] + b + res[m][q4]);
          *reinterpret_cast<v4f*>(dst + go[m] + k * OHW) = v;
        }
    }
  } else {
    constexpr int NU = kTB * 16 / 64;  // <= 32 tiles x 16 pixels per channel
    int go[NU], yo[NU];
    unit_table<1, NU>(a, bk, lane, go, yo);
    for (int j = 0; j < JW; ++j) {
      const int kk = wave + NW * j, k = bk.k0 + kk;
      if (k >= a.K) break;
      const float b = FINAL ? a.bias[k] : 0.f;
      float res[NU];
#pragma unroll
      for (int m = 0; m < NU; ++m)
        res[m] = (FINAL && a.residual && go[m] >= 0) ? a.residual[go[m] + k * OHW] : 0.f;
#pragma unroll
      for (int m = 0; m < NU; ++m)
        if (go[m] >= 0) dst[go[m] + k * OHW] = activate<ACT>(lds[kk * (kTB * 16) + yo[m]] + b + res[m]);
    }
  }
}

// 8 waves, 4 load + 4 MFMA, chunks of 8 channels in 2 x 72 KB of LDS (one
// workgroup per CU).  FINAL: write act(Y + bias (+ residual)) with
// activation ACT; otherwise the raw part of channel split cs.
template <int ACT, bool FINAL>
__global__ __launch_bounds__(kThreads, 1) void wino_fused_kernel(FusedArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const Block bk = block_of(a, kCB);

  if (wave >= 4) {
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

// ---- LDS-DMA variant --------------------------------------------------------
// The same 32 tiles x 32 output channels x 36 transform points per
// workgroup, with 4 waves that each own a 16 x 16 MFMA block and also move
// the operands: buffer_load_dwordx4 ... lds copies V and U slices from
// memory straight into LDS (lane l's 16 bytes land at the wave-uniform LDS
// base in M0 plus 16*l), so no registers hold data in flight.  Two LDS slots
// of 36 KB (chunks of 4 input channels) keep each workgroup at 74 KB and 175
// registers per lane, so two workgroups share a CU: while one waits at its
// per-chunk barrier or for its next chunk, the other's waves issue MFMAs
// (the chunk loop of a co-resident pair measured ~92% MFMA-busy).  The
// copies are issued from inline assembly: the compiler does not see them,
// so it inserts no waits of its own before the LDS reads; the kernel waits
// with explicit vmcnt counts (a wave's copies complete in issue order) and a
// workgroup barrier per chunk.  Chosen where the launch has enough
// workgroups for two per CU (measured: 64@56 at batch 32, 392 workgroups,
// 45.0 -> 37.3 us; with fewer workgroups the register-staged kernel, one
// workgroup of 8 waves per CU, is faster).
namespace dma {
constexpr int kThreads = 256;
constexpr int kCB = 4;                                // input channels per chunk
constexpr int kSlots = 2;                             // chunk slots per workgroup
constexpr int kVElems = 36 * kTB * kCB;               // [36][2 pairs][32 tiles][2]
constexpr int kUElems = 36 * kKB * kCB;               // [36][2 pairs][32 channels][2]
constexpr int kSlotElems = kVElems + kUElems;
constexpr int kLdsBytes = kSlots * kSlotElems * (int)sizeof(float);  // 73728
constexpr int kInstrV = kVElems * 4 / 1024;           // 1 KB copies per chunk: 18 for V
constexpr int kInstrU = kUElems * 4 / 1024;           // and 18 for U
constexpr int kPerWave = (kInstrV + kInstrU) / 4;     // 9 per wave and chunk
static_assert(kLdsBytes >= kKB * kTB * 16 * (int)sizeof(float), "the staged output tiles fit in the slots");
static_assert((kInstrV + kInstrU) % 4 == 0, "whole copies per wave");

// Wait until at most 9 * chunks of this wave's copies are outstanding.
__device__ __forceinline__ void wait_copies(int chunks) {
  static_assert(kPerWave == 9 && kSlots == 2, "the counts below are 9 copies per chunk, at most one chunk ahead");
  if (chunks >= 1) asm volatile("s_waitcnt vmcnt(9)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
}  // namespace dma

// Two workgroups per CU: at least 2 waves per SIMD (<= 256 registers).
template <int ACT, bool FINAL>
__global__ __launch_bounds__(dma::kThreads, 2) void wino_fused_dma_kernel(FusedArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const Block bk = block_of(a, dma::kCB);
  const uint32_t lds0 = (uint32_t)(uintptr_t)lds;

  // Copy sources.  V[xi][c/2][t][2]: copy j of a chunk covers xi = 2j, 2j+1
  // (lane bit 5), pairs 0, 1 of the chunk (lane bit 4), tiles t0 + 2*(l%16)
  // and +1.  U[c/8][xi][pair][k][2] likewise over k0 .. k0 + 31.
  const v4i vrs = ::nhip::dma::raw_rsrc(a.V, a.v_bytes), urs = ::nhip::dma::raw_rsrc(a.U, a.u_bytes);
  const int hp = a.c_pad / 2;
  const uint32_t v_lane =
      (uint32_t)((((lane >> 5) * hp + ((lane >> 4) & 1)) * a.t_pad + bk.t0 + 2 * (lane & 15)) * 8);
  const uint32_t u_lane = (uint32_t)(((((lane >> 5) * 4 + ((lane >> 4) & 1)) * a.m_pad) + bk.k0 + 2 * (lane & 15)) * 8);
  auto issue = [&](int c4, int slot) {  // chunk c4 (global 4-channel index) into slot
    const uint32_t sb = lds0 + (uint32_t)(slot * dma::kSlotElems * 4);
#pragma unroll
    for (int m = 0; m < dma::kPerWave; ++m) {
      const int q = wave + 4 * m;
      if (q < dma::kInstrV) {
        const uint32_t so = (uint32_t)(((2 * q) * hp + 2 * c4) * a.t_pad * 8);
        ::nhip::dma::copy16(sb + (uint32_t)(q * 1024), v_lane, vrs, so);
      } else {
        const int j = q - dma::kInstrV;
        const uint32_t so = (uint32_t)((((c4 >> 1) * 36 + 2 * j) * 4 + (c4 & 1) * 2) * a.m_pad * 8);
        ::nhip::dma::copy16(sb + (uint32_t)(dma::kVElems * 4 + j * 1024), u_lane, urs, so);
      }
    }
  };

  const int li = lane & 15, q = lane >> 4;
  const int wk = wave & 1, wt = wave >> 1;
  // lane (li, q) supplies reduction index q (channel q of the chunk):
  // A = U[xi][q/2][k = wk*16 + li][q%2], B = V[xi][q/2][t = wt*16 + li][q%2]
  const int a_off = dma::kVElems + ((q >> 1) * 32 + wk * 16 + li) * 2 + (q & 1);
  const int b_off = ((q >> 1) * 32 + wt * 16 + li) * 2 + (q & 1);
  constexpr int kXiStride = 2 * 32 * 2;  // floats per transform point in a slot part

  v4f acc[36];
#pragma unroll
  for (int xi = 0; xi < 36; ++xi) acc[xi] = v4f{0.f, 0.f, 0.f, 0.f};

  const int n = bk.n;
  for (int c = 0; c < min(dma::kSlots, n); ++c) issue(bk.ch_begin + c, c);
  dma::wait_copies(min(dma::kSlots, n) - 1);
  __syncthreads();  // chunk 0 in slot 0

  constexpr int kG = 6, kGroups = 36 / kG;
  static_assert(kGroups % 2 == 0, "a chunk's first group lands in register buffer 0");
  float av[2][kG], bv[2][kG];
  auto read_group = [&](const float* slot, int g, int buf) {
#pragma unroll
    for (int j = 0; j < kG; ++j) {
      av[buf][j] = slot[a_off + (g * kG + j) * kXiStride];
      bv[buf][j] = slot[b_off + (g * kG + j) * kXiStride];
    }
  };
  if (n > 0) read_group(lds, 0, 0);
  for (int i = 0; i < n; ++i) {
    const float* slot = lds + (i % dma::kSlots) * dma::kSlotElems;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
      if (g + 1 < kGroups) {
        read_group(slot, g + 1, (g + 1) & 1);
      } else {
        // chunk i is read (its operands are in registers): wait for this
        // wave's copies of chunk i + 1 (vmcnt(0) here: at most one chunk is
        // in flight), then the barrier hands slot i % kSlots back to the
        // copies (chunk i + kSlots) and publishes chunk i + 1
        dma::wait_copies(max(0, min(dma::kSlots - 1, n - 1 - i) - 1));
        __syncthreads();
        if (i + dma::kSlots < n) issue(bk.ch_begin + i + dma::kSlots, i % dma::kSlots);
        if (i + 1 < n) read_group(lds + ((i + 1) % dma::kSlots) * dma::kSlotElems, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < kG; ++j)
        acc[g * kG + j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[g & 1][j], bv[g & 1][j], acc[g * kG + j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // every copy has landed and every slot is read (the last barrier above)
  y_to_lds(acc, lds, wk, wt, li, q);
  __syncthreads();
  write_out<4, ACT, FINAL>(a, bk, lds, lane, wave);
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

template <int ACT, bool FINAL>
int launch_kernel(const FusedArgs& a, int64_t blocks, bool dma, hipStream_t s) {
  if (dma) {
    NHIP_TRY(ensure_dynamic_lds(reinterpret_cast<const void*>(&wino_fused_dma_kernel<ACT, FINAL>), dma::kLdsBytes));
    NHIP_LAUNCH("wino_fused", (wino_fused_dma_kernel<ACT, FINAL>), dim3((unsigned)blocks), dim3(dma::kThreads),
                dma::kLdsBytes, s, a);
    return check_launch("wino_fused");
  }
  NHIP_TRY(ensure_dynamic_lds(reinterpret_cast<const void*>(&wino_fused_kernel<ACT, FINAL>), kLdsBytes));
  NHIP_LAUNCH("wino_fused", (wino_fused_kernel<ACT, FINAL>), dim3((unsigned)blocks), dim3(kThreads),
              kLdsBytes, s, a);
  return check_launch("wino_fused");
}

template <int VEC, int ACT>
int launch_reduce(const float* parts, int splits, int64_t total, int ohw, int K, const float* bias,
                  const float* residual, float* out, hipStream_t s) {
  NHIP_LAUNCH("wino_split_reduce", (wino_fused_reduce<VEC, ACT>), dim3((unsigned)ceil_div(total / VEC, 256)),
              dim3(256), 0, s, parts, splits, total, ohw, K, bias, residual, out);
  return check_launch("wino_split_reduce");
}

struct FusedShape {
  int th, tw, nt, nk, nch, splits, per;
  bool dma;  // the LDS-DMA kernel (two workgroups per CU) rather than the register-staged one
};

// Tile blocks of 32 consecutive tiles; channel splits: the fewest that
// minimise (rounds of one workgroup per CU) x (chunks per workgroup), each
// split keeping at least 4 chunks.
FusedShape fused_shape(const nhip_conv_plan* p, int n, int oh, int ow) {
  FusedShape f;
  f.th = (int)ceil_div(oh, 4);
  f.tw = (int)ceil_div(ow, 4);
  f.nt = (int)ceil_div((int64_t)n * f.th * f.tw, kTB);
  f.nk = (int)ceil_div(p->g.k, kKB);
  const int64_t blocks = (int64_t)f.nt * f.nk;
  // The LDS-DMA kernel from 1.5 workgroups per CU without a channel split;
  // NHIP_WINO_FUSED=dma / reg forces one (tuning and tests).
  const char* force = setting("NHIP_WINO_FUSED");
  f.dma = force ? std::strcmp(force, "dma") == 0 : 2 * blocks >= 3 * (int64_t)cu_count();
  const int cb = f.dma ? dma::kCB : kCB;  // channels per chunk
  f.nch = p->c_pad / cb;
  const int64_t cus = cu_count() * (f.dma ? 2 : 1);  // workgroup slots
  f.splits = 1;
  int64_t best = ceil_div(blocks, cus) * f.nch;
  const int min_chunks = 32 / cb;  // at least 32 channels per split
  for (int s = 2; s <= 8 && ceil_div(f.nch, s) >= min_chunks; s *= 2) {
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

// a = the operand source (V) already set.
int launch_fused(const nhip_conv_plan* p, FusedArgs& a, const FusedShape& f, const float* residual, float* out,
                 int n, int oh, int ow, float* parts, hipStream_t s) {
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
  if ((int64_t)n * p->g.k * oh * ow >= (int64_t(1) << 31))  // 32-bit output offsets in the write-out
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "winograd GEMM: output above 2^31 elements");
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
  a.part_stride = (int64_t)n * p->g.k * oh * ow;
  a.m_pad = p->m_pad;
  a.c_pad = p->c_pad;
  a.nt = f.nt;
  a.nk = f.nk;
  a.splits = f.splits;
  a.per = f.per;
  const int64_t blocks = (int64_t)f.nt * f.nk * f.splits;
  if (f.splits == 1) {
    switch (p->g.act) {
      case NHIP_ACT_NONE: return launch_kernel<NHIP_ACT_NONE, true>(a, blocks, f.dma, s);
      case NHIP_ACT_RELU: return launch_kernel<NHIP_ACT_RELU, true>(a, blocks, f.dma, s);
      case NHIP_ACT_SIGMOID: return launch_kernel<NHIP_ACT_SIGMOID, true>(a, blocks, f.dma, s);
      default: return fail(NHIP_STATUS_UNSUPPORTED, "winograd GEMM: unsupported activation");
    }
  }
  NHIP_TRY((launch_kernel<NHIP_ACT_NONE, false>(a, blocks, f.dma, s)));
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
  return launch_fused(p, a, fused_shape(p, n, oh, ow), residual, out, n, oh, ow, parts, s);
}

}  // namespace nhip
