// Winograd F(4x4, 3x3) batched GEMM with the output transform fused: the
// 36 point-wise products M[xi] = U[xi] V[xi] and Y = A^T M A in one kernel,
// so M never leaves the CU (the three-kernel path in winograd.hip writes and
// re-reads M through HBM).  V comes from wino_input_transform<true>
// (winograd.hip) in the 4-channel-group layout [36][c_pad/4][t_pad][4]; U
// is prepacked on the host in the same layout, [36][c_pad/4][m_pad][4].
//
// The input transform: a separate, HBM-bound kernel, except for launches of
// paired channel blocks (XT below), where the kernel forms V itself.  On
// gfx950 the fp32 MFMA and fp32 VALU work of the waves on one SIMD do not
// overlap (measured: a VALU wave beside an MFMA wave adds its whole time),
// so transforming patches inside the GEMM costs MFMA time; with 64 output
// channels per workgroup each patch is transformed once for 64 channels'
// MFMAs, and the transform's VALU work (about a fifth of the MFMA time)
// costs less than the separate kernel's write and re-read of V (2.25x the
// input's bytes): 64@56 at batch 32, 17.6 + 30.5 us -> 40.0-40.6 us per
// conv.  With 32 output channels per workgroup (or channel splits) the same
// transform work meets half the MFMA work and the separate kernel wins.
//
// Work decomposition.  A workgroup owns a block of 32 tiles x 32 output
// channels and runs 12 waves: wave (p, h) owns row p of the 6 x 6 transform
// points, xi = 6p + q for q = 0..5, and input-channel chunk parity h (the
// two halves of the workgroup take alternate chunks of 8 channels).  For its
// six points a wave accumulates the whole 32 x 32 block with
// v_mfma_f32_32x32x2_f32, 6 x 16 accumulator registers, at the instruction's
// full issue rate (64 cycles, dependent chains included).  No operand is
// shared between waves, so each wave loads its own A (U) and B (V)
// fragments straight from memory into registers, 16 bytes per lane
// (lane l: row l % 32, channels 4 (l / 32) .. + 3 of the chunk; a half-wave
// reads 512 contiguous bytes): no LDS and no barrier in the main loop, and
// each point's operands for the chunk two ahead are requested as soon as
// its four MFMAs are issued, so about 10 KB per wave stay in flight.
//
// Output transform.  Y = A^T M A is applied along q inside each wave,
// Z_h[p][b] = sum_q M[p][q] A[q][b] (4 values per (channel, tile) pair),
// then along p across the waves: Z goes through LDS (per round of 16
// channels: 2 halves x 512 pairs x 6 rows x 4 floats, 112 KB with the
// records padded against bank conflicts) and thread
// tid < 512 of the workgroup sums the two halves and finishes its pair:
// Y[a][b] = sum_p A^T[a][p] Z[p][b], + bias (+ residual), activation, four
// row stores.
//
// Layers with few blocks split the input channels over `splits`
// workgroups (grid), each writing its partial Y (linear in M) to a
// workspace as tile rows, [splits][K][4 rows][T][4]: every part store is an
// aligned 16-byte row and a wave's 64 lanes (consecutive tiles) write 1 KB
// contiguously, whatever OW is; wino_fused_reduce sums the parts and
// applies bias, residual and activation.
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "nhip_internal.h"

namespace nhip {
namespace {

constexpr int kThreads = 768;       // 12 waves: 2 channel-chunk halves x 6 point rows
constexpr int kTB = 32;             // tiles per block
constexpr int kKB = 32;             // output channels per block
constexpr int kCB = 8;              // input channels per chunk
constexpr int kPairs = kTB * kKB / 2;  // (channel, tile) pairs per epilogue round
// Z record of one pair: 6 rows x 4 floats, padded to 28 floats so that the
// 16-byte accesses of 16 consecutive lanes (records 112 bytes apart) fall on
// distinct LDS banks.
constexpr int kZRec = 28;
constexpr int kLdsBytes = 2 * kPairs * kZRec * (int)sizeof(float);  // Z of both halves, 112 KB
constexpr int kXcds = 8;            // MI355X: workgroup L runs on XCD L % 8

struct FusedArgs {
  const float* V;       // [36][c_pad/4][t_pad][4] (not with XT)
  const float* x;       // XT: the input [N][C][H][W]
  uint32_t x_bytes;     // XT: its size (< 2^31)
  int C, H, W, pt, pl;  // XT: input channels, extent, top / left padding
  int xvec;             // XT: pl == 1, W % 4 == 0, 16-byte aligned input
  const float* U;       // [36][c_pad/4][m_pad][4]
  const float* bias;    // [m_pad]
  const float* residual;
  float* out;           // [N][K][OH][OW]; with splits > 1 the parts [splits][K][4][T][4]
  int K, OH, OW, th, tw, T, t_pad, m_pad, c_pad;
  int nt, nk, splits, per;  // tile blocks, channel blocks, channel splits, chunks per split
  int kb_fast;              // block order: channel block fastest (1) or tile block fastest (0)
  int64_t part_stride;      // K*16*T (< 2^31): elements per channel-split part
  uint32_t v_bytes;         // size of V (< 2^31)
  uint32_t u_bytes;         // size of U (< 2^31)
};

template <int ACT>
__device__ __forceinline__ float activate(float v) {
  if constexpr (ACT == NHIP_ACT_RELU) return v < 0.f ? 0.f : v;
  if constexpr (ACT == NHIP_ACT_SIGMOID) return __frcp_rn(1.0f + __expf(-v));
  return v;
}

// FINAL: write act(Y + bias (+ residual)) with activation ACT; otherwise
// the raw part of channel split s as tile rows.  VEC: OW % 4 == 0 (an
// output tile row is one aligned 16-byte vector).  KS: the two halves own
// the two 32-channel blocks of a 64-channel block (same tiles) and each
// runs every chunk; otherwise they share one 32-channel block and take
// alternate chunks.
// B^T (F(4x4, 3x3)) applied to six values, the rows sharing their partial
// sums (14 operations, fused multiply-adds):
//   o0 = 4 d0 - 5 d2 + d4          o3 = (d4 - d2) - 2 (d1 - d3)
//   o1 = (d3 + d4) - 4 (d1 + d2)   o4 = (d4 - d2) + 2 (d1 - d3)
//   o2 = (d4 - d3) + 4 (d1 - d2)   o5 = 4 d1 - 5 d3 + d5
__device__ __forceinline__ void bt6(float d0, float d1, float d2, float d3, float d4, float d5, float (&o)[6]) {
  const float a = d4 - d2, b = d1 - d3;
  o[0] = __builtin_fmaf(4.f, d0, __builtin_fmaf(-5.f, d2, d4));
  o[1] = __builtin_fmaf(-4.f, d1 + d2, d3 + d4);
  o[2] = __builtin_fmaf(4.f, d1 - d2, d4 - d3);
  o[3] = __builtin_fmaf(-2.f, b, a);
  o[4] = __builtin_fmaf(2.f, b, a);
  o[5] = __builtin_fmaf(4.f, d1, __builtin_fmaf(-5.f, d3, d5));
}

// XT: the input transform inside the GEMM (paired channel blocks, one
// part).  Per 8-channel chunk the workgroup's 256 (tile, channel) patches
// are transformed by its 768 threads, thread (tile, channel, g) taking rows
// 2g, 2g+1: first E = d B along its two patch rows (from registers loaded a
// chunk ahead) into LDS, then, a barrier later, columns 2g, 2g+1 of
// V = B^T E down the columns into LDS in the B-fragment layout
// [36][2][32][4], which the twelve waves read instead of V from memory.  One barrier per chunk:
// chunk c's MFMAs, chunk c+1's V rows and chunk c+2's E rows run between
// two barriers (two slots each for E and V, 147 KB of LDS).
constexpr int kXtSlot = 36 * 2 * 32 * 4;  // floats of one E or V slot
constexpr int kXtLdsBytes = 4 * kXtSlot * (int)sizeof(float);

// XV (XT only): the input rows are float4-aligned with one column of left
// padding (a.xvec), so a patch row's centre is one 16-byte load; a template
// argument rather than a branch, so the loop has one load sequence and the
// compiler's wait counts stay exact.
template <int ACT, bool FINAL, bool VEC, bool KS, bool XT = false, bool XV = false>
__global__ __launch_bounds__(kThreads, 1) void wino_fused_kernel(FusedArgs a) {
  static_assert(!XT || (KS && FINAL), "the in-kernel transform runs paired channel blocks in one part");
  extern __shared__ __attribute__((aligned(16))) float zs[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int p = wave % 6, h = wave / 6;

  // XCD-contiguous renumbering: each XCD takes a contiguous range of logical
  // blocks, ordered (block, split) with the split fastest; blocks ordered
  // so that consecutive ones share the larger operand (V: same tile block,
  // U: same channel block), which an XCD then fetches into its L2 once.
  // nk counts the workgroup's channel blocks (64 channels with KS).
  const int total = a.nt * a.nk * a.splits;
  const int L = blockIdx.x;
  const int xcd = L % kXcds, q8 = L / kXcds;
  const int logical = xcd * (total / kXcds) + min(xcd, total % kXcds) + q8;
  const int s = logical % a.splits, blk = logical / a.splits;
  const int kb = a.kb_fast ? blk % a.nk : blk / a.nt;
  const int tb = a.kb_fast ? blk / a.nk : blk % a.nt;
  const int kbase = kb * (KS ? 2 * kKB : kKB), t0 = tb * kTB;
  const int k0 = kbase + (KS ? h * kKB : 0);  // this wave's 32 output channels
  const int nch = a.c_pad / kCB;
  const int cb = s * a.per, ce = min(nch, cb + a.per);
  // KS with an odd number of 32-channel blocks: the last half has none
  const bool kvalid = k0 < a.m_pad;

  // Operand addressing: byte offsets, lane part in the per-lane offset,
  // the rest (point, chunk, block) in the scalar offset.
  const __amdgpu_buffer_rsrc_t ur = make_rsrc(a.U, a.u_bytes), vr = make_rsrc(a.V, a.v_bytes);
  const uint32_t uoff = (uint32_t)(((lane >> 5) * a.m_pad + (lane & 31)) * 16);
  const uint32_t voff = (uint32_t)(((lane >> 5) * a.t_pad + (lane & 31)) * 16);
  const uint32_t u_xi = (uint32_t)nch * a.m_pad * 32, u_ch = (uint32_t)a.m_pad * 32;
  const uint32_t v_xi = (uint32_t)nch * a.t_pad * 32, v_ch = (uint32_t)a.t_pad * 32;
  const uint32_t u_base = (uint32_t)(6 * p) * u_xi + (uint32_t)(kvalid ? k0 : 0) * 16;
  const uint32_t v_base = (uint32_t)(6 * p) * v_xi + (uint32_t)t0 * 16;

  v16f acc[6];
#pragma unroll
  for (int q = 0; q < 6; ++q) acc[q] = v16f{};
  v4f av[6], bv[6];
  // Chunks past this split's end are pointed out of range and read as 0
  // without touching memory (an unconditional load: a conditional one
  // would make the compiler wait for it at the join).
  auto load = [&](int c, int q) {
    const bool live = c < ce && kvalid;
    av[q] = __builtin_bit_cast(
        v4f, __builtin_amdgcn_raw_buffer_load_b128(ur, live ? uoff : kBufOOB, u_base + q * u_xi + (uint32_t)c * u_ch, 0));
    if constexpr (!XT)
      bv[q] = __builtin_bit_cast(
          v4f, __builtin_amdgcn_raw_buffer_load_b128(vr, live ? voff : kBufOOB, v_base + q * v_xi + (uint32_t)c * v_ch, 0));
  };
  // One chunk: per point its four MFMAs (reduction index: lane half l / 32
  // supplies channel 4 (l / 32) + st at step st, for both operands), then
  // that point's operands of the wave's next chunk into the same registers.
  // The scheduling groups keep this order (left alone, the compiler issues
  // all twelve loads after the last MFMA).
  constexpr int kStep = KS ? 1 : 2;  // chunk stride of a wave
  auto chunk = [&](int c) {
#pragma unroll
    for (int q = 0; q < 6; ++q) {
#pragma unroll
      for (int st = 0; st < 4; ++st)
        acc[q] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[q][st], bv[q][st], acc[q], 0, 0, 0);
      load(c + kStep, q);
    }
#pragma unroll
    for (int q = 0; q < 6; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);  // 4 MFMAs
      __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);  // 2 vector-memory reads
    }
  };
  int c = cb + (KS ? 0 : h);
  if constexpr (!XT) {
#pragma unroll
    for (int q = 0; q < 6; ++q) load(c, q);
#pragma unroll
    for (int q = 0; q < 6; ++q) __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);
  }

  // XT: this thread's patch: tile t0 + xtl, channel 4 xchq + xcq of each
  // chunk, patch rows 2 xg, 2 xg + 1.
  const int xg = wave >> 2, xchq = wave & 1, xtl = ((wave >> 1) & 1) * 16 + (lane >> 2), xcq = lane & 3;
  const int xt = t0 + xtl;
  int xrow0 = 0, xx0 = 0;  // (image * C) * H + first patch row; first patch column
  bool xrows_ok[2] = {false, false};
  // a patch row's six values: column 0, columns 1..4 (one 16-byte load on
  // the vector path, kept as a vector so that the loaded registers are used
  // in place and no copy waits for the load), column 5
  struct XRows {
    float l[2];
    v4f m[2];
    float r[2];
  };
  XRows dreg;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, XT ? a.x_bytes : 0u);
  if constexpr (XT) {
    if (xt < a.T) {
      const int per_img = a.th * a.tw;
      const int img = xt / per_img, rem = xt - img * per_img;
      const int ty = rem / a.tw, tx = rem - ty * a.tw;
      const int y = 4 * ty - a.pt + 2 * xg;
      xrow0 = img * a.C * a.H + y;
      xx0 = 4 * tx - a.pl;
      xrows_ok[0] = (unsigned)y < (unsigned)a.H;
      xrows_ok[1] = (unsigned)(y + 1) < (unsigned)a.H;
    }
  }
  // the two patch rows of chunk c (zero outside the image, past C, past T)
  // (byte offsets of chunk 0 and per-column validity fixed per thread; the
  // chunk moves the offset by 8 channel planes)
  uint32_t xoff[2] = {0u, 0u};
  if constexpr (XT) {
#pragma unroll
    for (int r = 0; r < 2; ++r) xoff[r] = (uint32_t)((xrow0 + (4 * xchq + xcq) * a.H + r) * a.W + xx0) * 4u;
  }
  const bool xl_ok = xx0 >= 0, xr_ok = xx0 + 5 < a.W, xm_ok = xx0 + 1 < a.W;
  const uint32_t xplane8 = (uint32_t)(kCB * a.H * a.W) * 4u;
  auto load_d = [&](int cc, XRows& dr) {
    const bool cok = (cc < ce) & (cc * kCB + 4 * xchq + xcq < a.C);
    const uint32_t cofs = (uint32_t)cc * xplane8;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const bool yok = cok & xrows_ok[r];
      const uint32_t o = xoff[r] + cofs;
      dr.l[r] = buf_load_f32(xr, (yok & xl_ok) ? o : kBufOOB);
      if constexpr (XV) {
        dr.m[r] = __builtin_bit_cast(
            v4f, __builtin_amdgcn_raw_buffer_load_b128(xr, (yok & xm_ok) ? o + 4u : kBufOOB, 0, 0));
      } else {
        v4f m;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bool jok = (unsigned)(xx0 + 1 + j) < (unsigned)a.W;
          m[j] = buf_load_f32(xr, (yok & jok) ? o + (uint32_t)(4 * (j + 1)) : kBufOOB);
        }
        dr.m[r] = m;
      }
      dr.r[r] = buf_load_f32(xr, (yok & xr_ok) ? o + 20u : kBufOOB);
    }
  };
  // E rows 2xg, 2xg+1 (E[i][q] = row i of d times column q of B) into slot eb,
  // layout [i][q][chq][tile][cq]
  auto e_phase = [&](float* eb, const XRows& dr) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const float d[6] = {dr.l[r], dr.m[r][0], dr.m[r][1], dr.m[r][2], dr.m[r][3], dr.r[r]};
      float* e = eb + ((((2 * xg + r) * 6) * 2 + xchq) * 32 + xtl) * 4 + xcq;
      float o[6];
      bt6(d[0], d[1], d[2], d[3], d[4], d[5], o);
#pragma unroll
      for (int q = 0; q < 6; ++q) e[q * 256] = o[q];
    }
  };
  // V rows p = 2G, 2G+1 (V[p][q] = row p of B^T times column q of E) from
  // slot eb into slot vb, layout [xi][chq][tile][cq]
  // V columns q = 2xg, 2xg+1 (V[p][q] = row p of B^T times column q of E)
  // from slot eb into slot vb, layout [xi][chq][tile][cq]: twelve E values
  // read, twelve V values written
  auto v_phase = [&](const float* eb, float* vb) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int q = 2 * xg + r;
      const float* e = eb + ((q * 2 + xchq) * 32 + xtl) * 4 + xcq;  // E[i][q] at + i * 6 * 256
      const float e0 = e[0], e1 = e[1536], e2 = e[3072], e3 = e[4608], e4 = e[6144], e5 = e[7680];
      float* v = vb + ((q * 2 + xchq) * 32 + xtl) * 4 + xcq;  // V[p][q] at + p * 6 * 256
      float o[6];
      bt6(e0, e1, e2, e3, e4, e5, o);
#pragma unroll
      for (int pp = 0; pp < 6; ++pp) v[pp * 1536] = o[pp];
    }
  };
  // XT: one chunk's MFMAs with the B fragments from V slot vb, then the
  // next chunk's A operands
  auto chunk_xt = [&](int cc, const float* vb) {
    const float* vl = vb + ((6 * p * 2 + (lane >> 5)) * 32 + (lane & 31)) * 4;
    // point q + 1's B fragment read while point q's MFMAs run
    v4f bq = *reinterpret_cast<const v4f*>(vl);
#pragma unroll
    for (int q = 0; q < 6; ++q) {
      const v4f bn = q < 5 ? *reinterpret_cast<const v4f*>(vl + (q + 1) * 256) : bq;
#pragma unroll
      for (int st = 0; st < 4; ++st)
        acc[q] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[q][st], bq[st], acc[q], 0, 0, 0);
      load(cc + 1, q);
      bq = bn;
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // point 0's LDS read
#pragma unroll
    for (int q = 0; q < 6; ++q) {
      if (q < 5) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // the next point's LDS read
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);  // 4 MFMAs
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // 1 vector-memory read
    }
  };

  // This thread's epilogue pairs (tid < 512), set up while the first
  // chunk's operands are in flight: tile t0 + tid % 32 and, per
  // round rr, channel kbase + tid / 32 + 16 rr (+ 32 for the second half's
  // pair with KS).
  const int OHW = a.OH * a.OW;
  const bool own = tid < kPairs;
  const int kk = kbase + ((tid >> 5) & 15), tt = t0 + (tid & 31);
  const bool live_t = own && tt < a.T;
  constexpr int NQ = KS ? 2 : 1;  // pairs per thread and round
  int obase = 0, rows = 0, cols = 0;
  float bias_r[2][NQ];
#pragma unroll
  for (int rr = 0; rr < 2; ++rr)
#pragma unroll
    for (int e = 0; e < NQ; ++e) bias_r[rr][e] = 0.f;
  if (live_t) {
    const int per_img = a.th * a.tw;
    const int img = tt / per_img, rem = tt - img * per_img;
    const int ty = rem / a.tw, tx = rem - ty * a.tw;
    obase = (img * a.K + kk) * OHW + 4 * ty * a.OW + 4 * tx;
    rows = min(4, a.OH - 4 * ty);
    cols = min(4, a.OW - 4 * tx);
    if (FINAL) {
#pragma unroll
      for (int rr = 0; rr < 2; ++rr)
#pragma unroll
        for (int e = 0; e < NQ; ++e)  // m_pad entries, zero past K
          bias_r[rr][e] = kk + 16 * rr + 32 * e < a.m_pad ? a.bias[kk + 16 * rr + 32 * e] : 0.f;
    }
  }

  if constexpr (XT) {
    float* const vs0 = zs;
    float* const vs1 = zs + kXtSlot;
    float* const es0 = zs + 2 * kXtSlot;
    float* const es1 = zs + 3 * kXtSlot;
    // Prologue: the first two chunks' rows requested together, then chunk
    // 0's A operands, E and V of chunk 0 and E of chunk 1 formed, chunk 2's
    // rows on their way: the loop is entered with chunk 0's A operands and
    // chunk 2's rows in flight in that order, as every iteration leaves the
    // next one, so the compiler's wait counts in the loop are exact (each
    // MFMA waits for its own A operand only, not for the rows behind it).
    {
      XRows d1;
      load_d(cb, dreg);
      load_d(cb + 1, d1);
#pragma unroll
      for (int q = 0; q < 6; ++q) load(cb, q);
      e_phase(es0, dreg);
      __syncthreads();
      v_phase(es0, vs0);
      e_phase(es1, d1);
      load_d(cb + 2, dreg);
      __syncthreads();
    }
    for (int cc = cb; cc < ce; ++cc) {
      const bool odd = ((cc - cb) & 1) != 0;
      chunk_xt(cc, odd ? vs1 : vs0);
      if (cc + 1 < ce) v_phase(odd ? es0 : es1, odd ? vs0 : vs1);
      if (cc + 2 < ce) e_phase(odd ? es1 : es0, dreg);
      // unconditional (chunks past the end read nothing, out of range): every
      // path through the loop then leaves the same loads in flight, and the
      // compiler's wait before each point's MFMAs counts the rows behind the
      // A operand instead of waiting for them
      load_d(cc + 3, dreg);
      __syncthreads();
    }
  } else if (c < ce) {
    // The first chunk is peeled, so the loop is entered with the loads in
    // flight in the loop's own order: the compiler's wait counts at the loop
    // head are then exact (vmcnt(10) before each point) rather than vmcnt(0).
    chunk(c);
    for (c += kStep; c < ce; c += kStep) chunk(c);
  }

  const int tl = lane & 31, hi = lane >> 5;
  float* dst_part = a.out + (FINAL ? 0 : (int64_t)s * a.part_stride);
  // Z_h[p][.] of accumulator register r: (sum_q M[p][q] A[q][b]) for b = 0..3.
  auto zrow = [&](int r) {
    const float m0 = acc[0][r], m1 = acc[1][r], m2 = acc[2][r], m3 = acc[3][r], m4 = acc[4][r], m5 = acc[5][r];
    const float s12 = m1 + m2, d12 = m1 - m2, s34 = m3 + m4, d34 = m3 - m4;
    return v4f{m0 + s12 + s34, d12 + 2.f * d34, s12 + 4.f * s34, d12 + 8.f * d34 + m5};
  };
  // Round 1's Z are computed here, before the first barrier, while the
  // workgroup's slower waves are still in their loops.
  v4f z_late[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) z_late[j] = zrow(8 + j);
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    // Residual rows of this round's pairs, requested before the exchange.
    float res[NQ][4][4];
#pragma unroll
    for (int e = 0; e < NQ; ++e)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool ok = FINAL && a.residual && live_t && kk + 16 * rr + 32 * e < a.K && i < rows;
        const float* src = a.residual + obase + (16 * rr + 32 * e) * OHW + i * a.OW;
        if (VEC) {
          const v4f v = ok ? *reinterpret_cast<const v4f*>(src) : v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int j = 0; j < 4; ++j) res[e][i][j] = v[j];
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) res[e][i][j] = (ok && j < cols) ? src[j] : 0.f;
        }
      }
    // Z_h[p][.] of the wave's 8 pairs in this round: accumulator register r
    // of lane l is channel (r%4) + 8(r/4) + 4(l/32) of the wave's block,
    // tile l%32.
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r = 8 * rr + j;
      const int row = (r & 3) + 8 * ((r >> 2) & 1) + 4 * hi;  // channel within the round's 16
      *reinterpret_cast<v4f*>(zs + (h * kPairs + row * 32 + tl) * kZRec + p * 4) = rr ? z_late[j] : zrow(j);
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < NQ; ++e) {
      const int k = kk + 16 * rr + 32 * e;
      if (!(live_t && k < a.K)) continue;
      float z[6][4];
#pragma unroll
      for (int pp = 0; pp < 6; ++pp) {
        if (KS) {  // the pair of half e
          const v4f z0 = *reinterpret_cast<const v4f*>(zs + (e * kPairs + tid) * kZRec + pp * 4);
#pragma unroll
          for (int j = 0; j < 4; ++j) z[pp][j] = z0[j];
        } else {  // the two halves' partial sums of one pair
          const v4f z0 = *reinterpret_cast<const v4f*>(zs + tid * kZRec + pp * 4);
          const v4f z1 = *reinterpret_cast<const v4f*>(zs + (kPairs + tid) * kZRec + pp * 4);
#pragma unroll
          for (int j = 0; j < 4; ++j) z[pp][j] = z0[j] + z1[j];
        }
      }
      float y[4][4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float s12 = z[1][j] + z[2][j], d12 = z[1][j] - z[2][j];
        const float s34 = z[3][j] + z[4][j], d34 = z[3][j] - z[4][j];
        y[0][j] = z[0][j] + s12 + s34;
        y[1][j] = d12 + 2.f * d34;
        y[2][j] = s12 + 4.f * s34;
        y[3][j] = d12 + 8.f * d34 + z[5][j];
      }
      if (FINAL) {
        const float b = bias_r[rr][e];
        float* dst = a.out + obase + (16 * rr + 32 * e) * OHW;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (i >= rows) break;
          float o[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) o[j] = activate<ACT>(y[i][j] + b + res[e][i][j]);
          if (VEC) {
            *reinterpret_cast<v4f*>(dst + i * a.OW) = v4f{o[0], o[1], o[2], o[3]};
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              if (j < cols) dst[i * a.OW + j] = o[j];
          }
        }
      } else {
        float* dst = dst_part + ((int64_t)k * 4 * a.T + tt) * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *reinterpret_cast<v4f*>(dst + (int64_t)i * a.T * 4) = v4f{y[i][0], y[i][1], y[i][2], y[i][3]};
      }
    }
    if (rr == 0) __syncthreads();  // round 1 overwrites Z
  }
}

// out = act(sum_s part[s] + bias[k] (+ residual)), parts [splits][K][4][T][4]
// (tile t, row i, column j of the 4x4 output tile).  One thread per output
// tile row (image n, channel k, output row y, tile column tx): one aligned
// 16-byte read per part, up to four outputs (VEC: OW % 4 == 0, one 16-byte
// store).  Consecutive threads take consecutive tile columns, so both the
// part reads and the output writes of a wave are contiguous runs.
struct ReduceArgs {
  const float* part;
  int splits;
  int rows_total;      // N*K*OH*tw (< 2^31)
  int part_stride;     // K*16*T (< 2^31)
  int OH, OW, K, th, tw, T;
  const float* bias;
  const float* residual;
  float* out;
};

template <bool VEC, int ACT>
__global__ void wino_fused_reduce(ReduceArgs a) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= a.rows_total) return;
  const int tx = idx % a.tw;
  const int r0 = idx / a.tw;
  const int y = r0 % a.OH;
  const int r1 = r0 / a.OH;
  const int k = r1 % a.K, n = r1 / a.K;
  const int t = (n * a.th + (y >> 2)) * a.tw + tx;
  const float* src = a.part + ((int64_t)(k * 4 + (y & 3)) * a.T + t) * 4;
  v4f sum = *reinterpret_cast<const v4f*>(src);
  for (int z = 1; z < a.splits; ++z) sum += *reinterpret_cast<const v4f*>(src + (int64_t)z * a.part_stride);
  const float b = a.bias[k];
  const int64_t o = ((int64_t)(n * a.K + k) * a.OH + y) * a.OW + 4 * tx;
  if constexpr (VEC) {
    const v4f rv = a.residual ? *reinterpret_cast<const v4f*>(a.residual + o) : v4f{0.f, 0.f, 0.f, 0.f};
    v4f v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = activate<ACT>(sum[j] + b + rv[j]);
    *reinterpret_cast<v4f*>(a.out + o) = v;
  } else {
    const int cols = min(4, a.OW - 4 * tx);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (j < cols) a.out[o + j] = activate<ACT>(sum[j] + b + (a.residual ? a.residual[o + j] : 0.f));
  }
}

template <int ACT, bool FINAL, bool VEC, bool KS, bool XT = false, bool XV = false>
int launch_one(const FusedArgs& a, int64_t blocks, hipStream_t s) {
  constexpr int lds = XT ? std::max(kXtLdsBytes, kLdsBytes) : kLdsBytes;
  NHIP_TRY(ensure_dynamic_lds(reinterpret_cast<const void*>(&wino_fused_kernel<ACT, FINAL, VEC, KS, XT, XV>), lds));
  NHIP_LAUNCH("wino_fused", (wino_fused_kernel<ACT, FINAL, VEC, KS, XT, XV>), dim3((unsigned)blocks),
              dim3(kThreads), lds, s, a);
  return check_launch("wino_fused");
}

template <int ACT>
int launch_xt(const FusedArgs& a, int64_t blocks, hipStream_t s) {
  if (a.xvec)
    return a.OW % 4 == 0 ? launch_one<ACT, true, true, true, true, true>(a, blocks, s)
                         : launch_one<ACT, true, false, true, true, true>(a, blocks, s);
  return a.OW % 4 == 0 ? launch_one<ACT, true, true, true, true, false>(a, blocks, s)
                       : launch_one<ACT, true, false, true, true, false>(a, blocks, s);
}

template <int ACT, bool FINAL>
int launch_kernel(const FusedArgs& a, int64_t blocks, bool ks, hipStream_t s) {
  if (a.OW % 4 == 0)
    return ks ? launch_one<ACT, FINAL, true, true>(a, blocks, s) : launch_one<ACT, FINAL, true, false>(a, blocks, s);
  return ks ? launch_one<ACT, FINAL, false, true>(a, blocks, s) : launch_one<ACT, FINAL, false, false>(a, blocks, s);
}

template <bool VEC, int ACT>
int launch_reduce(const ReduceArgs& r, hipStream_t s) {
  NHIP_LAUNCH("wino_split_reduce", (wino_fused_reduce<VEC, ACT>), dim3((unsigned)ceil_div(r.rows_total, 256)),
              dim3(256), 0, s, r);
  return check_launch("wino_split_reduce");
}

struct FusedShape {
  int th, tw, nt, nk, nch, splits, per;
  bool ks;  // workgroups of two 32-channel blocks (halves by channel block, not by chunk)
};

// Blocks of 32 consecutive tiles x 32 output channels, one 12-wave
// workgroup per CU.  Channel splits only where the blocks would leave more
// than a quarter of the CUs idle: the smallest power of two that brings the
// workgroups to 3/4 of the CUs, each split keeping at least 4 chunks of 8
// channels (two per half).  NHIP_WINO_SPLITS forces a split count (tests).
FusedShape fused_shape(const nhip_conv_plan* p, int n, int oh, int ow) {
  FusedShape f;
  f.th = (int)ceil_div(oh, 4);
  f.tw = (int)ceil_div(ow, 4);
  f.nt = (int)ceil_div((int64_t)n * f.th * f.tw, kTB);
  f.nk = (int)ceil_div(p->g.k, kKB);
  f.nch = p->c_pad / kCB;
  // Blocks beyond one round of CUs: pair the channel blocks (one fill and
  // one epilogue per 64 channels instead of two rounds of workgroups).
  // NHIP_WINO_KS=0/1 forces it off / on (tests).
  const int ks_forced = setting_int("NHIP_WINO_KS", -1);
  f.ks = ks_forced >= 0 ? ks_forced != 0 && f.nk >= 2
                        : (int64_t)f.nt * f.nk > (int64_t)cu_count() && f.nk >= 2;
  if (f.ks) f.nk = (f.nk + 1) / 2;
  const int64_t blocks = (int64_t)f.nt * f.nk;  // workgroups per split
  const int forced = setting_int("NHIP_WINO_SPLITS", 0);
  f.splits = 1;
  if (forced > 0) {
    while (f.splits * 2 <= std::min(forced, 8) && f.splits * 2 <= f.nch) f.splits *= 2;
  } else {
    while (!f.ks && f.splits < 8 && 4 * blocks * f.splits < 3 * (int64_t)cu_count() && f.nch / (2 * f.splits) >= 4)
      f.splits *= 2;
  }
  f.per = (int)ceil_div(f.nch, f.splits);
  return f;
}

}  // namespace

uint64_t wino_gemm_out_parts_bytes(const nhip_conv_plan* p, int n, int oh, int ow) {
  const FusedShape f = fused_shape(p, n, oh, ow);
  return f.splits > 1 ? (uint64_t)f.splits * p->g.k * 16 * ((uint64_t)n * f.th * f.tw) * sizeof(float) : 0;
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
  if ((int64_t)p->g.k * 16 * n * f.th * f.tw >= (int64_t(1) << 31))  // 32-bit tile offsets in a part
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "winograd GEMM: partial sums above 2^31 elements");
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
  a.part_stride = (int64_t)p->g.k * 16 * a.T;
  a.m_pad = p->m_pad;
  a.c_pad = p->c_pad;
  a.nt = f.nt;
  a.nk = f.nk;
  a.splits = f.splits;
  a.per = f.per;
  // consecutive blocks share V (the same tiles) when V is the larger
  // operand, U (the same output channels) otherwise
  a.kb_fast = a.t_pad >= p->m_pad ? 1 : 0;
  const int64_t blocks = (int64_t)f.nt * f.nk * f.splits;
  if (a.x != nullptr) {  // XT: the input transform inside the GEMM
    switch (p->g.act) {
      case NHIP_ACT_NONE: return launch_xt<NHIP_ACT_NONE>(a, blocks, s);
      case NHIP_ACT_RELU: return launch_xt<NHIP_ACT_RELU>(a, blocks, s);
      case NHIP_ACT_SIGMOID: return launch_xt<NHIP_ACT_SIGMOID>(a, blocks, s);
      default: return fail(NHIP_STATUS_UNSUPPORTED, "winograd GEMM: unsupported activation");
    }
  }
  if (f.splits == 1) {
    switch (p->g.act) {
      case NHIP_ACT_NONE: return launch_kernel<NHIP_ACT_NONE, true>(a, blocks, f.ks, s);
      case NHIP_ACT_RELU: return launch_kernel<NHIP_ACT_RELU, true>(a, blocks, f.ks, s);
      case NHIP_ACT_SIGMOID: return launch_kernel<NHIP_ACT_SIGMOID, true>(a, blocks, f.ks, s);
      default: return fail(NHIP_STATUS_UNSUPPORTED, "winograd GEMM: unsupported activation");
    }
  }
  NHIP_TRY((launch_kernel<NHIP_ACT_NONE, false>(a, blocks, f.ks, s)));
  ReduceArgs r{};
  r.part = parts;
  r.splits = f.splits;
  r.rows_total = n * p->g.k * oh * f.tw;
  r.part_stride = (int)a.part_stride;
  r.OH = oh;
  r.OW = ow;
  r.K = p->g.k;
  r.th = f.th;
  r.tw = f.tw;
  r.T = a.T;
  r.bias = p->bias;
  r.residual = residual;
  r.out = out;
#define NHIP_REDUCE(V_)                                                                           \
  switch (p->g.act) {                                                                             \
    case NHIP_ACT_RELU: return launch_reduce<V_, NHIP_ACT_RELU>(r, s);                            \
    case NHIP_ACT_SIGMOID: return launch_reduce<V_, NHIP_ACT_SIGMOID>(r, s);                      \
    default: return launch_reduce<V_, NHIP_ACT_NONE>(r, s);                                       \
  }
  if (ow % 4 == 0) {
    NHIP_REDUCE(true)
  } else {
    NHIP_REDUCE(false)
  }
#undef NHIP_REDUCE
}

}  // namespace

// The input transform inside the GEMM (XT) for launches of paired channel
// blocks in one part (no channel split), unless NHIP_WINO_XT=0: the
// separate transform's write and re-read of V (2.25x the input's bytes)
// and its launch go away, for VALU work inside the GEMM.
bool wino_xt_selected(const nhip_conv_plan* p, int n, int h, int w, int oh, int ow) {
  if (setting_int("NHIP_WINO_XT", 1) == 0) return false;
  if ((int64_t)n * p->g.c * h * w >= (int64_t(1) << 31) / 4) return false;  // 32-bit byte offsets into x
  const FusedShape f = fused_shape(p, n, oh, ow);
  return f.ks && f.splits == 1;
}

int launch_wino_gemm_xt(const nhip_conv_plan* p, const float* in, const float* residual, float* out, int n, int h,
                        int w, int oh, int ow, hipStream_t s) {
  const FusedShape f = fused_shape(p, n, oh, ow);
  if (!f.ks || f.splits != 1)
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "winograd GEMM (in-kernel transform): shape not supported");
  FusedArgs a{};
  a.x = in;
  a.x_bytes = (uint32_t)((size_t)n * p->g.c * h * w * sizeof(float));
  a.C = p->g.c;
  a.H = h;
  a.W = w;
  a.pt = p->g.pt;
  a.pl = p->g.pl;
  a.xvec = p->g.pl == 1 && w % 4 == 0 && (reinterpret_cast<uintptr_t>(in) & 15) == 0;
  a.t_pad = (int)round_up((int64_t)n * f.th * f.tw, kTB);
  return launch_fused(p, a, f, residual, out, n, oh, ow, nullptr, s);
}

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
