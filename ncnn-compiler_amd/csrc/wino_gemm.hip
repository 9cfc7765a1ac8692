// The 36 batched GEMMs of Winograd F(4,3):
//   M[s][xi] (m_pad x t_pad) = U[xi] (m_pad x c_pad) * V[xi] (c_pad x t_pad)
// over the K range of split s (the output transform sums the splits).
//
// One workgroup = 4 waves (2x2) computes a BM x BN tile of one xi, each wave a
// (BM/2) x (BN/2) tile of 32x32 blocks with v_mfma_f32_32x32x2_f32.  K advances
// in chunks of BK (16 or 32) through two LDS buffers, and global loads run two
// chunks ahead of the MFMAs: while chunk k is multiplied, chunk k+1 (already
// in registers) waits to be written to LDS and chunk k+2 is in flight.  The
// loop is unrolled by two so that each register stage is a fixed set of VGPRs.
//
// MFMA k mapping: inside each 16-wide sub-chunk, lane l supplies
// k = 8*(l/32)+s at step s (s = 0..7) to both operands.  Both LDS tiles hold k
// contiguously (B is transposed on the way in), so a lane's fragment of one
// operand is two ds_read_b128.
// Accumulator layout (32x32): register r of lane l = row (r%4)+8*(r/4)+4*(l/32),
// column l%32.
#include <cstdio>
#include <cstdlib>

#include "nhip_internal.h"

namespace nhip {
namespace {

constexpr int kThreads = 256;
constexpr int kBK = 16;   // MFMA k sub-chunk
constexpr int kPad = 4;   // LDS row padding (floats)
constexpr int kXcds = 8;  // MI355X: workgroup L runs on XCD L % 8

struct WinoArgs {
  const float* U;  // [36][m_pad][c_pad]
  const float* V;  // [36][c_pad][t_pad]
  float* M;        // [splits][36][m_pad][t_pad]
  int m_pad, c_pad, t_pad, splits;
};

template <int BM, int BN, int BK>
__global__ __launch_bounds__(kThreads) void wino_gemm_kernel(WinoArgs g) {
  constexpr int TM = BM / 64, TN = BN / 64;
  constexpr int AS = BK + kPad;     // As[BM][AS], Bs[BN][AS]: k contiguous
  static_assert(BK % 16 == 0 && AS % 8 == 4, "the B transpose mapping below");
  constexpr int KQ = BK / 4;        // float4 per row chunk
  constexpr int A_LD = BM * KQ / kThreads;  // float4 loads per thread per chunk
  constexpr int B_LD = BN * KQ / kThreads;
  constexpr int NSUB = BK / kBK;    // 16-wide MFMA k sub-chunks per chunk
  __shared__ __attribute__((aligned(16))) float As[2][BM * AS];
  __shared__ __attribute__((aligned(16))) float Bs[2][BN * AS];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 31, lh = lane >> 5;

  // XCD-contiguous renumbering of the workgroups (see kXcds).
  int bx, by, bz;
  {
    const int nbx = gridDim.x, nby = gridDim.y;
    const int total = nbx * nby * gridDim.z;
    const int L = blockIdx.x + nbx * (blockIdx.y + nby * blockIdx.z);
    const int x = L % kXcds, q = L / kXcds;
    const int logical = x * (total / kXcds) + min(x, total % kXcds) + q;
    bx = logical % nbx;
    by = (logical / nbx) % nby;
    bz = logical / (nbx * nby);
  }
  const int j0 = bx * BN, i0 = by * BM;
  const int xi = bz % 36, split = bz / 36;
  const float* A = g.U + (int64_t)xi * g.m_pad * g.c_pad + (int64_t)i0 * g.c_pad;
  const float* B = g.V + (int64_t)xi * g.c_pad * g.t_pad + j0;

  const int nk = g.c_pad / BK;
  const int per = (nk + g.splits - 1) / g.splits;
  const int kb = split * per;
  const int n = max(0, min(nk, kb + per) - kb);

  // Native 4-float vectors (not HIP's float4 struct, whose copies lower to
  // memcpy and keep the stage in scratch memory).
  struct Stage {
    v4f a[A_LD];
    v4f b[B_LD];
  };
  // A chunk: BM rows of BK contiguous k.  B chunk: BK rows of BN contiguous j
  // (V is [c][t]); stored transposed so that a lane's 8 k values of one
  // column are contiguous in LDS.  B element q (16 bytes: 4 columns of one
  // row) is row 16*(q / (4*BN)) + q % 16, column quad (q / 16) % (BN/4): a
  // half-wave holds 16 rows x 2 column quads, whose transposed 4-byte
  // stores (row stride AS = 4 mod 8 floats) hit 32 distinct banks; a wave
  // loads 16 rows x 64 contiguous bytes.
  auto gload = [&](Stage& st, int kt) {
#pragma unroll
    for (int u = 0; u < A_LD; ++u) {
      const int q = tid + u * kThreads;
      const int row = q / KQ, kq = (q % KQ) * 4;
      st.a[u] = *reinterpret_cast<const v4f*>(A + (int64_t)row * g.c_pad + kt * BK + kq);
    }
#pragma unroll
    for (int u = 0; u < B_LD; ++u) {
      const int q = tid + u * kThreads;
      const int row = (q / (4 * BN)) * 16 + (q & 15), jq = ((q >> 4) % (BN / 4)) * 4;
      st.b[u] = *reinterpret_cast<const v4f*>(B + (int64_t)(kt * BK + row) * g.t_pad + jq);
    }
  };
  auto lstore = [&](const Stage& st, int buf) {
#pragma unroll
    for (int u = 0; u < A_LD; ++u) {
      const int q = tid + u * kThreads;
      const int row = q / KQ, kq = (q % KQ) * 4;
      *reinterpret_cast<v4f*>(&As[buf][row * AS + kq]) = st.a[u];
    }
#pragma unroll
    for (int u = 0; u < B_LD; ++u) {
      const int q = tid + u * kThreads;
      const int k = (q / (4 * BN)) * 16 + (q & 15), jq = ((q >> 4) % (BN / 4)) * 4;
      float* dst = &Bs[buf][jq * AS + k];
      dst[0] = st.b[u].x;
      dst[AS] = st.b[u].y;
      dst[2 * AS] = st.b[u].z;
      dst[3 * AS] = st.b[u].w;
    }
  };

  v16f acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

  struct Frag {
    v4f a[TM][2];
    v4f b[TN][2];
  };
  auto fread = [&](Frag& f, int buf, int kc) {
#pragma unroll
    for (int a = 0; a < TM; ++a) {
      const float* pa = &As[buf][(wm * (BM / 2) + a * 32 + li) * AS + kc + lh * 8];
      f.a[a][0] = *reinterpret_cast<const v4f*>(pa);
      f.a[a][1] = *reinterpret_cast<const v4f*>(pa + 4);
    }
#pragma unroll
    for (int b = 0; b < TN; ++b) {
      const float* pb = &Bs[buf][(wn * (BN / 2) + b * 32 + li) * AS + kc + lh * 8];
      f.b[b][0] = *reinterpret_cast<const v4f*>(pb);
      f.b[b][1] = *reinterpret_cast<const v4f*>(pb + 4);
    }
  };
  auto fmma = [&](const Frag& f) {
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(f.a[a][s >> 2][s & 3], f.b[b][s >> 2][s & 3],
                                                           acc[a][b], 0, 0, 0);
  };
  // One chunk: the fragments of sub-chunk u+1 are read while sub-chunk u
  // multiplies.
  auto compute = [&](int buf) {
    Frag f0, f1;
    fread(f0, buf, 0);
#pragma unroll
    for (int u = 0; u < NSUB; u += 2) {
      if (u + 1 < NSUB) fread(f1, buf, (u + 1) * kBK);
      fmma(f0);
      if (u + 1 < NSUB) {
        if (u + 2 < NSUB) fread(f0, buf, (u + 2) * kBK);
        fmma(f1);
      }
    }
  };

  // The loop body is straight-line (two chunks per trip, odd tail peeled):
  // an exit in the middle of the body makes the register allocator give the
  // accumulators a different register range on each path and copy them
  // through VGPRs on every trip.
  if (n > 0) {
    Stage s0, s1;
    gload(s0, kb);
    if (n > 1) gload(s1, kb + 1);
    lstore(s0, 0);
    __syncthreads();
    int i = 0;
    for (; i + 1 < n; i += 2) {
      // chunk i in LDS buffer 0, chunk i+1 in s1
      if (i + 2 < n) gload(s0, kb + i + 2);
      compute(0);
      lstore(s1, 1);
      __syncthreads();
      // chunk i+1 in LDS buffer 1, chunk i+2 in s0
      if (i + 3 < n) gload(s1, kb + i + 3);
      compute(1);
      if (i + 2 < n) lstore(s0, 0);
      __syncthreads();
    }
    if (i < n) compute(0);  // odd n: the last chunk is in buffer 0
  }

  float* D = g.M + ((int64_t)split * 36 + xi) * g.m_pad * g.t_pad;
#pragma unroll
  for (int b = 0; b < TN; ++b) {
    const int j = j0 + wn * (BN / 2) + b * 32 + li;
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = i0 + wm * (BM / 2) + a * 32 + (r & 3) + 8 * (r >> 2) + 4 * lh;
        D[(int64_t)i * g.t_pad + j] = acc[a][b][r];
      }
  }
}

bool cfg_valid(const WinoGemmCfg& c, int m_pad, int c_pad, int t_pad) {
  return (c.bm == 64 || c.bm == 128) && (c.bn == 64 || c.bn == 128) && (c.bk == 16 || c.bk == 32) &&
         (c.splits == 1 || c.splits == 2 || c.splits == 4) && m_pad % c.bm == 0 && t_pad % c.bn == 0 &&
         c_pad % c.bk == 0 && c.splits <= c_pad / c.bk;
}

}  // namespace

WinoGemmCfg wino_gemm_config(int m_pad, int c_pad, int t_pad) {
  // Tuning override: NHIP_WINO_GEMM="bm,bn,bk,splits" (ignored when not
  // valid for the shape).
  if (const char* env = setting("NHIP_WINO_GEMM")) {
    WinoGemmCfg c{};
    if (std::sscanf(env, "%d,%d,%d,%d", &c.bm, &c.bn, &c.bk, &c.splits) == 4 && cfg_valid(c, m_pad, c_pad, t_pad))
      return c;
  }
  // 64x64 tiles (the most workgroups per batch: the stage shapes have small
  // M or small T), 32-wide K chunks when K is long enough, no K split
  // (partial buffers cost the output transform more than they save here).
  WinoGemmCfg c{64, 64, c_pad % 32 == 0 && c_pad >= 128 ? 32 : kBK, 1};
  if (!cfg_valid(c, m_pad, c_pad, t_pad)) c.bk = kBK;
  return c;
}

int launch_wino_gemm(const float* U, const float* V, float* M, int m_pad, int c_pad, int t_pad,
                     const WinoGemmCfg& c, hipStream_t s) {
  if (!cfg_valid(c, m_pad, c_pad, t_pad)) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "wino_gemm: bad tile config");
  const WinoArgs g{U, V, M, m_pad, c_pad, t_pad, c.splits};
  const dim3 grid(t_pad / c.bn, m_pad / c.bm, 36 * c.splits);
#define NHIP_WINO_CASE(BM_, BN_, BK_)                                                                   \
  if (c.bm == BM_ && c.bn == BN_ && c.bk == BK_) {                                                      \
    NHIP_LAUNCH("wino_gemm<" #BM_ "," #BN_ "," #BK_ ">", (wino_gemm_kernel<BM_, BN_, BK_>), grid, dim3(kThreads), 0, \
                s, g);                                                                                  \
    return check_launch("wino_gemm");                                                                   \
  }
  NHIP_WINO_CASE(64, 64, 16)
  NHIP_WINO_CASE(64, 128, 16)
  NHIP_WINO_CASE(128, 64, 16)
  NHIP_WINO_CASE(128, 128, 16)
  NHIP_WINO_CASE(64, 64, 32)
  NHIP_WINO_CASE(64, 128, 32)
  NHIP_WINO_CASE(128, 64, 32)
  NHIP_WINO_CASE(128, 128, 32)
#undef NHIP_WINO_CASE
  return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "wino_gemm: bad tile config");
}

}  // namespace nhip
