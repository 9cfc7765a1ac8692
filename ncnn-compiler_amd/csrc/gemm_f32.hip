// fp32 MFMA GEMM core (v_mfma_f32_32x32x2_f32, wave64) and the two
// contractions that use it (the Winograd batched GEMM has its own kernel in
// wino_gemm.hip):
//   - implicit-GEMM Convolution over NCHW blobs (reference ConvertConvolution
//     fp32 path, NCNNToTosa.cpp:1316-1529, lowered upstream to
//     linalg.conv_2d_nhwc_hwcf: out = bias + sum_{kh,kw,c} x*w);
//   - InnerProduct (NCNNToTosa.cpp:5254-5392: zero-init matmul, then bias).
//
// GEMM view: D[i][j] = sum_k A[i][k] * B[k][j].  A rows i are output channels
// (conv) or input rows m (InnerProduct); B columns j are output pixels or
// InnerProduct outputs.  One workgroup = 4 waves
// (2x2) computes a BM x BN tile; each wave a (BM/2) x (BN/2) tile built from
// 32x32 MFMA blocks.  K advances in chunks of 16 through double-buffered LDS.
//
// MFMA k mapping: in chunk-local step s (0..7) lane l supplies k = 8*(l/32)+s
// for both operands, so each lane reads 8 consecutive k of its A row (two
// ds_read_b128) instead of 16 scattered words.  Any permutation of k is valid
// for a dot product as long as A and B use the same one.
#include <cstdio>
#include <cstdlib>

#include "nhip_internal.h"

namespace nhip {
namespace {

constexpr int kThreads = 256;
constexpr int kBK = 16;      // K chunk of the MFMA k mapping; tiles use BK = 16 or 32
constexpr int kRowPad = 4;  // LDS row padding (floats): conflict-free b128 reads
constexpr int kXcds = 8;    // accelerator complex dies on MI355X

enum class Mode { Conv, IP };

struct GemmArgs {
  // A operand
  const float* a;        // conv: weights [m_pad][lda]; IP: input [M][lda]
  int lda;
  int m;                 // valid rows of the problem (out channels / IP rows)
  // B operand
  const float* b;        // conv: input NCHW; IP: W [n_pad][ldb]
  int ldb;
  int n;                 // valid columns (pixels / IP outputs)
  int kdim;              // reduction length (multiple of BK after padding)
  int k_valid;           // IP: valid input length (loads past it read 0)
  uint32_t b_bytes;      // conv: size of the input tensor (< 2^31)
  // conv geometry
  const int* ktab;
  int C, H, W, OW, OHW, sh, sw, pt, pl;
  int pointwise;         // 1x1, stride 1, no padding: reduction index k is channel k (no ktab lookup)
  // epilogue
  float* d;              // conv: out NCHW; IP: out [M][ldd]
  int ldd;
  const float* bias;
  const float* residual;
  int act;
  int splits;            // split-K factor (IP): >1 writes raw partials to d
  int a_vec4;            // IP: lda % 4 == 0 (float4 A loads allowed)
};

__device__ __forceinline__ float apply_act(float v, int act) {
  if (act == NHIP_ACT_RELU) return v < 0.0f ? 0.0f : v;
  if (act == NHIP_ACT_SIGMOID) return 1.0f / (1.0f + __expf(-v));
  return v;
}

template <int BM, int BN, int BK, Mode MODE>
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(GemmArgs g) {
  static_assert(BK % kBK == 0, "BK is a multiple of the 16-wide MFMA k chunk");
  constexpr int TM = BM / 64;  // 32x32 blocks per wave along i
  constexpr int TN = BN / 64;  // along j
  constexpr int AS = BK + kRowPad;                  // As[BM][AS], Bs[BN][AS]
  constexpr int B_ELEMS = BN * AS;
  // One LDS array: two A and two B operand buffers, reused by the conv
  // epilogue for a 64 x (BN+4) staging slab.
  constexpr int OPER = 2 * (BM * AS + B_ELEMS);
  constexpr int SLAB = (MODE == Mode::Conv) ? 64 * (BN + 4) : 0;
  __shared__ __attribute__((aligned(16))) float smem[OPER > SLAB ? OPER : SLAB];
  auto As = [&](int buf) { return smem + buf * BM * AS; };
  auto Bs = [&](int buf) { return smem + 2 * BM * AS + buf * B_ELEMS; };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 31, lh = lane >> 5;

  // Workgroups are dispatched round-robin over the XCDs (8 on MI355X, each
  // with its own L2): hardware id L runs on XCD L % 8.  Renumber so that each
  // XCD gets a contiguous range of logical tiles; tiles that share an A row
  // block (same i) then run on the same XCD and share its L2.
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
  const int j0 = bx * BN;
  const int i0 = by * BM;
  const int split = bz;  // K split (grid z)

  const float* A = g.a;
  const float* B = g.b;

  const int nk_total = g.kdim / BK;
  const int per = (nk_total + g.splits - 1) / g.splits;
  const int kt_begin = min(nk_total, split * per);
  const int kt_end = min(nk_total, kt_begin + per);

  // ---- operand stages.  A: BM x BK floats as float4 rows.  B (Conv): im2col
  // gather, thread owns pixel column jj = tid % BN and KPT consecutive k
  // (KPT = BK*BN/256).  B (IP): W [j][k] rows, like A.
  constexpr int A_Q = BK / 4;  // float4 per A row chunk
  constexpr int A_LD = BM * A_Q / kThreads;
  constexpr int KPT = BK * BN / kThreads;
  constexpr int B_LD4 = BN * A_Q / kThreads;
  // Native vectors: HIP's float4 struct copies would keep a stage in scratch.
  struct Stage {
    v4f a[A_LD];
    float b[(MODE == Mode::Conv) ? KPT : 1];
    v4f b4[(MODE == Mode::Conv) ? 1 : B_LD4];
  };

  // Conv per-thread pixel state (fixed for the whole block).
  const int jj = tid % BN;
  const int kg = __builtin_amdgcn_readfirstlane(tid / BN);
  // Conv: the whole input is one wave-uniform buffer resource (< 2^31 bytes);
  // zero padding reads through kBufOOB offsets.
  const __amdgpu_buffer_rsrc_t img_rs = make_rsrc(B, g.b_bytes);
  int iy0 = 0, ix0 = 0, img_plane0 = 0;
  bool pix_ok = false;
  if constexpr (MODE == Mode::Conv) {
    const int p = j0 + jj;
    pix_ok = p < g.n;
    const int pp = pix_ok ? p : 0;
    const int img = pp / g.OHW;
    const int rem = pp - img * g.OHW;
    const int oh = rem / g.OW;
    const int ow = rem - oh * g.OW;
    iy0 = oh * g.sh - g.pt;
    ix0 = ow * g.sw - g.pl;
    img_plane0 = img * g.C;
  }

  auto gload = [&](Stage& st, int kt) {
#pragma unroll
    for (int u = 0; u < A_LD; ++u) {
      const int q = tid + u * kThreads;
      const int row = q / A_Q, kq = (q % A_Q) * 4;
      const int k = kt * BK + kq;
      if constexpr (MODE == Mode::IP) {
        const int r = i0 + row;
        v4f v = {0.f, 0.f, 0.f, 0.f};
        if (r < g.m) {
          const float* src = A + (int64_t)r * g.lda;
          if (g.a_vec4) {
            if (k < g.k_valid) v = *reinterpret_cast<const v4f*>(src + k);
          } else {
            v.x = (k + 0 < g.k_valid) ? src[k + 0] : 0.f;
            v.y = (k + 1 < g.k_valid) ? src[k + 1] : 0.f;
            v.z = (k + 2 < g.k_valid) ? src[k + 2] : 0.f;
            v.w = (k + 3 < g.k_valid) ? src[k + 3] : 0.f;
          }
        }
        st.a[u] = v;
      } else {
        st.a[u] = *reinterpret_cast<const v4f*>(A + (int64_t)(i0 + row) * g.lda + k);
      }
    }
    if constexpr (MODE == Mode::Conv) {
      const int kbase = kt * BK + kg * KPT;
#pragma unroll
      for (int u = 0; u < KPT; ++u) {
        int c = kbase + u, dy = 0, dx = 0;
        if (!g.pointwise) {  // wave-uniform table entry
          const int t = g.ktab[kbase + u];
          c = t >> 16;
          dy = (t >> 8) & 255;
          dx = t & 255;
        }
        const int y = iy0 + dy, x = ix0 + dx;
        const bool in = pix_ok && c < g.C && (unsigned)y < (unsigned)g.H && (unsigned)x < (unsigned)g.W;
        st.b[u] = buf_load_f32(img_rs, in ? (uint32_t)((((img_plane0 + c) * g.H + y) * g.W + x) * (int)sizeof(float))
                                          : kBufOOB);
      }
    } else {
#pragma unroll
      for (int u = 0; u < B_LD4; ++u) {
        const int q = tid + u * kThreads;
        const int row = q / A_Q, kq = (q % A_Q) * 4;
        st.b4[u] = *reinterpret_cast<const v4f*>(B + (int64_t)(j0 + row) * g.ldb + kt * BK + kq);
      }
    }
  };
  auto lstore = [&](const Stage& st, int buf) {
#pragma unroll
    for (int u = 0; u < A_LD; ++u) {
      const int q = tid + u * kThreads;
      const int row = q / A_Q, kq = (q % A_Q) * 4;
      *reinterpret_cast<v4f*>(&As(buf)[row * AS + kq]) = st.a[u];
    }
    if constexpr (MODE == Mode::Conv) {
#pragma unroll
      for (int u = 0; u < KPT; u += 4)
        *reinterpret_cast<v4f*>(&Bs(buf)[jj * AS + kg * KPT + u]) = v4f{st.b[u], st.b[u + 1], st.b[u + 2], st.b[u + 3]};
    } else {
#pragma unroll
      for (int u = 0; u < B_LD4; ++u) {
        const int q = tid + u * kThreads;
        const int row = q / A_Q, kq = (q % A_Q) * 4;
        *reinterpret_cast<v4f*>(&Bs(buf)[row * AS + kq]) = st.b4[u];
      }
    }
  };

  v16f acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

  auto compute = [&](int buf) {
#pragma unroll
    for (int kc = 0; kc < BK; kc += kBK) {
      v4f af[TM][2], bf[TN][2];
#pragma unroll
      for (int a = 0; a < TM; ++a) {
        const float* pa = &As(buf)[(wm * (BM / 2) + a * 32 + li) * AS + kc + lh * 8];
        af[a][0] = *reinterpret_cast<const v4f*>(pa);
        af[a][1] = *reinterpret_cast<const v4f*>(pa + 4);
      }
#pragma unroll
      for (int b = 0; b < TN; ++b) {
        const float* pb = &Bs(buf)[(wn * (BN / 2) + b * 32 + li) * AS + kc + lh * 8];
        bf[b][0] = *reinterpret_cast<const v4f*>(pb);
        bf[b][1] = *reinterpret_cast<const v4f*>(pb + 4);
      }
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
          for (int b = 0; b < TN; ++b)
            acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[a][s >> 2][s & 3], bf[b][s >> 2][s & 3], acc[a][b],
                                                             0, 0, 0);
    }
  };

  // Two LDS buffers, global loads two stages ahead; the loop body is
  // straight-line (two stages per trip, odd tail peeled) so the accumulators
  // keep one register range.
  const int n = kt_end - kt_begin;
  if (n > 0) {
    Stage s0, s1;
    gload(s0, kt_begin);
    if (n > 1) gload(s1, kt_begin + 1);
    lstore(s0, 0);
    __syncthreads();
    int i = 0;
    for (; i + 1 < n; i += 2) {
      if (i + 2 < n) gload(s0, kt_begin + i + 2);
      compute(0);
      lstore(s1, 1);
      __syncthreads();
      if (i + 3 < n) gload(s1, kt_begin + i + 3);
      compute(1);
      if (i + 2 < n) lstore(s0, 0);
      __syncthreads();
    }
    if (i < n) compute(0);
  }

  // ---- epilogue.  32x32 accumulator layout: register r of lane l holds
  // row (r%4) + 8*(r/4) + 4*(l/32), column l%32.
  if constexpr (MODE == Mode::Conv) {
    if (g.splits == 1) {
      // Staged through LDS one 64-row slab (a) at a time: each thread then
      // writes runs of 4 pixels of one output channel with 16-byte accesses
      // (bias once per run, residual read as a vector), 32-bit offsets (a
      // launch's tensors stay below 2^31 bytes).  Same order as the direct
      // epilogue: acc + bias, + residual, then the activation.
      constexpr int TS = BN + 4;  // staged row stride (floats)
      float* tile = smem;
      const int ohw = g.OHW;
      const bool vec = (ohw & 3) == 0;
#pragma unroll
      for (int a = 0; a < TM; ++a) {
        __syncthreads();
#pragma unroll
        for (int b = 0; b < TN; ++b)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            tile[(wm * 32 + (r & 3) + 8 * (r >> 2) + 4 * lh) * TS + wn * (BN / 2) + b * 32 + li] = acc[a][b][r];
        __syncthreads();
        for (int q = tid; q < 64 * (BN / 4); q += kThreads) {
          const int lr = q / (BN / 4), lc = (q % (BN / 4)) * 4;
          const int i = i0 + (lr >> 5) * (BM / 2) + a * 32 + (lr & 31);
          const int j = j0 + lc;
          if (i >= g.m || j >= g.n) continue;
          const float bi = g.bias[i];
          const int img = j / ohw, rem = j - img * ohw;
          const int o = (img * g.m + i) * ohw + rem;
          const v4f t = *reinterpret_cast<const v4f*>(&tile[lr * TS + lc]);
          if (vec && j + 4 <= g.n) {  // a 4-run never crosses an image when ohw % 4 == 0
            v4f v = t + bi;
            if (g.residual) v += *reinterpret_cast<const v4f*>(g.residual + o);
            v.x = apply_act(v.x, g.act);
            v.y = apply_act(v.y, g.act);
            v.z = apply_act(v.z, g.act);
            v.w = apply_act(v.w, g.act);
            *reinterpret_cast<v4f*>(g.d + o) = v;
          } else {
            for (int e = 0; e < 4 && j + e < g.n; ++e) {
              const int je = j + e, ie = je / ohw;
              const int oe = (ie * g.m + i) * ohw + (je - ie * ohw);
              float v = t[e] + bi;
              if (g.residual) v += g.residual[oe];
              g.d[oe] = apply_act(v, g.act);
            }
          }
        }
      }
      return;
    }
  }
#pragma unroll
  for (int b = 0; b < TN; ++b) {
    const int j = j0 + wn * (BN / 2) + b * 32 + li;
    if constexpr (MODE == Mode::Conv) {
      if (j >= g.n) continue;
      if (g.splits > 1) {  // raw partial sums [split][m][n]; bias etc. in conv_splitk_reduce
        float* P = g.d + (int64_t)split * g.m * g.n;
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int i = i0 + wm * (BM / 2) + a * 32 + (r & 3) + 8 * (r >> 2) + 4 * lh;
            if (i < g.m) P[(int64_t)i * g.n + j] = acc[a][b][r];
          }
        continue;
      }
      const int img = j / g.OHW;
      const int rem = j - img * g.OHW;
      const int64_t obase = (int64_t)img * g.m * g.OHW + rem;
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int i = i0 + wm * (BM / 2) + a * 32 + (r & 3) + 8 * (r >> 2) + 4 * lh;
          if (i < g.m) {
            const int64_t o = obase + (int64_t)i * g.OHW;
            float v = acc[a][b][r] + g.bias[i];
            if (g.residual) v += g.residual[o];
            g.d[o] = apply_act(v, g.act);
          }
        }
    } else {
      if (j >= g.n) continue;
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int i = i0 + wm * (BM / 2) + a * 32 + (r & 3) + 8 * (r >> 2) + 4 * lh;
          if (i < g.m) {
            if (g.splits > 1) {
              g.d[((int64_t)split * g.m + i) * g.ldd + j] = acc[a][b][r];
            } else {
              g.d[(int64_t)i * g.ldd + j] = apply_act(acc[a][b][r] + g.bias[j], g.act);
            }
          }
        }
    }
  }
}

// Split-K reduction for the implicit-GEMM convolution: part [S][m][npix] ->
// out NCHW = act(sum_s part + bias (+ residual)), the order of the unsplit
// epilogue.
__global__ void conv_splitk_reduce(const float* __restrict__ part, int splits, int m, int npix, int ohw,
                                   const float* __restrict__ bias, const float* __restrict__ residual,
                                   float* __restrict__ out, int act) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)m * npix) return;
  const int i = (int)(idx / npix), j = (int)(idx - (int64_t)i * npix);
  float acc = part[idx];
  for (int s = 1; s < splits; ++s) acc += part[(int64_t)s * m * npix + idx];
  const int img = j / ohw, rem = j - img * ohw;
  const int64_t o = ((int64_t)img * m + i) * ohw + rem;
  float v = acc + bias[i];
  if (residual) v += residual[o];
  out[o] = apply_act(v, act);
}

// Split-K reduction for InnerProduct: out = act((sum_s part[s]) + bias).
__global__ void ip_splitk_reduce(const float* part, const float* bias,
                                 float* out, int m, int n, int ldp,
                                 int splits, int act) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)m * n) return;
  const int i = (int)(idx / n), j = (int)(idx - (int64_t)i * n);
  // splits are added in order; the loads of 8 splits are issued together
  const float* src = part + (int64_t)i * ldp + j;
  const int64_t stride = (int64_t)m * ldp;
  float s = 0.f;
  int z = 0;
  for (; z + 8 <= splits; z += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = src[(z + u) * stride];
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
  }
  for (; z < splits; ++z) s += src[z * stride];
  out[idx] = apply_act(s + bias[j], act);
}

template <int BM, int BN, Mode MODE, int BK = kBK>
int launch(const GemmArgs& g, dim3 grid, hipStream_t s, const char* name) {
  NHIP_LAUNCH(name, (gemm_f32_kernel<BM, BN, BK, MODE>), grid, dim3(kThreads), 0, s, g);
  return check_launch(name);
}

}  // namespace

// ------------------------------- Convolution ------------------------------
namespace {
struct IgemmCfg {
  int bm, bn, splits;
};
// Tile: the largest that still gives about two workgroups per CU (64x64
// otherwise).  K split: when even that leaves the CUs short of work and K is
// long, split K so that each workgroup keeps at least 4 chunks.
IgemmCfg igemm_config(const nhip_conv_plan* p, int64_t npix) {
  const int64_t target = 2LL * cu_count();
  const int64_t mt128 = ceil_div(p->g.k, 128), mt64 = ceil_div(p->g.k, 64);
  const int64_t nt128 = ceil_div(npix, 128);
  IgemmCfg c{64, 64, 1};
  // Short reductions (1x1 and stem convolutions, K <= 256) are bandwidth-bound:
  // the 64x64 tile gives the most workgroups and measures fastest there.
  if (p->kred_pad > 256) {
    if (p->m_pad % 128 == 0 && mt128 * nt128 >= target) c = {128, 128, 1};
    else if (mt64 * nt128 >= target) c = {64, 128, 1};
  }
  // Tuning override NHIP_IGEMM_TILE="bm,bn" (64x64, 64x128, 128x128).
  if (const char* env = setting("NHIP_IGEMM_TILE")) {
    int bm = 0, bn = 0;
    if (std::sscanf(env, "%d,%d", &bm, &bn) == 2 && (bm == 64 || (bm == 128 && p->m_pad % 128 == 0)) &&
        (bn == 64 || bn == 128) && !(bm == 128 && bn == 64))
      c = {bm, bn, 1};
  }
  const int64_t tiles = ceil_div(p->g.k, c.bm) * ceil_div(npix, c.bn);
  const int nk = p->kred_pad / kBK;
  while (c.splits < 16 && tiles * c.splits < cu_count() && nk / (c.splits * 2) >= 4) c.splits *= 2;
  return c;
}
}  // namespace

uint64_t conv_igemm_f32_workspace(const nhip_conv_plan* p, int n, int oh, int ow) {
  if (pointwise_selected(p, n, oh, ow)) return 0;
  if (pw_dma_supported(p, n, oh, ow)) return conv_pw_dma_workspace(p, n, oh, ow);
  const int64_t npix = (int64_t)n * oh * ow;
  const IgemmCfg c = igemm_config(p, npix);
  return c.splits > 1 ? (uint64_t)c.splits * p->g.k * npix * sizeof(float) : 0;
}

int launch_conv_igemm_f32(const nhip_conv_plan* p, const float* in,
                          const float* residual, float* out, int n, int h,
                          int w, int oh, int ow, void* ws, uint64_t ws_bytes,
                          hipStream_t s) {
  // (the short-reduction kernel needs no workspace; the size query above
  // keeps the implicit GEMM's, which is then unused)
  if (smallk_supported(p, n, h, w, oh, ow)) return launch_conv_smallk(p, in, residual, out, n, h, w, oh, ow, s);
  if (kq_supported(p, n, h, w, oh, ow)) return launch_conv_kq(p, in, residual, out, n, h, w, oh, ow, s);
  if (pointwise_selected(p, n, h, w)) return launch_conv_pointwise_f32(p, in, residual, out, n, h, w, s);
  if (pw_dma_supported(p, n, h, w)) return launch_conv_pw_dma(p, in, residual, out, n, h, w, ws, ws_bytes, s);
  GemmArgs g{};
  g.a = p->weight;
  g.lda = p->kred_pad;
  g.m = p->g.k;
  g.b = in;
  g.b_bytes = (uint32_t)((size_t)n * p->g.c * h * w * sizeof(float));
  g.n = n * oh * ow;
  g.kdim = p->kred_pad;
  g.ktab = p->ktab;
  g.C = p->g.c;
  g.H = h;
  g.W = w;
  g.OW = ow;
  g.OHW = oh * ow;
  g.sh = p->g.sh;
  g.sw = p->g.sw;
  g.pt = p->g.pt;
  g.pl = p->g.pl;
  g.pointwise = p->g.kh == 1 && p->g.kw == 1 && p->g.sh == 1 && p->g.sw == 1 && p->g.pt == 0 && p->g.pl == 0 &&
                p->g.pb == 0 && p->g.pr == 0;
  g.d = out;
  g.bias = p->bias;
  g.residual = residual;
  g.act = p->g.act;
  const IgemmCfg c = igemm_config(p, g.n);
  g.splits = c.splits;
  if (c.splits > 1) {
    const uint64_t need = conv_igemm_f32_workspace(p, n, oh, ow);
    if (ws == nullptr || ws_bytes < need)
      return fail(NHIP_STATUS_OUTPUT_CAPACITY_INSUFFICIENT,
                  "implicit-GEMM conv: workspace of " + std::to_string(need) + " bytes required");
    g.d = static_cast<float*>(ws);
  }
  const dim3 grid((unsigned)ceil_div(g.n, c.bn), (unsigned)ceil_div(p->g.k, c.bm), (unsigned)c.splits);
  if (c.bm == 128)
    NHIP_TRY((launch<128, 128, Mode::Conv>(g, grid, s, "conv_igemm_f32<128,128>")));
  else if (c.bn == 128)
    NHIP_TRY((launch<64, 128, Mode::Conv>(g, grid, s, "conv_igemm_f32<64,128>")));
  else
    NHIP_TRY((launch<64, 64, Mode::Conv>(g, grid, s, "conv_igemm_f32<64,64>")));
  if (c.splits > 1) {
    const int64_t total = (int64_t)p->g.k * g.n;
    NHIP_LAUNCH("conv_splitk_reduce", conv_splitk_reduce, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, s,
                static_cast<const float*>(ws), c.splits, p->g.k, g.n, g.OHW, p->bias, residual, out, p->g.act);
    return check_launch("conv_splitk_reduce");
  }
  return ok();
}

// ------------------------------- InnerProduct -----------------------------
static int ip_splits(const nhip_ip_plan* p, int m) {
  const int64_t tiles = ceil_div(m, 64) * ceil_div(p->n_out, 64);
  const int nk = p->k_pad / kBK;
  int splits = 1;
  while (tiles * splits < 2LL * cu_count() && nk / (splits * 2) >= 8) splits *= 2;
  return splits;
}

uint64_t innerproduct_workspace(const nhip_ip_plan* p, int m) {
  const int splits = ip_splits(p, m);
  const uint64_t own = splits == 1 ? 0 : (uint64_t)splits * m * p->n_pad * sizeof(float);
  // the direct-to-LDS kernel runs when the input is 16-byte aligned; this
  // kernel otherwise: room for either
  return ip_dma_supported(p, nullptr, m) ? std::max(own, innerproduct_dma_workspace(p, m)) : own;
}

// ------------------- global average pooling + InnerProduct -----------------
// The MobileNet / ResNet head: ConvertPooling's global average
// (NCNNToTosa.cpp:1880-1990, the mean of every [H,W] plane) feeding
// ConvertInnerProduct (:5254-5392), in one pass over the input.  A
// workgroup of 16 waves owns 16 images x 256 outputs x one slice of ks <= 64
// channels.  The slice of one image is one contiguous run of ks planes: ipp
// images at a time come into LDS through 16-byte loads, one lane per plane
// sums it in element order (the CPU loop's order, so the means equal
// nhip_global_avgpool_f32's bit for bit), then the LDS holds the weight
// slice, v_mfma_f32_16x16x4_f32 multiplies, and the workgroup writes a
// split-K partial [split][n][n_out]; ip_splitk_reduce adds the splits in
// order, the bias and the activation.  The ceil(n_out / 256) workgroups of
// a slice (4 for 1000 outputs) read its planes, mostly from L2; the head is
// two launches instead of three.
namespace {
constexpr int kGapRows = 16, kGapCols = 256, kGapMaxK = 64, kGapThreads = 1024;
constexpr int kGapStage = 25600;  // floats of LDS: staged planes, then the weight slice
static_assert(kGapCols * (kGapMaxK + 4) <= kGapStage, "the weight slice fits the staging area");
static_assert(kGapThreads / 64 * 16 == kGapCols, "one 16-output MFMA block per wave");

struct GapIpArgs {
  const float* x;   // [n][C][hw]
  const float* w;   // [n_pad][k_pad], zero padded
  float* part;      // [splits][n][n_out]
  int n, C, hw, n_out, n_pad, k_pad, ks, ipp;
};

__global__ __launch_bounds__(kGapThreads) void gap_ip_kernel(GapIpArgs a) {
  __shared__ __attribute__((aligned(16))) float S[kGapStage];
  __shared__ float P[kGapRows][kGapMaxK + 4];  // pooled [image][channel of the slice]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c0 = blockIdx.x * kGapCols, z = blockIdx.y, img0 = blockIdx.z * kGapRows;
  const int k0 = z * a.ks;
  const int kv = min(a.ks, a.C - k0);  // channels of the slice inside the tensor
  const int L = kv * a.hw, L4 = L >> 2, Ls = (L + 3) & ~3;  // floats of one image's run, its LDS stride
  for (int e = tid; e < kGapRows * (kGapMaxK + 4); e += kGapThreads) (&P[0][0])[e] = 0.f;
  for (int i0 = 0; i0 < kGapRows && img0 + i0 < a.n; i0 += a.ipp) {
    const int ni = min(a.ipp, a.n - img0 - i0);
    const float* src = a.x + ((int64_t)(img0 + i0) * a.C + k0) * a.hw;
    const int64_t img_stride = (int64_t)a.C * a.hw;
    // runs of ni images: 16-byte loads (4-byte aligned sources), four in flight per lane
    for (int v0 = tid; v0 < ni * L4; v0 += 4 * kGapThreads) {
      v4f t[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int v = v0 + u * kGapThreads, i = v / max(L4, 1), q = v - i * L4;
        if (v < ni * L4) __builtin_memcpy(&t[u], src + i * img_stride + 4 * q, 16);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int v = v0 + u * kGapThreads, i = v / max(L4, 1), q = v - i * L4;
        if (v < ni * L4) *reinterpret_cast<v4f*>(&S[i * Ls + 4 * q]) = t[u];
      }
    }
    const int rem = L - 4 * L4;
    for (int e = tid; e < ni * rem; e += kGapThreads) {
      const int i = e / rem, j = e - i * rem;
      S[i * Ls + 4 * L4 + j] = src[i * img_stride + 4 * L4 + j];
    }
    __syncthreads();
    if (tid < ni * a.ks) {
      const int i = tid / a.ks, j = tid - i * a.ks;
      if (j < kv) {
        const float* pl = S + i * Ls + j * a.hw;
        float sum = 0.f;
        for (int e = 0; e < a.hw; ++e) sum = sum + pl[e];
        P[i0 + i][j] = sum / (float)a.hw;
      }
    }
    __syncthreads();
  }
  // weight slice [256 outputs][ks channels], 16-byte loads (k_pad and ks are multiples of 4)
  float (*Ws)[kGapMaxK + 4] = reinterpret_cast<float (*)[kGapMaxK + 4]>(S);
  const int kq = a.ks / 4;
  for (int e = tid; e < kGapCols * kq; e += kGapThreads) {
    const int col = e / kq, q4 = e - col * kq, k = k0 + 4 * q4;
    v4f v = v4f{0.f, 0.f, 0.f, 0.f};
    if (c0 + col < a.n_pad && k < a.k_pad) v = *reinterpret_cast<const v4f*>(a.w + (int64_t)(c0 + col) * a.k_pad + k);
    *reinterpret_cast<v4f*>(&Ws[col][4 * q4]) = v;
  }
  __syncthreads();
  // one C[16 images][16 outputs] block per wave: lane (li, q) supplies
  // A = P[li][4s + q] and B = Ws[16 wave + li][4s + q]; register r holds
  // C[image 4q + r][output li]
  const int li = lane & 15, q = lane >> 4;
  v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < kq; ++s)
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(P[li][4 * s + q], Ws[wave * 16 + li][4 * s + q], acc, 0, 0, 0);
  float* dst = a.part + (int64_t)z * a.n * a.n_out;
  const int col = c0 + wave * 16 + li;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int img = img0 + 4 * q + r;
    if (img < a.n && col < a.n_out) dst[(int64_t)img * a.n_out + col] = acc[r];
  }
}

// Channels per split: about one workgroup per CU, 16 to 64 channels per
// slice, at most 16 splits (each split's partial is n x n_out floats), and
// at least one image's slice in the staging area (4 <= ks).
int gap_ip_ks(const nhip_ip_plan* p, int n, int hw) {
  const int64_t others = ceil_div(p->n_out, kGapCols) * ceil_div(n, kGapRows);
  const int64_t splits = std::min<int64_t>(16, std::max<int64_t>(1, cu_count() / others));
  int ks = (int)round_up(ceil_div(p->k_in, splits), 4);
  ks = std::min(std::max(ks, 16), kGapMaxK);
  const int fit = (kGapStage / hw) / 4 * 4;  // run stride rounds up to 4 floats
  return std::min(ks, fit);
}

// Images per staging pass: the largest power of two up to 16 whose runs fit.
int gap_ip_ipp(int ks, int hw) {
  const int run = (int)round_up((int64_t)ks * hw, 4);
  int ipp = kGapRows;
  while (ipp > 1 && ipp * run > kGapStage) ipp /= 2;
  return ipp;
}
}  // namespace

bool gap_innerproduct_supported(int hw) { return hw >= 1 && hw <= kGapStage / 4; }

uint64_t gap_innerproduct_workspace(const nhip_ip_plan* p, int n, int hw) {
  if (!gap_innerproduct_supported(hw)) return 0;
  const int splits = (int)ceil_div(p->k_in, gap_ip_ks(p, n, hw));
  return (uint64_t)splits * n * p->n_out * sizeof(float);
}

int launch_gap_innerproduct_f32(const nhip_ip_plan* p, const float* in, float* out, int n, int hw, void* ws,
                                uint64_t ws_bytes, hipStream_t s) {
  if (!gap_innerproduct_supported(hw))
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION,
                "global_avgpool_innerproduct: planes of at most " + std::to_string(kGapStage / 4) + " pixels");
  const int ks = gap_ip_ks(p, n, hw);
  const int splits = (int)ceil_div(p->k_in, ks);
  const uint64_t need = (uint64_t)splits * n * p->n_out * sizeof(float);
  if (ws == nullptr || ws_bytes < need)
    return fail(NHIP_STATUS_OUTPUT_CAPACITY_INSUFFICIENT,
                "global_avgpool_innerproduct: workspace of " + std::to_string(need) + " bytes required");
  GapIpArgs a{in, p->weight, static_cast<float*>(ws), n, p->k_in, hw, p->n_out, p->n_pad, p->k_pad, ks,
              gap_ip_ipp(ks, hw)};
  const dim3 grid((unsigned)ceil_div(p->n_out, kGapCols), (unsigned)splits, (unsigned)ceil_div(n, kGapRows));
  NHIP_LAUNCH("gap_innerproduct_f32", gap_ip_kernel, grid, dim3(kGapThreads), 0, s, a);
  NHIP_TRY(check_launch("gap_innerproduct_f32"));
  const int64_t total = (int64_t)n * p->n_out;
  NHIP_LAUNCH("ip_splitk_reduce", ip_splitk_reduce, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, s,
              static_cast<const float*>(ws), p->bias, out, n, p->n_out, p->n_out, splits, p->act);
  return check_launch("ip_splitk_reduce");
}

int launch_innerproduct_f32(const nhip_ip_plan* p, const float* in,
                            float* out, int m, void* ws, uint64_t ws_bytes,
                            hipStream_t s) {
  if (ip_kq_supported(p, in, m)) return launch_ip_kq(p, in, out, m, s);
  if (ip_dma_supported(p, in, m)) return launch_innerproduct_dma(p, in, out, m, ws, ws_bytes, s);
  GemmArgs g{};
  g.a = in;
  g.lda = p->k_in;
  g.m = m;
  g.k_valid = p->k_in;
  g.a_vec4 = (p->k_in % 4 == 0 && (reinterpret_cast<uintptr_t>(in) & 15) == 0) ? 1 : 0;
  g.b = p->weight;
  g.ldb = p->k_pad;
  g.n = p->n_out;
  g.kdim = p->k_pad;
  g.bias = p->bias;
  g.act = p->act;
  const int splits = ip_splits(p, m);
  g.splits = splits;
  if (splits > 1) {
    const uint64_t need = innerproduct_workspace(p, m);
    if (ws == nullptr || ws_bytes < need)
      return fail(NHIP_STATUS_OUTPUT_CAPACITY_INSUFFICIENT,
                  "innerproduct: workspace of " + std::to_string(need) +
                      " bytes required");
    g.d = static_cast<float*>(ws);
    g.ldd = p->n_pad;
  } else {
    g.d = out;
    g.ldd = p->n_out;
  }
  // B rows (weights) are padded to n_pad (multiple of 64); j bounds are
  // checked in the epilogue only.
  NHIP_TRY((launch<64, 64, Mode::IP>(g, dim3(p->n_pad / 64, (int)ceil_div(m, 64), splits), s,
                                     "innerproduct_f32<64,64>")));
  if (splits > 1) {
    const int64_t total = (int64_t)m * p->n_out;
    NHIP_LAUNCH("ip_splitk_reduce", ip_splitk_reduce, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, s,
                       static_cast<const float*>(ws), p->bias, out, m, p->n_out, p->n_pad,
                       splits, p->act);
    return check_launch("ip_splitk_reduce");
  }
  return ok();
}

}  // namespace nhip
