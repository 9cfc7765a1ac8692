// fp32 MFMA GEMM fed by direct-to-LDS loads, for the contractions whose
// tiles are too few, or whose reductions too short, to hide memory latency
// with register prefetch:
//   - InnerProduct (NCNNToTosa.cpp:5254-5392: zero-init matmul, then bias):
//     D[i][j] = sum_k X[i][k] W[j][k], X the input rows, W the weights;
//   - 1x1 stride-1 unpadded Convolution on NCHW (ConvertConvolution fp32,
//     NCNNToTosa.cpp:1316-1529): D[o][(n, p)] = sum_c W[o][c] x[n][c][p],
//     whose pixel columns run across images (7x7 and 14x14 layers: a few
//     thousand pixels, hundreds of channels).
//
// A workgroup (4 waves, 2x2) owns a BM x 64 tile of D (BM = 64 or 128).  K
// advances in stages of 32 through a ring of LDS slots: the loads of the
// next 3 (BM = 64) or 2 (BM = 128) stages are in flight while one stage is
// multiplied, with no register cost (67-74 KB of LDS: two workgroups per
// CU).
//   A stage (rows i, 32 k): 16-byte copies, 8 rows of 128 bytes per wave
//     copy; quad q of row r is stored at quad q ^ (r % 8), so the MFMA
//     operand reads (32 rows at one quad) spread over the banks.
//   B stage, InnerProduct: the weight rows j, like A.
//   B stage, convolution: row k = the 64 pixel columns of channel k, one
//     4-byte copy per row (lane = column, any image boundary inside), rows
//     68 floats apart so that rows k and k + 8 fall on different banks.
// MFMA v_mfma_f32_32x32x2_f32; within a 16-k chunk, step s takes
// k = s and 8 + s from lane halves 0 and 1 (the k order of gemm_f32.hip).
// Positions past the operands (rows, columns, k past the data) read zero
// through out-of-range buffer offsets; every in-range offset is below the
// operand's size (< 2^31 bytes, checked on the host).  Split K (grid z) writes raw partial
// sums [split][m][n] that ip_splitk_reduce / conv_splitk_reduce finish.
#include <algorithm>

#include "lds_dma.h"
#include "nhip_internal.h"

namespace nhip {
namespace {

constexpr int kThreads = 256;
constexpr int kBK = 32;      // k per stage
constexpr int kBN = 64;      // tile columns
constexpr int kBRow = 68;    // convolution B row stride (floats)
constexpr int kXcds = 8;

enum class Kind { IP, PW };

struct DmaGemmArgs {
  const float* a;       // rows [i][lda]: IP input, PW weights (zero past the reduction)
  uint32_t a_bytes;
  int lda, ka;          // row stride; k at or past ka reads zero
  const float* b;       // IP: weights [j][ldb]; PW: x NCHW
  uint32_t b_bytes;
  int ldb, kb;          // IP: row stride, k at or past kb reads zero; PW: channels C (k >= C reads zero)
  int hw;               // PW: pixels per plane
  int m, n;             // rows i and columns j of D
  int stages;           // K / 32
  int splits;           // grid z; > 1: raw partials [split][m][n] at d (row stride n)
  float* d;
  int ldd;              // IP output row stride
  const float* bias;
  const float* residual;
  int act;
};

template <int BM, Kind K>
struct Layout {
  // LDS stage slots: kSlots - 1 stages in flight while one is multiplied
  // (67 KB at BM = 64, 72 KB at BM = 128 for the InnerProduct: two
  // workgroups per CU either way)
  static constexpr int kSlots = BM == 64 ? 4 : 3;
  static constexpr int kA = BM * kBK;                                   // floats
  static constexpr int kB = K == Kind::IP ? kBN * kBK : kBK * kBRow;    // floats
  static constexpr int kSlot = kA + kB;
  static constexpr int kBytes = kSlots * kSlot * (int)sizeof(float);
  static_assert(2 * kBytes <= 160 * 1024, "two workgroups per CU");
  static constexpr int kCopiesA = BM / 8;                  // 1 KB copies per stage
  static constexpr int kCopiesB = K == Kind::IP ? kBN / 8 : kBK;  // 1 KB or 256 B copies
  static constexpr int kPerWave = (kCopiesA + kCopiesB) / 4;
  static_assert((kCopiesA % 4) == 0 && (kCopiesB % 4) == 0, "whole copies per wave");
  static_assert(kPerWave * (kSlots - 2) < 64, "outstanding copies fit the 6-bit vmcnt");
};

__device__ __forceinline__ float act_fn(float v, int act) {
  if (act == NHIP_ACT_RELU) return v < 0.0f ? 0.0f : v;
  if (act == NHIP_ACT_SIGMOID) return 1.0f / (1.0f + __expf(-v));
  return v;
}

template <int BM, Kind K>
__global__ __launch_bounds__(kThreads, 2) void gemm_dma_kernel(DmaGemmArgs g) {
  using L = Layout<BM, K>;
  constexpr int kSlots = L::kSlots;
  constexpr int TM = BM / 64;  // 32-row MFMA blocks per wave
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 31, lh = lane >> 5;

  // Workgroup L runs on XCD L % 8: give each XCD a contiguous range of
  // logical tiles, column tiles fastest, so the tiles of one row block (the
  // same A rows) share an L2.
  int bx, by, bz;
  {
    const int nbx = gridDim.x, nby = gridDim.y;
    const int total = nbx * nby * gridDim.z;
    const int Lh = blockIdx.x + nbx * (blockIdx.y + nby * blockIdx.z);
    const int x = Lh % kXcds, q = Lh / kXcds;
    const int logical = x * (total / kXcds) + min(x, total % kXcds) + q;
    bx = logical % nbx;
    by = (logical / nbx) % nby;
    bz = logical / (nbx * nby);
  }
  const int j0 = bx * kBN, i0 = by * BM;
  const int per = (g.stages + g.splits - 1) / g.splits;
  const int s_begin = min(g.stages, bz * per);
  const int n_st = min(g.stages, s_begin + per) - s_begin;

  const uint32_t lds0 = (uint32_t)(uintptr_t)lds;
  const v4i ars = dma::raw_rsrc(g.a, g.a_bytes), brs = dma::raw_rsrc(g.b, g.b_bytes);
  // 16-byte copies: lane l covers row t*8 + l/8 of the copy and, at LDS quad
  // l%8, the k quad (l%8) ^ (l/8).
  const int rr = lane >> 3, kq = 4 * ((lane & 7) ^ rr);
  // PW: lane = pixel column j0 + lane: byte offset of (image, channel 0, p)
  uint32_t pix = kBufOOB;
  if constexpr (K == Kind::PW) {
    const int j = j0 + lane;
    if (j < g.n) {
      const int img = j / g.hw;
      pix = (uint32_t)(((int64_t)img * g.kb * g.hw + (j - img * g.hw)) * 4);
    }
  }

  auto issue = [&](int st, int slot) {  // stage st of this split into slot
    const int k0 = (s_begin + st) * kBK;
    const uint32_t sa = lds0 + (uint32_t)(slot * L::kSlot * 4);
    const uint32_t sb = sa + (uint32_t)(L::kA * 4);
#pragma unroll
    for (int c = 0; c < L::kCopiesA / 4; ++c) {
      const int t = wave + 4 * c;
      const int k = k0 + kq, row = i0 + t * 8 + rr;
      const uint32_t off = (k < g.ka && row < g.m) ? (uint32_t)((row * g.lda + k) * 4) : kBufOOB;
      dma::copy16(sa + (uint32_t)(t * 1024), off, ars, 0);
    }
    if constexpr (K == Kind::IP) {
#pragma unroll
      for (int c = 0; c < L::kCopiesB / 4; ++c) {
        const int t = wave + 4 * c;
        const int k = k0 + kq, row = j0 + t * 8 + rr;
        const uint32_t off = (k < g.kb && row < g.n) ? (uint32_t)((row * g.ldb + k) * 4) : kBufOOB;
        dma::copy16(sb + (uint32_t)(t * 1024), off, brs, 0);
      }
    } else {
#pragma unroll
      for (int c = 0; c < L::kCopiesB / 4; ++c) {
        const int r = wave * (kBK / 4) + c;  // B row = k offset in the stage
        const int ch = k0 + r;
        const uint32_t off = ch < g.kb ? pix + (uint32_t)(ch * g.hw * 4) : kBufOOB;
        dma::copy4(sb + (uint32_t)(r * kBRow * 4), off, brs, 0);
      }
    }
  };

  v16f acc[TM];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[a][r] = 0.f;

  // All operand reads of a stage go out before its MFMAs (one wait).
  auto compute = [&](int slot) {
    const float* As = lds + slot * L::kSlot;
    const float* Bs = As + L::kA;
    v4f af[2][TM][2], bf[2][2];  // [16-k chunk][block][half]
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      // lane (li, lh) supplies k = 16h + 8*lh + s at step s: logical quads
      // q0 = 4h + 2*lh and q0 + 1 of its row
      const int q0 = 4 * h + 2 * lh;
#pragma unroll
      for (int a = 0; a < TM; ++a) {
        const int r = wm * (BM / 2) + a * 32 + li;
        const float* row = As + r * kBK;
        af[h][a][0] = *reinterpret_cast<const v4f*>(row + 4 * (q0 ^ (r & 7)));
        af[h][a][1] = *reinterpret_cast<const v4f*>(row + 4 * ((q0 + 1) ^ (r & 7)));
      }
      if constexpr (K == Kind::IP) {
        const int r = wn * 32 + li;
        const float* row = Bs + r * kBK;
        bf[h][0] = *reinterpret_cast<const v4f*>(row + 4 * (q0 ^ (r & 7)));
        bf[h][1] = *reinterpret_cast<const v4f*>(row + 4 * ((q0 + 1) ^ (r & 7)));
      } else {
        const float* col = Bs + (16 * h + 8 * lh) * kBRow + wn * 32 + li;
#pragma unroll
        for (int s = 0; s < 8; ++s) bf[h][s >> 2][s & 3] = col[s * kBRow];
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int a = 0; a < TM; ++a)
          acc[a] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[h][a][s >> 2][s & 3], bf[h][s >> 2][s & 3], acc[a], 0, 0,
                                                        0);
  };

  // Stage i is in slot i % kSlots.  At the top of iteration i the wave's
  // copies of stages i .. min(i + kSlots - 2, n - 1) are outstanding: wait
  // for stage i's, then the barrier makes every wave's copies visible and
  // tells that slot (i - 1) % kSlots, multiplied in iteration i - 1, is free
  // for stage i + kSlots - 1.
  for (int st = 0; st < min(kSlots - 1, n_st); ++st) issue(st, st);
  for (int i = 0; i < n_st; ++i) {
    const int ahead = min(kSlots - 2, n_st - 1 - i);
    if (kSlots > 3 && ahead >= 2) dma::wait_vmcnt<(kSlots > 3 ? 2 : 1) * L::kPerWave>();
    else if (ahead >= 1) dma::wait_vmcnt<L::kPerWave>();
    else dma::wait_vmcnt<0>();
    __syncthreads();
    if (i + kSlots - 1 < n_st) issue(i + kSlots - 1, (i + kSlots - 1) % kSlots);
    compute(i % kSlots);
  }

  // Epilogue.  Register r of a 32x32 block: row (r%4) + 8*(r/4) + 4*lh,
  // column li.
  const int j = j0 + wn * 32 + li;
  if (j >= g.n) return;
  int pimg = 0, pp = 0;
  if constexpr (K == Kind::PW) {
    pimg = j / g.hw;
    pp = j - pimg * g.hw;
  }
  auto row_of = [&](int a, int r) { return i0 + wm * (BM / 2) + a * 32 + (r & 3) + 8 * (r >> 2) + 4 * lh; };
  if (g.splits > 1) {
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (row_of(a, r) < g.m) g.d[((int64_t)bz * g.m + row_of(a, r)) * g.n + j] = acc[a][r];
    return;
  }
  // the activation, one wave-uniform branch for all of the lane's values
  auto activate = [&](v16f* v) {
    if (g.act == NHIP_ACT_RELU) {
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int r = 0; r < 16; ++r) v[a][r] = v[a][r] < 0.0f ? 0.0f : v[a][r];
    } else if (g.act == NHIP_ACT_SIGMOID) {
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int r = 0; r < 16; ++r) v[a][r] = act_fn(v[a][r], NHIP_ACT_SIGMOID);
    }
  };
  if constexpr (K == Kind::IP) {
    const float bj = g.bias[j];
#pragma unroll
    for (int a = 0; a < TM; ++a) acc[a] += bj;
    activate(acc);
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (row_of(a, r) < g.m) g.d[(int64_t)row_of(a, r) * g.ldd + j] = acc[a][r];
  } else {
    // every bias (and residual) load of the lane issued before the first use;
    // rows past m read row m - 1 and are not stored
    v16f bv[TM];
    float rv[TM][16];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int r = 0; r < 16; ++r) bv[a][r] = g.bias[min(row_of(a, r), g.m - 1)];
    if (g.residual) {
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          rv[a][r] = g.residual[((int64_t)pimg * g.m + min(row_of(a, r), g.m - 1)) * g.hw + pp];
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int r = 0; r < 16; ++r) bv[a][r] = (acc[a][r] + bv[a][r]) + rv[a][r];
    } else {
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int r = 0; r < 16; ++r) bv[a][r] = acc[a][r] + bv[a][r];
    }
    activate(bv);
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (row_of(a, r) < g.m) g.d[((int64_t)pimg * g.m + row_of(a, r)) * g.hw + pp] = bv[a][r];
  }
}

struct DmaCfg {
  int bm, splits;
};

// Tile rows: 64 (NHIP_GEMM_DMA_BM=128 selects 128 where M >= 128: tuning).
// Split K until the tiles give about per_cu workgroups per CU, keeping at
// least three stages per split (fewer cannot fill the load ring).
DmaCfg dma_config(int m, int n, int stages, int per_cu) {
  const int bm = (setting_int("NHIP_GEMM_DMA_BM", 64) == 128 && m >= 128) ? 128 : 64;
  const int64_t tiles = ceil_div(m, bm) * ceil_div(n, kBN);
  const int64_t target = (int64_t)per_cu * cu_count();
  int splits = 1;
  while (splits < 32 && tiles * splits < target && stages / (2 * splits) >= 3) splits *= 2;
  return DmaCfg{bm, splits};
}

template <Kind K>
int launch_dma(const DmaGemmArgs& g, int bm, hipStream_t s, const char* name) {
  auto go = [&](auto kernel, int bytes, int rows) {
    NHIP_TRY(ensure_dynamic_lds(reinterpret_cast<const void*>(kernel), bytes));
    const dim3 grid((unsigned)ceil_div(g.n, kBN), (unsigned)ceil_div(g.m, rows), (unsigned)g.splits);
    NHIP_LAUNCH(name, kernel, grid, dim3(kThreads), bytes, s, g);
    return check_launch(name);
  };
  if (bm == 128) return go(gemm_dma_kernel<128, K>, Layout<128, K>::kBytes, 128);
  return go(gemm_dma_kernel<64, K>, Layout<64, K>::kBytes, 64);
}

// Split-K reduction of the convolution: part [S][m][npix] -> NCHW.
__global__ void pw_splitk_reduce(const float* __restrict__ part, int splits, int m, int npix, int hw,
                                 const float* __restrict__ bias, const float* __restrict__ residual,
                                 float* __restrict__ out, int act) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)m * npix) return;
  const int i = (int)(idx / npix), j = (int)(idx - (int64_t)i * npix);
  float acc = part[idx];
  for (int s = 1; s < splits; ++s) acc += part[(int64_t)s * m * npix + idx];
  const int img = j / hw, rem = j - img * hw;
  const int64_t o = ((int64_t)img * m + i) * hw + rem;
  float v = acc + bias[i];
  if (residual) v += residual[o];
  out[o] = act_fn(v, act);
}

// Split-K reduction of the InnerProduct: out = act(sum_s part[s] + bias),
// the splits added in order.
__global__ void ipd_splitk_reduce(const float* __restrict__ part, const float* __restrict__ bias,
                                  float* __restrict__ out, int m, int n, int ldd, int splits, int act) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)m * n) return;
  const int i = (int)(idx / n), j = (int)(idx - (int64_t)i * n);
  float s = part[idx];
  for (int z = 1; z < splits; ++z) s += part[(int64_t)z * m * n + idx];
  out[(int64_t)i * ldd + j] = act_fn(s + bias[j], act);
}

}  // namespace

// ------------------------------- InnerProduct -----------------------------
bool ip_dma_supported(const nhip_ip_plan* p, const float* in, int m) {
  if (setting_int("NHIP_GEMM_DMA", 1) == 0) return false;
  // 16-byte aligned input rows and 32-bit buffer offsets
  return p->k_in % 4 == 0 && (reinterpret_cast<uintptr_t>(in) & 15) == 0 &&
         (int64_t)m * p->k_in * 4 < (int64_t(1) << 31) &&
         (int64_t)p->n_pad * p->k_pad * 4 < (int64_t(1) << 31);
}

static DmaCfg ip_dma_cfg(const nhip_ip_plan* p, int m) {
  // one workgroup per CU (256x2048 -> 1000: four splits, 18.0-18.7 us
  // with the reduce against 19.7-21.3 us for eight at two per CU)
  return dma_config(m, p->n_out, (int)ceil_div(p->k_in, kBK), 1);
}

uint64_t innerproduct_dma_workspace(const nhip_ip_plan* p, int m) {
  const DmaCfg c = ip_dma_cfg(p, m);
  return c.splits > 1 ? (uint64_t)c.splits * m * p->n_out * sizeof(float) : 0;
}

int launch_innerproduct_dma(const nhip_ip_plan* p, const float* in, float* out, int m, void* ws, uint64_t ws_bytes,
                            hipStream_t s) {
  const DmaCfg c = ip_dma_cfg(p, m);
  DmaGemmArgs g{};
  g.a = in;
  g.a_bytes = (uint32_t)((int64_t)m * p->k_in * 4);
  g.lda = p->k_in;
  g.ka = p->k_in;
  g.b = p->weight;
  g.b_bytes = (uint32_t)((int64_t)p->n_pad * p->k_pad * 4);
  g.ldb = p->k_pad;
  g.kb = p->k_pad;
  g.m = m;
  g.n = p->n_out;
  g.stages = (int)ceil_div(p->k_in, kBK);
  g.splits = c.splits;
  g.d = out;
  g.ldd = p->n_out;
  g.bias = p->bias;
  g.act = p->act;
  if (c.splits > 1) {
    const uint64_t need = innerproduct_dma_workspace(p, m);
    if (ws == nullptr || ws_bytes < need)
      return fail(NHIP_STATUS_OUTPUT_CAPACITY_INSUFFICIENT,
                  "innerproduct: workspace of " + std::to_string(need) + " bytes required");
    g.d = static_cast<float*>(ws);
  }
  NHIP_TRY(launch_dma<Kind::IP>(g, c.bm, s, "innerproduct_f32_dma"));
  if (c.splits > 1) {
    const int64_t total = (int64_t)m * p->n_out;
    NHIP_LAUNCH("ip_splitk_reduce", ipd_splitk_reduce, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, s,
                static_cast<const float*>(ws), p->bias, out, m, p->n_out, p->n_out, c.splits, p->act);
    return check_launch("ip_splitk_reduce");
  }
  return ok();
}

// ------------------------- 1x1 convolution (NCHW) -------------------------
static DmaCfg pw_dma_cfg(const nhip_conv_plan* p, int64_t npix) {
  // one workgroup per CU as well (MobileNetV2 at batch 32, whose 7x7 1x1
  // layers take this kernel: 0.786 -> 0.775 ms over the graph; four per CU
  // 0.785)
  return dma_config(p->g.k, (int)npix, (int)ceil_div(p->g.c, kBK), 1);
}

// Taken for launches of at most 2.5 workgroups per CU.  Measured on the
// MobileNetV2 7x7 layers at batch 32 against the register-prefetch implicit
// GEMM: 160->960 12.3 us against 16.5 (375 workgroups, no split),
// 576->160 15.2 against 17.6 (300: 4 splits), 960->160 + residual 21.5
// against 23.5 (600: 8 splits); at 1000 workgroups it measured slower
// (960->320 27.1 against 25.2, 320->1280 32.2 against 27.0).
// NHIP_GEMM_DMA=2 takes it for every supported shape (tests).
bool pw_dma_supported(const nhip_conv_plan* p, int n, int h, int w) {
  const ConvGeom& g = p->g;
  if (g.kh != 1 || g.kw != 1 || g.sh != 1 || g.sw != 1 || g.pt || g.pb || g.pl || g.pr) return false;
  const int mode = setting_int("NHIP_GEMM_DMA", 1);
  if (mode == 0) return false;
  const int64_t npix = (int64_t)n * h * w;
  if (npix * g.c * 4 >= (int64_t(1) << 31) || npix * g.k * 4 >= (int64_t(1) << 31) ||
      (int64_t)p->m_pad * p->kred_pad * 4 >= (int64_t(1) << 31))
    return false;
  if (mode == 2) return true;
  const DmaCfg c = pw_dma_cfg(p, npix);
  const int64_t wgs = ceil_div(g.k, c.bm) * ceil_div(npix, kBN) * c.splits;
  return 2 * wgs <= 5LL * cu_count();
}

uint64_t conv_pw_dma_workspace(const nhip_conv_plan* p, int n, int h, int w) {
  const int64_t npix = (int64_t)n * h * w;
  const DmaCfg c = pw_dma_cfg(p, npix);
  return c.splits > 1 ? (uint64_t)c.splits * p->g.k * npix * sizeof(float) : 0;
}

int launch_conv_pw_dma(const nhip_conv_plan* p, const float* in, const float* residual, float* out, int n, int h,
                       int w, void* ws, uint64_t ws_bytes, hipStream_t s) {
  const int64_t npix = (int64_t)n * h * w;
  const DmaCfg c = pw_dma_cfg(p, npix);
  DmaGemmArgs g{};
  g.a = p->weight;
  g.a_bytes = (uint32_t)((int64_t)p->m_pad * p->kred_pad * 4);
  g.lda = p->kred_pad;
  g.ka = p->kred_pad;
  g.b = in;
  g.b_bytes = (uint32_t)(npix * p->g.c * 4);
  g.kb = p->g.c;
  g.hw = h * w;
  g.m = p->g.k;
  g.n = (int)npix;
  g.stages = (int)ceil_div(p->g.c, kBK);
  g.splits = c.splits;
  g.d = out;
  g.bias = p->bias;
  g.residual = residual;
  g.act = p->g.act;
  if (c.splits > 1) {
    const uint64_t need = conv_pw_dma_workspace(p, n, h, w);
    if (ws == nullptr || ws_bytes < need)
      return fail(NHIP_STATUS_OUTPUT_CAPACITY_INSUFFICIENT,
                  "1x1 conv: workspace of " + std::to_string(need) + " bytes required");
    g.d = static_cast<float*>(ws);
  }
  NHIP_TRY(launch_dma<Kind::PW>(g, c.bm, s, "conv_pw_f32_dma"));
  if (c.splits > 1) {
    const int64_t total = (int64_t)p->g.k * npix;
    NHIP_LAUNCH("conv_splitk_reduce", pw_splitk_reduce, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, s,
                static_cast<const float*>(ws), c.splits, p->g.k, (int)npix, h * w, p->bias, residual, out,
                p->g.act);
    return check_launch("conv_splitk_reduce");
  }
  return ok();
}

}  // namespace nhip
