// 3x3 depthwise convolution (stride 1 or 2, padding 1) feeding a 1x1
// convolution with at most 32 output channels, in one kernel: an
// inverted-residual block's depthwise -> project pair (ncnn
// ConvolutionDepthWise, NCNNToTosa.cpp:3376-3503, then Convolution with a
// 1x1 kernel, NCNNToTosa.cpp:1316-1529), with the intermediate tensor kept
// on chip.
//
// A workgroup (4 waves) owns one image's band of R output rows and every
// output channel; the input channels stream through in chunks of 8:
//   * the chunk's input rows (the band's S*(R-1) + 3 rows of 8 channel
//     planes: for each channel one contiguous run of the NCHW input) go into
//     LDS by direct-to-LDS copies (1 KB per wave instruction, no registers),
//     rows outside the image read as zero, up to three later chunks'
//     copies in flight while the current chunk is computed (row slots as
//     many as two workgroups per CU leave room for, at most four);
//   * every thread forms runs of four horizontal depthwise outputs from
//     LDS (centre vectors plus the two halo columns, zero outside the
//     image) in the reference's order: zero, += x*w over (kh, kw), + bias,
//     activation, without fused multiply-adds, the same operations as the
//     standalone depthwise kernel, into a [8][pixels] LDS block;
//   * the waves multiply that block by the chunk's 1x1 weights on
//     v_mfma_f32_16x16x4_f32 (k-step s: channels 4s .. 4s+3 of the chunk,
//     lane l supplying channel 4s + l/16, as in the streaming 1x1 kernel, so
//     each output element accumulates the same products in the same order),
//     wave w taking the 16-pixel blocks w, w+4, ...;
//   * the epilogue adds the bias, the residual and the activation in the
//     1x1 kernel's order and stores 16 consecutive pixels per 16 lanes.
// Two barriers per chunk: the chunk's rows are in LDS; its depthwise block
// is complete (which also frees the rows' slot for the chunk ns - 1 later).
// The weights come from copies made with the plans (depthwise [C][12],
// 1x1 channel-major [C][32]), staged by the same direct-to-LDS copies: a
// per-element transposing load in the prologue cost each workgroup about
// 20 serialized load round trips (7 us per launch).
#include <algorithm>

#include "lds_dma.h"
#include "nhip_internal.h"

namespace nhip {
namespace {

constexpr int kThreads = 256;
constexpr int kCC = 8;        // input channels per chunk: two MFMA k-steps
constexpr int kXcds = 8;      // MI355X: workgroup L runs on XCD L % 8
constexpr int kMaxNi = 8;     // direct-to-LDS copies per thread and chunk
constexpr int kMaxSlots = 4;  // row slots: up to three chunks in flight
constexpr int kMaxItems = 4;  // depthwise work items (4 outputs each) per thread and chunk
constexpr int kMaxLds = 80 * 1024;  // two workgroups per CU

struct DwpwArgs {
  const float* x;      // [N][C][H][W]
  const float* dw12;   // [C][12]: taps, bias, zeros
  const float* ck;     // [C][32]: 1x1 weights channel-major, zero past K
  const float* pw_b;   // [m_pad]
  const float* res;    // [N][K][OH][OW] or null
  float* out;          // [N][K][OH][OW]
  int C, K, H, W, OH, OW;
  int dwv, ckv;          // 16-byte vectors of the two weight regions in LDS (multiples of 256)
  int R, nbands, total;  // output rows per workgroup, bands per image, workgroups
  int nr;                // input rows per band: S*(R-1) + 3
  int nbk;               // 16-pixel blocks per band: ceil(R*OW / 16)
  int chunk_f4;          // 16-byte vectors of one chunk's rows: kCC*nr*W/4
  int ni;                // copies per thread and chunk: ceil(chunk_f4 / 256)
  int pp;                // pitch of the depthwise block (floats), 16 mod 32
  int ns;                // row slots (2 .. kMaxSlots): ns - 1 chunks in flight
  int dw_relu, pw_act;
  uint32_t x_bytes, out_bytes;
};

__device__ __forceinline__ float pw_activate(float v, int act) {
  if (act == NHIP_ACT_RELU) return v < 0.f ? 0.f : v;
  if (act == NHIP_ACT_SIGMOID) return 1.0f / (1.0f + __expf(-v));
  return v;
}

// Wait until at most n (0 <= n < 32, wave-uniform) of this wave's vector
// memory loads are outstanding.
template <int N>
__device__ __forceinline__ void wait_upto(int n) {
  if constexpr (N < 32) {
    if (n == N) dma::wait_vmcnt<N>();
    else wait_upto<N + 1>(n);
  }
}

// S: depthwise stride; MB: 16-channel blocks of the 1x1 output (K <= 16 *
// MB); NBW: 16-pixel blocks per wave at most.
template <int S, int MB, int NBW>
__global__ __launch_bounds__(kThreads, 2) void dwpw_lds_kernel(DwpwArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  float* dww = lds;                          // [C][12]: 9 taps, bias
  float* pwl = dww + a.dwv * 4;              // [C][32]: 1x1 weights, zero past K
  const int rawf = a.ni * kThreads * 4;      // floats per row slot
  float* raw = pwl + a.ckv * 4;              // ns slots of [kCC][nr][W]
  float* dwb = raw + a.ns * rawf;            // [kCC][pp]
  const uint32_t lds0 = (uint32_t)(uintptr_t)lds;
  const uint32_t raw_lds = lds0 + (uint32_t)((a.dwv + a.ckv) * 16);

  // XCD-contiguous numbering: consecutive bands of an image (which share
  // their halo rows) run on one XCD.
  const int L = blockIdx.x;
  const int xcd = L % kXcds, q8 = L / kXcds;
  const int logical = xcd * (a.total / kXcds) + min(xcd, a.total % kXcds) + q8;
  const int img = logical / a.nbands, band = logical - img * a.nbands;
  const int oy0 = band * a.R;
  const int reff = min(a.R, a.OH - oy0);
  const int iy0 = S * oy0 - 1;

  // Per-thread copy offsets of chunk 0 (the chunk index moves only the
  // scalar offset): vector f = i*256 + tid of the chunk is channel f / rowf,
  // row, 4-float column; rows outside the image and vectors past the chunk
  // read as zero.
  const v4i xr = dma::raw_rsrc(a.x, a.x_bytes);
  const int w4 = a.W >> 2, rowf = a.nr * w4;
  uint32_t voff[kMaxNi];
#pragma unroll
  for (int i = 0; i < kMaxNi; ++i) {
    const int f = i * kThreads + tid;
    const int ch = f / rowf, rem = f - ch * rowf;
    const int row = rem / w4, c4 = rem - row * w4;
    const int iy = iy0 + row;
    const bool ok = i < a.ni && f < a.chunk_f4 && (unsigned)iy < (unsigned)a.H;
    voff[i] = ok ? (uint32_t)((((img * a.C + ch) * a.H + iy) * a.W + 4 * c4) * 4) : kBufOOB;
  }
  const uint32_t chunk_bytes = (uint32_t)(kCC * a.H * a.W * 4);
  auto issue = [&](int c, int slot) {
    const uint32_t base = raw_lds + (uint32_t)(slot * rawf * 4) + (uint32_t)(wave * 64 * 16);
#pragma unroll
    for (int i = 0; i < kMaxNi; ++i)
      if (i < a.ni) dma::copy16(base + (uint32_t)(i * kThreads * 16), voff[i], xr, (uint32_t)c * chunk_bytes);
  };
  const int nch = a.C / kCC;
  // The weights first (the same direct-to-LDS copies; the regions are
  // whole multiples of 256 vectors, the source's tail reads as zero), then
  // the first ns - 1 chunks: the waits below count them all in issue order.
  {
    const v4i dr = dma::raw_rsrc(a.dw12, (uint32_t)(a.C * 48));
    const v4i cr = dma::raw_rsrc(a.ck, (uint32_t)(a.C * 128));
    const uint32_t wl = lds0 + (uint32_t)(wave * 64 * 16);
    for (int v = 0; v < a.dwv; v += kThreads)
      dma::copy16(wl + (uint32_t)(v * 16), (uint32_t)((v + tid) * 16), dr, 0);
    for (int v = 0; v < a.ckv; v += kThreads)
      dma::copy16(wl + (uint32_t)((a.dwv + v) * 16), (uint32_t)((v + tid) * 16), cr, 0);
  }
  for (int c = 0; c < a.ns - 1 && c < nch; ++c) issue(c, c);

  v4f acc[MB][NBW];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < NBW; ++j) acc[mb][j] = v4f{0.f, 0.f, 0.f, 0.f};

  // This thread's depthwise work items, the same in every chunk: item
  // tid + 256j = (channel, band row, output quad), quads fastest; kept as
  // LDS offsets (row slab, depthwise block), the channel and the halo flags.
  const int qw = a.OW >> 2;              // output quads per row
  const int items = kCC * a.R * qw;      // (channel, row, quad) of a chunk
  int it_raw[kMaxItems], it_dwb[kMaxItems], it_ch[kMaxItems];
  bool it_on[kMaxItems], it_l[kMaxItems], it_r[kMaxItems];
#pragma unroll
  for (int j = 0; j < kMaxItems; ++j) {
    const int it = tid + kThreads * j;
    const int q = it % qw, t = it / qw;
    const int r = t % a.R, ch = t / a.R;
    it_on[j] = it < items && r < reff;
    it_raw[j] = (ch * a.nr + S * r) * a.W + 4 * S * q;
    it_dwb[j] = ch * a.pp + r * a.OW + 4 * q;
    it_ch[j] = ch;
    it_l[j] = q > 0;
    it_r[j] = 4 * q + 4 < a.W;
  }
  for (int c = 0, slot = 0; c < nch; ++c, slot = slot + 1 == a.ns ? 0 : slot + 1) {
    // chunk c + ns - 1 into the slot chunk c - 1 used (free since the last
    // barrier), then wait for chunk c: the copies of the later chunks stay
    // in flight (loads retire in issue order)
    const int ahead = c + a.ns - 1;
    if (ahead < nch) issue(ahead, slot == 0 ? a.ns - 1 : slot - 1);
    wait_upto<0>((min(ahead, nch - 1) - c) * a.ni);
    __syncthreads();
    const float* rs = raw + slot * rawf;
    {
#pragma clang fp contract(off)
#pragma unroll
      for (int jt = 0; jt < kMaxItems; ++jt) {
        if (!it_on[jt]) continue;
        const float* wq = dww + (c * kCC + it_ch[jt]) * 12;
        float w[12];
#pragma unroll
        for (int u = 0; u < 3; ++u) {
          const v4f wv = *reinterpret_cast<const v4f*>(wq + 4 * u);
          w[4 * u] = wv[0];
          w[4 * u + 1] = wv[1];
          w[4 * u + 2] = wv[2];
          w[4 * u + 3] = wv[3];
        }
        // window rows S*r .. S*r + 2, columns S*4q - 1 .. S*4q + 4S
        float in[3][4 * S + 2];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
          const float* row = rs + it_raw[jt] + i * a.W;
          in[i][0] = it_l[jt] ? row[-1] : 0.f;
#pragma unroll
          for (int v = 0; v < S; ++v) {
            const v4f m = *reinterpret_cast<const v4f*>(row + 4 * v);
            in[i][1 + 4 * v] = m[0];
            in[i][2 + 4 * v] = m[1];
            in[i][3 + 4 * v] = m[2];
            in[i][4 + 4 * v] = m[3];
          }
          if constexpr (S == 1) in[i][5] = it_r[jt] ? row[4] : 0.f;
        }
        v4f o;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          float s = 0.f;
#pragma unroll
          for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = 0; j < 3; ++j) s = s + in[i][u * S + j] * w[i * 3 + j];
          s = s + w[9];
          if (a.dw_relu) s = s < 0.f ? 0.f : s;
          o[u] = s;
        }
        *reinterpret_cast<v4f*>(dwb + it_dwb[jt]) = o;
      }
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < kCC / 4; ++s) {
      const int cl = 4 * s + (lane >> 4);
      float av[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) av[mb] = pwl[(c * kCC + cl) * 32 + mb * 16 + (lane & 15)];
#pragma unroll
      for (int j = 0; j < NBW; ++j) {
        const int nb = wave + 4 * j;
        if (nb >= a.nbk) break;
        const float bv = dwb[cl * a.pp + nb * 16 + (lane & 15)];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[mb][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[mb], bv, acc[mb][j], 0, 0, 0);
      }
    }
  }

  // Epilogue: lane l holds output channels 16mb + 4(l/16) + i (register i)
  // of pixel 16nb + l%16 of the band; a band's pixels are consecutive in
  // the output plane.
  const __amdgpu_buffer_rsrc_t orr = make_rsrc(a.out, a.out_bytes);
  const __amdgpu_buffer_rsrc_t rr = make_rsrc(a.res, a.res ? a.out_bytes : 0u);
  const int npx = reff * a.OW;
  float bias[MB][4];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = mb * 16 + 4 * (lane >> 4) + i;
      bias[mb][i] = k < a.K ? a.pw_b[k] : 0.f;
    }
  float rv[MB][NBW][4];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < NBW; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k = mb * 16 + 4 * (lane >> 4) + i, px = (wave + 4 * j) * 16 + (lane & 15);
        const bool ok = a.res && wave + 4 * j < a.nbk && k < a.K && px < npx;
        const uint32_t off = (uint32_t)((((img * a.K + k) * a.OH + oy0) * a.OW + px) * 4);
        rv[mb][j][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rr, ok ? off : kBufOOB, 0, 0));
      }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      if (wave + 4 * j >= a.nbk) break;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k = mb * 16 + 4 * (lane >> 4) + i, px = (wave + 4 * j) * 16 + (lane & 15);
        float o = acc[mb][j][i] + bias[mb][i];
        if (a.res) o += rv[mb][j][i];
        o = pw_activate(o, a.pw_act);
        const bool ok = k < a.K && px < npx;
        const uint32_t off = (uint32_t)((((img * a.K + k) * a.OH + oy0) * a.OW + px) * 4);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(o), orr, ok ? off : kBufOOB, 0, 0);
      }
    }
}

struct DwpwCfg {
  int R, nr, nbk, nbw, chunk_f4, ni, pp, ns;
  size_t lds;
};

// Largest band height R in {4, 2, 1} whose workgroups still cover the GPU
// one and a half times over (two fit per CU), within the LDS and register
// bounds; with too few pixels for that, the smallest R that fits.  Row
// slots: as many as the LDS share of two workgroups per CU holds, up to
// kMaxSlots (NHIP_DWPW_SLOTS caps them, for tests).
bool dwpw_lds_cfg(int C, int W, int OH, int OW, int S, int n, DwpwCfg* out) {
  bool found = false;
  const int ns_cap = std::max(2, std::min(kMaxSlots, setting_int("NHIP_DWPW_SLOTS", kMaxSlots)));
  for (int R : {4, 2, 1}) {
    DwpwCfg c;
    c.R = R;
    c.nr = S * (R - 1) + 3;
    c.nbk = (int)ceil_div((int64_t)R * OW, 16);
    c.nbw = (int)ceil_div(c.nbk, 4);
    c.chunk_f4 = kCC * c.nr * (W / 4);
    c.ni = (int)ceil_div(c.chunk_f4, kThreads);
    c.pp = (int)round_up(c.nbk * 16, 32) + 16;
    const size_t fixed = (size_t)((round_up(3 * C, kThreads) + round_up(8 * C, kThreads)) * 4 + kCC * c.pp) * sizeof(float);
    const size_t slot = (size_t)c.ni * kThreads * 16;
    if (c.nbw > 8 || c.ni > kMaxNi || fixed + 2 * slot > (size_t)kMaxLds ||
        kCC * R * (OW / 4) > kMaxItems * kThreads)
      continue;
    c.ns = (int)std::min<size_t>(ns_cap, (kMaxLds - fixed) / slot);
    if ((c.ns - 1) * c.ni >= 32) c.ns = 32 / c.ni;
    c.lds = fixed + c.ns * slot;
    *out = c;
    found = true;
    if ((int64_t)n * ceil_div(OH, R) * 2 >= 3LL * cu_count()) return true;
  }
  return found;
}

template <int S, int MB, int NBW>
int launch_one(const DwpwArgs& a, size_t lds, hipStream_t s) {
  const auto kernel = dwpw_lds_kernel<S, MB, NBW>;
  NHIP_TRY(ensure_dynamic_lds(reinterpret_cast<const void*>(kernel), (int)lds));
  NHIP_LAUNCH("dwpw_lds_f32", kernel, dim3((unsigned)a.total), dim3(kThreads), lds, s, a);
  return check_launch("dwpw_lds_f32");
}

template <int S, int MB>
int launch_nbw(const DwpwArgs& a, int nbw, size_t lds, hipStream_t s) {
  if (nbw <= 2) return launch_one<S, MB, 2>(a, lds, s);
  if (nbw <= 4) return launch_one<S, MB, 4>(a, lds, s);
  return launch_one<S, MB, 8>(a, lds, s);
}

}  // namespace

// The pair's shape rules for this kernel beyond the fused pair's own
// (3x3, stride 1 or 2 on both axes, padding 1, float4-aligned rows):
// channels a multiple of 8, at most 32 output channels, a depthwise
// activation of none or ReLU, 32-bit buffer offsets.  Taken at stride 2
// only, where it measured faster than the streaming kernel's depthwise mode
// (MobileNetV2 at batch 32, in the graph: 96@112 -> 24 44.6 against 46.9
// us, 144@56 -> 32 23.2 against 26.2 us); at stride 1 it measured slower
// (32@112 -> 16 41.6 against 26.8 us, 144@56 -> 24 + residual 42.2 against
// 39.7 us: the depthwise arithmetic of four waves per workgroup, two
// workgroups per CU, and the per-chunk barriers leave the SIMDs idle about
// half the time).  NHIP_DWPW_LDS=0: never; 2: at stride 1 too (tests).
bool dwpw_lds_supported(const nhip_conv_plan* dw, const nhip_conv_plan* pw, int n, int h, int w, int oh,
                        int ow) {
  const int mode = setting_int("NHIP_DWPW_LDS", 1);
  if (mode == 0 || (mode == 1 && dw->g.sh != 2)) return false;
  const int C = dw->g.c, S = dw->g.sh;
  if (C % kCC != 0 || pw->g.k > 32 || pw->g.k < 1 || (S != 1 && S != 2) || w % 4 != 0 || ow % 4 != 0)
    return false;
  if (dw->g.act != NHIP_ACT_NONE && dw->g.act != NHIP_ACT_RELU) return false;
  if ((int64_t)n * C * h * w * 4 >= (int64_t(1) << 31) || (int64_t)n * pw->g.k * oh * ow * 4 >= (int64_t(1) << 31))
    return false;
  if (dw->weight_dw12 == nullptr || pw->weight_ck == nullptr) return false;
  DwpwCfg c;
  return dwpw_lds_cfg(C, w, oh, ow, S, n, &c);
}

int launch_dwpw_lds_f32(const nhip_conv_plan* dw, const nhip_conv_plan* pw, const float* in,
                        const float* residual, float* out, int n, int h, int w, int oh, int ow, hipStream_t s) {
  DwpwCfg c;
  const int S = dw->g.sh;
  if (!dwpw_lds_cfg(dw->g.c, w, oh, ow, S, n, &c))
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "depthwise + 1x1 (LDS): unsupported shape");
  if ((reinterpret_cast<uintptr_t>(in) & 15) != 0)
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "depthwise + 1x1 (LDS): input must be 16-byte aligned");
  DwpwArgs a{};
  a.x = in;
  a.dw12 = dw->weight_dw12;
  a.ck = pw->weight_ck;
  a.pw_b = pw->bias;
  a.res = residual;
  a.out = out;
  a.C = dw->g.c;
  a.K = pw->g.k;
  a.H = h;
  a.W = w;
  a.OH = oh;
  a.OW = ow;
  a.dwv = (int)round_up(3 * a.C, kThreads);
  a.ckv = (int)round_up(8 * a.C, kThreads);
  a.R = c.R;
  a.nbands = (int)ceil_div(oh, c.R);
  a.total = n * a.nbands;
  a.nr = c.nr;
  a.nbk = c.nbk;
  a.chunk_f4 = c.chunk_f4;
  a.ni = c.ni;
  a.pp = c.pp;
  a.ns = c.ns;
  a.dw_relu = dw->g.act == NHIP_ACT_RELU;
  a.pw_act = pw->g.act;
  a.x_bytes = (uint32_t)((int64_t)n * a.C * h * w * 4);
  a.out_bytes = (uint32_t)((int64_t)n * a.K * oh * ow * 4);
  const bool mb2 = a.K > 16;
  if (S == 1) return mb2 ? launch_nbw<1, 2>(a, c.nbw, c.lds, s) : launch_nbw<1, 1>(a, c.nbw, c.lds, s);
  return mb2 ? launch_nbw<2, 2>(a, c.nbw, c.lds, s) : launch_nbw<2, 1>(a, c.nbw, c.lds, s);
}

}  // namespace nhip
