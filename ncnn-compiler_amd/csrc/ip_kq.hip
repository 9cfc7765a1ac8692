// InnerProduct (ncnn InnerProduct, NCNNToTosa.cpp:5254-5392: zero-initialised
// matmul, then bias, then the activation) as one workgroup per 32 x 32 block
// of the output, the reduction split over the workgroup's 16 waves.
//
//   out[m][n] = act(sum_k x[m][k] W[n][k] + b[n])
//
// A block's whole reduction runs inside its workgroup: wave w takes the
// reduction slice [w*kw, (w+1)*kw) (kw = k_kq / 16) in groups of 32, and
// keeps the 32 x 32 block in the 16 accumulator registers of
// v_mfma_f32_32x32x2_f32.
//   - The weights come from a prepacked copy in 4-k groups,
//     [n_pad/32][k_kq/4][32][4], straight into registers: a half-wave's
//     16-byte loads cover 512 contiguous bytes.
//   - The input rows come through a wave-private LDS double buffer: a
//     group's 32 rows x 128 bytes arrive in four direct-to-LDS loads of 8
//     whole rows (whole cache lines, instead of 32 B of 32 rows per load,
//     which re-fetched each line four times), slot s of row r holding the
//     16-byte segment s ^ (r & 7), so the MFMA-order reads (one segment of
//     32 rows) hit distinct banks.
// The 16 partial blocks are summed through LDS in wave order (the result
// does not depend on timing), bias and activation applied, and the block
// written row by row.  No split-K partials in memory and no reduce launch;
// one block per CU keeps 4 waves on every SIMD.
#include "nhip_internal.h"

namespace nhip {
namespace {

constexpr int kWaves = 16;
constexpr int kThreads = kWaves * 64;
constexpr int kGroupK = 32;                        // reduction indices per LDS group
constexpr int kStageBytes = kWaves * 2 * 4096;     // two 4 KB groups per wave
constexpr int kPad = 33;                           // LDS row pitch of a partial block
constexpr int kPartBytes = kWaves * 32 * kPad * 4;  // 16 partial 32 x 32 blocks
constexpr int kLdsBytes = kStageBytes > kPartBytes ? kStageBytes : kPartBytes;

struct IpKqArgs {
  const float* x;       // [m][k_in] row-major, k_in % 4 == 0
  const float* w;       // [n_pad/32][k_kq/4][32][4]
  const float* bias;    // [n_pad]
  float* out;           // [m][n_out]
  int m, n_out, k_in, k_kq;
  uint32_t x_bytes, w_bytes;
  int act;
};

// Wait until at most N of this wave's vector memory loads are outstanding,
// then keep later memory accesses (the LDS reads of the group) below it.
template <int N>
__device__ __forceinline__ void wait_loads() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit count");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");
}

// NG groups of 32 reduction indices per wave.
template <int NG>
__global__ __launch_bounds__(kThreads, 1) void ip_kq_kernel(IpKqArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nb = blockIdx.x, mb = blockIdx.y;
  const int n0 = nb * 32, m0 = mb * 32;
  const int k0 = wave * NG * kGroupK;
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, a.w_bytes), xr = make_rsrc(a.x, a.x_bytes);
  // MFMA operands: lane l supplies row l % 32 and reduction index
  // 4 (l / 32) + st of a chunk of 8 at step st
  const int row = lane & 31, hk = lane >> 5;
  const uint32_t w_lane = (uint32_t)((((size_t)nb * (a.k_kq / 4) + (k0 / 4) + hk) * 32 + row) * 16);
  float* xs = lds + wave * 2 * 1024;  // this wave's two 4 KB groups
  // input loads: lane l fills slot l % 8 of row 8q + l / 8
  const int lrow = lane >> 3, lslot = lane & 7;
  uint32_t x_row[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int m = m0 + 8 * q + lrow;
    x_row[q] = m < a.m ? (uint32_t)((size_t)m * a.k_in * 4) : kBufOOB;
  }
  auto load_x = [&](int g) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int k = k0 + kGroupK * g + 4 * (lslot ^ lrow);  // row & 7 == lrow
      const uint32_t off = (x_row[q] != kBufOOB && k < a.k_in) ? x_row[q] + (uint32_t)k * 4 : kBufOOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xr, (__attribute__((address_space(3))) void*)(xs + (g & 1) * 1024 + q * 256), 16, off, 0, 0, 0);
    }
  };
  v4f wv[NG * 4];
  auto load_w = [&](int g) {
#pragma unroll
    for (int c = 4 * g; c < 4 * g + 4; ++c)
      wv[c] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(wr, w_lane + (uint32_t)c * 1024, 0, 0));
  };
  // Issue group g: its input loads strictly before its weight loads (the
  // waits below count on that order), and only once this wave's LDS reads
  // of the group that used the buffer before have completed.
  auto issue = [&](int g) {
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));  // lgkmcnt(0)
    asm volatile("" ::: "memory");
    load_x(g);
    asm volatile("" ::: "memory");
    load_w(g);
    asm volatile("" ::: "memory");
  };
  v16f acc = v16f{};
  issue(0);
  if (NG > 1) issue(1);
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    // group g's input is in LDS once only its 4 weight loads and, when
    // issued, group g + 1's 8 loads may still be outstanding
    if (g + 1 < NG) wait_loads<12>(); else wait_loads<4>();
    v4f xv[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) xv[c] = *(const v4f*)(xs + (g & 1) * 1024 + row * 32 + (((2 * c + hk) ^ (row & 7)) * 4));
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int st = 0; st < 4; ++st) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(wv[4 * g + c][st], xv[c][st], acc, 0, 0, 0);
    if (g + 2 < NG) issue(g + 2);
  }
  __syncthreads();  // every wave's staging reads are done: the LDS now takes the partial blocks
  // partial block of this wave: register r of lane l is output n = (r % 4) +
  // 8 (r / 4) + 4 (l / 32), m = l % 32
  float* pw = lds + wave * 32 * kPad;
#pragma unroll
  for (int r = 0; r < 16; ++r) pw[((r & 3) + 8 * (r >> 2) + 4 * hk) * kPad + row] = acc[r];
  __syncthreads();
  // thread t: m = t / 32, n = t % 32 (consecutive threads, consecutive outputs)
  const int mo = m0 + (tid >> 5), no = n0 + (tid & 31);
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) s += lds[w * 32 * kPad + (tid & 31) * kPad + (tid >> 5)];
  if (mo < a.m && no < a.n_out) {
    float v = s + a.bias[no];
    if (a.act == NHIP_ACT_RELU) v = v < 0.f ? 0.f : v;
    a.out[(size_t)mo * a.n_out + no] = v;
  }
}

template <int NG>
int launch_ng(const IpKqArgs& a, hipStream_t s) {
  NHIP_TRY(ensure_dynamic_lds(reinterpret_cast<const void*>(&ip_kq_kernel<NG>), kLdsBytes));
  NHIP_LAUNCH("innerproduct_f32_kq", ip_kq_kernel<NG>, dim3((unsigned)ceil_div(a.n_out, 32), (unsigned)ceil_div(a.m, 32)),
              dim3(kThreads), kLdsBytes, s, a);
  return check_launch("innerproduct_f32_kq");
}

}  // namespace

int ip_kq_k_pad(int k_in) { return (int)round_up(k_in, kWaves * kGroupK); }

// The prepacked weights of the kernel above: [n_pad/32][k_kq/4][32][4].
int ip_kq_prepack(nhip_ip_plan* p, const float* weight) {
  const int k_kq = ip_kq_k_pad(p->k_in);
  if (k_kq > 4 * kWaves * kGroupK) return ok();  // reductions above 2048: the tiled GEMM only
  std::vector<float> wp((size_t)p->n_pad * k_kq, 0.f);
  for (int n = 0; n < p->n_out; ++n)
    for (int k = 0; k < p->k_in; ++k)
      wp[(((size_t)(n / 32) * (k_kq / 4) + k / 4) * 32 + n % 32) * 4 + k % 4] = weight[(size_t)n * p->k_in + k];
  NHIP_TRY(check_hip(hipMalloc(&p->weight_kq, wp.size() * sizeof(float)), "hipMalloc(ip weight, 4-k groups)"));
  return check_hip(hipMemcpy(p->weight_kq, wp.data(), wp.size() * sizeof(float), hipMemcpyHostToDevice),
                   "hipMemcpy(ip weight, 4-k groups)");
}

// Whether the kernel takes m rows: weights prepacked, 16-byte aligned rows
// (k_in % 4 == 0), and at least 3/4 of the CUs with a block each (below
// that the tiled GEMM's K split fills the GPU better).  NHIP_IP_KQ=0 / 1
// switches it off / on whatever the block count (tests).
bool ip_kq_supported(const nhip_ip_plan* p, const float* in, int m) {
  if (p->weight_kq == nullptr || p->k_in % 4 != 0 || (reinterpret_cast<uintptr_t>(in) & 15)) return false;
  if ((int64_t)m * p->k_in * 4 >= (int64_t(1) << 31) || ceil_div(m, 32) > 65535) return false;
  const int forced = setting_int("NHIP_IP_KQ", -1);
  if (forced >= 0) return forced != 0;
  return 4 * ceil_div(p->n_out, 32) * ceil_div(m, 32) >= 3 * (int64_t)cu_count();
}

int launch_ip_kq(const nhip_ip_plan* p, const float* in, float* out, int m, hipStream_t s) {
  IpKqArgs a{};
  a.x = in;
  a.w = p->weight_kq;
  a.bias = p->bias;
  a.out = out;
  a.m = m;
  a.n_out = p->n_out;
  a.k_in = p->k_in;
  a.k_kq = ip_kq_k_pad(p->k_in);
  a.x_bytes = (uint32_t)((size_t)m * p->k_in * 4);
  a.w_bytes = (uint32_t)((size_t)p->n_pad * a.k_kq * 4);
  a.act = p->act;
  switch (a.k_kq / (kWaves * kGroupK)) {
    case 1: return launch_ng<1>(a, s);
    case 2: return launch_ng<2>(a, s);
    case 3: return launch_ng<3>(a, s);
    case 4: return launch_ng<4>(a, s);
    default: return fail(NHIP_STATUS_UNSUPPORTED, "innerproduct: reduction length outside the kernel's range");
  }
}

}  // namespace nhip
