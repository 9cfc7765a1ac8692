// Internal declarations shared by the runtime's translation units.
// Device code targets gfx950 (CDNA4) only: wave64, fp32/int8 MFMA.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/nhip.h"

namespace nhip {

// ---- status / error plumbing ---------------------------------------------
int fail(int status, const std::string& message);
int ok();
int check_hip(hipError_t e, const char* what);
int check_launch(const char* kernel);

#define NHIP_TRY(expr)          \
  do {                          \
    int _st = (expr);           \
    if (_st != NHIP_STATUS_SUCCESS) return _st; \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Kernel timing for nhip_timer_*: when the timer is on and `kernel` matches
// its filter, holds a start/stop event pair that hipExtLaunchKernelGGL
// stamps from the kernel's own dispatch on its stream (no separate marker
// packets around the launch).
class LaunchTimer {
 public:
  explicit LaunchTimer(const char* kernel);
  bool active() const { return start_ != nullptr; }
  hipEvent_t start() const { return start_; }
  hipEvent_t stop() const { return stop_; }
  LaunchTimer(const LaunchTimer&) = delete;
  LaunchTimer& operator=(const LaunchTimer&) = delete;

 private:
  hipEvent_t start_ = nullptr;
  hipEvent_t stop_ = nullptr;
};

// NHIP_LAUNCH(name, kernel, grid, block, shmem, stream, args...): launch,
// timed under `name` while nhip_timer_start is in effect.
#define NHIP_LAUNCH(name, kernel, grid, block, shmem, strm, ...)                                      \
  do {                                                                                              \
    ::nhip::LaunchTimer _nhip_timer(name);                                                          \
    if (_nhip_timer.active())                                                                       \
      hipExtLaunchKernelGGL(kernel, grid, block, shmem, strm, _nhip_timer.start(), _nhip_timer.stop(), \
                            0, __VA_ARGS__);                                                        \
    else                                                                                            \
      hipLaunchKernelGGL(kernel, grid, block, shmem, strm, __VA_ARGS__);                            \
  } while (0)

int cu_count();  // compute units of the current device (cached)

// NHIP_* tuning / test switches from the settings snapshot (environment at
// first use or at the last nhip_reload_settings); nullptr when unset.
const char* setting(const char* name);
int setting_int(const char* name, int fallback);
uint64_t settings_generation();
// Dynamic LDS above 64 KB needs a per-kernel attribute, set once per device.
int ensure_dynamic_lds(const void* kernel, int bytes);
// Workgroups of `kernel` resident per CU at this block size and dynamic
// LDS (cached per device).
int resident_blocks(const void* kernel, int threads, size_t lds);

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

// ---- division by a divisor fixed at launch ------------------------------------
// n / d for 0 <= n < 2^31 and 1 <= d < 2^31 as (umulhi(n, m) + n) >> s, with
// s = ceil(log2 d) and m = floor(2^32 (2^s - d) / d) + 1 (Granlund and
// Montgomery, "Division by invariant integers using multiplication", PLDI
// 1994, section 4); n < 2^31 keeps the sum inside 32 bits.
struct FastDiv {
  uint32_t m, s;
};
inline FastDiv fast_div(uint32_t d) {
  uint32_t s = 0;
  while ((uint64_t(1) << s) < d) ++s;
  return FastDiv{(uint32_t)((((uint64_t(1) << s) - d) << 32) / d + 1), s};
}
__device__ __forceinline__ int fdiv(int n, FastDiv f) {
  return (int)((__umulhi((uint32_t)n, f.m) + (uint32_t)n) >> f.s);
}

// ---- int8 quantization (reference quantizeSignedI8, NCNNToTosa.cpp:322-389) --
// Round half away from zero of s = x * scale, saturated to [lo, 127] (lo =
// -127, or 0 for a ReLU that follows), NaN -> 0.  s + copysign(0.5, s) forms
// the same fp32 sum as floor(s + 0.5) for s >= 0 and ceil(s - 0.5) for s < 0,
// and truncating it toward zero equals that floor / ceil since the sum has
// the sign of s (s = -0.0 gives 0 both ways).  v_cvt_i32_f32 truncates toward
// zero, saturates out-of-range values and infinities to the int32 limits and
// converts NaN to 0 (GCN/CDNA ISA), so it is issued directly (a C++ cast of
// such values is undefined) and one integer median-of-three saturates.
// max(clamp(q, -127, 127), 0) = clamp(q, 0, 127), so a ReLU is the bound.
// The caller's multiply stays separately rounded: no contraction here.
__device__ __forceinline__ int quantize_q(float x, float scale, int lo = -127) {
#pragma clang fp contract(off)
  const float s = x * scale;
  const float t = s + __builtin_copysignf(0.5f, s);
  int q;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(q) : "v"(t));
  return max(min(q, 127), lo);
}
__device__ __forceinline__ int8_t quantize_i8(float x, float scale, int lo = -127) {
  return (int8_t)quantize_q(x, scale, lo);
}
// Four quantized values (low bytes of a, b, c, d) as one little-endian word.
__device__ __forceinline__ uint32_t pack_i8x4(int a, int b, int c, int d) {
  const uint32_t lo = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x0c0c0400u);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// ---- MFMA operand / accumulator types ---------------------------------------
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// ---- raw buffer loads ---------------------------------------------------------
// A raw buffer load whose byte offset is at or past the resource's size
// returns 0 without touching memory.  Gathers with zero padding therefore pass
// kBufOOB for out-of-image positions instead of branching around the load:
// no per-load branch, so the compiler can issue all loads before waiting.
// Resources here never exceed 2^31 bytes (checked on the host).
constexpr uint32_t kBufOOB = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  // word 3 = 0x00020000: the gfx9-family (incl. gfx950) raw-buffer format
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float buf_load_f32(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 0));
}
__device__ __forceinline__ int4 buf_load_b128(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}

// ---- plans ----------------------------------------------------------------
enum class PlanKind { ConvF32, ConvInt8, DwConvF32, DwConvInt8 };

struct ConvGeom {
  int32_t c, k;             // input channels, num_output
  int32_t kh, kw, sh, sw, dh, dw;
  int32_t pt, pb, pl, pr;
  int32_t act;              // NHIP_ACT_*
};

}  // namespace nhip

// Opaque handle of nhip.h.  Device buffers are owned by the plan.
struct nhip_conv_plan {
  nhip::PlanKind kind;
  nhip::ConvGeom g;
  int32_t algorithm;        // resolved NHIP_CONV_ALGO_* (never AUTO)
  int32_t has_bias;
  // implicit GEMM fp32: weights [m_pad][kred_pad], k = (c, kh, kw) order;
  // Winograd: weights U[36][m_pad][c_pad].
  float* weight = nullptr;
  // Winograd, fused kernel: the same U in 4-channel groups,
  // [36][c_pad/4][m_pad][4], so 32 output channels of one group are 512
  // contiguous bytes per transform point.
  float* weight_fused = nullptr;
  // Plans the one-kernel path of small launches can take (conv_kq.hip: 3x3
  // with 32 or 64 input channels, on either algorithm, and 1x1 with its
  // channel counts): the weights in groups of kq_vw reduction indices,
  // [m_pad/32][C*KH*KW/kq_vw][32][kq_vw] with k = c*KH*KW + kh*KW + kw, so
  // the 32 output channels of one group are contiguous.
  float* weight_kq = nullptr;
  int32_t kq_vw = 0;
  // Winograd plans of 256+ input channels: an implicit-GEMM plan of the same
  // layer, for launches of so few tiles that the Winograd GEMM's 128-tile
  // padding dominates (a single 7x7 or 14x14 image).
  nhip_conv_plan* igemm_twin = nullptr;
  // 1x1 plans with at most 32 output channels: the weights channel-major,
  // [C][32] (zero past K), the LDS layout of the depthwise -> 1x1 kernel.
  float* weight_ck = nullptr;
  // 3x3 depthwise plans: [C][12], the nine taps, the bias, two zeros.
  float* weight_dw12 = nullptr;
  float* bias = nullptr;      // [m_pad] zero-filled past k (always present)
  int32_t m_pad = 0, kred = 0, kred_pad = 0, c_pad = 0;
  // im2col gather table: one packed int per reduction index
  // (c << 16 | dy << 8 | dx), dy/dx = kh*dil_h, kw*dil_w; sentinel past kred.
  int32_t* ktab = nullptr;
  // int8: weights int8 [m_pad][kh*kw*c_pad] (k = (kh, kw, c) order),
  // reciprocal r[c] = ws==0 ? 0 : 1/(ws*is), bias, scales.
  int8_t* weight_i8 = nullptr;
  // The same int8 weights in MFMA fragment order for the register-weight
  // kernel, [m_pad/32][kred_pad/32][64 lanes][16 bytes]: lane l of k step s
  // of block b holds row 32b + l%32, bytes 32s + 16(l/32) .. +15, so one
  // wave's load of a k step is 1 KB contiguous.  Only when that kernel can
  // take the plan (kred_pad == kRwKred, m_pad a multiple of 128).
  int8_t* weight_i8_frag = nullptr;
  float* recip = nullptr;
  float input_scale = 1.0f, output_scale = 1.0f;
  int32_t scale_term = 0;
};

struct nhip_ip_plan {
  int32_t n_out, k_in, act;
  int32_t n_pad, k_pad;
  float* weight = nullptr;  // [n_pad][k_pad]
  float* bias = nullptr;    // [n_pad], zero past n_out
  // The same weights in 4-k groups for the one-block-per-workgroup kernel
  // (ip_kq.hip): [n_pad/32][k_kq/4][32][4], k_kq = k_in rounded up to 256;
  // null for reductions beyond that kernel's range.
  float* weight_kq = nullptr;
  // int8 InnerProduct: a 1x1 int8 convolution over m one-pixel images
  nhip_conv_plan* q8 = nullptr;
};

namespace nhip {
// Reduction length (bytes) of the int8 register-weight kernel: 36 k steps of
// 32 bytes (128 channels at 3x3).
constexpr int kRwKred = 36 * 32;
// Input channels from which a Winograd plan also holds an implicit-GEMM twin.
constexpr int kWinoTwinMinC = 256;
// Kernel launchers (defined in the .hip files).
int launch_conv_igemm_f32(const nhip_conv_plan* p, const float* in,
                          const float* residual, float* out, int n, int h,
                          int w, int oh, int ow, void* ws, uint64_t ws_bytes,
                          hipStream_t s);
uint64_t conv_igemm_f32_workspace(const nhip_conv_plan* p, int n, int oh,
                                  int ow);
// 1x1 stride-1 unpadded convolutions (pointwise.hip): true when the
// streaming pointwise kernel takes the layer (no workspace).
bool pointwise_selected(const nhip_conv_plan* p, int n, int h, int w);
int launch_conv_pointwise_f32(const nhip_conv_plan* p, const float* in, const float* residual, float* out, int n,
                              int h, int w, hipStream_t s);
// A 3x3 depthwise convolution feeding a 1x1 convolution, in one pass
// (pointwise.hip): dwpw_supported says whether the pair and shape qualify.
bool dwpw_supported(const nhip_conv_plan* dw, const nhip_conv_plan* pw, int n, int h, int w);
// expand_dw.hip: a 1x1 expand convolution and the 3x3 depthwise reading it,
// one kernel for planes of at most 256 pixels (the expanded tensor never
// reaches memory); pwdw_supported says whether the pair and shape qualify.
bool pwdw_supported(const nhip_conv_plan* pw, const nhip_conv_plan* dw, int n, int h, int w);
int launch_pwdw_f32(const nhip_conv_plan* pw, const nhip_conv_plan* dw, const float* in, float* out, int n, int h,
                    int w, hipStream_t s);
int launch_dwpw_f32(const nhip_conv_plan* dw, const nhip_conv_plan* pw, const float* in, const float* residual,
                    float* out, int n, int h, int w, hipStream_t s);
// dwpw_lds.hip: the pair with its input rows staged through LDS (up to 32
// output channels, channels a multiple of 8); taken by launch_dwpw_f32 when
// dwpw_lds_supported says so (NHIP_DWPW_LDS=0: never).
bool dwpw_lds_supported(const nhip_conv_plan* dw, const nhip_conv_plan* pw, int n, int h, int w, int oh, int ow);
int launch_dwpw_lds_f32(const nhip_conv_plan* dw, const nhip_conv_plan* pw, const float* in,
                        const float* residual, float* out, int n, int h, int w, int oh, int ow, hipStream_t s);
int launch_conv_winograd_f32(const nhip_conv_plan* p, const float* in,
                             const float* residual, float* out, int n, int h,
                             int w, int oh, int ow, void* ws,
                             uint64_t ws_bytes, hipStream_t s);
uint64_t conv_winograd_f32_workspace(const nhip_conv_plan* p, int n, int oh,
                                     int ow);
int winograd_prepack_weights(nhip_conv_plan* p, const float* weight);

// Tile shape and K split of the Winograd batched GEMM (gemm_f32.hip).
struct WinoGemmCfg {
  int bm, bn, bk, splits;
};
WinoGemmCfg wino_gemm_config(int m_pad, int c_pad, int t_pad);
int launch_wino_gemm(const float* U, const float* V, float* M, int m_pad, int c_pad, int t_pad,
                     const WinoGemmCfg& cfg, hipStream_t s);
int launch_conv_int8(const nhip_conv_plan* p, const void* in, int in_is_i8,
                     void* out, int n, int h, int w, int oh, int ow, void* ws,
                     uint64_t ws_bytes, hipStream_t s);
uint64_t conv_int8_workspace(const nhip_conv_plan* p, int n, int h, int w);
int launch_dwconv_f32(const nhip_conv_plan* p, const float* in, float* out,
                      int n, int h, int w, int oh, int ow, hipStream_t s);
int launch_dwconv_int8(const nhip_conv_plan* p, const void* in, int in_is_i8,
                       void* out, int n, int h, int w, int oh, int ow,
                       hipStream_t s);
int launch_innerproduct_f32(const nhip_ip_plan* p, const float* in,
                            float* out, int m, void* ws, uint64_t ws_bytes,
                            hipStream_t s);
uint64_t innerproduct_workspace(const nhip_ip_plan* p, int m);
// ip_kq.hip: one workgroup per 32 x 32 output block, the reduction split
// over its 16 waves and summed in LDS (no workspace).
int ip_kq_prepack(nhip_ip_plan* p, const float* weight);
bool ip_kq_supported(const nhip_ip_plan* p, const float* in, int m);
int launch_ip_kq(const nhip_ip_plan* p, const float* in, float* out, int m, hipStream_t s);
// fp32 GEMMs fed by direct-to-LDS loads (gemm_dma.hip): the InnerProduct
// and the 1x1 stride-1 unpadded convolution.  `in` may be null for the
// workspace query (alignment is then not part of the answer).
bool ip_dma_supported(const nhip_ip_plan* p, const float* in, int m);
uint64_t innerproduct_dma_workspace(const nhip_ip_plan* p, int m);
int launch_innerproduct_dma(const nhip_ip_plan* p, const float* in, float* out, int m, void* ws, uint64_t ws_bytes,
                            hipStream_t s);
// conv_smallk.hip: fp32 convolutions with a reduction of at most 32 and at
// most 32 output channels (network stems), one MFMA block per 32 pixels.
bool smallk_supported(const nhip_conv_plan* p, int n, int h, int w, int oh, int ow);
// conv_kq.hip: fp32 3x3 (32 or 64 input channels) and 1x1 convolutions with
// few output blocks, one workgroup per 32x32 block, the reduction over its
// waves (no workspace).
bool kq_supported(const nhip_conv_plan* p, int n, int h, int w, int oh, int ow);
// The weight copy above for a plan the kernel can take (nothing otherwise).
int conv_kq_prepack(nhip_conv_plan* p, const float* weight, int c, int k, int kh, int kw);
int launch_conv_kq(const nhip_conv_plan* p, const float* in, const float* residual, float* out, int n, int h, int w,
                   int oh, int ow, hipStream_t s);
int launch_conv_smallk(const nhip_conv_plan* p, const float* in, const float* residual, float* out, int n, int h,
                       int w, int oh, int ow, hipStream_t s);
bool pw_dma_supported(const nhip_conv_plan* p, int n, int h, int w);
uint64_t conv_pw_dma_workspace(const nhip_conv_plan* p, int n, int h, int w);
int launch_conv_pw_dma(const nhip_conv_plan* p, const float* in, const float* residual, float* out, int n, int h,
                       int w, void* ws, uint64_t ws_bytes, hipStream_t s);
// Global average pooling of [n][k_in][hw] feeding the InnerProduct, fused
// (gemm_f32.hip), for planes of 1 .. 6400 pixels.
bool gap_innerproduct_supported(int hw);
int launch_gap_innerproduct_f32(const nhip_ip_plan* p, const float* in, float* out, int n, int hw, void* ws,
                                uint64_t ws_bytes, hipStream_t s);
uint64_t gap_innerproduct_workspace(const nhip_ip_plan* p, int n, int hw);
}  // namespace nhip
