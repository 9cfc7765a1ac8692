// Host side of the runtime: status/error plumbing, device and memory calls,
// parameter validation (the checks the reference importer applies before a
// layer reaches the hot path), weight prepacking, and forward dispatch.
//
// This file is compiled with -ffp-contract=off: the host-side constant weight
// quantization and the dequantize reciprocals must be the same separately
// rounded fp32 operations as the reference's compile-time folding.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <limits>
#include <mutex>
#include <tuple>
#include <vector>

#include <unistd.h>

#include "nhip_internal.h"

namespace nhip {

namespace {
thread_local std::string g_last_error;

struct DeviceInfo {
  int cus = 0;
};
std::mutex g_dev_mutex;
DeviceInfo g_dev[64];
}  // namespace

int fail(int status, const std::string& message) {
  g_last_error = message;
  return status;
}

int ok() {
  g_last_error.clear();
  return NHIP_STATUS_SUCCESS;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  return fail(NHIP_STATUS_DEVICE_ERROR, std::string(what) + ": " + hipGetErrorString(e));
}

int check_launch(const char* kernel) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return ok();
  return fail(NHIP_STATUS_DEVICE_ERROR, std::string("launch of ") + kernel + ": " + hipGetErrorString(e));
}

// ---- kernel timer -----------------------------------------------------------
namespace {
struct TimerState {
  std::mutex mu;
  bool on = false;
  std::string filter;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> events;
};
TimerState& timer() {
  static TimerState t;
  return t;
}
}  // namespace

bool kernel_timer_active() {
  TimerState& t = timer();
  std::lock_guard<std::mutex> lock(t.mu);
  return t.on;
}

// Stream capture for the graph executor's replay (csrc/graph.cpp): the
// executor records one run of its call plan into a hipGraph and replays the
// instantiated graph on later calls with the same buffers.
// A failed capture call leaves HIP's thread-local last error set; it is
// cleared here so that the next launch check does not report it as its own
// failure.
bool stream_capturing(void* stream) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(as_stream(stream), &st) != hipSuccess) {
    (void)hipGetLastError();
    return true;  // unknown: treat as not capturable
  }
  return st != hipStreamCaptureStatusNone;
}

int graph_capture_begin(void* stream) {
  const int st = check_hip(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal),
                           "hipStreamBeginCapture");
  if (st != NHIP_STATUS_SUCCESS) (void)hipGetLastError();
  return st;
}

int graph_capture_end(void* stream, void** exec) {
  hipGraph_t graph = nullptr;
  *exec = nullptr;
  int st = check_hip(hipStreamEndCapture(as_stream(stream), &graph), "hipStreamEndCapture");
  if (st == NHIP_STATUS_SUCCESS) {
    hipGraphExec_t e = nullptr;
    st = check_hip(hipGraphInstantiate(&e, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    if (st == NHIP_STATUS_SUCCESS) *exec = e;
  }
  if (graph) (void)hipGraphDestroy(graph);
  if (st != NHIP_STATUS_SUCCESS) (void)hipGetLastError();
  return st;
}

// Device, stream and pinned host memory for the graph executor's host-buffer
// entry (csrc/graph.cpp is host-only C++ without HIP headers).
int device_current(int* dev) { return check_hip(hipGetDevice(dev), "hipGetDevice"); }
int device_set(int dev) { return check_hip(hipSetDevice(dev), "hipSetDevice"); }
void device_restore(int dev) {  // leaves the thread's last error message alone
  if (hipSetDevice(dev) != hipSuccess) (void)hipGetLastError();
}
int stream_create(void** s) {
  hipStream_t st = nullptr;  // default priority, never blocks on the legacy stream
  NHIP_TRY(check_hip(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), "hipStreamCreateWithFlags"));
  *s = st;
  return ok();
}
void stream_destroy(void* s) {
  if (s) (void)hipStreamDestroy(as_stream(s));
}
int host_pinned_alloc(void** p, uint64_t bytes) {
  *p = nullptr;
  return check_hip(hipHostMalloc(p, bytes ? bytes : 1, hipHostMallocDefault), "hipHostMalloc");
}
void host_pinned_free(void* p) {
  if (p) (void)hipHostFree(p);
}

int graph_exec_launch(void* exec, void* stream) {
  NHIP_TRY(check_hip(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(exec), as_stream(stream)), "hipGraphLaunch"));
  return check_launch("graph replay");
}

void graph_exec_destroy(void* exec) {
  if (exec) (void)hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(exec));
}

LaunchTimer::LaunchTimer(const char* kernel) {
  TimerState& t = timer();
  std::lock_guard<std::mutex> lock(t.mu);
  if (!t.on || (!t.filter.empty() && std::string(kernel).find(t.filter) == std::string::npos)) return;
  if (hipEventCreate(&start_) != hipSuccess) {
    start_ = nullptr;
    return;
  }
  if (hipEventCreate(&stop_) != hipSuccess) {
    (void)hipEventDestroy(start_);
    start_ = stop_ = nullptr;
    return;
  }
  t.events.emplace_back(start_, stop_);
}

// ---- NHIP_* switches ----------------------------------------------------------
// Tuning and test switches are read from the environment into an immutable
// snapshot at the first use; nhip_reload_settings() publishes a new one.
// Readers take the current snapshot with one atomic load, so launches never
// call getenv and a reload never invalidates a value a reader still holds
// (snapshots are kept until the process ends; a reload is a rare tuning or
// test action).
namespace {
struct Settings {
  std::vector<std::pair<std::string, std::string>> kv;
  uint64_t generation = 0;
};
std::atomic<const Settings*> g_settings{nullptr};
std::mutex g_settings_mu;

const Settings* load_settings_locked(uint64_t generation) {
  auto* s = new Settings;
  s->generation = generation;
  for (char** e = environ; e && *e; ++e) {
    if (std::strncmp(*e, "NHIP_", 5) != 0) continue;
    const char* eq = std::strchr(*e, '=');
    if (eq) s->kv.emplace_back(std::string(*e, (size_t)(eq - *e)), std::string(eq + 1));
  }
  return s;
}

const Settings* settings_snapshot() {
  const Settings* s = g_settings.load(std::memory_order_acquire);
  if (s) return s;
  std::lock_guard<std::mutex> lock(g_settings_mu);
  s = g_settings.load(std::memory_order_acquire);
  if (!s) {
    s = load_settings_locked(1);
    g_settings.store(s, std::memory_order_release);
  }
  return s;
}
}  // namespace

const char* setting(const char* name) {
  for (const auto& kv : settings_snapshot()->kv)
    if (kv.first == name) return kv.second.c_str();
  return nullptr;
}

int setting_int(const char* name, int fallback) {
  const char* v = setting(name);
  return v && *v ? std::atoi(v) : fallback;
}

uint64_t settings_generation() { return settings_snapshot()->generation; }

// ---- per-device kernel attributes and occupancy -----------------------------
namespace {
std::mutex g_attr_mu;
std::vector<std::tuple<int, const void*>> g_attr_done;
std::vector<std::tuple<int, const void*, int, size_t, int>> g_occupancy;
}  // namespace

int ensure_dynamic_lds(const void* kernel, int bytes) {
  int dev = 0;
  NHIP_TRY(check_hip(hipGetDevice(&dev), "hipGetDevice"));
  std::lock_guard<std::mutex> lock(g_attr_mu);
  for (const auto& d : g_attr_done)
    if (std::get<0>(d) == dev && std::get<1>(d) == kernel) return ok();
  NHIP_TRY(check_hip(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes),
                     "hipFuncSetAttribute(max dynamic LDS)"));
  g_attr_done.emplace_back(dev, kernel);
  return ok();
}

int resident_blocks(const void* kernel, int threads, size_t lds) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 1;
  std::lock_guard<std::mutex> lock(g_attr_mu);
  for (const auto& o : g_occupancy)
    if (std::get<0>(o) == dev && std::get<1>(o) == kernel && std::get<2>(o) == threads && std::get<3>(o) == lds)
      return std::get<4>(o);
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, threads, lds) != hipSuccess || occ < 1) {
    (void)hipGetLastError();
    occ = 1;
  }
  g_occupancy.emplace_back(dev, kernel, threads, lds, occ);
  return occ;
}

// ---- static scratch of nhip_conv2d_f32_forward_noalloc ----------------------
// Device memory for callers that cannot allocate: one array per GPU, set up
// once per device.  In host code `scratch` names a host-side stand-in, so the
// device address is taken with hipGetSymbolAddress (per device, with that
// device current) and only that address is handed to kernels.
constexpr uint64_t kScratchBytes = uint64_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[64];
}  // namespace

int scratch_address(void** out) {
  *out = nullptr;
  int dev = 0;
  NHIP_TRY(check_hip(hipGetDevice(&dev), "hipGetDevice"));
  if (dev < 0 || dev >= 64) return fail(NHIP_STATUS_UNSUPPORTED, "static scratch: device index above 63");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    NHIP_TRY(check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return ok();
}

int cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(g_dev_mutex);
  if (g_dev[dev].cus == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    g_dev[dev].cus = cus;
  }
  return g_dev[dev].cus;
}

namespace {

// ---- validation mirrors lib/Graph/graph.cpp:219-301 and the importers -----
int validate_common(const nhip_conv_desc* d) {
  if (!d) return fail(NHIP_STATUS_NULL_POINTER, "conv: null descriptor");
  if (d->input_channels <= 0 || d->num_output <= 0)
    return fail(NHIP_STATUS_INVALID_SHAPE, "conv: channels must be positive");
  if (d->kernel_w <= 0 || d->kernel_h <= 0)
    return fail(NHIP_STATUS_INVALID_SHAPE, "convolution kernel dimensions must be positive");
  if (d->dilation_w <= 0 || d->dilation_h <= 0)
    return fail(NHIP_STATUS_INVALID_SHAPE, "convolution dilation must be positive");
  if (d->stride_w <= 0 || d->stride_h <= 0)
    return fail(NHIP_STATUS_INVALID_SHAPE, "convolution stride must be positive");
  if (d->pad_left < 0 || d->pad_right < 0 || d->pad_top < 0 || d->pad_bottom < 0)
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION,
                "requires explicit non-negative padding; resolve SAME padding first");
  if (d->bias_term != 0 && d->bias_term != 1)
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "convolution bias_term must be 0 or 1");
  const int t = d->int8_scale_term;
  if (t != 0 && t != 1 && t != 2 && t != 101 && t != 102)
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION,
                "convolution int8_scale_term must be 0, 1, 2, 101, or 102");
  // The gather tables pack dy/dx in 8 bits and the channel in 15.
  if ((int64_t)(d->kernel_h - 1) * d->dilation_h > 255 || (int64_t)(d->kernel_w - 1) * d->dilation_w > 255 ||
      d->input_channels > 32000)
    return fail(NHIP_STATUS_UNSUPPORTED, "conv: kernel extent > 256 or more than 32000 channels");
  return ok();
}

ConvGeom geom_of(const nhip_conv_desc* d) {
  ConvGeom g;
  g.c = d->input_channels;
  g.k = d->num_output;
  g.kh = d->kernel_h;
  g.kw = d->kernel_w;
  g.sh = d->stride_h;
  g.sw = d->stride_w;
  g.dh = d->dilation_h;
  g.dw = d->dilation_w;
  g.pt = d->pad_top;
  g.pb = d->pad_bottom;
  g.pl = d->pad_left;
  g.pr = d->pad_right;
  g.act = d->activation_type;
  return g;
}

template <typename T>
int upload(T** dst, const std::vector<T>& host, const char* what) {
  NHIP_TRY(check_hip(hipMalloc(reinterpret_cast<void**>(dst), std::max<size_t>(host.size(), 1) * sizeof(T)), what));
  return check_hip(hipMemcpy(*dst, host.data(), host.size() * sizeof(T), hipMemcpyHostToDevice), what);
}

int upload_bias(nhip_conv_plan* p, const float* bias, int count, int padded) {
  std::vector<float> b((size_t)padded, 0.f);
  if (bias) std::copy(bias, bias + count, b.begin());
  return upload(&p->bias, b, "hipMalloc(bias)");
}

void free_plan(nhip_conv_plan* p) {
  if (!p) return;
  free_plan(p->igemm_twin);
  (void)hipFree(p->weight);
  (void)hipFree(p->weight_fused);
  (void)hipFree(p->weight_kq);
  (void)hipFree(p->weight_ck);
  (void)hipFree(p->weight_dw12);
  (void)hipFree(p->bias);
  (void)hipFree(p->ktab);
  (void)hipFree(p->weight_i8);
  (void)hipFree(p->weight_i8_frag);
  (void)hipFree(p->recip);
  delete p;
}

// quantizeConstantToI8 (NCNNToTosa.cpp:234-301) for one value.
int8_t quantize_host(float x, float scale) {
#pragma clang fp contract(off)
  const float s = x * scale;
  if (s != s) return 0;
  float r = (s >= 0.0f) ? std::floor(s + 0.5f) : std::ceil(s - 0.5f);
  if (r > 127.0f) r = 127.0f;
  if (r < -127.0f) r = -127.0f;
  return (int8_t)(int)r;
}

int conv_out(const ConvGeom& g, int h, int w, int* oh, int* ow) {
  const int64_t eh = (int64_t)(g.kh - 1) * g.dh + 1, ew = (int64_t)(g.kw - 1) * g.dw + 1;
  const int64_t ph = (int64_t)h + g.pt + g.pb - eh, pw = (int64_t)w + g.pl + g.pr - ew;
  if (ph < 0 || pw < 0) return fail(NHIP_STATUS_INVALID_SHAPE, "conv: input smaller than the kernel extent");
  *oh = (int)(ph / g.sh + 1);
  *ow = (int)(pw / g.sw + 1);
  return ok();
}

// Checks shared by every forward call: pointers, positive extents, and that
// per-batch element counts fit the kernels' 32-bit pixel indexing.
int check_forward(const nhip_conv_plan* p, const void* in, const void* out, int n, int h, int w,
                  int* oh, int* ow) {
  if (!p) return fail(NHIP_STATUS_NULL_POINTER, "conv: null plan");
  if (n < 0 || h <= 0 || w <= 0) return fail(NHIP_STATUS_INVALID_SHAPE, "conv: invalid input extent");
  // An empty batch has no elements to address: its buffers may be null.
  if (n > 0 && (!in || !out)) return fail(NHIP_STATUS_NULL_POINTER, "conv: null input or output");
  NHIP_TRY(conv_out(p->g, h, w, oh, ow));
  const int64_t lim = std::numeric_limits<int32_t>::max();
  if ((int64_t)p->g.c * h * w > lim / 4 || (int64_t)p->g.k * *oh * *ow > lim / 4 ||
      (int64_t)n * *oh * *ow > lim || (int64_t)n * h * w > lim)
    return fail(NHIP_STATUS_SHAPE_ARITHMETIC_OVERFLOW, "conv: tensor too large for 32-bit pixel indexing");
  return ok();
}

// Kernels address their input as one raw buffer resource with 32-bit byte
// offsets, so a launch must keep every tensor below 2^31 bytes.  Larger
// batches run as consecutive sub-batches of whole images on the same stream.
template <typename F>
int for_each_subbatch(int n, int64_t max_image_bytes, F&& run) {
  const int64_t lim = (int64_t)1 << 31;
  const int per = (int)std::max<int64_t>(1, (lim - 1) / std::max<int64_t>(max_image_bytes, 1));
  for (int i0 = 0; i0 < n; i0 += per) NHIP_TRY(run(i0, std::min(per, n - i0)));
  return ok();
}

}  // namespace
}  // namespace nhip

using namespace nhip;

extern "C" {

const char* nhip_last_error(void) { return g_last_error.c_str(); }

int nhip_init(int32_t device) {
  int count = 0;
  NHIP_TRY(check_hip(hipGetDeviceCount(&count), "hipGetDeviceCount"));
  if (device < 0 || device >= count)
    return fail(NHIP_STATUS_INVALID_SHAPE, "nhip_init: no such device " + std::to_string(device));
  NHIP_TRY(check_hip(hipSetDevice(device), "hipSetDevice"));
  NHIP_TRY(check_hip(hipFree(nullptr), "device initialisation"));
  cu_count();
  void* scratch_dev = nullptr;  // the static scratch's address on this device
  NHIP_TRY(scratch_address(&scratch_dev));
  return ok();
}

int nhip_reload_settings(void) {
  std::lock_guard<std::mutex> lock(nhip::g_settings_mu);
  const nhip::Settings* cur = nhip::g_settings.load(std::memory_order_acquire);
  nhip::g_settings.store(nhip::load_settings_locked(cur ? cur->generation + 1 : 1), std::memory_order_release);
  return ok();
}

int nhip_device_count(int32_t* count) {
  if (!count) return fail(NHIP_STATUS_NULL_POINTER, "device_count: null pointer");
  int c = 0;
  NHIP_TRY(check_hip(hipGetDeviceCount(&c), "hipGetDeviceCount"));
  *count = c;
  return ok();
}

int nhip_malloc(void** ptr, uint64_t bytes) {
  if (!ptr) return fail(NHIP_STATUS_NULL_POINTER, "malloc: null pointer");
  *ptr = nullptr;
  return check_hip(hipMalloc(ptr, bytes ? bytes : 1), "hipMalloc");
}

int nhip_free(void* ptr) { return check_hip(hipFree(ptr), "hipFree"); }

int nhip_memcpy_h2d(void* dst, const void* src, uint64_t bytes, void* stream) {
  if ((!dst || !src) && bytes) return fail(NHIP_STATUS_NULL_POINTER, "memcpy_h2d: null pointer");
  return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)), "hipMemcpyAsync(H2D)");
}

int nhip_memcpy_d2h(void* dst, const void* src, uint64_t bytes, void* stream) {
  if ((!dst || !src) && bytes) return fail(NHIP_STATUS_NULL_POINTER, "memcpy_d2h: null pointer");
  return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)), "hipMemcpyAsync(D2H)");
}

int nhip_memcpy_d2d(void* dst, const void* src, uint64_t bytes, void* stream) {
  if ((!dst || !src) && bytes) return fail(NHIP_STATUS_NULL_POINTER, "memcpy_d2d: null pointer");
  return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)), "hipMemcpyAsync(D2D)");
}

int nhip_stream_sync(void* stream) {
  return check_hip(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
}

int nhip_timer_start(const char* kernel_filter) {
  TimerState& t = timer();
  std::lock_guard<std::mutex> lock(t.mu);
  for (auto& e : t.events) {
    (void)hipEventDestroy(e.first);
    (void)hipEventDestroy(e.second);
  }
  t.events.clear();
  t.filter = kernel_filter ? kernel_filter : "";
  t.on = true;
  return ok();
}

int nhip_timer_stop(uint64_t* launches, double* total_ms) {
  if (!launches || !total_ms) return fail(NHIP_STATUS_NULL_POINTER, "timer_stop: null pointer");
  TimerState& t = timer();
  std::lock_guard<std::mutex> lock(t.mu);
  t.on = false;
  double sum = 0.0;
  int status = NHIP_STATUS_SUCCESS;
  for (auto& e : t.events) {
    float ms = 0.f;
    if (status == NHIP_STATUS_SUCCESS) {
      status = check_hip(hipEventSynchronize(e.second), "hipEventSynchronize(timer)");
      if (status == NHIP_STATUS_SUCCESS)
        status = check_hip(hipEventElapsedTime(&ms, e.first, e.second), "hipEventElapsedTime(timer)");
    }
    sum += ms;
    (void)hipEventDestroy(e.first);
    (void)hipEventDestroy(e.second);
  }
  *launches = t.events.size();
  *total_ms = sum;
  t.events.clear();
  if (status != NHIP_STATUS_SUCCESS) return status;
  return ok();
}

int nhip_conv_output_shape(const nhip_conv_desc* desc, int32_t h, int32_t w, int32_t* out_h, int32_t* out_w) {
  NHIP_TRY(validate_common(desc));
  if (!out_h || !out_w) return fail(NHIP_STATUS_NULL_POINTER, "conv_output_shape: null pointer");
  if (h <= 0 || w <= 0) return fail(NHIP_STATUS_INVALID_SHAPE, "conv_output_shape: invalid input extent");
  int oh = 0, ow = 0;
  NHIP_TRY(conv_out(geom_of(desc), h, w, &oh, &ow));
  *out_h = oh;
  *out_w = ow;
  return ok();
}

int nhip_conv2d_f32_create(const nhip_conv_desc* d, const float* weight, const float* bias,
                           nhip_conv_t* plan) {
  NHIP_TRY(validate_common(d));
  if (!weight || !plan) return fail(NHIP_STATUS_NULL_POINTER, "conv2d_f32_create: null pointer");
  if (d->bias_term && !bias) return fail(NHIP_STATUS_NULL_POINTER, "conv2d_f32_create: bias_term set but bias is null");
  if (d->int8_scale_term != 0)
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "conv2d_f32_create: int8_scale_term must be 0 (use conv2d_int8_create)");
  if (d->group != 0 && d->group != 1)
    return fail(NHIP_STATUS_UNSUPPORTED, "Convolution has no group parameter (ImportConvolution.cpp:55-56)");
  const int act = d->activation_type;
  if (act != NHIP_ACT_NONE && act != NHIP_ACT_RELU && act != NHIP_ACT_SIGMOID)
    return fail(NHIP_STATUS_UNSUPPORTED, "unsupported fused activation");
  *plan = nullptr;
  auto* p = new nhip_conv_plan();
  p->kind = PlanKind::ConvF32;
  p->g = geom_of(d);
  p->has_bias = d->bias_term;
  const bool wino_shape = d->kernel_h == 3 && d->kernel_w == 3 && d->stride_h == 1 && d->stride_w == 1 &&
                          d->dilation_h == 1 && d->dilation_w == 1;
  int algo = d->algorithm;
  if (algo == NHIP_CONV_ALGO_AUTO)
    algo = (wino_shape && d->input_channels >= 16 && d->num_output >= 16) ? NHIP_CONV_ALGO_WINOGRAD
                                                                         : NHIP_CONV_ALGO_IMPLICIT_GEMM;
  if (algo == NHIP_CONV_ALGO_WINOGRAD && !wino_shape) {
    free_plan(p);
    return fail(NHIP_STATUS_UNSUPPORTED, "winograd needs a 3x3 stride-1 dilation-1 convolution");
  }
  if (algo != NHIP_CONV_ALGO_WINOGRAD && algo != NHIP_CONV_ALGO_IMPLICIT_GEMM) {
    free_plan(p);
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "unknown convolution algorithm");
  }
  p->algorithm = algo;
  const int K = d->num_output, C = d->input_channels;
  p->m_pad = (int)round_up(K, 64);
  int st = NHIP_STATUS_SUCCESS;
  if (algo == NHIP_CONV_ALGO_WINOGRAD) {
    p->c_pad = (int)round_up(C, 16);
    st = winograd_prepack_weights(p, weight);
    if (st == NHIP_STATUS_SUCCESS) st = conv_kq_prepack(p, weight, C, K, 3, 3);
    if (st == NHIP_STATUS_SUCCESS && C >= kWinoTwinMinC) {
      nhip_conv_desc d2 = *d;
      d2.algorithm = NHIP_CONV_ALGO_IMPLICIT_GEMM;
      st = nhip_conv2d_f32_create(&d2, weight, bias, &p->igemm_twin);
    }
  } else {
    const int khw = d->kernel_h * d->kernel_w;
    p->kred = C * khw;
    p->kred_pad = (int)round_up(p->kred, 16);
    std::vector<float> wp((size_t)p->m_pad * p->kred_pad, 0.f);
    for (int k = 0; k < K; ++k)
      std::copy(weight + (size_t)k * p->kred, weight + (size_t)(k + 1) * p->kred, wp.begin() + (size_t)k * p->kred_pad);
    std::vector<int32_t> kt((size_t)p->kred_pad, 0x7fff << 16);
    for (int k = 0; k < p->kred; ++k) {
      const int c = k / khw, r = k % khw, kh = r / d->kernel_w, kw = r % d->kernel_w;
      kt[k] = (c << 16) | ((kh * d->dilation_h) << 8) | (kw * d->dilation_w);
    }
    st = upload(&p->weight, wp, "hipMalloc(conv weight)");
    if (st == NHIP_STATUS_SUCCESS) st = upload(&p->ktab, kt, "hipMalloc(conv ktab)");
    if (st == NHIP_STATUS_SUCCESS) st = conv_kq_prepack(p, weight, C, K, d->kernel_h, d->kernel_w);
    if (st == NHIP_STATUS_SUCCESS && khw == 1 && K <= 32) {
      std::vector<float> ck((size_t)C * 32, 0.f);
      for (int k = 0; k < K; ++k)
        for (int c = 0; c < C; ++c) ck[(size_t)c * 32 + k] = weight[(size_t)k * C + c];
      st = upload(&p->weight_ck, ck, "hipMalloc(1x1 weight, channel-major)");
    }
  }
  if (st == NHIP_STATUS_SUCCESS) st = upload_bias(p, d->bias_term ? bias : nullptr, K, p->m_pad);
  if (st != NHIP_STATUS_SUCCESS) {
    std::string msg = g_last_error;
    free_plan(p);
    return fail(st, msg);
  }
  *plan = p;
  return ok();
}

int nhip_conv2d_workspace_size(nhip_conv_t p, int32_t n, int32_t h, int32_t w, uint64_t* bytes) {
  if (!p || !bytes) return fail(NHIP_STATUS_NULL_POINTER, "workspace_size: null pointer");
  int oh = 0, ow = 0;
  if (n < 0 || h <= 0 || w <= 0) return fail(NHIP_STATUS_INVALID_SHAPE, "workspace_size: invalid extent");
  NHIP_TRY(conv_out(p->g, h, w, &oh, &ow));
  switch (p->kind) {
    case PlanKind::ConvF32:
      *bytes = p->algorithm == NHIP_CONV_ALGO_WINOGRAD ? conv_winograd_f32_workspace(p, n, oh, ow)
                                                       : conv_igemm_f32_workspace(p, n, oh, ow);
      break;
    case PlanKind::ConvInt8:
      *bytes = conv_int8_workspace(p, n, h, w);
      break;
    default:
      *bytes = 0;
  }
  return ok();
}

int nhip_conv2d_f32_forward(nhip_conv_t p, const float* input, const float* residual, float* output,
                            int32_t n, int32_t h, int32_t w, void* workspace, uint64_t workspace_bytes,
                            void* stream) {
  int oh = 0, ow = 0;
  NHIP_TRY(check_forward(p, input, output, n, h, w, &oh, &ow));
  if (p->kind != PlanKind::ConvF32) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "conv2d_f32_forward: not an fp32 conv plan");
  if (n == 0) return ok();
  const int64_t in_img = (int64_t)p->g.c * h * w, out_img = (int64_t)p->g.k * oh * ow;
  return for_each_subbatch(n, 4 * std::max(in_img, out_img), [&](int i0, int nb) {
    const float* in = input + i0 * in_img;
    const float* res = residual ? residual + i0 * out_img : nullptr;
    float* out = output + i0 * out_img;
    if (p->algorithm == NHIP_CONV_ALGO_WINOGRAD)
      return launch_conv_winograd_f32(p, in, res, out, nb, h, w, oh, ow, workspace, workspace_bytes,
                                      as_stream(stream));
    return launch_conv_igemm_f32(p, in, res, out, nb, h, w, oh, ow, workspace, workspace_bytes,
                                 as_stream(stream));
  });
}

int nhip_conv2d_f32_forward_noalloc(nhip_conv_t p, const float* input, const float* residual, float* output,
                                    int32_t n, int32_t h, int32_t w, void* stream) {
  int oh = 0, ow = 0;
  NHIP_TRY(check_forward(p, input, output, n, h, w, &oh, &ow));
  if (p->kind != PlanKind::ConvF32)
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "conv2d_f32_forward_noalloc: not an fp32 conv plan");
  if (n == 0) return ok();
  uint64_t need = 0;
  NHIP_TRY(nhip_conv2d_workspace_size(p, n, h, w, &need));
  if (need > kScratchBytes)
    return fail(NHIP_STATUS_OUTPUT_CAPACITY_INSUFFICIENT,
                "conv2d_f32_forward_noalloc: this batch needs " + std::to_string(need) +
                    " bytes of scratch; the static scratch holds " + std::to_string(kScratchBytes) +
                    " (use nhip_conv2d_f32_forward with a workspace, or a smaller batch)");
  void* ws = nullptr;
  NHIP_TRY(scratch_address(&ws));
  return nhip_conv2d_f32_forward(p, input, residual, output, n, h, w, ws, kScratchBytes, stream);
}

int nhip_conv2d_int8_create(const nhip_conv_desc* d, const void* weight, int32_t weight_is_i8, const float* bias,
                            const float* weight_scale, int32_t weight_scale_count, float input_scale,
                            float output_scale, nhip_conv_t* plan) {
  NHIP_TRY(validate_common(d));
  if (!weight || !plan || !weight_scale) return fail(NHIP_STATUS_NULL_POINTER, "conv2d_int8_create: null pointer");
  if (d->bias_term && !bias) return fail(NHIP_STATUS_NULL_POINTER, "conv2d_int8_create: bias_term set but bias is null");
  if (d->int8_scale_term == 0)
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "conv2d_int8_create: int8_scale_term must be nonzero");
  if (d->group != 0 && d->group != 1)
    return fail(NHIP_STATUS_UNSUPPORTED, "Convolution has no group parameter");
  if (d->activation_type != NHIP_ACT_NONE && d->activation_type != NHIP_ACT_RELU)
    return fail(NHIP_STATUS_UNSUPPORTED, "int8 convolution: activation must be 0 or 1");
  if (weight_scale_count != 1 && weight_scale_count != d->num_output)
    return fail(NHIP_STATUS_INVALID_SHAPE, "conv2d_int8_create: weight_scale count must be 1 or num_output");
  *plan = nullptr;
  auto* p = new nhip_conv_plan();
  p->kind = PlanKind::ConvInt8;
  p->g = geom_of(d);
  p->algorithm = NHIP_CONV_ALGO_IMPLICIT_GEMM;
  p->has_bias = d->bias_term;
  p->scale_term = d->int8_scale_term;
  p->input_scale = input_scale;
  p->output_scale = output_scale;
  const int K = d->num_output, C = d->input_channels, KH = d->kernel_h, KW = d->kernel_w;
  p->m_pad = (int)round_up(K, 64);
  p->c_pad = (int)round_up(C, 16);
  p->kred = KH * KW * p->c_pad;
  p->kred_pad = (int)round_up(p->kred, 128);  // whole 128-byte GEMM K stages (256-byte tiles where it divides)
  // Weights to int8 [m_pad][kh][kw][c_pad] (OHWI with channel padding).
  std::vector<int8_t> wq((size_t)p->m_pad * p->kred_pad, 0);
  for (int k = 0; k < K; ++k) {
    const float ws = weight_scale[weight_scale_count == 1 ? 0 : k];
    for (int c = 0; c < C; ++c)
      for (int kh = 0; kh < KH; ++kh)
        for (int kw = 0; kw < KW; ++kw) {
          const size_t src = (((size_t)k * C + c) * KH + kh) * KW + kw;
          const int8_t q = weight_is_i8 ? static_cast<const int8_t*>(weight)[src]
                                        : quantize_host(static_cast<const float*>(weight)[src], ws);
          wq[(size_t)k * p->kred_pad + (size_t)(kh * KW + kw) * p->c_pad + c] = q;
        }
  }
  // dequantizeAccumulator reciprocals (NCNNToTosa.cpp:577-637).
  std::vector<float> rc((size_t)p->m_pad, 0.f);
  for (int k = 0; k < K; ++k) {
#pragma clang fp contract(off)
    const float ws = weight_scale[weight_scale_count == 1 ? 0 : k];
    const float combined = ws * input_scale;
    const float r = 1.0f / combined;
    rc[k] = ws == 0.0f ? 0.0f : r;
  }
  std::vector<int32_t> kt((size_t)p->kred_pad / 16, 0x7fff << 16);
  for (int q = 0; q < p->kred / 16; ++q) {
    const int kidx = q * 16, r = kidx / p->c_pad, c0 = kidx % p->c_pad;
    const int kh = r / KW, kw = r % KW;
    kt[q] = (c0 << 16) | ((kh * d->dilation_h) << 8) | (kw * d->dilation_w);
  }
  int st = upload(&p->weight_i8, wq, "hipMalloc(int8 weight)");
  if (st == NHIP_STATUS_SUCCESS && p->kred_pad == nhip::kRwKred && p->m_pad % 128 == 0) {
    std::vector<int8_t> wf(wq.size());
    const int ks = p->kred_pad / 32;
    for (int b = 0; b < p->m_pad / 32; ++b)
      for (int s = 0; s < ks; ++s)
        for (int l = 0; l < 64; ++l)
          std::copy_n(wq.begin() + (size_t)(32 * b + l % 32) * p->kred_pad + 32 * s + 16 * (l / 32), 16,
                      wf.begin() + (((size_t)b * ks + s) * 64 + l) * 16);
    st = upload(&p->weight_i8_frag, wf, "hipMalloc(int8 fragment-order weight)");
  }
  if (st == NHIP_STATUS_SUCCESS) st = upload(&p->recip, rc, "hipMalloc(int8 reciprocal)");
  if (st == NHIP_STATUS_SUCCESS) st = upload(&p->ktab, kt, "hipMalloc(int8 ktab)");
  if (st == NHIP_STATUS_SUCCESS) st = upload_bias(p, d->bias_term ? bias : nullptr, K, p->m_pad);
  if (st != NHIP_STATUS_SUCCESS) {
    std::string msg = g_last_error;
    free_plan(p);
    return fail(st, msg);
  }
  *plan = p;
  return ok();
}

int nhip_conv2d_int8_forward(nhip_conv_t p, const void* input, int32_t input_is_i8, void* output, int32_t n,
                             int32_t h, int32_t w, void* workspace, uint64_t workspace_bytes, void* stream) {
  int oh = 0, ow = 0;
  NHIP_TRY(check_forward(p, input, output, n, h, w, &oh, &ow));
  if (p->kind != PlanKind::ConvInt8) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "conv2d_int8_forward: not an int8 conv plan");
  if (n == 0) return ok();
  const int64_t in_img = (int64_t)p->g.c * h * w, out_img = (int64_t)p->g.k * oh * ow;
  const int in_es = input_is_i8 ? 1 : 4, out_es = p->scale_term > 100 ? 1 : 4;
  const int64_t ws_img = (int64_t)h * w * p->c_pad;
  return for_each_subbatch(n, std::max({in_es * in_img, out_es * out_img, ws_img}), [&](int i0, int nb) {
    return launch_conv_int8(p, static_cast<const char*>(input) + i0 * in_img * in_es, input_is_i8 ? 1 : 0,
                            static_cast<char*>(output) + i0 * out_img * out_es, nb, h, w, oh, ow, workspace,
                            workspace_bytes, as_stream(stream));
  });
}

int nhip_dwconv2d_f32_create(const nhip_conv_desc* d, const float* weight, const float* bias, nhip_conv_t* plan) {
  NHIP_TRY(validate_common(d));
  if (!weight || !plan) return fail(NHIP_STATUS_NULL_POINTER, "dwconv2d_f32_create: null pointer");
  if (d->bias_term && !bias) return fail(NHIP_STATUS_NULL_POINTER, "dwconv2d_f32_create: bias_term set but bias is null");
  if (d->group != d->input_channels || d->num_output != d->input_channels)
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "depthwise group must equal input channels");
  if (d->int8_scale_term != 0)
    return fail(NHIP_STATUS_UNSUPPORTED, "dwconv2d_f32_create: int8 depthwise is not in this build");
  if (d->activation_type != NHIP_ACT_NONE && d->activation_type != NHIP_ACT_RELU)
    return fail(NHIP_STATUS_UNSUPPORTED, "depthwise activation must be 0 or 1");
  *plan = nullptr;
  auto* p = new nhip_conv_plan();
  p->kind = PlanKind::DwConvF32;
  p->g = geom_of(d);
  p->algorithm = NHIP_CONV_ALGO_IMPLICIT_GEMM;
  p->has_bias = d->bias_term;
  const size_t wcount = (size_t)d->num_output * d->kernel_h * d->kernel_w;
  std::vector<float> wv(weight, weight + wcount);
  int st = upload(&p->weight, wv, "hipMalloc(dw weight)");
  if (st == NHIP_STATUS_SUCCESS) st = upload_bias(p, d->bias_term ? bias : nullptr, d->num_output, d->num_output);
  if (st == NHIP_STATUS_SUCCESS && d->kernel_h == 3 && d->kernel_w == 3) {
    std::vector<float> w12((size_t)d->num_output * 12, 0.f);
    for (int c = 0; c < d->num_output; ++c) {
      std::copy(weight + (size_t)c * 9, weight + (size_t)c * 9 + 9, w12.begin() + (size_t)c * 12);
      w12[(size_t)c * 12 + 9] = d->bias_term ? bias[c] : 0.f;
    }
    st = upload(&p->weight_dw12, w12, "hipMalloc(dw weight, 12-float records)");
  }
  if (st != NHIP_STATUS_SUCCESS) {
    std::string msg = g_last_error;
    free_plan(p);
    return fail(st, msg);
  }
  *plan = p;
  return ok();
}

int nhip_dwconv2d_f32_forward(nhip_conv_t p, const float* input, float* output, int32_t n, int32_t h, int32_t w,
                              void* stream) {
  int oh = 0, ow = 0;
  NHIP_TRY(check_forward(p, input, output, n, h, w, &oh, &ow));
  if (p->kind != PlanKind::DwConvF32) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "dwconv2d_f32_forward: not a depthwise plan");
  if (n == 0) return ok();
  return launch_dwconv_f32(p, input, output, n, h, w, oh, ow, as_stream(stream));
}

int nhip_dwconv2d_pw_f32_supported(nhip_conv_t dw, nhip_conv_t pw, int32_t n, int32_t h, int32_t w,
                                   int32_t* supported) {
  if (!dw || !pw || !supported) return fail(NHIP_STATUS_NULL_POINTER, "dwconv2d_pw_supported: null pointer");
  if (n < 0 || h <= 0 || w <= 0) return fail(NHIP_STATUS_INVALID_SHAPE, "dwconv2d_pw_supported: invalid extent");
  *supported = 0;
  int oh = 0, ow = 0;
  if (conv_out(dw->g, h, w, &oh, &ow) != NHIP_STATUS_SUCCESS) return ok();
  // the forward call runs sub-batches of at most this many images
  const int64_t img = 4 * std::max((int64_t)dw->g.c * h * w, (int64_t)pw->g.k * oh * ow);
  const int per = (int)std::max<int64_t>(1, ((int64_t(1) << 31) - 1) / std::max<int64_t>(img, 1));
  *supported = dwpw_supported(dw, pw, std::max(1, std::min<int>(n, per)), h, w) ? 1 : 0;
  return ok();
}

int nhip_dwconv2d_pw_f32_forward(nhip_conv_t dw, nhip_conv_t pw, const float* input, const float* residual,
                                 float* output, int32_t n, int32_t h, int32_t w, void* stream) {
  int oh = 0, ow = 0;
  if (!pw) return fail(NHIP_STATUS_NULL_POINTER, "dwconv2d_pw_forward: null plan");
  NHIP_TRY(check_forward(dw, input, output, n, h, w, &oh, &ow));
  if (dw->kind != PlanKind::DwConvF32 || pw->kind != PlanKind::ConvF32 || pw->g.c != dw->g.c)
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION,
                "dwconv2d_pw_forward: needs an fp32 depthwise plan and an fp32 convolution over its channels");
  if (n == 0) return ok();
  const int64_t in_img = (int64_t)dw->g.c * h * w, out_img = (int64_t)pw->g.k * oh * ow;
  return for_each_subbatch(n, 4 * std::max(in_img, out_img), [&](int i0, int nb) {
    if (!dwpw_supported(dw, pw, nb, h, w))
      return fail(NHIP_STATUS_UNSUPPORTED, "dwconv2d_pw_forward: this pair or shape has no fused kernel");
    return launch_dwpw_f32(dw, pw, input + i0 * in_img, residual ? residual + i0 * out_img : nullptr,
                           output + i0 * out_img, nb, h, w, as_stream(stream));
  });
}

int nhip_conv1x1_dw_f32_supported(nhip_conv_t pw, nhip_conv_t dw, int32_t n, int32_t h, int32_t w,
                                  int32_t* supported) {
  if (!pw || !dw || !supported) return fail(NHIP_STATUS_NULL_POINTER, "conv1x1_dw_supported: null pointer");
  if (n < 0 || h <= 0 || w <= 0) return fail(NHIP_STATUS_INVALID_SHAPE, "conv1x1_dw_supported: invalid extent");
  *supported = pwdw_supported(pw, dw, std::max(1, std::min<int32_t>(n, 65535)), h, w) ? 1 : 0;
  return ok();
}

int nhip_conv1x1_dw_f32_forward(nhip_conv_t pw, nhip_conv_t dw, const float* input, float* output, int32_t n,
                                int32_t h, int32_t w, void* stream) {
  int oh = 0, ow = 0;
  if (!pw) return fail(NHIP_STATUS_NULL_POINTER, "conv1x1_dw_forward: null plan");
  NHIP_TRY(check_forward(dw, input, output, n, h, w, &oh, &ow));
  if (dw->kind != PlanKind::DwConvF32 || pw->kind != PlanKind::ConvF32 || dw->g.c != pw->g.k)
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION,
                "conv1x1_dw_forward: needs an fp32 convolution and an fp32 depthwise plan over its outputs");
  if (n == 0) return ok();
  const int64_t in_img = (int64_t)pw->g.c * h * w, out_img = (int64_t)dw->g.k * oh * ow;
  return for_each_subbatch(n, 4 * std::max(in_img, out_img), [&](int i0, int nb) {
    // the grid's y extent is the batch
    for (int j0 = 0; j0 < nb; j0 += 65535) {
      const int nj = std::min(65535, nb - j0);
      if (!pwdw_supported(pw, dw, nj, h, w))
        return fail(NHIP_STATUS_UNSUPPORTED, "conv1x1_dw_forward: this pair or shape has no fused kernel");
      NHIP_TRY(launch_pwdw_f32(pw, dw, input + (i0 + j0) * in_img, output + (i0 + j0) * out_img, nj, h, w,
                               as_stream(stream)));
    }
    return ok();
  });
}

int nhip_dwconv2d_int8_create(const nhip_conv_desc* d, const void* weight, int32_t weight_is_i8, const float* bias,
                              const float* weight_scale, int32_t weight_scale_count, float input_scale,
                              float output_scale, nhip_conv_t* plan) {
  NHIP_TRY(validate_common(d));
  if (!weight || !plan || !weight_scale) return fail(NHIP_STATUS_NULL_POINTER, "dwconv2d_int8_create: null pointer");
  if (d->bias_term && !bias) return fail(NHIP_STATUS_NULL_POINTER, "dwconv2d_int8_create: bias_term set but bias is null");
  if (d->group != d->input_channels || d->num_output != d->input_channels)
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "depthwise group must equal input channels");
  if (d->int8_scale_term == 0)
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "dwconv2d_int8_create: int8_scale_term must be nonzero");
  if (d->activation_type != NHIP_ACT_NONE && d->activation_type != NHIP_ACT_RELU)
    return fail(NHIP_STATUS_UNSUPPORTED, "depthwise activation must be 0 or 1");
  const int C = d->input_channels, KHW = d->kernel_h * d->kernel_w;
  if (weight_scale_count != 1 && weight_scale_count != C)
    return fail(NHIP_STATUS_INVALID_SHAPE, "dwconv2d_int8_create: weight_scale count must be 1 or C");
  *plan = nullptr;
  auto* p = new nhip_conv_plan();
  p->kind = PlanKind::DwConvInt8;
  p->g = geom_of(d);
  p->algorithm = NHIP_CONV_ALGO_IMPLICIT_GEMM;
  p->has_bias = d->bias_term;
  p->scale_term = d->int8_scale_term;
  p->input_scale = input_scale;
  p->output_scale = output_scale;
  std::vector<int8_t> wq((size_t)C * KHW);
  for (int c = 0; c < C; ++c) {
    const float ws = weight_scale[weight_scale_count == 1 ? 0 : c];
    for (int e = 0; e < KHW; ++e) {
      const size_t i = (size_t)c * KHW + e;
      wq[i] = weight_is_i8 ? static_cast<const int8_t*>(weight)[i] : quantize_host(static_cast<const float*>(weight)[i], ws);
    }
  }
  std::vector<float> rc((size_t)C, 0.f);
  for (int c = 0; c < C; ++c) {
#pragma clang fp contract(off)
    const float ws = weight_scale[weight_scale_count == 1 ? 0 : c];
    const float combined = ws * input_scale;
    const float r = 1.0f / combined;
    rc[c] = ws == 0.0f ? 0.0f : r;
  }
  int st = upload(&p->weight_i8, wq, "hipMalloc(dw int8 weight)");
  if (st == NHIP_STATUS_SUCCESS) st = upload(&p->recip, rc, "hipMalloc(dw int8 reciprocal)");
  if (st == NHIP_STATUS_SUCCESS) st = upload_bias(p, d->bias_term ? bias : nullptr, C, C);
  if (st != NHIP_STATUS_SUCCESS) {
    std::string msg = g_last_error;
    free_plan(p);
    return fail(st, msg);
  }
  *plan = p;
  return ok();
}

int nhip_dwconv2d_int8_forward(nhip_conv_t p, const void* input, int32_t input_is_i8, void* output, int32_t n,
                               int32_t h, int32_t w, void* stream) {
  int oh = 0, ow = 0;
  NHIP_TRY(check_forward(p, input, output, n, h, w, &oh, &ow));
  if (p->kind != PlanKind::DwConvInt8)
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "dwconv2d_int8_forward: not an int8 depthwise plan");
  if (n == 0) return ok();
  return launch_dwconv_int8(p, input, input_is_i8 ? 1 : 0, output, n, h, w, oh, ow, as_stream(stream));
}

int nhip_conv_destroy(nhip_conv_t p) {
  free_plan(p);
  return ok();
}

int nhip_innerproduct_f32_create(int32_t num_output, int32_t num_input, const float* weight, const float* bias,
                                 int32_t activation_type, nhip_ip_t* plan) {
  if (!weight || !plan) return fail(NHIP_STATUS_NULL_POINTER, "innerproduct_create: null pointer");
  if (num_output <= 0 || num_input <= 0) return fail(NHIP_STATUS_INVALID_SHAPE, "innerproduct: sizes must be positive");
  if (activation_type != NHIP_ACT_NONE && activation_type != NHIP_ACT_RELU)
    return fail(NHIP_STATUS_UNSUPPORTED, "innerproduct activation must be 0 or 1");
  *plan = nullptr;
  auto* p = new nhip_ip_plan();
  p->n_out = num_output;
  p->k_in = num_input;
  p->act = activation_type;
  p->n_pad = (int)round_up(num_output, 64);
  p->k_pad = (int)round_up(num_input, 16);
  std::vector<float> wp((size_t)p->n_pad * p->k_pad, 0.f);
  for (int j = 0; j < num_output; ++j)
    std::copy(weight + (size_t)j * num_input, weight + (size_t)(j + 1) * num_input, wp.begin() + (size_t)j * p->k_pad);
  std::vector<float> bv((size_t)p->n_pad, 0.f);
  if (bias) std::copy(bias, bias + num_output, bv.begin());
  int st = upload(&p->weight, wp, "hipMalloc(ip weight)");
  if (st == NHIP_STATUS_SUCCESS) st = upload(&p->bias, bv, "hipMalloc(ip bias)");
  if (st == NHIP_STATUS_SUCCESS) st = ip_kq_prepack(p, weight);
  if (st != NHIP_STATUS_SUCCESS) {
    std::string msg = g_last_error;
    (void)hipFree(p->weight);
    (void)hipFree(p->bias);
    (void)hipFree(p->weight_kq);
    delete p;
    return fail(st, msg);
  }
  *plan = p;
  return ok();
}

int nhip_innerproduct_workspace_size(nhip_ip_t p, int32_t m, uint64_t* bytes) {
  if (!p || !bytes) return fail(NHIP_STATUS_NULL_POINTER, "innerproduct_workspace_size: null pointer");
  if (m < 0) return fail(NHIP_STATUS_INVALID_SHAPE, "innerproduct: negative m");
  if (p->q8) return nhip_conv2d_workspace_size(p->q8, m, 1, 1, bytes);
  *bytes = m == 0 ? 0 : innerproduct_workspace(p, m);
  return ok();
}

int nhip_innerproduct_int8_create(int32_t num_output, int32_t num_input, const void* weight, int32_t weight_is_i8,
                                  const float* bias, const float* weight_scale, float input_scale,
                                  int32_t activation_type, nhip_ip_t* plan) {
  if (!weight || !plan || !weight_scale) return fail(NHIP_STATUS_NULL_POINTER, "innerproduct_int8_create: null pointer");
  if (num_output <= 0 || num_input <= 0) return fail(NHIP_STATUS_INVALID_SHAPE, "innerproduct: sizes must be positive");
  if (activation_type != NHIP_ACT_NONE && activation_type != NHIP_ACT_RELU)
    return fail(NHIP_STATUS_UNSUPPORTED, "innerproduct activation must be 0 or 1");
  *plan = nullptr;
  // A 1x1 int8 convolution with fp32 output over m one-pixel "images" is
  // exactly the quantized matmul + dequantize + bias of the InnerProduct.
  nhip_conv_desc d{};
  d.input_channels = num_input;
  d.num_output = num_output;
  d.kernel_w = d.kernel_h = 1;
  d.dilation_w = d.dilation_h = 1;
  d.stride_w = d.stride_h = 1;
  d.bias_term = bias ? 1 : 0;
  d.int8_scale_term = 2;
  d.activation_type = activation_type;
  d.group = 1;
  nhip_conv_t c = nullptr;
  NHIP_TRY(nhip_conv2d_int8_create(&d, weight, weight_is_i8, bias, weight_scale, num_output, input_scale, 1.0f, &c));
  auto* p = new nhip_ip_plan();
  p->n_out = num_output;
  p->k_in = num_input;
  p->act = activation_type;
  p->q8 = c;
  *plan = p;
  return ok();
}

int nhip_innerproduct_int8_forward(nhip_ip_t p, const void* input, int32_t input_is_i8, float* output, int32_t m,
                                   void* workspace, uint64_t workspace_bytes, void* stream) {
  if (!p) return fail(NHIP_STATUS_NULL_POINTER, "innerproduct_int8_forward: null plan");
  if (!p->q8) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "innerproduct_int8_forward: not an int8 plan");
  if (m < 0) return fail(NHIP_STATUS_INVALID_SHAPE, "innerproduct: negative m");
  return nhip_conv2d_int8_forward(p->q8, input, input_is_i8, output, m, 1, 1, workspace, workspace_bytes, stream);
}

int nhip_innerproduct_f32_forward(nhip_ip_t p, const float* input, float* output, int32_t m, void* workspace,
                                  uint64_t workspace_bytes, void* stream) {
  if (!p) return fail(NHIP_STATUS_NULL_POINTER, "innerproduct_forward: null plan");
  if (p->q8) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "innerproduct_f32_forward: int8 plan");
  if (m < 0) return fail(NHIP_STATUS_INVALID_SHAPE, "innerproduct: negative m");
  if (m > 0 && (!input || !output)) return fail(NHIP_STATUS_NULL_POINTER, "innerproduct_forward: null pointer");
  if ((int64_t)m * std::max(p->k_in, p->n_pad) > std::numeric_limits<int32_t>::max())
    return fail(NHIP_STATUS_SHAPE_ARITHMETIC_OVERFLOW, "innerproduct: m too large");
  if (m == 0) return ok();
  return launch_innerproduct_f32(p, input, output, m, workspace, workspace_bytes, as_stream(stream));
}

int nhip_global_avgpool_innerproduct_f32_workspace_size(nhip_ip_t p, int32_t n, int32_t h, int32_t w,
                                                        uint64_t* bytes) {
  if (!p || !bytes) return fail(NHIP_STATUS_NULL_POINTER, "gap_innerproduct_workspace_size: null pointer");
  if (p->q8) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "gap_innerproduct: int8 plan");
  if (n < 0 || h <= 0 || w <= 0) return fail(NHIP_STATUS_INVALID_SHAPE, "gap_innerproduct: invalid shape");
  if ((int64_t)h * w > std::numeric_limits<int32_t>::max() || !gap_innerproduct_supported(h * w))
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "gap_innerproduct: planes of at most 6400 pixels");
  *bytes = n == 0 ? 0 : gap_innerproduct_workspace(p, n, h * w);
  return ok();
}

int nhip_global_avgpool_innerproduct_f32_forward(nhip_ip_t p, const float* input, float* output, int32_t n,
                                                 int32_t c, int32_t h, int32_t w, void* workspace,
                                                 uint64_t workspace_bytes, void* stream) {
  if (!p) return fail(NHIP_STATUS_NULL_POINTER, "gap_innerproduct_forward: null plan");
  if (p->q8) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "gap_innerproduct_forward: int8 plan");
  if (n < 0 || c <= 0 || h <= 0 || w <= 0) return fail(NHIP_STATUS_INVALID_SHAPE, "gap_innerproduct: invalid shape");
  if (c != p->k_in)
    return fail(NHIP_STATUS_INVALID_SHAPE, "gap_innerproduct: input has " + std::to_string(c) +
                                               " channels, weights expect " + std::to_string(p->k_in));
  if ((int64_t)n * c * h * w > std::numeric_limits<int32_t>::max() ||
      (int64_t)n * p->n_out > std::numeric_limits<int32_t>::max())
    return fail(NHIP_STATUS_SHAPE_ARITHMETIC_OVERFLOW, "gap_innerproduct: tensor too large");
  if (!gap_innerproduct_supported(h * w))
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "gap_innerproduct: planes of at most 6400 pixels");
  if (n == 0) return ok();
  if (!input || !output) return fail(NHIP_STATUS_NULL_POINTER, "gap_innerproduct_forward: null pointer");
  return launch_gap_innerproduct_f32(p, input, output, n, h * w, workspace, workspace_bytes, as_stream(stream));
}

int nhip_innerproduct_destroy(nhip_ip_t p) {
  if (p) {
    if (p->q8) free_plan(p->q8);
    (void)hipFree(p->weight);
    (void)hipFree(p->bias);
    (void)hipFree(p->weight_kq);
    delete p;
  }
  return ok();
}

}  // extern "C"
