// ncnn model execution on libnhip (include/nhip_graph.h): .param/.bin
// parsing, lowering of the layer graph to a call plan of nhip_* kernels, and
// the executor.  Host-only C++; every device operation goes through the
// public nhip_* C ABI.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <sstream>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/nhip_graph.h"

// Internal helpers of libnhip (csrc/runtime.hip): stream capture into a
// hipGraph and its replay, whether the kernel timer is recording, and the
// NHIP_* settings snapshot.
namespace nhip {
bool kernel_timer_active();
bool stream_capturing(void* stream);
int setting_int(const char* name, int fallback);
uint64_t settings_generation();
int graph_capture_begin(void* stream);
int graph_capture_end(void* stream, void** exec);
int graph_exec_launch(void* exec, void* stream);
void graph_exec_destroy(void* exec);
int device_current(int* dev);
int device_set(int dev);
void device_restore(int dev);
int stream_create(void** s);
void stream_destroy(void* s);
int host_pinned_alloc(void** p, uint64_t bytes);
void host_pinned_free(void* p);
}  // namespace nhip

namespace nhip {
int fail(int status, const std::string& message);  // runtime.hip
int ok();
}  // namespace nhip

namespace {

using nhip::fail;
using nhip::ok;

#define TRY(expr)                                \
  do {                                           \
    int _st = (expr);                            \
    if (_st != NHIP_STATUS_SUCCESS) return _st;  \
  } while (0)

// ---------------------------------------------------------------- model IR
struct Param {
  bool is_array = false;
  bool is_float = false;
  std::vector<int64_t> i;
  std::vector<float> f;
};

struct Tensor {
  int dtype = NHIP_DTYPE_F32;
  std::vector<float> f;
  std::vector<int8_t> q;
  size_t count() const { return dtype == NHIP_DTYPE_F32 ? f.size() : q.size(); }
};

struct Layer {
  std::string type, name;
  std::vector<std::string> bottoms, tops;
  std::map<int, Param> params;
  std::vector<Tensor> weights;
  bool removed = false;
  // lowering annotations
  int act = 0;                 // fused activation (NHIP_ACT_*)
  std::string residual;        // fused BinaryOp/Eltwise operand

  bool has(int id) const { return params.count(id) != 0; }
  int64_t geti(int id, int64_t def) const {
    auto it = params.find(id);
    if (it == params.end() || it->second.is_array) return def;
    return it->second.is_float ? (int64_t)it->second.f[0] : it->second.i[0];
  }
  float getf(int id, float def) const {
    auto it = params.find(id);
    if (it == params.end() || it->second.is_array) return def;
    return it->second.is_float ? it->second.f[0] : (float)it->second.i[0];
  }
  std::vector<int64_t> geta(int id) const {
    auto it = params.find(id);
    if (it == params.end() || !it->second.is_array) return {};
    if (!it->second.is_float) return it->second.i;
    std::vector<int64_t> r;
    for (float v : it->second.f) r.push_back((int64_t)v);
    return r;
  }
};

std::string where(const Layer& L) { return L.type + " '" + L.name + "': "; }

// ------------------------------------------------------------ .param parser
// Text format (lib/Graph/parser.cpp): magic 7767517, "layers blobs", then per
// layer "type name nbottom ntop bottoms... tops... id=value...".  Array
// parameters use id -(23300 + id) with value "count,v1,...".  A token with
// '.', 'e' or 'E' (or nan/inf) is a float.
bool token_is_float(const std::string& t) {
  std::string s = t;
  if (!s.empty() && (s[0] == '-' || s[0] == '+')) s = s.substr(1);
  std::string low;
  for (char c : s) low.push_back((char)std::tolower((unsigned char)c));
  if (low == "nan" || low == "inf" || low == "infinity") return true;
  return t.find_first_of(".eE") != std::string::npos;
}

int parse_number(const std::string& tok, bool as_float, int64_t* iv, float* fv) {
  try {
    size_t used = 0;
    if (as_float) {
      *fv = std::stof(tok, &used);
    } else {
      *iv = std::stoll(tok, &used);
    }
    if (used != tok.size()) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "bad number in .param: " + tok);
  } catch (...) {
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "bad number in .param: " + tok);
  }
  return ok();
}

int parse_param_text(const std::string& text, std::vector<Layer>& layers) {
  std::istringstream in(text);
  std::string line;
  auto next_line = [&](std::string& out) {
    while (std::getline(in, out)) {
      const auto p = out.find_first_not_of(" \t\r");
      if (p != std::string::npos) return true;
    }
    return false;
  };
  // Header (graph.cpp:2139-2170): the magic 7767517 on a line of its own,
  // or the legacy form with only the "layer_count blob_count" line.
  if (!next_line(line)) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, ".param: empty param file");
  {
    std::istringstream hs(line);
    std::vector<std::string> toks;
    std::string t;
    while (hs >> t) toks.push_back(t);
    if (toks.size() == 1) {
      int64_t magic = 0;
      if (parse_number(toks[0], false, &magic, nullptr) != NHIP_STATUS_SUCCESS || magic != 7767517)
        return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, ".param: magic mismatch (expected 7767517)");
      if (!next_line(line)) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, ".param: missing layer/blob count header");
    } else if (toks.size() != 2) {
      return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, ".param: bad magic / header line");
    }
  }
  int64_t layer_count = 0, blob_count = 0;
  {
    std::istringstream hs(line);
    std::string a, b, extra;
    if (!(hs >> a >> b) || (hs >> extra) || parse_number(a, false, &layer_count, nullptr) != NHIP_STATUS_SUCCESS ||
        parse_number(b, false, &blob_count, nullptr) != NHIP_STATUS_SUCCESS)
      return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, ".param: bad layer/blob count header");
    if (layer_count < 0 || blob_count < 0 || layer_count > (1 << 24) || blob_count > (1 << 24))
      return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, ".param: layer and blob counts must be non-negative");
  }
  std::map<std::string, int> producer;  // blob -> producing layer (declared blobs so far)
  while ((int64_t)layers.size() < layer_count && next_line(line)) {
    std::istringstream ls(line);
    Layer L;
    int64_t nb = 0, nt = 0;
    if (!(ls >> L.type >> L.name >> nb >> nt) || nb < 0 || nt < 0 || nb > 1024 || nt > 1024)
      return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, ".param: malformed layer line: " + line);
    for (int64_t i = 0; i < nb; ++i) {
      std::string b;
      if (!(ls >> b)) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, where(L) + "missing bottom blob");
      L.bottoms.push_back(b);
    }
    for (int64_t i = 0; i < nt; ++i) {
      std::string t;
      if (!(ls >> t)) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, where(L) + "missing top blob");
      L.tops.push_back(t);
    }
    std::string kv;
    while (ls >> kv) {
      const auto eq = kv.find('=');
      if (eq == std::string::npos || kv.find('=', eq + 1) != std::string::npos)
        return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, where(L) + "bad param " + kv);
      int64_t id = 0;
      TRY(parse_number(kv.substr(0, eq), false, &id, nullptr));
      const std::string val = kv.substr(eq + 1);
      Param P;
      if (id <= -23300) {
        id = -id - 23300;
        P.is_array = true;
        std::vector<std::string> toks;
        std::string t;
        std::istringstream vs(val);
        while (std::getline(vs, t, ',')) toks.push_back(t);
        if (toks.empty()) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, where(L) + "empty array param");
        int64_t n = 0;
        TRY(parse_number(toks[0], false, &n, nullptr));
        if (n != (int64_t)toks.size() - 1)
          return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, where(L) + "array param count mismatch");
        P.is_float = std::any_of(toks.begin() + 1, toks.end(), token_is_float);
        for (size_t k = 1; k < toks.size(); ++k) {
          int64_t iv = 0;
          float fv = 0.f;
          TRY(parse_number(toks[k], P.is_float, &iv, &fv));
          if (P.is_float) P.f.push_back(fv); else P.i.push_back(iv);
        }
      } else {
        if (id < 0 || id > 31) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, where(L) + "param id out of range");
        P.is_float = token_is_float(val);
        int64_t iv = 0;
        float fv = 0.f;
        TRY(parse_number(val, P.is_float, &iv, &fv));
        if (P.is_float) P.f.push_back(fv); else P.i.push_back(iv);
      }
      L.params[(int)id] = P;
    }
    // Blob bookkeeping (graph.cpp:2257-2282): bottoms are produced by an
    // earlier layer, every blob has one producer, and no more blobs are
    // created than the header declares.
    const int index = (int)layers.size();
    for (const std::string& b : L.bottoms)
      if (!producer.count(b))
        return fail(NHIP_STATUS_CONSTRAINT_VIOLATION,
                    "layer " + std::to_string(index) + " has unresolved bottom blob: " + b);
    for (const std::string& t : L.tops) {
      if (producer.count(t)) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "blob has multiple producers: " + t);
      if ((int64_t)producer.size() >= blob_count)
        return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, ".param: model creates more blobs than declared");
      producer[t] = index;
    }
    layers.push_back(std::move(L));
  }
  if ((int64_t)layers.size() != layer_count)
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, ".param: truncated before all layers were read");
  if (next_line(line)) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, ".param: contains trailing layer lines");
  return ok();
}

// -------------------------------------------------------------- .bin loader
// Tagged payloads (lib/Graph/graph.cpp:1260-1327): a u32 flag, 0 or
// 0x0002C056 = fp32, 0x01306B47 = fp16, 0x000D4B38 = int8; fp16/int8 data
// is padded to 4 bytes.  "Raw" payloads (type 1) are plain fp32.
constexpr uint32_t kFlagF32 = 0x0002C056, kFlagF16 = 0x01306B47, kFlagI8 = 0x000D4B38;

float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ff;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {  // subnormal: normalise
      int e = -1;
      do {
        ++e;
        man <<= 1;
      } while ((man & 0x400) == 0);
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ff) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

struct BinCursor {
  const uint8_t* data;
  size_t size, pos = 0;
  int read(void* dst, size_t n, const std::string& what) {
    if (n > size - pos) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, ".bin: truncated " + what);
    std::memcpy(dst, data + pos, n);
    pos += n;
    return ok();
  }
  // fp16 / int8 payloads are padded to 4 bytes; the padding must be present
  int align4(const std::string& what) {
    const size_t to = (pos + 3) & ~(size_t)3;
    if (to > size) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, ".bin: weight alignment padding missing after " + what);
    pos = to;
    return ok();
  }
};

int load_weight(BinCursor& c, int64_t count, bool tagged, Tensor& t, const std::string& what) {
  if (count <= 0 || count > (int64_t)1 << 31) return fail(NHIP_STATUS_INVALID_SHAPE, what + ": bad element count");
  uint32_t flag = 0;
  if (tagged) TRY(c.read(&flag, 4, what + " flag"));
  if (tagged && flag != 0 && flag != kFlagF32 && flag != kFlagF16 && flag != kFlagI8) {
    char buf[64];
    std::snprintf(buf, sizeof buf, " flag 0x%08x is unsupported", flag);
    return fail(NHIP_STATUS_UNSUPPORTED, what + buf);
  }
  // The payload must be present before anything is allocated for it (a
  // count taken from a hostile .param cannot force a large allocation).
  const uint64_t esz = (!tagged || flag == 0 || flag == kFlagF32) ? 4 : flag == kFlagF16 ? 2 : 1;
  if ((uint64_t)count * esz > (uint64_t)(c.size - c.pos))
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, ".bin: truncated " + what);
  if (!tagged || flag == 0 || flag == kFlagF32) {
    t.dtype = NHIP_DTYPE_F32;
    t.f.resize((size_t)count);
    return c.read(t.f.data(), (size_t)count * 4, what);
  }
  if (flag == kFlagF16) {
    std::vector<uint16_t> h((size_t)count);
    TRY(c.read(h.data(), (size_t)count * 2, what));
    TRY(c.align4(what));
    t.dtype = NHIP_DTYPE_F32;  // fp16 storage is promoted, as the importer does
    t.f.resize((size_t)count);
    for (size_t i = 0; i < h.size(); ++i) t.f[i] = half_to_float(h[i]);
    return ok();
  }
  if (flag == kFlagI8) {
    t.dtype = NHIP_DTYPE_I8;
    t.q.resize((size_t)count);
    TRY(c.read(t.q.data(), (size_t)count, what));
    TRY(c.align4(what));
    return ok();
  }
  char buf[64];
  std::snprintf(buf, sizeof buf, " flag 0x%08x is unsupported", flag);
  return fail(NHIP_STATUS_UNSUPPORTED, what + buf);
}

// Parameter rules applied before any .bin read: decode_convolution_params
// and its depthwise twin (graph.cpp:219-397) and decode_inner_product_params
// (:486-515).  Extents are also bounded so that the shape arithmetic below
// cannot overflow.
int check_layer_params(const Layer& L) {
  const std::string& ty = L.type;
  constexpr int64_t kMaxExtent = 1 << 16, kMaxCount = (int64_t)1 << 31;
  auto bad = [&](const std::string& m) { return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, where(L) + m); };
  if (ty == "Convolution" || ty == "ConvolutionDepthWise") {
    const int64_t k = L.geti(0, 0), kw = L.geti(1, 0), kh = L.geti(11, kw), dw = L.geti(2, 1), dh = L.geti(12, dw),
                  sw = L.geti(3, 1), sh = L.geti(13, sw), wsize = L.geti(6, 0), bias = L.geti(5, 0),
                  term = L.geti(8, 0);
    if (k <= 0 || k > kMaxCount) return bad("convolution num_output must be positive");
    if (wsize <= 0 || wsize > kMaxCount) return bad("convolution weight count must be positive");
    if (kw <= 0 || kh <= 0 || kw > kMaxExtent || kh > kMaxExtent) return bad("convolution kernel dimensions must be positive");
    if (dw <= 0 || dh <= 0 || dw > kMaxExtent || dh > kMaxExtent) return bad("convolution dilation must be positive");
    if (sw <= 0 || sh <= 0 || sw > kMaxExtent || sh > kMaxExtent) return bad("convolution stride must be positive");
    for (int id : {4, 14, 15, 16}) {
      const int64_t v = L.geti(id, 0);
      if (v > kMaxExtent || (v < 0 && v != -233 && v != -234)) return bad("convolution padding out of range");
    }
    if (bias != 0 && bias != 1) return bad("convolution bias_term must be 0 or 1");
    if (term != 0 && term != 1 && term != 2 && term != 101 && term != 102)
      return bad("convolution int8_scale_term must be 0, 1, 2, 101, or 102");
    if (ty == "Convolution") {
      if (wsize % (k * kh * kw) != 0) return bad("convolution weight count is not divisible by num_output*kernel_h*kernel_w");
    } else {
      const int64_t group = L.geti(7, 1);
      if (group <= 0 || group > kMaxCount || wsize % group != 0)
        return bad("convolution depthwise group must be positive and divide the weight count");
    }
  } else if (ty == "InnerProduct") {
    const int64_t n = L.geti(0, 0), wsize = L.geti(2, 0), bias = L.geti(1, 0), term = L.geti(8, 0);
    if (n <= 0 || n > kMaxCount) return bad("inner product num_output must be positive");
    if (wsize <= 0 || wsize > kMaxCount || wsize % n != 0)
      return bad("inner product weight count must be positive and divisible by num_output");
    if (bias != 0 && bias != 1) return bad("inner product bias_term must be 0 or 1");
    if (term != 0 && term != 1 && term != 2) return bad("inner product int8_scale_term must be 0, 1, or 2");
  } else if (ty == "Input") {
    for (int id : {0, 1, 2})
      if (L.geti(id, 0) > kMaxCount || L.geti(id, 0) < -1) return bad("Input extent out of range");
  }
  return ok();
}

int load_layer_weights(Layer& L, BinCursor& c) {
  TRY(check_layer_params(L));
  auto add = [&](int64_t count, bool tagged, const char* what) {
    Tensor t;
    TRY(load_weight(c, count, tagged, t, where(L) + what));
    L.weights.push_back(std::move(t));
    return ok();
  };
  const std::string& ty = L.type;
  if (ty == "Convolution" || ty == "ConvolutionDepthWise") {
    if (L.geti(19, 0) != 0) return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "dynamic weights are unsupported");
    const int64_t k = L.geti(0, 0), term = L.geti(8, 0);
    TRY(add(L.geti(6, 0), true, "weight"));
    if (L.geti(5, 0)) TRY(add(k, false, "bias"));
    if (term != 0) {
      const int64_t scales = ty == "Convolution" ? k : ((term == 1 || term == 101) ? L.geti(7, 1) : 1);
      TRY(add(scales, false, "weight int8 scales"));
      TRY(add(1, false, "bottom int8 scale"));
    }
    if (term > 100) TRY(add(1, false, "top int8 scale"));
  } else if (ty == "InnerProduct") {
    TRY(add(L.geti(2, 0), true, "weight"));
    if (L.geti(1, 0)) TRY(add(L.geti(0, 0), false, "bias"));
    if (L.geti(8, 0) != 0) {
      TRY(add(L.geti(0, 0), false, "weight int8 scales"));
      TRY(add(1, false, "bottom int8 scale"));
    }
  } else if (ty == "BatchNorm") {
    for (const char* w : {"slope", "mean", "variance", "bias"}) TRY(add(L.geti(0, 0), false, w));
  } else if (ty == "Quantize") {
    // decode_quantize_params / load_quantize_weights (graph.cpp:748-756,1960-1973)
    if (L.geti(0, 1) <= 0) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, where(L) + "Quantize scale count must be positive");
    TRY(add(L.geti(0, 1), false, "scale"));
  } else if (ty == "Dequantize") {
    // decode_dequantize_params / load_dequantize_weights (graph.cpp:758-770,1975-1996)
    const int64_t scales = L.geti(0, 1), bias = L.geti(1, 0);
    if (scales <= 0 || bias < 0)
      return fail(NHIP_STATUS_CONSTRAINT_VIOLATION,
                  where(L) + "Dequantize scale count must be positive and bias count non-negative");
    TRY(add(scales, false, "Dequantize scale"));
    if (bias != 0) TRY(add(bias, false, "Dequantize bias"));
  } else if (ty == "Requantize") {
    // decode_requantize_params / load_requantize_weights (graph.cpp:772-790,1998-2022)
    const int64_t in = L.geti(0, 1), out = L.geti(1, 1), bias = L.geti(2, 0), act = L.geti(3, 0);
    if (in <= 0 || out <= 0 || bias < 0 || act < 0 || act > 6)
      return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, where(L) + "invalid Requantize scale, bias, or activation");
    TRY(add(in, false, "Requantize input scale"));
    TRY(add(out, false, "Requantize output scale"));
    if (bias != 0) TRY(add(bias, false, "Requantize bias"));
  } else if (ty == "PReLU" || ty == "Gemm" || ty == "MemoryData" ||
             ty == "Deconvolution" || ty == "LayerNorm" || ty == "Embed" || ty == "MultiHeadAttention") {
    return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "layer type is not on this runtime's path");
  }
  return ok();
}

// -------------------------------------------------------------- lowering
struct Use {
  std::map<std::string, int> producer;                // blob -> layer index
  std::map<std::string, std::vector<int>> consumers;  // blob -> layer indices
};

Use uses(const std::vector<Layer>& layers) {
  Use u;
  for (int i = 0; i < (int)layers.size(); ++i) {
    if (layers[i].removed) continue;
    for (auto& t : layers[i].tops) u.producer[t] = i;
    for (auto& b : layers[i].bottoms) u.consumers[b].push_back(i);
    if (!layers[i].residual.empty()) u.consumers[layers[i].residual].push_back(i);
  }
  return u;
}

bool is_fp32_conv(const Layer& L) {
  return (L.type == "Convolution" || L.type == "ConvolutionDepthWise") && L.geti(8, 0) == 0;
}

// fold-ncnn-batchnorm (FoldNCNNBatchNorm.cpp:56-177): a constant BatchNorm
// whose input comes from a single-use fp32 (depthwise) convolution without
// a fused activation is folded into its weights and bias:
//   v = var + eps; k = v == 0 ? 1e4 : pow(v, -0.5); scale = slope * k;
//   W' = W * scale[o]; b' = b * scale + (beta - scale * mean).
void fold_batchnorm(std::vector<Layer>& layers) {
  for (int i = 0; i < (int)layers.size(); ++i) {
    Layer& bn = layers[i];
    if (bn.removed || bn.type != "BatchNorm" || bn.bottoms.size() != 1 || bn.tops.size() != 1) continue;
    const Use u = uses(layers);
    auto pit = u.producer.find(bn.bottoms[0]);
    if (pit == u.producer.end()) continue;
    Layer& cv = layers[pit->second];
    if (!is_fp32_conv(cv) || cv.geti(9, 0) != 0 || cv.act != 0 || !cv.residual.empty() ||
        u.consumers.at(bn.bottoms[0]).size() != 1)
      continue;
    const int64_t k = cv.geti(0, 0);
    if ((int64_t)bn.weights[0].f.size() != k || cv.weights.empty() || cv.weights[0].dtype != NHIP_DTYPE_F32) continue;
    const float eps = bn.getf(1, 0.f);
    const auto &slope = bn.weights[0].f, &mean = bn.weights[1].f, &var = bn.weights[2].f, &beta = bn.weights[3].f;
    bool finite = true;
    for (int64_t o = 0; o < k; ++o) {
      const float v = var[o] + eps;
      const float inv = v == 0.0f ? 10000.0f : std::pow(v, -0.5f);
      if (!std::isfinite(inv)) finite = false;
    }
    if (!finite) continue;
    std::vector<float>& w = cv.weights[0].f;
    const int64_t per = (int64_t)w.size() / k;
    std::vector<float> bias((size_t)k, 0.f);
    const bool has_bias = cv.geti(5, 0) != 0;
    for (int64_t o = 0; o < k; ++o) {
      const float v = var[o] + eps;
      const float inv = v == 0.0f ? 10000.0f : std::pow(v, -0.5f);
      const float scale = slope[o] * inv;
      const float sm = scale * mean[o];
      const float offset = beta[o] - sm;
      for (int64_t e = 0; e < per; ++e) w[o * per + e] = w[o * per + e] * scale;
      if (has_bias) {
        const float bs = cv.weights[1].f[o] * scale;
        bias[o] = bs + offset;
      } else {
        bias[o] = offset;
      }
    }
    if (has_bias) {
      cv.weights[1].f = bias;
    } else {
      Tensor t;
      t.f = bias;
      cv.weights.insert(cv.weights.begin() + 1, std::move(t));
      cv.params[5].is_array = false;
      cv.params[5].is_float = false;
      cv.params[5].i = {1};
      cv.params[5].f.clear();
    }
    cv.tops[0] = bn.tops[0];
    bn.removed = true;
  }
}

// A BinaryOp add / Eltwise sum of an fp32 Convolution's single-use output
// (no activation yet) and a blob computed earlier becomes that convolution's
// residual operand: out = conv + bias + other, in the reference's order.
void fuse_residual(std::vector<Layer>& layers) {
  for (int i = 0; i < (int)layers.size(); ++i) {
    Layer& add = layers[i];
    if (add.removed || add.bottoms.size() != 2 || add.tops.size() != 1) continue;
    const bool is_add = (add.type == "BinaryOp" && add.geti(0, 0) == 0 && add.geti(1, 0) == 0) ||
                        (add.type == "Eltwise" && add.geti(0, 1) == 1 && add.geta(1).empty());
    if (!is_add || add.bottoms[0] == add.bottoms[1]) continue;
    const Use u = uses(layers);
    for (int side = 1; side >= 0; --side) {
      const std::string& mine = add.bottoms[side];
      const std::string& other = add.bottoms[1 - side];
      auto p = u.producer.find(mine);
      auto q = u.producer.find(other);
      if (p == u.producer.end() || q == u.producer.end()) continue;
      Layer& cv = layers[p->second];
      if (cv.type != "Convolution" || cv.geti(8, 0) != 0 || cv.geti(9, 0) != 0 || cv.act != 0 ||
          !cv.residual.empty() || u.consumers.at(mine).size() != 1 || q->second >= p->second)
        continue;
      cv.residual = other;
      cv.tops[0] = add.tops[0];
      add.removed = true;
      break;
    }
  }
}

// The importer's fused activation (ImportConvolution.cpp:236-248) and a
// standalone ReLU (slope 0) on a single-use fp32 conv / depthwise /
// InnerProduct output both become the producer's epilogue activation.
void fuse_relu(std::vector<Layer>& layers) {
  for (auto& L : layers)
    if (!L.removed && (L.type == "Convolution" || L.type == "ConvolutionDepthWise" || L.type == "InnerProduct"))
      if (L.act == 0) L.act = (int)L.geti(9, 0);
  for (int i = 0; i < (int)layers.size(); ++i) {
    Layer& r = layers[i];
    if (r.removed || r.type != "ReLU" || r.getf(0, 0.f) != 0.f || r.bottoms.size() != 1) continue;
    const Use u = uses(layers);
    auto p = u.producer.find(r.bottoms[0]);
    if (p == u.producer.end()) continue;
    Layer& src = layers[p->second];
    const bool can = (is_fp32_conv(src) || (src.type == "InnerProduct" && src.geti(8, 0) == 0)) && src.act == 0 &&
                     u.consumers.at(r.bottoms[0]).size() == 1;
    if (!can) continue;
    src.act = NHIP_ACT_RELU;
    src.tops[0] = r.tops[0];
    r.removed = true;
  }
}

// ------------------------------------------------------------- call plan
enum class OpKind {
  Input, ConvF32, ConvInt8, DwF32, DwInt8, IP, IPInt8, Relu, Add, Gap, Quantize, Dequantize, Requantize, Alias
};

struct Shape {
  int rank = 0;
  int64_t d[4] = {0, 0, 0, 0};
  // -1 when an extent is dynamic; saturates at INT64_MAX instead of
  // overflowing (the shape checks then reject it)
  int64_t elems() const {
    int64_t e = 1;
    for (int i = 0; i < rank; ++i) {
      if (d[i] < 0) return -1;
      if (__builtin_mul_overflow(e, d[i], &e)) return INT64_MAX;
    }
    return e;
  }
};

struct Op {
  OpKind kind = OpKind::Alias;
  std::string name;
  std::vector<int> in;  // blob ids
  int out = -1;
  int residual = -1;
  nhip_conv_desc desc{};
  nhip_conv_t conv = nullptr;
  nhip_ip_t ip = nullptr;
  int64_t ip_k = 0, ip_n = 0;
  // Quantize: scale; Dequantize: scale (+ bias); Requantize: input scale,
  // output scale (+ bias).  Device copies, counts 1 or the channel extent.
  float* scale_dev = nullptr;
  int32_t scale_count = 0;
  float* scale2_dev = nullptr;
  int32_t scale2_count = 0;
  float* bias_dev = nullptr;
  int32_t bias_count = 0;
  int32_t quant_act = 0;
  int out_dtype = NHIP_DTYPE_F32;
  // Alias view rules
  enum class View { Same, Flatten, Reshape, Squeeze } view = View::Same;
  std::vector<int64_t> reshape;  // (w, h, c) targets, -1 infer, 0 absent
  std::vector<int64_t> squeeze_axes;
  // Depthwise -> 1x1 fusion (nhip_dwconv2d_pw_f32_*), and global average
  // pooling -> InnerProduct (nhip_global_avgpool_innerproduct_f32_*): on
  // the first op, the index of the op that is its output's only consumer;
  // on that op, the first op's index.
  int fuse_into = -1, fuse_from = -1;
  // a 1x1 convolution whose only consumer is a depthwise op: that op's index
  // (the pair may run as one kernel, decided at run time)
  int pwdw_dw = -1;
};

struct Blob {
  std::string name;
  int dtype = NHIP_DTYPE_F32;
  Shape declared;     // from load-time propagation (-1 = dynamic)
  int alias_of = -1;  // view of another blob's memory
  void* buf = nullptr;
  uint64_t cap = 0;   // bytes
};

}  // namespace

struct nhip_graph {
  std::vector<Blob> blobs;
  std::vector<Op> ops;
  std::vector<int> inputs, outputs;
  void* ws = nullptr;
  uint64_t ws_cap = 0;
  // nhip_graph_run_host: device copies of one image's inputs and outputs,
  // pinned host staging for them, and the graph's own stream
  std::vector<void*> host_in;
  std::vector<uint64_t> host_in_cap;
  std::vector<void*> pinned;
  std::vector<uint64_t> pinned_cap;
  void* host_stream = nullptr;
  int device = 0;  // the device the plans were uploaded to (current at load)
  std::mutex mu;
  bool host_only = false;  // from nhip_graph_describe: no device plans
  // The last call plan recorded as a hipGraph (nhip_graph_run on a stream),
  // valid for calls with the same key: batch, input shapes, input and output
  // pointers and NHIP_* settings (the buffers it uses stay allocated).
  void* exec = nullptr;
  std::string exec_key;
  std::vector<const void*> exec_bufs;  // the internal buffers the recorded plan uses
  std::string seen_key;   // the previous call's key: a plan is recorded on its second call
  std::string nocap_key;  // a key whose capture failed: runs eagerly
  // Once a call has run inside a caller's stream capture, the caller's graph
  // may still reference the blob buffers and workspace of that call: buffers
  // superseded by a later, larger call are kept here until destroy instead
  // of being freed.
  bool caller_captured = false;
  std::vector<void*> retired;
  ~nhip_graph() {
    nhip::graph_exec_destroy(exec);
    for (void* p : retired) nhip_free(p);
    for (auto& op : ops) {
      if (op.conv) nhip_conv_destroy(op.conv);
      if (op.ip) nhip_innerproduct_destroy(op.ip);
      if (op.scale_dev) nhip_free(op.scale_dev);
      if (op.scale2_dev) nhip_free(op.scale2_dev);
      if (op.bias_dev) nhip_free(op.bias_dev);
    }
    for (auto& b : blobs)
      if (b.buf) nhip_free(b.buf);
    if (ws) nhip_free(ws);
    for (void* p : host_in)
      if (p) nhip_free(p);
    for (void* p : pinned) nhip::host_pinned_free(p);
    nhip::stream_destroy(host_stream);
  }
};

namespace {

// Candidates for the depthwise -> 1x1 fusion: an fp32 depthwise op whose
// output blob is read by exactly one op, an fp32 convolution taking it as its
// main input (not as a residual), and is no graph output.  Whether the pair's
// shapes have a fused kernel is asked at run time.
void mark_dw_pw_pairs(nhip_graph& g) {
  std::vector<int> uses(g.blobs.size(), 0);
  for (const Op& op : g.ops) {
    for (int b : op.in) ++uses[b];
    if (op.residual >= 0) ++uses[op.residual];
  }
  for (int b : g.outputs) ++uses[b];
  for (size_t i = 0; i < g.ops.size(); ++i) {
    Op& d = g.ops[i];
    if (d.kind != OpKind::DwF32 || uses[d.out] != 1) continue;
    for (size_t j = i + 1; j < g.ops.size(); ++j) {
      Op& c = g.ops[j];
      if (c.kind == OpKind::ConvF32 && !c.in.empty() && c.in[0] == d.out && c.residual != d.out) {
        d.fuse_into = (int)j;
        c.fuse_from = (int)i;
        break;
      }
    }
  }
}

// Candidates for the 1x1 -> depthwise fusion (an inverted-residual block's
// expand and depthwise): an fp32 convolution without residual, not itself the
// consumer of a depthwise fusion, whose output blob is read by exactly one op,
// a depthwise op taking it as input, and is no graph output.  Whether the
// pair's shapes have a fused kernel is asked at run time.
void mark_pw_dw_pairs(nhip_graph& g) {
  std::vector<int> uses(g.blobs.size(), 0);
  std::vector<int> consumer(g.blobs.size(), -1);
  for (size_t j = 0; j < g.ops.size(); ++j) {
    for (int b : g.ops[j].in) {
      ++uses[b];
      consumer[b] = (int)j;
    }
    if (g.ops[j].residual >= 0) ++uses[g.ops[j].residual];
  }
  for (int b : g.outputs) ++uses[b];
  for (size_t i = 0; i < g.ops.size(); ++i) {
    Op& c = g.ops[i];
    if (c.kind != OpKind::ConvF32 || c.residual >= 0 || c.fuse_from >= 0 || uses[c.out] != 1 || consumer[c.out] < 0)
      continue;
    const Op& d = g.ops[consumer[c.out]];
    if (d.kind == OpKind::DwF32 && d.in.size() == 1 && d.in[0] == c.out) c.pwdw_dw = consumer[c.out];
  }
}

// Global average pooling whose output reaches exactly one fp32
// InnerProduct, directly or through at most two views (Flatten, Reshape,
// Squeeze), and is no graph output: the pair runs as one fused launch.
void mark_gap_ip_pairs(nhip_graph& g) {
  std::vector<int> uses(g.blobs.size(), 0);
  std::vector<int> consumer(g.blobs.size(), -1);
  for (size_t j = 0; j < g.ops.size(); ++j) {
    for (int b : g.ops[j].in) {
      ++uses[b];
      consumer[b] = (int)j;
    }
    if (g.ops[j].residual >= 0) ++uses[g.ops[j].residual];
  }
  for (int b : g.outputs) ++uses[b];
  for (size_t i = 0; i < g.ops.size(); ++i) {
    Op& gap = g.ops[i];
    if (gap.kind != OpKind::Gap || g.blobs[gap.in[0]].dtype != NHIP_DTYPE_F32) continue;
    int b = gap.out;
    for (int hop = 0; hop < 3 && b >= 0; ++hop) {
      if (uses[b] != 1 || consumer[b] < 0) break;
      Op& c = g.ops[consumer[b]];
      if (c.kind == OpKind::IP && c.in.size() == 1 && c.in[0] == b) {
        gap.fuse_into = consumer[b];
        c.fuse_from = (int)i;
        break;
      }
      if (c.kind != OpKind::Alias || c.in.size() != 1) break;
      b = c.out;
    }
  }
}

int64_t out_extent(int64_t in, int64_t k, int64_t s, int64_t d, int64_t pa, int64_t pb) {
  if (in < 0) return -1;
  const int64_t eff = (k - 1) * d + 1;
  const int64_t v = in + pa + pb - eff;
  return v < 0 ? 0 : v / s + 1;
}

// Shape of op's output from its input shapes; dims of -1 propagate.
int infer_op(const nhip_graph& g, const Op& op, const std::vector<Shape>& sh, Shape& out) {
  const Shape& a = sh[op.in.empty() ? 0 : op.in[0]];
  switch (op.kind) {
    case OpKind::ConvF32:
    case OpKind::ConvInt8:
    case OpKind::DwF32:
    case OpKind::DwInt8: {
      if (a.rank != 3) return fail(NHIP_STATUS_INVALID_SHAPE, op.name + ": convolution needs a [C,H,W] input");
      if (a.d[0] != op.desc.input_channels)
        return fail(NHIP_STATUS_INVALID_SHAPE, op.name + ": input has " + std::to_string(a.d[0]) +
                                                   " channels, weights expect " + std::to_string(op.desc.input_channels));
      const nhip_conv_desc& d = op.desc;
      out.rank = 3;
      out.d[0] = d.num_output;
      out.d[1] = out_extent(a.d[1], d.kernel_h, d.stride_h, d.dilation_h, d.pad_top, d.pad_bottom);
      out.d[2] = out_extent(a.d[2], d.kernel_w, d.stride_w, d.dilation_w, d.pad_left, d.pad_right);
      if (out.d[1] == 0 || out.d[2] == 0)
        return fail(NHIP_STATUS_INVALID_SHAPE, op.name + ": input smaller than the kernel extent");
      if (op.residual >= 0) {
        const Shape& r = sh[op.residual];
        if (r.rank != 3 || r.d[0] != out.d[0] || (r.d[1] >= 0 && out.d[1] >= 0 && (r.d[1] != out.d[1] || r.d[2] != out.d[2])))
          return fail(NHIP_STATUS_INVALID_SHAPE, op.name + ": residual operand shape differs from the output");
      }
      return ok();
    }
    case OpKind::IP:
    case OpKind::IPInt8: {
      int64_t k = 0;
      if (a.rank == 2) {
        k = a.d[1];
        out.rank = 2;
        out.d[0] = a.d[0];
        out.d[1] = op.ip_n;
      } else {
        k = a.elems();
        for (int i = 0; i < a.rank; ++i)
          if (a.d[i] < 0) k = -1;
        out.rank = 1;
        out.d[0] = op.ip_n;
      }
      if (k >= 0 && k != op.ip_k)
        return fail(NHIP_STATUS_INVALID_SHAPE, op.name + ": input has " + std::to_string(k) + " features, weights expect " +
                                                   std::to_string(op.ip_k));
      return ok();
    }
    case OpKind::Relu:
      out = a;
      return ok();
    case OpKind::Quantize:
    case OpKind::Dequantize:
    case OpKind::Requantize: {
      // validateScale / validateOptionalBias (NCNNOps.cpp:1378-1416): a
      // count is one or the extent of dimension zero (the channel of a
      // [C,H,W] blob).
      for (int32_t cnt : {op.scale_count, op.scale2_count, op.bias_count})
        if (cnt > 1 && (a.rank == 0 || a.d[0] != cnt))
          return fail(NHIP_STATUS_INVALID_SHAPE,
                      op.name + ": scale and bias counts must be one or match dimension zero");
      out = a;
      return ok();
    }
    case OpKind::Add: {
      const Shape& b = sh[op.in[1]];
      if (a.rank != b.rank) return fail(NHIP_STATUS_INVALID_SHAPE, op.name + ": add operands differ in rank");
      for (int i = 0; i < a.rank; ++i)
        if (a.d[i] >= 0 && b.d[i] >= 0 && a.d[i] != b.d[i])
          return fail(NHIP_STATUS_INVALID_SHAPE, op.name + ": add operands differ in shape (broadcast is unsupported)");
      out = a;
      return ok();
    }
    case OpKind::Gap:
      if (a.rank != 3) return fail(NHIP_STATUS_INVALID_SHAPE, op.name + ": global pooling needs [C,H,W]");
      out.rank = 1;
      out.d[0] = a.d[0];
      return ok();
    case OpKind::Alias: {
      if (op.view == Op::View::Same) {
        out = a;
      } else if (op.view == Op::View::Flatten) {
        out.rank = 1;
        out.d[0] = a.elems();
        for (int i = 0; i < a.rank; ++i)
          if (a.d[i] < 0) out.d[0] = -1;
      } else if (op.view == Op::View::Squeeze) {
        out.rank = 0;
        for (int i = 0; i < a.rank; ++i) {
          const bool sq = std::find(op.squeeze_axes.begin(), op.squeeze_axes.end(), i) != op.squeeze_axes.end();
          if (sq) {
            if (a.d[i] > 1) return fail(NHIP_STATUS_INVALID_SHAPE, op.name + ": squeezed axis has extent > 1");
            continue;
          }
          out.d[out.rank++] = a.d[i];
        }
      } else {  // Reshape to (c, h, w) given as (w, h, c)
        std::vector<int64_t> dims;
        const int64_t w = op.reshape[0], h = op.reshape[1], c = op.reshape[2];
        if (c != 0) dims = {c, h, w};
        else if (h != 0) dims = {h, w};
        else dims = {w};
        int64_t known = 1, infer = -1;
        for (size_t i = 0; i < dims.size(); ++i) {
          if (dims[i] == -1) {
            if (infer >= 0) return fail(NHIP_STATUS_UNSUPPORTED, op.name + ": more than one inferred extent");
            infer = (int64_t)i;
          } else if (dims[i] <= 0 || dims[i] > ((int64_t)1 << 31)) {
            return fail(NHIP_STATUS_INVALID_SHAPE, op.name + ": reshape extents must be positive or -1");
          } else if (__builtin_mul_overflow(known, dims[i], &known)) {
            return fail(NHIP_STATUS_SHAPE_ARITHMETIC_OVERFLOW, op.name + ": reshape extents overflow");
          }
        }
        int64_t total = a.elems();
        for (int i = 0; i < a.rank; ++i)
          if (a.d[i] < 0) total = -1;
        if (infer >= 0 && total >= 0 && total % known != 0)
          return fail(NHIP_STATUS_INVALID_SHAPE, op.name + ": reshape extents do not divide the element count");
        if (infer >= 0) dims[(size_t)infer] = total < 0 ? -1 : total / known;
        else if (total >= 0 && total != known)
          return fail(NHIP_STATUS_INVALID_SHAPE, op.name + ": reshape changes the element count");
        out.rank = (int)dims.size();
        for (size_t i = 0; i < dims.size(); ++i) out.d[i] = dims[i];
      }
      return ok();
    }
    default:
      return fail(NHIP_STATUS_UNSUPPORTED, op.name + ": no shape rule");
  }
  (void)g;
}

int propagate(const nhip_graph& g, const int64_t* input_shapes, std::vector<Shape>& sh, bool concrete) {
  sh.assign(g.blobs.size(), Shape{});
  for (size_t i = 0; i < g.inputs.size(); ++i) {
    Shape s = g.blobs[g.inputs[i]].declared;
    if (input_shapes) {
      for (int k = 0; k < 3; ++k) {
        const int64_t v = input_shapes[3 * i + k];
        if (s.d[k] >= 0 && v != s.d[k])
          return fail(NHIP_STATUS_INVALID_SHAPE, "input " + std::to_string(i + 1) + " extent " + std::to_string(k) +
                                                     " must be " + std::to_string(s.d[k]));
        if (v <= 0) return fail(NHIP_STATUS_INVALID_SHAPE, "input extents must be positive");
        if (v > ((int64_t)1 << 31)) return fail(NHIP_STATUS_SHAPE_ARITHMETIC_OVERFLOW, "input extent too large");
        s.d[k] = v;
      }
    } else if (concrete) {
      for (int k = 0; k < s.rank; ++k)
        if (s.d[k] < 0) return fail(NHIP_STATUS_INVALID_SHAPE, "dynamic input extents need input_shapes");
    }
    sh[g.inputs[i]] = s;
  }
  for (const Op& op : g.ops) {
    if (op.kind == OpKind::Input) continue;
    Shape o;
    TRY(infer_op(g, op, sh, o));
    if (concrete) {
      const int64_t lim = (int64_t)1 << 40;
      int64_t e = 1;
      for (int i = 0; i < o.rank; ++i) {
        if (o.d[i] <= 0) return fail(NHIP_STATUS_INVALID_SHAPE, op.name + ": empty output");
        if (e > lim / o.d[i]) return fail(NHIP_STATUS_SHAPE_ARITHMETIC_OVERFLOW, op.name + ": output too large");
        e *= o.d[i];
      }
    }
    sh[op.out] = o;
  }
  return ok();
}

int upload_floats(const std::vector<float>& v, float** dev) {
  TRY(nhip_malloc(reinterpret_cast<void**>(dev), v.size() * sizeof(float)));
  TRY(nhip_memcpy_h2d(*dev, v.data(), v.size() * sizeof(float), nullptr));
  return nhip_stream_sync(nullptr);
}

nhip_conv_desc conv_desc_of(const Layer& L, int64_t c) {
  nhip_conv_desc d{};
  d.input_channels = (int32_t)c;
  d.num_output = (int32_t)L.geti(0, 0);
  d.kernel_w = (int32_t)L.geti(1, 0);
  d.kernel_h = (int32_t)L.geti(11, d.kernel_w);
  d.dilation_w = (int32_t)L.geti(2, 1);
  d.dilation_h = (int32_t)L.geti(12, d.dilation_w);
  d.stride_w = (int32_t)L.geti(3, 1);
  d.stride_h = (int32_t)L.geti(13, d.stride_w);
  d.pad_left = (int32_t)L.geti(4, 0);
  d.pad_right = (int32_t)L.geti(15, d.pad_left);
  d.pad_top = (int32_t)L.geti(14, d.pad_left);
  d.pad_bottom = (int32_t)L.geti(16, d.pad_top);
  d.bias_term = (int32_t)L.geti(5, 0);
  d.int8_scale_term = (int32_t)L.geti(8, 0);
  d.activation_type = L.act;
  d.group = L.type == "ConvolutionDepthWise" ? (int32_t)L.geti(7, 1) : 1;
  d.algorithm = NHIP_CONV_ALGO_AUTO;
  return d;
}

// SAME padding sentinels -233 / -234 (NormalizeNCNN.cpp:31-66), resolved for
// a known input extent.
int resolve_same(nhip_conv_desc& d, const Shape& in, const std::string& name) {
  auto same = [](int64_t input, int64_t k, int64_t s, int64_t dl, bool lower, int32_t* a, int32_t* b) {
    const int64_t extent = dl * (k - 1) + 1;
    const int64_t out = 1 + (input - 1) / s;
    const int64_t need = (out - 1) * s + extent;
    const int64_t total = need > input ? need - input : 0;
    const int64_t before = lower ? total / 2 + total % 2 : total / 2;
    *a = (int32_t)before;
    *b = (int32_t)(total - before);
  };
  const bool sh = d.pad_left == -233 || d.pad_left == -234;
  if (!sh) return ok();
  if (in.d[1] < 0 || in.d[2] < 0)
    return fail(NHIP_STATUS_UNSUPPORTED, name + ": SAME padding with a dynamic input extent");
  const bool lower = d.pad_left == -234;
  same(in.d[1], d.kernel_h, d.stride_h, d.dilation_h, lower, &d.pad_top, &d.pad_bottom);
  same(in.d[2], d.kernel_w, d.stride_w, d.dilation_w, lower, &d.pad_left, &d.pad_right);
  return ok();
}

// dry: lower and infer shapes only, creating no device plans (for the
// compiler and for output-shape queries on hosts without a GPU).
int build(nhip_graph& g, std::vector<Layer>& layers, const int64_t* input_shapes, int32_t input_shape_count,
          bool dry) {
  fold_batchnorm(layers);
  fuse_residual(layers);
  fuse_relu(layers);
  std::map<std::string, int> blob_id;
  auto blob = [&](const std::string& name) {
    auto it = blob_id.find(name);
    if (it != blob_id.end()) return it->second;
    Blob b;
    b.name = name;
    g.blobs.push_back(b);
    return blob_id[name] = (int)g.blobs.size() - 1;
  };
  // Integer input storage (NCNNImporter.cpp:370-376, ImportInput.cpp:78-80):
  // the reference gives an Input blob i32 elements when an Embed layer reads
  // it; Dequantize and Requantize need i32 operands
  // (NCNNOps.cpp:1434-1470), so an Input blob they read is i32 here as well
  // (the reference rejects such a graph at import, so no graph it accepts
  // changes meaning).
  std::set<std::string> integer_inputs;
  for (const Layer& L : layers)
    if (!L.removed && (L.type == "Embed" || L.type == "Dequantize" || L.type == "Requantize"))
      integer_inputs.insert(L.bottoms.begin(), L.bottoms.end());
  std::vector<Shape> sh;
  int next_input = 0;
  for (Layer& L : layers) {
    if (L.removed) continue;
    Op op;
    op.name = L.type + " '" + L.name + "'";
    for (auto& b : L.bottoms) {
      auto it = blob_id.find(b);
      if (it == blob_id.end()) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, where(L) + "unknown bottom blob " + b);
      op.in.push_back(it->second);
    }
    if (!L.residual.empty()) op.residual = blob_id.at(L.residual);
    const std::string& ty = L.type;
    auto in_shape = [&]() -> const Shape& { return sh[op.in[0]]; };
    if (ty == "Input") {
      if (L.tops.size() != 1) return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "one output per Input");
      const int id = blob(L.tops[0]);
      Shape s;
      s.rank = 3;
      s.d[0] = L.geti(2, 0);
      s.d[1] = L.geti(1, 0);
      s.d[2] = L.geti(0, 0);
      const bool omitted = s.d[0] == 0 && s.d[1] == 0 && s.d[2] == 0;
      if (input_shapes && next_input < input_shape_count) {
        for (int k = 0; k < 3; ++k) s.d[k] = input_shapes[3 * next_input + k];
      } else if (omitted) {
        return fail(NHIP_STATUS_INVALID_SHAPE, where(L) + "Input dimensions are omitted without an override");
      }
      for (int k = 0; k < 3; ++k)
        if (s.d[k] == 0 || s.d[k] < -1 || s.d[k] > ((int64_t)1 << 31))
          return fail(NHIP_STATUS_INVALID_SHAPE, where(L) + "Input requires positive or dynamic (-1) extents");
      ++next_input;
      if (integer_inputs.count(L.tops[0])) g.blobs[id].dtype = NHIP_DTYPE_I32;
      g.blobs[id].declared = s;
      g.inputs.push_back(id);
      if (sh.size() < g.blobs.size()) sh.resize(g.blobs.size());
      sh[id] = s;
      op.kind = OpKind::Input;
      op.out = id;
      g.ops.push_back(op);
      continue;
    }
    if (op.in.empty()) return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "layer without inputs");
    if (ty == "Convolution" || ty == "ConvolutionDepthWise") {
      if (L.bottoms.size() != 1 || L.tops.size() != 1) return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "one input and output");
      if (L.getf(18, 0.f) != 0.f || L.has(10)) return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "pad value / activation params");
      const Shape& a = in_shape();
      const int64_t k = L.geti(0, 0), kw = L.geti(1, 0), kh = L.geti(11, kw);
      if (k <= 0 || kw <= 0 || kh <= 0 || L.weights.empty())
        return fail(NHIP_STATUS_INVALID_SHAPE, where(L) + "bad num_output/kernel/weights");
      const int64_t c = ty == "Convolution" ? (int64_t)L.weights[0].count() / (k * kh * kw) : a.d[0];
      op.desc = conv_desc_of(L, c);
      TRY(resolve_same(op.desc, a, op.name));
      const int term = op.desc.int8_scale_term;
      const int input_i8 = g.blobs[op.in[0]].dtype == NHIP_DTYPE_I8;
      const float* bias = op.desc.bias_term ? L.weights[1].f.data() : nullptr;
      const size_t s0 = op.desc.bias_term ? 2 : 1;
      nhip_conv_desc d = op.desc;
      if (ty == "ConvolutionDepthWise" && term != 0) {
        if (L.act != 0 && L.act != NHIP_ACT_RELU) return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "int8 activation");
        const Tensor& ws = L.weights[s0];
        const float is = L.weights[s0 + 1].f[0];
        const float os = term > 100 ? L.weights[s0 + 2].f[0] : 1.0f;
        const bool wi8 = L.weights[0].dtype == NHIP_DTYPE_I8;
        if (!dry)
          TRY(nhip_dwconv2d_int8_create(&d, wi8 ? (const void*)L.weights[0].q.data() : (const void*)L.weights[0].f.data(),
                                        wi8 ? 1 : 0, bias, ws.f.data(), (int32_t)ws.f.size(), is, os, &op.conv));
        op.kind = OpKind::DwInt8;
        op.out_dtype = term > 100 ? NHIP_DTYPE_I8 : NHIP_DTYPE_F32;
      } else if (ty == "ConvolutionDepthWise") {
        if (L.weights[0].dtype != NHIP_DTYPE_F32) return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "int8 weights without scale term");
        if (input_i8) return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "int8 input to an fp32 depthwise convolution");
        if (!dry) TRY(nhip_dwconv2d_f32_create(&d, L.weights[0].f.data(), bias, &op.conv));
        op.kind = OpKind::DwF32;
      } else if (term == 0) {
        if (L.weights[0].dtype != NHIP_DTYPE_F32)
          return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, where(L) + "convolution kernel element type does not match scale term");
        if (input_i8) return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "int8 input to an fp32 convolution");
        if (op.residual >= 0 && g.blobs[op.residual].dtype != NHIP_DTYPE_F32)
          return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "int8 residual operand");
        if (!dry) TRY(nhip_conv2d_f32_create(&d, L.weights[0].f.data(), bias, &op.conv));
        op.kind = OpKind::ConvF32;
      } else {
        if (L.act != 0 && L.act != NHIP_ACT_RELU) return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "int8 activation");
        const Tensor& ws = L.weights[s0];
        const float is = L.weights[s0 + 1].f[0];
        const float os = term > 100 ? L.weights[s0 + 2].f[0] : 1.0f;
        const bool wi8 = L.weights[0].dtype == NHIP_DTYPE_I8;
        if (!dry)
          TRY(nhip_conv2d_int8_create(&d, wi8 ? (const void*)L.weights[0].q.data() : (const void*)L.weights[0].f.data(),
                                    wi8 ? 1 : 0, bias, ws.f.data(), (int32_t)ws.f.size(), is, os, &op.conv));
        op.kind = OpKind::ConvInt8;
        op.out_dtype = term > 100 ? NHIP_DTYPE_I8 : NHIP_DTYPE_F32;
      }
    } else if (ty == "InnerProduct") {
      const int64_t n = L.geti(0, 0), count = L.geti(2, 0);
      const bool q = L.geti(8, 0) != 0;
      if (n <= 0 || count <= 0 || count % n != 0 || L.weights.empty())
        return fail(NHIP_STATUS_INVALID_SHAPE, where(L) + "bad num_output / weight_data_size");
      if (L.act != 0 && L.act != NHIP_ACT_RELU) return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "activation");
      op.ip_n = n;
      op.ip_k = count / n;
      const bool has_bias = L.geti(1, 0) != 0;
      const float* bias = has_bias ? L.weights[1].f.data() : nullptr;
      if (q) {
        const size_t s0 = has_bias ? 2 : 1;
        const bool wi8 = L.weights[0].dtype == NHIP_DTYPE_I8;
        if (!dry)
          TRY(nhip_innerproduct_int8_create((int32_t)n, (int32_t)op.ip_k,
                                            wi8 ? (const void*)L.weights[0].q.data() : (const void*)L.weights[0].f.data(),
                                            wi8 ? 1 : 0, bias, L.weights[s0].f.data(), L.weights[s0 + 1].f[0], L.act,
                                            &op.ip));
        op.kind = OpKind::IPInt8;
      } else {
        if (g.blobs[op.in[0]].dtype != NHIP_DTYPE_F32) return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "int8 input");
        if (L.weights[0].dtype != NHIP_DTYPE_F32)
          return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, where(L) + "int8 weights without scale term");
        if (!dry) TRY(nhip_innerproduct_f32_create((int32_t)n, (int32_t)op.ip_k, L.weights[0].f.data(), bias, L.act, &op.ip));
        op.kind = OpKind::IP;
      }
    } else if (ty == "ReLU") {
      if (L.getf(0, 0.f) != 0.f) return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "leaky slope");
      op.kind = OpKind::Relu;
      op.out_dtype = g.blobs[op.in[0]].dtype;
    } else if (ty == "BinaryOp" || ty == "Eltwise") {
      const bool is_add = (ty == "BinaryOp" && L.geti(0, 0) == 0 && L.geti(1, 0) == 0) ||
                          (ty == "Eltwise" && L.geti(0, 1) == 1 && L.geta(1).empty());
      if (!is_add || op.in.size() != 2) return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "only two-operand add / sum");
      if (g.blobs[op.in[0]].dtype != NHIP_DTYPE_F32 || g.blobs[op.in[1]].dtype != NHIP_DTYPE_F32)
        return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "int8 operands");
      op.kind = OpKind::Add;
    } else if (ty == "Pooling") {
      if (L.geti(0, 0) != 1 || L.geti(4, 0) != 1)
        return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "only global average pooling is on this path");
      op.kind = OpKind::Gap;
    } else if (ty == "Quantize") {
      // import_quantize (ImportQuantization.cpp:37-62); computeQuantizeResult
      // (NCNNOps.cpp:1420-1432): an f32 input
      if (L.weights.size() != 1 || L.bottoms.size() != 1) return fail(NHIP_STATUS_INVALID_SHAPE, where(L) + "unexpected weight count");
      if (g.blobs[op.in[0]].dtype != NHIP_DTYPE_F32)
        return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, where(L) + "Quantize input must be ranked f32");
      if (!dry) TRY(upload_floats(L.weights[0].f, &op.scale_dev));
      op.scale_count = (int32_t)L.weights[0].f.size();
      op.kind = OpKind::Quantize;
      op.out_dtype = NHIP_DTYPE_I8;
    } else if (ty == "Dequantize" || ty == "Requantize") {
      // import_dequantize / import_requantize (ImportQuantization.cpp:65-161),
      // ConvertDequantize / ConvertRequantize (NCNNToTosa.cpp:4823-4888):
      // an i32 input; Dequantize scale [+ bias] -> f32; Requantize input
      // scale, output scale [+ bias], activation none or ReLU -> i8.
      const bool deq = ty == "Dequantize";
      if (L.bottoms.size() != 1) return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "one input");
      if (g.blobs[op.in[0]].dtype != NHIP_DTYPE_I32)
        return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, where(L) + ty + " input must be ranked i32");
      if (!deq) {
        const int64_t act = L.geti(3, 0);
        if (act != 0 && act != 1)
          return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "Requantize supports no activation or ReLU only");
        op.quant_act = (int32_t)act;
      }
      const size_t nscale = deq ? 1 : 2;
      op.scale_count = (int32_t)L.weights[0].f.size();
      if (!dry) TRY(upload_floats(L.weights[0].f, &op.scale_dev));
      if (!deq) {
        op.scale2_count = (int32_t)L.weights[1].f.size();
        if (!dry) TRY(upload_floats(L.weights[1].f, &op.scale2_dev));
      }
      if (L.weights.size() > nscale) {
        op.bias_count = (int32_t)L.weights[nscale].f.size();
        if (!dry) TRY(upload_floats(L.weights[nscale].f, &op.bias_dev));
      }
      op.kind = deq ? OpKind::Dequantize : OpKind::Requantize;
      op.out_dtype = deq ? NHIP_DTYPE_F32 : NHIP_DTYPE_I8;
    } else if (ty == "Split" || ty == "Dropout" || ty == "Noop") {
      op.kind = OpKind::Alias;
      op.view = Op::View::Same;
    } else if (ty == "Flatten") {
      op.kind = OpKind::Alias;
      op.view = Op::View::Flatten;
    } else if (ty == "Reshape") {
      op.kind = OpKind::Alias;
      op.view = Op::View::Reshape;
      op.reshape = {L.geti(0, -233), L.geti(1, 0), L.geti(2, 0)};
      if (L.geti(11, 0) != 0 || L.has(3)) return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "4-d or permuted reshape");
      if (op.reshape[0] == -233) op.reshape[0] = -1;
    } else if (ty == "Squeeze") {
      op.kind = OpKind::Alias;
      op.view = Op::View::Squeeze;
      op.squeeze_axes = L.geta(3);
      if (op.squeeze_axes.empty()) {  // flags 0=w 1=h 2=c on [C,H,W]
        if (L.geti(2, 0)) op.squeeze_axes.push_back(0);
        if (L.geti(1, 0)) op.squeeze_axes.push_back(1);
        if (L.geti(0, 0)) op.squeeze_axes.push_back(2);
      }
    } else {
      return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "layer type is not on this runtime's path");
    }
    if (op.kind != OpKind::Alias || op.view != Op::View::Same) {
      if (L.tops.size() != 1) return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "one output expected");
    }
    // i32 blobs (integer-storage inputs) are read only by the layers that
    // take accumulators, or viewed
    if (op.kind != OpKind::Dequantize && op.kind != OpKind::Requantize && op.kind != OpKind::Alias)
      for (int b : op.in)
        if (g.blobs[b].dtype == NHIP_DTYPE_I32)
          return fail(NHIP_STATUS_UNSUPPORTED, where(L) + "int32 operand (only Dequantize / Requantize read i32 blobs)");
    // outputs (Split fans its input out to several aliases of it, so that
    // each top can also be a graph output)
    for (size_t t = 0; t < L.tops.size(); ++t) {
      Op o = op;
      o.out = blob(L.tops[t]);
      Blob& ob = g.blobs[o.out];
      ob.dtype = o.kind == OpKind::Alias ? g.blobs[o.in[0]].dtype : o.out_dtype;
      if (o.kind == OpKind::Alias) ob.alias_of = o.in[0];
      if (sh.size() < g.blobs.size()) sh.resize(g.blobs.size());
      Shape s;
      TRY(infer_op(g, o, sh, s));
      sh[o.out] = s;
      ob.declared = s;
      g.ops.push_back(o);
    }
  }
  // Graph outputs: blobs no remaining layer consumes (ncnn's convention).
  std::set<int> consumed;
  for (const Op& op : g.ops) {
    for (int b : op.in) consumed.insert(b);
    if (op.residual >= 0) consumed.insert(op.residual);
  }
  for (const Op& op : g.ops)
    if (op.kind != OpKind::Input && !consumed.count(op.out)) g.outputs.push_back(op.out);
  if (g.inputs.empty() || g.outputs.empty()) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "graph needs inputs and outputs");
  mark_dw_pw_pairs(g);
  mark_pw_dw_pairs(g);
  mark_gap_ip_pairs(g);
  return ok();
}

int esize(int dtype) { return dtype == NHIP_DTYPE_I8 ? 1 : 4; }  // f32 and i32: 4 bytes

int ensure(void** buf, uint64_t* cap, uint64_t bytes) {
  if (*cap >= bytes) return ok();
  if (*buf) TRY(nhip_free(*buf));
  *buf = nullptr;
  *cap = 0;
  TRY(nhip_malloc(buf, bytes));
  *cap = bytes;
  return ok();
}

// Grows a blob buffer or the workspace of the executor.  Inside a stream
// capture (the caller's or the executor's own recording) nothing may grow: a
// hipFree or hipMalloc there would invalidate the capture, so the call fails
// instead, naming the fix (run that batch and shape once before capturing).
// After a caller's capture has been seen, superseded buffers are retired,
// not freed, because the caller's graph may still replay over them.
int grow(nhip_graph& g, void** buf, uint64_t* cap, uint64_t bytes, bool capturing) {
  if (*cap >= bytes) return ok();
  if (capturing)
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION,
                "graph_run: the stream is being captured and the executor's buffers would have to grow to " +
                    std::to_string(bytes) + " bytes; run this batch size and these shapes once before capturing");
  if (*buf) {
    if (g.caller_captured) g.retired.push_back(*buf);
    else TRY(nhip_free(*buf));
  }
  *buf = nullptr;
  *cap = 0;
  TRY(nhip_malloc(buf, bytes));
  *cap = bytes;
  return ok();
}

// A marked pooling -> InnerProduct pair runs fused when the pooled planes
// fit nhip_global_avgpool_innerproduct_f32 (at most 6400 pixels).
bool gap_ip_fusable(const nhip_graph& g, const std::vector<Shape>& sh, const Op& ip) {
  if (ip.fuse_from < 0) return false;
  const Shape& a = sh[g.ops[ip.fuse_from].in[0]];
  return a.rank == 3 && a.d[1] > 0 && a.d[2] > 0 && a.d[1] * a.d[2] <= 6400;
}

int run_ops(nhip_graph& g, int n, const std::vector<Shape>& sh, const void* const* inputs, void* const* outputs,
            void* stream, bool capturing) {
  std::vector<char*> ptr(g.blobs.size(), nullptr);
  // device buffers for computed blobs; the graph's inputs are the caller's
  uint64_t ws_need = 0;
  for (const Op& op : g.ops) {
    if (op.kind == OpKind::Input || op.kind == OpKind::Alias) continue;
    Blob& b = g.blobs[op.out];
    TRY(grow(g, &b.buf, &b.cap, (uint64_t)n * sh[op.out].elems() * esize(b.dtype), capturing));
    const Shape& a = sh[op.in[0]];
    uint64_t w = 0;
    if (op.kind == OpKind::ConvF32 || op.kind == OpKind::ConvInt8)
      TRY(nhip_conv2d_workspace_size(op.conv, n, (int32_t)a.d[1], (int32_t)a.d[2], &w));
    else if (op.kind == OpKind::IP || op.kind == OpKind::IPInt8) {
      TRY(nhip_innerproduct_workspace_size(op.ip, (int32_t)(a.rank == 2 ? n * a.d[0] : n), &w));
      if (op.kind == OpKind::IP && gap_ip_fusable(g, sh, op)) {  // fused or not, as the switch says at run time
        const Shape& pa = sh[g.ops[op.fuse_from].in[0]];
        uint64_t wf = 0;
        TRY(nhip_global_avgpool_innerproduct_f32_workspace_size(op.ip, n, (int32_t)pa.d[1], (int32_t)pa.d[2], &wf));
        w = std::max(w, wf);
      }
    }
    ws_need = std::max(ws_need, w);
  }
  TRY(grow(g, &g.ws, &g.ws_cap, std::max<uint64_t>(ws_need, 256), capturing));
  for (size_t i = 0; i < g.inputs.size(); ++i) ptr[g.inputs[i]] = (char*)inputs[i];
  // Outputs written in place: a graph output computed by an op goes
  // straight into the caller's buffer (no copy after the last op) when that
  // buffer is 256-byte aligned (as the kernels' own buffers are) and overlaps
  // none of the graph's inputs (which later ops may still read).  Views and
  // pass-through inputs, and a blob listed twice after its first listing,
  // are copied as before.
  std::vector<char*> direct(g.blobs.size(), nullptr);
  std::vector<char> copied(g.outputs.size(), 1);
  {
    std::vector<char> computed(g.blobs.size(), 0);
    for (const Op& op : g.ops)
      if (op.kind != OpKind::Input && op.kind != OpKind::Alias) computed[op.out] = 1;
    for (size_t j = 0; j < g.outputs.size(); ++j) {
      const int b = g.outputs[j];
      char* o = static_cast<char*>(outputs[j]);
      const uint64_t ob = (uint64_t)n * sh[b].elems() * esize(g.blobs[b].dtype);
      bool ok = computed[b] && direct[b] == nullptr && (reinterpret_cast<uintptr_t>(o) & 255) == 0;
      for (size_t i = 0; ok && i < g.inputs.size(); ++i) {
        const int ib = g.inputs[i];
        const char* in = static_cast<const char*>(inputs[i]);
        const uint64_t inb = (uint64_t)n * sh[ib].elems() * esize(g.blobs[ib].dtype);
        if (o < in + inb && in < o + ob) ok = false;
      }
      if (ok) {
        direct[b] = o;
        copied[j] = 0;
      }
    }
  }
  auto out_buf = [&](int b) { return direct[b] ? direct[b] : (char*)g.blobs[b].buf; };
  std::vector<char> fused(g.ops.size(), 0);  // ops folded into their consumer
  // Pooling -> InnerProduct runs fused only with NHIP_GAP_IP=1.  Measured on
  // the MobileNetV2 head at batch 32 (1280@7x7 -> 1000): fused 13.5 us +
  // the split-K reduce against 4.0 us pooling + 9.8 us InnerProduct + 1.7 us
  // reduce unfused - pooling wants every CU on the 8 MB input, the GEMM an
  // output split, and one kernel gets either re-read planes or large split-K
  // partials.
  const bool gap_ip = nhip::setting_int("NHIP_GAP_IP", 0) != 0;
  std::vector<char> done(g.ops.size(), 0);  // depthwise ops run with their 1x1 producer
  for (size_t oi = 0; oi < g.ops.size(); ++oi) {
    const Op& op = g.ops[oi];
    if (op.kind == OpKind::Input || done[oi]) continue;
    if (op.kind == OpKind::ConvF32 && op.pwdw_dw >= 0) {
      // expand -> depthwise in one kernel where that kernel takes the pair
      // (its shape policy says where it is preferred); the depthwise's own
      // fusion into the 1x1 after it is then not used
      const Op& d = g.ops[op.pwdw_dw];
      const Shape& a = sh[op.in[0]];
      int32_t sup = 0;
      TRY(nhip_conv1x1_dw_f32_supported(op.conv, d.conv, n, (int32_t)a.d[1], (int32_t)a.d[2], &sup));
      if (sup) {
        ptr[d.out] = out_buf(d.out);
        TRY(nhip_conv1x1_dw_f32_forward(op.conv, d.conv, (const float*)ptr[op.in[0]], (float*)ptr[d.out], n,
                                        (int32_t)a.d[1], (int32_t)a.d[2], stream));
        done[op.pwdw_dw] = 1;
        continue;
      }
    }
    if (op.kind == OpKind::DwF32 && op.fuse_into >= 0) {
      const Shape& a = sh[op.in[0]];
      int32_t sup = 0;
      TRY(nhip_dwconv2d_pw_f32_supported(op.conv, g.ops[op.fuse_into].conv, n, (int32_t)a.d[1], (int32_t)a.d[2], &sup));
      if (sup) {
        fused[oi] = 1;
        continue;
      }
    }
    if (op.kind == OpKind::Gap && op.fuse_into >= 0 && gap_ip && gap_ip_fusable(g, sh, g.ops[op.fuse_into])) {
      // runs inside its InnerProduct
      fused[oi] = 1;
      continue;
    }
    if (op.kind == OpKind::IP && op.fuse_from >= 0 && fused[op.fuse_from]) {
      const Op& gp = g.ops[op.fuse_from];
      const Shape& a = sh[gp.in[0]];
      ptr[op.out] = out_buf(op.out);
      TRY(nhip_global_avgpool_innerproduct_f32_forward(op.ip, (const float*)ptr[gp.in[0]], (float*)ptr[op.out], n,
                                                       (int32_t)a.d[0], (int32_t)a.d[1], (int32_t)a.d[2], g.ws,
                                                       g.ws_cap, stream));
      continue;
    }
    if (op.kind == OpKind::ConvF32 && op.fuse_from >= 0 && fused[op.fuse_from]) {
      const Op& d = g.ops[op.fuse_from];
      const Shape& a = sh[d.in[0]];
      ptr[op.out] = out_buf(op.out);
      TRY(nhip_dwconv2d_pw_f32_forward(d.conv, op.conv, (const float*)ptr[d.in[0]],
                                       op.residual >= 0 ? (const float*)ptr[op.residual] : nullptr,
                                       (float*)ptr[op.out], n, (int32_t)a.d[1], (int32_t)a.d[2], stream));
      continue;
    }
    if (op.kind == OpKind::Alias) {
      ptr[op.out] = ptr[op.in[0]];
      continue;
    }
    ptr[op.out] = out_buf(op.out);
    const Shape& a = sh[op.in[0]];
    char* in = ptr[op.in[0]];
    char* out = ptr[op.out];
    switch (op.kind) {
      case OpKind::ConvF32:
        TRY(nhip_conv2d_f32_forward(op.conv, (const float*)in, op.residual >= 0 ? (const float*)ptr[op.residual] : nullptr,
                                    (float*)out, n, (int32_t)a.d[1], (int32_t)a.d[2], g.ws, g.ws_cap, stream));
        break;
      case OpKind::ConvInt8:
        TRY(nhip_conv2d_int8_forward(op.conv, in, g.blobs[op.in[0]].dtype == NHIP_DTYPE_I8, out, n, (int32_t)a.d[1],
                                     (int32_t)a.d[2], g.ws, g.ws_cap, stream));
        break;
      case OpKind::DwF32:
        TRY(nhip_dwconv2d_f32_forward(op.conv, (const float*)in, (float*)out, n, (int32_t)a.d[1], (int32_t)a.d[2], stream));
        break;
      case OpKind::DwInt8:
        TRY(nhip_dwconv2d_int8_forward(op.conv, in, g.blobs[op.in[0]].dtype == NHIP_DTYPE_I8, out, n, (int32_t)a.d[1],
                                       (int32_t)a.d[2], stream));
        break;
      case OpKind::IPInt8:
        TRY(nhip_innerproduct_int8_forward(op.ip, in, g.blobs[op.in[0]].dtype == NHIP_DTYPE_I8, (float*)out,
                                           (int32_t)(a.rank == 2 ? n * a.d[0] : n), g.ws, g.ws_cap, stream));
        break;
      case OpKind::IP:
        TRY(nhip_innerproduct_f32_forward(op.ip, (const float*)in, (float*)out, (int32_t)(a.rank == 2 ? n * a.d[0] : n),
                                          g.ws, g.ws_cap, stream));
        break;
      case OpKind::Relu:
        if (g.blobs[op.in[0]].dtype == NHIP_DTYPE_I8)
          TRY(nhip_relu_i8((const int8_t*)in, (int8_t*)out, n * a.elems(), stream));
        else
          TRY(nhip_relu_f32((const float*)in, (float*)out, n * a.elems(), stream));
        break;
      case OpKind::Add:
        TRY(nhip_add_f32((const float*)in, (const float*)ptr[op.in[1]], (float*)out, n * a.elems(), 0, stream));
        break;
      case OpKind::Gap:
        TRY(nhip_global_avgpool_f32((const float*)in, (float*)out, n, (int32_t)a.d[0], (int32_t)a.d[1], (int32_t)a.d[2],
                                    stream));
        break;
      // per-channel parameters index dimension zero of the blob
      // (quantizeSignedI8 / dequantizeNcnn scale dimension, NCNNToTosa.cpp:
      // 322-389,411-460): the channel of [C,H,W], the first extent of a
      // rank-1/2 view
      case OpKind::Quantize: {
        const int64_t c = a.rank >= 1 ? a.d[0] : 1;
        TRY(nhip_quantize_f32_i8((const float*)in, (int8_t*)out, n, (int32_t)c, a.elems() / c, op.scale_dev,
                                 op.scale_count, stream));
        break;
      }
      case OpKind::Dequantize: {
        const int64_t c = a.rank >= 1 ? a.d[0] : 1;
        TRY(nhip_dequantize_i32_f32((const int32_t*)in, (float*)out, n, (int32_t)c, a.elems() / c, op.scale_dev,
                                    op.scale_count, op.bias_dev, op.bias_count, stream));
        break;
      }
      case OpKind::Requantize: {
        const int64_t c = a.rank >= 1 ? a.d[0] : 1;
        TRY(nhip_requantize_i32_i8((const int32_t*)in, (int8_t*)out, n, (int32_t)c, a.elems() / c, op.scale_dev,
                                   op.scale_count, op.scale2_dev, op.scale2_count, op.bias_dev, op.bias_count,
                                   op.quant_act, stream));
        break;
      }
      default:
        return fail(NHIP_STATUS_UNSUPPORTED, op.name + ": no executor");
    }
  }
  for (size_t j = 0; j < g.outputs.size(); ++j) {
    if (!copied[j]) continue;
    const int b = g.outputs[j];
    TRY(nhip_memcpy_d2d(outputs[j], ptr[b], (uint64_t)n * sh[b].elems() * esize(g.blobs[b].dtype), stream));
  }
  return ok();
}

}  // namespace

extern "C" {

static int load_impl(const char* param_text, uint64_t param_len, const void* bin, uint64_t bin_len,
                     const int64_t* input_shapes, int32_t input_shape_count, nhip_graph_t* graph, bool dry) {
  if (!graph) return fail(NHIP_STATUS_NULL_POINTER, "graph_load: null graph pointer");
  *graph = nullptr;
  if (!param_text || (!bin && bin_len)) return fail(NHIP_STATUS_NULL_POINTER, "graph_load: null model data");
  if (input_shape_count < 0 || (input_shape_count > 0 && !input_shapes))
    return fail(NHIP_STATUS_NULL_POINTER, "graph_load: null input shapes");
  try {
    std::vector<Layer> layers;
    TRY(parse_param_text(std::string(param_text, param_len), layers));
    BinCursor cur{static_cast<const uint8_t*>(bin), (size_t)bin_len};
    for (Layer& L : layers) TRY(load_layer_weights(L, cur));
    if (bin && cur.pos != cur.size)  // graph.cpp:2299-2306
      return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, ".bin: size mismatch: consumed " + std::to_string(cur.pos) +
                                                        " bytes of " + std::to_string(cur.size));
    auto g = std::make_unique<nhip_graph>();
    g->host_only = dry;
    if (!dry) TRY(nhip::device_current(&g->device));  // plans are uploaded to the caller's current device
    TRY(build(*g, layers, input_shape_count ? input_shapes : nullptr, input_shape_count, dry));
    *graph = g.release();
    return ok();
  } catch (const std::bad_alloc&) {
    return fail(NHIP_STATUS_SHAPE_ARITHMETIC_OVERFLOW, "graph_load: out of host memory");
  } catch (const std::exception& e) {
    return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, std::string("graph_load: ") + e.what());
  }
}

int nhip_graph_load(const char* param_text, uint64_t param_len, const void* bin, uint64_t bin_len,
                    const int64_t* input_shapes, int32_t input_shape_count, nhip_graph_t* graph) {
  return load_impl(param_text, param_len, bin, bin_len, input_shapes, input_shape_count, graph, false);
}

int nhip_graph_describe(const char* param_text, uint64_t param_len, const void* bin, uint64_t bin_len,
                        const int64_t* input_shapes, int32_t input_shape_count, nhip_graph_t* graph) {
  return load_impl(param_text, param_len, bin, bin_len, input_shapes, input_shape_count, graph, true);
}

int nhip_graph_num_io(nhip_graph_t g, int32_t* inputs, int32_t* outputs) {
  if (!g || !inputs || !outputs) return fail(NHIP_STATUS_NULL_POINTER, "graph_num_io: null pointer");
  *inputs = (int32_t)g->inputs.size();
  *outputs = (int32_t)g->outputs.size();
  return ok();
}

int nhip_graph_io_info(nhip_graph_t g, int32_t is_output, int32_t index, int32_t* rank, int64_t dims[4], int32_t* dtype,
                       const char** name) {
  if (!g || !rank || !dims || !dtype) return fail(NHIP_STATUS_NULL_POINTER, "graph_io_info: null pointer");
  const std::vector<int>& list = is_output ? g->outputs : g->inputs;
  if (index < 0 || index >= (int32_t)list.size()) return fail(NHIP_STATUS_INVALID_SHAPE, "graph_io_info: bad index");
  const Blob& b = g->blobs[list[index]];
  *rank = b.declared.rank;
  for (int i = 0; i < 4; ++i) dims[i] = b.declared.d[i];
  *dtype = b.dtype;
  if (name) *name = b.name.c_str();
  return ok();
}

int nhip_graph_infer_shapes(nhip_graph_t g, const int64_t* input_shapes, int64_t* output_shapes, int32_t* output_ranks) {
  if (!g || !output_shapes || !output_ranks) return fail(NHIP_STATUS_NULL_POINTER, "graph_infer_shapes: null pointer");
  std::vector<Shape> sh;
  TRY(propagate(*g, input_shapes, sh, true));
  for (size_t j = 0; j < g->outputs.size(); ++j) {
    const Shape& s = sh[g->outputs[j]];
    output_ranks[j] = s.rank;
    for (int i = 0; i < 4; ++i) output_shapes[4 * j + i] = i < s.rank ? s.d[i] : 0;
  }
  return ok();
}

}  // extern "C"

namespace {

// Makes the graph's device current for one call and restores the caller's
// afterwards (a call never changes the calling thread's current device).
class DeviceGuard {
 public:
  explicit DeviceGuard(int dev) {
    if (nhip::device_current(&prev_) != NHIP_STATUS_SUCCESS) {
      status_ = NHIP_STATUS_DEVICE_ERROR;
      return;
    }
    if (prev_ != dev) {
      status_ = nhip::device_set(dev);
      switched_ = status_ == NHIP_STATUS_SUCCESS;
    }
  }
  ~DeviceGuard() {
    if (switched_) nhip::device_restore(prev_);
  }
  int status() const { return status_; }

 private:
  int prev_ = 0, status_ = NHIP_STATUS_SUCCESS;
  bool switched_ = false;
};

// One run of the call plan on `stream`, with replay.  When two calls in a
// row on a stream have the same key, the second runs eagerly (every buffer
// is already sized) and is also recorded into a hipGraph, and later calls
// with that key launch the recorded graph: one launch instead of one per
// kernel (each eager launch costs a few microseconds of dispatch that the
// short late layers of a network cannot hide).  Calls whose pointers change
// every time stay eager and record nothing.  The legacy default stream
// cannot be captured and runs eagerly, as do runs while the kernel timer
// records per-launch events and runs on a stream the caller is capturing
// itself (the launches then become part of the caller's graph; such a call
// fails with status 3 if the executor's buffers would have to grow, and
// from then on buffers that a larger call supersedes stay allocated until
// the graph is destroyed, since the caller's graph may replay over them);
// NHIP_GRAPH_REPLAY=0 turns replay off.  The graph's mutex is held.
int run_with_replay(nhip_graph& g, int32_t n, const std::vector<Shape>& sh, const void* const* inputs,
                    void* const* outputs, void* stream) {
  if (stream != nullptr && nhip::stream_capturing(stream)) {
    g.caller_captured = true;  // from here on, superseded buffers are retired, not freed
    return run_ops(g, n, sh, inputs, outputs, stream, true);
  }
  if (stream == nullptr || nhip::setting_int("NHIP_GRAPH_REPLAY", 1) == 0 || nhip::kernel_timer_active())
    return run_ops(g, n, sh, inputs, outputs, stream, false);
  std::ostringstream key;
  key << n;
  for (int b : g.inputs) {
    key << "|";
    for (int d = 0; d < sh[b].rank; ++d) key << sh[b].d[d] << ",";
  }
  for (size_t i = 0; i < g.inputs.size(); ++i) key << "|" << inputs[i];
  for (size_t j = 0; j < g.outputs.size(); ++j) key << "|" << outputs[j];
  key << "|stream " << stream << "|settings " << nhip::settings_generation();
  // The blob buffers and workspace grow (free + malloc) when a call needs
  // more: a recorded plan is only replayed while they are the ones it was
  // recorded with.
  auto internal_bufs = [&]() {
    std::vector<const void*> v;
    v.reserve(g.blobs.size() + 1);
    for (const Blob& b : g.blobs) v.push_back(b.buf);
    v.push_back(g.ws);
    return v;
  };
  if (g.exec && key.str() == g.exec_key) {
    if (internal_bufs() == g.exec_bufs) return nhip::graph_exec_launch(g.exec, stream);
    nhip::graph_exec_destroy(g.exec);
    g.exec = nullptr;
    g.exec_key.clear();
  }
  TRY(run_ops(g, n, sh, inputs, outputs, stream, false));
  if (key.str() != g.seen_key || key.str() == g.nocap_key) {
    g.seen_key = key.str();
    return ok();
  }
  nhip::graph_exec_destroy(g.exec);
  g.exec = nullptr;
  g.exec_key.clear();
  bool recorded = false;
  if (nhip::graph_capture_begin(stream) == NHIP_STATUS_SUCCESS) {
    const int st = run_ops(g, n, sh, inputs, outputs, stream, true);
    void* exec = nullptr;
    const int st2 = nhip::graph_capture_end(stream, &exec);
    if (st == NHIP_STATUS_SUCCESS && st2 == NHIP_STATUS_SUCCESS && exec) {
      g.exec = exec;
      g.exec_key = key.str();
      g.exec_bufs = internal_bufs();
      recorded = true;
    } else {
      nhip::graph_exec_destroy(exec);
    }
  }
  if (!recorded) g.nocap_key = key.str();
  return ok();
}

int ensure_pinned(nhip_graph& g, size_t slot, uint64_t bytes) {
  if (g.pinned.size() <= slot) {
    g.pinned.resize(slot + 1, nullptr);
    g.pinned_cap.resize(slot + 1, 0);
  }
  if (g.pinned_cap[slot] >= bytes) return ok();
  nhip::host_pinned_free(g.pinned[slot]);
  g.pinned[slot] = nullptr;
  g.pinned_cap[slot] = 0;
  TRY(nhip::host_pinned_alloc(&g.pinned[slot], bytes));
  g.pinned_cap[slot] = bytes;
  return ok();
}

}  // namespace

extern "C" {

int nhip_graph_run(nhip_graph_t g, int32_t n, const int64_t* input_shapes, const void* const* inputs,
                   void* const* outputs, void* stream) {
  if (!g || !inputs || !outputs) return fail(NHIP_STATUS_NULL_POINTER, "graph_run: null pointer");
  if (g->host_only) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "graph_run: graph was only described, not loaded");
  if (n < 0) return fail(NHIP_STATUS_INVALID_SHAPE, "graph_run: negative batch");
  if (n == 0) return ok();
  for (size_t i = 0; i < g->inputs.size(); ++i)
    if (!inputs[i]) return fail(NHIP_STATUS_NULL_POINTER, "graph_run: null input");
  for (size_t j = 0; j < g->outputs.size(); ++j)
    if (!outputs[j]) return fail(NHIP_STATUS_NULL_POINTER, "graph_run: null output");
  std::vector<Shape> sh;
  TRY(propagate(*g, input_shapes, sh, true));
  std::lock_guard<std::mutex> lock(g->mu);
  DeviceGuard dev(g->device);
  TRY(dev.status());
  return run_with_replay(*g, n, sh, inputs, outputs, stream);
}

int nhip_graph_run_host(nhip_graph_t g, const int64_t* input_shapes, const void* const* inputs, void* const* outputs,
                        const uint64_t* output_capacity) {
  if (!g || !inputs || !outputs) return fail(NHIP_STATUS_NULL_POINTER, "graph_run_host: null pointer");
  if (g->host_only) return fail(NHIP_STATUS_CONSTRAINT_VIOLATION, "graph_run_host: graph was only described, not loaded");
  for (size_t i = 0; i < g->inputs.size(); ++i)
    if (!inputs[i]) return fail(NHIP_STATUS_NULL_POINTER, "graph_run_host: null input");
  for (size_t j = 0; j < g->outputs.size(); ++j)
    if (!outputs[j]) return fail(NHIP_STATUS_NULL_POINTER, "graph_run_host: null output");
  std::lock_guard<std::mutex> lock(g->mu);
  std::vector<Shape> sh;
  TRY(propagate(*g, input_shapes, sh, true));
  if (output_capacity)
    for (size_t j = 0; j < g->outputs.size(); ++j)
      if ((uint64_t)sh[g->outputs[j]].elems() > output_capacity[j])
        return fail(NHIP_STATUS_OUTPUT_CAPACITY_INSUFFICIENT,
                    "output " + std::to_string(j + 1) + " needs " + std::to_string(sh[g->outputs[j]].elems()) + " elements");
  DeviceGuard dev(g->device);
  TRY(dev.status());
  if (!g->host_stream) TRY(nhip::stream_create(&g->host_stream));
  void* const s = g->host_stream;
  const size_t nin = g->inputs.size(), nout = g->outputs.size();
  g->host_in.resize(nin + nout, nullptr);
  g->host_in_cap.resize(nin + nout, 0);
  std::vector<const void*> din(nin);
  std::vector<void*> dout(nout);
  std::vector<uint64_t> out_bytes(nout);
  // inputs: caller buffer -> pinned staging -> device (DMA on the graph's stream)
  for (size_t i = 0; i < nin; ++i) {
    const int b = g->inputs[i];
    const uint64_t bytes = (uint64_t)sh[b].elems() * esize(g->blobs[b].dtype);
    TRY(ensure(&g->host_in[i], &g->host_in_cap[i], bytes));
    TRY(ensure_pinned(*g, i, bytes));
    std::memcpy(g->pinned[i], inputs[i], bytes);
    TRY(nhip_memcpy_h2d(g->host_in[i], g->pinned[i], bytes, s));
    din[i] = g->host_in[i];
  }
  for (size_t j = 0; j < nout; ++j) {
    const int b = g->outputs[j];
    out_bytes[j] = (uint64_t)sh[b].elems() * esize(g->blobs[b].dtype);
    TRY(ensure(&g->host_in[nin + j], &g->host_in_cap[nin + j], out_bytes[j]));
    TRY(ensure_pinned(*g, nin + j, out_bytes[j]));
    dout[j] = g->host_in[nin + j];
  }
  // the device buffers stay the same from call to call, so repeated calls
  // replay one recorded hipGraph of the plan
  TRY(run_with_replay(*g, 1, sh, din.data(), dout.data(), s));
  for (size_t j = 0; j < nout; ++j) TRY(nhip_memcpy_d2h(g->pinned[nin + j], dout[j], out_bytes[j], s));
  TRY(nhip_stream_sync(s));
  for (size_t j = 0; j < nout; ++j) std::memcpy(outputs[j], g->pinned[nin + j], out_bytes[j]);
  return ok();
}

int nhip_graph_destroy(nhip_graph_t g) {
  delete g;
  return ok();
}

}  // extern "C"
