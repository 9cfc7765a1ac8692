// ncnn-compile for MI355X: the reference's product CLI
// (tools/ncnn-compile.cpp:40-198 options, :946-1218 header, :805-913
// manifest, :2046-2196 link and export audit, :2235-2351 publish), producing
// the same artifact set — <model>.h and lib<model>.so with the entry
// `int <model>(const T* input1, ..., T* output1, ...)` — whose body runs the
// model on the GPU through libnhip (include/nhip_graph.h) instead of
// LLVM-generated CPU loops.
//
// The model is validated and lowered at compile time with
// nhip_graph_describe (no GPU needed); the .param/.bin bytes are embedded in
// the library and loaded onto the device at the first call.
#include <sys/stat.h>
#include <sys/wait.h>
#include <unistd.h>

#include <cctype>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <fstream>
#include <iostream>
#include <set>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/nhip_graph.h"

namespace {

// --input-dim-constraint=INPUT:DIM:min=N,multiple=N (the reference's
// tools/ncnn-mlir-driver.cpp:191-243 grammar): INPUT indexes the Input
// layers in source order, DIM is a CHW dimension that must be dynamic.
struct DimConstraint {
  int64_t input = 0, dim = 0, minimum = 0, multiple_of = 0;
};

struct Options {
  std::string param, bin, model_name, output_dir, runtime_dir, precision = "auto";
  std::vector<std::vector<int64_t>> input_shapes;
  std::vector<DimConstraint> constraints;
  bool emit_manifest = false, verbose = false, keep_source = false, verify_execution = false;
};

[[noreturn]] void die(const std::string& msg, int code = 1) {
  std::cerr << "ncnn-compile: error: " << msg << "\n";
  std::exit(code);
}

void usage() {
  std::cout << "usage: ncnn-compile [options] <model.param>\n"
               "  --bin=<path>            weights (default: <model>.bin)\n"
               "  --model-name=<name>     entry/header/library name (default: from the .param file name)\n"
               "  -o, --output-dir=<dir>  output directory (default: ./<model-name>)\n"
               "  --input-shape=<CxHxW>   Input extents, '?' = given at run time (repeatable)\n"
               "  --input-dim-constraint=<INPUT:DIM:min=N,multiple=N>\n"
               "                          run-time minimum and divisor of a '?' extent (repeatable)\n"
               "  --verify-execution      build and run an ABI harness against the library before publishing\n"
               "  --emit-manifest         also write <model-name>.json\n"
               "  --precision=<p>         auto|f32|int8 (recorded; int8 comes from the model's scale terms)\n"
               "  --runtime-dir=<dir>     directory holding libnhip.so (default: next to this tool)\n"
               "  --keep-source           keep the generated wrapper source in the output directory\n"
               "  -v, --verbose           echo every subprocess command\n"
               "  --threads=N --vector-width=N -O0..-O3   accepted for compatibility (no CPU code is generated)\n";
}

std::vector<int64_t> parse_shape(const std::string& s) {
  std::vector<int64_t> dims;
  std::string tok;
  std::stringstream ss(s);
  while (std::getline(ss, tok, 'x')) {
    std::stringstream inner(tok);
    std::string t2;
    while (std::getline(inner, t2, 'X')) {
      if (t2 == "?") {
        dims.push_back(-1);
      } else {
        char* end = nullptr;
        const long long v = std::strtoll(t2.c_str(), &end, 10);
        if (t2.empty() || *end || v <= 0) die("--input-shape extent must be a positive integer or '?': " + s);
        dims.push_back(v);
      }
    }
  }
  if (dims.size() != 3) die("--input-shape needs exactly three extents CxHxW: " + s);
  return dims;
}

bool parse_int(const std::string& t, int64_t* v) {
  if (t.empty()) return false;
  char* end = nullptr;
  errno = 0;
  const long long r = std::strtoll(t.c_str(), &end, 10);
  if (*end || errno) return false;
  *v = r;
  return true;
}

// Both fields are required, once each, with positive values.
bool parse_constraint(const std::string& text, DimConstraint* c) {
  const auto a = text.find(':');
  const auto b = a == std::string::npos ? a : text.find(':', a + 1);
  if (b == std::string::npos) return false;
  if (!parse_int(text.substr(0, a), &c->input) || !parse_int(text.substr(a + 1, b - a - 1), &c->dim)) return false;
  bool saw_min = false, saw_mult = false;
  std::stringstream fields(text.substr(b + 1));
  std::string f;
  while (std::getline(fields, f, ',')) {
    const auto eq = f.find('=');
    if (eq == std::string::npos) return false;
    const std::string name = f.substr(0, eq), value = f.substr(eq + 1);
    if (name == "min" && !saw_min) {
      saw_min = parse_int(value, &c->minimum) && c->minimum > 0;
      if (!saw_min) return false;
    } else if (name == "multiple" && !saw_mult) {
      saw_mult = parse_int(value, &c->multiple_of) && c->multiple_of > 0;
      if (!saw_mult) return false;
    } else {
      return false;
    }
  }
  return saw_min && saw_mult && c->input >= 0 && c->dim >= 0;
}

Options parse_args(int argc, char** argv) {
  Options o;
  auto value = [&](int& i, const std::string& a, const std::string& key) -> std::string {
    if (a.size() > key.size() && a[key.size()] == '=') return a.substr(key.size() + 1);
    if (i + 1 >= argc) die("missing value for " + key);
    return argv[++i];
  };
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    auto is = [&](const std::string& key) { return a == key || a.rfind(key + "=", 0) == 0; };
    if (a == "-h" || a == "--help") {
      usage();
      std::exit(0);
    } else if (is("--bin")) {
      o.bin = value(i, a, "--bin");
    } else if (is("--model-name")) {
      o.model_name = value(i, a, "--model-name");
    } else if (is("--output-dir")) {
      o.output_dir = value(i, a, "--output-dir");
    } else if (a == "-o") {
      if (i + 1 >= argc) die("missing value for -o");
      o.output_dir = argv[++i];
    } else if (is("--input-shape")) {
      const std::string v = value(i, a, "--input-shape");
      if (v == "*") die("--input-shape=* (dynamic rank) is not supported by the GPU runtime", 2);
      o.input_shapes.push_back(parse_shape(v));
    } else if (is("--input-dim-constraint")) {
      DimConstraint c;
      if (!parse_constraint(value(i, a, "--input-dim-constraint"), &c))
        die("--input-dim-constraint must be INPUT:DIM:min=N,multiple=N with positive values");
      o.constraints.push_back(c);
    } else if (a == "--emit-manifest") {
      o.emit_manifest = true;
    } else if (a == "--verify-execution") {
      o.verify_execution = true;
    } else if (is("--precision")) {
      o.precision = value(i, a, "--precision");
      if (o.precision != "auto" && o.precision != "f32" && o.precision != "int8")
        die("--precision must be auto, f32 or int8 on this backend");
    } else if (is("--runtime-dir")) {
      o.runtime_dir = value(i, a, "--runtime-dir");
    } else if (a == "--keep-source") {
      o.keep_source = true;
    } else if (a == "-v" || a == "--verbose") {
      o.verbose = true;
    } else if (is("--threads") || is("--vector-width")) {
      if (a.find('=') == std::string::npos) ++i;
    } else if (a.size() == 3 && a[0] == '-' && a[1] == 'O' && std::isdigit((unsigned char)a[2])) {
    } else if (!a.empty() && a[0] == '-') {
      die("unknown option " + a);
    } else if (o.param.empty()) {
      o.param = a;
    } else {
      die("more than one input .param file");
    }
  }
  if (o.param.empty()) {
    usage();
    die("no input .param file");
  }
  return o;
}

// The reference's name rule (docs/ncnn-compile-command-line.md section 2.3):
// ASCII identifier characters kept, runs of others become one underscore;
// names starting with a digit or underscore, C23 keywords and "main" get the
// prefix "ncnn_".
std::string c_identifier(const std::string& raw) {
  std::string out;
  bool last_sub = false;
  for (unsigned char c : raw) {
    if (std::isalnum(c) || c == '_') {
      out.push_back((char)c);
      last_sub = false;
    } else if (!last_sub) {
      out.push_back('_');
      last_sub = true;
    }
  }
  static const std::set<std::string> kKeywords = {
      "alignas", "alignof", "auto", "bool", "break", "case", "char", "const", "constexpr", "continue",
      "default", "do", "double", "else", "enum", "extern", "false", "float", "for", "goto", "if",
      "inline", "int", "long", "nullptr", "register", "restrict", "return", "short", "signed", "sizeof",
      "static", "static_assert", "struct", "switch", "thread_local", "true", "typedef", "typeof",
      "typeof_unqual", "union", "unsigned", "void", "volatile", "while", "main"};
  if (out.empty() || std::isdigit((unsigned char)out[0]) || out[0] == '_' || kKeywords.count(out)) out = "ncnn_" + out;
  return out;
}

std::string read_file(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) die("cannot read " + path);
  std::ostringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

void write_file(const std::string& path, const std::string& data) {
  std::ofstream f(path, std::ios::binary);
  if (!f || !(f << data)) die("cannot write " + path);
}

std::string dirname_of(const std::string& p) {
  const auto s = p.find_last_of('/');
  return s == std::string::npos ? "." : p.substr(0, s);
}

std::string basename_of(const std::string& p) {
  const auto s = p.find_last_of('/');
  return s == std::string::npos ? p : p.substr(s + 1);
}

std::string self_dir() {
  char buf[4096];
  const ssize_t n = readlink("/proc/self/exe", buf, sizeof buf - 1);
  if (n <= 0) return ".";
  buf[n] = 0;
  return dirname_of(buf);
}

std::string abs_path(const std::string& p) {
  char buf[4096];
  if (realpath(p.c_str(), buf)) return buf;
  return p;
}

// Runs a subprocess; with `capture`, its stdout goes to that file.
int run(const std::vector<std::string>& cmd, bool verbose, const std::string& capture = "") {
  std::string line;
  for (auto& c : cmd) line += (line.empty() ? "" : " ") + c;
  if (verbose) std::cerr << "+ " << line << (capture.empty() ? "" : " > " + capture) << "\n";
  const pid_t pid = fork();
  if (pid < 0) die("fork failed");
  if (pid == 0) {
    if (!capture.empty()) {
      FILE* f = std::fopen(capture.c_str(), "w");
      if (!f || dup2(fileno(f), 1) < 0) _exit(126);
    }
    std::vector<char*> av;
    for (auto& c : cmd) av.push_back(const_cast<char*>(c.c_str()));
    av.push_back(nullptr);
    execvp(av[0], av.data());
    _exit(127);
  }
  int st = 0;
  waitpid(pid, &st, 0);
  return WIFEXITED(st) ? WEXITSTATUS(st) : 128;
}

struct Arg {
  std::string name, ctype, etype;
  std::vector<int64_t> shape;
  uint32_t mask = 0;
  std::vector<DimConstraint> constraints;  // inputs: on dynamic dimensions, by dimension
};

std::string upper(std::string s) {
  for (auto& c : s) c = (char)std::toupper((unsigned char)c);
  return s;
}

std::string macro(const std::string& fn, const Arg& a, const std::string& suffix) {
  return upper(fn + "_" + a.name + "_" + suffix);
}

// Header text: the same structure as the reference's write_header
// (tools/ncnn-compile.cpp:946-1218) for fixed-rank arguments.
std::string header_text(const std::string& fn, const std::vector<Arg>& ins, const std::vector<Arg>& outs) {
  std::ostringstream h;
  const std::string guard = upper("NCNN_" + fn + "_H");
  h << "#ifndef " << guard << "\n#define " << guard << "\n\n#include <stdint.h>\n\n"
    << "#define NCNN_DYNAMIC_DIM INT64_C(-1)\n#define NCNN_MAX_RANK 4\n"
    << "#define NCNN_STATUS_SUCCESS 0\n#define NCNN_STATUS_NULL_POINTER 1\n#define NCNN_STATUS_INVALID_SHAPE 2\n"
    << "#define NCNN_STATUS_CONSTRAINT_VIOLATION 3\n#define NCNN_STATUS_SHAPE_ARITHMETIC_OVERFLOW 4\n"
    << "#define NCNN_STATUS_OUTPUT_CAPACITY_INSUFFICIENT 5\n\n"
    << "typedef uint16_t ncnn_float16_t;\ntypedef uint16_t ncnn_bfloat16_t;\n\n"
    << "#define " << upper(fn) << "_INPUT_COUNT " << ins.size() << "\n"
    << "#define " << upper(fn) << "_OUTPUT_COUNT " << outs.size() << "\n\n";
  auto emit = [&](const Arg& a, bool is_out) {
    h << "#define " << macro(fn, a, "rank") << " " << a.shape.size() << "\n";
    for (size_t i = 0; i < a.shape.size(); ++i)
      h << "#define " << macro(fn, a, "dim" + std::to_string(i)) << " "
        << (a.shape[i] < 0 ? std::string("NCNN_DYNAMIC_DIM") : "INT64_C(" + std::to_string(a.shape[i]) + ")") << "\n";
    char mask[32];
    std::snprintf(mask, sizeof mask, "UINT32_C(0x%x)", a.mask);
    h << "#define " << macro(fn, a, "dynamic_dim_mask") << " " << mask << "\n";
    for (const DimConstraint& c : a.constraints)  // tools/ncnn-compile.cpp:1059-1073
      h << "#define " << macro(fn, a, "dim" + std::to_string(c.dim) + "_minimum") << " INT64_C(" << c.minimum << ")\n"
        << "#define " << macro(fn, a, "dim" + std::to_string(c.dim) + "_multiple_of") << " INT64_C(" << c.multiple_of
        << ")\n";
    if (a.mask == 0) {
      uint64_t e = 1;
      for (int64_t d : a.shape) e *= (uint64_t)d;
      h << "#define " << macro(fn, a, "elements") << " UINT64_C(" << e << ")\n";
    }
    if (is_out) h << "#define " << macro(fn, a, "shape_depends_on_data") << " 0\n";
    h << "\n";
  };
  for (auto& a : ins) emit(a, false);
  for (auto& a : outs) emit(a, true);
  h << "\n#ifdef __cplusplus\nextern \"C\" {\n#endif\n\nint " << fn << "(";
  bool first = true;
  for (auto& a : ins) {
    h << (first ? "" : ", ") << "const " << a.ctype << " *" << a.name;
    if (a.mask) h << ", const int64_t " << a.name << "_shape[" << macro(fn, a, "rank") << "]";
    first = false;
  }
  for (auto& a : outs) {
    h << (first ? "" : ", ") << a.ctype << " *" << a.name;
    first = false;
  }
  bool dyn_out = false;
  for (auto& a : outs)
    if (a.mask) {
      h << ", uint64_t " << a.name << "_capacity";
      dyn_out = true;
    }
  h << ");\n";
  if (dyn_out) {
    h << "\nint " << fn << "_infer_output_shapes(";
    first = true;
    for (auto& a : ins)
      if (a.mask) {
        h << (first ? "" : ", ") << "const int64_t " << a.name << "_shape[" << macro(fn, a, "rank") << "]";
        first = false;
      }
    for (auto& a : outs)
      if (a.mask) {
        h << (first ? "" : ", ") << "int64_t " << a.name << "_shape[" << macro(fn, a, "rank") << "]";
        first = false;
      }
    h << ");\n";
  }
  h << "\n#ifdef __cplusplus\n}\n#endif\n\n#endif  // " << guard << "\n";
  return h.str();
}

std::string manifest_text(const std::string& fn, const std::vector<Arg>& ins, const std::vector<Arg>& outs,
                          const std::string& precision) {
  std::ostringstream j;
  auto arr = [&](const std::vector<Arg>& v) {
    j << "[";
    for (size_t i = 0; i < v.size(); ++i) {
      j << (i ? ",\n    " : "\n    ") << "{\n";
      if (!v[i].constraints.empty()) {  // tools/ncnn-compile.cpp:818-830
        j << "      \"dimension_constraints\": [";
        for (size_t c = 0; c < v[i].constraints.size(); ++c)
          j << (c ? ", " : "") << "{\"dimension\": " << v[i].constraints[c].dim << ", \"minimum\": "
            << v[i].constraints[c].minimum << ", \"multiple_of\": " << v[i].constraints[c].multiple_of << "}";
        j << "],\n";
      }
      j << "      \"dynamic_dim_mask\": " << v[i].mask << ",\n      \"element_type\": \""
        << v[i].etype << "\",\n      \"name\": \"" << v[i].name << "\",\n      \"shape\": [";
      for (size_t k = 0; k < v[i].shape.size(); ++k) j << (k ? ", " : "") << v[i].shape[k];
      j << "]\n    }";
    }
    j << "\n  ]";
  };
  j << "{\n  \"function\": \"" << fn << "\",\n  \"inputs\": ";
  arr(ins);
  j << ",\n  \"outputs\": ";
  arr(outs);
  j << ",\n  \"precision_policy\": {\n    \"storage\": \"" << (precision == "int8" ? "int8" : "f32")
    << "\",\n    \"fallback\": \"none\"\n  },\n  \"target\": {\n    \"triple\": \"amdgcn-amd-amdhsa\",\n"
    << "    \"cpu\": \"gfx950\",\n    \"execution_profile\": \"libnhip\"\n  }\n}\n";
  return j.str();
}

// The wrapper library: embedded model bytes, one device graph loaded at the
// first call (pthread_once), the reference's typed entry, and the
// shape-inference entry for dynamic outputs (host-only, no GPU needed).
std::string wrapper_source(const std::string& fn, const std::vector<Arg>& ins, const std::vector<Arg>& outs,
                           const std::string& param_path, const std::string& bin_path,
                           const std::vector<int64_t>& flat_shapes) {
  std::ostringstream s;
  s << "// Generated by ncnn-compile (MI355X / libnhip backend) for model '" << fn << "'.\n"
    << "#include <pthread.h>\n#include <stdint.h>\n#include \"nhip_graph.h\"\n\n"
    << "__asm__(\".section .rodata\\n.balign 16\\n.hidden nhip_model_param\\n.hidden nhip_model_param_end\\n"
    << "nhip_model_param:\\n.incbin \\\"" << param_path << "\\\"\\nnhip_model_param_end:\\n"
    << ".balign 16\\n.hidden nhip_model_bin\\n.hidden nhip_model_bin_end\\n"
    << "nhip_model_bin:\\n.incbin \\\"" << bin_path << "\\\"\\nnhip_model_bin_end:\\n.previous\\n\");\n"
    << "extern \"C\" const char nhip_model_param[], nhip_model_param_end[], nhip_model_bin[], nhip_model_bin_end[];\n\n"
    << "static const int64_t kShapes[" << std::max<size_t>(flat_shapes.size(), 1) << "] = {";
  for (size_t i = 0; i < flat_shapes.size(); ++i) s << (i ? ", " : "") << flat_shapes[i];
  if (flat_shapes.empty()) s << "0";
  s << "};\nstatic const int32_t kNumShapes = " << flat_shapes.size() / 3 << ";\n"
    << "static nhip_graph_t g_exec, g_desc;\nstatic int g_exec_status, g_desc_status;\n"
    << "static pthread_once_t g_exec_once = PTHREAD_ONCE_INIT, g_desc_once = PTHREAD_ONCE_INIT;\n"
    << "/* The model is loaded onto the device current in the thread of the first call (device 0\n"
    << "   unless that thread chose another); every call then runs there on the graph's own stream,\n"
    << "   leaving the calling thread's current device as it was. */\n"
    << "static void init_exec(void) {\n"
    << "  g_exec_status = nhip_graph_load(nhip_model_param, (uint64_t)(nhip_model_param_end - nhip_model_param),\n"
    << "                                    nhip_model_bin, (uint64_t)(nhip_model_bin_end - nhip_model_bin),\n"
    << "                                    kNumShapes ? kShapes : 0, kNumShapes, &g_exec);\n}\n"
    << "static void init_desc(void) {\n"
    << "  g_desc_status = nhip_graph_describe(nhip_model_param, (uint64_t)(nhip_model_param_end - nhip_model_param),\n"
    << "                                      nhip_model_bin, (uint64_t)(nhip_model_bin_end - nhip_model_bin),\n"
    << "                                      kNumShapes ? kShapes : 0, kNumShapes, &g_desc);\n}\n\n";
  // run-time input shapes: static extents from the model, dynamic from the caller
  auto shape_block = [&]() {
    std::ostringstream b;
    b << "  int64_t shapes[" << 3 * ins.size() << "];\n";
    for (size_t i = 0; i < ins.size(); ++i)
      for (int k = 0; k < 3; ++k) {
        b << "  shapes[" << 3 * i + k << "] = ";
        // a dynamic input passes every caller extent, so static ones are checked too
        if (ins[i].mask) b << ins[i].name << "_shape[" << k << "];\n";
        else b << ins[i].shape[k] << ";\n";
      }
    // The reference wrapper's order (GenerateCAPI.cpp:1440-1480): invalid
    // extents are status 2 before constraint violations are status 3.
    for (size_t i = 0; i < ins.size(); ++i)
      for (int k = 0; k < 3; ++k)
        if (ins[i].mask & (1u << k)) b << "  if (shapes[" << 3 * i + k << "] <= 0) return 2;\n";
    for (size_t i = 0; i < ins.size(); ++i)
      for (const DimConstraint& c : ins[i].constraints)
        b << "  if (shapes[" << 3 * i + c.dim << "] < INT64_C(" << c.minimum << ") || shapes[" << 3 * i + c.dim
          << "] % INT64_C(" << c.multiple_of << ") != 0) return 3;  /* NCNN_STATUS_CONSTRAINT_VIOLATION */\n";
    return b.str();
  };
  s << "extern \"C\" __attribute__((visibility(\"default\"))) int " << fn << "(";
  bool first = true;
  for (auto& a : ins) {
    s << (first ? "" : ", ") << "const " << a.ctype << " *" << a.name;
    if (a.mask) s << ", const int64_t " << a.name << "_shape[" << a.shape.size() << "]";
    first = false;
  }
  for (auto& a : outs) {
    s << (first ? "" : ", ") << a.ctype << " *" << a.name;
    first = false;
  }
  bool dyn_out = false;
  for (auto& a : outs)
    if (a.mask) {
      s << ", uint64_t " << a.name << "_capacity";
      dyn_out = true;
    }
  s << ") {\n  if (";
  first = true;
  for (auto& a : ins) {
    s << (first ? "" : " || ") << "!" << a.name;
    if (a.mask) s << " || !" << a.name << "_shape";
    first = false;
  }
  for (auto& a : outs) s << " || !" << a.name;
  s << ") return 1;  /* NCNN_STATUS_NULL_POINTER */\n"
    << shape_block() << "  pthread_once(&g_exec_once, init_exec);\n  if (g_exec_status != 0) return g_exec_status;\n"
    << "  const void* ins[] = {";
  for (size_t i = 0; i < ins.size(); ++i) s << (i ? ", " : "") << ins[i].name;
  s << "};\n  void* outs[] = {";
  for (size_t j = 0; j < outs.size(); ++j) s << (j ? ", " : "") << outs[j].name;
  s << "};\n";
  if (dyn_out) {
    s << "  const uint64_t caps[] = {";
    for (size_t j = 0; j < outs.size(); ++j) {
      s << (j ? ", " : "");
      if (outs[j].mask) {
        s << outs[j].name << "_capacity";
      } else {
        uint64_t e = 1;
        for (int64_t d : outs[j].shape) e *= (uint64_t)d;
        s << e << "u";
      }
    }
    s << "};\n  return nhip_graph_run_host(g_exec, shapes, ins, outs, caps);\n}\n";
  } else {
    s << "  return nhip_graph_run_host(g_exec, shapes, ins, outs, 0);\n}\n";
  }
  if (dyn_out) {
    s << "\nextern \"C\" __attribute__((visibility(\"default\"))) int " << fn << "_infer_output_shapes(";
    first = true;
    for (auto& a : ins)
      if (a.mask) {
        s << (first ? "" : ", ") << "const int64_t " << a.name << "_shape[" << a.shape.size() << "]";
        first = false;
      }
    for (auto& a : outs)
      if (a.mask) {
        s << (first ? "" : ", ") << "int64_t " << a.name << "_shape[" << a.shape.size() << "]";
        first = false;
      }
    s << ") {\n  if (";
    first = true;
    for (auto& a : ins)
      if (a.mask) {
        s << (first ? "" : " || ") << "!" << a.name << "_shape";
        first = false;
      }
    for (auto& a : outs)
      if (a.mask) {
        s << (first ? "" : " || ") << "!" << a.name << "_shape";
        first = false;
      }
    s << ") return 1;\n" << shape_block()
      << "  pthread_once(&g_desc_once, init_desc);\n  if (g_desc_status != 0) return g_desc_status;\n"
      << "  int64_t oshape[" << 4 * outs.size() << "];\n  int32_t orank[" << outs.size() << "];\n"
      << "  const int st = nhip_graph_infer_shapes(g_desc, shapes, oshape, orank);\n  if (st != 0) return st;\n";
    for (size_t j = 0; j < outs.size(); ++j)
      if (outs[j].mask)
        for (size_t k = 0; k < outs[j].shape.size(); ++k)
          s << "  " << outs[j].name << "_shape[" << k << "] = oshape[" << 4 * j + k << "];\n";
    s << "  return 0;\n}\n";
  }
  return s.str();
}

// Symbol names from `nm -D` output (the last column, version suffix dropped).
std::set<std::string> nm_symbols(const std::string& text) {
  std::set<std::string> out;
  std::istringstream in(text);
  std::string line;
  while (std::getline(in, line)) {
    std::istringstream ls(line);
    std::string tok, last;
    while (ls >> tok) last = tok;
    if (last.empty()) continue;
    const auto at = last.find('@');
    out.insert(at == std::string::npos ? last : last.substr(0, at));
  }
  return out;
}

// The reference's artifact audit (tools/ncnn-compile.cpp:2070-2196), with
// its allowlists extended by exactly what a GPU-backed library needs: the
// libnhip graph entry points (nhip_*) and pthread_once (the one-time graph
// load) as undefined symbols, libnhip.so (and the HIP runtime it loads) as a
// DT_NEEDED entry.  Returns "" or the failure.
std::string audit_library(const std::string& lib, const std::string& fn, bool dynamic_output,
                          const std::string& scratch_dir, bool verbose) {
  const std::string cap = scratch_dir + "/audit.txt";
  if (run({"nm", "-D", "--undefined-only", lib}, verbose, cap) != 0) return "nm failed on " + lib;
  static const std::set<std::string> kAllowed = {"ceilf", "erfcf", "erff",   "expf",   "floorf",      "free",
                                                 "malloc", "memcpy", "memset", "powf", "tanhf", "pthread_once"};
  std::string unexpected;
  for (const std::string& s : nm_symbols(read_file(cap)))
    if (!kAllowed.count(s) && s.rfind("nhip_", 0) != 0) unexpected += (unexpected.empty() ? "" : ", ") + s;
  if (!unexpected.empty()) return "shared library contains unexpected undefined symbols: " + unexpected;
  if (run({"nm", "-D", "--defined-only", lib}, verbose, cap) != 0) return "nm failed on " + lib;
  std::set<std::string> expected = {fn};
  if (dynamic_output) expected.insert(fn + "_infer_output_shapes");
  if (nm_symbols(read_file(cap)) != expected) return "shared library exports symbols outside the model ABI entry points";
  if (run({"readelf", "-d", "-W", lib}, verbose, cap) != 0) return "readelf failed on " + lib;
  {
    std::istringstream in(read_file(cap));
    std::string line;
    while (std::getline(in, line)) {
      if (line.find("(NEEDED)") == std::string::npos) continue;
      const auto a = line.find('['), b = line.find(']');
      if (a == std::string::npos || b == std::string::npos || b < a) return "unreadable DT_NEEDED entry: " + line;
      const std::string name = line.substr(a + 1, b - a - 1);
      auto starts = [&](const char* p) { return name.rfind(p, 0) == 0; };
      if (!starts("libc.so") && !starts("libm.so") && name != "libnhip.so" && !starts("libamdhip64.so"))
        return "shared library has an unexpected dependency: " + name;
    }
  }
  if (run({"nm", "-D", lib}, verbose, cap) != 0) return "nm failed on " + lib;
  const std::string all = read_file(cap);
  for (const char* forbidden : {"memrefCopy", "runner_utils", "RunnerUtils", "ncnn_runtime"})
    if (all.find(forbidden) != std::string::npos) return "forbidden runtime symbol found in shared library";
  std::remove(cap.c_str());
  return "";
}

// --verify-execution: the reference's ABI harness (tools/ncnn-compile.cpp:
// 1383-1636) for fixed-rank models: zero inputs (dynamic extents 2, or the
// smallest extent a constraint allows), output shapes from
// <model>_infer_output_shapes, one call that must succeed with finite
// floating-point outputs, every pointer argument rejected when NULL, and a
// dynamic output's capacity one short rejected with status 5.
std::string harness_source(const std::string& fn, const std::vector<Arg>& ins, const std::vector<Arg>& outs) {
  std::ostringstream c;
  c << "#include <math.h>\n#include <stddef.h>\n#include <stdio.h>\n#include <stdlib.h>\n#include \"" << fn
    << ".h\"\n\nstatic size_t element_count(const int64_t *shape, size_t rank) {\n  size_t count = 1;\n"
    << "  for (size_t i = 0; i < rank; ++i) count *= (size_t)shape[i];\n  return count;\n}\n\nint main(void) {\n";
  std::vector<std::string> args;
  for (const Arg& a : ins) {
    if (a.mask) {
      c << "  int64_t " << a.name << "_shape[" << a.shape.size() << "] = {";
      for (size_t k = 0; k < a.shape.size(); ++k) {
        int64_t e = 2;
        for (const DimConstraint& d : a.constraints)
          if (d.dim == (int64_t)k) e = (d.minimum + d.multiple_of - 1) / d.multiple_of * d.multiple_of;
        c << (k ? ", " : "") << (a.shape[k] < 0 ? e : a.shape[k]);
      }
      c << "};\n  size_t " << a.name << "_count = element_count(" << a.name << "_shape, " << a.shape.size() << ");\n";
    } else {
      uint64_t e = 1;
      for (int64_t d : a.shape) e *= (uint64_t)d;
      c << "  size_t " << a.name << "_count = " << e << ";\n";
    }
    c << "  " << a.ctype << " *" << a.name << " = calloc(" << a.name << "_count, sizeof(" << a.ctype << "));\n"
      << "  if (!" << a.name << ") { fprintf(stderr, \"ABI verification failed: cannot allocate " << a.name
      << "\\n\"); return 2; }\n";
  }
  bool dyn_out = false;
  std::string shape_call = fn + "_infer_output_shapes(";
  bool first = true;
  for (const Arg& a : ins)
    if (a.mask) {
      shape_call += (first ? "" : ", ") + a.name + "_shape";
      first = false;
    }
  for (const Arg& a : outs)
    if (a.mask) {
      dyn_out = true;
      c << "  int64_t " << a.name << "_shape[" << a.shape.size() << "] = {0};\n";
      shape_call += (first ? "" : ", ") + a.name + "_shape";
      first = false;
    }
  shape_call += ")";
  if (dyn_out) c << "  if (" << shape_call << " != 0) return 6;\n";
  for (const Arg& a : outs) {
    if (a.mask) {
      c << "  size_t " << a.name << "_count = element_count(" << a.name << "_shape, " << a.shape.size() << ");\n"
        << "  uint64_t " << a.name << "_capacity = " << a.name << "_count;\n";
    } else {
      uint64_t e = 1;
      for (int64_t d : a.shape) e *= (uint64_t)d;
      c << "  size_t " << a.name << "_count = " << e << ";\n";
    }
    c << "  " << a.ctype << " *" << a.name << " = calloc(" << a.name << "_count, sizeof(" << a.ctype << "));\n"
      << "  if (!" << a.name << ") return 2;\n";
  }
  for (const Arg& a : ins) {
    args.push_back(a.name);
    if (a.mask) args.push_back(a.name + "_shape");
  }
  for (const Arg& a : outs) args.push_back(a.name);
  for (const Arg& a : outs)
    if (a.mask) args.push_back(a.name + "_capacity");
  auto call = [&](long null_index, long short_index) {
    std::string r = fn + "(";
    for (size_t i = 0; i < args.size(); ++i)
      r += (i ? ", " : "") + ((long)i == null_index ? std::string("NULL") : args[i] + ((long)i == short_index ? " - 1" : ""));
    return r + ")";
  };
  c << "  int model_status = " << call(-1, -1) << ";\n"
    << "  if (model_status != 0) { fprintf(stderr, \"ABI verification failed: model returned %d\\n\", model_status); "
       "return 4; }\n";
  for (const Arg& a : outs)
    if (a.etype == "f32")
      c << "  for (size_t i = 0; i < " << a.name << "_count; ++i) if (!isfinite(" << a.name
        << "[i])) { fprintf(stderr, \"ABI verification failed: output " << a.name
        << "[%zu] is not finite\\n\", i); return 5; }\n";
  for (size_t i = 0; i < args.size(); ++i) {
    if (args[i].size() > 9 && args[i].compare(args[i].size() - 9, 9, "_capacity") == 0) continue;
    c << "  if (" << call((long)i, -1) << " == 0) { fprintf(stderr, \"ABI verification failed: NULL argument "
      << args[i] << " was accepted\\n\"); return 3; }\n";
  }
  for (size_t i = 0; i < args.size(); ++i)
    if (args[i].size() > 9 && args[i].compare(args[i].size() - 9, 9, "_capacity") == 0)
      c << "  if (" << call(-1, (long)i) << " != NCNN_STATUS_OUTPUT_CAPACITY_INSUFFICIENT) return 14;\n";
  for (const Arg& a : ins) c << "  free(" << a.name << ");\n";
  for (const Arg& a : outs) c << "  free(" << a.name << ");\n";
  c << "  return 0;\n}\n";
  return c.str();
}

}  // namespace

int main(int argc, char** argv) {
  Options o = parse_args(argc, argv);
  if (o.bin.empty()) {
    o.bin = o.param;
    if (o.bin.size() > 6 && o.bin.compare(o.bin.size() - 6, 6, ".param") == 0) o.bin.replace(o.bin.size() - 6, 6, ".bin");
    else o.bin += ".bin";
  }
  std::string stem = basename_of(o.param);
  if (stem.size() > 6 && stem.compare(stem.size() - 6, 6, ".param") == 0) stem.resize(stem.size() - 6);
  const std::string fn = c_identifier(o.model_name.empty() ? stem : o.model_name);
  if (o.output_dir.empty()) o.output_dir = fn;
  const std::string runtime_dir = abs_path(o.runtime_dir.empty() ? self_dir() + "/.." : o.runtime_dir);
  const std::string include_dir = abs_path(runtime_dir + "/../include");

  const std::string param = read_file(o.param), bin = read_file(o.bin);
  std::vector<int64_t> flat;
  for (auto& sh : o.input_shapes) flat.insert(flat.end(), sh.begin(), sh.end());
  nhip_graph_t g = nullptr;
  if (nhip_graph_describe(param.data(), param.size(), bin.data(), bin.size(), flat.empty() ? nullptr : flat.data(),
                          (int32_t)(flat.size() / 3), &g) != 0)
    die(std::string("model rejected: ") + nhip_last_error());
  int32_t ni = 0, no = 0;
  nhip_graph_num_io(g, &ni, &no);
  std::vector<Arg> ins, outs;
  for (int io = 0; io < 2; ++io)
    for (int32_t i = 0; i < (io ? no : ni); ++i) {
      int32_t rank = 0, dtype = 0;
      int64_t dims[4];
      nhip_graph_io_info(g, io, i, &rank, dims, &dtype, nullptr);
      Arg a;
      a.name = (io ? "output" : "input") + std::to_string(i + 1);
      // ABI element types of GenerateCAPI.cpp:50-80
      a.ctype = dtype == NHIP_DTYPE_I8 ? "int8_t" : dtype == NHIP_DTYPE_I32 ? "int32_t" : "float";
      a.etype = dtype == NHIP_DTYPE_I8 ? "i8" : dtype == NHIP_DTYPE_I32 ? "i32" : "f32";
      for (int k = 0; k < rank; ++k) {
        a.shape.push_back(dims[k]);
        if (dims[k] < 0) a.mask |= 1u << k;
      }
      (io ? outs : ins).push_back(a);
    }
  // Constraints name dynamic extents of existing inputs, once each.
  for (size_t a = 0; a < o.constraints.size(); ++a) {
    const DimConstraint& c = o.constraints[a];
    if (c.input >= (int64_t)ins.size())
      die("--input-dim-constraint: input index " + std::to_string(c.input) + " is out of range");
    Arg& in = ins[(size_t)c.input];
    if (c.dim >= (int64_t)in.shape.size())
      die("--input-dim-constraint: dimension " + std::to_string(c.dim) + " is out of range");
    if (in.shape[(size_t)c.dim] >= 0)
      die("--input-dim-constraint: input " + std::to_string(c.input) + " dimension " + std::to_string(c.dim) +
          " is static; constraints apply to '?' extents");
    for (const DimConstraint& d : in.constraints)
      if (d.dim == c.dim) die("--input-dim-constraint: duplicate constraint on input " + std::to_string(c.input) +
                              " dimension " + std::to_string(c.dim));
    in.constraints.push_back(c);
  }
  for (Arg& in : ins)
    std::sort(in.constraints.begin(), in.constraints.end(),
              [](const DimConstraint& x, const DimConstraint& y) { return x.dim < y.dim; });
  // Inputs with a dynamic extent need the full [C,H,W] in kShapes.
  if (flat.empty()) {
    for (auto& a : ins) flat.insert(flat.end(), a.shape.begin(), a.shape.end());
  }
  nhip_graph_destroy(g);

  // Stage everything next to the output directory, then publish.
  const std::string out_abs = abs_path(dirname_of(o.output_dir)) + "/" + basename_of(o.output_dir);
  const std::string stage = out_abs + ".ncnn-compile-tmp." + std::to_string(getpid());
  if (mkdir(stage.c_str(), 0755) != 0) die("cannot create staging directory " + stage);
  write_file(stage + "/" + fn + ".h", header_text(fn, ins, outs));
  if (o.emit_manifest) write_file(stage + "/" + fn + ".json", manifest_text(fn, ins, outs, o.precision));
  const std::string src_dir = stage + "/.src";
  mkdir(src_dir.c_str(), 0755);
  write_file(src_dir + "/model.param", param);
  write_file(src_dir + "/model.bin", bin);
  write_file(src_dir + "/" + fn + "_wrapper.cpp",
             wrapper_source(fn, ins, outs, src_dir + "/model.param", src_dir + "/model.bin", flat));
  std::string exports = "{\n  global:\n    " + fn + ";\n";
  for (auto& a : outs)
    if (a.mask) {
      exports += "    " + fn + "_infer_output_shapes;\n";
      break;
    }
  exports += "  local: *;\n};\n";
  write_file(src_dir + "/exports.map", exports);
  const char* cxx = std::getenv("CXX");
  // Linked like the reference's artifact (tools/ncnn-compile.cpp:2045-2069):
  // no start files or default libraries, every symbol resolved at link time,
  // exports from a version script; the wrapper needs no C++ runtime.
  const std::string lib = stage + "/lib" + fn + ".so";
  std::vector<std::string> cmd = {cxx && *cxx ? cxx : "g++", "-O2", "-fPIC", "-shared", "-std=c++17",
                                  "-fvisibility=hidden", "-fno-exceptions", "-fno-rtti", "-fno-stack-protector",
                                  "-nostdlib", "-I" + include_dir, src_dir + "/" + fn + "_wrapper.cpp", "-o", lib,
                                  "-L" + runtime_dir, "-lnhip", "-Wl,-rpath," + runtime_dir,
                                  "-Wl,--version-script=" + src_dir + "/exports.map", "-Wl,-z,defs",
                                  "-Wl,--no-undefined", "-Wl,--build-id=none", "-lc"};
  if (run(cmd, o.verbose) != 0) {
    run({"rm", "-rf", stage}, o.verbose);
    die("compiling the model library failed");
  }
  bool dynamic_output = false;
  for (auto& a : outs) dynamic_output |= a.mask != 0;
  const std::string audit = audit_library(lib, fn, dynamic_output, src_dir, o.verbose);
  if (!audit.empty()) {
    run({"rm", "-rf", stage}, o.verbose);
    die(audit);
  }
  if (o.verify_execution) {
    const char* cc = std::getenv("CC");
    write_file(src_dir + "/harness.c", harness_source(fn, ins, outs));
    if (run({cc && *cc ? cc : "gcc", "-std=c11", src_dir + "/harness.c", "-I", stage, "-L", stage, "-l" + fn,
             "-Wl,-rpath," + stage, "-lm", "-o", src_dir + "/harness"},
            o.verbose) != 0) {
      run({"rm", "-rf", stage}, o.verbose);
      die("ABI verification harness compilation failed");
    }
    const int st = run({src_dir + "/harness"}, o.verbose);
    if (st != 0) {
      run({"rm", "-rf", stage}, o.verbose);
      die("ABI execution verification failed with harness exit code " + std::to_string(st), st);
    }
    std::cerr << "ncnn-compile: ABI execution verification passed\n";
  }
  if (o.keep_source) {
    std::rename((src_dir + "/" + fn + "_wrapper.cpp").c_str(), (stage + "/" + fn + "_wrapper.cpp").c_str());
  }
  run({"rm", "-rf", src_dir}, o.verbose);
  // Atomic publish: old directory -> backup, staging -> output, drop backup.
  struct stat st {};
  const std::string backup = out_abs + ".ncnn-compile-old." + std::to_string(getpid());
  const bool had_old = stat(out_abs.c_str(), &st) == 0;
  if (had_old && std::rename(out_abs.c_str(), backup.c_str()) != 0) die("cannot move the old output directory aside");
  if (std::rename(stage.c_str(), out_abs.c_str()) != 0) {
    if (had_old) std::rename(backup.c_str(), out_abs.c_str());
    die("cannot publish " + out_abs);
  }
  if (had_old) run({"rm", "-rf", backup}, o.verbose);
  if (o.verbose) std::cerr << "wrote " << out_abs << "/" << fn << ".h and lib" << fn << ".so\n";
  return 0;
}
