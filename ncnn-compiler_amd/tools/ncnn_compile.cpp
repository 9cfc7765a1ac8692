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
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <set>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/nhip_graph.h"

namespace {

struct Options {
  std::string param, bin, model_name, output_dir, runtime_dir, precision = "auto";
  std::vector<std::vector<int64_t>> input_shapes;
  bool emit_manifest = false, verbose = false, keep_source = false;
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
    } else if (a == "--emit-manifest") {
      o.emit_manifest = true;
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

int run(const std::vector<std::string>& cmd, bool verbose) {
  std::string line;
  for (auto& c : cmd) line += (line.empty() ? "" : " ") + c;
  if (verbose) std::cerr << "+ " << line << "\n";
  const pid_t pid = fork();
  if (pid < 0) die("fork failed");
  if (pid == 0) {
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
      j << (i ? ",\n    " : "\n    ") << "{\n      \"dynamic_dim_mask\": " << v[i].mask << ",\n      \"element_type\": \""
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
    << "static void init_exec(void) {\n  g_exec_status = nhip_init(0);\n  if (g_exec_status == 0)\n"
    << "    g_exec_status = nhip_graph_load(nhip_model_param, (uint64_t)(nhip_model_param_end - nhip_model_param),\n"
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
    << "  pthread_once(&g_exec_once, init_exec);\n  if (g_exec_status != 0) return g_exec_status;\n"
    << shape_block() << "  const void* ins[] = {";
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
    s << ") return 1;\n  pthread_once(&g_desc_once, init_desc);\n  if (g_desc_status != 0) return g_desc_status;\n"
      << shape_block() << "  int64_t oshape[" << 4 * outs.size() << "];\n  int32_t orank[" << outs.size() << "];\n"
      << "  const int st = nhip_graph_infer_shapes(g_desc, shapes, oshape, orank);\n  if (st != 0) return st;\n";
    for (size_t j = 0; j < outs.size(); ++j)
      if (outs[j].mask)
        for (size_t k = 0; k < outs[j].shape.size(); ++k)
          s << "  " << outs[j].name << "_shape[" << k << "] = oshape[" << 4 * j + k << "];\n";
    s << "  return 0;\n}\n";
  }
  return s.str();
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
      a.ctype = dtype == NHIP_DTYPE_I8 ? "int8_t" : "float";
      a.etype = dtype == NHIP_DTYPE_I8 ? "i8" : "f32";
      for (int k = 0; k < rank; ++k) {
        a.shape.push_back(dims[k]);
        if (dims[k] < 0) a.mask |= 1u << k;
      }
      (io ? outs : ins).push_back(a);
    }
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
  std::vector<std::string> cmd = {cxx && *cxx ? cxx : "g++", "-O2", "-fPIC", "-shared", "-std=c++17",
                                  "-fvisibility=hidden", "-I" + include_dir,
                                  src_dir + "/" + fn + "_wrapper.cpp", "-o", stage + "/lib" + fn + ".so",
                                  "-L" + runtime_dir, "-lnhip", "-Wl,-rpath," + runtime_dir,
                                  "-Wl,--version-script=" + src_dir + "/exports.map", "-Wl,-z,defs",
                                  "-Wl,--build-id=none", "-lpthread"};
  if (run(cmd, o.verbose) != 0) die("compiling the model library failed");
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
