// CPU sanitizer driver for the model front end (parser, weight loader,
// lowering and shape inference of csrc/graph.cpp), built with
// -fsanitize=address,undefined by tests/test_cpu_sanitize.py.  Everything
// goes through nhip_graph_describe, which does no device work.
//
//   describe_fuzz describe <model.param> <model.bin | -> [CxHxW ...]
//       prints "<status> <message>" for one model
//   describe_fuzz fuzz <model.param> <model.bin> <iterations> <seed> [CxHxW ...]
//       describes seeded mutants of the model (corrupted numbers, flipped
//       bytes, dropped or repeated lines, truncated or extended payloads)
//       and prints how many were accepted; a sanitizer report aborts.
// CxHxW: Input shape overrides in source order ('?' = dynamic).
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include "nhip_graph.h"

namespace {

std::string slurp(const char* path) {
  std::ifstream f(path, std::ios::binary);
  std::ostringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

uint64_t splitmix(uint64_t& s) {
  uint64_t z = (s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

std::vector<int64_t> g_shapes;  // 3 extents per Input override

void parse_shapes(int first, int argc, char** argv) {
  for (int a = first; a < argc; ++a) {
    std::string s = argv[a];
    size_t pos = 0;
    for (int k = 0; k < 3; ++k) {
      const size_t x = s.find('x', pos);
      const std::string tok = s.substr(pos, x == std::string::npos ? std::string::npos : x - pos);
      g_shapes.push_back(tok == "?" ? -1 : std::atoll(tok.c_str()));
      pos = x == std::string::npos ? s.size() : x + 1;
    }
  }
}

int describe(const std::string& param, const std::string* bin, std::string* msg) {
  nhip_graph_t g = nullptr;
  const int st = nhip_graph_describe(param.data(), param.size(), bin ? bin->data() : nullptr, bin ? bin->size() : 0,
                                     g_shapes.empty() ? nullptr : g_shapes.data(), (int32_t)(g_shapes.size() / 3), &g);
  if (msg) *msg = nhip_last_error();
  if (st == 0) {
    int32_t ni = 0, no = 0;
    nhip_graph_num_io(g, &ni, &no);
    for (int32_t i = 0; i < ni + no; ++i) {
      int32_t rank = 0, dtype = 0;
      int64_t dims[4];
      const char* name = nullptr;
      nhip_graph_io_info(g, i >= ni, i >= ni ? i - ni : i, &rank, dims, &dtype, &name);
    }
    std::vector<int64_t> oshape(4 * (size_t)(no > 0 ? no : 1));
    std::vector<int32_t> orank((size_t)(no > 0 ? no : 1));
    (void)nhip_graph_infer_shapes(g, nullptr, oshape.data(), orank.data());
    nhip_graph_destroy(g);
  }
  return st;
}

// One mutation of the .param text or the .bin payload.
void mutate(std::string& param, std::string& bin, uint64_t& rng) {
  static const char* kValues[] = {"0",          "-1",   "1",     "2147483647", "2147483648", "9223372036854775807",
                                  "-233",       "-234", "65536", "1e30",       "nan",        "-23301=2,1,2",
                                  "3.5",        "",     "x",     "-2147483648", "4294967296", "1,2"};
  const uint64_t r = splitmix(rng);
  switch (r % 7) {
    case 0: {  // replace the value of one key=value token
      std::vector<size_t> eqs;
      for (size_t i = 0; i < param.size(); ++i)
        if (param[i] == '=') eqs.push_back(i);
      if (eqs.empty()) break;
      const size_t at = eqs[splitmix(rng) % eqs.size()] + 1;
      size_t end = at;
      while (end < param.size() && param[end] != ' ' && param[end] != '\n') ++end;
      param.replace(at, end - at, kValues[splitmix(rng) % (sizeof kValues / sizeof *kValues)]);
      break;
    }
    case 1: {  // replace one whitespace-separated token anywhere
      std::vector<size_t> starts;
      for (size_t i = 0; i < param.size(); ++i)
        if (param[i] != ' ' && param[i] != '\n' && (i == 0 || param[i - 1] == ' ' || param[i - 1] == '\n'))
          starts.push_back(i);
      if (starts.empty()) break;
      const size_t at = starts[splitmix(rng) % starts.size()];
      size_t end = at;
      while (end < param.size() && param[end] != ' ' && param[end] != '\n') ++end;
      param.replace(at, end - at, kValues[splitmix(rng) % (sizeof kValues / sizeof *kValues)]);
      break;
    }
    case 2: {  // drop or repeat a line
      std::vector<std::string> lines;
      std::istringstream in(param);
      std::string l;
      while (std::getline(in, l)) lines.push_back(l);
      if (lines.empty()) break;
      const size_t i = splitmix(rng) % lines.size();
      if (splitmix(rng) & 1) lines.erase(lines.begin() + (long)i);
      else lines.insert(lines.begin() + (long)i, lines[i]);
      param.clear();
      for (auto& x : lines) param += x + "\n";
      break;
    }
    case 3:  // flip a byte of the text
      if (!param.empty()) param[splitmix(rng) % param.size()] ^= (char)(1 + splitmix(rng) % 255);
      break;
    case 4:  // truncate the payload
      if (!bin.empty()) bin.resize(splitmix(rng) % bin.size());
      break;
    case 5:  // flip payload bytes (weight flags, counts, values)
      for (int k = 0; k < 4 && !bin.empty(); ++k) bin[splitmix(rng) % bin.size()] ^= (char)(1 + splitmix(rng) % 255);
      break;
    default:  // extend the payload
      bin.append(1 + splitmix(rng) % 9, (char)splitmix(rng));
      break;
  }
}

}  // namespace

int main(int argc, char** argv) {
  if (argc >= 4 && std::strcmp(argv[1], "describe") == 0) {
    parse_shapes(4, argc, argv);
    const std::string param = slurp(argv[2]);
    std::string bin;
    const bool has_bin = std::strcmp(argv[3], "-") != 0;
    if (has_bin) bin = slurp(argv[3]);
    std::string msg;
    const int st = describe(param, has_bin ? &bin : nullptr, &msg);
    std::printf("%d %s\n", st, msg.c_str());
    return 0;
  }
  if (argc >= 6 && std::strcmp(argv[1], "fuzz") == 0) {
    parse_shapes(6, argc, argv);
    const std::string param0 = slurp(argv[2]), bin0 = slurp(argv[3]);
    const long iters = std::atol(argv[4]);
    uint64_t rng = std::strtoull(argv[5], nullptr, 10);
    long accepted = 0;
    for (long it = 0; it < iters; ++it) {
      std::string param = param0, bin = bin0;
      const int edits = 1 + (int)(splitmix(rng) % 3);
      for (int e = 0; e < edits; ++e) mutate(param, bin, rng);
      if (describe(param, &bin, nullptr) == 0) ++accepted;
    }
    std::printf("mutants %ld accepted %ld\n", iters, accepted);
    return 0;
  }
  std::fprintf(stderr, "usage: describe_fuzz describe <param> <bin|->\n       describe_fuzz fuzz <param> <bin> <n> <seed>\n");
  return 2;
}
