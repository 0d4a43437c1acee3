// shlo_hip — run a StableHLO module on the MI355X.
//
//   shlo_hip <module.mlir> <out-prefix> <arg0.bin> [arg1.bin ...] [--no-compile] [--repeat N]
//
// The surface of the reference's shlo_mlx (Main.lean:16-48): each argument
// file holds @main's argument as raw little-endian elements in row-major
// order; each result is written to <out-prefix><i>.bin the same way.  The
// module is hipGraph-compiled unless --no-compile; --repeat N calls it N times
// and prints the per-call time.  Built on the C ABI only (include/shlo_hip.h).
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iterator>
#include <string>
#include <vector>

#include "shlo_hip.h"

namespace {

bool is_nat(const std::string &s) {
  if (s.empty()) return false;
  for (char c : s)
    if (c < '0' || c > '9') return false;
  return true;
}

bool read_file(const std::string &p, std::string *out) {
  std::ifstream f(p, std::ios::binary);
  if (!f) return false;
  out->assign(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
  return true;
}

size_t dtype_size(uint8_t dt) {
  switch (dt) {
    case 0: case 1: case 5: return 1;
    case 2: case 6: case 9: return 2;
    case 3: case 7: case 10: return 4;
    default: return 8;
  }
}

int die(const char *what) {
  fprintf(stderr, "%s: %s\n", what, shlo_last_error());
  return 1;
}

double now_ms() {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

}  // namespace

int main(int argc, char **argv) {
  std::vector<std::string> args(argv + 1, argv + argc);
  bool compile = true;
  long repeat = 1;
  for (size_t i = 0; i < args.size(); i++) {
    if (args[i] == "--no-compile") compile = false;
    if (args[i] == "--repeat" && i + 1 < args.size()) repeat = std::atol(args[i + 1].c_str());
  }
  std::vector<std::string> pos;  // positional: not a flag, not a number (Main.lean:66)
  for (auto &a : args)
    if (a.rfind("--", 0) != 0 && !is_nat(a)) pos.push_back(a);
  if (pos.size() < 2) {
    fprintf(stderr, "usage: shlo_hip <module.mlir> <out-prefix> <arg0.bin> [arg1.bin ...] [--no-compile] [--repeat N]\n");
    return 2;
  }
  std::string text;
  if (!read_file(pos[0], &text)) {
    fprintf(stderr, "cannot read %s\n", pos[0].c_str());
    return 1;
  }
  shlo_module *m = nullptr;
  if (shlo_module_load(text.data(), text.size(), &m)) return die("load");
  size_t nargs = 0;
  shlo_module_nargs(m, &nargs);
  if (nargs != pos.size() - 2) {
    fprintf(stderr, "@main takes %zu arguments, %zu files given\n", nargs, pos.size() - 2);
    return 2;
  }
  std::vector<shlo_arr *> ins;
  for (size_t i = 0; i < nargs; i++) {
    int64_t shape[16];
    size_t rank = 0;
    uint8_t dt = 0;
    if (shlo_module_arg(m, i, shape, 16, &rank, &dt)) return die("argTys");
    std::string bytes;
    if (!read_file(pos[2 + i], &bytes)) {
      fprintf(stderr, "cannot read %s\n", pos[2 + i].c_str());
      return 1;
    }
    size_t count = 1;
    for (size_t k = 0; k < rank; k++) count *= (size_t)shape[k];
    if (bytes.size() != count * dtype_size(dt)) {
      fprintf(stderr, "%s: %zu bytes, argument %zu needs %zu\n", pos[2 + i].c_str(), bytes.size(), i,
              count * dtype_size(dt));
      return 1;
    }
    shlo_arr *a = nullptr;
    if (shlo_of_bytes(bytes.data(), bytes.size(), shape, rank, dt, &a)) return die("ofBytes");
    ins.push_back(a);
  }
  if (shlo_eval(ins.data(), ins.size())) return die("eval");
  const double t0 = now_ms();
  shlo_fn *f = nullptr;
  if (shlo_module_prepare(m, 0, compile ? 1 : 0, &f)) return die("prepare");
  std::vector<shlo_arr *> outs(64, nullptr);
  size_t nout = 0;
  if (shlo_call(f, ins.data(), ins.size(), outs.data(), outs.size(), &nout)) return die("call");
  const double t1 = now_ms();
  printf("first call (trace + compile + run): %f ms\n", t1 - t0);
  if (repeat > 1) {
    const double t2 = now_ms();
    for (long r = 1; r < repeat; r++) {
      for (size_t k = 0; k < nout; k++) shlo_arr_free(outs[k]);
      if (shlo_call(f, ins.data(), ins.size(), outs.data(), outs.size(), &nout)) return die("call");
    }
    const double t3 = now_ms();
    printf("per call over %ld: %f ms\n", repeat - 1, (t3 - t2) / (double)(repeat - 1));
  }
  for (size_t k = 0; k < nout; k++) {
    size_t nb = 0;
    if (shlo_to_bytes(outs[k], nullptr, 0, &nb)) return die("toBytes");
    std::vector<char> buf(nb);
    if (shlo_to_bytes(outs[k], buf.data(), buf.size(), &nb)) return die("toBytes");
    const std::string p = pos[1] + std::to_string(k) + ".bin";
    std::ofstream o(p, std::ios::binary);
    o.write(buf.data(), (std::streamsize)buf.size());
    if (!o) {
      fprintf(stderr, "cannot write %s\n", p.c_str());
      return 1;
    }
    shlo_arr_free(outs[k]);
  }
  for (auto *a : ins) shlo_arr_free(a);
  shlo_fn_free(f);
  shlo_module_free(m);
  return 0;
}
