// The StableHLO front end: AST, parser, op table and executor.
//
// The same surface as the reference's Lean front end: the AST of
// StablehloMlx/Ast.lean, the generic-form reader of StablehloMlx/Parse.lean,
// the op table of StablehloMlx/Lower.lean and the load/prepare/call of
// StablehloMlx/Exec.lean, re-expressed in C++ over this executor's runtime.
#pragma once

#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "ops.h"

namespace shlo {

// ---- AST (StablehloMlx/Ast.lean:12-60) -----------------------------------------

struct Ty {
  std::vector<int64_t> dims;  // slowest first, as MLIR writes them
  std::string el;
  int64_t count() const { return shape_count(dims); }
  std::string str() const;
};

struct Block;

struct Op {
  std::vector<std::string> results;
  std::string name;
  std::vector<std::string> operands;
  std::vector<std::pair<std::string, std::string>> attrs;  // raw attribute text
  std::vector<Block> regions;
  std::vector<Ty> in_tys, out_tys;
  const std::string *attr(const std::string &k) const;
};

struct Block {
  std::vector<std::pair<std::string, Ty>> args;
  std::vector<Op> ops;
  std::vector<std::string> ret;
};

struct Func {
  std::string name;
  Block body;
  std::vector<Ty> out_tys;
};

struct Module {
  std::vector<Func> funcs;
  const Func *func(const std::string &n) const;
};

// Parse.parse (StablehloMlx/Parse.lean:247).  Throws Error("parse error at …").
Module parse_module(const std::string &text);

// ---- the op table (StablehloMlx/Lower.lean) ---------------------------------------

// Planted wrong lowerings (Lower.lean:53-69), one bit each in this order.
struct Faults {
  bool dot_builtin = false, dot_plain = false, soft_max_float_sum = false, norm_gpu_ops = false,
       silu_gpu_ops = false, gelu_tanh = false, divide_builtin = false, sqrt_builtin = false,
       binary_half = false, broadcast_first = false, concat_swap = false, transpose_identity = false,
       slice_shift = false, f64_as_f32 = false, while_short = false;
  static Faults from_bits(uint64_t b);
};

uint8_t el_dtype(const std::string &el);  // Lower.elDtype (Lower.lean:97-107)
size_t el_bytes(const std::string &el);   // Lower.elBytes (Lower.lean:109-110)

std::vector<ArrayP> run_func(const Module &m, const Faults &f, const Func &fn, const std::vector<ArrayP> &args);

// ---- the executor (StablehloMlx/Exec.lean:17-43) -----------------------------------

struct Loaded {
  Module module;
  const Func &main() const { return *module.func("main"); }
};
Loaded load_module(const std::string &text);

}  // namespace shlo
