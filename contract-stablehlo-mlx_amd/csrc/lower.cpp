// The op table: each StableHLO op as executor ops (StablehloMlx/Lower.lean).
//
// Exactness, op by op, is the reference's policy (Lower.lean:12-44): data
// movement and single-rounding arithmetic are exact in any order; f32 divide
// and sqrt are the correctly rounded GPU operations; dot_general is
// ggml_vec_dot_f32's order; composites / custom_calls named ggml.norm,
// ggml.soft_max, ggml.silu and ggml.gelu_erf run ggml-cpu's routine, any other
// composite its decomposition.  Binary32 attributes are hex bit patterns.
//
// Differences from the reference, each giving the same bits:
// * dot_general reads its operands in place through (batch, free, k) strides
//   when the dims flatten, instead of transposing both to [B*free, K] first
//   (Lower.lean:173-175);
// * f64 tensors are native binary64 arrays (the reference carries them as
//   uint64 bit patterns with soft-float kernels because Metal has no binary64,
//   Lower.lean:253-298); the .bin bytes are the same.
#include <algorithm>
#include <cstring>

#include "stablehlo.h"

namespace shlo {

Faults Faults::from_bits(uint64_t b) {
  Faults f;
  bool *fs[] = {&f.dot_builtin, &f.dot_plain, &f.soft_max_float_sum, &f.norm_gpu_ops, &f.silu_gpu_ops,
                &f.gelu_tanh, &f.divide_builtin, &f.sqrt_builtin, &f.binary_half, &f.broadcast_first,
                &f.concat_swap, &f.transpose_identity, &f.slice_shift, &f.f64_as_f32, &f.while_short};
  for (size_t i = 0; i < sizeof fs / sizeof fs[0]; i++) *fs[i] = (b >> i) & 1;
  return f;
}

namespace {

using Env = std::unordered_map<std::string, ArrayP>;
using Known = std::unordered_map<std::string, int64_t>;

ArrayP get(const Env &env, const std::string &n) {
  auto it = env.find(n);
  if (it == env.end()) fail("undefined value " + n);
  return it->second;
}

bool starts_with(const std::string &s, const std::string &p) { return s.compare(0, p.size(), p) == 0; }
bool ends_with(const std::string &s, const std::string &p) {
  return s.size() >= p.size() && s.compare(s.size() - p.size(), p.size(), p) == 0;
}
std::vector<std::string> split(const std::string &s, const std::string &sep) {
  std::vector<std::string> r;
  size_t b = 0;
  for (;;) {
    size_t e = s.find(sep, b);
    if (e == std::string::npos) {
      r.push_back(s.substr(b));
      return r;
    }
    r.push_back(s.substr(b, e - b));
    b = e + sep.size();
  }
}
std::string trim(const std::string &s) {
  size_t a = s.find_first_not_of(" \t\n\r"), e = s.find_last_not_of(" \t\n\r");
  return a == std::string::npos ? std::string() : s.substr(a, e - a + 1);
}
std::string replace_all(std::string s, const std::string &a, const std::string &b) {
  size_t p = 0;
  while ((p = s.find(a, p)) != std::string::npos) {
    s.replace(p, a.size(), b);
    p += b.size();
  }
  return s;
}
std::string attr_or(const Op &o, const char *k, const std::string &d) {
  const std::string *v = o.attr(k);
  return v ? *v : d;
}

// The integers in `array<i64: 1, 2>`, `[1, 2]` or `dense<[1, 2]> : …`
// (Lower.lean:82-89).
std::vector<int64_t> ints(const std::string &s) {
  std::string body;
  auto parts = split(s, ":");
  if (parts.size() >= 2) {
    if (starts_with(s, "array<")) {
      body = s.substr(s.find(':') + 1);
    } else {
      body = s;
    }
  } else {
    body = starts_with(s, "array<") ? std::string() : s;
  }
  std::vector<int64_t> r;
  int64_t cur = -1;
  for (char c : body) {
    if (c >= '0' && c <= '9') cur = (cur < 0 ? 0 : cur * 10) + (c - '0');
    else if (cur >= 0) r.push_back(cur), cur = -1;
  }
  if (cur >= 0) r.push_back(cur);
  return r;
}

// The value of `key = …` inside a `#stablehlo.dot<…>`-style text (Lower.lean:92-95).
std::string field(const std::string &s, const std::string &key) {
  auto parts = split(s, key + " = ");
  if (parts.size() < 2) return "";
  return split(parts[1], "]")[0] + "]";
}

// One literal of a dense<…> attribute as its bit pattern (Lower.lean:113-125).
uint64_t literal_bits(const std::string &el, const std::string &lit) {
  const std::string t = trim(lit);
  if (t == "true") return 1;
  if (t == "false") return 0;
  if (starts_with(t, "0x") || starts_with(t, "0X")) {
    uint64_t v = 0;
    for (size_t i = 2; i < t.size(); i++) {
      const char c = (char)std::tolower(t[i]);
      v = v * 16 + (uint64_t)(std::isdigit(c) ? c - '0' : c - 'a' + 10);
    }
    return v;
  }
  if (starts_with(el, "f")) fail("decimal float literal " + t + " for " + el + ": write it as a hex bit pattern so it is exact");
  const bool neg = starts_with(t, "-");
  const uint64_t mag = std::stoull(neg ? t.substr(1) : t);
  const size_t w = 8 * el_bytes(el);
  if (!neg) return mag;
  return w >= 64 ? (uint64_t)0 - mag : (((uint64_t)1 << w) - mag);
}

std::vector<uint8_t> bytes_of(const std::string &el, const std::vector<uint64_t> &bits) {
  const size_t w = el_bytes(el);
  std::vector<uint8_t> b;
  b.reserve(w * bits.size());
  for (uint64_t x : bits)
    for (size_t k = 0; k < w; k++) b.push_back((uint8_t)(x >> (8 * k)));
  return b;
}

ArrayP constant_op(const Op &o) {  // Lower.lean:134-147
  const std::string *v = o.attr("value");
  if (!v) fail("constant without value");
  const Ty &t = o.out_tys.at(0);
  auto dp = split(*v, "dense<");
  std::string inner = dp.size() > 1 ? dp[1] : "";
  inner = split(inner, ">")[0];
  inner = replace_all(replace_all(inner, "[", ""), "]", "");
  std::vector<uint64_t> bits;
  for (auto &l : split(inner, ","))
    if (!trim(l).empty()) bits.push_back(literal_bits(t.el, l));
  const uint8_t dt = el_dtype(t.el);
  if (bits.size() == 1 && t.count() != 1) {
    auto b = bytes_of(t.el, bits);
    return broadcast_to(array_from_host(b.data(), b.size(), Shape{}, dt), t.dims);
  }
  if ((int64_t)bits.size() != t.count()) fail(strf("constant has %zu values for %s", bits.size(), t.str().c_str()));
  auto b = bytes_of(t.el, bits);
  return array_from_host(b.data(), b.size(), t.dims, dt);
}

// The f32 bit pattern of `key = 0x… : f32` in a composite's attributes (Lower.lean:150-153).
uint32_t f32_attr(const std::string &attrs, const std::string &key) {
  auto parts = split(attrs, key + " = ");
  if (parts.size() < 2) fail("composite attribute " + key + " missing");
  return (uint32_t)literal_bits("f32", split(parts[1], " ")[0]);
}

// ---- dot_general ---------------------------------------------------------------------

// Express dims `ds` of `a` (in that order) as one stride, if they flatten.
bool flat_stride(const ArrayP &a, const std::vector<int64_t> &ds, int64_t *stride) {
  std::vector<int64_t> nz;  // the non-unit dims, outer to inner
  for (int64_t d : ds)
    if (a->shape[d] != 1) nz.push_back(d);
  for (size_t i = 0; i + 1 < nz.size(); i++)
    if (a->strides[nz[i]] != a->strides[nz[i + 1]] * a->shape[nz[i + 1]]) return false;
  *stride = nz.empty() ? 0 : a->strides[nz.back()];
  return true;
}

DotOperand dot_operand(const ArrayP &a, const std::vector<int64_t> &batch, const std::vector<int64_t> &free,
                       int64_t contract) {
  DotOperand op;
  int64_t sb = 0, sf = 0;
  if (flat_stride(a, free, &sf)) {
    if (flat_stride(a, batch, &sb)) {
      op.arr = a;
      op.sb = sb;
      op.sf = sf;
      op.sk = a->strides[contract];
      return op;
    }
    // Two batch levels: outer dims [0, k) and inner dims [k, end), each flat
    // (per-head views such as [B, H, T, dh] over a [B, T, H*dh] buffer).
    for (size_t k = 1; k < batch.size(); k++) {
      const std::vector<int64_t> outer(batch.begin(), batch.begin() + k), inner(batch.begin() + k, batch.end());
      int64_t s1 = 0, s2 = 0, n2 = 1;
      for (int64_t d : inner) n2 *= a->shape[d];
      if (n2 > 1 && flat_stride(a, outer, &s1) && flat_stride(a, inner, &s2)) {
        op.arr = a;
        op.sb = s1;
        op.sb2 = s2;
        op.nb2 = n2;
        op.sf = sf;
        op.sk = a->strides[contract];
        return op;
      }
    }
  }
  // Not flattenable: copy to [batch, free, contract] (the reference's layout).
  std::vector<int64_t> perm(batch);
  perm.insert(perm.end(), free.begin(), free.end());
  perm.push_back(contract);
  ArrayP c = contiguous(transpose(a, perm));
  int64_t F = 1, K = a->shape[contract];
  for (int64_t d : free) F *= a->shape[d];
  op.arr = c;
  op.sb = F * K;
  op.sf = K;
  op.sk = 1;
  return op;
}

// An element-wise op that follows a producer: `other` is its second operand,
// `rev` says the produced value is its right operand; code kEpiGeluErf is
// ggml.gelu_erf (no operand).
struct Chained {
  uint32_t code;
  bool rev;
  ArrayP other;
};

// Applies the chain's ops from `from` on as separate kernels.
ArrayP apply_chain(ArrayP v, const std::vector<Chained> &chain, size_t from) {
  for (size_t i = from; i < chain.size(); i++) {
    const Chained &c = chain[i];
    if (c.code == kEpiGeluErf) v = reshape(gelu_erf(v, false), v->shape);
    else v = c.rev ? binary(c.code, c.other, v) : binary(c.code, v, c.other);
  }
  return v;
}

// The chain's leading ops that a producer with output index (i0, i1, i2) over
// the dim groups g0, g1, g2 of `dims` can fuse: each other operand f32 of
// shape `dims`, its strides flat over every group.
std::vector<FusedOp> fusable_prefix(const std::vector<Chained> &chain, const Shape &dims,
                                    const std::vector<int64_t> (&g)[3], bool gelu_ok) {
  std::vector<FusedOp> out;
  for (const Chained &c : chain) {
    if ((int)out.size() == kMaxEpi) break;
    if (c.code == kEpiGeluErf) {
      if (!gelu_ok) break;
      FusedOp op;
      op.code = kEpiGeluErf;
      out.push_back(op);
      continue;
    }
    if (c.other->dtype != kF32 || c.other->shape != dims || !c.other->buf) break;
    FusedOp op;
    if (!flat_stride(c.other, g[0], &op.s0) || !flat_stride(c.other, g[1], &op.s1) ||
        !flat_stride(c.other, g[2], &op.s2))
      break;
    op.arr = c.other;
    op.code = c.code;
    op.rev = c.rev;
    out.push_back(op);
  }
  return out;
}

// dot_general's dimension numbers: false when the lowering would refuse them.
bool dot_dims(const Op &o, std::vector<int64_t> *lb, std::vector<int64_t> *rb, std::vector<int64_t> *lc,
              std::vector<int64_t> *rc) {
  const std::string dn = attr_or(o, "dot_dimension_numbers", "");
  *lb = ints(field(dn, "lhs_batching_dimensions"));
  *rb = ints(field(dn, "rhs_batching_dimensions"));
  *lc = ints(field(dn, "lhs_contracting_dimensions"));
  *rc = ints(field(dn, "rhs_contracting_dimensions"));
  if (o.in_tys.size() != 2 || o.out_tys.size() != 1) return false;
  return lc->size() == 1 && rc->size() == 1 && lb->size() == rb->size();
}

ArrayP dot_general(const Faults &f, const Op &o, const ArrayP &a, const ArrayP &b,
                   const std::vector<Chained> &chain = {}) {  // Lower.lean:157-182
  const std::string dn = attr_or(o, "dot_dimension_numbers", "");
  const auto lb = ints(field(dn, "lhs_batching_dimensions"));
  const auto rb = ints(field(dn, "rhs_batching_dimensions"));
  const auto lc = ints(field(dn, "lhs_contracting_dimensions"));
  const auto rc = ints(field(dn, "rhs_contracting_dimensions"));
  const Ty &ta = o.in_tys.at(0), &tb = o.in_tys.at(1);
  if (lc.size() != 1 || rc.size() != 1) fail("dot_general: one contracting dimension is carried");
  if (lb.size() != rb.size()) fail("dot_general: batching dimensions differ in number");
  auto contains = [](const std::vector<int64_t> &v, int64_t d) { return std::find(v.begin(), v.end(), d) != v.end(); };
  std::vector<int64_t> lf, rf;
  for (int64_t d = 0; d < (int64_t)ta.dims.size(); d++)
    if (!contains(lb, d) && !contains(lc, d)) lf.push_back(d);
  for (int64_t d = 0; d < (int64_t)tb.dims.size(); d++)
    if (!contains(rb, d) && !contains(rc, d)) rf.push_back(d);
  auto prod = [](const Ty &t, const std::vector<int64_t> &ds) {
    int64_t n = 1;
    for (int64_t d : ds) n *= t.dims.at(d);
    return n;
  };
  const int64_t B = prod(ta, lb), N = prod(ta, lf), M = prod(tb, rf), K = ta.dims.at(lc[0]);
  if (tb.dims.at(rc[0]) != K) fail("dot_general: contracting dimensions differ");
  if (prod(tb, rb) != B) fail("dot_general: batch extents differ");
  const Ty &out = o.out_tys.at(0);
  if (a->shape != ta.dims || b->shape != tb.dims) fail("dot_general: operand shapes differ from the op's types");
  if (f.dot_builtin) {  // planted: a built-in matmul's own order (Lower.lean:177-180)
    std::vector<int64_t> pa(lb), pb(rb);
    pa.insert(pa.end(), lf.begin(), lf.end());
    pa.push_back(lc[0]);
    pb.insert(pb.end(), rf.begin(), rf.end());
    pb.push_back(rc[0]);
    ArrayP a3 = reshape(transpose(a, pa), Shape{B, N, K});
    ArrayP b3 = transpose(reshape(transpose(b, pb), Shape{B, M, K}), {0, 2, 1});
    return apply_chain(reshape(matmul_builtin(a3, b3), out.dims), chain, 0);
  }
  DotOperand L = dot_operand(a, lb, lf, lc[0]);
  DotOperand R = dot_operand(b, rb, rf, rc[0]);
  // Output dims: the batch dims, lhs free dims, rhs free dims (index b, n, m).
  std::vector<int64_t> g[3];
  const size_t nb = lb.size(), nl = lf.size();
  for (size_t d = 0; d < out.dims.size(); d++) g[d < nb ? 0 : d < nb + nl ? 1 : 2].push_back((int64_t)d);
  const std::vector<FusedOp> epi = fusable_prefix(chain, out.dims, g, true);
  ArrayP y = dot_ggml(L, R, B, N, M, K, f.dot_plain ? (int)kTailPlain : default_dot_tail(), epi);
  return apply_chain(reshape(y, out.dims), chain, epi.size());
}

// ---- op codes --------------------------------------------------------------------------

bool unary_code(const std::string &n, uint32_t *c) {  // Lower.lean:186-194
  static const std::pair<const char *, uint32_t> t[] = {
      {"stablehlo.negate", kNeg}, {"stablehlo.abs", kAbs}, {"stablehlo.floor", kFloor},
      {"stablehlo.not", kInvert}, {"stablehlo.exponential", kExp}, {"stablehlo.tanh", kTanh},
      {"stablehlo.logistic", kSigmoid}};
  for (auto &kv : t)
    if (n == kv.first) return *c = kv.second, true;
  return false;
}

bool binary_code(const std::string &n, uint32_t *c) {  // Lower.lean:196-208
  static const std::pair<const char *, uint32_t> t[] = {
      {"stablehlo.add", kAdd}, {"stablehlo.subtract", kSub}, {"stablehlo.multiply", kMul},
      {"stablehlo.maximum", kMax}, {"stablehlo.minimum", kMin}, {"stablehlo.and", kAnd},
      {"stablehlo.or", kOr}, {"stablehlo.xor", kXor}, {"stablehlo.shift_left", kShl},
      {"stablehlo.shift_right_logical", kShr}, {"stablehlo.remainder", kRem}};
  for (auto &kv : t)
    if (n == kv.first) return *c = kv.second, true;
  return false;
}

std::string direction(const Op &o) {  // Lower.lean:211-213
  const std::string t = attr_or(o, "comparison_direction", "");
  auto parts = split(t, "comparison_direction ");
  return trim(replace_all(parts.back(), ">", ""));
}

uint32_t compare_code(const std::string &dir) {
  if (ends_with(dir, "EQ")) return kEq;
  if (ends_with(dir, "NE")) return kNe;
  if (ends_with(dir, "LT")) return kLt;
  if (ends_with(dir, "LE")) return kLe;
  if (ends_with(dir, "GT")) return kGt;
  if (ends_with(dir, "GE")) return kGe;
  fail("comparison " + dir);
}

bool is_int_el(const std::string &el) {
  static const char *t[] = {"i1", "i8", "ui8", "i32", "si32", "ui32", "i64", "si64", "ui64"};
  for (auto *x : t)
    if (el == x) return true;
  return false;
}

// Scalars known at trace time (Lower.lean:228-251).
bool const_eval(const Known &known, const Op &o, int64_t *out) {
  if (o.out_tys.empty()) return false;
  const Ty &t = o.out_tys[0];
  if (!t.dims.empty() || !is_int_el(t.el)) return false;
  auto k = [&](size_t i, int64_t *v) {
    if (i >= o.operands.size()) return false;
    auto it = known.find(o.operands[i]);
    if (it == known.end()) return false;
    *v = it->second;
    return true;
  };
  int64_t a, b;
  if (o.name == "stablehlo.constant") {
    const std::string *v = o.attr("value");
    if (!v) return false;
    auto dp = split(*v, "dense<");
    const std::string s = trim(split(dp.size() > 1 ? dp[1] : "", ">")[0]);
    if (s == "true") return *out = 1, true;
    if (s == "false") return *out = 0, true;
    try {
      size_t pos = 0;
      const long long x = std::stoll(s, &pos);
      if (pos != s.size()) return false;
      *out = x;
      return true;
    } catch (...) {
      return false;
    }
  }
  if (o.name == "stablehlo.add") return k(0, &a) && k(1, &b) ? (*out = a + b, true) : false;
  if (o.name == "stablehlo.subtract") return k(0, &a) && k(1, &b) ? (*out = a - b, true) : false;
  if (o.name == "stablehlo.multiply") return k(0, &a) && k(1, &b) ? (*out = a * b, true) : false;
  if (o.name == "stablehlo.convert") return k(0, out);
  if (o.name == "stablehlo.compare") {
    if (!k(0, &a) || !k(1, &b)) return false;
    const std::string d = direction(o);
    bool r = ends_with(d, "EQ") ? a == b : ends_with(d, "NE") ? a != b : ends_with(d, "LT") ? a < b
           : ends_with(d, "LE") ? a <= b : ends_with(d, "GT") ? a > b : a >= b;
    *out = r ? 1 : 0;
    return true;
  }
  return false;
}

std::pair<int64_t, int64_t> rows_cols(const Ty &t) {  // Lower.lean:301-303
  const int64_t c = t.dims.empty() ? 1 : t.dims.back();
  return {t.count() / std::max<int64_t>(c, 1), c};
}

ArrayP convert_op(const ArrayP &a, const Ty &src, const Ty &out) {  // Lower.lean:306-315
  // binary64 converts only to and from binary32 and to int64 (toward zero,
  // saturating, NaN to 0), as the reference's soft-float kernels do.
  if (src.el == "f64" && out.el != "f32" && out.el != "f64" && out.el != "i64" && out.el != "si64")
    fail("convert f64 to " + out.el + " is not carried");
  if (out.el == "f64" && src.el != "f32" && src.el != "f64") fail("convert " + src.el + " to f64 is not carried");
  return astype(a, el_dtype(out.el));
}

ArrayP gather1d(const Op &o, const ArrayP &table, const ArrayP &idx) {  // Lower.lean:319-331
  const std::string dn = attr_or(o, "dimension_numbers", "");
  const Ty &t = o.in_tys.at(0), &it = o.in_tys.at(1);
  const bool ok = t.dims.size() == 1 && field(dn, "collapsed_slice_dims") == "[0]" &&
                  field(dn, "start_index_map") == "[0]" &&
                  dn.find("index_vector_dim = " + std::to_string(it.dims.size())) != std::string::npos &&
                  ints(attr_or(o, "slice_sizes", "")) == std::vector<int64_t>{1};
  if (!ok) fail("gather: only a 1-D table indexed elementwise is carried (" + dn + ")");
  return take(table, astype(idx, kI64), 0);  // take clamps each index to the table
}

struct Lowerer {
  const Module &m;
  const Faults &f;

  std::vector<ArrayP> run_op(const Env &env, const Known &known, const Op &o) {  // Lower.lean:334-473
    std::vector<ArrayP> args;
    for (auto &n : o.operands) args.push_back(get(env, n));
    const Ty out = o.out_tys.empty() ? Ty{} : o.out_tys[0];
    const std::string &n = o.name;
    const std::string el0 = o.in_tys.empty() ? std::string() : o.in_tys[0].el;
    uint32_t c;
    if (el0 == "f64" && f.f64_as_f32 && binary_code(n, &c) &&
        (n == "stablehlo.add" || n == "stablehlo.subtract" || n == "stablehlo.multiply")) {
      return {astype(binary(c, astype(args[0], kF32), astype(args[1], kF32)), kF64)};
    }
    if (el0 == "f64" && f.f64_as_f32 && n == "stablehlo.divide")
      return {astype(binary(kDiv, astype(args[0], kF32), astype(args[1], kF32)), kF64)};
    if (el0 == "f64" && (n == "stablehlo.sqrt" || n == "stablehlo.exponential" || n == "stablehlo.tanh" ||
                         n == "stablehlo.logistic" || n == "stablehlo.remainder"))
      fail(n + " on f64 is not carried");
    if (el0 == "i1") {  // booleans: logical, not bitwise
      if (n == "stablehlo.and") return {binary(kLAnd, args[0], args[1])};
      if (n == "stablehlo.or") return {binary(kLOr, args[0], args[1])};
      if (n == "stablehlo.xor") return {binary(kNe, args[0], args[1])};
      if (n == "stablehlo.not") return {unary(kNot, args[0])};
    }
    if (n == "stablehlo.shift_right_logical" && !starts_with(el0, "ui"))
      fail("shift_right_logical on " + el0 + " (a signed type) is not carried");
    if (unary_code(n, &c)) return {unary(c, args[0])};
    if (binary_code(n, &c)) {
      if (f.binary_half && out.el == "f32")
        return {astype(binary(c, astype(args[0], kF16), astype(args[1], kF16)), kF32)};
      return {binary(c, args[0], args[1])};
    }
    if (n == "stablehlo.constant") return {constant_op(o)};
    if (n == "stablehlo.divide") {
      if (out.el == "f32") return {binary(f.divide_builtin ? kDivApprox : (uint32_t)kDiv, args[0], args[1])};
      return {binary(kDiv, args[0], args[1])};
    }
    if (n == "stablehlo.sqrt") {
      if (out.el == "f32" && f.sqrt_builtin) return {unary(kSqrtApprox, args[0])};
      return {unary(kSqrt, args[0])};
    }
    if (n == "stablehlo.compare") return {binary(compare_code(direction(o)), args[0], args[1])};
    if (n == "stablehlo.select") return {where(args[0], args[1], args[2])};
    if (n == "stablehlo.reshape") return {reshape(args[0], out.dims)};
    if (n == "stablehlo.transpose") {
      if (f.transpose_identity) return {reshape(args[0], out.dims)};
      return {transpose(args[0], ints(attr_or(o, "permutation", "")))};
    }
    if (n == "stablehlo.broadcast_in_dim") {  // Lower.lean:398-407
      const auto map = ints(attr_or(o, "broadcast_dimensions", ""));
      const Ty &src = o.in_tys.at(0);
      if (f.broadcast_first) {
        ArrayP first = slice(reshape(args[0], Shape{src.count()}), Shape{0}, Shape{1}, Shape{1});
        return {broadcast_to(reshape(first, Shape(out.dims.size(), 1)), out.dims)};
      }
      Shape shp(out.dims.size(), 1);
      for (size_t k = 0; k < map.size(); k++) shp.at(map[k]) = src.dims.at(k);
      return {broadcast_to(reshape(args[0], shp), out.dims)};
    }
    if (n == "stablehlo.slice") {  // Lower.lean:408-416
      Shape st = ints(attr_or(o, "start_indices", "")), li = ints(attr_or(o, "limit_indices", ""));
      Shape sd = ints(attr_or(o, "strides", ""));
      if (sd.empty()) sd.assign(st.size(), 1);
      if (f.slice_shift && !st.empty()) {
        st.back() += 1;
        li.back() += 1;
      }
      return {slice(args[0], st, li, sd)};
    }
    if (n == "stablehlo.dynamic_slice") {  // Lower.lean:417-428
      const Ty &src = o.in_tys.at(0);
      const auto sizes = ints(attr_or(o, "slice_sizes", ""));
      Shape st;
      for (size_t d = 0; d + 1 < o.operands.size(); d++) {
        auto it = known.find(o.operands[d + 1]);
        if (it == known.end())
          fail(strf("dynamic_slice: start %zu (%s) depends on data, which is not carried", d,
                    o.operands[d + 1].c_str()));
        const int64_t hi = src.dims.at(d) - sizes.at(d);
        st.push_back(std::max<int64_t>(0, std::min<int64_t>(it->second, hi)));
      }
      Shape li(st.size()), one(st.size(), 1);
      for (size_t d = 0; d < st.size(); d++) li[d] = st[d] + sizes.at(d);
      return {slice(args[0], st, li, one)};
    }
    if (n == "stablehlo.gather") return {gather1d(o, args.at(0), args.at(1))};
    if (n == "stablehlo.reduce") {  // Lower.lean:430-439
      auto dims = ints(attr_or(o, "dimensions", ""));
      if (o.regions.empty()) fail("reduce without a body");
      const Block &body = o.regions[0];
      if (!(body.ops.size() == 1 && body.ops[0].name == "stablehlo.maximum" && o.operands.size() == 2))
        fail("reduce: only a single-operand maximum is carried");
      if (el0 == "f64") fail("reduce on f64 is not carried");
      ArrayP r = args[0];
      std::sort(dims.begin(), dims.end(), std::greater<int64_t>());
      for (int64_t d : dims) r = max_axis(r, (int)d);
      return {binary(kMax, r, args[1])};
    }
    if (n == "stablehlo.concatenate") {
      const int64_t d = ints(attr_or(o, "dimension", "0")).at(0);
      std::vector<ArrayP> xs(args);
      if (f.concat_swap) std::reverse(xs.begin(), xs.end());
      return {concat(xs, (int)d)};
    }
    if (n == "stablehlo.convert") return {convert_op(args[0], o.in_tys.at(0), out)};
    if (n == "stablehlo.bitcast_convert") return {view_dtype(args[0], el_dtype(out.el))};
    if (n == "stablehlo.iota") {  // Lower.lean:445-452
      const int64_t d = ints(attr_or(o, "iota_dimension", "0")).at(0);
      return {iota(el_dtype(out.el), out.dims, (int)d)};
    }
    if (n == "stablehlo.dot_general") return {dot_general(f, o, args.at(0), args.at(1))};
    if (n == "stablehlo.while") {  // Lower.lean:454-470
      if (o.regions.size() < 2) fail("while without its two regions");
      const Block &cond = o.regions[0], &body = o.regions[1];
      std::vector<ArrayP> st = args, prev = args;
      std::vector<std::pair<bool, int64_t>> stk;
      for (auto &nm : o.operands) {
        auto it = known.find(nm);
        stk.push_back(it == known.end() ? std::make_pair(false, (int64_t)0) : std::make_pair(true, it->second));
      }
      for (;;) {
        auto cr = run_region(env, known, cond, st, stk);
        if (cr.second.empty() || !cr.second[0].first)
          fail("while: the condition depends on data, which is not carried (the loop is unrolled when traced)");
        if (cr.second[0].second == 0) break;
        auto br = run_region(env, known, body, st, stk);
        prev = st;
        st = br.first;
        stk = br.second;
      }
      return f.while_short ? prev : st;
    }
    if (n == "stablehlo.composite" || n == "stablehlo.custom_call") return run_composite(o, args);
    fail("op " + n + " is not in the lowering table");
  }

  // ggml.norm over the rows of the output's last dim, then `chain` (the fused
  // prefix at index (0, row, column)).
  ArrayP run_norm(const Op &o, const ArrayP &x, const std::vector<Chained> &chain) {
    const std::string attrs = attr_or(o, "composite_attributes", attr_or(o, "backend_config", ""));
    const Ty &out = o.out_tys.at(0);
    auto rc = rows_cols(out);
    std::vector<int64_t> g[3];
    for (size_t d = 0; d < out.dims.size(); d++) g[d + 1 < out.dims.size() ? 1 : 2].push_back((int64_t)d);
    const bool can = !f.norm_gpu_ops && rc.second <= 4 * 64 * kNormEpiJ;
    const std::vector<FusedOp> epi = can ? fusable_prefix(chain, out.dims, g, false) : std::vector<FusedOp>{};
    ArrayP y = norm(x, rc.first, rc.second, f32_attr(attrs, "eps"), f.norm_gpu_ops, epi);
    return apply_chain(reshape(y, out.dims), chain, epi.size());
  }

  std::vector<ArrayP> run_composite(const Op &o, const std::vector<ArrayP> &args) {  // Lower.lean:475-498
    const std::string name = replace_all(attr_or(o, "name", attr_or(o, "call_target_name", "")), "\"", "");
    const std::string attrs = attr_or(o, "composite_attributes", attr_or(o, "backend_config", ""));
    const Ty &out = o.out_tys.at(0);
    auto rc = rows_cols(out);
    const int64_t rows = rc.first, cols = rc.second;
    if (name == "ggml.norm") return {run_norm(o, args.at(0), {})};
    // A row tail (cols % 4) is refused unless the pinned flavour's correctly
    // rounded expf carries it (Lower.lean:485-486 refuses it always).
    if (name == "ggml.soft_max") {
      require_tail_expf("ggml.soft_max", cols);
      return {reshape(soft_max(args.at(0), rows, cols, f32_attr(attrs, "scale"), f.soft_max_float_sum), out.dims)};
    }
    if (name == "ggml.silu") {
      require_tail_expf("ggml.silu", cols);
      return {reshape(silu(args.at(0), rows, cols, f.silu_gpu_ops), out.dims)};
    }
    if (name == "ggml.gelu_erf") return {reshape(gelu_erf(args.at(0), f.gelu_tanh), out.dims)};
    const std::string dec = replace_all(attr_or(o, "decomposition", ""), "@", "");
    const Func *fn = m.func(dec);
    if (!fn) fail("composite " + name + ": no decomposition @" + dec);
    return run_func_(*fn, args);
  }

  // ---- fusion of element-wise chains into their producer (the mx::compile
  // role): a dot_general or ggml.norm whose result's one use is an f32 add /
  // subtract / multiply / divide / maximum / minimum of the same shape, whose
  // result's one use is the next such op, and so on, runs as one kernel that
  // applies the chain to each output before storing it.  Each op is one IEEE
  // rounding of the same operands, so the bits are those of the separate ops.

  // An attention group: S = dot_general(q, k) with its chain, P = ggml.soft_max(S),
  // O = dot_general(P, v) with its chain, run by attention_ggml when it carries them.
  struct AttnGroup {
    int qk = -1, sm = -1, pv = -1;
    std::vector<int> ch1, ch2;
  };

  struct Fusion {
    std::vector<char> skip;               // the producer and the chain's inner ops
    std::vector<int> producer;            // at a chain's last op: its producer's index
    std::vector<std::vector<int>> chain;  // at a producer: its chain's op indices
    std::vector<int> attn;                // at an attention group's last op: the group's index
    std::vector<AttnGroup> groups;
  };

  static void count_uses(const Block &b, std::unordered_map<std::string, int> *uses) {
    for (const Op &o : b.ops) {
      for (auto &n : o.operands) (*uses)[n]++;
      for (const Block &r : o.regions) count_uses(r, uses);
    }
    for (auto &r : b.ret) (*uses)[r]++;
  }

  // Whether `e` can take the value `cur` of type `vt` into a fused chain;
  // *other = the index of its other operand.
  bool chainable(const Op &e, const Ty &vt, const std::string &cur, int *other) const {
    if ((e.name == "stablehlo.custom_call" || e.name == "stablehlo.composite") &&
        composite_name(e) == "ggml.gelu_erf") {  // unary: any operand count but one is refused
      if (f.gelu_tanh || e.operands.size() != 1 || e.operands[0] != cur || e.results.size() != 1 ||
          e.out_tys.size() != 1 || e.out_tys[0].el != "f32" || e.out_tys[0].dims != vt.dims)
        return false;
      *other = -1;
      return true;
    }
    if (f.binary_half) return false;  // planted: binary ops through f16
    uint32_t c = 0;
    const bool div = e.name == "stablehlo.divide" && !f.divide_builtin;
    if (!div && !(binary_code(e.name, &c) && (c == kAdd || c == kSub || c == kMul || c == kMax || c == kMin)))
      return false;
    if (e.operands.size() != 2 || e.results.size() != 1 || e.in_tys.size() != 2 || e.out_tys.size() != 1 ||
        !e.regions.empty())
      return false;
    for (const Ty *t : {&e.in_tys[0], &e.in_tys[1], &e.out_tys[0]})
      if (t->el != "f32" || t->dims != vt.dims) return false;
    const bool l = e.operands[0] == cur, r = e.operands[1] == cur;
    if (l == r) return false;
    *other = l ? 1 : 0;
    return true;
  }

  static std::string composite_name(const Op &o) {
    return replace_all(attr_or(o, "name", attr_or(o, "call_target_name", "")), "\"", "");
  }

  // A dot_general the lowering accepts, or a ggml.norm (not planted), with one f32 result.
  bool fusable_producer(const Op &o) const {
    if (o.results.size() != 1 || o.out_tys.size() != 1 || o.out_tys[0].el != "f32" || o.operands.empty()) return false;
    std::vector<int64_t> lb, rb, lc, rc;
    if (o.name == "stablehlo.dot_general") return o.operands.size() == 2 && dot_dims(o, &lb, &rb, &lc, &rc);
    if (o.name == "stablehlo.composite" || o.name == "stablehlo.custom_call")
      return composite_name(o) == "ggml.norm" && !f.norm_gpu_ops && o.operands.size() == 1;
    return false;
  }

  Fusion plan_fusion(const Block &b) const {
    const size_t n = b.ops.size();
    Fusion fu{std::vector<char>(n, 0), std::vector<int>(n, -1), std::vector<std::vector<int>>(n),
              std::vector<int>(n, -1), {}};
    std::unordered_map<std::string, int> uses, user;
    count_uses(b, &uses);
    for (size_t k = 0; k < n; k++)
      for (auto &nm : b.ops[k].operands) user[nm] = (int)k;
    std::vector<char> claimed(n, 0);
    for (size_t i = 0; i < n; i++) {
      const Op &o = b.ops[i];
      if (!fusable_producer(o)) continue;
      const Ty &vt = o.out_tys[0];
      std::string cur = o.results[0];
      std::vector<int> ch;
      while ((int)ch.size() < kMaxEpi && uses[cur] == 1) {
        auto it = user.find(cur);
        int other = 0;
        if (it == user.end() || it->second <= (ch.empty() ? (int)i : ch.back()) || claimed[it->second] ||
            !chainable(b.ops[it->second], vt, cur, &other))
          break;
        ch.push_back(it->second);
        cur = b.ops[it->second].results[0];
      }
      if (ch.empty()) continue;
      fu.skip[i] = 1;
      for (size_t k = 0; k + 1 < ch.size(); k++) fu.skip[ch[k]] = 1;
      for (int k : ch) claimed[k] = 1;
      fu.producer[ch.back()] = (int)i;
      fu.chain[i] = ch;
    }
    plan_attention(b, uses, user, &fu);
    return fu;
  }

  // Attention groups among the planned chains: a dot_general (with its chain)
  // whose value's one use is a ggml.soft_max, whose result's one use is the
  // lhs of a dot_general (with its chain).  Not under the planted faults that
  // change a product or the softmax (the separate kernels carry those).
  void plan_attention(const Block &b, std::unordered_map<std::string, int> &uses,
                      const std::unordered_map<std::string, int> &user, Fusion *fu) const {
    if (f.dot_builtin || f.dot_plain || f.soft_max_float_sum) return;
    const size_t n = b.ops.size();
    auto one_user = [&](const std::string &v, int after) -> int {
      if (uses[v] != 1) return -1;
      auto it = user.find(v);
      return it == user.end() || it->second <= after ? -1 : it->second;
    };
    for (size_t i = 0; i < n; i++) {
      const Op &qk = b.ops[i];
      if (qk.name != "stablehlo.dot_general" || !fusable_producer(qk) || fu->attn[i] >= 0) continue;
      const std::vector<int> &ch1 = fu->chain[i];
      const int end1 = ch1.empty() ? (int)i : ch1.back();
      const int s = one_user(b.ops[end1].results[0], end1);
      if (s < 0) continue;
      const Op &sm = b.ops[s];
      if ((sm.name != "stablehlo.custom_call" && sm.name != "stablehlo.composite") ||
          composite_name(sm) != "ggml.soft_max" || sm.operands.size() != 1 || sm.results.size() != 1 ||
          sm.out_tys.size() != 1 || sm.out_tys[0].el != "f32")
        continue;
      const int p = one_user(sm.results[0], s);
      if (p < 0) continue;
      const Op &pv = b.ops[p];
      if (pv.name != "stablehlo.dot_general" || !fusable_producer(pv) || pv.operands[0] != sm.results[0] ||
          pv.operands[1] == sm.results[0] || (fu->skip[p] && fu->chain[p].empty()))
        continue;
      AttnGroup g{(int)i, s, p, ch1, fu->chain[p]};
      const int last = g.ch2.empty() ? p : g.ch2.back();
      fu->skip[i] = 1;
      for (int k : g.ch1) fu->skip[k] = 1, fu->producer[k] = -1;
      fu->skip[s] = 1;
      fu->skip[p] = p != last;
      fu->producer[last] = -1;
      fu->skip[last] = 0;
      fu->attn[last] = (int)fu->groups.size();
      fu->groups.push_back(std::move(g));
    }
  }

  std::vector<Chained> chain_of(const Env &env, const std::vector<Op> &ops, int p, const std::vector<int> &ch) {
    std::string cur = ops[p].results[0];
    std::vector<Chained> chain;
    for (int k : ch) {
      const Op &e = ops[k];
      if (e.operands.size() == 1) {  // ggml.gelu_erf
        chain.push_back(Chained{kEpiGeluErf, false, nullptr});
        cur = e.results[0];
        continue;
      }
      const bool rev = e.operands[1] == cur;
      uint32_t c = kDiv;
      if (e.name != "stablehlo.divide") binary_code(e.name, &c);
      chain.push_back(Chained{c, rev, get(env, e.operands[rev ? 0 : 1])});
      cur = e.results[0];
    }
    return chain;
  }

  // The fused attention kernel when it carries the group's shapes and
  // layouts, else the group's ops one by one (the same bits either way).
  std::vector<ArrayP> run_attention(const Env &env, const std::vector<Op> &ops, const AttnGroup &g) {
    const Op &qk = ops[g.qk], &sm = ops[g.sm], &pv = ops[g.pv];
    const ArrayP q = get(env, qk.operands.at(0)), k = get(env, qk.operands.at(1)), v = get(env, pv.operands.at(1));
    const std::vector<Chained> c1 = chain_of(env, ops, g.qk, g.ch1), c2 = chain_of(env, ops, g.pv, g.ch2);
    const Ty &st = qk.out_tys.at(0), &ot = pv.out_tys.at(0);
    const std::string attrs = attr_or(sm, "composite_attributes", attr_or(sm, "backend_config", ""));
    const uint32_t scale = f32_attr(attrs, "scale");
    std::vector<int64_t> lb, rb, lc, rc, lb2, rb2, lc2, rc2;
    if (dot_dims(qk, &lb, &rb, &lc, &rc) && dot_dims(pv, &lb2, &rb2, &lc2, &rc2) && sm.out_tys[0].dims == st.dims &&
        q->shape == qk.in_tys.at(0).dims && k->shape == qk.in_tys.at(1).dims && v->shape == pv.in_tys.at(1).dims) {
      const Ty &ta = qk.in_tys[0], &tb = qk.in_tys[1], &tv = pv.in_tys[1];
      auto contains = [](const std::vector<int64_t> &x, int64_t d) { return std::find(x.begin(), x.end(), d) != x.end(); };
      auto prod = [](const Ty &t, const std::vector<int64_t> &ds) {
        int64_t m = 1;
        for (int64_t d : ds) m *= t.dims.at(d);
        return m;
      };
      std::vector<int64_t> lf, rf, vf;
      for (int64_t d = 0; d < (int64_t)ta.dims.size(); d++)
        if (!contains(lb, d) && !contains(lc, d)) lf.push_back(d);
      for (int64_t d = 0; d < (int64_t)tb.dims.size(); d++)
        if (!contains(rb, d) && !contains(rc, d)) rf.push_back(d);
      for (int64_t d = 0; d < (int64_t)tv.dims.size(); d++)
        if (!contains(rb2, d) && !contains(rc2, d)) vf.push_back(d);
      const int64_t nb = (int64_t)lb.size(), nl = (int64_t)lf.size(), rank = (int64_t)st.dims.size();
      // P's batch dims are S's, in order; P contracts its last dim, the one key dim.
      std::vector<int64_t> sb(nb);
      for (int64_t d = 0; d < nb; d++) sb[d] = d;
      const int64_t B = prod(ta, lb), NQ = prod(ta, lf), NK = prod(tb, rf), DH = ta.dims.at(lc[0]);
      if (rf.size() == 1 && lb2 == sb && lc2.size() == 1 && lc2[0] == rank - 1 && rank == nb + nl + 1 &&
          tv.dims.at(rc2[0]) == NK && prod(tv, rb2) == B && tb.dims.at(rc[0]) == DH && prod(tb, rb) == B) {
        std::vector<int64_t> g1[3], g2[3];
        for (int64_t d = 0; d < rank; d++) g1[d < nb ? 0 : d < nb + nl ? 1 : 2].push_back(d);
        for (int64_t d = 0; d < (int64_t)ot.dims.size(); d++) g2[d < nb ? 0 : d < nb + nl ? 1 : 2].push_back(d);
        const std::vector<FusedOp> e1 = fusable_prefix(c1, st.dims, g1, false);
        const std::vector<FusedOp> e2 = fusable_prefix(c2, ot.dims, g2, false);
        if (e1.size() == c1.size()) {
          const DotOperand Q = dot_operand(q, lb, lf, lc[0]), K = dot_operand(k, rb, rf, rc[0]);
          const DotOperand V = dot_operand(v, rb2, vf, rc2[0]);
          if (ArrayP y = attention_ggml(Q, K, V, B, NQ, NK, DH, prod(tv, vf), e1, scale, e2))
            return {apply_chain(reshape(y, ot.dims), c2, e2.size())};
        }
      }
    }
    ArrayP s = dot_general(f, qk, q, k, c1);
    const auto rcs = rows_cols(sm.out_tys[0]);
    require_tail_expf("ggml.soft_max", rcs.second);
    ArrayP pr = reshape(soft_max(s, rcs.first, rcs.second, scale, f.soft_max_float_sum), sm.out_tys[0].dims);
    return {dot_general(f, pv, pr, v, c2)};
  }

  std::vector<ArrayP> run_fused(const Env &env, const std::vector<Op> &ops, int p, const std::vector<int> &ch) {
    const Op &d = ops[p];
    const std::vector<Chained> chain = chain_of(env, ops, p, ch);
    if (d.name == "stablehlo.dot_general")
      return {dot_general(f, d, get(env, d.operands.at(0)), get(env, d.operands.at(1)), chain)};
    return {run_norm(d, get(env, d.operands.at(0)), chain)};
  }

  // Run a block whose arguments are `args`, seeing the enclosing env (Lower.lean:503-519).
  std::pair<std::vector<ArrayP>, std::vector<std::pair<bool, int64_t>>> run_region(
      const Env &env0, const Known &known0, const Block &b, const std::vector<ArrayP> &args,
      const std::vector<std::pair<bool, int64_t>> &argk) {
    Env env = env0;
    Known known = known0;
    for (size_t i = 0; i < b.args.size() && i < args.size(); i++) {
      env[b.args[i].first] = args[i];
      if (i < argk.size() && argk[i].first) known[b.args[i].first] = argk[i].second;
      else known.erase(b.args[i].first);
    }
    const Fusion fu = plan_fusion(b);
    for (size_t i = 0; i < b.ops.size(); i++) {
      const Op &o = b.ops[i];
      if (fu.skip[i]) continue;  // a fused producer or inner chain op: runs with the chain's last op
      auto rs = fu.attn[i] >= 0        ? run_attention(env, b.ops, fu.groups[fu.attn[i]])
                : fu.producer[i] >= 0 ? run_fused(env, b.ops, fu.producer[i], fu.chain[fu.producer[i]])
                                      : run_op(env, known, o);
      if (rs.size() != o.results.size())
        fail(strf("%s: %zu results for %zu names", o.name.c_str(), rs.size(), o.results.size()));
      for (size_t j = 0; j < rs.size(); j++) env[o.results[j]] = rs[j];
      if (o.results.size() == 1) {
        int64_t v;
        if (const_eval(known, o, &v)) known[o.results[0]] = v;
        else known.erase(o.results[0]);
      }
    }
    std::vector<ArrayP> outs;
    std::vector<std::pair<bool, int64_t>> ks;
    for (auto &r : b.ret) {
      outs.push_back(get(env, r));
      auto it = known.find(r);
      ks.push_back(it == known.end() ? std::make_pair(false, (int64_t)0) : std::make_pair(true, it->second));
    }
    return {outs, ks};
  }

  std::vector<ArrayP> run_func_(const Func &fn, const std::vector<ArrayP> &args) {  // Lower.lean:521-526
    if (args.size() != fn.body.args.size())
      fail(strf("@%s takes %zu arguments, got %zu", fn.name.c_str(), fn.body.args.size(), args.size()));
    std::vector<std::pair<bool, int64_t>> none(args.size(), {false, 0});
    return run_region(Env{}, Known{}, fn.body, args, none).first;
  }
};

}  // namespace

uint8_t el_dtype(const std::string &el) {
  if (el == "f32") return kF32;
  if (el == "i32" || el == "si32") return kI32;
  if (el == "ui32") return kU32;
  if (el == "i64" || el == "si64") return kI64;
  if (el == "ui64") return kU64;
  if (el == "i1") return kBool;
  if (el == "ui8") return kU8;
  if (el == "f64") return kF64;
  fail("element type " + el + " is not carried");
}

size_t el_bytes(const std::string &el) {
  if (el == "f64" || el == "i64" || el == "ui64" || el == "si64") return 8;
  if (el == "i1" || el == "ui8") return 1;
  return 4;
}

std::vector<ArrayP> run_func(const Module &m, const Faults &f, const Func &fn, const std::vector<ArrayP> &args) {
  Lowerer l{m, f};
  return l.run_func_(fn, args);
}

}  // namespace shlo
