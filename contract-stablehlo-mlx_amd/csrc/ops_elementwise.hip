// Elementwise and data-movement kernels: the single-rounding built-ins the
// reference takes from MLX (c/smlx_shim.c:148-264; exact in any order,
// StablehloMlx/Lower.lean:12-17).  One generic strided kernel per arity: the
// operands' dims are collapsed on the host, then each thread maps its linear
// output index to operand offsets with magic-number division.
#include <hip/hip_runtime.h>

#include <cmath>

#include "epilogue.h"
#include "ops.h"

namespace shlo {
namespace {

constexpr int kND = 6;       // dims after collapsing
constexpr int kBlock = 256;

struct FastDiv {
  uint32_t d = 1, m = 1, s = 0;
};
FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  uint32_t s = 0;
  while ((1ull << s) < d) s++;
  f.s = s;
  f.m = (uint32_t)(((1ull << 32) * ((1ull << s) - d)) / d + 1);
  return f;
}
__device__ __forceinline__ uint32_t fdiv(const FastDiv &f, uint32_t n) {
  const uint32_t t = __umulhi(n, f.m);
  return (t + n) >> f.s;
}

template <int NOP>
struct NDMap {
  int rank = 1;
  uint32_t dim[kND] = {};
  FastDiv div[kND];
  uint32_t st[NOP][kND] = {};

  __device__ __forceinline__ void offsets(uint32_t i, uint32_t *off) const {
#pragma unroll
    for (int j = 0; j < NOP; j++) off[j] = 0;
    for (int d = rank - 1; d > 0; d--) {
      const uint32_t q = fdiv(div[d], i);
      const uint32_t c = i - q * dim[d];
      i = q;
#pragma unroll
      for (int j = 0; j < NOP; j++) off[j] += c * st[j][d];
    }
#pragma unroll
    for (int j = 0; j < NOP; j++) off[j] += i * st[j][0];
  }
};

// Collapse the iteration space of `shape` for NOP operands whose element
// strides are given (each already broadcast to `shape`).
template <int NOP>
NDMap<NOP> make_map(const Shape &shape, const std::vector<const Shape *> &strides) {
  std::vector<int64_t> dims;
  std::vector<std::vector<int64_t>> st(NOP);
  for (size_t d = 0; d < shape.size(); d++) {
    if (shape[d] == 1) continue;
    dims.push_back(shape[d]);
    for (int j = 0; j < NOP; j++) st[j].push_back((*strides[j])[d]);
  }
  if (dims.empty()) {
    dims.push_back(1);
    for (int j = 0; j < NOP; j++) st[j].push_back(0);
  }
  // merge d-1 and d when every operand walks them as one run
  std::vector<int64_t> md{dims[0]};
  std::vector<std::vector<int64_t>> ms(NOP);
  for (int j = 0; j < NOP; j++) ms[j].push_back(st[j][0]);
  for (size_t d = 1; d < dims.size(); d++) {
    bool ok = true;
    for (int j = 0; j < NOP && ok; j++) ok = ms[j].back() == st[j][d] * dims[d];
    if (ok) {
      md.back() *= dims[d];
      for (int j = 0; j < NOP; j++) ms[j].back() = st[j][d];
    } else {
      md.push_back(dims[d]);
      for (int j = 0; j < NOP; j++) ms[j].push_back(st[j][d]);
    }
  }
  if ((int)md.size() > kND) fail(strf("elementwise: %d dims after collapsing (at most %d)", (int)md.size(), kND));
  NDMap<NOP> m;
  m.rank = (int)md.size();
  for (int d = 0; d < m.rank; d++) {
    if (md[d] > 0x7FFFFFFF) fail("elementwise: dimension above 2^31");
    m.dim[d] = (uint32_t)md[d];
    m.div[d] = make_fastdiv((uint32_t)md[d]);
    for (int j = 0; j < NOP; j++) {
      if (ms[j][d] < 0 || ms[j][d] > 0x7FFFFFFF) fail("elementwise: stride out of range");
      m.st[j][d] = (uint32_t)ms[j][d];
    }
  }
  return m;
}

unsigned grid_for(int64_t n) {
  int64_t g = (n + kBlock - 1) / kBlock;
  if (g > 65536) g = 65536;
  return (unsigned)std::max<int64_t>(g, 1);
}

void check_elems(int64_t n) {
  if (n > 0x7FFFFFFF) fail("elementwise: more than 2^31 elements in one array");
}

// ---- generic kernels ----------------------------------------------------------

template <class F, class TA, class TO>
__global__ void __launch_bounds__(kBlock) ew1(NDMap<1> map, uint32_t n, const TA *a, TO *o, F f) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    uint32_t off[1];
    map.offsets(i, off);
    o[i] = f(a[off[0]]);
  }
}

template <class F, class TA, class TB, class TO>
__global__ void __launch_bounds__(kBlock) ew2(NDMap<2> map, uint32_t n, const TA *a, const TB *b, TO *o, F f) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    uint32_t off[2];
    map.offsets(i, off);
    o[i] = f(a[off[0]], b[off[1]]);
  }
}

template <class F, class TA, class TB, class TC, class TO>
__global__ void __launch_bounds__(kBlock) ew3(NDMap<3> map, uint32_t n, const TA *a, const TB *b, const TC *c, TO *o,
                                             F f) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    uint32_t off[3];
    map.offsets(i, off);
    o[i] = f(a[off[0]], b[off[1]], c[off[2]]);
  }
}

// Contiguous binary f32 fast path, four elements per thread.
template <class F>
__global__ void __launch_bounds__(kBlock) ew2_f32x4(uint32_t n4, const float4 *a, const float4 *b, float4 *o, F f) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += gridDim.x * blockDim.x) {
    const float4 x = a[i], y = b[i];
    o[i] = make_float4(f(x.x, y.x), f(x.y, y.y), f(x.z, y.z), f(x.w, y.w));
  }
}

// Strided copy: operand 0 is the source, operand 1 the destination.
template <class T>
__global__ void __launch_bounds__(kBlock) copy_nd(NDMap<2> map, uint32_t n, const T *src, T *dst) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    uint32_t off[2];
    map.offsets(i, off);
    dst[off[1]] = src[off[0]];
  }
}

// ---- four elements per thread ---------------------------------------------------
//
// For 4-byte element types whose collapsed innermost dim has a length that is a
// multiple of 4 and that every operand walks with stride 0 or 1: the map runs
// over groups of four (innermost length / 4, innermost strides x 4), a stride-1
// operand's group is one 16-byte access, a stride-0 operand's one scalar.
// Results are the same elements computed by the same functor, so the bits
// match the one-element kernels.

template <class T>
struct V4 {
  T v[4];
};

template <class T>
__device__ __forceinline__ V4<T> ld_v4(const T *p, bool unit) {
  V4<T> r;
  if (unit) {
    const uint4 u = *reinterpret_cast<const uint4 *>(p);
    r.v[0] = __builtin_bit_cast(T, u.x);
    r.v[1] = __builtin_bit_cast(T, u.y);
    r.v[2] = __builtin_bit_cast(T, u.z);
    r.v[3] = __builtin_bit_cast(T, u.w);
  } else {
    r.v[0] = r.v[1] = r.v[2] = r.v[3] = *p;
  }
  return r;
}

template <class T>
__device__ __forceinline__ void st_v4(T *p, const V4<T> &r) {
  *reinterpret_cast<uint4 *>(p) = make_uint4(__builtin_bit_cast(uint32_t, r.v[0]), __builtin_bit_cast(uint32_t, r.v[1]),
                                             __builtin_bit_cast(uint32_t, r.v[2]), __builtin_bit_cast(uint32_t, r.v[3]));
}

// unit[j]: operand j walks the innermost dim with stride 1 (else 0).
template <class F, class TA, class TO>
__global__ void __launch_bounds__(kBlock) ew1_v4(NDMap<1> map, uint32_t n4, const TA *a, TO *o, F f, bool ua) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += gridDim.x * blockDim.x) {
    uint32_t off[1];
    map.offsets(i, off);
    const V4<TA> x = ld_v4(a + off[0], ua);
    V4<TO> y;
#pragma unroll
    for (int k = 0; k < 4; k++) y.v[k] = f(x.v[k]);
    st_v4(o + 4 * (size_t)i, y);
  }
}

template <class F, class TA, class TB, class TO>
__global__ void __launch_bounds__(kBlock) ew2_v4(NDMap<2> map, uint32_t n4, const TA *a, const TB *b, TO *o, F f,
                                                bool ua, bool ub) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += gridDim.x * blockDim.x) {
    uint32_t off[2];
    map.offsets(i, off);
    const V4<TA> x = ld_v4(a + off[0], ua);
    const V4<TB> y = ld_v4(b + off[1], ub);
    V4<TO> z;
#pragma unroll
    for (int k = 0; k < 4; k++) z.v[k] = f(x.v[k], y.v[k]);
    st_v4(o + 4 * (size_t)i, z);
  }
}

template <class T>
__global__ void __launch_bounds__(kBlock) copy_v4(NDMap<2> map, uint32_t n4, const T *src, T *dst, bool us) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += gridDim.x * blockDim.x) {
    uint32_t off[2];
    map.offsets(i, off);
    st_v4(dst + off[1], ld_v4(src + off[0], us));
  }
}

// The group map for `m` (element offsets in units of T), or false when the
// four-element kernels do not apply: the innermost length is not a multiple
// of 4, an operand walks it with a stride other than 0 or 1, or a stride-1
// operand's groups would not be 16-byte aligned.  `ptrs[j]` is operand j's
// base; `must_unit` marks operands (outputs) that need stride 1.
template <int NOP>
bool group_map(const NDMap<NOP> &m, const void *const (&ptrs)[NOP], const bool (&must_unit)[NOP], NDMap<NOP> &g,
               bool (&unit)[NOP]) {
  const int l = m.rank - 1;
  if (m.dim[l] % 4) return false;
  for (int j = 0; j < NOP; j++) {
    const uint32_t sl = m.st[j][l];
    if (sl > 1 || (must_unit[j] && sl != 1)) return false;
    unit[j] = sl == 1;
    if (unit[j]) {
      if ((uintptr_t)ptrs[j] % 16) return false;
      for (int d = 0; d < l; d++)
        if (m.st[j][d] % 4) return false;
    }
  }
  g = m;
  g.dim[l] = m.dim[l] / 4;
  g.div[l] = make_fastdiv(g.dim[l]);
  for (int j = 0; j < NOP; j++) g.st[j][l] = m.st[j][l] * 4;
  return true;
}

// ---- dtype dispatch -----------------------------------------------------------

using f16 = _Float16;

template <class F>
void dispatch_dtype(uint8_t dt, F &&f) {
  switch (dt) {
    case kBool: f(uint8_t{}); break;
    case kU8: f(uint8_t{}); break;
    case kI8: f(int8_t{}); break;
    case kU16: f(uint16_t{}); break;
    case kI16: f(int16_t{}); break;
    case kU32: f(uint32_t{}); break;
    case kI32: f(int32_t{}); break;
    case kU64: f(uint64_t{}); break;
    case kI64: f(int64_t{}); break;
    case kF16: f(f16{}); break;
    case kF32: f(float{}); break;
    case kF64: f(double{}); break;
    default: fail(strf("dtype %u is not carried", dt));
  }
}

template <class T>
constexpr bool is_flt() {
  return std::is_same<T, float>::value || std::is_same<T, f16>::value || std::is_same<T, double>::value;
}

// ---- binary64 with the reference's NaN and conversion rules ---------------------
//
// The reference carries binary64 tensors as bit patterns through soft-float
// kernels (StablehloMlx/Kernels/SoftFloat.lean) that behave as arm64 with
// FPCR.DN clear: a NaN operand comes back quieted, sign and payload kept, the
// first operand's when both are NaN (f64Add/f64Sub/f64Mul/f64Div,
// SoftFloat.lean:137-259); an invalid operation (inf - inf, 0 * inf, 0 / 0,
// inf / inf) gives the default NaN +0x7FF8000000000000.  gfx950's binary64
// instructions round to nearest even with subnormals, as those kernels do;
// the NaN choices are made explicit here, since the hardware's own (and the
// compiler's freedom to commute operands) need not match them.
constexpr uint64_t kSign64 = 0x8000000000000000ull, kQuiet64 = 0x0008000000000000ull;
constexpr uint64_t kInf64 = 0x7FF0000000000000ull, kNan64 = 0x7FF8000000000000ull;
__device__ __forceinline__ uint64_t d_bits(double x) { return __builtin_bit_cast(uint64_t, x); }
__device__ __forceinline__ double bits_d(uint64_t u) { return __builtin_bit_cast(double, u); }
__device__ __forceinline__ bool d_isnan(double x) { return (d_bits(x) & ~kSign64) > kInf64; }
__device__ __forceinline__ double d_quiet(double x) { return bits_d(d_bits(x) | kQuiet64); }

__device__ __forceinline__ double f64_binary(uint32_t op, double x, double y) {
  if (d_isnan(x)) return d_quiet(x);
  if (d_isnan(y)) return d_quiet(y);
  double r;
  switch (op) {
    case kAdd: r = x + y; break;
    case kSub: r = x - y; break;  // a + (-b) (f64Sub, SoftFloat.lean:197-202)
    case kMul: r = x * y; break;
    case kDiv: r = x / y; break;  // IEEE division (the HIP lowering is correctly rounded)
    // maximum / minimum: -0 below +0, the first operand on a tie
    // (f64MaxMin, Lower.lean:290-296)
    case kMax:
      if (x == y) return std::signbit(x) ? y : x;
      return x > y ? x : y;
    case kMin:
      if (x == y) return std::signbit(x) ? x : y;
      return x < y ? x : y;
    case kRem: r = std::fmod(x, y); break;
    default: return x;
  }
  return d_isnan(r) ? bits_d(kNan64) : r;
}

// f64ToI64 (SoftFloat.lean:219-236, arm64 fcvtzs): toward zero, saturating,
// NaN to 0.
__device__ __forceinline__ int64_t f64_to_i64(double x) {
  if (d_isnan(x)) return 0;
  if (x >= 0x1p63) return INT64_MAX;
  if (x <= -0x1p63) return INT64_MIN;
  return (int64_t)x;
}
// f64ToF32 (SoftFloat.lean:95-120): round to nearest even with binary32
// subnormals; a NaN keeps its sign and the top of its payload, quieted.
__device__ __forceinline__ float f64_to_f32(double x) {
  if (d_isnan(x)) {
    const uint64_t u = d_bits(x);
    return __builtin_bit_cast(float, (uint32_t)((u >> 32) & 0x80000000u) | 0x7FC00000u |
                                         (uint32_t)((u & 0x000FFFFFFFFFFFFFull) >> 29));
  }
  return (float)x;
}
// f64FromF32 (SoftFloat.lean:73-86): exact; a NaN keeps its sign and payload
// (it is not quieted).
__device__ __forceinline__ double f32_to_f64(float x) {
  const uint32_t b = __builtin_bit_cast(uint32_t, x);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u)
    return bits_d(((uint64_t)(b >> 31) << 63) | kInf64 | ((uint64_t)(b & 0x7FFFFFu) << 29));
  return (double)x;
}

// ---- unary functors ------------------------------------------------------------

template <class T>
struct UnaryF {
  uint32_t op;
  __device__ T operator()(T x) const {
    if constexpr (is_flt<T>()) {
      using C = typename std::conditional<std::is_same<T, double>::value, double, float>::type;
      const C v = (C)x;
      switch (op) {
        case kNeg: return (T)(-v);
        case kAbs: return (T)std::fabs(v);  // clears the sign bit, of a NaN too (Lower.lean:360)
        case kSqrt: return (T)std::sqrt(v);
        case kFloor:
          if constexpr (std::is_same<T, double>::value)  // f64Floor (SoftFloat.lean:204-217)
            if (d_isnan(v)) return d_quiet(v);
          return (T)std::floor(v);
        case kExp: return (T)std::exp(v);
        case kErf: return (T)std::erf(v);
        case kNot: return (T)(v == (C)0 ? 1 : 0);
        case kRsqrt: return (T)((C)1 / std::sqrt(v));
        case kTanh: return (T)std::tanh(v);
        case kSigmoid: return (T)((C)1 / ((C)1 + std::exp(-v)));
        case kSqrtApprox:
          if constexpr (std::is_same<T, float>::value) return __builtin_amdgcn_sqrtf(v);
          else return (T)std::sqrt(v);
        default: return x;
      }
    } else {
      switch (op) {
        case kNeg: return (T)(T(0) - x);
        case kAbs:
          if constexpr (std::is_signed<T>::value) return x < 0 ? (T)(T(0) - x) : x;
          else return x;
        case kNot: return (T)(x == 0 ? 1 : 0);
        case kInvert: return (T)~x;
        default: return x;
      }
    }
  }
};

template <class TI, class TO>
struct CastF {
  __device__ TO operator()(TI x) const {
    if constexpr (std::is_same<TI, double>::value && std::is_same<TO, int64_t>::value) {
      return f64_to_i64(x);
    } else if constexpr (std::is_same<TI, double>::value && std::is_same<TO, float>::value) {
      return f64_to_f32(x);
    } else if constexpr (std::is_same<TI, float>::value && std::is_same<TO, double>::value) {
      return f32_to_f64(x);
    } else {
      return (TO)x;
    }
  }
};
template <class TI>
struct ToBoolF {
  __device__ uint8_t operator()(TI x) const { return x != (TI)0 ? 1 : 0; }
};

// ---- binary functors ------------------------------------------------------------

template <class T>
struct BinaryF {
  uint32_t op;
  __device__ T operator()(T a, T b) const {
    if constexpr (std::is_same<T, float>::value) {  // shared with the fused epilogues
      if (op == kDivApprox) return a * __builtin_amdgcn_rcpf(b);
      if (op == kRem) return std::fmod(a, b);
      return f32_binary(op, a, b);
    } else if constexpr (std::is_same<T, double>::value) {
      return f64_binary(op == kDivApprox ? (uint32_t)kDiv : op, a, b);
    } else if constexpr (is_flt<T>()) {
      using C = typename std::conditional<std::is_same<T, double>::value, double, T>::type;
      const C x = (C)a, y = (C)b;
      switch (op) {
        case kAdd: return (T)(x + y);
        case kSub: return (T)(x - y);
        case kMul: return (T)(x * y);
        case kDiv: return (T)(x / y);
        case kMax:
          if (x != x || y != y) return (T)(x + y);
          if (x == y) return std::signbit((float)x) ? b : a;
          return x > y ? a : b;
        case kMin:
          if (x != x || y != y) return (T)(x + y);
          if (x == y) return std::signbit((float)x) ? a : b;
          return x < y ? a : b;
        case kRem:
          if constexpr (std::is_same<T, double>::value) return std::fmod(x, y);
          else return (T)std::fmod((float)x, (float)y);
        case kDivApprox:
          if constexpr (std::is_same<T, float>::value) return x * __builtin_amdgcn_rcpf(y);
          else return (T)(x / y);
        default: return a;
      }
    } else {
      constexpr int bits = 8 * sizeof(T);
      using U = typename std::make_unsigned<T>::type;
      switch (op) {
        case kAdd: return (T)((U)a + (U)b);
        case kSub: return (T)((U)a - (U)b);
        case kMul: return (T)((U)a * (U)b);
        case kDiv:
          if (b == 0) return (T)0;
          if constexpr (std::is_signed<T>::value)
            if (b == (T)-1) return (T)((U)0 - (U)a);
          return (T)(a / b);
        case kRem:
          if (b == 0) return a;
          if constexpr (std::is_signed<T>::value)
            if (b == (T)-1) return (T)0;
          return (T)(a % b);
        case kMax: return a > b ? a : b;
        case kMin: return a < b ? a : b;
        case kAnd: return (T)(a & b);
        case kOr: return (T)(a | b);
        case kXor: return (T)(a ^ b);
        case kShl: return (U)b >= (U)bits ? (T)0 : (T)((U)a << (U)b);
        case kShr: return (U)b >= (U)bits ? (T)0 : (T)((U)a >> (U)b);
        case kLAnd: return (T)((a != 0) && (b != 0));
        case kLOr: return (T)((a != 0) || (b != 0));
        default: return a;
      }
    }
  }
};

template <class T>
struct CompareF {
  uint32_t op;
  __device__ uint8_t operator()(T a, T b) const {
    switch (op) {
      case kEq: return a == b;
      case kNe: return a != b;
      case kLt: return a < b;
      case kLe: return a <= b;
      case kGt: return a > b;
      case kGe: return a >= b;
      default: return 0;
    }
  }
};

template <class T>
struct WhereF {
  __device__ T operator()(uint8_t c, T a, T b) const { return c ? a : b; }
};

// ---- launch helpers ------------------------------------------------------------

template <class F, class TA, class TO>
void launch1(const ArrayP &a, const std::shared_ptr<Array> &o, F f) {
  const int64_t n = o->size();
  if (n == 0) return;
  check_elems(n);
  auto m = make_map<1>(o->shape, {&a->strides});
  const TA *pa = (const TA *)a->data();
  TO *po = (TO *)o->data();
  ArrayP keep = a;
  if constexpr (sizeof(TA) == 4 && sizeof(TO) == 4) {
    NDMap<1> g;
    bool unit[1];
    if ((uintptr_t)po % 16 == 0 && group_map<1>(m, {pa}, {false}, g, unit)) {
      const uint32_t n4 = (uint32_t)(n / 4);
      const bool ua = unit[0];
      launch([=](hipStream_t s) {
        (void)keep;
        ew1_v4<F, TA, TO><<<grid_for(n4), kBlock, 0, s>>>(g, n4, pa, po, f, ua);
      });
      return;
    }
  }
  launch([=](hipStream_t s) {
    (void)keep;
    ew1<F, TA, TO><<<grid_for(n), kBlock, 0, s>>>(m, (uint32_t)n, pa, po, f);
  });
}

template <class F, class TA, class TB, class TO>
void launch2(const ArrayP &a, const ArrayP &b, const std::shared_ptr<Array> &o, F f) {
  const int64_t n = o->size();
  if (n == 0) return;
  check_elems(n);
  const TA *pa = (const TA *)a->data();
  const TB *pb = (const TB *)b->data();
  TO *po = (TO *)o->data();
  ArrayP ka = a, kb = b;
  if constexpr (std::is_same<TA, float>::value && std::is_same<TB, float>::value && std::is_same<TO, float>::value) {
    if (a->contiguous() && b->contiguous() && a->shape == o->shape && b->shape == o->shape && n % 4 == 0 &&
        ((uintptr_t)pa % 16) == 0 && ((uintptr_t)pb % 16) == 0) {
      const uint32_t n4 = (uint32_t)(n / 4);
      launch([=](hipStream_t s) {
        (void)ka, (void)kb;
        ew2_f32x4<F><<<grid_for(n4), kBlock, 0, s>>>(n4, (const float4 *)pa, (const float4 *)pb, (float4 *)po, f);
      });
      return;
    }
  }
  auto m = make_map<2>(o->shape, {&a->strides, &b->strides});
  if constexpr (sizeof(TA) == 4 && sizeof(TB) == 4 && sizeof(TO) == 4) {
    NDMap<2> g;
    bool unit[2];
    if ((uintptr_t)po % 16 == 0 && group_map<2>(m, {pa, pb}, {false, false}, g, unit)) {
      const uint32_t n4 = (uint32_t)(n / 4);
      const bool ua = unit[0], ub = unit[1];
      launch([=](hipStream_t s) {
        (void)ka, (void)kb;
        ew2_v4<F, TA, TB, TO><<<grid_for(n4), kBlock, 0, s>>>(g, n4, pa, pb, po, f, ua, ub);
      });
      return;
    }
  }
  launch([=](hipStream_t s) {
    (void)ka, (void)kb;
    ew2<F, TA, TB, TO><<<grid_for(n), kBlock, 0, s>>>(m, (uint32_t)n, pa, pb, po, f);
  });
}

template <class T>
void launch_copy(const ArrayP &src, const Shape &dst_strides, char *dst_base, const Shape &shape) {
  const int64_t n = shape_count(shape);
  if (n == 0) return;
  check_elems(n);
  auto m = make_map<2>(shape, {&src->strides, &dst_strides});
  const T *ps = (const T *)src->data();
  T *pd = (T *)dst_base;
  ArrayP keep = src;
  if constexpr (sizeof(T) == 4) {
    NDMap<2> g;
    bool unit[2];
    if (group_map<2>(m, {ps, pd}, {false, true}, g, unit)) {
      const uint32_t n4 = (uint32_t)(n / 4);
      const bool us = unit[0];
      launch([=](hipStream_t s) {
        (void)keep;
        copy_v4<T><<<grid_for(n4), kBlock, 0, s>>>(g, n4, ps, pd, us);
      });
      return;
    }
  }
  launch([=](hipStream_t s) {
    (void)keep;
    copy_nd<T><<<grid_for(n), kBlock, 0, s>>>(m, (uint32_t)n, ps, pd);
  });
}

void copy_strided(const ArrayP &src, const Shape &dst_strides, char *dst_base) {
  switch (dtype_size(src->dtype)) {
    case 1: launch_copy<uint8_t>(src, dst_strides, dst_base, src->shape); break;
    case 2: launch_copy<uint16_t>(src, dst_strides, dst_base, src->shape); break;
    case 4: launch_copy<uint32_t>(src, dst_strides, dst_base, src->shape); break;
    case 8: launch_copy<uint64_t>(src, dst_strides, dst_base, src->shape); break;
    default: fail("copy: bad dtype");
  }
}

}  // namespace

// ---- public ops -------------------------------------------------------------------

void copy_to_strides(const ArrayP &src, const Shape &dst_strides, char *dst_base) {
  if (dst_strides.size() != src->shape.size()) fail("copy: stride count does not match the rank");
  copy_strided(src, dst_strides, dst_base);
}

ArrayP contiguous(const ArrayP &a) {
  if (a->contiguous()) return a;
  auto o = new_array(a->dtype, a->shape);
  copy_strided(a, o->strides, o->data());
  return o;
}

void copy_into(const std::shared_ptr<Array> &dst, const ArrayP &src) {
  if (dst->dtype != src->dtype || dst->shape != src->shape) fail("copy: dtype or shape mismatch");
  if (src->size() == 0) return;
  if (src->contiguous()) {
    if (tracing()) {
      char *d = dst->data();
      const char *p = src->data();
      const size_t nb = src->nbytes();
      ArrayP keep = src;
      launch([=](hipStream_t s) {
        (void)keep;
        SHLO_HIP(hipMemcpyAsync(d, p, nb, hipMemcpyDeviceToDevice, s));
      });
    } else {
      SHLO_HIP(hipMemcpyAsync(dst->data(), src->data(), src->nbytes(), hipMemcpyDeviceToDevice, stream()));
    }
    return;
  }
  copy_strided(src, dst->strides, dst->data());
}

ArrayP concat(const std::vector<ArrayP> &xs, int axis) {
  if (xs.empty()) fail("concatenate: no operands");
  const int r = xs[0]->rank();
  if (axis < 0) axis += r;
  if (axis < 0 || axis >= r) fail(strf("concatenate: axis %d of a rank-%d array", axis, r));
  Shape out = xs[0]->shape;
  out[axis] = 0;
  for (auto &x : xs) {
    if (x->rank() != r || x->dtype != xs[0]->dtype) fail("concatenate: operands differ in rank or dtype");
    for (int d = 0; d < r; d++)
      if (d != axis && x->shape[d] != xs[0]->shape[d]) fail("concatenate: operand shapes differ off the axis");
    out[axis] += x->shape[axis];
  }
  auto o = new_array(xs[0]->dtype, out);
  int64_t at = 0;
  const size_t es = dtype_size(o->dtype);
  for (auto &x : xs) {
    copy_strided(x, o->strides, o->data() + at * o->strides[axis] * (int64_t)es);
    at += x->shape[axis];
  }
  return o;
}

ArrayP astype(const ArrayP &a, uint8_t dtype) {
  if (!dtype_valid(dtype)) fail(strf("astype: dtype %u is not carried", dtype));
  if (a->dtype == dtype) return a;
  auto o = new_array(dtype, a->shape);
  dispatch_dtype(a->dtype, [&](auto ti) {
    using TI = decltype(ti);
    if (dtype == kBool) {
      launch1<ToBoolF<TI>, TI, uint8_t>(a, o, ToBoolF<TI>{});
      return;
    }
    dispatch_dtype(dtype, [&](auto to) {
      using TO = decltype(to);
      launch1<CastF<TI, TO>, TI, TO>(a, o, CastF<TI, TO>{});
    });
  });
  return o;
}

ArrayP view_dtype(const ArrayP &a, uint8_t dtype) {
  if (!dtype_valid(dtype)) fail(strf("view: dtype %u is not carried", dtype));
  ArrayP c = contiguous(a);
  const size_t si = dtype_size(c->dtype), so = dtype_size(dtype);
  Shape s = c->shape;
  if (si != so) {
    if (s.empty()) fail("view: a scalar cannot change element size");
    const int64_t bytes = s.back() * (int64_t)si;
    if (bytes % (int64_t)so) fail("view: the last dimension does not divide");
    s.back() = bytes / (int64_t)so;
  }
  auto v = std::make_shared<Array>();
  v->buf = c->buf;
  v->offset = c->offset * (int64_t)si / (int64_t)so;
  if ((c->offset * (int64_t)si) % (int64_t)so) fail("view: misaligned offset");
  v->dtype = dtype;
  v->shape = s;
  v->strides = contiguous_strides(s);
  v->shadow = c->shadow;
  return v;
}

ArrayP unary(uint32_t op, const ArrayP &a) {
  if (op > kSigmoid && op != kSqrtApprox) fail("unary: unknown op code");
  auto o = new_array(a->dtype, a->shape);
  dispatch_dtype(a->dtype, [&](auto t) {
    using T = decltype(t);
    if constexpr (!is_flt<T>()) {
      if (op != kNeg && op != kAbs && op != kNot && op != kInvert)
        fail(strf("unary op %u on %s is not carried", op, dtype_name(a->dtype)));
    } else {
      if (op == kInvert) fail("invert on a float is not carried");
    }
    launch1<UnaryF<T>, T, T>(a, o, UnaryF<T>{op});
  });
  return o;
}

ArrayP binary(uint32_t op, const ArrayP &a0, const ArrayP &b0) {
  if (op == kMatmul) return matmul_builtin(a0, b0);
  if (op > kLOr && op != kDivApprox) fail("binary: unknown op code");
  if (a0->dtype != b0->dtype)
    fail(strf("binary: operand dtypes differ (%s, %s)", dtype_name(a0->dtype), dtype_name(b0->dtype)));
  const Shape out = broadcast_shapes(a0->shape, b0->shape);
  ArrayP a = a0->shape == out ? a0 : broadcast_to(a0, out);
  ArrayP b = b0->shape == out ? b0 : broadcast_to(b0, out);
  const bool cmp = op >= kEq && op <= kGe;
  auto o = new_array(cmp ? (uint8_t)kBool : a->dtype, out);
  dispatch_dtype(a->dtype, [&](auto t) {
    using T = decltype(t);
    if (cmp) {
      launch2<CompareF<T>, T, T, uint8_t>(a, b, o, CompareF<T>{op});
      return;
    }
    if constexpr (is_flt<T>()) {
      if (op == kAnd || op == kOr || op == kXor || op == kShl || op == kShr || op == kLAnd || op == kLOr)
        fail(strf("binary op %u on %s is not carried", op, dtype_name(a->dtype)));
    }
    launch2<BinaryF<T>, T, T, T>(a, b, o, BinaryF<T>{op});
  });
  return o;
}

ArrayP where(const ArrayP &c0, const ArrayP &a0, const ArrayP &b0) {
  if (a0->dtype != b0->dtype) fail("where: operand dtypes differ");
  const Shape out = broadcast_shapes(broadcast_shapes(c0->shape, a0->shape), b0->shape);
  ArrayP c = broadcast_to(c0->dtype == kBool ? c0 : astype(c0, kBool), out);
  ArrayP a = broadcast_to(a0, out), b = broadcast_to(b0, out);
  auto o = new_array(a->dtype, out);
  const int64_t n = o->size();
  if (n == 0) return o;
  check_elems(n);
  auto m = make_map<3>(out, {&c->strides, &a->strides, &b->strides});
  dispatch_dtype(a->dtype, [&](auto t) {
    using T = decltype(t);
    const uint8_t *pc = (const uint8_t *)c->data();
    const T *pa = (const T *)a->data();
    const T *pb = (const T *)b->data();
    T *po = (T *)o->data();
    ArrayP kc = c, ka = a, kb = b;
    launch([=](hipStream_t s) {
      (void)kc, (void)ka, (void)kb;
      ew3<WhereF<T>, uint8_t, T, T, T><<<grid_for(n), kBlock, 0, s>>>(m, (uint32_t)n, pc, pa, pb, po, WhereF<T>{});
    });
  });
  return o;
}

// ---- take, max over an axis, iota, count_nonzero ----------------------------------

namespace {

template <class T, class I>
__global__ void take_k(uint64_t n, uint64_t inner, uint64_t nidx, uint64_t dim, const T *a, const I *idx, T *o) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t in = i % inner;
    const uint64_t j = (i / inner) % nidx;
    const uint64_t pre = i / (inner * nidx);
    int64_t k = (int64_t)idx[j];
    k = k < 0 ? 0 : (k >= (int64_t)dim ? (int64_t)dim - 1 : k);
    o[i] = a[(pre * dim + (uint64_t)k) * inner + in];
  }
}

template <class T>
__global__ void max_axis_k(uint64_t n, uint64_t inner, uint64_t len, const T *a, T *o) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t in = i % inner, pre = i / inner;
    const T *p = a + pre * len * inner + in;
    T m = p[0];
    for (uint64_t k = 1; k < len; k++) {
      const T v = p[k * inner];
      if constexpr (is_flt<T>()) {
        if (m != m) continue;
        if (v != v || v > m) m = v;
      } else {
        if (v > m) m = v;
      }
    }
    o[i] = m;
  }
}

template <class T>
__global__ void iota_k(uint64_t n, uint64_t inner, uint64_t len, T *o) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
    o[i] = (T)((i / inner) % len);
}

template <class T>
__global__ void nonzero_k(uint64_t n, const T *a, unsigned long long *count) {
  __shared__ unsigned long long part[kBlock];
  unsigned long long c = 0;
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
    c += a[i] != (T)0;
  part[threadIdx.x] = c;
  __syncthreads();
  for (int w = kBlock / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) atomicAdd(count, part[0]);
}

__global__ void zero_u64_k(unsigned long long *p) { *p = 0; }

}  // namespace

ArrayP take(const ArrayP &a0, const ArrayP &idx0, int axis) {
  ArrayP a = contiguous(a0), idx = contiguous(idx0);
  const int r = a->rank();
  if (axis < 0) axis += r;
  if (axis < 0 || axis >= r) fail("take: axis out of range");
  Shape out(a->shape.begin(), a->shape.begin() + axis);
  for (int64_t d : idx->shape) out.push_back(d);
  for (int d = axis + 1; d < r; d++) out.push_back(a->shape[d]);
  auto o = new_array(a->dtype, out);
  const uint64_t n = o->size();
  if (!n) return o;
  uint64_t inner = 1;
  for (int d = axis + 1; d < r; d++) inner *= a->shape[d];
  const uint64_t nidx = idx->size(), dim = a->shape[axis];
  if (dim == 0) fail("take: empty axis");
  dispatch_dtype(a->dtype, [&](auto t) {
    using T = decltype(t);
    auto go = [&](auto it) {
      using I = decltype(it);
      const T *pa = (const T *)a->data();
      const I *pi = (const I *)idx->data();
      T *po = (T *)o->data();
      ArrayP ka = a, ki = idx;
      launch([=](hipStream_t s) {
        (void)ka, (void)ki;
        take_k<T, I><<<grid_for((int64_t)n), kBlock, 0, s>>>(n, inner, nidx, dim, pa, pi, po);
      });
    };
    switch (idx->dtype) {
      case kI32: go(int32_t{}); break;
      case kU32: go(uint32_t{}); break;
      case kI64: go(int64_t{}); break;
      case kU64: go(uint64_t{}); break;
      default: fail("take: indices must be 32- or 64-bit integers");
    }
  });
  return o;
}

ArrayP max_axis(const ArrayP &a0, int axis) {
  ArrayP a = contiguous(a0);
  const int r = a->rank();
  if (axis < 0) axis += r;
  if (axis < 0 || axis >= r) fail("max_axis: axis out of range");
  if (a->shape[axis] == 0) fail("max_axis: empty axis");
  Shape out;
  uint64_t inner = 1;
  for (int d = 0; d < r; d++)
    if (d != axis) out.push_back(a->shape[d]);
  for (int d = axis + 1; d < r; d++) inner *= a->shape[d];
  auto o = new_array(a->dtype, out);
  const uint64_t n = o->size(), len = a->shape[axis];
  if (!n) return o;
  dispatch_dtype(a->dtype, [&](auto t) {
    using T = decltype(t);
    const T *pa = (const T *)a->data();
    T *po = (T *)o->data();
    ArrayP ka = a;
    launch([=](hipStream_t s) {
      (void)ka;
      max_axis_k<T><<<grid_for((int64_t)n), kBlock, 0, s>>>(n, inner, len, pa, po);
    });
  });
  return o;
}

ArrayP iota(uint8_t dtype, const Shape &shape, int dim) {
  auto o = new_array(dtype, shape);
  const uint64_t n = o->size();
  if (!n) return o;
  if (dim < 0 || dim >= (int)shape.size()) fail("iota: dimension out of range");
  uint64_t inner = 1;
  for (size_t d = dim + 1; d < shape.size(); d++) inner *= shape[d];
  const uint64_t len = shape[dim];
  dispatch_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    T *po = (T *)o->data();
    launch([=](hipStream_t s) { iota_k<T><<<grid_for((int64_t)n), kBlock, 0, s>>>(n, inner, len, po); });
  });
  return o;
}

int64_t count_nonzero(const ArrayP &a0) {
  if (tracing()) fail("count_nonzero: not available while a function is being traced");
  ArrayP a = contiguous(a0);
  auto cnt = new_array(kU64, Shape{1});
  unsigned long long *pc = (unsigned long long *)cnt->data();
  const uint64_t n = a->size();
  zero_u64_k<<<1, 1, 0, stream()>>>(pc);
  check_launch("count_nonzero");
  if (n) {
    switch (dtype_size(a->dtype)) {
      case 1: nonzero_k<uint8_t><<<grid_for((int64_t)n), kBlock, 0, stream()>>>(n, (const uint8_t *)a->data(), pc); break;
      case 2: nonzero_k<uint16_t><<<grid_for((int64_t)n), kBlock, 0, stream()>>>(n, (const uint16_t *)a->data(), pc); break;
      case 4: nonzero_k<uint32_t><<<grid_for((int64_t)n), kBlock, 0, stream()>>>(n, (const uint32_t *)a->data(), pc); break;
      case 8: nonzero_k<uint64_t><<<grid_for((int64_t)n), kBlock, 0, stream()>>>(n, (const uint64_t *)a->data(), pc); break;
    }
    check_launch("count_nonzero");
  }
  uint64_t h = 0;
  array_to_host(cnt, &h);
  return (int64_t)h;
}

// ---- the planted built-in matmul -------------------------------------------------

namespace {
// One thread per output, products fused into one running sum in k order: a
// different accumulation order from ggml_vec_dot_f32.
__global__ void matmul_natural_k(uint64_t n, uint64_t N, uint64_t M, uint64_t K, uint64_t bsa, uint64_t bsb,
                                 const float *a, const float *b, float *o) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t m = i % M, nn = (i / M) % N, bt = i / (M * N);
    const float *pa = a + bt * bsa + nn * K;
    const float *pb = b + bt * bsb + m;
    float s = 0.0f;
    for (uint64_t k = 0; k < K; k++) s = fmaf(pa[k], pb[k * M], s);
    o[i] = s;
  }
}
}  // namespace

ArrayP matmul_builtin(const ArrayP &a0, const ArrayP &b0) {
  if (a0->dtype != kF32 || b0->dtype != kF32) fail("matmul: f32 only");
  if (a0->rank() < 2 || b0->rank() < 2) fail("matmul: operands need rank 2 or more");
  const int64_t N = a0->shape[a0->rank() - 2], K = a0->shape[a0->rank() - 1];
  const int64_t K2 = b0->shape[b0->rank() - 2], M = b0->shape[b0->rank() - 1];
  if (K != K2) fail("matmul: inner dimensions differ");
  Shape ba(a0->shape.begin(), a0->shape.end() - 2), bb(b0->shape.begin(), b0->shape.end() - 2);
  Shape bo = broadcast_shapes(ba, bb);
  Shape sa = bo, sb = bo, so = bo;
  sa.push_back(N), sa.push_back(K);
  sb.push_back(K), sb.push_back(M);
  so.push_back(N), so.push_back(M);
  ArrayP a = contiguous(broadcast_to(a0, sa)), b = contiguous(broadcast_to(b0, sb));
  auto o = new_array(kF32, so);
  const uint64_t n = o->size();
  if (!n) return o;
  const float *pa = (const float *)a->data(), *pb = (const float *)b->data();
  float *po = (float *)o->data();
  ArrayP ka = a, kb = b;
  launch([=](hipStream_t s) {
    (void)ka, (void)kb;
    matmul_natural_k<<<grid_for((int64_t)n), kBlock, 0, s>>>(n, N, M, K, N * K, K * M, pa, pb, po);
  });
  return o;
}

}  // namespace shlo

// ---- synthetic inputs from the splitmix32 stream -----------------------------------

namespace shlo {
namespace {

// Draw t (0-based) of the stream seeded with `seed` (ref/ggml_ref.c:21-28).
__device__ __forceinline__ uint32_t splitmix32_at(uint32_t seed, uint64_t t) {
  uint32_t z = seed + (uint32_t)((t + 1) * 0x9e3779b9ull);
  z = (z ^ (z >> 16)) * 0x85ebca6bu;
  z = (z ^ (z >> 13)) * 0xc2b2ae35u;
  return z ^ (z >> 16);
}

__global__ void fill_unif_k(uint64_t n, uint32_t seed, uint64_t skip, float a, float *o) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
    const float u = (float)(splitmix32_at(seed, skip + i) >> 8) * (1.0f / 8388608.0f);
    o[i] = a * (u - 1.0f);
  }
}

__global__ void fill_normal_k(uint64_t n, uint32_t seed, uint64_t skip, double sigma, float *o) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
    double s = 0.0;
    for (int k = 0; k < 12; k++) s = s + (double)(splitmix32_at(seed, skip + 12 * i + k) >> 8) * 0x1p-24;
    o[i] = (float)((s - 6.0) * sigma);
  }
}

}  // namespace

ArrayP fill_random(const Shape &shape, uint32_t seed, uint64_t skip, int dist, double param) {
  auto o = new_array(kF32, shape);
  const uint64_t n = o->size();
  if (!n) return o;
  float *po = (float *)o->data();
  if (dist == 0) {
    const float a = (float)param;
    launch([=](hipStream_t s) { fill_unif_k<<<grid_for((int64_t)n), kBlock, 0, s>>>(n, seed, skip, a, po); });
  } else if (dist == 1) {
    launch([=](hipStream_t s) { fill_normal_k<<<grid_for((int64_t)n), kBlock, 0, s>>>(n, seed, skip, param, po); });
  } else {
    fail("fill_random: dist 0 (uniform) or 1 (normal)");
  }
  return o;
}

}  // namespace shlo

// ---- an order-free checksum of u32 words (test helper) ----------------------------------

namespace shlo {
namespace {

// sum over t of (w[t] + 1) * (2(start + t) + 1) * 0x9E3779B97F4A7C15 mod 2^64.
// Integer addition mod 2^64 is associative, so the atomic accumulation is exact.
__global__ void checksum_u32_k(uint64_t n, uint64_t start, const uint32_t *w, unsigned long long *out) {
  __shared__ unsigned long long part[kBlock];
  unsigned long long s = 0;
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
    s += ((unsigned long long)w[i] + 1ull) * (2ull * (start + i) + 1ull) * 0x9E3779B97F4A7C15ull;
  part[threadIdx.x] = s;
  __syncthreads();
  for (int k = kBlock / 2; k > 0; k >>= 1) {
    if ((int)threadIdx.x < k) part[threadIdx.x] += part[threadIdx.x + k];
    __syncthreads();
  }
  if (threadIdx.x == 0) atomicAdd(out, part[0]);
}

}  // namespace

uint64_t checksum_u32(const ArrayP &a0, uint64_t start) {
  if (tracing()) fail("checksum: not available while a function is being traced");
  if (dtype_size(a0->dtype) != 4) fail("checksum: 32-bit words only");
  ArrayP a = contiguous(a0);
  auto cnt = new_array(kU64, Shape{1});
  unsigned long long *pc = (unsigned long long *)cnt->data();
  zero_u64_k<<<1, 1, 0, stream()>>>(pc);
  check_launch("checksum");
  const uint64_t n = a->size();
  if (n) {
    checksum_u32_k<<<grid_for((int64_t)n), kBlock, 0, stream()>>>(n, start, (const uint32_t *)a->data(), pc);
    check_launch("checksum");
  }
  uint64_t h = 0;
  array_to_host(cnt, &h);
  return h;
}

}  // namespace shlo
