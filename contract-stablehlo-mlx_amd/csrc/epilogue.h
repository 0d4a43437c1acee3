// Element-wise binary32 operations and the fused epilogue a producing kernel
// (dot_general, norm) applies to each output before it stores it.
//
// A StableHLO add / subtract / multiply / divide / maximum / minimum is one
// correctly rounded IEEE operation per element (Lower.lean:13-17, :375-452),
// so applying it to a value in registers right after the producing kernel
// computed it gives the same bits as the separate element-wise kernel reading
// the stored value back: f32_binary below is the one definition both use.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "ops.h"

namespace shlo {

// Binary32 semantics of the arithmetic binary op codes
// (StablehloMlx/Mlx.lean:88-108): maximum / minimum order -0 below +0
// (mx::maximum).  A NaN operand propagates as on arm64 and x86 (the first
// NaN operand, quieted, sign kept): the result is x + y, which the GPU's add
// returns that way, where its subtract would flip a NaN's sign.  The NaN case
// is a select, not a branch, so a wave never diverges over it.
__host__ __device__ inline float f32_binary(uint32_t op, float x, float y) {
  float r;
  switch (op) {
    case kAdd: r = x + y; break;
    case kSub: r = x - y; break;
    case kMul: r = x * y; break;
    case kDiv: r = x / y; break;  // correctly rounded: built with -fhip-fp32-correctly-rounded-divide-sqrt
    case kMax: r = x == y ? (std::signbit(x) ? y : x) : (x > y ? x : y); break;
    case kMin: r = x == y ? (std::signbit(x) ? x : y) : (x < y ? x : y); break;
    default: r = x; break;
  }
  return __builtin_isunordered(x, y) ? x + y : r;
}

// Up to kMaxEpi ops applied in order to an output value v at index
// (i0, i1, i2) of the producer's output: a binary op v = op(v, p[i0*s0 +
// i1*s1 + i2*s2]), or op(p[...], v) when `rev` (the produced value was the
// op's right operand); or the unary ggml gelu_erf (code kEpiGeluErf, no
// operand; the producer supplies the routine).
struct EpiOp {
  const float *p;
  int64_t s0, s1, s2;
  uint32_t code, rev;
};
struct Epilogue {
  EpiOp op[kMaxEpi];
  int n = 0;
  int gelu = 0;  // some op is kEpiGeluErf
};

// The identity for producers whose chains hold no unary op.
struct NoUnary {
  __device__ float operator()(float v) const { return v; }
};

// A chain's unary op on all NV values a lane holds.  A producer's routine
// may overload this for its own type (found by argument-dependent lookup) to
// share work across the values; its results must be the value-by-value ones.
template <class Unary, int NV>
__device__ __forceinline__ void unary_all(const Unary &un, float (&v)[NV]) {
#pragma unroll
  for (int r = 0; r < NV; r++) v[r] = un(v[r]);
}

// Whether an op's operand takes one value over the NV values a lane holds
// (then one load serves them all); by default never.
struct NeverUniform {
  __device__ bool operator()(const EpiOp &) const { return false; }
};

template <class Unary = NoUnary>
__device__ __forceinline__ float epi_apply(const Epilogue &e, float v, int64_t i0, int64_t i1, int64_t i2,
                                           Unary un = Unary()) {
#pragma unroll
  for (int k = 0; k < kMaxEpi; k++) {
    if (k < e.n) {
      const EpiOp &o = e.op[k];
      if (o.code == kEpiGeluErf) {
        v = un(v);
        continue;
      }
      const float w = o.p[i0 * o.s0 + i1 * o.s1 + i2 * o.s2];
      v = o.rev ? f32_binary(o.code, w, v) : f32_binary(o.code, v, w);
    }
  }
  return v;
}

// The fused ops on NV output values a lane holds: value r sits at element
// offset off(op, r) of each op's operand (a producer clamps the offsets of
// values it discards into range).  One uniform switch per op, then the op on
// all NV values, their operand loads issued together.  The operand order is
// a branch around the whole loop, not a select per value.
template <uint32_t C, bool REV, int NV>
__device__ __forceinline__ void epi_op_in(float (&v)[NV], const float (&w)[NV]) {
#pragma unroll
  for (int r = 0; r < NV; r++) v[r] = REV ? f32_binary(C, w[r], v[r]) : f32_binary(C, v[r], w[r]);
}
template <uint32_t C, int NV>
__device__ __forceinline__ void epi_op(float (&v)[NV], const float (&w)[NV], uint32_t rev) {
  if (rev)
    epi_op_in<C, true>(v, w);
  else
    epi_op_in<C, false>(v, w);
}

// The same in two steps, for a producer that can issue the operand loads
// long before its values are ready: epi_load_n, then epi_ops_n, for the first
// NE ops (epi_apply_n's `from` then takes the rest).
template <int NE, int NV, class Off, class Uni = NeverUniform>
__device__ __forceinline__ void epi_load_n(const Epilogue &e, float (&w)[NE][NV], Off off, Uni uni = Uni()) {
#pragma unroll
  for (int k = 0; k < NE; k++) {
    if (k >= e.n) break;
    if (e.op[k].code == kEpiGeluErf) continue;
    if (uni(e.op[k])) {
      const float w0 = e.op[k].p[off(e.op[k], 0)];
#pragma unroll
      for (int r = 0; r < NV; r++) w[k][r] = w0;
      continue;
    }
#pragma unroll
    for (int r = 0; r < NV; r++) w[k][r] = e.op[k].p[off(e.op[k], r)];
  }
}


template <int NE, int NV, class Unary = NoUnary>
__device__ __forceinline__ void epi_ops_n(const Epilogue &e, float (&v)[NV], const float (&w)[NE][NV],
                                          Unary un = Unary()) {
#pragma unroll
  for (int k = 0; k < NE; k++) {
    if (k >= e.n) break;
    const EpiOp &o = e.op[k];
    switch (o.code) {
      case kEpiGeluErf: unary_all(un, v); break;
      case kAdd: epi_op<kAdd>(v, w[k], o.rev); break;
      case kSub: epi_op<kSub>(v, w[k], o.rev); break;
      case kMul: epi_op<kMul>(v, w[k], o.rev); break;
      case kDiv: epi_op<kDiv>(v, w[k], o.rev); break;
      case kMax: epi_op<kMax>(v, w[k], o.rev); break;
      case kMin: epi_op<kMin>(v, w[k], o.rev); break;
      default: break;
    }
  }
}

template <int NV, class Off, class Unary = NoUnary, class Uni = NeverUniform>
__device__ __forceinline__ void epi_apply_n(const Epilogue &e, float (&v)[NV], Off off, int from = 0,
                                            Unary un = Unary(), Uni uni = Uni()) {
#pragma unroll
  for (int k = 0; k < kMaxEpi; k++) {
    if (k < from) continue;
    if (k >= e.n) break;
    const EpiOp &o = e.op[k];
    if (o.code == kEpiGeluErf) {
      unary_all(un, v);
      continue;
    }
    float w[NV];
    if (uni(o)) {
      const float w0 = o.p[off(o, 0)];
#pragma unroll
      for (int r = 0; r < NV; r++) w[r] = w0;
    } else {
#pragma unroll
      for (int r = 0; r < NV; r++) w[r] = o.p[off(o, r)];
    }
    switch (o.code) {
      case kAdd: epi_op<kAdd>(v, w, o.rev); break;
      case kSub: epi_op<kSub>(v, w, o.rev); break;
      case kMul: epi_op<kMul>(v, w, o.rev); break;
      case kDiv: epi_op<kDiv>(v, w, o.rev); break;
      case kMax: epi_op<kMax>(v, w, o.rev); break;
      case kMin: epi_op<kMin>(v, w, o.rev); break;
      default: break;
    }
  }
}

}  // namespace shlo
