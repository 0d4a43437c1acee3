// Correctly rounded binary32 exp, host and device.
//
// ggml-cpu sends a soft_max row's last cols % 4 elements, and silu's, through
// the platform expf (ggml_vec_soft_max_f32; Shaders.lean:100-123, :172-179 of
// the reference restate the four-lane body only).  The reference's pinned ggml
// build links CORE-MATH's correctly rounded expf (ref/build.sh:52).  A
// correctly rounded function is fixed by the mathematics, so this routine is
// our own:
//
//   k = rint(64 x / ln2),  r = x - k ln2/64  (binary64, two FMAs),
//   R = 2^(k >> 6) * T[k & 63] * P(r),  y = RN_binary32(R).
//
// The relative error of R is below 2^-51.3 (table 2^-54, P 2^-54.7, three
// binary64 roundings).  When R lies within R * 2^-49 of a binary32 rounding
// midpoint the rounding is undecided, and the input's correctly rounded value
// is looked up in expf_exceptions.h, which lists every such input.  The whole
// function is checked on all 2^32 inputs against MPFR.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "expf_exceptions.h"
#include "expf_tables.h"

namespace shlo {
namespace expfk {

__host__ __device__ inline uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ inline float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// Binary search of the sorted exception list (x bits -> exp bits).
__host__ __device__ inline uint32_t exception_lookup(uint32_t xb, uint32_t fallback) {
  int lo = 0, hi = kNumExceptions - 1;
  while (lo <= hi) {
    const int mid = (lo + hi) >> 1;
    const uint32_t k = kExceptions[mid][0];
    if (k == xb) return kExceptions[mid][1];
    if (k < xb) lo = mid + 1;
    else hi = mid - 1;
  }
  return fallback;
}

// R ~ exp(x) in binary64 for kMinBits <= x <= kMaxBits (as values).
__host__ __device__ inline double exp_R(float x) {
  const double xd = (double)x;
  const double kd = __builtin_rint(xd * kInvLn2x64);
  const int k = (int)kd;
  double r = __builtin_fma(-kd, kLn2d64Hi, xd);
  r = __builtin_fma(-kd, kLn2d64Lo, r);
  double p = kP[5];
  p = __builtin_fma(p, r, kP[4]);
  p = __builtin_fma(p, r, kP[3]);
  p = __builtin_fma(p, r, kP[2]);
  p = __builtin_fma(p, r, kP[1]);
  p = __builtin_fma(p, r, kP[0]);
  const double scale = __builtin_bit_cast(double, (uint64_t)(1023 + (k >> 6)) << 52);  // 2^(k>>6), normal
  return kT[k & 63] * p * scale;
}

// Whether R (> 0) lies within R * 2^-49 of the binary32 rounding midpoint
// nearest to it; y = RN_binary32(R), finite.
__host__ __device__ inline bool rounding_undecided(double R, float y) {
  const uint32_t yb = f2u(y);
  const double yd = (double)y;
  double mid;
  if (R >= yd) mid = yb == 0x7F7FFFFFu ? yd + 0x1p103 : 0.5 * (yd + (double)u2f(yb + 1));
  else mid = 0.5 * (yd + (double)u2f(yb - 1));  // y > 0 here: R < y and R > 0
  const double d = R - mid;
  return (d < 0 ? -d : d) <= R * 0x1p-49;
}

__host__ __device__ inline float expf_cr(float x) {
  const uint32_t xb = f2u(x);
  if ((xb & 0x7FFFFFFFu) > 0x7F800000u) return x + x;  // NaN: the input, quieted
  if (x > u2f(kMaxBits)) return __builtin_inff();
  if (x < u2f(kMinBits)) return 0.0f;
  const double R = exp_R(x);
  const float y = (float)R;
  return rounding_undecided(R, y) ? u2f(exception_lookup(xb, f2u(y))) : y;
}

}  // namespace expfk
}  // namespace shlo
