// Correctly rounded binary32 erf, host and device.
//
// ggml_vec_gelu_erf_f32 calls the platform erff (StablehloMlx/Kernels/
// Shaders.lean:24, :186-199).  The reference's pinned ggml build links a
// correctly rounded erff (CORE-MATH, ref/build.sh:52); its stock build's Apple
// libsystem_m erff is closed code and not reproduced here.  A correctly rounded
// function is fixed by the mathematics, so this routine is our own:
//
//   a = |x| in binary64;  R = a*S(a^2) (a < 1/16)  or  P_i(a - c_i) (table);
//   y = RN_binary32(R), sign restored.
//
// The tables (erff_tables.h) bound |R - erf(a)| by 2^-49.3 relative.  When R
// lies within 2^7 binary64 units (2^-45 relative) of a binary32 rounding
// boundary the rounding is undecided, and the input's correctly rounded value
// is looked up in erff_exceptions.h, which lists every such input.  The whole
// function is checked on all 2^32 inputs against MPFR.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "erff_exceptions.h"
#include "erff_tables.h"

namespace shlo {
namespace erffk {

__host__ __device__ inline uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ inline float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
__host__ __device__ inline uint64_t d2u(double d) { return __builtin_bit_cast(uint64_t, d); }

// erf(|x|) in binary64 for |x| < kOneBits, non-NaN; `tab` is kPoly (global,
// constant or LDS copy).  Sets *undecided when the binary32 rounding of the
// result is not certain.
__host__ __device__ inline double erf_abs_binary64(uint32_t ax, const double *tab, bool *undecided) {
  const float a = u2f(ax);
  const double A = (double)a;
  double R;
  if (ax < 0x3D800000u) {  // a < 1/16
    const double t = A * A;
    double s = kSmall[5];
    s = __builtin_fma(s, t, kSmall[4]);
    s = __builtin_fma(s, t, kSmall[3]);
    s = __builtin_fma(s, t, kSmall[2]);
    s = __builtin_fma(s, t, kSmall[1]);
    s = __builtin_fma(s, t, kSmall[0]);
    R = A * s;
  } else {
    const int i = (int)(a * 64.0f);              // exact scaling, a < 4
    const double h = A - (double)(2 * i + 1) * 0x1p-7;  // exact
    const double *p = tab + 6 * i;
    double s = p[5];
    s = __builtin_fma(s, h, p[4]);
    s = __builtin_fma(s, h, p[3]);
    s = __builtin_fma(s, h, p[2]);
    s = __builtin_fma(s, h, p[1]);
    s = __builtin_fma(s, h, p[0]);
    R = s;
  }
  // The binary32 rounding of R is decided by R's low 29 fraction bits (for a
  // normal binary32 result): undecided within 2^7 units of the midpoint 2^28.
  const uint32_t low = (uint32_t)d2u(R) & 0x1FFFFFFFu;
  *undecided = (uint32_t)(low - (0x10000000u - 0x80u)) < 0x100u;
  return R;
}

// Binary search of the sorted exception list (|x| bits -> |erf| bits).
__host__ __device__ inline uint32_t exception_lookup(uint32_t ax, uint32_t fallback) {
  int lo = 0, hi = kNumExceptions - 1;
  while (lo <= hi) {
    const int mid = (lo + hi) >> 1;
    const uint32_t k = kExceptions[mid][0];
    if (k == ax) return kExceptions[mid][1];
    if (k < ax) lo = mid + 1;
    else hi = mid - 1;
  }
  return fallback;
}

__host__ __device__ inline float erff_cr(float x, const double *tab) {
  const uint32_t ux = f2u(x);
  const uint32_t ax = ux & 0x7FFFFFFFu;
  if (ax > 0x7F800000u) return x + x;  // NaN: the input, quieted
  uint32_t r;
  if (ax >= kOneBits) {
    r = 0x3F800000u;
  } else if (ax == 0) {
    r = 0;
  } else {
    bool undecided;
    const double R = erf_abs_binary64(ax, tab, &undecided);
    r = f2u((float)R);
    if (undecided) r = exception_lookup(ax, r);
  }
  return u2f(r | (ux & 0x80000000u));
}

}  // namespace erffk
}  // namespace shlo
