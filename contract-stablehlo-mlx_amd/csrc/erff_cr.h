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

// erf(|x|) as binary32 bits before the exception lookup and without the
// |x| >= kOneBits saturation, branch-free.  One Horner evaluation serves both
// ranges: row i = floor(64|x|) of `tab` holds, for i < 4 (|x| < 1/16), the
// small-argument polynomial S in t = x^2 (R = |x|*S(t)), and otherwise the
// interval polynomial in h = |x| - c_i (R = P_i(h)).  The index is clamped so
// NaN, infinity and |x| >= 4 stay in range (their results are replaced by the
// caller).  *undecided is set when R's binary32 rounding is not certain.
__host__ __device__ inline uint32_t erf_abs_bits_fast(uint32_t ax, const double *tab, bool *undecided) {
  const float a = u2f(ax);
  const double A = (double)a;
  const float a64 = a * 64.0f;                                              // exact scaling
  const int i = (int)(a64 < (float)(kTab - 1) ? a64 : (float)(kTab - 1));  // NaN -> kTab-1
  const bool small = ax < 0x3D800000u;                                      // |x| < 1/16, i < 4
  const double v = small ? A * A : A - (double)(2 * i + 1) * 0x1p-7;       // both exact
  const double *p = tab + 6 * i;
  double q = p[5];
  q = __builtin_fma(q, v, p[4]);
  q = __builtin_fma(q, v, p[3]);
  q = __builtin_fma(q, v, p[2]);
  q = __builtin_fma(q, v, p[1]);
  q = __builtin_fma(q, v, p[0]);
  const double R = small ? A * q : q;
  // The binary32 rounding of R is decided by R's low 29 fraction bits: it is
  // undecided within 2^7 units of the midpoint 2^28 (R = +0 is never flagged).
  const uint32_t low = (uint32_t)d2u(R) & 0x1FFFFFFFu;
  *undecided = ax < kOneBits && (uint32_t)(low - (0x10000000u - 0x80u)) < 0x100u;
  return f2u((float)R);
}

// The correctly rounded erf of x's magnitude as bits, from the fast bits and
// the undecided flag: the exception lookup, then saturation to 1.
__host__ __device__ inline uint32_t erf_abs_bits_finish(uint32_t ax, uint32_t r, bool undecided) {
  if (undecided) r = exception_lookup(ax, r);
  return ax >= kOneBits ? 0x3F800000u : r;
}

__host__ __device__ inline float erff_cr(float x, const double *tab) {
  const uint32_t ux = f2u(x);
  const uint32_t ax = ux & 0x7FFFFFFFu;
  bool undecided;
  const uint32_t r = erf_abs_bits_finish(ax, erf_abs_bits_fast(ax, tab, &undecided), undecided);
  const float y = u2f(r | (ux & 0x80000000u));
  return ax > 0x7F800000u ? x + x : y;  // NaN: the input, quieted
}

}  // namespace erffk
}  // namespace shlo
