// Correctly rounded binary32 erf, host and device.
//
// ggml_vec_gelu_erf_f32 calls the platform erff (StablehloMlx/Kernels/
// Shaders.lean:24, :186-199).  The reference's pinned ggml build links a
// correctly rounded erff (CORE-MATH, ref/build.sh:52); its stock build's Apple
// libsystem_m erff is closed code and not reproduced here.  A correctly rounded
// function is fixed by the mathematics, so this routine is our own:
//
//   a = min(|x|, 255/64);  R = a * Q_i(64 a - i), i = floor(64 a)  (table,
//   binary64);  y = RN_binary32(R), sign restored.
//
// The tables (erff_tables.h) bound |Q_i - erf(a)/a| by 2^-51.8 relative.  When
// R lies within 2^5 binary64 units (2^-47 relative) of a binary32 rounding
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

// Inputs are clamped to kClampA = 255/64, the start of the last interval:
// erf(kClampA) rounds to 1, as erf of every larger input (and infinity) does.
constexpr float kClampA = 3.984375f;
constexpr uint32_t kClampBits = 0x407F0000u;

// R ~ erf(a64 / 64) in binary64 for a64 in [0, 255] (a quiet NaN is clamped
// there by the callers' v_min_f32 / fminf, which return the number),
// branch-free: i = floor(a64), u = a64 - i, R = a64 * (Q_i(u) / 64) with
// row(i) pointing at Q_i / 64's six coefficients (tab + 6 i for a whole
// table; a caller may hold the table in pieces).  u is exact (the fraction of
// a binary64 copy of a binary32).
template <class Row>
__host__ __device__ inline double erf_R64_at(float a64, Row row) {
  const double ad = (double)a64;
#if defined(__HIP_DEVICE_COMPILE__)
  const double u = __builtin_amdgcn_fract(ad);  // ad - floor(ad), exact for ad >= 0
#else
  const double u = ad - __builtin_floor(ad);
#endif
  const unsigned i = (unsigned)(int)a64 & (unsigned)(kTab - 1);
  const double *p = row(i);
  double q = p[5];
  q = __builtin_fma(q, u, p[4]);
  q = __builtin_fma(q, u, p[3]);
  q = __builtin_fma(q, u, p[2]);
  q = __builtin_fma(q, u, p[1]);
  q = __builtin_fma(q, u, p[0]);
  return ad * q;
}

__host__ __device__ inline double erf_R64(float a64, const double *tab) {
  return erf_R64_at(a64, [tab](unsigned i) { return tab + 6 * i; });
}

// R ~ erf(min(a, kClampA)) for a = |x| >= 0 or a quiet NaN.
__host__ __device__ inline double erf_abs_R(float a, const double *tab) {
  return erf_R64(__builtin_fminf(a, kClampA) * 64.0f, tab);  // exact scaling
}

// The binary32 rounding of R is decided by R's low 29 fraction bits: it is
// undecided within 2^5 units of the midpoint 2^28.  undecided_distance(R) < 64
// exactly when R is undecided (R = +0 never is).
__host__ __device__ inline uint32_t undecided_distance(double R) {
  return ((uint32_t)d2u(R) & 0x1FFFFFFFu) - (0x10000000u - 0x20u);
}

// The correctly rounded erf of |x| as bits, for |x|'s bits ax (NaN excluded).
__host__ __device__ inline uint32_t erf_abs_bits(uint32_t ax, const double *tab) {
  const double R = erf_abs_R(u2f(ax), tab);
  const uint32_t r = f2u((float)R);
  return undecided_distance(R) < 0x40u ? exception_lookup(ax, r) : r;
}

__host__ __device__ inline float erff_cr(float x, const double *tab) {
  const uint32_t ux = f2u(x);
  const uint32_t ax = ux & 0x7FFFFFFFu;
  const float y = u2f(erf_abs_bits(ax, tab) | (ux & 0x80000000u));
  return ax > 0x7F800000u ? x + x : y;  // NaN: the input, quieted
}

}  // namespace erffk
}  // namespace shlo
