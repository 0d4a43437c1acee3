// ggml-cpu's arm64 ggml_v_expf, one lane at a time (host and device).
//
// Restated from StablehloMlx/Kernels/Math.lean:28-49 (ggml vec.h, "adapted
// from arm limited optimized routine"): each vfmaq_f32(a, b, c) is
// fma(b, c, a), each vfmsq_f32(a, b, c) is fma(-b, c, a), and every constant
// is the same binary32 bit pattern.  The NEON code branches on all four lanes
// at once, but each lane's value depends only on that lane.  The two rare
// branches are computed as selects so a wave never diverges.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace shlo {

__host__ __device__ inline float bits_f(uint32_t u) { return __builtin_bit_cast(float, u); }
__host__ __device__ inline uint32_t f_bits(float f) { return __builtin_bit_cast(uint32_t, f); }

__host__ __device__ inline float ggml_v_expf(float x) {
  const float r = bits_f(0x4B400000u);                                  // 0x1.8p23f
  const float z = __builtin_fmaf(x, bits_f(0x3FB8AA3Bu), r);            // r + x*log2(e)
  const float n = z - r;
  const float b = __builtin_fmaf(-n, bits_f(0x35BFBE8Eu), __builtin_fmaf(-n, bits_f(0x3F317200u), x));
  const uint32_t e = f_bits(z) << 23;
  const float k = bits_f(e + 0x3F800000u);
  const float u = b * b;
  const float p1 = __builtin_fmaf(bits_f(0x3E2AAF33u), b, bits_f(0x3EFFFEDBu));
  const float p2 = __builtin_fmaf(bits_f(0x3C072010u), b, bits_f(0x3D2B9F17u));
  const float p3 = __builtin_fmaf(p2, u, p1);
  const float j = __builtin_fmaf(p3, u, bits_f(0x3F7FFFF6u) * b);
  const float an = __builtin_fabsf(n);
  const uint32_t d = n <= 0.0f ? 0x82000000u : 0u;
  const float s1 = bits_f(d + 0x7F000000u);
  const float s2 = bits_f(e - d);
  const float big = s1 * s1;                                             // |n| > 192
  const float mid = __builtin_fmaf(s2, j, s2) * s1;                      // |n| > 126
  const float nrm = __builtin_fmaf(k, j, k);
  return an > bits_f(0x43400000u) ? big : (an > bits_f(0x42FC0000u) ? mid : nrm);
}

// ggml_v_expf for arguments that are <= 0, -inf or NaN (a softmax row minus
// its maximum), with the same bits: there the |n| > 192 branch gives exactly
// +0 (2^-125 squared underflows), so only the 126 < |n| <= 192 branch needs its
// own formula.  *mid is set when x falls in that branch; the caller then
// recomputes x with ggml_v_expf.
__host__ __device__ inline float ggml_v_expf_nonpos(float x, bool *mid) {
  const float r = bits_f(0x4B400000u);
  const float z = __builtin_fmaf(x, bits_f(0x3FB8AA3Bu), r);
  const float n = z - r;
  const float b = __builtin_fmaf(-n, bits_f(0x35BFBE8Eu), __builtin_fmaf(-n, bits_f(0x3F317200u), x));
  const uint32_t e = f_bits(z) << 23;
  const float k = bits_f(e + 0x3F800000u);
  const float u = b * b;
  const float p1 = __builtin_fmaf(bits_f(0x3E2AAF33u), b, bits_f(0x3EFFFEDBu));
  const float p2 = __builtin_fmaf(bits_f(0x3C072010u), b, bits_f(0x3D2B9F17u));
  const float p3 = __builtin_fmaf(p2, u, p1);
  const float j = __builtin_fmaf(p3, u, bits_f(0x3F7FFFF6u) * b);
  const float an = __builtin_fabsf(n);
  const bool big = an > bits_f(0x43400000u);
  *mid = !big && an > bits_f(0x42FC0000u);
  return big ? 0.0f : __builtin_fmaf(k, j, k);
}

}  // namespace shlo
