/*
 * CPU oracle of ggml-cpu's arm64 NEON semantics — TEST INFRASTRUCTURE ONLY.
 *
 * Nothing in the product (the HIP library, its host code, the CLI) may link,
 * load or call this.  It is the checker: tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg use it, nothing else.
 *
 * Every routine is a plain C11 restatement of the ggml-cpu routine that the
 * reference executor reproduces on its GPU, in the order ggml accumulates.
 * Build: -O2 -ffp-contract=off, no fast-math, explicit fmaf() only where ggml
 * fuses (see oracle/Makefile).
 *
 * How each function is pinned (checked against something that is not this
 * file) is listed next to it; the tests under tests/test_oracle*.py do the
 * checking.
 */
#ifndef SHLO_ORACLE_H
#define SHLO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- input streams ----------------------------------------------------- */

/* splitmix32 stream and `unif`, ref/ggml_ref.c:21-30.  Pinned by the in*.f32
 * hashes of evidence/ref-*.sha256 (every case's inputs). */
uint32_t orc_rnd(uint32_t *state);
float orc_unif(uint32_t *state, float a);
void orc_fill_unif(uint32_t *state, float a, float *dst, size_t n);

/* Portable normal: Irwin-Hall sum of 12 of the stream's 24-bit uniforms,
 * centred, times sigma, one rounding to binary32.  Every step before the last
 * multiply is exact in binary64, so the bits are host-independent.  Used only
 * for the measurement configs (no reference fixture exists for them). */
float orc_normal(uint32_t *state, double sigma);
void orc_fill_normal(uint32_t *state, double sigma, float *dst, size_t n);

/* ---- ggml_vec_dot_f32 (mul_mat) ---------------------------------------- */

/* Tail flavours of the dot product past the last full block of 16.
 *   ORC_TAIL_STOCK  : tail >= 4 -> groups of four as separately rounded
 *                     products added in order, the rest fused
 *                     (StablehloMlx/Kernels/Shaders.lean:80-90);
 *   ORC_TAIL_PINNED : every tail element an unfused multiply then add
 *                     (-ffp-contract=off build, evidence/README.md:44-46);
 *   ORC_TAIL_PLAIN  : the planted wrong lowering, a sequential binary32 sum
 *                     without FMA over the whole row (Shaders.lean:65-68). */
enum { ORC_TAIL_STOCK = 0, ORC_TAIL_PINNED = 1, ORC_TAIL_PLAIN = 2 };

/* One output: dot(w[0..K), x[0..K)) in ggml order.  Pinned by the ten
 * mul_mat_* out.f32 hashes in both flavours. */
float orc_vec_dot(const float *w, const float *x, int64_t K, int tail);

/* The ggml mul_mat layout used by the reference's Run.mulMat (Run.lean:64-65,
 * Shaders.lean:49-64): y[r*M + m] = dot(w + ((r / N) * wBatchStride + m*K),
 * x + r*K), for R rows of x (wBatchStride is in elements; 0 = shared w).
 * nthreads > 1 splits rows of x over pthreads; each output is still one
 * thread's serial loop, so the bits do not depend on it. */
void orc_mul_mat(const float *w, const float *x, float *y, int64_t K, int64_t M, int64_t R,
                 int64_t N, int64_t wBatchStride, int tail, int nthreads);

/* ---- ggml_v_expf and the row ops --------------------------------------- */

/* ggml_v_expf one lane at a time, StablehloMlx/Kernels/Math.lean:28-49.
 * Pinned by the soft_max_* and silu_* hashes, and against exp() within its
 * documented error (a few ulp) on a sweep. */
float orc_ggml_v_expf(float x);

/* Correctly rounded binary32 exp and erf (what the pinned ggml build links,
 * CORE-MATH expf/erff, ref/build.sh:52).  expf: libquadmath expq at 113 bits,
 * rounded once.  erff: glibc's binary64 erf rounded to binary32 where that
 * rounding is provably the correct one, else erfq at 113 bits (see
 * oracle.c).  Pinned against MPFR on all 2^32 inputs (the chunk checksums in
 * tests/golden, checked by tests/test_oracle_erff.py) and by the gelu_erf_* /
 * *_tail hashes. */
float orc_expf_cr(float x);
float orc_erff_cr(float x);

/* ggml_soft_max over rows of `cols`, scale `scale` (no mask): ggml_vec_max_f32,
 * ggml_vec_soft_max_f32 (ggml_v_expf on groups of 4, each vaddvq_f32 group sum
 * added to a double in group order; tail elements via expf),
 * ggml_vec_scale_f32 with (float)(1.0/sum) (Shaders.lean:100-123).
 * float_sum != 0: the planted wrong lowering (binary32 denominator,
 * Shaders.lean:120-122).  Tail elements use orc_expf_cr (the pinned build's
 * expf). */
void orc_soft_max(const float *x, float *y, int64_t rows, int64_t cols, float scale, int float_sum,
                  int nthreads);

/* ggml_norm (Accelerate off): double sum, mean in binary32, cvar in groups of
 * four plus the scalar tail, 1/sqrtf(var+eps) (Shaders.lean:147-166).
 * gpu_ops != 0: the planted wrong lowering (binary32 sums, Shaders.lean:137-146). */
void orc_norm(const float *x, float *y, int64_t rows, int64_t cols, float eps, int gpu_ops,
              int nthreads);

/* ggml_vec_gelu_erf_f32: (0.5f*x)*(1.0f + erff(x*SQRT_2_INV)), NaN -> the
 * input quieted (Shaders.lean:186-199).  tanh_form != 0: the planted wrong
 * lowering (GELU's tanh form, Shaders.lean:192-194). */
float orc_gelu_erf1(float x, int tanh_form);
void orc_gelu_erf(const float *x, float *y, size_t n, int tanh_form, int nthreads);

/* ggml_vec_silu_f32 per row of `cols`: x / (1 + ggml_v_expf(0 - x)) on the
 * four-lane body, x / (1 + expf(-x)) on the row tail (Shaders.lean:172-179). */
void orc_silu(const float *x, float *y, int64_t rows, int64_t cols);

/* erff over `count` consecutive binary32 bit patterns from `base` (the CPU side
 * of the exhaustive check, Tests/OpTests.lean:273-296). */
void orc_erff_range(uint32_t base, uint32_t count, uint32_t *out, int nthreads);
/* orc_expf_cr over count consecutive binary32 patterns from base. */
void orc_expf_range(uint32_t base, uint32_t count, uint32_t *out, int nthreads);

/* An order-sensitive 64-bit checksum of `count` words: sum over t of
 * (w[t] + 1) * (2t + 1) * 0x9E3779B97F4A7C15 (mod 2^64).  Used to pin the
 * 256 chunks of the exhaustive erff sweep in a small committed fixture. */
uint64_t orc_checksum_words(const uint32_t *w, size_t count, uint64_t start_index);

/* ---- binary64 on the generic path --------------------------------------- */

/* The reference's soft-float binary64 (StablehloMlx/Kernels/SoftFloat.lean),
 * on bit patterns.  op: 0 add, 1 subtract, 2 multiply, 3 divide, 4 floor of
 * a, 5 a to int64 (the f64_ew op codes, Run.lean:87-92).  Rounding is the
 * host's IEEE binary64; the NaN, signed-zero and saturation rules are the
 * reference's.  Pinned by exact rational arithmetic (Python Fraction,
 * correctly rounded back) on random, subnormal and boundary operands, and by
 * the special cases SoftFloat.lean states (tests/test_oracle_f64.py). */
uint64_t orc_f64_ew(int op, uint64_t a, uint64_t b);
/* maximum (is_max) / minimum of binary64 (Lower.lean:290-296). */
uint64_t orc_f64_maxmin(int is_max, uint64_t a, uint64_t b);
/* binary32 -> binary64 and back (SoftFloat.lean:73-86, :95-120). */
uint64_t orc_f64_of_f32(uint32_t x);
uint32_t orc_f32_of_f64(uint64_t d);
/* Element-wise forms over n values (b may be NULL for ops 4 and 5). */
void orc_f64_ew_n(int op, const uint64_t *a, const uint64_t *b, uint64_t *out, size_t n);
void orc_f64_maxmin_n(int is_max, const uint64_t *a, const uint64_t *b, uint64_t *out, size_t n);
void orc_f64_of_f32_n(const uint32_t *x, uint64_t *out, size_t n);
void orc_f32_of_f64_n(const uint64_t *x, uint32_t *out, size_t n);

/* ---- the fixture generator's cases (ref/ggml_ref.c:152-283) ------------- */

/* Writes <outdir>/<case>/in<i>.f32, out.f32, meta.txt for one case, in the
 * given flavour ("stock" or "pinned").  Returns 0, or -1 for an unknown case,
 * -2 for an I/O error. */
int orc_write_case(const char *outdir, const char *name, int pinned);
/* Number of cases and the i-th case name (the order of ref/ggml_ref.c:286-295). */
int orc_case_count(void);
const char *orc_case_name(int i);

#ifdef __cplusplus
}
#endif
#endif
