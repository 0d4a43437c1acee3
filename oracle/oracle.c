/*
 * CPU oracle of ggml-cpu's arm64 NEON semantics — TEST INFRASTRUCTURE ONLY.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
 * this file (as the checker); the product never links it.
 *
 * Build with -O2 -ffp-contract=off (oracle/Makefile): every multiply and add
 * below is its own IEEE operation unless it is written as fmaf().
 *
 * Each routine restates the ggml-cpu routine that the reference reproduces on
 * its GPU.  Citations are into the reference repository
 * (V-Sekai-fire/contract-stablehlo-mlx); ggml itself (V-Sekai-fire/ggml
 * @29cae86726d8ae2b4d699d8e432fd1bb1801e959, ref/build.sh:24) is not in the
 * reference tree, so the reference's own restatements in
 * StablehloMlx/Kernels/Shaders.lean and Math.lean, its case table
 * (ref/ggml_ref.c) and its fixture hashes (evidence/ref-*.sha256) are the
 * anchors.  Parity status of every function is listed in oracle.h.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <errno.h>
#include <math.h>
#include <pthread.h>
#include <quadmath.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ---- a tiny pthread parallel-for over [0, n) ------------------------------ */

typedef void (*orc_body)(void *ctx, int64_t lo, int64_t hi);
struct orc_job { orc_body body; void *ctx; int64_t lo, hi; };
static void *orc_job_run(void *p) {
	struct orc_job *j = (struct orc_job *)p;
	j->body(j->ctx, j->lo, j->hi);
	return NULL;
}
static void orc_parallel(int64_t n, int nthreads, orc_body body, void *ctx) {
	if (nthreads <= 1 || n < 2) { body(ctx, 0, n); return; }
	if (nthreads > 256) nthreads = 256;
	if (nthreads > n) nthreads = (int)n;
	pthread_t th[256];
	struct orc_job jobs[256];
	for (int t = 0; t < nthreads; t++) {
		jobs[t].body = body;
		jobs[t].ctx = ctx;
		jobs[t].lo = n * t / nthreads;
		jobs[t].hi = n * (t + 1) / nthreads;
		pthread_create(&th[t], NULL, orc_job_run, &jobs[t]);
	}
	for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
}

/* ---- input streams (ref/ggml_ref.c:21-30) --------------------------------- */

uint32_t orc_rnd(uint32_t *state) {
	uint32_t z = (*state += 0x9e3779b9u);
	z = (z ^ (z >> 16)) * 0x85ebca6bu;
	z = (z ^ (z >> 13)) * 0xc2b2ae35u;
	return z ^ (z >> 16);
}

/* a * (u24 * 2^-23 - 1): the 24-bit draw, scaled and centred exactly, then one
 * rounding for the multiply by a (ref/ggml_ref.c:30). */
float orc_unif(uint32_t *state, float a) {
	float u = (float)(orc_rnd(state) >> 8) * (1.0f / 8388608.0f);
	return a * (u - 1.0f);
}

void orc_fill_unif(uint32_t *state, float a, float *dst, size_t n) {
	for (size_t i = 0; i < n; i++) dst[i] = orc_unif(state, a);
}

float orc_normal(uint32_t *state, double sigma) {
	double s = 0.0;
	for (int k = 0; k < 12; k++) s += (double)(orc_rnd(state) >> 8) * 0x1p-24;
	return (float)((s - 6.0) * sigma);
}

void orc_fill_normal(uint32_t *state, double sigma, float *dst, size_t n) {
	for (size_t i = 0; i < n; i++) dst[i] = orc_normal(state, sigma);
}

/* ---- ggml_vec_dot_f32 (Shaders.lean:55-91) ------------------------------ */

float orc_vec_dot(const float *w, const float *x, int64_t K, int tail) {
	if (tail == ORC_TAIL_PLAIN) {
		float s = 0.0f;
		for (int64_t i = 0; i < K; i++) s = s + w[i] * x[i];
		return s;
	}
	/* Four float32x4 accumulators over blocks of 16 (GGML_F32_STEP 16,
	 * GGML_F32_EPR 4): lane j of the block feeds accumulator j. */
	float a[16] = { 0 };
	const int64_t np = K & ~(int64_t)15;
	for (int64_t i = 0; i < np; i += 16)
		for (int j = 0; j < 16; j++) a[j] = fmaf(w[i + j], x[i + j], a[j]);
	/* GGML_F32x4_REDUCE: sum[0]+=sum[2], sum[1]+=sum[3], sum[0]+=sum[1] (each a
	 * four-lane add), then vaddvq_f32 = (v0+v1)+(v2+v3). */
	for (int l = 0; l < 4; l++) a[l] = a[l] + a[8 + l];
	for (int l = 0; l < 4; l++) a[4 + l] = a[4 + l] + a[12 + l];
	for (int l = 0; l < 4; l++) a[l] = a[l] + a[4 + l];
	float sumf = (a[0] + a[1]) + (a[2] + a[3]);
	if (tail == ORC_TAIL_PINNED) {
		for (int64_t i = np; i < K; i++) {
			float p = w[i] * x[i];
			sumf = sumf + p;
		}
		return sumf;
	}
	/* stock: Shaders.lean:80-90 */
	const int64_t tl = K - np;
	const int64_t nq = tl >= 4 ? (tl & ~(int64_t)3) : 0;
	for (int64_t i = np; i < np + nq; i++) {
		float p = w[i] * x[i];
		sumf = sumf + p;
	}
	for (int64_t i = np + nq; i < K; i++) sumf = fmaf(w[i], x[i], sumf);
	return sumf;
}

struct mm_ctx {
	const float *w, *x;
	float *y;
	int64_t K, M, N, wbs;
	int tail;
};
static void mm_rows(void *p, int64_t lo, int64_t hi) {
	struct mm_ctx *c = (struct mm_ctx *)p;
	for (int64_t r = lo; r < hi; r++) {
		const float *xr = c->x + r * c->K;
		const float *wb = c->w + (r / c->N) * c->wbs;
		for (int64_t m = 0; m < c->M; m++) c->y[r * c->M + m] = orc_vec_dot(wb + m * c->K, xr, c->K, c->tail);
	}
}

void orc_mul_mat(const float *w, const float *x, float *y, int64_t K, int64_t M, int64_t R,
                 int64_t N, int64_t wBatchStride, int tail, int nthreads) {
	struct mm_ctx c = { w, x, y, K, M, N > 0 ? N : 1, wBatchStride, tail };
	orc_parallel(R, nthreads, mm_rows, &c);
}

/* ---- ggml_v_expf, lane by lane (Math.lean:28-49) ------------------------- */

float orc_ggml_v_expf(float x) {
	const float r = u2f(0x4B400000u);                 /* 0x1.8p23f */
	const float z = fmaf(x, u2f(0x3FB8AA3Bu), r);
	const float n = z - r;
	const float b = fmaf(-n, u2f(0x35BFBE8Eu), fmaf(-n, u2f(0x3F317200u), x));
	const uint32_t e = f2u(z) << 23;
	const float k = u2f(e + 0x3F800000u);
	const float uu = b * b;
	const float p1 = fmaf(u2f(0x3E2AAF33u), b, u2f(0x3EFFFEDBu));
	const float p2 = fmaf(u2f(0x3C072010u), b, u2f(0x3D2B9F17u));
	const float p3 = fmaf(p2, uu, p1);
	const float j = fmaf(p3, uu, u2f(0x3F7FFFF6u) * b);
	const float an = fabsf(n);
	const uint32_t d = n <= 0.0f ? 0x82000000u : 0u;
	const float s1 = u2f(d + 0x7F000000u);
	if (an > u2f(0x43400000u)) return s1 * s1;        /* |n| > 192 */
	if (an > u2f(0x42FC0000u)) {                       /* |n| > 126 */
		const float s2 = u2f(e - d);
		return fmaf(s2, j, s2) * s1;
	}
	return fmaf(k, j, k);
}

/* ---- correctly rounded expf / erff -------------------------------------- */

float orc_expf_cr(float x) {
	if (x != x) return x + x;
	return (float)expq((__float128)x);
}

/* erf(x) rounded once to binary32.  Fast path: glibc's binary64 erf, whose
 * error is below one binary64 ulp (2^-52 relative), rounded to binary32.  That
 * rounding is the correct one unless erf(x) can lie on the other side of the
 * binary32 rounding boundary nearest to the binary64 value r, i.e. unless r
 * lies within r's error of that boundary.  The boundaries around f = (float)r
 * are the midpoints between f and its two binary32 neighbours (exact in
 * binary64); r within 2^-45 |r| of either (128 times the error bound) is
 * decided by libquadmath's erfq at 113 bits instead.  About 2^-20 of the
 * inputs take that path. */
float orc_erff_cr(float x) {
	if (x != x) return x + x;
	if (x == 0.0f) return x;
	const double r = erf((double)x);
	const float f = (float)r;
	const double lo = ((double)f + (double)nextafterf(f, -INFINITY)) * 0.5;
	const double hi = ((double)f + (double)nextafterf(f, INFINITY)) * 0.5;
	const double margin = fabs(r) * 0x1p-45;
	if (fabs(r - lo) > margin && fabs(hi - r) > margin) return f;
	return (float)erfq((__float128)x);
}

/* ---- ggml_soft_max (Shaders.lean:100-123) -------------------------------- */

struct sm_ctx {
	const float *x;
	float *y;
	int64_t cols;
	float scale;
	int float_sum;
};
static void sm_rows(void *p, int64_t lo, int64_t hi) {
	struct sm_ctx *c = (struct sm_ctx *)p;
	const int64_t N = c->cols;
	for (int64_t row = lo; row < hi; row++) {
		const float *x = c->x + row * N;
		float *y = c->y + row * N;
		float mx = -INFINITY;
		for (int64_t i = 0; i < N; i++) {
			const float wv = x[i] * c->scale;
			mx = mx > wv ? mx : wv;
		}
		double sum = 0.0;
		float fs = 0.0f;
		int64_t i = 0;
		for (; i + 3 < N; i += 4) {
			float e[4];
			for (int l = 0; l < 4; l++) {
				e[l] = orc_ggml_v_expf(x[i + l] * c->scale - mx);
				y[i + l] = e[l];
			}
			const float part = (e[0] + e[1]) + (e[2] + e[3]);
			sum += (double)part;
			fs = fs + part;
		}
		for (; i < N; i++) {  /* the row tail: the scalar expf */
			const float v = orc_expf_cr(x[i] * c->scale - mx);
			sum += (double)v;
			fs = fs + v;
			y[i] = v;
		}
		float inv = (float)(1.0 / sum);
		if (c->float_sum) inv = 1.0f / fs;
		for (int64_t q = 0; q < N; q++) y[q] = y[q] * inv;
	}
}

void orc_soft_max(const float *x, float *y, int64_t rows, int64_t cols, float scale, int float_sum,
                  int nthreads) {
	struct sm_ctx c = { x, y, cols, scale, float_sum };
	orc_parallel(rows, nthreads, sm_rows, &c);
}

/* ---- ggml_norm (Shaders.lean:130-166) ------------------------------------ */

struct nm_ctx {
	const float *x;
	float *y;
	int64_t cols;
	float eps;
	int gpu_ops;
};
static void nm_rows(void *p, int64_t lo, int64_t hi) {
	struct nm_ctx *c = (struct nm_ctx *)p;
	const int64_t N = c->cols;
	for (int64_t row = lo; row < hi; row++) {
		const float *x = c->x + row * N;
		float *y = c->y + row * N;
		if (c->gpu_ops) {
			float s = 0.0f;
			for (int64_t i = 0; i < N; i++) s = s + x[i];
			const float mean = s / (float)N;
			float s2 = 0.0f;
			for (int64_t i = 0; i < N; i++) {
				const float d = x[i] - mean;
				s2 = s2 + d * d;
			}
			const float scl = 1.0f / sqrtf(s2 / (float)N + c->eps);
			for (int64_t i = 0; i < N; i++) y[i] = (x[i] - mean) * scl;
			continue;
		}
		double sum = 0.0;
		for (int64_t i = 0; i < N; i++) sum += (double)x[i];
		const float mean = (float)sum / (float)N;
		double s2 = 0.0;
		const int64_t nb = N & ~(int64_t)3;
		for (int64_t i = 0; i < nb; i += 4) {
			float q[4];
			for (int l = 0; l < 4; l++) {
				const float d = x[i + l] - mean;
				q[l] = d * d;
			}
			s2 += (double)((q[0] + q[1]) + (q[2] + q[3]));
		}
		for (int64_t i = nb; i < N; i++) {
			const float d = x[i] - mean;
			const float q = d * d;
			s2 += (double)q;
		}
		const float var = (float)(s2 / (double)N);
		const float scl = 1.0f / sqrtf(var + c->eps);
		for (int64_t i = 0; i < N; i++) y[i] = (x[i] - mean) * scl;
	}
}

void orc_norm(const float *x, float *y, int64_t rows, int64_t cols, float eps, int gpu_ops,
              int nthreads) {
	struct nm_ctx c = { x, y, cols, eps, gpu_ops };
	orc_parallel(rows, nthreads, nm_rows, &c);
}

/* ---- gelu_erf (Shaders.lean:186-199) ------------------------------------- */

float orc_gelu_erf1(float x, int tanh_form) {
	float ev;
	if (tanh_form)
		ev = tanhf(u2f(0x3F4C422Au) * x * (1.0f + u2f(0x3D372713u) * x * x));
	else
		ev = orc_erff_cr(x * u2f(0x3F3504F3u));          /* SQRT_2_INV */
	float y = (0.5f * x) * (1.0f + ev);
	if ((f2u(x) & 0x7FFFFFFFu) > 0x7F800000u) y = u2f(f2u(x) | 0x00400000u);
	return y;
}

struct ge_ctx { const float *x; float *y; int tanh_form; };
static void ge_body(void *p, int64_t lo, int64_t hi) {
	struct ge_ctx *c = (struct ge_ctx *)p;
	for (int64_t i = lo; i < hi; i++) c->y[i] = orc_gelu_erf1(c->x[i], c->tanh_form);
}

void orc_gelu_erf(const float *x, float *y, size_t n, int tanh_form, int nthreads) {
	struct ge_ctx c = { x, y, tanh_form };
	orc_parallel((int64_t)n, nthreads, ge_body, &c);
}

/* ---- silu (Shaders.lean:172-179) ----------------------------------------- */

void orc_silu(const float *x, float *y, int64_t rows, int64_t cols) {
	for (int64_t r = 0; r < rows; r++) {
		const float *xr = x + r * cols;
		float *yr = y + r * cols;
		int64_t i = 0;
		/* the four-lane body covers the first cols & ~3 elements */
		for (; i < (cols & ~(int64_t)3); i++) yr[i] = xr[i] / (1.0f + orc_ggml_v_expf(0.0f - xr[i]));
		for (; i < cols; i++) yr[i] = xr[i] / (1.0f + orc_expf_cr(-xr[i]));
	}
}

/* ---- the exhaustive erff sweep's CPU side --------------------------------- */

struct er_ctx { uint32_t base; uint32_t *out; };
static void er_body(void *p, int64_t lo, int64_t hi) {
	struct er_ctx *c = (struct er_ctx *)p;
	for (int64_t i = lo; i < hi; i++) c->out[i] = f2u(orc_erff_cr(u2f(c->base + (uint32_t)i)));
}

void orc_erff_range(uint32_t base, uint32_t count, uint32_t *out, int nthreads) {
	struct er_ctx c = { base, out };
	orc_parallel((int64_t)count, nthreads, er_body, &c);
}

/* The same sweep for the correctly rounded expf (the row tails' expf). */
static void ex_body(void *p, int64_t lo, int64_t hi) {
	struct er_ctx *c = (struct er_ctx *)p;
	for (int64_t i = lo; i < hi; i++) c->out[i] = f2u(orc_expf_cr(u2f(c->base + (uint32_t)i)));
}

void orc_expf_range(uint32_t base, uint32_t count, uint32_t *out, int nthreads) {
	struct er_ctx c = { base, out };
	orc_parallel((int64_t)count, nthreads, ex_body, &c);
}

uint64_t orc_checksum_words(const uint32_t *w, size_t count, uint64_t start_index) {
	uint64_t s = 0;
	for (size_t i = 0; i < count; i++) {
		const uint64_t t = start_index + i;
		s += ((uint64_t)w[i] + 1u) * (2u * t + 1u) * 0x9E3779B97F4A7C15ull;
	}
	return s;
}

/* ---- binary64 on the generic path (StablehloMlx/Kernels/SoftFloat.lean) ----
 *
 * The reference carries f64 tensors as uint64 bit patterns through integer
 * soft-float kernels.  Their rounding is IEEE binary64 round-to-nearest-even
 * with subnormals, which the host's SSE2 arithmetic computes directly; what
 * follows restates their choices for NaNs, signed zeros and conversions. */

#define Q64 0x0008000000000000ull
#define INF64 0x7FF0000000000000ull
#define NAN64 0x7FF8000000000000ull  /* arm64's default NaN (invalid operations) */
#define SIGN64 0x8000000000000000ull
static inline uint64_t d2u(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
static inline double u2d(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }
static inline int nan64(uint64_t u) { return (u & ~SIGN64) > INF64; }

/* f64Add / f64Sub / f64Mul / f64Div (SoftFloat.lean:137-202, :239-259): a NaN
 * operand comes back quieted with its sign, the first operand's when both are
 * NaN; an invalid operation gives NAN64.  f64Floor (:204-217): exact, NaN
 * quieted, -0 kept.  f64ToI64 (:219-236): toward zero, saturating, NaN -> 0. */
uint64_t orc_f64_ew(int op, uint64_t a, uint64_t b) {
	if (op == 5) {
		if (nan64(a)) return 0;
		const double x = u2d(a);
		if (x >= 0x1p63) return 0x7FFFFFFFFFFFFFFFull;
		if (x <= -0x1p63) return SIGN64;
		return (uint64_t)(int64_t)x;
	}
	if (op == 4) {
		if (nan64(a)) return a | Q64;
		return d2u(floor(u2d(a)));
	}
	if (nan64(a)) return a | Q64;
	if (nan64(b)) return b | Q64;
	const double x = u2d(a), y = u2d(b);
	double r;
	switch (op) {
	case 0: r = x + y; break;
	case 1: r = x - y; break;
	case 2: r = x * y; break;
	case 3: r = x / y; break;
	default: return 0;
	}
	const uint64_t u = d2u(r);
	return nan64(u) ? NAN64 : u;
}

/* f64MaxMin (Lower.lean:290-296): a NaN operand (the first one) quieted; else
 * the larger (smaller) in an order with -0 below +0, the first operand on a
 * tie. */
uint64_t orc_f64_maxmin(int is_max, uint64_t a, uint64_t b) {
	if (nan64(a)) return a | Q64;
	if (nan64(b)) return b | Q64;
	/* f64Key: a uint64 whose unsigned order is the numeric order */
	const uint64_t ka = (a >> 63) ? ~a : (a | SIGN64), kb = (b >> 63) ? ~b : (b | SIGN64);
	return is_max ? (ka >= kb ? a : b) : (ka <= kb ? a : b);
}

/* f64FromF32 (SoftFloat.lean:73-86): exact widening; a NaN keeps its sign and
 * payload shifted up, without setting the quiet bit. */
uint64_t orc_f64_of_f32(uint32_t x) {
	if ((x & 0x7FFFFFFFu) > 0x7F800000u)
		return ((uint64_t)(x >> 31) << 63) | INF64 | ((uint64_t)(x & 0x7FFFFFu) << 29);
	return d2u((double)u2f(x));
}

/* f64ToF32 (SoftFloat.lean:95-120): round to nearest even with binary32
 * subnormals, overflow to infinity; a NaN keeps its sign and the top of its
 * payload, quieted. */
uint32_t orc_f32_of_f64(uint64_t d) {
	if (nan64(d))
		return (uint32_t)((d >> 32) & 0x80000000u) | 0x7FC00000u | (uint32_t)((d & 0xFFFFFFFFFFFFFull) >> 29);
	return f2u((float)u2d(d));
}

void orc_f64_ew_n(int op, const uint64_t *a, const uint64_t *b, uint64_t *out, size_t n) {
	for (size_t i = 0; i < n; i++) out[i] = orc_f64_ew(op, a[i], b ? b[i] : a[i]);
}
void orc_f64_maxmin_n(int is_max, const uint64_t *a, const uint64_t *b, uint64_t *out, size_t n) {
	for (size_t i = 0; i < n; i++) out[i] = orc_f64_maxmin(is_max, a[i], b[i]);
}
void orc_f64_of_f32_n(const uint32_t *x, uint64_t *out, size_t n) {
	for (size_t i = 0; i < n; i++) out[i] = orc_f64_of_f32(x[i]);
}
void orc_f32_of_f64_n(const uint64_t *x, uint32_t *out, size_t n) {
	for (size_t i = 0; i < n; i++) out[i] = orc_f32_of_f64(x[i]);
}

/* ---- fixture writer: the case table of ref/ggml_ref.c:152-295 ------------- */

struct tensor { int64_t ne[4]; float *d; };

static int64_t tcount(const struct tensor *t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }

static struct tensor tnew(int64_t ne0, int64_t ne1, int64_t ne2) {
	struct tensor t = { { ne0, ne1, ne2, 1 }, NULL };
	t.d = (float *)calloc((size_t)tcount(&t), sizeof(float));
	return t;
}

/* input(): a new [ne0, ne1, ne2] tensor filled from the stream (ggml_ref.c:38-43). */
static struct tensor tinput(uint32_t *st, int64_t ne0, int64_t ne1, int64_t ne2, float a) {
	struct tensor t = tnew(ne0, ne1, ne2);
	orc_fill_unif(st, a, t.d, (size_t)tcount(&t));
	return t;
}

struct writer { char dir[1024]; FILE *meta; int nin; int err; };

static void wsave(struct writer *w, const char *name, const struct tensor *t) {
	char p[1200];
	snprintf(p, sizeof p, "%s/%s.f32", w->dir, name);
	FILE *f = fopen(p, "wb");
	if (!f) { w->err = 1; return; }
	if (fwrite(t->d, sizeof(float), (size_t)tcount(t), f) != (size_t)tcount(t)) w->err = 1;
	fclose(f);
	fprintf(w->meta, "%s %lld %lld %lld %lld\n", name, (long long)t->ne[0], (long long)t->ne[1],
	        (long long)t->ne[2], (long long)t->ne[3]);
}

static void win(struct writer *w, const struct tensor *t) {
	char n[16];
	snprintf(n, sizeof n, "in%d", w->nin++);
	wsave(w, n, t);
}

static int wbegin(struct writer *w, const char *outdir, const char *name) {
	snprintf(w->dir, sizeof w->dir, "%s/%s", outdir, name);
	mkdir(outdir, 0755);
	mkdir(w->dir, 0755);
	char p[1200];
	snprintf(p, sizeof p, "%s/meta.txt", w->dir);
	w->meta = fopen(p, "w");
	w->nin = 0;
	w->err = w->meta == NULL;
	return w->err ? -2 : 0;
}

static int wfinish(struct writer *w, struct tensor *out) {
	wsave(w, "out", out);
	fclose(w->meta);
	return w->err ? -2 : 0;
}

enum { OP_MUL_MAT, OP_ADD, OP_MUL, OP_REPEAT, OP_NORM, OP_SCALE, OP_SOFT_MAX, OP_GELU, OP_SILU,
       OP_CONCAT, OP_TRANSPOSE, OP_VIEW };

/* One row per case of ref/ggml_ref.c:244-283 (same names, ops, shapes and
 * amplitudes; the per-op seed is ggml_ref.c:152-239's begin() argument). */
struct ocase { const char *name; int op; int64_t a[5]; float amp0, amp1; };

static const struct ocase CASES[] = {
	{ "mul_mat_small", OP_MUL_MAT, { 37, 5, 3, 1 }, 1.0f, 1.0f },
	{ "mul_mat_k2", OP_MUL_MAT, { 2, 7, 1, 3 }, 1.0f, 1.0f },
	{ "add_small", OP_ADD, { 7, 3, 2 }, 4.0f, 0 },
	{ "mul_small", OP_MUL, { 7, 3, 2 }, 4.0f, 0 },
	{ "repeat_small", OP_REPEAT, { 7, 3, 2 }, 1.0f, 0 },
	{ "norm_small", OP_NORM, { 37, 3, 1 }, 3.0f, 0 },
	{ "scale_small", OP_SCALE, { 13, 4 }, 40.0f, 0 },
	{ "soft_max_small", OP_SOFT_MAX, { 16, 4 }, 30.0f, 0 },
	{ "soft_max_tail", OP_SOFT_MAX, { 13, 4 }, 30.0f, 0 },
	{ "gelu_erf_small", OP_GELU, { 64, 4, 1 }, 6.0f, 0 },
	{ "silu_small", OP_SILU, { 16, 2, 1 }, 12.0f, 0 },
	{ "silu_tail", OP_SILU, { 7, 2, 1 }, 12.0f, 0 },
	{ "concat0_small", OP_CONCAT, { 0, 5, 3, 2, 4 }, 1.0f, 0 },
	{ "concat1_small", OP_CONCAT, { 1, 5, 3, 2, 4 }, 1.0f, 0 },
	{ "concat2_small", OP_CONCAT, { 2, 5, 3, 2, 4 }, 1.0f, 0 },
	{ "transpose_small", OP_TRANSPOSE, { 5, 3 }, 1.0f, 0 },
	{ "view_small", OP_VIEW, { 24, 3, 4, 8 }, 1.0f, 0 },
	{ "mul_mat_qkv", OP_MUL_MAT, { 1024, 3072, 352, 3 }, 0.05f, 2.0f },
	{ "mul_mat_ffn2", OP_MUL_MAT, { 2048, 1024, 352, 3 }, 0.05f, 2.0f },
	{ "mul_mat_text", OP_MUL_MAT, { 4096, 1024, 50, 3 }, 0.05f, 2.0f },
	{ "mul_mat_heading", OP_MUL_MAT, { 2, 1024, 1, 3 }, 0.5f, 1.0f },
	{ "mul_mat_root_in", OP_MUL_MAT, { 738, 1024, 300, 3 }, 0.05f, 2.0f },
	{ "mul_mat_body_in", OP_MUL_MAT, { 737, 1024, 300, 3 }, 0.05f, 2.0f },
	{ "mul_mat_scores", OP_MUL_MAT, { 128, 352, 352, 1 }, 2.0f, 2.0f },
	{ "mul_mat_value", OP_MUL_MAT, { 352, 128, 352, 1 }, 0.01f, 2.0f },
	{ "add_kimodo", OP_ADD, { 3072, 352, 3 }, 4.0f, 0 },
	{ "mul_kimodo", OP_MUL, { 1024, 352, 3 }, 4.0f, 0 },
	{ "repeat_kimodo", OP_REPEAT, { 1024, 352, 3 }, 1.0f, 0 },
	{ "norm_kimodo", OP_NORM, { 1024, 352, 3 }, 3.0f, 0 },
	{ "scale_kimodo", OP_SCALE, { 352, 352 }, 40.0f, 0 },
	{ "soft_max_kimodo", OP_SOFT_MAX, { 352, 352 }, 30.0f, 0 },
	{ "gelu_erf_kimodo", OP_GELU, { 2048, 352, 3 }, 6.0f, 0 },
	{ "silu_kimodo", OP_SILU, { 1024, 1, 3 }, 12.0f, 0 },
	{ "concat0_kimodo", OP_CONCAT, { 0, 896, 352, 1, 128 }, 1.0f, 0 },
	{ "concat1_kimodo", OP_CONCAT, { 1, 1024, 52, 3, 300 }, 1.0f, 0 },
	{ "concat2_kimodo", OP_CONCAT, { 2, 1024, 352, 2, 1 }, 1.0f, 0 },
	{ "transpose_kimodo", OP_TRANSPOSE, { 128, 352 }, 1.0f, 0 },
	{ "view_kimodo", OP_VIEW, { 3072, 352, 128, 1024 + 3 * 128 }, 1.0f, 0 },
};

/* ---- graph.txt: ggml's graph of a case, "ghlo-graph 1" (ggml_ref.c:94-134) --
 * One line per tensor: the arguments (tensors the nodes read that are not
 * nodes themselves, in the order the nodes first read them, a view's source
 * after its srcs), then the nodes in graph order:
 *   T <i> <op> <unary op or -> <node> <output> <type> <ne0..3> <nb0..3>
 *     <view source index or -1> <view offset> <src0..9 index or -1> <op_params 0..15>
 * <op> is ggml_op_name(); a node is an output when no later tensor reads it.
 * The op_params are ggml's for the ops of these cases: NORM {eps},
 * SCALE {s, bias 0}, SOFT_MAX {scale 1, max_bias 0}, UNARY {unary op},
 * CONCAT {dim}, VIEW {byte offset as a size_t}. */
struct gtensor {
	const char *op, *un;
	int node;
	int64_t ne[4];
	int64_t nb[4];
	int view_src;
	int64_t view_offs;
	int src[10];
	int32_t par[16];
};
struct graph { struct gtensor t[8]; int n; };

/* ggml_unary_op values at the reference's ggml (GGML_UNARY_OP_SILU, _GELU_ERF); pinned by
 * the graph.txt hashes of the silu and gelu_erf cases. */
enum { GGML_UNARY_SILU = 10, GGML_UNARY_GELU_ERF = 16 };

static int gadd(struct graph *g, const char *op, const char *un, int node, int64_t ne0, int64_t ne1, int64_t ne2,
                int64_t ne3) {
	struct gtensor *t = &g->t[g->n];
	memset(t, 0, sizeof *t);
	t->op = op;
	t->un = un;
	t->node = node;
	t->ne[0] = ne0; t->ne[1] = ne1; t->ne[2] = ne2; t->ne[3] = ne3;
	t->nb[0] = 4;
	for (int i = 1; i < 4; i++) t->nb[i] = t->nb[i - 1] * t->ne[i - 1];
	t->view_src = -1;
	for (int i = 0; i < 10; i++) t->src[i] = -1;
	return g->n++;
}

static int32_t fbits(float f) { int32_t b; memcpy(&b, &f, 4); return b; }

static void build_graph(const struct ocase *c, struct graph *g) {
	const int64_t *a = c->a;
	g->n = 0;
	int x, y, n;
	switch (c->op) {
	case OP_MUL_MAT:
		x = gadd(g, "NONE", "-", 0, a[0], a[1], 1, 1);
		y = gadd(g, "NONE", "-", 0, a[0], a[2], a[3], 1);
		n = gadd(g, "MUL_MAT", "-", 1, a[1], a[2], a[3], 1);
		g->t[n].src[0] = x; g->t[n].src[1] = y;
		break;
	case OP_ADD:
	case OP_MUL:
		x = gadd(g, "NONE", "-", 0, a[0], a[1], a[2], 1);
		y = gadd(g, "NONE", "-", 0, a[0], a[1], a[2], 1);
		n = gadd(g, c->op == OP_ADD ? "ADD" : "MUL", "-", 1, a[0], a[1], a[2], 1);
		g->t[n].src[0] = x; g->t[n].src[1] = y;
		break;
	case OP_REPEAT:
		x = gadd(g, "NONE", "-", 0, a[0], 1, 1, 1);
		n = gadd(g, "REPEAT", "-", 1, a[0], a[1], a[2], 1);
		g->t[n].src[0] = x;
		break;
	case OP_NORM:
		x = gadd(g, "NONE", "-", 0, a[0], a[1], a[2], 1);
		n = gadd(g, "NORM", "-", 1, a[0], a[1], a[2], 1);
		g->t[n].src[0] = x; g->t[n].par[0] = fbits(1.e-5f);
		break;
	case OP_SCALE:
		x = gadd(g, "NONE", "-", 0, a[0], a[1], 1, 1);
		n = gadd(g, "SCALE", "-", 1, a[0], a[1], 1, 1);
		g->t[n].src[0] = x; g->t[n].par[0] = fbits(1.f / sqrtf(128.0f));
		break;
	case OP_SOFT_MAX:
		x = gadd(g, "NONE", "-", 0, a[0], a[1], 1, 1);
		n = gadd(g, "SOFT_MAX", "-", 1, a[0], a[1], 1, 1);
		g->t[n].src[0] = x; g->t[n].par[0] = fbits(1.0f);
		break;
	case OP_GELU:
	case OP_SILU:
		x = gadd(g, "NONE", "-", 0, a[0], a[1], a[2], 1);
		n = gadd(g, "UNARY", c->op == OP_GELU ? "GELU_ERF" : "SILU", 1, a[0], a[1], a[2], 1);
		g->t[n].src[0] = x; g->t[n].par[0] = c->op == OP_GELU ? GGML_UNARY_GELU_ERF : GGML_UNARY_SILU;
		break;
	case OP_CONCAT: {
		const int dim = (int)a[0];
		int64_t bn[3] = { a[1], a[2], a[3] }, on[3] = { a[1], a[2], a[3] };
		bn[dim] = a[4];
		on[dim] += a[4];
		x = gadd(g, "NONE", "-", 0, a[1], a[2], a[3], 1);
		y = gadd(g, "NONE", "-", 0, bn[0], bn[1], bn[2], 1);
		n = gadd(g, "CONCAT", "-", 1, on[0], on[1], on[2], 1);
		g->t[n].src[0] = x; g->t[n].src[1] = y; g->t[n].par[0] = dim;
		break;
	}
	case OP_TRANSPOSE: {  /* cont(transpose(x)): the transpose is a view of x with ne and nb swapped */
		x = gadd(g, "NONE", "-", 0, a[0], a[1], 1, 1);
		const int v = gadd(g, "TRANSPOSE", "-", 1, a[1], a[0], 1, 1);
		struct gtensor *t = &g->t[v];
		t->nb[0] = g->t[x].nb[1]; t->nb[1] = g->t[x].nb[0]; t->nb[2] = g->t[x].nb[2]; t->nb[3] = g->t[x].nb[3];
		t->view_src = x; t->src[0] = x;
		n = gadd(g, "CONT", "-", 1, a[1], a[0], 1, 1);
		g->t[n].src[0] = v;
		break;
	}
	case OP_VIEW: {  /* cont(view_2d(x, hw, seq, x->nb[1], off * 4)) */
		const int64_t W = a[0], S = a[1], HW = a[2], off = a[3] * 4;
		x = gadd(g, "NONE", "-", 0, W, S, 1, 1);
		const int v = gadd(g, "VIEW", "-", 1, HW, S, 1, 1);
		struct gtensor *t = &g->t[v];
		t->nb[1] = g->t[x].nb[1]; t->nb[2] = t->nb[1] * S; t->nb[3] = t->nb[2];
		t->view_src = x; t->view_offs = off; t->src[0] = x;
		t->par[0] = (int32_t)(uint32_t)(uint64_t)off; t->par[1] = (int32_t)(uint32_t)((uint64_t)off >> 32);
		n = gadd(g, "CONT", "-", 1, HW, S, 1, 1);
		g->t[n].src[0] = v;
		break;
	}
	}
}

static int wgraph(struct writer *w, const struct ocase *c) {
	struct graph g;
	build_graph(c, &g);
	char p[1200];
	snprintf(p, sizeof p, "%s/graph.txt", w->dir);
	FILE *f = fopen(p, "w");
	if (!f) return -2;
	fprintf(f, "ghlo-graph 1\n");
	for (int i = 0; i < g.n; i++) {
		const struct gtensor *t = &g.t[i];
		int output = 0;
		if (t->node) {
			int used = 0;
			for (int j = i + 1; j < g.n; j++)
				for (int s = 0; s < 10; s++) used |= g.t[j].src[s] == i || g.t[j].view_src == i;
			output = !used;
		}
		fprintf(f, "T %d %s %s %d %d f32 %lld %lld %lld %lld %lld %lld %lld %lld %d %lld", i, t->op, t->un, t->node,
		        output, (long long)t->ne[0], (long long)t->ne[1], (long long)t->ne[2], (long long)t->ne[3],
		        (long long)t->nb[0], (long long)t->nb[1], (long long)t->nb[2], (long long)t->nb[3], t->view_src,
		        (long long)t->view_offs);
		for (int s = 0; s < 10; s++) fprintf(f, " %d", t->src[s]);
		for (int q = 0; q < 16; q++) fprintf(f, " %d", t->par[q]);
		fprintf(f, "\n");
	}
	return fclose(f) ? -2 : 0;
}

int orc_case_count(void) { return (int)(sizeof CASES / sizeof CASES[0]); }
const char *orc_case_name(int i) { return i >= 0 && i < orc_case_count() ? CASES[i].name : NULL; }

static const uint32_t SEED[] = { 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12 };

int orc_write_case(const char *outdir, const char *name, int pinned) {
	const struct ocase *c = NULL;
	for (int i = 0; i < orc_case_count(); i++)
		if (strcmp(CASES[i].name, name) == 0) c = &CASES[i];
	if (!c) return -1;
	struct writer w;
	if (wbegin(&w, outdir, name)) return -2;
	uint32_t st = SEED[c->op];
	const int64_t *a = c->a;
	struct tensor out = { { 0 }, NULL };
	struct tensor t0 = { { 0 }, NULL }, t1 = { { 0 }, NULL };
	switch (c->op) {
	case OP_MUL_MAT: {  /* mul_mat(n, k, m, r, b, aw, ax), ggml_ref.c:152-157 */
		const int64_t K = a[0], M = a[1], R = a[2], B = a[3];
		t0 = tinput(&st, K, M, 1, c->amp0);
		t1 = tinput(&st, K, R, B, c->amp1);
		win(&w, &t0);
		win(&w, &t1);
		out = tnew(M, R, B);
		orc_mul_mat(t0.d, t1.d, out.d, K, M, R * B, R, 0, pinned ? ORC_TAIL_PINNED : ORC_TAIL_STOCK, 8);
		break;
	}
	case OP_ADD:
	case OP_MUL: {
		t0 = tinput(&st, a[0], a[1], a[2], c->amp0);
		t1 = tinput(&st, a[0], a[1], a[2], c->amp0);
		win(&w, &t0);
		win(&w, &t1);
		out = tnew(a[0], a[1], a[2]);
		for (int64_t i = 0; i < tcount(&out); i++)
			out.d[i] = c->op == OP_ADD ? t0.d[i] + t1.d[i] : t0.d[i] * t1.d[i];
		break;
	}
	case OP_REPEAT: {
		t0 = tinput(&st, a[0], 1, 1, c->amp0);
		win(&w, &t0);
		out = tnew(a[0], a[1], a[2]);
		for (int64_t i = 0; i < tcount(&out); i++) out.d[i] = t0.d[i % a[0]];
		break;
	}
	case OP_NORM: {
		t0 = tinput(&st, a[0], a[1], a[2], c->amp0);
		win(&w, &t0);
		out = tnew(a[0], a[1], a[2]);
		orc_norm(t0.d, out.d, a[1] * a[2], a[0], 1.e-5f, 0, 8);
		break;
	}
	case OP_SCALE: {
		t0 = tinput(&st, a[0], a[1], 1, c->amp0);
		win(&w, &t0);
		out = tnew(a[0], a[1], 1);
		const float s = 1.f / sqrtf(128.0f);
		for (int64_t i = 0; i < tcount(&out); i++) out.d[i] = t0.d[i] * s;
		break;
	}
	case OP_SOFT_MAX: {
		t0 = tinput(&st, a[0], a[1], 1, c->amp0);
		win(&w, &t0);
		out = tnew(a[0], a[1], 1);
		orc_soft_max(t0.d, out.d, a[1], a[0], 1.0f, 0, 8);
		break;
	}
	case OP_GELU: {
		t0 = tinput(&st, a[0], a[1], a[2], c->amp0);
		win(&w, &t0);
		out = tnew(a[0], a[1], a[2]);
		orc_gelu_erf(t0.d, out.d, (size_t)tcount(&out), 0, 8);
		break;
	}
	case OP_SILU: {
		t0 = tinput(&st, a[0], a[1], a[2], c->amp0);
		win(&w, &t0);
		out = tnew(a[0], a[1], a[2]);
		orc_silu(t0.d, out.d, a[1] * a[2], a[0]);
		break;
	}
	case OP_CONCAT: {  /* concat_c(n, dim, a0, a1, a2, b), ggml_ref.c:217-224 */
		const int dim = (int)a[0];
		int64_t bn[3] = { a[1], a[2], a[3] };
		bn[dim] = a[4];
		t0 = tinput(&st, a[1], a[2], a[3], c->amp0);
		t1 = tinput(&st, bn[0], bn[1], bn[2], c->amp0);
		win(&w, &t0);
		win(&w, &t1);
		int64_t on[3] = { a[1], a[2], a[3] };
		on[dim] += bn[dim];
		out = tnew(on[0], on[1], on[2]);
		for (int64_t i2 = 0; i2 < on[2]; i2++)
			for (int64_t i1 = 0; i1 < on[1]; i1++)
				for (int64_t i0 = 0; i0 < on[0]; i0++) {
					int64_t ix[3] = { i0, i1, i2 };
					const int64_t o = i0 + on[0] * (i1 + on[1] * i2);
					if (ix[dim] < t0.ne[dim]) {
						out.d[o] = t0.d[ix[0] + t0.ne[0] * (ix[1] + t0.ne[1] * ix[2])];
					} else {
						ix[dim] -= t0.ne[dim];
						out.d[o] = t1.d[ix[0] + t1.ne[0] * (ix[1] + t1.ne[1] * ix[2])];
					}
				}
		break;
	}
	case OP_TRANSPOSE: {  /* cont(transpose(x)), ggml_ref.c:226-231 */
		t0 = tinput(&st, a[0], a[1], 1, c->amp0);
		win(&w, &t0);
		out = tnew(a[1], a[0], 1);
		for (int64_t i1 = 0; i1 < a[0]; i1++)
			for (int64_t i0 = 0; i0 < a[1]; i0++) out.d[i0 + a[1] * i1] = t0.d[i1 + a[0] * i0];
		break;
	}
	case OP_VIEW: {  /* cont(view_2d(x, hw, seq, nb1, off)), ggml_ref.c:234-239 */
		const int64_t W = a[0], S = a[1], HW = a[2], OFF = a[3];
		t0 = tinput(&st, W, S, 1, c->amp0);
		win(&w, &t0);
		out = tnew(HW, S, 1);
		for (int64_t s = 0; s < S; s++)
			for (int64_t i = 0; i < HW; i++) out.d[i + HW * s] = t0.d[OFF + i + W * s];
		break;
	}
	}
	int rc = wfinish(&w, &out);
	if (rc == 0) rc = wgraph(&w, c);
	free(t0.d);
	free(t1.d);
	free(out.d);
	return rc;
}
