// The exact kernels: ggml-cpu's arm64 routines restated for gfx950 wave64 in
// ggml's accumulation order, so every output has the same bits as ggml-cpu
// (StablehloMlx/Kernels/Shaders.lean:55-208 restates the same routines for
// Metal).  No atomics: every output has one writer and a fixed order, so
// eager and graph-replayed runs give identical bits.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "epilogue.h"
#include "erff_cr.h"
#include "expf_cr.h"
#include "ggml_expf.h"
#include "ops.h"

namespace shlo {

namespace {

constexpr int kWave = 64;

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }

// Orders one wave's LDS writes before its later LDS reads by other lanes.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
__device__ __forceinline__ void st4(float *p, float4 v) { *reinterpret_cast<float4 *>(p) = v; }

// Streaming loads and stores for operands touched once: they bypass cache
// allocation (the `nt` bit).
__device__ __forceinline__ float4 ld4_nt(const float *p) {
  float4 v;
  v.x = __builtin_nontemporal_load(p);
  v.y = __builtin_nontemporal_load(p + 1);
  v.z = __builtin_nontemporal_load(p + 2);
  v.w = __builtin_nontemporal_load(p + 3);
  return v;
}
__device__ __forceinline__ void st4_nt(float *p, float4 v) {
  __builtin_nontemporal_store(v.x, p);
  __builtin_nontemporal_store(v.y, p + 1);
  __builtin_nontemporal_store(v.z, p + 2);
  __builtin_nontemporal_store(v.w, p + 3);
}


// ---- gelu_erf's per-element routine (also a fused epilogue op of dot_general) ----------

constexpr int kPolyWords = erffk::kTab * 6;

// Stages the coefficient table in LDS (16-byte loads; the table is read from
// L2 after the first blocks).
__device__ __forceinline__ void load_poly(double *tab) {
  const double2 *src = reinterpret_cast<const double2 *>(&erffk::kPoly[0][0]);
  for (int i = threadIdx.x; i < kPolyWords / 2; i += blockDim.x) reinterpret_cast<double2 *>(tab)[i] = src[i];
  __syncthreads();
}

template <int TANH>
__device__ __forceinline__ float gelu1(float x, const double *tab) {
  float ev;
  if (TANH)  // planted: the tanh form of GELU (Shaders.lean:192-194)
    ev = tanhf(bits_f(0x3F4C422Au) * x * (1.0f + bits_f(0x3D372713u) * x * x));
  else
    ev = erffk::erff_cr(x * bits_f(0x3F3504F3u), tab);  // SQRT_2_INV
  float y = (0.5f * x) * (1.0f + ev);
  // A NaN input gives the input quieted, payload kept (Shaders.lean:196-199).
  if ((f_bits(x) & 0x7FFFFFFFu) > 0x7F800000u) y = bits_f(f_bits(x) | 0x00400000u);
  return y;
}

// NV elements at once, the same results as gelu1 element by element.
//
// 64 |x*SQRT_2_INV| is taken as one product |x| * (64*SQRT_2_INV) (the
// scaling is exact), clamped to 255: the same value wherever x*SQRT_2_INV is
// a normal binary32, and where it is subnormal (|x| < 1.7e-38) erf of it is
// below 2^-125, so 1 + ev rounds to 1 either way.  The NV erf evaluations
// share one (rarely taken) branch into the exception table, keyed by
// |x*SQRT_2_INV|.  NaN inputs need no select: the clamp maps them to erf = 1,
// ev = +-1, and (0.5f*x)*(1 + ev) multiplies the quieted x, payload kept, by
// 2 or 0, which returns it.
// row(i): the erff table's row i (erffk::erf_R64_at).
template <int NV, class Row>
__device__ __forceinline__ void gelu_erf_n_at(float (&x)[NV], Row row) {
  uint32_t r[NV], d[NV];
#pragma unroll
  for (int k = 0; k < NV; k++) {
    const float a64 = __builtin_fminf(__builtin_fabsf(x[k]) * bits_f(0x423504F3u), 255.0f);  // 64*SQRT_2_INV
    const double R = erffk::erf_R64_at(a64, row);
    r[k] = f_bits((float)R);
    d[k] = erffk::undecided_distance(R);
  }
  uint32_t dmin = d[0];
#pragma unroll
  for (int k = 1; k < NV; k++) dmin = dmin < d[k] ? dmin : d[k];
  if (dmin < 0x40u) {
#pragma unroll
    for (int k = 0; k < NV; k++)
      if (d[k] < 0x40u) r[k] = erffk::exception_lookup(f_bits(x[k] * bits_f(0x3F3504F3u)) & 0x7FFFFFFFu, r[k]);
  }
#pragma unroll
  for (int k = 0; k < NV; k++) {
    const float ev = bits_f(r[k] | (f_bits(x[k]) & 0x80000000u));
    x[k] = (0.5f * x[k]) * (1.0f + ev);
  }
}
template <int NV>
__device__ __forceinline__ void gelu_erf_n(float (&x)[NV], const double *tab) {
  gelu_erf_n_at(x, [tab](unsigned i) { return tab + 6 * i; });
}

// ggml.gelu_erf as a fused op of the dot kernels' epilogues: one output
// through gelu1, all of a lane's outputs at once through gelu_erf_n
// (epilogue.h's unary_all, found by argument-dependent lookup).
struct GeluErfOp {
  const double *tab;
  __device__ float operator()(float x) const { return gelu1<0>(x, tab); }
};
template <int NV>
__device__ __forceinline__ void unary_all(const GeluErfOp &g, float (&v)[NV]) {
  gelu_erf_n(v, g.tab);
}

// The same with the table held in two pieces of LDS: rows 0 .. 127 at lo,
// 128 .. 255 at hi (the four-wave matrix kernel stages it in its two free
// lhs stage buffers for the epilogue).
constexpr int kPolyHalfRows = erffk::kTab / 2;
struct GeluErfSplitOp {
  const double *lo, *hi;
  __device__ const double *row(unsigned i) const {
    return i < (unsigned)kPolyHalfRows ? lo + 6 * i : hi + 6 * (i - kPolyHalfRows);
  }
  __device__ float operator()(float x) const {
    float v[1] = {x};
    gelu_erf_n_at(v, [this](unsigned i) { return row(i); });
    return v[0];
  }
};
template <int NV>
__device__ __forceinline__ void unary_all(const GeluErfSplitOp &g, float (&v)[NV]) {
  gelu_erf_n_at(v, [&g](unsigned i) { return g.row(i); });
}

// ---- dot_general in ggml_vec_dot_f32 order --------------------------------------

// The tail and the final combination shared by every dot kernel: `a` holds the
// 16 block accumulators; returns the finished output.
template <int TAIL>
__device__ __forceinline__ float dot_finish(float a[16], const float *w, int64_t wk, const float *x, int64_t xk,
                                            int64_t np, int64_t K) {
  // GGML_F32x4_REDUCE (sum[0]+=sum[2], sum[1]+=sum[3], sum[0]+=sum[1]) and
  // vaddvq_f32 = (v0+v1)+(v2+v3), Shaders.lean:75-79.
#pragma unroll
  for (int l = 0; l < 4; l++) a[l] = a[l] + a[8 + l];
#pragma unroll
  for (int l = 0; l < 4; l++) a[4 + l] = a[4 + l] + a[12 + l];
#pragma unroll
  for (int l = 0; l < 4; l++) a[l] = a[l] + a[4 + l];
  float s = (a[0] + a[1]) + (a[2] + a[3]);
  if (TAIL == kTailPinned) {
    for (int64_t i = np; i < K; i++) {
      const float p = w[i * wk] * x[i * xk];
      s = s + p;
    }
  } else {
    // stock: Shaders.lean:80-90
    const int64_t tl = K - np;
    const int64_t nq = tl >= 4 ? (tl & ~(int64_t)3) : 0;
    for (int64_t i = np; i < np + nq; i++) {
      const float p = w[i * wk] * x[i * xk];
      s = s + p;
    }
    for (int64_t i = np + nq; i < K; i++) s = __builtin_fmaf(w[i * wk], x[i * xk], s);
  }
  return s;
}

// One operand of a dot kernel: element (b, f, k) at p + boff(b) + f*sf + k*sk,
// where batch b = b1 * nb2 + b2 sits at b1*sb + b2*sb2 (two batch levels, so
// per-head views of a [tokens, heads*dh] buffer need no copy; nb2 = 1 for one).
struct MfmaOperand {
  const float *p;
  int64_t sb, sf, sk;
  int64_t rows;  // N or M
  int64_t sb2, nb2;
};

__host__ __device__ __forceinline__ int64_t boff(const MfmaOperand &o, int64_t b) {  // b < 2^31 (the host checks)
  if (o.nb2 == 1) return b * o.sb;
  const uint32_t q = (uint32_t)b / (uint32_t)o.nb2, r = (uint32_t)b - q * (uint32_t)o.nb2;
  return (int64_t)q * o.sb + (int64_t)r * o.sb2;
}

// One thread per output; any strides.  The reference kernel's mapping
// (one thread per output, Shaders.lean:60-64), used for small and irregular
// shapes and as the parity baseline.
template <int TAIL>
__global__ void __launch_bounds__(256) dot_ggml_simple(int64_t n_out, int64_t N, int64_t M, int64_t K,
                                                       MfmaOperand X, MfmaOperand W, Epilogue ep,
                                                       float *__restrict__ y) {
  __shared__ double gtab[kPolyWords];  // a fused gelu_erf's table
  if (ep.gelu) load_poly(gtab);
  const GeluErfOp gelu{gtab};
  const int64_t lk = X.sk, rk = W.sk;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n_out; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = i % M, t = i / M, n = t % N, b = t / N;
    const float *x = X.p + boff(X, b) + n * X.sf;
    const float *w = W.p + boff(W, b) + m * W.sf;
    if (TAIL == kTailPlain) {  // planted: sequential binary32 sum, no FMA (Shaders.lean:65-68)
      float s = 0.0f;
      for (int64_t k = 0; k < K; k++) {
        const float p = w[k * rk] * x[k * lk];
        s = s + p;
      }
      y[i] = epi_apply(ep, s, b, n, m, gelu);
      continue;
    }
    float a[16];
#pragma unroll
    for (int j = 0; j < 16; j++) a[j] = 0.0f;
    const int64_t np = K & ~(int64_t)15;
    for (int64_t k0 = 0; k0 < np; k0 += 16) {
#pragma unroll
      for (int j = 0; j < 16; j++) a[j] = __builtin_fmaf(w[(k0 + j) * rk], x[(k0 + j) * lk], a[j]);
    }
    y[i] = epi_apply(ep, dot_finish<TAIL>(a, w, rk, x, lk, np, K), b, n, m, gelu);
  }
}

// ---- dot_general on the matrix cores ------------------------------------------------
//
// ggml_vec_dot_f32 keeps 16 accumulators per output, accumulator j taking
// fma(w[16b+j], x[16b+j], acc_j) over the blocks b in order.  Each chain is
// an ordinary GEMM over the k = j (mod 16) slice, so it maps onto
// v_mfma_f32_32x32x1_2b_f32: per instruction every output of two 32x32 blocks
// gets exactly one fused multiply-add, acc = fma(a_i, b_j, acc), with one
// rounding (checked bit for bit against fmaf, subnormals included).  Block 0
// of an instruction carries one residue and block 1 the residue 8 above it, so
// the 16 chains of a 32x32 output tile take 8 accumulator sets (256 registers).
// After the last block the fixed GGML_F32x4_REDUCE / vaddvq_f32 tree and the
// serial tail run per output, exactly as in dot_finish.
//
// Workgroup: 8 waves (two per SIMD) on a 64 (n) x 64 (m) output tile, the two
// waves of each 32x32 quadrant holding half of its chains each; operands staged
// in LDS as [row][k] (row stride KC + 4 floats), KC = 128 (eight k-blocks) per
// stage, double-buffered (135 KB of gfx950's 160 KB), the next stage loaded
// into registers while the matrix cores work on the current one.

typedef float v32f __attribute__((ext_vector_type(32)));

constexpr int kMT = 64;        // tile rows (n) and columns (m)
constexpr int kKC = 128;       // k per stage (8 blocks of 16)
constexpr int kLS = kKC + 4;   // LDS row stride (floats): rows start 4 banks apart
constexpr int kDotStageFloats = 2 * 2 * kMT * kLS;  // two buffers of both operands; a fused gelu_erf's table follows
// float4 per thread per operand per stage for a workgroup of TH threads.
template <int TH>
constexpr int regs_of() {
  return kMT * kKC / 4 / TH;
}
static_assert(regs_of<512>() % 4 == 0 && kMT == 64 && kKC == 128,
              "the loaders' thread mappings assume these");

// How an operand tile is loaded: kLoadRowVec = rows contiguous in k (sk == 1),
// float4 along k; kLoadColVec = free dim contiguous (sf == 1), four scalar
// loads per thread (four consecutive k of one row, each load coalesced across
// the wave along the free dim); kLoadColQuad = the same operand 16-byte
// aligned with rows % 4 == 0: each thread loads 4x4 (k x row) sub-blocks as
// four 16-byte loads along the free dim and transposes them in registers;
// kLoadScalar = any strides.  Every thread then writes 16-byte [row][k]
// chunks to LDS.  kLoadRowVecB and kLoadColQuadB read the same elements as
// kLoadRowVec and kLoadColQuad through buffer loads: one per-lane byte offset
// fixed for the whole kernel, and every per-load and per-stage advance in the
// scalar offset, so a stage's loads cost no vector ALU work and no branches.
// They are chosen only when every read is in range by construction (rows a
// multiple of 64, every stage full, offsets below 2^31).
enum { kLoadRowVec = 0, kLoadColVec = 1, kLoadScalar = 2, kLoadColQuad = 3, kLoadRowVecB = 4, kLoadColQuadB = 5 };

// The LDS layout a loader's stash writes: the buffer loaders share their
// plain counterparts'.
constexpr int stash_kind(int load) {
  return load == kLoadRowVecB ? kLoadRowVec : load == kLoadColQuadB ? kLoadColQuad : load;
}

// A buffer loader's per-workgroup state: the batch's buffer resource and the
// lane's byte offset within it.
struct BufOp {
  __amdgpu_buffer_rsrc_t r;
  int voff;
  const float *base;  // the batch's first element (every loader)
};

template <int LOAD>
__device__ __forceinline__ BufOp buf_op(const MfmaOperand &o, int64_t b, int64_t r0) {  // any TH <= 512
  BufOp bo;
  const int t = threadIdx.x;
  bo.base = o.p + boff(o, b);
  bo.r = __builtin_amdgcn_make_buffer_rsrc((void *)bo.base, (short)0, 0x7FFFFFFF, 0x00020000);
  if (LOAD == kLoadRowVecB) {  // row t / 32, k quad t % 32 (as kLoadRowVec's load 0)
    bo.voff = (int)(((r0 + t / 32) * o.sf + (t % 32) * 4) * 4);
  } else if (LOAD == kLoadColQuadB) {  // row quad (t % 64) / 4, k 4 (t % 4) + 16 (t / 64) (as kLoadColQuad's group 0)
    bo.voff = (int)((r0 + 4 * ((t % 64) / 4) + (4 * (t % 4) + 16 * (t / 64)) * o.sk) * 4);
  } else {
    bo.voff = 0;
  }
  return bo;
}

__device__ __forceinline__ float4 buf_ld4(const BufOp &bo, int soff) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  const f4 v = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(bo.r, bo.voff, soff, 0));
  return make_float4(v.x, v.y, v.z, v.w);
}

// Stage s of one operand into registers: kMT * kKC floats per tile.
// kLoadColQuad: sub-block u = t + TH * (i / 4) of the tile's 16 x 32
// (row quads x k quads); lane l of wave chunk c takes row quad l / 4 and k quad
// l % 4 + 4 c, so the 16 lanes an LDS write serves together hit 16 distinct
// bank quads, and each load reads four 256-byte runs along the free dim.
// reg[4 (i / 4) + mm] ends up holding k quad kq of row 4 rq + mm.
__device__ __forceinline__ void colquad_coords(int u, int &rq, int &kq) {
  const int l = u % 64, c = u / 64;
  rq = l / 4;
  kq = l % 4 + 4 * c;
}

// Registers [I0, I1) of stage s for a workgroup of TH threads (all of it by
// default; the 4x4 loaders in whole groups of 4).
template <int LOAD, int TH, int I0 = 0, int I1 = regs_of<TH>()>
__device__ __forceinline__ void mfma_fetch(const MfmaOperand &o, const BufOp &bo, int64_t r0, int s, int nb,
                                           float4 (&reg)[regs_of<TH>()]) {
  static_assert((LOAD != kLoadColQuad && LOAD != kLoadColQuadB) || (I0 % 4 == 0 && I1 % 4 == 0), "whole groups");
  const int t = threadIdx.x;
  if (LOAD == kLoadRowVecB) {  // load i: rows TH / 32 * i further, stage s: k 128 s further
#pragma unroll
    for (int i = I0; i < I1; i++) reg[i] = buf_ld4(bo, (int)(((TH / 32) * i * o.sf + s * kKC) * 4));
    return;
  }
  if (LOAD == kLoadColQuadB) {  // group g: k TH / 4 * g further, load mm: k mm further
#pragma unroll
    for (int g = I0 / 4; g < I1 / 4; g++) {
      float4 v[4];
#pragma unroll
      for (int mm = 0; mm < 4; mm++) v[mm] = buf_ld4(bo, (int)((s * kKC + (TH / 4) * g + mm) * o.sk * 4));
      reg[4 * g + 0] = make_float4(v[0].x, v[1].x, v[2].x, v[3].x);
      reg[4 * g + 1] = make_float4(v[0].y, v[1].y, v[2].y, v[3].y);
      reg[4 * g + 2] = make_float4(v[0].z, v[1].z, v[2].z, v[3].z);
      reg[4 * g + 3] = make_float4(v[0].w, v[1].w, v[2].w, v[3].w);
    }
    return;
  }
  if (LOAD == kLoadColQuad) {
#pragma unroll
    for (int g = I0 / 4; g < I1 / 4; g++) {
      int rq, kq;
      colquad_coords(t + TH * g, rq, kq);
      const int k = s * kKC + 4 * kq;
      int64_t row = r0 + 4 * rq;
      if (row > o.rows - 4) row = o.rows - 4;  // stays in bounds (rows % 4 == 0); discarded outputs
      if (k / 16 < nb) {
        const float *q = bo.base + row + (int64_t)k * o.sk;
        const float4 v0 = ld4(q), v1 = ld4(q + o.sk), v2 = ld4(q + 2 * o.sk), v3 = ld4(q + 3 * o.sk);
        reg[4 * g + 0] = make_float4(v0.x, v1.x, v2.x, v3.x);
        reg[4 * g + 1] = make_float4(v0.y, v1.y, v2.y, v3.y);
        reg[4 * g + 2] = make_float4(v0.z, v1.z, v2.z, v3.z);
        reg[4 * g + 3] = make_float4(v0.w, v1.w, v2.w, v3.w);
      }
    }
    return;
  }
#pragma unroll
  for (int i = I0; i < I1; i++) {
    const int f = t + TH * i;
    if (LOAD == kLoadColVec) {
      // Lane-consecutive rows (the contiguous free dim, so each of the four
      // loads is coalesced across the wave), four consecutive k per thread:
      // the thread then writes one 16-byte [row][k] chunk to LDS.
      const int row_l = f % kMT, kq = (f / kMT) * 4;
      const int k = s * kKC + kq;
      int64_t row = r0 + row_l;
      if (row > o.rows - 1) row = o.rows - 1;  // stays in bounds; those outputs are discarded
      if (k / 16 < nb) {
        const float *q = bo.base + row + (int64_t)k * o.sk;
        reg[i] = make_float4(q[0], q[o.sk], q[2 * o.sk], q[3 * o.sk]);
      }
    } else {
      const int row_l = f / (kKC / 4), kq = (f % (kKC / 4)) * 4;
      const int k = s * kKC + kq;
      int64_t row = r0 + row_l;
      if (row > o.rows - 1) row = o.rows - 1;
      if (k / 16 < nb) {
        const float *q = bo.base + row * o.sf;
        if (LOAD == kLoadRowVec) {
          reg[i] = ld4(q + k);
        } else {
          reg[i] = make_float4(q[(int64_t)k * o.sk], q[(int64_t)(k + 1) * o.sk], q[(int64_t)(k + 2) * o.sk],
                               q[(int64_t)(k + 3) * o.sk]);
        }
      }
    }
  }
}

// Registers [I0, I1) of a stage (all of it by default) into LDS.
template <int LOAD_, int TH, int I0 = 0, int I1 = regs_of<TH>()>
__device__ __forceinline__ void mfma_stash(float *lds, const float4 (&reg)[regs_of<TH>()]) {
  constexpr int LOAD = stash_kind(LOAD_);
  const int t = threadIdx.x;
#pragma unroll
  for (int i = I0; i < I1; i++) {
    if (LOAD == kLoadColQuad) {
      int rq, kq;
      colquad_coords(t + TH * (i / 4), rq, kq);
      st4(lds + (4 * rq + i % 4) * kLS + 4 * kq, reg[i]);
    } else if (LOAD == kLoadColVec) {
      const int f = t + TH * i;
      const int row_l = f % kMT, kq = (f / kMT) * 4;
      st4(lds + row_l * kLS + kq, reg[i]);  // rows 132 floats apart: 16 lanes, 16 distinct bank quads
    } else {
      const int f = t + TH * i;
      const int row_l = f / (kKC / 4), kq = (f % (kKC / 4)) * 4;
      st4(lds + row_l * kLS + kq, reg[i]);
    }
  }
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef const volatile __attribute__((address_space(3))) f32x4 lds_f32x4;
__device__ __forceinline__ float4 ld4_lds_v(const float *p) {
  const f32x4 v = *(lds_f32x4 *)(p);
  return make_float4(v.x, v.y, v.z, v.w);
}

// Eight waves, two per SIMD, so that one wave's matrix instructions issue
// while the other waits on memory, LDS or the barrier (with all 16 chains in
// one wave, 256 accumulator registers leave room for one wave per SIMD, and
// config 3 ran at 6.38 ms instead of 5.12).  The two waves of an output
// quadrant split ggml's 16 chains: wave half rh
// holds residues 4 rh .. 4 rh + 3 (block 0 of its four instructions) and
// 4 rh + 8 .. 4 rh + 11 (block 1): 4 accumulator sets, 128 AGPRs.  Per block a
// wave reads one float4 of each operand (k 16 b + 8 h + 4 rh ..) and issues 4
// instructions.  In the epilogue the rh = 0 wave holds a[q] + a[8+q] (q = 0..3,
// GGML_F32x4_REDUCE's sum[0] += sum[2]) and the rh = 1 wave a[4+q] + a[12+q]
// (sum[1] += sum[3]); each hands the other the four values of the rows the
// other finishes (tree, tail and store): rows 0..7 of the quadrant's 16 per
// lane go to rh = 0, rows 8..15 to rh = 1.
__device__ __forceinline__ void mfma_block4(v32f (&acc)[4], const float4 &a, const float4 &b) {
  acc[0] = __builtin_amdgcn_mfma_f32_32x32x1f32(a.x, b.x, acc[0], 0, 0, 0);
  acc[1] = __builtin_amdgcn_mfma_f32_32x32x1f32(a.y, b.y, acc[1], 0, 0, 0);
  acc[2] = __builtin_amdgcn_mfma_f32_32x32x1f32(a.z, b.z, acc[2], 0, 0, 0);
  acc[3] = __builtin_amdgcn_mfma_f32_32x32x1f32(a.w, b.w, acc[3], 0, 0, 0);
}

// A tile's first block: the accumulators start from +0 as ggml's do, given
// as the instruction's inline zero operand instead of 128 register moves.
__device__ __forceinline__ void mfma_block4_first(v32f (&acc)[4], const float4 &a, const float4 &b) {
  const v32f z = {};
  acc[0] = __builtin_amdgcn_mfma_f32_32x32x1f32(a.x, b.x, z, 0, 0, 0);
  acc[1] = __builtin_amdgcn_mfma_f32_32x32x1f32(a.y, b.y, z, 0, 0, 0);
  acc[2] = __builtin_amdgcn_mfma_f32_32x32x1f32(a.z, b.z, z, 0, 0, 0);
  acc[3] = __builtin_amdgcn_mfma_f32_32x32x1f32(a.w, b.w, z, 0, 0, 0);
}

// The fused ops whose operands the matrix kernels load before the products
// (16 registers), so their latency hides under the tile's instructions.
constexpr int kEpiEarly = 2;

// Element offset of output (row, col)'s operand of a fused op, the indices
// clamped into range (a discarded output reads a valid element).
template <class RowF, class ColF>
__device__ __forceinline__ int64_t dot_epi_off(const EpiOp &o, int64_t b, int64_t N, int64_t M, int r, RowF row,
                                               ColF col) {
  const int64_t nr = row(r), mr = col(r);
  return b * o.s0 + (nr < N ? nr : N - 1) * o.s1 + (mr < M ? mr : M - 1) * o.s2;
}

// Whether a fused op's operand is one value over a lane's 8 outputs: the
// 32x32-layout kernels' 8 outputs share a column (COLCONST), so an operand
// broadcast along rows (a bias) or a scalar is; in the 16x16 layout only a
// scalar per batch is.
template <bool COLCONST>
struct DotUniform {
  __device__ bool operator()(const EpiOp &o) const { return o.s1 == 0 && (COLCONST || o.s2 == 0); }
};

template <bool COLCONST, class RowF, class ColF>
__device__ __forceinline__ void dot_epi_early(const Epilogue &ep, int64_t b, int64_t N, int64_t M,
                                              float (&pre)[kEpiEarly][8], RowF row, ColF col) {
  epi_load_n(
      ep, pre, [&](const EpiOp &o, int r) { return dot_epi_off(o, b, N, M, r, row, col); }, DotUniform<COLCONST>());
}

// Stores the 8 outputs a lane finishes, output r at row row(r) and column
// col(r), after the serial tail of dot_finish when K % 16 != 0 and the fused
// element-wise ops (the first kEpiEarly with operands `pre` loaded by
// dot_epi_early).  `whole` (wave-uniform) says every output is in range and
// there is no tail.  `gelu` is a fused ggml.gelu_erf's routine (GeluErfOp or
// GeluErfSplitOp, by where the kernel holds the erff table).
template <bool COLCONST, int NE = kEpiEarly, class Gelu, class RowF, class ColF>
__device__ __forceinline__ void dot_store8(const MfmaOperand &X, const MfmaOperand &W, int64_t b, int64_t N,
                                           int64_t M, int64_t K, int64_t np, int tail, bool whole,
                                           const float (&out)[8], const Epilogue &ep, const float (&pre)[kEpiEarly][8],
                                           const Gelu &gelu, float *__restrict__ Y, RowF row, ColF col) {
  float v[8];
#pragma unroll
  for (int r = 0; r < 8; r++) v[r] = out[r];
  if (!whole && np < K) {
#pragma unroll
    for (int r = 0; r < 8; r++) {
      const int64_t nr = row(r), mr = col(r);
      if (nr >= N || mr >= M) continue;
      const float *xr = X.p + boff(X, b) + nr * X.sf;
      const float *wr = W.p + boff(W, b) + mr * W.sf;
      float sumf = v[r];
      if (tail == kTailPinned) {
        for (int64_t k = np; k < K; k++) {
          const float p = wr[k * W.sk] * xr[k * X.sk];
          sumf = sumf + p;
        }
      } else {
        const int64_t tl = K - np;
        const int64_t nq = tl >= 4 ? (tl & ~(int64_t)3) : 0;
        for (int64_t k = np; k < np + nq; k++) {
          const float p = wr[k * W.sk] * xr[k * X.sk];
          sumf = sumf + p;
        }
        for (int64_t k = np + nq; k < K; k++) sumf = __builtin_fmaf(wr[k * W.sk], xr[k * X.sk], sumf);
      }
      v[r] = sumf;
    }
  }
  if (ep.n > 0) {
    if (NE > 0) epi_ops_n(ep, v, pre, gelu);
    epi_apply_n(
        ep, v, [&](const EpiOp &o, int r) { return dot_epi_off(o, b, N, M, r, row, col); }, NE, gelu,
        DotUniform<COLCONST>());
  }
  float *y = Y + b * N * M;
  if (whole) {
#pragma unroll
    for (int r = 0; r < 8; r++) y[row(r) * M + col(r)] = v[r];
    return;
  }
#pragma unroll
  for (int r = 0; r < 8; r++)
    if (row(r) < N && col(r) < M) y[row(r) * M + col(r)] = v[r];
}


template <int LX, int LW>
__global__ void __launch_bounds__(512) dot_mfma8_k(MfmaOperand X, MfmaOperand W, int64_t N, int64_t M, int64_t K,
                                                   int tail, int tiles_m, Epilogue ep, float *__restrict__ Y) {
  constexpr int TH = 512, R = regs_of<TH>();
  extern __shared__ float lds_m[];  // [buffer][operand][kMT * kLS]; the epilogue's exchange reuses it
  auto tile = [&](int buf, int op) { return lds_m + (buf * 2 + op) * (kMT * kLS); };
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int quad = wave & 3, rh = wave >> 2;
  const int wn = quad >> 1, wm = quad & 1;
  const int64_t b = blockIdx.y;
  const int64_t n0 = (int64_t)(blockIdx.x / tiles_m) * kMT, m0 = (int64_t)(blockIdx.x % tiles_m) * kMT;
  const int64_t np = K & ~(int64_t)15;
  const int nb = (int)(np / 16);
  const int nst = (nb + kKC / 16 - 1) / (kKC / 16);

  v32f acc[4];
  if (nst == 0) {  // K < 16: no block; the tail starts from the +0 tree
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
      for (int r = 0; r < 32; r++) acc[q][r] = 0.0f;
  }

  // This lane's 8 outputs: rows nl + 8 (r / 4) + r % 4 of column ml.
  const int64_t nl = n0 + wn * 32 + 4 * (lane >> 5) + 16 * rh, ml = m0 + wm * 32 + (lane & 31);
  auto orow = [&](int r) { return nl + 8 * (r / 4) + r % 4; };
  auto ocol = [&](int) { return ml; };
  float pre[kEpiEarly][8];
  dot_epi_early<true>(ep, b, N, M, pre, orow, ocol);
  double *gtab = reinterpret_cast<double *>(lds_m + kDotStageFloats);  // a fused gelu_erf's table
  if (ep.gelu) load_poly(gtab);

  float4 rx[R], rw[R];
  const BufOp bx = buf_op<LX>(X, b, n0), bw = buf_op<LW>(W, b, m0);
  if (nst > 0) {
    mfma_fetch<LX, TH>(X, bx, n0, 0, nb, rx);
    mfma_fetch<LW, TH>(W, bw, m0, 0, nb, rw);
    mfma_stash<LX, TH>(tile(0, 0), rx);
    mfma_stash<LW, TH>(tile(0, 1), rw);
  }
  __syncthreads();
  const int h = lane >> 5, li = lane & 31;
  for (int s = 0; s < nst; s++) {
    const int buf = s & 1;
    const float *xs = tile(buf, 0) + (wn * 32 + li) * kLS + 8 * h + 4 * rh;
    const float *ws = tile(buf, 1) + (wm * 32 + li) * kLS + 8 * h + 4 * rh;
    const int blocks = min(kKC / 16, nb - s * (kKC / 16));
    // Straight-line code over the stage's kKC / 16 blocks (a loop header
    // between blocks costs a full LDS wait); blocks past the end of a short
    // last stage skip their instructions.  Block blk + 1's operands are read
    // before block blk's instructions issue: the reads are volatile so that
    // the compiler keeps them where they are written instead of sinking them
    // next to their use, and a scheduling barrier keeps them ahead of the
    // instructions.  The next stage's loads follow blocks 0 and 1 (a burst of
    // loads holds up the instructions queued behind it) and its LDS writes
    // blocks 4 and 5, four blocks after the loads (a short last stage has no
    // next stage).
    auto rd = [&](int k, float4 &x, float4 &w) {
      const int o = 16 * (k < blocks ? k : blocks - 1);  // blocks >= 1 in every stage
      x = ld4_lds_v(xs + o);
      w = ld4_lds_v(ws + o);
    };
    const bool more = s + 1 < nst;
    auto part = [&](int q) {
      if (more) {
        if (q == 0) mfma_fetch<LX, TH>(X, bx, n0, s + 1, nb, rx);
        if (q == 1) mfma_fetch<LW, TH>(W, bw, m0, s + 1, nb, rw);
        if (q == 4) mfma_stash<LX, TH>(tile(buf ^ 1, 0), rx);
        if (q == 5) mfma_stash<LW, TH>(tile(buf ^ 1, 1), rw);
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    float4 pa, qa, pb, qb;  // set p: even blocks, set q: odd blocks
    rd(0, pa, qa);
#pragma unroll
    for (int blk = 0; blk < kKC / 16; blk += 2) {
      rd(blk + 1, pb, qb);
      __builtin_amdgcn_sched_barrier(0);
      if (blk == 0 && s == 0) mfma_block4_first(acc, pa, qa);
      else if (blk < blocks) mfma_block4(acc, pa, qa);
      if (blk == 0 || blk == 4) part(blk);
      if (blk + 2 < kKC / 16) rd(blk + 2, pa, qa);
      __builtin_amdgcn_sched_barrier(0);
      if (blk + 1 < blocks) mfma_block4(acc, pb, qb);
      if (blk == 0 || blk == 4) part(blk + 1);
    }
    __syncthreads();
  }

  // Epilogue: register r of set q holds block r/16 of output row
  // i = 8*((r%16)/4) + 4*h + r%4, column j = lane%32.  Wave half rh finishes
  // rows r in [8 rh, 8 rh + 8) of its quadrant and hands the other half its
  // partial sums for the rest through LDS (every wave stores).
  float t4[16][4];
#pragma unroll
  for (int r = 0; r < 16; r++)
#pragma unroll
    for (int q = 0; q < 4; q++) t4[r][q] = acc[q][r] + acc[q][r + 16];  // rh 0: sum[0] += sum[2]; rh 1: sum[1] += sum[3]
  float *give = lds_m + wave * (8 * 4 * 64);                            // [r % 8][q][lane]
  const float *take = lds_m + (wave ^ 4) * (8 * 4 * 64);
#pragma unroll
  for (int r = 0; r < 8; r++)
#pragma unroll
    for (int q = 0; q < 4; q++) give[(r * 4 + q) * 64 + lane] = rh ? t4[r][q] : t4[8 + r][q];
  __syncthreads();
  float out[8];
#pragma unroll
  for (int r = 0; r < 8; r++) {
    float w[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const float mine = rh ? t4[8 + r][q] : t4[r][q], other = take[(r * 4 + q) * 64 + lane];
      w[q] = rh ? other + mine : mine + other;  // sum[0] += sum[1]
    }
    out[r] = (w[0] + w[1]) + (w[2] + w[3]);  // vaddvq_f32
  }
  dot_store8<true>(X, W, b, N, M, K, np, tail, np == K && n0 + kMT <= N && m0 + kMT <= M, out, ep, pre,
                   GeluErfOp{gtab}, Y, orow, ocol);
}


// ---- dot_mfma8_k with both operands loaded straight into LDS ----------------------
//
// For an lhs read along k and an rhs read along its free dim or along k,
// every read in range by construction: buffer_load_dwordx4 with
// the lds bit writes each lane's 16 bytes to LDS at the instruction's LDS base
// + 16 lane (checked on the device), so a stage needs no staging registers and
// no LDS store instructions, and the next stage's loads go out at the start of
// this stage, a whole stage before the barrier that waits for them.  One
// instruction fills 1 KB of LDS contiguously, so rows are unpadded:
//   lhs [64 rows][32 k-quads]: k-quad q of row r sits at chunk 32 r + (q ^ (r & 15)),
//     so 16 consecutive rows reading one k-quad hit 16 distinct bank quads;
//   rhs along its free dim (LW = kLoadColQuadB): [KC k][16 m-quads], as in
//     HBM: a lane reads its column one k at a time, 32 lanes on 32
//     consecutive floats;
//   rhs along k (LW = kLoadRowVecB): [64 columns][KC / 4 k-quads], swizzled
//     and read as the lhs.
// KC = 128 k per stage, or 64 for contractions in multiples of 64 (Q K^T
// with K = 64: rows of 16 chunks, 4 rows per instruction).  WAVES = 8: a
// 64 x 64 tile, 140 KB of LDS, one workgroup per CU.  WAVES = 4 (KC = 64): a
// 32 x 64 tile (two quadrants, two waves each) in 60 KB, so two workgroups
// share a CU and one's loads and epilogue overlap the other's products.
// The two stage buffers are separate LDS variables and the stage loop is
// unrolled by two, so the buffer being filled and the one being read are
// different objects to the compiler.  Chains, epilogue and stores are
// dot_mfma8_k's.
typedef __attribute__((address_space(3))) void lds_void;
typedef const volatile __attribute__((address_space(3))) float lds_f32;
__device__ __forceinline__ float ld1_lds_v(const float *p) { return *(lds_f32 *)(p); }
typedef const __attribute__((address_space(3))) float lds_f32n;

// MI355X hands the workgroups of a launch to its 8 XCDs in turn (linear id
// mod 8), and each XCD has its own 4 MB L2.  Consecutive tiles share operand
// strips (a row of tiles reads one lhs strip; a batch's tiles read one pair of
// operands), so renumber: XCD x takes the x-th contiguous run of ids, in
// order.  The runs are [x(q+1), (x+1)(q+1)) for x < r and r(q+1) + (x-r)q
// onward for the rest (q = total / 8, r = total % 8), which cover [0, total)
// once each: the set of tiles computed, and every output's bits, are
// unchanged.  Grids of 2^32 workgroups or more keep launch order.
constexpr uint32_t kXcds = 8;
__device__ __forceinline__ void xcd_tile(uint32_t &tx, uint32_t &ty) {
  const uint64_t total64 = (uint64_t)gridDim.x * gridDim.y;
  if (total64 > 0xFFFFFFFFull) return;
  const uint32_t gx = gridDim.x, total = (uint32_t)total64;
  const uint32_t lin = tx + gx * ty;
  const uint32_t q = total / kXcds, r = total % kXcds, x = lin % kXcds, i = lin / kXcds;
  const uint32_t id = (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + i;
  tx = id % gx;
  ty = id / gx;
}

template <int LX, int LW, int KC, int WAVES, bool EDGE>
__global__ void __launch_bounds__(WAVES * 64, 2) dot_mfma8d_k(MfmaOperand X, MfmaOperand W, int64_t N, int64_t M,
                                                           int64_t K, int tail, int tiles_m, Epilogue ep,
                                                           float *__restrict__ Y) {
  static_assert(LX == kLoadRowVecB && (LW == kLoadColQuadB || LW == kLoadRowVecB), "direct loads: lhs along k");
  static_assert(KC == 128 || KC == 64, "stages of 128 or 64 k");
  static_assert(WAVES == 8 || (WAVES == 4 && KC == 64), "four waves with stages of 64");
  constexpr int TN = WAVES == 8 ? kMT : 32;  // tile rows
  // 16-byte chunks per buffer: the eight-wave kernel keeps 32 KB buffers (its
  // epilogue exchange, 8 KB per wave, uses the lhs buffers); the four-wave one
  // exchanges through the rhs buffers.
  constexpr int XCH = WAVES == 8 ? kMT * kKC / 4 : TN * KC / 4, WCH = WAVES == 8 ? kMT * kKC / 4 : kMT * KC / 4;
  constexpr int CPR = KC / 4, RPI = 64 / CPR;  // chunks per row, rows per instruction
  constexpr int NIX = TN * KC / 4 / 64 / WAVES, NIW = kMT * KC / 4 / 64 / WAVES;  // instructions per wave
  static_assert((RPI * WAVES) % 16 == 0, "the swizzle key of a row does not depend on the instruction");
  __shared__ float4 dx0[XCH], dx1[XCH], dw0[WCH], dw1[WCH];
  extern __shared__ double gtab[];  // a fused gelu_erf's table (dynamic LDS, only with one)
  // The eight-wave kernel loads the first fused ops' operands before the
  // products; the four-wave one at the end (two more workgroups hide it, and
  // 16 fewer registers let three share a CU).
  constexpr int NE = WAVES == 8 ? kEpiEarly : 0;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int quad = wave % (WAVES / 2), rh = wave / (WAVES / 2);
  const int wn = WAVES == 8 ? quad >> 1 : 0, wm = WAVES == 8 ? quad & 1 : quad;
  // Batched four-wave launches (per-head products such as Q K^T and P V, whose
  // operands per batch are small) renumber their workgroups so that each XCD
  // walks whole batches (xcd_tile).  An unbatched one keeps launch order: each
  // XCD then takes every 8th column tile, so it keeps only an eighth of the rhs
  // hot in its L2 instead of all of it.  The eight-wave form (long
  // contractions) keeps launch order too, in which all XCDs share one batch's
  // operands in the MALL.
  uint32_t tx = blockIdx.x, ty = blockIdx.y;
  if (WAVES == 4 && gridDim.y > 1) xcd_tile(tx, ty);
  const int64_t b = ty;
  const int64_t n0 = (int64_t)(tx / tiles_m) * TN, m0 = (int64_t)(tx % tiles_m) * kMT;
  // The stages cover the blocks of 16 (np = K & ~15, a whole number of
  // stages: the host checks).  Every row a tile loads exists (rows padded to
  // the tile: the host checks).  EDGE: a serial tail (np < K) and outputs
  // past N or M (not stored); without it, np == K and every tile is whole.
  const int64_t np = EDGE ? K & ~(int64_t)15 : K;
  const int nst = (int)(np / KC);

  const int64_t nl = n0 + wn * 32 + 4 * (lane >> 5) + 16 * rh, ml = m0 + wm * 32 + (lane & 31);
  auto orow = [&](int r) { return nl + 8 * (r / 4) + r % 4; };
  auto ocol = [&](int) { return ml; };
  float pre[kEpiEarly][8];
  if (NE > 0) dot_epi_early<true>(ep, b, N, M, pre, orow, ocol);
  // A fused GELU's erff table: the eight-wave form stages it in dynamic LDS
  // at the start.  The four-wave form keeps its LDS at 48 KB, so that three
  // workgroups share a CU: with edge tiles it reads the table from global
  // memory (cached); without, it stages the table after the products in its
  // lhs stage buffers (LDS_TAB below).
  constexpr bool LDS_TAB = WAVES == 4 && !EDGE;
  const double *gt = WAVES == 4 ? &erffk::kPoly[0][0] : gtab;
  if (WAVES == 8 && ep.gelu) load_poly(gtab);

  // Loads.  Instruction i (0..NI-1) of wave w fills chunks 64 (8 i + w) .. + 63
  // of each operand: lhs rows RPI (8 i + w) + lane / CPR (lane % CPR is the
  // chunk's position in its row; the swizzle key, row & 15, does not depend
  // on i); a free-dim rhs k rows 32 i + 4 w + lane / 16, m-quad lane % 16; a
  // k-contiguous rhs as the lhs.  The per-instruction and per-stage advances
  // go in the scalar offset.
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const __amdgpu_buffer_rsrc_t bx =
      __builtin_amdgcn_make_buffer_rsrc((void *)(X.p + boff(X, b)), (short)0, 0x7FFFFFFF, 0x00020000);
  const __amdgpu_buffer_rsrc_t bw =
      __builtin_amdgcn_make_buffer_rsrc((void *)(W.p + boff(W, b)), (short)0, 0x7FFFFFFF, 0x00020000);
  const int xr = RPI * wave + lane / CPR;  // row of instruction 0
  const int xvoff = (int)(((n0 + xr) * X.sf + 4 * ((lane % CPR) ^ (xr & 15))) * 4);
  const int wvoff = LW == kLoadColQuadB
                        ? (int)((m0 + 4 * (lane % 16) + (int64_t)(4 * wave + lane / 16) * W.sk) * 4)
                        : (int)(((m0 + xr) * W.sf + 4 * ((lane % CPR) ^ (xr & 15))) * 4);
  auto dma_x = [&](float4 *dx, int s) {
#pragma unroll
    for (int i = 0; i < NIX; i++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(bx, (lds_void *)(dx + 64 * (WAVES * i + wv)), 16, xvoff,
                                               (int)((WAVES * RPI * i * X.sf + (int64_t)KC * s) * 4), 0, 0);
  };
  auto dma_w = [&](float4 *dw, int s) {
#pragma unroll
    for (int i = 0; i < NIW; i++) {
      const int so = LW == kLoadColQuadB ? (int)(((int64_t)4 * WAVES * i + (int64_t)KC * s) * W.sk * 4)
                                         : (int)((WAVES * RPI * i * W.sf + (int64_t)KC * s) * 4);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(bw, (lds_void *)(dw + 64 * (WAVES * i + wv)), 16, wvoff, so, 0, 0);
    }
  };

  // Reads.  lhs: row wn 32 + li, k-quad 4 blk + 2 h + rh at chunk
  // row CPR + 4 (blk ^ kh) + kx (kh, kx: the row key's high and low bits);
  // a free-dim rhs: float (16 blk + 8 h + 4 rh + q) 64 + wm 32 + li; a
  // k-contiguous rhs: column wm 32 + li as an lhs row (the same key).
  const int h = lane >> 5, li = lane & 31;
  const int key = li & 15;  // (wn 32 + li) & 15 and (wm 32 + li) & 15
  const int kx = (2 * h + rh) ^ (key & 3), kh = key >> 2;
  int xa[4], wa4[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {  // floats; block blk: xa[blk & 3] + 64 (blk >> 2)
    xa[j] = (wn * 32 + li) * KC + 4 * (4 * (j ^ kh) + kx);
    wa4[j] = (wm * 32 + li) * KC + 4 * (4 * (j ^ kh) + kx);
  }
  const int wa = (8 * h + 4 * rh) * kMT + wm * 32 + li;

  v32f acc[4];
  auto stage = [&](const float4 *cx, const float4 *cw, float4 *nx, float4 *nw, int s) {
    const float *xs = reinterpret_cast<const float *>(cx), *ws = reinterpret_cast<const float *>(cw);
    const bool more = s + 1 < nst;
    auto rd = [&](int k, float4 &x, float4 &w) {
      x = ld4_lds_v(xs + xa[k & 3] + 64 * (k >> 2));
      if (LW == kLoadRowVecB) {
        w = ld4_lds_v(ws + wa4[k & 3] + 64 * (k >> 2));
      } else {
        // Plain (not volatile) reads: the compiler pairs rows k, k + 1 into
        // ds_read2st64_b32 (config 3 -1.5%).
        const lds_f32n *q = (const lds_f32n *)(ws + wa + 16 * k * kMT);
        w = make_float4(q[0], q[kMT], q[2 * kMT], q[3 * kMT]);
      }
    };
    float4 pa, qa, pb, qb;  // set p: even blocks, set q: odd blocks
    rd(0, pa, qa);
#pragma unroll
    for (int blk = 0; blk < KC / 16; blk += 2) {
      rd(blk + 1, pb, qb);
      __builtin_amdgcn_sched_barrier(0);
      if (blk == 0 && s == 0) mfma_block4_first(acc, pa, qa);
      else mfma_block4(acc, pa, qa);
      if (blk == 0 && more) dma_x(nx, s + 1);
      if (blk + 2 < KC / 16) rd(blk + 2, pa, qa);
      __builtin_amdgcn_sched_barrier(0);
      mfma_block4(acc, pb, qb);
      if (blk == 0 && more) dma_w(nw, s + 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads have landed in LDS
    __syncthreads();
  };
  dma_x(dx0, 0);
  dma_w(dw0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int s = 0; s < nst; s += 2) {
    stage(dx0, dw0, dx1, dw1, s);
    if (s + 1 < nst) stage(dx1, dw1, dx0, dw0, s + 1);
  }

  // LDS_TAB with a fused GELU: after the last stage's barrier no wave reads
  // the lhs stage buffers and no load into them is outstanding, so the erff
  // table goes there, straight from memory (buffer_load_dwordx4 lds, no
  // registers): twelve 1 KB chunks, three per wave, chunks 0 .. 5 (rows
  // 0 .. 127) to dx0 and 6 .. 11 (rows 128 .. 255) to dx1.  The wave waits for
  // its chunks before the exchange's barrier.
  static_assert(!LDS_TAB || (WAVES == 4 && kPolyWords * 8 == 12 * 1024 && kPolyHalfRows * 6 * 8 == 6 * 1024 &&
                             6 * 64 <= XCH),
                "the erff table is twelve 1 KB chunks, six per lhs stage buffer, three per wave");
  const bool stage_tab = LDS_TAB && ep.gelu;
  if (stage_tab) {
    const __amdgpu_buffer_rsrc_t tr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)&erffk::kPoly[0][0], (short)0, kPolyWords * (int)sizeof(double), 0x00020000);
#pragma unroll
    for (int j = 0; j < 3; j++) {
      const int c = 4 * j + wv;  // wave-uniform
      float4 *dst = c < 6 ? dx0 + 64 * c : dx1 + 64 * (c - 6);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(tr, (lds_void *)dst, 16, 16 * lane, 1024 * c, 0, 0);
    }
  }

  // Epilogue: dot_mfma8_k's, the exchange in the lhs buffers (waves 0..3 in
  // dx0, 4..7 in dx1; four waves: the rhs buffers; no load is outstanding
  // after the last stage).
  float t4[16][4];
#pragma unroll
  for (int r = 0; r < 16; r++)
#pragma unroll
    for (int q = 0; q < 4; q++) t4[r][q] = acc[q][r] + acc[q][r + 16];
  static_assert((WAVES / 2) * 8 * 4 * 64 <= 4 * (WAVES == 8 ? XCH : WCH), "the exchange fits its buffers");
  float *give = reinterpret_cast<float *>(WAVES == 8 ? (rh ? dx1 : dx0) : (rh ? dw1 : dw0)) + quad * (8 * 4 * 64);
  const float *take =
      reinterpret_cast<const float *>(WAVES == 8 ? (rh ? dx0 : dx1) : (rh ? dw0 : dw1)) + quad * (8 * 4 * 64);
#pragma unroll
  for (int r = 0; r < 8; r++)
#pragma unroll
    for (int q = 0; q < 4; q++) give[(r * 4 + q) * 64 + lane] = rh ? t4[r][q] : t4[8 + r][q];
  if (stage_tab) __builtin_amdgcn_s_waitcnt(0);  // this wave's table chunks have landed in LDS
  __syncthreads();
  // EDGE with a tail: the tile's tail operands (lhs rows n0.., rhs rows m0..,
  // k in [np, K)) go to LDS once, in the buffers the exchange leaves free
  // (rows past N or M read row N - 1 or M - 1; those outputs are discarded).
  const int tl = (int)(K - np);
  float *tlx = reinterpret_cast<float *>(WAVES == 8 ? dw0 : dx0), *tlw = tlx + TN * 16;
  static_assert((TN + kMT) * 16 <= 4 * (WAVES == 8 ? WCH : XCH), "the tail operands fit their buffer");
  if (EDGE && tl > 0) {
    const float *xb = X.p + boff(X, b), *wb = W.p + boff(W, b);
    for (int i = threadIdx.x; i < (TN + kMT) * tl; i += WAVES * 64) {
      const int r = i / tl, k = i - r * tl;
      if (r < TN) {
        const int64_t row = n0 + r < N ? n0 + r : N - 1;
        tlx[r * 16 + k] = xb[row * X.sf + (np + k) * X.sk];
      } else {
        const int64_t row = m0 + (r - TN) < M ? m0 + (r - TN) : M - 1;
        tlw[(r - TN) * 16 + k] = wb[row * W.sf + (np + k) * W.sk];
      }
    }
  }
  if (EDGE) __syncthreads();
  float out[8];
#pragma unroll
  for (int r = 0; r < 8; r++) {
    float w[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const float mine = rh ? t4[8 + r][q] : t4[r][q], other = take[(r * 4 + q) * 64 + lane];
      w[q] = rh ? other + mine : mine + other;  // sum[0] += sum[1]
    }
    out[r] = (w[0] + w[1]) + (w[2] + w[3]);  // vaddvq_f32
  }
  if (EDGE && tl > 0) {  // the serial tail of dot_finish, operands from LDS
    // Products k < nq are rounded and then added, the rest fused (the stock
    // rule: nq = tl & ~3 when tl >= 4, else 0; the pinned rule: all rounded),
    // k in order for each of the lane's eight outputs.  One loop over k with
    // a wave-uniform choice per k: two loops with run-time bounds, one after
    // the other, ran the [8192,263] x [263,512] product in 59 us instead of
    // the 35 us a 264-long contraction took.
    const float *wt = tlw + (ocol(0) - m0) * 16;
    const int nq = tail == kTailPinned ? tl : (tl >= 4 ? (tl & ~3) : 0);
    for (int k = 0; k < tl; k++) {
      const float w = wt[k];
      if (k < nq) {
#pragma unroll
        for (int r = 0; r < 8; r++) {
          const float p = w * tlx[(orow(r) - n0) * 16 + k];
          out[r] = out[r] + p;
        }
      } else {
#pragma unroll
        for (int r = 0; r < 8; r++) out[r] = __builtin_fmaf(w, tlx[(orow(r) - n0) * 16 + k], out[r]);
      }
    }
  }
  const bool whole = !EDGE || (n0 + TN <= N && m0 + kMT <= M);
  if constexpr (LDS_TAB) {
    const GeluErfSplitOp gelu{reinterpret_cast<const double *>(dx0), reinterpret_cast<const double *>(dx1)};
    dot_store8<true, NE>(X, W, b, N, M, K, K, tail, whole, out, ep, pre, gelu, Y, orow, ocol);
  } else {
    dot_store8<true, NE>(X, W, b, N, M, K, K, tail, whole, out, ep, pre, GeluErfOp{gt}, Y, orow, ocol);
  }
}


constexpr int kDotLds = kDotStageFloats * (int)sizeof(float);                     // 135,168 bytes
constexpr int kDotLdsGelu = kDotLds + kPolyWords * (int)sizeof(double);            // 147,456 bytes
static_assert(kDotStageFloats % 4 == 0, "the gelu table starts 16-byte aligned");
static_assert(8 * 8 * 4 * 64 <= 4 * kMT * kLS, "dot_mfma8_k's epilogue exchange fits the LDS");

// ---- soft_max ---------------------------------------------------------------------
//
// ggml_vec_soft_max_f32 adds each four-element group's part (a binary32
// value >= 0) to a binary64 sum in group order, then the scalar tail values
// (Shaders.lean:111-120).  That serial chain can be shortened wherever none of
// its additions rounds.  Take a run of additions s + p_1 + ... + p_n (s the
// running binary64 sum, p_i parts) and let u be the smallest ulp among s and
// the nonzero p_i: a binary32 value is an integer multiple of its ulp
// (2^(e-150) for exponent field e, 2^-149 for subnormals), a binary64 value
// of its own.  If the exact total is below 2^53 u, every partial sum, in any
// order, is a multiple of u below 2^53 u, hence a binary64 number: no addition
// rounds, and the in-order chain, a tree sum and the exact total coincide.
// The computed total t decides it: over at most 2^11 additions of
// non-negative terms t falls short of the exact total by a relative 2^-42 at
// most, so t <= (1 - 2^-20) 2^53 u implies an exact total below 2^53 u, and
// then t is that total.
//
// ordered_sum_apply first tests the whole row at once (a wave's tree sum T).
// A row that fails (parts spread over more than about 2^50, a NaN, an
// infinity) still needs only a monotone f(S) of the in-order sum S: softmax's
// inv = (float)(1.0 / S), non-increasing, or norm's variance
// (float)(S / cols), non-decreasing.  For n <= 2^11 non-negative terms S lies
// within a relative (n-1) 2^-53 < 2^-42 of the exact total and T within 2^-48
// of it, so S lies in [T (1 - 2^-41), T (1 + 2^-41)], inside
// [lo, hi] = T (1 -+ 2^-40) computed in binary64; f(lo) == f(hi) then fixes
// f(S).  Only a row whose f(S) falls within about 2^-40 of a binary32 rounding
// boundary fails that as well (about one row in 10^5 of those); it walks its
// parts in segments of 16 consecutive groups (one 16-lane row of the wave,
// reduced with DPP), adding a segment's tree sum in one step when the exactness
// test holds for the running sum and that segment, and the segment's parts one
// by one in group order when it does not.

// Biased exponent e of p's ulp 2^(e-150) for a part p >= 0: its exponent
// field, 1 for subnormals, 255 (no constraint) for +0.
__device__ __forceinline__ int part_ulp_exp(float p) {
  const uint32_t u = f_bits(p) & 0x7FFFFFFFu;
  if (u == 0) return 255;
  const int e = (int)(u >> 23);
  return e > 1 ? e : 1;
}

// (1 - 2^-20) 2^53 u for u = 2^(e-150), i.e. 2^(e-98) (2 - 2^-19): exponent
// field e + 925, the top 19 fraction bits set.
__device__ __forceinline__ double exact_limit(int e) {
  return __builtin_bit_cast(double, ((uint64_t)(e + 925) << 52) | (((1ull << 19) - 1) << 33));
}

// The biased exponent e (in part_ulp_exp's units: the bit is 2^(e-150)) of the
// lowest set bit of a binary64 s, 255 for 0: every partial sum that s and
// multiples of that bit make is a multiple of it.
__device__ __forceinline__ int low_bit_exp(double s) {
  const uint64_t b = __builtin_bit_cast(uint64_t, s) & 0x7FFFFFFFFFFFFFFFull;
  if (b == 0) return 255;
  const int E = (int)(b >> 52);
  const uint64_t m = b & ((1ull << 52) - 1);
  const uint64_t sig = E ? (m | (1ull << 52)) : m;
  return (E ? E : 1) - 1075 + __builtin_ctzll(sig) + 150;
}

// DPP within 16-lane rows: quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror, row_mirror.  After the four steps every lane of a row holds
// a reduction over the row's 16 lanes.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) { return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true); }
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)dpp_i<CTRL>((int)(uint32_t)u), hi = (uint32_t)dpp_i<CTRL>((int)(uint32_t)(u >> 32));
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double row16_sum(double v) {
  v = v + dpp_d<kDppXor1>(v);
  v = v + dpp_d<kDppXor2>(v);
  v = v + dpp_d<kDppHalfMirror>(v);
  return v + dpp_d<kDppMirror>(v);
}
__device__ __forceinline__ int row16_min(int v) {
  v = min(v, dpp_i<kDppXor1>(v));
  v = min(v, dpp_i<kDppXor2>(v));
  v = min(v, dpp_i<kDppHalfMirror>(v));
  return min(v, dpp_i<kDppMirror>(v));
}
// Whole-wave binary64 sum and int minimum, the same on every lane: rows of 16
// through DPP, then the four row results read as scalars and added as
// (r0 + r1) + (r2 + r3).  Six levels, as a butterfly over 64 lanes; the
// callers' error bounds count only the depth.
__device__ __forceinline__ double wave_sum_d(double v);
__device__ __forceinline__ int wave_min_i(int v);
__device__ __forceinline__ float lane_f(float v, int l) {
  return bits_f((uint32_t)__builtin_amdgcn_readlane((int)f_bits(v), l));
}
__device__ __forceinline__ double lane_d(double v, int l) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double wave_sum_d(double v) {
  v = row16_sum(v);
  return (lane_d(v, 0) + lane_d(v, 16)) + (lane_d(v, 32) + lane_d(v, 48));
}
__device__ __forceinline__ float wave_max_f(float v) {
  v = __builtin_fmaxf(v, bits_f((uint32_t)dpp_i<kDppXor1>((int)f_bits(v))));
  v = __builtin_fmaxf(v, bits_f((uint32_t)dpp_i<kDppXor2>((int)f_bits(v))));
  v = __builtin_fmaxf(v, bits_f((uint32_t)dpp_i<kDppHalfMirror>((int)f_bits(v))));
  v = __builtin_fmaxf(v, bits_f((uint32_t)dpp_i<kDppMirror>((int)f_bits(v))));
  return __builtin_fmaxf(__builtin_fmaxf(lane_f(v, 0), lane_f(v, 16)), __builtin_fmaxf(lane_f(v, 32), lane_f(v, 48)));
}
__device__ __forceinline__ int wave_min_i(int v) {
  v = row16_min(v);
  return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// fin(S) for the in-order binary64 sum S of a row's parts: group part
// g = l + 64 j, held by lane l as part[j] (+0 for g >= G), then tail values
// on lanes < T.  fin must be monotone (either way) on binary64 values; the
// result is the same on every lane.
template <int J, bool FULL, class Fin>
__device__ __forceinline__ float ordered_sum_apply(const float (&part)[J], int G, float tail, int T, Fin fin) {
  const int lane = threadIdx.x % kWave;
  double ls = 0.0;
  int le = 255;
#pragma unroll
  for (int j = 0; j < J; j++) {
    ls = ls + (double)part[j];
    le = min(le, part_ulp_exp(part[j]));
  }
  if (lane < T) {
    ls = ls + (double)tail;
    le = min(le, part_ulp_exp(tail));
  }
  ls = wave_sum_d(ls);
  le = wave_min_i(le);
  if (ls <= exact_limit(le)) return fin(ls);
  const double d = ls * 0x1p-40;  // exact: ls >= 2^-149 or ls = 0
  const float f_lo = fin(ls - d), f_hi = fin(ls + d);
  if (f_lo == f_hi) return f_lo;  // false for NaN and infinity
  // In order, segment by segment: segment q = 4 j + r holds groups
  // 64 j + 16 r .. 64 j + 16 r + 15 (lanes 16 r .. 16 r + 15 of slice j).
  double s = 0.0;
#pragma unroll
  for (int j = 0; j < J; j++) {
    if (!FULL && kWave * j >= G) break;
    const double seg = row16_sum((double)part[j]);
    const int sege = row16_min(part_ulp_exp(part[j]));
#pragma unroll
    for (int r = 0; r < 4; r++) {
      if (!FULL && kWave * j + 16 * r >= G) break;
      // u = min(ulp(s), the segment's smallest part ulp): the test splits
      // into the segment's limit and s's own, (1 - 2^-20) 2^53 ulp(s), which
      // is s's binade top 2^(E+1) less 2^-20 of it (no constraint for s = 0).
      const double t = s + lane_d(seg, 16 * r);
      const double lim_p = exact_limit(__builtin_amdgcn_readlane(sege, 16 * r));
      const uint32_t hs = (uint32_t)(__builtin_bit_cast(uint64_t, s) >> 32);
      const double lim_s = __builtin_bit_cast(double, (uint64_t)((hs & 0xFFF00000u) | 0x000FFFFEu) << 32);
      if (t <= lim_p && (s == 0.0 || t <= lim_s)) {
        s = t;
      } else {
#pragma unroll 1
        for (int i = 0; i < 16; i++) s = s + (double)lane_f(part[j], 16 * r + i);
      }
    }
  }
  for (int l = 0; l < T; l++) s = s + (double)lane_f(tail, l);
  return fin(s);
}

// softmax's inv = (float)(1.0 / S), S as in ordered_sum_apply.
template <int J, bool FULL>
__device__ __forceinline__ float softmax_inv(const float (&part)[J], int G, float tail, int T, int float_sum) {
  if (float_sum) {  // planted: the denominator summed in binary32 (Shaders.lean:120-122)
    float fs = 0.0f;
#pragma unroll
    for (int j = 0; j < J; j++) {
      const int n = FULL ? kWave : min(kWave, G - kWave * j);
      for (int l = 0; l < n; l++) fs = fs + lane_f(part[j], l);
    }
    for (int l = 0; l < T; l++) fs = fs + lane_f(tail, l);
    return 1.0f / fs;
  }
  return ordered_sum_apply<J, FULL>(part, G, tail, T, [](double x) { return (float)(1.0 / x); });
}

// ggml soft_max, one wave per row.  Lane l owns the four-element groups
// g = l + 64j, loaded as float4 (coalesced).  Loads and stores are both
// nontemporal: ordinary loads keep the logits in the MALL across back-to-back
// calls of softmax alone (4.8 us instead of 5.6 on [4096,1024]) but evict the
// data of the kernels around it (the config-2 module, softmax then a 64 Mi
// GELU, ran 97 us per call instead of 89).  The row maximum is a wave reduction of v_max_f32: on rows without
// NaN it equals ggml's (mx > w ? mx : w) chain in any order, and a +0/-0 tie
// cannot change an output since exp(x - (+0)) = exp(x - (-0)); a NaN anywhere
// in a row makes every output NaN through the sum, whatever the maximum.
// Each group's e = ggml_v_expf(x*sc - mx) stays in registers, its
// vaddvq_f32 part goes into softmax_inv, and y = e*inv.
// FULL: every lane owns exactly J groups (cols == 256*J), so no group index
// needs a bounds check.  UNIT: scale == 1, so x*sc is x (a NaN x makes the
// whole row NaN either way, through its own part of the sum).
template <int J, bool FULL, bool UNIT>
__device__ __forceinline__ void softmax_row(float4 (&e)[J], int G, float sc, int float_sum) {
  const int lane = threadIdx.x % kWave;
  float mx = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < J; j++) {
    const int g = lane + kWave * j;
    if (FULL || g < G) {
      if (!UNIT) e[j] = make_float4(e[j].x * sc, e[j].y * sc, e[j].z * sc, e[j].w * sc);
      mx = __builtin_fmaxf(mx, __builtin_fmaxf(__builtin_fmaxf(e[j].x, e[j].y), __builtin_fmaxf(e[j].z, e[j].w)));
    }
  }
  mx = wave_max_f(mx);
  // The arguments x*sc - mx are <= 0 (or -inf, or NaN): the fast form, with
  // the rare 126 < |n| <= 192 elements recomputed when any lane has one.
  float4 v[J];
  bool mid = false;
#pragma unroll
  for (int j = 0; j < J; j++) {
    const int g = lane + kWave * j;
    if (FULL || g < G) {
      bool m0, m1, m2, m3;
      v[j] = make_float4(e[j].x - mx, e[j].y - mx, e[j].z - mx, e[j].w - mx);  // e holds x*sc
      e[j].x = ggml_v_expf_nonpos(v[j].x, &m0);
      e[j].y = ggml_v_expf_nonpos(v[j].y, &m1);
      e[j].z = ggml_v_expf_nonpos(v[j].z, &m2);
      e[j].w = ggml_v_expf_nonpos(v[j].w, &m3);
      mid |= m0 | m1 | m2 | m3;
    }
  }
  if (__any(mid)) {
#pragma unroll
    for (int j = 0; j < J; j++) {
      const int g = lane + kWave * j;
      if (FULL || g < G) {
        e[j].x = ggml_v_expf(v[j].x);
        e[j].y = ggml_v_expf(v[j].y);
        e[j].z = ggml_v_expf(v[j].z);
        e[j].w = ggml_v_expf(v[j].w);
      }
    }
  }
  float part[J];
#pragma unroll
  for (int j = 0; j < J; j++) {
    const int g = lane + kWave * j;
    part[j] = (FULL || g < G) ? (e[j].x + e[j].y) + (e[j].z + e[j].w) : 0.0f;
  }
  const float inv = softmax_inv<J, FULL>(part, G, 0.0f, 0, float_sum);
#pragma unroll
  for (int j = 0; j < J; j++) e[j] = make_float4(e[j].x * inv, e[j].y * inv, e[j].z * inv, e[j].w * inv);
}

// ggml soft_max, one wave per row.  Lane l owns the four-element groups
// g = l + 64j, loaded as float4 (coalesced).  Loads and stores are both
// nontemporal: ordinary loads keep the logits in the MALL across back-to-back
// calls of softmax alone (4.8 us instead of 5.6 on [4096,1024]) but evict the
// data of the kernels around it (the config-2 module, softmax then a 64 Mi
// GELU, ran 97 us per call instead of 89).  The row maximum is a wave reduction of v_max_f32: on rows without
// NaN it equals ggml's (mx > w ? mx : w) chain in any order, and a +0/-0 tie
// cannot change an output since exp(x - (+0)) = exp(x - (-0)); a NaN anywhere
// in a row makes every output NaN through the sum, whatever the maximum.
// Each group's e = ggml_v_expf(x*sc - mx) stays in registers, its
// vaddvq_f32 part goes into softmax_inv, and y = e*inv (softmax_row).
// FULL: every lane owns exactly J groups (cols == 256*J), so no group index
// needs a bounds check.  UNIT: scale == 1, so x*sc is x (a NaN x makes the
// whole row NaN either way, through its own part of the sum).
template <int J, bool FULL, bool UNIT = false>
__global__ void __launch_bounds__(256) soft_max_rows_k(int64_t rows, int cols, float sc, int float_sum,
                                                       const float *__restrict__ X, float *__restrict__ Y) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int G = cols / 4;
  const int64_t row = blockIdx.x * 4LL + wave;
  if (row >= rows) return;  // the whole wave; no barrier follows
  const float *x = X + row * cols;
  float4 e[J];
#pragma unroll
  for (int j = 0; j < J; j++) {
    const int g = lane + kWave * j;
    e[j] = (FULL || g < G) ? ld4_nt(x + 4 * g) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  softmax_row<J, FULL, UNIT>(e, G, sc, float_sum);
  float *y = Y + row * cols;
#pragma unroll
  for (int j = 0; j < J; j++) {
    const int g = lane + kWave * j;
    if (FULL || g < G) st4_nt(y + 4 * g, e[j]);
  }
}

// Rows whose length is not a multiple of 4 (the pinned flavour only): ggml
// runs the four-lane body over the first 4*G elements and sends the last
// cols % 4 through the scalar expf, the correctly rounded one here, adding
// each tail value to the binary64 sum after the group parts
// (ggml_vec_soft_max_f32).  Rows are not 16-byte aligned, so elements are read
// one by one; wave w of a block owns row 4*blockIdx.x + w.
template <int J>
__global__ void __launch_bounds__(256) soft_max_tail_k(int64_t rows, int cols, float sc, int float_sum,
                                                       const float *__restrict__ X, float *__restrict__ Y) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int G = cols / 4, T = cols % 4;
  const int64_t row = blockIdx.x * 4LL + wave;
  if (row >= rows) return;  // the whole wave; no barrier follows
  const float *x = X + row * cols;
  float *y = Y + row * cols;
  float4 e[J];
  float et = 0.0f;
  float mx = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < J; j++) {
    const int g = lane + kWave * j;
    if (g < G) {
      e[j] = make_float4(x[4 * g], x[4 * g + 1], x[4 * g + 2], x[4 * g + 3]);
      const float w0 = e[j].x * sc, w1 = e[j].y * sc, w2 = e[j].z * sc, w3 = e[j].w * sc;
      mx = mx > w0 ? mx : w0;
      mx = mx > w1 ? mx : w1;
      mx = mx > w2 ? mx : w2;
      mx = mx > w3 ? mx : w3;
    }
  }
  if (lane < T) {
    et = x[4 * G + lane];
    const float w = et * sc;
    mx = mx > w ? mx : w;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float other = __shfl_xor(mx, o, kWave);
    mx = mx > other ? mx : other;
  }
  float part[J];
#pragma unroll
  for (int j = 0; j < J; j++) {
    const int g = lane + kWave * j;
    part[j] = 0.0f;
    if (g < G) {
      e[j].x = ggml_v_expf(e[j].x * sc - mx);
      e[j].y = ggml_v_expf(e[j].y * sc - mx);
      e[j].z = ggml_v_expf(e[j].z * sc - mx);
      e[j].w = ggml_v_expf(e[j].w * sc - mx);
      part[j] = (e[j].x + e[j].y) + (e[j].z + e[j].w);
    }
  }
  if (lane < T) et = expfk::expf_cr(et * sc - mx);
  const float inv = softmax_inv<J, false>(part, G, et, T, float_sum);
#pragma unroll
  for (int j = 0; j < J; j++) {
    const int g = lane + kWave * j;
    if (g < G) {
      y[4 * g] = e[j].x * inv;
      y[4 * g + 1] = e[j].y * inv;
      y[4 * g + 2] = e[j].z * inv;
      y[4 * g + 3] = e[j].w * inv;
    }
  }
  if (lane < T) y[4 * G + lane] = et * inv;
}

// ---- softmax over 16-lane rows --------------------------------------------------------
//
// For rows of 64 NJ elements in LDS a wave takes four rows at once: lane
// 16 q + i holds row q's four-element groups g = i + 16 j (j < NJ).  Every
// reduction stays inside the row's 16 lanes (DPP), so the per-row work (the
// maximum, the binary64 sum and its decision, the reciprocal) is shared by
// four rows and needs no lane reads.  The values are softmax_row's.

__device__ __forceinline__ float row16_max_f(float v) {
  v = __builtin_fmaxf(v, bits_f((uint32_t)dpp_i<kDppXor1>((int)f_bits(v))));
  v = __builtin_fmaxf(v, bits_f((uint32_t)dpp_i<kDppXor2>((int)f_bits(v))));
  v = __builtin_fmaxf(v, bits_f((uint32_t)dpp_i<kDppHalfMirror>((int)f_bits(v))));
  return __builtin_fmaxf(v, bits_f((uint32_t)dpp_i<kDppMirror>((int)f_bits(v))));
}

// fin(S) for the in-order binary64 sum S of a 16-lane row's parts (part[j]
// of lane i is group i + 16 j), decided as in ordered_sum_apply: exact, or
// inside an interval fin maps to one value (the sum's error over its NJ + 4
// levels is far below 2^-40 of it: every part is >= 0), or else walked in
// order, segment j (groups 16 j .. 16 j + 15) at a time.
template <int NJ, class Fin>
__device__ __forceinline__ float ordered_sum16(const float (&part)[NJ], Fin fin) {
  double ls = 0.0;
  int le = 255;
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    ls = ls + (double)part[j];
    le = min(le, part_ulp_exp(part[j]));
  }
  ls = row16_sum(ls);
  le = row16_min(le);
  if (ls <= exact_limit(le)) return fin(ls);
  const double d = ls * 0x1p-40;  // exact: ls >= 2^-149 or ls = 0
  const float f_lo = fin(ls - d), f_hi = fin(ls + d);
  if (f_lo == f_hi) return f_lo;  // false for NaN and infinity
  const int base = threadIdx.x & 48;  // the row's first lane
  double s = 0.0;
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const double seg = row16_sum((double)part[j]);
    const int sege = row16_min(part_ulp_exp(part[j]));
    const double t = s + seg;
    const double lim_p = exact_limit(sege);
    const uint32_t hs = (uint32_t)(__builtin_bit_cast(uint64_t, s) >> 32);
    const double lim_s = __builtin_bit_cast(double, (uint64_t)((hs & 0xFFF00000u) | 0x000FFFFEu) << 32);
    if (t <= lim_p && (s == 0.0 || t <= lim_s)) {
      s = t;
    } else {
#pragma unroll 1
      for (int i = 0; i < 16; i++) s = s + (double)__shfl(part[j], base + i);
    }
  }
  return fin(s);
}

// softmax_row on a 16-lane row of 16 NJ groups (every group present), the
// row's values e also stored at rp (4 (i + 16 j) for group j): the rare
// recomputation of the 126 < |n| <= 192 exponentials reads them back rather
// than keeping the arguments in registers.
//
// Returns (the same in every lane) bit j set when slice j of all four rows
// came out +0 exactly: the slice was set to zeros and every row's reciprocal
// is finite (a NaN reciprocal, from a NaN in the row, makes the slice NaN).
template <int NJ, bool UNIT>
__device__ __forceinline__ uint32_t softmax_row16(float4 (&e)[NJ], float sc, float *rp) {
  const int li = threadIdx.x & 15;
  float mx = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    *reinterpret_cast<float4 *>(rp + 4 * (li + 16 * j)) = e[j];
    if (!UNIT) e[j] = make_float4(e[j].x * sc, e[j].y * sc, e[j].z * sc, e[j].w * sc);
    mx = __builtin_fmaxf(mx, __builtin_fmaxf(__builtin_fmaxf(e[j].x, e[j].y), __builtin_fmaxf(e[j].z, e[j].w)));
  }
  mx = row16_max_f(mx);
  // A slice j that holds only -inf on every lane, with each row's maximum
  // neither -inf nor NaN, gives ggml_v_expf(-inf - mx) = +0 throughout (its
  // |n| > 192 branch): it is set, not computed (a causal mask's upper half).
  const bool mx_ok = mx > -__builtin_inff();
  bool mid = false;
  uint32_t zero = 0;
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    // maximum (IEEE 754-2019: a NaN operand gives NaN) of the four is -inf
    // exactly when all four are -inf: two v_maximum3_f32 and one compare
    const float m4 = __builtin_elementwise_maximum(__builtin_elementwise_maximum(e[j].x, e[j].y),
                                                   __builtin_elementwise_maximum(e[j].z, e[j].w));
    if (__all(mx_ok && m4 == -__builtin_inff())) {
      e[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      zero |= 1u << j;
      continue;
    }
    bool m0, m1, m2, m3;
    e[j].x = ggml_v_expf_nonpos(e[j].x - mx, &m0);
    e[j].y = ggml_v_expf_nonpos(e[j].y - mx, &m1);
    e[j].z = ggml_v_expf_nonpos(e[j].z - mx, &m2);
    e[j].w = ggml_v_expf_nonpos(e[j].w - mx, &m3);
    mid |= m0 | m1 | m2 | m3;
  }
  if (__any(mid)) {
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      float4 x = *reinterpret_cast<const float4 *>(rp + 4 * (li + 16 * j));
      if (!UNIT) x = make_float4(x.x * sc, x.y * sc, x.z * sc, x.w * sc);
      e[j].x = ggml_v_expf(x.x - mx);
      e[j].y = ggml_v_expf(x.y - mx);
      e[j].z = ggml_v_expf(x.z - mx);
      e[j].w = ggml_v_expf(x.w - mx);
    }
  }
  float part[NJ];
#pragma unroll
  for (int j = 0; j < NJ; j++) part[j] = (e[j].x + e[j].y) + (e[j].z + e[j].w);
  const float inv = ordered_sum16<NJ>(part, [](double x) { return (float)(1.0 / x); });
#pragma unroll
  for (int j = 0; j < NJ; j++) e[j] = make_float4(e[j].x * inv, e[j].y * inv, e[j].z * inv, e[j].w * inv);
  return __all(__builtin_isfinite(inv)) ? zero : 0u;
}

// ---- fused attention: S = Q K^T, its element-wise chain, ggml.soft_max, O = P V ----------
//
// One workgroup per (batch, 32 query rows): S and then P stay in LDS, so the
// score matrix never goes through HBM.  Every value is the one the separate
// kernels give: S in ggml_vec_dot_f32 order, then the fused chain (the same
// IEEE operations; attn_chain_ops says where a NaN's payload may differ),
// each row through softmax_row16 or softmax_row (the soft_max kernel's
// decisions), and O in ggml order again.  Work whose result is fixed without
// it is skipped: softmax slices that are -inf on every row, and key tiles
// that a mask sets to -inf on all 32 rows (attn_skip_plan).
//
// The products run on v_mfma_f32_16x16x1_4b_f32 (K = 1: one fused
// multiply-add per output per instruction, as the 32x32 form): lane l
// supplies A and B of block l / 16, row / column l % 16, and block b's output
// (i, j) lands in lane j + 16 (i / 4), register 4 b + i % 4.  Lane l of block
// bl = l / 16 supplies the k-quad 16 blk + 4 bl .. + 3 and instruction g its
// component g, so block b of accumulator set g holds chain 4 b + g: an
// output's 16 chains are registers r, 4 + r, 8 + r, 12 + r (r = i % 4) of the
// four sets, in one lane, and ggml's tree needs no exchange (tree16).
typedef float v16f __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v16f mfma16(float a, float b, const v16f &c) {
  return __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, c, 0, 0, 0);
}

// dot_finish's GGML_F32x4_REDUCE and vaddvq_f32 on a lane's four outputs.
__device__ __forceinline__ void tree16(const v16f (&acc)[4], float (&out)[4]) {
#pragma unroll
  for (int r = 0; r < 4; r++) {
    float w[4];
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const float u = acc[g][r] + acc[g][8 + r];       // sum[0] += sum[2]
      const float v = acc[g][4 + r] + acc[g][12 + r];  // sum[1] += sum[3]
      w[g] = u + v;                                    // sum[0] += sum[1]
    }
    out[r] = (w[0] + w[1]) + (w[2] + w[3]);  // vaddvq_f32
  }
}

// The 16 instructions of one 16x16 tile over a k-range of 64 (four blocks),
// A and B float4 k-quads per block; the first block of a product starts from
// the inline +0 accumulator, as ggml's accumulators do.
__device__ __forceinline__ void mfma16_block(v16f (&acc)[4], const float4 &a, const float4 &b, bool first) {
  const v16f z = {};
  acc[0] = mfma16(a.x, b.x, first ? z : acc[0]);
  acc[1] = mfma16(a.y, b.y, first ? z : acc[1]);
  acc[2] = mfma16(a.z, b.z, first ? z : acc[2]);
  acc[3] = mfma16(a.w, b.w, first ? z : acc[3]);
}

constexpr int kAttnRows = 32;  // query rows per workgroup
constexpr int kAttnDh = 64;    // head dim (the Q K^T contraction)
constexpr int kAttnDv = 64;    // value columns

// J = keys / 256.  Q (b, n, d) and K (b, m, d) along d (16-byte aligned rows),
// V (b, m, e) along e; O [B, NQ, 64] contiguous.  A block is 32 query rows of
// one batch; its score tile S, then P, is 32 rows of NK + 4 floats in LDS
// (rows 4 floats apart: the writes spread over banks).  Three phases, each
// split over four waves w = 0 .. 3: S for key tiles w, w + 4, ... (both query
// tiles); the chain and softmax for eight of the rows; O for value columns
// 16 w .. 16 w + 15 (both query tiles).

// K and V load through buffer resources: one 32-bit per-lane byte offset for
// a whole phase, every per-tile and per-block advance in the scalar offset
// (each batch's K and V slices are below 2^31 bytes: the host checks).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t attn_rsrc(const MfmaOperand &o, int64_t b) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)(o.p + boff(o, b)), (short)0, 0x7FFFFFFF, 0x00020000);
}

// Phase one's operands: the block's Q rows (both query tiles) and the first
// key tile, loaded before the phase runs.
struct AttnQk {
  float4 qa[2][4];
  float4 ka[4];
};

__device__ __forceinline__ float4 attn_kload(const MfmaOperand &Kk, const __amdgpu_buffer_rsrc_t &kr, int wave,
                                             int kt, int blk) {
  const int lane = threadIdx.x & 63, bl = lane >> 4, li = lane & 15;
  const int kvo = (int)(((int64_t)(16 * wave + li) * Kk.sf + 4 * bl) * 4);
  return buf_ld4(BufOp{kr, kvo, nullptr}, (int)((int64_t)16 * (kt - wave) * Kk.sf * 4 + 64 * blk));
}

__device__ __forceinline__ void attn_qk_load(const MfmaOperand &Q, const MfmaOperand &Kk, int64_t b, int64_t n0,
                                             int wave, AttnQk &st) {
  const int lane = threadIdx.x & 63, bl = lane >> 4, li = lane & 15;
  const float *qb = Q.p + boff(Q, b);
#pragma unroll
  for (int qt = 0; qt < 2; qt++)
#pragma unroll
    for (int blk = 0; blk < 4; blk++) st.qa[qt][blk] = ld4(qb + (n0 + 16 * qt + li) * Q.sf + 16 * blk + 4 * bl);
  const __amdgpu_buffer_rsrc_t kr = attn_rsrc(Kk, b);
#pragma unroll
  for (int blk = 0; blk < 4; blk++) st.ka[blk] = attn_kload(Kk, kr, wave, wave, blk);
}

// The largest exponent field (bits 23..30) among a wave's values, the same
// on every lane.
__device__ __forceinline__ int wave_max_expfield(int v) {
  v = max(v, dpp_i<kDppXor1>(v));
  v = max(v, dpp_i<kDppXor2>(v));
  v = max(v, dpp_i<kDppHalfMirror>(v));
  v = max(v, dpp_i<kDppMirror>(v));
  v = max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
          max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
  return v >> 23;
}
__device__ __forceinline__ int expfield4(const float4 &x, int v) {
  v = max(v, (int)(f_bits(x.x) & 0x7F800000u));
  v = max(v, (int)(f_bits(x.y) & 0x7F800000u));
  v = max(v, (int)(f_bits(x.z) & 0x7F800000u));
  return max(v, (int)(f_bits(x.w) & 0x7F800000u));
}

// Masked key tiles (mskip = 1: the chain is one add of a row operand, the
// mask, shared by every batch; mskip = 2: a multiply by one scalar c, then
// that add).  attn_prep_k finds the masked tiles and K's largest exponents
// in a launch of its own before the kernel.  A key tile of
// 16 keys whose mask is -inf on all 32 rows of the block needs no products
// when Q, K (and c) are finite and small enough that no partial sum of a
// score can overflow: then every score S is finite, S c is finite, and the
// chain gives S (c) + -inf = -inf whatever S is, the same as from S = 0, which
// is written instead.  With |q| < 2^(eq+1) and |k| < 2^(ek+1) (exponents of
// the largest magnitudes) every partial sum of the 64 products, rounding
// included, stays below 2^(eq+ek+9), so eq + ek + 9 <= 127, or
// eq + ek + ec + 10 <= 127 with the multiply, keeps everything finite.
struct AttnSkip {
  uint32_t bits;  // bit i: the wave's tile w + 4 i is skipped
  uint32_t vbad;  // bit c: V may hold an infinite or NaN value among keys 64 c .. 64 c + 63
};

template <int J>
__device__ __forceinline__ AttnSkip attn_skip_plan(const Epilogue &e1, int mskip, const int *__restrict__ prep,
                                                   int64_t b, int64_t n0, int64_t NQ, int64_t B, int wave,
                                                   const AttnQk &st) {
  constexpr int NK = 256 * J, KT = NK / 16, NC = NK / 64;
  AttnSkip sk;
  sk.bits = 0;
  sk.vbad = ~0u;
  if (!mskip) return sk;
  // attn_prep_k's output: K's exponent fields per (batch, 64 keys), then per
  // (block of 32 rows, 64 keys) the masked-tile bits of its four key tiles.
  // Tile w + 4 i is tile w of chunk i.
  const int *mb = prep + B * NC + (n0 / kAttnRows) * NC;
#pragma unroll
  for (int i = 0; i < KT / 4; i++) sk.bits |= (uint32_t)((mb[i] >> wave) & 1) << i;
  int q = 0;
#pragma unroll
  for (int qt = 0; qt < 2; qt++)
#pragma unroll
    for (int blk = 0; blk < 4; blk++) q = expfield4(st.qa[qt][blk], q);
  const int qf = wave_max_expfield(q);
  const int cf = mskip == 2 ? (int)((f_bits(e1.op[0].p[0]) >> 23) & 0xFF) : 0;
  int kf = 0;
  sk.vbad = 0;
#pragma unroll
  for (int c = 0; c < NC; c++) {
    const int pk = prep[b * NC + c];
    kf = max(kf, pk & 0xFF);
    sk.vbad |= (uint32_t)((pk >> 8) & 1) << c;
  }
  // inf or NaN anywhere in Q, K or c (field 255), or a bound too large:
  // compute every tile
  if (qf == 255 || cf == 255 || kf == 255 || qf + kf + cf > (mskip == 2 ? 498 : 372)) sk.bits = 0;
  return sk;
}

// attn_skip_plan's inputs, one launch of B NC + (NQ / 32) NC workgroups
// (NC = NK / 64): the first B NC take the largest exponent field of K per
// (batch, 64 keys), with bit 8 set when V has an infinite or NaN value among
// those keys; the rest take a block of 32 mask rows (the mask is shared by
// every batch: s0 = 0) by 64 keys and set bit t of their int when the
// block's key tile 4 c + t is -inf on all 32 rows.  K rows and mask rows are
// 16-byte aligned (the host checks).
__global__ void __launch_bounds__(256) attn_prep_k(MfmaOperand Kk, MfmaOperand V, int NK, int64_t B,
                                                   const float *__restrict__ mask, int64_t ms1, int *__restrict__ out) {
  __shared__ int part[4], vpart[4];
  const int NC = NK / 64;
  const int64_t wg = blockIdx.x;
  int v = 0;
  if (wg < B * NC) {
    const int64_t bb = wg / NC, c = wg % NC;
    const float *kb = Kk.p + boff(Kk, bb) + 64 * c * Kk.sf;
    const float *vb = V.p + boff(V, bb) + 64 * c * V.sk;
    float4 kv[4];
    float vv[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {  // 64 keys x 16 float4s, four per thread
      const int g = threadIdx.x + 256 * i;
      kv[i] = ld4(kb + (int64_t)(g >> 4) * Kk.sf + 4 * (g & 15));
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {  // 64 keys x 64 values (unit stride along values), 16 per thread
      const int g = threadIdx.x + 256 * i;
      vv[i] = vb[(int64_t)(g >> 6) * V.sk + (g & 63)];
    }
#pragma unroll
    for (int i = 0; i < 4; i++) v = expfield4(kv[i], v);
    v = wave_max_expfield(v) << 23;
    int w = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) w = expfield4(make_float4(vv[4 * i], vv[4 * i + 1], vv[4 * i + 2], vv[4 * i + 3]), w);
    w = wave_max_expfield(w);
    if ((threadIdx.x & 63) == 0) vpart[threadIdx.x >> 6] = w;
  } else {
    // 32 rows x 16 float4s: two per thread, rows t / 16 and t / 16 + 16, key
    // quad t % 16 (tile (t % 16) / 4); the bits of tiles with an entry that
    // is not -inf, ORed over the workgroup
    const int64_t blk = (wg - B * NC) / NC, c = (wg - B * NC) % NC;
    const float *m = mask + (blk * kAttnRows + (threadIdx.x >> 4)) * ms1 + 64 * c + 4 * (threadIdx.x & 15);
    const float ninf = -__builtin_inff();
    const float4 x = ld4(m), y = ld4(m + 16 * ms1);
    const bool all = x.x == ninf && x.y == ninf && x.z == ninf && x.w == ninf && y.x == ninf && y.y == ninf &&
                     y.z == ninf && y.w == ninf;
    v = all ? 0 : 1 << ((threadIdx.x & 15) >> 2);
    v |= dpp_i<kDppXor1>(v);
    v |= dpp_i<kDppXor2>(v);
    v |= dpp_i<kDppHalfMirror>(v);
    v |= dpp_i<kDppMirror>(v);
    v = (__builtin_amdgcn_readlane(v, 0) | __builtin_amdgcn_readlane(v, 16)) |
        (__builtin_amdgcn_readlane(v, 32) | __builtin_amdgcn_readlane(v, 48));
  }
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    if (wg < B * NC) {
      const int vf = max(max(vpart[0], vpart[1]), max(vpart[2], vpart[3]));
      out[wg] = (max(max(part[0], part[1]), max(part[2], part[3])) >> 23) | (vf == 255 ? 0x100 : 0);
    } else {
      out[wg] = ~(part[0] | part[1] | part[2] | part[3]) & 15;
    }
  }
}

// Phase one: S = Q K^T in ggml order.  Key tiles in two register sets that
// take turns (a wave's KT / 4 tiles are an even count): one set's loads fly
// while the other's products run.
template <int J, bool SKIP>
__device__ __forceinline__ void attn_qk(const MfmaOperand &Kk, int64_t b, int wave, AttnQk &st, float *S,
                                        const AttnSkip &sk) {
  constexpr int NK = 256 * J, KT = NK / 16, LS = NK + 4;
  const int lane = threadIdx.x & 63, bl = lane >> 4, li = lane & 15;
  const __amdgpu_buffer_rsrc_t kr = attn_rsrc(Kk, b);
  // A skipped tile (masked on every row, the bound holding) loads nothing
  // and stores S = 0.  Without skipping (SKIP false) every load is
  // unconditional, so the wait before a tile's products counts the next
  // tile's loads as still in flight rather than waiting for them.
  auto skipped = [&](int kt) { return SKIP && ((sk.bits >> ((kt - wave) >> 2)) & 1u) != 0; };
  auto qk_tile = [&](const float4 (&ks)[4], int kt) {
    const int m = 16 * kt + li;
    if (skipped(kt)) {
#pragma unroll
      for (int qt = 0; qt < 2; qt++)
#pragma unroll
        for (int r = 0; r < 4; r++) S[(16 * qt + 4 * bl + r) * LS + m] = 0.0f;
      return;
    }
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
      v16f acc[4];
#pragma unroll
      for (int blk = 0; blk < 4; blk++) mfma16_block(acc, st.qa[qt][blk], ks[blk], blk == 0);
      float out[4];
      tree16(acc, out);
#pragma unroll
      for (int r = 0; r < 4; r++) S[(16 * qt + 4 * bl + r) * LS + m] = out[r];
    }
  };
  float4 kc[4];
#pragma unroll 1
  for (int kt = wave; kt < KT; kt += 8) {
    if (!skipped(kt + 4)) {
#pragma unroll
      for (int blk = 0; blk < 4; blk++) kc[blk] = attn_kload(Kk, kr, wave, kt + 4, blk);
    }
    qk_tile(st.ka, kt);
    const int kn = kt + 8 < KT ? kt + 8 : kt;  // past the end: reloads, in bounds
    if (!skipped(kn)) {
#pragma unroll
      for (int blk = 0; blk < 4; blk++) st.ka[blk] = attn_kload(Kk, kr, wave, kn, blk);
    }
    qk_tile(kc, kt + 4);
  }
}

// Phase two: the chain on S, then P = softmax(S), rows r0 .. r0 + nr - 1 in
// place, one row at a time over the wave.  The chain's ops (the same
// f32_binary, in order, per element) run here rather than after each product
// tile: a row's operands (a mask row) load as coalesced float4s, the next
// row's while this one is computed.  Operand r of a lane's row holds element
// 4 (lane + 64 (r / 4)) + r % 4.
template <int J, bool UNIT>
__device__ __forceinline__ void attn_rows(const Epilogue &e1, float sm_sc, int64_t b, int64_t n0, float *S, int r0,
                                          int nr) {
  constexpr int NK = 256 * J, LS = NK + 4;
  const int lane = threadIdx.x & 63;
  auto chain_off = [&](const EpiOp &o, int row, int r) {
    return b * o.s0 + (n0 + row) * o.s1 + (int64_t)(4 * (lane + kWave * (r / 4)) + r % 4) * o.s2;
  };
  auto chain_load = [&](int row, float (&w)[kEpiEarly][4 * J]) {
#pragma unroll
    for (int k = 0; k < kEpiEarly; k++) {
      if (k >= e1.n) break;
      const EpiOp &o = e1.op[k];
      if (o.s2 == 0) {  // one value over the row
        const float w0 = o.p[chain_off(o, row, 0)];
#pragma unroll
        for (int r = 0; r < 4 * J; r++) w[k][r] = w0;
      } else if (o.s2 == 1 && (((uintptr_t)(o.p + chain_off(o, row, 0))) & 15) == 0) {
#pragma unroll
        for (int j = 0; j < J; j++) {
          const float4 q = ld4(o.p + chain_off(o, row, 4 * j));
          w[k][4 * j] = q.x, w[k][4 * j + 1] = q.y, w[k][4 * j + 2] = q.z, w[k][4 * j + 3] = q.w;
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4 * J; r++) w[k][r] = o.p[chain_off(o, row, r)];
      }
    }
  };
  float wn[kEpiEarly][4 * J];
  chain_load(r0, wn);
#pragma unroll 1
  for (int rr = 0; rr < nr; rr++) {
    const int ri = r0 + rr;
    float *row = S + ri * LS;
    float wc[kEpiEarly][4 * J];
#pragma unroll
    for (int k = 0; k < kEpiEarly; k++)
#pragma unroll
      for (int r = 0; r < 4 * J; r++) wc[k][r] = wn[k][r];
    if (rr + 1 < nr) chain_load(ri + 1, wn);
    float v[4 * J];
#pragma unroll
    for (int j = 0; j < J; j++) {
      const float4 q = *reinterpret_cast<const float4 *>(row + 4 * (lane + kWave * j));
      v[4 * j] = q.x, v[4 * j + 1] = q.y, v[4 * j + 2] = q.z, v[4 * j + 3] = q.w;
    }
    epi_ops_n(e1, v, wc);
    epi_apply_n(e1, v, [&](const EpiOp &o, int r) { return chain_off(o, ri, r); }, kEpiEarly);
    float4 e[J];
#pragma unroll
    for (int j = 0; j < J; j++) e[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
    softmax_row<J, true, UNIT>(e, 64 * J, sm_sc, 0);
#pragma unroll
    for (int j = 0; j < J; j++) *reinterpret_cast<float4 *>(row + 4 * (lane + kWave * j)) = e[j];
  }
}

// The first kEpiEarly chain ops inside the fused kernel.  Add, subtract,
// multiply and divide run as the plain IEEE operation: only which operand's
// NaN comes out can differ from f32_binary, never whether the result is NaN,
// and a NaN anywhere in a row makes that softmax row, and so its rows of P
// and O, NaN in the separate kernels and here alike.  Maximum and minimum
// decide NaN-ness by their NaN rule, so they keep f32_binary.
// w[k] holds op k's operand for each element of the lane's row, or, when it
// is one value along the row (s2 = 0), wu[k] holds that value.
template <int NV>
__device__ __forceinline__ void attn_chain_op(const EpiOp &o, float (&v)[NV], const float (&w)[NV]) {
  switch (o.code) {
    case kAdd:
#pragma unroll
      for (int r = 0; r < NV; r++) v[r] = v[r] + w[r];
      break;
    case kMul:
#pragma unroll
      for (int r = 0; r < NV; r++) v[r] = v[r] * w[r];
      break;
    case kSub:
      if (o.rev) {
#pragma unroll
        for (int r = 0; r < NV; r++) v[r] = w[r] - v[r];
      } else {
#pragma unroll
        for (int r = 0; r < NV; r++) v[r] = v[r] - w[r];
      }
      break;
    case kDiv:
      if (o.rev) {
#pragma unroll
        for (int r = 0; r < NV; r++) v[r] = w[r] / v[r];
      } else {
#pragma unroll
        for (int r = 0; r < NV; r++) v[r] = v[r] / w[r];
      }
      break;
    case kMax: epi_op<kMax>(v, w, o.rev); break;
    case kMin: epi_op<kMin>(v, w, o.rev); break;
    default: break;
  }
}

template <int NV>
__device__ __forceinline__ void attn_chain_ops(const Epilogue &e, float (&v)[NV], const float (&w)[kEpiEarly][NV],
                                               const float (&wu)[kEpiEarly]) {
#pragma unroll
  for (int k = 0; k < kEpiEarly; k++) {
    if (k >= e.n) break;
    const EpiOp &o = e.op[k];
    if (o.s2 == 0) {
      float t[NV];
#pragma unroll
      for (int r = 0; r < NV; r++) t[r] = wu[k];
      attn_chain_op(o, v, t);
    } else {
      attn_chain_op(o, v, w[k]);
    }
  }
}

// Phase two for keys 256 and 512: rows r0 .. r0 + 7 as two passes of four
// 16-lane rows (softmax_row16), the second pass's chain operands loaded while
// the first pass's softmax runs.  Operand r of a lane's row holds element
// 4 (i + 16 (r / 4)) + r % 4 (i = lane % 16); an operand constant along the
// row (s2 = 0) is one load.  Returns the 64-key slices whose P is +0 on all
// eight rows (bit j: keys 64 j .. 64 j + 63).
// Offset of operand value r of a lane's row (lane l: i = l % 16) in op o's
// operand.  The element stride goes through an empty asm: left visible, the
// compiler hoists all NV element offsets of the (rare) strided operands out
// of the pass code and spills them.
__device__ __forceinline__ int64_t attn_chain_off(const EpiOp &o, int64_t b, int64_t n0, int row, int r) {
  const int li = threadIdx.x & 15;
  int64_t s2 = o.s2;
  asm volatile("" : "+s"(s2));
  return b * o.s0 + (n0 + row) * o.s1 + (int64_t)(4 * (li + 16 * (r / 4)) + r % 4) * s2;
}

// The chain operands of one 16-lane row pass (see attn_chain_ops).
template <int J>
__device__ __forceinline__ void attn_chain_load16(const Epilogue &e1, int64_t b, int64_t n0, int row,
                                                  float (&w)[kEpiEarly][16 * J], float (&wu)[kEpiEarly]) {
  constexpr int NJ = 4 * J, NV = 4 * NJ;
  const int li = threadIdx.x & 15;
#pragma unroll
  for (int k = 0; k < kEpiEarly; k++) {
    if (k >= e1.n) break;
    const EpiOp &o = e1.op[k];
    const float *p = o.p + b * o.s0 + (n0 + row) * o.s1;
    if (o.s2 == 0) {
      wu[k] = *p;
    } else if (o.s2 == 1 && ((uintptr_t)p & 15) == 0) {
#pragma unroll
      for (int j = 0; j < NJ; j++) {
        const float4 f = ld4(p + 4 * (li + 16 * j));
        w[k][4 * j] = f.x, w[k][4 * j + 1] = f.y, w[k][4 * j + 2] = f.z, w[k][4 * j + 3] = f.w;
      }
    } else {
#pragma unroll
      for (int r = 0; r < NV; r++) w[k][r] = o.p[attn_chain_off(o, b, n0, row, r)];
    }
  }
}

// Called before the barrier that ends phase one: the first pass's operands
// load first, and their wait overlaps the barrier's.
template <int J, bool UNIT>
__device__ __forceinline__ uint32_t attn_rows16(const Epilogue &e1, float sm_sc, int64_t b, int64_t n0, float *S,
                                                int r0) {
  constexpr int NK = 256 * J, LS = NK + 4, NJ = 4 * J, NV = 4 * NJ;
  const int lane = threadIdx.x & 63, q = lane >> 4, li = lane & 15;
  float wa[kEpiEarly][NV], wua[kEpiEarly], wb[kEpiEarly][NV], wub[kEpiEarly];
  attn_chain_load16<J>(e1, b, n0, r0 + q, wa, wua);
  __syncthreads();
  auto pass = [&](int ps, const float (&w)[kEpiEarly][NV], const float (&wu)[kEpiEarly])
                  __attribute__((always_inline)) {
    const int row = r0 + 4 * ps + q;
    float *rp = S + row * LS;
    float v[NV];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const float4 f = *reinterpret_cast<const float4 *>(rp + 4 * (li + 16 * j));
      v[4 * j] = f.x, v[4 * j + 1] = f.y, v[4 * j + 2] = f.z, v[4 * j + 3] = f.w;
    }
    attn_chain_ops(e1, v, w, wu);
    if (ps == 0) attn_chain_load16<J>(e1, b, n0, r0 + 4 + q, wb, wub);  // loads under this pass's softmax
    epi_apply_n(e1, v, [&](const EpiOp &o, int r) { return attn_chain_off(o, b, n0, row, r); }, kEpiEarly);
    float4 e[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) e[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
    const uint32_t zero = softmax_row16<NJ, UNIT>(e, sm_sc, rp);
#pragma unroll
    for (int j = 0; j < NJ; j++) *reinterpret_cast<float4 *>(rp + 4 * (li + 16 * j)) = e[j];
    return zero;
  };
  // Each pass has its own operand registers and both passes are inlined, so
  // the second pass's operands need no copy between the passes.
  const uint32_t z0 = pass(0, wa, wua);
  return z0 & pass(1, wb, wub);
}

// V's operands for phase three: lane l (bl = l / 16, li = l % 16) of wave w
// takes keys 16 blk + 4 bl + g (g < 4) of value column 16 w + li, through a
// buffer resource (one per-lane offset per g, the block in the scalar offset).
struct AttnVLoad {
  __amdgpu_buffer_rsrc_t r;
  int vo[4];
  int vstep;
  __device__ AttnVLoad(const MfmaOperand &V, int64_t b, int wave) : r(attn_rsrc(V, b)) {
    const int lane = threadIdx.x & 63, bl = lane >> 4, li = lane & 15;
#pragma unroll
    for (int g = 0; g < 4; g++) vo[g] = (int)(((int64_t)(16 * wave + li) * V.sf + (int64_t)(4 * bl + g) * V.sk) * 4);
    vstep = (int)((int64_t)16 * V.sk * 4);  // one block of 16 keys
  }
  __device__ float4 operator()(int blk) const {
    float x[4];
#pragma unroll
    for (int g = 0; g < 4; g++) x[g] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, vo[g], blk * vstep, 0));
    return make_float4(x[0], x[1], x[2], x[3]);
  }
};

// Phase three: O = P V in ggml order, then the chain after it, stored.  V's
// operands load four blocks ahead of their products, in two register sets
// that take turns: the loads of one set fly while the other feeds the MFMAs,
// and no register moves between them.
//
// The products run over the first nzb blocks of 16 keys (a multiple of 4,
// at least 4).  The blocks after them have P = +0 on all 32 rows (a causal
// mask's upper part) and finite V (the caller checks both): each of their
// products adds +0 * v = +-0 to a chain, which leaves the chain's value
// unchanged, bit for bit, unless the chain is -0 (-0 + +0 = +0).  If any of
// the wave's chains is -0 the remaining products run as well, in order.
template <int J>
__device__ __forceinline__ void attn_pv(const MfmaOperand &V, int64_t b, int64_t n0, int64_t NQ, int wave,
                                        const float *S, const uint32_t *zs, uint32_t vbad, const Epilogue &e2,
                                        float *__restrict__ O) {
  constexpr int NK = 256 * J, LS = NK + 4, NB = NK / 16;
  const int lane = threadIdx.x & 63, bl = lane >> 4, li = lane & 15;
  const AttnVLoad vl(V, b, wave);
  auto vload = [&](int blk) { return vl(blk); };
  // Called before the barrier that ends phase two: the first V blocks load
  // first (eight in two sets of four; for 256 keys four in two sets of two,
  // which keeps the kernel within three workgroups' registers per CU).  A
  // second set goes unused when the products stop after the first.
  constexpr int VS = J >= 2 ? 4 : 2;  // V blocks per register set
  float4 va[VS], vb[VS];
#pragma unroll
  for (int i = 0; i < VS; i++) va[i] = vload(i);
#pragma unroll
  for (int i = 0; i < VS; i++) vb[i] = vload(VS + i);
  __syncthreads();
  // Products run up to the last slice with a nonzero P on any of the 32 rows,
  // when V is finite on the slices after it (else over all keys).
  const uint32_t live = ~(zs[0] & zs[1] & zs[2] & zs[3]) & ((1u << (NK / 64)) - 1);
  int nzb = live ? 4 * (32 - __builtin_clz(live)) : 4;
  if (vbad >> (nzb / 4)) nzb = NB;
  auto pload = [&](int qt, int blk) {
    return *reinterpret_cast<const float4 *>(S + (16 * qt + li) * LS + 16 * blk + 4 * bl);
  };
  v16f acc[2][4];
  if constexpr (J >= 2) {
    // Block 0 starts the accumulators from the inline +0 (first).
    auto pv4 = [&](const float4 (&vs)[4], const float4 (&ps)[4][2], bool first) {
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int qt = 0; qt < 2; qt++) mfma16_block(acc[qt], ps[i][qt], vs[i], first && i == 0);
    };
    auto pl4 = [&](float4 (&ps)[4][2], int blk0) {
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int qt = 0; qt < 2; qt++) ps[i][qt] = pload(qt, min(blk0 + i, nzb - 1));
    };
    float4 pa[4][2], pb[4][2];
    pl4(pa, 0);
    pl4(pb, 4);
    pv4(va, pa, true);
#pragma unroll 1
    for (int b0 = 4; b0 < nzb; b0 += 8) {  // vb, pb hold blocks b0 .. b0 + 3
#pragma unroll
      for (int i = 0; i < 4; i++) va[i] = vload(min(b0 + 4 + i, nzb - 1));
      pl4(pa, b0 + 4);
      __builtin_amdgcn_sched_barrier(0);
      pv4(vb, pb, false);
      __builtin_amdgcn_sched_barrier(0);
      if (b0 + 4 >= nzb) break;
#pragma unroll
      for (int i = 0; i < 4; i++) vb[i] = vload(min(b0 + 8 + i, nzb - 1));
      pl4(pb, b0 + 8);
      __builtin_amdgcn_sched_barrier(0);
      pv4(va, pa, false);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    // Sets of VS = 2 blocks, in block order; block 0 starts the accumulators
    // from the inline +0 (first).  nzb is a multiple of 4, so the sets end on
    // it; loads past it reload block nzb - 1 (in range, unused).
    auto pvs = [&](const float4 (&vs)[VS], int blk0, bool first) {
#pragma unroll
      for (int i = 0; i < VS; i++)
#pragma unroll
        for (int qt = 0; qt < 2; qt++) mfma16_block(acc[qt], pload(qt, blk0 + i), vs[i], first && i == 0);
    };
    pvs(va, 0, true);
#pragma unroll 1
    for (int b0 = VS; b0 < nzb; b0 += 2 * VS) {  // vb holds blocks b0 .. b0 + VS - 1
#pragma unroll
      for (int i = 0; i < VS; i++) va[i] = vload(min(b0 + VS + i, nzb - 1));
      pvs(vb, b0, false);
      if (b0 + VS >= nzb) break;
#pragma unroll
      for (int i = 0; i < VS; i++) vb[i] = vload(min(b0 + 2 * VS + i, nzb - 1));
      pvs(va, b0 + VS, false);
    }
  }
  if (nzb < NB) {
    bool neg0 = false;
#pragma unroll
    for (int qt = 0; qt < 2; qt++)
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) neg0 |= __builtin_amdgcn_classf(acc[qt][i][r], 32);  // -0
    if (__any(neg0)) {
#pragma unroll 1
      for (int blk = nzb; blk < NB; blk++) {
        const float4 v = vload(blk);
#pragma unroll
        for (int qt = 0; qt < 2; qt++) mfma16_block(acc[qt], pload(qt, blk), v, false);
      }
    }
  }
  const int64_t d = 16 * wave + li;
#pragma unroll
  for (int qt = 0; qt < 2; qt++) {
    float out[4];
    tree16(acc[qt], out);
    const int64_t nq = n0 + 16 * qt + 4 * bl;
    if (e2.n > 0)
      epi_apply_n(e2, out, [&](const EpiOp &o, int r) { return b * o.s0 + (nq + r) * o.s1 + d * o.s2; }, 0,
                  NoUnary(), DotUniform<true>());
    float *y = O + (b * NQ + nq) * kAttnDv + d;
#pragma unroll
    for (int r = 0; r < 4; r++) y[r * kAttnDv] = out[r];
  }
}

// One workgroup of four waves per block, the phases in turn.  Consecutive
// query blocks of one batch share K and V: each XCD takes a contiguous run of
// workgroups (whole batches), whose K and V stay in its L2.  The register
// budget follows the workgroups per CU that the scores' LDS allows, up to
// three: 256 keys (33 KB) three, 512 keys (66 KB) two, 768 or 1024 keys (99
// or 132 KB) one.
template <int J, bool UNIT, bool SKIP>
__global__ void __launch_bounds__(256, J == 1 ? 3 : J == 2 ? 2 : 1)
    attention_k(MfmaOperand Q, MfmaOperand Kk, MfmaOperand V, int64_t NQ, Epilogue e1, int mskip,
                const int *__restrict__ prep, float sm_sc, Epilogue e2, float *__restrict__ O) {
  constexpr int NK = 256 * J, LS = NK + 4;
  __shared__ __attribute__((aligned(16))) float S[kAttnRows * LS];
  __shared__ uint32_t zs[4];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // an SGPR
  uint32_t tx = blockIdx.x, ty = blockIdx.y;
  if (SKIP) {
    // Masked tiles make blocks unequal (a causal mask leaves the first query
    // blocks the least work).  Blocks are ranked h = 0 (heaviest: the last
    // query block of every batch) .. nb - 1, and dispatched so that the two
    // workgroups a CU starts with are a heavy and a light one: ids 0 .. 255
    // (one per CU of the 256) take the heaviest ranks, ids 256 .. 511 (each
    // CU's second) the lightest, the rest the middle ranks, heaviest first.
    // A heavy block's waves wait on their own dependences as much as they
    // issue, and a light block fills those gaps, where two light blocks
    // together would leave the CU mostly idle.  Consecutive ranks walk the
    // batches.  The lightest ranks go in reverse order within each aligned
    // run of 8 ids, which keeps every id's rank congruent to the id mod 8
    // (C is a multiple of 8; so is nb whenever the batch count is): XCD x,
    // which takes the ids = x mod 8, then computes only batches = x mod 8
    // (for a batch count that is a multiple of 8), and their K and V stay in
    // its L2.  Every mapping here is a bijection on the grid.
    const uint32_t lin = blockIdx.x + gridDim.x * blockIdx.y;
    const uint32_t nb = gridDim.x * gridDim.y, C = 256;
    uint32_t h = lin;
    if (nb >= 2 * C) h = lin < C ? lin : lin < 2 * C ? nb - 1 - ((lin - C) ^ 7u) : lin - C;
    ty = h % gridDim.y;
    tx = gridDim.x - 1 - h / gridDim.y;
  } else if (gridDim.y > 1) {
    xcd_tile(tx, ty);
  }
  const int64_t b = ty, n0 = (int64_t)tx * kAttnRows;
  AttnQk st;
  attn_qk_load(Q, Kk, b, n0, wave, st);
  const AttnSkip sk = attn_skip_plan<J>(e1, mskip, prep, b, n0, NQ, gridDim.y, wave, st);
  attn_qk<J, SKIP>(Kk, b, wave, st, S, sk);
  // Global loads issued before a barrier stay in flight across it: phases
  // two and three each start their first loads, then wait at the barrier
  // for the other waves to finish the phase before.
  uint32_t zero = 0;  // 64-key slices whose P is +0 on this wave's rows
  if constexpr (J <= 2) {
    zero = attn_rows16<J, UNIT>(e1, sm_sc, b, n0, S, 8 * wave);
  } else {
    __syncthreads();
    attn_rows<J, UNIT>(e1, sm_sc, b, n0, S, 8 * wave, 8);
  }
  if ((threadIdx.x & 63) == 0) zs[wave] = zero;
  attn_pv<J>(V, b, n0, NQ, wave, S, zs, sk.vbad, e2, O);
}

// ---- rows longer than 4096 columns -------------------------------------------------
//
// A row that does not fit one wave's registers is streamed: each lane takes
// the four-element groups g = lane + 64 j (j = 0 .. J - 1, J = ceil(G / 64))
// in passes over global memory.  The in-order binary64 sums are decided as
// in ordered_sum_apply, with the interval re-derived for n terms: the
// in-order chain S lies within (n - 1) 2^-53 of the exact total and the tree
// sum T (a lane's serial sum of J parts and one tail value, then six
// butterfly levels) within (J + 7) 2^-53, so S lies in T (1 -+ delta) with
// delta = (n + J + 8) 2^-52, twice their sum; f(T (1 - delta)) == f(T (1 +
// delta)) fixes f(S).  The exactness test holds unchanged: T falls short of
// the exact total by a relative (J + 7) 2^-53 < 2^-20 for any row below 2^31
// columns.  The walk takes the parts again, in group order, from `part_at`.
template <class PartAt, class Fin>
__device__ float ordered_sum_long(double ls, int le, int G, float tail, int T, PartAt part_at, Fin fin) {
  const int lane = threadIdx.x % kWave;
  if (lane < T) {
    ls = ls + (double)tail;
    le = min(le, part_ulp_exp(tail));
  }
  ls = wave_sum_d(ls);
  le = wave_min_i(le);
  if (ls <= exact_limit(le)) return fin(ls);
  const int J = (G + kWave - 1) / kWave;
  const double d = ls * ((double)(G + T + J + 8) * 0x1p-52);
  const float f_lo = fin(ls - d), f_hi = fin(ls + d);
  if (f_lo == f_hi) return f_lo;  // false for NaN and infinity
  double s = 0.0;
  for (int j = 0; j < J; j++) {
    const int g = kWave * j + lane;
    const float p = g < G ? part_at(g) : 0.0f;
    const double seg = row16_sum((double)p);
    const int sege = row16_min(part_ulp_exp(p));
#pragma unroll
    for (int r = 0; r < 4; r++) {
      if (kWave * j + 16 * r >= G) break;
      const double t = s + lane_d(seg, 16 * r);
      const double lim_p = exact_limit(__builtin_amdgcn_readlane(sege, 16 * r));
      const uint32_t hs = (uint32_t)(__builtin_bit_cast(uint64_t, s) >> 32);
      const double lim_s = __builtin_bit_cast(double, (uint64_t)((hs & 0xFFF00000u) | 0x000FFFFEu) << 32);
      if (t <= lim_p && (s == 0.0 || t <= lim_s)) {
        s = t;
      } else {
        const int n = min(16, G - (kWave * j + 16 * r));
#pragma unroll 1
        for (int i = 0; i < n; i++) s = s + (double)lane_f(p, 16 * r + i);
      }
    }
  }
  for (int l = 0; l < T; l++) s = s + (double)lane_f(tail, l);
  return fin(s);
}

// Group g of a row (four elements from p + 4 g): a float4 load when rows are
// 16-byte aligned (cols % 4 == 0), else four scalar loads.
template <bool ALIGNED>
__device__ __forceinline__ float4 row_group(const float *p, int g) {
  if (ALIGNED) return ld4(p + 4 * (int64_t)g);
  const float *q = p + 4 * (int64_t)g;
  return make_float4(q[0], q[1], q[2], q[3]);
}
template <bool ALIGNED>
__device__ __forceinline__ void row_group_st(float *p, int g, float4 v) {
  if (ALIGNED) {
    st4(p + 4 * (int64_t)g, v);
    return;
  }
  float *q = p + 4 * (int64_t)g;
  q[0] = v.x, q[1] = v.y, q[2] = v.z, q[3] = v.w;
}

// ggml soft_max on rows of any length (Shaders.lean:100-123), one wave per
// row: pass 1 the maximum of x*sc; pass 2 e = ggml_v_expf(x*sc - mx) stored
// to y (as ggml does) with each group's vaddvq_f32 part summed per lane, the
// row tail (pinned flavour) through the correctly rounded expf; the
// denominator decided by ordered_sum_long, whose walk re-reads e from y (each
// lane reads back only the groups it wrote); pass 3 y *= inv.
template <bool ALIGNED>
__global__ void __launch_bounds__(256) soft_max_long_k(int64_t rows, int cols, float sc, int float_sum,
                                                       const float *__restrict__ X, float *__restrict__ Y) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int G = cols / 4, T = cols % 4;
  const int64_t row = blockIdx.x * 4LL + wave;
  if (row >= rows) return;  // the whole wave; no barrier follows
  const float *x = X + row * cols;
  float *y = Y + row * cols;
  float mx = -__builtin_inff();
  for (int g = lane; g < G; g += kWave) {
    const float4 v = row_group<ALIGNED>(x, g);
    mx = __builtin_fmaxf(mx, __builtin_fmaxf(__builtin_fmaxf(v.x * sc, v.y * sc),
                                             __builtin_fmaxf(v.z * sc, v.w * sc)));
  }
  if (lane < T) mx = __builtin_fmaxf(mx, x[4 * G + lane] * sc);
  mx = wave_max_f(mx);
  double ls = 0.0;
  int le = 255;
  auto part_of = [](float4 e) { return (e.x + e.y) + (e.z + e.w); };
  for (int g = lane; g < G; g += kWave) {
    const float4 v = row_group<ALIGNED>(x, g);
    const float4 e = make_float4(ggml_v_expf(v.x * sc - mx), ggml_v_expf(v.y * sc - mx),
                                 ggml_v_expf(v.z * sc - mx), ggml_v_expf(v.w * sc - mx));
    row_group_st<ALIGNED>(y, g, e);
    const float p = part_of(e);
    ls = ls + (double)p;
    le = min(le, part_ulp_exp(p));
  }
  float et = 0.0f;
  if (lane < T) {
    et = expfk::expf_cr(x[4 * G + lane] * sc - mx);
    y[4 * G + lane] = et;
  }
  auto part_at = [&](int g) { return part_of(row_group<ALIGNED>(y, g)); };
  float inv;
  if (float_sum) {  // planted: the denominator summed in binary32 in group order (Shaders.lean:120-122)
    float fs = 0.0f;
    const int J = (G + kWave - 1) / kWave;
    for (int j = 0; j < J; j++) {
      const int g = kWave * j + lane;
      const float p = g < G ? part_at(g) : 0.0f;
      const int n = min(kWave, G - kWave * j);
      for (int l = 0; l < n; l++) fs = fs + lane_f(p, l);
    }
    for (int l = 0; l < T; l++) fs = fs + lane_f(et, l);
    inv = 1.0f / fs;
  } else {
    inv = ordered_sum_long(ls, le, G, et, T, part_at, [](double v) { return (float)(1.0 / v); });
  }
  for (int g = lane; g < G; g += kWave) {
    const float4 e = row_group<ALIGNED>(y, g);
    row_group_st<ALIGNED>(y, g, make_float4(e.x * inv, e.y * inv, e.z * inv, e.w * inv));
  }
  if (lane < T) y[4 * G + lane] = et * inv;
}

// ggml norm on rows of any length (Shaders.lean:130-166), one wave per row:
// pass 1 the mean's binary64 sum (decided as in norm_rows_k, the walk
// re-reading x 64 elements at a time); pass 2 the variance's group parts of
// q = (x - mean)^2, decided by ordered_sum_long (the walk recomputes them
// from x); pass 3 y = (x - mean) * scale.
template <bool ALIGNED>
__global__ void __launch_bounds__(256) norm_long_k(int64_t rows, int cols, float eps, const float *__restrict__ X,
                                                   float *__restrict__ Y) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int G = cols / 4, T = cols - 4 * G;
  const int J = (G + kWave - 1) / kWave;
  const int64_t row = blockIdx.x * 4LL + wave;
  if (row >= rows) return;  // the whole wave; no barrier follows
  const float *x = X + row * cols;
  float *y = Y + row * cols;
  double ls = 0.0, la = 0.0;
  int le = 255;
  auto take = [&](float v) {
    ls = ls + (double)v;
    la = la + (double)__builtin_fabsf(v);
    le = min(le, part_ulp_exp(v));
  };
  for (int g = lane; g < G; g += kWave) {
    const float4 v = row_group<ALIGNED>(x, g);
    take(v.x);
    take(v.y);
    take(v.z);
    take(v.w);
  }
  const float et = lane < T ? x[4 * G + lane] : 0.0f;
  take(et);
  ls = wave_sum_d(ls);
  la = wave_sum_d(la);
  le = wave_min_i(le);
  const float fc = (float)cols;
  float mean;
  if (la <= exact_limit(le)) {
    mean = (float)ls / fc;
  } else {
    const double d = la * ((double)(cols + 4 * J + 8) * 0x1p-52);
    const float lo = (float)(ls - d) / fc, hi = (float)(ls + d) / fc;
    if (lo == hi) {  // false for NaN
      mean = lo;
    } else {
      double s = 0.0;
      for (int j = 0; j < J; j++) {
        const int g = kWave * j + lane;
        const float4 q = g < G ? row_group<ALIGNED>(x, g) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const double seg = row16_sum(((double)q.x + (double)q.y) + ((double)q.z + (double)q.w));
        const double sega = row16_sum(((double)__builtin_fabsf(q.x) + (double)__builtin_fabsf(q.y)) +
                                      ((double)__builtin_fabsf(q.z) + (double)__builtin_fabsf(q.w)));
        const int sege = row16_min(min(min(part_ulp_exp(q.x), part_ulp_exp(q.y)),
                                       min(part_ulp_exp(q.z), part_ulp_exp(q.w))));
#pragma unroll
        for (int r = 0; r < 4; r++) {
          if (kWave * j + 16 * r >= G) break;
          const int e_min = min(__builtin_amdgcn_readlane(sege, 16 * r), low_bit_exp(s));
          if (__builtin_fabs(s) + lane_d(sega, 16 * r) <= exact_limit(e_min)) {
            s = s + lane_d(seg, 16 * r);
          } else {
            const int n = min(16, G - (kWave * j + 16 * r));
#pragma unroll 1
            for (int i = 16 * r; i < 16 * r + n; i++) {
              s = s + (double)lane_f(q.x, i);
              s = s + (double)lane_f(q.y, i);
              s = s + (double)lane_f(q.z, i);
              s = s + (double)lane_f(q.w, i);
            }
          }
        }
      }
      for (int l = 0; l < T; l++) s = s + (double)lane_f(et, l);
      mean = (float)s / fc;
    }
  }
  auto part_at = [&](int g) {
    const float4 v = row_group<ALIGNED>(x, g);
    const float d0 = v.x - mean, d1 = v.y - mean, d2 = v.z - mean, d3 = v.w - mean;
    return (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
  };
  double vs = 0.0;
  int ve = 255;
  for (int g = lane; g < G; g += kWave) {
    const float p = part_at(g);
    vs = vs + (double)p;
    ve = min(ve, part_ulp_exp(p));
  }
  const float dt = et - mean, qt = dt * dt;
  const double dc = (double)cols;
  const float var = ordered_sum_long(vs, ve, G, qt, T, part_at, [dc](double v) { return (float)(v / dc); });
  const float scl = 1.0f / sqrtf(var + eps);
  for (int g = lane; g < G; g += kWave) {
    const float4 v = row_group<ALIGNED>(x, g);
    row_group_st<ALIGNED>(y, g, make_float4((v.x - mean) * scl, (v.y - mean) * scl, (v.z - mean) * scl,
                                            (v.w - mean) * scl));
  }
  if (lane < T) y[4 * G + lane] = dt * scl;
}

int env_int(const char *name, int dflt) {
  const char *s = getenv(name);
  return s ? atoi(s) : dflt;
}

// ---- norm ---------------------------------------------------------------------------

// The planted norm (Shaders.lean:137-146: binary32 sums and the GPU's own
// approximate reciprocal and square root): one wave per row, the sequential
// sums on lane 0 reading the row from global memory (rows of any length).
__global__ void __launch_bounds__(256) norm_planted_k(int64_t rows, int cols, float eps,
                                                      const float *__restrict__ X, float *__restrict__ Y) {
  const int waves = blockDim.x / kWave;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  for (int64_t row = blockIdx.x * (int64_t)waves + wave; row < rows; row += (int64_t)gridDim.x * waves) {
    const float *x = X + row * cols;
    const float *xr = x;
    float *y = Y + row * cols;
    float mean = 0.0f, scl = 0.0f;
    if (lane == 0) {
      float s = 0.0f;
      for (int i = 0; i < cols; i++) s = s + xr[i];
      mean = s / (float)cols;
      float s2 = 0.0f;
      for (int i = 0; i < cols; i++) {
        const float d = xr[i] - mean;
        s2 = s2 + d * d;
      }
      scl = __builtin_amdgcn_rcpf(__builtin_amdgcn_sqrtf(s2 / (float)cols + eps));
    }
    mean = __shfl(mean, 0, kWave);
    scl = __shfl(scl, 0, kWave);
    for (int i = lane; i < cols; i += kWave) y[i] = (xr[i] - mean) * scl;
  }
}

// ggml norm, one wave per row (rows of at most 4096 columns): lane l holds the
// four-element groups g = l + 64 j as float4 and, on lanes < cols % 4, one
// tail element.  Both binary64 sums of Shaders.lean:130-166 are taken in
// ggml's order only where the order can matter:
// * The mean's sum of the elements x_i (any signs).  Every x_i is a multiple
//   of u, the smallest ulp among the nonzero x_i, and every partial sum in any
//   order is bounded by A = sum |x_i|: if A < 2^53 u, no addition rounds and
//   the in-order chain equals a tree sum.  A wave computes the tree sum t, the
//   tree sum a of |x_i| and u, and takes a <= (1 - 2^-20) 2^53 u as the test
//   (the softmax argument, on |x_i|).  Otherwise the chain lies within
//   (cols - 1) 2^-53 A of the exact sum (cols - 1 additions, each rounding
//   by at most 2^-53 of a partial sum bounded by A) and t within
//   (4 J + 7) 2^-53 A (a lane's serial sum, then six butterfly levels), so
//   mean = (float)s / cols, monotone in s, is fixed when it agrees at
//   t -+ a (cols + 4 J + 8) 2^-52, twice that bound.  A row that fails both
//   (a NaN, an infinity, or a mean within about cols 2^-52 A of a rounding
//   boundary) adds its elements in order, 64 at a time where no addition in
//   them can round.
// * The variance's sum of the group parts (q0 + q1) + (q2 + q3) of
//   q = (x - mean)^2 and the tail's q, all >= 0: ordered_sum_apply with
//   f(S) = (float)(S / cols).
// Then scale = 1 / sqrtf(var + eps) and y = (x - mean) * scale, followed (EPI)
// by the fused element-wise ops at index (0, row, column).
template <int J, bool FULL, bool EPI>
__global__ void __launch_bounds__(256) norm_rows_k(int64_t rows, int cols, float eps, Epilogue ep,
                                                   const float *__restrict__ X, float *__restrict__ Y) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int G = cols / 4, T = cols - 4 * G;
  const int64_t row = blockIdx.x * 4LL + wave;
  if (row >= rows) return;  // the whole wave; no barrier follows
  const float *x = X + row * cols;
  float4 e[J];
#pragma unroll
  for (int j = 0; j < J; j++) {  // rows start 16-byte aligned only when cols % 4 == 0
    const int g = lane + kWave * j;
    const float *p = x + 4 * g;
    e[j] = (FULL || g < G) ? (T == 0 ? ld4(p) : make_float4(p[0], p[1], p[2], p[3]))
                           : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  const float et = lane < T ? x[4 * G + lane] : 0.0f;
  // The fused ops' operands do not depend on the row's sums.  For rows of
  // more than 512 columns their loads go out now and land under the
  // reductions; for 512 and fewer they go out after the sums (LATE): held
  // through the reductions, their registers would keep the kernel above 64,
  // the budget at which all eight waves per SIMD of a [8192, 512] row set
  // are resident at once.
  constexpr bool LATE = J <= 2;
  float w[kEpiEarly][4 * J], wt[kEpiEarly][1];  // the first kEpiEarly ops' operands; later ops load at the end
  auto load_ops = [&]() {
    if (EPI) {
      // An operand along columns with unit stride from a 16-byte aligned start
      // (LayerNorm's gain and bias) loads float4 groups, as the row does;
      // any other, one element at a time.
#pragma unroll
      for (int k = 0; k < kEpiEarly; k++) {
        if (k >= ep.n) break;
        const EpiOp &o = ep.op[k];
        if (o.code == kEpiGeluErf) continue;
        const float *base = o.p + row * o.s1;
        if (o.s2 == 1 && T == 0 && ((uintptr_t)base & 15) == 0) {
#pragma unroll
          for (int j = 0; j < J; j++) {
            const int g = lane + kWave * j;
            const float4 q = ld4(base + 4 * ((FULL || g < G) ? g : 0));  // a discarded group reads group 0
            w[k][4 * j] = q.x, w[k][4 * j + 1] = q.y, w[k][4 * j + 2] = q.z, w[k][4 * j + 3] = q.w;
          }
        } else {
#pragma unroll
          for (int r = 0; r < 4 * J; r++) {
            const int g = lane + kWave * (r / 4);
            const int c = (FULL || g < G) ? 4 * g + r % 4 : 0;  // a discarded group reads column 0
            w[k][r] = o.p[row * o.s1 + c * o.s2];
          }
        }
      }
      if (T > 0)
        epi_load_n(ep, wt, [&](const EpiOp &o, int) { return row * o.s1 + (lane < T ? 4 * G + lane : 0) * o.s2; });
    }
  };
  if (!LATE) load_ops();
  double ls = 0.0, la = 0.0;
  int le = 255;
  auto take = [&](float v) {
    ls = ls + (double)v;
    la = la + (double)__builtin_fabsf(v);
    le = min(le, part_ulp_exp(v));
  };
#pragma unroll
  for (int j = 0; j < J; j++) {  // groups past G hold +0: no effect on any of the three
    take(e[j].x);
    take(e[j].y);
    take(e[j].z);
    take(e[j].w);
  }
  take(et);
  ls = wave_sum_d(ls);
  la = wave_sum_d(la);
  le = wave_min_i(le);
  const float fc = (float)cols;
  float mean;
  if (la <= exact_limit(le)) {
    mean = (float)ls / fc;
  } else {
    const double d = la * ((double)(cols + 4 * J + 8) * 0x1p-52);
    const float lo = (float)(ls - d) / fc, hi = (float)(ls + d) / fc;
    if (lo == hi) {  // false for NaN
      mean = lo;
    } else {
      // In order, 64 elements (16 lanes of one slice) at a time: a segment
      // whose additions to the running sum s cannot round (|s| plus the
      // segment's sum of |x| below 2^53 times the smaller of s's lowest set
      // bit and the segment's smallest ulp) is added as its tree sum, any
      // other element by element.
      double s = 0.0;
#pragma unroll
      for (int j = 0; j < J; j++) {
        if (!FULL && kWave * j >= G) break;
        const float4 q = e[j];  // +0 past G
        const double seg = row16_sum(((double)q.x + (double)q.y) + ((double)q.z + (double)q.w));
        const double sega = row16_sum(((double)__builtin_fabsf(q.x) + (double)__builtin_fabsf(q.y)) +
                                      ((double)__builtin_fabsf(q.z) + (double)__builtin_fabsf(q.w)));
        const int sege = row16_min(min(min(part_ulp_exp(q.x), part_ulp_exp(q.y)),
                                       min(part_ulp_exp(q.z), part_ulp_exp(q.w))));
#pragma unroll
        for (int r = 0; r < 4; r++) {
          if (!FULL && kWave * j + 16 * r >= G) break;
          const int e_min = min(__builtin_amdgcn_readlane(sege, 16 * r), low_bit_exp(s));
          if (__builtin_fabs(s) + lane_d(sega, 16 * r) <= exact_limit(e_min)) {
            s = s + lane_d(seg, 16 * r);
          } else {
#pragma unroll 1
            for (int i = 16 * r; i < 16 * r + 16; i++) {
              s = s + (double)lane_f(q.x, i);
              s = s + (double)lane_f(q.y, i);
              s = s + (double)lane_f(q.z, i);
              s = s + (double)lane_f(q.w, i);
            }
          }
        }
      }
      for (int l = 0; l < T; l++) s = s + (double)lane_f(et, l);
      mean = (float)s / fc;
    }
  }
  float part[J];
#pragma unroll
  for (int j = 0; j < J; j++) {
    const int g = lane + kWave * j;
    e[j] = make_float4(e[j].x - mean, e[j].y - mean, e[j].z - mean, e[j].w - mean);
    const float q0 = e[j].x * e[j].x, q1 = e[j].y * e[j].y, q2 = e[j].z * e[j].z, q3 = e[j].w * e[j].w;
    part[j] = (FULL || g < G) ? (q0 + q1) + (q2 + q3) : 0.0f;
  }
  const float dt = et - mean, qt = dt * dt;
  const double dc = (double)cols;
  const float var = ordered_sum_apply<J, FULL>(part, G, qt, T, [dc](double v) { return (float)(v / dc); });
  if (LATE) load_ops();
  const float scl = 1.0f / sqrtf(var + eps);
  float v[4 * J];
#pragma unroll
  for (int j = 0; j < J; j++) {
    v[4 * j] = e[j].x * scl;
    v[4 * j + 1] = e[j].y * scl;
    v[4 * j + 2] = e[j].z * scl;
    v[4 * j + 3] = e[j].w * scl;
  }
  float tv[1] = {dt * scl};
  if (EPI) {
    auto off = [&](const EpiOp &o, int r) {
      const int g = lane + kWave * (r / 4);
      const int c = (FULL || g < G) ? 4 * g + r % 4 : 0;
      return row * o.s1 + c * o.s2;
    };
    epi_ops_n(ep, v, w);
    epi_apply_n(ep, v, off, kEpiEarly);
    if (T > 0) {
      epi_ops_n(ep, tv, wt);
      epi_apply_n(ep, tv, [&](const EpiOp &o, int) { return row * o.s1 + (lane < T ? 4 * G + lane : 0) * o.s2; },
                  kEpiEarly);
    }
  }
  float *y = Y + row * cols;
#pragma unroll
  for (int j = 0; j < J; j++) {
    const int g = lane + kWave * j;
    if (!(FULL || g < G)) continue;
    float *p = y + 4 * g;
    if (T == 0) {
      st4(p, make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]));
    } else {
      p[0] = v[4 * j];
      p[1] = v[4 * j + 1];
      p[2] = v[4 * j + 2];
      p[3] = v[4 * j + 3];
    }
  }
  if (lane < T) y[4 * G + lane] = tv[0];
}

// ---- silu -----------------------------------------------------------------------

// x / (1 + ggml_v_expf(0 - x)) on the four-lane body (Shaders.lean:172-179);
// rows must be multiples of 4 (tails are refused by the lowering).
// With rows of `cols` not a multiple of 4 (pinned flavour only), each row's
// last cols % 4 elements take x / (1 + expf(-x)) with the correctly rounded
// expf (ggml_vec_silu_f32's scalar loop).
template <int TAIL>
__global__ void __launch_bounds__(256) silu_k(int64_t n, int64_t cols, int gpu_ops, const float *__restrict__ X,
                                              float *__restrict__ Y) {
  const int64_t body = cols & ~(int64_t)3;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float x = X[i];
    if (gpu_ops) Y[i] = x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));  // planted: GPU exp and /
    else if (TAIL && i % cols >= body) Y[i] = x / (1.0f + expfk::expf_cr(-x));
    else Y[i] = x / (1.0f + ggml_v_expf(0.0f - x));
  }
}

// ---- gelu_erf and the erff map ------------------------------------------------------

template <int TANH>
__device__ __forceinline__ float4 gelu4(float4 v, const double *tab) {
  if (TANH) return make_float4(gelu1<1>(v.x, tab), gelu1<1>(v.y, tab), gelu1<1>(v.z, tab), gelu1<1>(v.w, tab));
  float x[4] = {v.x, v.y, v.z, v.w};
  gelu_erf_n(x, tab);
  return make_float4(x[0], x[1], x[2], x[3]);
}

// Block b owns the float4s [b*chunk, (b+1)*chunk) (contiguous, so each block
// streams whole DRAM pages); each thread takes kGeluU float4s 256 apart per
// step.  Loads are ordinary (cached), stores nontemporal: on gfx950 that mix
// streams 64 Mi at 6.9 TB/s, against 6.4 TB/s with both nontemporal and
// 5.7 TB/s with both cached.  The first step's loads are issued before the
// table is staged in LDS, so they are in flight during the staging.  The last
// block also maps the n % 4 scalar tail.
constexpr int kGeluU = 4;

template <int TANH>
__global__ void __launch_bounds__(256) gelu_erf_k(int64_t n, int64_t chunk, const float *__restrict__ X,
                                                  float *__restrict__ Y) {
  __shared__ double tab[kPolyWords];
  const int64_t n4 = n / 4;
  const int64_t b0 = blockIdx.x * chunk;
  const int64_t e = b0 + chunk < n4 ? b0 + chunk : n4;
  int64_t i = b0 + threadIdx.x;
  float4 v[kGeluU];
  bool loaded = i + (kGeluU - 1) * 256 < e;
  if (loaded) {
#pragma unroll
    for (int u = 0; u < kGeluU; u++) v[u] = ld4(X + 4 * (i + u * 256));
  }
  load_poly(tab);
  for (; i + (kGeluU - 1) * 256 < e; i += kGeluU * 256) {
    if (!loaded) {
#pragma unroll
      for (int u = 0; u < kGeluU; u++) v[u] = ld4(X + 4 * (i + u * 256));
    }
    loaded = false;
#pragma unroll
    for (int u = 0; u < kGeluU; u++) st4_nt(Y + 4 * (i + u * 256), gelu4<TANH>(v[u], tab));
  }
  for (; i < e; i += 256) st4_nt(Y + 4 * i, gelu4<TANH>(ld4(X + 4 * i), tab));
  if (blockIdx.x == gridDim.x - 1)
    for (int64_t t = 4 * n4 + threadIdx.x; t < n; t += 256) Y[t] = gelu1<TANH>(X[t], tab);
}

__global__ void __launch_bounds__(256) erff_map_k(uint32_t base, uint32_t count, uint32_t *__restrict__ Y) {
  __shared__ double tab[kPolyWords];
  load_poly(tab);
  for (uint32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < count; t += gridDim.x * blockDim.x)
    Y[t] = f_bits(erffk::erff_cr(bits_f(base + t), tab));
}

__global__ void __launch_bounds__(256) expf_map_k(uint32_t base, uint32_t count, uint32_t *__restrict__ Y) {
  for (uint32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < count; t += gridDim.x * blockDim.x)
    Y[t] = f_bits(expfk::expf_cr(bits_f(base + t)));
}

unsigned grid_cap(int64_t n, int block, int64_t cap) {
  int64_t g = (n + block - 1) / block;
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(g, cap));
}

}  // namespace

// ---- host side --------------------------------------------------------------------------

namespace {
int g_default_tail = kTailStock;
std::string g_last_dot = "";  // the kernel the last dot_ggml call chose

const char *loader_name(int l) {
  static const char *const n[] = {"RowVec", "ColVec", "Scalar", "ColQuad", "RowVecB", "ColQuadB"};
  return l >= 0 && l < 6 ? n[l] : "?";
}
}  // namespace
int default_dot_tail() { return g_default_tail; }
const std::string &last_dot_kernel() { return g_last_dot; }
void set_default_dot_tail(int t) {
  if (t != kTailStock && t != kTailPinned) fail("flavor: 0 (stock) or 1 (pinned)");
  g_default_tail = t;
}

Epilogue make_epilogue(const std::vector<FusedOp> &ops, std::vector<ArrayP> *keep) {
  if (ops.size() > (size_t)kMaxEpi) fail(strf("fused epilogue: at most %d ops", kMaxEpi));
  Epilogue ep;
  for (const FusedOp &o : ops) {
    if (o.code == kEpiGeluErf) {
      ep.op[ep.n++] = EpiOp{nullptr, 0, 0, 0, o.code, 0u};
      ep.gelu = 1;
      continue;
    }
    if (!o.arr || o.arr->dtype != kF32 || !o.arr->buf) fail("fused epilogue: f32 operands only");
    ep.op[ep.n++] = EpiOp{(const float *)o.arr->data(), o.s0, o.s1, o.s2, o.code, o.rev ? 1u : 0u};
    keep->push_back(o.arr);
  }
  return ep;
}

// A copy of a dot operand (element (b, r, k) for b < B, r < rows, k < K) in a
// layout the direct kernel reads: [B][R][Kp] (along k, rows Kp = K rounded up
// to 4 floats apart) or [B][K][R] (rows contiguous), R = rows rounded up to
// the tile.  Padding never reaches a stored output: padded rows feed only
// outputs past N or M, which are not stored, and k past K is never read.
DotOperand padded_operand(const DotOperand &d, int64_t B, int64_t rows, int64_t K, bool along_k) {
  const int64_t R = (rows + kMT - 1) / kMT * kMT, Kp = (K + 3) / 4 * 4;
  auto p = new_array(kF32, along_k ? Shape{B, R, Kp} : Shape{B, K, R});
  auto src = std::make_shared<Array>();
  src->buf = d.arr->buf;
  src->offset = d.arr->offset;
  src->dtype = kF32;
  src->shape = Shape{B / d.nb2, d.nb2, rows, K};
  src->strides = Shape{d.sb, d.sb2, d.sf, d.sk};
  copy_to_strides(src, along_k ? Shape{d.nb2 * R * Kp, R * Kp, Kp, 1} : Shape{d.nb2 * K * R, K * R, 1, R},
                  p->data());
  DotOperand o{p, along_k ? R * Kp : K * R, along_k ? Kp : 1, along_k ? 1 : R, 0, 1};
  o.rows_alloc = R;
  return o;
}

ArrayP dot_ggml(const DotOperand &lhs, const DotOperand &rhs, int64_t B, int64_t N, int64_t M, int64_t K, int tail,
                const std::vector<FusedOp> &epi) {
  if (lhs.arr->dtype != kF32 || rhs.arr->dtype != kF32) fail("dot_general: f32 operands only");
  if (B < 0 || N < 0 || M < 0 || K < 0) fail("dot_general: negative extent");
  std::vector<ArrayP> ek;
  const Epilogue ep = make_epilogue(epi, &ek);
  auto y = new_array(kF32, Shape{B * N * M});
  const int64_t n_out = B * N * M;
  if (n_out == 0) return y;
  if (K > 0 && (!lhs.arr->buf || !rhs.arr->buf)) fail("dot_general: empty operand");
  const float *L = (const float *)lhs.arr->data();
  const float *R = (const float *)rhs.arr->data();
  float *Y = (float *)y->data();
  ArrayP kl = lhs.arr, kr = rhs.arr;
  const int64_t lb = lhs.sb, ln = lhs.sf, lk = lhs.sk, rb = rhs.sb, rm = rhs.sf, rk = rhs.sk;
  if (lhs.nb2 < 1 || rhs.nb2 < 1 || B % lhs.nb2 || B % rhs.nb2) fail("dot_general: inner batch count does not divide");
  if (B > 0x7FFFFFFF) fail("dot_general: more than 2^31 - 1 batches");
  const MfmaOperand X{L, lb, ln, lk, N, lhs.sb2, lhs.nb2}, W{R, rb, rm, rk, M, rhs.sb2, rhs.nb2};
  if (tail != kTailPlain && B <= 65535) {
    auto loader = [&](const float *p, int64_t sb, int64_t sf, int64_t sk, int64_t rows, const DotOperand &d) {
      const bool al = ((uintptr_t)p % 16) == 0 && (sb % 4 == 0 || B == 1) && (d.nb2 == 1 || d.sb2 % 4 == 0);
      if (al && sk == 1 && (sf % 4 == 0 || rows == 1)) return (int)kLoadRowVec;
      if (al && sf == 1 && sk % 4 == 0 && rows % 4 == 0) return (int)kLoadColQuad;
      if (sf == 1) return (int)kLoadColVec;
      return (int)kLoadScalar;
    };
    // Rows readable per batch: a padded copy's, else the logical rows.
    const int64_t Nr = lhs.rows_alloc ? lhs.rows_alloc : N, Mr = rhs.rows_alloc ? rhs.rows_alloc : M;
    int lx = loader(L, lb, ln, lk, Nr, lhs), lw = loader(R, rb, rm, rk, Mr, rhs);
    // The buffer loaders need every read in range by construction: rows a
    // multiple of the tile, every stage full, non-negative strides, and the
    // largest byte offset within a batch below 2^31.
    const bool full_stages = ((K / 16) % (kKC / 16)) == 0 && K >= kKC;
    auto in_range = [&](int64_t sf, int64_t sk, int64_t sb, int64_t rows) {
      if (rows % kMT || sf < 0 || sk < 0 || sb < 0 || lhs.sb2 < 0 || rhs.sb2 < 0) return false;
      const int64_t top = ((rows - 1) * sf + (K - 1) * sk + 4) * 4;
      return top < ((int64_t)1 << 31);
    };
    auto buf_ok = [&](int64_t sf, int64_t sk, int64_t sb, int64_t rows) {
      return full_stages && in_range(sf, sk, sb, rows);
    };
    if (((lx == kLoadRowVec && ln % 4 == 0) || lx == kLoadColQuad) && buf_ok(ln, lk, lb, Nr) &&
        ((lw == kLoadRowVec && rm % 4 == 0) || lw == kLoadColQuad) && buf_ok(rm, rk, rb, Mr)) {
      lx = lx == kLoadRowVec ? (int)kLoadRowVecB : (int)kLoadColQuadB;
      lw = lw == kLoadRowVec ? (int)kLoadRowVecB : (int)kLoadColQuadB;
    }
    static const bool lds_ok = [] {  // 135 KB of dynamic LDS, above the 64 KB default
#define DOT_ATTR(a, c)                                                                                       \
  SHLO_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&dot_mfma8_k<a, c>),                         \
                               hipFuncAttributeMaxDynamicSharedMemorySize, kDotLdsGelu));
      DOT_ATTR(kLoadRowVec, kLoadRowVec) DOT_ATTR(kLoadRowVec, kLoadColVec) DOT_ATTR(kLoadRowVec, kLoadScalar)
      DOT_ATTR(kLoadColVec, kLoadRowVec) DOT_ATTR(kLoadColVec, kLoadColVec) DOT_ATTR(kLoadColVec, kLoadScalar)
      DOT_ATTR(kLoadScalar, kLoadRowVec) DOT_ATTR(kLoadScalar, kLoadColVec) DOT_ATTR(kLoadScalar, kLoadScalar)
      DOT_ATTR(kLoadRowVec, kLoadColQuad) DOT_ATTR(kLoadColQuad, kLoadRowVec) DOT_ATTR(kLoadColQuad, kLoadColQuad)
      DOT_ATTR(kLoadColQuad, kLoadColVec) DOT_ATTR(kLoadColVec, kLoadColQuad) DOT_ATTR(kLoadColQuad, kLoadScalar)
      DOT_ATTR(kLoadScalar, kLoadColQuad)
      DOT_ATTR(kLoadColQuadB, kLoadRowVecB) DOT_ATTR(kLoadColQuadB, kLoadColQuadB)
#undef DOT_ATTR
      return true;
    }();
    (void)lds_ok;
    const int64_t tiles_m64 = (M + kMT - 1) / kMT, tiles_n64 = (N + kMT - 1) / kMT;
    if (tiles_m64 > 0x7FFFFFFF || tiles_n64 > 0x7FFFFFFF || tiles_m64 * tiles_n64 > 0x7FFFFFFF)
      fail("dot_general: too many output tiles");
    const int tiles_m = (int)tiles_m64;
    const int64_t tiles_b = tiles_n64 * tiles_m64;
    // One workgroup per tile.  An lhs along k with an rhs along its free dim
    // or along k, every read in range, loads both operands straight into LDS
    // (dot_mfma8d_k; both along k also in stages of 64, as Q K^T with K = 64);
    // any other layout stages them through registers (dot_mfma8_k).  A
    // persistent kernel walking tiles with the next tile's loads under this
    // tile's epilogue was slower in every case measured (the denoiser's
    // K = 256 and 512 products 6.11 against 5.57 ms, its [8192,512] x
    // [512,263] output projection 64 against 57 us, config 3 5.44 against
    // 5.16 ms).
    // The direct kernel's stages cover the blocks of 16 (np = K & ~15, a
    // whole number of stages); the serial tail runs in its store.
    const int64_t np = K & ~(int64_t)15;
    int dkc = 0;
    if (lx == kLoadRowVecB && (lw == kLoadColQuadB || lw == kLoadRowVecB)) {
      dkc = kKC;
    } else if (lx == kLoadRowVec && lw == kLoadRowVec && np % 64 == 0 && np >= 64 && ln % 4 == 0 && rm % 4 == 0 &&
               in_range(ln, lk, lb, Nr) && in_range(rm, rk, rb, Mr)) {
      dkc = 64;
      lx = lw = kLoadRowVecB;
    }
    const bool direct = dkc > 0;
    // A large product with an lhs along k and an rhs along its free dim or
    // along k that cannot go direct in place (rows not 16-byte aligned, row
    // counts not multiples of the tile, e.g. the denoiser's 263-wide
    // projections) runs on padded copies: one pass over each operand buys the
    // direct kernel.
    if (!direct && lhs.rows_alloc == 0 && rhs.rows_alloc == 0 && lk == 1 && (rm == 1 || rk == 1) &&
        np >= kKC && np % kKC == 0 && (double)B * (double)N * (double)M * (double)np >= (double)(1 << 27) &&
        ((double)std::max(N, M) + kMT) * ((double)K + 4) * 4.0 < (double)(1LL << 31)) {
      const DotOperand pl = padded_operand(lhs, B, N, K, true);
      const DotOperand pr = padded_operand(rhs, B, M, K, rm != 1);
      return dot_ggml(pl, pr, B, N, M, K, tail, epi);
    }
    // The register-staged kernel is instantiated with the buffer loaders only
    // for a column-read lhs: a row-read lhs that did not go direct takes the
    // plain loaders (same elements, bounds-checked addressing).
    if (!direct && lx == kLoadRowVecB) {
      lx = kLoadRowVec;
      lw = lw == kLoadRowVecB ? (int)kLoadRowVec : (int)kLoadColQuad;
    }
    if (!direct) {
      static const int kCases[][2] = {
          {kLoadRowVec, kLoadRowVec},   {kLoadRowVec, kLoadColVec},     {kLoadRowVec, kLoadScalar},
          {kLoadColVec, kLoadRowVec},   {kLoadColVec, kLoadColVec},     {kLoadColVec, kLoadScalar},
          {kLoadScalar, kLoadRowVec},   {kLoadScalar, kLoadColVec},     {kLoadScalar, kLoadScalar},
          {kLoadRowVec, kLoadColQuad},  {kLoadColQuad, kLoadRowVec},    {kLoadColQuad, kLoadColQuad},
          {kLoadColQuad, kLoadColVec},  {kLoadColVec, kLoadColQuad},    {kLoadColQuad, kLoadScalar},
          {kLoadScalar, kLoadColQuad},  {kLoadColQuadB, kLoadRowVecB}, {kLoadColQuadB, kLoadColQuadB}};
      bool have = false;
      for (auto &c : kCases) have |= c[0] == lx && c[1] == lw;
      if (!have) fail(strf("dot_general: no kernel for loaders %s, %s", loader_name(lx), loader_name(lw)));
    }
    // Short direct contractions: four-wave workgroups on 32 x 64 tiles, three per CU.
    const bool small = direct && K <= 512;
    const unsigned glds = ep.gelu ? kPolyWords * (unsigned)sizeof(double) : 0;  // the eight-wave direct kernel's dynamic LDS
    const dim3 grid_s((unsigned)(tiles_n64 * 2 * tiles_m64), (unsigned)B);
    const unsigned lds = ep.gelu ? kDotLdsGelu : kDotLds;
    const dim3 grid1((unsigned)tiles_b, (unsigned)B);
    if ((small ? 2 * tiles_b : tiles_b) > 0x7FFFFFFF) fail("dot_general: too many output tiles");
    const int tl = tail;
    if (direct)
      g_last_dot = strf("dot_mfma8d_k<RowVecB,%s,%d,%d>", loader_name(lw), small ? 64 : dkc, small ? 4 : 8);
    else
      g_last_dot = strf("dot_mfma8_k<%s,%s>", loader_name(lx), loader_name(lw));
    // Tiles that are not whole (rows past N or M, a tail) take the EDGE
    // instances; the rest keep the leaner code (and three workgroups per CU).
    const bool edge = np < K || N % (small ? 32 : kMT) != 0 || M % kMT != 0;
    launch([=](hipStream_t s) {
      (void)kl, (void)kr, (void)ek;
#define DOT_D(lw_, kc_, waves_, grid_, th_, lds_)                                                              \
  do {                                                                                                        \
    if (edge)                                                                                                 \
      dot_mfma8d_k<kLoadRowVecB, lw_, kc_, waves_, true><<<grid_, th_, lds_, s>>>(X, W, N, M, K, tl, tiles_m, ep, Y); \
    else                                                                                                      \
      dot_mfma8d_k<kLoadRowVecB, lw_, kc_, waves_, false><<<grid_, th_, lds_, s>>>(X, W, N, M, K, tl, tiles_m, ep, Y); \
  } while (0)
      if (direct && small) {
        if (lw == kLoadColQuadB) DOT_D(kLoadColQuadB, 64, 4, grid_s, 256, 0);
        else DOT_D(kLoadRowVecB, 64, 4, grid_s, 256, 0);
        return;
      }
      if (direct) {
        if (lw == kLoadColQuadB) DOT_D(kLoadColQuadB, kKC, 8, grid1, 512, glds);
        else if (dkc == kKC) DOT_D(kLoadRowVecB, kKC, 8, grid1, 512, glds);
        else DOT_D(kLoadRowVecB, 64, 8, grid1, 512, glds);
        return;
      }
#undef DOT_D
#define DOT_CASE(a, c)                                                                    \
  if (lx == a && lw == c) {                                                               \
    dot_mfma8_k<a, c><<<grid1, 512, lds, s>>>(X, W, N, M, K, tl, tiles_m, ep, Y);         \
    return;                                                                               \
  }
      DOT_CASE(kLoadRowVec, kLoadRowVec) DOT_CASE(kLoadRowVec, kLoadColVec) DOT_CASE(kLoadRowVec, kLoadScalar)
      DOT_CASE(kLoadColVec, kLoadRowVec) DOT_CASE(kLoadColVec, kLoadColVec) DOT_CASE(kLoadColVec, kLoadScalar)
      DOT_CASE(kLoadScalar, kLoadRowVec) DOT_CASE(kLoadScalar, kLoadColVec) DOT_CASE(kLoadScalar, kLoadScalar)
      DOT_CASE(kLoadRowVec, kLoadColQuad) DOT_CASE(kLoadColQuad, kLoadRowVec) DOT_CASE(kLoadColQuad, kLoadColQuad)
      DOT_CASE(kLoadColQuad, kLoadColVec) DOT_CASE(kLoadColVec, kLoadColQuad) DOT_CASE(kLoadColQuad, kLoadScalar)
      DOT_CASE(kLoadScalar, kLoadColQuad)
      DOT_CASE(kLoadColQuadB, kLoadRowVecB) DOT_CASE(kLoadColQuadB, kLoadColQuadB)
#undef DOT_CASE
    });
    return y;
  }
  const unsigned grid = grid_cap(n_out, 256, 1 << 20);
  g_last_dot = strf("dot_ggml_simple<%s>", tail == kTailStock ? "stock" : tail == kTailPinned ? "pinned" : "plain");
  launch([=](hipStream_t s) {
    (void)kl, (void)kr, (void)ek;
    switch (tail) {
      case kTailStock:
        dot_ggml_simple<kTailStock><<<grid, 256, 0, s>>>(n_out, N, M, K, X, W, ep, Y);
        break;
      case kTailPinned:
        dot_ggml_simple<kTailPinned><<<grid, 256, 0, s>>>(n_out, N, M, K, X, W, ep, Y);
        break;
      default:
        dot_ggml_simple<kTailPlain><<<grid, 256, 0, s>>>(n_out, N, M, K, X, W, ep, Y);
        break;
    }
  });
  return y;
}


// One attention_k launch: the instance for J keys / 256, a unit softmax
// scale or not, masked-tile skipping or not (a no-op unless `on`).
template <int J>
void attention_launch(bool on, bool unit, bool skip, dim3 grid, hipStream_t s, const MfmaOperand &Q,
                      const MfmaOperand &Kk, const MfmaOperand &V, int64_t NQ, const Epilogue &e1, int mskip,
                      const int *prep, float sc, const Epilogue &e2, float *Y) {
  if (!on) return;
  if (skip) {
    if (unit) attention_k<J, true, true><<<grid, 256, 0, s>>>(Q, Kk, V, NQ, e1, mskip, prep, sc, e2, Y);
    else attention_k<J, false, true><<<grid, 256, 0, s>>>(Q, Kk, V, NQ, e1, mskip, prep, sc, e2, Y);
  } else {
    if (unit) attention_k<J, true, false><<<grid, 256, 0, s>>>(Q, Kk, V, NQ, e1, mskip, prep, sc, e2, Y);
    else attention_k<J, false, false><<<grid, 256, 0, s>>>(Q, Kk, V, NQ, e1, mskip, prep, sc, e2, Y);
  }
}

ArrayP attention_ggml(const DotOperand &q, const DotOperand &k, const DotOperand &v, int64_t B, int64_t NQ,
                      int64_t NK, int64_t DH, int64_t DV, const std::vector<FusedOp> &epi1, uint32_t sm_scale_bits,
                      const std::vector<FusedOp> &epi2) {
  for (const DotOperand *d : {&q, &k, &v})
    if (d->arr->dtype != kF32 || !d->arr->buf || d->nb2 < 1 || B % d->nb2) return nullptr;
  if (DH != kAttnDh || DV != kAttnDv || NK % 256 || NK < 256 || NK > 1024 || NQ <= 0 || NQ % kAttnRows) return nullptr;
  if (B < 1 || B > 65535 || NQ / kAttnRows > 0x7FFFFFFF) return nullptr;
  auto rows_ok = [&](const DotOperand &d) {  // float4 loads along d from 16-byte aligned rows
    const float *p = (const float *)d.arr->data();
    return d.sk == 1 && d.sf % 4 == 0 && (uintptr_t)p % 16 == 0 && (d.sb % 4 == 0 || B == 1) &&
           (d.nb2 == 1 || d.sb2 % 4 == 0);
  };
  if (!rows_ok(q) || !rows_ok(k) || v.sf != 1) return nullptr;
  // K's and V's buffer offsets within a batch stay below 2^31 bytes
  if (((NK - 1) * k.sf + DH) * 4 >= ((int64_t)1 << 31) || (DV + (NK + 16) * v.sk) * 4 >= ((int64_t)1 << 31) ||
      k.sf < 0 || v.sk < 0)
    return nullptr;
  for (auto *ep : {&epi1, &epi2})
    for (const FusedOp &o : *ep)
      if (o.code == kEpiGeluErf) return nullptr;
  std::vector<ArrayP> keep;
  const Epilogue e1 = make_epilogue(epi1, &keep), e2 = make_epilogue(epi2, &keep);
  // Masked-tile skipping (attn_skip_plan): the chain is [add mask] or
  // [multiply by a scalar, add mask], the mask along keys with 16-byte
  // aligned rows.
  int mskip = 0;
  {
    auto mask_ok = [](const EpiOp &o) {
      return o.code == kAdd && o.s0 == 0 && o.s2 == 1 && (uintptr_t)o.p % 16 == 0 && o.s1 % 4 == 0;
    };
    if (e1.n == 1 && mask_ok(e1.op[0])) mskip = 1;
    if (e1.n == 2 && e1.op[0].code == kMul && e1.op[0].s0 == 0 && e1.op[0].s1 == 0 && e1.op[0].s2 == 0 &&
        mask_ok(e1.op[1]))
      mskip = 2;
  }
  auto y = new_array(kF32, Shape{B * NQ * DV});
  const MfmaOperand Q{(const float *)q.arr->data(), q.sb, q.sf, q.sk, NQ, q.sb2, q.nb2};
  const MfmaOperand Kk{(const float *)k.arr->data(), k.sb, k.sf, k.sk, NK, k.sb2, k.nb2};
  const MfmaOperand V{(const float *)v.arr->data(), v.sb, v.sf, v.sk, DV, v.sb2, v.nb2};
  float *Y = (float *)y->data();
  const float sc = bits_f(sm_scale_bits);
  const bool unit = sm_scale_bits == 0x3F800000u;
  const dim3 grid((unsigned)(NQ / kAttnRows), (unsigned)B);
  const int J = (int)(NK / 256);
  ArrayP kq = q.arr, kk = k.arr, kvv = v.arr;
  // attn_prep_k's ints: K's exponent fields per (batch, 64 keys), then the
  // masked-tile bits per (block of 32 query rows, 64 keys)
  const int64_t nprep = (B + NQ / kAttnRows) * (NK / 64);
  ArrayP kxa = mskip ? new_array(kF32, Shape{nprep}) : nullptr;
  int *kx = kxa ? (int *)kxa->data() : nullptr;
  const float *mp = mskip ? e1.op[mskip - 1].p : nullptr;
  const int64_t ms1 = mskip ? e1.op[mskip - 1].s1 : 0;
  g_last_dot = strf("attention_k<%d>", J);
  launch([=](hipStream_t s) {
    (void)kq, (void)kk, (void)kvv, (void)keep, (void)kxa;
    if (mskip)
      attn_prep_k<<<(unsigned)nprep, 256, 0, s>>>(Kk, V, (int)NK, B, mp, ms1, kx);
    attention_launch<1>(J == 1, unit, mskip != 0, grid, s, Q, Kk, V, NQ, e1, mskip, kx, sc, e2, Y);
    attention_launch<2>(J == 2, unit, mskip != 0, grid, s, Q, Kk, V, NQ, e1, mskip, kx, sc, e2, Y);
    attention_launch<3>(J == 3, unit, mskip != 0, grid, s, Q, Kk, V, NQ, e1, mskip, kx, sc, e2, Y);
    attention_launch<4>(J == 4, unit, mskip != 0, grid, s, Q, Kk, V, NQ, e1, mskip, kx, sc, e2, Y);
  });
  return y;
}

ArrayP mul_mat(const ArrayP &w0, const ArrayP &x0, int64_t K, int64_t M, int64_t R, int64_t N, int64_t wbs,
               int tail) {
  if (N <= 0 || R % N) fail("mul_mat: R must be a multiple of N > 0");
  ArrayP w = contiguous(w0), x = contiguous(x0);
  const int64_t B = R / N;
  if (x->size() < R * K) fail("mul_mat: x holds fewer than R*K elements");
  if (w->size() < (B - 1) * wbs + M * K) fail("mul_mat: w holds fewer elements than the batch stride needs");
  return dot_ggml(DotOperand{x, N * K, K, 1}, DotOperand{w, wbs, K, 1}, B, N, M, K, tail);
}

// The row kernels load four-element groups as 16-byte loads from the start
// of the array: a contiguous view at an offset that is not a multiple of 16
// bytes is first copied to a fresh (256-byte aligned) block.
ArrayP aligned_rows(const ArrayP &x) {
  if (!x->buf || (uintptr_t)x->data() % 16 == 0) return x;
  auto c = new_array(x->dtype, x->shape);
  copy_into(c, x);
  return c;
}

// A row tail (cols % 4 elements) goes through ggml-cpu's scalar expf: the
// pinned flavour's is correctly rounded and carried; the stock flavour's is
// Apple libsystem_m's, closed code, and refused as the reference refuses it
// (Lower.lean:485-486).
void require_tail_expf(const char *op, int64_t cols) {
  if (cols % 4 && default_dot_tail() != kTailPinned)
    fail(strf("%s: a row of %lld has a %lld-element tail that ggml-cpu sends through the platform expf, which is "
              "not carried (the pinned flavour carries it with the correctly rounded expf)",
              op, (long long)cols, (long long)(cols % 4)));
}

ArrayP soft_max(const ArrayP &x0, int64_t rows, int64_t cols, uint32_t scale_bits, bool float_sum) {
  if (x0->dtype != kF32) fail("ggml.soft_max: f32 only");
  if (rows * cols != x0->size()) fail("ggml.soft_max: rows*cols is not the element count");
  require_tail_expf("ggml.soft_max", cols);
  if (cols > 0x7FFFFFFF) fail("ggml.soft_max: rows of 2^31 columns or more are not carried");
  ArrayP x = aligned_rows(contiguous(x0));
  auto y = new_array(kF32, x->shape);
  if (rows == 0 || cols == 0) return y;
  const float sc = bits_f(scale_bits);
  if (cols > 4 * kWave * 16) {  // rows that do not fit one wave's registers
    const int64_t nblk = (rows + 3) / 4;
    if (nblk > 0x7FFFFFFF) fail("ggml.soft_max: too many rows");
    const unsigned grid = (unsigned)nblk;
    const float *px = (const float *)x->data();
    float *py = (float *)y->data();
    const int c = (int)cols, fs = float_sum ? 1 : 0;
    ArrayP kx = x;
    launch([=](hipStream_t s) {
      (void)kx;
      if (c % 4) soft_max_long_k<false><<<grid, 256, 0, s>>>(rows, c, sc, fs, px, py);
      else soft_max_long_k<true><<<grid, 256, 0, s>>>(rows, c, sc, fs, px, py);
    });
    return y;
  }
  if (cols % 4) {
    const int G = (int)(cols / 4);
    const int Jt = std::max(1, (G + kWave - 1) / kWave);
    const int64_t nblk = (rows + 3) / 4;
    if (nblk > 0x7FFFFFFF) fail("ggml.soft_max: too many rows");
    const unsigned grid = (unsigned)nblk;
    const float *px = (const float *)x->data();
    float *py = (float *)y->data();
    const int c = (int)cols;
    const int fs = float_sum ? 1 : 0;
    ArrayP kx = x;
    launch([=](hipStream_t s) {
      (void)kx;
#define SMT_CASE(n) \
  case n: soft_max_tail_k<n><<<grid, 256, 0, s>>>(rows, c, sc, fs, px, py); break;
      switch (Jt) {
        SMT_CASE(1) SMT_CASE(2) SMT_CASE(3) SMT_CASE(4) SMT_CASE(5) SMT_CASE(6) SMT_CASE(7) SMT_CASE(8)
        SMT_CASE(9) SMT_CASE(10) SMT_CASE(11) SMT_CASE(12) SMT_CASE(13) SMT_CASE(14) SMT_CASE(15) SMT_CASE(16)
        default: break;
      }
#undef SMT_CASE
    });
    return y;
  }
  const int J = (int)((cols / 4 + kWave - 1) / kWave);
  const float *px = (const float *)x->data();
  float *py = (float *)y->data();
  const int c = (int)cols;
  const int fs = float_sum ? 1 : 0;
  ArrayP kx = x;
  const int64_t nblk = (rows + 3) / 4;
  if (nblk > 0x7FFFFFFF) fail("ggml.soft_max: too many rows");
  const unsigned grid = (unsigned)nblk;
  const bool full = cols == 4LL * kWave * J;
  const bool unit = scale_bits == 0x3F800000u;
  launch([=](hipStream_t s) {
    (void)kx;
#define SM_CASE(n)                                                                                  \
  case n:                                                                                           \
    if (full && unit) soft_max_rows_k<n, true, true><<<grid, 256, 0, s>>>(rows, c, sc, fs, px, py); \
    else if (full) soft_max_rows_k<n, true><<<grid, 256, 0, s>>>(rows, c, sc, fs, px, py);          \
    else soft_max_rows_k<n, false><<<grid, 256, 0, s>>>(rows, c, sc, fs, px, py);                   \
    break;
    switch (J) {
      SM_CASE(1) SM_CASE(2) SM_CASE(3) SM_CASE(4) SM_CASE(5) SM_CASE(6) SM_CASE(7) SM_CASE(8)
      SM_CASE(9) SM_CASE(10) SM_CASE(11) SM_CASE(12) SM_CASE(13) SM_CASE(14) SM_CASE(15) SM_CASE(16)
      default: break;
    }
#undef SM_CASE
  });
  return y;
}

ArrayP norm(const ArrayP &x0, int64_t rows, int64_t cols, uint32_t eps_bits, bool gpu_ops,
            const std::vector<FusedOp> &epi) {
  if (x0->dtype != kF32) fail("ggml.norm: f32 only");
  if (rows * cols != x0->size()) fail("ggml.norm: rows*cols is not the element count");
  if (cols > 0x7FFFFFFF) fail("ggml.norm: rows of 2^31 columns or more are not carried");
  if (gpu_ops && !epi.empty()) fail("ggml.norm: no fused ops with the planted binary32 sums");
  for (const FusedOp &o : epi)
    if (o.code == kEpiGeluErf) fail("ggml.norm: gelu_erf is not a fused op of norm");
  ArrayP x = aligned_rows(contiguous(x0));
  auto y = new_array(kF32, x->shape);
  if (rows == 0 || cols == 0) return y;
  const float *px = (const float *)x->data();
  float *py = (float *)y->data();
  const float eps = bits_f(eps_bits);
  const int c = (int)cols;
  ArrayP kx = x;
  if (gpu_ops) {  // planted: binary32 sums and the GPU's own / and sqrt
    const unsigned grid = grid_cap(rows, 4, 1 << 20);
    launch([=](hipStream_t s) {
      (void)kx;
      norm_planted_k<<<grid, kWave * 4, 0, s>>>(rows, c, eps, px, py);
    });
    return y;
  }
  std::vector<ArrayP> ek;
  const Epilogue ep = make_epilogue(epi, &ek);
  if (cols > 4096) {  // rows that do not fit one wave's registers
    if (ep.n > 0) fail("ggml.norm: fused ops need rows of at most 1024 columns");
    const int64_t nblk = (rows + 3) / 4;
    if (nblk > 0x7FFFFFFF) fail("ggml.norm: too many rows");
    const unsigned grid = (unsigned)nblk;
    launch([=](hipStream_t s) {
      (void)kx;
      if (c % 4) norm_long_k<false><<<grid, 256, 0, s>>>(rows, c, eps, px, py);
      else norm_long_k<true><<<grid, 256, 0, s>>>(rows, c, eps, px, py);
    });
    return y;
  }
  const int J = std::max<int>(1, (int)((cols / 4 + kWave - 1) / kWave));
  if (ep.n > 0 && J > kNormEpiJ) fail("ggml.norm: fused ops need rows of at most 1024 columns");
  const bool full = cols == 4LL * kWave * J, fused = ep.n > 0;
  const int64_t nblk = (rows + 3) / 4;
  if (nblk > 0x7FFFFFFF) fail("ggml.norm: too many rows");
  const unsigned grid = (unsigned)nblk;
  launch([=](hipStream_t s) {
    (void)kx, (void)ek;
#define NORM_CASE(n)                                                                                    \
  case n:                                                                                               \
    if (full) norm_rows_k<n, true, false><<<grid, 256, 0, s>>>(rows, c, eps, ep, px, py);               \
    else norm_rows_k<n, false, false><<<grid, 256, 0, s>>>(rows, c, eps, ep, px, py);                   \
    break;
#define NORM_EPI_CASE(n)                                                                                \
  case n:                                                                                               \
    if (full) norm_rows_k<n, true, true><<<grid, 256, 0, s>>>(rows, c, eps, ep, px, py);                \
    else norm_rows_k<n, false, true><<<grid, 256, 0, s>>>(rows, c, eps, ep, px, py);                    \
    break;
    if (fused) {
      switch (J) {
        NORM_EPI_CASE(1) NORM_EPI_CASE(2) NORM_EPI_CASE(3) NORM_EPI_CASE(4)
        default: break;
      }
      return;
    }
    switch (J) {
      NORM_CASE(1) NORM_CASE(2) NORM_CASE(3) NORM_CASE(4) NORM_CASE(5) NORM_CASE(6) NORM_CASE(7) NORM_CASE(8)
      NORM_CASE(9) NORM_CASE(10) NORM_CASE(11) NORM_CASE(12) NORM_CASE(13) NORM_CASE(14) NORM_CASE(15)
      NORM_CASE(16)
      default: break;
    }
#undef NORM_CASE
#undef NORM_EPI_CASE
  });
  return y;
}

ArrayP silu(const ArrayP &x0, int64_t rows, int64_t cols, bool gpu_ops) {
  if (x0->dtype != kF32) fail("ggml.silu: f32 only");
  require_tail_expf("ggml.silu", cols);
  if (cols <= 0 && x0->size() > 0) fail("ggml.silu: rows of zero columns");
  ArrayP x = contiguous(x0);
  auto y = new_array(kF32, x->shape);
  const int64_t n = x->size();
  if (!n) return y;
  const float *px = (const float *)x->data();
  float *py = (float *)y->data();
  const int go = gpu_ops ? 1 : 0;
  ArrayP kx = x;
  const int64_t c = cols;
  launch([=](hipStream_t s) {
    (void)kx;
    if (c % 4) silu_k<1><<<grid_cap(n, 256, 1 << 16), 256, 0, s>>>(n, c, go, px, py);
    else silu_k<0><<<grid_cap(n, 256, 1 << 16), 256, 0, s>>>(n, c, go, px, py);
  });
  return y;
}

ArrayP gelu_erf(const ArrayP &x0, bool tanh_form) {
  if (x0->dtype != kF32) fail("ggml.gelu_erf: f32 only");
  ArrayP x = contiguous(x0);
  auto y = new_array(kF32, x->shape);
  const int64_t n = x->size();
  if (!n) return y;
  if ((uintptr_t)x->data() % 16) {  // a view at an odd offset: the float4 path needs an aligned copy
    auto c = new_array(kF32, x->shape);
    copy_into(c, x);
    x = c;
  }
  const float *px = (const float *)x->data();
  float *py = (float *)y->data();
  const int tf = tanh_form ? 1 : 0;
  ArrayP kx = x;
  // 8192 blocks (32 per CU) of at least 4 float4 steps each
  static const int blocks = env_int("SHLO_GELU_BLOCKS", 8192);
  const int64_t n4 = n / 4;
  const int64_t per = kGeluU * 256;
  const int64_t steps = std::max<int64_t>(1, (n4 + per - 1) / per);
  const int64_t nb = std::max<int64_t>(1, std::min<int64_t>(blocks, steps));
  const int64_t chunk = (steps + nb - 1) / nb * per;
  const unsigned grid = (unsigned)std::max<int64_t>(1, (n4 + chunk - 1) / chunk);
  launch([=](hipStream_t s) {
    (void)kx;
    if (tf) gelu_erf_k<1><<<grid, 256, 0, s>>>(n, chunk, px, py);
    else gelu_erf_k<0><<<grid, 256, 0, s>>>(n, chunk, px, py);
  });
  return y;
}

ArrayP erff_map(uint32_t base, uint32_t count) {
  auto y = new_array(kU32, Shape{(int64_t)count});
  if (!count) return y;
  uint32_t *py = (uint32_t *)y->data();
  launch([=](hipStream_t s) { erff_map_k<<<grid_cap(count, 256, 256 * 16), 256, 0, s>>>(base, count, py); });
  return y;
}

ArrayP divide_exact(const ArrayP &a, const ArrayP &b) {
  if (a->dtype != kF32 || b->dtype != kF32) fail("divide: f32 only");
  return binary(kDiv, a, b);  // binary32 `/` is correctly rounded on gfx950 (IEEE division sequence)
}

ArrayP sqrt_exact(const ArrayP &a) {
  if (a->dtype != kF32) fail("sqrt: f32 only");
  return unary(kSqrt, a);  // correctly rounded sqrtf (the default HIP lowering)
}

ArrayP expf_map(uint32_t base, uint32_t count) {
  auto y = new_array(kU32, Shape{(int64_t)count});
  if (!count) return y;
  uint32_t *py = (uint32_t *)y->data();
  launch([=](hipStream_t s) { expf_map_k<<<grid_cap(count, 256, 256 * 16), 256, 0, s>>>(base, count, py); });
  return y;
}

float expf_host(float x) { return expfk::expf_cr(x); }

float erff_host(float x) { return erffk::erff_cr(x, &erffk::kPoly[0][0]); }

}  // namespace shlo
