// Array operations: the MI355X counterparts of the mlx-c calls the reference
// shim makes (c/smlx_shim.c:142-264, :301-323, :388-414) and of the exact
// kernels its Run.lean dispatches (StablehloMlx/Kernels/Run.lean:64-104).
#pragma once

#include "runtime.h"

namespace shlo {

// Unary op codes (StablehloMlx/Mlx.lean:76-87).
enum UnaryOp : uint32_t {
  kNeg = 0, kAbs = 1, kSqrt = 2, kFloor = 3, kExp = 4, kErf = 5, kNot = 6,
  kInvert = 7, kRsqrt = 8, kTanh = 9, kSigmoid = 10
};
// Binary op codes (StablehloMlx/Mlx.lean:88-108).
enum BinaryOp : uint32_t {
  kAdd = 0, kSub = 1, kMul = 2, kDiv = 3, kMax = 4, kMin = 5, kAnd = 6, kOr = 7,
  kXor = 8, kShl = 9, kShr = 10, kEq = 11, kNe = 12, kLt = 13, kLe = 14, kGt = 15,
  kGe = 16, kMatmul = 17, kRem = 18, kLAnd = 19, kLOr = 20
};
// Internal codes for the planted "built-in" lowerings only: the GPU's
// reciprocal-based binary32 divide and its raw v_sqrt_f32, neither correctly
// rounded (the role of MLX's own / and sqrt, Lower.lean:383-390).
constexpr uint32_t kDivApprox = 100;
constexpr uint32_t kSqrtApprox = 101;

// ---- views (no device work) -------------------------------------------------
ArrayP reshape(const ArrayP &a, const Shape &shape);
ArrayP transpose(const ArrayP &a, const std::vector<int64_t> &perm);
ArrayP broadcast_to(const ArrayP &a, const Shape &shape);
ArrayP slice(const ArrayP &a, const Shape &start, const Shape &stop, const Shape &step);
ArrayP empty_array();

// ---- data movement and elementwise kernels ----------------------------------
ArrayP contiguous(const ArrayP &a);
// Copies src's elements (in its logical order) to dst_base laid out with
// dst_strides (elements, one per dim of src), on the executor's stream.
void copy_to_strides(const ArrayP &src, const Shape &dst_strides, char *dst_base);
void copy_into(const std::shared_ptr<Array> &dst, const ArrayP &src);  // eager
ArrayP concat(const std::vector<ArrayP> &xs, int axis);
ArrayP astype(const ArrayP &a, uint8_t dtype);
ArrayP view_dtype(const ArrayP &a, uint8_t dtype);
ArrayP unary(uint32_t op, const ArrayP &a);
ArrayP binary(uint32_t op, const ArrayP &a, const ArrayP &b);
ArrayP where(const ArrayP &c, const ArrayP &a, const ArrayP &b);
ArrayP take(const ArrayP &a, const ArrayP &idx, int axis);
ArrayP max_axis(const ArrayP &a, int axis);
ArrayP iota(uint8_t dtype, const Shape &shape, int dim);
int64_t count_nonzero(const ArrayP &a);
// sum over t of (w[t]+1)*(2(start+t)+1)*0x9E3779B97F4A7C15 mod 2^64 over 32-bit words.
uint64_t checksum_u32(const ArrayP &a, uint64_t start);
Shape broadcast_shapes(const Shape &a, const Shape &b);

// Device-side fill from the splitmix32 stream of ref/ggml_ref.c:21-30:
// dist 0 = unif(param) one draw per element; dist 1 = the Irwin-Hall normal
// (12 draws per element) times sigma = param.  `skip` draws are skipped first.
ArrayP fill_random(const Shape &shape, uint32_t seed, uint64_t skip, int dist, double param);

// MLX-style matmul of [..., N, K] x [..., K, M] in a natural (non-ggml) order:
// the planted "built-in matmul" lowering (StablehloMlx/Lower.lean:177-180).
ArrayP matmul_builtin(const ArrayP &a, const ArrayP &b);

// ---- the exact ggml kernels -------------------------------------------------

// Tail flavour of ggml_vec_dot_f32 past the last full block of 16
// (Shaders.lean:80-90; evidence/README.md:41-46).
enum DotTail : int { kTailStock = 0, kTailPinned = 1, kTailPlain = 2 };
int default_dot_tail();          // process-wide flavour for dot_general
void set_default_dot_tail(int);  // 0 stock (the reference kernel), 1 pinned

// One operand of a dot product, addressed as (batch, free, k) with element
// strides: element (b, f, k) is at data + b*sb + f*sf + k*sk.
// With nb2 > 1 the batch index b = b1 * nb2 + b2 takes two strides:
// element (b, f, k) is at data + b1*sb + b2*sb2 + f*sf + k*sk.
struct DotOperand {
  ArrayP arr;       // keeps the buffer alive
  int64_t sb = 0, sf = 0, sk = 0;
  int64_t sb2 = 0, nb2 = 1;
  int64_t rows_alloc = 0;  // rows readable in each batch (a padded copy's), 0: the logical rows
};

// One element-wise binary32 op fused into a producer's store: v = op(v, o)
// (op(o, v) when `rev`), o the element of `arr` at i0*s0 + i1*s1 + i2*s2 for
// the producer's output index (i0, i1, i2).  Same bits as the separate op.
constexpr int kMaxEpi = 4;  // fused ops per producer
constexpr uint32_t kEpiGeluErf = 0x100;  // FusedOp code of ggml gelu_erf (no operand)
struct FusedOp {
  ArrayP arr;  // f32; keeps the buffer alive
  int64_t s0 = 0, s1 = 0, s2 = 0;
  uint32_t code = 0;  // kAdd, kSub, kMul, kDiv, kMax, kMin
  bool rev = false;
};

// y[(b*N + n)*M + m] = dot over k of lhs(b, n, k) and rhs(b, m, k), each
// output in ggml_vec_dot_f32's order (16 FMA accumulators over blocks of 16,
// GGML_F32x4_REDUCE, vaddvq_f32, then the tail), then the fused ops `epi` at
// index (b, n, m) in order (at most 4).  Output shape [B*N*M].
ArrayP dot_ggml(const DotOperand &lhs, const DotOperand &rhs, int64_t B, int64_t N, int64_t M,
                int64_t K, int tail, const std::vector<FusedOp> &epi = {});

// softmax(chain1(Q K^T)) V in one kernel (S and P stay in LDS), for q, k
// (b, query / key, d) and v (b, key, e) with DH = 64 head dims, DV = 64 value
// columns, NK keys a multiple of 256 up to 1024 and NQ queries a multiple of
// 32: the same bits as dot_ggml, its chain, soft_max and dot_ggml again.
// chain2 applies to the output at (b, n, e).  Returns null when the shapes or
// layouts are not carried (the caller runs the separate ops).  Output
// [B*NQ*DV].
ArrayP attention_ggml(const DotOperand &q, const DotOperand &k, const DotOperand &v, int64_t B, int64_t NQ,
                      int64_t NK, int64_t DH, int64_t DV, const std::vector<FusedOp> &epi1, uint32_t sm_scale_bits,
                      const std::vector<FusedOp> &epi2);

// The kernel the last dot_ggml call chose, e.g. "dot_mfma8d_k<RowVecB,ColQuadB,128,8>"
// (host bookkeeping for tests and profiles; "" before the first call).
const std::string &last_dot_kernel();

// The reference's Run.mulMat surface (Run.lean:64-65): w rows of K, x rows
// of K; y[r*M + m] = dot(w row (r/N)*wBatchStride/K + m, x row r).
ArrayP mul_mat(const ArrayP &w, const ArrayP &x, int64_t K, int64_t M, int64_t R, int64_t N,
               int64_t wBatchStride, int tail);

// ggml soft_max over `rows` rows of `cols` (Shaders.lean:100-123).  A row
// tail (cols % 4 elements) is carried in the pinned flavour only, through the
// correctly rounded expf.
ArrayP soft_max(const ArrayP &x, int64_t rows, int64_t cols, uint32_t scale_bits, bool float_sum);
// ggml norm (Shaders.lean:130-166), then the fused ops `epi` at index
// (0, row, column) (none with the planted gpu_ops; rows of at most
// 4 * 64 * kNormEpiJ columns).
constexpr int kNormEpiJ = 4;
ArrayP norm(const ArrayP &x, int64_t rows, int64_t cols, uint32_t eps_bits, bool gpu_ops,
            const std::vector<FusedOp> &epi = {});
// ggml silu on rows of `cols` (Shaders.lean:172-179); row tails as soft_max.
ArrayP silu(const ArrayP &x, int64_t rows, int64_t cols, bool gpu_ops);
// ggml gelu_erf (Shaders.lean:186-199) with a correctly rounded erff.
ArrayP gelu_erf(const ArrayP &x, bool tanh_form);
// y[t] = bits(erff(bits^-1(base + t))), t < count (Shaders.lean:204-208).
ArrayP erff_map(uint32_t base, uint32_t count);
// Correctly rounded binary32 / and sqrt (Shaders.lean:213-221).
ArrayP divide_exact(const ArrayP &a, const ArrayP &b);
ArrayP sqrt_exact(const ArrayP &a);

// Host copy of the product's erff (the same routine the kernels run), for the
// CPU side of the exhaustive check (c/smlx_shim.c:388-403).
float erff_host(float x);
// y[t] = bits(expf(bits^-1(base + t))) with the correctly rounded expf of the
// row tails (no reference counterpart: the exhaustive check of that expf).
ArrayP expf_map(uint32_t base, uint32_t count);
float expf_host(float x);
// count_nonzero over `count` elements of elem_bytes (1, 2, 4, 8) at device
// address `data`, written to the device word `out`, queued on the executor's
// stream; its partial counts live in a static device array, so it allocates
// nothing (noalloc.hip).
void count_nonzero_noalloc(const void *data, uint64_t count, uint32_t elem_bytes, uint64_t *out);
// Refuses a row tail (cols % 4 != 0) unless the pinned flavour is selected.
void require_tail_expf(const char *op, int64_t cols);

}  // namespace shlo
