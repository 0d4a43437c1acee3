// The C ABI (include/shlo_hip.h): one entry point per smlx_* function of the
// reference shim (c/smlx_shim.c), each a thin wrapper that unpacks handles,
// makes one executor call and boxes the result.  No numerics live here (the
// policy of c/smlx_shim.c:1-3).
#include "../../include/shlo_hip.h"

#include <cstring>
#include <string>

#include "stablehlo.h"

struct shlo_arr {
  shlo::ArrayP a;
};
struct shlo_kernel {
  std::string name;
};
struct shlo_fn {
  shlo::CompiledFn f;
  void *payload = nullptr;
  void (*payload_free)(void *) = nullptr;
  ~shlo_fn() {
    if (payload_free) payload_free(payload);
  }
};
struct shlo_module {
  shlo::Loaded l;
};

namespace {

thread_local std::string g_err;

template <class F>
int guard(const char *what, F &&f) {
  try {
    f();
    return 0;
  } catch (const std::exception &e) {
    g_err = std::string(what) + ": " + e.what();
  } catch (...) {
    g_err = std::string(what) + ": unknown error";
  }
  return 1;
}

shlo::ArrayP A(const shlo_arr *a) {
  if (!a || !a->a) shlo::fail("null array handle");
  return a->a;
}
shlo_arr *box(shlo::ArrayP a) { return new shlo_arr{std::move(a)}; }
void need(const void *p, const char *what) {
  if (!p) shlo::fail(std::string(what) + " is NULL");
}
shlo::Shape shape_of(const int64_t *s, size_t rank) {
  if (rank > (size_t)shlo::kMaxRank) shlo::fail("rank above 16");
  if (rank && !s) shlo::fail("shape is NULL");
  return shlo::Shape(s, s + rank);
}

// Scalar parameters of a kernel_apply: the u32 words of the last input
// (Run.lean:51-52), read from its host shadow when it has one.
std::vector<uint32_t> params_of(const shlo::ArrayP &p) {
  std::vector<uint8_t> bytes;
  if (!p->shadow.empty() && p->contiguous()) {
    bytes = p->shadow;
  } else {
    shlo::ArrayP c = shlo::contiguous(p);
    bytes.resize(c->nbytes());
    shlo::array_to_host(c, bytes.data());
  }
  if (shlo::dtype_size(p->dtype) != 4) shlo::fail("kernel parameters must be 32-bit words");
  std::vector<uint32_t> w(bytes.size() / 4);
  memcpy(w.data(), bytes.data(), w.size() * 4);
  w.resize(std::max<size_t>(w.size(), 8), 0);
  return w;
}

}  // namespace

extern "C" {

const char *shlo_last_error(void) { return g_err.c_str(); }
void shlo_set_error(const char *msg) { g_err = msg ? msg : ""; }

void shlo_arr_free(shlo_arr *a) { delete a; }

int shlo_empty(shlo_arr **out) {
  return guard("empty", [&] {
    need(out, "out");
    *out = box(shlo::empty_array());
  });
}

int shlo_of_bytes(const void *data, size_t nbytes, const int64_t *shape, size_t rank, uint8_t dtype, shlo_arr **out) {
  return guard("ofBytes", [&] {
    need(out, "out");
    if (nbytes) need(data, "data");
    *out = box(shlo::array_from_host(data, nbytes, shape_of(shape, rank), dtype));
  });
}

int shlo_to_bytes(const shlo_arr *a, void *dst, size_t cap, size_t *nbytes) {
  return guard("toBytes", [&] {
    shlo::ArrayP x = A(a);
    const size_t n = x->nbytes();
    if (nbytes) *nbytes = n;
    if (!dst) return;
    if (cap < n) shlo::fail(shlo::strf("buffer of %zu bytes for %zu", cap, n));
    shlo::ArrayP c = shlo::contiguous(x);
    shlo::array_to_host(c, dst);
  });
}

int shlo_shape(const shlo_arr *a, int64_t *shape, size_t cap, size_t *rank) {
  return guard("shape", [&] {
    shlo::ArrayP x = A(a);
    if (rank) *rank = x->shape.size();
    for (size_t i = 0; i < x->shape.size() && i < cap; i++) shape[i] = x->shape[i];
  });
}

int shlo_dtype(const shlo_arr *a, uint8_t *dtype) {
  return guard("dtype", [&] {
    need(dtype, "dtype");
    *dtype = A(a)->dtype;
  });
}

int shlo_unary(uint32_t op, const shlo_arr *a, shlo_arr **out) {
  return guard("unary", [&] { *out = box(shlo::unary(op, A(a))); });
}

int shlo_binary(uint32_t op, const shlo_arr *a, const shlo_arr *b, shlo_arr **out) {
  return guard("binary", [&] { *out = box(shlo::binary(op, A(a), A(b))); });
}

int shlo_where(const shlo_arr *c, const shlo_arr *a, const shlo_arr *b, shlo_arr **out) {
  return guard("where", [&] { *out = box(shlo::where(A(c), A(a), A(b))); });
}

int shlo_reshape(const shlo_arr *a, const int64_t *shape, size_t rank, shlo_arr **out) {
  return guard("reshape", [&] { *out = box(shlo::reshape(A(a), shape_of(shape, rank))); });
}

int shlo_transpose(const shlo_arr *a, const int64_t *perm, size_t n, shlo_arr **out) {
  return guard("transpose", [&] { *out = box(shlo::transpose(A(a), shape_of(perm, n))); });
}

int shlo_broadcast(const shlo_arr *a, const int64_t *shape, size_t rank, shlo_arr **out) {
  return guard("broadcast", [&] { *out = box(shlo::broadcast_to(A(a), shape_of(shape, rank))); });
}

int shlo_slice(const shlo_arr *a, const int64_t *start, const int64_t *stop, const int64_t *step, size_t n,
               shlo_arr **out) {
  return guard("slice", [&] {
    *out = box(shlo::slice(A(a), shape_of(start, n), shape_of(stop, n), shape_of(step, n)));
  });
}

int shlo_concat(const shlo_arr *const *xs, size_t n, uint32_t axis, shlo_arr **out) {
  return guard("concatenate", [&] {
    std::vector<shlo::ArrayP> v;
    for (size_t i = 0; i < n; i++) v.push_back(A(xs[i]));
    *out = box(shlo::concat(v, (int)axis));
  });
}

int shlo_astype(const shlo_arr *a, uint8_t dtype, shlo_arr **out) {
  return guard("astype", [&] { *out = box(shlo::astype(A(a), dtype)); });
}

int shlo_view(const shlo_arr *a, uint8_t dtype, shlo_arr **out) {
  return guard("view", [&] { *out = box(shlo::view_dtype(A(a), dtype)); });
}

int shlo_take(const shlo_arr *a, const shlo_arr *idx, uint32_t axis, shlo_arr **out) {
  return guard("take", [&] { *out = box(shlo::take(A(a), A(idx), (int)axis)); });
}

int shlo_max_axis(const shlo_arr *a, uint32_t axis, shlo_arr **out) {
  return guard("max_axis", [&] { *out = box(shlo::max_axis(A(a), (int)axis)); });
}

int shlo_contiguous(const shlo_arr *a, shlo_arr **out) {
  return guard("contiguous", [&] { *out = box(shlo::contiguous(A(a))); });
}

int shlo_eval(const shlo_arr *const *xs, size_t n) {
  return guard("eval", [&] {
    for (size_t i = 0; i < n; i++) (void)A(xs[i]);
    shlo::synchronize();
  });
}

// ---- kernels ---------------------------------------------------------------------

static const char *kKernels[] = {"mul_mat", "soft_max", "norm", "silu", "gelu_erf", "erff_map", "expf_map",
                                 "divide", "sqrt", "f64_ew", "f64_of_f32", "f32_of_f64"};

int shlo_kernel_new(const char *name, const char *const *inputs, size_t nin, const char *const *outputs, size_t nout,
                    const char *source, const char *header, shlo_kernel **out) {
  (void)inputs, (void)nin, (void)outputs, (void)nout, (void)source, (void)header;
  return guard("kernel", [&] {
    need(name, "name");
    need(out, "out");
    std::string n = name;
    if (n.compare(0, 5, "smlx_") == 0) n = n.substr(5);
    bool ok = false;
    for (auto *k : kKernels) ok |= n == k;
    if (!ok) shlo::fail("no precompiled kernel named " + std::string(name));
    *out = new shlo_kernel{n};
  });
}

void shlo_kernel_free(shlo_kernel *k) { delete k; }

int shlo_kernel_apply(const shlo_kernel *k, const shlo_arr *const *inputs, size_t nin, const int64_t *out_shapes,
                      const size_t *out_ranks, const uint8_t *out_dtypes, size_t nout, const int64_t *grid,
                      size_t grid_n, const int64_t *tg, size_t tg_n, shlo_arr **outs) {
  return guard("kernel apply", [&] {
    using namespace shlo;
    need(k, "kernel");
    (void)grid, (void)tg;
    if (grid_n != 3 || tg_n != 3) fail("kernel: grid and threadgroup need 3 entries");
    if (nout != 1) fail("kernel: one output is carried");
    std::vector<ArrayP> in;
    for (size_t i = 0; i < nin; i++) in.push_back(A(inputs[i]));
    const std::string &n = k->name;
    auto want = [&](size_t c) {
      if (in.size() != c) fail(strf("%s takes %zu inputs, got %zu", n.c_str(), c, in.size()));
    };
    ArrayP y;
    if (n == "mul_mat") {  // Run.lean:64-65: [w, x, p = K, M, R, wBatchStride, N, plain]
      want(3);
      auto p = params_of(in[2]);
      y = mul_mat(in[0], in[1], p[0], p[1], p[2], p[4], p[3], p[5] ? (int)kTailPlain : default_dot_tail());
    } else if (n == "soft_max") {  // [x, p = ncols, rows, scaleBits, floatSum]
      want(2);
      auto p = params_of(in[1]);
      y = soft_max(in[0], p[1], p[0], p[2], p[3] != 0);
    } else if (n == "norm") {  // [x, p = ncols, rows, epsBits, gpuOps]
      want(2);
      auto p = params_of(in[1]);
      y = norm(in[0], p[1], p[0], p[2], p[3] != 0);
    } else if (n == "silu") {  // [x, p = count, gpuOps]
      want(2);
      auto p = params_of(in[1]);
      ArrayP x = reshape(slice(reshape(in[0], Shape{in[0]->size()}), Shape{0}, Shape{(int64_t)p[0]}, Shape{1}),
                         Shape{(int64_t)p[0]});
      y = silu(x, 1, p[0], p[1] != 0);
    } else if (n == "gelu_erf") {  // [x, erffTable, p = count, gpuErf]; the table is the reference's, unused
      want(3);
      auto p = params_of(in[2]);
      ArrayP x = slice(reshape(in[0], Shape{in[0]->size()}), Shape{0}, Shape{(int64_t)p[0]}, Shape{1});
      y = gelu_erf(x, p[1] != 0);
    } else if (n == "erff_map") {  // [erffTable, p = base, count]
      want(2);
      auto p = params_of(in[1]);
      y = erff_map(p[0], p[1]);
    } else if (n == "expf_map") {  // [p = base, count]: the row tails' correctly rounded expf (no reference kernel)
      want(1);
      auto p = params_of(in[0]);
      y = expf_map(p[0], p[1]);
    } else if (n == "divide") {  // [a, b, p = count]
      want(3);
      y = divide_exact(in[0], in[1]);
    } else if (n == "sqrt") {  // [a, p = count]
      want(2);
      y = sqrt_exact(in[0]);
    } else if (n == "f64_ew") {  // [a, b, p = count, op] on binary64 bit patterns
      want(3);
      auto p = params_of(in[2]);
      ArrayP a = view_dtype(in[0], kF64), b = view_dtype(in[1], kF64);
      ArrayP r;
      switch (p[1]) {
        case 0: r = binary(kAdd, a, b); break;
        case 1: r = binary(kSub, a, b); break;
        case 2: r = binary(kMul, a, b); break;
        case 3: r = binary(kDiv, a, b); break;
        case 4: r = unary(kFloor, a); break;
        case 5: r = astype(a, kI64); break;
        default: fail("f64_ew: unknown op");
      }
      y = view_dtype(r, kU64);
    } else if (n == "f64_of_f32") {
      want(2);
      y = view_dtype(astype(in[0], kF64), kU64);
    } else if (n == "f32_of_f64") {
      want(2);
      y = astype(view_dtype(in[0], kF64), kF32);
    } else {
      fail("unknown kernel " + n);
    }
    Shape os = shape_of(out_shapes, out_ranks ? out_ranks[0] : 0);
    if (shape_count(os) != y->size()) fail("kernel: output shape does not match the kernel's output");
    if (out_dtypes && out_dtypes[0] != y->dtype) fail("kernel: output dtype does not match the kernel's output");
    outs[0] = box(reshape(y, os));
  });
}

// ---- compile / apply ----------------------------------------------------------------

int shlo_compile(shlo_traced_fn fn, void *payload, void (*payload_free)(void *), int enable, shlo_fn **out) {
  return guard("compile", [&] {
    if (!fn) shlo::fail("fn is NULL");
    need(out, "out");
    auto *f = new shlo_fn;
    f->payload = payload;
    f->payload_free = payload_free;
    f->f.compile = enable != 0;
    f->f.fn = [fn, payload](const std::vector<shlo::ArrayP> &ins) {
      std::vector<shlo_arr *> hin;
      for (auto &a : ins) hin.push_back(box(a));
      std::vector<shlo_arr *> hout(256, nullptr);
      size_t nout = 0;
      g_err.clear();
      const int rc = fn(payload, hin.data(), hin.size(), hout.data(), hout.size(), &nout);
      for (auto *h : hin) delete h;
      std::vector<shlo::ArrayP> res;
      for (size_t i = 0; i < nout && i < hout.size(); i++) {
        if (hout[i]) res.push_back(hout[i]->a);
        delete hout[i];
      }
      if (rc) shlo::fail("traced function: " + g_err);
      return res;
    };
    *out = f;
  });
}

void shlo_fn_free(shlo_fn *f) { delete f; }

static void apply_into(shlo_fn *f, const shlo_arr *const *inputs, size_t nin, shlo_arr **outs, size_t out_cap,
                       size_t *nout) {
  need(f, "fn");
  std::vector<shlo::ArrayP> in;
  for (size_t i = 0; i < nin; i++) in.push_back(A(inputs[i]));
  std::vector<shlo::ArrayP> r = shlo::apply_fn(f->f, in);
  if (nout) *nout = r.size();
  if (r.size() > out_cap) shlo::fail(shlo::strf("%zu outputs for room of %zu", r.size(), out_cap));
  for (size_t i = 0; i < r.size(); i++) outs[i] = box(r[i]);
}

int shlo_apply(shlo_fn *f, const shlo_arr *const *inputs, size_t nin, shlo_arr **outs, size_t out_cap,
               size_t *nout) {
  return guard("apply", [&] { apply_into(f, inputs, nin, outs, out_cap, nout); });
}

// ---- helpers -------------------------------------------------------------------------

int shlo_libm_erff_range(uint32_t base, uint32_t count, uint32_t *out) {
  return guard("libm_erff_range", [&] {
    if (count) need(out, "out");
    for (uint32_t i = 0; i < count; i++) {
      const float y = shlo::erff_host(__builtin_bit_cast(float, base + i));
      out[i] = __builtin_bit_cast(uint32_t, y);
    }
  });
}

int shlo_expf_range(uint32_t base, uint32_t count, uint32_t *out) {
  return guard("expf_range", [&] {
    if (count) need(out, "out");
    for (uint32_t i = 0; i < count; i++) {
      const float y = shlo::expf_host(__builtin_bit_cast(float, base + i));
      out[i] = __builtin_bit_cast(uint32_t, y);
    }
  });
}

int shlo_count_nonzero(const shlo_arr *a, uint64_t *out) {
  return guard("count_nonzero", [&] {
    need(out, "out");
    *out = (uint64_t)shlo::count_nonzero(A(a));
  });
}

// ---- executor surface -------------------------------------------------------------------

int shlo_module_load(const char *text, size_t len, shlo_module **out) {
  return guard("load", [&] {
    need(text, "text");
    need(out, "out");
    auto *m = new shlo_module;
    try {
      m->l = shlo::load_module(std::string(text, len));
    } catch (...) {
      delete m;
      throw;
    }
    *out = m;
  });
}

void shlo_module_free(shlo_module *m) { delete m; }

int shlo_module_nargs(const shlo_module *m, size_t *n) {
  return guard("argTys", [&] {
    need(m, "module");
    *n = m->l.main().body.args.size();
  });
}

int shlo_module_arg(const shlo_module *m, size_t i, int64_t *shape, size_t cap, size_t *rank, uint8_t *dtype) {
  return guard("argTys", [&] {
    need(m, "module");
    const auto &args = m->l.main().body.args;
    if (i >= args.size()) shlo::fail("argument index out of range");
    const shlo::Ty &t = args[i].second;
    if (rank) *rank = t.dims.size();
    for (size_t k = 0; k < t.dims.size() && k < cap; k++) shape[k] = t.dims[k];
    if (dtype) *dtype = shlo::el_dtype(t.el);
  });
}

int shlo_module_prepare(const shlo_module *m, uint64_t faults, int compile, shlo_fn **out) {
  return guard("prepare", [&] {
    need(m, "module");
    need(out, "out");
    auto *f = new shlo_fn;
    auto loaded = std::make_shared<shlo::Loaded>(m->l);
    const shlo::Faults fl = shlo::Faults::from_bits(faults);
    f->f.compile = compile != 0;
    f->f.fn = [loaded, fl](const std::vector<shlo::ArrayP> &ins) {
      return shlo::run_func(loaded->module, fl, loaded->main(), ins);
    };
    *out = f;
  });
}

int shlo_call(shlo_fn *f, const shlo_arr *const *inputs, size_t nin, shlo_arr **outs, size_t out_cap,
              size_t *nout) {
  return guard("call", [&] {
    apply_into(f, inputs, nin, outs, out_cap, nout);
    shlo::synchronize();
  });
}

int shlo_set_flavor(int flavor) {
  return guard("flavor", [&] { shlo::set_default_dot_tail(flavor); });
}
int shlo_get_flavor(void) { return shlo::default_dot_tail(); }

int shlo_set_graph_min_ops(int n, int *prev) {
  return guard("graph_min_ops", [&] {
    if (n < 1) shlo::fail("graph_min_ops: n must be at least 1");
    const size_t old = shlo::set_graph_min_ops((size_t)n);
    if (prev) *prev = (int)old;
  });
}

int shlo_fill_random(const int64_t *shape, size_t rank, uint32_t seed, uint64_t skip, int dist, double param,
                     shlo_arr **out) {
  return guard("fill_random", [&] {
    need(out, "out");
    *out = box(shlo::fill_random(shape_of(shape, rank), seed, skip, dist, param));
  });
}

int shlo_checksum_u32(const shlo_arr *a, uint64_t start_index, uint64_t *out) {
  return guard("checksum", [&] {
    need(out, "out");
    *out = shlo::checksum_u32(A(a), start_index);
  });
}

int shlo_sync(void) {
  return guard("sync", [&] { shlo::synchronize(); });
}

static hipEvent_t g_ev[2];
int shlo_timer_start(void) {
  return guard("timer", [&] {
    if (!g_ev[0]) {
      SHLO_HIP(hipEventCreate(&g_ev[0]));
      SHLO_HIP(hipEventCreate(&g_ev[1]));
    }
    SHLO_HIP(hipEventRecord(g_ev[0], shlo::stream()));
  });
}
int shlo_timer_stop(float *ms) {
  return guard("timer", [&] {
    need(ms, "ms");
    if (!g_ev[0]) shlo::fail("timer not started");
    SHLO_HIP(hipEventRecord(g_ev[1], shlo::stream()));
    SHLO_HIP(hipEventSynchronize(g_ev[1]));
    SHLO_HIP(hipEventElapsedTime(ms, g_ev[0], g_ev[1]));
  });
}

int shlo_time_apply(shlo_fn *f, const shlo_arr *const *inputs, size_t nin, int reps, float *ms) {
  return guard("time_apply", [&] {
    need(f, "fn");
    need(ms, "ms");
    if (reps < 1) shlo::fail("reps must be >= 1");
    std::vector<shlo::ArrayP> in;
    for (size_t i = 0; i < nin; i++) in.push_back(A(inputs[i]));
    (void)shlo::apply_fn(f->f, in);  // trace/instantiate outside the timed region
    SHLO_HIP(hipStreamSynchronize(shlo::stream()));
    hipEvent_t e0, e1;
    SHLO_HIP(hipEventCreate(&e0));
    SHLO_HIP(hipEventCreate(&e1));
    SHLO_HIP(hipEventRecord(e0, shlo::stream()));
    for (int r = 0; r < reps; r++) (void)shlo::apply_fn(f->f, in);
    SHLO_HIP(hipEventRecord(e1, shlo::stream()));
    SHLO_HIP(hipEventSynchronize(e1));
    float t = 0;
    SHLO_HIP(hipEventElapsedTime(&t, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *ms = t / (float)reps;
  });
}

int shlo_device_info(char *name, size_t cap, int *cus, uint64_t *pool_bytes) {
  return guard("device_info", [&] {
    const hipDeviceProp_t &p = shlo::device_props();
    if (name && cap) {
      snprintf(name, cap, "%s (%s)", p.name, p.gcnArchName);
    }
    if (cus) *cus = p.multiProcessorCount;
    if (pool_bytes) *pool_bytes = shlo::pool_reserved_bytes();
  });
}

int shlo_count_nonzero_noalloc(const void *data, uint64_t count, uint32_t elem_bytes, uint64_t *out_device) {
  return guard("count_nonzero_noalloc", [&] { shlo::count_nonzero_noalloc(data, count, elem_bytes, out_device); });
}

int shlo_last_dot_kernel(char *name, size_t cap) {
  return guard("last_dot_kernel", [&] {
    need(name, "name");
    if (!cap) shlo::fail("cap must be at least 1");
    snprintf(name, cap, "%s", shlo::last_dot_kernel().c_str());
  });
}

int shlo_data_ptr(const shlo_arr *a, void **ptr) {
  return guard("data_ptr", [&] {
    need(ptr, "ptr");
    *ptr = A(a)->data();
  });
}

}  // extern "C"
