// Device-array runtime: pool, stream, tracing and hipGraph replay.
#include "runtime.h"

#include <algorithm>
#include <cstdarg>
#include <cstdlib>
#include <map>
#include <mutex>

#include "ops.h"

namespace shlo {

// ---- errors and small helpers ----------------------------------------------

[[noreturn]] void fail(const std::string &msg) { throw Error(msg); }

std::string strf(const char *fmt, ...) {
  char buf[2048];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return buf;
}

std::string shape_str(const Shape &s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); i++) r += (i ? "," : "") + std::to_string(s[i]);
  return r + "]";
}

const char *dtype_name(uint8_t dt) {
  switch (dt) {
    case kBool: return "bool";
    case kU8: return "u8";
    case kU16: return "u16";
    case kU32: return "u32";
    case kU64: return "u64";
    case kI8: return "i8";
    case kI16: return "i16";
    case kI32: return "i32";
    case kI64: return "i64";
    case kF16: return "f16";
    case kF32: return "f32";
    case kF64: return "f64";
    default: return "?";
  }
}

// ---- the caching pool ------------------------------------------------------

namespace {

struct Pool {
  std::mutex mu;
  std::multimap<size_t, void *> free_blocks;  // capacity -> block
  size_t reserved = 0;

  static size_t round_up(size_t b) {
    if (b == 0) b = 1;
    size_t q = b <= (1u << 20) ? 256 : b <= (64u << 20) ? (64u << 10) : (2u << 20);
    return (b + q - 1) / q * q;
  }

  void *get(size_t bytes, size_t *cap) {
    const size_t want = round_up(bytes);
    {
      std::lock_guard<std::mutex> g(mu);
      auto it = free_blocks.lower_bound(want);
      // Accept a cached block up to 25% (plus 2 MiB) larger than asked.
      if (it != free_blocks.end() && it->first <= want + want / 4 + (2u << 20)) {
        void *p = it->second;
        *cap = it->first;
        free_blocks.erase(it);
        return p;
      }
    }
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) {
      // Release the cache and try once more.
      (void)hipGetLastError();
      trim();
      e = hipMalloc(&p, want);
      if (e != hipSuccess) fail(strf("hipMalloc(%zu): %s", want, hipGetErrorString(e)));
    }
    std::lock_guard<std::mutex> g(mu);
    reserved += want;
    *cap = want;
    return p;
  }

  void put(void *p, size_t cap) {
    std::lock_guard<std::mutex> g(mu);
    free_blocks.emplace(cap, p);
  }

  void trim() {
    (void)hipStreamSynchronize(stream());
    std::lock_guard<std::mutex> g(mu);
    for (auto &kv : free_blocks) {
      (void)hipFree(kv.second);
      reserved -= kv.first;
    }
    free_blocks.clear();
  }
};

// Never destroyed: arrays held by the host program may outlive static
// destructors at exit.
Pool &pool() {
  static Pool *p = new Pool;
  return *p;
}

thread_local Trace *g_trace = nullptr;

}  // namespace

Buffer::~Buffer() {
  if (ptr && owned) pool().put(ptr, bytes);
}

BufferP alloc_buffer(size_t bytes) {
  auto b = std::make_shared<Buffer>();
  b->ptr = pool().get(bytes, &b->bytes);
  if (g_trace) g_trace->keep.push_back(b);
  return b;
}

size_t pool_reserved_bytes() {
  std::lock_guard<std::mutex> g(pool().mu);
  return pool().reserved;
}

void pool_trim() { pool().trim(); }

// ---- arrays ----------------------------------------------------------------

Shape contiguous_strides(const Shape &shape) {
  Shape s(shape.size());
  int64_t acc = 1;
  for (int i = (int)shape.size() - 1; i >= 0; i--) {
    s[i] = acc;
    acc *= shape[i];
  }
  return s;
}

bool Array::contiguous() const {
  int64_t acc = 1;
  for (int i = rank() - 1; i >= 0; i--) {
    if (shape[i] != 1 && strides[i] != acc) return false;
    acc *= shape[i];
  }
  return true;
}

std::shared_ptr<Array> new_array(uint8_t dtype, const Shape &shape) {
  if (!dtype_valid(dtype)) fail(strf("dtype %u is not carried", dtype));
  if ((int)shape.size() > kMaxRank) fail("rank above 16");
  for (int64_t d : shape)
    if (d < 0) fail("negative dimension in " + shape_str(shape));
  auto a = std::make_shared<Array>();
  a->dtype = dtype;
  a->shape = shape;
  a->strides = contiguous_strides(shape);
  const size_t n = a->nbytes();
  if (n) a->buf = alloc_buffer(n);
  return a;
}

// ---- device and stream -----------------------------------------------------

namespace {
struct Dev {
  int id = 0;
  hipStream_t s = nullptr;
  hipDeviceProp_t props{};
};
Dev &dev() {
  static Dev *d = [] {
    auto *x = new Dev;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) fail("no HIP device is visible (the executor needs an MI355X)");
    SHLO_HIP(hipGetDevice(&x->id));
    SHLO_HIP(hipGetDeviceProperties(&x->props, x->id));
    // Default priority, non-blocking with respect to the null stream.
    SHLO_HIP(hipStreamCreateWithFlags(&x->s, hipStreamNonBlocking));
    return x;
  }();
  return *d;
}
}  // namespace

hipStream_t stream() { return dev().s; }
int device_id() { return dev().id; }
const hipDeviceProp_t &device_props() { return dev().props; }

Trace *current_trace() { return g_trace; }
void set_trace(Trace *t) { g_trace = t; }

void check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail(strf("%s: launch failed: %s", what, hipGetErrorString(e)));
}

void launch(LaunchFn fn) {
  if (g_trace) {
    g_trace->ops.push_back(std::move(fn));
    return;
  }
  fn(stream());
  check_launch("kernel");
}

void synchronize() {
  if (g_trace) return;  // nothing has run yet; the graph runs at apply time
  SHLO_HIP(hipStreamSynchronize(stream()));
}

ArrayP array_from_host(const void *data, size_t nbytes, const Shape &shape, uint8_t dtype) {
  auto a = new_array(dtype, shape);
  if (a->nbytes() != nbytes) fail("ofBytes: byte count does not match the shape");
  if (nbytes) {
    // Ordered on the executor's stream: the pool may hand out a block that a
    // kernel queued earlier on that stream still writes (the stream is
    // non-blocking, so a copy on the null stream would not wait for it).
    // Constants made while tracing are uploaded once, here, outside the
    // recorded launches; the graph only reads them.
    SHLO_HIP(hipMemcpyAsync(a->data(), data, nbytes, hipMemcpyHostToDevice, stream()));
    SHLO_HIP(hipStreamSynchronize(stream()));
  }
  if (nbytes <= Array::kShadowBytes) a->shadow.assign((const uint8_t *)data, (const uint8_t *)data + nbytes);
  return a;
}

void array_to_host(const ArrayP &a, void *dst) {
  if (g_trace) fail("toBytes: not available while a function is being traced");
  if (!a->contiguous()) fail("toBytes: array is not contiguous");
  if (a->nbytes() == 0) return;
  SHLO_HIP(hipMemcpyAsync(dst, a->data(), a->nbytes(), hipMemcpyDeviceToHost, stream()));
  SHLO_HIP(hipStreamSynchronize(stream()));
}

// ---- compiled functions -----------------------------------------------------

struct CompiledFn::Variant {
  std::vector<std::pair<uint8_t, Shape>> sig;
  Trace trace;
  std::vector<std::shared_ptr<Array>> slots;
  std::vector<std::weak_ptr<const Array>> last_in;
  std::vector<ArrayP> outs;
  // Buffers handed to the caller by the last apply: they alias the graph's
  // output buffers (no copy on the common path).
  std::vector<std::weak_ptr<Buffer>> handed;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  ~Variant();
};

// Outputs of the last apply that the caller still holds move to blocks of
// their own before the graph overwrites its buffers or the function goes away
// (their contents are unchanged: arrays stay immutable).
static void evacuate(CompiledFn::Variant &v) {
  for (auto &w : v.handed) {
    if (std::shared_ptr<Buffer> b = w.lock()) {
      size_t cap = 0;
      void *p = pool().get(b->bytes, &cap);
      SHLO_HIP(hipMemcpyAsync(p, b->ptr, b->bytes, hipMemcpyDeviceToDevice, stream()));
      b->ptr = p;
      b->bytes = cap;
      b->owned = true;
    }
  }
  v.handed.clear();
}

CompiledFn::Variant::~Variant() {
  try {
    evacuate(*this);
  } catch (...) {
  }
  (void)hipStreamSynchronize(stream());
  if (exec) (void)hipGraphExecDestroy(exec);
  if (graph) (void)hipGraphDestroy(graph);
}

CompiledFn::~CompiledFn() {
  if (!variants.empty()) (void)hipStreamSynchronize(stream());
}

namespace {
struct TraceScope {
  Trace *prev;
  explicit TraceScope(Trace *t) : prev(g_trace) { g_trace = t; }
  ~TraceScope() { g_trace = prev; }
};
}  // namespace

// Traces of fewer launches than this replay their recorded launches straight
// onto the stream; longer ones are captured into a hipGraph.  A graph launch
// costs the stream a gap of several microseconds before its first kernel, more
// than issuing a few dozen kernels (which queue back to back behind a busy
// GPU); a graph saves host time on long traces.  SHLO_GRAPH_MIN_OPS sets the
// initial value.
static size_t &graph_min_ops_ref() {
  static size_t n = [] {
    const char *e = getenv("SHLO_GRAPH_MIN_OPS");
    return e ? (size_t)std::max(1, atoi(e)) : (size_t)32;
  }();
  return n;
}
size_t graph_min_ops() { return graph_min_ops_ref(); }
size_t set_graph_min_ops(size_t n) {
  const size_t prev = graph_min_ops_ref();
  graph_min_ops_ref() = std::max<size_t>(1, n);
  return prev;
}

static CompiledFn::Variant &variant_for(CompiledFn &f, const std::vector<ArrayP> &in) {
  for (auto &v : f.variants) {
    if (v->sig.size() != in.size()) continue;
    bool same = true;
    for (size_t i = 0; i < in.size() && same; i++)
      same = v->sig[i].first == in[i]->dtype && v->sig[i].second == in[i]->shape;
    if (same) return *v;
  }
  if (g_trace) fail("compile: a compiled function cannot be traced inside another trace");
  auto v = std::make_shared<CompiledFn::Variant>();
  for (auto &a : in) {
    v->sig.emplace_back(a->dtype, a->shape);
    v->slots.push_back(new_array(a->dtype, a->shape));
    v->last_in.emplace_back();
  }
  {
    TraceScope ts(&v->trace);
    std::vector<ArrayP> ins(v->slots.begin(), v->slots.end());
    std::vector<ArrayP> outs = f.fn(ins);
    for (auto &o : outs) v->outs.push_back(o->contiguous() ? o : contiguous(o));
  }
  if (v->trace.ops.size() >= graph_min_ops()) {
    hipStream_t s = stream();
    SHLO_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    try {
      for (auto &op : v->trace.ops) op(s);
    } catch (...) {
      hipGraph_t g = nullptr;
      (void)hipStreamEndCapture(s, &g);
      if (g) (void)hipGraphDestroy(g);
      throw;
    }
    SHLO_HIP(hipStreamEndCapture(s, &v->graph));
    SHLO_HIP(hipGraphInstantiate(&v->exec, v->graph, nullptr, nullptr, 0));
  }
  f.variants.push_back(std::move(v));
  return *f.variants.back();
}

std::vector<ArrayP> apply_fn(CompiledFn &f, const std::vector<ArrayP> &inputs) {
  if (!f.compile || g_trace) return f.fn(inputs);
  CompiledFn::Variant &v = variant_for(f, inputs);
  hipStream_t s = stream();
  evacuate(v);
  for (size_t i = 0; i < inputs.size(); i++) {
    if (v.last_in[i].lock() == inputs[i]) continue;  // arrays are immutable
    copy_into(v.slots[i], inputs[i]);
    v.last_in[i] = inputs[i];
  }
  if (v.exec) {
    SHLO_HIP(hipGraphLaunch(v.exec, s));
  } else {
    for (auto &op : v.trace.ops) op(s);  // a short trace: its launches, re-issued
  }
  std::vector<ArrayP> res;
  for (auto &o : v.outs) {
    auto r = std::make_shared<Array>();
    r->dtype = o->dtype;
    r->shape = o->shape;
    r->strides = o->strides;
    r->offset = o->offset;
    if (o->buf) {
      auto alias = std::make_shared<Buffer>();
      alias->ptr = o->buf->ptr;
      alias->bytes = o->buf->bytes;
      alias->owned = false;
      r->buf = alias;
      v.handed.push_back(alias);
    }
    res.push_back(r);
  }
  return res;
}

}  // namespace shlo
