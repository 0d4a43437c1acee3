// The device-array runtime: the MI355X replacement for what mlx-c provides
// to the reference shim (c/smlx_shim.c:43-127, :266-273, :359-386).
//
// * One HIP stream per process (default priority), created on first use.
//   Every kernel and copy is ordered on it, so a buffer returned to the pool
//   can be handed to the next op without a host wait.
// * Arrays are immutable: every op returns a new Array.  Views (reshape of a
//   contiguous array, transpose, broadcast, slice) share the buffer and carry
//   element strides; kernels that need contiguous operands copy first.
// * Compiled mode: while a Trace is active, ops record their launches instead
//   of running them and every allocation is pinned to the trace.  The recorded
//   launches are then captured into one hipGraph (hipStreamBeginCapture /
//   hipStreamEndCapture / hipGraphInstantiate) and replayed per call.
#pragma once

#include <hip/hip_runtime.h>

#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "common.h"

namespace shlo {

#define SHLO_HIP(call)                                                        \
  do {                                                                        \
    hipError_t e_ = (call);                                                   \
    if (e_ != hipSuccess)                                                     \
      ::shlo::fail(::shlo::strf("%s: %s", #call, hipGetErrorString(e_)));     \
  } while (0)

// ---- device buffers ---------------------------------------------------------

struct Buffer {
  void *ptr = nullptr;
  size_t bytes = 0;    // capacity handed out by the pool
  bool owned = true;   // false: an alias of a compiled function's output buffer
  Buffer() = default;
  Buffer(const Buffer &) = delete;
  Buffer &operator=(const Buffer &) = delete;
  ~Buffer();  // returns the block to the pool
};
using BufferP = std::shared_ptr<Buffer>;

// A block of at least `bytes` (256-byte aligned) from the caching pool.
BufferP alloc_buffer(size_t bytes);

// Bytes the pool holds from hipMalloc (live + cached), and a full release of
// the cached blocks (after a device sync).
size_t pool_reserved_bytes();
void pool_trim();

// ---- arrays -----------------------------------------------------------------

struct Array {
  BufferP buf;           // null when size() == 0
  int64_t offset = 0;    // in elements
  uint8_t dtype = kF32;
  Shape shape;
  Shape strides;         // in elements, one per dim
  // A host copy of the bytes of small arrays made from host data (at most
  // kShadowBytes).  Kernel parameter arrays are read from it, so a dispatch
  // never waits on the device for its scalars.
  std::vector<uint8_t> shadow;
  static constexpr size_t kShadowBytes = 256;

  int rank() const { return (int)shape.size(); }
  int64_t size() const { return shape_count(shape); }
  size_t nbytes() const { return (size_t)size() * dtype_size(dtype); }
  bool contiguous() const;
  char *data() const {
    return buf ? (char *)buf->ptr + offset * (int64_t)dtype_size(dtype) : nullptr;
  }
};
using ArrayP = std::shared_ptr<const Array>;

Shape contiguous_strides(const Shape &shape);

// A new contiguous array of `shape` (uninitialised device memory).
std::shared_ptr<Array> new_array(uint8_t dtype, const Shape &shape);

// ---- stream, launches, tracing ---------------------------------------------

hipStream_t stream();
int device_id();
const hipDeviceProp_t &device_props();

using LaunchFn = std::function<void(hipStream_t)>;

// Run `fn` on the stream now, or record it when a trace is active.
void launch(LaunchFn fn);
// Check the last launch's error (eager mode).
void check_launch(const char *what);

struct Trace {
  std::vector<LaunchFn> ops;
  std::vector<BufferP> keep;  // every buffer allocated while tracing
};
Trace *current_trace();
void set_trace(Trace *t);
inline bool tracing() { return current_trace() != nullptr; }

// Host <-> device (synchronous with respect to the stream).
ArrayP array_from_host(const void *data, size_t nbytes, const Shape &shape, uint8_t dtype);
void array_to_host(const ArrayP &a, void *dst);  // a must be contiguous
void synchronize();

// ---- compiled functions (the mx::compile replacement) -----------------------

using HostFn = std::function<std::vector<ArrayP>(const std::vector<ArrayP> &)>;

struct CompiledFn {
  HostFn fn;
  bool compile = true;
  struct Variant;  // one per input signature
  std::vector<std::shared_ptr<Variant>> variants;
  ~CompiledFn();
};

std::vector<ArrayP> apply_fn(CompiledFn &f, const std::vector<ArrayP> &inputs);

// Fewest recorded launches a compiled function captures into a hipGraph
// (shorter traces re-issue their launches); the setter returns the old value.
size_t graph_min_ops();
size_t set_graph_min_ops(size_t n);

}  // namespace shlo
