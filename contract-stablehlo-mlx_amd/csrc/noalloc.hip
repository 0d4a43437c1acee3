// count_nonzero for callers that cannot allocate device memory (code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// shlo_count_nonzero (the comparator of the exhaustive erff check,
// c/smlx_shim.c:405-414) takes an array handle and allocates a device counter
// from the pool.  This variant takes plain device pointers and keeps its
// per-block partial counts in `scratch`, a file-scope device array: a first
// kernel writes one partial count per block (every slot it uses is written,
// so nothing needs clearing), a second sums the used slots in order into the
// caller's device word.  Both are queued on the executor's stream; nothing is
// allocated or freed, and no memset is recorded.
//
// Each GPU holds its own copy of `scratch` (4096 words, 32 KiB) for the life
// of the process.  Calls on one GPU share it: calls that overlap on one GPU
// from different streams or processes race on it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "ops.h"
#include "runtime.h"

namespace shlo {
namespace {

constexpr int kNzBlocks = 4096;  // partial counts held in the scratch array
constexpr int kNzThreads = 256;
constexpr int kMaxDevices = 64;
constexpr uint64_t kNzMaxCount = 1ull << 40;  // elements per call

static __device__ __align__(256) unsigned long long scratch[kNzBlocks];

__device__ __forceinline__ unsigned long long block_sum(unsigned long long v) {
  __shared__ unsigned long long w[kNzThreads / 64];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  if (threadIdx.x % 64 == 0) w[threadIdx.x / 64] = v;
  __syncthreads();
  unsigned long long t = 0;
#pragma unroll
  for (int i = 0; i < kNzThreads / 64; i++) t += w[i];
  return t;
}

// Block b counts the nonzero elements at b*256 + t + k*gridDim*256 and
// writes its count to part[b].
template <class T>
__global__ void __launch_bounds__(kNzThreads) nz_partial_k(const T *__restrict__ x, uint64_t n,
                                                           unsigned long long *__restrict__ part) {
  unsigned long long c = 0;
  for (uint64_t i = blockIdx.x * (uint64_t)kNzThreads + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kNzThreads)
    c += x[i] != (T)0;
  c = block_sum(c);
  if (threadIdx.x == 0) part[blockIdx.x] = c;
}

// One block: out = part[0] + ... + part[nparts - 1] (integers, exact).
__global__ void __launch_bounds__(kNzThreads) nz_final_k(const unsigned long long *__restrict__ part, int nparts,
                                                         unsigned long long *__restrict__ out) {
  unsigned long long c = 0;
  for (int i = threadIdx.x; i < nparts; i += kNzThreads) c += part[i];
  c = block_sum(c);
  if (threadIdx.x == 0) *out = c;
}

// The device address of `scratch` on each GPU, looked up once per device with
// that device current.  Host code uses these, never the array's name.
struct ScratchAddrs {
  std::mutex mu;
  unsigned long long *p[kMaxDevices] = {};
};
ScratchAddrs &scratch_addrs() {
  static ScratchAddrs *s = new ScratchAddrs;
  return *s;
}

unsigned long long *scratch_on(int dev) {
  if (dev < 0 || dev >= kMaxDevices) fail(strf("count_nonzero_noalloc: device %d is beyond the %d supported", dev,
                                               kMaxDevices));
  ScratchAddrs &s = scratch_addrs();
  std::lock_guard<std::mutex> g(s.mu);
  if (!s.p[dev]) {
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      fail(strf("count_nonzero_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e)));
    s.p[dev] = (unsigned long long *)ptr;
  }
  return s.p[dev];
}

// [p, p + bytes) must lie inside one device allocation: a kernel must never
// read or write outside the memory the caller owns.
void require_device_range(const void *p, uint64_t bytes, const char *what) {
  hipPointerAttribute_t at{};
  if (hipPointerGetAttributes(&at, p) != hipSuccess || at.type != hipMemoryTypeDevice) {
    (void)hipGetLastError();
    fail(strf("count_nonzero_noalloc: %s is not a device pointer", what));
  }
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)p) != hipSuccess) {
    (void)hipGetLastError();
    fail(strf("count_nonzero_noalloc: %s is not inside a device allocation", what));
  }
  const uint64_t off = (uint64_t)((const char *)p - (const char *)base);
  if (off > size || bytes > size - off)
    fail(strf("count_nonzero_noalloc: %s: %llu bytes from offset %llu overrun its %zu-byte allocation", what,
              (unsigned long long)bytes, (unsigned long long)off, size));
}

struct DeviceScope {
  int prev = -1;
  explicit DeviceScope(int dev) {
    SHLO_HIP(hipGetDevice(&prev));
    if (prev != dev) SHLO_HIP(hipSetDevice(dev));
  }
  ~DeviceScope() {
    int cur = -1;
    if (hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

}  // namespace

void count_nonzero_noalloc(const void *data, uint64_t count, uint32_t elem_bytes, uint64_t *out) {
  if (tracing()) fail("count_nonzero_noalloc: not available while a function is being traced");
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8)
    fail("count_nonzero_noalloc: elem_bytes must be 1, 2, 4 or 8");
  if (count > kNzMaxCount) fail(strf("count_nonzero_noalloc: at most %llu elements per call",
                                     (unsigned long long)kNzMaxCount));
  if (!out) fail("count_nonzero_noalloc: out is NULL");
  if (count && !data) fail("count_nonzero_noalloc: data is NULL");
  hipStream_t s = stream();  // the executor's device and stream
  const int dev = device_id();
  DeviceScope scope(dev);
  if (count) require_device_range(data, count * elem_bytes, "data");
  require_device_range(out, sizeof(uint64_t), "out");
  unsigned long long *part = scratch_on(dev);
  const uint64_t want = (count + kNzThreads - 1) / kNzThreads;
  const int blocks = (int)(want < (uint64_t)kNzBlocks ? want : (uint64_t)kNzBlocks);  // 0 when count == 0
  if (blocks > 0) {
    switch (elem_bytes) {
      case 1: nz_partial_k<uint8_t><<<blocks, kNzThreads, 0, s>>>((const uint8_t *)data, count, part); break;
      case 2: nz_partial_k<uint16_t><<<blocks, kNzThreads, 0, s>>>((const uint16_t *)data, count, part); break;
      case 4: nz_partial_k<uint32_t><<<blocks, kNzThreads, 0, s>>>((const uint32_t *)data, count, part); break;
      default: nz_partial_k<uint64_t><<<blocks, kNzThreads, 0, s>>>((const uint64_t *)data, count, part); break;
    }
    check_launch("count_nonzero_noalloc");
  }
  nz_final_k<<<1, kNzThreads, 0, s>>>(part, blocks, (unsigned long long *)out);
  check_launch("count_nonzero_noalloc");
}

}  // namespace shlo
