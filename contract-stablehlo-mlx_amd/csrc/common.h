// Shared definitions of the MI355X StableHLO executor: dtype codes, errors,
// and the small value types every layer uses.  Host-side only.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>
#include <vector>

namespace shlo {

// dtype codes: the mlx_dtype enum order the reference binds
// (StablehloMlx/Mlx.lean:28-37): bool 0, u8 1, u16 2, u32 3, u64 4, i8 5,
// i16 6, i32 7, i64 8, f16 9, f32 10.
enum DType : uint8_t {
  kBool = 0, kU8 = 1, kU16 = 2, kU32 = 3, kU64 = 4, kI8 = 5, kI16 = 6,
  kI32 = 7, kI64 = 8, kF16 = 9, kF32 = 10, kF64 = 11
};

inline size_t dtype_size(uint8_t dt) {
  switch (dt) {
    case kBool: case kU8: case kI8: return 1;
    case kU16: case kI16: case kF16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
    default: return 0;
  }
}

inline bool dtype_valid(uint8_t dt) { return dtype_size(dt) != 0; }
inline bool dtype_is_float(uint8_t dt) { return dt == kF16 || dt == kF32 || dt == kF64; }
inline bool dtype_is_signed(uint8_t dt) {
  return dt == kI8 || dt == kI16 || dt == kI32 || dt == kI64;
}
const char *dtype_name(uint8_t dt);

// Every failure is raised as shlo::Error with a "what: detail" message; the
// C-ABI catches it, stores the text as the thread's last error and returns a
// nonzero status (the convention of c/smlx_shim.c:15-41).
struct Error : std::runtime_error {
  explicit Error(const std::string &m) : std::runtime_error(m) {}
};

[[noreturn]] void fail(const std::string &msg);
std::string strf(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

constexpr int kMaxRank = 16;

using Shape = std::vector<int64_t>;
inline int64_t shape_count(const Shape &s) {
  int64_t n = 1;
  for (int64_t d : s) n *= d;
  return n;
}
std::string shape_str(const Shape &s);

}  // namespace shlo
