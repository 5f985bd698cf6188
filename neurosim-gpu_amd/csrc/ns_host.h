// Host-side helpers shared by the C-ABI entry points: thread-local error
// text, operand conversion and overlap checks.  All validation runs before
// any launch, so a failing call leaves every buffer untouched.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "ns_common.h"
#include "ns_error.h"

namespace ns {

inline int fail_launch(const char* what, hipError_t err) {
  snprintf(error_buffer(), 512, "%s launch failed: %s", what, hipGetErrorString(err));
  return NS_ERR_LAUNCH;
}

// Byte range [lo, hi) touched by a strided [B,N] float32 view (empty if absent).
struct Extent {
  uintptr_t lo, hi;
};

inline Extent extent_of(const void* data, int64_t sb, int64_t sn, int64_t batch, int64_t n) {
  if (!data || batch <= 0 || n <= 0) return Extent{0, 0};
  const uintptr_t lo = reinterpret_cast<uintptr_t>(data);
  const int64_t last = (batch - 1) * (sb < 0 ? -sb : sb) + (n - 1) * (sn < 0 ? -sn : sn);
  return Extent{lo, lo + static_cast<uintptr_t>((last + 1) * 4)};
}

inline Extent extent(const ns_plane& p, int64_t b, int64_t n) {
  return extent_of(p.data, p.stride_b, p.stride_n, b, n);
}
inline Extent extent(const ns_out_plane& p, int64_t b, int64_t n) {
  return extent_of(p.data, p.stride_b, p.stride_n, b, n);
}

// Whether a [B,N] view with strides (sb, sn) gives every (b, n) its own element
// (no zero stride, and the two strides do not interleave).
inline bool distinct_elements(int64_t sb, int64_t sn, int64_t B, int64_t N) {
  sb = sb < 0 ? -sb : sb;
  sn = sn < 0 ? -sn : sn;
  if (B <= 1) return N <= 1 || sn > 0;
  if (N <= 1) return sb > 0;
  return (sn > 0 && sb >= N * sn) || (sb > 0 && sn >= B * sb);
}

inline bool overlaps(const Extent& x, const Extent& y) {
  if (x.lo == x.hi || y.lo == y.hi) return false;
  return x.lo < y.hi && y.lo < x.hi;
}

// `valid` is any readable device float, used as the address of a scalar plane.
inline Plane plane(const ns_plane& p, const float* valid) {
  if (p.data) return Plane{p.data, p.stride_b, p.stride_n, p.scalar, ~0u};
  return Plane{valid, 0, 0, p.scalar, 0u};
}
inline OutPlane out_plane(const ns_out_plane& p) {
  return OutPlane{p.data, p.stride_b, p.stride_n};
}

}  // namespace ns
