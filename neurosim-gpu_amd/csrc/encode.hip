// Device encoders of the reduced-precision CSR weight payloads (gfx950),
// bit-exact with the reference's torch encoders (precision.py:45-90):
//
//  * fp8:   scale = max(amax/448, tiny); code = e4m3(clamp(w/scale, +-448)).
//  * NVFP4: global = max(amax/(6*448), tiny); per 16 consecutive weights
//           block = e4m3(min(block_amax/(6*global), 448)), unit = global *
//           block, code = nearest e2m1 level of |w|/unit (an exact midpoint
//           goes to the even code), sign in bit 3; two codes per byte, the
//           even weight in the low nibble.
//
// Every quotient is a correctly rounded float32 division and every product a
// float32 multiply, in the reference's order; e4m3 rounding is
// round-to-nearest-even written from the OCP 8-bit float specification
// (e4m3fn: bias 7, 3 mantissa bits, subnormals, largest finite 448).
//
// Two launches: per-workgroup maxima of |w| (as integer bit patterns, whose
// order on non-negative floats is the float order), then the encoder, in
// which every workgroup first reduces those maxima itself, so no launch waits
// on a single-workgroup reduction and no memory needs clearing beforehand.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>

#include "ns_common.h"
#include "ns_host.h"

namespace ns {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));
typedef uint32_t v2u32 __attribute__((ext_vector_type(2)));

constexpr int kEncodeThreads = 256;
constexpr int kEncodePartials = 1024;   // maxima written by the first launch, at most
constexpr float kTiny = 1.17549435e-38f;  // smallest normal float32

// Round |x| <= 448 (any sign, -0 included) to an e4m3fn code, nearest even;
// NaN becomes 0x7F with its sign, as torch's float8_e4m3fn conversion does.
__device__ __forceinline__ uint32_t e4m3_code(float x) {
  const uint32_t bits = __float_as_uint(x);
  const uint32_t sign = (bits >> 24) & 0x80u;
  const uint32_t mag = bits & 0x7FFFFFFFu;
  uint32_t code;
  if (mag > 0x7F800000u) {
    code = 0x7Fu;
  } else if (mag < 0x3C800000u) {
    // Below 2^-6: multiples of 2^-9 (the scaling by 512 is exact); a result
    // of 8 is the smallest normal, code 0x08.
    code = static_cast<uint32_t>(rintf(__uint_as_float(mag) * 512.0f));
  } else {
    // Normal: keep 3 of the 23 fraction bits, nearest even; a carry moves
    // into the exponent.
    const uint32_t rounded = (mag + 0x7FFFFu + ((mag >> 20) & 1u)) & ~0xFFFFFu;
    const uint32_t exponent = (rounded >> 23) - 127u + 7u;
    code = (exponent << 3) | ((rounded >> 20) & 7u);
  }
  return code | sign;
}

// torch.clamp(x, lo, hi): NaN stays NaN.
__device__ __forceinline__ float clamp_to(float x, float lo, float hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}

// tensor.clamp_min(tiny): NaN stays NaN.
__device__ __forceinline__ float at_least_tiny(float x) { return x < kTiny ? kTiny : x; }

__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = max(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), off, 64)));
  return v;
}

// Maximum over the workgroup of each thread's `v`; every thread gets it.
__device__ __forceinline__ uint32_t block_max(uint32_t v) {
  __shared__ uint32_t per_wave[kEncodeThreads / 64];
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) per_wave[threadIdx.x >> 6] = v;
  __syncthreads();
  uint32_t all = per_wave[0];
#pragma unroll
  for (int w = 1; w < kEncodeThreads / 64; ++w) all = max(all, per_wave[w]);
  __syncthreads();
  return all;
}

// First launch: partials[blockIdx.x] = bits of max |w| over a grid-stride share.
__global__ __launch_bounds__(kEncodeThreads) void amax_partials_kernel(const float* w, int64_t m,
                                                                       uint32_t* partials) {
  uint32_t best = 0u;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kEncodeThreads;
  const int64_t quads = m / 4;
  const v4u32* w4 = reinterpret_cast<const v4u32*>(w);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kEncodeThreads + threadIdx.x; i < quads; i += stride) {
    const v4u32 q = w4[i];
    best = max(best, max(max(q.x & 0x7FFFFFFFu, q.y & 0x7FFFFFFFu),
                         max(q.z & 0x7FFFFFFFu, q.w & 0x7FFFFFFFu)));
  }
  if (blockIdx.x == 0 && threadIdx.x < m - quads * 4)
    best = max(best, __float_as_uint(w[quads * 4 + threadIdx.x]) & 0x7FFFFFFFu);
  best = block_max(best);
  if (threadIdx.x == 0) partials[blockIdx.x] = best;
}

// max |w| over the whole vector, from the first launch's partials.
__device__ __forceinline__ float reduce_amax(const uint32_t* partials, int n_partials) {
  uint32_t best = 0u;
  for (int i = threadIdx.x; i < n_partials; i += kEncodeThreads) best = max(best, partials[i]);
  return __uint_as_float(block_max(best));
}

__global__ __launch_bounds__(kEncodeThreads) void encode_e4m3_kernel(
    const float* w, int64_t m, const uint32_t* partials, int n_partials, uint8_t* codes,
    float* scale_out) {
  const float amax = reduce_amax(partials, n_partials);
  const float scale = at_least_tiny(amax / 448.0f);
  if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = scale;
  auto code_of = [&](float x) { return e4m3_code(clamp_to(x / scale, -448.0f, 448.0f)); };
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kEncodeThreads;
  const int64_t quads = m / 4;
  const v4f* w4 = reinterpret_cast<const v4f*>(w);
  uint32_t* c4 = reinterpret_cast<uint32_t*>(codes);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kEncodeThreads + threadIdx.x; i < quads; i += stride) {
    const v4f q = w4[i];
    c4[i] = code_of(q.x) | (code_of(q.y) << 8) | (code_of(q.z) << 16) | (code_of(q.w) << 24);
  }
  if (blockIdx.x == 0 && threadIdx.x < m - quads * 4) {
    const int64_t e = quads * 4 + threadIdx.x;
    codes[e] = static_cast<uint8_t>(code_of(w[e]));
  }
}

// Index of the nearest e2m1 level of x >= 0: the number of midpoints
// (.25 .75 1.25 1.75 2.5 3.5 5) below x, plus one at an exact midpoint whose
// lower level is odd, so that ties go to the even code.
__device__ __forceinline__ uint32_t e2m1_index(float x) {
  constexpr float mid[7] = {0.25f, 0.75f, 1.25f, 1.75f, 2.5f, 3.5f, 5.0f};
  uint32_t below = 0u, tie_up = 0u;
#pragma unroll
  for (int i = 0; i < 7; ++i) {
    below += x > mid[i] ? 1u : 0u;
    if (i % 2 == 1) tie_up |= x == mid[i] ? 1u : 0u;
  }
  return below + tie_up;
}

// One thread per 16-weight block: block scale, 16 codes, 8 packed bytes.
__global__ __launch_bounds__(kEncodeThreads) void encode_nvfp4_kernel(
    const float* w, int64_t m, const uint32_t* partials, int n_partials, uint8_t* packed,
    uint8_t* block_scales, float* scale_out) {
  const float amax = reduce_amax(partials, n_partials);
  const float global = at_least_tiny(amax / 2688.0f);
  const float six_global = 6.0f * global;
  if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = global;
  const int64_t n_blocks = (m + 15) / 16;
  const int64_t full = m / 16;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kEncodeThreads;
  for (int64_t blk = static_cast<int64_t>(blockIdx.x) * kEncodeThreads + threadIdx.x; blk < n_blocks; blk += stride) {
    float v[16];
    if (blk < full) {
      const v4f* src = reinterpret_cast<const v4f*>(w + blk * 16);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const v4f x = src[q];
        v[4 * q] = x.x; v[4 * q + 1] = x.y; v[4 * q + 2] = x.z; v[4 * q + 3] = x.w;
      }
    } else {                 // the last, partial block: zero padding on the right
#pragma unroll
      for (int k = 0; k < 16; ++k) v[k] = blk * 16 + k < m ? w[blk * 16 + k] : 0.0f;
    }
    uint32_t bamax_bits = 0u;
#pragma unroll
    for (int k = 0; k < 16; ++k) bamax_bits = max(bamax_bits, __float_as_uint(v[k]) & 0x7FFFFFFFu);
    const float ratio = clamp_to(__uint_as_float(bamax_bits) / six_global, -448.0f, 448.0f);
    const uint32_t block_code = e4m3_code(ratio);
    const float unit = global * e4m3_to_float(block_code);
    const float safe = unit > 0.0f ? unit : 1.0f;
    uint32_t word[2] = {0u, 0u};
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const uint32_t sign = __float_as_uint(v[k]) >> 31;
      const uint32_t code = e2m1_index(fabsf(v[k]) / safe) | (sign << 3);
      word[k / 8] |= code << (4 * (k % 8));
    }
    block_scales[blk] = static_cast<uint8_t>(block_code);
    if (blk < full) {
      *reinterpret_cast<v2u32*>(packed + blk * 8) = v2u32{word[0], word[1]};
    } else {
      const int64_t bytes = ((m + 1) / 2) - blk * 8;   // packed bytes of the partial block
      for (int64_t b = 0; b < bytes; ++b) packed[blk * 8 + b] = static_cast<uint8_t>(word[b / 4] >> (8 * (b % 4)));
    }
  }
}

// The partials of ns_encode_weights_no_alloc: a library-owned device array,
// one per GPU (each device holds its own copy at its own address), alive until
// the process ends.  Host code never passes `scratch` itself to a kernel (on
// the host the name is a stand-in, not a device address): it looks up each
// device's address once and passes that.
static __device__ __align__(256) uint32_t scratch[kEncodePartials];

constexpr int kMaxDevices = 64;

// The device address of `scratch` on the current device, looked up on the
// first call on that device (with it current) and kept; null with the error
// set on failure.
uint32_t* scratch_on_current_device() {
  static std::mutex mu;
  static uint32_t* address[kMaxDevices] = {};
  int device = -1;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) {
    fail("no usable current HIP device (device %d)", device);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!address[device]) {
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr) {
      fail("could not find the encoder's scratch array on device %d: %s", device,
           hipGetErrorString(err));
      return nullptr;
    }
    address[device] = static_cast<uint32_t*>(ptr);
  }
  return address[device];
}

int partial_blocks(int64_t m) {
  const int64_t quads = (m + 3) / 4;
  return static_cast<int>(std::min<int64_t>(kEncodePartials,
                                            std::max<int64_t>(1, (quads + kEncodeThreads - 1) / kEncodeThreads)));
}

}  // namespace ns

using namespace ns;

extern "C" int64_t ns_encode_workspace_bytes(void) { return 4 * int64_t{kEncodePartials}; }

namespace {

// Every argument but the workspace.
int check_args(const ns_encode_args& a) {
  if (a.n_edges < 0 || a.n_edges >= (int64_t{1} << 40)) return fail("n_edges must be in [0, 2^40)");
  if (a.format != NS_WEIGHT_E4M3 && a.format != NS_WEIGHT_NVFP4)
    return fail("weight encoding needs format E4M3 or NVFP4, not %d", a.format);
  if (!a.global_scale) return fail("global_scale is required");
  if (a.n_edges > 0 && (!a.weight || !a.codes)) return fail("weight and codes are required");
  if (a.format == NS_WEIGHT_NVFP4 && a.n_edges > 0 && !a.block_scales)
    return fail("NVFP4 encoding requires block_scales");
  if (reinterpret_cast<uintptr_t>(a.weight) % 16)
    return fail("weight must be 16-byte aligned");
  if (a.format == NS_WEIGHT_E4M3 && reinterpret_cast<uintptr_t>(a.codes) % 4)
    return fail("E4M3 codes must be 4-byte aligned");
  if (a.format == NS_WEIGHT_NVFP4 && reinterpret_cast<uintptr_t>(a.codes) % 8)
    return fail("NVFP4 codes must be 8-byte aligned");
  return NS_OK;
}

// Launches the two kernels of checked arguments with the amax partials in
// `partials` (room for kEncodePartials entries).
int encode(const ns_encode_args& a, uint32_t* partials, void* stream) {
  const hipStream_t s = static_cast<hipStream_t>(stream);
  // Every partial the encoder reads is written by the first launch: nothing
  // in `partials` needs to be cleared beforehand.
  const int parts = partial_blocks(a.n_edges);
  amax_partials_kernel<<<dim3(parts), dim3(kEncodeThreads), 0, s>>>(a.weight, a.n_edges, partials);
  if (hipGetLastError() != hipSuccess) return fail("amax launch failed");
  if (a.format == NS_WEIGHT_E4M3) {
    const int64_t quads = a.n_edges / 4;
    const int grid = static_cast<int>(std::min<int64_t>(2048, std::max<int64_t>(1, (quads + kEncodeThreads - 1) / kEncodeThreads)));
    encode_e4m3_kernel<<<dim3(grid), dim3(kEncodeThreads), 0, s>>>(
        a.weight, a.n_edges, partials, parts, a.codes, a.global_scale);
  } else {
    const int64_t blocks = (a.n_edges + 15) / 16;
    const int grid = static_cast<int>(std::min<int64_t>(2048, std::max<int64_t>(1, (blocks + kEncodeThreads - 1) / kEncodeThreads)));
    encode_nvfp4_kernel<<<dim3(grid), dim3(kEncodeThreads), 0, s>>>(
        a.weight, a.n_edges, partials, parts, a.codes, a.block_scales, a.global_scale);
  }
  if (hipGetLastError() != hipSuccess) return fail("encode launch failed");
  return NS_OK;
}

}  // namespace

extern "C" int ns_encode_weights(const ns_encode_args* args, void* stream) {
  clear_error();
  if (!args) return fail("arguments are required");
  const ns_encode_args& a = *args;
  if (!a.global_scale || !a.workspace) return fail("global_scale and workspace are required");
  if (int rc = check_args(a)) return rc;
  if (reinterpret_cast<uintptr_t>(a.workspace) % 4) return fail("workspace must be 4-byte aligned");
  return encode(a, a.workspace, stream);
}

extern "C" int ns_encode_weights_no_alloc(const ns_encode_args* args, void* stream) {
  clear_error();
  if (!args) return fail("arguments are required");
  const ns_encode_args& a = *args;
  if (int rc = check_args(a)) return rc;
  if (a.workspace) return fail("the no-allocation encoder takes no workspace (pass NULL)");
  // The partials of any M in range fit the scratch array: at most
  // kEncodePartials workgroups write them (partial_blocks).
  if (partial_blocks(a.n_edges) > kEncodePartials)
    return fail("%lld edges need more than the %d partials of the scratch array",
                (long long)a.n_edges, kEncodePartials);
  if (stream) {
    int current = -1, owner = -1;
    if (hipGetDevice(&current) != hipSuccess ||
        hipStreamGetDevice(static_cast<hipStream_t>(stream), &owner) != hipSuccess)
      return fail("could not query the current device or the stream's device");
    if (current != owner)
      return fail("the stream belongs to device %d but device %d is current", owner, current);
  }
  uint32_t* partials = scratch_on_current_device();
  if (!partials) return NS_ERR_INVALID;
  return encode(a, partials, stream);
}
