// Weights of a CSR payload rearranged into a slot layout's order (gfx950).
//
// The panel and band kernels stream their weights in slot order (a layout
// built once per graph: slot k holds CSR edge perm[k], or padding).  When the
// weights change, the slot-order copy is rebuilt by this gather: one thread
// per slot pair reads the pair's two edge numbers (one 8-byte load), gathers
// their weights (the edges of one tile lie in a short stretch of the CSR, so
// the gathers stay within an L2-sized window, and those of one row's lanes
// in a few cache lines) and writes the pair's words.
//
// Per format, slot pair (2i, 2i+1) with edges e0, e1 (negative: padding,
// code 0):
//   F32 / F16 / E4M3: the two weights (4 / 2 / 1 bytes each);
//   NVFP4:            one byte, the two edges' nibbles (slot 2i low), plus one
//                     block-scale byte per slot;
//   NVFP4 pairs:      one uint16: the two nibbles in the low byte and, in the
//                     high byte, the block-scale code of the pair's first real
//                     edge (both edges of a pair lie in one weight block).
#include <hip/hip_runtime.h>

#include "ns_common.h"
#include "ns_host.h"

namespace ns {

namespace {

// Slot pairs of one workgroup: gather_rounds<FMT>() consecutive runs of
// kGatherThreads pairs.  A row's lanes hold consecutive CSR edges at every
// step of its group, so consecutive steps re-read the same cache lines of the
// weights: a workgroup that covers many consecutive steps finds them in its
// compute unit's L1 instead of asking L2 again.  At the 25M-edge headline
// layout, µs per gather for 256 / 1024 threads (one run): fp32 82 / 68, fp8
// 64 / 50, NVFP4 pairs 72 / 61; for 1024 threads and 1 / 4 / 8 runs: fp32
// 68 / 75 / 90, fp8 50 / 44 / 49, NVFP4 pairs 61 / 56 / 58.
constexpr int kGatherThreads = 1024;

template <int FMT>
constexpr int gather_rounds() {
  return FMT == NS_WEIGHT_F32 ? 1 : 4;
}

typedef int32_t v2i32 __attribute__((ext_vector_type(2)));

struct GatherArgs {
  const v2i32* perm;     // [pairs]
  int64_t pairs, n_edges;
  const void* weight;
  const uint8_t* block_scales;
  void* slots;
  uint8_t* slot_scales;
};

// Nibble of edge e of a packed NVFP4 payload.
__device__ __forceinline__ uint32_t nibble_of(const uint8_t* codes, int32_t e) {
  return (codes[e >> 1] >> ((e & 1) * 4)) & 15u;
}

template <int FMT, bool PAIRS>
__device__ __forceinline__ void gather_pair(const GatherArgs& a, int64_t i) {
  v2i32 e = a.perm[i];
  // An edge number outside the payload reads as padding.
  const bool r0 = e.x >= 0 && e.x < a.n_edges, r1 = e.y >= 0 && e.y < a.n_edges;
  if constexpr (FMT == NS_WEIGHT_F32) {
    const float* w = static_cast<const float*>(a.weight);
    typedef float v2f __attribute__((ext_vector_type(2)));
    v2f out;
    out.x = r0 ? w[e.x] : 0.0f;
    out.y = r1 ? w[e.y] : 0.0f;
    static_cast<v2f*>(a.slots)[i] = out;
  } else if constexpr (FMT == NS_WEIGHT_F16) {
    const uint16_t* w = static_cast<const uint16_t*>(a.weight);
    const uint32_t lo = r0 ? w[e.x] : 0u, hi = r1 ? w[e.y] : 0u;
    static_cast<uint32_t*>(a.slots)[i] = lo | (hi << 16);
  } else if constexpr (FMT == NS_WEIGHT_E4M3) {
    const uint8_t* w = static_cast<const uint8_t*>(a.weight);
    const uint32_t lo = r0 ? w[e.x] : 0u, hi = r1 ? w[e.y] : 0u;
    static_cast<uint16_t*>(a.slots)[i] = static_cast<uint16_t>(lo | (hi << 8));
  } else {
    const uint8_t* codes = static_cast<const uint8_t*>(a.weight);
    const uint32_t nibbles = (r0 ? nibble_of(codes, e.x) : 0u) | ((r1 ? nibble_of(codes, e.y) : 0u) << 4);
    if constexpr (PAIRS) {
      const uint32_t scale = r0 ? a.block_scales[e.x >> 4] : r1 ? a.block_scales[e.y >> 4] : 0u;
      static_cast<uint16_t*>(a.slots)[i] = static_cast<uint16_t>(nibbles | (scale << 8));
    } else {
      static_cast<uint8_t*>(a.slots)[i] = static_cast<uint8_t>(nibbles);
      const uint32_t s0 = r0 ? a.block_scales[e.x >> 4] : 0u;
      const uint32_t s1 = r1 ? a.block_scales[e.y >> 4] : 0u;
      reinterpret_cast<uint16_t*>(a.slot_scales)[i] = static_cast<uint16_t>(s0 | (s1 << 8));
    }
  }
}

template <int FMT, bool PAIRS>
__global__ __launch_bounds__(kGatherThreads) void gather_slots_kernel(GatherArgs a) {
  constexpr int kRounds = gather_rounds<FMT>();
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kRounds * kGatherThreads;
#pragma unroll
  for (int k = 0; k < kRounds; ++k) {
    const int64_t i = first + k * kGatherThreads + threadIdx.x;
    if (i < a.pairs) gather_pair<FMT, PAIRS>(a, i);
  }
}

template <int FMT, bool PAIRS>
hipError_t launch(const GatherArgs& a, hipStream_t stream) {
  constexpr int64_t per_block = int64_t{kGatherThreads} * gather_rounds<FMT>();
  const int64_t blocks = (a.pairs + per_block - 1) / per_block;
  gather_slots_kernel<FMT, PAIRS><<<dim3(static_cast<unsigned>(blocks)), dim3(kGatherThreads), 0,
                                    stream>>>(a);
  return hipGetLastError();
}

}  // namespace

}  // namespace ns

using namespace ns;

extern "C" int ns_gather_slot_weights(const int32_t* perm, int64_t n_slots, int64_t n_edges,
                                      int32_t format, int32_t pairs, const void* weight,
                                      const uint8_t* block_scales, void* slots,
                                      uint8_t* slot_scales, void* stream) {
  clear_error();
  if (n_slots < 0 || n_slots % 2 || n_slots >= (int64_t{1} << 32))
    return fail("n_slots must be even and in [0, 2^32)");
  if (n_edges < 0 || n_edges >= (int64_t{1} << 31)) return fail("n_edges must be in [0, 2^31)");
  if (format < NS_WEIGHT_F32 || format > NS_WEIGHT_NVFP4)
    return fail("unknown weight format %d", format);
  if (pairs && format != NS_WEIGHT_NVFP4) return fail("the pair layout applies to NVFP4 only");
  if (n_slots == 0) return NS_OK;
  if (!perm || !slots) return fail("perm and slots are required");
  if (n_edges > 0 && !weight) return fail("weight is required");
  const bool nvfp4 = format == NS_WEIGHT_NVFP4;
  if (nvfp4 && n_edges > 0 && !block_scales) return fail("NVFP4 weights require block scales");
  if (nvfp4 && !pairs && !slot_scales) return fail("NVFP4 slots without pairs need slot_scales");
  if (reinterpret_cast<uintptr_t>(perm) % 8) return fail("perm must be 8-byte aligned");
  const uintptr_t need = format == NS_WEIGHT_F32 ? 8 : format == NS_WEIGHT_F16 ? 4
                         : (format == NS_WEIGHT_E4M3 || pairs) ? 2 : 1;
  if (reinterpret_cast<uintptr_t>(slots) % need) return fail("slots are misaligned");
  if (nvfp4 && !pairs && reinterpret_cast<uintptr_t>(slot_scales) % 2)
    return fail("slot_scales must be 2-byte aligned");
  GatherArgs a{};
  a.perm = reinterpret_cast<const v2i32*>(perm);
  a.pairs = n_slots / 2;
  a.n_edges = n_edges;
  a.weight = weight;
  a.block_scales = block_scales;
  a.slots = slots;
  a.slot_scales = slot_scales;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t err;
  switch (format) {
    case NS_WEIGHT_F32: err = launch<NS_WEIGHT_F32, false>(a, s); break;
    case NS_WEIGHT_F16: err = launch<NS_WEIGHT_F16, false>(a, s); break;
    case NS_WEIGHT_E4M3: err = launch<NS_WEIGHT_E4M3, false>(a, s); break;
    default:
      err = pairs ? launch<NS_WEIGHT_NVFP4, true>(a, s) : launch<NS_WEIGHT_NVFP4, false>(a, s);
  }
  if (err != hipSuccess) return fail_launch("slot gather", err);
  return NS_OK;
}
