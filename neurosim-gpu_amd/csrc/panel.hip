// Column-panel matrix tick for batch widths 1 and 2 (gfx950).
//
// The row-block tick gathers s[col] from L2 for every edge; each 4-byte
// gather moves a whole cache line into the CU, so at 25M edges the gather
// traffic, not HBM, bounds the tick.  Here the columns are cut into panels
// whose slice of s fits in LDS, and the CSR is re-laid out once per graph
// (ns_plan_panels) as sliced rows:
//
//  * a workgroup (16 wavefronts) owns one tile: one panel and a range of
//    destination rows.  It stages the panel's slice of s in LDS, plus one zero
//    that padding slots point at;
//  * the tile's rows are grouped by segment length; a group gives each row
//    2^lg lanes, and lane j of a row accumulates items j, j+2^lg, ... of the
//    row's segment in one float32 FMA chain, so the inner loop has no row
//    boundaries.  The items are the segment's edges in CSR order or, in the
//    pair layout (NS_PANEL_PAIRS), grouped by 16-edge weight block with each
//    block's run padded to even length, so that two neighbouring lanes of a
//    row hold edges of one NVFP4 block and share one scale byte;
//  * each wavefront owns a run of consecutive groups (balanced by the planner)
//    whose slots are one contiguous stream of 64-lane steps (16-bit
//    panel-local source index plus the weight in its encoding).  The stream
//    is read in register blocks of D steps, the next block in flight while
//    the current one is consumed;
//  * a bitmap over steps marks each group's last step: inside a block the
//    sums are only snapshotted there, and after the block the groups that
//    ended are closed in order (xor butterfly over the row's lanes, one lane
//    per row stores the sum at the group's row-table entries);
//  * after its stream each wavefront maps its row-table entries back to rows:
//    with one panel it updates those rows, with several it stores the
//    panel's partial sums by row;
//  * rows are cut into ranges shared by all panels, so the tiles of one range
//    (one per panel) together hold every panel's sums of the range's rows.
//    Each tile counts itself in on its range's counter once its sums are
//    stored, and the tile that completes the count adds the range's sums in
//    panel order and applies the update: one launch per tick.  The sums are
//    written through to, and read back from, the device-coherent level
//    (agent-scope atomic stores and loads), ordered by the count (a release
//    by every tile, an acquire by the last).  A second kernel that does the
//    same adds after the tick kernel (NS_PANEL_COMBINE_LAUNCH, the default)
//    gives bitwise the same results.
//
// Results are bitwise repeatable and, on one layout, identical across weight
// encodings that decode to the same float32 values.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "ns_common.h"
#include "ns_host.h"

namespace ns {

// Neurons of one panel that fit in LDS next to the sentinel zero, in whole
// 4-neuron groups.
template <int BT>
constexpr int panel_capacity_neurons() {
  return ((163840 - 64) / (4 * BT) - 1) & ~3;
}

// NVFP4 weights of a pair layout (NS_PANEL_PAIRS): one uint16 word per slot
// pair, the two nibbles in the low byte and the pair's block-scale code in the
// high byte.  A kernel template format of its own, next to the NS_WEIGHT_* ones.
constexpr int kNvfp4Pairs = 4;
// Float32 weights read in place (NS_PANEL_INDEXED): the slot stream carries each
// slot's CSR edge number (int32, -1 for padding) and the tick gathers the
// weight from the CSR-order array.  A weight version ticked once then needs no
// slot-order copy; a row's lanes read consecutive edges, which stay in L1.
constexpr int kIndexedF32 = 5;

// Wave priority follows each wave's remaining stream.
constexpr bool kPacedWaves = true;

// Steps per register block: enough 64-lane loads in flight per wavefront to
// cover HBM latency with 16 wavefronts per compute unit, within 128 VGPRs.
// Measured at N=166k, M=25M, B=1 (µs per tick, graph replays): fp32 8/9/10/11/12
// steps 33.7/33.3/32.4/33.9/35.1; fp16 8/10/12/14 25.1/25.0/26.4/27.4; e4m3
// 8/10/12/16 22.0/22.1/22.7/23.7; NVFP4 pairs 10/12/13/16 23.0/22.6/23.2/23.7.
template <int BT, int FMT>
constexpr int block_steps() {
  if constexpr (FMT == NS_WEIGHT_F32) return BT == 1 ? 10 : 8;
  else if constexpr (FMT == NS_WEIGHT_F16) return BT == 1 ? 10 : 8;
  else if constexpr (FMT == NS_WEIGHT_E4M3) return BT == 1 ? 10 : 12;
  else if constexpr (FMT == kNvfp4Pairs) return 12;
  else if constexpr (FMT == kIndexedF32) return BT == 1 ? 10 : 8;
  else return BT == 1 ? 12 : 8;
}

struct PanelArgs {
  int64_t N, B;
  Plane s, d, a, u, v;
  Params p;
  int32_t width, n_panels;
  const int32_t* tiles;
  const int32_t* tile_ranges;
  uint32_t* counters;  // [n_ranges]; null: a second kernel combines the panels
  const int32_t* wave_groups;
  const int32_t* groups;
  const uint16_t* rows;
  const uint32_t* last_steps;
  const uint16_t* col;
  const void* weight;
  const uint8_t* slot_scales;
  const float* gscale;
  const float* csr_weight;  // kIndexedF32: the float32 weights in CSR order
  float* sorted;     // [rows-table entries][BT]: row sums in row-table order
  float* partials;   // [n_panels][N][BT]: row sums by row (several panels)
  OutPlane os, od, oa;
  OutPlane oj;       // optional: j as well (data null: not written)
  int32_t s_vec;   // s.sn == 1 (B == 1) or neuron-major B == 2, 16-byte aligned
  int32_t product;  // 0: the tick; 1: W @ s stored into os; 2: W @ s added to os
};

// The product modes' store of one row's sum.
__device__ __forceinline__ void store_product(const PanelArgs& A, int64_t n, int64_t b, float j) {
  float* const at = A.os.data + b * A.os.sb + n * A.os.sn;
  *at = A.product == 2 ? *at + j : j;
}

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef const int32_t __attribute__((address_space(4)))* const_i32_ptr;
typedef const uint32_t __attribute__((address_space(4)))* const_u32_ptr;
typedef const __attribute__((address_space(1))) void* global_void_ptr;
typedef __attribute__((address_space(3))) void* lds_void_ptr;

// One lane's raw slot: source index, weight bits (F32/F16/E4M3 code, or the
// NVFP4 byte holding its nibble) and, for NVFP4, the block-scale code.
struct Slot {
  uint32_t c, w, sc;
};

// Slots of one register block: this lane's slot of step k is q0 + 64k.
template <int FMT>
__device__ __forceinline__ Slot load_slot(const PanelArgs& A, int64_t q0, int k) {
  Slot x;
  x.c = A.col[q0 + 64 * k];
  if constexpr (FMT == NS_WEIGHT_F32) {
    x.w = static_cast<const uint32_t*>(A.weight)[q0 + 64 * k];
  } else if constexpr (FMT == NS_WEIGHT_F16) {
    x.w = static_cast<const uint16_t*>(A.weight)[q0 + 64 * k];
  } else if constexpr (FMT == NS_WEIGHT_E4M3) {
    x.w = static_cast<const uint8_t*>(A.weight)[q0 + 64 * k];
  } else if constexpr (FMT == kNvfp4Pairs) {
    x.w = static_cast<const uint16_t*>(A.weight)[(q0 >> 1) + 32 * k];
  } else {
    x.w = static_cast<const uint8_t*>(A.weight)[(q0 >> 1) + 32 * k];
  }
  x.sc = FMT == NS_WEIGHT_NVFP4 ? A.slot_scales[q0 + 64 * k] : 0u;
  return x;
}

// `p` kept a scalar operand of the loads made through it (scalar base plus
// 32-bit lane offset) instead of being folded into per-lane 64-bit addresses.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* scalar_base(const T* p) {
  typedef const __attribute__((address_space(1))) T* global_ptr;
  global_ptr q = (global_ptr)p;
  asm volatile("" : "+s"(q));
  return q;
}

// One register block of D steps starting at slot block0 (a multiple of 64).
// For float32 weights the loads take a scalar base per block and a 32-bit
// lane offset: with per-lane 64-bit addresses the compiler reuses a register
// of the block in flight for the next block's address and so waits for that
// block before issuing the next one.  lane32 is the lane made opaque once per
// kernel, so it stays in one register for the whole stream (neither a 64-bit
// copy nor a register a load may target).  NVFP4 pair words take the same
// path.  The other narrow encodings keep per-lane addresses: they compile
// without the wait, or (e4m3) measure no faster without it.
template <int FMT, int D>
__device__ __forceinline__ void load_block(const PanelArgs& A, int64_t block0, int lane,
                                           uint32_t lane32, Slot (&dst)[D]) {
  if constexpr (FMT == NS_WEIGHT_F32 || FMT == kIndexedF32) {
    const auto col = scalar_base(A.col + block0);
    const auto weight = scalar_base(static_cast<const uint32_t*>(A.weight) + block0);
#pragma unroll
    for (int k = 0; k < D; ++k) {
      const uint32_t at = lane32 + 64u * k;
      dst[k].c = col[at];
      dst[k].w = weight[at];
      dst[k].sc = 0u;
    }
  } else if constexpr (FMT == kNvfp4Pairs) {
    const auto col = scalar_base(A.col + block0);
    const auto words = scalar_base(static_cast<const uint16_t*>(A.weight) + block0 / 2);
#pragma unroll
    for (int k = 0; k < D; ++k) {
      dst[k].c = col[lane32 + 64u * k];
      dst[k].w = words[(lane32 >> 1) + 32u * k];
      dst[k].sc = 0u;
    }
  } else {
#pragma unroll
    for (int k = 0; k < D; ++k) dst[k] = load_slot<FMT>(A, block0 + lane, k);
  }
}

// Slots of a group start at multiples of 64, so a slot's nibble half is the lane's parity.
template <int FMT>
__device__ __forceinline__ float decode_slot(const Slot& x, int lane, float gscale) {
  if constexpr (FMT == NS_WEIGHT_F32 || FMT == kIndexedF32) {
    // kIndexedF32: `w` was replaced by the gathered weight (gather_block).
    return __builtin_bit_cast(float, x.w);
  } else if constexpr (FMT == NS_WEIGHT_F16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(x.w)));
  } else if constexpr (FMT == NS_WEIGHT_E4M3) {
    return e4m3_to_float(x.w) * gscale;
  } else if constexpr (FMT == kNvfp4Pairs) {
    const ns_v2f pair = e2m1_pair(x.w & 0xFFu);
    return ((lane & 1) ? pair.y : pair.x) * (e4m3_to_float(x.w >> 8) * gscale);
  } else {
    const ns_v2f pair = e2m1_pair(x.w & 0xFFu);
    return ((lane & 1) ? pair.y : pair.x) * (e4m3_to_float(x.sc) * gscale);
  }
}

// kIndexedF32: replaces each slot's edge number by its float32 weight, all D
// gathers issued before the first is used.  Padding (-1) reads edge 0 and
// contributes +0.0 (its source is the slice's zero, and the weight is zeroed).
template <int FMT, int D>
__device__ __forceinline__ void gather_block(const PanelArgs& A, Slot (&x)[D]) {
  if constexpr (FMT == kIndexedF32) {
    const auto w = scalar_base(A.csr_weight);
    uint32_t got[D];
#pragma unroll
    for (int k = 0; k < D; ++k) {
      const int32_t e = static_cast<int32_t>(x[k].w);
      got[k] = __builtin_bit_cast(uint32_t, w[e < 0 ? 0u : static_cast<uint32_t>(e)]);
    }
#pragma unroll
    for (int k = 0; k < D; ++k) x[k].w = static_cast<int32_t>(x[k].w) < 0 ? 0u : got[k];
  }
}

// The kernel's arguments read again from the kernel argument segment.  The
// opaque pointer makes the compiler load the fields a caller uses where it
// uses them, instead of keeping them in scalar registers since kernel entry.
__device__ __forceinline__ PanelArgs fresh_args() {
  static_assert(sizeof(PanelArgs) % 4 == 0, "kernel arguments are copied in 32-bit words");
  typedef const __attribute__((address_space(4))) uint32_t* kernarg_ptr;
  kernarg_ptr p = (kernarg_ptr)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(p));
  PanelArgs out;
  uint32_t* words = reinterpret_cast<uint32_t*>(&out);
#pragma unroll
  for (unsigned i = 0; i < sizeof(PanelArgs) / 4; ++i) words[i] = p[i];
  return out;
}

__device__ __forceinline__ void update(const PanelArgs& A, int64_t n, int64_t b, float j) {
  const NextState x = advance_one(A.p, n, j, A.s.get(b, n), A.d.get(b, n), A.a.get(b, n),
                                  A.u.get(b, n), A.v.get(b, n));
  A.os.put(b, n, x.soma);
  A.od.put(b, n, x.dendrite);
  A.oa.put(b, n, x.adaptation);
  if (A.oj.data) A.oj.put(b, n, j);
}

// A group descriptor held in scalar registers.
struct Group {
  int lg, nrows, rowtab;
};

__device__ __forceinline__ Group load_group(const PanelArgs& A, int g) {
  const_i32_ptr desc = (const_i32_ptr)(A.groups + 4 * static_cast<int64_t>(g));
  return Group{desc[2] & 255, desc[2] >> 8, desc[3]};
}

// Boundary bits of steps [k0, k0 + D) of the whole slot array.
template <int D>
__device__ __forceinline__ uint32_t boundary_bits(const PanelArgs& A, int64_t k0) {
  const_u32_ptr w = (const_u32_ptr)(A.last_steps + (k0 >> 5));
  const uint64_t both = w[0] | (static_cast<uint64_t>(w[1]) << 32);
  return static_cast<uint32_t>(both >> (k0 & 31)) & ((1u << D) - 1u);
}

// Panel sums loaded per round before they are added.
constexpr int kCombineBatch = 8;

// Rows per thread per round of the finish below: a range of up to
// kPanelThreads * finish_rows rows with at most kCombineBatch panels finishes
// in one round.
template <int BT>
constexpr int rows_per_finisher() {
  return BT == 1 ? 4 : 2;
}

// One launch per tick with several panels: called by every tile after its
// wavefronts have stored the panel's sums of rows [r0, r1) (agent-scope atomic
// stores).  The tile counts itself in on its range's counter; the tile that
// completes the count (all n_panels tiles of the range have stored their
// sums) sets the counter back to zero for the next launch, then adds each
// row's sums in panel order and applies the update.  Each round issues every
// load of its rows (parameters, states, drives, the first kCombineBatch
// panels' sums) before the first add, so it waits on memory once.
// Operand views for the finish: global-address-space pointers (the arguments
// read afresh come back as generic ones) and 32-bit offset arithmetic.
typedef const __attribute__((address_space(1))) float* gcfloat;
typedef __attribute__((address_space(1))) float* gfloat;

// Element `i` of `p` as a 32-bit byte offset from the (uniform) base, which
// the loads and stores take as scalar base plus vector offset.
template <typename T>
__device__ __forceinline__ T* element(T* p, uint32_t i) {
  typedef const __attribute__((address_space(1))) char* raw;
  return (T*)((raw)p + i * 4u);
}

template <typename I>
struct FinishPlane {
  gcfloat data;
  I sb, sn;
  float scalar;
  uint32_t mask;
  __device__ __forceinline__ float get(I b, I n) const {
    const uint32_t x = __builtin_bit_cast(uint32_t, *element(data, b * sb + n * sn));
    return __builtin_bit_cast(float, (x & mask) | (__builtin_bit_cast(uint32_t, scalar) & ~mask));
  }
};

template <typename I>
struct FinishOut {
  gfloat data;
  I sb, sn;
  __device__ __forceinline__ void put(I b, I n, float x) const { *element(data, b * sb + n * sn) = x; }
};

template <typename I>
struct FinishVec {
  gcfloat data;
  I stride;
  __device__ __forceinline__ float get(I n) const { return *element(data, n * stride); }
};

template <typename I>
__device__ __forceinline__ FinishPlane<I> finish_view(const Plane& p) {
  return FinishPlane<I>{(gcfloat)p.data, static_cast<I>(p.sb), static_cast<I>(p.sn), p.scalar, p.mask};
}
template <typename I>
__device__ __forceinline__ FinishOut<I> finish_view(const OutPlane& p) {
  return FinishOut<I>{(gfloat)p.data, static_cast<I>(p.sb), static_cast<I>(p.sn)};
}

// Adds the range's sums in panel order and updates rows [r0, r1), with 32-bit
// offsets (the host launches this path only when every offset fits).
template <int BT>
__device__ __forceinline__ void finish_rows(const PanelArgs& A, uint32_t r0, uint32_t r1) {
  typedef uint32_t I;
  constexpr int R = rows_per_finisher<BT>();
  const FinishPlane<I> s = finish_view<I>(A.s), d = finish_view<I>(A.d), a = finish_view<I>(A.a);
  const FinishPlane<I> u = finish_view<I>(A.u), v = finish_view<I>(A.v);
  const FinishOut<I> os = finish_view<I>(A.os), od = finish_view<I>(A.od), oa = finish_view<I>(A.oa);
  const FinishOut<I> oj = finish_view<I>(A.oj);
  FinishVec<I> prm_v[6];
#pragma unroll
  for (int i = 0; i < 6; ++i) prm_v[i] = FinishVec<I>{(gcfloat)A.p.v[i].data, static_cast<I>(A.p.v[i].stride)};
  const int64_t plane = A.N * BT;
  auto partial = [&](int p, I n, int j) {
    const gcfloat base = (gcfloat)A.partials + p * plane;   // uniform
    return __hip_atomic_load(element(base, n * BT + j), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  };
  for (I n0 = r0 + threadIdx.x; n0 < r1; n0 += kPanelThreads * R) {
    NeuronParams prm[R];
    float sv[R][BT], dv[R][BT], av[R][BT], uv[R][BT], vv[R][BT];
    float part[R][kCombineBatch][BT];
#pragma unroll
    for (int k = 0; k < R; ++k) {
      // Rows past the range and panels past the last reread the last ones
      // (not used), so that no load waits behind a branch.
      const I n = min(n0 + static_cast<I>(k * kPanelThreads), r1 - 1);
      prm[k] = NeuronParams{prm_v[0].get(n), prm_v[1].get(n), prm_v[2].get(n),
                            prm_v[3].get(n), prm_v[4].get(n), prm_v[5].get(n)};
#pragma unroll
      for (int j = 0; j < BT; ++j) {
        sv[k][j] = s.get(j, n); dv[k][j] = d.get(j, n); av[k][j] = a.get(j, n);
        uv[k][j] = u.get(j, n); vv[k][j] = v.get(j, n);
      }
#pragma unroll
      for (int q = 0; q < kCombineBatch; ++q)
#pragma unroll
        for (int j = 0; j < BT; ++j) part[k][q][j] = partial(min(q, A.n_panels - 1), n, j);
    }
    float sum[R][BT];
#pragma unroll
    for (int k = 0; k < R; ++k)
#pragma unroll
      for (int j = 0; j < BT; ++j) {
        sum[k][j] = 0.0f;
#pragma unroll
        for (int q = 0; q < kCombineBatch; ++q)
          if (q < A.n_panels) sum[k][j] += part[k][q][j];
      }
    for (int p0 = kCombineBatch; p0 < A.n_panels; p0 += kCombineBatch) {
#pragma unroll
      for (int k = 0; k < R; ++k) {
        const I n = min(n0 + static_cast<I>(k * kPanelThreads), r1 - 1);
#pragma unroll
        for (int q = 0; q < kCombineBatch; ++q)
#pragma unroll
          for (int j = 0; j < BT; ++j) part[k][q][j] = partial(min(p0 + q, A.n_panels - 1), n, j);
      }
#pragma unroll
      for (int k = 0; k < R; ++k)
#pragma unroll
        for (int q = 0; q < kCombineBatch; ++q)
#pragma unroll
          for (int j = 0; j < BT; ++j)
            if (p0 + q < A.n_panels) sum[k][j] += part[k][q][j];
    }
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const I n = n0 + static_cast<I>(k * kPanelThreads);
      if (n < r1) {
#pragma unroll
        for (int j = 0; j < BT; ++j) {
          const NextState x = advance_loaded(prm[k], sum[k][j], sv[k][j], dv[k][j], av[k][j],
                                             uv[k][j], vv[k][j]);
          os.put(j, n, x.soma);
          od.put(j, n, x.dendrite);
          oa.put(j, n, x.adaptation);
          if (A.oj.data) oj.put(j, n, sum[k][j]);
        }
      }
    }
  }
}

// One launch per tick with several panels: called by every tile after its
// wavefronts have stored the panel's sums of rows [r0, r1) (agent-scope atomic
// stores).  The tile counts itself in on its range's counter; the tile that
// completes the count (all n_panels tiles of the range have stored their
// sums) sets the counter back to zero for the next launch, then adds each
// row's sums in panel order and applies the update.  Each round issues every
// load of its rows (parameters, states, drives, the first kCombineBatch
// panels' sums) before the first add, so it waits on memory once.
//
// Ordering: the workgroup barrier makes every lane's sums part of the counting
// thread's history; the count is a release at agent scope (every tile) and the
// last tile's is also an acquire, so the sums of all the range's tiles happen
// before its reads.  The counter goes back to zero in the launch that completes
// it; after a failed launch the caller must zero the counters again.
template <int BT>
__device__ __forceinline__ void finish_range(const PanelArgs& A, int64_t r0, int64_t r1) {
  __shared__ int last;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t* const counter = A.counters + A.tile_ranges[blockIdx.x];
    const uint32_t before = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL,
                                                   __HIP_MEMORY_SCOPE_AGENT);
    const bool done = before == static_cast<uint32_t>(A.n_panels - 1);
    if (done) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = done;
  }
  __syncthreads();
  if (!last) return;
  finish_rows<BT>(A, static_cast<uint32_t>(r0), static_cast<uint32_t>(r1));
}

template <int BT, int FMT>
__global__ __launch_bounds__(kPanelThreads) void panel_tick_kernel(PanelArgs A) {
  constexpr int D = block_steps<BT, FMT>();
  static_assert(D <= kPanelMaxPrefetch, "tail padding too short");
  constexpr int CAP = panel_capacity_neurons<BT>();
  __shared__ __attribute__((aligned(16))) float lds_s[(CAP + 1) * BT];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  uint32_t lane32 = static_cast<uint32_t>(lane);
  asm volatile("" : "+v"(lane32));
  __builtin_assume(lane32 < 64u);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const_i32_ptr tile = (const_i32_ptr)(A.tiles + 4 * static_cast<int64_t>(blockIdx.x));
  const int panel = tile[0];
  const int64_t base = static_cast<int64_t>(panel) * A.width;
  const int len = static_cast<int>(min<int64_t>(A.width, A.N - base));
  const float gscale =
      (FMT == NS_WEIGHT_E4M3 || FMT == NS_WEIGHT_NVFP4 || FMT == kNvfp4Pairs) ? *A.gscale : 1.0f;

  // A contiguous slice of s is staged with direct global -> LDS loads, issued
  // first since they need only the panel: wavefront chunk ch covers float4s
  // [64ch, 64ch + 64) (each lane's 16 bytes land at its own offset).  (Staging
  // through registers, in the same order or with each workgroup of an XCD
  // starting at its own place in the slice, measured no faster.)
  const v4f* src = reinterpret_cast<const v4f*>(A.s.data + base * BT);
  const int n4 = len * BT / 4;
  if (A.s_vec) {
    for (int ch = wave; ch * 64 < n4; ch += kPanelWaves) {
      const int i = ch * 64 + lane;
      if (i < n4)
        __builtin_amdgcn_global_load_lds((const global_void_ptr)(src + i),
                                         (lds_void_ptr)(lds_s + ch * 256), 16, 0, 0);
    }
  }

  // This wavefront's stream: groups [g, g_end), steps [first/64, first/64 + total).
  const_i32_ptr wg = (const_i32_ptr)(A.wave_groups + static_cast<int64_t>(blockIdx.x) * kPanelWaves + wave);
  int g = wg[0];
  const int g_end = wg[1];
  int64_t first = 0;
  int total = 0;
  if (g < g_end) {
    const_i32_ptr head = (const_i32_ptr)(A.groups + 4 * static_cast<int64_t>(g));
    const_i32_ptr last = (const_i32_ptr)(A.groups + 4 * static_cast<int64_t>(g_end - 1));
    first = head[0];
    total = (last[0] - head[0]) / 64 + last[1];
  }

  // First register block in flight while the panel is staged.
  Slot buf_a[D], buf_b[D];
  load_block<FMT, D>(A, first, lane, lane32, buf_a);
  uint32_t bits = boundary_bits<D>(A, first / 64);
  Group now{0, 0, 0}, next{0, 0, 0};
  if (g < g_end) now = load_group(A, g);
  if (g + 1 < g_end) next = load_group(A, g + 1);

  // Finish staging: the slice's last floats (not a whole float4) or, for a
  // strided state, the whole slice; then the zero that padding slots read.
  if (A.s_vec) {
    __builtin_amdgcn_s_waitcnt(0);
    for (int i = n4 * 4 + tid; i < len * BT; i += kPanelThreads) lds_s[i] = A.s.data[base * BT + i];
  } else {
    for (int i = tid; i < len * BT; i += kPanelThreads) {
      const int nn = i / BT, j = i - nn * BT;
      lds_s[i] = A.s.data[j * A.s.sb + (base + nn) * A.s.sn];
    }
  }
  if (tid < BT) lds_s[A.width * BT + tid] = 0.0f;
  __syncthreads();

  float acc[BT];
#pragma unroll
  for (int j = 0; j < BT; ++j) acc[j] = 0.0f;

  // One register block: prefetch the block after it into `ahead`, accumulate,
  // then close the groups that ended.  A closed group's row sums go to the
  // row-table-ordered buffer at the group's row-table entries (an address
  // made of scalars and the lane id, so closing waits on no vector load).
  // kIndexedF32: the block's weights are gathered once its edge numbers are
  // in (a pipeline that gathers one block ahead measured slower: 82 against
  // 77 us for a headline tick on new weights).
  auto block = [&](Slot (&here)[D], Slot (&ahead)[D], int b) {
    const int64_t ahead0 = first + static_cast<int64_t>(b + 1) * D * 64;
    load_block<FMT, D>(A, ahead0, lane, lane32, ahead);
    gather_block<FMT, D>(A, here);
    const int rem = total - b * D;
    uint32_t ends = rem < D ? bits & ((1u << rem) - 1u) : bits;
    bits = boundary_bits<D>(A, ahead0 / 64);

    float fin[D][BT];
#pragma unroll
    for (int i = 0; i < D; ++i) {
      const float w = decode_slot<FMT>(here[i], lane, gscale);
      if constexpr (BT == 1) {
        acc[0] = __builtin_fmaf(w, lds_s[here[i].c], acc[0]);
      } else {
        const v2f sv = *reinterpret_cast<const v2f*>(lds_s + 2 * here[i].c);
        acc[0] = __builtin_fmaf(w, sv.x, acc[0]);
        acc[1] = __builtin_fmaf(w, sv.y, acc[1]);
      }
      const bool end = (ends >> i) & 1u;
#pragma unroll
      for (int j = 0; j < BT; ++j) {
        fin[i][j] = acc[j];
        acc[j] = end ? 0.0f : acc[j];
      }
    }

    while (ends) {
      const int i = __builtin_ctz(ends);
      ends &= ends - 1u;
      float t[BT];
#pragma unroll
      for (int j = 0; j < BT; ++j) t[j] = fin[0][j];
#pragma unroll
      for (int k = 1; k < D; ++k)
        if (k == i) {
#pragma unroll
          for (int j = 0; j < BT; ++j) t[j] = fin[k][j];
        }
      const int lanes = 1 << now.lg;
#pragma unroll
      for (int j = 0; j < BT; ++j)
        for (int off = 1; off < lanes; off <<= 1) t[j] += __shfl_xor(t[j], off, 64);
      const int k = lane >> now.lg;
      if ((lane & (lanes - 1)) == 0 && k < now.nrows) {
#pragma unroll
        for (int j = 0; j < BT; ++j)
          A.sorted[(static_cast<int64_t>(now.rowtab) + k) * BT + j] = t[j];
      }
      ++g;
      now = next;
      if (g + 1 < g_end) next = load_group(A, g + 1);
    }
  };
  // The waves of a compute unit take turns by age, so with equal streams the
  // oldest would finish well before the youngest and leave the tile's last
  // stretch to a few waves.  A wave's priority instead follows the share of
  // its stream still ahead of it, which keeps the waves abreast.
  auto pace = [&](int b) {
    if constexpr (kPacedWaves) {
      const int ahead = 4 * (total - b * D);
      if (ahead > 3 * total) __builtin_amdgcn_s_setprio(3);
      else if (ahead > 2 * total) __builtin_amdgcn_s_setprio(2);
      else if (ahead > total) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
  };
  for (int b = 0; b * D < total; b += 2) {
    pace(b);
    block(buf_a, buf_b, b);
    if ((b + 1) * D >= total) break;
    pace(b + 1);
    block(buf_b, buf_a, b + 1);
  }
  if constexpr (kPacedWaves) __builtin_amdgcn_s_setprio(0);

  // Map the row-table entries back to rows.  The arguments are read afresh,
  // so the stream loop above need not keep them in scalar registers.
  const PanelArgs E = fresh_args();
  const_i32_ptr tile_e = (const_i32_ptr)(E.tiles + 4 * static_cast<int64_t>(blockIdx.x));
  const int64_t row0_e = tile_e[1];
  if (E.n_panels == 1) {
    // One panel: each wavefront updates the rows of its own entries (one
    // contiguous range: its groups' rows in order) as soon as its stream is
    // done.  The entries were stored by this wavefront's lanes; the fence
    // orders those stores before the loads below.
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
    const_i32_ptr wg_e =
        (const_i32_ptr)(E.wave_groups + static_cast<int64_t>(blockIdx.x) * kPanelWaves + wave);
    const int g_first = wg_e[0], g_last = wg_e[1];
    if (g_first < g_last) {
      const_i32_ptr head = (const_i32_ptr)(E.groups + 4 * static_cast<int64_t>(g_first));
      const_i32_ptr last = (const_i32_ptr)(E.groups + 4 * static_cast<int64_t>(g_last - 1));
      const int e_begin = head[3], e_end = last[3] + (last[2] >> 8);
      for (int e = e_begin + lane; e < e_end; e += 64) {
        const int64_t row = row0_e + static_cast<int64_t>(E.rows[e]);
#pragma unroll
        for (int j = 0; j < BT; ++j) {
          const float sum = E.sorted[static_cast<int64_t>(e) * BT + j];
          if (E.product) store_product(E, row, j, sum);
          else update(E, row, j, sum);
        }
      }
    }
    return;
  }

  // Several panels: the tile's sums (one entry per row of the tile) are
  // gathered into LDS by row, which the panel slice no longer needs, and
  // stored in row order, so that the stores of a wavefront fill whole cache
  // lines.  With more rows than LDS holds this goes in chunks of rows.
  // kMapUnroll entries per thread per round: every load of a round is issued
  // before its first LDS store (an entry past the end rereads the last one
  // and is not stored), so a round waits on memory once.
  constexpr int kMapUnroll = 4;
  constexpr int kChunkRows = CAP + 1;
  const int e0 = tile_e[3];
  const int nrows = static_cast<int>(tile_e[2] - row0_e);
  float* const out = E.partials + (static_cast<int64_t>(tile_e[0]) * E.N + row0_e) * BT;
  const bool coherent = E.counters != nullptr;
  __syncthreads();   // every wavefront's entries stored, the panel slice no longer read
  for (int c0 = 0; c0 < nrows; c0 += kChunkRows) {
    const int c1 = min(nrows, c0 + kChunkRows);
    for (int i0 = tid; i0 < nrows; i0 += kPanelThreads * kMapUnroll) {
      int r[kMapUnroll];
      float value[kMapUnroll][BT];
#pragma unroll
      for (int u = 0; u < kMapUnroll; ++u) {
        const int e = e0 + min(i0 + u * kPanelThreads, nrows - 1);
        r[u] = E.rows[e];
#pragma unroll
        for (int j = 0; j < BT; ++j) value[u][j] = E.sorted[static_cast<int64_t>(e) * BT + j];
      }
#pragma unroll
      for (int u = 0; u < kMapUnroll; ++u)
        if (i0 + u * kPanelThreads < nrows && r[u] >= c0 && r[u] < c1) {
#pragma unroll
          for (int j = 0; j < BT; ++j) lds_s[(r[u] - c0) * BT + j] = value[u][j];
        }
    }
    __syncthreads();
    for (int i = tid; i < (c1 - c0) * BT; i += kPanelThreads) {
      float* const at = out + c0 * BT + i;
      // The combine kernel reads each sum once: stored non-temporally, they leave
      // no dirty lines in this XCD's L2 for the end of the launch to write back
      // (MALL-flushed tick 42.1 against 42.5 us, warm unchanged; the combine's
      // state planes stored the same way cost the next tick's staging 0.35 us).
      if (coherent)
        __hip_atomic_store(at, lds_s[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else
        __builtin_nontemporal_store(lds_s[i], at);
    }
    __syncthreads();
  }
  if (coherent) finish_range<BT>(E, row0_e, tile_e[2]);
}

// Several panels, NS_PANEL_COMBINE_LAUNCH: add each row's panel partial sums
// in panel order, then update; one neuron (all BT columns) per thread.  Every
// load (state, parameters, the first CB panels' sums) is issued before the
// first add, so the kernel waits on memory about once rather than once per
// panel.  CB is the number of panels, up to kCombineBatch, so that no load
// rereads a panel's sum: each load instruction costs address-unit cycles.

template <int BT, int CB>
__global__ __launch_bounds__(kThreads) void panel_combine_kernel(PanelArgs A) {
  const int64_t n = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (n >= A.N) return;
  const int64_t plane = A.N * BT;
  if (A.product) {
    // W @ s alone: the panels' sums in panel order, stored or added.
#pragma unroll
    for (int j = 0; j < BT; ++j) {
      float sum = 0.0f;
      for (int p = 0; p < A.n_panels; ++p) sum += A.partials[p * plane + n * BT + j];
      store_product(A, n, j, sum);
    }
    return;
  }
  const NeuronParams prm = load_params(A.p, n);
  float s[BT], d[BT], a[BT], u[BT], v[BT];
#pragma unroll
  for (int j = 0; j < BT; ++j) {
    s[j] = A.s.get(j, n); d[j] = A.d.get(j, n); a[j] = A.a.get(j, n);
    u[j] = A.u.get(j, n); v[j] = A.v.get(j, n);
  }
  float sum[BT];
#pragma unroll
  for (int j = 0; j < BT; ++j) sum[j] = 0.0f;
  for (int p0 = 0; p0 < A.n_panels; p0 += CB) {
    float part[CB][BT];
#pragma unroll
    for (int q = 0; q < CB; ++q) {
      // Past the last panel, reread the last panel's sum (not added) so that
      // no load waits behind a branch.
      const int p = min(p0 + q, A.n_panels - 1);
#pragma unroll
      for (int j = 0; j < BT; ++j) part[q][j] = A.partials[p * plane + n * BT + j];
    }
#pragma unroll
    for (int q = 0; q < CB; ++q)
#pragma unroll
      for (int j = 0; j < BT; ++j)
        if (p0 + q < A.n_panels) sum[j] += part[q][j];
  }
#pragma unroll
  for (int j = 0; j < BT; ++j) {
    const NextState x = advance_loaded(prm, sum[j], s[j], d[j], a[j], u[j], v[j]);
    A.os.put(j, n, x.soma);
    A.od.put(j, n, x.dendrite);
    A.oa.put(j, n, x.adaptation);
    if (A.oj.data) A.oj.put(j, n, sum[j]);
  }
}

template <int BT>
hipError_t launch_panels(const PanelArgs& A, int fmt, int n_tiles, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(n_tiles)), block(kPanelThreads);
  switch (fmt) {
    case NS_WEIGHT_F32: panel_tick_kernel<BT, NS_WEIGHT_F32><<<grid, block, 0, stream>>>(A); break;
    case NS_WEIGHT_F16: panel_tick_kernel<BT, NS_WEIGHT_F16><<<grid, block, 0, stream>>>(A); break;
    case NS_WEIGHT_E4M3: panel_tick_kernel<BT, NS_WEIGHT_E4M3><<<grid, block, 0, stream>>>(A); break;
    case kNvfp4Pairs: panel_tick_kernel<BT, kNvfp4Pairs><<<grid, block, 0, stream>>>(A); break;
    case kIndexedF32: panel_tick_kernel<BT, kIndexedF32><<<grid, block, 0, stream>>>(A); break;
    default: panel_tick_kernel<BT, NS_WEIGHT_NVFP4><<<grid, block, 0, stream>>>(A); break;
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || A.n_panels == 1 || A.counters) return err;
  const dim3 cgrid(static_cast<unsigned>((A.N + kThreads - 1) / kThreads)), cblock(kThreads);
  switch (std::min(A.n_panels, kCombineBatch)) {
    case 2: panel_combine_kernel<BT, 2><<<cgrid, cblock, 0, stream>>>(A); break;
    case 3: panel_combine_kernel<BT, 3><<<cgrid, cblock, 0, stream>>>(A); break;
    case 4: panel_combine_kernel<BT, 4><<<cgrid, cblock, 0, stream>>>(A); break;
    case 5: panel_combine_kernel<BT, 5><<<cgrid, cblock, 0, stream>>>(A); break;
    case 6: panel_combine_kernel<BT, 6><<<cgrid, cblock, 0, stream>>>(A); break;
    case 7: panel_combine_kernel<BT, 7><<<cgrid, cblock, 0, stream>>>(A); break;
    default: panel_combine_kernel<BT, kCombineBatch><<<cgrid, cblock, 0, stream>>>(A); break;
  }
  return hipGetLastError();
}

int panel_geometry(int64_t batch, int32_t* width, int32_t* waves) {
  if (batch == 1) *width = panel_capacity_neurons<1>();
  else if (batch == 2) *width = panel_capacity_neurons<2>();
  else return fail("column panels support batch widths 1 and 2, not %lld", (long long)batch);
  *waves = kPanelWaves;
  return NS_OK;
}

// Validation and launch of the panel path for ns_dendritic_step (product 0)
// and for the product W @ s alone (1: stored into out_state, 2: added to it).
// With launch false it only validates.
int panel_step(const ns_step_args& a, hipStream_t stream, int product, bool launch) {
  const ns_panel_plan& pl = *a.panels;
  int32_t cap = 0, waves = 0;
  if (int rc = panel_geometry(a.batch, &cap, &waves)) return rc;
  if (pl.waves != waves)
    return fail("panel plan was built for %d wavefronts per workgroup, the kernel runs %d",
                pl.waves, waves);
  if (pl.panel_width < 4 || pl.panel_width > cap || pl.panel_width % 4)
    return fail("panel width %d is not a multiple of 4 in [4, %d]", pl.panel_width, cap);
  if (pl.n_panels < 1 || static_cast<int64_t>(pl.n_panels) * pl.panel_width < a.n_neurons ||
      static_cast<int64_t>(pl.n_panels - 1) * pl.panel_width >= a.n_neurons)
    return fail("%d panels of width %d do not cover N=%lld", pl.n_panels, pl.panel_width,
                (long long)a.n_neurons);
  if (pl.n_tiles < pl.n_panels || pl.n_groups < 0)
    return fail("panel plan needs at least one tile per panel");
  if (pl.n_slots < kPanelTailSlots) return fail("panel plan lacks its tail padding");
  if (!pl.tiles || !pl.wave_groups || !pl.groups || !pl.rows || !pl.last_steps || !pl.col ||
      !pl.weight)
    return fail("panel plan tables are required");
  if (pl.n_step_words < pl.n_slots / 64 / 32 + 2) return fail("panel plan's step bitmap is short");
  if (pl.flags & ~(NS_PANEL_PAIRS | NS_PANEL_COMBINE_LAUNCH | NS_PANEL_INDEXED))
    return fail("unknown panel plan flags %d", pl.flags);
  const bool pairs = (pl.flags & NS_PANEL_PAIRS) != 0;
  const bool indexed = (pl.flags & NS_PANEL_INDEXED) != 0;
  if (indexed && a.matrix.format != NS_WEIGHT_F32)
    return fail("an indexed panel plan reads float32 CSR weights");
  if (indexed && a.matrix.n_edges > 0 && !a.matrix.weight)
    return fail("an indexed panel plan needs the CSR weights");
  // The products always finish in the second kernel.
  const bool one_launch = !product && pl.n_panels > 1 && !(pl.flags & NS_PANEL_COMBINE_LAUNCH);
  if (one_launch) {
    if (!pl.tile_ranges || !pl.range_counters)
      return fail("panel tile ranges and range counters are required with several panels");
    if (pl.n_ranges < 1 || static_cast<int64_t>(pl.n_ranges) * pl.n_panels != pl.n_tiles)
      return fail("%d tiles are not one per panel for each of %d row ranges", pl.n_tiles,
                  pl.n_ranges);
  }
  if (a.matrix.format == NS_WEIGHT_NVFP4 && !pairs && !pl.slot_scales)
    return fail("NVFP4 panels require per-slot block scales");
  if (product) {
    if (!a.out_state.data) return fail("the product needs an output plane");
    if (overlaps(extent(a.out_state, a.batch, a.n_neurons), extent(a.state, a.batch, a.n_neurons)))
      return fail("the product's output must not overlap its source");
    if (!distinct_elements(a.out_state.stride_b, a.out_state.stride_n, a.batch, a.n_neurons))
      return fail("the product's output must not overlap itself (strides %lld, %lld)",
                  (long long)a.out_state.stride_b, (long long)a.out_state.stride_n);
  }
  if (!pl.partials) return fail("the panel path needs its partials workspace");
  const uintptr_t need = (a.matrix.format == NS_WEIGHT_F32 || indexed) ? 4
                         : (a.matrix.format == NS_WEIGHT_F16 ||
                            (a.matrix.format == NS_WEIGHT_NVFP4 && pairs)) ? 2 : 1;
  if (reinterpret_cast<uintptr_t>(pl.col) % 2 || reinterpret_cast<uintptr_t>(pl.weight) % need)
    return fail("panel arrays are misaligned");
  {
    // Tiles write partial sums while other workgroups still read the state and
    // drives, so the workspace may overlap no operand at all.
    const int64_t B = a.batch, N = a.n_neurons;
    const Extent part = extent_of(pl.partials, 1, 1, 1, 2 * int64_t{pl.n_panels} * N * B);
    const Extent others[9] = {extent(a.out_state, B, N), extent(a.out_dendrite, B, N),
                              extent(a.out_adaptation, B, N), extent(a.out_current, B, N),
                              extent(a.state, B, N), extent(a.dendrite, B, N),
                              extent(a.adaptation, B, N), extent(a.drive, B, N),
                              extent(a.dendritic_drive, B, N)};
    for (int i = 0; i < 9; ++i)
      if (overlaps(part, others[i]))
        return fail(i < 4 ? "the partials workspace overlaps an output"
                          : "the partials workspace overlaps an input");
    if (one_launch) {
      const Extent counters = extent_of(pl.range_counters, 1, 1, 1, pl.n_ranges);
      if (overlaps(counters, part)) return fail("the range counters overlap the partials workspace");
      for (int i = 0; i < 9; ++i)
        if (overlaps(counters, others[i]))
          return fail(i < 4 ? "the range counters overlap an output"
                            : "the range counters overlap an input");
    }
  }

  PanelArgs A{};
  A.N = a.n_neurons; A.B = a.batch;
  A.s = plane(a.state, a.state.data); A.d = plane(a.dendrite, a.state.data);
  A.a = plane(a.adaptation, a.state.data);
  A.u = plane(a.drive, a.state.data); A.v = plane(a.dendritic_drive, a.state.data);
  for (int i = 0; i < 6; ++i) A.p.v[i] = Vec{a.params[i].data, a.params[i].stride};
  A.width = pl.panel_width; A.n_panels = pl.n_panels;
  A.tiles = pl.tiles; A.wave_groups = pl.wave_groups;
  A.groups = pl.groups; A.rows = pl.rows;
  if (one_launch) { A.tile_ranges = pl.tile_ranges; A.counters = pl.range_counters; }
  A.last_steps = pl.last_steps;
  A.col = pl.col; A.weight = pl.weight; A.slot_scales = pl.slot_scales;
  A.gscale = a.matrix.global_scale;
  // An indexed plan gathers from the CSR weights; with no edges every slot is
  // padding, which reads element 0 of the (then non-null) slot array instead.
  A.csr_weight = indexed ? (a.matrix.n_edges > 0 ? static_cast<const float*>(a.matrix.weight)
                                                 : static_cast<const float*>(pl.weight))
                         : nullptr;
  A.partials = pl.partials;
  A.sorted = pl.partials + int64_t{pl.n_panels} * a.n_neurons * a.batch;
  A.os = out_plane(a.out_state); A.od = out_plane(a.out_dendrite);
  A.oa = out_plane(a.out_adaptation); A.oj = out_plane(a.out_current);
  const bool aligned = reinterpret_cast<uintptr_t>(a.state.data) % 16 == 0;
  A.product = product;
  A.s_vec = aligned && ((a.batch == 1 && a.state.stride_n == 1) ||
                        (a.batch == 2 && a.state.stride_b == 1 && a.state.stride_n == 2));
  {
    // 32-bit offsets in the one-launch finish: every stride non-negative and
    // every element offset (and n * B + b of the partials) below 2^30, so
    // byte offsets fit 32 bits.
    const int64_t B = a.batch, N = a.n_neurons, limit = int64_t{1} << 30;
    auto fits = [&](int64_t sb, int64_t sn) {
      return sb >= 0 && sn >= 0 && (B - 1) * sb + (N - 1) * sn < limit;
    };
    bool ok = N * B < limit;
    const Plane ins[5] = {A.s, A.d, A.a, A.u, A.v};
    for (const Plane& q : ins) ok = ok && fits(q.sb, q.sn);
    const OutPlane outs[4] = {A.os, A.od, A.oa, A.oj};
    for (const OutPlane& q : outs) ok = ok && fits(q.sb, q.sn);
    for (int i = 0; i < 6; ++i) ok = ok && fits(0, A.p.v[i].stride);
    // The one-launch finish addresses with 32-bit offsets; otherwise the
    // combine kernel finishes the tick (bitwise the same results).
    if (!ok) { A.tile_ranges = nullptr; A.counters = nullptr; }
  }
  if (!launch) return NS_OK;
  const int fmt = indexed ? kIndexedF32
                 : a.matrix.format == NS_WEIGHT_NVFP4 && pairs ? kNvfp4Pairs : a.matrix.format;
  const hipError_t err = a.batch == 1 ? launch_panels<1>(A, fmt, pl.n_tiles, stream)
                                      : launch_panels<2>(A, fmt, pl.n_tiles, stream);
  if (err != hipSuccess) return fail_launch("panel tick", err);
  return NS_OK;
}

}  // namespace ns

using namespace ns;

extern "C" int ns_panel_geometry(int64_t batch, int32_t* max_panel_width, int32_t* waves) {
  clear_error();
  int32_t w = 0, v = 0;
  if (int rc = panel_geometry(batch, &w, &v)) return rc;
  if (max_panel_width) *max_panel_width = w;
  if (waves) *waves = v;
  return NS_OK;
}
