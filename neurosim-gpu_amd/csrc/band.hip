// Fused dendritic matrix tick over source bands, for wide batches (16 state
// columns per workgroup; 8 when the batch is an odd multiple of 8, 4 when it
// is an odd multiple of 4) whose state is larger than an XCD's L2.
//
// Semantics follow the reference's fused kernel (csrc/compartmental.cu:121-140
// and :72-90): j = W @ s over the batch columns, then the three-state update.
// The work decomposition is this library's own (ns_plan_bands):
//
//  * A gather of one source's 16 columns is a 64-byte row of the neuron-major
//    state.  Random 64-byte gathers over a state far larger than L2 are served
//    by the MALL; confined to a band of a few MB they hit the XCD's L2 and run
//    about twice as fast.  So sources are cut into bands, and every
//    workgroup walks the bands in the same order: the workgroups resident on
//    one XCD gather from about one band at a time.
//  * One 1024-lane workgroup (one per compute unit) owns a block of
//    destination rows and one tile of C = 16 (or 8, or 4) columns.  Its row sums
//    live in LDS for the whole tick, so no partial sums leave the compute
//    unit.  A row's edges in one band lie in one group of one wavefront, so
//    within a band its LDS updates race with no other wavefront; its groups
//    of different bands may lie in different wavefronts, which the barrier
//    after each band orders.  The wavefronts finish each band before any
//    starts the next: a compute unit's sixteen
//    wavefronts then gather from one band, and the workgroups of an XCD, which
//    start together with equal work, stay within a band or two of each other.
//    (Two 256-lane workgroups per compute unit drifted apart by up to a dozen
//    bands, the older one issuing first; L2 then held about half the
//    gathers, against nearly nine in ten with the barrier.)
//  * Per band the block's rows are packed 64 lanes at a time, longest
//    segments first, and each group goes to the wavefront with the fewest
//    steps in the band so far; lane l walks its row's segment.  The four lanes
//    of a quad gather their four rows' 64-byte source rows together, each
//    lane one 16-byte quarter of each, and each lane keeps the running sums
//    of its quarter's four columns for the quad's four rows (16 registers);
//    with 8 columns a pair of lanes does the same for its two rows' 32-byte
//    source rows, and with 4 each lane loads its own 16-byte row.  A lane
//    whose row ends early may take a second, shorter row in the group's
//    remaining steps: at the switch step it adds its sums to the first row's
//    LDS sums and starts again from zero.  At the group's end the lane adds
//    them to its (last) row's LDS sums.
//  * A group is cut into register blocks of D steps whose slots are
//    lane-major, so a lane loads its D source indices and its D weight codes
//    in one load each.  Blocks are software-pipelined: the slots of block b+1
//    are loaded while block b's gathers are in flight, and steps past a
//    block's count issue no gathers.  Every vector-memory instruction costs
//    the address units cycles whatever its lanes read, so the loop is built
//    to issue few of them.
//  * After the last band the workgroup applies the update to its rows.
//
// Summation order: per row, bands in order; within a band, the row's edges in
// CSR order, accumulated one at a time.  It depends only on the plan, so the
// tick is bitwise repeatable and identical across weight encodings that decode
// to the same float32 values.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "ns_common.h"
#include "ns_host.h"

namespace ns {

struct BandArgs {
  int64_t N, B;
  Plane s, d, a, u, v;
  Params p;
  const float* s_rows;   // neuron-major state: source n's columns at s_rows + n * s_stride
  int64_t s_stride;
  int32_t band_width, block_rows;
  int32_t n_bands, reserved;
  uint32_t row_bytes;    // s_stride * 4
  int32_t band_bytes;    // band_width * row_bytes: the buffer range of one band
  const int32_t* wave_blocks;
  const int32_t* blocks;
  const uint32_t* rows;   // lane words: first row, second row, switch step
  const uint16_t* col;
  const void* weight;
  const uint8_t* slot_scales;
  const float* gscale;
  OutPlane os, od, oa;
  OutPlane oj;   // optional: j as well (data null: not written)
};

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr uint32_t kBandPad = 0xFFFFu;

struct BandSlot {
  uint32_t c, w, sc;
};

struct BandBlock {
  int32_t step0, band, steps, last, t0, group;   // t0: the block's first step in its group
};

__device__ __forceinline__ BandBlock load_band_block(const BandArgs& A, int32_t b) {
  const int32_t* q = A.blocks + 4 * static_cast<int64_t>(b);
  const int32_t info = q[2];
  return BandBlock{q[0], q[1], info & 0xFF, (info >> 8) & 1, info >> 9, q[3]};
}

// BYTES consecutive bytes at p (1, 2, 4, 8, 16 or 32; aligned to their size,
// at most 16) as little-endian 32-bit words, in one or two load instructions.
template <int BYTES>
__device__ __forceinline__ void load_run(const void* p, uint32_t (&w)[(BYTES + 3) / 4]) {
  if constexpr (BYTES == 1) {
    w[0] = *static_cast<const uint8_t*>(p);
  } else if constexpr (BYTES == 2) {
    w[0] = *static_cast<const uint16_t*>(p);
  } else if constexpr (BYTES == 4) {
    w[0] = *static_cast<const uint32_t*>(p);
  } else if constexpr (BYTES == 8) {
    const uint2 v = *static_cast<const uint2*>(p);
    w[0] = v.x; w[1] = v.y;
  } else {
    static_assert(BYTES == 16 || BYTES == 32, "runs of 1 to 32 bytes");
#pragma unroll
    for (int h = 0; h < BYTES / 16; ++h) {
      const uint4 v = static_cast<const uint4*>(p)[h];
      w[4 * h + 0] = v.x; w[4 * h + 1] = v.y; w[4 * h + 2] = v.z; w[4 * h + 3] = v.w;
    }
  }
}

// Field k of BITS bits (4, 8, 16 or 32) of a run of little-endian words.
template <int BITS, int N>
__device__ __forceinline__ uint32_t run_field(const uint32_t (&w)[N], int k) {
  if constexpr (BITS == 32) {
    return w[k];
  } else {
    constexpr int per = 32 / BITS;
    return (w[k / per] >> (BITS * (k % per))) & ((1u << BITS) - 1u);
  }
}

// This lane's D slots of the block and its lane word in the block's group.  A
// block's slots are lane-major (lane l's steps at 64*first_step + l*D + k), so
// the lane's D source indices come in one load and its D weight codes in
// another, rather than one load per step.  The loads do not depend on the
// block's step count (the slot array has D padding steps past its end, the
// block table a sentinel record), so the compiler can count them and wait for
// exactly the ones it needs.
template <int FMT, int D>
__device__ __forceinline__ void load_band_slots(const BandArgs& A, const BandBlock& blk, int lane,
                                                BandSlot (&x)[D], uint32_t& row) {
  const int64_t q0 = int64_t{64} * blk.step0 + int64_t{D} * lane;
  uint32_t cw[(2 * D + 3) / 4];
  load_run<2 * D>(A.col + q0, cw);
#pragma unroll
  for (int k = 0; k < D; ++k) {
    x[k].c = run_field<16>(cw, k);
    x[k].sc = 0u;
  }
  if constexpr (FMT == NS_WEIGHT_F32) {
    uint32_t ww[D];
    load_run<4 * D>(static_cast<const uint32_t*>(A.weight) + q0, ww);
#pragma unroll
    for (int k = 0; k < D; ++k) x[k].w = ww[k];
  } else if constexpr (FMT == NS_WEIGHT_F16) {
    uint32_t ww[(2 * D + 3) / 4];
    load_run<2 * D>(static_cast<const uint16_t*>(A.weight) + q0, ww);
#pragma unroll
    for (int k = 0; k < D; ++k) x[k].w = run_field<16>(ww, k);
  } else if constexpr (FMT == NS_WEIGHT_E4M3) {
    uint32_t ww[(D + 3) / 4];
    load_run<D>(static_cast<const uint8_t*>(A.weight) + q0, ww);
#pragma unroll
    for (int k = 0; k < D; ++k) x[k].w = run_field<8>(ww, k);
  } else {
    // Two nibbles per byte in slot order (q0 is even): step k's nibble is
    // nibble k of the lane's D/2 bytes; one block-scale code per slot.
    uint32_t ww[(D / 2 + 3) / 4], sw[(D + 3) / 4];
    load_run<D / 2>(static_cast<const uint8_t*>(A.weight) + q0 / 2, ww);
    load_run<D>(A.slot_scales + q0, sw);
#pragma unroll
    for (int k = 0; k < D; ++k) {
      x[k].w = run_field<4>(ww, k);
      x[k].sc = run_field<8>(sw, k);
    }
  }
  row = A.rows[int64_t{64} * blk.group + lane];
}

// Adds four running sums (acc[4j .. 4j+3]: columns 4*seg .. 4*seg+3 of one
// row) to that row's LDS sums; a row holds G groups of four columns.
template <int G>
__device__ __forceinline__ void add_piece(v4f* sums4, uint32_t row, int seg,
                                          float (&acc)[4 * G], int j) {
  v4f t = sums4[row * G + seg];
  t.x += acc[4 * j + 0]; t.y += acc[4 * j + 1];
  t.z += acc[4 * j + 2]; t.w += acc[4 * j + 3];
  sums4[row * G + seg] = t;
}

// Buffer resource word 3 of a raw (unswizzled, stride 0) buffer on gfx9.
constexpr int kRawBufferWord3 = 0x00020000;
// A byte offset beyond every band's buffer range: the load returns zeros.
constexpr uint32_t kBandOutOfRange = 0x80000000u;

// An NVFP4 slot carries its own nibble (see load_band_slots).
template <int FMT>
__device__ __forceinline__ float decode_band(const BandSlot& x, float gscale) {
  if constexpr (FMT == NS_WEIGHT_F32) {
    return __builtin_bit_cast(float, x.w);
  } else if constexpr (FMT == NS_WEIGHT_F16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(x.w)));
  } else if constexpr (FMT == NS_WEIGHT_E4M3) {
    return e4m3_to_float(x.w) * gscale;
  } else {
    return e2m1_pair(x.w).x * (e4m3_to_float(x.sc) * gscale);
  }
}

// Value `v` of lane J of each group of G lanes (G = 4: a quad; G = 2: a pair
// within a quad), for every lane of the group: a DPP quad permutation.
template <int G, int J>
__device__ __forceinline__ uint32_t from_group_lane(uint32_t v) {
  constexpr int sel = G == 4 ? J | (J << 2) | (J << 4) | (J << 6)
                             : J | (J << 2) | ((2 + J) << 4) | ((2 + J) << 6);
  return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), sel, 0xF, 0xF, false));
}
template <int G>
__device__ __forceinline__ void group_values(uint32_t v, uint32_t (&out)[G]) {
  if constexpr (G == 1) {
    out[0] = v;   // a lane gathers its own row
  } else {
    out[0] = from_group_lane<G, 0>(v);
    out[1] = from_group_lane<G, 1>(v);
    if constexpr (G == 4) {
      out[2] = from_group_lane<G, 2>(v);
      out[3] = from_group_lane<G, 3>(v);
    }
  }
}

// C: state columns per workgroup, 16 (a 64-byte source row, gathered by the
// four lanes of a quad), 8 (a 32-byte row, gathered by a pair of lanes) or 4
// (a 16-byte row, gathered by its own lane).
template <int FMT, int D, int C>
__global__ __launch_bounds__(kBandWaves * 64) void band_tick_kernel(BandArgs A) {
  constexpr int G = C / 4;   // lanes that gather a row together, 16 bytes each
  extern __shared__ __attribute__((aligned(16))) float sums[];   // [block_rows][C]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * A.block_rows;
  const int nrows = static_cast<int>(min<int64_t>(A.block_rows, A.N - r0));
  const int64_t b0 = int64_t{C} * blockIdx.y;
  const float gscale = (FMT == NS_WEIGHT_E4M3 || FMT == NS_WEIGHT_NVFP4) ? *A.gscale : 1.0f;
  v4f* const sums4 = reinterpret_cast<v4f*>(sums);
  for (int i = tid; i < nrows * G; i += kBandWaves * 64) sums4[i] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  __syncthreads();

  const int32_t* wb = A.wave_blocks + static_cast<int64_t>(blockIdx.x) * kBandWaves + wave;
  const int32_t b_begin = wb[0], b_end = wb[1];
  const float* const srow = A.s_rows + b0;
  float acc[4 * G];
#pragma unroll
  for (int j = 0; j < 4 * G; ++j) acc[j] = 0.0f;

  BandBlock cur{};
  BandSlot here[D];
  uint32_t row = kBandNoRow | (kBandNoRow << kBandRowBits);
  if (b_begin < b_end) {
    cur = load_band_block(A, b_begin);
    load_band_slots<FMT, D>(A, cur, lane, here, row);
  }
  // Every wavefront passes exactly n_bands barriers, whatever its blocks.
  int32_t b = b_begin;
  for (int32_t band = 0; band < A.n_bands; ++band) {
  for (; b < b_end && cur.band == band; ++b) {
    // Gathers of this block: each slot's whole C-column source row, as buffer
    // loads over the band's rows (32-bit offsets, so no 64-bit address per
    // load is held in registers).
    const int64_t base = static_cast<int64_t>(cur.band) * A.band_width;
    const __amdgpu_buffer_rsrc_t band_rows = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(srow + base * A.s_stride), 0, A.band_bytes, kRawBufferWord3);
    // The G lanes of a group gather together: at step k, instruction j loads
    // piece `seg` (16 bytes) of the source row of the group's lane j, so one
    // load instruction touches 64/G rows, each in one 4G-float piece, rather
    // than 64 rows as when each lane loads its own row in G instructions: 1/G
    // of the cache-line accesses.  Lane l then accumulates columns
    // 4*seg .. 4*seg+3 of the rows of its group's G lanes (acc[4j..4j+3] for
    // lane j's row), in step order, and adds them to those rows' LDS sums at
    // each row's switch or end.  A padding slot loads at an offset beyond the
    // band's range, which reads zeros.
    const int seg = lane & (G - 1);
    v4f g[D][G];
#pragma unroll
    for (int k = 0; k < D; ++k) {
      // Steps past the block's end issue no loads (a wave-uniform test): each
      // load instruction costs address-unit cycles whatever its lanes read.
      if (k >= cur.steps) {
#pragma unroll
        for (int j = 0; j < G; ++j) g[k][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        continue;
      }
      uint32_t cq[G];
      group_values<G>(here[k].c, cq);
#pragma unroll
      for (int j = 0; j < G; ++j) {
        const bool real = cq[j] != kBandPad;
        const uint32_t at = real ? cq[j] * A.row_bytes + 16u * seg : kBandOutOfRange;
        g[k][j] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(band_rows, at, 0, 0));
      }
    }
    // The next block's slots load while the gathers are in flight (past the
    // wavefront's last block this reads the next wavefront's first block or
    // the sentinel; those values go unused).
    const BandBlock nxt = load_band_block(A, b + 1);
    BandSlot ahead[D];
    uint32_t row_ahead;
    load_band_slots<FMT, D>(A, nxt, lane, ahead, row_ahead);
    // The group's lane words: lane j's rows and the step where it switches.
    uint32_t rowq[G];
    group_values<G>(row, rowq);
#pragma unroll
    for (int k = 0; k < D; ++k) {
      if (k < cur.steps) {
        const float w = decode_band<FMT>(here[k], gscale);
        uint32_t wq[G];
        group_values<G>(__builtin_bit_cast(uint32_t, w), wq);
#pragma unroll
        for (int j = 0; j < G; ++j) {
          const float wj = __builtin_bit_cast(float, wq[j]);
          acc[4 * j + 0] += wj * g[k][j].x;
          acc[4 * j + 1] += wj * g[k][j].y;
          acc[4 * j + 2] += wj * g[k][j].z;
          acc[4 * j + 3] += wj * g[k][j].w;
        }
#pragma unroll
        for (int j = 0; j < G; ++j) {
          const int turn_j = static_cast<int>(rowq[j] >> 24) - cur.t0 - 1;
          if (k == turn_j) {   // lane j moves on to its second row
            add_piece<G>(sums4, rowq[j] & kBandNoRow, seg, acc, j);
            acc[4 * j + 0] = acc[4 * j + 1] = acc[4 * j + 2] = acc[4 * j + 3] = 0.0f;
          }
        }
      }
    }
    if (cur.last) {
#pragma unroll
      for (int j = 0; j < G; ++j) {
        const uint32_t first_j = rowq[j] & kBandNoRow;
        const uint32_t second_j = (rowq[j] >> kBandRowBits) & kBandNoRow;
        const uint32_t r = second_j != kBandNoRow ? second_j : first_j;
        if (r != kBandNoRow) add_piece<G>(sums4, r, seg, acc, j);
      }
#pragma unroll
      for (int j = 0; j < 4 * G; ++j) acc[j] = 0.0f;
    }
    cur = nxt;
    row = row_ahead;
#pragma unroll
    for (int k = 0; k < D; ++k) here[k] = ahead[k];
  }
  __syncthreads();
  }

  // The update: consecutive lanes take consecutive columns of a row.
  for (int i = tid; i < nrows * C; i += kBandWaves * 64) {
    const int64_t n = r0 + i / C;
    const int64_t b = b0 + i % C;
    const NextState x = advance_one(A.p, n, sums[i], A.s.get(b, n), A.d.get(b, n),
                                    A.a.get(b, n), A.u.get(b, n), A.v.get(b, n));
    A.os.put(b, n, x.soma);
    A.od.put(b, n, x.dendrite);
    A.oa.put(b, n, x.adaptation);
    if (A.oj.data) A.oj.put(b, n, sums[i]);
  }
}

template <int D, int C>
hipError_t launch_bands(const BandArgs& A, int fmt, int n_row_blocks, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(n_row_blocks), static_cast<unsigned>(A.B / C));
  const dim3 block(kBandWaves * 64);
  const size_t lds = static_cast<size_t>(A.block_rows) * C * sizeof(float);
  switch (fmt) {
    case NS_WEIGHT_F32: band_tick_kernel<NS_WEIGHT_F32, D, C><<<grid, block, lds, stream>>>(A); break;
    case NS_WEIGHT_F16: band_tick_kernel<NS_WEIGHT_F16, D, C><<<grid, block, lds, stream>>>(A); break;
    case NS_WEIGHT_E4M3: band_tick_kernel<NS_WEIGHT_E4M3, D, C><<<grid, block, lds, stream>>>(A); break;
    default: band_tick_kernel<NS_WEIGHT_NVFP4, D, C><<<grid, block, lds, stream>>>(A); break;
  }
  return hipGetLastError();
}

template <int D>
hipError_t launch_bands(const BandArgs& A, int fmt, int n_row_blocks, hipStream_t stream) {
  return A.B % 16 == 0  ? launch_bands<D, 16>(A, fmt, n_row_blocks, stream)
         : A.B % 8 == 0 ? launch_bands<D, 8>(A, fmt, n_row_blocks, stream)
                        : launch_bands<D, 4>(A, fmt, n_row_blocks, stream);
}

template <int D, int C>
hipError_t allow_band_lds() {
  const int bytes = band_max_rows(C) * C * static_cast<int>(sizeof(float));
  const void* kernels[4] = {reinterpret_cast<const void*>(&band_tick_kernel<NS_WEIGHT_F32, D, C>),
                            reinterpret_cast<const void*>(&band_tick_kernel<NS_WEIGHT_F16, D, C>),
                            reinterpret_cast<const void*>(&band_tick_kernel<NS_WEIGHT_E4M3, D, C>),
                            reinterpret_cast<const void*>(&band_tick_kernel<NS_WEIGHT_NVFP4, D, C>)};
  for (const void* k : kernels) {
    const hipError_t err =
        hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

template <int D>
hipError_t allow_band_lds() {
  hipError_t e = allow_band_lds<D, 16>();
  if (e == hipSuccess) e = allow_band_lds<D, 8>();
  return e != hipSuccess ? e : allow_band_lds<D, 4>();
}

int check_step_head(const ns_step_args& a);
int check_step_planes(const ns_step_args& a);

int band_step(const ns_step_args& a, const ns_band_plan& pl, hipStream_t stream) {
  if (a.batch % 4) return fail("the band kernel needs a batch that is a multiple of 4, not %lld",
                               (long long)a.batch);
  if (a.state.stride_b != 1 || a.state.stride_n < a.batch || a.state.stride_n % 4 ||
      reinterpret_cast<uintptr_t>(a.state.data) % 16)
    return fail("the band kernel needs a neuron-major state with 16-byte aligned rows");
  if (pl.band_width < 1 || pl.band_width > 65535) return fail("band width must be in [1, 65535]");
  if (pl.n_bands != (a.n_neurons + pl.band_width - 1) / pl.band_width)
    return fail("%d bands of width %d do not cover N=%lld", pl.n_bands, pl.band_width,
                (long long)a.n_neurons);
  if (pl.block_rows < 1 || pl.block_rows > band_max_rows(a.batch))
    return fail("block_rows must be in [1, %d] at batch %lld", band_max_rows(a.batch),
                (long long)a.batch);
  if (pl.n_row_blocks != (a.n_neurons + pl.block_rows - 1) / pl.block_rows)
    return fail("%d row blocks of %d rows do not cover N=%lld", pl.n_row_blocks, pl.block_rows,
                (long long)a.n_neurons);
  if (pl.block_steps != 2 && pl.block_steps != 4 && pl.block_steps != 8)
    return fail("band plans are cut into register blocks of 2, 4 or 8 steps, not %d",
                pl.block_steps);
  if (pl.n_blocks < 0 || pl.n_groups < 1 || pl.n_slots < int64_t{kBandMaxBlockSteps} * 64)
    return fail("band plan lacks its sentinel group or tail padding");
  if (!pl.wave_blocks || !pl.blocks || !pl.rows || !pl.col || !pl.weight)
    return fail("band plan tables are required");
  if (a.matrix.format == NS_WEIGHT_NVFP4 && !pl.slot_scales)
    return fail("NVFP4 bands require per-slot block scales");
  // A lane loads its block's source indices, weight codes and block scales
  // as runs of up to 16 bytes (lane-major slots).
  if (reinterpret_cast<uintptr_t>(pl.col) % 16 || reinterpret_cast<uintptr_t>(pl.weight) % 16 ||
      reinterpret_cast<uintptr_t>(pl.rows) % 4 ||
      (pl.slot_scales && reinterpret_cast<uintptr_t>(pl.slot_scales) % 16))
    return fail("band arrays are misaligned (col, weight and slot_scales need 16-byte alignment)");
  if (int64_t{pl.band_width} * a.state.stride_n * 4 >= int64_t{kBandOutOfRange})
    return fail("a band of the state (band width x row stride) must be under 2 GiB");
  if (static_cast<int64_t>(pl.n_row_blocks) > 0x7FFFFFFF || a.batch / 4 > 65535)
    return fail("band grid too large");

  BandArgs A{};
  A.N = a.n_neurons; A.B = a.batch;
  A.s = plane(a.state, a.state.data); A.d = plane(a.dendrite, a.state.data);
  A.a = plane(a.adaptation, a.state.data);
  A.u = plane(a.drive, a.state.data); A.v = plane(a.dendritic_drive, a.state.data);
  for (int i = 0; i < 6; ++i) A.p.v[i] = Vec{a.params[i].data, a.params[i].stride};
  A.s_rows = a.state.data; A.s_stride = a.state.stride_n;
  A.row_bytes = static_cast<uint32_t>(a.state.stride_n * 4);
  A.band_bytes = static_cast<int32_t>(int64_t{pl.band_width} * a.state.stride_n * 4);
  A.band_width = pl.band_width; A.block_rows = pl.block_rows; A.n_bands = pl.n_bands;
  A.wave_blocks = pl.wave_blocks; A.blocks = pl.blocks; A.rows = pl.rows; A.col = pl.col;
  A.weight = pl.weight; A.slot_scales = pl.slot_scales; A.gscale = a.matrix.global_scale;
  A.os = out_plane(a.out_state); A.od = out_plane(a.out_dendrite);
  A.oa = out_plane(a.out_adaptation); A.oj = out_plane(a.out_current);
  static const hipError_t lds_ok = [] {
    hipError_t e = allow_band_lds<2>();
    if (e == hipSuccess) e = allow_band_lds<4>();
    return e != hipSuccess ? e : allow_band_lds<8>();
  }();
  if (lds_ok != hipSuccess) return fail_launch("band tick (LDS limit)", lds_ok);
  const hipError_t err =
      pl.block_steps == 2   ? launch_bands<2>(A, a.matrix.format, pl.n_row_blocks, stream)
      : pl.block_steps == 4 ? launch_bands<4>(A, a.matrix.format, pl.n_row_blocks, stream)
                            : launch_bands<8>(A, a.matrix.format, pl.n_row_blocks, stream);
  if (err != hipSuccess) return fail_launch("band tick", err);
  return NS_OK;
}

}  // namespace ns

using namespace ns;

extern "C" int ns_dendritic_step_bands(const ns_step_args* args, const ns_band_plan* plan,
                                       void* stream) {
  clear_error();
  if (!args || !plan) return fail("arguments and a band plan are required");
  if (int rc = check_step_head(*args)) return rc;
  if (args->batch == 0) return NS_OK;  // empty planes may carry null pointers
  if (int rc = check_step_planes(*args)) return rc;
  return band_step(*args, *plan, static_cast<hipStream_t>(stream));
}
