// Column-panel matrix tick for batch widths 1 and 2 (gfx950).
//
// The row-block tick gathers s[col] from L2 for every edge; each 4-byte
// gather moves a whole cache line into the CU, so at 25M edges the gather
// traffic, not HBM, bounds the tick.  Here the columns are cut into panels
// whose slice of s fits in LDS and the CSR is re-laid out (once per graph) so
// that tile (panel p, row stripe s) holds the stripe's edges whose source lies
// in panel p, in row order, with 16-bit panel-local source indices:
//
//  * one workgroup per tile (a panel and a run of stripes) stages its panel of
//    s in LDS, then streams the tile's chunks (512 lanes x `pad` edge slots,
//    16-byte loads; the next chunk's slots and the header after it are in
//    flight while the current chunk is reduced; two barriers per chunk);
//  * each lane decodes its slots, gathers s from LDS, and sums its products
//    per row segment in registers; a row-parallel pass adds the pieces of
//    rows that span lanes in lane order (deterministic, no atomics);
//  * with one panel the lane that finishes a row applies the neuron update;
//    with several, per-panel partial sums go to a workspace and a second,
//    fully parallel kernel adds them in panel order and applies the update
//    (stream order publishes the partials; an in-kernel hand-off would need
//    agent-scope fences, which write back and invalidate L2 on this part).
//
// Results are bitwise repeatable and identical across weight encodings that
// decode to the same float32 values.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "ns_common.h"
#include "ns_host.h"

namespace ns {

template <int BT>
struct PanelCfg;
template <>
struct PanelCfg<1> { static constexpr int pad = 16; };
template <>
struct PanelCfg<2> { static constexpr int pad = 8; };

template <int BT>
constexpr int panel_chunk() { return kPanelThreads * PanelCfg<BT>::pad; }

// LDS left for the panel after the per-chunk scratch (row offsets, segment
// sums, double-buffered), in floats, rounded to whole 4-neuron groups.
template <int BT>
constexpr int panel_capacity_neurons() {
  constexpr int scratch = 2 * (kPanelThreads * 4 + 3 * BT * kPanelThreads * 4) + 512;
  return ((163840 - scratch) / 4 / BT) & ~3;
}

struct PanelArgs {
  int64_t N, B;
  Plane s, d, a, u, v;
  Params p;
  int32_t width, n_panels;
  const int32_t* tiles;
  const int32_t* chunks;
  const uint16_t* row_offsets;
  const uint16_t* lane_rows;
  const int32_t* stripes;
  const uint16_t* col;
  const void* weight;
  const uint8_t* slot_scales;
  const float* gscale;
  float* partials;
  OutPlane os, od, oa;
  int32_t s_vec;   // s.sn == 1 (B == 1) or neuron-major B == 2, 16-byte aligned
};

typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

// One lane's raw slots: PAD 16-bit columns and PAD weights in the matrix encoding.
template <int PAD, int FMT>
struct Raw {
  static constexpr int kColWords = PAD / 2;                       // uint32 words of columns
  static constexpr int kWeightWords = FMT == NS_WEIGHT_F32 ? PAD
                                      : FMT == NS_WEIGHT_F16 ? PAD / 2
                                      : FMT == NS_WEIGHT_E4M3 ? PAD / 4
                                                              : PAD / 8;
  static constexpr int kScaleWords = FMT == NS_WEIGHT_NVFP4 ? PAD / 4 : 0;
  uint32_t col[kColWords];
  uint32_t w[kWeightWords];
  uint32_t sc[kScaleWords > 0 ? kScaleWords : 1];
};

template <int WORDS>
__device__ __forceinline__ void load_words(const void* base, int64_t byte_offset, uint32_t* out) {
  const char* p = static_cast<const char*>(base) + byte_offset;
  if constexpr (WORDS % 4 == 0) {
#pragma unroll
    for (int i = 0; i < WORDS / 4; ++i) {
      const v4u v = *reinterpret_cast<const v4u*>(p + 16 * i);
      out[4 * i] = v.x; out[4 * i + 1] = v.y; out[4 * i + 2] = v.z; out[4 * i + 3] = v.w;
    }
  } else if constexpr (WORDS == 2) {
    const v2u v = *reinterpret_cast<const v2u*>(p);
    out[0] = v.x; out[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < WORDS; ++i) out[i] = reinterpret_cast<const uint32_t*>(p)[i];
  }
}

template <int PAD, int FMT>
__device__ __forceinline__ void load_raw(const PanelArgs& A, int64_t slot, Raw<PAD, FMT>& r) {
  using R = Raw<PAD, FMT>;
  load_words<R::kColWords>(A.col, slot * 2, r.col);
  constexpr int bytes_per_slot_x8 = FMT == NS_WEIGHT_F32 ? 32 : FMT == NS_WEIGHT_F16 ? 16
                                    : FMT == NS_WEIGHT_E4M3 ? 8 : 4;
  load_words<R::kWeightWords>(A.weight, slot * bytes_per_slot_x8 / 8, r.w);
  if constexpr (FMT == NS_WEIGHT_NVFP4) load_words<R::kScaleWords>(A.slot_scales, slot, r.sc);
}

template <int FMT>
__device__ __forceinline__ float decode_slot(const uint32_t* w, const uint32_t* sc, int k,
                                             float gscale) {
  if constexpr (FMT == NS_WEIGHT_F32) {
    return __builtin_bit_cast(float, w[k]);
  } else if constexpr (FMT == NS_WEIGHT_F16) {
    const uint16_t h = static_cast<uint16_t>(w[k >> 1] >> (16 * (k & 1)));
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
  } else if constexpr (FMT == NS_WEIGHT_E4M3) {
    return e4m3_to_float((w[k >> 2] >> (8 * (k & 3))) & 0xFFu) * gscale;
  } else {
    const uint32_t nibble = (w[k >> 3] >> (4 * (k & 7))) & 15u;
    const float bs = e4m3_to_float((sc[k >> 2] >> (8 * (k & 3))) & 0xFFu) * gscale;
    return nvfp4_weight(nibble, bs);
  }
}

__device__ __forceinline__ void update(const PanelArgs& A, int64_t n, int64_t b, float j) {
  const NextState x = advance_one(A.p, n, j, A.s.get(b, n), A.d.get(b, n), A.a.get(b, n),
                                  A.u.get(b, n), A.v.get(b, n));
  A.os.put(b, n, x.soma);
  A.od.put(b, n, x.dendrite);
  A.oa.put(b, n, x.adaptation);
}

typedef const int32_t __attribute__((address_space(4)))* const_i32_ptr;

// Chunk header through the constant address space: scalar loads on their own
// counter, so waiting for a header never waits for the streamed slots.
struct Header {
  int slot0, nedge, row0, nrows, off0, flags, lanes;
};

__device__ __forceinline__ Header load_header(const PanelArgs& A, int c) {
  const_i32_ptr h = (const_i32_ptr)(A.chunks + 8 * static_cast<int64_t>(c));
  return Header{h[0], h[1], h[2], h[3], h[4], h[5], h[6]};
}

template <int BT, int FMT>
__global__ __launch_bounds__(kPanelThreads) void panel_tick_kernel(PanelArgs A) {
  constexpr int PAD = PanelCfg<BT>::pad;
  constexpr int CAP = panel_capacity_neurons<BT>();
  __shared__ __attribute__((aligned(16))) float lds_s[CAP * BT];
  __shared__ int32_t offs[2][kPanelThreads];
  __shared__ float rowsum[2][BT][kPanelThreads];
  __shared__ float head[2][BT][kPanelThreads];
  __shared__ float tail[2][BT][kPanelThreads];
  __shared__ float carry[BT];

  const int tid = threadIdx.x;
  const_i32_ptr tile = (const_i32_ptr)(A.tiles + 4 * static_cast<int64_t>(blockIdx.x));
  const int panel = tile[0], c_begin = tile[1], c_end = tile[2];
  const int64_t base = static_cast<int64_t>(panel) * A.width;
  const int len = static_cast<int>(min<int64_t>(A.width, A.N - base));
  const float gscale = (FMT == NS_WEIGHT_E4M3 || FMT == NS_WEIGHT_NVFP4) ? *A.gscale : 1.0f;

  // Pipeline: slots, row offset and lane row of chunk c+1 are in flight while
  // chunk c is reduced; headers run one chunk further ahead.
  Raw<PAD, FMT> next;
  int next_off = 0, next_lane_row = 0;
  Header h_next{}, h_after{};
  auto fetch = [&](const Header& h) {
    if (tid * PAD < h.nedge) load_raw<PAD, FMT>(A, h.slot0 + tid * PAD, next);
    next_off = tid <= h.nrows ? A.row_offsets[h.off0 + tid] : 0;
    next_lane_row = A.lane_rows[static_cast<int64_t>(h.lanes) * kPanelThreads + tid];
  };
  if (c_begin < c_end) {
    h_next = load_header(A, c_begin);
    fetch(h_next);
    if (c_begin + 1 < c_end) h_after = load_header(A, c_begin + 1);
  }

  // Stage this panel's slice of s (neuron-major, BT columns per neuron), 8 loads deep.
  if (A.s_vec) {
    const v4f* src = reinterpret_cast<const v4f*>(A.s.data + base * BT);
    v4f* dst = reinterpret_cast<v4f*>(lds_s);
    const int n4 = len * BT / 4;
    for (int i0 = tid; i0 < n4; i0 += 8 * kPanelThreads) {
      v4f v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = src[min(i0 + u * kPanelThreads, n4 - 1)];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (i0 + u * kPanelThreads < n4) dst[i0 + u * kPanelThreads] = v[u];
    }
    for (int i = n4 * 4 + tid; i < len * BT; i += kPanelThreads) lds_s[i] = A.s.data[base * BT + i];
  } else {
    for (int i = tid; i < len * BT; i += kPanelThreads) {
      const int nn = i / BT, j = i - nn * BT;
      lds_s[i] = A.s.data[j * A.s.sb + (base + nn) * A.s.sn];
    }
  }
  if (tid < BT) carry[tid] = 0.0f;
  if (tid <= h_next.nrows) offs[0][tid] = next_off;
  __syncthreads();

  for (int c = c_begin; c < c_end; ++c) {
    const int buf = (c - c_begin) & 1;
    const Raw<PAD, FMT> raw = next;
    const Header h = h_next;
    const int lane_row = next_lane_row;
    if (c + 1 < c_end) {
      h_next = h_after;
      fetch(h_next);
      if (c + 2 < c_end) h_after = load_header(A, c + 2);
    }

    // Lane phase: products of this lane's slots (all LDS gathers in flight),
    // then sums per row segment; pieces of lane-spanning rows go to LDS.
    const int first = tid * PAD;
    const int count = h.nedge - first < PAD ? h.nedge - first : PAD;
    float prod[PAD][BT];
#pragma unroll
    for (int k = 0; k < PAD; ++k) {
      const uint32_t word = raw.col[k >> 1];
      const int local = static_cast<int>((word >> (16 * (k & 1))) & 0xFFFFu);
      const float w = decode_slot<FMT>(raw.w, raw.sc, k, gscale);
#pragma unroll
      for (int j = 0; j < BT; ++j) prod[k][j] = k < count ? w * lds_s[local * BT + j] : 0.0f;
    }
    if (count > 0) {
      int r = lane_row;
      int row_end = offs[buf][r + 1];
      bool started_here = offs[buf][r] == first;
      float acc[BT];
#pragma unroll
      for (int j = 0; j < BT; ++j) acc[j] = 0.0f;
      auto store = [&](bool continues) {
#pragma unroll
        for (int j = 0; j < BT; ++j) {
          if (!started_here) head[buf][j][tid] = acc[j];
          else if (continues) tail[buf][j][tid] = acc[j];
          else rowsum[buf][j][r] = acc[j];
        }
      };
#pragma unroll
      for (int k = 0; k < PAD; ++k) {
        if (k < count) {
          while (first + k >= row_end) {   // close row r, skip rows with no edges here
            store(false);
            started_here = true;
            ++r;
            row_end = offs[buf][r + 1];
#pragma unroll
            for (int j = 0; j < BT; ++j) acc[j] = 0.0f;
          }
#pragma unroll
          for (int j = 0; j < BT; ++j) acc[j] += prod[k][j];
        }
      }
      store(first + count < row_end);
    }
    __syncthreads();

    // Row phase: lane i < nrows finishes row i of the chunk; the next chunk's
    // row offsets go to the other buffer.
    if (tid < h.nrows) {
      const int lo = offs[buf][tid], hi = offs[buf][tid + 1];
      float total[BT];
#pragma unroll
      for (int j = 0; j < BT; ++j) total[j] = 0.0f;
      if (lo < hi) {
        const int t0 = lo / PAD, t1 = (hi - 1) / PAD;
        if (t0 == t1) {
#pragma unroll
          for (int j = 0; j < BT; ++j) total[j] = rowsum[buf][j][tid];
        } else {
#pragma unroll
          for (int j = 0; j < BT; ++j) {
            float sum = tail[buf][j][t0];
            for (int t = t0 + 1; t <= t1; ++t) sum += head[buf][j][t];
            total[j] = sum;
          }
        }
      }
      const bool continued = tid == 0 && (h.flags & 1);
      const bool continues = tid == h.nrows - 1 && (h.flags & 2);
#pragma unroll
      for (int j = 0; j < BT; ++j) {
        const float value = continued ? carry[j] + total[j] : total[j];
        if (continues) {
          carry[j] = value;
        } else if (j < A.B) {
          const int64_t row = h.row0 + tid;
          if (A.n_panels == 1) update(A, row, j, value);
          else A.partials[(static_cast<int64_t>(panel) * A.N + row) * A.B + j] = value;
        }
      }
    }
    if (c + 1 < c_end && tid <= h_next.nrows) offs[buf ^ 1][tid] = next_off;
    __syncthreads();
  }
}

// Several panels: add each row's panel partial sums in panel order, then update.
__global__ __launch_bounds__(kThreads) void panel_combine_kernel(PanelArgs A) {
  const int64_t count = A.N * A.B;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < count; i += stride) {
    const int64_t n = i / A.B, b = i - n * A.B;
    float sum = 0.0f;
    for (int p = 0; p < A.n_panels; ++p)
      sum += __builtin_nontemporal_load(A.partials + p * count + i);
    update(A, n, b, sum);
  }
}

template <int BT>
hipError_t launch_panels(const PanelArgs& A, int fmt, int n_tiles, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(n_tiles)), block(kPanelThreads);
  switch (fmt) {
    case NS_WEIGHT_F32: panel_tick_kernel<BT, NS_WEIGHT_F32><<<grid, block, 0, stream>>>(A); break;
    case NS_WEIGHT_F16: panel_tick_kernel<BT, NS_WEIGHT_F16><<<grid, block, 0, stream>>>(A); break;
    case NS_WEIGHT_E4M3: panel_tick_kernel<BT, NS_WEIGHT_E4M3><<<grid, block, 0, stream>>>(A); break;
    default: panel_tick_kernel<BT, NS_WEIGHT_NVFP4><<<grid, block, 0, stream>>>(A); break;
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || A.n_panels == 1) return err;
  const int64_t blocks = std::min<int64_t>((A.N * A.B + kThreads - 1) / kThreads, 16384);
  panel_combine_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, stream>>>(A);
  return hipGetLastError();
}

int panel_geometry(int64_t batch, int32_t* width, int32_t* chunk, int32_t* pad) {
  if (batch == 1) {
    *width = panel_capacity_neurons<1>(); *chunk = panel_chunk<1>(); *pad = PanelCfg<1>::pad;
  } else if (batch == 2) {
    *width = panel_capacity_neurons<2>(); *chunk = panel_chunk<2>(); *pad = PanelCfg<2>::pad;
  } else {
    return fail("column panels support batch widths 1 and 2, not %lld", (long long)batch);
  }
  return NS_OK;
}

// Validation and launch of the panel path for ns_dendritic_step.
int panel_step(const ns_step_args& a, hipStream_t stream) {
  const ns_panel_plan& pl = *a.panels;
  int32_t cap = 0, chunk = 0, pad = 0;
  if (int rc = panel_geometry(a.batch, &cap, &chunk, &pad)) return rc;
  if (pl.chunk_edges != chunk || pl.pad != pad)
    return fail("panel plan was built for chunks of %d x %d, batch %lld needs %d x %d",
                pl.chunk_edges / (pl.pad ? pl.pad : 1), pl.pad, (long long)a.batch,
                chunk / pad, pad);
  if (pl.panel_width < 4 || pl.panel_width > cap || pl.panel_width % 4)
    return fail("panel width %d is not a multiple of 4 in [4, %d]", pl.panel_width, cap);
  if (pl.n_panels < 1 || static_cast<int64_t>(pl.n_panels) * pl.panel_width < a.n_neurons ||
      static_cast<int64_t>(pl.n_panels - 1) * pl.panel_width >= a.n_neurons)
    return fail("%d panels of width %d do not cover N=%lld", pl.n_panels, pl.panel_width,
                (long long)a.n_neurons);
  if (pl.n_tiles < pl.n_panels || pl.n_stripes < 1)
    return fail("panel plan needs at least one tile per panel and one stripe");
  if (!pl.tiles || !pl.chunks || !pl.row_offsets || !pl.lane_rows || !pl.stripes)
    return fail("panel plan tables are required");
  if (pl.n_slots > 0 && (!pl.col || !pl.weight)) return fail("panel columns and weights are required");
  if (a.matrix.format == NS_WEIGHT_NVFP4 && pl.n_slots > 0 && !pl.slot_scales)
    return fail("NVFP4 panels require per-slot block scales");
  if (pl.n_panels > 1 && !pl.partials) return fail("several panels need the partials workspace");
  const uintptr_t need = a.matrix.format == NS_WEIGHT_NVFP4 ? 8 : 16;
  if (reinterpret_cast<uintptr_t>(pl.col) % 16 || reinterpret_cast<uintptr_t>(pl.weight) % need ||
      reinterpret_cast<uintptr_t>(pl.slot_scales) % 16)
    return fail("panel arrays must be 16-byte aligned");
  if (pl.partials) {
    const Extent part = extent_of(pl.partials, 1, 1, 1, int64_t{pl.n_panels} * a.n_neurons * a.batch);
    const Extent outs[3] = {extent(a.out_state, a.batch, a.n_neurons),
                            extent(a.out_dendrite, a.batch, a.n_neurons),
                            extent(a.out_adaptation, a.batch, a.n_neurons)};
    for (const Extent& o : outs)
      if (overlaps(part, o)) return fail("the partials workspace overlaps an output");
  }

  PanelArgs A{};
  A.N = a.n_neurons; A.B = a.batch;
  A.s = plane(a.state); A.d = plane(a.dendrite); A.a = plane(a.adaptation);
  A.u = plane(a.drive); A.v = plane(a.dendritic_drive);
  for (int i = 0; i < 6; ++i) A.p.v[i] = Vec{a.params[i].data, a.params[i].stride};
  A.width = pl.panel_width; A.n_panels = pl.n_panels;
  A.tiles = pl.tiles; A.chunks = pl.chunks; A.row_offsets = pl.row_offsets;
  A.lane_rows = pl.lane_rows; A.stripes = pl.stripes;
  A.col = pl.col; A.weight = pl.weight; A.slot_scales = pl.slot_scales;
  A.gscale = a.matrix.global_scale;
  A.partials = pl.partials;
  A.os = out_plane(a.out_state); A.od = out_plane(a.out_dendrite);
  A.oa = out_plane(a.out_adaptation);
  const bool aligned = reinterpret_cast<uintptr_t>(a.state.data) % 16 == 0;
  A.s_vec = aligned && ((a.batch == 1 && a.state.stride_n == 1) ||
                        (a.batch == 2 && a.state.stride_b == 1 && a.state.stride_n == 2));
  const hipError_t err = a.batch == 1 ? launch_panels<1>(A, a.matrix.format, pl.n_tiles, stream)
                                      : launch_panels<2>(A, a.matrix.format, pl.n_tiles, stream);
  if (err != hipSuccess) return fail_launch("panel tick", err);
  return NS_OK;
}

}  // namespace ns

using namespace ns;

extern "C" int ns_panel_geometry(int64_t batch, int32_t* max_panel_width, int32_t* chunk_edges,
                                 int32_t* pad) {
  clear_error();
  int32_t w = 0, c = 0, p = 0;
  if (int rc = panel_geometry(batch, &w, &c, &p)) return rc;
  if (max_panel_width) *max_panel_width = w;
  if (chunk_edges) *chunk_edges = c;
  if (pad) *pad = p;
  return NS_OK;
}
