// Fused dendritic matrix tick for gfx950: CSR gather-product over B columns,
// then the three-state update, with fp32 / fp16 / fp8 e4m3 / nvfp4 weights
// decoded in-register and accumulated in float32.
//
// Semantics follow the reference's fused kernel (csrc/compartmental.cu:121-140
// and :72-90) and its PyTorch twin (runtime.py:78-79, compartmental.py:152-183);
// the work decomposition is this library's own:
//
//  * Rows are cut on the host into row blocks of consecutive rows whose edges
//    fit one workgroup's edge capacity (ns_plan_row_blocks).  One 256-lane
//    workgroup owns one row block and one tile of BT batch columns.
//  * Phase 1 streams the block's contiguous edge range with aligned 16-byte
//    loads of col_idx (4 edges per lane per pass) and the matching weight
//    bytes, decodes, gathers s[col] for the BT columns and writes the products
//    to LDS ([column][edge] layout, padded).
//  * Phase 2 assigns a power-of-two group of lanes to every row (more lanes
//    to fewer, longer rows), reduces the row's products from LDS, finishes
//    with cross-lane xor shuffles and applies the update on one lane per
//    (row, column).
//  * A block that does not fit (a row longer than the capacity) is reduced
//    row by row by the whole workgroup.
//
// The summation order depends only on the plan, the batch tile and the
// weights' position, so results are bitwise repeatable and identical across
// weight encodings that decode to the same float32 values.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>

#include "ns_common.h"
#include "ns_host.h"

namespace ns {

template <int BT>
struct TileCfg;
template <>
struct TileCfg<1> { static constexpr int passes = 2; };
template <>
struct TileCfg<2> { static constexpr int passes = 2; };
template <>
struct TileCfg<4> { static constexpr int passes = 1; };
template <>
struct TileCfg<8> { static constexpr int passes = 1; };
template <>
struct TileCfg<16> { static constexpr int passes = 1; };

template <int BT>
constexpr int block_capacity() { return kThreads * 4 * TileCfg<BT>::passes; }

struct TickArgs {
  int64_t N, B, M;
  Plane s, d, a, u, v;
  Params p;
  const int32_t* rowptr;
  const int32_t* col;
  const void* weight;
  const uint8_t* scales;
  const float* gscale;
  const int32_t* bounds;
  int64_t n_blocks;
  OutPlane os, od, oa;
  OutPlane oj;          // optional: j as well (data null: not written)
  int32_t quad_loads;   // col/weight pointers aligned for one-quad vector loads
  int32_t s_vec4;       // s is neuron-major with 16-byte aligned column groups
  int32_t spmm_only;    // write j to `os` instead of advancing
  int32_t spmm_accumulate;  // with spmm_only: add j to `os` instead
};

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

// Decode the four weights of the aligned quad [q, q+4) (q % 4 == 0).
// Lanes past the end of the arrays read nothing; those edges are masked later.
template <int FMT>
__device__ __forceinline__ void load_quad(const TickArgs& A, int64_t q, bool vec, int c[4],
                                          float w[4], float gscale) {
  if (vec) {
    const v4i cv = *reinterpret_cast<const v4i*>(A.col + q);
    c[0] = cv.x; c[1] = cv.y; c[2] = cv.z; c[3] = cv.w;
    if constexpr (FMT == NS_WEIGHT_F32) {
      const v4f wv = *reinterpret_cast<const v4f*>(static_cast<const float*>(A.weight) + q);
      w[0] = wv.x; w[1] = wv.y; w[2] = wv.z; w[3] = wv.w;
    } else if constexpr (FMT == NS_WEIGHT_F16) {
      const v4h hv = *reinterpret_cast<const v4h*>(static_cast<const _Float16*>(A.weight) + q);
      w[0] = static_cast<float>(hv.x); w[1] = static_cast<float>(hv.y);
      w[2] = static_cast<float>(hv.z); w[3] = static_cast<float>(hv.w);
    } else if constexpr (FMT == NS_WEIGHT_E4M3) {
      const uint32_t codes = *reinterpret_cast<const uint32_t*>(
          static_cast<const uint8_t*>(A.weight) + q);
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = e4m3_to_float((codes >> (8 * k)) & 0xFFu) * gscale;
    } else {
      const uint32_t nibbles = *reinterpret_cast<const uint16_t*>(
          static_cast<const uint8_t*>(A.weight) + (q >> 1));
      const float bs = e4m3_to_float(A.scales[q >> 4]) * gscale;
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = nvfp4_weight((nibbles >> (4 * k)) & 15u, bs);
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t e = q + k;
    c[k] = 0;
    w[k] = 0.0f;
    if (e < A.M) {
      c[k] = A.col[e];
      if constexpr (FMT == NS_WEIGHT_F32) {
        w[k] = static_cast<const float*>(A.weight)[e];
      } else if constexpr (FMT == NS_WEIGHT_F16) {
        w[k] = static_cast<float>(static_cast<const _Float16*>(A.weight)[e]);
      } else if constexpr (FMT == NS_WEIGHT_E4M3) {
        w[k] = e4m3_to_float(static_cast<const uint8_t*>(A.weight)[e]) * gscale;
      } else {
        const uint32_t byte = static_cast<const uint8_t*>(A.weight)[e >> 1];
        const float bs = e4m3_to_float(A.scales[e >> 4]) * gscale;
        w[k] = nvfp4_weight((byte >> (4 * (e & 1))) & 15u, bs);
      }
    }
  }
}

template <int FMT>
__device__ __forceinline__ float load_weight(const TickArgs& A, int64_t e, float gscale) {
  if constexpr (FMT == NS_WEIGHT_F32) {
    return static_cast<const float*>(A.weight)[e];
  } else if constexpr (FMT == NS_WEIGHT_F16) {
    return static_cast<float>(static_cast<const _Float16*>(A.weight)[e]);
  } else if constexpr (FMT == NS_WEIGHT_E4M3) {
    return e4m3_to_float(static_cast<const uint8_t*>(A.weight)[e]) * gscale;
  } else {
    const uint32_t byte = static_cast<const uint8_t*>(A.weight)[e >> 1];
    const float bs = e4m3_to_float(A.scales[e >> 4]) * gscale;
    return nvfp4_weight((byte >> (4 * (e & 1))) & 15u, bs);
  }
}

__device__ __forceinline__ void finish(const TickArgs& A, int64_t n, int64_t b, float j) {
  if (A.spmm_only) {
    A.os.put(b, n, A.spmm_accumulate ? A.os.data[b * A.os.sb + n * A.os.sn] + j : j);
    return;
  }
  const NextState x = advance_one(A.p, n, j, A.s.get(b, n), A.d.get(b, n), A.a.get(b, n),
                                  A.u.get(b, n), A.v.get(b, n));
  A.os.put(b, n, x.soma);
  A.od.put(b, n, x.dendrite);
  A.oa.put(b, n, x.adaptation);
  if (A.oj.data) A.oj.put(b, n, j);
}

// Rows of a block that does not fit the LDS path: the whole workgroup reduces
// one row at a time (long rows, or a plan built for another capacity).
template <int BT, int FMT>
__device__ void rows_one_by_one(const TickArgs& A, int r0, int r1, int b0, float gscale,
                                float* red) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  for (int r = r0; r < r1; ++r) {
    const int64_t rs = A.rowptr[r], re = A.rowptr[r + 1];
    float acc[BT];
#pragma unroll
    for (int j = 0; j < BT; ++j) acc[j] = 0.0f;
    for (int64_t e = rs + tid; e < re; e += kThreads) {
      const float w = load_weight<FMT>(A, e, gscale);
      const int64_t c = A.col[e];
#pragma unroll
      for (int j = 0; j < BT; ++j)
        if (b0 + j < A.B) acc[j] += w * A.s.data[(b0 + j) * A.s.sb + c * A.s.sn];
    }
#pragma unroll
    for (int j = 0; j < BT; ++j) {
      float x = acc[j];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
      if (lane == 0) red[wave * BT + j] = x;
    }
    __syncthreads();
    if (tid < BT && b0 + tid < A.B) {
      const float j = ((red[tid] + red[BT + tid]) + red[2 * BT + tid]) + red[3 * BT + tid];
      finish(A, r, b0 + tid, j);
    }
    __syncthreads();
  }
}

template <int BT, int FMT>
__global__ __launch_bounds__(kThreads) void tick_kernel(TickArgs A) {
  constexpr int kPasses = TileCfg<BT>::passes;
  constexpr int kCap = block_capacity<BT>();
  constexpr int kStride = kCap + 4;  // padded [column][edge] rows keep 16-byte alignment
  __shared__ __attribute__((aligned(16))) float prod[BT * kStride];
  __shared__ int32_t srow[kMaxRows + 1];

  const int tid = threadIdx.x;
  const int64_t blk = blockIdx.x;
  const int b0 = blockIdx.y * BT;
  const float gscale = (FMT == NS_WEIGHT_E4M3 || FMT == NS_WEIGHT_NVFP4) ? *A.gscale : 1.0f;

  // The plan's boundary pairs carry each block's first row and first edge, so
  // the edge range needs no rowptr load (clamped into the edge arrays).
  const int32_t* bnd = A.bounds + 2 * blk;
  const int r0 = min(max(bnd[0], 0), static_cast<int>(A.N));
  const int r1 = min(max(bnd[2], r0), static_cast<int>(A.N));
  const int nrows = r1 - r0;
  if (nrows == 0) return;
  const int e0 = static_cast<int>(min<int64_t>(max(bnd[1], 0), A.M));
  const int e1 = static_cast<int>(min<int64_t>(max(bnd[3], e0), A.M));
  const int base = e0 & ~3;
  if (nrows > kMaxRows || e1 - base > kCap) {
    rows_one_by_one<BT, FMT>(A, r0, r1, b0, gscale, prod);
    return;
  }

  // Phase 1 loads first: the block's col/weight quads.
  int cq[kPasses][4];
  float wq[kPasses][4];
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const int q = base + (p * kThreads + tid) * 4;
    if (q < e1) {
      const bool vec = A.quad_loads && (static_cast<int64_t>(q) + 4 <= A.M);
      load_quad<FMT>(A, q, vec, cq[p], wq[p], gscale);
    }
  }

  // Phase 2's geometry depends only on the row count, so each lane's update
  // operands (its row's parameters and its columns' five planes) load now,
  // alongside the quads, and the update at the end waits on nothing.
  int group = kThreads / nrows;                  // lanes per row, power of two, <= 64
  group = 1 << (31 - __builtin_clz(group));
  group = group > 64 ? 64 : group;
  const int cols_at_once = group < BT ? group : BT;
  const int slices = group / cols_at_once;
  const int col_rounds = BT / cols_at_once;
  const int i = tid / group;
  const int lane = tid & (group - 1);
  const int cpos = lane & (cols_at_once - 1);
  const int h = lane / cols_at_once;
  const bool row_ok = i < nrows;
  const bool updates = row_ok && h == 0 && !A.spmm_only;
  const int64_t n = r0 + i;
  NeuronParams prm{};
  float us[BT], ud[BT], ua[BT], uu[BT], uv[BT];
  if (updates) {
    prm = load_params(A.p, n);
#pragma unroll
    for (int round = 0; round < BT; ++round) {
      const int64_t b = b0 + cpos + round * cols_at_once;
      if (round < col_rounds && b < A.B) {
        us[round] = A.s.get(b, n); ud[round] = A.d.get(b, n); ua[round] = A.a.get(b, n);
        uu[round] = A.u.get(b, n); uv[round] = A.v.get(b, n);
      }
    }
  }
  for (int r = tid; r <= nrows; r += kThreads) srow[r] = A.rowptr[r0 + r];

  // Phase 1: decode, gather, multiply, stage in LDS.
  bool paired = false;
  if constexpr (BT == 8 && kPasses == 1) {
    // Eight columns of neuron-major s: an edge's source row is 32 bytes.  The
    // two lanes of a pair take the pair's eight edges together, each loading one
    // 16-byte half of every edge's row, so one load instruction reads 32 rows
    // whole and the L2 sees one request per row rather than up to two (the
    // lanes trade column indices and weights with shuffles).  The products and
    // their LDS places are those of the per-lane path below, so the sums are
    // bitwise the same.  N=50k, M=1M, B=8: 14.8 to 13.7 us per tick.
    if (A.s_vec4 && b0 + 8 <= A.B) {
      paired = true;
      const bool have = base + tid * 4 < e1;
      int c_own[4], c_par[4];
      float w_own[4], w_par[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        c_own[k] = have ? cq[0][k] : 0;
        w_own[k] = have ? wq[0][k] : 0.0f;
        c_par[k] = __shfl_xor(c_own[k], 1, 64);
        w_par[k] = __shfl_xor(w_own[k], 1, 64);
      }
      const int h = tid & 1;                         // the half of the row this lane loads
      const int pair0 = base + (tid & ~1) * 4;       // the pair's first edge
      v4f g[8];
      float w[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        // Edges 0-3 are the even lane's quad, 4-7 the odd lane's.
        const int e = pair0 + i;
        const int c = i < 4 ? (h ? c_par[i] : c_own[i]) : (h ? c_own[i - 4] : c_par[i - 4]);
        w[i] = i < 4 ? (h ? w_par[i] : w_own[i]) : (h ? w_own[i - 4] : w_par[i - 4]);
        g[i] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        if (e >= e0 && e < e1)
          g[i] = *reinterpret_cast<const v4f*>(A.s.data + static_cast<int64_t>(c) * A.s.sn +
                                               (b0 + 4 * h));
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        v4f lo, hi;
        lo.x = w[0] * g[0][t]; lo.y = w[1] * g[1][t]; lo.z = w[2] * g[2][t]; lo.w = w[3] * g[3][t];
        hi.x = w[4] * g[4][t]; hi.y = w[5] * g[5][t]; hi.z = w[6] * g[6][t]; hi.w = w[7] * g[7][t];
        float* const at = prod + (4 * h + t) * kStride + (pair0 - base);
        *reinterpret_cast<v4f*>(at) = lo;
        *reinterpret_cast<v4f*>(at + 4) = hi;
      }
    }
  }
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    if (paired) break;
    const int q = base + (p * kThreads + tid) * 4;
    if (q < e1) {
      float g[4][BT];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int e = q + k;
        const bool valid = e >= e0 && e < e1;
        const int64_t c = cq[p][k];
        if constexpr (BT >= 4) {
          if (A.s_vec4) {
#pragma unroll
            for (int j = 0; j < BT; j += 4) {
              v4f sv = {0.0f, 0.0f, 0.0f, 0.0f};
              if (valid && b0 + j < A.B)
                sv = *reinterpret_cast<const v4f*>(A.s.data + c * A.s.sn + (b0 + j));
              g[k][j] = sv.x; g[k][j + 1] = sv.y; g[k][j + 2] = sv.z; g[k][j + 3] = sv.w;
            }
            continue;
          }
        }
#pragma unroll
        for (int j = 0; j < BT; ++j)
          g[k][j] = (valid && b0 + j < A.B) ? A.s.data[(b0 + j) * A.s.sb + c * A.s.sn] : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < BT; ++j) {
        v4f pv;
        pv.x = wq[p][0] * g[0][j];
        pv.y = wq[p][1] * g[1][j];
        pv.z = wq[p][2] * g[2][j];
        pv.w = wq[p][3] * g[3][j];
        *reinterpret_cast<v4f*>(prod + j * kStride + (q - base)) = pv;
      }
    }
  }
  __syncthreads();

  // Phase 2: per-row reduction from LDS, then the update.
  int rs = 0, re = 0;
  if (row_ok) {
    rs = max(srow[i], e0);
    re = min(srow[i + 1], e1);
  }
#pragma unroll
  for (int round = 0; round < BT; ++round) {
    if (round >= col_rounds) continue;   // (not break: the loop must fully unroll)
    const int j = cpos + round * cols_at_once;
    float acc = 0.0f;
    if (row_ok) {
      // Four running sums over interleaved products, so the LDS reads of a
      // row overlap instead of waiting on one add chain.
      const float* row = prod + j * kStride - base;
      float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
      int e = rs + h;
      for (; e + 3 * slices < re; e += 4 * slices) {
        a0 += row[e];
        a1 += row[e + slices];
        a2 += row[e + 2 * slices];
        a3 += row[e + 3 * slices];
      }
      for (; e < re; e += slices) a0 += row[e];
      acc = (a0 + a1) + (a2 + a3);
    }
    for (int off = cols_at_once; off < group; off <<= 1) acc += __shfl_xor(acc, off, 64);
    if (row_ok && h == 0 && b0 + j < A.B) {
      if (A.spmm_only) {
        const int64_t b = b0 + j;
        A.os.put(b, n, A.spmm_accumulate ? A.os.data[b * A.os.sb + n * A.os.sn] + acc : acc);
      } else {
        const NextState x = advance_loaded(prm, acc, us[round], ud[round], ua[round], uu[round],
                                           uv[round]);
        A.os.put(b0 + j, n, x.soma);
        A.od.put(b0 + j, n, x.dendrite);
        A.oa.put(b0 + j, n, x.adaptation);
        if (A.oj.data) A.oj.put(b0 + j, n, acc);
      }
    }
  }
}

int column_tile(int64_t batch) {
  if (batch <= 1) return 1;
  if (batch <= 2) return 2;
  if (batch <= 4) return 4;
  if (batch <= 8) return 8;
  return 16;
}

int32_t capacity_for(int64_t batch) {
  switch (column_tile(batch)) {
    case 1: return block_capacity<1>();
    case 2: return block_capacity<2>();
    case 4: return block_capacity<4>();
    case 8: return block_capacity<8>();
    default: return block_capacity<16>();
  }
}

template <int BT>
hipError_t launch_tile(const TickArgs& A, int fmt, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(A.n_blocks),
                  static_cast<unsigned>((A.B + BT - 1) / BT));
  const dim3 block(kThreads);
  switch (fmt) {
    case NS_WEIGHT_F32: tick_kernel<BT, NS_WEIGHT_F32><<<grid, block, 0, stream>>>(A); break;
    case NS_WEIGHT_F16: tick_kernel<BT, NS_WEIGHT_F16><<<grid, block, 0, stream>>>(A); break;
    case NS_WEIGHT_E4M3: tick_kernel<BT, NS_WEIGHT_E4M3><<<grid, block, 0, stream>>>(A); break;
    default: tick_kernel<BT, NS_WEIGHT_NVFP4><<<grid, block, 0, stream>>>(A); break;
  }
  return hipGetLastError();
}

hipError_t launch_tick(const TickArgs& A, int fmt, hipStream_t stream) {
  switch (column_tile(A.B)) {
    case 1: return launch_tile<1>(A, fmt, stream);
    case 2: return launch_tile<2>(A, fmt, stream);
    case 4: return launch_tile<4>(A, fmt, stream);
    case 8: return launch_tile<8>(A, fmt, stream);
    default: return launch_tile<16>(A, fmt, stream);
  }
}

int panel_step(const ns_step_args& a, hipStream_t stream, int product, bool launch);

// Host-side validation shared by the tick and the plain product.
int check_csr(const ns_csr& m, int64_t n) {
  if (m.n_rows != n) return fail("CSR row count %lld does not match N=%lld",
                                 (long long)m.n_rows, (long long)n);
  if (m.n_edges < 0 || m.n_edges >= (int64_t{1} << 31))
    return fail("edge count must be in [0, 2^31)");
  if (!m.rowptr) return fail("CSR rowptr is required");
  if (m.n_edges > 0 && (!m.col || !m.weight)) return fail("CSR col and weight are required");
  switch (m.format) {
    case NS_WEIGHT_F32:
    case NS_WEIGHT_F16:
      if (m.block_scales || m.global_scale)
        return fail("floating-point CSR weights take no scales");
      break;
    case NS_WEIGHT_E4M3:
      if (!m.global_scale) return fail("quantized CSR weights require a global scale");
      if (m.block_scales) return fail("fp8 weights take no block scales");
      break;
    case NS_WEIGHT_NVFP4:
      if (!m.global_scale) return fail("quantized CSR weights require a global scale");
      if (m.n_edges > 0 && !m.block_scales) return fail("NVFP4 weights require block scales");
      break;
    default:
      return fail("unknown CSR weight format %d", m.format);
  }
  return NS_OK;
}

int check_matrix(const ns_csr& m, int64_t n, const ns_row_plan& plan, int64_t batch) {
  if (int rc = check_csr(m, n)) return rc;
  if (!plan.bounds || plan.n_blocks < 1) return fail("a row plan is required");
  if (plan.n_blocks > 0x7FFFFFFF) return fail("row plan has too many blocks");
  if (plan.block_edges < 8 || plan.block_edges % 4 || plan.block_edges > capacity_for(batch))
    return fail("row plan was built for %d edges per block, batch %lld takes a multiple of 4 "
                "from 8 to %d", plan.block_edges, (long long)batch, capacity_for(batch));
  return NS_OK;
}

int32_t quad_aligned(const ns_csr& m) {
  const uintptr_t col = reinterpret_cast<uintptr_t>(m.col);
  const uintptr_t w = reinterpret_cast<uintptr_t>(m.weight);
  uintptr_t need = 16;
  switch (m.format) {
    case NS_WEIGHT_F32: need = 16; break;
    case NS_WEIGHT_F16: need = 8; break;
    case NS_WEIGHT_E4M3: need = 4; break;
    default: need = 2; break;
  }
  return (col % 16 == 0) && (w % need == 0);
}

int32_t neuron_major_vec4(const ns_plane& s, int64_t batch) {
  if (column_tile(batch) < 4) return 0;
  // Exactly neuron-major ([N][B] contiguous, B % 4 == 0): every 4-column group
  // starting below B lies inside the neuron's row.
  return s.stride_b == 1 && s.stride_n == batch && batch % 4 == 0 &&
         reinterpret_cast<uintptr_t>(s.data) % 16 == 0;
}

}  // namespace ns

using namespace ns;

extern "C" int32_t ns_block_edges(int64_t batch) { return capacity_for(batch); }

namespace ns {

// Checks shared by every matrix-tick entry: sizes, parameters and the CSR's
// weight encoding (check_step_head), then the planes, which must be present
// and must not overlap where outputs are concerned (check_step_planes).
int check_step_head(const ns_step_args& a) {
  if (a.n_neurons <= 0) return fail("state must be [B,N], N > 0");
  if (a.batch < 0) return fail("batch must be non-negative");
  if (a.n_neurons >= (int64_t{1} << 31)) return fail("N must be below 2^31");
  for (int i = 0; i < 6; ++i)
    if (!a.params[i].data) return fail("six neuron parameter vectors are required");
  return check_csr(a.matrix, a.n_neurons);
}

int check_step_planes(const ns_step_args& a) {
  if (!a.state.data || !a.dendrite.data || !a.adaptation.data)
    return fail("state, dendrite and adaptation data are required");
  if (!a.out_state.data || !a.out_dendrite.data || !a.out_adaptation.data)
    return fail("three output planes are required");
  const Extent outs[4] = {extent(a.out_state, a.batch, a.n_neurons),
                          extent(a.out_dendrite, a.batch, a.n_neurons),
                          extent(a.out_adaptation, a.batch, a.n_neurons),
                          extent(a.out_current, a.batch, a.n_neurons)};
  const Extent ins[5] = {extent(a.state, a.batch, a.n_neurons),
                         extent(a.dendrite, a.batch, a.n_neurons),
                         extent(a.adaptation, a.batch, a.n_neurons),
                         extent(a.drive, a.batch, a.n_neurons),
                         extent(a.dendritic_drive, a.batch, a.n_neurons)};
  for (int o = 0; o < 4; ++o) {
    for (int i = 0; i < 5; ++i)
      if (overlaps(outs[o], ins[i])) return fail("output planes must not overlap inputs");
    for (int p = o + 1; p < 4; ++p)
      if (overlaps(outs[o], outs[p])) return fail("output planes must not overlap each other");
  }
  return NS_OK;
}

}  // namespace ns

extern "C" int ns_dendritic_step(const ns_step_args* args, void* stream) {
  clear_error();
  if (!args) return fail("arguments are required");
  const ns_step_args& a = *args;
  if (int rc = check_step_head(a)) return rc;
  if (!a.panels)
    if (int rc = check_matrix(a.matrix, a.n_neurons, a.plan, a.batch)) return rc;
  if (a.batch == 0) return NS_OK;  // empty planes may carry null pointers
  if (int rc = check_step_planes(a)) return rc;
  if (a.panels) return panel_step(a, static_cast<hipStream_t>(stream), 0, true);

  TickArgs A{};
  A.N = a.n_neurons; A.B = a.batch; A.M = a.matrix.n_edges;
  A.s = plane(a.state, a.state.data); A.d = plane(a.dendrite, a.state.data);
  A.a = plane(a.adaptation, a.state.data);
  A.u = plane(a.drive, a.state.data); A.v = plane(a.dendritic_drive, a.state.data);
  for (int i = 0; i < 6; ++i) A.p.v[i] = Vec{a.params[i].data, a.params[i].stride};
  A.rowptr = a.matrix.rowptr; A.col = a.matrix.col; A.weight = a.matrix.weight;
  A.scales = a.matrix.block_scales; A.gscale = a.matrix.global_scale;
  A.bounds = a.plan.bounds; A.n_blocks = a.plan.n_blocks;
  A.os = out_plane(a.out_state); A.od = out_plane(a.out_dendrite);
  A.oa = out_plane(a.out_adaptation); A.oj = out_plane(a.out_current);
  A.quad_loads = quad_aligned(a.matrix);
  A.s_vec4 = neuron_major_vec4(a.state, a.batch);
  A.spmm_only = 0;
  const hipError_t err = launch_tick(A, a.matrix.format, static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail_launch("dendritic tick", err);
  return NS_OK;
}

extern "C" int ns_csr_spmm(const ns_spmm_args* args, void* stream) {
  clear_error();
  if (!args) return fail("arguments are required");
  const ns_spmm_args& a = *args;
  if (a.n_neurons <= 0) return fail("source must be [B,N], N > 0");
  if (a.batch < 0) return fail("batch must be non-negative");
  if (a.n_neurons >= (int64_t{1} << 31)) return fail("N must be below 2^31");
  if (a.panels) {
    if (int rc = check_csr(a.matrix, a.n_neurons)) return rc;
  } else if (int rc = check_matrix(a.matrix, a.n_neurons, a.plan, a.batch)) {
    return rc;
  }
  if (a.batch == 0) return NS_OK;  // empty planes may carry null pointers
  if (!a.source.data) return fail("source data is required");
  if (!a.out.data) return fail("an output plane is required");
  if (overlaps(extent(a.out, a.batch, a.n_neurons), extent(a.source, a.batch, a.n_neurons)))
    return fail("output plane must not overlap the source");
  if (a.accumulate && !distinct_elements(a.out.stride_b, a.out.stride_n, a.batch, a.n_neurons))
    return fail("an accumulated output plane must not overlap itself (strides %lld, %lld)",
                (long long)a.out.stride_b, (long long)a.out.stride_n);
  if (a.panels) {
    // The panel kernel in product mode: per-panel sums, then the combine
    // kernel adds them in panel order and stores (1) or adds (2) them.
    ns_step_args step{};
    step.n_neurons = a.n_neurons; step.batch = a.batch;
    step.state = a.source; step.matrix = a.matrix; step.panels = a.panels;
    step.out_state = a.out;
    return panel_step(step, static_cast<hipStream_t>(stream), a.accumulate ? 2 : 1, true);
  }

  TickArgs A{};
  A.N = a.n_neurons; A.B = a.batch; A.M = a.matrix.n_edges;
  A.s = plane(a.source, a.source.data);
  A.rowptr = a.matrix.rowptr; A.col = a.matrix.col; A.weight = a.matrix.weight;
  A.scales = a.matrix.block_scales; A.gscale = a.matrix.global_scale;
  A.bounds = a.plan.bounds; A.n_blocks = a.plan.n_blocks;
  A.os = out_plane(a.out);
  A.quad_loads = quad_aligned(a.matrix);
  A.s_vec4 = neuron_major_vec4(a.source, a.batch);
  A.spmm_only = 1;
  A.spmm_accumulate = a.accumulate != 0;
  const hipError_t err = launch_tick(A, a.matrix.format, static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail_launch("CSR product", err);
  return NS_OK;
}
