// Device builder of the coalesced graph and both CSR views (gfx950), bitwise
// equal to the reference's SparseTopology.from_edges on the CPU
// (topology.py:32-115):
//
//  * canonical edges: candidates stably sorted by src*N + dst; equal keys are
//    one edge whose weight is the sum, from zero, of the candidates' weights
//    in their input order (zeros(...).index_add(0, inverse, sorted_weight));
//  * out_rowptr over canonical src; the destination-major view in_rowptr /
//    in_col / in_weight in (dst, src) order; out_weight_index mapping each
//    canonical edge to its destination-major position.
//
// The sorts are stable LSD radix sorts (hipCUB) over just the key bits N*N
// needs; each run of equal keys is summed in order by one lane, so the sums
// are deterministic, unlike an atomic index_add.  The unique-edge count stays
// on the device: every launch after the first sort covers all candidate
// slots and reads the count itself, so nothing waits for the host.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <algorithm>

#include "ns_common.h"
#include "ns_host.h"

namespace ns {
namespace {

constexpr int kTopoThreads = 256;

inline unsigned grid_for(int64_t items) {
  return static_cast<unsigned>(std::max<int64_t>(1, (items + kTopoThreads - 1) / kTopoThreads));
}

__global__ void candidate_keys_kernel(const int64_t* src, const int64_t* dst, int64_t n,
                                      int64_t m, int64_t* keys) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kTopoThreads + threadIdx.x;
  if (i < m) keys[i] = src[i] * n + dst[i];
}

// flags[i] = 1 where a run of equal sorted keys starts.
__global__ void run_starts_kernel(const int64_t* keys, int64_t m, int32_t* flags) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kTopoThreads + threadIdx.x;
  if (i < m) flags[i] = (i == 0 || keys[i] != keys[i - 1]) ? 1 : 0;
}

// rank[i] = number of run starts in [0, i]; run u starts at position starts[u].
__global__ void run_offsets_kernel(const int32_t* flags, const int32_t* rank, int64_t m,
                                   int32_t* starts, int64_t* n_unique) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kTopoThreads + threadIdx.x;
  if (i < m && flags[i]) starts[rank[i] - 1] = static_cast<int32_t>(i);
  if (i == m - 1) {
    starts[rank[i]] = static_cast<int32_t>(m);
    *n_unique = rank[i];
  }
  if (m == 0 && i == 0) {
    starts[0] = 0;
    *n_unique = 0;
  }
}

// One lane per canonical edge: its (src, dst), its summed weight, and the key
// of its destination-major position.  Slots past the count get the largest
// key the sort sees, `pad`; that may equal a real key (n a power of two), but
// the stable sort keeps every real edge, whose slot is lower, ahead of them.
__global__ void canonical_edges_kernel(const int64_t* keys, const float* weights,
                                       const int32_t* starts, const int64_t* n_unique,
                                       int64_t n, int64_t capacity, int64_t pad, int32_t* out_src,
                                       int32_t* out_dst, float* out_weight, int64_t* in_keys,
                                       int32_t* in_values) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * kTopoThreads + threadIdx.x;
  if (u >= capacity) return;
  in_values[u] = static_cast<int32_t>(u);
  if (u >= *n_unique) {
    in_keys[u] = pad;
    return;
  }
  const int32_t first = starts[u], end = starts[u + 1];
  float sum = 0.0f;
  for (int32_t j = first; j < end; ++j) sum += weights[j];
  const int64_t key = keys[first];
  const int64_t s = key / n, d = key - s * n;
  out_src[u] = static_cast<int32_t>(s);
  out_dst[u] = static_cast<int32_t>(d);
  out_weight[u] = sum;
  in_keys[u] = d * n + s;
}

// Destination-major view from the (dst, src)-sorted keys and canonical ids.
__global__ void in_view_kernel(const int64_t* in_keys, const int32_t* in_order,
                               const float* canonical_weight, const int64_t* n_unique,
                               int64_t n, int64_t capacity, int32_t* in_col, float* in_weight,
                               int32_t* out_weight_index) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kTopoThreads + threadIdx.x;
  if (i >= capacity || i >= *n_unique) return;
  const int64_t key = in_keys[i];
  const int32_t u = in_order[i];
  in_col[i] = static_cast<int32_t>(key - (key / n) * n);
  in_weight[i] = canonical_weight[u];
  out_weight_index[u] = static_cast<int32_t>(i);
}

// rowptr[r] = number of edges whose row (key / n) is below r, over sorted keys.
__global__ void row_pointer_kernel(const int64_t* sorted_keys, const int32_t* rows32,
                                   const int64_t* n_unique, int64_t n, int32_t* rowptr) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kTopoThreads + threadIdx.x;
  if (r > n) return;
  int64_t lo = 0, hi = *n_unique;
  while (lo < hi) {
    const int64_t mid = (lo + hi) / 2;
    const int64_t row = rows32 ? rows32[mid] : sorted_keys[mid] / n;
    if (row < r) lo = mid + 1;
    else hi = mid;
  }
  rowptr[r] = static_cast<int32_t>(lo);
}

int key_bits(int64_t n) {
  const uint64_t top = static_cast<uint64_t>(n) * static_cast<uint64_t>(n);   // keys < n*n
  int bits = 1;
  while (bits < 63 && (uint64_t{1} << bits) < top) ++bits;
  return bits;
}

// Workspace carve-up (all offsets 256-byte aligned).
struct Layout {
  size_t keys, sorted_keys, sorted_weights, flags, rank, starts, in_keys, in_keys_sorted,
      in_values, in_order, temp, temp_bytes, total;
};

int layout(int64_t n, int64_t m, Layout* L) {
  auto up = [](size_t x) { return (x + 255) & ~size_t{255}; };
  const size_t cap = static_cast<size_t>(std::max<int64_t>(m, 1));
  size_t at = 0;
  auto take = [&](size_t bytes) { const size_t here = at; at += up(bytes); return here; };
  L->keys = take(8 * cap);
  L->sorted_keys = take(8 * cap);
  L->sorted_weights = take(4 * cap);
  L->flags = take(4 * cap);
  L->rank = take(4 * cap);
  L->starts = take(4 * (cap + 1));
  L->in_keys = take(8 * cap);
  L->in_keys_sorted = take(8 * cap);
  L->in_values = take(4 * cap);
  L->in_order = take(4 * cap);
  const int bits = key_bits(n);
  size_t sort1 = 0, sort2 = 0, scan = 0;
  if (hipcub::DeviceRadixSort::SortPairs(nullptr, sort1, static_cast<const int64_t*>(nullptr),
                                         static_cast<int64_t*>(nullptr),
                                         static_cast<const float*>(nullptr),
                                         static_cast<float*>(nullptr), static_cast<int>(cap), 0,
                                         bits) != hipSuccess ||
      hipcub::DeviceRadixSort::SortPairs(nullptr, sort2, static_cast<const int64_t*>(nullptr),
                                         static_cast<int64_t*>(nullptr),
                                         static_cast<const int32_t*>(nullptr),
                                         static_cast<int32_t*>(nullptr), static_cast<int>(cap), 0,
                                         bits) != hipSuccess ||
      hipcub::DeviceScan::InclusiveSum(nullptr, scan, static_cast<const int32_t*>(nullptr),
                                       static_cast<int32_t*>(nullptr), static_cast<int>(cap)) !=
          hipSuccess)
    return fail("temporary storage query failed");
  L->temp_bytes = std::max({sort1, sort2, scan});
  L->temp = take(L->temp_bytes);
  L->total = at;
  return NS_OK;
}

}  // namespace
}  // namespace ns

using namespace ns;

extern "C" int64_t ns_topology_workspace_bytes(int64_t n_neurons, int64_t n_candidates) {
  clear_error();
  if (n_neurons < 1 || n_neurons > (int64_t{1} << 31) || n_candidates < 0 ||
      n_candidates >= (int64_t{1} << 31)) {
    fail("N must be in [1, 2^31] and the candidate count in [0, 2^31)");
    return -1;
  }
  Layout L{};
  if (layout(n_neurons, n_candidates, &L) != NS_OK) return -1;
  return static_cast<int64_t>(L.total);
}

extern "C" int ns_build_topology(const ns_topology_args* args, void* stream) {
  clear_error();
  if (!args) return fail("arguments are required");
  const ns_topology_args& a = *args;
  const int64_t n = a.n_neurons, m = a.n_candidates;
  if (n < 1 || n > (int64_t{1} << 31)) return fail("N must be in [1, 2^31]");
  if (m < 0 || m >= (int64_t{1} << 31))
    return fail("this compact topology supports fewer than 2^31 edges");
  if (m > 0 && (!a.src || !a.dst || !a.weight)) return fail("src, dst and weight are required");
  if (!a.out_rowptr || !a.in_rowptr || !a.n_edges || !a.workspace)
    return fail("out_rowptr, in_rowptr, n_edges and workspace are required");
  if (m > 0 && (!a.out_src || !a.out_dst || !a.out_weight || !a.in_col || !a.in_weight ||
                !a.out_weight_index))
    return fail("every edge output is required");
  Layout L{};
  if (int rc = layout(n, m, &L)) return rc;
  if (a.workspace_bytes < static_cast<int64_t>(L.total))
    return fail("workspace of %lld bytes is below the %lld required",
                (long long)a.workspace_bytes, (long long)L.total);
  if (reinterpret_cast<uintptr_t>(a.workspace) % 256) return fail("workspace must be 256-byte aligned");
  char* ws = static_cast<char*>(a.workspace);
  int64_t* keys = reinterpret_cast<int64_t*>(ws + L.keys);
  int64_t* sorted_keys = reinterpret_cast<int64_t*>(ws + L.sorted_keys);
  float* sorted_weights = reinterpret_cast<float*>(ws + L.sorted_weights);
  int32_t* flags = reinterpret_cast<int32_t*>(ws + L.flags);
  int32_t* rank = reinterpret_cast<int32_t*>(ws + L.rank);
  int32_t* starts = reinterpret_cast<int32_t*>(ws + L.starts);
  int64_t* in_keys = reinterpret_cast<int64_t*>(ws + L.in_keys);
  int64_t* in_keys_sorted = reinterpret_cast<int64_t*>(ws + L.in_keys_sorted);
  int32_t* in_values = reinterpret_cast<int32_t*>(ws + L.in_values);
  int32_t* in_order = reinterpret_cast<int32_t*>(ws + L.in_order);
  void* temp = ws + L.temp;
  size_t temp_bytes = L.temp_bytes;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int items = static_cast<int>(m);
  const int bits = key_bits(n);

  if (m > 0) {
    candidate_keys_kernel<<<grid_for(m), kTopoThreads, 0, s>>>(a.src, a.dst, n, m, keys);
    if (hipcub::DeviceRadixSort::SortPairs(temp, temp_bytes, keys, sorted_keys, a.weight,
                                           sorted_weights, items, 0, bits, s) != hipSuccess)
      return fail("candidate sort failed");
    run_starts_kernel<<<grid_for(m), kTopoThreads, 0, s>>>(sorted_keys, m, flags);
    temp_bytes = L.temp_bytes;
    if (hipcub::DeviceScan::InclusiveSum(temp, temp_bytes, flags, rank, items, s) != hipSuccess)
      return fail("run scan failed");
  }
  run_offsets_kernel<<<grid_for(std::max<int64_t>(m, 1)), kTopoThreads, 0, s>>>(
      flags, rank, m, starts, a.n_edges);
  if (m > 0) {
    canonical_edges_kernel<<<grid_for(m), kTopoThreads, 0, s>>>(
        sorted_keys, sorted_weights, starts, a.n_edges, n, m, (int64_t{1} << bits) - 1, a.out_src,
        a.out_dst, a.out_weight, in_keys, in_values);
    temp_bytes = L.temp_bytes;
    if (hipcub::DeviceRadixSort::SortPairs(temp, temp_bytes, in_keys, in_keys_sorted, in_values,
                                           in_order, items, 0, bits, s) != hipSuccess)
      return fail("destination-major sort failed");
    in_view_kernel<<<grid_for(m), kTopoThreads, 0, s>>>(in_keys_sorted, in_order, a.out_weight,
                                                        a.n_edges, n, m, a.in_col, a.in_weight,
                                                        a.out_weight_index);
  }
  row_pointer_kernel<<<grid_for(n + 1), kTopoThreads, 0, s>>>(nullptr, m > 0 ? a.out_src : nullptr,
                                                              a.n_edges, n, a.out_rowptr);
  row_pointer_kernel<<<grid_for(n + 1), kTopoThreads, 0, s>>>(in_keys_sorted, nullptr, a.n_edges,
                                                              n, a.in_rowptr);
  if (hipGetLastError() != hipSuccess) return fail("topology launch failed");
  return NS_OK;
}
