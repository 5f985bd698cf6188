// PELS event tick for gfx950: (1) three-state advance driven by the
// persistent current plus the emission threshold, (2) scatter of every
// emitter's out-edges into the persistent current with float32 atomics.
//
// Semantics: the reference's dendritic_event (csrc/compartmental.cu:142-173)
// and DendriticPELSRuntime.step with HybridPELSRuntime._emit
// (compartmental.py:322-348, runtime.py:225-253): residual = s' - emitted,
// active = |residual| >= theta, delta = active ? residual : 0,
// emitted' = emitted + delta, current += W @ delta.  Entries with a zero
// delta push nothing (compartmental.cu:168).
//
// Work decomposition (this library's own): kernel 1 walks (neuron, column)
// pairs in neuron-major order, one lane each.  Kernel 2 gives each wavefront
// 64 consecutive pairs and spreads their emitters' source-major out-edges
// over its lanes (see scatter_chunk).  Inactive stretches cost a few
// coalesced loads and a prefix sum.
//
// One-launch tick (pending buffers given): the scatter cannot add into the
// current that other wavefronts of the same launch still have to read, so it
// adds into a zeroed pending buffer instead, and the next tick folds that
// buffer into the current as it reads it (j = current + pending).  A
// wavefront advances its 64 pairs and scatters their deltas straight from
// registers; the launch boundary orders one tick's scatter before the next
// tick's reads.  Two buffers alternate, so the buffer a tick scatters into is
// never the one it reads and zeroes.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "ns_common.h"
#include "ns_host.h"

namespace ns {

struct EventArgs {
  int64_t N, B, count;
  Plane s, d, a, u, v, emitted;
  Params p;
  float* current;
  int64_t csb, csn;
  Vec theta;
  OutPlane os, od, oa, oe;
  float* delta;
  const int32_t* out_rowptr;
  const int32_t* dst;
  const int32_t* weight_index;
  const float* weight;
  const float* out_weight;
  float* pending_in;
  float* pending_out;
  unsigned long long* activity;
  int32_t column_log2;  // log2 B when B is a power of two in [2, 64], else 0
};

// Everything pair (n, b) reads besides its current.
struct PairInputs {
  NeuronParams p;
  float s, d, a, u, v, emitted, theta;
};

__device__ __forceinline__ PairInputs load_pair(const EventArgs& A, int64_t n, int64_t b) {
  return PairInputs{load_params(A.p, n), A.s.get(b, n), A.d.get(b, n), A.a.get(b, n),
                    A.u.get(b, n),       A.v.get(b, n), A.emitted.get(b, n), A.theta.get(n)};
}

// Advances pair (n, b) on current j, stores the three states and the
// emitted state, and returns the pair's delta; `active` tells whether the
// residual reached the threshold (the reference's emission mask, which at
// theta = 0 includes pairs whose residual is zero).
__device__ __forceinline__ float advance_loaded_pair(const EventArgs& A, int64_t n, int64_t b,
                                                     float j, const PairInputs& in,
                                                     bool& active) {
  const NextState x = advance_loaded(in.p, j, in.s, in.d, in.a, in.u, in.v);
  float dl;
  {
#pragma clang fp contract(off)
    const float residual = x.soma - in.emitted;
    active = fabsf(residual) >= in.theta;
    dl = active ? residual : 0.0f;
    A.oe.put(b, n, in.emitted + dl);
  }
  A.os.put(b, n, x.soma);
  A.od.put(b, n, x.dendrite);
  A.oa.put(b, n, x.adaptation);
  return dl;
}

__device__ __forceinline__ float advance_pair(const EventArgs& A, int64_t n, int64_t b,
                                              float j) {
  bool active;
  return advance_loaded_pair(A, n, b, j, load_pair(A, n, b), active);
}

__global__ __launch_bounds__(kThreads) void event_advance_kernel(EventArgs A) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < A.count;
       i += stride) {
    const int64_t n = i / A.B;
    const int64_t b = i - n * A.B;
    A.delta[i] = advance_pair(A, n, b, A.current[b * A.csb + n * A.csn]);
  }
}

// Edges per lane per round of the scatter, loaded before any is added.
constexpr int kScatterUnroll = 2;

// Adds W[:, n] * delta for the emitters among one wavefront's 64 pairs into
// target[b*tb + dst*tn].  Pair chunk*64 + lane holds `mine` and its neuron's
// source-major out-edge range [start, end).  The emitters' out-edges are
// numbered wave-wide by an inclusive prefix sum over their degrees; lane l
// takes edges l, l + 64, ... and finds each one's emitter by a binary search
// over the prefix sums.  Every lane has work whatever the degrees, and an
// edge's loads (target index, weight) do not wait on each other.
__device__ __forceinline__ void scatter_chunk(const EventArgs& A, int64_t chunk, int lane,
                                              float mine, int64_t start, int64_t end,
                                              float* target, int64_t tb, int64_t tn) {
  const int64_t count = mine != 0.0f ? end - start : 0;
  // A wavefront without an emitting out-edge has nothing to scatter.
  if (__ballot(count != 0) == 0) return;
  int64_t incl = count;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int64_t up = __shfl_up(incl, d, 64);
    if (lane >= d) incl += up;
  }
  const int64_t first = incl - count;  // number of this pair's first edge
  const int64_t total = __shfl(incl, 63, 64);
  const int64_t pair = chunk * 64 + lane;
  const int column = static_cast<int>(pair - (pair / A.B) * A.B);
  for (int64_t base = 0; base < total; base += 64 * kScatterUnroll) {
    int64_t edge[kScatterUnroll];
    float scale[kScatterUnroll];
    int col[kScatterUnroll];
    bool live[kScatterUnroll];
#pragma unroll
    for (int r = 0; r < kScatterUnroll; ++r) {
      const int64_t k = base + r * 64 + lane;
      // owner: the lowest lane whose inclusive sum exceeds k (all lanes search)
      int o = 0;
#pragma unroll
      for (int step = 32; step > 0; step >>= 1)
        if (__shfl(incl, o + step - 1, 64) <= k) o += step;
      // Every lane takes part in each shuffle: a lane left out of one supplies
      // zero to the lanes that read from it.
      const int64_t owner_start = __shfl(start, o, 64);
      const int64_t owner_first = __shfl(first, o, 64);
      scale[r] = __shfl(mine, o, 64);
      col[r] = __shfl(column, o, 64);
      live[r] = k < total;
      // a lane past the last edge reads edge 0 (total > 0, so it exists) and adds nothing
      edge[r] = live[r] ? owner_start + (k - owner_first) : 0;
    }
    int32_t to[kScatterUnroll];
    float w[kScatterUnroll];
#pragma unroll
    for (int r = 0; r < kScatterUnroll; ++r) {
      to[r] = A.dst[edge[r]];
      w[r] = A.out_weight ? A.out_weight[edge[r]] : A.weight[A.weight_index[edge[r]]];
    }
#pragma unroll
    for (int r = 0; r < kScatterUnroll; ++r)
      if (live[r])
        unsafeAtomicAdd(target + col[r] * tb + static_cast<int64_t>(to[r]) * tn,
                        scale[r] * w[r]);
  }
}

// The same scatter with each source's B columns taken together, for B = 2^lg
// from 2 to 64 (a wavefront's 64 pairs are then 64/B whole sources, columns in
// lane order).  Work item k of a source with `na` emitting columns is its
// out-edge k / na in its (k mod na)-th emitting column, so neighbouring lanes
// add into neighbouring columns of one destination: in a neuron-major target
// one 4B-byte run, which the memory-side atomic units serve as one request
// (random float32 atomics: 21 G/s; eight lanes per 32-byte run: 151 G/s).
// Items are numbered per source by an inclusive prefix sum held by the
// source's first lane; lane l takes items l, l + 64, ...
__device__ __forceinline__ void scatter_chunk_columns(const EventArgs& A, int lane, float mine,
                                                      int64_t start, int64_t end, float* target,
                                                      int64_t tb, int64_t tn, int lg) {
  const unsigned long long act = __ballot(mine != 0.0f);
  if (act == 0) return;
  const int B = 1 << lg;
  const int g0 = lane & ~(B - 1);  // this lane's source's first lane
  const unsigned long long all = lg == 6 ? ~0ull : (1ull << B) - 1;
  const unsigned long long mask = (act >> g0) & all;  // its emitting columns
  const int64_t work = lane == g0 ? (end - start) * __popcll(mask) : 0;
  int64_t incl = work;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int64_t up = __shfl_up(incl, d, 64);
    if (lane >= d) incl += up;
  }
  const int64_t first = incl - work;
  const int64_t total = __shfl(incl, 63, 64);
  for (int64_t base = 0; base < total; base += 64 * kScatterUnroll) {
    int64_t edge[kScatterUnroll];
    float scale[kScatterUnroll];
    int col[kScatterUnroll];
    bool live[kScatterUnroll];
#pragma unroll
    for (int r = 0; r < kScatterUnroll; ++r) {
      const int64_t k = base + r * 64 + lane;
      // owner: the lowest lane whose inclusive sum exceeds k, the first lane of
      // a source with work (every lane takes part in each shuffle)
      int o = 0;
#pragma unroll
      for (int step = 32; step > 0; step >>= 1)
        if (__shfl(incl, o + step - 1, 64) <= k) o += step;
      const int64_t owner_start = __shfl(start, o, 64);
      const int64_t owner_first = __shfl(first, o, 64);
      const unsigned long long owner_mask = __shfl(mask, o, 64);
      live[r] = k < total;
      int64_t e = 0;
      int c = 0;
      if (live[r]) {
        const int64_t local = k - owner_first;
        const int na = __popcll(owner_mask);     // at least 1: the owner has work
        if (na == B) {
          e = local >> lg;
          c = static_cast<int>(local & (B - 1));
        } else {
          int64_t rank;
          if (local < (int64_t{1} << 32)) {
            const uint32_t u = static_cast<uint32_t>(local);
            const uint32_t q = u / static_cast<uint32_t>(na);
            e = q;
            rank = u - q * static_cast<uint32_t>(na);
          } else {
            e = local / na;
            rank = local - e * na;
          }
          unsigned long long bits = owner_mask;
          for (int64_t t = 0; t < rank; ++t) bits &= bits - 1;  // drop the lowest `rank` columns
          c = __builtin_ctzll(bits);
        }
      }
      // o + c stays in the owner's B lanes (a lane past the end reads lane o, unused)
      scale[r] = __shfl(mine, o + c, 64);
      col[r] = c;
      edge[r] = live[r] ? owner_start + e : 0;
    }
    int32_t to[kScatterUnroll];
    float w[kScatterUnroll];
#pragma unroll
    for (int r = 0; r < kScatterUnroll; ++r) {
      to[r] = A.dst[edge[r]];
      w[r] = A.out_weight ? A.out_weight[edge[r]] : A.weight[A.weight_index[edge[r]]];
    }
#pragma unroll
    for (int r = 0; r < kScatterUnroll; ++r)
      if (live[r])
        unsafeAtomicAdd(target + col[r] * tb + static_cast<int64_t>(to[r]) * tn,
                        scale[r] * w[r]);
  }
}

// The wavefront's scatter in the form its batch width allows.
__device__ __forceinline__ void scatter_wave(const EventArgs& A, int64_t chunk, int lane,
                                             float mine, int64_t start, int64_t end,
                                             float* target, int64_t tb, int64_t tn) {
  if (A.column_log2 > 0)
    scatter_chunk_columns(A, lane, mine, start, end, target, tb, tn, A.column_log2);
  else
    scatter_chunk(A, chunk, lane, mine, start, end, target, tb, tn);
}

__global__ __launch_bounds__(kThreads) void event_scatter_kernel(EventArgs A) {
  const int lane = threadIdx.x & 63;
  const int64_t chunk = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) >> 6;
  const int64_t i = chunk * 64 + lane;
  float mine = 0.0f;
  int64_t start = 0, end = 0;
  if (i < A.count) {
    const int64_t n = i / A.B;
    mine = A.delta[i];
    start = A.out_rowptr[n];
    end = A.out_rowptr[n + 1];
  }
  scatter_wave(A, chunk, lane, mine, start, end, A.current, A.csb, A.csn);
}

// Adds the out-degrees of a workgroup's active pairs (`edges` per lane) to
// one of NS_EVENT_ACTIVITY_SLOTS counters, NS_EVENT_ACTIVITY_STRIDE apart
// (workgroup w uses slot w mod the slot count): a wavefront sum by
// shuffles, then one atomic per workgroup, so that few workgroups meet on one
// address.  Every lane of the workgroup must call it.
__device__ __forceinline__ void count_activity(const EventArgs& A, int64_t edges) {
  __shared__ unsigned long long wave_sum[kThreads / 64];
  unsigned long long v = static_cast<unsigned long long>(edges);
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
  if ((threadIdx.x & 63) == 0) wave_sum[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long total = 0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) total += wave_sum[w];
    if (total)
      __hip_atomic_fetch_add(A.activity + (blockIdx.x % NS_EVENT_ACTIVITY_SLOTS) *
                                              NS_EVENT_ACTIVITY_STRIDE,
                             total, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The one-launch tick: one lane per pair, one wavefront per 64 pairs.  It
// reads j = current + pending_in and folds it into the current.  kScatter:
// the wavefront scatters its deltas into pending_out; else (the fused
// advance-only tick) the deltas go to `delta` for the caller to propagate.
// kCount: the out-degrees of the active pairs are added to `activity`.
template <bool kScatter, bool kCount>
__global__ __launch_bounds__(kThreads) void event_tick_kernel(EventArgs A) {
  const int lane = threadIdx.x & 63;
  const int64_t chunk = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) >> 6;
  const int64_t i = chunk * 64 + lane;
  float dl = 0.0f;
  bool active = false;
  int64_t start = 0, end = 0;
  if (i < A.count) {
    const int64_t n = i / A.B;
    const int64_t b = i - n * A.B;
    // Every load of the pair is issued before its first store, so the pair
    // waits on memory once.
    start = A.out_rowptr[n];
    end = A.out_rowptr[n + 1];
    float* at = A.current + b * A.csb + n * A.csn;
    const float current = *at, pending = A.pending_in[i];
    const PairInputs in = load_pair(A, n, b);
    const float j = current + pending;
    *at = j;
    A.pending_in[i] = 0.0f;
    dl = advance_loaded_pair(A, n, b, j, in, active);
    if constexpr (!kScatter) A.delta[i] = dl;
  }
  if constexpr (kCount) count_activity(A, active ? end - start : 0);
  if constexpr (kScatter) scatter_wave(A, chunk, lane, dl, start, end, A.pending_out, 1, A.B);
}

}  // namespace ns

using namespace ns;

extern "C" int ns_dendritic_event(const ns_event_args* args, void* stream) {
  clear_error();
  if (!args) return fail("arguments are required");
  const ns_event_args& a = *args;
  if (a.n_neurons <= 0) return fail("state must be [B,N], N > 0");
  if (a.batch < 0) return fail("batch must be non-negative");
  if (a.n_neurons >= (int64_t{1} << 31)) return fail("N must be below 2^31");
  for (int i = 0; i < 6; ++i)
    if (!a.params[i].data) return fail("six neuron parameter vectors are required");
  if (!a.theta.data) return fail("theta must have N values");
  if (a.n_edges < 0 || a.n_edges >= (int64_t{1} << 31))
    return fail("edge count must be in [0, 2^31)");
  if (!a.out_rowptr) return fail("out_rowptr is required");
  if (a.n_edges > 0 && (!a.dst || !a.weight_index || !a.weight))
    return fail("dst, weight_index and weight are required");
  if (a.batch == 0) return NS_OK;  // empty planes may carry null pointers
  if (!a.state.data || !a.dendrite.data || !a.adaptation.data || !a.emitted.data)
    return fail("state, dendrite, adaptation and emitted data are required");
  if (!a.current) return fail("persistent current is required");
  {
    // The current is updated in place, one element per (b, n): no two pairs
    // may share an element (a zero stride, or strides that interleave).
    if (!distinct_elements(a.current_stride_b, a.current_stride_n, a.batch, a.n_neurons))
      return fail("the persistent current must not overlap itself (strides %lld, %lld)",
                  (long long)a.current_stride_b, (long long)a.current_stride_n);
  }
  if (!a.out_state.data || !a.out_dendrite.data || !a.out_adaptation.data ||
      !a.out_emitted.data)
    return fail("four output planes are required");
  if (a.flags & ~NS_EVENT_ADVANCE_ONLY) return fail("unknown event flags %d", a.flags);
  const bool advance_only = (a.flags & NS_EVENT_ADVANCE_ONLY) != 0;
  // The one-launch forms read j = current + pending_in; the scattering one
  // also needs pending_out, the advance-only one writes `delta` instead.
  const bool fused = a.pending_in != nullptr;
  if (advance_only) {
    if (a.pending_out) return fail("the advance-only tick scatters nothing: pending_out must be NULL");
    if (!a.delta) return fail("a delta workspace is required");
  } else {
    if (fused != (a.pending_out != nullptr)) return fail("pending_in and pending_out go together");
    if (!fused && !a.delta) return fail("a delta workspace is required");
  }
  if (a.activity && !fused)
    return fail("activity counts need the one-launch tick (pending_in)");
  const int64_t B = a.batch, N = a.n_neurons;
  // Written memory: the four planes, then the workspaces (pending buffers and
  // delta, entry n*B + b) and the activity counters.
  Extent outs[8] = {extent(a.out_state, B, N), extent(a.out_dendrite, B, N),
                    extent(a.out_adaptation, B, N), extent(a.out_emitted, B, N)};
  int n_outs = 4;
  if (a.pending_in) outs[n_outs++] = extent_of(a.pending_in, 1, B, B, N);
  if (a.pending_out) outs[n_outs++] = extent_of(a.pending_out, 1, B, B, N);
  if (a.delta && (advance_only || !fused)) outs[n_outs++] = extent_of(a.delta, N, 1, B, N);
  if (a.activity)
    outs[n_outs++] = extent_of(a.activity, 0, 1, 1,
                               2 * NS_EVENT_ACTIVITY_SLOTS * NS_EVENT_ACTIVITY_STRIDE);
  const Extent ins[8] = {extent(a.state, B, N), extent(a.dendrite, B, N),
                         extent(a.adaptation, B, N), extent(a.drive, B, N),
                         extent(a.dendritic_drive, B, N), extent(a.emitted, B, N),
                         extent_of(a.current, a.current_stride_b, a.current_stride_n, B, N),
                         extent_of(a.out_weight, 0, 1, 1, a.n_edges)};
  for (int o = 0; o < n_outs; ++o) {
    for (int i = 0; i < 8; ++i)
      if (overlaps(outs[o], ins[i]))
        return fail(o < 4 ? "output planes must not overlap inputs"
                          : "event workspaces must not overlap inputs or the current");
    for (int p = o + 1; p < n_outs; ++p)
      if (overlaps(outs[o], outs[p]))
        return fail(p < 4 ? "output planes must not overlap each other"
                          : "event workspaces must not overlap outputs or each other");
  }
  if ((B * N + kThreads - 1) / kThreads > 0x7FFFFFFF)
    return fail("B*N is too large for one scatter launch");

  EventArgs A{};
  A.N = N; A.B = B; A.count = B * N;
  A.s = plane(a.state, a.state.data); A.d = plane(a.dendrite, a.state.data);
  A.a = plane(a.adaptation, a.state.data);
  A.u = plane(a.drive, a.state.data); A.v = plane(a.dendritic_drive, a.state.data);
  A.emitted = plane(a.emitted, a.state.data);
  for (int i = 0; i < 6; ++i) A.p.v[i] = Vec{a.params[i].data, a.params[i].stride};
  A.current = a.current; A.csb = a.current_stride_b; A.csn = a.current_stride_n;
  A.theta = Vec{a.theta.data, a.theta.stride};
  A.os = out_plane(a.out_state); A.od = out_plane(a.out_dendrite);
  A.oa = out_plane(a.out_adaptation); A.oe = out_plane(a.out_emitted);
  A.delta = a.delta;
  A.out_rowptr = a.out_rowptr; A.dst = a.dst; A.weight_index = a.weight_index;
  A.weight = a.weight;
  A.out_weight = a.out_weight;
  A.pending_in = a.pending_in; A.pending_out = a.pending_out;
  A.activity = reinterpret_cast<unsigned long long*>(a.activity);
  // Column-grouped scatter for B = 2, 4, ..., 64 (a wavefront then holds whole sources).
  A.column_log2 = 0;
  for (int lg = 1; lg <= 6; ++lg)
    if (B == (int64_t{1} << lg)) A.column_log2 = lg;

  hipStream_t s = static_cast<hipStream_t>(stream);
  if (fused) {
    const dim3 grid(static_cast<unsigned>((A.count + kThreads - 1) / kThreads));
    if (advance_only) {
      if (A.activity) event_tick_kernel<false, true><<<grid, dim3(kThreads), 0, s>>>(A);
      else event_tick_kernel<false, false><<<grid, dim3(kThreads), 0, s>>>(A);
    } else {
      if (A.activity) event_tick_kernel<true, true><<<grid, dim3(kThreads), 0, s>>>(A);
      else event_tick_kernel<true, false><<<grid, dim3(kThreads), 0, s>>>(A);
    }
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? NS_OK : fail_launch("event tick", err);
  }
  const int64_t advance_blocks = std::min<int64_t>((A.count + kThreads - 1) / kThreads, 65536);
  event_advance_kernel<<<dim3(static_cast<unsigned>(advance_blocks)), dim3(kThreads), 0, s>>>(A);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail_launch("event advance", err);
  if (advance_only) return NS_OK;
  const int64_t scatter_blocks = (A.count + kThreads - 1) / kThreads;
  event_scatter_kernel<<<dim3(static_cast<unsigned>(scatter_blocks)), dim3(kThreads), 0, s>>>(A);
  err = hipGetLastError();
  if (err != hipSuccess) return fail_launch("event scatter", err);
  return NS_OK;
}
