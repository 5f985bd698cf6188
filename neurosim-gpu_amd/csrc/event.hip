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
// 64 consecutive pairs: a ballot over their deltas finds the emitters, and
// four 16-lane groups walk four emitters' source-major out-edge lists at a
// time.  Inactive stretches cost one coalesced load and one ballot.
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
};

constexpr int kScatterGroup = 16;  // lanes walking one emitter's out-edges

__global__ __launch_bounds__(kThreads) void event_advance_kernel(EventArgs A) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < A.count;
       i += stride) {
    const int64_t n = i / A.B;
    const int64_t b = i - n * A.B;
    const float j = A.current[b * A.csb + n * A.csn];
    const NextState x = advance_one(A.p, n, j, A.s.get(b, n), A.d.get(b, n), A.a.get(b, n),
                                    A.u.get(b, n), A.v.get(b, n));
    const float previous = A.emitted.get(b, n);
    float dl;
    {
#pragma clang fp contract(off)
      const float residual = x.soma - previous;
      const bool active = fabsf(residual) >= A.theta.get(n);
      dl = active ? residual : 0.0f;
      A.oe.put(b, n, previous + dl);
    }
    A.os.put(b, n, x.soma);
    A.od.put(b, n, x.dendrite);
    A.oa.put(b, n, x.adaptation);
    A.delta[i] = dl;
  }
}

__global__ __launch_bounds__(kThreads) void event_scatter_kernel(EventArgs A) {
  const int lane = threadIdx.x & 63;
  const int64_t chunk = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) >> 6;
  const int64_t i = chunk * 64 + lane;
  const float mine = i < A.count ? A.delta[i] : 0.0f;
  uint64_t pending = __ballot(mine != 0.0f);
  const int group = lane / kScatterGroup;
  const int glane = lane & (kScatterGroup - 1);
  while (pending) {
    // The g-th lowest pending bit goes to group g (the same sequence on every lane).
    int pick = -1;
#pragma unroll
    for (int g = 0; g < 64 / kScatterGroup; ++g) {
      const int bit = pending ? __builtin_ctzll(pending) : -1;
      if (bit >= 0) pending &= pending - 1;
      if (g == group) pick = bit;
    }
    const float dl = __shfl(mine, pick < 0 ? 0 : pick, 64);
    if (pick >= 0) {
      const int64_t entry = chunk * 64 + pick;
      const int64_t n = entry / A.B;
      const int64_t b = entry - n * A.B;
      const int64_t start = A.out_rowptr[n], end = A.out_rowptr[n + 1];
      float* target = A.current + b * A.csb;
      for (int64_t e = start + glane; e < end; e += kScatterGroup)
        unsafeAtomicAdd(target + static_cast<int64_t>(A.dst[e]) * A.csn,
                        dl * A.weight[A.weight_index[e]]);
    }
  }
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
  if (!a.out_state.data || !a.out_dendrite.data || !a.out_adaptation.data ||
      !a.out_emitted.data)
    return fail("four output planes are required");
  if (!a.delta) return fail("a delta workspace is required");
  const int64_t B = a.batch, N = a.n_neurons;
  const Extent outs[5] = {extent(a.out_state, B, N), extent(a.out_dendrite, B, N),
                          extent(a.out_adaptation, B, N), extent(a.out_emitted, B, N),
                          extent_of(a.delta, N, 1, B, N)};
  const Extent ins[7] = {extent(a.state, B, N), extent(a.dendrite, B, N),
                         extent(a.adaptation, B, N), extent(a.drive, B, N),
                         extent(a.dendritic_drive, B, N), extent(a.emitted, B, N),
                         extent_of(a.current, a.current_stride_b, a.current_stride_n, B, N)};
  for (int o = 0; o < 5; ++o) {
    for (int i = 0; i < 7; ++i)
      if (overlaps(outs[o], ins[i])) return fail("output planes must not overlap inputs");
    for (int p = o + 1; p < 5; ++p)
      if (overlaps(outs[o], outs[p])) return fail("output planes must not overlap each other");
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

  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t advance_blocks = std::min<int64_t>((A.count + kThreads - 1) / kThreads, 65536);
  event_advance_kernel<<<dim3(static_cast<unsigned>(advance_blocks)), dim3(kThreads), 0, s>>>(A);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail_launch("event advance", err);
  const int64_t scatter_blocks = (A.count + kThreads - 1) / kThreads;
  event_scatter_kernel<<<dim3(static_cast<unsigned>(scatter_blocks)), dim3(kThreads), 0, s>>>(A);
  err = hipGetLastError();
  if (err != hipSuccess) return fail_launch("event scatter", err);
  return NS_OK;
}
