// Float32 backward of the fused matrix tick (gfx950).
//
// The tick computes, per (column b, neuron n), with j = (W @ s)[b, n]:
//   d' = rho_d*d + (1-rho_d)*tanh(j + v)
//   u_ = ((1-c)*j + c*d') - k*a
//   s' = clamp(alpha*s + (1-alpha)*(gain*tanh(u_ + drive)), 0, 1)
//   a' = rho_a*a + (1-rho_a)*s'
// This file propagates upstream gradients of (s', d', a') to the states, the
// drives, the six parameters and the CSR weights, as autograd does through
// the reference's torch path (compartmental.py:152-183 and the CSR product of
// runtime.py:78-79, whose weight and source gradients compartmental.py:40-56
// spells out: a sampled product over the stored entries, and the transposed
// product through out_weight_index).  clamp passes the gradient where its
// input lies in [0, 1], ends included, and tanh's derivative is 1 - y^2 of its
// output, as in torch.
//
// Launches: j = W @ s again (the row-block product, as in ns_csr_spmm), the
// elementwise backward (one lane per neuron, columns in order, so the
// parameter sums are deterministic), the transposed product added into the
// state gradient (one wavefront per source neuron over its out-edges) and the
// weight gradient (one wavefront per destination row; each edge sums its
// columns in order).  No atomics: every result has a single writer.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "ns_common.h"
#include "ns_host.h"

namespace ns {
namespace {

constexpr int kGradThreads = 256;
constexpr int kGradChunk = 8;   // columns per pass of the wavefront kernels
constexpr int kGradUnroll = 4;  // edges per lane per round of the edge loops

struct GradArgs {
  int64_t N, B;
  Plane s, d, a, u, v;
  Params p;
  const float* j;        // [N][B]: j[n*B + b]
  Plane gs_up, gd_up, ga_up;
  OutPlane gs, gd, ga, gu, gv;
  float* gj;             // [N][B]
  float* gp[6];
};

__global__ __launch_bounds__(kGradThreads) void advance_backward_kernel(GradArgs A) {
#pragma clang fp contract(off)
  const int64_t n = static_cast<int64_t>(blockIdx.x) * kGradThreads + threadIdx.x;
  if (n >= A.N) return;
  const NeuronParams P = load_params(A.p, n);
  float g_alpha = 0.0f, g_gain = 0.0f, g_rho_d = 0.0f, g_rho_a = 0.0f, g_c = 0.0f, g_k = 0.0f;
  for (int64_t b = 0; b < A.B; ++b) {
    const float j = A.j[n * A.B + b];
    const float s = A.s.get(b, n), d = A.d.get(b, n), a = A.a.get(b, n);
    const float u = A.u.get(b, n), v = A.v.get(b, n);
    // Forward, rounded as the tick rounds it.
    const float t1 = tanhf(j + v);
    const float dn = P.rho_d * d + (1.0f - P.rho_d) * t1;
    const float m = (1.0f - P.coupling) * j + P.coupling * dn;
    const float cur = m - P.strength * a;
    const float t2 = tanhf(cur + u);
    const float eq = P.gain * t2;
    const float pre = P.alpha * s + (1.0f - P.alpha) * eq;
    const float sn = clamp01(pre);
    // Backward.
    const float gS = A.gs_up.get(b, n), gD = A.gd_up.get(b, n), gA = A.ga_up.get(b, n);
    g_rho_a += gA * (a - sn);
    const float g_sn = gS + (1.0f - P.rho_a) * gA;
    const float g_pre = (pre >= 0.0f && pre <= 1.0f) ? g_sn : 0.0f;
    g_alpha += g_pre * (s - eq);
    const float g_eq = (1.0f - P.alpha) * g_pre;
    g_gain += g_eq * t2;
    const float g_x2 = (g_eq * P.gain) * (1.0f - t2 * t2);
    g_k += -(a * g_x2);
    g_c += g_x2 * (dn - j);
    const float g_dn = gD + P.coupling * g_x2;
    g_rho_d += g_dn * (d - t1);
    const float g_x1 = ((1.0f - P.rho_d) * g_dn) * (1.0f - t1 * t1);
    A.gs.put(b, n, P.alpha * g_pre);
    A.gd.put(b, n, P.rho_d * g_dn);
    A.ga.put(b, n, P.rho_a * gA - P.strength * g_x2);
    if (A.gu.data) A.gu.put(b, n, g_x2);
    if (A.gv.data) A.gv.put(b, n, g_x1);
    A.gj[n * A.B + b] = (1.0f - P.coupling) * g_x2 + g_x1;
  }
  const float sums[6] = {g_alpha, g_gain, g_rho_d, g_rho_a, g_c, g_k};
#pragma unroll
  for (int i = 0; i < 6; ++i)
    if (A.gp[i]) A.gp[i][n] = sums[i];
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// gs[b, c] += sum over out-edges e of source c of w[owi[e]] * gj[dst[e], b].
__global__ __launch_bounds__(kGradThreads) void transposed_product_kernel(
    const int32_t* out_rowptr, const int32_t* dst, const int32_t* owi, const float* w,
    const float* w_out, const float* gj, int64_t N, int64_t B, OutPlane gs) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * (kGradThreads / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (c >= N) return;
  const int32_t e0 = out_rowptr[c], e1 = out_rowptr[c + 1];
  for (int64_t b0 = 0; b0 < B; b0 += kGradChunk) {
    float acc[kGradChunk];
#pragma unroll
    for (int q = 0; q < kGradChunk; ++q) acc[q] = 0.0f;
    // kGradUnroll edges per lane per round, every load of a round issued before
    // the first multiply (an edge past the row's end rereads the row's last edge
    // and adds nothing), so a round waits on memory once.
    for (int32_t e = e0 + lane; e < e1; e += 64 * kGradUnroll) {
      float weight[kGradUnroll];
      int64_t t[kGradUnroll];
#pragma unroll
      for (int u = 0; u < kGradUnroll; ++u) {
        const int32_t at = min(e + 64 * u, e1 - 1);
        // Source-major weights stream; otherwise each one is a gather into the CSR order.
        weight[u] = w_out ? w_out[at] : w[owi[at]];
        t[u] = dst[at];
      }
#pragma unroll
      for (int u = 0; u < kGradUnroll; ++u) {
        if (e + 64 * u >= e1) break;
#pragma unroll
        for (int q = 0; q < kGradChunk; ++q)
          if (b0 + q < B) acc[q] = __builtin_fmaf(weight[u], gj[t[u] * B + b0 + q], acc[q]);
      }
    }
#pragma unroll
    for (int q = 0; q < kGradChunk; ++q) {
      const float total = wave_sum(acc[q]);
      if (lane == 0 && b0 + q < B) {
        float* at = gs.data + (b0 + q) * gs.sb + c * gs.sn;
        *at = *at + total;
      }
    }
  }
}

// gw[e] = sum over columns b (in order) of gj[row, b] * s[b, col[e]], for the
// edges e of each destination row.
__global__ __launch_bounds__(kGradThreads) void weight_gradient_kernel(
    const int32_t* rowptr, const int32_t* col, const float* gj, Plane s, int64_t N, int64_t B,
    float* gw) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * (kGradThreads / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= N) return;
  const int32_t e0 = rowptr[r], e1 = rowptr[r + 1];
  // kGradUnroll edges per lane per round: the round's column indices load
  // together, then their state gathers, then the stores.
  for (int32_t e = e0 + lane; e < e1; e += 64 * kGradUnroll) {
    int64_t c[kGradUnroll];
#pragma unroll
    for (int u = 0; u < kGradUnroll; ++u) c[u] = col[min(e + 64 * u, e1 - 1)];
    float sum[kGradUnroll];
#pragma unroll
    for (int u = 0; u < kGradUnroll; ++u) sum[u] = 0.0f;
    for (int64_t b = 0; b < B; ++b) {
      const float g = gj[r * B + b];
#pragma unroll
      for (int u = 0; u < kGradUnroll; ++u) sum[u] = __builtin_fmaf(g, s.get(b, c[u]), sum[u]);
    }
#pragma unroll
    for (int u = 0; u < kGradUnroll; ++u)
      if (e + 64 * u < e1) gw[e + 64 * u] = sum[u];
  }
}

}  // namespace
}  // namespace ns

namespace ns {
int panel_step(const ns_step_args& a, hipStream_t stream, int product, bool launch);
}  // namespace ns

using namespace ns;

extern "C" int64_t ns_step_backward_workspace_floats(int64_t n_neurons, int64_t batch) {
  return 2 * std::max<int64_t>(n_neurons, 0) * std::max<int64_t>(batch, 0);
}

extern "C" int ns_dendritic_step_backward(const ns_step_grad_args* args, void* stream) {
  clear_error();
  if (!args) return fail("arguments are required");
  const ns_step_grad_args& a = *args;
  const int64_t n = a.n_neurons, batch = a.batch;
  if (n <= 0 || n >= (int64_t{1} << 31)) return fail("N must be in [1, 2^31)");
  if (batch < 0) return fail("batch must be non-negative");
  if (a.matrix.format != NS_WEIGHT_F32) return fail("the backward needs float32 weights");
  for (int i = 0; i < 6; ++i)
    if (!a.params[i].data) return fail("six neuron parameter vectors are required");
  if (batch == 0) return NS_OK;
  if (!a.state.data || !a.dendrite.data || !a.adaptation.data)
    return fail("state, dendrite and adaptation data are required");
  if (!a.d_state.data || !a.d_dendrite.data || !a.d_adaptation.data)
    return fail("the three state gradient planes are required");
  if (!a.out_rowptr || !a.dst || !a.out_weight_index)
    return fail("the source-major view (out_rowptr, dst, out_weight_index) is required");
  if (!a.workspace) return fail("a workspace of 2*B*N floats is required");
  if (a.transposed_panels && batch > 2) return fail("transposed panels need batch 1 or 2");
  const Extent outs[5] = {extent(a.d_state, batch, n), extent(a.d_dendrite, batch, n),
                          extent(a.d_adaptation, batch, n), extent(a.d_drive, batch, n),
                          extent(a.d_dendritic_drive, batch, n)};
  const Extent ins[9] = {extent(a.state, batch, n), extent(a.dendrite, batch, n),
                         extent(a.adaptation, batch, n), extent(a.drive, batch, n),
                         extent(a.dendritic_drive, batch, n), extent(a.grad_state, batch, n),
                         extent(a.grad_dendrite, batch, n), extent(a.grad_adaptation, batch, n),
                         extent_of(a.current, 1, 1, 1, batch * n)};
  const Extent work = extent_of(a.workspace, 1, 1, 1, 2 * batch * n);
  if (overlaps(ins[8], work)) return fail("the forward's current must not overlap the workspace");
  for (int o = 0; o < 5; ++o) {
    if (overlaps(outs[o], work)) return fail("gradient planes must not overlap the workspace");
    for (int i = 0; i < 9; ++i)
      if (overlaps(outs[o], ins[i])) return fail("gradient planes must not overlap inputs");
    for (int p = o + 1; p < 5; ++p)
      if (overlaps(outs[o], outs[p])) return fail("gradient planes must not overlap each other");
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  float* gj = a.workspace + batch * n;

  // j = W @ s, neuron-major: the forward's, or recomputed into the workspace.
  const float* j = a.current;
  if (!j) {
    ns_spmm_args prod{};
    prod.n_neurons = n; prod.batch = batch; prod.source = a.state; prod.matrix = a.matrix;
    prod.plan = a.plan; prod.out = ns_out_plane{a.workspace, 1, batch};
    if (int rc = ns_csr_spmm(&prod, stream)) return rc;
    j = a.workspace;
  }

  GradArgs G{};
  G.N = n; G.B = batch;
  G.s = plane(a.state, a.state.data); G.d = plane(a.dendrite, a.state.data);
  G.a = plane(a.adaptation, a.state.data);
  G.u = plane(a.drive, a.state.data); G.v = plane(a.dendritic_drive, a.state.data);
  for (int i = 0; i < 6; ++i) G.p.v[i] = Vec{a.params[i].data, a.params[i].stride};
  G.j = j;
  G.gs_up = plane(a.grad_state, a.state.data);
  G.gd_up = plane(a.grad_dendrite, a.state.data);
  G.ga_up = plane(a.grad_adaptation, a.state.data);
  G.gs = out_plane(a.d_state); G.gd = out_plane(a.d_dendrite); G.ga = out_plane(a.d_adaptation);
  G.gu = out_plane(a.d_drive); G.gv = out_plane(a.d_dendritic_drive);
  G.gj = gj;
  for (int i = 0; i < 6; ++i) G.gp[i] = a.d_params[i];
  // The transposed product on panels: W^T @ gj added into d_state.
  ns_step_args transposed{};
  if (a.transposed_panels && a.matrix.n_edges > 0) {
    transposed.n_neurons = n; transposed.batch = batch;
    transposed.state = ns_plane{gj, 1, batch, 0.0f};
    transposed.matrix.n_rows = n; transposed.matrix.n_edges = a.matrix.n_edges;
    transposed.matrix.format = NS_WEIGHT_F32;
    // An indexed plan (NS_PANEL_INDEXED) reads each slot's weight from the CSR
    // weights through the slot's edge number.
    transposed.matrix.weight = a.matrix.weight;
    transposed.panels = a.transposed_panels;
    transposed.out_state = a.d_state;
    if (int rc = panel_step(transposed, s, 2, false)) return rc;
    const ns_panel_plan& tp = *a.transposed_panels;
    const Extent part = extent_of(tp.partials, 1, 1, 1, 2 * int64_t{tp.n_panels} * n * batch);
    if (overlaps(part, work)) return fail("the transposed panels' partials overlap the workspace");
    for (int o = 0; o < 5; ++o)
      if (overlaps(part, outs[o]))
        return fail("the transposed panels' partials overlap a gradient plane");
  }
  const unsigned per_neuron = static_cast<unsigned>((n + kGradThreads - 1) / kGradThreads);
  const unsigned per_row = static_cast<unsigned>((n + kGradThreads / 64 - 1) / (kGradThreads / 64));
  advance_backward_kernel<<<per_neuron, kGradThreads, 0, s>>>(G);
  if (a.matrix.n_edges > 0) {
    if (a.transposed_panels) {
      // d_state += W^T @ gj on the transposed matrix's panel layout (checked
      // before the first launch).
      if (const hipError_t e = hipGetLastError(); e != hipSuccess)
        return fail_launch("tick backward", e);
      if (int rc = panel_step(transposed, s, 2, true)) return rc;
    } else {
      transposed_product_kernel<<<per_row, kGradThreads, 0, s>>>(
          a.out_rowptr, a.dst, a.out_weight_index, static_cast<const float*>(a.matrix.weight),
          a.out_weight, gj, n, batch, out_plane(a.d_state));
    }
    if (a.d_weight)
      weight_gradient_kernel<<<per_row, kGradThreads, 0, s>>>(
          a.matrix.rowptr, a.matrix.col, gj, plane(a.state, a.state.data), n, batch, a.d_weight);
  }
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail_launch("tick backward", err);
  return NS_OK;
}
