// Host-side pieces of the C ABI: error storage, version, and the row-block
// planner that cuts a destination-major CSR into the workgroup-sized blocks
// consumed by the tick kernels.
#include <stdint.h>

#include <algorithm>
#include <cstdio>
#include <vector>

#include "ns_host.h"

namespace ns {

char* error_buffer() {
  static thread_local char buffer[512];
  return buffer;
}

}  // namespace ns

using namespace ns;

extern "C" int ns_abi_version(void) { return NS_ABI_VERSION; }

extern "C" const char* ns_last_error(void) { return error_buffer(); }

// Greedy cut: a block starts at row r with aligned base (rowptr[r] & ~3) and
// takes following rows while all their edges stay within base + block_edges
// and the block holds at most kMaxRows rows.  A row that cannot fit even
// alone becomes a one-row block; the kernels reduce such rows with the whole
// workgroup.
extern "C" int ns_plan_row_blocks(const int32_t* rowptr, int64_t n_rows, int32_t block_edges,
                                  int32_t* bounds, int64_t capacity, int64_t* n_blocks) {
  clear_error();
  if (!rowptr || !n_blocks) return fail("rowptr and n_blocks are required");
  if (n_rows <= 0 || n_rows >= (int64_t{1} << 31)) return fail("N must be in [1, 2^31)");
  if (block_edges < 8 || block_edges % 4 != 0) return fail("block_edges must be a multiple of 4");
  if (rowptr[0] != 0) return fail("rowptr[0] must be 0");
  for (int64_t r = 0; r < n_rows; ++r)
    if (rowptr[r + 1] < rowptr[r]) return fail("rowptr must be non-decreasing");

  int64_t count = 0;
  int64_t r = 0;
  auto emit = [&](int64_t row) {
    if (bounds && 2 * count + 1 < capacity) {
      bounds[2 * count] = static_cast<int32_t>(row);
      bounds[2 * count + 1] = rowptr[row];
    }
  };
  while (r < n_rows) {
    emit(r);
    ++count;
    const int64_t start = r;
    const int64_t base = rowptr[r] & ~int64_t{3};
    if (rowptr[r + 1] - base > block_edges) {
      r += 1;  // a long row gets a block of its own
      continue;
    }
    while (r < n_rows && r - start < kMaxRows && rowptr[r + 1] - base <= block_edges) ++r;
  }
  emit(n_rows);
  *n_blocks = count;
  if (bounds && 2 * (count + 1) > capacity)
    return fail("bounds capacity %lld is below the %lld entries required",
                (long long)capacity, (long long)(2 * (count + 1)));
  return NS_OK;
}

namespace {

// The whole panel layout in host vectors (built twice: size query, then fill).
struct PanelLayout {
  int32_t panel_width = 0, n_panels = 0, n_stripes = 0;
  std::vector<int32_t> tiles, chunks, stripes, perm;
  std::vector<uint16_t> row_offsets, col, lane_rows;
};

// Appends the chunks of one (panel, stripe) pair: the stripe's rows in order,
// each with its edges whose source lies in the panel.  A row longer than a
// chunk continues in the next chunk (flags 1/2); the stripe's last chunk gets
// flag 4.  Every chunk is padded with perm = -1 slots to whole lanes.
void append_chunks(PanelLayout& out, const int32_t* rowptr, const int32_t* col,
                   const std::vector<int32_t>& order, const std::vector<int32_t>& bucket,
                   int32_t P, int64_t width, int32_t panel, int32_t stripe, int64_t r0, int64_t r1,
                   int32_t chunk_edges, int32_t pad) {
  int64_t c_edges = 0, c_rows = 0, c_flags = 0, c_first_row = r0, c_slot = 0, c_off = 0;
  auto open_chunk = [&](int64_t first_row, int64_t flags) {
    c_edges = 0; c_rows = 0; c_flags = flags; c_first_row = first_row;
    c_slot = static_cast<int64_t>(out.perm.size());
    c_off = static_cast<int64_t>(out.row_offsets.size());
    out.row_offsets.push_back(0);
  };
  auto close_chunk = [&](bool last_row_continues, bool stripe_done) {
    if (last_row_continues) c_flags |= 2;
    if (stripe_done) c_flags |= 4;
    const int64_t lanes_at = static_cast<int64_t>(out.lane_rows.size());
    const int32_t rec[8] = {static_cast<int32_t>(c_slot), static_cast<int32_t>(c_edges),
                            static_cast<int32_t>(c_first_row), static_cast<int32_t>(c_rows),
                            static_cast<int32_t>(c_off), static_cast<int32_t>(c_flags),
                            static_cast<int32_t>(lanes_at / kPanelThreads), stripe};
    out.chunks.insert(out.chunks.end(), rec, rec + 8);
    // Local row holding each lane's first slot (c_rows past the edges).
    const uint16_t* offs = &out.row_offsets[c_off];
    int64_t row = 0;
    for (int64_t lane = 0; lane < kPanelThreads; ++lane) {
      const int64_t first = lane * pad;
      if (first >= c_edges) {
        out.lane_rows.push_back(static_cast<uint16_t>(c_rows));
        continue;
      }
      while (offs[row + 1] <= first) ++row;
      out.lane_rows.push_back(static_cast<uint16_t>(row));
    }
    while ((static_cast<int64_t>(out.perm.size()) - c_slot) % pad) {   // whole lanes
      out.perm.push_back(-1);
      out.col.push_back(0);
    }
  };
  open_chunk(r0, 0);
  for (int64_t r = r0; r < r1; ++r) {
    const int32_t* b = &bucket[r * (P + 1)];
    int64_t lo = rowptr[r] + b[panel], hi = rowptr[r] + b[panel + 1];
    bool continued = false;
    while (true) {
      if (c_rows == kPanelMaxRows || (c_rows > 0 && c_edges + (hi - lo) > chunk_edges)) {
        close_chunk(false, false);
        open_chunk(r, 0);
      }
      const int64_t take = std::min<int64_t>(hi - lo, chunk_edges - c_edges);
      if (continued && c_rows == 0) c_flags |= 1;
      for (int64_t k = lo; k < lo + take; ++k) {
        const int32_t e = order[k];
        out.perm.push_back(e);
        out.col.push_back(static_cast<uint16_t>(col[e] - panel * width));
      }
      c_edges += take;
      ++c_rows;
      out.row_offsets.push_back(static_cast<uint16_t>(c_edges));
      lo += take;
      if (lo == hi) break;
      close_chunk(true, false);          // the row continues in a fresh chunk
      open_chunk(r, 0);
      continued = true;
    }
  }
  close_chunk(false, true);
}

int build_panels(const int32_t* rowptr, const int32_t* col, int64_t n, int32_t max_width,
                 int32_t want_stripes, int32_t groups_wanted, int32_t chunk_edges, int32_t pad,
                 PanelLayout& out) {
  const int64_t m = rowptr[n];
  max_width &= ~3;                       // panel widths are whole 4-neuron groups
  const int64_t panels = (n + max_width - 1) / max_width;
  int64_t width = (n + panels - 1) / panels;
  width = (width + 3) & ~int64_t{3};
  out.panel_width = static_cast<int32_t>(width);
  out.n_panels = static_cast<int32_t>((n + width - 1) / width);
  const int32_t P = out.n_panels;

  // Stripes: rows split at equal edge counts (equal row counts when M == 0).
  const int64_t stripes_wanted = std::max<int64_t>(1, std::min<int64_t>(want_stripes, n));
  out.stripes.assign(1, 0);
  for (int64_t k = 1; k < stripes_wanted; ++k) {
    int64_t row;
    if (m > 0) {
      const int64_t target = (m * k) / stripes_wanted;
      row = std::lower_bound(rowptr, rowptr + n + 1, static_cast<int32_t>(target)) - rowptr;
    } else {
      row = (n * k) / stripes_wanted;
    }
    if (row > out.stripes.back() && row < n) out.stripes.push_back(static_cast<int32_t>(row));
  }
  out.stripes.push_back(static_cast<int32_t>(n));
  out.n_stripes = static_cast<int32_t>(out.stripes.size() - 1);
  const int32_t S = out.n_stripes;
  const int32_t groups = std::max<int32_t>(1, std::min<int32_t>(groups_wanted, S));

  // Each row's edges grouped by panel (stable counting sort).
  std::vector<int32_t> order(m), bucket((n) * (P + 1), 0), fill(P);
  for (int64_t r = 0; r < n; ++r) {
    int32_t* b = &bucket[r * (P + 1)];
    for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e) {
      const int64_t c = col[e];
      if (c < 0 || c >= n) return fail("CSR column %lld out of range", (long long)c);
      ++b[c / width + 1];
    }
    for (int32_t p = 0; p < P; ++p) b[p + 1] += b[p];
    for (int32_t p = 0; p < P; ++p) fill[p] = b[p];
    for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e)
      order[rowptr[r] + fill[col[e] / width]++] = static_cast<int32_t>(e);
  }

  // Work item (panel p, group g) walks stripes [g*S/groups, (g+1)*S/groups) of panel p.
  for (int32_t p = 0; p < P; ++p) {
    for (int32_t g = 0; g < groups; ++g) {
      const int32_t s0 = static_cast<int32_t>((int64_t{g} * S) / groups);
      const int32_t s1 = static_cast<int32_t>((int64_t{g + 1} * S) / groups);
      const int32_t first_chunk = static_cast<int32_t>(out.chunks.size() / 8);
      for (int32_t st = s0; st < s1; ++st)
        append_chunks(out, rowptr, col, order, bucket, P, width, p, st, out.stripes[st],
                      out.stripes[st + 1], chunk_edges, pad);
      const int32_t tile[4] = {p, first_chunk, static_cast<int32_t>(out.chunks.size() / 8), g};
      out.tiles.insert(out.tiles.end(), tile, tile + 4);
    }
  }
  if (static_cast<int64_t>(out.perm.size()) >= (int64_t{1} << 31))
    return fail("panel layout needs 2^31 or more slots");
  return NS_OK;
}

}  // namespace

extern "C" int ns_plan_panels(const int32_t* rowptr, const int32_t* col, int64_t n_rows,
                              int32_t max_panel_width, int32_t n_stripes, int32_t n_groups,
                              int32_t chunk_edges, int32_t pad, ns_panel_plan* plan,
                              int64_t* n_row_offsets, int32_t* tiles, int32_t* chunks,
                              uint16_t* row_offsets, uint16_t* lane_rows, int32_t* stripes,
                              int32_t* perm, uint16_t* col_out) {
  clear_error();
  if (!rowptr || !plan || !n_row_offsets) return fail("rowptr, plan and n_row_offsets are required");
  if (n_rows <= 0 || n_rows >= (int64_t{1} << 31)) return fail("N must be in [1, 2^31)");
  if (rowptr[0] != 0) return fail("rowptr[0] must be 0");
  for (int64_t r = 0; r < n_rows; ++r)
    if (rowptr[r + 1] < rowptr[r]) return fail("rowptr must be non-decreasing");
  if (rowptr[n_rows] > 0 && !col) return fail("col is required");
  if (max_panel_width < 4 || max_panel_width > 65536)
    return fail("max_panel_width must be in [4, 65536]");
  if (n_stripes < 1 || n_groups < 1) return fail("n_stripes and n_groups must be positive");
  if (pad < 1 || chunk_edges != pad * kPanelThreads || chunk_edges > 65535)
    return fail("chunk_edges must be pad * %d and below 65536", kPanelThreads);
  PanelLayout layout;
  if (int rc = build_panels(rowptr, col, n_rows, max_panel_width, n_stripes, n_groups,
                            chunk_edges, pad, layout))
    return rc;
  plan->panel_width = layout.panel_width;
  plan->n_panels = layout.n_panels;
  plan->n_stripes = layout.n_stripes;
  plan->n_tiles = static_cast<int32_t>(layout.tiles.size() / 4);
  plan->n_chunks = static_cast<int32_t>(layout.chunks.size() / 8);
  plan->chunk_edges = chunk_edges;
  plan->pad = pad;
  plan->n_slots = static_cast<int64_t>(layout.perm.size());
  *n_row_offsets = static_cast<int64_t>(layout.row_offsets.size());
  if (tiles) std::copy(layout.tiles.begin(), layout.tiles.end(), tiles);
  if (chunks) std::copy(layout.chunks.begin(), layout.chunks.end(), chunks);
  if (row_offsets) std::copy(layout.row_offsets.begin(), layout.row_offsets.end(), row_offsets);
  if (lane_rows) std::copy(layout.lane_rows.begin(), layout.lane_rows.end(), lane_rows);
  if (stripes) std::copy(layout.stripes.begin(), layout.stripes.end(), stripes);
  if (perm) std::copy(layout.perm.begin(), layout.perm.end(), perm);
  if (col_out) std::copy(layout.col.begin(), layout.col.end(), col_out);
  return NS_OK;
}
