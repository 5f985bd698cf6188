// Host-side pieces of the C ABI: error storage, version, and the row-block
// planner that cuts a destination-major CSR into the workgroup-sized blocks
// consumed by the tick kernels.
#include <stdint.h>

#include <algorithm>
#include <atomic>
#include <functional>
#include <map>
#include <system_error>
#include <thread>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "ns_error.h"
#include "ns_limits.h"

static_assert(ns::kBandWaves == NS_BAND_WAVES, "band wavefronts match the ABI");

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

// Host threads a planner may use (the hosts this runs on give a process
// about 16 cores).
constexpr unsigned kPlanThreads = 16;

// Rows per work item of the planners' row-parallel passes.
constexpr int64_t kPlanRowChunk = 4096;

// Host threads the planners use: min(kPlanThreads, hardware threads), or the
// positive value of NEUROSIM_PLAN_THREADS (capped at kPlanThreads).  Layouts do
// not depend on it; the variable exists so that a one-thread build of a plan
// can be compared with a threaded one.
int64_t plan_threads() {
  const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
  int64_t n = std::min<int64_t>(kPlanThreads, hw);
  if (const char* env = std::getenv("NEUROSIM_PLAN_THREADS")) {
    const long v = std::strtol(env, nullptr, 10);
    if (v > 0) n = std::min<int64_t>(kPlanThreads, v);
  }
  return n;
}

// Runs `work` on min(plan_threads(), items) threads, this one included;
// `work` takes its items from a shared counter.  Without threads (creation
// fails) it runs on this thread alone.
template <typename Work>
void run_on_threads(Work& work, int64_t items) {
  const int64_t n = std::min<int64_t>(plan_threads(), std::max<int64_t>(items, 1));
  std::vector<std::thread> pool;
  try {
    for (int64_t t = 1; t < n; ++t) pool.emplace_back(std::ref(work));
  } catch (const std::system_error&) {
  }
  work();
  for (std::thread& t : pool) t.join();
}

// The sliced layout of one graph, in host vectors (built twice: size query, then fill).
struct PanelLayout {
  int32_t panel_width = 0, n_panels = 0, n_ranges = 0;
  std::vector<int32_t> tiles, tile_ranges, wave_groups, groups, perm;
  std::vector<uint16_t> rows, col;
  std::vector<uint32_t> last_steps;   // bit k: step k (slots 64k..64k+63) ends a group
};

int32_t log2_lanes(int64_t len, int32_t lane_target, int32_t min_lg) {
  // Lanes per row: the smallest power of two (at least 2^min_lg) that leaves
  // each lane at most lane_target items, capped at a whole wavefront.
  int32_t lg = min_lg;
  while (lg < 6 && len > (int64_t{lane_target} << lg)) ++lg;
  return lg;
}

struct Group {
  int32_t lg, nrows, steps, first;   // first: index of its first row in the sorted order
};

// A row's items in one panel: its edges there, in the order lanes take them,
// plus (for pair layouts) padding items (-1).  Row r's items for panel p are
// items[base[r] + bucket[r*(P+1)+p] .. base[r] + bucket[r*(P+1)+p+1]).
struct Items {
  std::vector<int32_t> items, bucket;
  std::vector<int64_t> base;
};

// Lays out tile (panel p, rows [r0, r1)): rows sorted by segment length
// (descending, ties by row), cut into groups of 64 >> lg rows sharing one
// lanes-per-row width, groups dealt longest first onto the least-loaded of the
// tile's wavefronts, then every wavefront's groups emitted back to back.
void append_tile(PanelLayout& out, const int32_t* col, const Items& it, int32_t P, int64_t width,
                 int32_t p, int64_t r0, int64_t r1, int32_t waves, int32_t lane_target,
                 int32_t min_lg) {
  const int64_t nr = r1 - r0;
  const std::vector<int32_t>& bucket = it.bucket;
  auto seg_len = [&](int64_t r) -> int64_t {
    const int32_t* b = bucket.data() + r * (P + 1);
    return b[p + 1] - b[p];
  };
  std::vector<int32_t> sorted(nr);
  for (int64_t i = 0; i < nr; ++i) sorted[i] = static_cast<int32_t>(r0 + i);
  std::stable_sort(sorted.begin(), sorted.end(),
                   [&](int32_t x, int32_t y) { return seg_len(x) > seg_len(y); });
  std::vector<Group> groups;
  for (int64_t i = 0; i < nr;) {
    const int64_t len = seg_len(sorted[i]);
    const int32_t lg = log2_lanes(len, lane_target, min_lg);
    const int64_t cap = 64 >> lg;
    int64_t n = 1;
    while (n < cap && i + n < nr && log2_lanes(seg_len(sorted[i + n]), lane_target, min_lg) == lg)
      ++n;
    const int64_t lanes = int64_t{1} << lg;
    // Every group takes at least one step (rows with no edges read one padding
    // step), so each group ends on a step the boundary bitmap can mark.
    const int64_t steps = std::max<int64_t>(1, (len + lanes - 1) / lanes);
    groups.push_back(Group{lg, static_cast<int32_t>(n), static_cast<int32_t>(steps),
                           static_cast<int32_t>(i)});
    i += n;
  }
  // Longest-processing-time assignment (steps + 1 per group for its reduction).
  std::vector<int32_t> by_cost(groups.size());
  for (size_t g = 0; g < groups.size(); ++g) by_cost[g] = static_cast<int32_t>(g);
  std::stable_sort(by_cost.begin(), by_cost.end(),
                   [&](int32_t x, int32_t y) { return groups[x].steps > groups[y].steps; });
  std::vector<int64_t> load(waves, 0);
  std::vector<std::vector<int32_t>> mine(waves);
  for (int32_t g : by_cost) {
    const int32_t w = static_cast<int32_t>(std::min_element(load.begin(), load.end()) - load.begin());
    load[w] += groups[g].steps + 1;
    mine[w].push_back(g);
  }
  const int32_t rec[4] = {p, static_cast<int32_t>(r0), static_cast<int32_t>(r1),
                          static_cast<int32_t>(out.rows.size())};
  out.tiles.insert(out.tiles.end(), rec, rec + 4);
  for (int32_t w = 0; w < waves; ++w) {
    out.wave_groups.push_back(static_cast<int32_t>(out.groups.size() / 4));
    for (int32_t g : mine[w]) {
      const Group& grp = groups[g];
      const int32_t lanes = 1 << grp.lg;
      const int32_t rec_g[4] = {static_cast<int32_t>(out.perm.size()), grp.steps,
                                grp.lg | (grp.nrows << 8), static_cast<int32_t>(out.rows.size())};
      out.groups.insert(out.groups.end(), rec_g, rec_g + 4);
      const int64_t last = static_cast<int64_t>(out.perm.size()) / 64 + grp.steps - 1;
      if (static_cast<int64_t>(out.last_steps.size()) <= last / 32)
        out.last_steps.resize(last / 32 + 1, 0u);
      out.last_steps[last / 32] |= 1u << (last % 32);
      for (int32_t k = 0; k < grp.nrows; ++k)
        out.rows.push_back(static_cast<uint16_t>(sorted[grp.first + k] - r0));
      // Step-major slots: lane l = (row k, part j) takes the row's edges j, j+lanes, ...
      for (int32_t step = 0; step < grp.steps; ++step) {
        for (int32_t lane = 0; lane < 64; ++lane) {
          const int32_t k = lane >> grp.lg, j = lane & (lanes - 1);
          int32_t edge = -1;
          if (k < grp.nrows) {
            const int64_t r = sorted[grp.first + k];
            const int64_t idx = int64_t{step} * lanes + j;
            if (idx < seg_len(r)) edge = it.items[it.base[r] + bucket[r * (P + 1) + p] + idx];
          }
          out.perm.push_back(edge);
          out.col.push_back(edge < 0 ? static_cast<uint16_t>(width)
                                     : static_cast<uint16_t>(col[edge] - p * width));
        }
      }
    }
  }
}

int build_panels(const int32_t* rowptr, const int32_t* col, int64_t n, int32_t max_width,
                 int32_t tiles_per_panel, int32_t waves, int32_t lane_target, bool pairs,
                 PanelLayout& out) {
  const int64_t m = rowptr[n];
  max_width &= ~3;                       // panel widths are whole 4-neuron groups
  const int64_t panels = (n + max_width - 1) / max_width;
  int64_t width = (n + panels - 1) / panels;
  width = (width + 3) & ~int64_t{3};
  out.panel_width = static_cast<int32_t>(width);
  out.n_panels = static_cast<int32_t>((n + width - 1) / width);
  const int32_t P = out.n_panels;

  // Rows are independent below: chunks of kPlanRowChunk rows go to up to
  // kPlanThreads threads, and each row writes only its own ranges.
  // Each row's edges grouped by panel (stable counting sort).
  // Columns are checked first, on all rows: the passes below index by them.
  // The first offending edge (lowest index) is reported, whatever the threads.
  const int64_t n_chunks = (n + kPlanRowChunk - 1) / kPlanRowChunk;
  auto for_rows = [&](auto&& body) {
    std::atomic<int64_t> next_chunk{0};
    auto work = [&] {
      for (int64_t q = next_chunk.fetch_add(1); q < n_chunks; q = next_chunk.fetch_add(1))
        for (int64_t r = q * kPlanRowChunk; r < std::min(n, (q + 1) * kPlanRowChunk); ++r) body(r);
    };
    run_on_threads(work, n_chunks);
  };
  constexpr int64_t kNoEdge = INT64_MAX;
  std::atomic<int64_t> bad_edge{kNoEdge};
  for_rows([&](int64_t r) {
    for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e)
      if (col[e] < 0 || col[e] >= n) {
        int64_t seen = bad_edge.load();
        while (e < seen && !bad_edge.compare_exchange_weak(seen, e)) {
        }
        return;
      }
  });
  if (const int64_t e = bad_edge.load(); e != kNoEdge)
    return fail("CSR column %lld out of range (edge %lld)", (long long)col[e], (long long)e);

  std::vector<int32_t> order(m), bucket(n * (P + 1), 0);
  for_rows([&](int64_t r) {
    int32_t* b = bucket.data() + r * (P + 1);
    for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e) ++b[col[e] / width + 1];
    for (int32_t p = 0; p < P; ++p) b[p + 1] += b[p];
    std::vector<int32_t> fill(b, b + P);
    for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e)
      order[rowptr[r] + fill[col[e] / width]++] = static_cast<int32_t>(e);
  });

  // Items.  Plain layouts: the edges as grouped above.  Pair layouts: within
  // each (row, panel) segment the edges grouped by 16-edge weight block (stable,
  // so a column-sorted CSR keeps its order) and each block's run padded to an
  // even length, so items 2i and 2i+1 share a block.  Every row gets at least
  // two lanes, so lanes 2q and 2q+1 of a step hold items 2i and 2i+1 of one row.
  Items it;
  it.base.resize(n + 1);
  if (!pairs) {
    it.items = std::move(order);
    it.bucket = std::move(bucket);
    for (int64_t r = 0; r <= n; ++r) it.base[r] = rowptr[r];
  } else {
    // Per row: its segments regrouped by weight block into `regrouped` (in
    // place of `order`) with the padded length of each segment in it.bucket;
    // then the rows' item ranges by a prefix sum, and the items written.
    it.bucket.assign(n * (P + 1), 0);
    std::vector<int32_t> regrouped(m);
    for_rows([&](int64_t r) {
      const int32_t* b = bucket.data() + r * (P + 1);
      int32_t* ib = it.bucket.data() + r * (P + 1);
      int32_t* seg = regrouped.data() + rowptr[r];
      std::copy(order.begin() + rowptr[r], order.begin() + rowptr[r + 1], seg);
      int32_t padded = 0;
      for (int32_t p = 0; p < P; ++p) {
        std::stable_sort(seg + b[p], seg + b[p + 1],
                         [](int32_t x, int32_t y) { return (x >> 4) < (y >> 4); });
        for (int32_t i = b[p]; i < b[p + 1];) {
          int32_t j = i;
          while (j < b[p + 1] && (seg[j] >> 4) == (seg[i] >> 4)) ++j;
          padded += (j - i) + ((j - i) % 2);
          i = j;
        }
        ib[p + 1] = padded;
      }
    });
    it.base[0] = 0;
    for (int64_t r = 0; r < n; ++r) it.base[r + 1] = it.base[r] + it.bucket[r * (P + 1) + P];
    it.items.assign(static_cast<size_t>(it.base[n]), -1);
    for_rows([&](int64_t r) {
      const int32_t* b = bucket.data() + r * (P + 1);
      const int32_t* seg = regrouped.data() + rowptr[r];
      int32_t* out_items = it.items.data() + it.base[r];
      int32_t k = 0;
      for (int32_t p = 0; p < P; ++p)
        for (int32_t i = b[p]; i < b[p + 1];) {
          int32_t j = i;
          while (j < b[p + 1] && (seg[j] >> 4) == (seg[i] >> 4)) out_items[k++] = seg[j++];
          if ((j - i) % 2) out_items[k++] = -1;
          i = j;
        }
    });
  }
  const int32_t min_lg = pairs ? 1 : 0;

  // Row ranges shared by every panel: consecutive rows of about equal cost
  // over all panels (items + 1 per row and panel), at most 65536 rows each
  // (16-bit tile-local rows).  Panel p's tile of range k covers the range's
  // rows, so the tiles of one range together cover its rows in every panel.
  const int64_t min_ranges = (n + 65535) / 65536;
  const int64_t T = std::min<int64_t>(n, std::max<int64_t>(tiles_per_panel, min_ranges));
  std::vector<int64_t> cost(n + 1, 0);
  for (int64_t r = 0; r < n; ++r) cost[r + 1] = cost[r] + (it.base[r + 1] - it.base[r]) + P;
  std::vector<int64_t> range_rows{0};
  for (int64_t t = 1; range_rows.back() < n; ++t) {
    const int64_t r0 = range_rows.back();
    int64_t r1 = n;
    if (t < T) r1 = std::lower_bound(cost.begin(), cost.end(), (cost[n] * t) / T) - cost.begin();
    r1 = std::min<int64_t>(n, std::min<int64_t>(r0 + 65536, std::max<int64_t>(r1, r0 + 1)));
    range_rows.push_back(r1);
  }
  const int64_t n_ranges = static_cast<int64_t>(range_rows.size()) - 1;
  out.n_ranges = static_cast<int32_t>(n_ranges);
  struct Cut { int32_t p; int64_t r0, r1, k; };
  std::vector<Cut> cuts;                 // panel-major
  for (int32_t p = 0; p < P; ++p)
    for (int64_t k = 0; k < n_ranges; ++k) cuts.push_back(Cut{p, range_rows[k], range_rows[k + 1], k});
  // Workgroups are dealt to the XCDs round-robin by workgroup id.  Tile k of
  // the emitted order runs on XCD k % kXcds, so the panel-major list is cut
  // into runs, one per XCD, that fill that XCD's workgroup ids in turn: the
  // tiles of one XCD then come from one or two panels, and the workgroups
  // staging the same panel slice share that XCD's L2.
  const int64_t nt = static_cast<int64_t>(cuts.size());
  std::vector<int64_t> slot_tile(nt);
  int64_t next = 0;
  for (int64_t x = 0; x < kXcds; ++x)
    for (int64_t k = x; k < nt; k += kXcds) slot_tile[k] = next++;
  // Tiles are laid out independently, on up to kPlanThreads threads, then
  // concatenated in emitted order with their slot, group and row numbers (and
  // group-end bits) shifted: the result does not depend on the thread count.
  std::vector<PanelLayout> parts(static_cast<size_t>(nt));
  std::atomic<int64_t> next_tile{0};
  auto work = [&] {
    for (int64_t k = next_tile.fetch_add(1); k < nt; k = next_tile.fetch_add(1)) {
      const Cut& c = cuts[slot_tile[k]];
      append_tile(parts[k], col, it, P, width, c.p, c.r0, c.r1, waves, lane_target, min_lg);
    }
  };
  run_on_threads(work, nt);
  for (int64_t k = 0; k < nt; ++k) out.tile_ranges.push_back(static_cast<int32_t>(cuts[slot_tile[k]].k));
  for (PanelLayout& part : parts) {
    const int64_t slot0 = static_cast<int64_t>(out.perm.size());
    const int64_t group0 = static_cast<int64_t>(out.groups.size() / 4);
    const int64_t row0 = static_cast<int64_t>(out.rows.size());
    if (slot0 + static_cast<int64_t>(part.perm.size()) >= (int64_t{1} << 31))
      return fail("panel layout needs 2^31 or more slots");
    const int32_t rec[4] = {part.tiles[0], part.tiles[1], part.tiles[2],
                            static_cast<int32_t>(part.tiles[3] + row0)};
    out.tiles.insert(out.tiles.end(), rec, rec + 4);
    for (int32_t w : part.wave_groups) out.wave_groups.push_back(static_cast<int32_t>(w + group0));
    for (size_t g = 0; g < part.groups.size(); g += 4) {
      const int32_t rec_g[4] = {static_cast<int32_t>(part.groups[g] + slot0), part.groups[g + 1],
                                part.groups[g + 2], static_cast<int32_t>(part.groups[g + 3] + row0)};
      out.groups.insert(out.groups.end(), rec_g, rec_g + 4);
    }
    out.rows.insert(out.rows.end(), part.rows.begin(), part.rows.end());
    out.perm.insert(out.perm.end(), part.perm.begin(), part.perm.end());
    out.col.insert(out.col.end(), part.col.begin(), part.col.end());
    for (size_t wd = 0; wd < part.last_steps.size(); ++wd)
      for (uint32_t bits = part.last_steps[wd]; bits; bits &= bits - 1) {
        const int64_t step = slot0 / 64 + static_cast<int64_t>(wd) * 32 + __builtin_ctz(bits);
        if (static_cast<int64_t>(out.last_steps.size()) <= step / 32)
          out.last_steps.resize(step / 32 + 1, 0u);
        out.last_steps[step / 32] |= 1u << (step % 32);
      }
    part = PanelLayout();   // release the part's memory as it is copied
  }
  out.wave_groups.push_back(static_cast<int32_t>(out.groups.size() / 4));
  // Trailing padding: prefetches run up to two blocks of steps past a stream's end.
  for (int64_t k = 0; k < kPanelTailSlots; ++k) {
    out.perm.push_back(-1);
    out.col.push_back(static_cast<uint16_t>(width));
  }
  if (static_cast<int64_t>(out.perm.size()) >= (int64_t{1} << 31))
    return fail("panel layout needs 2^31 or more slots");
  // One word per 32 steps of the whole slot array, plus one spare word so a
  // 64-bit read at any step stays inside.
  out.last_steps.resize(static_cast<int64_t>(out.perm.size()) / 64 / 32 + 2, 0u);
  return NS_OK;
}

}  // namespace

extern "C" int ns_plan_panels(const int32_t* rowptr, const int32_t* col, int64_t n_rows,
                              int32_t max_panel_width, int32_t tiles_per_panel, int32_t waves,
                              int32_t lane_target, int32_t flags, ns_panel_plan* plan,
                              int64_t* n_row_entries,
                              int32_t* tiles, int32_t* tile_ranges, int32_t* wave_groups,
                              int32_t* groups, uint16_t* rows, uint32_t* last_steps,
                              int32_t* perm, uint16_t* col_out) {
  clear_error();
  if (!rowptr || !plan || !n_row_entries) return fail("rowptr, plan and n_row_entries are required");
  if (n_rows <= 0 || n_rows >= (int64_t{1} << 31)) return fail("N must be in [1, 2^31)");
  if (rowptr[0] != 0) return fail("rowptr[0] must be 0");
  for (int64_t r = 0; r < n_rows; ++r)
    if (rowptr[r + 1] < rowptr[r]) return fail("rowptr must be non-decreasing");
  if (rowptr[n_rows] > 0 && !col) return fail("col is required");
  if (max_panel_width < 4 || max_panel_width > 65532)
    return fail("max_panel_width must be in [4, 65532]");
  if (tiles_per_panel < 1) return fail("tiles_per_panel must be positive");
  if (waves != kPanelWaves) return fail("the panel kernel runs %d wavefronts per workgroup", kPanelWaves);
  if (lane_target < 1) return fail("lane_target must be positive");
  if (flags & ~NS_PANEL_PAIRS) return fail("unknown panel layout flags %d", flags);
  PanelLayout layout;
  if (int rc = build_panels(rowptr, col, n_rows, max_panel_width, tiles_per_panel, waves,
                            lane_target, (flags & NS_PANEL_PAIRS) != 0, layout))
    return rc;
  plan->panel_width = layout.panel_width;
  plan->n_panels = layout.n_panels;
  plan->n_tiles = static_cast<int32_t>(layout.tiles.size() / 4);
  plan->n_groups = static_cast<int32_t>(layout.groups.size() / 4);
  plan->waves = waves;
  plan->flags = flags;
  plan->n_ranges = layout.n_ranges;
  plan->n_slots = static_cast<int64_t>(layout.perm.size());
  plan->n_step_words = static_cast<int64_t>(layout.last_steps.size());
  *n_row_entries = static_cast<int64_t>(layout.rows.size());
  if (tiles) std::copy(layout.tiles.begin(), layout.tiles.end(), tiles);
  if (tile_ranges) std::copy(layout.tile_ranges.begin(), layout.tile_ranges.end(), tile_ranges);
  if (wave_groups) std::copy(layout.wave_groups.begin(), layout.wave_groups.end(), wave_groups);
  if (groups) std::copy(layout.groups.begin(), layout.groups.end(), groups);
  if (rows) std::copy(layout.rows.begin(), layout.rows.end(), rows);
  if (last_steps) std::copy(layout.last_steps.begin(), layout.last_steps.end(), last_steps);
  if (perm) std::copy(layout.perm.begin(), layout.perm.end(), perm);
  if (col_out) std::copy(layout.col.begin(), layout.col.end(), col_out);
  return NS_OK;
}

namespace {

// The band layout of one graph, in host vectors (built twice: size query, then fill).
struct BandLayout {
  int64_t n_groups = 0, n_slots = 0;
  std::vector<int32_t> wave_blocks, blocks, perm;
  std::vector<uint32_t> rows;
  std::vector<uint16_t> col;
};


// Lays out row block [r0, r1).  Per band, the block's rows with edges in the
// band are packed into groups of 64 lanes, cut into register blocks: a lane
// takes one row's segment (the group's 64 longest left, longest first) and, in
// the steps after it, a second, shorter row's segment where one fits.  Each
// group goes to the wavefront with the fewest steps in that band so far, so
// the band's work is balanced across the wavefronts; the kernel's barrier
// after each band lets a row's groups of different bands lie in different
// wavefronts.  A wavefront's blocks are band-ordered and its slots contiguous.
void append_band_block(BandLayout& out, const int32_t* rowptr, const int32_t* col,
                       int64_t r0, int64_t r1, int32_t band_width, int32_t n_bands,
                       int32_t block_steps, bool fill) {
  const int64_t nr = r1 - r0;
  // Each row's edges grouped by band (stable counting sort): start[i][k].
  std::vector<int32_t> start(nr * (n_bands + 1), 0);
  std::vector<int64_t> row_base(nr + 1, 0);
  for (int64_t i = 0; i < nr; ++i) {
    const int64_t r = r0 + i;
    int32_t* st = start.data() + i * (n_bands + 1);
    for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e) ++st[col[e] / band_width + 1];
    for (int32_t k = 0; k < n_bands; ++k) st[k + 1] += st[k];
    row_base[i + 1] = row_base[i] + (rowptr[r + 1] - rowptr[r]);
  }
  std::vector<int32_t> order;   // per row, its edges in band order (CSR order within a band)
  if (fill) {
    order.assign(row_base[nr], 0);
    std::vector<int32_t> at(n_bands);
    for (int64_t i = 0; i < nr; ++i) {
      const int32_t* st = start.data() + i * (n_bands + 1);
      for (int32_t k = 0; k < n_bands; ++k) at[k] = st[k];
      for (int64_t e = rowptr[r0 + i]; e < rowptr[r0 + i + 1]; ++e)
        order[row_base[i] + at[col[e] / band_width]++] = static_cast<int32_t>(e);
    }
  }
  // The wavefronts' parts, concatenated in wavefront order at the end.
  std::vector<BandLayout> waves(kBandWaves);
  // Rows with edges in the band, by segment length (within a length, in row
  // order): a cursor into each length's list, the length dropped once empty.
  std::map<int32_t, std::pair<size_t, std::vector<int32_t>>> by_len;
  auto take = [&](std::map<int32_t, std::pair<size_t, std::vector<int32_t>>>::iterator it) {
    const int32_t i = it->second.second[it->second.first++];
    if (it->second.first == it->second.second.size()) by_len.erase(it);
    return i;
  };
  for (int32_t k = 0; k < n_bands; ++k) {
    auto seg_len = [&](int32_t i) -> int32_t {
      const int32_t* st = start.data() + static_cast<int64_t>(i) * (n_bands + 1);
      return st[k + 1] - st[k];
    };
    auto edge_at = [&](int32_t i, int32_t t) -> int32_t {
      return order[row_base[i] + start[static_cast<int64_t>(i) * (n_bands + 1) + k] + t];
    };
    by_len.clear();
    for (int64_t i = 0; i < nr; ++i)
      if (seg_len(static_cast<int32_t>(i)) > 0)
        by_len[seg_len(static_cast<int32_t>(i))].second.push_back(static_cast<int32_t>(i));
    std::vector<int64_t> band_steps(kBandWaves, 0);
    while (!by_len.empty()) {
      // A group's first rows: the 64 longest segments left, longest first;
      // the group lasts as many steps as the first of them.
      int32_t first[64], second[64];
      int gn = 0;
      while (gn < 64 && !by_len.empty()) first[gn++] = take(std::prev(by_len.end()));
      const int32_t steps = seg_len(first[0]);
      // Second rows: a lane's steps after its first row's segment take the
      // longest segment left that fits them, lanes with the most such steps
      // first.  The lane's word holds the switch step in 8 bits.
      for (int l = 0; l < 64; ++l) second[l] = -1;
      for (int l = gn - 1; l >= 0 && !by_len.empty(); --l) {
        const int32_t len = seg_len(first[l]);
        if (len > kBandMaxSwitch) break;
        auto it = by_len.upper_bound(steps - len);
        if (it == by_len.begin()) break;   // no lane after this one has more room
        second[l] = take(std::prev(it));
      }
      // The wavefront with the fewest steps in this band takes the group.
      const int32_t w = static_cast<int32_t>(
          std::min_element(band_steps.begin(), band_steps.end()) - band_steps.begin());
      band_steps[w] += steps;
      BandLayout& part = waves[w];
      const int32_t group = static_cast<int32_t>(part.n_groups++);
      if (fill)
        for (int l = 0; l < 64; ++l) {
          uint32_t word = kBandNoRow | (kBandNoRow << kBandRowBits);
          if (l < gn) {
            word = static_cast<uint32_t>(first[l]);
            word |= second[l] < 0 ? kBandNoRow << kBandRowBits
                                  : (static_cast<uint32_t>(second[l]) << kBandRowBits) |
                                        (static_cast<uint32_t>(seg_len(first[l])) << 24);
          }
          part.rows.push_back(word);
        }
      // A block spans block_steps steps (those past the group's end are
      // padding) and its slots are lane-major: lane l's steps are the
      // consecutive slots 64*first_step + l*block_steps + (0 .. block_steps-1),
      // so the kernel loads each lane's columns, and its weights, at once.
      for (int32_t t0 = 0; t0 < steps; t0 += block_steps) {
        const int32_t nst = std::min(block_steps, steps - t0);
        const int32_t last = t0 + block_steps >= steps ? 1 : 0;
        const int32_t rec[4] = {static_cast<int32_t>(part.n_slots / 64), k,
                                nst | (last << 8) | (t0 << 9), group};
        part.blocks.insert(part.blocks.end(), rec, rec + 4);
        part.n_slots += int64_t{64} * block_steps;
        if (!fill) continue;
        for (int l = 0; l < 64; ++l)
          for (int32_t t = t0; t < t0 + block_steps; ++t) {
            int32_t edge = -1;
            if (l < gn && t < t0 + nst) {
              const int32_t la = seg_len(first[l]);
              if (t < la) edge = edge_at(first[l], t);
              else if (second[l] >= 0 && t - la < seg_len(second[l])) edge = edge_at(second[l], t - la);
            }
            part.perm.push_back(edge);
            part.col.push_back(edge < 0 ? uint16_t{0xFFFF}
                                        : static_cast<uint16_t>(col[edge] - int64_t{k} * band_width));
          }
      }
    }
  }
  // Concatenate the wavefronts' parts, shifting their step and group numbers.
  for (const BandLayout& part : waves) {
    out.wave_blocks.push_back(static_cast<int32_t>(out.blocks.size() / 4));
    for (size_t q = 0; q < part.blocks.size(); q += 4) {
      const int32_t rec[4] = {static_cast<int32_t>(part.blocks[q] + out.n_slots / 64),
                              part.blocks[q + 1], part.blocks[q + 2],
                              static_cast<int32_t>(part.blocks[q + 3] + out.n_groups)};
      out.blocks.insert(out.blocks.end(), rec, rec + 4);
    }
    out.rows.insert(out.rows.end(), part.rows.begin(), part.rows.end());
    out.perm.insert(out.perm.end(), part.perm.begin(), part.perm.end());
    out.col.insert(out.col.end(), part.col.begin(), part.col.end());
    out.n_slots += part.n_slots;
    out.n_groups += part.n_groups;
  }
}

}  // namespace

extern "C" int32_t ns_band_max_block_rows(int64_t batch) { return band_max_rows(batch); }

extern "C" int ns_plan_bands(const int32_t* rowptr, const int32_t* col, int64_t n_rows,
                             int32_t band_width, int32_t block_rows, int32_t block_steps,
                             ns_band_plan* plan, int32_t* wave_blocks, int32_t* blocks,
                             uint32_t* rows, int32_t* perm, uint16_t* col_out) {
  clear_error();
  if (!rowptr || !plan) return fail("rowptr and plan are required");
  if (n_rows <= 0 || n_rows >= (int64_t{1} << 31)) return fail("N must be in [1, 2^31)");
  if (rowptr[0] != 0) return fail("rowptr[0] must be 0");
  for (int64_t r = 0; r < n_rows; ++r)
    if (rowptr[r + 1] < rowptr[r]) return fail("rowptr must be non-decreasing");
  if (rowptr[n_rows] > 0 && !col) return fail("col is required");
  if (band_width < 1 || band_width > 65535) return fail("band_width must be in [1, 65535]");
  if (block_rows < 1 || block_rows > kBandMaxNarrowRows)
    return fail("block_rows must be in [1, %d]", kBandMaxNarrowRows);
  if (block_steps < 1 || block_steps > kBandMaxBlockSteps)
    return fail("block_steps must be in [1, %d]", kBandMaxBlockSteps);
  for (int64_t e = 0; e < rowptr[n_rows]; ++e)
    if (col[e] < 0 || col[e] >= n_rows) return fail("CSR column %lld out of range", (long long)col[e]);
  const int64_t n_bands = (n_rows + band_width - 1) / band_width;
  const int64_t n_row_blocks = (n_rows + block_rows - 1) / block_rows;
  const bool fill = wave_blocks || blocks || rows || perm || col_out;
  if (fill && !(wave_blocks && blocks && rows && perm && col_out))
    return fail("all output arrays are required together");
  // Row blocks are laid out independently, on up to kPlanThreads threads,
  // then concatenated in order with their slot, group and block numbers
  // shifted: the result does not depend on the thread count.
  std::vector<BandLayout> parts(static_cast<size_t>(n_row_blocks));
  std::atomic<int64_t> next{0};
  auto work = [&] {
    for (int64_t q = next.fetch_add(1); q < n_row_blocks; q = next.fetch_add(1)) {
      const int64_t r0 = q * block_rows, r1 = std::min<int64_t>(n_rows, r0 + block_rows);
      append_band_block(parts[q], rowptr, col, r0, r1, band_width, static_cast<int32_t>(n_bands),
                        block_steps, fill);
    }
  };
  run_on_threads(work, n_row_blocks);
  int64_t n_slots = 0, n_groups = 0, n_blocks64 = 0;
  for (const BandLayout& part : parts) {
    n_slots += part.n_slots;
    n_groups += part.n_groups;
    n_blocks64 += static_cast<int64_t>(part.blocks.size() / 4);
  }
  if (n_slots + int64_t{kBandMaxBlockSteps} * 64 >= (int64_t{1} << 37) ||
      n_blocks64 + 1 >= (int64_t{1} << 31) || n_groups + 1 >= (int64_t{1} << 31))
    return fail("band layout needs too many slots");
  const int32_t n_blocks = static_cast<int32_t>(n_blocks64);
  // The sentinel group (no rows) and block record follow the row blocks, then
  // the tail padding: the kernel loads one block ahead and a whole register
  // block of slots.
  const int32_t sentinel_group = static_cast<int32_t>(n_groups++);
  n_slots += int64_t{kBandMaxBlockSteps} * 64;
  if (fill) {
    int64_t slot0 = 0, group0 = 0, block0 = 0;
    int32_t* wb = wave_blocks;
    for (const BandLayout& part : parts) {
      for (int32_t w : part.wave_blocks) *wb++ = static_cast<int32_t>(w + block0);
      for (size_t b = 0; b < part.blocks.size(); b += 4) {
        int32_t* rec = blocks + 4 * block0 + b;
        rec[0] = static_cast<int32_t>(part.blocks[b] + slot0 / 64);
        rec[1] = part.blocks[b + 1];
        rec[2] = part.blocks[b + 2];
        rec[3] = static_cast<int32_t>(part.blocks[b + 3] + group0);
      }
      std::copy(part.rows.begin(), part.rows.end(), rows + 64 * group0);
      std::copy(part.perm.begin(), part.perm.end(), perm + slot0);
      std::copy(part.col.begin(), part.col.end(), col_out + slot0);
      slot0 += part.n_slots;
      group0 += part.n_groups;
      block0 += static_cast<int64_t>(part.blocks.size() / 4);
    }
    *wb = n_blocks;
    const int32_t sentinel[4] = {0, 0, 0, sentinel_group};
    std::copy(sentinel, sentinel + 4, blocks + 4 * block0);
    std::fill(rows + 64 * group0, rows + 64 * (group0 + 1), kBandNoRow | (kBandNoRow << kBandRowBits));
    std::fill(perm + slot0, perm + slot0 + kBandMaxBlockSteps * 64, -1);
    std::fill(col_out + slot0, col_out + slot0 + kBandMaxBlockSteps * 64, uint16_t{0xFFFF});
  }
  plan->band_width = band_width;
  plan->n_bands = static_cast<int32_t>(n_bands);
  plan->block_rows = block_rows;
  plan->n_row_blocks = static_cast<int32_t>(n_row_blocks);
  plan->n_blocks = n_blocks;
  plan->n_groups = static_cast<int32_t>(n_groups);
  plan->block_steps = block_steps;
  plan->reserved = 0;
  plan->n_slots = n_slots;
  return NS_OK;
}
