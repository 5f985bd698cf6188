// Host driver for sanitizer builds of the layout planners (csrc/plan.cpp):
// compiled with g++ under -fsanitize=address,undefined or -fsanitize=thread
// together with plan.cpp, it plans a set of CSR graphs (random, hub rows,
// trailing empty rows, no edges, one neuron) as panels (plain and pair
// layouts), bands and row blocks, once on one host thread and once on 16,
// requires identical layouts, and requires rejection of out-of-range columns.
// Prints "ok" and exits 0 on success.
#include <stdint.h>
#include <stdlib.h>

#include <cstdio>
#include <random>
#include <vector>

#include "neurosim_hip.h"

namespace {

struct Csr {
  std::vector<int32_t> rowptr, col;
};

Csr random_csr(int64_t n, int64_t m, uint32_t seed, int64_t hub_row, int64_t hub_len,
               int64_t empty_tail) {
  std::mt19937 rng(seed);
  std::vector<std::vector<int32_t>> rows(n);
  const int64_t live = n - empty_tail;
  for (int64_t e = 0; live > 0 && e < m; ++e)
    rows[rng() % live].push_back(static_cast<int32_t>(rng() % n));
  if (hub_row >= 0)
    for (int64_t e = 0; e < hub_len; ++e) rows[hub_row].push_back(static_cast<int32_t>(rng() % n));
  Csr g;
  g.rowptr.push_back(0);
  for (auto& r : rows) {
    g.col.insert(g.col.end(), r.begin(), r.end());
    g.rowptr.push_back(static_cast<int32_t>(g.col.size()));
  }
  return g;
}

int failures = 0;

void check(bool ok, const char* what) {
  if (!ok) {
    std::fprintf(stderr, "FAILED: %s (%s)\n", what, ns_last_error());
    ++failures;
  }
}

struct PanelOut {
  ns_panel_plan plan{};
  int64_t entries = 0;
  std::vector<int32_t> tiles, tile_ranges, wave_groups, groups, perm;
  std::vector<uint16_t> rows, col;
  std::vector<uint32_t> last_steps;
  bool operator==(const PanelOut& o) const {
    return plan.n_panels == o.plan.n_panels && plan.n_slots == o.plan.n_slots &&
           plan.n_ranges == o.plan.n_ranges && tile_ranges == o.tile_ranges &&
           tiles == o.tiles && wave_groups == o.wave_groups && groups == o.groups &&
           perm == o.perm && rows == o.rows && col == o.col && last_steps == o.last_steps;
  }
};

PanelOut plan_panels(const Csr& g, int32_t width, int32_t tiles, int32_t flags) {
  PanelOut o;
  const int64_t n = static_cast<int64_t>(g.rowptr.size()) - 1;
  const int32_t* col = g.col.empty() ? nullptr : g.col.data();
  int rc = ns_plan_panels(g.rowptr.data(), col, n, width, tiles, 16, 24, flags, &o.plan,
                          &o.entries, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                          nullptr, nullptr);
  check(rc == 0, "panel size query");
  if (rc) return o;
  o.tiles.resize(4 * o.plan.n_tiles);
  o.tile_ranges.resize(o.plan.n_tiles);
  o.wave_groups.resize(o.plan.n_tiles * 16 + 1);
  o.groups.resize(4 * o.plan.n_groups);
  o.rows.resize(o.entries);
  o.last_steps.resize(o.plan.n_step_words);
  o.perm.resize(o.plan.n_slots);
  o.col.resize(o.plan.n_slots);
  rc = ns_plan_panels(g.rowptr.data(), col, n, width, tiles, 16, 24, flags, &o.plan, &o.entries,
                      o.tiles.data(), o.tile_ranges.data(), o.wave_groups.data(), o.groups.data(), o.rows.data(),
                      o.last_steps.data(), o.perm.data(), o.col.data());
  check(rc == 0, "panel fill");
  return o;
}

struct BandOut {
  ns_band_plan plan{};
  std::vector<int32_t> wave_blocks, blocks, perm;
  std::vector<uint32_t> rows;
  std::vector<uint16_t> col;
  bool operator==(const BandOut& o) const {
    return plan.n_slots == o.plan.n_slots && wave_blocks == o.wave_blocks &&
           blocks == o.blocks && perm == o.perm && rows == o.rows && col == o.col;
  }
};

BandOut plan_bands(const Csr& g, int32_t width, int32_t rows, int32_t steps) {
  BandOut o;
  const int64_t n = static_cast<int64_t>(g.rowptr.size()) - 1;
  const int32_t* col = g.col.empty() ? nullptr : g.col.data();
  int rc = ns_plan_bands(g.rowptr.data(), col, n, width, rows, steps, &o.plan, nullptr, nullptr,
                         nullptr, nullptr, nullptr);
  check(rc == 0, "band size query");
  if (rc) return o;
  o.wave_blocks.resize(NS_BAND_WAVES * o.plan.n_row_blocks + 1);
  o.blocks.resize(4 * (o.plan.n_blocks + 1));
  o.rows.resize(64 * o.plan.n_groups);
  o.perm.resize(o.plan.n_slots);
  o.col.resize(o.plan.n_slots);
  rc = ns_plan_bands(g.rowptr.data(), col, n, width, rows, steps, &o.plan, o.wave_blocks.data(),
                     o.blocks.data(), o.rows.data(), o.perm.data(), o.col.data());
  check(rc == 0, "band fill");
  return o;
}

}  // namespace

int main() {
  const Csr graphs[] = {
      random_csr(30000, 300000, 1, 17, 5000, 0),
      random_csr(20000, 90000, 2, -1, 0, 9000),   // trailing empty rows
      random_csr(50, 0, 3, -1, 0, 0),             // no edges
      random_csr(1, 0, 4, -1, 0, 0),              // one neuron
      random_csr(9000, 40000, 5, 0, 9000, 100),
  };
  for (const Csr& g : graphs) {
    const int64_t n = static_cast<int64_t>(g.rowptr.size()) - 1;
    for (int32_t flags : {0, NS_PANEL_PAIRS}) {
      const int32_t width = n > 4000 ? 4000 : 40940;
      setenv("NEUROSIM_PLAN_THREADS", "1", 1);
      const PanelOut one = plan_panels(g, width, 7, flags);
      setenv("NEUROSIM_PLAN_THREADS", "16", 1);
      const PanelOut many = plan_panels(g, width, 7, flags);
      check(one == many, "panel layout independent of threads");
    }
    setenv("NEUROSIM_PLAN_THREADS", "1", 1);
    const BandOut one = plan_bands(g, 3000, 257, 4);
    setenv("NEUROSIM_PLAN_THREADS", "16", 1);
    const BandOut many = plan_bands(g, 3000, 257, 4);
    check(one == many, "band layout independent of threads");
    int64_t blocks = 0;
    check(ns_plan_row_blocks(g.rowptr.data(), n, 1024, nullptr, 0, &blocks) == 0, "row blocks");
    std::vector<int32_t> bounds(2 * (blocks + 1));
    check(ns_plan_row_blocks(g.rowptr.data(), n, 1024, bounds.data(),
                             static_cast<int64_t>(bounds.size()), &blocks) == 0, "row block fill");
  }
  // Out-of-range columns, -1 included, are rejected by both planners.
  Csr bad = random_csr(12, 60, 6, -1, 0, 0);
  bad.col[41] = -1;
  ns_panel_plan p{};
  int64_t entries = 0;
  for (int32_t flags : {0, NS_PANEL_PAIRS})
    check(ns_plan_panels(bad.rowptr.data(), bad.col.data(), 12, 4, 1, 16, 12, flags, &p, &entries,
                         nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                         nullptr) != 0,
          "panel planner rejects column -1");
  ns_band_plan b{};
  check(ns_plan_bands(bad.rowptr.data(), bad.col.data(), 12, 4, 4, 4, &b, nullptr, nullptr,
                      nullptr, nullptr, nullptr) != 0,
        "band planner rejects column -1");
  if (failures) return 1;
  std::printf("ok\n");
  return 0;
}
