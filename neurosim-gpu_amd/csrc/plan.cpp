// Host-side pieces of the C ABI: error storage, version, and the row-block
// planner that cuts a destination-major CSR into the workgroup-sized blocks
// consumed by the tick kernels.
#include <stdint.h>

#include <cstdio>

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
