// Launch geometry shared by the kernels and the host-side planners (plain
// C++: the planners compile without the HIP headers).
#pragma once

#include <cstdint>

namespace ns {

constexpr int kThreads = 256;   // 4 wavefronts of 64 lanes
// XCDs of the target (gfx950); workgroups are dealt to them round-robin by id.
constexpr int kXcds = 8;
constexpr int kMaxRows = 256;   // rows per row block (one lane per row at most density)

// Column-panel kernel (batch widths 1 and 2): 16 wavefronts per workgroup
// stream their own runs of 64-lane steps; a slot stream ends with
// kPanelTailSlots padding slots so prefetches may run past a stream's end.
constexpr int kPanelWaves = 16;
constexpr int kPanelThreads = kPanelWaves * 64;
constexpr int kPanelMaxPrefetch = 16;                  // steps per register block, at most
constexpr int kPanelTailSlots = 2 * kPanelMaxPrefetch * 64;
constexpr int kBandWaves = 16;                          // wavefronts per band workgroup (one per CU)
constexpr int kBandMaxBlockRows = 2496;                 // 16 float row sums each in LDS (156 KB)
constexpr int kBandMaxNarrowRows = 4095;                // 8 or 4 sums each (128 KB at 8), the lane word's limit
constexpr int kBandMaxBlockSteps = 8;                   // steps per register block, at most
// A band lane word: first row (bits 0-11), second row (bits 12-23) and the
// step at which the lane moves on to its second row (bits 24-31).
constexpr unsigned kBandNoRow = 0xFFF;
constexpr int kBandRowBits = 12;
constexpr int kBandMaxSwitch = 255;
static_assert(kBandMaxBlockRows <= static_cast<int>(kBandNoRow), "block rows fit a lane word");
static_assert(kBandMaxNarrowRows <= static_cast<int>(kBandNoRow), "block rows fit a lane word");

// Most destination rows per band workgroup for a batch: its LDS holds each
// row's sums over the workgroup's column tile (16 columns, or 8 or 4).
constexpr int band_max_rows(int64_t batch) {
  return batch % 16 == 0 ? kBandMaxBlockRows : kBandMaxNarrowRows;
}

}  // namespace ns
