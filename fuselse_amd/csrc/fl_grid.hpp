// Launch-size arithmetic shared by the launchers (plain C++, no HIP types, so
// a host compiler can test it alone).
//
// A kernel dispatch packet holds the grid size as a 32-bit count of
// work-items per dimension, so one launch of blocks of `threads` threads
// carries at most max_grid_blocks(threads) blocks.  The cap is rounded down to
// a multiple of 8, the XCD count, so that a launch split in several keeps each
// block's position modulo 8 (the hardware deals blocks out to the XCDs in
// turn).
#pragma once

#include <stdint.h>

namespace fl {

constexpr int64_t kMaxDispatchWorkItems = 0xFFFFFFFFll;

constexpr int64_t max_grid_blocks(int64_t threads) { return (kMaxDispatchWorkItems / threads) & ~(int64_t)7; }

// Calls launch(first, count) for consecutive block ranges that cover
// [0, total) in order, each of at most max_grid_blocks(threads) blocks.
template <typename F>
inline void for_grid_chunks(int64_t total, int64_t threads, F launch) {
    const int64_t cap = max_grid_blocks(threads);
    for (int64_t first = 0; first < total; first += cap) launch(first, total - first < cap ? total - first : cap);
}

// A grid-stride launch of at most `want` blocks, capped to one dispatch.
constexpr int64_t grid_stride_blocks(int64_t want, int64_t threads) {
    return want < max_grid_blocks(threads) ? want : max_grid_blocks(threads);
}

}  // namespace fl
