// Host-side sizing rules of the batched step's split tile products
// (batch.hip), kept free of device code so a CPU test can check them.
#pragma once

#include <cstddef>

namespace wsp::batch
{
constexpr int kTileColumns = 64; // output columns of one tile block
constexpr int kMaxSplits = 8;    // most k-splits a tile launch takes

// Row tiles of 16 a launch over `rows` rows covers, a power of two.
inline int row_tiles(int rows)
{
    const int tiles = (rows + 15) / 16;
    int t = 1;
    while (t < tiles)
        t *= 2;
    return t;
}

// k-blocks (32 inner values each) per split, and the splits, of a product
// over `inner` values: eight runs of whole k-blocks when splitting is allowed.
inline void plan_split_runs(int inner, bool can_split, int& kb_per_split, int& splits)
{
    const int kblocks = inner / 32;
    const int most = can_split ? (kMaxSplits < kblocks ? kMaxSplits : kblocks) : 1;
    kb_per_split = (kblocks + most - 1) / most;
    splits = (kblocks + kb_per_split - 1) / kb_per_split;
}

// Partial floats a split launch of `out` columns, `rows` rows and `splits`
// k-splits writes: 64 columns x 16 rows per row tile, per split, per column
// group.
inline std::size_t split_partials(int out, int rows, int splits)
{
    const std::size_t groups = (std::size_t) (out + kTileColumns - 1) / kTileColumns;
    return groups * (std::size_t) splits * kTileColumns * 16 * (std::size_t) row_tiles(rows);
}

// Whether that launch fits buffers of `partials_capacity` floats and
// `counters_capacity` column-group counters; a launch that does not is
// refused before it is issued.
inline bool split_launch_fits(int out, int rows, int splits, std::size_t partials_capacity,
                              std::size_t counters_capacity)
{
    if (splits <= 1)
        return true;
    const std::size_t groups = (std::size_t) (out + kTileColumns - 1) / kTileColumns;
    return split_partials(out, rows, splits) <= partials_capacity && groups <= counters_capacity;
}

// The buffers a batch of `rows_padded` rows (a multiple of 16 covering
// row_tiles(rows)) reserves for launches of up to `split_groups` column
// groups: the partial floats, then the counters.
inline std::size_t split_partials_capacity(int split_groups, int rows_padded)
{
    return (std::size_t) kMaxSplits * (std::size_t) split_groups * (std::size_t) rows_padded * kTileColumns;
}
} // namespace wsp::batch
