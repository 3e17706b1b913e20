// The batched step's split-product sizing (whispereacp_amd/csrc/batch_plan.h)
// on the CPU: every launch the batch plans fits the buffers it reserves at
// create, and a launch one column group, one row tile or one split past them
// is refused. Prints "ok <case>" per passing case; exits 1 on the first
// failure.
#include "../../whispereacp_amd/csrc/batch_plan.h"

#include <cstdio>
#include <cstdlib>

using namespace wsp::batch;

static void expect(bool condition, const char* what)
{
    if (!condition)
    {
        std::printf("FAIL %s\n", what);
        std::exit(1);
    }
    std::printf("ok %s\n", what);
}

int main()
{
    // (width, feed-forward width, streams x tokens per step) of the batched
    // configurations and a few odd ones.
    const int shapes[][3] = {{1024, 4096, 16}, {1280, 5120, 32}, {1280, 5120, 128}, {384, 1536, 5}, {512, 2048, 33}};
    for (const auto& shape : shapes)
    {
        const int d = shape[0], f = shape[1], rows_cap = shape[2];
        const int split_groups = (d + kTileColumns - 1) / kTileColumns; // fc2's output columns
        const int rows_padded = 16 * row_tiles(rows_cap);
        const std::size_t partials = split_partials_capacity(split_groups, rows_padded);
        const std::size_t counters = (std::size_t) split_groups;
        int kb = 0, splits = 0;
        plan_split_runs(f, true, kb, splits);
        expect(splits >= 1 && splits <= kMaxSplits && kb * splits >= f / 32, "fc2 plans at most kMaxSplits whole runs");
        for (int rows = 1; rows <= rows_cap; ++rows)
            if (!split_launch_fits(d, rows, splits, partials, counters))
                expect(false, "every planned fc2 launch fits the reserved buffers");
        expect(true, "every planned fc2 launch fits the reserved buffers");
        expect(!split_launch_fits(d + kTileColumns, rows_cap, splits, partials, counters),
               "one column group more is refused");
        expect(!split_launch_fits(d, rows_padded + 1, kMaxSplits, partials, counters),
               "one row tile past the padded rows is refused at full splits");
        expect(!split_launch_fits(d, rows_cap, kMaxSplits + 1, partials, counters), "one split more is refused");
        expect(split_launch_fits(d + kTileColumns, rows_cap, 1, partials, counters),
               "an unsplit launch needs no partials");
    }
    int kb = 0, splits = 0;
    plan_split_runs(4096, false, kb, splits);
    expect(splits == 1 && kb == 128, "no split when splitting is not allowed");
    plan_split_runs(96, true, kb, splits);
    expect(splits == 3 && kb == 1, "three k-blocks split three ways");
    return 0;
}
