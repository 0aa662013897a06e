// mnb_sched.h -- the work list of a prefill GEMM launch (host and device
// side), free of HIP headers so the schedule builds and is checked on its own.
#pragma once

#include <stdint.h>

#include <vector>

namespace mnb {

// One product of a GEMM launch (M > 16): the weight's tiled buffers, x, y and
// the sizes; ibeg is its first (tile, stage) iteration in the launch.
struct SkItem {
    const void *q_t;
    const void *s_t;
    const uint8_t *zp_t;
    const void *x;              // fp16 [M][ldx]
    void *y;
    int32_t ldx, kx, M, N;
    int32_t NT, ST, MT, T;      // n-tiles, super-tiles (stages), m-tiles, output tiles
    int32_t y_f16, accumulate;
    int32_t y_vec;              // N % 4 == 0 and y aligned for 4-element stores
    int32_t ibeg;
};

// Tile-list order of a GEMM launch: tile t of item `item` (m-tile t % MT,
// n-group t / MT), and the start of one workgroup's tiles (list position,
// first iteration).
struct SkTile {
    int32_t item, t;
};
struct SkRange {
    int32_t pos, iter;
};

// Tile list of a launch over `items` on G workgroups (logical workgroups
// [x G / 8, (x + 1) G / 8) run on XCD x when G is a multiple of 8): the
// tiles in blocks of 32 that share x rows and weight columns (up to 4
// m-tiles by 32 / that many n-groups), cut into one contiguous chunk of
// equal stages per XCD,
// each chunk dealt tile by tile, longest tiles first (stable), to the least
// loaded workgroup of that XCD.
// Fills seq (workgroup-major, every tile of every item once) and wg (G + 1
// entries; workgroup g owns seq[wg[g].pos, wg[g + 1].pos), whose stages are
// the iterations [wg[g].iter, wg[g + 1].iter)).
void sk_tile_list(const std::vector<SkItem> &items, int G, std::vector<SkTile> &seq, std::vector<SkRange> &wg);

}  // namespace mnb
