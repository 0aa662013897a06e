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
    float unfold;               // 2^-fold_exp of the weight: undoes its stored scale factor
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

// Static schedule of a group of M = 1 products on the persistent streaming
// kernel (mnb_stream.hip).  A unit is one 16-row n-tile of one item over its
// whole K, coded (item << 16) | n-tile; item i has NT[i] n-tiles of ST[i]
// super-tiles.  Units are dealt longest first (cost = super-tiles + 1, the
// unit's output write counted as one) to the least loaded of `waves` waves;
// each wave keeps its units in group order.  Fills units (wave-major) and
// wave_begin (2 * waves + 1 entries: per wave its first unit and the number of
// super-tiles of its units, then the end of the list).  Returns false when
// there are 65536 items or more, an item has more than 65536 n-tiles, or a
// wave's super-tiles do not fit 31 bits.
bool stream_schedule(const std::vector<int32_t> &NT, const std::vector<int32_t> &ST, int64_t waves,
                     std::vector<uint32_t> &units, std::vector<int32_t> &wave_begin);

}  // namespace mnb
