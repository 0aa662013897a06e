// mnb_sched.h -- the work list of a prefill GEMM launch (host and device
// side), free of HIP headers so the schedule builds and is checked on its own.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <vector>

#if defined(__HIPCC__)
#define MNB_HD __host__ __device__
#else
#define MNB_HD
#endif

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
// n-group t / MT), its stages [st0, st0 + nst) (a whole tile: 0 and ST) and,
// for a part of a tile cut along K, the index of the fp32 partial tile it
// writes into the workspace (-1: a whole tile, which writes y); and the start
// of one workgroup's tiles (list position, first iteration).
struct SkTile {
    int32_t item, t;
    int32_t st0 = 0, nst = 0;
    int32_t part = -1;
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

// The tile list of ONE item in closed form: exactly what sk_tile_list gives a
// launch of a single item (every tile costs the same, so each XCD's chunk is
// dealt round robin), computed from the tile count instead of read from a
// table, so a single product can run in tile-list order without a device
// table.  X = 8 XCDs when G is a multiple of 8, else 1; per = G / X logical
// workgroups per XCD; the item's tiles in block order are cut at
// sk_cf_xcd_start(T, X, x), and logical workgroup g = x * per + r owns the
// block-order positions sk_cf_xcd_start(T, X, x) + r + j * per below the next
// XCD's start.
MNB_HD inline int32_t sk_cf_xcd_start(int32_t T, int32_t X, int32_t x) {
    // tile i goes to XCD min(X - 1, floor((2 i + 1) X / (2 T))) (the equal-cost
    // cut of sk_tile_list), so XCD x starts at ceil((2 T x - X) / (2 X))
    if (x <= 0) return 0;
    if (x >= X) return T;
    const int64_t v = 2 * (int64_t)T * x - X;
    return v <= 0 ? 0 : (int32_t)((v + 2 * X - 1) / (2 * X));
}
// Tiles owned by the logical workgroups before g (g = G gives T).
MNB_HD inline int32_t sk_cf_first(int32_t T, int32_t G, int32_t g) {
    const int32_t X = G % 8 == 0 ? 8 : 1, per = G / X, x = g / per, r = g % per;
    const int32_t c = sk_cf_xcd_start(T, X, x), L = sk_cf_xcd_start(T, X, x + 1) - c;
    return c + (L / per) * r + (r < L % per ? r : L % per);
}
// Block-order position of logical workgroup g's first tile; its j-th tile
// is at that position + j * per.
MNB_HD inline int32_t sk_cf_base(int32_t T, int32_t G, int32_t g) {
    const int32_t X = G % 8 == 0 ? 8 : 1, per = G / X;
    return sk_cf_xcd_start(T, X, g / per) + g % per;
}
MNB_HD inline int32_t sk_cf_step(int32_t G) { return G % 8 == 0 ? G / 8 : G; }
// Tile (m-tile + n-group * MT) at block-order position q of an item with MT
// m-tiles and NG n-groups: chunks of up to 4 m-tiles, each cut into blocks of
// 32 / (its m-tiles) n-groups, a block's tiles m-tile-major.
MNB_HD inline int32_t sk_cf_tile(int32_t MT, int32_t NG, int32_t q) {
    const int32_t full = MT / 4;
    int32_t m0, mc, local;
    if (q < full * 4 * NG) {
        const int32_t c = q / (4 * NG);
        m0 = 4 * c;
        mc = 4;
        local = q - c * 4 * NG;
    } else {
        m0 = full * 4;
        mc = MT - m0;
        local = q - full * 4 * NG;
    }
    const int32_t nb = 32 / mc, blk = local / (mc * nb), n0 = blk * nb;
    const int32_t nn = NG - n0 < nb ? NG - n0 : nb;
    const int32_t within = local - blk * mc * nb;
    return m0 + within / nn + (n0 + within % nn) * MT;
}

// ---- GEMM launch shapes and the single-product planner (host only) ----
//
// n-tiles (16 rows) per wave of the GEMM: 2 (256-column tiles), or 4
// (512-column tiles, in tile-list order only); 32-row fragments per tile: 4
// (128 rows), 2 (64-row tiles) or 1 (32-row tiles), both with 512 columns in
// tile-list order only.
constexpr int kGemmNTW = 2, kGemmWideNTW = 4;
constexpr int kGemmFM = 4, kGemmHalfFM = 2, kGemmSkinnyFM = 1;
// Cost of a 512-column stage in 256-column stages (same-box A/B of the
// Phi-3 groups with the 512-column kernel's current stage order: 256-column
// against 512-column tiles 947 vs 1103 TFLOP/s at M=128, 1008 vs 1172 at
// M=256, 1038 vs 1254 at M=512, so 2 x 0.83-0.86).
constexpr double kGemmWideStageCost = 1.70;
// One fp32 partial tile of a split 128 x 256 tile (floats).
constexpr int kSkPartialFloats = 128 * 256;
// Most workgroups of one GEMM launch: the partial-tile workspace (and the
// fixed scratch array of mnb_matmul_noalloc) is sized for this many.
constexpr int kSkMaxGrid = 256;

// Output tiles of 32 fm rows x 128 ntw columns of an M x (16 NT) product.
int sk_tiles(int M, int NT, int ntw = kGemmNTW, int fm = kGemmFM);
// Whether the weight variant has a 512-column kernel: a wave's four n-tiles
// of scales must fit one 1 KiB window.
bool sk_wide_supported(int scale_f32, int sps);
// Largest workgroup count of a GEMM launch on cu_count CUs: one persistent
// workgroup per CU, at most kSkMaxGrid.  Every grid the planners pick is at
// most this.
inline int sk_max_grid(int cu_count) { return cu_count < kSkMaxGrid ? (cu_count < 1 ? 1 : cu_count) : kSkMaxGrid; }
// Bytes of the stream-K workspace of a G-workgroup launch: two fp32 partial
// tiles per workgroup (slot 0 for its first tile, 1 for its last).
constexpr size_t sk_workspace_bytes(int G) { return (size_t)G * 2 * kSkPartialFloats * sizeof(float); }
// Workgroup count for T tiles of ST stages on cu_count CUs (a cost model:
// whole tiles per workgroup when that is cheapest, else stream-K with split
// tiles summed by a reduce launch); at most sk_max_grid(cu_count) and at most
// T * ST.
int sk_grid(int T, int ST, int cu_count);
// Estimated time (us) of T tiles of ST stages on G workgroups in stream-K
// order (the model sk_grid minimises).
double sk_cost(int64_t T, int64_t ST, int64_t G, int cu_count);
// How one product with M > 16 runs on the GEMM: stream-K over 128 x 256
// tiles on sk_grid workgroups, or whole 128 x 512 tiles in closed-form
// tile-list order when the cost model, with a 512-column stage costing
// kGemmWideStageCost 256-column stages, expects the busiest workgroup to
// finish first that way.
struct SinglePlan {
    bool closed;
    int ntw, fm, G;
    double est;   // the cost model's time (us)
};
SinglePlan sk_single_plan(int M, int NT, int ST, int scale_f32, int sps, int cu_count);

// The K-sliced kernel (one product, M > 16, where the GEMM would have few
// tiles): workgroup (m-block, n-group) owns 16 mb rows x 16 ntw columns of y
// over the whole K, its ks_waves(ST) waves on contiguous K slices.
constexpr int kKsMaxWaves = 8;
struct KsConfig {
    int mb, ntw;   // 16-row blocks of x and 16-row n-tiles per workgroup
};
bool ks_config_supported(int mb, int ntw, int scale_f32, int has_zp, int sps);
int ks_waves(int ST);
int64_t ks_workgroups(int M, int NT, const KsConfig &c);
// The block this kernel would run one product with and the cost model's
// estimate (us) for it, which the caller compares with the GEMM's
// (sk_single_plan).
struct KsPlan {
    KsConfig c;
    double est;
    int64_t wgs;
};
KsPlan ks_single_plan(int M, int NT, int ST, int scale_f32, int has_zp, int sps, int cu_count);

// The split tiles of one launch, passed by value in the reduce kernel's
// arguments, so nothing is allocated: tile t of item `item` and its
// contributors first .. last in K order.
// - Stream-K (the ranges of G logical workgroups over `iters` iterations,
//   range g = [g iters / G, (g + 1) iters / G), listed by the host at launch
//   time): first .. last are the workgroups whose ranges hold some of the
//   tile's stages; first's partial tile is in its slot 0 when the tile starts
//   its range, else slot 1 (bit 31); the others' are in their slot 0.
// - Tile list with parts (bit 30): first .. last are the indices of the
//   parts' partial tiles.
// t < 2^30: a split tile has at least two stages and a launch fewer than
// 2^31 iterations.
constexpr uint32_t kSkSplitSlot1 = 0x80000000u, kSkSplitParts = 0x40000000u, kSkSplitTile = 0x3fffffffu;
struct SkSplit {
    int32_t t_slot;     // t | kSkSplitSlot1 | kSkSplitParts
    uint16_t item;
    uint8_t first, last;
};
constexpr int kSkMaxSplits = kSkMaxGrid - 1;   // at most one split tile per range boundary
struct SkSplitList {
    int32_t n;
    SkSplit e[kSkMaxSplits];
};
// Fills `list` for items host[0 .. count) (ibeg ascending, iters in all,
// G <= kSkMaxGrid): each split tile once, at the first range boundary inside it.
void sk_split_list(const SkItem *host, int32_t count, int64_t iters, int G, SkSplitList &list);

// A tile list whose tiles of more than split_above stages are cut along K
// into ceil(ST / split_above) parts of equal stages (to within one), so that
// one long tile no longer sets the busiest workgroup.  The parts of a tile
// are listed side by side in block order and dealt like tiles; each writes
// an fp32 partial tile (workspace index `part`, numbered tile by tile), and
// `list` names every cut tile with its parts first .. last (tile-list flag
// set), for the reduce kernel to sum in K order.  Returns false when the
// parts would need more than kSkMaxParts partial tiles or kSkMaxSplits cut
// tiles (seq, wg and list are then unspecified).  split_above <= 0 cuts
// nothing (sk_tile_list).
constexpr int kSkMaxParts = 256;
bool sk_tile_list_parts(const std::vector<SkItem> &items, int G, int64_t split_above, std::vector<SkTile> &seq,
                        std::vector<SkRange> &wg, SkSplitList &list);

// The streaming kernel's unit of issue: up to kStreamJobTiles consecutive
// super-tiles of one n-tile (a unit of ST super-tiles is stream_jobs(ST)
// jobs; the last job of a unit whose ST is not a multiple loads its last
// super-tile again for the missing ones and does not compute them).
constexpr int32_t kStreamJobTiles = 4;
MNB_HD inline int32_t stream_jobs(int32_t ST) { return (ST + kStreamJobTiles - 1) / kStreamJobTiles; }

// Static schedule of a group of M = 1 products on the persistent streaming
// kernel (mnb_stream.hip).  A unit is one 16-row n-tile of one item over its
// whole K, coded (item << 16) | n-tile; item i has NT[i] n-tiles of ST[i]
// super-tiles.  Units are dealt longest first (cost = the super-tiles its
// jobs read + 1, the unit's output write counted as one) to the least loaded
// of `waves` waves; each wave keeps its units in group order.  Fills units
// (wave-major) and wave_begin (2 * waves + 1 entries: per wave its first unit
// and the number of jobs of its units, then the end of the list).  Returns
// false when there are 65536 items or more, an item has more than 65536
// n-tiles, or a wave's jobs do not fit 31 bits.
bool stream_schedule(const std::vector<int32_t> &NT, const std::vector<int32_t> &ST, int64_t waves,
                     std::vector<uint32_t> &units, std::vector<int32_t> &wave_begin);

}  // namespace mnb
