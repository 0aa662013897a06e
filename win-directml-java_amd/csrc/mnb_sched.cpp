// mnb_sched.cpp -- host-side work list of a prefill GEMM launch (tile-list
// order, see mnb_sched.h).
#include "mnb_sched.h"

#include <algorithm>
#include <functional>
#include <limits>
#include <queue>
#include <utility>

namespace mnb {

bool sk_tile_list_parts(const std::vector<SkItem> &items, int G, int64_t split_above, std::vector<SkTile> &seq,
                        std::vector<SkRange> &wg, SkSplitList &list) {
    constexpr int kBlock = 32;    // tiles of one block: what the workgroups of one XCD run side by side
    constexpr int kBlockM = 4;    // m-tiles per block (so 8 n-groups): the fewest x and weight bytes per stage
    constexpr int kTileCost = 2;  // epilogue of a tile, in stages (balance only)
    list.n = 0;
    int32_t parts = 0;
    // (1) the launch's tiles in block order: per item, chunks of kBlockM
    // m-tiles; per chunk, blocks of nb n-groups (consecutive blocks of a
    // chunk share its x rows); a tile longer than split_above stages as its
    // parts, side by side
    std::vector<SkTile> order;
    for (int i = 0; i < (int)items.size(); ++i) {
        const SkItem &it = items[(size_t)i];
        const int MT = it.MT, NG = it.T / it.MT;
        const int np = split_above > 0 && it.ST > split_above ? (int)((it.ST + split_above - 1) / split_above) : 1;
        for (int m0 = 0; m0 < MT; m0 += kBlockM) {
            const int m1 = std::min(MT, m0 + kBlockM), nb = kBlock / (m1 - m0);
            for (int n0 = 0; n0 < NG; n0 += nb)
                for (int m = m0; m < m1; ++m)
                    for (int n = n0; n < std::min(NG, n0 + nb); ++n) {
                        const int t = m + n * MT;
                        if (np == 1) {
                            order.push_back(SkTile{i, t, 0, it.ST, -1});
                            continue;
                        }
                        if (list.n == kSkMaxSplits || parts + np > kSkMaxParts) return false;
                        SkSplit &e = list.e[list.n++];
                        e.t_slot = (int32_t)((uint32_t)t | kSkSplitParts);
                        e.item = (uint16_t)i;
                        e.first = (uint8_t)parts;
                        e.last = (uint8_t)(parts + np - 1);
                        for (int j = 0; j < np; ++j) {
                            const int s0 = (int)((int64_t)j * it.ST / np), s1 = (int)((int64_t)(j + 1) * it.ST / np);
                            order.push_back(SkTile{i, t, s0, s1 - s0, parts++});
                        }
                    }
        }
    }
    // (2) one contiguous chunk of equal cost per XCD
    const int X = G % 8 == 0 ? 8 : 1, per = G / X;
    int64_t total = 0;
    for (const SkTile &e : order) total += e.nst + kTileCost;
    // (3) each chunk dealt to its XCD's workgroups, least loaded first, its
    // longest tiles first (a stable order, so each item's tiles keep their
    // block order and still run side by side; longest first keeps the
    // busiest workgroup close to the mean when tile lengths differ)
    std::vector<std::vector<SkTile>> chunks((size_t)X);
    int64_t before = 0;
    for (const SkTile &e : order) {
        const int64_t c = e.nst + kTileCost;
        const int x = (int)std::min<int64_t>(X - 1, (2 * before + c) * X / (2 * total));
        before += c;
        chunks[(size_t)x].push_back(e);
    }
    std::vector<std::vector<SkTile>> lists((size_t)G);
    std::vector<int64_t> load((size_t)G, 0);
    for (int x = 0; x < X; ++x) {
        std::vector<SkTile> &ch = chunks[(size_t)x];
        std::stable_sort(ch.begin(), ch.end(), [](const SkTile &a, const SkTile &b) { return a.nst > b.nst; });
        for (const SkTile &e : ch) {
            const int64_t c = e.nst + kTileCost;
            int best = x * per;
            for (int w = x * per + 1; w < (x + 1) * per; ++w)
                if (load[(size_t)w] < load[(size_t)best]) best = w;
            lists[(size_t)best].push_back(e);
            load[(size_t)best] += c;
        }
    }
    // (4) workgroup-major list and the workgroup starts
    seq.clear();
    wg.assign((size_t)G + 1, SkRange{0, 0});
    int64_t iter = 0;
    for (int g = 0; g < G; ++g) {
        wg[(size_t)g] = SkRange{(int32_t)seq.size(), (int32_t)iter};
        for (const SkTile &e : lists[(size_t)g]) {
            seq.push_back(e);
            iter += e.nst;
        }
    }
    wg[(size_t)G] = SkRange{(int32_t)seq.size(), (int32_t)iter};
    return true;
}

void sk_tile_list(const std::vector<SkItem> &items, int G, std::vector<SkTile> &seq, std::vector<SkRange> &wg) {
    SkSplitList none;
    sk_tile_list_parts(items, G, 0, seq, wg, none);
}

bool stream_schedule(const std::vector<int32_t> &NT, const std::vector<int32_t> &ST, int64_t waves,
                     std::vector<uint32_t> &units, std::vector<int32_t> &wave_begin) {
    units.clear();
    wave_begin.clear();
    if (waves < 1 || NT.size() != ST.size() || NT.size() > 65536) return false;
    std::vector<std::pair<int32_t, uint32_t>> order;   // (cost, code)
    for (size_t i = 0; i < NT.size(); ++i) {
        if (NT[i] < 1 || NT[i] > 65536 || ST[i] < 1) return false;
        const int32_t cost = kStreamJobTiles * stream_jobs(ST[i]) + 1;
        for (int32_t nt = 0; nt < NT[i]; ++nt) order.emplace_back(cost, ((uint32_t)i << 16) | (uint32_t)nt);
    }
    std::stable_sort(order.begin(), order.end(),
                     [](const std::pair<int32_t, uint32_t> &a, const std::pair<int32_t, uint32_t> &b) {
                         return a.first > b.first;
                     });
    typedef std::pair<int64_t, int64_t> Load;   // (cost, wave)
    std::priority_queue<Load, std::vector<Load>, std::greater<Load>> heap;
    for (int64_t w = 0; w < waves; ++w) heap.push(Load(0, w));
    std::vector<std::vector<uint32_t>> per((size_t)waves);
    for (const auto &u : order) {
        Load l = heap.top();
        heap.pop();
        per[(size_t)l.second].push_back(u.second);
        l.first += u.first;
        heap.push(l);
    }
    wave_begin.reserve(2 * (size_t)waves + 1);
    units.reserve(order.size());
    for (auto &v : per) {
        std::sort(v.begin(), v.end());
        int64_t jobs = 0;
        for (uint32_t c : v) jobs += stream_jobs(ST[c >> 16]);
        if (jobs > std::numeric_limits<int32_t>::max()) return false;
        wave_begin.push_back((int32_t)units.size());
        wave_begin.push_back((int32_t)jobs);
        units.insert(units.end(), v.begin(), v.end());
    }
    wave_begin.push_back((int32_t)units.size());
    return true;
}

}  // namespace mnb

namespace mnb {

int sk_tiles(int M, int NT, int ntw, int fm) {
    const int bn = 8 * ntw * 16, bm = 32 * fm;   // 8 waves of 16 ntw columns, 32 fm rows
    return ((M + bm - 1) / bm) * ((NT * 16 + bn - 1) / bn);
}

bool sk_wide_supported(int scale_f32, int sps) {
    // a wave's scales of its four n-tiles (16 rows each) must fit one 1 KiB window
    return kGemmWideNTW * 16 * sps * (scale_f32 ? 4 : 2) <= 1024;
}

// Estimated time of G workgroups (us).  A least-squares fit (4% median error)
// to 300 timings on MI355X of the Phi-3 projections at M = 128, 512 and 2048
// over every candidate G: a stage costs 1.16 us plus 0.38 us times the busy
// fraction of the chip, each tile a workgroup touches 8.6 us (pipeline fill
// and epilogue), and split tiles 0.28 us per MB of partial tiles (stored, then
// read by the reduce kernel) less 2 us, plus 1.7 us when every CU holds a
// split workgroup.
static constexpr double kStageUs = 1.16, kStageBusyUs = 0.38, kTileUs = 8.6;

double sk_cost(int64_t T, int64_t ST, int64_t G, int cu_count) {
    const int64_t I = T * ST;
    const int64_t per_wg = (I + G - 1) / G;
    bool split = false;
    for (int64_t b = 1; b < G && !split; ++b) split = (b * I / G) % ST != 0;
    const double load = (double)std::min<int64_t>(G, cu_count) / cu_count;
    const double tiles = (double)((per_wg + ST - 1) / ST + (split ? 1 : 0));
    double t = (double)per_wg * (kStageUs + kStageBusyUs * load) + kTileUs * tiles;
    if (split) {
        const double partial_mb = (double)(G + std::min<int64_t>(G, T)) * kSkPartialFloats * 4.0 / 1.0e6;
        t += 0.28 * partial_mb - 2.0 + (G > cu_count - 8 ? 1.7 : 0.0);
    }
    return t;
}

// Candidates: every workgroup count that gives each workgroup whole tiles (G
// dividing T), every tile cut into m equal pieces (G = m T), one workgroup per
// CU, and two CUs per XCD fewer; the cheapest by sk_cost wins.
int sk_grid(int T, int ST, int cu_count) {
    const int64_t I = (int64_t)T * ST;
    const int64_t cap = std::min<int64_t>(sk_max_grid(cu_count), I);
    int64_t best = 0;
    double best_t = 0.0;
    auto consider = [&](int64_t G) {
        if (G < 1 || G > cap) return;
        const double t = sk_cost(T, ST, G, cu_count);
        if (best == 0 || t < best_t) best = G, best_t = t;
    };
    for (int64_t k = 1; k <= T; ++k)
        if (T % k == 0) consider(T / k);
    for (int64_t G = 2 * (int64_t)T; G <= cap; G += T) consider(G);
    consider(cap);
    consider(cap - 16);
    return (int)best;
}

SinglePlan sk_single_plan(int M, int NT, int ST, int scale_f32, int sps, int cu_count) {
    const int T = sk_tiles(M, NT);
    SinglePlan plan{false, kGemmNTW, kGemmFM, sk_grid(T, ST, cu_count), 0.0};
    const double stream_k = sk_cost(T, ST, plan.G, cu_count);
    plan.est = stream_k;
    if (!sk_wide_supported(scale_f32, sps)) return plan;
    const int Tw = sk_tiles(M, NT, kGemmWideNTW, kGemmFM);
    const int Gw = std::min(sk_max_grid(cu_count), Tw);
    int busiest = 0;   // tiles of the busiest workgroup in closed-form order
    for (int g = 0; g < Gw; ++g) busiest = std::max(busiest, sk_cf_first(Tw, Gw, g + 1) - sk_cf_first(Tw, Gw, g));
    const double load = (double)Gw / cu_count;
    const double wide = busiest * (ST * (kStageUs + kStageBusyUs * load) * kGemmWideStageCost + kTileUs);
    if (wide < stream_k) plan = SinglePlan{true, kGemmWideNTW, kGemmFM, Gw, wide};
    return plan;
}

}  // namespace mnb

namespace mnb {

void sk_split_list(const SkItem *host, int32_t count, int64_t iters, int G, SkSplitList &list) {
    list.n = 0;
    auto start = [&](int64_t g) { return g * iters / G; };
    int32_t k = 0;
    for (int b = 1; b < G && b <= kSkMaxSplits; ++b) {
        const int64_t s = start(b);
        while (k + 1 < count && host[k + 1].ibeg <= s) ++k;
        const SkItem &it = host[k];
        const int64_t local = s - it.ibeg;
        if (local % it.ST == 0) continue;                // between tiles
        const int64_t t = local / it.ST, ts = it.ibeg + t * it.ST;
        if (start(b - 1) > ts) continue;                 // an earlier boundary lies inside t
        int64_t g_last = b;                              // the owner of the tile's last iteration
        while (g_last + 1 < G && start(g_last + 1) <= ts + it.ST - 1) ++g_last;
        SkSplit &e = list.e[list.n++];
        e.t_slot = (int32_t)((uint32_t)t | (start(b - 1) == ts ? 0u : kSkSplitSlot1));
        e.item = (uint16_t)k;
        e.first = (uint8_t)(b - 1);
        e.last = (uint8_t)g_last;
    }
}


// ---- the K-sliced kernel's planner (host-only; the kernel is csrc/mnb_gemm_ks.hip) ----

bool ks_config_supported(int mb, int ntw, int scale_f32, int has_zp, int sps) {
    if (mb == 2 && (ntw == 1 || ntw == 2 || ntw == 4)) return true;
    if (mb == 1 && ntw == 4) return true;   // 9 <= M <= 16 (ks_skinny_plan)
    // 16 output units per wave leave registers for the weights of one
    // super-tile only where their scales and zero points are small
    return mb == 4 && ntw == 4 && sps != 8 && !(scale_f32 && has_zp);
}

int ks_waves(int ST) { return ST < kKsMaxWaves ? ST : kKsMaxWaves; }

// Cost model of one launch, fitted to single-product timings of the Phi-3
// projections (K 3072 and 8192, N 3072 to 32064, M 17 to 512): a workgroup
// alone on its CU takes c + k us per super-tile of each wave; with more
// workgroups than CUs the chip sustains thr wave-super-tiles per us (at 256
// CUs).  The launch takes the longer of the two.  (Output blocks of 64 x 16,
// 64 x 32 and 128 x 32 were measured too; with their fitted costs the model
// never prefers them over 2100 shapes from K 256 to 14336 and N 64 to 151936.)
//
// For products of 6 or more super-tiles (K > 640) the block and the estimate
// returned (which the caller compares with the GEMM's) come from a second fit
// that also charges each round of workgroups a fixed cost r (the round's
// launch, the LDS reduction, the epilogue): c2 + max(rounds x (super-tiles
// per wave x k2 + r), the same chip-rate term), fitted to every block forced
// on the Phi-3 and Qwen2.5-0.5B projections (K 896 to 8192, N 896 to 151936,
// M 32 to 512; median error 2.6-5% against 6.5-10% for the first model,
// whose error grows with the rounds).  Measured on random shapes where the
// two fits choose differently: its blocks 5% faster in total (36 shapes, 12
// of them 13-21% faster, one 2% slower); with its estimate also deciding
// against the GEMM, 5.2% faster in total (40 shapes: 18 of them 8-31%
// faster, 8 of them 1-12% slower, where the GEMM's model underestimates its
// short tiles).  On shorter K, where several workgroups share a CU, it
// misjudged the blocks, so those keep the first model.
struct KsCost {
    int mb, ntw;
    double c, k, thr;
    double c2, k2, r2, thr2;
};
static const KsCost kKsCosts[] = {
    {2, 1, 3.06, 0.88, 2114.0, 2.417, 0.878, 0.687, 2223.1},
    {2, 2, 2.92, 1.16, 1138.0, 1.346, 1.311, 1.715, 1376.7},
    {2, 4, 3.86, 1.58, 757.0, 1.177, 1.754, 2.901, 693.6},
    {4, 4, 5.50, 2.30, 469.0, 0.932, 2.543, 4.603, 422.6},
};
constexpr int kKsRoundCostMinST = 6;

KsPlan ks_single_plan(int M, int NT, int ST, int scale_f32, int has_zp, int sps, int cu_count) {
    KsPlan best{{0, 0}, 0.0, 0};
    KsConfig block{0, 0};
    double block_est = 0.0;
    const int cu = cu_count > 0 ? cu_count : 256;
    const int W = ks_waves(ST);
    const double spw = (double)ST / W;
    for (const KsCost &k : kKsCosts) {
        if (!ks_config_supported(k.mb, k.ntw, scale_f32, has_zp, sps)) continue;
        const KsConfig c{k.mb, k.ntw};
        const int64_t wgs = ks_workgroups(M, NT, c);
        const double rounds = (double)((wgs + cu - 1) / cu);
        const double alone = rounds * spw * k.k;
        const double busy = (double)wgs * W * spw / (k.thr * cu / 256.0);
        const double est = k.c + std::max(alone, busy);
        if (best.wgs == 0 || est < best.est) best = KsPlan{c, est, wgs};
        const double est2 =
            k.c2 + std::max(rounds * (spw * k.k2 + k.r2), (double)wgs * W * spw / (k.thr2 * cu / 256.0));
        if (block.mb == 0 || est2 < block_est) {
            block = c;
            block_est = est2;
        }
    }
    if (best.wgs > 0 && ST >= kKsRoundCostMinST) {
        best.c = block;
        best.est = block_est;
        best.wgs = ks_workgroups(M, NT, block);
    }
    return best;
}

int64_t ks_workgroups(int M, int NT, const KsConfig &c) {
    return (int64_t)((NT + c.ntw - 1) / c.ntw) * ((M + 16 * c.mb - 1) / (16 * c.mb));
}

}  // namespace mnb
