// Checks the tile-list schedule of a grouped prefill GEMM (mnb::sk_tile_list)
// on the CPU.  Input (stdin): G, then one line "MT NG ST" per item.  Exits 1
// on the first broken invariant; prints balance and locality figures.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <set>
#include <vector>

#include "mnb_sched.h"

using namespace mnb;

static int fail(const char *what, long a, long b) {
    printf("FAIL %s (%ld, %ld)\n", what, a, b);
    return 1;
}

int main() {
    int G = 0;
    if (scanf("%d", &G) != 1 || G < 1) return fail("input", G, 0);
    std::vector<SkItem> items;
    int MT, NG, ST;
    long ibeg = 0;
    while (scanf("%d %d %d", &MT, &NG, &ST) == 3) {
        SkItem it{};
        it.MT = MT;
        it.T = MT * NG;
        it.ST = ST;
        it.ibeg = (int32_t)ibeg;
        ibeg += (long)it.T * ST;
        items.push_back(it);
    }
    std::vector<SkTile> seq;
    std::vector<SkRange> wg;
    sk_tile_list(items, G, seq, wg);
    long tiles = 0, iters = 0;
    for (const SkItem &it : items) tiles += it.T, iters += (long)it.T * it.ST;
    // every tile of every item exactly once
    if ((long)seq.size() != tiles) return fail("tile count", (long)seq.size(), tiles);
    std::vector<std::vector<char>> seen(items.size());
    for (size_t i = 0; i < items.size(); ++i) seen[i].assign((size_t)items[i].T, 0);
    for (const SkTile &e : seq) {
        if (e.item < 0 || e.item >= (int)items.size()) return fail("item index", e.item, (long)items.size());
        if (e.t < 0 || e.t >= items[(size_t)e.item].T) return fail("tile index", e.t, items[(size_t)e.item].T);
        if (seen[(size_t)e.item][(size_t)e.t]++) return fail("tile twice", e.item, e.t);
    }
    // workgroup ranges: contiguous, covering, stages consistent with the tiles
    if ((int)wg.size() != G + 1) return fail("wg size", (long)wg.size(), G + 1);
    if (wg[0].pos != 0 || wg[0].iter != 0) return fail("wg[0]", wg[0].pos, wg[0].iter);
    if (wg[(size_t)G].pos != tiles || wg[(size_t)G].iter != iters) return fail("wg[G]", wg[(size_t)G].pos, wg[(size_t)G].iter);
    long maxload = 0;
    for (int g = 0; g < G; ++g) {
        const SkRange a = wg[(size_t)g], b = wg[(size_t)g + 1];
        if (b.pos < a.pos || b.iter < a.iter) return fail("wg order", g, b.pos - a.pos);
        long st = 0;
        for (int k = a.pos; k < b.pos; ++k) st += items[(size_t)seq[(size_t)k].item].ST;
        if (st != b.iter - a.iter) return fail("wg stages", g, st);
        maxload = std::max(maxload, st);
    }
    // locality: the r-th tiles of one XCD's workgroups run side by side; count
    // the distinct x row blocks (item, m-tile) and weight column blocks
    // (item, n-group) they read
    const int X = G % 8 == 0 ? 8 : 1, per = G / X;
    double xb = 0, wb = 0;
    long rounds = 0;
    for (int x = 0; x < X; ++x) {
        for (int r = 0;; ++r) {
            std::set<long> xs, ws;
            for (int g = x * per; g < (x + 1) * per; ++g) {
                const int k = wg[(size_t)g].pos + r;
                if (k >= wg[(size_t)g + 1].pos) continue;
                const SkTile e = seq[(size_t)k];
                const int mt = items[(size_t)e.item].MT;
                xs.insert((long)e.item << 32 | (e.t % mt));
                ws.insert((long)e.item << 32 | (e.t / mt));
            }
            if (xs.empty()) break;
            xb += (double)xs.size();
            wb += (double)ws.size();
            ++rounds;
        }
    }
    printf("ok tiles=%ld iters=%ld max_wg_stages=%ld mean=%.1f imbalance=%.4f x_blocks=%.2f w_blocks=%.2f\n", tiles,
           iters, maxload, (double)iters / G, (double)maxload * G / (double)iters - 1.0, xb / (double)rounds,
           wb / (double)rounds);
    return 0;
}
