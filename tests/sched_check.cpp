// Checks the schedules of a group launch on the CPU.  Input (stdin):
//   tile list of a grouped prefill GEMM (mnb::sk_tile_list): G, then one line
//     "MT NG ST" per item;
//   streaming M = 1 schedule (mnb::stream_schedule): the word "stream", the
//     wave count, then one line "NT ST" per item;
//   closed-form tile list of a single item (mnb::sk_cf_*): the word "closed",
//     then lines "G MT NG ST", each checked against sk_tile_list of that item;
//   "grid", "split" and "parts": see check_grid, check_split, check_parts;
//   K-sliced plan of single products (mnb::ks_single_plan): the word
//   "ksplan", then lines "M NT ST scale_f32 has_zp sps", each answered with
//   "mb ntw est wgs" (mb 0: no supported block).
// Exits 1 on the first broken invariant; prints balance (and, for the tile
// list, locality) figures.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <set>
#include <vector>

#include "mnb_sched.h"

using namespace mnb;

static int fail(const char *what, long a, long b) {
    printf("FAIL %s (%ld, %ld)\n", what, a, b);
    return 1;
}

// Every (item, n-tile) unit exactly once, each wave's units in group order,
// the wave table consistent with the units, and the longest-first bound:
// no wave carries more than the mean cost plus one unit.
static int check_stream() {
    long waves = 0;
    if (scanf("%ld", &waves) != 1 || waves < 1) return fail("input", waves, 0);
    std::vector<int32_t> NT, ST;
    int nt, st;
    while (scanf("%d %d", &nt, &st) == 2) {
        NT.push_back(nt);
        ST.push_back(st);
    }
    std::vector<uint32_t> units;
    std::vector<int32_t> wb;
    if (!stream_schedule(NT, ST, waves, units, wb)) {
        printf("refused\n");
        return 0;
    }
    long total = 0, cost = 0, maxunit = 0;
    for (size_t i = 0; i < NT.size(); ++i) {
        total += NT[i];
        const long job_tiles = 4L * ((ST[i] + 3) / 4);   // 4-tile jobs, the last one padded
        cost += (long)NT[i] * (job_tiles + 1);
        maxunit = std::max<long>(maxunit, job_tiles + 1);
    }
    if ((long)units.size() != total) return fail("unit count", (long)units.size(), total);
    if ((long)wb.size() != 2 * waves + 1) return fail("wave table size", (long)wb.size(), 2 * waves + 1);
    std::vector<std::vector<char>> seen(NT.size());
    for (size_t i = 0; i < NT.size(); ++i) seen[i].assign((size_t)NT[i], 0);
    long maxcost = 0, busy = 0;
    for (long w = 0; w < waves; ++w) {
        const long b = wb[(size_t)(2 * w)], e = wb[(size_t)(2 * w + 2)];
        if (b > e || e > (long)units.size()) return fail("wave range", b, e);
        if (w == 0 && b != 0) return fail("first wave start", b, 0);
        long jobs = 0, c = 0;
        for (long k = b; k < e; ++k) {
            const uint32_t u = units[(size_t)k];
            const size_t it = u >> 16, t = u & 0xFFFFu;
            if (it >= NT.size() || (long)t >= NT[it]) return fail("unit code", (long)it, (long)t);
            if (seen[it][t]++) return fail("unit twice", (long)it, (long)t);
            if (k > b && units[(size_t)k - 1] >= u) return fail("wave order", w, k);
            jobs += (ST[it] + 3) / 4;
            c += 4L * ((ST[it] + 3) / 4) + 1;
        }
        if (jobs != wb[(size_t)(2 * w + 1)]) return fail("wave jobs", w, jobs);
        maxcost = std::max(maxcost, c);
        busy += e > b;
    }
    if (wb[(size_t)(2 * waves)] != (long)units.size()) return fail("end of list", wb[(size_t)(2 * waves)], (long)units.size());
    const double mean = (double)cost / (double)waves;
    if ((double)maxcost > mean + (double)maxunit) return fail("longest-first bound", maxcost, (long)mean);
    printf("ok units=%ld waves=%ld busy=%ld max_wave_cost=%ld mean=%.1f imbalance=%.4f\n", total, waves, busy, maxcost,
           mean, (double)maxcost / mean - 1.0);
    return 0;
}

// The closed form must give every workgroup exactly the tiles, in the same
// order, and the same first iteration as the table sk_tile_list builds for
// the same single item.
static int check_closed() {
    int G, MT, NG, ST, cases = 0;
    while (scanf("%d %d %d %d", &G, &MT, &NG, &ST) == 4) {
        std::vector<SkItem> items(1);
        SkItem &it = items[0];
        it = SkItem{};
        it.MT = MT;
        it.T = MT * NG;
        it.ST = ST;
        std::vector<SkTile> seq;
        std::vector<SkRange> wg;
        sk_tile_list(items, G, seq, wg);
        for (int g = 0; g <= G; ++g) {
            const int first = sk_cf_first(it.T, G, g);
            if (wg[(size_t)g].pos != first || wg[(size_t)g].iter != first * ST) return fail("workgroup start", g, first);
            if (g == G) break;
            const int n = sk_cf_first(it.T, G, g + 1) - first;
            for (int j = 0; j < n; ++j) {
                const int t = sk_cf_tile(MT, NG, sk_cf_base(it.T, G, g) + j * sk_cf_step(G));
                if (seq[(size_t)(first + j)].t != t || seq[(size_t)(first + j)].item != 0)
                    return fail("tile", g * 100000L + j, t);
            }
        }
        ++cases;
    }
    printf("ok closed cases=%d\n", cases);
    return 0;
}

// The single-product planner's grids against the workspace they need: for
// lines "cu_count M NT ST scale_f32 sps", sk_grid and sk_single_plan never
// pick more than sk_max_grid(cu_count) <= kSkMaxGrid workgroups, nor more
// workgroups than iterations, so the partial tiles of any plan fit
// sk_workspace_bytes(kSkMaxGrid) -- the size of the context's workspace on a
// device of at least kSkMaxGrid CUs and of mnb_matmul_noalloc's fixed array.
static int check_grid() {
    int cu, M, NT, ST, f32, sps, cases = 0;
    while (scanf("%d %d %d %d %d %d", &cu, &M, &NT, &ST, &f32, &sps) == 6) {
        const int cap = sk_max_grid(cu);
        if (cap < 1 || cap > kSkMaxGrid || cap > cu) return fail("max grid", cu, cap);
        const int T = sk_tiles(M, NT);
        const int G = sk_grid(T, ST, cu);
        if (G < 1 || G > cap || (int64_t)G > (int64_t)T * ST) return fail("sk_grid", cu * 100000L + T, G);
        if (sk_workspace_bytes(G) > sk_workspace_bytes(kSkMaxGrid)) return fail("workspace", G, kSkMaxGrid);
        const SinglePlan p = sk_single_plan(M, NT, ST, f32, sps, cu);
        if (p.G < 1 || p.G > cap) return fail("single plan grid", cu, p.G);
        if (p.closed ? (p.ntw != kGemmWideNTW || !sk_wide_supported(f32, sps)) : (p.ntw != kGemmNTW || p.G != G))
            return fail("single plan shape", p.ntw, p.G);
        ++cases;
    }
    printf("ok grid cases=%d\n", cases);
    return 0;
}

// The reduce launch's split list against the partial tiles the GEMM writes:
// for lines "G ST T [ST T ...]" (a stream-K launch of items with ST stages
// and T tiles each), the GEMM's walk of each workgroup's range (segments of
// one tile each; a segment shorter than its tile is written as a partial
// tile, in slot 0 for the workgroup's first segment, else slot 1) must give,
// for every split tile, exactly the contributors and slots that
// mnb::sk_split_list lists, in workgroup order.
static int check_split() {
    char line[8192];
    int cases = 0;
    while (fgets(line, sizeof line, stdin)) {
        std::vector<long> v;
        for (char *tok = strtok(line, " \n"); tok; tok = strtok(nullptr, " \n")) v.push_back(atol(tok));
        if (v.size() < 3 || v.size() % 2 == 0) continue;
        const int G = (int)v[0];
        std::vector<SkItem> items;
        long ibeg = 0;
        for (size_t i = 1; i + 1 < v.size(); i += 2) {
            SkItem it{};
            it.ST = (int32_t)v[i];
            it.T = (int32_t)v[i + 1];
            it.ibeg = (int32_t)ibeg;
            ibeg += (long)it.ST * it.T;
            items.push_back(it);
        }
        const long iters = ibeg;
        if (G < 1 || G > kSkMaxGrid || G > iters) return fail("input", G, iters);
        // the GEMM's partial tiles: key (item, tile) -> (workgroup, slot) in workgroup order
        std::map<std::pair<int, long>, std::vector<std::pair<int, int>>> want;
        for (int g = 0; g < G; ++g) {
            long i = (long)g * iters / G;
            const long i1 = (long)(g + 1) * iters / G;
            bool first = true;
            while (i < i1) {
                int k = 0;
                while (k + 1 < (int)items.size() && items[(size_t)k + 1].ibeg <= i) ++k;
                const SkItem &it = items[(size_t)k];
                const long t = (i - it.ibeg) / it.ST, ts = it.ibeg + t * it.ST;
                const long end = std::min(i1, ts + it.ST);
                if (end - i < it.ST) want[{k, t}].push_back({g, first ? 0 : 1});
                first = false;
                i = end;
            }
        }
        SkSplitList list;
        sk_split_list(items.data(), (int32_t)items.size(), iters, G, list);
        if ((size_t)list.n != want.size()) return fail("split count", list.n, (long)want.size());
        for (int j = 0; j < list.n; ++j) {
            const SkSplit &e = list.e[j];
            const long t = e.t_slot & kSkSplitTile;
            const int slot0 = (int)((uint32_t)e.t_slot >> 31);
            if ((uint32_t)e.t_slot & kSkSplitParts) return fail("parts flag in a stream-K list", j, t);
            auto w = want.find({(int)e.item, t});
            if (w == want.end()) return fail("unknown split tile", e.item, t);
            if ((int)w->second.size() != e.last - e.first + 1) return fail("contributors", j, e.last - e.first + 1);
            for (int c = 0; c < (int)w->second.size(); ++c) {
                const int slot = c == 0 ? slot0 : 0;
                if (w->second[(size_t)c].first != e.first + c || w->second[(size_t)c].second != slot)
                    return fail("contributor slot", j, c);
            }
        }
        ++cases;
    }
    printf("ok split cases=%d\n", cases);
    return 0;
}

// Tile lists with parts (mnb::sk_tile_list_parts): for lines "G split_above
// MT NG ST [MT NG ST ...]", every tile of every item is covered exactly once:
// whole (stages 0 .. ST, no partial) when ST <= split_above, else by
// ceil(ST / split_above) parts whose stage ranges tile [0, ST) in K order,
// each shorter than split_above + 1, with consecutive partial indices that
// the reduce list names (tile, item, first .. last, parts flag); the
// workgroup ranges agree with the listed stages; and the busiest workgroup
// exceeds the mean by less than the longest unit.  Prints per line the
// busiest workgroup's stages with and without parts.
static int check_parts() {
    char line[8192];
    int cases = 0;
    while (fgets(line, sizeof line, stdin)) {
        std::vector<long> v;
        for (char *tok = strtok(line, " \n"); tok; tok = strtok(nullptr, " \n")) v.push_back(atol(tok));
        if (v.size() < 5 || (v.size() - 2) % 3 != 0) continue;
        const int G = (int)v[0];
        const long split = v[1];
        std::vector<SkItem> items;
        long ibeg = 0;
        for (size_t i = 2; i + 2 < v.size(); i += 3) {
            SkItem it{};
            it.MT = (int32_t)v[i];
            it.T = (int32_t)(v[i] * v[i + 1]);
            it.ST = (int32_t)v[i + 2];
            it.ibeg = (int32_t)ibeg;
            ibeg += (long)it.T * it.ST;
            items.push_back(it);
        }
        const long iters = ibeg;
        std::vector<SkTile> seq, seq0;
        std::vector<SkRange> wg, wg0;
        SkSplitList list;
        if (!sk_tile_list_parts(items, G, split, seq, wg, list)) {
            printf("refused %d\n", cases);
            ++cases;
            continue;
        }
        sk_tile_list(items, G, seq0, wg0);
        // coverage: per (item, tile) the stage ranges, in the order listed
        std::map<std::pair<int, long>, std::vector<SkTile>> got;
        for (const SkTile &e : seq) {
            if (e.item < 0 || e.item >= (int)items.size()) return fail("item index", e.item, (long)items.size());
            if (e.t < 0 || e.t >= items[(size_t)e.item].T) return fail("tile index", e.t, items[(size_t)e.item].T);
            got[{e.item, (long)e.t}].push_back(e);
        }
        long tiles = 0;
        for (const SkItem &it : items) tiles += it.T;
        if ((long)got.size() != tiles) return fail("tiles covered", (long)got.size(), tiles);
        std::vector<char> part_seen((size_t)kSkMaxParts, 0);
        int cut = 0;
        long longest = 0;
        for (auto &kv : got) {
            const SkItem &it = items[(size_t)kv.first.first];
            std::vector<SkTile> &ps = kv.second;
            std::sort(ps.begin(), ps.end(), [](const SkTile &a, const SkTile &b) { return a.st0 < b.st0; });
            const long np = split > 0 && it.ST > split ? (it.ST + split - 1) / split : 1;
            if ((long)ps.size() != np) return fail("parts of a tile", (long)ps.size(), np);
            long s0 = 0;
            for (size_t j = 0; j < ps.size(); ++j) {
                const SkTile &e = ps[j];
                if (e.st0 != s0 || e.nst < 1) return fail("stage ranges", e.st0, s0);
                if (np > 1 && e.nst > split) return fail("part longer than split", e.nst, split);
                if (np == 1 && e.part != -1) return fail("whole tile with a partial", e.part, 0);
                if (np > 1) {
                    if (e.part < 0 || e.part >= kSkMaxParts || part_seen[(size_t)e.part]++) return fail("part index", e.part, 0);
                    if (e.part != ps[0].part + (int)j) return fail("part indices not consecutive", e.part, ps[0].part);
                }
                s0 += e.nst;
                longest = std::max<long>(longest, e.nst);
            }
            if (s0 != it.ST) return fail("stages covered", s0, it.ST);
            if (np > 1) {
                // the reduce list names this tile once, with its parts in K order
                int found = 0;
                for (int j = 0; j < list.n; ++j) {
                    const SkSplit &e = list.e[j];
                    if (!((uint32_t)e.t_slot & kSkSplitParts) || ((uint32_t)e.t_slot & kSkSplitSlot1)) return fail("flags", j, 0);
                    if (e.item == kv.first.first && (long)(e.t_slot & kSkSplitTile) == kv.first.second) {
                        ++found;
                        if (e.first != ps[0].part || e.last != ps.back().part) return fail("list parts", e.first, ps[0].part);
                    }
                }
                if (found != 1) return fail("cut tile listed", found, 1);
                ++cut;
            }
        }
        if (cut != list.n) return fail("list length", list.n, cut);
        // workgroup ranges
        if ((int)wg.size() != G + 1 || wg[0].pos != 0 || wg[0].iter != 0) return fail("wg[0]", wg[0].pos, wg[0].iter);
        if (wg[(size_t)G].pos != (long)seq.size() || wg[(size_t)G].iter != iters) return fail("wg[G]", wg[(size_t)G].pos, iters);
        long busiest = 0, busiest0 = 0;
        for (int g = 0; g < G; ++g) {
            long st = 0;
            for (int k = wg[(size_t)g].pos; k < wg[(size_t)g + 1].pos; ++k) st += seq[(size_t)k].nst;
            if (st != wg[(size_t)g + 1].iter - wg[(size_t)g].iter) return fail("wg stages", g, st);
            busiest = std::max(busiest, st);
            busiest0 = std::max<long>(busiest0, wg0[(size_t)g + 1].iter - wg0[(size_t)g].iter);
        }
        // the deal's bound (per XCD chunk, with each unit's epilogue cost of 2 stages)
        if ((double)busiest > (double)iters / G * 1.15 + longest + 2 * 8) return fail("balance", busiest, iters / G);
        printf("ok parts busiest=%ld unsplit=%ld mean=%.1f cut=%d\n", busiest, busiest0, (double)iters / G, cut);
        ++cases;
    }
    printf("ok parts cases=%d\n", cases);
    return 0;
}

static int print_ksplan() {
    int M, NT, ST, f32, zp, sps;
    while (scanf("%d %d %d %d %d %d", &M, &NT, &ST, &f32, &zp, &sps) == 6) {
        const KsPlan p = ks_single_plan(M, NT, ST, f32, zp, sps, 256);
        if (p.wgs > 0 && (p.wgs != ks_workgroups(M, NT, p.c) || !ks_config_supported(p.c.mb, p.c.ntw, f32, zp, sps)))
            return fail("ksplan block", p.c.mb, p.c.ntw);
        printf("%d %d %.3f %lld\n", p.wgs > 0 ? p.c.mb : 0, p.c.ntw, p.est, (long long)p.wgs);
    }
    return 0;
}

int main() {
    char first[32] = {0};
    if (scanf("%31s", first) != 1) return fail("input", 0, 0);
    if (strcmp(first, "stream") == 0) return check_stream();
    if (strcmp(first, "closed") == 0) return check_closed();
    if (strcmp(first, "grid") == 0) return check_grid();
    if (strcmp(first, "split") == 0) return check_split();
    if (strcmp(first, "parts") == 0) return check_parts();
    if (strcmp(first, "ksplan") == 0) return print_ksplan();
    const int G = atoi(first);
    if (G < 1) return fail("input", G, 0);
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
