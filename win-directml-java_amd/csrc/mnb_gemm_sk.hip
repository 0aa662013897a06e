// mnb_gemm_sk.hip -- prefill-shaped MatMulNBits (M > 16): stream-K GEMM on
// fp16 MFMA with the int4 weights dequantized in registers.
//
// Replaces the tiled HLSL batch GEMM INT4_MATMUL_BATCH_TILED_HLSL
// (directml-windows-bindings/src/main/java/com/aresstack/windirectml/windows/
// MatMulNBitsKernel.java:732-820) and its 256-row host chunking (:2374-2387).
//
// Output tile 128 (M) x 256 (N) per workgroup of 8 waves (two per SIMD, so
// one wave's LDS and dequant latency hides behind the other's MFMAs), each
// wave 128 x 32: four 32-row x fragments against one 32-column weight
// fragment of v_mfma_f32_32x32x16_f16, fp32 accumulators (512-column tiles:
// two weight fragments per wave, see the work split below).  The weight
// fragment is the MFMA's A operand and x its B operand, so the accumulators
// hold y transposed: each lane owns four consecutive columns of one row per
// 4-register group and writes them with one 8-byte (fp16) or 16-byte (fp32)
// store.
// Operand pipeline, one 128-k stage at a time: every operand of stage s + 2 --
// the x tile (32 KiB), the packed weight tiles (16 KiB), their scales and zero
// points -- is copied straight from HBM into a 3-slot LDS ring by direct
// global->LDS loads while stage s computes, so no load ever passes through
// registers and two stages of latency are hidden (a 2-slot ring, one stage,
// where three slots do not fit the 160 KiB LDS).  Per 16-k step a wave
// dequantizes its weight fragment in registers (w = (q - zp) * scale, scale
// folded into the fp16 operand) and runs 4 MFMAs against four x fragments.
// x rows are stored with chunk c of row m at slot c ^ (m & 15), so the
// fragment reads are free of bank conflicts.
//
// Work split: the grid is one persistent workgroup per CU.  A launch covers
// one product (mnb_matmul) or a recorded group of independent products
// (mnb_group_*, M > 16), in one of two orders:
// - Stream-K: the (tile, stage) iterations of the launch (the items' tiles
//   one after another) are cut into equal contiguous ranges, one per
//   workgroup, so every CU gets the same MFMA work whatever the tile count; a
//   range may run from one item into the next.  A workgroup that owns all
//   stages of a tile writes y directly.  A tile whose stages span several
//   workgroups is written as fp32 partial tiles, one per contributor, and
//   summed in contributor order by sk_reduce_kernel, launched right after on
//   the same stream over the whole chip; no workgroup ever waits for another.
// - Tile list (groups with several tiles per workgroup, and single products
//   with many tiles): a list (a host-built table, mnb_sched.cpp, or for one
//   product the same list in closed form) gives each workgroup whole tiles,
//   ordered so that the workgroups of one XCD run tiles sharing x rows and
//   weight columns side by side; no tile is split.  These launches may use
//   512-column tiles (8 waves of 128 x 64), which halve the LDS reads of x
//   per MFMA, and stage whole fp16 output tiles through 20 KiB of LDS so that
//   each store writes 16 rows x 64 bytes; for groups whose M is at most 32
//   (down to M = 2), 32 x 512 tiles (one 32-row fragment per wave): then the
//   kernel is a weight stream whose x rows are shared in LDS; and for groups
//   whose M is at most 64, 64 x 512 tiles (two 32-row fragments per wave),
//   half the MFMA work of 128-row tiles.  The ring has three slots where
//   three fit the 160 KiB of LDS beside the staging (32 x 512 tiles with fp16
//   scales at bs >= 32 or fp32 scales at bs >= 64), else two (128- and
//   64-row 512-column tiles, and 32-row tiles with fp32 scales at bs 32 or
//   fp16 scales at bs 16).
// Logical workgroup ids are laid out XCD-contiguous, so neighbouring
// workgroups (which share tiles and weight columns) sit on the same XCD.
#include <algorithm>

#include "mnb_device.h"

namespace mnb {

constexpr int kSkBM = 128;          // rows per tile
constexpr int kSkWaves = 8;         // two per SIMD
constexpr int kSkNTW = kGemmNTW;    // n-tiles (16 rows of W) per wave: 32 columns
constexpr int kSkBN = kSkWaves * kSkNTW * kTileRows;   // 256 columns per tile
constexpr int kSkWideNTW = kGemmWideNTW;   // wide tiles (tile-list launches only): 64 columns per wave, 512 per tile
constexpr int kSkFM = kSkBM / 32;   // 32-row A fragments per wave
constexpr int kSkSkinnyFM = kGemmSkinnyFM;   // skinny tiles (tile-list launches only): 32 rows
constexpr int kSkHalfFM = kGemmHalfFM;       // half-height tiles (tile-list launches only): 64 rows
// Epilogue staging of 512-column tiles: per wave one 32 x 32 fp16 block,
// rows padded to 80 bytes against bank conflicts.
constexpr int kSkStageRow = 80, kSkStageWave = 32 * kSkStageRow, kSkStageBytes = kSkWaves * kSkStageWave;
constexpr int kSkThreads = 64 * kSkWaves;
static_assert(kSkPartialFloats == kSkBM * kSkBN, "one fp32 partial tile, [kSkBM][kSkBN] row-major");
constexpr int kSkReduceThreads = 256;             // each thread: 4 rows x 4 columns

typedef float float16_t __attribute__((ext_vector_type(16)));
// LDS staging of the epilogue is written in 8-byte and read in 16-byte
// pieces: both types may alias anything, so the compiler keeps every store
// and never moves a read above the stores it depends on.
typedef uint32_t u32x2_alias_t __attribute__((ext_vector_type(2), may_alias));
typedef uint32_t u32x4_alias_t __attribute__((ext_vector_type(4), may_alias));

__device__ __forceinline__ float16_t mfma32x32x16(half8_t a, half8_t b, float16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// The launch's parameters: its items and how their iterations are shared.
// Stream-K order (seq == nullptr): the items' tiles follow one another in
// group order, tile t of an item covering m-tile t % MT and n-group t / MT,
// and logical workgroup g owns iterations [g I / G, (g + 1) I / G).
// Tile-list order (seq != nullptr): the tiles are listed in seq, workgroup
// after workgroup, and logical workgroup g owns the tiles seq[wg[g].pos ..]
// with iterations [wg[g].iter, wg[g + 1].iter): whole tiles, or parts of a
// tile cut along K (stages [st0, st0 + nst)), each written as the fp32
// partial tile ws[part] for the reduce kernel.
struct SkParams {
    SkItem one;             // the item when count == 1 (a single product)
    const SkItem *items;    // device table of count items (count > 1), ibeg ascending
    const SkTile *seq;      // tile-list order: the tiles, workgroup-major (else nullptr)
    const SkRange *wg;      // tile-list order: G + 1 workgroup starts
    int32_t count;
    int32_t closed;         // 1: tile-list order of the single item `one` in closed form (sk_cf_*), no table
    int32_t G;              // workgroups
    int32_t I;              // iterations of all items (below 2^31)
    float *ws;              // partial tiles: stream-K [G][2] (slot 0 for a workgroup's first tile, 1 for its
                            // last); tile list [part]
};

// Item i (uniform index).  The table is read through the constant address
// space: it is never written by the kernel, so these are scalar loads and the
// fields stay in scalar registers.
__device__ __forceinline__ SkItem sk_item(const SkParams &p, int i) {
    if (p.count == 1) return p.one;
    static_assert(sizeof(SkItem) % 4 == 0, "dword copy");
    const __attribute__((address_space(4))) uint32_t *src =
        (const __attribute__((address_space(4))) uint32_t *)(p.items + i);
    SkItem r;
    uint32_t *dst = (uint32_t *)&r;
#pragma unroll
    for (int k = 0; k < (int)(sizeof(SkItem) / 4); ++k) dst[k] = src[k];
    return r;
}

// Item that owns iteration i (binary search over the items' first iterations).
__device__ __forceinline__ int sk_find_item(const SkParams &p, int i) {
    if (p.count == 1) return 0;
    int lo = 0, hi = p.count - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (((const __attribute__((address_space(4))) SkItem *)p.items)[mid].ibeg <= i) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// Entry i of the tile list (uniform index, scalar load).
__device__ __forceinline__ SkTile sk_seq(const SkParams &p, int i) {
    const __attribute__((address_space(4))) SkTile *s = (const __attribute__((address_space(4))) SkTile *)p.seq;
    SkTile e;
    e.item = s[i].item;
    e.t = s[i].t;
    e.st0 = s[i].st0;
    e.nst = s[i].nst;
    e.part = s[i].part;
    return e;
}

__device__ __forceinline__ SkRange sk_wg(const SkParams &p, int g) {
    const __attribute__((address_space(4))) SkRange *s = (const __attribute__((address_space(4))) SkRange *)p.wg;
    SkRange r;
    r.pos = s[g].pos;
    r.iter = s[g].iter;
    return r;
}

// first iteration of logical workgroup g (g = G gives I)
__device__ __forceinline__ int sk_start(int g, const SkParams &p) {
    if (p.seq) return sk_wg(p, g).iter;
    if (p.closed) return sk_cf_first(p.one.T, p.G, g) * p.one.ST;
    return (int)((int64_t)g * p.I / p.G);
}

// A cursor over the launch's tiles is item ci (fields ic), tile t of that
// item, its stages [st0, end) and partial tile `part` (-1 for a whole tile
// and in stream-K order, where the workgroup's range decides; a tile list
// has parts only in the PARTS kernels) and, in tile-list order, the list
// position pos (closed form: the workgroup's own tile count so far, its
// tiles at block-order positions cf_base + pos * cf_step).  Steps it to the
// next tile of the launch (the caller knows there is one).
template <bool PARTS>
__device__ __forceinline__ void sk_next_tile(const SkParams &p, int &ci, int &t, int &pos, SkItem &ic, int cf_base,
                                             int cf_step, int &st0, int &end, int &part) {
    if (p.closed) {
        ++pos;
        t = sk_cf_tile(ic.MT, ic.T / ic.MT, cf_base + pos * cf_step);
        st0 = 0;
        end = ic.ST;
        part = -1;
    } else if (p.seq) {
        const SkTile e = sk_seq(p, ++pos);
        if (e.item != ci) {
            ci = e.item;
            ic = sk_item(p, ci);
        }
        t = e.t;
        if constexpr (PARTS) {
            st0 = e.st0;
            end = e.st0 + e.nst;
            part = e.part;
        } else {
            st0 = 0;
            end = ic.ST;
            part = -1;
        }
    } else {
        if (++t == ic.T) {
            t = 0;
            ic = sk_item(p, ++ci);
        }
        st0 = 0;
        end = ic.ST;
        part = -1;
    }
}

// k extent and first stage of the tile after the cursor's (the caller knows
// there is one).
template <bool PARTS>
__device__ __forceinline__ int sk_next_kx(const SkParams &p, int ci, int t, int pos, const SkItem &ic, int &st0) {
    st0 = 0;
    if (p.closed) return ic.kx;
    if (p.seq) {
        const SkTile e = sk_seq(p, pos + 1);
        if constexpr (PARTS) st0 = e.st0;
        return e.item == ci ? ic.kx : sk_item(p, e.item).kx;
    }
    return t + 1 < ic.T ? ic.kx : sk_item(p, ci + 1).kx;
}

// logical workgroup owning iteration i
__device__ __forceinline__ int sk_owner(int i, const SkParams &p) {
    int g = (int)((int64_t)i * p.G / p.I);
    while (g + 1 < p.G && sk_start(g + 1, p) <= i) ++g;
    while (g > 0 && sk_start(g, p) > i) --g;
    return g;
}

// Four consecutive outputs y[m, n..n+3] (=|+=) v, m < M checked by the
// caller; columns >= N are dropped.  One 8-byte (fp16) or 16-byte (fp32)
// store when the row segment is whole and aligned.
__device__ __forceinline__ void store_y4(const SkItem &p, int m, int n, float4_t v) {
    const size_t idx = (size_t)m * p.N + n;
    const bool acc = p.accumulate != 0;
    if (p.y_vec && n + 3 < p.N) {
        if (p.y_f16) {
            __attribute__((address_space(1))) u32x2_t *q = (__attribute__((address_space(1))) u32x2_t *)((_Float16 *)p.y + idx);
            if (acc) {
                const u32x2_t o = *q;
                const half2_t o0 = as_half2(o[0]), o1 = as_half2(o[1]);
                v[0] += (float)o0[0];
                v[1] += (float)o0[1];
                v[2] += (float)o1[0];
                v[3] += (float)o1[1];
            }
            half2_t h0, h1;
            h0[0] = (_Float16)v[0];
            h0[1] = (_Float16)v[1];
            h1[0] = (_Float16)v[2];
            h1[1] = (_Float16)v[3];
            *q = (u32x2_t){as_u32(h0), as_u32(h1)};
        } else {
            __attribute__((address_space(1))) float4_t *q = (__attribute__((address_space(1))) float4_t *)((float *)p.y + idx);
            if (acc) v += *q;
            *q = v;
        }
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (n + e < p.N) {
                if (p.y_f16) store_y<true>(p.y, idx + e, v[e], acc);
                else store_y<false>(p.y, idx + e, v[e], acc);
            }
        }
    }
}


// Ring slot layout (bytes) for one stage, and the direct loads that fill it.
template <typename ScaleT, bool HAS_ZP, int SPS, int NTW, int FM>
struct SkSlot {
    static constexpr int BM = 32 * FM;                              // rows per tile
    static constexpr int ZB = SPS <= 2 ? 1 : SPS / 2;
    static constexpr int kNT = kSkWaves * NTW;                      // n-tiles per tile (16 or 32)
    static constexpr int kX = 0;                                    // x tile [128][16 chunks]
    static constexpr int kQ = BM * kTileK * 2;                      // packed tiles [16][64 lanes][16 B] after the x tile
    static constexpr int kWin = 1024;                               // bytes of one 64-lane direct load
    static constexpr int kS = kQ + kNT * kTileBytes;                // scales [16 tiles][16 rows][SPS]
    static constexpr int kTileS = kTileRows * SPS * (int)sizeof(ScaleT);   // scale bytes per tile
    static constexpr int kSRegion = kNT * kTileS > kWin ? kNT * kTileS : kWin;   // padded to one window
    static constexpr int kZ = kS + kSRegion;                        // zero points [16 tiles][16 rows][ZB]
    static constexpr int kTileZ = kTileRows * ZB;
    static constexpr int kZRegion = HAS_ZP ? (kNT * kTileZ > kWin ? kNT * kTileZ : kWin) : 0;
    static constexpr int kBytes = kZ + kZRegion;
    // ring slots: three when they fit the 160 KiB LDS beside the epilogue
    // staging of 512-column tiles, else two (the staging pays more than a
    // third slot: 64 x 512 tiles at K = 896, 113 -> 100 us per Qwen step)
    static constexpr int kDepth = 3 * kBytes + (NTW == kSkWideNTW ? kSkStageBytes : 0) <= 160 * 1024 ? 3 : 2;
    // per wave and stage: x pieces of 4 rows, its packed tiles, and one
    // 1 KiB window each of the scale and zero-point regions that contains
    // the wave's own tiles (all 64 lanes load: no lane mask, no branch)
    static constexpr int kXDma = BM * kTileK * 2 / kWin / kSkWaves;
    static constexpr int kDma = kXDma + NTW + 1 + (HAS_ZP ? 1 : 0);
    static_assert(kTileS % 16 == 0 && kTileZ % 16 == 0, "16-byte pieces");
    static_assert(NTW * kTileS <= kWin && NTW * kTileZ <= kWin, "a wave's scales fit one window");
};

// PARTS: a tile list with parts (tiles cut along K, written as partial
// tiles); the other launches (stream-K, closed form, whole-tile lists) run
// the kernel without the parts' bookkeeping.
template <typename ScaleT, bool HAS_ZP, int SPS, int NTW, int FM, bool PARTS>
__global__ __launch_bounds__(kSkThreads, 1) void gemm_sk_kernel(SkParams p) {
    using L = SkSlot<ScaleT, HAS_ZP, SPS, NTW, FM>;
    constexpr int BM = L::BM;                        // rows per tile (128, 64, or 32 for skinny tiles)
    constexpr int BN = kSkWaves * NTW * kTileRows;   // columns per tile
    constexpr int FN = NTW / 2;                      // 32-column weight fragments per wave
    constexpr int ZB = L::ZB;
    constexpr int D = L::kDepth;
    __shared__ __align__(1024) unsigned char ring[D][L::kBytes];
    // Epilogue staging (512-column tiles, where the LDS has room)
    constexpr int kStageRow = kSkStageRow, kStageWave = kSkStageWave;
    constexpr bool kStaged = NTW == kSkWideNTW && D * L::kBytes + kSkStageBytes <= 160 * 1024;
    __shared__ __align__(16) unsigned char stage_all[kStaged ? kSkStageBytes : 16];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c32 = lane & 31, h = lane >> 5;   // MFMA row/column and k half
    // XCD-contiguous logical id: physical workgroup b runs on XCD b % 8
    const int per_xcd = p.G / 8;
    const int g = (p.G % 8 == 0) ? (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8) : (int)blockIdx.x;
    const int i0 = sk_start(g, p), i1 = sk_start(g + 1, p);
    if (i0 >= i1) return;
    // compute cursor: the tile (item fields ic, tile t of the item), the
    // stage cst of the tile and the end cend of the tile's stages in this
    // entry (the partial tile of a tile-list part is read from the list in
    // the epilogue)
    int ci, t, cpos, cst, cend = 0;
    const int cf_base = p.closed ? sk_cf_base(p.one.T, p.G, g) : 0, cf_step = sk_cf_step(p.G);
    if (p.closed) {
        cpos = 0;
        ci = 0;
        t = sk_cf_tile(p.one.MT, p.one.T / p.one.MT, cf_base);
        cst = 0;
    } else if (p.seq) {
        cpos = sk_wg(p, g).pos;
        const SkTile e = sk_seq(p, cpos);
        ci = e.item;
        t = e.t;
        cst = PARTS ? e.st0 : 0;
        cend = e.st0 + e.nst;
    } else {
        cpos = 0;
        ci = sk_find_item(p, i0);
    }
    SkItem ic = sk_item(p, ci);
    if (!p.seq && !p.closed) {
        t = (i0 - ic.ibeg) / ic.ST;
        cst = (i0 - ic.ibeg) - t * ic.ST;
    }
    if (!PARTS || !p.seq) cend = ic.ST;

    const uint32_t k6400 = vgpr_const(0x64006400u);
    const uint32_t ring0 = __builtin_amdgcn_readfirstlane(lds_addr(&ring[0][0]));

    // ---- issue: all operands of one stage into one ring slot ----
    // The issue cursor (tile lt, stage lst) stops at this workgroup's last
    // iteration, so every stage issues the same loads (the final ones re-load
    // the last stage into a slot nobody reads).  Lane byte offsets are set
    // per tile; a stage only moves the scalar bases.  issue_dma is straight
    // -line code (no branch, no lane mask), so it can be interleaved with
    // MFMAs; advance moves the cursor.
    // Scales and zero points: the wave loads the 1 KiB window of the region
    // that starts at its own tiles, moved back to end at the region's end;
    // waves write identical bytes where windows overlap, and lanes past the
    // workgroup's 16 n-tiles fill the padding.
    constexpr int s_win_max = L::kSRegion - L::kWin;
    constexpr int z_win_max = L::kZRegion - L::kWin;
    const int s_win = min(wave * NTW * L::kTileS, s_win_max);
    const int z_win = HAS_ZP ? min(wave * NTW * L::kTileZ, z_win_max) : 0;
    // issue cursor: the tile (item fields iq, tile lt of the item), stage lst
    // (of the entry's stages up to lend), iteration li
    int ii = ci, lt = t, ipos = cpos, lst = cst, lend = cend, li = i0, lslot = 0;
    SkItem iq = ic;
    uint32_t xrow[L::kXDma], xcolk[L::kXDma], qoff[NTW], soff = 0, zoff = 0;
    auto set_tile = [&]() __attribute__((always_inline)) {
        const int m0 = (lt % iq.MT) * BM, ntg = (lt / iq.MT) * L::kNT, nt0 = ntg + wave * NTW;
#pragma unroll
        for (int u = 0; u < L::kXDma; ++u) {
            const int row = (wave * L::kXDma + u) * 4 + (lane >> 4);
            xrow[u] = (uint32_t)min(m0 + row, iq.M - 1) * (uint32_t)iq.ldx * 2u;
            xcolk[u] = (uint32_t)(((lane & 15) ^ (row & 15)) * 8);   // k of the chunk this lane loads
        }
#pragma unroll
        for (int b = 0; b < NTW; ++b)
            qoff[b] = ((uint32_t)min(nt0 + b, iq.NT - 1) * (uint32_t)iq.ST * 64u + (uint32_t)lane) * 16u;
        {
            const int byte = s_win + lane * 16;
            soff = (uint32_t)min(ntg + byte / L::kTileS, iq.NT - 1) * (uint32_t)iq.ST * L::kTileS +
                   (uint32_t)(byte % L::kTileS);
        }
        if constexpr (HAS_ZP) {
            const int byte = z_win + lane * 16;
            zoff = (uint32_t)min(ntg + byte / L::kTileZ, iq.NT - 1) * (uint32_t)iq.ST * L::kTileZ +
                   (uint32_t)(byte % L::kTileZ);
        }
    };
    set_tile();
    // x piece u of this wave (4 rows); chunks at k >= kx (a k tail) re-read
    // the row's last chunk, stay inside x, and are zeroed in LDS on landing
    auto dma_x = [&](uint32_t base, int u) __attribute__((always_inline)) {
        const uint32_t k = (uint32_t)min(lst * kTileK + (int)xcolk[u], iq.kx - 8);
        dma16(base + L::kX + (uint32_t)(wave * L::kXDma + u) * 1024u, xrow[u] + k * 2u, iq.x);
    };
    auto dma_q = [&](uint32_t base, int b) __attribute__((always_inline)) {
        const unsigned char *qb = (const unsigned char *)iq.q_t + (size_t)lst * kTileBytes;
        dma16(base + L::kQ + (uint32_t)(wave * NTW + b) * kTileBytes, qoff[b], qb);
    };
    auto dma_sz = [&](uint32_t base) __attribute__((always_inline)) {
        dma16(base + L::kS + (uint32_t)s_win, soff, (const unsigned char *)iq.s_t + (size_t)lst * L::kTileS);
        if constexpr (HAS_ZP) dma16(base + L::kZ + (uint32_t)z_win, zoff, iq.zp_t + (size_t)lst * L::kTileZ);
    };
    auto slot_base = [&]() __attribute__((always_inline)) { return ring0 + (uint32_t)(lslot * L::kBytes); };
    auto advance = [&]() __attribute__((always_inline)) {
        if (li + 1 < i1) {
            ++li;
            if (++lst == (PARTS ? lend : iq.ST)) {
                int lpart;
                sk_next_tile<PARTS>(p, ii, lt, ipos, iq, cf_base, cf_step, lst, lend, lpart);
                set_tile();
            }
        }
        lslot = lslot == D - 1 ? 0 : lslot + 1;
    };
    auto issue = [&]() __attribute__((always_inline)) {
        const uint32_t base = slot_base();
#pragma unroll
        for (int u = 0; u < L::kXDma; ++u) dma_x(base, u);
#pragma unroll
        for (int b = 0; b < NTW; ++b) dma_q(base, b);
        dma_sz(base);
        advance();
    };

    // ---- land: wait for the oldest stage in flight, zero its x pieces at
    // k >= kx, and meet the other waves ----
    bool drain = false;   // set after y stores: stores and loads may complete out of order
    bool first_seg = true;   // the segment being computed is this workgroup's first (partial slot 0)
    auto land = [&](int slot, int st, int kx) __attribute__((always_inline)) {
        if (drain || D == 2) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            drain = false;
        } else {
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(L::kDma) : "memory");   // only the newest stage in flight
        }
        if ((st + 1) * kTileK > kx) {
            unsigned char *xs = &ring[slot][L::kX];
#pragma unroll
            for (int u = 0; u < L::kXDma; ++u) {
                const int row = (wave * L::kXDma + u) * 4 + (lane >> 4);
                const int chunk = (lane & 15) ^ (row & 15);
                if (st * kTileK + chunk * 8 >= kx)
                    *(u32x4_t *)(xs + (wave * L::kXDma + u) * 1024 + lane * 16) = (u32x4_t){0u, 0u, 0u, 0u};
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };

    float16_t acc[FM][FN];
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int f = 0; f < FN; ++f)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[a][f][v] = 0.f;

    // ---- epilogue of tile t after nst of its stages ----
    // Fragment (a, f), register v of lane (c32, h): row a * 32 + c32 of the
    // tile, column 32 f + 8 (v / 4) + 4 h + v % 4 of the wave's 32 columns.
    auto epilogue = [&](int nst) __attribute__((always_inline)) {
        // undo the stored scales' 2^fold_exp (exact), for whole and partial tiles alike
#pragma unroll
        for (int a = 0; a < FM; ++a)
#pragma unroll
            for (int f = 0; f < FN; ++f)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[a][f][v] *= ic.unfold;
        const int m0 = (t % ic.MT) * BM, ng = t / ic.MT;
        const int c_wave = wave * NTW * kTileRows;   // first column of this wave in the tile
        if (nst == ic.ST) {
            const int n_wave = ng * BN + c_wave;
            // The common case: the wave's 128 x (16 NTW) block lies inside y,
            // rows are 4-element aligned and y is overwritten.  Then every
            // lane writes its four rows with one address each and immediate
            // offsets, without per-group tests.
            const bool whole = ic.y_vec && !ic.accumulate && m0 + BM <= ic.M && n_wave + NTW * kTileRows <= ic.N;
            const bool staged = kStaged && whole && ic.y_f16 && ic.N % 8 == 0 && ((uintptr_t)ic.y & 15) == 0;
            if (staged) {
                // Per 32 x 32 block: each lane's four 4-column pieces of its
                // row go to the wave's LDS block, then every lane reads 16
                // contiguous bytes, so 4 lanes cover a row's 64 bytes and one
                // store writes 16 rows x 64 bytes (the direct stores write 32
                // rows x 16 bytes).  The wave's LDS operations run in order,
                // so the reads see the writes and the next block's writes
                // follow the reads.
                unsigned char *sb = stage_all + wave * kStageWave;
#pragma unroll
                for (int a = 0; a < FM; ++a)
#pragma unroll
                    for (int f = 0; f < FN; ++f) {
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            half2_t h0, h1;
                            h0[0] = (_Float16)acc[a][f][4 * j];
                            h0[1] = (_Float16)acc[a][f][4 * j + 1];
                            h1[0] = (_Float16)acc[a][f][4 * j + 2];
                            h1[1] = (_Float16)acc[a][f][4 * j + 3];
                            *(u32x2_alias_t *)(sb + c32 * kStageRow + (8 * j + 4 * h) * 2) =
                                (u32x2_alias_t){as_u32(h0), as_u32(h1)};
                        }
                        asm volatile("" ::: "memory");   // the reads below follow the writes
#pragma unroll
                        for (int k = 0; k < 2; ++k) {
                            const int r = (lane >> 2) + 16 * k, cc = lane & 3;
                            const u32x4_alias_t v = *(const u32x4_alias_t *)(sb + r * kStageRow + cc * 16);
                            *(__attribute__((address_space(1))) u32x4_t *)((_Float16 *)ic.y +
                                (size_t)(m0 + a * 32 + r) * ic.N + n_wave + f * 32 + cc * 8) = (u32x4_t)v;
                        }
                        asm volatile("" ::: "memory");   // the next block's writes follow these reads
                    }
            } else if (whole) {
#pragma unroll
                for (int a = 0; a < FM; ++a) {
                    const size_t row = (size_t)(m0 + a * 32 + c32) * ic.N + n_wave + 4 * h;
                    if (ic.y_f16) {
                        __attribute__((address_space(1))) u32x2_t *q =
                            (__attribute__((address_space(1))) u32x2_t *)((_Float16 *)ic.y + row);
#pragma unroll
                        for (int f = 0; f < FN; ++f)
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                half2_t h0, h1;
                                h0[0] = (_Float16)acc[a][f][4 * j];
                                h0[1] = (_Float16)acc[a][f][4 * j + 1];
                                h1[0] = (_Float16)acc[a][f][4 * j + 2];
                                h1[1] = (_Float16)acc[a][f][4 * j + 3];
                                q[(f * 32 + 8 * j) / 4] = (u32x2_t){as_u32(h0), as_u32(h1)};
                            }
                    } else {
                        __attribute__((address_space(1))) float4_t *q =
                            (__attribute__((address_space(1))) float4_t *)((float *)ic.y + row);
#pragma unroll
                        for (int f = 0; f < FN; ++f)
#pragma unroll
                            for (int j = 0; j < 4; ++j)
                                q[(f * 32 + 8 * j) / 4] = (float4_t){acc[a][f][4 * j], acc[a][f][4 * j + 1],
                                                                     acc[a][f][4 * j + 2], acc[a][f][4 * j + 3]};
                    }
                }
            } else {
#pragma unroll
                for (int a = 0; a < FM; ++a) {
                    const int m = m0 + a * 32 + c32;
                    if (m < ic.M) {
#pragma unroll
                        for (int f = 0; f < FN; ++f)
#pragma unroll
                            for (int j = 0; j < 4; ++j)
                                store_y4(ic, m, n_wave + f * 32 + 8 * j + 4 * h,
                                         (float4_t){acc[a][f][4 * j], acc[a][f][4 * j + 1], acc[a][f][4 * j + 2],
                                                    acc[a][f][4 * j + 3]});
                    }
                }
            }
        } else if constexpr (PARTS ? BM * BN <= kSkPartialFloats : NTW == kSkNTW && FM == kSkFM) {
            // partial tile of a split tile: [BM][BN] fp32, summed by sk_reduce_kernel
            // (stream-K, 128 x 256 tiles only: this workgroup's slot; a tile list with
            // parts: the entry's part); rows past M are neither stored nor summed
            const size_t pidx = PARTS ? (size_t)sk_seq(p, cpos).part : (size_t)g * 2 + (first_seg ? 0 : 1);
            __attribute__((address_space(1))) float *part =
                (__attribute__((address_space(1))) float *)p.ws + pidx * kSkPartialFloats;
#pragma unroll
            for (int a = 0; a < FM; ++a)
                if (m0 + a * 32 + c32 < ic.M) {
#pragma unroll
                    for (int f = 0; f < FN; ++f)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            *(__attribute__((address_space(1))) float4_t *)(part + (a * 32 + c32) * BN + c_wave +
                                                                             f * 32 + 8 * j + 4 * h) =
                                (float4_t){acc[a][f][4 * j], acc[a][f][4 * j + 1], acc[a][f][4 * j + 2],
                                           acc[a][f][4 * j + 3]};
                }
        }
#pragma unroll
        for (int a = 0; a < FM; ++a)
#pragma unroll
            for (int f = 0; f < FN; ++f)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[a][f][v] = 0.f;
        drain = true;
        first_seg = false;
    };

    // ---- main loop: segments of one tile, one stage per inner trip ----
    // The epilogue sits outside the stage loop, so the accumulators stay in
    // the MFMA registers across stages.  A stage is: the head (DMA issue of
    // stage + 2, the stage's raw weights, scales and zero points, step 0's x
    // fragments and dequant), steps 0..5 (MFMAs of step s while step s + 1's
    // operands are read and dequantized), step 7's x fragments read into
    // registers, the barrier that lands the next stage, and then the MFMAs
    // of steps 6 and 7 issued together with the DMAs of a later stage and
    // step 7's dequantization, before the next stage's head, so the matrix
    // core keeps running through the barrier.  Nothing reads a slot
    // after the barrier that follows its last stage, so the DMA that the next
    // head issues into it is safe.
    //
    // B fragment f covers local n-tiles 4 wave + 2 f + {0, 1}; lane (c32, h)
    // needs, at 16-k step s, the 8 nibbles of row c32 % 16 of tile c32 / 16 at
    // k-group 2 s + h: word s / 2 of tile lane ((2 s + h) % 4) * 16 + c32 % 16.
    // Two 16-byte reads per fragment hold all of them: qb[f][0] for even s,
    // qb[f][1] for odd s.
    u32x4_t qb[FN][2];
    ScaleT sc[FN][SPS];
    uint32_t zb[FN];
    auto load_stage = [&](int slot) __attribute__((always_inline)) {
        const unsigned char *sl = ring[slot];
#pragma unroll
        for (int f = 0; f < FN; ++f) {
            const int ntl = wave * NTW + 2 * f + (c32 >> 4);
            const unsigned char *qt = sl + L::kQ + ntl * kTileBytes;
            qb[f][0] = *(const u32x4_t *)(qt + (h * 16 + (c32 & 15)) * 16);
            qb[f][1] = *(const u32x4_t *)(qt + ((2 + h) * 16 + (c32 & 15)) * 16);
            const ScaleT *sp = (const ScaleT *)(sl + L::kS + ntl * L::kTileS) + (c32 & 15) * SPS;
#pragma unroll
            for (int e = 0; e < SPS; ++e) sc[f][e] = sp[e];
            if constexpr (HAS_ZP) {
                const unsigned char *zp = sl + L::kZ + ntl * L::kTileZ + (c32 & 15) * ZB;
                uint32_t z = 0;
#pragma unroll
                for (int e = 0; e < ZB; ++e) z |= (uint32_t)zp[e] << (8 * e);
                zb[f] = z;
            } else {
                zb[f] = 0x88888888u;
            }
        }
    };
    auto read_x = [&](half8_t(&af)[FM], int slot, int s) __attribute__((always_inline)) {
        // row a * 32 + c32 (row & 15 == c32 & 15), k-chunk 2 s + h
        const _Float16 *xs = (const _Float16 *)(ring[slot] + L::kX);
#pragma unroll
        for (int a = 0; a < FM; ++a)
            af[a] = *(const half8_t *)(xs + (a * 32 + c32) * kTileK + (((2 * s + h) ^ (c32 & 15)) * 8));
    };
    auto dequant = [&](half8_t(&bf)[FN], int s) __attribute__((always_inline)) {
        const int si = s * SPS / 8;   // scale block of k-group 2 s + h (same for both h)
#pragma unroll
        for (int f = 0; f < FN; ++f) {
            const uint32_t z = HAS_ZP ? zp_nibble(zb[f], si) : 8u;
            half8_t w = unpack_q_minus_zp(qb[f][s & 1][s >> 1], bias_lo_pair(z), bias_hi_pair(z), k6400);
            if constexpr (sizeof(ScaleT) == 2) {
                w = w * (_Float16)sc[f][si];
            } else {
                const float sf = (float)sc[f][si];
#pragma unroll
                for (int e = 0; e < 8; ++e) w[e] = (_Float16)((float)w[e] * sf);
            }
            bf[f] = w;
        }
    };
    auto mfma_step = [&](const half8_t(&af)[FM], const half8_t(&bf)[FN]) __attribute__((always_inline)) {
#pragma unroll
        for (int a = 0; a < FM; ++a)
#pragma unroll
            for (int f = 0; f < FN; ++f) acc[a][f] = mfma32x32x16(bf[f], af[a], acc[a][f]);
    };
    int cslot = 0;                           // ring slot of the stage being computed
    constexpr int kSteps = kTileK / 16;      // 8 MFMA k-steps per stage
    half8_t af[2][FM], bf[2][FN];      // steps 0..6, alternating
    half8_t af7[FM], bf7[FN];          // step 7: x read before the barrier, weights dequantized in the tail
    auto head_reads = [&]() __attribute__((always_inline)) {
        load_stage(cslot);
        read_x(af[0], cslot, 0);
        dequant(bf[0], 0);
    };
    int remaining = i1 - i0;
    int seg_n = min(remaining, cend - cst);   // stages of tile t done by this workgroup
    issue();                                   // stages 0 and 1 (three-slot ring: and 2)
    issue();
    land(0, cst, ic.kx);
    if (D == 3) issue();
    head_reads();
    int kk = 0;                                // stages of the current segment done
    while (true) {
#pragma unroll
        for (int s = 0; s + 2 < kSteps; ++s) {
            read_x(af[(s + 1) & 1], cslot, s + 1);
            dequant(bf[(s + 1) & 1], s + 1);
            mfma_step(af[s & 1], bf[s & 1]);
            // order within the step: the next step's dequant VALU fills the
            // shadow of the first MFMAs, and the next step's x reads go out
            // between the last FM MFMAs (same box, M=512 group: +2.4% over
            // issuing the x reads first).  VALU per MFMA: 5 + 2 for 128 x 512
            // tiles; 7 + 6 for 64 x 512 tiles, which place all 26 of a step
            // (+1.2% on the M=64 groups over 4 + 3); 4 + 3 for the others
            // (32-row groups lose with 5 + 2 or with all 26 placed)
            constexpr bool kWide128 = FM == kSkFM && NTW == kSkWideNTW, kWide64 = FM == kSkHalfFM && NTW == kSkWideNTW;
            constexpr int kVa = kWide128 ? 5 : kWide64 ? 7 : 4;
            constexpr int kVb = kWide128 ? 2 : kWide64 ? 6 : 3;
#pragma unroll
            for (int i = 0; i < FM * FN - FM; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);     // MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, kVa, 0);   // VALU
            }
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);     // MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);     // DS read
                __builtin_amdgcn_sched_group_barrier(0x002, kVb, 0);   // VALU
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // af[0], bf[0] hold step 6; step 7 goes to its own registers
        read_x(af7, cslot, kSteps - 1);   // step 7's weights are dequantized in the tail
        cslot = cslot == D - 1 ? 0 : cslot + 1;
        // the stage to land: the next of this segment, else the first of the
        // next tile (of this item or the next); after the last stage of the
        // range it is a re-load nobody reads
        int nkx = ic.kx;
        if (kk + 1 < seg_n) {
            ++cst;
        } else {
            cst = 0;
            if (remaining > seg_n) nkx = sk_next_kx<PARTS>(p, ci, t, cpos, ic, cst);
        }
        land(cslot, cst, nkx);
        // MFMAs of steps 6 and 7 with the DMA of a later stage between them,
        // then the next stage's head (at the end of the range these load and
        // read stages nobody uses: the issue cursor stays on the last one)
        {
            const uint32_t base = slot_base();
            // the wave that has passed the barrier issues these first: the
            // SIMD's other wave is still in its own tail or stage (+0.7%)
            __builtin_amdgcn_s_setprio(1);
            // the DMAs spread over the tail MFMAs: after every second one
            // for 128 x 512 tiles, after every one for the others (those
            // left after the last MFMA follow it); step 7's dequantization
            // after the fourth step-6 MFMA (the last one for skinny tiles),
            // where the matrix core hides it (same box: +1.7% on the M=512
            // group, +1-2% on the M <= 64 groups against issuing it before
            // the barrier with one DMA per MFMA)
            constexpr int kTailMfma = 2 * FM * FN, kTailDma = L::kXDma + NTW + 1;
            constexpr int kDmaGap = (FM == kSkFM && NTW == kSkWideNTW) ? 2 : 1;
            constexpr int kDq7 = FM * FN - 1 < 3 ? FM * FN - 1 : 3;
            auto dma_j = [&](int j) __attribute__((always_inline)) {
                if (j < L::kXDma) dma_x(base, j);
                else if (j < L::kXDma + NTW) dma_q(base, j - L::kXDma);
                else dma_sz(base);
            };
#pragma unroll
            for (int i = 0; i < kTailMfma; ++i) {
                const int a = (i / FN) % FM, f = i % FN;
                if (i < FM * FN) acc[a][f] = mfma32x32x16(bf[0][f], af[0][a], acc[a][f]);
                else acc[a][f] = mfma32x32x16(bf7[f], af7[a], acc[a][f]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < kTailDma; ++j)
                    if ((kDmaGap * j < kTailMfma ? kDmaGap * j : kTailMfma - 1) == i) dma_j(j);
                __builtin_amdgcn_sched_barrier(0);
                if (i == kDq7) dequant(bf7, kSteps - 1);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __builtin_amdgcn_s_setprio(0);
        advance();
        head_reads();
        if (++kk == seg_n) {
            remaining -= seg_n;
            epilogue(seg_n);
            if (remaining == 0) break;
            int st0, part;   // st0 equals cst, set when this stage landed
            sk_next_tile<PARTS>(p, ci, t, cpos, ic, cf_base, cf_step, st0, cend, part);
            seg_n = min(remaining, cend - st0);
            kk = 0;
        }
    }
    // drain every direct load before the workgroup's LDS is released
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Sums the partial tiles of every split tile in contributor order and writes
// y.  The tiles are BM x BN ([BM][BN] fp32 partial tiles); workgroup (j, rb)
// reduces rows [rb * RB, +RB) of split tile j of the list (RB = 16 rows of
// 256 columns or 8 of 512); each thread owns four rows of one 4-column group
// and keeps the loads of up to kBatch contributors (4 kBatch 16-byte loads)
// in flight before it adds them in contributor order.
template <int BM, int BN>
__global__ __launch_bounds__(kSkReduceThreads) void sk_reduce_kernel(SkParams p, SkSplitList list) {
    constexpr int RB = kSkReduceThreads * 16 / BN;
    constexpr int kRowBlocks = BM / RB;
    constexpr int kColGroups = BN / 4;
    constexpr int kRowsPerThread = RB * kColGroups / kSkReduceThreads;
    constexpr int kRowStep = kSkReduceThreads / kColGroups;
    constexpr int kBatch = 8;
    static_assert(kRowsPerThread == 4 && BM % RB == 0 && BM * BN <= kSkPartialFloats, "reduce shape");
    const SkSplit e = list.e[blockIdx.x / kRowBlocks];
    const int rb = (int)blockIdx.x % kRowBlocks;
    const uint32_t flags = (uint32_t)e.t_slot;
    const int t = (int)(flags & kSkSplitTile);
    const bool parts = (flags & kSkSplitParts) != 0;
    const size_t slot0 = (flags & kSkSplitSlot1) ? 1 : 0;
    const SkItem it = sk_item(p, e.item);
    const int first = e.first, nc = (int)e.last - (int)e.first + 1;
    const int tid = (int)threadIdx.x;
    const int c = (tid % kColGroups) * 4;
    const int r0 = rb * RB + tid / kColGroups;
    const int m0 = (t % it.MT) * BM, n = (t / it.MT) * BN + c;
    // rows past M hold no partial sums (the GEMM does not store them): a
    // workgroup whose rows all lie past M has nothing to do; in the block
    // that M cuts, the loads of rows past M read values that are never stored
    if (n >= it.N || m0 + rb * RB >= it.M) return;
    auto part = [&](int i, int k) __attribute__((always_inline)) {
        // tile list: the parts' partial tiles in K order; stream-K: the
        // contributors' slots (the first one's slot0, the others' slot 0)
        const size_t pt = parts ? (size_t)(first + i) : (size_t)(first + i) * 2 + (i == 0 ? slot0 : 0);
        return gld((const float4_t *)(p.ws + pt * kSkPartialFloats + (size_t)(r0 + k * kRowStep) * BN + c));
    };
    float4_t sum[kRowsPerThread];
    for (int i0 = 0; i0 < nc; i0 += kBatch) {
        const int nb = min(kBatch, nc - i0);
        float4_t v[kBatch][kRowsPerThread];
#pragma unroll
        for (int j = 0; j < kBatch; ++j)
            if (j < nb)
#pragma unroll
                for (int k = 0; k < kRowsPerThread; ++k) v[j][k] = part(i0 + j, k);
#pragma unroll
        for (int j = 0; j < kBatch; ++j)
            if (j < nb)
#pragma unroll
                for (int k = 0; k < kRowsPerThread; ++k) sum[k] = i0 + j == 0 ? v[j][k] : sum[k] + v[j][k];
    }
#pragma unroll
    for (int k = 0; k < kRowsPerThread; ++k) {
        const int m = m0 + r0 + k * kRowStep;
        if (m < it.M) store_y4(it, m, n, sum[k]);
    }
}

// The reduce launch over `list` for tiles of 32 fm rows x 128 ntw columns.
static hipError_t launch_reduce(int ntw, int fm, hipStream_t stream, const SkParams &p, const SkSplitList &list) {
    if (list.n <= 0) return hipSuccess;
    const int bm = 32 * fm, bn = 128 * ntw;
    const int blocks = list.n * (bm / (kSkReduceThreads * 16 / bn));
    if (bm == kSkBM && bn == kSkBN)
        hipLaunchKernelGGL((sk_reduce_kernel<kSkBM, kSkBN>), dim3(blocks), dim3(kSkReduceThreads), 0, stream, p, list);
    else if (bm == 32 * kSkHalfFM && bn == 128 * kSkWideNTW)
        hipLaunchKernelGGL((sk_reduce_kernel<32 * kSkHalfFM, 128 * kSkWideNTW>), dim3(blocks), dim3(kSkReduceThreads), 0,
                           stream, p, list);
    else if (bm == 32 * kSkSkinnyFM && bn == 128 * kSkWideNTW)
        hipLaunchKernelGGL((sk_reduce_kernel<32 * kSkSkinnyFM, 128 * kSkWideNTW>), dim3(blocks), dim3(kSkReduceThreads), 0,
                           stream, p, list);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

SkItem sk_make_item(const mnb_weight *w, const MatmulArgs &a, int32_t ibeg, int ntw, int fm) {
    const WeightGeom &g = w->g;
    SkItem it{};
    it.q_t = w->q_t;
    it.s_t = w->s_t;
    it.zp_t = (const uint8_t *)w->zp_t;
    it.x = (const void *)a.x;
    it.y = a.y;
    it.ldx = a.ldx;
    it.kx = a.kx;
    it.M = a.M;
    it.N = g.N;
    it.NT = g.NT;
    it.ST = g.ST;
    it.MT = (a.M + 32 * fm - 1) / (32 * fm);
    it.T = sk_tiles(a.M, g.NT, ntw, fm);
    it.y_f16 = a.y_type == MNB_F16;
    it.accumulate = a.accumulate;
    it.y_vec = (g.N % 4 == 0) && ((uintptr_t)a.y % (it.y_f16 ? 8 : 16) == 0);
    it.unfold = pow2f(-g.fold_exp);
    it.ibeg = ibeg;
    return it;
}

// The kernel of one weight variant at tile width ntw and height 32 fm (wide
// and skinny tiles exist for the variants whose four n-tiles of scales fit
// one 1 KiB window), with or without parts (never for 128 x 512 tiles).
template <typename ScaleT, bool HAS_ZP, int SPS, int NTW, int FM>
static void launch_sk_parts(bool parts, dim3 grid, dim3 block, hipStream_t stream, const SkParams &p) {
    if (parts)
        hipLaunchKernelGGL((gemm_sk_kernel<ScaleT, HAS_ZP, SPS, NTW, FM, true>), grid, block, 0, stream, p);
    else
        hipLaunchKernelGGL((gemm_sk_kernel<ScaleT, HAS_ZP, SPS, NTW, FM, false>), grid, block, 0, stream, p);
}
template <typename ScaleT, bool HAS_ZP, int SPS>
static void launch_sk_variant(int ntw, int fm, bool parts, dim3 grid, dim3 block, hipStream_t stream,
                              const SkParams &p) {
    if (ntw == kSkNTW) {
        launch_sk_parts<ScaleT, HAS_ZP, SPS, kSkNTW, kSkFM>(parts, grid, block, stream, p);
    } else if constexpr (kSkWideNTW * kTileRows * SPS * sizeof(ScaleT) <= 1024) {
        if (fm == kSkFM)
            hipLaunchKernelGGL((gemm_sk_kernel<ScaleT, HAS_ZP, SPS, kSkWideNTW, kSkFM, false>), grid, block, 0, stream, p);
        else if (fm == kSkHalfFM)
            launch_sk_parts<ScaleT, HAS_ZP, SPS, kSkWideNTW, kSkHalfFM>(parts, grid, block, stream, p);
        else
            launch_sk_parts<ScaleT, HAS_ZP, SPS, kSkWideNTW, kSkSkinnyFM>(parts, grid, block, stream, p);
    }
}

// Launches the GEMM over the items (count == 1: `one`, else the device table
// `items` with host copy `host`) and, when some workgroup range boundary falls
// inside a tile, the reduce kernel.  A stream-K launch needs ws_bytes of at
// least sk_workspace_bytes(G); else nothing is launched.
static hipError_t launch_sk(const SkItem &one, const SkItem *items, const SkItem *host, int32_t count,
                            const SkTile *seq, const SkRange *wg, const SkSplitList *parts, bool closed, int ntw,
                            int fm, int64_t iters, int scale_f32, int has_zp, int sps, int G, float *ws,
                            size_t ws_bytes, hipStream_t stream) {
    if (iters >= (int64_t)1 << 31 || G < 1 || G > kSkMaxGrid) return hipErrorInvalidValue;
    if (closed && (count != 1 || seq)) return hipErrorInvalidValue;
    if (parts && (!seq || parts->n < 0 || parts->n > kSkMaxSplits)) return hipErrorInvalidValue;
    // a stream-K launch may split tiles: the workspace must hold the partial
    // tiles of its G workgroups; a tile list with parts, its parts' partials
    if (!seq && !closed && (!ws || ws_bytes < sk_workspace_bytes(G))) return hipErrorInvalidValue;
    if (parts && parts->n > 0) {
        int n_parts = 0;
        for (int j = 0; j < parts->n; ++j) {
            if (!((uint32_t)parts->e[j].t_slot & kSkSplitParts)) return hipErrorInvalidValue;
            n_parts = std::max(n_parts, (int)parts->e[j].last + 1);
        }
        if (!ws || ws_bytes < (size_t)n_parts * kSkPartialFloats * sizeof(float) ||
            32 * fm * 128 * ntw > kSkPartialFloats)
            return hipErrorInvalidValue;
    }
    // 256 x 128 tiles, or wide (512 x 128), half (512 x 64) and skinny (512 x 32) tiles in
    // tile-list order only (split only into listed parts, never 512 x 128 tiles)
    const bool narrow = ntw == kSkNTW && fm == kSkFM;
    const bool wide = ntw == kSkWideNTW && (fm == kSkFM || fm == kSkHalfFM || fm == kSkSkinnyFM);
    if (!narrow && (!wide || !(seq || closed) || !sk_wide_supported(scale_f32, sps))) return hipErrorInvalidValue;
    SkParams p;
    p.one = one;
    p.items = items;
    p.seq = seq;
    p.wg = wg;
    p.count = count;
    p.closed = closed ? 1 : 0;
    p.G = G;
    p.I = (int32_t)iters;
    p.ws = ws;
    dim3 grid(G), block(kSkThreads);
    const bool with_parts = parts && parts->n > 0;
#define MNB_SK_LAUNCH(ST_, ZP_, SPS_) launch_sk_variant<ST_, ZP_, SPS_>(ntw, fm, with_parts, grid, block, stream, p)
#define MNB_SK_SPS(ST_, ZP_)                           \
    switch (sps) {                                     \
        case 1: MNB_SK_LAUNCH(ST_, ZP_, 1); break;     \
        case 2: MNB_SK_LAUNCH(ST_, ZP_, 2); break;     \
        case 4: MNB_SK_LAUNCH(ST_, ZP_, 4); break;     \
        case 8: MNB_SK_LAUNCH(ST_, ZP_, 8); break;     \
        default: return hipErrorInvalidValue;          \
    }
    if (scale_f32) {
        if (has_zp) { MNB_SK_SPS(float, true) } else { MNB_SK_SPS(float, false) }
    } else {
        if (has_zp) { MNB_SK_SPS(_Float16, true) } else { MNB_SK_SPS(_Float16, false) }
    }
#undef MNB_SK_SPS
#undef MNB_SK_LAUNCH
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || closed) return e;
    if (seq) return parts ? launch_reduce(ntw, fm, stream, p, *parts) : hipSuccess;
    // stream-K: split tiles exist when some range boundary falls inside a tile
    SkSplitList list;
    sk_split_list(host, count, iters, G, list);
    return launch_reduce(ntw, fm, stream, p, list);
}

hipError_t launch_gemm_sk(const mnb_weight *w, const MatmulArgs &a, int G, float *ws, size_t ws_bytes,
                          hipStream_t stream) {
    const WeightGeom &g = w->g;
    const SkItem one = sk_make_item(w, a, 0);
    return launch_sk(one, nullptr, &one, 1, nullptr, nullptr, nullptr, false, kSkNTW, kSkFM, (int64_t)one.T * g.ST,
                     g.scale_f32, g.has_zp, g.SPS, G, ws, ws_bytes, stream);
}

hipError_t launch_gemm_closed(const mnb_weight *w, const MatmulArgs &a, int ntw, int fm, int G, hipStream_t stream) {
    const WeightGeom &g = w->g;
    const SkItem one = sk_make_item(w, a, 0, ntw, fm);
    return launch_sk(one, nullptr, &one, 1, nullptr, nullptr, nullptr, true, ntw, fm, (int64_t)one.T * g.ST,
                     g.scale_f32, g.has_zp, g.SPS, std::min(G, one.T), nullptr, 0, stream);
}

hipError_t launch_gemm_group(const GemmGroupPlan &g, float *ws, size_t ws_bytes, hipStream_t stream) {
    return launch_sk(g.host[0], (const SkItem *)g.items, g.host.data(), g.count, (const SkTile *)g.seq,
                     (const SkRange *)g.wg, g.parts.n > 0 ? &g.parts : nullptr, false, g.ntw, g.fm, g.iters,
                     g.scale_f32, g.has_zp, g.sps, g.G, ws, ws_bytes, stream);
}

}  // namespace mnb
