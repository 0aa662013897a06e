// mnb_gemv.hip -- decode-shaped MatMulNBits (M <= 16), HBM-bound.
//
// Replaces the one-thread-per-row HLSL GEMV INT4_MATVEC_HLSL
// (directml-windows-bindings/src/main/java/com/aresstack/windirectml/windows/
// MatMulNBitsKernel.java:235-292) and the WARP row-group variants (:299-714).
// Same result: y[m,n] = sum_blk scale[n,blk] * sum_k (q[n,k]-zp[n,blk]) * x[m,k].
//
// Work decomposition: one workgroup per 16-row n-tile, W waves split the
// n-tile's super-tiles (128 k each) and reduce their partial sums in LDS.
// Per super-tile a lane issues ONE 16-byte load that holds its part of the
// 16x128 tile in MFMA operand order, so a wave streams 1 KiB per load.
// Per 32-k step: 9 VALU ops turn 8 nibbles into 8 exact fp16 (q - zp), one
// v_mfma_f32_16x16x32_f16 multiplies them with x (A operand; rows 0..15 are
// the activation rows, M = 1 broadcasts x to every row), and the block
// scale is applied to the fp32 MFMA result (bs >= 32), so no weight is ever
// rounded.  bs = 16 (two scales per 32-k step) folds the scale into the fp16
// weight instead.
#include "mnb_device.h"

namespace mnb {

// LDS bytes of 4 x rows of one super-tile (128 k of fp16).  When M > 1 a
// wave's x block holds XR of them: 4 XR rows.
constexpr int kXGroupBytes = 4 * kTileK * 2;

// x row groups of 4 rows a product with M rows loads: M <= 4 XR.
inline int gemv_rows_xr(int M) { return M <= 4 ? 1 : M <= 8 ? 2 : 4; }

// M1: x has one row, staged once per workgroup in LDS (A operand = x
// broadcast to all 16 MFMA rows).  !M1: the wave's x block holds 4 XR rows
// of the super-tile (rows >= M repeat row M-1), and MFMA row m reads block
// row m * XR / 4: with M <= 4 (XR = 1) the four MFMA rows of lane group g
// all read x row g, so the lanes of group g hold output row g, one sum per
// lane; with M <= 8 (XR = 2) group g holds rows 2g and 2g+1, two sums; with
// M <= 16 (XR = 4) rows 4g..4g+3, four sums.  A smaller block means fewer
// LDS stores and less LDS per workgroup (more resident workgroups); the
// duplicated MFMA rows cost nothing, the MFMA issues either way.
// STW: super-tiles per wave; all of a wave's weight, scale and zero-point
// loads are issued before any arithmetic.
// One workgroup computes the 16 outputs of n-tile `nt` (per activation row):
// its W waves take chunks of STW super-tiles; waves beyond the chunk count
// only take part in the final LDS reduction.
template <typename ScaleT, bool HAS_ZP, bool M1, int SPS, int STW, int XR = 4>
__device__ __forceinline__ void gemv_tile(const GemvParams &p, const int nt, unsigned char *smem) {
    constexpr int ZB = SPS <= 2 ? 1 : SPS / 2;
    static_assert(XR == 1 || XR == 2 || XR == 4, "x row groups: 1, 2 or 4");
    // !M1: MFMA row m reads x block row m >> RSH; the D values of a lane that
    // are distinct rows are acc[0], acc[AST], ... (AST = 1 << RSH).  M1
    // keeps acc[0] only.
    constexpr int RSH = XR == 4 ? 0 : XR == 2 ? 1 : 2;
    constexpr int AST = M1 ? 4 : 1 << RSH;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int W = blockDim.x >> 6;
    float4_t *red = (float4_t *)smem;                              // [W][64]
    // wave-private x region after the reduction slots: M1, the wave's slice
    // of x (STW*128 halves); !M1, the 4 XR-row x block of a super-tile
    unsigned char *xw = smem + (size_t)W * 64 * sizeof(float4_t) + (size_t)wave * (M1 ? STW * kTileK * 2 : XR * kXGroupBytes);
    _Float16 *xs = (_Float16 *)xw;
    const int r = lane & 15, gg = lane >> 4;
    const int nchunks = (p.ST + STW - 1) / STW;

    const size_t tile0 = (size_t)nt * p.ST;
    const u32x4_t *qp = (const u32x4_t *)p.q_t + tile0 * 64 + lane;
    const ScaleT *sp = (const ScaleT *)p.s_t + (tile0 * kTileRows + r) * SPS;
    const uint8_t *zpp = HAS_ZP ? p.zp_t + (tile0 * kTileRows + r) * ZB : nullptr;
    const u32x4_t zero4 = {0u, 0u, 0u, 0u};
    const uint32_t k6400 = vgpr_const(0x64006400u);

    u32x4_t raw[STW];
    ScaleT sv[STW][SPS];
    uint32_t zb[STW];
    // !M1: the x rows of each super-tile are loaded row-contiguous -- lane l
    // brings 16 bytes at k = 8 (l % 16) of row 4 i + l / 16, so one load
    // covers four whole 256-byte row pieces -- then go through the wave's LDS
    // block into MFMA operand order.  (Loading the operand order directly
    // touches 16 rows, 64 bytes each, per load: four times the cache-line
    // requests for the same bytes.)  Rows >= M repeat row M - 1.
    u32x4_t xrw[M1 ? 1 : STW][XR];
    const _Float16 *xrow[XR];
#pragma unroll
    for (int i = 0; i < XR; ++i) {
        const int row = 4 * i + (lane >> 4);
        xrow[i] = p.x + (size_t)(row < p.M ? row : p.M - 1) * p.ldx;
    }
    // Straight-line loads (no per-lane branches, so the compiler's wait
    // counters stay exact).  A super-tile index past the end is clamped to the
    // last tile: its k range lies at or beyond kx, where x is zero, so the
    // repeated tile contributes exactly zero.
    auto issue = [&](int c) {
#pragma unroll
        for (int t = 0; t < STW; ++t) {
            const int st = min(c * STW + t, p.ST - 1);
            if constexpr (!M1) {
                // clamped into the row; pieces at k >= kx are zeroed in LDS
                const int k = min((c * STW + t) * kTileK + 8 * (lane & 15), p.kx - 8);
                // XR groups of 4 rows are loaded (M <= 4 XR)
#pragma unroll
                for (int i = 0; i < XR; ++i) xrw[t][i] = *(const u32x4_t *)(xrow[i] + k);
            }
            raw[t] = gld_nt(qp + (size_t)st * 64);
            load_scale_row<ScaleT, SPS>(sp + (size_t)st * kTileRows * SPS, sv[t]);
            if constexpr (HAS_ZP) zb[t] = load_zp<ZB>(zpp + (size_t)st * kTileRows * ZB);
            else zb[t] = 0x88888888u;
            // keep each super-tile's weights and scales together in issue
            // order: loads complete in order, so super-tile t can be computed
            // while the later ones are still arriving (the compiler would
            // otherwise issue every scale after the last weight load)
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // M1: one coalesced 16-byte load per lane brings the wave's x slice
    // (issued before the weights, so it is the first to arrive).  The lane
    // mask is applied when the slice is written to LDS, not here: a select
    // on the loaded value would wait for it before the weight loads issue.
    bool xok = false;
    auto load_x_slice = [&](int c) -> u32x4_t {
        const int k = c * STW * kTileK + 8 * lane;
        xok = lane < STW * (kTileK / 8) && k < p.kx;
        return *(const u32x4_t *)(p.x + min(k, p.kx - 8));
    };

    float4_t acc = {0.f, 0.f, 0.f, 0.f};
    u32x4_t xv = zero4;
    auto compute_chunk = [&](int c) {
        if constexpr (M1) {
            // wave-private LDS: a wave's LDS accesses complete in order, no barrier needed
            if (lane < STW * (kTileK / 8)) ((u32x4_t *)xs)[lane] = xok ? xv : zero4;
        }
#pragma unroll
        for (int t = 0; t < STW; ++t) {
            half8_t xa[4];
            const int kst = (c * STW + t) * kTileK;
            if constexpr (M1) {
#pragma unroll
                for (int j = 0; j < 4; ++j) xa[j] = *(const half8_t *)(xs + t * kTileK + 32 * j + 8 * gg);
            } else {
                // 16-byte piece (row, chunk) at row * 256 + ((chunk ^ row) % 16) * 16:
                // eight consecutive lanes of a write (one row, eight chunks) or
                // of a read (eight rows, one chunk each) hit distinct banks.
                // The wave's LDS accesses run in order, so the block can be
                // rewritten for the next super-tile right after these reads.
                const bool kok = kst + 8 * (lane & 15) < p.kx;
#pragma unroll
                for (int i = 0; i < XR; ++i) {
                    const int row = 4 * i + (lane >> 4);
                    *(u32x4_t *)(xw + row * 256 + (((lane & 15) ^ row) & 15) * 16) = kok ? xrw[t][i] : zero4;
                }
                const int xq = r >> RSH;
#pragma unroll
                for (int j = 0; j < 4; ++j) xa[j] = *(const half8_t *)(xw + xq * 256 + (((4 * j + gg) ^ xq) & 15) * 16);
            }
            if constexpr (SPS == 8) {
                // bs = 16: the lane's 8 k lie in block 2j + gg/2; fold the scale.
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int i = 2 * j + (gg >> 1);
                    const uint32_t z = HAS_ZP ? zp_nibble(zb[t], i) : 8u;
                    half8_t b = unpack_q_minus_zp(raw[t][j], bias_lo_pair(z), bias_hi_pair(z), k6400);
                    b = b * (_Float16)(float)sv[t][i];
                    acc = mfma16x16x32(xa[j], b, acc);
                }
            } else {
                constexpr int KPB = 4 / SPS;   // 32-k steps per scale block inside the super-tile
#pragma unroll
                for (int i = 0; i < SPS; ++i) {
                    const uint32_t z = HAS_ZP ? zp_nibble(zb[t], i) : 8u;
                    const uint32_t blo = bias_lo_pair(z), bhi = bias_hi_pair(z);
                    float4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int u = 0; u < KPB; ++u) {
                        const int j = i * KPB + u;
                        d = mfma16x16x32(xa[j], unpack_q_minus_zp(raw[t][j], blo, bhi, k6400), d);
                    }
                    const float s = (float)sv[t][i];
#pragma unroll
                    for (int e = 0; e < 4; e += AST) acc[e] = fmaf(s, d[e], acc[e]);
                }
            }
        }
    };

    if (wave < nchunks) {
        // The first chunk is straight-line code after its loads; further
        // chunks (K > W x STW x 128) loop.
        if constexpr (M1) xv = load_x_slice(wave);
        issue(wave);
        __builtin_amdgcn_sched_barrier(0);   // every load of the chunk is issued before any arithmetic
        compute_chunk(wave);
        for (int c = wave + W; c < nchunks; c += W) {
            if constexpr (M1) xv = load_x_slice(c);
            issue(c);
            __builtin_amdgcn_sched_barrier(0);
            compute_chunk(c);
        }
    }

    if (W > 1) {
        red[wave * 64 + lane] = acc;
        __syncthreads();
        if (wave != 0) return;
        for (int w2 = 1; w2 < W; ++w2) {
            const float4_t o = red[w2 * 64 + lane];
#pragma unroll
            for (int e = 0; e < 4; e += AST) acc[e] += o[e];
        }
    }

    // undo the stored scales' factor 2^fold_exp (exact)
#pragma unroll
    for (int e = 0; e < 4; e += AST) acc[e] *= p.unfold;
    // D layout of the 16x16 MFMA result: lane (gg*16 + r) holds MFMA rows
    // 4*gg+i, column r; MFMA row m is x row m >> RSH.
    const int n = nt * kTileRows + r;
    if (n >= p.N) return;
    const bool accum = p.accumulate != 0;
    if constexpr (M1) {
        if (gg == 0) {
            if (p.y_f16) store_y<true>(p.y, (size_t)n, acc[0], accum);
            else store_y<false>(p.y, (size_t)n, acc[0], accum);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; i += AST) {
            const int mm = (4 * gg + i) >> RSH;
            if (mm < p.M) {
                const size_t idx = (size_t)mm * p.N + n;
                if (p.y_f16) store_y<true>(p.y, idx, acc[i], accum);
                else store_y<false>(p.y, idx, acc[i], accum);
            }
        }
    }
}

template <typename ScaleT, bool HAS_ZP, bool M1, int SPS, int STW, int XR>
__global__ __launch_bounds__(M1 ? 64 * kGemvMaxWaves : 64 * kGemvMaxWavesRows) void gemv_kernel(GemvParams p) {
    extern __shared__ __align__(16) unsigned char smem[];
    gemv_tile<ScaleT, HAS_ZP, M1, SPS, STW, XR>(p, blockIdx.x, smem);
}

// A group of independent projections in one launch: workgroup b computes
// n-tile b - first_wg of item wg_item[b].
template <typename ScaleT, bool HAS_ZP, bool M1, int SPS, int STW, int XR>
__global__ __launch_bounds__(M1 ? 64 * kGemvMaxWaves : 64 * kGemvMaxWavesRows) void gemv_group_kernel(const GroupItem *__restrict__ items,
                                                          const uint16_t *__restrict__ wg_item) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int it = wg_item[blockIdx.x];
    const GemvParams p = items[it].p;
    gemv_tile<ScaleT, HAS_ZP, M1, SPS, STW, XR>(p, (int)blockIdx.x - items[it].first_wg, smem);
}

struct GemvLaunch {
    dim3 grid, block;
    size_t lds;
    int stw;
};

template <typename ScaleT, bool HAS_ZP, bool M1, int SPS>
static hipError_t gemv_stw(const GemvLaunch &L, const GemvParams &p, hipStream_t s) {
    if constexpr (!M1) {
        if (L.stw != kGemvRowsSTW) return hipErrorInvalidValue;
        // x row groups to load: one per 4 rows of M (the LDS size follows)
        const int xr = gemv_rows_xr(p.M);
        if (xr == 1)
            hipLaunchKernelGGL((gemv_kernel<ScaleT, HAS_ZP, false, SPS, kGemvRowsSTW, 1>), L.grid, L.block, L.lds, s, p);
        else if (xr == 2)
            hipLaunchKernelGGL((gemv_kernel<ScaleT, HAS_ZP, false, SPS, kGemvRowsSTW, 2>), L.grid, L.block, L.lds, s, p);
        else
            hipLaunchKernelGGL((gemv_kernel<ScaleT, HAS_ZP, false, SPS, kGemvRowsSTW, 4>), L.grid, L.block, L.lds, s, p);
    } else {
        switch (L.stw) {
            case 2: hipLaunchKernelGGL((gemv_kernel<ScaleT, HAS_ZP, true, SPS, 2, 4>), L.grid, L.block, L.lds, s, p); break;
            case 4: hipLaunchKernelGGL((gemv_kernel<ScaleT, HAS_ZP, true, SPS, 4, 4>), L.grid, L.block, L.lds, s, p); break;
            default: return hipErrorInvalidValue;
        }
    }
    return hipGetLastError();
}

template <typename ScaleT, bool HAS_ZP, bool M1>
static hipError_t gemv_sps(const WeightGeom &g, const GemvLaunch &L, const GemvParams &p, hipStream_t s) {
    switch (g.SPS) {
        case 1: return gemv_stw<ScaleT, HAS_ZP, M1, 1>(L, p, s);
        case 2: return gemv_stw<ScaleT, HAS_ZP, M1, 2>(L, p, s);
        case 4: return gemv_stw<ScaleT, HAS_ZP, M1, 4>(L, p, s);
        case 8: return gemv_stw<ScaleT, HAS_ZP, M1, 8>(L, p, s);
        default: return hipErrorInvalidValue;
    }
}

template <typename ScaleT>
static hipError_t gemv_zp(const WeightGeom &g, const GemvLaunch &L, const GemvParams &p, bool m1, hipStream_t s) {
    if (g.has_zp) return m1 ? gemv_sps<ScaleT, true, true>(g, L, p, s) : gemv_sps<ScaleT, true, false>(g, L, p, s);
    return m1 ? gemv_sps<ScaleT, false, true>(g, L, p, s) : gemv_sps<ScaleT, false, false>(g, L, p, s);
}

// Super-tiles per wave: 4 (4 KiB of weights in flight per wave), or 2 when
// the grid would otherwise have fewer than 8 waves per CU.  M > 1 always
// takes 2 (kGemvRowsSTW): each super-tile also holds 4 XR registers of x rows.
// K above 16 waves x 4 x 128 = 8192 (12 waves x 2 x 128 = 3072 when M > 1)
// loops over further chunks per wave.
static int gemv_stw_for(const WeightGeom &g, int cu_count, bool m1) {
    if (!m1) return kGemvRowsSTW;
    if ((g.ST + 3) / 4 <= 16 && (int64_t)g.NT * ((g.ST + 3) / 4) >= 8LL * cu_count) return 4;
    if ((g.ST + 1) / 2 <= 16) return 2;
    return 4;
}

hipError_t launch_gemv(const mnb_weight *w, const MatmulArgs &a, int32_t cu_count, hipStream_t stream) {
    const WeightGeom &g = w->g;
    if (a.M < 1 || a.M > kSkinnyMaxM) return hipErrorInvalidValue;
    GemvParams p;
    p.q_t = (const u32x4_t *)w->q_t;
    p.s_t = w->s_t;
    p.zp_t = (const uint8_t *)w->zp_t;
    p.x = a.x;
    p.ldx = a.ldx;
    p.kx = a.kx;
    p.M = a.M;
    p.N = g.N;
    p.ST = g.ST;
    p.y = a.y;
    p.y_f16 = a.y_type == MNB_F16;
    p.accumulate = a.accumulate;
    p.unfold = pow2f(-g.fold_exp);
    GemvLaunch L;
    const bool m1 = a.M == 1;
    L.stw = gemv_stw_for(g, cu_count > 0 ? cu_count : 256, m1);
    int waves = (g.ST + L.stw - 1) / L.stw;
    waves = min(waves, m1 ? kGemvMaxWaves : kGemvMaxWavesRows);
    L.grid = dim3(g.NT);
    L.block = dim3(64 * waves);
    L.lds = (size_t)waves * 64 * sizeof(float4_t) + (size_t)waves * (m1 ? L.stw * kTileK * 2 : gemv_rows_xr(a.M) * kXGroupBytes);
    return g.scale_f32 ? gemv_zp<float>(g, L, p, m1, stream) : gemv_zp<_Float16>(g, L, p, m1, stream);
}

hipError_t launch_gemv_group(const GemvGroupPlan &g, hipStream_t stream) {
    dim3 grid(g.total_wgs), block(64 * g.waves);
    // M > 1: x row groups to load, from the largest M of the items (the LDS size follows)
    const int xr = g.m1 ? 4 : gemv_rows_xr(g.max_m);
    const size_t lds = (size_t)g.waves * 64 * sizeof(float4_t) + (size_t)g.waves * (g.m1 ? 4 * kTileK * 2 : xr * kXGroupBytes);
    const GroupItem *it = (const GroupItem *)g.items;
    const uint16_t *wi = (const uint16_t *)g.wg_item;
#define MNB_GROUP_XR(ST_, ZP_, M1_, SPS_, XR_) \
    hipLaunchKernelGGL((gemv_group_kernel<ST_, ZP_, M1_, SPS_, M1_ ? 4 : kGemvRowsSTW, XR_>), grid, block, lds, stream, it, wi)
#define MNB_GROUP_LAUNCH(ST_, ZP_, M1_, SPS_)                                    \
    if (M1_ || xr == 4) { MNB_GROUP_XR(ST_, ZP_, M1_, SPS_, 4); }                \
    else if (xr == 2) { MNB_GROUP_XR(ST_, ZP_, M1_, SPS_, (M1_ ? 4 : 2)); }      \
    else { MNB_GROUP_XR(ST_, ZP_, M1_, SPS_, (M1_ ? 4 : 1)); }
#define MNB_GROUP_SPS(ST_, ZP_, M1_)                              \
    switch (g.sps) {                                              \
        case 1: MNB_GROUP_LAUNCH(ST_, ZP_, M1_, 1); break;        \
        case 2: MNB_GROUP_LAUNCH(ST_, ZP_, M1_, 2); break;        \
        case 4: MNB_GROUP_LAUNCH(ST_, ZP_, M1_, 4); break;        \
        case 8: MNB_GROUP_LAUNCH(ST_, ZP_, M1_, 8); break;        \
        default: return hipErrorInvalidValue;                     \
    }
    if (g.scale_f32) {
        if (g.has_zp) { if (g.m1) { MNB_GROUP_SPS(float, true, true) } else { MNB_GROUP_SPS(float, true, false) } }
        else { if (g.m1) { MNB_GROUP_SPS(float, false, true) } else { MNB_GROUP_SPS(float, false, false) } }
    } else {
        if (g.has_zp) { if (g.m1) { MNB_GROUP_SPS(_Float16, true, true) } else { MNB_GROUP_SPS(_Float16, true, false) } }
        else { if (g.m1) { MNB_GROUP_SPS(_Float16, false, true) } else { MNB_GROUP_SPS(_Float16, false, false) } }
    }
#undef MNB_GROUP_SPS
#undef MNB_GROUP_LAUNCH
#undef MNB_GROUP_XR
    return hipGetLastError();
}

}  // namespace mnb
