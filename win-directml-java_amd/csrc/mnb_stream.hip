// mnb_stream.hip -- persistent streaming kernel for a group of M = 1 products.
//
// A recorded group (mnb_group_create) of independent decode projections is
// cut into units: one unit = one 16-row n-tile of one item, over its whole K.
// Groups of products with 2 <= M <= 4 rows (small-batch decode) run the same
// kernel with MR = M rows of x per job: MR 1 KiB activation loads instead of
// one, the rows interleaved in LDS in 16-byte chunks, and MFMA row m taking x
// row min(m / 4, MR - 1), so that lane group g's four results all belong to
// x row g: each lane keeps one sum, as for M = 1, and lane group g stores row
// g.
// Each wavefront owns a list of units (balanced by bytes on the host, see
// mnb_sched.cpp) and streams them as jobs of kStreamJobTiles (4) consecutive
// super-tiles through a 2-deep register pipeline that runs across unit
// boundaries, so every wave keeps 8 KiB of tile loads in flight at all times.
// A job's loads are four 1 KiB weight tiles (one 16-byte non-temporal load per
// lane each), ONE scale load and ONE zero-point load for all four tiles (lane
// group g brings tile g's row), and ONE 1 KiB load of the four tiles'
// activations: per tile, a third of the load instructions of a per-tile
// pipeline (the scale and activation loads, not their bytes, cost 13% of the
// launch).  The scales, zero points and activations go through a
// wave-private LDS block to the lanes that multiply them.  A wave finishes a
// unit on its own (no split-K, no cross-wave reduction, no barrier) and writes
// the unit's 16 outputs.  The grid is sized to the device's resident capacity;
// the kernel is a plain loop over a static list, so no wave ever waits for
// another.
#include "mnb_device.h"

namespace mnb {

constexpr int kStreamDepth = 2;      // jobs in flight per wave (three measured the same, four slower)
constexpr int kStreamWaves = 4;      // waves per workgroup
constexpr int kJT = kStreamJobTiles;

typedef uint32_t u32x4_st_alias_t __attribute__((ext_vector_type(4), may_alias));
typedef _Float16 half8_st_alias_t __attribute__((ext_vector_type(8), may_alias));

// Per-unit view of one item, resolved with uniform (scalar) loads.
template <typename ScaleT>
struct UnitRef {
    const u32x4_t *q;      // first tile of the n-tile, + lane
    const ScaleT *s;       // first scale row of the n-tile, + row r
    const uint8_t *z;      // first zero-point row of the n-tile, + row r
    const _Float16 *x;     // activation rows, ldx apart
    void *y;
    int32_t ST, NJ, kx, N, nt, y_f16, accumulate, M, ldx;
    float unfold;
};

template <typename ScaleT, int SPS, int ZB>
__device__ __forceinline__ UnitRef<ScaleT> resolve_unit(const GroupItem *__restrict__ items, uint32_t code, int lane,
                                                        int r) {
    const int it = (int)(code >> 16);
    const int nt = (int)(code & 0xFFFFu);
    const GemvParams &p = items[it].p;
    UnitRef<ScaleT> u;
    const size_t tile0 = (size_t)nt * p.ST;
    u.q = (const u32x4_t *)p.q_t + tile0 * 64 + lane;
    u.s = (const ScaleT *)p.s_t + (tile0 * kTileRows + r) * SPS;
    u.z = p.zp_t ? p.zp_t + (tile0 * kTileRows + r) * ZB : nullptr;
    u.x = p.x;
    u.y = p.y;
    u.ST = p.ST;
    u.NJ = stream_jobs(p.ST);
    u.kx = p.kx;
    u.N = p.N;
    u.nt = nt;
    u.y_f16 = p.y_f16;
    u.accumulate = p.accumulate;
    u.M = p.M;
    u.ldx = p.ldx;
    u.unfold = p.unfold;
    return u;
}

template <typename ScaleT, bool HAS_ZP, int SPS, int MR>
__global__ __launch_bounds__(64 * kStreamWaves) void gemv_stream_kernel(const GroupItem *__restrict__ items,
                                                                        const uint32_t *__restrict__ units,
                                                                        const int32_t *__restrict__ wave_begin) {
    constexpr int ZB = SPS <= 2 ? 1 : SPS / 2;
    constexpr int SB = SPS * (int)sizeof(ScaleT);               // scale bytes per row per tile
    constexpr int D = kStreamDepth;
    static_assert(MR >= 1 && MR <= 4, "rows of x per job");
    // per wave: a job's activations (MR rows of 4 x 128 fp16; 16-byte chunk c
    // of row i at (c * MR + i) * 16), scale rows and zero-point entries (4
    // tiles x 16 rows each)
    constexpr int kXB = MR * kJT * kTileK * 2, kSB = kJT * kTileRows * SB, kZB = HAS_ZP ? kJT * kTileRows * ZB : 0;
    constexpr int kWaveLds = kXB + kSB + kZB;
    __shared__ __align__(16) unsigned char lds_all[kStreamWaves * kWaveLds];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, gg = lane >> 4;
    const int gw = blockIdx.x * kStreamWaves + wave;
    const int ubeg = wave_begin[2 * gw], uend = wave_begin[2 * gw + 2];
    const int njobs = wave_begin[2 * gw + 1];   // jobs over all of this wave's units
    if (ubeg >= uend) return;
    const uint32_t k6400 = vgpr_const(0x64006400u);
    const u32x4_t zero4 = {0u, 0u, 0u, 0u};
    unsigned char *xw = lds_all + wave * kWaveLds;   // activations
    unsigned char *sw = xw + kXB;                    // scale rows
    unsigned char *zw = sw + kSB;                    // zero-point entries

    u32x4_t raw[D][kJT];
    ScaleT sv[D][SPS];   // lane group g: tile g's scale row r
    uint32_t zb[D];
    u32x4_t xv[D][MR];   // row i: this lane's 16-byte piece of x row min(i, M - 1)
    bool xok[D];         // this lane's activation piece lies below kx (applied when it is written to LDS)

    // issue cursor: unit index iu, job ij
    int iu = ubeg, ij = 0;
    UnitRef<ScaleT> iref = resolve_unit<ScaleT, SPS, ZB>(items, units[iu], lane, r);
    // Every call issues the same loads (past the last job it re-loads the last
    // job, which is never computed; past a unit's last super-tile a job
    // re-loads that super-tile, which compute() skips), so the loop below
    // has a fixed number of loads in flight and exact wait counts.
    auto issue = [&](int d) {
        const int st0 = ij * kJT;
#pragma unroll
        for (int t = 0; t < kJT; ++t) raw[d][t] = gld_nt(iref.q + (size_t)min(st0 + t, iref.ST - 1) * 64);
        const int stg = min(st0 + gg, iref.ST - 1);
        load_scale_row<ScaleT, SPS>(iref.s + (size_t)stg * kTileRows * SPS, sv[d]);
        if constexpr (HAS_ZP) zb[d] = load_zp<ZB>(iref.z + (size_t)stg * kTileRows * ZB);
        else zb[d] = 0x88888888u;
        // lane l brings activations k = st0 * 128 + 8 l .. + 7 (tile l / 16)
        // of each row (rows past M re-read row M - 1, never stored)
        const int k = st0 * kTileK + 8 * lane;
#pragma unroll
        for (int i = 0; i < MR; ++i)
            xv[d][i] = gld((const u32x4_t *)(iref.x + (size_t)min(i, iref.M - 1) * iref.ldx + min(k, iref.kx - 8)));
        xok[d] = k < iref.kx;
        if (ij + 1 < iref.NJ) {
            ++ij;
        } else if (iu + 1 < uend) {
            ij = 0;
            iref = resolve_unit<ScaleT, SPS, ZB>(items, units[++iu], lane, r);
        }
    };

    // compute cursor: unit index cu, job cj
    int cu = ubeg, cj = 0;
    UnitRef<ScaleT> cref = iref;
    float acc = 0.f;
    // x row of MFMA row r (A operand): lane group g's results are MFMA rows 4 g .. 4 g + 3
    const int xrow = MR == 1 ? 0 : min(r >> 2, MR - 1);
    auto compute = [&](int d) {
        // wave-private LDS: a wave's LDS accesses complete in order, and the
        // compiler barriers keep this job's writes after the previous job's
        // reads and its reads after its writes
#pragma unroll
        for (int i = 0; i < MR; ++i) *(u32x4_st_alias_t *)(xw + (lane * MR + i) * 16) = xok[d] ? xv[d][i] : zero4;
        __builtin_memcpy(sw + (gg * kTileRows + r) * SB, &sv[d][0], SB);
        if constexpr (HAS_ZP) __builtin_memcpy(zw + (gg * kTileRows + r) * ZB, &zb[d], ZB);
        asm volatile("" ::: "memory");
#pragma unroll
        for (int t = 0; t < kJT; ++t) {
            // past the unit's last super-tile (K not a multiple of 512): loaded
            // again for a fixed load count, not computed (a uniform branch)
            if (cj * kJT + t >= cref.ST) break;
            half8_t xa[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)   // MFMA row r: x row xrow, k chunk 16 t + 4 j + gg
                xa[j] = *(const half8_st_alias_t *)(xw + ((16 * t + 4 * j + gg) * MR + xrow) * 16);
            ScaleT sc[SPS];
            __builtin_memcpy(&sc[0], sw + (t * kTileRows + r) * SB, SB);
            uint32_t zt = 0x88888888u;
            if constexpr (HAS_ZP) __builtin_memcpy(&zt, zw + (t * kTileRows + r) * ZB, ZB);
            if constexpr (SPS == 8) {
                float4_t dd = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int i = 2 * j + (gg >> 1);
                    const uint32_t z = HAS_ZP ? zp_nibble(zt, i) : 8u;
                    half8_t b = unpack_q_minus_zp(raw[d][t][j], bias_lo_pair(z), bias_hi_pair(z), k6400);
                    b = b * (_Float16)(float)((gg >> 1) ? sc[2 * j + 1] : sc[2 * j]);
                    dd = mfma16x16x32(xa[j], b, dd);
                }
                acc += dd[0];
            } else {
                constexpr int KPB = 4 / SPS;
#pragma unroll
                for (int i = 0; i < SPS; ++i) {
                    const uint32_t z = HAS_ZP ? zp_nibble(zt, i) : 8u;
                    const uint32_t blo = bias_lo_pair(z), bhi = bias_hi_pair(z);
                    float4_t dd = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int u = 0; u < KPB; ++u) {
                        const int j = i * KPB + u;
                        dd = mfma16x16x32(xa[j], unpack_q_minus_zp(raw[d][t][j], blo, bhi, k6400), dd);
                    }
                    acc = fmaf((float)sc[i], dd[0], acc);
                }
            }
        }
        asm volatile("" ::: "memory");
        if (++cj == cref.NJ) {
            // lane group g holds x row g (for M = 1 every group holds row 0):
            // group g stores row g of its column r
            const int n = cref.nt * kTileRows + r;
            if (gg < MR && gg < cref.M && n < cref.N) {
                const float v = acc * cref.unfold;   // undo the stored scales' 2^fold_exp
                const size_t idx = (size_t)gg * cref.N + n;
                if (cref.y_f16) store_y<true>(cref.y, idx, v, cref.accumulate != 0);
                else store_y<false>(cref.y, idx, v, cref.accumulate != 0);
            }
            acc = 0.f;
            cj = 0;
            if (cu + 1 < uend) cref = resolve_unit<ScaleT, SPS, ZB>(items, units[++cu], lane, r);
        }
    };

#pragma unroll
    for (int d = 0; d < D; ++d) issue(d);
    int j = 0;
    for (; j + D <= njobs; j += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            compute(d);
            issue(d);
        }
    }
#pragma unroll
    for (int d = 0; d < D - 1; ++d)
        if (j + d < njobs) compute(d);
}

hipError_t launch_gemv_stream(const GemvGroupPlan &g, hipStream_t stream) {
    dim3 grid(g.stream_wgs), block(64 * kStreamWaves);
    const GroupItem *it = (const GroupItem *)g.items;
    const uint32_t *un = (const uint32_t *)g.units;
    const int32_t *wb = (const int32_t *)g.wave_begin;
    if (g.stream_rows < 1 || g.stream_rows > 4) return hipErrorInvalidValue;
#define MNB_STREAM_MR(ST_, ZP_, SPS_, MR_) \
    hipLaunchKernelGGL((gemv_stream_kernel<ST_, ZP_, SPS_, MR_>), grid, block, 0, stream, it, un, wb)
#define MNB_STREAM_LAUNCH(ST_, ZP_, SPS_)                                       \
    if (g.stream_rows == 1) { MNB_STREAM_MR(ST_, ZP_, SPS_, 1); }              \
    else if (g.stream_rows == 2) { MNB_STREAM_MR(ST_, ZP_, SPS_, 2); }         \
    else if (g.stream_rows == 3) { MNB_STREAM_MR(ST_, ZP_, SPS_, 3); }         \
    else { MNB_STREAM_MR(ST_, ZP_, SPS_, 4); }
#define MNB_STREAM_SPS(ST_, ZP_)                               \
    switch (g.sps) {                                           \
        case 1: MNB_STREAM_LAUNCH(ST_, ZP_, 1); break;         \
        case 2: MNB_STREAM_LAUNCH(ST_, ZP_, 2); break;         \
        case 4: MNB_STREAM_LAUNCH(ST_, ZP_, 4); break;         \
        case 8: MNB_STREAM_LAUNCH(ST_, ZP_, 8); break;         \
        default: return hipErrorInvalidValue;                  \
    }
    if (g.scale_f32) {
        if (g.has_zp) { MNB_STREAM_SPS(float, true) } else { MNB_STREAM_SPS(float, false) }
    } else {
        if (g.has_zp) { MNB_STREAM_SPS(_Float16, true) } else { MNB_STREAM_SPS(_Float16, false) }
    }
#undef MNB_STREAM_SPS
#undef MNB_STREAM_LAUNCH
#undef MNB_STREAM_MR
    return hipGetLastError();
}

int stream_kernel_waves_per_cu(int scale_f32, int has_zp, int sps, int rows) {
    int blocks = 0;
    hipError_t e = hipSuccess;
#define MNB_OCC_MR(ST_, ZP_, SPS_, MR_) \
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, gemv_stream_kernel<ST_, ZP_, SPS_, MR_>, 64 * kStreamWaves, 0)
#define MNB_OCC(ST_, ZP_, SPS_)                                  \
    if (rows == 1) { MNB_OCC_MR(ST_, ZP_, SPS_, 1); }            \
    else if (rows == 2) { MNB_OCC_MR(ST_, ZP_, SPS_, 2); }       \
    else if (rows == 3) { MNB_OCC_MR(ST_, ZP_, SPS_, 3); }       \
    else { MNB_OCC_MR(ST_, ZP_, SPS_, 4); }
#define MNB_OCC_SPS(ST_, ZP_)                  \
    switch (sps) {                             \
        case 1: MNB_OCC(ST_, ZP_, 1); break;   \
        case 2: MNB_OCC(ST_, ZP_, 2); break;   \
        case 4: MNB_OCC(ST_, ZP_, 4); break;   \
        default: MNB_OCC(ST_, ZP_, 8); break;  \
    }
    if (scale_f32) {
        if (has_zp) { MNB_OCC_SPS(float, true) } else { MNB_OCC_SPS(float, false) }
    } else {
        if (has_zp) { MNB_OCC_SPS(_Float16, true) } else { MNB_OCC_SPS(_Float16, false) }
    }
#undef MNB_OCC_SPS
#undef MNB_OCC
#undef MNB_OCC_MR
    if (e != hipSuccess || blocks < 1) blocks = 1;
    return blocks * kStreamWaves;
}

}  // namespace mnb
