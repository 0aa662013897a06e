// mnb_stream.hip -- persistent streaming kernel for a group of M = 1 products.
//
// A recorded group (mnb_group_create) of independent decode projections is
// cut into units: one unit = one 16-row n-tile of one item, over its whole K.
// Each wavefront owns a list of units (balanced by bytes on the host, see
// mnb_api.cpp) and streams their 16x128 weight tiles through a 4-deep
// register pipeline that runs across unit boundaries, so every wave keeps
// four 1 KiB tile loads in flight at all times.  A wave finishes a unit on
// its own (no split-K, no cross-wave reduction, no barrier) and writes the
// unit's 16 outputs.  The grid is sized to the device's resident capacity;
// the kernel is a plain loop over a static list, so no wave ever waits for
// another.
#include "mnb_device.h"

namespace mnb {

#ifndef MNB_STREAM_DEPTH
#define MNB_STREAM_DEPTH 4
#endif
constexpr int kStreamDepth = MNB_STREAM_DEPTH;   // tiles in flight per wave
constexpr int kStreamWaves = 4;      // waves per workgroup

// Per-unit view of one item, resolved with uniform (scalar) loads.
template <typename ScaleT>
struct UnitRef {
    const u32x4_t *q;      // first tile of the n-tile, + lane
    const ScaleT *s;       // first scale row of the n-tile
    const uint8_t *z;      // first zero-point row of the n-tile
    const _Float16 *x;     // activation row
    void *y;
    int32_t ST, kx, N, nt, y_f16, accumulate;
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
    u.kx = p.kx;
    u.N = p.N;
    u.nt = nt;
    u.y_f16 = p.y_f16;
    u.accumulate = p.accumulate;
    u.unfold = p.unfold;
    return u;
}

template <typename ScaleT, bool HAS_ZP, int SPS>
__global__ __launch_bounds__(64 * kStreamWaves) void gemv_stream_kernel(const GroupItem *__restrict__ items,
                                                                        const uint32_t *__restrict__ units,
                                                                        const int32_t *__restrict__ wave_begin) {
    constexpr int ZB = SPS <= 2 ? 1 : SPS / 2;
    constexpr int D = kStreamDepth;
    __shared__ __align__(16) _Float16 xs_all[kStreamWaves][D][kTileK];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, gg = lane >> 4;
    const int gw = blockIdx.x * kStreamWaves + wave;
    const int ubeg = wave_begin[2 * gw], uend = wave_begin[2 * gw + 2];
    const int njobs = wave_begin[2 * gw + 1];   // super-tiles over all of this wave's units
    if (ubeg >= uend) return;
    const uint32_t k6400 = vgpr_const(0x64006400u);
    const u32x4_t zero4 = {0u, 0u, 0u, 0u};

    u32x4_t raw[D];
    ScaleT sv[D][SPS];
    uint32_t zb[D];
    u32x4_t xv[D];
    bool xok[D];   // this lane's x piece lies below kx (applied at compute time, not at load time)

    // issue cursor: unit index iu, super-tile ist
    int iu = ubeg, ist = 0;
    UnitRef<ScaleT> iref = resolve_unit<ScaleT, SPS, ZB>(items, units[iu], lane, r);
    // Every call issues the same loads (past the last job it re-loads the last
    // tile, which is never computed), so the loop below has a fixed number of
    // loads in flight and exact wait counts.
    auto issue = [&](int d) {
        raw[d] = gld_nt(iref.q + (size_t)ist * 64);
        load_scale_row<ScaleT, SPS>(iref.s + (size_t)ist * kTileRows * SPS, sv[d]);
        if constexpr (HAS_ZP) zb[d] = load_zp<ZB>(iref.z + (size_t)ist * kTileRows * ZB);
        else zb[d] = 0x88888888u;
        // lanes 0..15 bring this tile's 128 activations
        const int k = ist * kTileK + 8 * lane;
        xv[d] = gld((const u32x4_t *)(iref.x + min(k, iref.kx - 8)));
        xok[d] = lane < kTileK / 8 && k < iref.kx;
        if (ist + 1 < iref.ST) {
            ++ist;
        } else if (iu + 1 < uend) {
            ist = 0;
            iref = resolve_unit<ScaleT, SPS, ZB>(items, units[++iu], lane, r);
        }
    };

    // compute cursor: unit index cu, super-tile cst
    int cu = ubeg, cst = 0;   // compute cursor (unit, super-tile)
    UnitRef<ScaleT> cref = iref;
    float acc = 0.f;
    auto compute = [&](int d) {
        _Float16 *xs = xs_all[wave][d];
        if (lane < kTileK / 8) ((u32x4_t *)xs)[lane] = xok[d] ? xv[d] : zero4;   // wave-private, in-order LDS
        half8_t xa[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) xa[j] = *(const half8_t *)(xs + 32 * j + 8 * gg);
        if constexpr (SPS == 8) {
            float4_t dd = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = 2 * j + (gg >> 1);
                const uint32_t z = HAS_ZP ? zp_nibble(zb[d], i) : 8u;
                half8_t b = unpack_q_minus_zp(raw[d][j], bias_lo_pair(z), bias_hi_pair(z), k6400);
                b = b * (_Float16)(float)sv[d][i];
                dd = mfma16x16x32(xa[j], b, dd);
            }
            acc += dd[0];
        } else {
            constexpr int KPB = 4 / SPS;
#pragma unroll
            for (int i = 0; i < SPS; ++i) {
                const uint32_t z = HAS_ZP ? zp_nibble(zb[d], i) : 8u;
                const uint32_t blo = bias_lo_pair(z), bhi = bias_hi_pair(z);
                float4_t dd = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int u = 0; u < KPB; ++u) {
                    const int j = i * KPB + u;
                    dd = mfma16x16x32(xa[j], unpack_q_minus_zp(raw[d][j], blo, bhi, k6400), dd);
                }
                acc = fmaf((float)sv[d][i], dd[0], acc);
            }
        }
        if (++cst == cref.ST) {
            // x was broadcast to all 16 MFMA rows: lanes 0..15 hold row 0, column r
            const int n = cref.nt * kTileRows + r;
            if (gg == 0 && n < cref.N) {
                const float v = acc * cref.unfold;   // undo the stored scales' 2^fold_exp
                if (cref.y_f16) store_y<true>(cref.y, (size_t)n, v, cref.accumulate != 0);
                else store_y<false>(cref.y, (size_t)n, v, cref.accumulate != 0);
            }
            acc = 0.f;
            cst = 0;
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
#define MNB_STREAM_LAUNCH(ST_, ZP_, SPS_) \
    hipLaunchKernelGGL((gemv_stream_kernel<ST_, ZP_, SPS_>), grid, block, 0, stream, it, un, wb)
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
    return hipGetLastError();
}

int stream_kernel_waves_per_cu(int scale_f32, int has_zp, int sps) {
    int blocks = 0;
    hipError_t e = hipSuccess;
#define MNB_OCC(ST_, ZP_, SPS_) \
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, gemv_stream_kernel<ST_, ZP_, SPS_>, 64 * kStreamWaves, 0)
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
    if (e != hipSuccess || blocks < 1) blocks = 1;
    return blocks * kStreamWaves;
}

}  // namespace mnb
