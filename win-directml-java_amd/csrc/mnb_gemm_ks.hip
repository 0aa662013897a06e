// mnb_gemm_ks.hip -- one product of a few hundred rows or fewer, K sliced
// over the waves of a workgroup.
//
// Replaces, for single products, the batched shader INT4_MATMUL_BATCH_TILED_HLSL
// (directml-windows-bindings/src/main/java/com/aresstack/windirectml/windows/
// MatMulNBitsKernel.java:732-820) where the stream-K GEMM has too few tiles,
// and for 9 <= M <= 16 the matvec shader's role (INT4_MATVEC_HLSL, :235-292)
// where its cost model beats the GEMV's:
// y[m,n] = sum_blk scale[n,blk] * sum_k (q[n,k]-zp[n,blk]) * x[m,k].
//
// Work decomposition: workgroup (m-block, n-group) computes 16 MB rows of y by
// 16 NTW columns (NTW n-tiles).  Its W waves take contiguous slices of the
// super-tiles (128 k each) and each wave keeps the whole output block in
// registers; the waves' partial blocks are summed in LDS in wave order, so
// results do not depend on timing.  No tile is split between workgroups:
// nothing goes through memory but y, and there is no second launch.
//
// Per super-tile a wave loads its NTW weight tiles (one 16-byte load per lane
// each, already in MFMA operand order), dequantizes them once into fp16
// ((q - zp) * scale, as the GEMM does) and uses them for all MB row blocks of
// x.  Each 16-row x block (16 x 128 fp16) is loaded row-contiguous (lane l
// brings 16 bytes of row 4 i + l / 16, so a load covers four whole 256-byte
// row pieces), goes through a 4 KiB wave-private LDS block into operand
// order, and feeds 4 x NTW
// v_mfma_f32_16x16x32_f16 (weights as A, x as B, so a lane's four results
// are four consecutive columns of one row).  The next x
// block is in flight while the current one is multiplied, and the next
// super-tile's weights while the current one's row blocks run.  All loads are
// ordinary loads, so the compiler places every wait.  (Two x blocks, or two
// and three super-tiles of weights, in flight measured no faster: at these
// sizes a workgroup is bound by its CU's dequantization and MFMA issue.)
#include <algorithm>

#include "mnb_device.h"

namespace mnb {

typedef uint32_t u32x4_ks_alias_t __attribute__((ext_vector_type(4), may_alias));
typedef _Float16 half8_ks_alias_t __attribute__((ext_vector_type(8), may_alias));
typedef float float4_ks_alias_t __attribute__((ext_vector_type(4), may_alias));

constexpr int kKsRoundUnits = 4;   // 16x16 output units per LDS reduction round

template <typename ScaleT, bool HAS_ZP, int SPS, int MB, int NTW>
__global__ __launch_bounds__(64 * kKsMaxWaves) void gemm_ks_kernel(KsParams p) {
    constexpr int ZB = SPS <= 2 ? 1 : SPS / 2;
    constexpr int U = MB * NTW;
    // wave-private x blocks in the main loop; the reduction rounds reuse the
    // space (kKsMaxWaves x kKsRoundUnits x 1 KiB)
    __shared__ __align__(16) unsigned char smem[kKsMaxWaves * 4096];
    static_assert(kKsRoundUnits * 1024 <= 4096, "a round must fit the x blocks' space");

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int W = blockDim.x >> 6;
    const int r = lane & 15, gg = lane >> 4;
    const int mblk = blockIdx.x % p.mblk;
    const int ng = blockIdx.x / p.mblk;
    const int m0 = mblk * 16 * MB;
    const int s0 = wave * p.ST / W, s1 = (wave + 1) * p.ST / W;   // s0 < s1: W <= ST
    const uint32_t k6400 = vgpr_const(0x64006400u);
    const u32x4_t zero4 = {0u, 0u, 0u, 0u};

    float4_t acc[MB][NTW];
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int t = 0; t < NTW; ++t) acc[b][t] = (float4_t){0.f, 0.f, 0.f, 0.f};

    unsigned char *xw = smem + wave * 4096;
    // byte offset of this lane's x row piece in row block b, load i: row
    // m0 + 16 b + 4 i + gg, where rows >= M repeat row M - 1 (their results
    // are never stored)
    const uint32_t ldx2 = (uint32_t)p.ldx * 2u;
    const uint32_t xrow0 = (uint32_t)(m0 + gg) * ldx2, xlast = (uint32_t)(p.M - 1) * ldx2;
    auto xr = [&](int b, int i) __attribute__((always_inline)) -> uint32_t {
        return min(xrow0 + (uint32_t)(16 * b + 4 * i) * ldx2, xlast);
    };
    const unsigned char *xb0 = (const unsigned char *)p.x;
    // tiles of this workgroup's n-tiles (past the last n-tile: the last one
    // again, whose extra results are never stored)
    size_t tile0[NTW];
#pragma unroll
    for (int t = 0; t < NTW; ++t) tile0[t] = (size_t)min(ng * NTW + t, p.NT - 1) * p.ST;

    u32x4_t raw[NTW];
    ScaleT sv[NTW][SPS];
    uint32_t zb[NTW];
    auto issue_w = [&](int s) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < NTW; ++t) {
            const size_t tile = tile0[t] + s;
            raw[t] = gld((const u32x4_t *)p.q_t + tile * 64 + lane);
            load_scale_row<ScaleT, SPS>((const ScaleT *)p.s_t + (tile * kTileRows + r) * SPS, sv[t]);
            if constexpr (HAS_ZP) zb[t] = load_zp<ZB>(p.zp_t + (tile * kTileRows + r) * ZB);
            else zb[t] = 0x88888888u;
        }
    };
    // x block (s, b): k offset of the lane's 16 bytes, clamped into the row
    // where the super-tile runs past kx (those pieces are zeroed when written
    // to LDS)
    auto x_off = [&](int s) __attribute__((always_inline)) -> uint32_t {
        return (uint32_t)min(s * kTileK + 8 * r, p.kx - 8) * 2u;
    };
    u32x4_t xc[4], xn[4];
    auto issue_x = [&](u32x4_t(&v)[4], int b, uint32_t ko) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = gld((const u32x4_t *)(xb0 + xr(b, i) + ko));
    };

    half8_t wq[NTW][4];
    auto dequant = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < NTW; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                // scale block of k-step j: the lane's 8 k lie in block 2 j + gg / 2 when bs = 16
                ScaleT sc;
                uint32_t z;
                if constexpr (SPS == 8) {
                    sc = (gg >> 1) ? sv[t][2 * j + 1] : sv[t][2 * j];
                    z = HAS_ZP ? zp_nibble(zb[t], 2 * j + (gg >> 1)) : 8u;
                } else {
                    sc = sv[t][j * SPS / 4];
                    z = HAS_ZP ? zp_nibble(zb[t], j * SPS / 4) : 8u;
                }
                half8_t w = unpack_q_minus_zp(raw[t][j], bias_lo_pair(z), bias_hi_pair(z), k6400);
                if constexpr (sizeof(ScaleT) == 2) {
                    w = w * (_Float16)sc;
                } else {
                    const float sf = (float)sc;
#pragma unroll
                    for (int e = 0; e < 8; ++e) w[e] = (_Float16)((float)w[e] * sf);
                }
                wq[t][j] = w;
            }
    };

    issue_w(s0);
    issue_x(xc, 0, x_off(s0));
    for (int s = s0; s < s1; ++s) {
        dequant();
        __builtin_amdgcn_sched_barrier(0);
        // the next super-tile's weights (the last one again at the end:
        // loaded, never used)
        const int sn = min(s + 1, s1 - 1);
        issue_w(sn);
        const uint32_t ko = x_off(s), kn = x_off(sn);
        const bool kok = s * kTileK + 8 * r < p.kx;
#pragma unroll
        for (int b = 0; b < MB; ++b) {
            if (b + 1 < MB) issue_x(xn, b + 1, ko);
            else issue_x(xn, 0, kn);
            // keep each phase in place: the scheduler would otherwise pull the
            // next block's LDS writes, which wait for its loads, into this
            // block's MFMAs
            __builtin_amdgcn_sched_barrier(0);
            // 16-byte piece (row, chunk) at row * 256 + ((chunk ^ row) % 16) * 16:
            // the eight lanes of a write (one row, eight chunks) or of a read
            // (eight rows, one chunk each) hit distinct banks.  The wave's LDS
            // operations run in order; the compiler barriers keep the reads
            // after the writes and the next block's writes after the reads.
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 4 * i + gg;
                *(u32x4_ks_alias_t *)(xw + row * 256 + ((r ^ row) & 15) * 16) = kok ? xc[i] : zero4;
            }
            asm volatile("" ::: "memory");
            half8_t xa[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) xa[j] = *(const half8_ks_alias_t *)(xw + r * 256 + (((4 * j + gg) ^ r) & 15) * 16);
            asm volatile("" ::: "memory");
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int t = 0; t < NTW; ++t) acc[b][t] = mfma16x16x32(wq[t][j], xa[j], acc[b][t]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 4; ++i) xc[i] = xn[i];
        }
    }

    // Sum the waves' partial blocks: per round, every wave writes
    // kKsRoundUnits of its 16x16 units to LDS, then unit q of the round is
    // summed over waves 0..W-1 (in that order) and stored by wave q mod W.
    __syncthreads();   // every wave is done with its ring
    float4_ks_alias_t *red = (float4_ks_alias_t *)smem;
    const int n_grp = ng * NTW * kTileRows;
#pragma unroll
    for (int r0 = 0; r0 < U; r0 += kKsRoundUnits) {
#pragma unroll
        for (int q = 0; q < kKsRoundUnits; ++q)
            if (r0 + q < U) red[(wave * kKsRoundUnits + q) * 64 + lane] = acc[(r0 + q) / NTW][(r0 + q) % NTW];
        __syncthreads();
        for (int q = wave; q < kKsRoundUnits && r0 + q < U; q += W) {
            float4_t v = red[q * 64 + lane];
            for (int w2 = 1; w2 < W; ++w2) {
                const float4_t o = red[(w2 * kKsRoundUnits + q) * 64 + lane];
                v[0] += o[0];
                v[1] += o[1];
                v[2] += o[2];
                v[3] += o[3];
            }
            // unit (b, t): lane (gg, r) holds row m0 + 16 b + r, columns n .. n + 3
            const int u = r0 + q, b = u / NTW, t = u % NTW;
            const int m = m0 + 16 * b + r;
            const int n = n_grp + t * kTileRows + 4 * gg;
            if (m < p.M && n < p.N) {
                // undo the stored scales' factor 2^fold_exp (exact)
                v[0] *= p.unfold;
                v[1] *= p.unfold;
                v[2] *= p.unfold;
                v[3] *= p.unfold;
                const size_t idx = (size_t)m * p.N + n;
                const bool acc_y = p.accumulate != 0;
                if (p.y_vec && n + 3 < p.N) {
                    if (p.y_f16) {
                        __attribute__((address_space(1))) half2_t *yp =
                            (__attribute__((address_space(1))) half2_t *)((_Float16 *)p.y + idx);
                        if (acc_y) {
                            const half2_t o0 = yp[0], o1 = yp[1];
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
                        *(__attribute__((address_space(1))) u32x2_t *)yp = (u32x2_t){as_u32(h0), as_u32(h1)};
                    } else {
                        __attribute__((address_space(1))) float4_t *yp =
                            (__attribute__((address_space(1))) float4_t *)((float *)p.y + idx);
                        if (acc_y) v += *yp;
                        *yp = v;
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n + e < p.N) {
                            if (p.y_f16) store_y<true>(p.y, idx + e, v[e], acc_y);
                            else store_y<false>(p.y, idx + e, v[e], acc_y);
                        }
                }
            }
        }
        __syncthreads();   // the next round overwrites the LDS
    }
}

template <typename ScaleT, bool HAS_ZP, int SPS>
static hipError_t ks_shape(const KsConfig &c, dim3 grid, dim3 block, hipStream_t s, const KsParams &p) {
#define MNB_KS(MB_, NTW_)                                                                               \
    if (c.mb == MB_ && c.ntw == NTW_) {                                                                 \
        hipLaunchKernelGGL((gemm_ks_kernel<ScaleT, HAS_ZP, SPS, MB_, NTW_>), grid, block, 0, s, p);     \
        return hipGetLastError();                                                                       \
    }
    MNB_KS(1, 4)
    MNB_KS(2, 1)
    MNB_KS(2, 2)
    MNB_KS(2, 4)
    // 16 output units per wave: compiled where ks_config_supported allows it
    if constexpr (SPS != 8 && !(sizeof(ScaleT) == 4 && HAS_ZP)) MNB_KS(4, 4)
#undef MNB_KS
    return hipErrorInvalidValue;
}

template <typename ScaleT, bool HAS_ZP>
static hipError_t ks_sps(int sps, const KsConfig &c, dim3 grid, dim3 block, hipStream_t s, const KsParams &p) {
    switch (sps) {
        case 1: return ks_shape<ScaleT, HAS_ZP, 1>(c, grid, block, s, p);
        case 2: return ks_shape<ScaleT, HAS_ZP, 2>(c, grid, block, s, p);
        case 4: return ks_shape<ScaleT, HAS_ZP, 4>(c, grid, block, s, p);
        case 8: return ks_shape<ScaleT, HAS_ZP, 8>(c, grid, block, s, p);
        default: return hipErrorInvalidValue;
    }
}

// Products with 9 <= M <= 16: the GEMV (one workgroup per n-tile, so every
// n-tile reads all 16 x rows again) or this kernel with 16 x 64 output blocks
// (x read once per four n-tiles, each weight tile dequantized once).  Model
// of either launch, fitted to timings on MI355X of 40 shapes (K 896 to
// 14336, N 896 to 151936, the weights read from HBM) at M = 12 and 16 for the
// GEMV (median error 4%) and M = 2 to 16 for this kernel (at M <= 8 a copy
// that loaded only the x row groups below M; median error 5.5% at M = 12 and
// 16; a fit to M = 12 and 16 alone misjudged the 3072 -> 9216 product by 20%
// and lost its 24% gain): c plus the
// longest of a workgroup's chain of super-tiles per wave (per round of
// workgroups), the weight bytes at the chip's rate, the weight bytes at the
// rate of the CUs the grid occupies, and the L2 reads (1 KiB of weights and
// 4 KiB of x per tile of an n-tile group), plus a cost per workgroup.  Sizes
// in KiB, times in us.  With M <= 8 the GEMV loads only one or two groups of
// four x rows; there it was faster than this kernel, or within the models'
// error, on every shape timed, and it always runs.  (16 x 16 and 16 x 32
// blocks were timed too: with their fitted costs the choice gained nothing.)
struct SkinnyCost {
    double c, lat, bw, bw_cu, bw_l2, per_wg;
};
static const SkinnyCost kSkinnyGemv = {2.6154, 0.3196, 2343.2, 11.564, 11678.7, 0.0};
static const SkinnyCost kSkinnyKs = {2.6868, 1.3758, 4589.1, 22.452, 8273.8, 1.4969};
constexpr int kSkinnyMinM = 9, kSkinnyNTW = 4;
// This kernel runs only where its estimate is this fraction of the GEMV's or
// less.  Over the shapes timed at M = 12 and 16: the GEMV alone 840 us in
// total, this choice 738 (no shape slower than with the GEMV), the faster
// kernel per shape 737.
constexpr double kSkinnyMargin = 0.92;

static double skinny_est(const SkinnyCost &k, int64_t wgs, int spw, double w_kib, double l2_kib, int cu) {
    const double chain = (double)((wgs + cu - 1) / cu) * spw * k.lat;
    const double occupied = (double)std::min<int64_t>(wgs, cu);
    const double t = std::max(std::max(chain, w_kib / k.bw), std::max(w_kib / (k.bw_cu * occupied), l2_kib / k.bw_l2));
    return k.c + t + k.per_wg * (double)wgs / cu;
}

KsPlan ks_skinny_plan(const WeightGeom &g, int32_t M, int32_t cu_count) {
    KsPlan none{{0, 0}, 0.0, 0};
    if (M < kSkinnyMinM || M > kSkinnyMaxM || g.ST < 1) return none;
    // the launch limits of launch_gemm_ks (x rows padded to a multiple of 8)
    if ((uint64_t)g.NT * (uint64_t)g.ST * kTileBytes >= ((uint64_t)1 << 32)) return none;
    if ((int64_t)M * ((g.K + 7) & ~7) * 2 > ((int64_t)1 << 31)) return none;
    const KsConfig c{1, kSkinnyNTW};
    if (!ks_config_supported(c.mb, c.ntw, g.scale_f32, g.has_zp, g.SPS)) return none;
    const int cu = cu_count > 0 ? cu_count : 256;
    const int ST = g.ST;
    const double w_kib = (double)g.NT * ST;
    // the GEMV: waves of 2 super-tiles, at most kGemvMaxWavesRows of them, looping beyond
    const int gw = std::min((ST + 1) / 2, kGemvMaxWavesRows);
    const int gspw = std::min(ST > 2 * gw ? (ST + 2 * gw - 1) / (2 * gw) * 2 : 2, ST);
    none.est = skinny_est(kSkinnyGemv, g.NT, gspw, w_kib, w_kib * 5.0, cu);
    // this kernel: ks_waves(ST) waves on contiguous K slices
    const int kw = ks_waves(ST);
    const int64_t wgs = ks_workgroups(M, g.NT, c);
    const double est = skinny_est(kSkinnyKs, wgs, (ST + kw - 1) / kw, w_kib, w_kib * (1.0 + 4.0 / c.ntw), cu);
    return est <= kSkinnyMargin * none.est ? KsPlan{c, est, wgs} : none;
}


hipError_t launch_gemm_ks(const mnb_weight *w, const MatmulArgs &a, const KsConfig &c, hipStream_t stream) {
    const WeightGeom &g = w->g;
    if (!ks_config_supported(c.mb, c.ntw, g.scale_f32, g.has_zp, g.SPS) || a.M < 1 || g.ST < 1) return hipErrorInvalidValue;
    // 32-bit byte offsets into x (rows come in chunks of at most 2 GiB) and
    // into the scales and zero points (packed weights below 4 GiB)
    if ((int64_t)a.M * a.ldx * 2 > ((int64_t)1 << 31)) return hipErrorInvalidValue;
    if ((uint64_t)g.NT * (uint64_t)g.ST * kTileBytes >= ((uint64_t)1 << 32)) return hipErrorInvalidValue;
    const int64_t wgs = ks_workgroups(a.M, g.NT, c);
    if (wgs > 0x7fffffff) return hipErrorInvalidValue;
    KsParams p;
    p.q_t = w->q_t;
    p.s_t = w->s_t;
    p.zp_t = (const uint8_t *)w->zp_t;
    p.x = a.x;
    p.y = a.y;
    p.ldx = a.ldx;
    p.kx = a.kx;
    p.M = a.M;
    p.N = g.N;
    p.NT = g.NT;
    p.ST = g.ST;
    p.mblk = (a.M + 16 * c.mb - 1) / (16 * c.mb);
    p.y_f16 = a.y_type == MNB_F16;
    p.accumulate = a.accumulate;
    p.y_vec = (g.N % 4 == 0) && ((uintptr_t)a.y % (p.y_f16 ? 8 : 16) == 0);
    p.unfold = pow2f(-g.fold_exp);
    const dim3 grid((unsigned)wgs), block(64 * ks_waves(g.ST));
    if (g.scale_f32)
        return g.has_zp ? ks_sps<float, true>(g.SPS, c, grid, block, stream, p)
                        : ks_sps<float, false>(g.SPS, c, grid, block, stream, p);
    return g.has_zp ? ks_sps<_Float16, true>(g.SPS, c, grid, block, stream, p)
                    : ks_sps<_Float16, false>(g.SPS, c, grid, block, stream, p);
}

}  // namespace mnb
