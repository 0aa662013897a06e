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
// the M activation rows, M = 1 broadcasts x to every row), and the block
// scale is applied to the fp32 MFMA result (bs >= 32), so no weight is ever
// rounded.  bs = 16 (two scales per 32-k step) folds the scale into the fp16
// weight instead.
#include "mnb_device.h"

namespace mnb {

struct GemvParams {
    const u32x4_t *q_t;
    const void *s_t;
    const uint8_t *zp_t;
    const _Float16 *x;
    int32_t ldx, kx, M, N, ST;
    void *y;
    int32_t y_f16, accumulate;
};

template <bool F16>
__device__ __forceinline__ void store_y(void *y, size_t idx, float v, bool accumulate) {
    if constexpr (F16) {
        _Float16 *p = (_Float16 *)y + idx;
        if (accumulate) v += (float)*p;
        *p = (_Float16)v;
    } else {
        float *p = (float *)y + idx;
        if (accumulate) v += *p;
        *p = v;
    }
}

template <typename ScaleT, bool HAS_ZP, bool M1, int SPS>
__global__ __launch_bounds__(1024) void gemv_kernel(GemvParams p) {
    constexpr int ZB = SPS <= 2 ? 1 : SPS / 2;
    __shared__ float4_t red[16 * 64];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int W = blockDim.x >> 6;
    const int r = lane & 15, gg = lane >> 4;
    const int nt = blockIdx.x;
    const int st0 = (wave * p.ST) / W, st1 = ((wave + 1) * p.ST) / W;

    const size_t tile0 = (size_t)nt * p.ST;
    const u32x4_t *qp = p.q_t + tile0 * 64 + lane;
    const ScaleT *sp = (const ScaleT *)p.s_t + (tile0 * kTileRows + r) * SPS;
    const uint8_t *zpp = HAS_ZP ? p.zp_t + (tile0 * kTileRows + r) * ZB : nullptr;
    const int m = M1 ? 0 : (r < p.M ? r : p.M - 1);
    const _Float16 *xr = p.x + (size_t)m * p.ldx + 8 * gg;
    const half8_t zero8 = {};

    float4_t acc = {0.f, 0.f, 0.f, 0.f};

    for (int st = st0; st < st1; ++st) {
        const u32x4_t raw = qp[(size_t)st * 64];
        float s[SPS];
        load_scales<ScaleT, SPS>(sp + (size_t)st * kTileRows * SPS, s);
        uint32_t zb = 0x88888888u;
        if constexpr (HAS_ZP) zb = load_zp<ZB>(zpp + (size_t)st * kTileRows * ZB);
        half8_t xa[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = st * kTileK + 32 * j;
            xa[j] = (k + 8 * gg < p.kx) ? *(const half8_t *)(xr + k) : zero8;
        }
        if constexpr (SPS == 8) {
            // bs = 16: the lane's 8 k lie in block 2j + gg/2; fold the scale.
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = 2 * j + (gg >> 1);
                const uint32_t z = zp_nibble(zb, i);
                half8_t b = unpack_q_minus_zp(raw[j], bias_lo_pair(z), bias_hi_pair(z));
                b = b * (_Float16)s[i];
                acc = mfma16x16x32(xa[j], b, acc);
            }
        } else {
            constexpr int KPB = 4 / SPS;   // 32-k steps per scale block inside the super-tile
#pragma unroll
            for (int i = 0; i < SPS; ++i) {
                const uint32_t z = zp_nibble(zb, i);
                const uint32_t blo = bias_lo_pair(z), bhi = bias_hi_pair(z);
                float4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int t = 0; t < KPB; ++t) {
                    const int j = i * KPB + t;
                    d = mfma16x16x32(xa[j], unpack_q_minus_zp(raw[j], blo, bhi), d);
                }
                if constexpr (M1) {
                    acc[0] = fmaf(s[i], d[0], acc[0]);
                } else {
                    acc[0] = fmaf(s[i], d[0], acc[0]);
                    acc[1] = fmaf(s[i], d[1], acc[1]);
                    acc[2] = fmaf(s[i], d[2], acc[2]);
                    acc[3] = fmaf(s[i], d[3], acc[3]);
                }
            }
        }
    }

    if (W > 1) {
        red[wave * 64 + lane] = acc;
        __syncthreads();
        if (wave != 0) return;
        for (int w2 = 1; w2 < W; ++w2) {
            const float4_t o = red[w2 * 64 + lane];
            acc[0] += o[0];
            acc[1] += o[1];
            acc[2] += o[2];
            acc[3] += o[3];
        }
    }

    // D layout of the 16x16 MFMA result: lane (gg*16 + r) holds rows 4*gg+i, column r.
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
        for (int i = 0; i < 4; ++i) {
            const int mm = 4 * gg + i;
            if (mm < p.M) {
                const size_t idx = (size_t)mm * p.N + n;
                if (p.y_f16) store_y<true>(p.y, idx, acc[i], accum);
                else store_y<false>(p.y, idx, acc[i], accum);
            }
        }
    }
}

template <typename ScaleT, bool HAS_ZP, bool M1>
static hipError_t gemv_sps(const WeightGeom &g, dim3 grid, dim3 block, const GemvParams &p, hipStream_t s) {
    switch (g.SPS) {
        case 1: hipLaunchKernelGGL((gemv_kernel<ScaleT, HAS_ZP, M1, 1>), grid, block, 0, s, p); break;
        case 2: hipLaunchKernelGGL((gemv_kernel<ScaleT, HAS_ZP, M1, 2>), grid, block, 0, s, p); break;
        case 4: hipLaunchKernelGGL((gemv_kernel<ScaleT, HAS_ZP, M1, 4>), grid, block, 0, s, p); break;
        case 8: hipLaunchKernelGGL((gemv_kernel<ScaleT, HAS_ZP, M1, 8>), grid, block, 0, s, p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <typename ScaleT>
static hipError_t gemv_zp(const WeightGeom &g, dim3 grid, dim3 block, const GemvParams &p, bool m1, hipStream_t s) {
    if (g.has_zp) return m1 ? gemv_sps<ScaleT, true, true>(g, grid, block, p, s) : gemv_sps<ScaleT, true, false>(g, grid, block, p, s);
    return m1 ? gemv_sps<ScaleT, false, true>(g, grid, block, p, s) : gemv_sps<ScaleT, false, false>(g, grid, block, p, s);
}

// Waves per workgroup: about three super-tiles (3 x 16 B in flight) per wave.
static int gemv_waves(int ST) {
    int w = (ST + 2) / 3;
    if (w < 1) w = 1;
    if (w > 16) w = 16;
    return w;
}

hipError_t launch_gemv(const mnb_weight *w, const MatmulArgs &a, int32_t /*cu_count*/, hipStream_t stream) {
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
    dim3 grid(g.NT), block(64 * gemv_waves(g.ST));
    const bool m1 = a.M == 1;
    return g.scale_f32 ? gemv_zp<float>(g, grid, block, p, m1, stream)
                       : gemv_zp<_Float16>(g, grid, block, p, m1, stream);
}

}  // namespace mnb
