// mnb_gemm.hip -- prefill-shaped MatMulNBits (M > 16) on fp16 MFMA.
//
// Replaces the tiled HLSL batch GEMM INT4_MATMUL_BATCH_TILED_HLSL
// (directml-windows-bindings/src/main/java/com/aresstack/windirectml/windows/
// MatMulNBitsKernel.java:732-820) and its 256-row host chunking (:2374-2387):
// any M runs in one launch.
//
// Per 128-k stage a workgroup stages an x tile [BM x 128] and the packed
// weight tiles of its BN rows into registers, dequantizes the weights once
// into LDS as fp16 (w = (q - zp) * scale, the scale folded into the fp16
// operand), and its waves run v_mfma_f32_16x16x32_f16 over the two LDS
// tiles with fp32 accumulation.  Global loads for stage s+1 are issued
// before the MFMAs of stage s.
#include "mnb_device.h"

namespace mnb {

struct GemmParams {
    const u32x4_t *q_t;
    const void *s_t;
    const uint8_t *zp_t;
    const _Float16 *x;
    int32_t ldx, kx, M, N, NT, ST;
    void *y;
    int32_t y_f16, accumulate;
};

constexpr int kLdsRow = kTileK + 8;   // halves per LDS row (16-byte pad against bank conflicts)

template <typename ScaleT, bool HAS_ZP, int SPS, int WM, int WN, int SM, int SN>
__global__ __launch_bounds__(64 * WM * WN) void gemm_kernel(GemmParams p) {
    constexpr int ZB = SPS <= 2 ? 1 : SPS / 2;
    constexpr int NTHR = 64 * WM * WN;
    constexpr int BM = WM * SM * 16;
    constexpr int BN = WN * SN * 16;
    constexpr int BNT = BN / kTileRows;                 // n-tiles per workgroup
    constexpr int A_PER_T = BM * (kTileK / 8) / NTHR;    // 16-byte x chunks per thread per stage
    constexpr int B_PER_T = BNT * 64 / NTHR;             // 16-byte weight chunks per thread per stage
    static_assert(A_PER_T * NTHR == BM * (kTileK / 8), "x tile must split evenly");
    static_assert(B_PER_T * NTHR == BNT * 64, "weight tile must split evenly");

    __shared__ _Float16 As[BM * kLdsRow];
    __shared__ _Float16 Bs[BN * kLdsRow];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int r = lane & 15, gg = lane >> 4;
    const int m0 = blockIdx.x * BM;
    const int nt0 = blockIdx.y * BNT;
    const ScaleT *sbase = (const ScaleT *)p.s_t;
    const uint32_t k6400 = vgpr_const(0x64006400u);

    u32x4_t a_reg[A_PER_T];
    u32x4_t b_reg[B_PER_T];
    ScaleT b_s[B_PER_T][SPS];
    uint32_t b_z[B_PER_T];

    auto load_stage = [&](int st) {
#pragma unroll
        for (int i = 0; i < A_PER_T; ++i) {
            const int c = tid + i * NTHR;
            const int row = c >> 4, cc = c & 15;
            int gm = m0 + row;
            gm = gm < p.M ? gm : p.M - 1;
            const int k = st * kTileK + cc * 8;
            const u32x4_t z4 = {0u, 0u, 0u, 0u};
            a_reg[i] = k < p.kx ? *(const u32x4_t *)(p.x + (size_t)gm * p.ldx + k) : z4;
        }
#pragma unroll
        for (int i = 0; i < B_PER_T; ++i) {
            const int c = tid + i * NTHR;
            const int ntl = c >> 6, ln = c & 63;
            const int nt = nt0 + ntl;
            const u32x4_t z4 = {0u, 0u, 0u, 0u};
            if (nt < p.NT) {
                const size_t tile = (size_t)nt * p.ST + st;
                b_reg[i] = p.q_t[tile * 64 + ln];
                const ScaleT *sp = sbase + (tile * kTileRows + (ln & 15)) * SPS;
#pragma unroll
                for (int t = 0; t < SPS; ++t) b_s[i][t] = sp[t];
                if constexpr (HAS_ZP) b_z[i] = load_zp<ZB>(p.zp_t + (tile * kTileRows + (ln & 15)) * ZB);
                else b_z[i] = 0x88888888u;
            } else {
                b_reg[i] = z4;
#pragma unroll
                for (int t = 0; t < SPS; ++t) b_s[i][t] = (ScaleT)0;
                b_z[i] = 0u;
            }
        }
    };

    auto store_stage = [&]() {
#pragma unroll
        for (int i = 0; i < A_PER_T; ++i) {
            const int c = tid + i * NTHR;
            const int row = c >> 4, cc = c & 15;
            *(u32x4_t *)&As[row * kLdsRow + cc * 8] = a_reg[i];
        }
#pragma unroll
        for (int i = 0; i < B_PER_T; ++i) {
            const int c = tid + i * NTHR;
            const int ntl = c >> 6, ln = c & 63;
            const int rr = ln & 15, g2 = ln >> 4;
            _Float16 *dst = &Bs[(ntl * kTileRows + rr) * kLdsRow + 8 * g2];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int si = SPS == 8 ? 2 * j + (g2 >> 1) : (SPS == 1 ? 0 : j / (4 / SPS));
                const uint32_t z = HAS_ZP ? zp_nibble(b_z[i], si) : 8u;
                half8_t w = unpack_q_minus_zp(b_reg[i][j], bias_lo_pair(z), bias_hi_pair(z), k6400);
                if constexpr (sizeof(ScaleT) == 2) {
                    w = w * (_Float16)b_s[i][si];
                } else {
                    const float sf = (float)b_s[i][si];
#pragma unroll
                    for (int e = 0; e < 8; ++e) w[e] = (_Float16)((float)w[e] * sf);
                }
                *(half8_t *)(dst + 32 * j) = w;
            }
        }
    };

    float4_t acc[SM][SN];
#pragma unroll
    for (int a = 0; a < SM; ++a)
#pragma unroll
        for (int b = 0; b < SN; ++b) acc[a][b] = (float4_t){0.f, 0.f, 0.f, 0.f};

    load_stage(0);
    for (int st = 0; st < p.ST; ++st) {
        store_stage();
        __syncthreads();
        if (st + 1 < p.ST) load_stage(st + 1);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            half8_t af[SM], bf[SN];
#pragma unroll
            for (int a = 0; a < SM; ++a)
                af[a] = *(const half8_t *)&As[((wm * SM + a) * 16 + r) * kLdsRow + 32 * j + 8 * gg];
#pragma unroll
            for (int b = 0; b < SN; ++b)
                bf[b] = *(const half8_t *)&Bs[((wn * SN + b) * 16 + r) * kLdsRow + 32 * j + 8 * gg];
#pragma unroll
            for (int a = 0; a < SM; ++a)
#pragma unroll
                for (int b = 0; b < SN; ++b) acc[a][b] = mfma16x16x32(af[a], bf[b], acc[a][b]);
        }
        __syncthreads();
    }

    const bool accum = p.accumulate != 0;
#pragma unroll
    for (int a = 0; a < SM; ++a) {
#pragma unroll
        for (int b = 0; b < SN; ++b) {
            const int n = (nt0 + wn * SN + b) * 16 + r;
            if (n >= p.N) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int mm = m0 + (wm * SM + a) * 16 + 4 * gg + i;
                if (mm < p.M) {
                    const size_t idx = (size_t)mm * p.N + n;
                    float v = acc[a][b][i];
                    if (p.y_f16) {
                        _Float16 *yp = (_Float16 *)p.y + idx;
                        if (accum) v += (float)*yp;
                        *yp = (_Float16)v;
                    } else {
                        float *yp = (float *)p.y + idx;
                        if (accum) v += *yp;
                        *yp = v;
                    }
                }
            }
        }
    }
}

template <typename ScaleT, bool HAS_ZP>
static hipError_t gemm_sps(const WeightGeom &g, const GemmParams &p, hipStream_t s) {
    constexpr int WM = 2, WN = 2, SM = 4, SN = 4;
    constexpr int BM = WM * SM * 16, BNT = WN * SN;
    dim3 grid((p.M + BM - 1) / BM, (g.NT + BNT - 1) / BNT), block(64 * WM * WN);
    switch (g.SPS) {
        case 1: hipLaunchKernelGGL((gemm_kernel<ScaleT, HAS_ZP, 1, WM, WN, SM, SN>), grid, block, 0, s, p); break;
        case 2: hipLaunchKernelGGL((gemm_kernel<ScaleT, HAS_ZP, 2, WM, WN, SM, SN>), grid, block, 0, s, p); break;
        case 4: hipLaunchKernelGGL((gemm_kernel<ScaleT, HAS_ZP, 4, WM, WN, SM, SN>), grid, block, 0, s, p); break;
        case 8: hipLaunchKernelGGL((gemm_kernel<ScaleT, HAS_ZP, 8, WM, WN, SM, SN>), grid, block, 0, s, p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemm(const mnb_weight *w, const MatmulArgs &a, int32_t /*cu_count*/, hipStream_t stream) {
    const WeightGeom &g = w->g;
    GemmParams p;
    p.q_t = (const u32x4_t *)w->q_t;
    p.s_t = w->s_t;
    p.zp_t = (const uint8_t *)w->zp_t;
    p.x = a.x;
    p.ldx = a.ldx;
    p.kx = a.kx;
    p.M = a.M;
    p.N = g.N;
    p.NT = g.NT;
    p.ST = g.ST;
    p.y = a.y;
    p.y_f16 = a.y_type == MNB_F16;
    p.accumulate = a.accumulate;
    if (g.scale_f32) return g.has_zp ? gemm_sps<float, true>(g, p, stream) : gemm_sps<float, false>(g, p, stream);
    return g.has_zp ? gemm_sps<_Float16, true>(g, p, stream) : gemm_sps<_Float16, false>(g, p, stream);
}

}  // namespace mnb
