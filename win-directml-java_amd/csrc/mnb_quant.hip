// mnb_quant.hip -- int4 quantization of a dense matrix on the device, and the
// read-back of a resident weight into the reference's arrays.
//
// The quantizer restates Qwen2Weights.quantizeDenseRowsToUInt4 with
// calculateUInt4QuantizationBlock and quantizeDenseBlockToUInt4
// (directml-inference/src/main/java/com/aresstack/windirectml/inference/qwen/
// Qwen2Weights.java:1352-1422): per block of bs values of a row,
//   max == min: |max| < 1e-8 -> scale 1, zp 0; max > 0 -> scale max/15, zp 0;
//               otherwise scale -min/15, zp 15
//   else:       scale = (max - min)/15, zp = clamp(round(-min/scale), 0, 15)
//   q = clamp(round(v/scale + zp), 0, 15)
// with fp32 IEEE division and addition and Java's Math.round (floor(v + 1/2),
// NaN -> 0, saturating), so the bytes equal the reference's.  It writes the
// tiled HBM layout directly: one wave per 16-row x 128-k tile, lane
// l = g*16 + r holding row r, k = 32j + 8g + (0..7) -- exactly the lane's
// 16-byte chunk of packed nibbles.
#include "mnb_device.h"

namespace mnb {

__device__ __forceinline__ int java_round_f(float a) {
    if (a != a) return 0;
    if (a >= 2147483647.0f) return 2147483647;
    if (a <= -2147483648.0f) return -2147483647 - 1;
    const float fl = floorf(a);
    const float diff = a - fl;  // exact
    return (int)fl + (diff >= 0.5f ? 1 : 0);
}

__device__ __forceinline__ int clamp_u4(int v) { return v < 0 ? 0 : (v > 15 ? 15 : v); }

template <typename InT>
__device__ __forceinline__ void load8(const InT *p, float *v);

template <>
__device__ __forceinline__ void load8<float>(const float *p, float *v) {
    const float4_t a = *(const float4_t *)p, b = *(const float4_t *)(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = a[i];
        v[4 + i] = b[i];
    }
}

template <>
__device__ __forceinline__ void load8<_Float16>(const _Float16 *p, float *v) {
    const half8_t a = *(const half8_t *)p;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (float)a[i];
}

template <typename InT, int BS>
__global__ __launch_bounds__(256) void quantize_tiles_kernel(WeightGeom g, const InT *__restrict__ data,
                                                             uint32_t *__restrict__ q_t, float *__restrict__ s_t,
                                                             uint8_t *__restrict__ zp_t) {
    constexpr int SPS = kTileK / BS;  // blocks of a row inside one super-tile
    constexpr int ZB = SPS <= 2 ? 1 : SPS / 2;
    const int lane = threadIdx.x & 63;
    const size_t t = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= (size_t)g.NT * g.ST) return;
    const int st = (int)(t % g.ST), nt = (int)(t / g.ST);
    const int r = lane & 15, gg = lane >> 4;
    const int n = nt * kTileRows + r;
    const int cols = g.K;  // a multiple of BS, so a block is entirely inside or outside [0, cols)

    float v[4][8];
    bool ok[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k0 = st * kTileK + 32 * j + 8 * gg;
        ok[j] = n < g.N && k0 < cols;
        if (ok[j]) {
            load8<InT>(data + (size_t)n * cols + k0, v[j]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[j][i] = 0.0f;
        }
    }

    // per-block min / max: lane-local, then across the four lanes of the row
    float mn[SPS], mx[SPS];
#pragma unroll
    for (int s = 0; s < SPS; ++s) {
        mn[s] = __builtin_inff();
        mx[s] = -__builtin_inff();
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (ok[j] && (32 * j + 8 * gg) / BS == s) {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    mn[s] = v[j][i] < mn[s] ? v[j][i] : mn[s];
                    mx[s] = v[j][i] > mx[s] ? v[j][i] : mx[s];
                }
            }
        }
#pragma unroll
        for (int m = 16; m <= 32; m <<= 1) {
            const float o_mn = __shfl_xor(mn[s], m), o_mx = __shfl_xor(mx[s], m);
            mn[s] = o_mn < mn[s] ? o_mn : mn[s];
            mx[s] = o_mx > mx[s] ? o_mx : mx[s];
        }
    }

    float sc[SPS];
    int zv[SPS];
#pragma unroll
    for (int s = 0; s < SPS; ++s) {
        const bool valid = n < g.N && st * kTileK + s * BS < cols;
        float scale = 0.0f;
        int z = 0;
        if (valid) {
            if (mx[s] == mn[s]) {
                if (fabsf(mx[s]) < 1.0e-8f) {
                    scale = 1.0f;
                } else if (mx[s] > 0.0f) {
                    scale = mx[s] / 15.0f;
                } else {
                    scale = -mn[s] / 15.0f;
                    z = 15;
                }
            } else {
                scale = (mx[s] - mn[s]) / 15.0f;
                z = clamp_u4(java_round_f(-mn[s] / scale));
            }
        }
        sc[s] = scale;
        zv[s] = z;
    }

    u32x4_t out;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float scj = 0.0f;
        int zj = 0;
#pragma unroll
        for (int s = 0; s < SPS; ++s)
            if ((32 * j + 8 * gg) / BS == s) {
                scj = sc[s];
                zj = zv[s];
            }
        uint32_t d = 0;
        if (ok[j]) {
            const float zf = (float)zj;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float tq = v[j][i] / scj + zf;
                const uint32_t nib = (uint32_t)clamp_u4(java_round_f(tq));
                d |= nib << ((i & 1) ? 16 + 4 * (i >> 1) : 4 * (i >> 1));
            }
        }
        out[j] = d;
    }
    *(u32x4_t *)(q_t + (t * 64 + lane) * 4) = out;

    if (gg == 0) {
        uint32_t bits = 0;
#pragma unroll
        for (int s = 0; s < SPS; ++s) {
            s_t[(t * kTileRows + r) * SPS + s] = sc[s];
            bits |= (uint32_t)zv[s] << (4 * s);
        }
#pragma unroll
        for (int b = 0; b < ZB; ++b) zp_t[(t * kTileRows + r) * ZB + b] = (uint8_t)(bits >> (8 * b));
    }
}

template <typename InT>
static hipError_t quantize_dispatch(const WeightGeom &g, const InT *data, void *q_t, float *s_t, uint8_t *zp_t,
                                    hipStream_t stream) {
    const size_t tiles = (size_t)g.NT * g.ST;
    const dim3 grid((unsigned)((tiles + 3) / 4)), block(256);
    switch (g.bs) {
    case 16:
        hipLaunchKernelGGL((quantize_tiles_kernel<InT, 16>), grid, block, 0, stream, g, data, (uint32_t *)q_t, s_t, zp_t);
        break;
    case 32:
        hipLaunchKernelGGL((quantize_tiles_kernel<InT, 32>), grid, block, 0, stream, g, data, (uint32_t *)q_t, s_t, zp_t);
        break;
    case 64:
        hipLaunchKernelGGL((quantize_tiles_kernel<InT, 64>), grid, block, 0, stream, g, data, (uint32_t *)q_t, s_t, zp_t);
        break;
    case 128:
        hipLaunchKernelGGL((quantize_tiles_kernel<InT, 128>), grid, block, 0, stream, g, data, (uint32_t *)q_t, s_t,
                           zp_t);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_quantize(const WeightGeom &g, const void *data, int32_t data_type, void *q_t, float *s_t,
                           uint8_t *zp_t, hipStream_t stream) {
    if (data_type == MNB_F32) return quantize_dispatch(g, (const float *)data, q_t, s_t, zp_t, stream);
    return quantize_dispatch(g, (const _Float16 *)data, q_t, s_t, zp_t, stream);
}

// ---------------------------------------------------------------------------
// read-back: tiled layout -> the reference's arrays
// ---------------------------------------------------------------------------

// Tiled dword -> natural dword (k0 in the low nibble ... k7 in the high one).
__device__ __forceinline__ uint32_t zip_nibbles(uint32_t t) {
    uint32_t s = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int pos = (i & 1) ? 16 + 4 * (i >> 1) : 4 * (i >> 1);
        s |= ((t >> pos) & 0xFu) << (4 * i);
    }
    return s;
}

__global__ void unpack_q_kernel(WeightGeom g, const uint32_t *__restrict__ q_t, uint8_t *__restrict__ q_nat) {
    const size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= (size_t)g.NT * g.ST * 64) return;
    const int lane = (int)(c & 63);
    const size_t tile = c >> 6;
    const int st = (int)(tile % g.ST), nt = (int)(tile / g.ST);
    const int r = lane & 15, gg = lane >> 4;
    const int n = nt * kTileRows + r;
    if (n >= g.N) return;
    const size_t row_bytes = (size_t)g.Kpad / 2;
    const u32x4_t in = *(const u32x4_t *)(q_t + c * 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k0 = st * kTileK + 32 * j + 8 * gg;
        if (k0 < g.Kpad) *(uint32_t *)(q_nat + (size_t)n * row_bytes + (size_t)(k0 / 2)) = zip_nibbles(in[j]);
    }
}

// One thread per (tile, row): the row's SPS scales and zero points of this
// super-tile; a block longer than a super-tile is written once, from the
// super-tile where it starts.  Zero points come out one byte per block (8
// when the weight has the implicit zero point).
template <typename ScaleT>
__global__ void unpack_scales_zp_kernel(WeightGeom g, const ScaleT *__restrict__ s_t, const uint8_t *__restrict__ zp_t,
                                        float *__restrict__ s_nat, uint8_t *__restrict__ zp_blocks) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= (size_t)g.NT * g.ST * kTileRows) return;
    const int r = (int)(e % kTileRows);
    const size_t tile = e / kTileRows;
    const int st = (int)(tile % g.ST), nt = (int)(tile / g.ST);
    const int n = nt * kTileRows + r;
    if (n >= g.N) return;
    uint32_t bits = 0;
    if (zp_t)
        for (int b = 0; b < g.ZB; ++b) bits |= (uint32_t)zp_t[e * g.ZB + b] << (8 * b);
    for (int i = 0; i < g.SPS; ++i) {
        const int blk = g.bs >= kTileK ? (st * kTileK) / g.bs : st * g.SPS + i;
        if (blk >= g.kb) continue;
        if (g.bs > kTileK && st * kTileK != blk * g.bs) continue;
        s_nat[(size_t)n * g.kb + blk] = (float)s_t[e * g.SPS + i] * pow2f(-g.fold_exp);
        zp_blocks[(size_t)n * g.kb + blk] = zp_t ? (uint8_t)((bits >> (4 * i)) & 0xFu) : (uint8_t)8;
    }
}

hipError_t launch_unpack(const mnb_weight *w, uint8_t *q_nat, float *s_nat, uint8_t *zp_blocks, hipStream_t stream) {
    const WeightGeom &g = w->g;
    const unsigned T = 256;
    const size_t nq = (size_t)g.NT * g.ST * 64;
    hipLaunchKernelGGL(unpack_q_kernel, dim3((unsigned)((nq + T - 1) / T)), dim3(T), 0, stream, g,
                       (const uint32_t *)w->q_t, q_nat);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const size_t ns = (size_t)g.NT * g.ST * kTileRows;
    const dim3 grid((unsigned)((ns + T - 1) / T));
    if (g.scale_f32)
        hipLaunchKernelGGL(unpack_scales_zp_kernel<float>, grid, dim3(T), 0, stream, g, (const float *)w->s_t,
                           (const uint8_t *)w->zp_t, s_nat, zp_blocks);
    else
        hipLaunchKernelGGL(unpack_scales_zp_kernel<_Float16>, grid, dim3(T), 0, stream, g, (const _Float16 *)w->s_t,
                           (const uint8_t *)w->zp_t, s_nat, zp_blocks);
    return hipGetLastError();
}

}  // namespace mnb
