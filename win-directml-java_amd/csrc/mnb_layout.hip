// mnb_layout.hip -- one-time weight repack into the tiled HBM layout, the
// activation staging kernel and the dequantize-only kernel.
//
// The dequantize-only kernel restates MatMulNBitsKernel.dequantizeInt4
// (directml-windows-bindings/src/main/java/com/aresstack/windirectml/windows/
// MatMulNBitsKernel.java:2674-2705): w = float(nibble - zp) * scale in fp32,
// low nibble first.  Its fp32 output is bit-identical to that function.
#include "mnb_device.h"

namespace mnb {

WeightGeom make_geom(int32_t N, int32_t K, int32_t bs) {
    WeightGeom g;
    g.N = N;
    g.K = K;
    g.bs = bs;
    g.kb = (K + bs - 1) / bs;
    g.Kpad = g.kb * bs;
    g.NT = (N + kTileRows - 1) / kTileRows;
    g.ST = (g.Kpad + kTileK - 1) / kTileK;
    g.SPS = bs >= kTileK ? 1 : kTileK / bs;
    g.ZB = g.SPS <= 2 ? 1 : g.SPS / 2;
    return g;
}

// Natural packed dword (k0 | k1<<4 | ... | k7<<28, bytes low nibble first)
// -> tiled order (k0,k2,k4,k6 in bits 0..15; k1,k3,k5,k7 in bits 16..31).
__device__ __forceinline__ uint32_t unzip_nibbles(uint32_t s) {
    uint32_t t = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint32_t nib = (s >> (4 * i)) & 0xFu;
        int pos = (i & 1) ? 16 + 4 * (i >> 1) : 4 * (i >> 1);
        t |= nib << pos;
    }
    return t;
}

// Tiled dword -> natural nibble i (0..7) of its 8 consecutive k.
__device__ __forceinline__ uint32_t tiled_nibble(uint32_t t, int i) {
    int pos = (i & 1) ? 16 + 4 * (i >> 1) : 4 * (i >> 1);
    return (t >> pos) & 0xFu;
}

__global__ void repack_q_kernel(WeightGeom g, const uint8_t *__restrict__ q_nat, uint32_t *__restrict__ q_t) {
    const size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x;   // one lane chunk (16 bytes)
    const size_t total = (size_t)g.NT * g.ST * 64;
    if (c >= total) return;
    const int lane = (int)(c & 63);
    const size_t tile = c >> 6;
    const int st = (int)(tile % g.ST);
    const int nt = (int)(tile / g.ST);
    const int r = lane & 15, gg = lane >> 4;
    const int n = nt * kTileRows + r;
    const size_t row_bytes = (size_t)g.Kpad / 2;
    u32x4_t out;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int k0 = st * kTileK + 32 * j + 8 * gg;
        uint32_t v = 0;
        if (n < g.N && k0 < g.Kpad) {
            const uint32_t s = *(const uint32_t *)(q_nat + (size_t)n * row_bytes + (size_t)(k0 / 2));
            v = unzip_nibbles(s);
        }
        out[j] = v;
    }
    *(u32x4_t *)(q_t + c * 4) = out;
}

// s * 2^e rounded to the scale type (exact: the product stays within the
// type's finite range by the choice of the exponents).  The fp32 product is
// kept in a register first: fused into one mixed-precision multiply-add with a
// +0 addend, a -0 scale would come out as +0.
template <typename ScaleT, typename SrcT>
__device__ __forceinline__ ScaleT scaled(SrcT s, float factor) {
    float f = (float)s * factor;
    asm volatile("" : "+v"(f));
    return (ScaleT)f;
}

// Scales in tile order, times 2^fold_exp.
template <typename ScaleT>
__global__ void repack_scales_kernel(WeightGeom g, const ScaleT *__restrict__ s_nat, ScaleT *__restrict__ s_t) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)g.NT * g.ST * kTileRows * g.SPS;
    if (e >= total) return;
    const int i = (int)(e % g.SPS);
    const size_t rest = e / g.SPS;
    const int r = (int)(rest % kTileRows);
    const size_t tile = rest / kTileRows;
    const int st = (int)(tile % g.ST);
    const int nt = (int)(tile / g.ST);
    const int n = nt * kTileRows + r;
    const int blk = g.bs >= kTileK ? (st * kTileK) / g.bs : st * g.SPS + i;
    ScaleT v = (ScaleT)0;
    if (n < g.N && blk < g.kb) v = scaled<ScaleT>(s_nat[(size_t)n * g.kb + blk], pow2f(g.fold_exp));
    s_t[e] = v;
}

__global__ void repack_zp_kernel(WeightGeom g, const uint8_t *__restrict__ zp_flat, uint8_t *__restrict__ zp_t) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)g.NT * g.ST * kTileRows;
    if (e >= total) return;
    const int r = (int)(e % kTileRows);
    const size_t tile = e / kTileRows;
    const int st = (int)(tile % g.ST);
    const int nt = (int)(tile / g.ST);
    const int n = nt * kTileRows + r;
    uint32_t bits = 0;
    for (int i = 0; i < g.SPS; ++i) {
        const int blk = g.bs >= kTileK ? (st * kTileK) / g.bs : st * g.SPS + i;
        if (n < g.N && blk < g.kb) {
            const size_t idx = (size_t)n * g.kb + blk;
            const uint32_t nib = (zp_flat[idx / 2] >> (4 * (idx & 1))) & 0xFu;
            bits |= nib << (4 * i);
        }
    }
    for (int b = 0; b < g.ZB; ++b) zp_t[e * g.ZB + b] = (uint8_t)(bits >> (8 * b));
}

static inline unsigned blocks_for(size_t n, unsigned t) { return (unsigned)((n + t - 1) / t); }

hipError_t launch_repack(const WeightGeom &g, const uint8_t *q_nat, const void *s_nat, const uint8_t *zp_flat,
                         void *q_t, void *s_t, void *zp_t, hipStream_t stream) {
    const unsigned T = 256;
    size_t nq = (size_t)g.NT * g.ST * 64;
    hipLaunchKernelGGL(repack_q_kernel, dim3(blocks_for(nq, T)), dim3(T), 0, stream, g, q_nat, (uint32_t *)q_t);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    size_t ns = (size_t)g.NT * g.ST * kTileRows * g.SPS;
    if (g.scale_f32)
        hipLaunchKernelGGL(repack_scales_kernel<float>, dim3(blocks_for(ns, T)), dim3(T), 0, stream, g,
                           (const float *)s_nat, (float *)s_t);
    else
        hipLaunchKernelGGL(repack_scales_kernel<_Float16>, dim3(blocks_for(ns, T)), dim3(T), 0, stream, g,
                           (const _Float16 *)s_nat, (_Float16 *)s_t);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (g.has_zp) {
        size_t nz = (size_t)g.NT * g.ST * kTileRows;
        hipLaunchKernelGGL(repack_zp_kernel, dim3(blocks_for(nz, T)), dim3(T), 0, stream, g, zp_flat,
                           (uint8_t *)zp_t);
        e = hipGetLastError();
    }
    return e;
}

// Row fusion: one thread per (source row, super-tile) moves that row's four
// 16-byte lane chunks of packed nibbles, its SPS scales and its ZB zero-point
// bytes to the destination row.  Both weights share K and the block size, so
// ST, SPS and ZB agree; padding k, blocks >= kb and rows past the end stay as
// the zeroed destination holds them.
template <typename SrcS, typename DstS>
__global__ void copy_rows_kernel(WeightGeom sg, const uint32_t *__restrict__ sq, const SrcS *__restrict__ ss,
                                 const uint8_t *__restrict__ sz, WeightGeom dg, uint32_t *__restrict__ dq,
                                 DstS *__restrict__ ds, uint8_t *__restrict__ dz, int32_t row0) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= (size_t)sg.N * sg.ST) return;
    const int st = (int)(e % sg.ST);
    const int rs = (int)(e / sg.ST);
    const int rd = row0 + rs;
    const size_t ts = (size_t)(rs / kTileRows) * sg.ST + st;
    const size_t td = (size_t)(rd / kTileRows) * dg.ST + st;
    const int ls = rs % kTileRows, ld = rd % kTileRows;
#pragma unroll
    for (int gg = 0; gg < 4; ++gg)
        *(u32x4_t *)(dq + (td * 64 + gg * 16 + ld) * 4) = *(const u32x4_t *)(sq + (ts * 64 + gg * 16 + ls) * 4);
    const float factor = pow2f(dg.fold_exp - sg.fold_exp);
    for (int i = 0; i < sg.SPS; ++i)
        ds[(td * kTileRows + ld) * dg.SPS + i] = scaled<DstS>(ss[(ts * kTileRows + ls) * sg.SPS + i], factor);
    if (!dz) return;
    if (sz) {
        for (int b = 0; b < sg.ZB; ++b) dz[(td * kTileRows + ld) * dg.ZB + b] = sz[(ts * kTileRows + ls) * sg.ZB + b];
        return;
    }
    uint32_t bits = 0;  // implicit zero point 8 for the blocks the row holds
    for (int i = 0; i < sg.SPS; ++i) {
        const int blk = sg.bs >= kTileK ? (st * kTileK) / sg.bs : st * sg.SPS + i;
        if (blk < sg.kb) bits |= 8u << (4 * i);
    }
    for (int b = 0; b < dg.ZB; ++b) dz[(td * kTileRows + ld) * dg.ZB + b] = (uint8_t)(bits >> (8 * b));
}

hipError_t launch_copy_rows(const WeightGeom &sg, const void *sq, const void *ss, const void *sz, const WeightGeom &dg,
                            void *dq, void *ds, void *dz, int32_t row0, hipStream_t stream) {
    const unsigned T = 256;
    const size_t n = (size_t)sg.N * sg.ST;
    if (n == 0) return hipSuccess;
    const dim3 grid(blocks_for(n, T)), block(T);
    if (!dg.scale_f32)
        hipLaunchKernelGGL((copy_rows_kernel<_Float16, _Float16>), grid, block, 0, stream, sg, (const uint32_t *)sq,
                           (const _Float16 *)ss, (const uint8_t *)sz, dg, (uint32_t *)dq, (_Float16 *)ds,
                           (uint8_t *)dz, row0);
    else if (sg.scale_f32)
        hipLaunchKernelGGL((copy_rows_kernel<float, float>), grid, block, 0, stream, sg, (const uint32_t *)sq,
                           (const float *)ss, (const uint8_t *)sz, dg, (uint32_t *)dq, (float *)ds, (uint8_t *)dz,
                           row0);
    else
        hipLaunchKernelGGL((copy_rows_kernel<_Float16, float>), grid, block, 0, stream, sg, (const uint32_t *)sq,
                           (const _Float16 *)ss, (const uint8_t *)sz, dg, (uint32_t *)dq, (float *)ds,
                           (uint8_t *)dz, row0);
    return hipGetLastError();
}

__global__ void scale_f32_kernel(float *__restrict__ s, size_t n, float factor) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e < n) s[e] *= factor;
}

hipError_t launch_scale_f32(float *s, size_t n, float factor, hipStream_t stream) {
    const unsigned T = 256;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(scale_f32_kernel, dim3(blocks_for(n, T)), dim3(T), 0, stream, s, n, factor);
    return hipGetLastError();
}

template <typename XT>
__global__ void stage_x_kernel(const XT *__restrict__ x, int32_t M, int32_t K, int32_t ldx, _Float16 *__restrict__ out) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)M * ldx;
    if (e >= total) return;
    const int m = (int)(e / ldx);
    const int k = (int)(e % ldx);
    out[e] = k < K ? (_Float16)x[(size_t)m * K + k] : (_Float16)0.0f;
}

hipError_t launch_stage_x(const void *x, int32_t x_type, int32_t M, int32_t K, int32_t ldx, _Float16 *out,
                          hipStream_t stream) {
    const unsigned T = 256;
    size_t n = (size_t)M * ldx;
    if (x_type == MNB_F32)
        hipLaunchKernelGGL(stage_x_kernel<float>, dim3(blocks_for(n, T)), dim3(T), 0, stream, (const float *)x, M,
                           K, ldx, out);
    else
        hipLaunchKernelGGL(stage_x_kernel<_Float16>, dim3(blocks_for(n, T)), dim3(T), 0, stream,
                           (const _Float16 *)x, M, K, ldx, out);
    return hipGetLastError();
}

// One thread per (row n, group of 8 consecutive k).  w = float(q - zp) * scale,
// formed as (float(q - zp) * stored scale) * 2^-fold_exp: the power of two
// makes the two roundings one.
template <typename ScaleT, typename OutT, bool HAS_ZP>
__global__ void dequant_kernel(WeightGeom g, const uint32_t *__restrict__ q_t, const ScaleT *__restrict__ s_t,
                               const uint8_t *__restrict__ zp_t, OutT *__restrict__ out) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int groups = (g.K + 7) / 8;
    const size_t total = (size_t)g.N * groups;
    if (e >= total) return;
    const int n = (int)(e / groups);
    const int k0 = (int)(e % groups) * 8;
    const int nt = n / kTileRows, r = n % kTileRows;
    const int st = k0 / kTileK, kk = k0 % kTileK;
    const int j = kk / 32, gg = (kk % 32) / 8;
    const size_t tile = (size_t)nt * g.ST + st;
    const uint32_t t = q_t[(tile * 64 + gg * 16 + r) * 4 + j];
    const int si = g.bs >= kTileK ? 0 : kk / g.bs;
    const float scale = (float)s_t[(tile * kTileRows + r) * g.SPS + si];
    const float unfold = pow2f(-g.fold_exp);
    int z = 8;
    if constexpr (HAS_ZP) {
        const uint8_t *zp = zp_t + (tile * kTileRows + r) * g.ZB;
        z = (int)((zp[si / 2] >> (4 * (si & 1))) & 0xFu);
    }
    OutT *o = out + (size_t)n * g.K + k0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (k0 + i < g.K) {
            const int w = (int)tiled_nibble(t, i) - z;
            float v = (float)w * scale * unfold;
            // Keep the binary32 product in a register before the fp16 rounding:
            // otherwise the multiply and the conversion are fused into
            // v_fma_mix(scale, w, +0), which turns a -0 product into +0.
            asm volatile("" : "+v"(v));
            o[i] = (OutT)v;
        }
    }
}

template <typename ScaleT>
static hipError_t dequant_dispatch(const mnb_weight *w, void *out, int32_t out_type, hipStream_t stream) {
    const WeightGeom &g = w->g;
    const unsigned T = 256;
    size_t n = (size_t)g.N * ((g.K + 7) / 8);
    const uint32_t *q = (const uint32_t *)w->q_t;
    const ScaleT *s = (const ScaleT *)w->s_t;
    const uint8_t *z = (const uint8_t *)w->zp_t;
    dim3 grid(blocks_for(n, T)), block(T);
    if (out_type == MNB_F32) {
        if (g.has_zp) hipLaunchKernelGGL((dequant_kernel<ScaleT, float, true>), grid, block, 0, stream, g, q, s, z, (float *)out);
        else hipLaunchKernelGGL((dequant_kernel<ScaleT, float, false>), grid, block, 0, stream, g, q, s, z, (float *)out);
    } else {
        if (g.has_zp) hipLaunchKernelGGL((dequant_kernel<ScaleT, _Float16, true>), grid, block, 0, stream, g, q, s, z, (_Float16 *)out);
        else hipLaunchKernelGGL((dequant_kernel<ScaleT, _Float16, false>), grid, block, 0, stream, g, q, s, z, (_Float16 *)out);
    }
    return hipGetLastError();
}

hipError_t launch_dequant(const mnb_weight *w, void *out, int32_t out_type, hipStream_t stream) {
    return w->g.scale_f32 ? dequant_dispatch<float>(w, out, out_type, stream)
                          : dequant_dispatch<_Float16>(w, out, out_type, stream);
}

}  // namespace mnb
