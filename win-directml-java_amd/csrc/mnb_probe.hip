// mnb_probe.hip -- libmnb_probe.so: the measured MFMA ceiling the benchmark
// reports beside the GEMM (not part of libmnb_hip.so, nothing in the
// library calls it).
//
// The prefill GEMM's roofline is the fp16 dense MFMA peak, 2.5 PFLOP/s
// (256 CUs x 4 SIMDs x 1024 flop per clock x 2.4 GHz).  Under a sustained
// matrix load the MI355X lowers its clock to stay within its power limit, so
// that peak is not what the chip sustains.  This kernel measures what it does
// sustain: nothing but v_mfma_f32_32x32x16_f16, the GEMM's instruction, at the
// GEMM's occupancy (256 workgroups of 8 waves, two per SIMD), on operands
// drawn like the GEMM's (activations of unit scale against weights of about
// 0.1; each wave cycles through 64 different operand pairs so operand bits
// toggle as they do in the GEMM), with four independent accumulators per wave
// so the matrix core never waits for a result.  No memory is touched inside the loop.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int kWaves = 8;       // per workgroup, two per SIMD, as the GEMM
constexpr int kSets = 8;        // operand pairs cycled by each wave
constexpr int kChains = 4;      // independent accumulators per wave

// A deterministic fp16 value in [-scale, scale) from a 32-bit hash.
__device__ __forceinline__ _Float16 draw(uint32_t h, float scale) {
    h ^= h >> 16;
    h *= 0x7feb352du;
    h ^= h >> 15;
    h *= 0x846ca68bu;
    h ^= h >> 16;
    return (_Float16)(((float)(h >> 8) * (1.0f / 16777216.0f) * 2.0f - 1.0f) * scale);
}

__global__ __launch_bounds__(64 * kWaves, 1) void mfma_ceiling_kernel(int iters, float *out) {
    const uint32_t lane = threadIdx.x + blockIdx.x * blockDim.x;
    half8_t a[kSets], b[kSets];
#pragma unroll
    for (int s = 0; s < kSets; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            a[s][e] = draw(lane * 131u + (uint32_t)(s * 8 + e), 0.1f);
            b[s][e] = draw(lane * 137u + (uint32_t)(s * 8 + e) + 0x9e3779b9u, 1.0f);
        }
    float16_t acc[kChains];
#pragma unroll
    for (int c = 0; c < kChains; ++c)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[c][v] = 0.f;
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int r = 0; r < kSets; ++r)
#pragma unroll
            for (int s = 0; s < kSets; ++s)
                acc[s % kChains] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[s], b[(s + r) % kSets], acc[s % kChains], 0, 0, 0);
    }
    float r = 0.f;
#pragma unroll
    for (int c = 0; c < kChains; ++c)
#pragma unroll
        for (int v = 0; v < 16; ++v) r += acc[c][v];
    out[lane] = r;   // keeps the loop; one store per lane after it
}

}  // namespace

extern "C" {

// Runs `launches` back-to-back launches of `workgroups` workgroups, each wave
// issuing iters * 64 MFMAs of 32 x 32 x 16 (32768 flops each), on `stream`
// (out: 64 * 8 * workgroups floats).  Returns the HIP status.
int32_t mnb_probe_mfma(int32_t workgroups, int32_t iters, int32_t launches, float *out, void *stream) {
    if (workgroups < 1 || iters < 1 || launches < 1 || !out) return (int32_t)hipErrorInvalidValue;
    for (int l = 0; l < launches; ++l)
        hipLaunchKernelGGL(mfma_ceiling_kernel, dim3(workgroups), dim3(64 * kWaves), 0, (hipStream_t)stream, iters, out);
    return (int32_t)hipGetLastError();
}

// Flops of one launch.
double mnb_probe_mfma_flops(int32_t workgroups, int32_t iters) {
    return (double)workgroups * kWaves * (double)iters * kSets * kSets * 32.0 * 32.0 * 16.0 * 2.0;
}

}  // extern "C"
