// mnb_device.h -- device-side helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mnb_internal.h"

namespace mnb {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half2_t as_half2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t as_u32(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// fp16 pair constants used by the nibble -> fp16 conversion.
//   (0x6400 | q) is the fp16 value 1024 + q   (q in bits 0..3)
//   (0x6400 | q<<4) is 1024 + 16 q; times 1/16 it is 64 + q exactly.
__device__ __forceinline__ uint32_t bias_lo_pair(uint32_t zp) {   // fp16 (1024 + zp) in both halves
    return 0x64006400u | (zp * 0x00010001u);
}
__device__ __forceinline__ uint32_t bias_hi_pair(uint32_t zp) {   // fp16 (64 + zp) in both halves
    return 0x54005400u | ((zp << 4) * 0x00010001u);
}

// Eight packed nibbles of one dword of the tiled layout -> eight fp16 values
// (q_i - zp), exact.  Result halves are k0..k7 in MFMA operand order.
//   d & 0x000F000F             -> (k0, k1) as 1024+q   -> minus (1024+zp)
//   d & 0x00F000F0             -> (k2, k3) as 1024+16q -> /16 minus (64+zp)
//   (d>>8) & 0x000F000F        -> (k4, k5)
//   (d>>8) & 0x00F000F0        -> (k6, k7)
// Every intermediate is an fp16 integer (or integer + 1024) below 2048, so
// the subtraction and the fused 1/16 scaling are exact.
//
// `k6400` must hold 0x64006400 in a VGPR (see vgpr_const): gfx9 VOP3
// instructions take no literal operand and at most one SGPR, so with the
// mask in an SGPR and this constant in a VGPR each (d & mask) | 0x64006400
// is a single v_and_or_b32.
__device__ __forceinline__ half8_t unpack_q_minus_zp(uint32_t d, uint32_t blo, uint32_t bhi, uint32_t k6400) {
    const half2_t lo = as_half2(blo);
    const half2_t hi = as_half2(bhi);
    const half2_t sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
    const uint32_t d8 = d >> 8;
    half2_t p0 = as_half2((d & 0x000F000Fu) | k6400) - lo;
    half2_t p1 = as_half2((d & 0x00F000F0u) | k6400) * sixteenth - hi;
    half2_t p2 = as_half2((d8 & 0x000F000Fu) | k6400) - lo;
    half2_t p3 = as_half2((d8 & 0x00F000F0u) | k6400) * sixteenth - hi;
    half8_t r;
    r[0] = p0[0]; r[1] = p0[1];
    r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1];
    r[6] = p3[0]; r[7] = p3[1];
    return r;
}

// A constant the compiler must keep in a VGPR (opaque to constant folding).
__device__ __forceinline__ uint32_t vgpr_const(uint32_t c) {
    asm volatile("" : "+v"(c));
    return c;
}

// Load through the global address space: pointers read from memory are
// generic to the compiler and would otherwise become flat loads, whose wait
// counter is shared with LDS and forces full waits.
template <typename T>
__device__ __forceinline__ T gld(const T *p) {
    return *(const __attribute__((address_space(1))) T *)p;
}

// Non-temporal load through the global address space, for the packed weights
// in the M <= 16 kernels, which one launch reads exactly once in whole 1 KiB
// tiles: the lines are not kept in the caches, which leaves L2 and the MALL to
// the activations that are re-read for every n-tile.  Measured on the
// 129-projection decode step: 5.6 -> 6.2 TB/s.  (The same hint on the small
// scale and zero-point reads measured slower, so those stay cached loads.)
template <typename T>
__device__ __forceinline__ T gld_nt(const T *p) {
    return __builtin_nontemporal_load((const __attribute__((address_space(1))) T *)p);
}

// The i-th nibble (low first) of a zero-point entry.
__device__ __forceinline__ uint32_t zp_nibble(uint32_t zbits, int i) { return (zbits >> (4 * i)) & 0xFu; }

template <typename T>
__device__ __forceinline__ float to_f32(T v) { return (float)v; }

__device__ __forceinline__ float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Load SPS consecutive scales (SPS in {1,2,4,8}) as floats.
template <typename ScaleT, int SPS>
__device__ __forceinline__ void load_scales(const ScaleT *p, float (&s)[SPS]) {
#pragma unroll
    for (int i = 0; i < SPS; ++i) s[i] = (float)p[i];
}

// Load one zero-point entry of ZB bytes.
template <int ZB>
__device__ __forceinline__ uint32_t load_zp(const uint8_t *p) {
    if constexpr (ZB == 1) return gld(p);
    else if constexpr (ZB == 2) return gld((const uint16_t *)p);
    else return gld((const uint32_t *)p);
}

template <bool F16>
__device__ __forceinline__ void store_y(void *y, size_t idx, float v, bool accumulate) {
    if constexpr (F16) {
        __attribute__((address_space(1))) _Float16 *p = (__attribute__((address_space(1))) _Float16 *)y + idx;
        if (accumulate) v += (float)*p;
        *p = (_Float16)v;
    } else {
        __attribute__((address_space(1))) float *p = (__attribute__((address_space(1))) float *)y + idx;
        if (accumulate) v += *p;
        *p = v;
    }
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// A wave-uniform pointer held in scalar registers.  The builtin returns a
// signed int: each half goes back through uint32_t, so the low dword is
// zero-extended (a sign extension would set the high dword to all ones
// whenever bit 31 of the address is set).
__device__ __forceinline__ const void *uniform_ptr(const void *p) {
    const uint64_t b = (uint64_t)(uintptr_t)p;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
    return (const void *)(uintptr_t)((uint64_t)lo | ((uint64_t)hi << 32));
}

// One direct global->LDS load of 16 bytes per active lane from base + off
// (scalar base, 32-bit lane offset): lane l writes LDS[m0 + 16 l].  Issued as
// inline asm, so the compiler neither tracks it nor moves memory accesses
// across it; the kernel waits for it explicitly.
//
// The compiler's hazard recognizer does not look inside inline asm, so it
// inserts none of the wait states this load needs.  gfx9 requires 1 between
// an SALU write of M0 and an LDS DMA: the s_nop 0 here provides it (the
// compiler sets M0 right before the statement).  It also requires 5 between
// a VALU write of an SGPR and a vector memory instruction that reads it: the
// scalar base must not come from a v_readfirstlane or from a v_readlane
// reload of a spilled SGPR within the 5 instructions before this load.  A
// build of the GEMM without its MFMAs (a timing copy) placed such a reload
// right before the load, which then read a stale base and faulted on the
// address.  Padding every load with s_nop 4 instead costs the M = 512 group
// launch 1% (the tail that issues these loads is issue-bound), so the
// library's code objects are checked instead: tests/test_code_objects.py
// disassembles the built library and fails on any direct-to-LDS load within
// 5 wait states of a VALU write of its base, on every path to it.
__device__ __forceinline__ void dma16(uint32_t m0, uint32_t off, const void *base) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"{m0}"(m0), "v"(off), "s"(uniform_ptr(base)) : "memory");
}

// Load the SPS scales of one row of one tile (SPS * sizeof(ScaleT) bytes,
// naturally aligned in the tiled layout) with the widest vector load.
template <typename ScaleT, int SPS>
__device__ __forceinline__ void load_scale_row(const ScaleT *p, ScaleT (&s)[SPS]) {
    constexpr int BYTES = SPS * (int)sizeof(ScaleT);
    if constexpr (BYTES == 2) {
        uint16_t v = gld((const uint16_t *)p);
        __builtin_memcpy(&s, &v, 2);
    } else if constexpr (BYTES == 4) {
        uint32_t v = gld((const uint32_t *)p);
        __builtin_memcpy(&s, &v, 4);
    } else if constexpr (BYTES == 8) {
        u32x2_t v = gld((const u32x2_t *)p);
        __builtin_memcpy(&s, &v, 8);
    } else if constexpr (BYTES == 16) {
        u32x4_t v = gld((const u32x4_t *)p);
        __builtin_memcpy(&s, &v, 16);
    } else {
        u32x4_t v0 = gld((const u32x4_t *)p), v1 = gld((const u32x4_t *)p + 1);
        __builtin_memcpy(&s, &v0, 16);
        __builtin_memcpy((char *)&s + 16, &v1, 16);
    }
}

}  // namespace mnb
