// mnb_gemm_sk.hip -- prefill-shaped MatMulNBits (M > 16): stream-K GEMM on
// fp16 MFMA with the int4 weights dequantized in registers.
//
// Replaces the tiled HLSL batch GEMM INT4_MATMUL_BATCH_TILED_HLSL
// (directml-windows-bindings/src/main/java/com/aresstack/windirectml/windows/
// MatMulNBitsKernel.java:732-820) and its 256-row host chunking (:2374-2387).
//
// Output tile 128 (M) x 256 (N) per workgroup of 8 waves (two per SIMD, so
// one wave's LDS and dequant latency hides behind the other's MFMAs), each
// wave 64 x 64 (4 x 4 fragments of v_mfma_f32_16x16x32_f16, fp32 accumulators).
// Operand pipeline, one 128-k stage at a time: every operand of stage s + 2 --
// the x tile (32 KiB), the packed weight tiles (16 KiB), their scales and zero
// points -- is copied straight from HBM into a 3-slot LDS ring by direct
// global->LDS loads while stage s computes, so no load ever passes through
// registers and two stages of latency are hidden.  Per 32-k step a wave reads
// its four raw weight fragments from the ring, dequantizes them in registers
// (w = (q - zp) * scale, scale folded into the fp16 operand) and runs 16 MFMAs
// against four x fragments (the two waves of an N quarter dequantize the same
// tiles).  x rows are stored with chunk c of row m at slot c ^ (m & 15), so
// the fragment reads are free of bank conflicts.
//
// Stream-K: the grid is one persistent workgroup per CU.  The (tile, stage)
// iterations of the whole product are cut into equal contiguous ranges, one
// per workgroup, so every CU gets the same MFMA work whatever the tile count.
// A tile whose stages span several workgroups is finished by whichever
// contributor arrives last (fp32 partials in a workspace, a per-tile arrival
// counter that the finisher resets); no workgroup ever waits for another.
// Logical workgroup ids are laid out XCD-contiguous, so neighbouring
// workgroups (which share tiles and weight columns) sit on the same XCD.
#include <algorithm>

#include "mnb_device.h"

namespace mnb {

constexpr int kSkBM = 128;          // rows per tile
constexpr int kSkWaves = 8;         // two per SIMD
constexpr int kSkNTW = 2;           // n-tiles (16 rows of W) per wave: 32 columns
constexpr int kSkBN = kSkWaves * kSkNTW * kTileRows;   // 256 columns per tile
constexpr int kSkFM = kSkBM / 32;   // 32-row A fragments per wave
constexpr int kSkFN = kSkNTW / 2;   // 32-column B fragments per wave
constexpr int kSkThreads = 64 * kSkWaves;
constexpr int kSkPartialFloats = kSkThreads * kSkFM * kSkFN * 16;   // one partial tile

typedef float float16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float16_t mfma32x32x16(half8_t a, half8_t b, float16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

struct SkParams {
    const u32x4_t *q_t;
    const void *s_t;
    const uint8_t *zp_t;
    const _Float16 *x;
    int32_t ldx, kx, M, N, NT, ST;
    void *y;
    int32_t y_f16, accumulate;
    int32_t MT, T, G;       // m-tiles, tiles, workgroups
    int32_t I;              // iterations = T * ST (below 2^31)
    float *ws;              // [G][2] partial tiles
    int32_t *cnt;           // [T] arrival counters (zero between launches)
};

// first iteration of logical workgroup g (g = G gives I)
__device__ __forceinline__ int sk_start(int g, const SkParams &p) { return (int)((int64_t)g * p.I / p.G); }

// logical workgroup owning iteration i
__device__ __forceinline__ int sk_owner(int i, const SkParams &p) {
    int g = (int)((int64_t)i * p.G / p.I);
    while (g + 1 < p.G && sk_start(g + 1, p) <= i) ++g;
    while (g > 0 && sk_start(g, p) > i) --g;
    return g;
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// One direct global->LDS load of 16 bytes per active lane from base + off
// (scalar base, 32-bit lane offset): lane l writes LDS[m0 + 16 l].  Issued as
// inline asm, so the compiler neither tracks it nor moves memory accesses
// across it; the kernel waits for it explicitly.
__device__ __forceinline__ void dma16(uint32_t m0, uint32_t off, const void *base) {
    asm volatile("global_load_lds_dwordx4 %1, %2" ::"{m0}"(m0), "v"(off), "s"(base) : "memory");
}

// Ring slot layout (bytes) for one stage, and the direct loads that fill it.
template <typename ScaleT, bool HAS_ZP, int SPS>
struct SkSlot {
    static constexpr int ZB = SPS <= 2 ? 1 : SPS / 2;
    static constexpr int kNT = kSkBN / kTileRows;                   // 16 n-tiles per tile
    static constexpr int kX = 0;                                    // x tile [128][16 chunks]
    static constexpr int kQ = kSkBM * kTileK * 2;                   // 32 KiB: packed tiles [16][64 lanes][16 B]
    static constexpr int kS = kQ + kNT * kTileBytes;                // scales [16 tiles][16 rows][SPS]
    static constexpr int kTileS = kTileRows * SPS * (int)sizeof(ScaleT);   // scale bytes per tile
    static constexpr int kZ = kS + kNT * kTileS;                    // zero points [16 tiles][16 rows][ZB]
    static constexpr int kTileZ = kTileRows * ZB;
    static constexpr int kBytes = kZ + (HAS_ZP ? kNT * kTileZ : 0);
    static constexpr int kDepth = 3 * kBytes <= 160 * 1024 ? 3 : 2;   // ring slots (fits the 160 KiB LDS)
    // per wave and stage: x pieces of 4 rows, its 4 packed tiles, their
    // scales and zero points
    static constexpr int kXDma = kSkBM * kTileK * 2 / 1024 / kSkWaves;
    static constexpr int kSDma = (kSkNTW * kTileS + 1023) / 1024;
    static constexpr int kDma = kXDma + kSkNTW + kSDma + (HAS_ZP ? 1 : 0);
    static_assert(kTileS % 16 == 0 && kTileZ % 16 == 0 && kSkNTW * kTileZ <= 1024, "16-byte pieces");
};

template <typename ScaleT, bool HAS_ZP, int SPS>
__global__ __launch_bounds__(kSkThreads, 1) void gemm_sk_kernel(SkParams p) {
    using L = SkSlot<ScaleT, HAS_ZP, SPS>;
    constexpr int ZB = L::ZB;
    constexpr int D = L::kDepth;
    __shared__ __align__(1024) unsigned char ring[D][L::kBytes];
    __shared__ int s_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c32 = lane & 31, h = lane >> 5;   // MFMA row/column and k half
    // XCD-contiguous logical id: physical workgroup b runs on XCD b % 8
    const int per_xcd = p.G / 8;
    const int g = (p.G % 8 == 0) ? (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8) : (int)blockIdx.x;
    const int i0 = sk_start(g, p), i1 = sk_start(g + 1, p);
    if (i0 >= i1) return;

    const uint32_t k6400 = vgpr_const(0x64006400u);
    const uint32_t ring0 = __builtin_amdgcn_readfirstlane(lds_addr(&ring[0][0]));

    // ---- issue: all operands of one stage into one ring slot ----
    // The issue cursor (tile lt, stage lst) stops at this workgroup's last
    // iteration, so every stage issues the same loads (the final ones re-load
    // the last stage into a slot nobody reads).  Lane byte offsets are set
    // per tile; a stage only moves the scalar bases.
    constexpr int SL = L::kTileS / 16;   // 16-byte scale pieces per tile
    constexpr int ZL = L::kTileZ / 16;   // 16-byte zero-point pieces per tile
    int lt = i0 / p.ST, lst = i0 - lt * p.ST, li = i0, lslot = 0;
    uint32_t xrow[L::kXDma], xcol[L::kXDma], qoff[kSkNTW], soff[L::kSDma], zoff = 0;
    auto set_tile = [&]() __attribute__((always_inline)) {
        const int m0 = (lt % p.MT) * kSkBM, nt0 = (lt / p.MT) * L::kNT + wave * kSkNTW;
#pragma unroll
        for (int u = 0; u < L::kXDma; ++u) {
            const int row = (wave * L::kXDma + u) * 4 + (lane >> 4);
            xrow[u] = (uint32_t)min(m0 + row, p.M - 1) * (uint32_t)p.ldx * 2u;
            xcol[u] = (uint32_t)(((lane & 15) ^ (row & 15)) * 16);
        }
#pragma unroll
        for (int b = 0; b < kSkNTW; ++b)
            qoff[b] = ((uint32_t)min(nt0 + b, p.NT - 1) * (uint32_t)p.ST * 64u + (uint32_t)lane) * 16u;
#pragma unroll
        for (int v = 0; v < L::kSDma; ++v) {
            const int l = min(v * 64 + lane, kSkNTW * SL - 1);
            soff[v] = (uint32_t)min(nt0 + l / SL, p.NT - 1) * (uint32_t)p.ST * L::kTileS + (uint32_t)(l % SL) * 16u;
        }
        if constexpr (HAS_ZP) {
            const int l = min(lane, kSkNTW * ZL - 1);
            zoff = (uint32_t)min(nt0 + l / ZL, p.NT - 1) * (uint32_t)p.ST * L::kTileZ + (uint32_t)(l % ZL) * 16u;
        }
    };
    set_tile();
    auto issue = [&]() __attribute__((always_inline)) {
        const uint32_t base = ring0 + (uint32_t)(lslot * L::kBytes);
        // x: this wave's kXDma pieces of 4 rows each; lane -> (row, slot)
        if ((lst + 1) * kTileK <= p.kx) {
            const unsigned char *xb = (const unsigned char *)p.x + (size_t)lst * kTileK * 2;
#pragma unroll
            for (int u = 0; u < L::kXDma; ++u)
                dma16(base + L::kX + (uint32_t)(wave * L::kXDma + u) * 1024u, xrow[u] + xcol[u], xb);
        } else {
            // last stage with a k tail: chunks at k >= kx re-read the row's
            // last chunk (zeroed in LDS on landing) and stay inside x
#pragma unroll
            for (int u = 0; u < L::kXDma; ++u) {
                const uint32_t k = (uint32_t)min(lst * kTileK + (int)(xcol[u] / 2), p.kx - 8);
                dma16(base + L::kX + (uint32_t)(wave * L::kXDma + u) * 1024u, xrow[u] + k * 2u, p.x);
            }
        }
        // this wave's packed tiles, scales and zero points
        const int ntl = wave * kSkNTW;   // first local n-tile
        const unsigned char *qb = (const unsigned char *)p.q_t + (size_t)lst * kTileBytes;
#pragma unroll
        for (int b = 0; b < kSkNTW; ++b) dma16(base + L::kQ + (uint32_t)(ntl + b) * kTileBytes, qoff[b], qb);
        const unsigned char *sb = (const unsigned char *)p.s_t + (size_t)lst * L::kTileS;
#pragma unroll
        for (int v = 0; v < L::kSDma; ++v) {
            if (v * 64 + lane < kSkNTW * SL) dma16(base + L::kS + (uint32_t)(ntl * L::kTileS + v * 1024), soff[v], sb);
        }
        if constexpr (HAS_ZP) {
            const unsigned char *zb = p.zp_t + (size_t)lst * L::kTileZ;
            if (lane < kSkNTW * ZL) dma16(base + L::kZ + (uint32_t)(ntl * L::kTileZ), zoff, zb);
        }
        if (li + 1 < i1) {
            ++li;
            if (++lst == p.ST) {
                lst = 0;
                ++lt;
                set_tile();
            }
        }
        lslot = lslot == D - 1 ? 0 : lslot + 1;
    };

    // ---- land: wait for the oldest stage in flight, zero its x pieces at
    // k >= kx, and meet the other waves ----
    bool drain = false;   // set after y stores: stores and loads may complete out of order
    auto land = [&](int slot, int st) __attribute__((always_inline)) {
        if (drain || D == 2) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            drain = false;
        } else {
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(L::kDma) : "memory");   // only the newest stage in flight
        }
        if ((st + 1) * kTileK > p.kx) {
            unsigned char *xs = &ring[slot][L::kX];
#pragma unroll
            for (int u = 0; u < L::kXDma; ++u) {
                const int row = (wave * L::kXDma + u) * 4 + (lane >> 4);
                const int chunk = (lane & 15) ^ (row & 15);
                if (st * kTileK + chunk * 8 >= p.kx)
                    *(u32x4_t *)(xs + (wave * L::kXDma + u) * 1024 + lane * 16) = (u32x4_t){0u, 0u, 0u, 0u};
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };

    float16_t acc[kSkFM][kSkFN];
#pragma unroll
    for (int a = 0; a < kSkFM; ++a)
#pragma unroll
        for (int f = 0; f < kSkFN; ++f)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[a][f][v] = 0.f;

    // ---- epilogue of tile t after nst of its stages ----
    int t = i0 / p.ST;
    auto epilogue = [&](int nst) __attribute__((always_inline)) {
        const int m0 = (t % p.MT) * kSkBM, ng = t / p.MT;
        const int n_wave = (ng * L::kNT + wave * kSkNTW) * kTileRows;
        bool write_out = nst == p.ST;
        if (!write_out) {
            // Partial tiles travel through agent-scope relaxed atomics (stores
            // and loads that are coherent across XCDs without writing back or
            // invalidating any L2): each thread waits for its own stores to
            // complete before the workgroup bumps the tile's arrival counter,
            // and the finisher reads only after the counter told it so.
            typedef unsigned long long u64;
            const int slot = i0 / p.ST == t ? 0 : 1;   // 0 if t is this workgroup's first tile
            u64 *mine = (u64 *)(p.ws + ((size_t)g * 2 + slot) * kSkPartialFloats) + tid;
#pragma unroll
            for (int a = 0; a < kSkFM; ++a)
#pragma unroll
                for (int f = 0; f < kSkFN; ++f)
#pragma unroll
                    for (int v2 = 0; v2 < 8; ++v2) {
                        const u64 bits = (u64)__float_as_uint(acc[a][f][2 * v2]) |
                                         ((u64)__float_as_uint(acc[a][f][2 * v2 + 1]) << 32);
                        __hip_atomic_store(mine + ((a * kSkFN + f) * 8 + v2) * kSkThreads, bits, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                    }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            const int g_first = sk_owner(t * p.ST, p);
            const int g_last = sk_owner((t + 1) * p.ST - 1, p);
            if (tid == 0)
                s_last = __hip_atomic_fetch_add(&p.cnt[t], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                         g_last - g_first;
            __syncthreads();
            if (s_last) {
                // every contributor's partial (this workgroup's included) is read
                // back and summed in contributor order, whoever finishes: the
                // result does not depend on arrival order
                for (int og = g_first; og <= g_last; ++og) {
                    const int oslot = sk_start(og, p) / p.ST == t ? 0 : 1;
                    const u64 *part = (const u64 *)(p.ws + ((size_t)og * 2 + oslot) * kSkPartialFloats) + tid;
#pragma unroll
                    for (int a = 0; a < kSkFM; ++a)
#pragma unroll
                        for (int f = 0; f < kSkFN; ++f)
#pragma unroll
                            for (int v2 = 0; v2 < 8; ++v2) {
                                const u64 bits = __hip_atomic_load(part + ((a * kSkFN + f) * 8 + v2) * kSkThreads,
                                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                                const float lo = __uint_as_float((uint32_t)bits), hi = __uint_as_float((uint32_t)(bits >> 32));
                                acc[a][f][2 * v2] = og == g_first ? lo : acc[a][f][2 * v2] + lo;
                                acc[a][f][2 * v2 + 1] = og == g_first ? hi : acc[a][f][2 * v2 + 1] + hi;
                            }
                }
                if (tid == 0) __hip_atomic_store(&p.cnt[t], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // ready for the next launch
                write_out = true;
            }
        }
        if (write_out) {
            // fragment (a, f): lane holds column c32, rows 8 (v / 4) + 4 h + v % 4
            const bool accum = p.accumulate != 0;
#pragma unroll
            for (int f = 0; f < kSkFN; ++f) {
                const int n = n_wave + f * 32 + c32;
                if (n >= p.N) continue;
#pragma unroll
                for (int a = 0; a < kSkFM; ++a) {
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int mm = m0 + a * 32 + 8 * (v / 4) + 4 * h + (v % 4);
                        if (mm < p.M) {
                            const size_t idx = (size_t)mm * p.N + n;
                            if (p.y_f16) store_y<true>(p.y, idx, acc[a][f][v], accum);
                            else store_y<false>(p.y, idx, acc[a][f][v], accum);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int a = 0; a < kSkFM; ++a)
#pragma unroll
            for (int f = 0; f < kSkFN; ++f)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[a][f][v] = 0.f;
        drain = true;
    };

    // ---- main loop: segments of one tile, one stage per inner trip ----
    // The epilogue sits outside the stage loop, so the accumulators stay in
    // the MFMA registers across stages.
    int cslot = 0, cst = i0 - t * p.ST;
    int remaining = i1 - i0;
    int seg_n = min(remaining, p.ST - cst);   // stages of tile t done by this workgroup
    issue();
    if (D == 3) issue();
    land(0, cst);
    while (true) {
        for (int kk = 0; kk < seg_n; ++kk) {
            issue();   // stage + 2 (three-slot ring) or stage + 1 (two slots)
            const unsigned char *sl = ring[cslot];
            // B fragment f covers local n-tiles 4 wave + 2 f + {0, 1}; lane
            // (c32, h) needs, at 16-k step s, the 8 nibbles of row c32 % 16 of
            // tile c32 / 16 at k-group 2 s + h: word s / 2 of tile lane
            // ((2 s + h) % 4) * 16 + c32 % 16.  Two 16-byte reads per fragment
            // hold all of them: qb[f][0] for even s, qb[f][1] for odd s.
            u32x4_t qb[kSkFN][2];
            ScaleT sc[kSkFN][SPS];
            uint32_t zb[kSkFN];
#pragma unroll
            for (int f = 0; f < kSkFN; ++f) {
                const int ntl = wave * kSkNTW + 2 * f + (c32 >> 4);
                const unsigned char *qt = sl + L::kQ + ntl * kTileBytes;
                qb[f][0] = *(const u32x4_t *)(qt + (h * 16 + (c32 & 15)) * 16);
                qb[f][1] = *(const u32x4_t *)(qt + ((2 + h) * 16 + (c32 & 15)) * 16);
                const ScaleT *sp = (const ScaleT *)(sl + L::kS + ntl * L::kTileS) + (c32 & 15) * SPS;
#pragma unroll
                for (int e = 0; e < SPS; ++e) sc[f][e] = sp[e];
                if constexpr (HAS_ZP) {
                    const unsigned char *zp = sl + L::kZ + ntl * L::kTileZ + (c32 & 15) * ZB;
                    uint32_t z = 0;
#pragma unroll
                    for (int e = 0; e < ZB; ++e) z |= (uint32_t)zp[e] << (8 * e);
                    zb[f] = z;
                } else {
                    zb[f] = 0x88888888u;
                }
            }
            const _Float16 *xs = (const _Float16 *)(sl + L::kX);
            auto read_x = [&](half8_t(&af)[kSkFM], int s) __attribute__((always_inline)) {
                // row a * 32 + c32 (row & 15 == c32 & 15), k-chunk 2 s + h
#pragma unroll
                for (int a = 0; a < kSkFM; ++a)
                    af[a] = *(const half8_t *)(xs + (a * 32 + c32) * kTileK + (((2 * s + h) ^ (c32 & 15)) * 8));
            };
            auto dequant = [&](half8_t(&bf)[kSkFN], int s) __attribute__((always_inline)) {
                const int si = s * SPS / 8;   // scale block of k-group 2 s + h (same for both h)
#pragma unroll
                for (int f = 0; f < kSkFN; ++f) {
                    const uint32_t z = HAS_ZP ? zp_nibble(zb[f], si) : 8u;
                    half8_t w = unpack_q_minus_zp(qb[f][s & 1][s >> 1], bias_lo_pair(z), bias_hi_pair(z), k6400);
                    if constexpr (sizeof(ScaleT) == 2) {
                        w = w * (_Float16)sc[f][si];
                    } else {
                        const float sf = (float)sc[f][si];
#pragma unroll
                        for (int e = 0; e < 8; ++e) w[e] = (_Float16)((float)w[e] * sf);
                    }
                    bf[f] = w;
                }
            };
            // step s + 1's x fragments are read and its weights dequantized while
            // the MFMAs of step s run
            half8_t af[2][kSkFM], bf[2][kSkFN];
            read_x(af[0], 0);
            dequant(bf[0], 0);
#pragma unroll
            for (int s = 0; s < kTileK / 16; ++s) {
                if (s + 1 < kTileK / 16) {
                    read_x(af[(s + 1) & 1], s + 1);
                    dequant(bf[(s + 1) & 1], s + 1);
                }
#pragma unroll
                for (int a = 0; a < kSkFM; ++a)
#pragma unroll
                    for (int f = 0; f < kSkFN; ++f) acc[a][f] = mfma32x32x16(af[s & 1][a], bf[s & 1][f], acc[a][f]);
                // order within the step: the next step's x reads go out first,
                // between the MFMAs, and its dequant VALU fills the MFMA shadow
                if (s + 1 < kTileK / 16) {
#pragma unroll
                    for (int i = 0; i < kSkFM; ++i) {
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);   // VALU
                    }
#pragma unroll
                    for (int i = 0; i < kSkFM * kSkFN - kSkFM; ++i) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // VALU
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            cslot = cslot == D - 1 ? 0 : cslot + 1;
            cst = cst + 1 == p.ST ? 0 : cst + 1;
            land(cslot, cst);   // after the last stage this waits for re-loads nobody reads
        }
        remaining -= seg_n;
        epilogue(seg_n);
        if (remaining == 0) break;
        ++t;
        seg_n = min(remaining, p.ST);
    }
    // drain every direct load before the workgroup's LDS is released
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

size_t sk_workspace_bytes(int G) { return (size_t)G * 2 * kSkPartialFloats * sizeof(float); }

int sk_tiles(int M, int NT) { return ((M + kSkBM - 1) / kSkBM) * ((NT * kTileRows + kSkBN - 1) / kSkBN); }

// Candidates: G = m T (m = 1, 2, ...: every tile split into about m pieces)
// and G = cu_count.  Estimated time, fitted to measurements on MI355X over
// the Phi-3 projection shapes at M = 128..2048: a stage costs 1.5 us on a
// lightly loaded chip up to 2.4 us with every CU busy; a split tile costs a
// fixed 8 us plus 3 us per contributing workgroup (partial tiles written and
// read back through the coherent path).
int sk_grid(int T, int ST, int cu_count) {
    const int64_t I = (int64_t)T * ST;
    auto cost = [&](int64_t G) {
        const double per_wg = (double)((I + G - 1) / G);
        const double t_stage = 1.5 + 0.9 * (double)std::min<int64_t>(G, cu_count) / cu_count;
        double t = per_wg * t_stage;
        if (G > T) t += 8.0 + 3.0 * (double)((ST + (int64_t)per_wg - 1) / (int64_t)per_wg + 1);
        return t;
    };
    const int64_t cap = std::min<int64_t>(cu_count, I);
    int64_t best = std::min<int64_t>(T, cap);
    double best_t = cost(best);
    for (int64_t G = 2 * (int64_t)T; G < cap; G += T) {
        const double t = cost(G);
        if (t < best_t) best = G, best_t = t;
    }
    if (cost(cap) < best_t) best = cap;
    return (int)best;
}

hipError_t launch_gemm_sk(const mnb_weight *w, const MatmulArgs &a, int G, float *ws, int32_t *cnt,
                          hipStream_t stream) {
    const WeightGeom &g = w->g;
    SkParams p;
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
    p.MT = (a.M + kSkBM - 1) / kSkBM;
    p.T = sk_tiles(a.M, g.NT);
    p.G = G;
    const int64_t iters = (int64_t)p.T * g.ST;
    if (iters >= (int64_t)1 << 31) return hipErrorInvalidValue;
    p.I = (int32_t)iters;
    p.ws = ws;
    p.cnt = cnt;
    dim3 grid(G), block(kSkThreads);
#define MNB_SK_LAUNCH(ST_, ZP_, SPS_) hipLaunchKernelGGL((gemm_sk_kernel<ST_, ZP_, SPS_>), grid, block, 0, stream, p)
#define MNB_SK_SPS(ST_, ZP_)                           \
    switch (g.SPS) {                                   \
        case 1: MNB_SK_LAUNCH(ST_, ZP_, 1); break;     \
        case 2: MNB_SK_LAUNCH(ST_, ZP_, 2); break;     \
        case 4: MNB_SK_LAUNCH(ST_, ZP_, 4); break;     \
        case 8: MNB_SK_LAUNCH(ST_, ZP_, 8); break;     \
        default: return hipErrorInvalidValue;          \
    }
    if (g.scale_f32) {
        if (g.has_zp) { MNB_SK_SPS(float, true) } else { MNB_SK_SPS(float, false) }
    } else {
        if (g.has_zp) { MNB_SK_SPS(_Float16, true) } else { MNB_SK_SPS(_Float16, false) }
    }
#undef MNB_SK_SPS
#undef MNB_SK_LAUNCH
    return hipGetLastError();
}

}  // namespace mnb
