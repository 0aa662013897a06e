/*
 * mnb_oracle.c -- CPU restatement of the reference's int4 MatMulNBits path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this file.  It is the checker that the HIP kernels are compared
 * against (tests/, the smoke check and the CPU-baseline leg of bench.py).
 *
 * Every function names the reference file:line it restates.  Paths are
 * relative to the reference repository root:
 *   P3W = directml-inference/src/main/java/com/aresstack/windirectml/inference/phi3/Phi3Weights.java
 *   Q2W = directml-inference/src/main/java/com/aresstack/windirectml/inference/qwen/Qwen2Weights.java
 *   MNK = directml-windows-bindings/src/main/java/com/aresstack/windirectml/windows/MatMulNBitsKernel.java
 *   QGK = directml-inference/src/main/java/com/aresstack/windirectml/inference/qwen/QwenGpuKernels.java
 *   SFO = directml-inference/src/main/java/com/aresstack/windirectml/inference/simd/ScalarFloatMathOps.java
 *   VFO = directml-inference/src/main/java/com/aresstack/windirectml/inference/simd/vector/VectorFloatMathOps.java
 *
 * Floating point follows Java's strict semantics: every float multiply and
 * add is rounded to binary32 on its own.  The file MUST be compiled with
 * -ffp-contract=off (the recipe in oracle/Makefile does) so that the C
 * compiler does not fuse a*b+c where Java would not.  The only fused
 * operation is the Vector-API lane FMA of VFO:60, restated with fmaf().
 *
 * How each function is pinned (tests/test_oracle.py):
 *   fp16_to_fp32 ........ exhaustive over all 65536 bit patterns against the
 *                         IEEE value (normals, inf, nan) and the closed form
 *                         m*2^-150 for subnormals.
 *   fp32_to_fp16 ........ against numpy astype(float16) on 2^20 samples that
 *                         include every rounding tie class.
 *   dequantize .......... bit-exact against an exact rational computation
 *                         (tests/golden fixtures) incl. nibble order, odd
 *                         blocksPerRow zero-point indexing, q==zp -> +0.
 *   dot_scalar / lanes .. FloatMathOpsTest closed form (dot = 32) and the
 *                         17-element tail case; against fsum within the
 *                         standard gamma_n bound.
 *   matvec / matmul ..... QuantizedWeightMatvecTest closed forms (128, 0,
 *                         128, accumulate), matmul == repeated matvec bitwise,
 *                         and the exact rational result within gamma_n.
 *   zero-point layouts .. byte-level known answers for odd blocksPerRow.
 *   quantizer ........... closed forms for constant / zero / ramp blocks and
 *                         Java Math.round tie cases.
 *   row fusion .......... byte concatenation identity and the odd-nibble
 *                         refusal case.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define MNB_ORACLE_EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* fp16 <-> fp32                                                            */
/* ------------------------------------------------------------------------ */

static inline float bits_to_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline uint32_t f32_to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

/* P3W:665-683 (identical copy at Q2W:1730-1743).  Subnormal fp16 inputs are
 * mapped to intBitsToFloat(s<<31 | m<<13) * 2^-14 = m * 2^-150 (rounded to
 * the binary32 grid), which is not the IEEE value m * 2^-24.  Restated as the
 * reference computes it, including that quirk. */
MNB_ORACLE_EXPORT float mnb_ref_fp16_to_fp32(uint16_t bits) {
    uint32_t s = (bits >> 15) & 1u;
    uint32_t e = (bits >> 10) & 0x1Fu;
    uint32_t m = bits & 0x3FFu;
    if (e == 0) {
        if (m == 0) return s == 0 ? 0.0f : -0.0f;
        return bits_to_f32((s << 31) | (m << 13)) * (1.0f / 16384.0f);
    } else if (e == 31) {
        return bits_to_f32((s << 31) | 0x7F800000u | (m << 13));
    }
    return bits_to_f32((s << 31) | ((e - 15 + 127) << 23) | (m << 13));
}

/* P3W:643-652 readFp16Floats: element-wise fp16ToFp32 over a scale tensor. */
MNB_ORACLE_EXPORT void mnb_ref_scales_fp16_to_fp32(const uint16_t *in, float *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = mnb_ref_fp16_to_fp32(in[i]);
}

/* IEEE-754 binary32 -> binary16, round to nearest even.  Not a reference
 * function: the reference never produces fp16.  Used to state what an fp16
 * output of the exact binary32 value must be, and to round the synthetic
 * fp32 draws of scales and activations to fp16. */
MNB_ORACLE_EXPORT uint16_t mnb_ref_fp32_to_fp16(float f) {
    uint32_t x = f32_to_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7FFFFFFFu;
    if (absx >= 0x7F800000u) {                       /* inf or nan */
        if (absx == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | ((absx >> 13) & 0x3FFu));
    }
    int32_t e = (int32_t)(absx >> 23) - 127;          /* unbiased exponent */
    uint32_t mant = absx & 0x7FFFFFu;
    if (e > 15) return (uint16_t)(sign | 0x7C00u);    /* overflow -> inf */
    if (e >= -14) {                                   /* normal fp16 range */
        uint32_t m = mant;
        uint32_t h = ((uint32_t)(e + 15) << 10) | (m >> 13);
        uint32_t rem = m & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1;  /* may carry into exponent: correct */
        return (uint16_t)(sign | h);
    }
    /* subnormal fp16 or zero: value = (1.mant) * 2^e, target grid 2^-24 */
    if (e < -25) return (uint16_t)sign;               /* below half the smallest subnormal */
    uint32_t full = mant | 0x800000u;                 /* 24-bit significand, value = full * 2^(e-23) */
    int shift = (-14 - e) + 13;                       /* bits to drop to reach the 2^-24 grid */
    uint32_t h = full >> shift;
    uint32_t rem = full & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) h += 1;
    return (uint16_t)(sign | h);
}

/* ------------------------------------------------------------------------ */
/* Dequantization                                                           */
/* ------------------------------------------------------------------------ */

/* MNK:2674-2705 dequantizeInt4.  K here is the reference's K = blocksPerRow *
 * blockSize (the padded width); out is float[N*K] row-major.  Zero points are
 * the flat nibble stream indexed n*blocksPerRow+blk, low nibble first. */
MNB_ORACLE_EXPORT void mnb_ref_dequantize(const uint8_t *q, const float *scales, const uint8_t *zp,
                                          int32_t N, int32_t K, int32_t bs, float *out) {
    int32_t bpr = K / bs;
    for (int32_t n = 0; n < N; ++n) {
        int64_t qOffset = (int64_t)n * bpr * (bs / 2);
        int64_t scaleOffset = (int64_t)n * bpr;
        for (int32_t blk = 0; blk < bpr; ++blk) {
            float scale = scales[scaleOffset + blk];
            int64_t zpIdx = (int64_t)n * bpr + blk;
            int zpByte = zp[zpIdx / 2];
            int z = (zpIdx % 2 == 0) ? (zpByte & 0xF) : (zpByte >> 4);
            int64_t kBase = (int64_t)blk * bs;
            int64_t qBase = qOffset + (int64_t)blk * (bs / 2);
            int64_t rowBase = (int64_t)n * K;
            for (int32_t j = 0; j < bs / 2; ++j) {
                int packed = q[qBase + j];
                int w0 = (packed & 0xF) - z;
                int w1 = (packed >> 4) - z;
                out[rowBase + kBase + 2 * j] = (float)w0 * scale;
                out[rowBase + kBase + 2 * j + 1] = (float)w1 * scale;
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Block dot products                                                       */
/* ------------------------------------------------------------------------ */

/* SFO:16-22 ScalarFloatMathOps.dot: sequential binary32 sum of rounded
 * products. */
MNB_ORACLE_EXPORT float mnb_ref_dot_scalar(const float *a, const float *b, int32_t len) {
    float sum = 0.0f;
    for (int32_t k = 0; k < len; ++k) sum += a[k] * b[k];
    return sum;
}

/* VFO:47-68 VectorFloatMathOps.dot with `lanes` lanes: lane-wise FMA over
 * loopBound(len), then reduceLanes(ADD), then a scalar tail.  The JDK leaves
 * the order of reduceLanes(ADD) unspecified; it is restated here as a
 * left-to-right sum over lanes.  Bitwise output of this function is
 * therefore parity unpinned; it is used for timing and tolerance checks. */
#define MNB_MAX_LANES 16
MNB_ORACLE_EXPORT float mnb_ref_dot_lanes(const float *a, const float *b, int32_t len, int32_t lanes) {
    if (lanes < 4 || lanes > MNB_MAX_LANES) return mnb_ref_dot_scalar(a, b, len);
    float v[MNB_MAX_LANES] = {0};
    int32_t upper = len - (len % lanes);
    int32_t k = 0;
    for (; k < upper; k += lanes)
        for (int32_t l = 0; l < lanes; ++l) v[l] = fmaf(a[k + l], b[k + l], v[l]);
    float sum = 0.0f;
    for (int32_t l = 0; l < lanes; ++l) sum += v[l];
    for (; k < len; ++k) sum += a[k] * b[k];
    return sum;
}

/* 8-lane variant with the lane loop unrolled so that gcc emits one AVX2 FMA
 * per step.  Same arithmetic as mnb_ref_dot_lanes(a, b, len, 8). */
__attribute__((target("avx2,fma")))
static float dot_lanes8_avx2(const float *a, const float *b, int32_t len) {
    float v0 = 0, v1 = 0, v2 = 0, v3 = 0, v4 = 0, v5 = 0, v6 = 0, v7 = 0;
    int32_t upper = len - (len % 8);
    int32_t k = 0;
    for (; k < upper; k += 8) {
        v0 = fmaf(a[k + 0], b[k + 0], v0);
        v1 = fmaf(a[k + 1], b[k + 1], v1);
        v2 = fmaf(a[k + 2], b[k + 2], v2);
        v3 = fmaf(a[k + 3], b[k + 3], v3);
        v4 = fmaf(a[k + 4], b[k + 4], v4);
        v5 = fmaf(a[k + 5], b[k + 5], v5);
        v6 = fmaf(a[k + 6], b[k + 6], v6);
        v7 = fmaf(a[k + 7], b[k + 7], v7);
    }
    float sum = 0.0f;
    sum += v0; sum += v1; sum += v2; sum += v3;
    sum += v4; sum += v5; sum += v6; sum += v7;
    for (; k < len; ++k) sum += a[k] * b[k];
    return sum;
}

static float block_dot(const float *a, const float *b, int32_t len, int32_t lanes) {
    if (lanes == 0) return mnb_ref_dot_scalar(a, b, len);
    if (lanes == 8 && __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma"))
        return dot_lanes8_avx2(a, b, len);
    return mnb_ref_dot_lanes(a, b, len, lanes);
}

/* ------------------------------------------------------------------------ */
/* MatMulNBits on the CPU (the Java QuantizedWeight.matvec / matmul)        */
/* ------------------------------------------------------------------------ */

/* One output element of P3W:129-151 (matvec) / P3W:166-191 (matmul):
 * per block, unpack bs nibbles into a float buffer as ((nib) - zpVal) * scale,
 * low nibble first, then sum += dot(wBuf, x[kBase..], bs).  Returns `sum`;
 * the caller performs y += sum. */
static float row_sum(const uint8_t *q, const float *sc, const uint8_t *zp, int32_t n, int32_t K, int32_t bs,
                     const float *x, int32_t lanes) {
    float wBuf[512];
    int32_t bpr = K / bs;
    float sum = 0.0f;
    int64_t qOffset = (int64_t)n * bpr * (bs / 2);
    int64_t scaleOffset = (int64_t)n * bpr;
    for (int32_t blk = 0; blk < bpr; ++blk) {
        float scale = sc[scaleOffset + blk];
        int64_t zpIdx = (int64_t)n * bpr + blk;
        int zpByte = zp[zpIdx / 2];
        float zpVal = (float)((zpIdx % 2 == 0) ? (zpByte & 0xF) : (zpByte >> 4));
        int64_t kBase = (int64_t)blk * bs;
        const uint8_t *qb = q + qOffset + (int64_t)blk * (bs / 2);
        for (int32_t j = 0; j < bs / 2; ++j) {
            int packed = qb[j];
            wBuf[2 * j] = ((float)(packed & 0xF) - zpVal) * scale;
            wBuf[2 * j + 1] = ((float)(packed >> 4) - zpVal) * scale;
        }
        sum += block_dot(wBuf, x + kBase, bs, lanes);
    }
    return sum;
}

typedef struct {
    const uint8_t *q;
    const float *sc;
    const uint8_t *zp;
    int32_t N, K, bs, lanes;
    const float *x;
    float *y;
    int64_t begin, end;   /* flat (s, n) index range, s-major as P3W:167-168 */
} mm_job;

static void *mm_worker(void *arg) {
    mm_job *j = (mm_job *)arg;
    for (int64_t idx = j->begin; idx < j->end; ++idx) {
        int64_t s = idx / j->N;
        int32_t n = (int32_t)(idx - s * j->N);
        float sum = row_sum(j->q, j->sc, j->zp, n, j->K, j->bs, j->x + s * (int64_t)j->K, j->lanes);
        j->y[s * (int64_t)j->N + n] += sum;
    }
    return NULL;
}

/* P3W:157-192 matmul (Q2W:114-147 is the same loop over byte[]): Y += X @ W^T
 * for seqLen rows.  The reference parallelises IntStream.range(0, seqLen*N)
 * over the ForkJoin pool; each (s, n) element is computed by one thread, so
 * the result does not depend on the thread count.  `threads` <= 1 runs the
 * loop on the calling thread.  `lanes` = 0 uses the scalar dot (SFO),
 * otherwise the Vector-API dot with that many lanes (VFO). */
MNB_ORACLE_EXPORT int mnb_ref_matmul(const uint8_t *q, const float *scales, const uint8_t *zp, int32_t N,
                                     int32_t K, int32_t bs, const float *x, float *y, int32_t seqLen,
                                     int32_t lanes, int32_t threads) {
    if (N <= 0 || K <= 0 || bs <= 0 || bs > 512 || (bs & 1) || K % bs || seqLen <= 0) return -1;
    int64_t total = (int64_t)seqLen * N;
    if (threads <= 1) {
        mm_job j = {q, scales, zp, N, K, bs, lanes, x, y, 0, total};
        mm_worker(&j);
        return 0;
    }
    if (threads > 256) threads = 256;
    pthread_t tid[256];
    mm_job jobs[256];
    int64_t per = (total + threads - 1) / threads;
    int started = 0;
    for (int t = 0; t < threads; ++t) {
        int64_t b = per * t, e = b + per;
        if (b >= total) break;
        if (e > total) e = total;
        jobs[t] = (mm_job){q, scales, zp, N, K, bs, lanes, x, y, b, e};
        if (pthread_create(&tid[t], NULL, mm_worker, &jobs[t]) != 0) {
            mm_worker(&jobs[t]);
            tid[t] = 0;
        }
        started = t + 1;
    }
    for (int t = 0; t < started; ++t)
        if (tid[t]) pthread_join(tid[t], NULL);
    return 0;
}

/* P3W:123-152 matvec: y += x @ W^T, parallel over output rows. */
MNB_ORACLE_EXPORT int mnb_ref_matvec(const uint8_t *q, const float *scales, const uint8_t *zp, int32_t N,
                                     int32_t K, int32_t bs, const float *x, float *y, int32_t lanes,
                                     int32_t threads) {
    return mnb_ref_matmul(q, scales, zp, N, K, bs, x, y, 1, lanes, threads);
}

/* Float64 product of the dequantized weights for error analysis: y[s,n] =
 * sum_k x[s,k] * w[n,k] with w from mnb_ref_dequantize, accumulated in double.
 * Not a reference function; it is the "exact enough" side of tolerance
 * checks (double accumulation error is ~2^-29 relative to the fp32 oracle's). */
MNB_ORACLE_EXPORT int mnb_ref_matmul_f64(const uint8_t *q, const float *scales, const uint8_t *zp, int32_t N,
                                         int32_t K, int32_t bs, const float *x, double *y, int32_t seqLen) {
    if (N <= 0 || K <= 0 || bs <= 0 || (bs & 1) || K % bs || seqLen <= 0) return -1;
    int32_t bpr = K / bs;
    for (int32_t n = 0; n < N; ++n) {
        for (int32_t s = 0; s < seqLen; ++s) {
            double acc = 0.0;
            const float *xs = x + (int64_t)s * K;
            for (int32_t blk = 0; blk < bpr; ++blk) {
                double scale = scales[(int64_t)n * bpr + blk];
                int64_t zpIdx = (int64_t)n * bpr + blk;
                int zpByte = zp[zpIdx / 2];
                int z = (zpIdx % 2 == 0) ? (zpByte & 0xF) : (zpByte >> 4);
                const uint8_t *qb = q + ((int64_t)n * bpr + blk) * (bs / 2);
                for (int32_t j = 0; j < bs / 2; ++j) {
                    int packed = qb[j];
                    acc += (double)xs[(int64_t)blk * bs + 2 * j] * (double)((packed & 0xF) - z) * scale;
                    acc += (double)xs[(int64_t)blk * bs + 2 * j + 1] * (double)((packed >> 4) - z) * scale;
                }
            }
            y[(int64_t)s * N + n] = acc;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Zero-point layouts (Q2W:986-1121, P3W:589-598)                           */
/* ------------------------------------------------------------------------ */

/* Q2W:1119-1121 unpackUInt4 */
static int unpack_u4(const uint8_t *data, int64_t nibbleIndex) {
    int packed = data[nibbleIndex / 2];
    return (nibbleIndex & 1) == 0 ? (packed & 0x0F) : (packed >> 4);
}

/* Q2W:1400-1408 packUInt4 */
MNB_ORACLE_EXPORT void mnb_ref_pack_u4(uint8_t *out, int64_t nibbleIndex, int value) {
    int64_t byteIndex = nibbleIndex / 2;
    int v = value & 0x0F;
    if ((nibbleIndex & 1) == 0)
        out[byteIndex] = (uint8_t)((out[byteIndex] & 0xF0) | v);
    else
        out[byteIndex] = (uint8_t)((out[byteIndex] & 0x0F) | (v << 4));
}

/* Q2W:1410-1418 clampUInt4 */
static int clamp_u4(int v) { return v < 0 ? 0 : (v > 15 ? 15 : v); }

/* Java Math.round(float): the closest int, ties toward +infinity; NaN -> 0;
 * saturates at the int range.  Used by Q2W:1076 and Q2W:1396-1397. */
MNB_ORACLE_EXPORT int32_t mnb_ref_java_round(float a) {
    if (a != a) return 0;
    if (a >= 2147483647.0f) return 2147483647;
    if (a <= -2147483648.0f) return (int32_t)-2147483647 - 1;
    float fl = floorf(a);
    float diff = a - fl;   /* exact: both operands share the binade or fl is 0 */
    double r = (double)fl + (diff >= 0.5f ? 1.0 : 0.0);
    return (int32_t)r;
}

/* Q2W:1107-1112 createDefaultZeroPoints (and P3W:593-598): (n+1)/2 bytes of 0x88. */
MNB_ORACLE_EXPORT int64_t mnb_ref_zp_default(int64_t blockCount, uint8_t *out) {
    int64_t bytes = (blockCount + 1) / 2;
    memset(out, 0x88, (size_t)bytes);
    return bytes;
}

/* Q2W:1055-1075 repackRowPaddedUInt4ZeroPoints: ONNX [rows, ceil(bpr/2)]
 * row-padded nibbles -> flat nibble stream indexed row*bpr+block. */
MNB_ORACLE_EXPORT int64_t mnb_ref_zp_repack_row_padded(const uint8_t *rowPacked, int64_t len, int32_t rows,
                                                       int32_t bpr, uint8_t *out) {
    int64_t rowPackedBytes = (bpr + 1) / 2;
    if (len < rows * rowPackedBytes) return -1;
    int64_t outBytes = ((int64_t)rows * bpr + 1) / 2;
    memset(out, 0, (size_t)outBytes);
    for (int32_t row = 0; row < rows; ++row) {
        int64_t rowOffset = row * rowPackedBytes;
        int64_t blockBase = (int64_t)row * bpr;
        for (int32_t block = 0; block < bpr; ++block) {
            int value = unpack_u4(rowPacked, rowOffset * 2 + block);
            mnb_ref_pack_u4(out, blockBase + block, value);
        }
    }
    return outBytes;
}

/* Q2W:1077-1090 packUnpackedUInt4ZeroPoints(byte[]): one value per byte,
 * masked to the low nibble. */
MNB_ORACLE_EXPORT int64_t mnb_ref_zp_pack_unpacked_u8(const uint8_t *vals, int64_t len, int32_t rows,
                                                      int32_t bpr, uint8_t *out) {
    int64_t blockCount = (int64_t)rows * bpr;
    if (len < blockCount) return -1;
    int64_t outBytes = (blockCount + 1) / 2;
    memset(out, 0, (size_t)outBytes);
    for (int64_t i = 0; i < blockCount; ++i) mnb_ref_pack_u4(out, i, vals[i] & 0x0F);
    return outBytes;
}

/* Q2W:1092-1105 packUnpackedUInt4ZeroPoints(float[]): clampUInt4(Math.round(v)). */
MNB_ORACLE_EXPORT int64_t mnb_ref_zp_pack_unpacked_f32(const float *vals, int64_t len, int32_t rows,
                                                       int32_t bpr, uint8_t *out) {
    int64_t blockCount = (int64_t)rows * bpr;
    if (len < blockCount) return -1;
    int64_t outBytes = (blockCount + 1) / 2;
    memset(out, 0, (size_t)outBytes);
    for (int64_t i = 0; i < blockCount; ++i) mnb_ref_pack_u4(out, i, clamp_u4(mnb_ref_java_round(vals[i])));
    return outBytes;
}

/* Q2W:1023-1053 normalizeRawUInt4ZeroPoints: the decision tree that maps a
 * raw uint8 zero-point tensor (dims, bytes) to the flat runtime stream.
 * Returns the output byte count, or -1 for the IOException branch. */
MNB_ORACLE_EXPORT int64_t mnb_ref_zp_normalize_raw(const uint8_t *data, int64_t len, const int64_t *dims,
                                                   int32_t ndims, int32_t rows, int32_t bpr, uint8_t *out) {
    int64_t blockCount = (int64_t)rows * bpr;
    int64_t runtimePackedBytes = (blockCount + 1) / 2;
    int64_t rowPackedBytes = (bpr + 1) / 2;
    int64_t rowPackedTotal = (int64_t)rows * rowPackedBytes;
    if (ndims == 2 && dims[0] == rows && dims[1] == rowPackedBytes)
        return mnb_ref_zp_repack_row_padded(data, len, rows, bpr, out);
    if (ndims == 2 && dims[0] == rows && dims[1] == bpr)
        return mnb_ref_zp_pack_unpacked_u8(data, len, rows, bpr, out);
    if (len == rowPackedTotal && rowPackedTotal != runtimePackedBytes)
        return mnb_ref_zp_repack_row_padded(data, len, rows, bpr, out);
    if (len == runtimePackedBytes) {
        memcpy(out, data, (size_t)len);
        return len;
    }
    if (len == blockCount) return mnb_ref_zp_pack_unpacked_u8(data, len, rows, bpr, out);
    return -1;
}

/* ------------------------------------------------------------------------ */
/* Tied lm_head uint4 quantizer (Q2W:1339-1398)                              */
/* ------------------------------------------------------------------------ */

/* Q2W:1339-1346 chooseTiedLmHeadBlockSize */
MNB_ORACLE_EXPORT int32_t mnb_ref_choose_tied_block_size(int32_t hidden) {
    static const int32_t cand[4] = {128, 64, 32, 16};
    for (int i = 0; i < 4; ++i)
        if (hidden % cand[i] == 0) return cand[i];
    return 0;
}

/* Q2W:1373-1398 calculateUInt4QuantizationBlock */
MNB_ORACLE_EXPORT void mnb_ref_quant_block_params(const float *data, int32_t length, float *scaleOut,
                                                  int32_t *zpOut) {
    float mn = INFINITY, mx = -INFINITY;
    for (int32_t i = 0; i < length; ++i) {
        float v = data[i];
        if (v < mn) mn = v;
        if (v > mx) mx = v;
    }
    if (mx == mn) {
        if (fabsf(mx) < 1.0e-8f) { *scaleOut = 1.0f; *zpOut = 0; return; }
        if (mx > 0.0f) { *scaleOut = mx / 15.0f; *zpOut = 0; return; }
        *scaleOut = -mn / 15.0f; *zpOut = 15; return;
    }
    float scale = (mx - mn) / 15.0f;
    *scaleOut = scale;
    *zpOut = clamp_u4(mnb_ref_java_round(-mn / scale));
}

/* Q2W:1348-1371 quantizeDenseRowsToUInt4 (+ Q2W:1390-1398 per block):
 * q[i] = clampUInt4(Math.round(v / scale + zp)). */
MNB_ORACLE_EXPORT int mnb_ref_quantize_rows_u4(const float *data, int32_t rows, int32_t cols, int32_t bs,
                                               uint8_t *q, float *scales, uint8_t *zp) {
    if (bs <= 0 || cols % bs) return -1;
    int32_t bpr = cols / bs;
    int64_t rowBytes = cols / 2;
    memset(q, 0, (size_t)(rows * rowBytes));
    memset(zp, 0, (size_t)(((int64_t)rows * bpr + 1) / 2));
    for (int32_t row = 0; row < rows; ++row) {
        for (int32_t block = 0; block < bpr; ++block) {
            const float *v = data + (int64_t)row * cols + (int64_t)block * bs;
            float scale;
            int32_t z;
            mnb_ref_quant_block_params(v, bs, &scale, &z);
            int64_t blockIndex = (int64_t)row * bpr + block;
            scales[blockIndex] = scale;
            mnb_ref_pack_u4(zp, blockIndex, z);
            int64_t outOffset = (int64_t)row * rowBytes + (int64_t)block * (bs / 2);
            for (int32_t i = 0; i < bs; ++i) {
                float t = v[i] / scale + (float)z;
                mnb_ref_pack_u4(q, outOffset * 2 + i, clamp_u4(mnb_ref_java_round(t)));
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Row fusion (QGK:243-315)                                                  */
/* ------------------------------------------------------------------------ */

/* tryFuseQuantizedRowwise: concatenate q, scales and flat zero points of
 * `parts` weights along N.  Returns the fused N, or -1 when the reference
 * would refuse (K/blockSize mismatch, or a non-last part whose
 * N_i*blocksPerRow is odd, i.e. its zero-point stream ends mid-byte). */
MNB_ORACLE_EXPORT int32_t mnb_ref_fuse_rows(int32_t parts, const int32_t *Ns, const int32_t *Ks,
                                            const int32_t *bss, const uint8_t *const *qs,
                                            const float *const *scales, const uint8_t *const *zps,
                                            uint8_t *outQ, float *outS, uint8_t *outZ) {
    if (parts <= 0) return -1;
    int32_t K = Ks[0], bs = bss[0];
    int32_t bpr = K / bs;
    for (int32_t i = 0; i < parts; ++i) {
        if (Ks[i] != K || bss[i] != bs) return -1;
        if (i < parts - 1 && ((int64_t)Ns[i] * bpr) % 2 != 0) return -1;
    }
    int64_t rowBytes = K / 2;
    int64_t qOff = 0, sOff = 0, zOff = 0;
    int32_t fusedN = 0;
    for (int32_t i = 0; i < parts; ++i) {
        int64_t partBytes = (int64_t)Ns[i] * rowBytes;
        memcpy(outQ + qOff, qs[i], (size_t)partBytes);
        qOff += partBytes;
        int64_t partFloats = (int64_t)Ns[i] * bpr;
        memcpy(outS + sOff, scales[i], (size_t)partFloats * sizeof(float));
        sOff += partFloats;
        int64_t partZpBytes = (partFloats + 1) / 2;
        memcpy(outZ + zOff, zps[i], (size_t)partZpBytes);
        zOff += partZpBytes;
        fusedN += Ns[i];
    }
    return fusedN;
}
