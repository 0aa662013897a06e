/*
 * mnb.h -- C ABI of libmnb_hip.so, the MI355X (gfx950) int4 MatMulNBits library.
 *
 * One weight object holds one MatMulNBits weight triplet (packed uint4 nibbles,
 * per-block scales, optional packed uint4 zero points) resident in HBM.  The
 * library owns every device buffer it creates; weights are uploaded once.
 *
 * Each entry point names the reference interface it replaces.  Paths are
 * relative to the reference repository root:
 *   MNK = directml-windows-bindings/src/main/java/com/aresstack/windirectml/windows/MatMulNBitsKernel.java
 *   P3W = directml-inference/src/main/java/com/aresstack/windirectml/inference/phi3/Phi3Weights.java
 *   Q2W = directml-inference/src/main/java/com/aresstack/windirectml/inference/qwen/Qwen2Weights.java
 *   QLK = directml-windows-bindings/src/main/java/com/aresstack/windirectml/runtime/kernels/QuantizedLinearKernel.java
 *
 * Conventions
 *   - Every function returns an int32_t status (MNB_OK = 0).  On failure a
 *     message is available from mnb_last_error() on the calling thread.
 *   - Status codes map onto the reference's exceptions:
 *       MNB_ERR_INVALID_ARGUMENT -> IllegalArgumentException
 *       MNB_ERR_INVALID_STATE    -> IllegalStateException ("Kernel not prepared")
 *       everything else          -> RuntimeException("MatMulNBitsKernel.<op> failed")
 *   - Calls on one context share its workspace (the GEMM's split-tile
 *     partial sums) and its staging buffers, the same as one reference
 *     kernel instance shares its command list (MNK:77-81).  Calls that use
 *     them must not overlap: host-memory calls, products with M > 16, products
 *     whose x is staged (fp32 x, x not 16-byte aligned, K not a multiple of
 *     8) and M > 16 groups in stream-K order or with parts
 *     (MNB_ORDER_TILE_LIST_PARTS).  Issue those on one stream or order them.
 *     The other device-pointer calls (M <= 16 with 16-byte aligned fp16 x
 *     and K a multiple of 8, mnb_group_run of M <= 16 groups and of M > 16
 *     groups in plain tile-list order) touch no shared buffer and may run
 *     concurrently on distinct streams.
 *   - Pointers: by default x/y/out are DEVICE pointers and the call is
 *     asynchronous on `stream` (a hipStream_t; NULL = the context's stream).
 *     With MNB_HOST_MEMORY they are host pointers, the call copies through
 *     device staging buffers and returns when the result is in host memory
 *     (the reference's float[] contract, MNK:1847-1914).
 */
#ifndef MNB_H
#define MNB_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MNB_ABI_VERSION 1

/* status codes */
#define MNB_OK 0
#define MNB_ERR_INVALID_ARGUMENT 1
#define MNB_ERR_INVALID_STATE 2
#define MNB_ERR_OUT_OF_MEMORY 3
#define MNB_ERR_DEVICE 4
#define MNB_ERR_NO_DEVICE 5
#define MNB_ERR_UNSUPPORTED 6
#define MNB_ERR_IO 7 /* weight-file errors: the reference's IOException */

/* element types */
#define MNB_F32 0
#define MNB_F16 1

/* zero-point layouts accepted by mnb_weight_create */
#define MNB_ZP_NONE 0       /* no tensor: implicit zero point 8 (P3W:593-598, Q2W:1107-1112) */
#define MNB_ZP_FLAT 1       /* flat nibble stream, nibble n*kb+blk, low nibble first, (N*kb+1)/2 bytes (MNK:258-262) */
#define MNB_ZP_ROW_PADDED 2 /* ONNX MatMulNBits layout [N, ceil(kb/2)] (Q2W:1055-1075) */

/* flags */
#define MNB_HOST_MEMORY 0x1u /* x/y/out are host pointers; the call is synchronous */
#define MNB_ACCUMULATE 0x2u  /* y += x W^T (QuantizedWeight.matvec/matmul, P3W:123-192) instead of y = x W^T */

typedef struct mnb_context mnb_context;
typedef struct mnb_weight mnb_weight;

typedef struct mnb_device_info {
    char name[64];
    char arch[64];
    int32_t compute_units;
    int32_t clock_khz;
    int32_t memory_clock_khz;
    int32_t memory_bus_width;
    int64_t total_memory;
    int32_t l2_bytes;
    int32_t lds_bytes_per_block;
    int32_t wavefront_size;
    int32_t device;
} mnb_device_info;

/* Library version (MNB_ABI_VERSION).  No reference counterpart. */
int32_t mnb_version(void);

/* Message of the last failed call on this thread ("" if none).  Replaces the
 * exception messages of MNK:1849-1850, 1909-1913 and 966-969. */
const char *mnb_last_error(void);

/* Open the library on HIP device `device`.  Replaces WindowsBindings.init
 * plus the per-kernel command allocator/queue/fence set-up (MNK:1168-1247,
 * prepareExecInfraInt4).  Fails with MNB_ERR_NO_DEVICE when no gfx950 device
 * is present. */
int32_t mnb_context_create(int32_t device, mnb_context **out);

/* Release the context's stream and staging buffers.  Weights created on it
 * must be destroyed first (MNB_ERR_INVALID_STATE otherwise). */
int32_t mnb_context_destroy(mnb_context *ctx);

/* Device properties used for the roofline (peak clocks, CU count, memory). */
int32_t mnb_context_info(const mnb_context *ctx, mnb_device_info *out);

/* Upload one weight triplet once.  Replaces the INT4 constructor
 * `new MatMulNBitsKernel(wb, N, K, byte[] qWeight, float[] scales,
 * byte[] zeroPoints, int blockSize)` (MNK:940-970 -> prepareInt4Gpu
 * MNK:1168-1247) and QLK:25-31's weight/scales/zeros operands.
 *
 *   N, K        output and input features.  K may be the true K; the packed
 *               tensors always hold kb = ceil(K/block_size) full blocks per
 *               row.  Passing the reference's K (= kb*block_size) is the
 *               same call as the reference.
 *   block_size  power of two in [16, 4096]
 *   bits        must be 4
 *   q           uint8 [N, kb, block_size/2], two nibbles per byte, low first; q_bytes >= N*kb*block_size/2
 *   scales      [N, kb] of scale_type (MNB_F16 bit patterns or MNB_F32); scale_count >= N*kb.
 *               F32 scales are kept exactly (device copy is fp16 when every
 *               value is exactly representable, else fp32).
 *   zero_points layout per zp_layout; NULL with MNB_ZP_NONE
 *   flags       0 (host pointers for all tensors)
 */
int32_t mnb_weight_create(mnb_context *ctx, int32_t N, int32_t K, int32_t block_size, int32_t bits,
                          const uint8_t *q, int64_t q_bytes, const void *scales, int32_t scale_type,
                          int64_t scale_count, const uint8_t *zero_points, int64_t zp_bytes, int32_t zp_layout,
                          uint32_t flags, mnb_weight **out);

/* New weight whose rows are the rows of parts[0], then parts[1], ... (all
 * created on ctx with the same K and block size), built on the device from
 * the parts' resident buffers.  Replaces QwenGpuKernels.tryFuseQuantizedRowwise
 * (directml-inference/.../qwen/QwenGpuKernels.java:243-315) and
 * Phi3GpuKernels.createFusedQKV (directml-inference/.../phi3/Phi3GpuKernels.java:
 * 114-137).  The fused weight equals the weight created from the concatenated
 * triplet; the parts stay valid and independent of it.  Unlike the reference,
 * any N_i works (zero points are stored per row on the device, so the
 * byte-alignment condition and its FP32 fallback do not arise), and the Phi-3
 * QKV stays int4 (the reference concatenates fp32 dequantized rows: the same
 * values).  Parts may differ in scale type (fp16 widens to fp32 exactly) and
 * in having zero points (implicit 8 where absent).  A part with another K or
 * block size fails with "part i has K=.. blockSize=.. but expected K=..
 * blockSize=..". */
int32_t mnb_weight_fuse_rows(mnb_context *ctx, const mnb_weight *const *parts, int32_t count, mnb_weight **out);

/* Quantize a dense matrix data[rows, cols] (row-major, MNB_F32 or MNB_F16)
 * to an int4 weight on the device: asymmetric min/max uint4 per block of
 * block_size columns with the reference's arithmetic, so the weight's bytes
 * equal those of Qwen2Weights.quantizeDenseRowsToUInt4 (Q2W:1352-1422; the
 * tied lm_head of Q2W:1329-1350).  block_size 0 picks the reference's choice,
 * the largest of 128, 64, 32, 16 dividing cols (chooseTiedLmHeadBlockSize,
 * Q2W:1339-1346); otherwise one of those four dividing cols.  fp16 data is
 * widened exactly (pass fp32 for the reference's own fp16 widening).  The
 * weight keeps fp32 scales and zero points.  flags: MNB_HOST_MEMORY when
 * data is a host pointer (copied through a temporary device buffer); device
 * data must be 16-byte aligned.  Synchronous on the context's stream. */
int32_t mnb_weight_quantize(mnb_context *ctx, const void *data, int32_t data_type, int32_t rows, int32_t cols,
                            int32_t block_size, uint32_t flags, mnb_weight **out);

/* Host copy of a resident weight as the reference's arrays: q [N, kb,
 * bs/2] (q_cap >= N*kb*bs/2), fp32 scales [N*kb], flat zero points
 * ((N*kb+1)/2 bytes; the 0x88 fill when the weight has the implicit zero
 * point).  The accessors QuantizedWeight.qWeight()/scales()/zeroPoints()
 * (P3W:83-110) for weights that exist only on the device (fused, quantized
 * on the device, loaded from a file). */
int32_t mnb_weight_read(mnb_context *ctx, const mnb_weight *w, uint8_t *q, int64_t q_cap, float *scales,
                        int64_t scale_cap, uint8_t *zero_points, int64_t zp_cap);

/* Free the weight's device buffers.  Replaces MatMulNBitsKernel.close()
 * (MNK:2740-2800).  NULL is accepted. */
int32_t mnb_weight_destroy(mnb_weight *w);

/* N, K (as passed at creation) and block size.  Replaces getN()/getK()
 * (MNK:2803-2812). */
int32_t mnb_weight_shape(const mnb_weight *w, int32_t *N, int32_t *K, int32_t *block_size);

/* Bytes of HBM the weight occupies (packed nibbles, scales, zero points). */
int64_t mnb_weight_device_bytes(const mnb_weight *w);

/* y[M, N] = x[M, K] W^T  (or += with MNB_ACCUMULATE).
 * Replaces matvec(float[] x, float[] out) (M = 1, overwrite, MNK:1847-1914),
 * matmulBatch(float[] xBatch, float[] outBatch, int M) (overwrite,
 * MNK:2145-2263), the resident variants (MNK:1687-1832, 2276-2358) when
 * called with device pointers, QuantizedWeight.matvec/matmul (accumulate,
 * P3W:123-192, Q2W:80-147) with MNB_ACCUMULATE, and QLK:25-31 dispatch.
 *
 *   x_type, y_type  MNB_F16 or MNB_F32; x is [M, K] row-major, y is [M, N]
 *   x_elems         number of elements the caller's x holds; M == 1 requires
 *                   x_elems == K ("Input length L != K=K"), M > 1 requires >= M*K
 *   y_elems         elements in y; must be >= M*N
 *   M               any M >= 1 (no 256-row chunking is needed; x beyond 2 GiB
 *                   runs in row chunks); with packed weights of 4 GiB or more
 *                   only M <= 16 (else MNB_ERR_UNSUPPORTED)
 * Arithmetic: products of fp16 operands accumulated in fp32.  The output is
 * within 1e-3*sqrt(K)*max|x|*max|w| of the reference's fp32 CPU path, for any
 * block scales (the device copy of a weight's scales carries a power of two
 * that keeps every fp16 weight operand normal; results are scaled back
 * exactly).  fp32 x is rounded to fp16 once, so |x| must stay below 65504.
 */
int32_t mnb_matmul(mnb_context *ctx, const mnb_weight *w, int32_t M, const void *x, int32_t x_type,
                   int64_t x_elems, void *y, int32_t y_type, int64_t y_elems, uint32_t flags, void *stream);

/* mnb_matmul on device pointers that allocates nothing: no counterpart in
 * the reference; for callers that cannot allocate device memory while they
 * run (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, checks, kernels and results as mnb_matmul
 * without MNB_HOST_MEMORY (which it refuses).  The GEMM's split-tile partial
 * sums and the fp16 copy of x (made when x is fp32, not 16-byte aligned or K
 * is not a multiple of 8) live in a fixed 80 MiB device array of the library
 * instead of context buffers: 64 MiB of partial tiles and at most 16 MiB of
 * staged x, M * roundup(K, 8) * 2 bytes (a larger staging need fails with
 * MNB_ERR_INVALID_ARGUMENT).  Each GPU holds its own array for the life of
 * the process; every call on one GPU shares it, so calls that overlap on one
 * GPU (concurrent streams, other threads) race: order them. */
int32_t mnb_matmul_noalloc(mnb_context *ctx, const mnb_weight *w, int32_t M, const void *x, int32_t x_type,
                           int64_t x_elems, void *y, int32_t y_type, int64_t y_elems, uint32_t flags, void *stream);

/* Dequantize to out[N, K] (K as passed at creation), w = (q - zp) * scale
 * computed in fp32 and written as fp32, or rounded to nearest-even fp16.
 * Replaces MatMulNBitsKernel.dequantizeInt4 (MNK:2674-2705); the fp32 output
 * is bit-identical to it. */
int32_t mnb_dequantize(mnb_context *ctx, const mnb_weight *w, void *out, int32_t out_type, int64_t out_elems,
                       uint32_t flags, void *stream);

/* Always true for a created weight.  Replaces supportsBatch() (MNK:2128). */
int32_t mnb_supports_batch(const mnb_weight *w);

/* Largest M one mnb_matmul call accepts.  Replaces maxBatchRows()
 * (MNK:2361, which is 256 there). */
int32_t mnb_max_batch_rows(void);

/* A recorded group of independent products executed as ONE launch.  No
 * reference counterpart: the reference records every MatMulNBits dispatch
 * into its command list with a UAV barrier after it (recordResidentInto /
 * recordBatchDispatchOnly, MNK:1935-2117; WarpExecutionContext.java:131-160;
 * the layer chain o_proj -> add -> rmsnorm -> gate_up -> swiglu -> down -> add
 * of Phi3GpuPipeline.java:183-244).  That dependent form maps to
 * stream-ordered device-pointer mnb_matmul calls (captured in a HIP graph to
 * replay them); a group is for products that do not depend on each other
 * (projections of one input, or of independent sequences): the items may run
 * concurrently, so no item may read another item's output.
 * Each item: device pointers, fp16 x [M, K] (K a multiple of 8, 16-byte
 * aligned), y [M, N] fp16 or fp32, M >= 1; all items share the weight variant
 * (scale type, zero points or not, block size class) and one M class: all
 * M == 1 (one persistent streaming launch), all 1 < M <= 16 (when no item
 * has more than 4 rows, the streaming launch with the group's largest M rows
 * of x per job),
 * or all M > 16 (prefill-shaped products: one GEMM launch over all items'
 * tiles).  A GEMM
 * group with few tiles splits tiles across workgroups (stream-K) and then
 * uses the context's GEMM workspace, so it must not overlap other M > 16
 * calls on the context; a group with many tiles (also one of 1 < M <= 16),
 * or whose items have M <= 64 and whose 64-row tiles balance well enough,
 * gives each workgroup whole tiles and uses no workspace, unless a few of
 * its tiles are much longer than a workgroup's share: those are then cut
 * along K into parts whose fp32 partial tiles go to the context's GEMM
 * workspace and are summed by a second launch (MNB_ORDER_TILE_LIST_PARTS,
 * reported by mnb_group_plan), so such a group run must not overlap other
 * M > 16 calls on the context either.  An item whose x
 * is 2 GiB or more, or whose packed weight is 4 GiB or more, is refused with
 * MNB_ERR_UNSUPPORTED (mnb_matmul runs such x in row chunks).  The group keeps
 * its own device descriptor table, so mnb_group_run allocates nothing and can
 * be captured in a HIP graph. */
typedef struct mnb_group mnb_group;
typedef struct mnb_group_item {
    const mnb_weight *weight;
    int32_t M;
    const void *x;
    int32_t x_type;
    int64_t x_elems;
    void *y;
    int32_t y_type;
    int64_t y_elems;
    uint32_t flags; /* 0 or MNB_ACCUMULATE */
} mnb_group_item;
int32_t mnb_group_create(mnb_context *ctx, int32_t count, const mnb_group_item *items, mnb_group **out);
int32_t mnb_group_run(mnb_context *ctx, const mnb_group *group, void *stream);
int32_t mnb_group_destroy(mnb_group *group);

/* Which kernel and work order a product or a recorded group runs (no
 * reference counterpart: the schedule is chosen by cost models, and this
 * lets callers and tests see the choice). */
#define MNB_KERNEL_GEMV 1        /* one workgroup per 16-row n-tile, waves split K (M <= 16) */
#define MNB_KERNEL_STREAM 2      /* persistent weight stream over (product, n-tile) units (groups with M <= 4) */
#define MNB_KERNEL_GEMV_GROUP 3  /* the GEMV kernel over every product's n-tiles (4 < M <= 16 groups) */
#define MNB_KERNEL_GEMM 4        /* the MFMA GEMM */
#define MNB_KERNEL_KSLICE 5      /* one product, M >= 9: workgroup per output block, its waves split K (no split tiles) */
#define MNB_ORDER_NONE 0         /* one unit of work per workgroup or a static unit list */
#define MNB_ORDER_STREAM_K 1     /* (tile, k-stage) iterations cut into equal ranges; split tiles reduced after */
#define MNB_ORDER_TILE_LIST 2    /* whole tiles per workgroup from a tile list (a table, or closed form for one product) */
#define MNB_ORDER_TILE_LIST_PARTS 3 /* a group's tile list whose longest tiles are cut along K into parts (fp32 partial
                                       tiles, summed in K order by a reduce launch after) */
typedef struct mnb_plan_info {
    int32_t kernel;      /* MNB_KERNEL_* */
    int32_t order;       /* MNB_ORDER_* */
    int32_t tile_rows;   /* output tile: rows of x (GEMM 32, 64 or 128; K-sliced 16 (M <= 16), 32, 64 or 128;
                            streaming kernel: the group's largest M when 2 <= M <= 4); 0 otherwise */
    int32_t tile_cols;   /* output tile: columns (GEMM 256 or 512; K-sliced 16, 32 or 64); 16 for the GEMV kernels */
    int32_t workgroups;  /* grid size */
} mnb_plan_info;
/* The plan of mnb_matmul(ctx, w, M, ...) with device pointers (for M
 * beyond 2 GiB of x rows, the plan of the first chunk of rows). */
int32_t mnb_matmul_plan(const mnb_context *ctx, const mnb_weight *w, int32_t M, mnb_plan_info *out);
/* The plan recorded by mnb_group_create. */
int32_t mnb_group_plan(const mnb_group *group, mnb_plan_info *out);

/* Device buffers for resident activations (WarpGpuBuffer in the reference,
 * used by MNK:1687-1832). */
int32_t mnb_device_alloc(mnb_context *ctx, int64_t bytes, void **out);
int32_t mnb_device_free(mnb_context *ctx, void *ptr);

#define MNB_COPY_H2D 0
#define MNB_COPY_D2H 1
#define MNB_COPY_D2D 2
/* Synchronous copy on the context's stream. */
int32_t mnb_memcpy(mnb_context *ctx, void *dst, const void *src, int64_t bytes, int32_t kind);

/* Wait for all work on the context's stream.  Replaces the fence wait
 * (MNK:1894-1901). */
int32_t mnb_synchronize(mnb_context *ctx);

/* ---------------------------------------------------------------------------
 * Weight files.  A pack is a read-only memory mapping of a file that holds
 * MatMulNBits weight triplets, with its directory parsed and checked:
 *
 *   MNB_PACK_PHI3   .wdmlpack whose manifest says architecture "phi3": one
 *                   triplet per role ("layers.<l>.q_proj", ..., "lm_head"):
 *                   <role>.qweight UINT8 dims [N, K, blockSize], <role>.scales
 *                   FLOAT [N*kb], <role>.zeropoints UINT8 flat nibble stream
 *                   (PRP:35-46,132-152; Phi3WdmlPackCompiler.java:236-264).
 *   MNB_PACK_QWEN2  .wdmlpack whose model.architecture is "qwen2": the ONNX
 *                   initializers stored in the payload plus the MatMulNBits
 *                   nodes of the manifest's runtimeGraph (QWS:59-185).  A
 *                   manifest-only package opens its source ONNX model instead
 *                   (QWS:76-86) and reports MNB_PACK_ONNX.
 *   MNB_PACK_ONNX   ONNX model; MatMulNBits inputs [A, B, scales, zero_points?]
 *                   (Q2W:534-545); external data in model.onnx_data or
 *                   model.onnx.data beside the model (QwenModelDirValidator.java:163-174).
 *   MNB_PACK_SAFETENSORS  a *.safetensors file: dense tensors only (no
 *                   MatMulNBits triplets), checked as SafeTensorsReader.read
 *                   does (directml-inference/.../model/SafeTensorsReader.java:
 *                   84-277, its IOException texts); weight names are its tensor
 *                   names in directory order.  A dense matrix of any pack
 *                   becomes an int4 weight with mnb_pack_weight_quantize.
 *
 * Weight names are the Phi-3 roles, or the first output of each MatMulNBits
 * node in graph order.  A triplet is resolved as the reference loads it
 * (Q2W:936-976, 986-1121; PRP:132-145): N = dims[0], blockSize = 2*dims[2],
 * K = kb*blockSize for ONNX; fp16 scales are widened with the reference's
 * fp16ToFp32 (P3W:665-683, including its subnormal rounding); zero points are
 * normalized to the flat nibble stream; a missing zero-point tensor means
 * every zero point is 8.  Failures return MNB_ERR_IO with the reference's
 * IOException text (WdmlPackWriter.java:114-177,254-259; WdmlPackManifest.java:
 * 108-123; WdmlPackReader.java:67-96; Q2W:936-976,1017-1048,2063-2131).
 *   PRP = directml-inference/src/main/java/com/aresstack/windirectml/inference/phi3/Phi3RuntimePackage.java
 *   QWS = directml-inference/src/main/java/com/aresstack/windirectml/inference/qwen/QwenWdmlPackModelSource.java
 * A pack is immutable after mnb_pack_open: concurrent calls on it are safe.
 */
#define MNB_PACK_PHI3 1
#define MNB_PACK_QWEN2 2
#define MNB_PACK_ONNX 3
#define MNB_PACK_SAFETENSORS 4

typedef struct mnb_pack mnb_pack;
typedef struct mnb_triplet_info {
    int32_t N;
    int32_t K;              /* kb * block_size, as the reference derives it */
    int32_t block_size;
    int32_t blocks_per_row; /* K / block_size for Phi-3 (P3W:51-60), dims[1] for ONNX */
    int64_t q_bytes;        /* packed nibbles as stored */
    int64_t scale_count;    /* fp32 scales after widening */
    int64_t zp_bytes;       /* flat zero-point stream (the 0x88 fill when zp_implicit) */
    int32_t zp_implicit;    /* 1: no zero-point tensor, every zero point is 8 (Q2W:1107-1112) */
    int32_t scale_dtype;    /* ONNX element type of the stored scales: 1 FLOAT, 10 FLOAT16 */
} mnb_triplet_info;

/* Open and check a weight file.  Replaces Phi3RuntimePackage.open (PRP:35-46)
 * with its runtimeTensorCatalog (WdmlPackReader.java:37-96), the Qwen package
 * and ONNX sources (QWS:59-185; Q2W:495-545, 1809-1938) and their tensor type
 * checks (Q2W:2063-2117).  A file named *.wdmlpack or starting with the bytes
 * "WDMLPACK" is read as a package; any other file as an ONNX model. */
int32_t mnb_pack_open(const char *path, mnb_pack **out);

/* Unmap the file.  Weights created from the pack stay valid (they live in
 * HBM); this is the release of the host copies (Q2W:1754-1785).  NULL is
 * accepted. */
int32_t mnb_pack_close(mnb_pack *pack);

int32_t mnb_pack_kind(const mnb_pack *pack, int32_t *kind);
int32_t mnb_pack_weight_count(const mnb_pack *pack, int32_t *count);

/* Name of weight `index` (0-based, in file order), NUL-terminated into buf
 * (truncated to cap-1 bytes); *length receives the full length. */
int32_t mnb_pack_weight_name(const mnb_pack *pack, int32_t index, char *buf, int64_t cap, int64_t *length);

/* First weight whose name contains both "layers.<layer>" and `projection`,
 * the lookup of Qwen2Weights.loadQuantizedProjection (Q2W:800-815); fails with
 * "Quantized weight not found for layer <l> <projection>". */
int32_t mnb_pack_find_projection(const mnb_pack *pack, int32_t layer, const char *projection, char *buf, int64_t cap,
                                 int64_t *length);

/* Shape and sizes of one triplet, resolved as above. */
int32_t mnb_pack_weight_info(const mnb_pack *pack, const char *name, mnb_triplet_info *out);

/* Host copy of one resolved triplet: the reference's QuantizedWeight arrays
 * (qWeight bytes, fp32 scales, flat zero points; P3W:51-110, Q2W:58-79).
 * Buffers must hold info.q_bytes, info.scale_count and info.zp_bytes. */
int32_t mnb_pack_read_weight(const mnb_pack *pack, const char *name, uint8_t *q, int64_t q_cap, float *scales,
                             int64_t scale_cap, uint8_t *zp, int64_t zp_cap);

/* Upload one triplet straight from the mapping to HBM: mnb_weight_create on
 * the resolved triplet (no host copy of the packed nibbles is made).  The
 * same call as constructing the reference's GPU kernel from the loaded
 * QuantizedWeight (MNK:940-970).  A zero-point stream whose nibbles are all 8
 * is uploaded as the implicit zero point (identical values). */
int32_t mnb_pack_weight_create(mnb_context *ctx, const mnb_pack *pack, const char *name, mnb_weight **out);

/* Element type (ONNX code: 1 FLOAT, 10 FLOAT16, 16 BFLOAT16, ...) and shape
 * of any tensor of the pack (up to dims_cap dimensions written; *ndims gets
 * the rank).  No reference counterpart beyond the tensor catalogs of its
 * readers (SafeTensorsReader.SafeTensorEntry, OnnxModelReader.OnnxTensor). */
int32_t mnb_pack_tensor_info(const mnb_pack *pack, const char *name, int32_t *dtype, int64_t *dims, int32_t dims_cap,
                             int32_t *ndims);

/* The runtime-quantized tied lm_head from a weight file: the dense matrix
 * `name` (e.g. "model.embed_tokens.weight" of a safetensors file or an ONNX
 * model) read as the reference reads its embedding table (Q2W:599-704:
 * FLOAT as stored, FLOAT16 through fp16ToFp32, other types fail), its shape
 * checked against [rows, cols] ("Unexpected dimensions for ..."; Q2W:1637),
 * then quantized on the device exactly as mnb_weight_quantize (createTiedLmHead
 * + quantizeDenseRowsToUInt4, Q2W:1329-1422; block_size 0 is the reference's
 * choice).  Failures to read return MNB_ERR_IO. */
int32_t mnb_pack_weight_quantize(mnb_context *ctx, const mnb_pack *pack, const char *name, int32_t rows, int32_t cols,
                                 int32_t block_size, mnb_weight **out);

#ifdef __cplusplus
}
#endif

#endif /* MNB_H */
