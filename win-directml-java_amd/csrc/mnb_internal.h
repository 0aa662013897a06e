// mnb_internal.h -- shared definitions of libmnb_hip: the HBM layout of a
// resident weight, the context, and the kernel launchers.
//
// HBM layout of one weight (N rows, kb blocks of bs nibbles per row):
//
//   The weight is cut into tiles of 16 rows x 128 k ("n-tile" x "super-tile"),
//   NT = ceil(N/16) n-tiles and ST = ceil(kb*bs/128) super-tiles per row.
//   Each tile is 1 KiB of packed nibbles stored so that ONE 16-byte load per
//   lane of a 64-lane wavefront brings a whole tile into registers already in
//   the operand order of v_mfma_f32_16x16x32_f16:
//
//     byte offset of tile (nt, st)   = ((nt*ST + st) * 64) * 16
//     lane l = g*16 + r  (r = row within the tile, g = 8-k group)  -> 16 bytes
//     dword j (0..3) of that lane    = 8 nibbles of row nt*16+r,
//                                      k = st*128 + 32*j + 8*g + (0..7)
//     nibble order inside the dword  = k0,k2,k4,k6 in bits 0..15 and
//                                      k1,k3,k5,k7 in bits 16..31, so that
//                                      (d & 0x000F000F) holds (k0,k1) in the two
//                                      fp16 halves, (d & 0x00F000F0) holds (k2,k3),
//                                      and the same on d >> 8 gives (k4,k5),(k6,k7).
//
//   Scales: [NT][ST][16][SPS] of fp16 (or fp32 when the caller's fp32 scales
//   are not all fp16-exact), SPS = max(1, 128/bs) scales per row per
//   super-tile; entry i is the scale of block (st*128)/bs + i.
//   The stored scales are the caller's times 2^fold_exp (fold_exp >= 0, per
//   weight, chosen so that 15 * max|scale| * 2^fold_exp <= 65504): where a
//   kernel folds the scale into an fp16 weight operand, (q - zp) * scale *
//   2^fold_exp stays in fp16's normal range however small the scales are, and
//   every consumer multiplies its fp32 result by 2^-fold_exp (exact, so
//   results are those of the unscaled scales wherever the unscaled fp16 fold
//   would not have been subnormal).
//   Zero points (optional): [NT][ST][16] entries of ZB = max(1, SPS/2) bytes,
//   nibble i (low nibble first) belongs to the same block as scale i.
//   Rows >= N, blocks >= kb and k >= kb*bs are stored as zero nibbles, zero
//   scales and zero zero-points, so they contribute exact zeros.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <vector>

#include "mnb.h"
#include "mnb_sched.h"

namespace mnb {

constexpr int kTileRows = 16;     // rows per n-tile (MFMA N dimension)
constexpr int kTileK = 128;       // k per super-tile (4 MFMA K-steps of 32)
constexpr int kTileBytes = 1024;  // packed bytes per tile

struct WeightGeom {
    int32_t N = 0, K = 0, bs = 0;
    int32_t kb = 0, Kpad = 0;     // blocks per row, kb*bs
    int32_t NT = 0, ST = 0;       // n-tiles, super-tiles
    int32_t SPS = 0, ZB = 0;      // scales per row per super-tile, zp bytes per row per super-tile
    int32_t scale_f32 = 0;        // 1: device scales are fp32
    int32_t has_zp = 0;           // 0: implicit zero point 8
    int32_t fold_exp = 0;         // stored scales = scales * 2^fold_exp
};

// Packed weights of 4 GiB or more: the GEMM and K-sliced kernels address the
// scales and zero points with 32-bit offsets, so such weights run only on
// the M <= 16 kernels (64-bit offsets).
inline bool weight_over_4gib(const WeightGeom &g) {
    return (uint64_t)g.NT * (uint64_t)g.ST * (uint64_t)kTileBytes >= ((uint64_t)1 << 32);
}

WeightGeom make_geom(int32_t N, int32_t K, int32_t bs);

// 2^e as a float, -126 <= e <= 127 (exact).
__host__ __device__ inline float pow2f(int e) { return __builtin_bit_cast(float, (uint32_t)(e + 127) << 23); }

// The largest e in [0, 100] with 15 * max_abs_scale * 2^e <= 65504 (0 for a
// zero, infinite or NaN maximum).
int32_t fold_exponent(double max_abs_scale);

}  // namespace mnb

struct mnb_context {
    int32_t device = 0;
    hipStream_t stream = nullptr;
    int32_t cu_count = 0;
    int64_t live_weights = 0;
    // staging buffers for host-memory calls and for x conversion (grown on demand)
    void *stage_raw = nullptr;
    size_t stage_raw_cap = 0;
    void *stage_x = nullptr;
    size_t stage_x_cap = 0;
    void *stage_y = nullptr;
    size_t stage_y_cap = 0;
    // stream-K GEMM: fp32 partial tiles of split tiles
    void *sk_ws = nullptr;
    size_t sk_ws_cap = 0;
    // device address of the fixed scratch array of mnb_matmul_noalloc on this
    // context's device (shared by every context on the device)
    void *scratch = nullptr;
    mnb_device_info info{};
};

struct mnb_weight {
    mnb_context *ctx = nullptr;
    mnb::WeightGeom g;
    void *q_t = nullptr;    // tiled packed nibbles
    void *s_t = nullptr;    // tiled scales
    void *zp_t = nullptr;   // tiled zero points (nullptr when implicit 8)
    int64_t bytes = 0;
};

namespace mnb {

// Makes `dev` the current device for the guard's lifetime.
struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

// Device address of mnb_matmul_noalloc's fixed scratch array on `device`
// (which must be current), looked up once per device (mnb_noalloc.hip).
hipError_t noalloc_scratch(int device, void **out);

// Kernel launchers (defined in the .hip files).  All take device pointers and
// enqueue on `stream`; they return the launch status.

// Records `message` as this thread's mnb_last_error() text and returns `code`.
int32_t report(int32_t code, const char *message);

// natural layout (device copies of the caller's tensors) -> tiled layout
hipError_t launch_repack(const WeightGeom &g, const uint8_t *q_nat, const void *s_nat, const uint8_t *zp_flat,
                         void *q_t, void *s_t, void *zp_t, hipStream_t stream);

// Copies the N_src rows of one tiled weight into rows [row0, row0 + N_src) of
// another with the same K and block size (row fusion).  dst must be zero
// beforehand.  Scales widen fp16 -> fp32 when dst keeps fp32 scales and are
// multiplied by 2^(dst fold_exp - src fold_exp) (dst's exponent is at most
// src's, so the stored value only moves toward the caller's); a source
// without zero points writes zero point 8 for its blocks < kb.
hipError_t launch_copy_rows(const WeightGeom &src_g, const void *src_q, const void *src_s, const void *src_zp,
                            const WeightGeom &dst_g, void *dst_q, void *dst_s, void *dst_zp, int32_t row0,
                            hipStream_t stream);

// s[i] *= factor for the n tiled fp32 scales of a weight (a power of two).
hipError_t launch_scale_f32(float *s, size_t n, float factor, hipStream_t stream);

// data[N, K] (f32 or f16, row stride K, K a multiple of g.bs, g.bs in
// {16, 32, 64, 128}) -> tiled weight with fp32 scales and zero points: the
// reference's per-block min/max uint4 quantizer.
hipError_t launch_quantize(const WeightGeom &g, const void *data, int32_t data_type, void *q_t, float *s_t,
                           uint8_t *zp_t, hipStream_t stream);

// tiled weight -> q [N, Kpad/2] natural packing, fp32 scales [N*kb], one zero
// point per block [N*kb] (8 where the weight has the implicit zero point)
hipError_t launch_unpack(const mnb_weight *w, uint8_t *q_nat, float *s_nat, uint8_t *zp_blocks, hipStream_t stream);

// x[M, K] (f16 or f32, row stride K) -> fp16 [M, ldx] with zeros in k in [K, ldx)
hipError_t launch_stage_x(const void *x, int32_t x_type, int32_t M, int32_t K, int32_t ldx, _Float16 *out,
                          hipStream_t stream);

// out[N, K] = dequantized weight (f32 or f16)
hipError_t launch_dequant(const mnb_weight *w, void *out, int32_t out_type, hipStream_t stream);

// y[M, N] (=|+=) x[M, kx] W^T; x fp16 with row stride ldx (multiple of 8,
// 16-byte aligned), k >= kx contributes zero (kx = K rounded up to 8, the
// x values in [K, kx) must be zero).
struct MatmulArgs {
    const _Float16 *x;
    int32_t ldx, kx, M;
    void *y;
    int32_t y_type;
    int32_t accumulate;
};
hipError_t launch_gemv(const mnb_weight *w, const MatmulArgs &a, int32_t cu_count, hipStream_t stream);

// Kernel parameters of one skinny (M <= 16) product.
struct GemvParams {
    const void *q_t;
    const void *s_t;
    const uint8_t *zp_t;
    const _Float16 *x;
    int32_t ldx, kx, M, N, ST;
    void *y;
    int32_t y_f16, accumulate;
    float unfold;     // 2^-fold_exp of the weight
};

// One item of a group launch (device-resident array).
struct GroupItem {
    GemvParams p;
    int32_t first_wg;   // first workgroup of this item in the group grid
    int32_t pad;
};

// A recorded group of independent skinny products (all items share the
// kernel variant: scale type, zero points, scales per super-tile, M == 1 or not).
struct GemvGroupPlan {
    void *items = nullptr;     // device GroupItem[count]
    void *wg_item = nullptr;   // device uint16_t[total_wgs]: item of each workgroup (M > 1)
    int32_t count = 0, total_wgs = 0, waves = 0;
    int32_t scale_f32 = 0, has_zp = 0, sps = 0, m1 = 0;
    int32_t max_m = 0;         // largest M of the items (M > 1: x row groups to load)
    // the persistent streaming kernel with this many x rows per job (1: M == 1
    // groups; 2 to 4: the largest M of groups with 2 <= M <= 4), 0: the GEMV
    // group kernel
    int32_t stream_rows = 0;
    // persistent streaming schedule
    void *units = nullptr;       // device uint32_t[U]: (item << 16) | n-tile, grouped by wave
    void *wave_begin = nullptr;  // device int32_t[2 * waves + 1]: per wave its first unit and 4-super-tile job count, then the end
    int32_t stream_wgs = 0;
};
hipError_t launch_gemv_group(const GemvGroupPlan &g, hipStream_t stream);
hipError_t launch_gemv_stream(const GemvGroupPlan &g, hipStream_t stream);
int stream_kernel_waves_per_cu(int scale_f32, int has_zp, int sps, int rows);
constexpr int kStreamWavesPerBlock = 4;

// A recorded group of independent products with M > 16 (all items share the
// kernel variant): one launch over all their iterations, in stream-K order
// (seq == nullptr) or in a tile list built at record time.
struct GemmGroupPlan {
    void *items = nullptr;          // device SkItem[count]
    void *seq = nullptr;            // device SkTile[tiles] (tile-list order)
    void *wg = nullptr;             // device SkRange[G + 1] (tile-list order)
    std::vector<SkItem> host;       // host copy
    int32_t count = 0, G = 0;
    int32_t ntw = kGemmNTW;         // n-tiles per wave (kGemmWideNTW: tile-list order only)
    int32_t fm = kGemmFM;           // 32-row fragments per tile (kGemmSkinnyFM: tile-list order, wide)
    int64_t iters = 0;
    int32_t scale_f32 = 0, has_zp = 0, sps = 0;
    SkSplitList parts{};            // tile list with parts: the cut tiles, summed by the reduce launch (n = 0: none)
};

// Stream-K GEMM (M > 16): G persistent workgroups share the (tile, k-stage)
// iterations; the tiles whose stages span workgroups are written as fp32
// partial tiles into ws (ws_bytes bytes, at least sk_workspace_bytes(G), else
// hipErrorInvalidValue and nothing is launched), which a second kernel on the
// same stream sums in contributor order.
hipError_t launch_gemm_sk(const mnb_weight *w, const MatmulArgs &a, int G, float *ws, size_t ws_bytes,
                          hipStream_t stream);
// One product in tile-list order with whole tiles of 32 fm rows x 128 ntw
// columns on min(G, tiles) workgroups, the list in closed form (sk_cf_*): no
// table, no split tile, no workspace.  Wide tiles (ntw = kGemmWideNTW) need
// sk_wide_supported.
hipError_t launch_gemm_closed(const mnb_weight *w, const MatmulArgs &a, int ntw, int fm, int G, hipStream_t stream);
SkItem sk_make_item(const mnb_weight *w, const MatmulArgs &a, int32_t ibeg, int ntw = kGemmNTW, int fm = kGemmFM);
hipError_t launch_gemm_group(const GemmGroupPlan &g, float *ws, size_t ws_bytes, hipStream_t stream);

// One product with K sliced over the waves of each workgroup (single
// products, M > 16): workgroup (m-block, n-group) owns 16 mb rows x 16 ntw
// columns of y over the whole K; no split tile, no workspace, no second
// launch.  Rows of x come in chunks of at most 2 GiB (32-bit offsets).
struct KsParams {
    const void *q_t;
    const void *s_t;
    const uint8_t *zp_t;
    const _Float16 *x;
    void *y;
    int32_t ldx, kx, M, N, NT, ST;
    int32_t mblk;                      // m-blocks (the fastest-varying workgroup index)
    int32_t y_f16, accumulate, y_vec;  // y_vec: four-column stores are aligned
    float unfold;                      // 2^-fold_exp of the weight
};
hipError_t launch_gemm_ks(const mnb_weight *w, const MatmulArgs &a, const KsConfig &c, hipStream_t stream);
// How one product (one chunk of at most 2 GiB of x rows, M > 16) runs: the
// K-sliced kernel when its cost model expects it to finish before the GEMM's
// plan, else that plan.
// How one product with M <= 16 runs: for 9 <= M <= 16 the K-sliced kernel
// with 16-row blocks where its cost model expects it to beat the GEMV's by a
// margin, else the GEMV (wgs == 0).
KsPlan ks_skinny_plan(const WeightGeom &g, int32_t M, int32_t cu_count);
struct ProductPlan {
    bool ks;
    KsConfig kc;
    SinglePlan sp;
};
ProductPlan product_plan(const WeightGeom &g, int32_t M, int32_t cu_count);

// Argument checks of a product (the reference's messages); MNB_OK or the
// status, with the message recorded.
int32_t check_matmul(const mnb_context *ctx, const mnb_weight *w, int32_t M, const void *x, int32_t x_type,
                     int64_t x_elems, const void *y, int32_t y_type, int64_t y_elems, uint32_t flags);
// Bytes of staged fp16 x a product needs: 0 when x is 16-byte aligned fp16
// and K is a multiple of 8 (the kernels read it in place), else M rows of K
// rounded up to 8.
size_t stage_x_bytes(const mnb_weight *w, int32_t M, const void *x, int32_t x_type);
// Bytes of GEMM workspace the product of M > 16 rows needs: the largest
// sk_workspace_bytes(G) over the stream-K grids of its row chunks (0 when no
// chunk runs stream-K).
size_t prefill_workspace_bytes(const WeightGeom &g, int32_t M, int32_t cu_count);
// One product on device pointers: x staged into stage_x when stage_x_bytes
// says so, then the GEMV (M <= 16) or the GEMM, whose split tiles use
// sk_ws (ws_bytes bytes, at least sk_workspace_bytes(sk_max_grid(cu_count))).
// Allocates nothing.
hipError_t launch_product(const mnb_weight *w, int cu_count, int32_t M, const void *x, int32_t x_type, void *y,
                          int32_t y_type, bool accumulate, void *stage_x, void *sk_ws, size_t ws_bytes, hipStream_t s);

// largest M handled by the skinny (GEMV-style) kernel
constexpr int kSkinnyMaxM = 16;
// waves per workgroup of the GEMV-style kernel: 16, or 12 for M > 1, whose
// waves each hold a 4 KiB x block in LDS (dynamic LDS stays below 64 KiB;
// the waves loop over further K chunks)
constexpr int kGemvMaxWaves = 16, kGemvMaxWavesRows = 12;
// super-tiles per wave of the GEMV-style kernel for M > 1 (groups and single
// products alike)
constexpr int kGemvRowsSTW = 2;

}  // namespace mnb
