// mnb_api.cpp -- the C ABI of libmnb_hip.so (declared in include/mnb.h).
//
// Host half of the reference's MatMulNBitsKernel
// (directml-windows-bindings/src/main/java/com/aresstack/windirectml/windows/
// MatMulNBitsKernel.java): argument validation with the reference's messages,
// one-time weight residency (prepareInt4Gpu, :1168-1247), the host-array
// call path (matvec :1847-1914, matmulBatch :2145-2263) and the
// device-resident path.  The D3D12 command lists, fences and upload heaps
// of the reference are replaced by one HIP stream per context.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <limits>
#include <string>
#include <vector>

#include "mnb_internal.h"

using mnb::DeviceGuard;
using mnb::WeightGeom;

namespace {

thread_local std::string g_last_error;

int32_t fail(int32_t code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int32_t ok() { return MNB_OK; }

int32_t hip_fail(hipError_t e, const char *op) {
    int32_t code = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? MNB_ERR_OUT_OF_MEMORY
                                                                              : MNB_ERR_DEVICE;
    return fail(code, "MatMulNBitsKernel.%s failed: %s (%s)", op, hipGetErrorString(e), hipGetErrorName(e));
}

// Fault injection for host-side error-path tests: MNB_FAULT_INJECT=alloc makes
// every device allocation of the library fail as out-of-memory.
bool inject_alloc_failure() {
    const char *v = getenv("MNB_FAULT_INJECT");
    return v && strcmp(v, "alloc") == 0;
}

hipError_t dev_alloc(void **p, size_t bytes) {
    *p = nullptr;
    if (inject_alloc_failure()) return hipErrorOutOfMemory;
    if (bytes == 0) bytes = 16;
    return hipMalloc(p, bytes);
}

// grow-only staging buffer
hipError_t ensure(void **buf, size_t *cap, size_t bytes) {
    if (*cap >= bytes && *buf) return hipSuccess;
    if (*buf) {
        hipError_t e = hipFree(*buf);
        *buf = nullptr;
        *cap = 0;
        if (e != hipSuccess) return e;
    }
    size_t want = bytes < 4096 ? 4096 : bytes;
    hipError_t e = dev_alloc(buf, want);
    if (e == hipSuccess) *cap = want;
    return e;
}

// Rows of x per launch of a product: at most 2 GiB of x (32-bit offsets),
// a multiple of 128.
static int64_t prefill_chunk_rows(int32_t ldx) {
    return std::max<int64_t>(128, (((int64_t)1 << 31) / ((int64_t)ldx * 2)) / 128 * 128);
}

// IEEE binary32 -> binary16 bits, round to nearest even.
uint16_t f32_to_f16_bits(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t a = x & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return (uint16_t)(sign | (a == 0x7F800000u ? 0x7C00u : 0x7E00u | ((a >> 13) & 0x3FFu)));
    const int e = (int)(a >> 23) - 127;
    const uint32_t mant = a & 0x7FFFFFu;
    if (e > 15) return (uint16_t)(sign | 0x7C00u);
    if (e >= -14) {
        uint32_t h = ((uint32_t)(e + 15) << 10) | (mant >> 13);
        const uint32_t rem = mant & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
        return (uint16_t)(sign | h);
    }
    if (e < -25) return (uint16_t)sign;
    const uint32_t full = mant | 0x800000u;
    const int shift = (-14 - e) + 13;
    uint32_t h = full >> shift;
    const uint32_t rem = full & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

// IEEE binary16 bits -> binary32 (exact).
float f16_bits_to_f32(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = s;
        } else {   // normalise the subnormal
            int ee = -1;
            do { ++ee; m <<= 1; } while ((m & 0x400u) == 0);
            bits = s | ((uint32_t)(127 - 15 - ee) << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 31) {
        bits = s | 0x7F800000u | (m << 13);
    } else {
        bits = s | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

size_t dtype_size(int32_t t) { return t == MNB_F32 ? 4 : 2; }

}  // namespace

int32_t mnb::fold_exponent(double max_abs_scale) {
    if (!(max_abs_scale > 0.0) || !std::isfinite(max_abs_scale)) return 0;
    int32_t e = 0;
    while (e < 100 && std::ldexp(15.0 * max_abs_scale, e + 1) <= 65504.0) ++e;
    return e;
}

int32_t mnb::report(int32_t code, const char *message) {
    g_last_error = message ? message : "";
    return code;
}

extern "C" {

int32_t mnb_version(void) { return MNB_ABI_VERSION; }

const char *mnb_last_error(void) { return g_last_error.c_str(); }

int32_t mnb_context_create(int32_t device, mnb_context **out) {
    if (!out) return fail(MNB_ERR_INVALID_ARGUMENT, "out must not be null");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0)
        return fail(MNB_ERR_NO_DEVICE, "no HIP device available (%s)", e != hipSuccess ? hipGetErrorString(e) : "0 devices");
    if (device < 0 || device >= count)
        return fail(MNB_ERR_INVALID_ARGUMENT, "device %d out of range [0, %d)", device, count);
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return hip_fail(e, "init");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(MNB_ERR_NO_DEVICE, "device %d is %s; this library is built for gfx950 (MI355X)", device,
                    prop.gcnArchName);
    DeviceGuard guard(device);
    mnb_context *c = new mnb_context();
    c->device = device;
    c->cu_count = prop.multiProcessorCount;
    e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete c;
        return hip_fail(e, "init");
    }
    // the stream-K GEMM's partial-tile workspace (for the largest grid) is
    // allocated here, so products on device pointers allocate nothing and can
    // be captured into a HIP graph from the first call
    e = ensure(&c->sk_ws, &c->sk_ws_cap, mnb::sk_workspace_bytes(mnb::sk_max_grid(c->cu_count)));
    if (e != hipSuccess) {
        (void)hipStreamDestroy(c->stream);
        delete c;
        return hip_fail(e, "init");
    }
    // the fixed scratch array of mnb_matmul_noalloc: its address on this device
    e = mnb::noalloc_scratch(device, &c->scratch);
    if (e != hipSuccess) {
        (void)hipFree(c->sk_ws);
        (void)hipStreamDestroy(c->stream);
        delete c;
        return hip_fail(e, "init");
    }
    mnb_device_info &i = c->info;
    snprintf(i.name, sizeof i.name, "%s", prop.name);
    snprintf(i.arch, sizeof i.arch, "%s", prop.gcnArchName);
    i.compute_units = prop.multiProcessorCount;
    i.clock_khz = prop.clockRate;
    i.memory_clock_khz = prop.memoryClockRate;
    i.memory_bus_width = prop.memoryBusWidth;
    i.total_memory = (int64_t)prop.totalGlobalMem;
    i.l2_bytes = prop.l2CacheSize;
    i.lds_bytes_per_block = (int32_t)prop.sharedMemPerBlock;
    i.wavefront_size = prop.warpSize;
    i.device = device;
    *out = c;
    return ok();
}

int32_t mnb_context_destroy(mnb_context *ctx) {
    if (!ctx) return ok();
    if (ctx->live_weights > 0)
        return fail(MNB_ERR_INVALID_STATE, "context still owns %lld weight(s); destroy them first",
                    (long long)ctx->live_weights);
    DeviceGuard guard(ctx->device);
    hipError_t first = hipSuccess;
    auto note = [&](hipError_t e) { if (first == hipSuccess && e != hipSuccess) first = e; };
    note(hipStreamSynchronize(ctx->stream));
    if (ctx->stage_raw) note(hipFree(ctx->stage_raw));
    if (ctx->stage_x) note(hipFree(ctx->stage_x));
    if (ctx->stage_y) note(hipFree(ctx->stage_y));
    if (ctx->sk_ws) note(hipFree(ctx->sk_ws));
    note(hipStreamDestroy(ctx->stream));
    delete ctx;
    if (first != hipSuccess) return hip_fail(first, "close");
    return ok();
}

int32_t mnb_context_info(const mnb_context *ctx, mnb_device_info *out) {
    if (!ctx || !out) return fail(MNB_ERR_INVALID_ARGUMENT, "context and out must not be null");
    *out = ctx->info;
    return ok();
}

int32_t mnb_weight_create(mnb_context *ctx, int32_t N, int32_t K, int32_t block_size, int32_t bits, const uint8_t *q,
                          int64_t q_bytes, const void *scales, int32_t scale_type, int64_t scale_count,
                          const uint8_t *zero_points, int64_t zp_bytes, int32_t zp_layout, uint32_t flags,
                          mnb_weight **out) {
    if (!out) return fail(MNB_ERR_INVALID_ARGUMENT, "out must not be null");
    *out = nullptr;
    if (!ctx) return fail(MNB_ERR_INVALID_STATE, "Kernel not prepared: no context");
    if (bits != 4) return fail(MNB_ERR_UNSUPPORTED, "bits=%d: only 4-bit MatMulNBits is supported", bits);
    if (N < 1 || K < 1) return fail(MNB_ERR_INVALID_ARGUMENT, "N=%d and K=%d must be positive", N, K);
    if (!is_pow2(block_size) || block_size < 16 || block_size > 4096)
        return fail(MNB_ERR_INVALID_ARGUMENT, "block_size=%d must be a power of two in [16, 4096]", block_size);
    if (flags != 0) return fail(MNB_ERR_INVALID_ARGUMENT, "unknown flags 0x%x", flags);
    if (!q || !scales) return fail(MNB_ERR_INVALID_ARGUMENT, "qWeight and scales must not be null");
    if (scale_type != MNB_F16 && scale_type != MNB_F32)
        return fail(MNB_ERR_INVALID_ARGUMENT, "scale_type=%d must be MNB_F16 or MNB_F32", scale_type);
    WeightGeom g = mnb::make_geom(N, K, block_size);
    const int64_t blocks = (int64_t)N * g.kb;
    const int64_t need_q = (int64_t)N * g.Kpad / 2;
    if (q_bytes < need_q)
        return fail(MNB_ERR_INVALID_ARGUMENT, "qWeight too short: %lld bytes < N*kb*blockSize/2 = %lld",
                    (long long)q_bytes, (long long)need_q);
    if (scale_count < blocks)
        return fail(MNB_ERR_INVALID_ARGUMENT, "scales too short: %lld < N*kb = %lld", (long long)scale_count,
                    (long long)blocks);

    // zero points -> flat nibble stream (Qwen2Weights.java:1023-1112)
    std::vector<uint8_t> zp_flat;
    if (zp_layout == MNB_ZP_NONE) {
        if (zero_points) return fail(MNB_ERR_INVALID_ARGUMENT, "zero_points given with MNB_ZP_NONE");
    } else if (zp_layout == MNB_ZP_FLAT || zp_layout == MNB_ZP_ROW_PADDED) {
        if (!zero_points) return fail(MNB_ERR_INVALID_ARGUMENT, "zero_points must not be null for this layout");
        const int64_t flat_bytes = (blocks + 1) / 2;
        zp_flat.assign((size_t)flat_bytes, 0);
        if (zp_layout == MNB_ZP_FLAT) {
            if (zp_bytes < flat_bytes)
                return fail(MNB_ERR_INVALID_ARGUMENT, "zero points truncated: %lld bytes, expected %lld",
                            (long long)zp_bytes, (long long)flat_bytes);
            memcpy(zp_flat.data(), zero_points, (size_t)flat_bytes);
        } else {
            const int64_t row_bytes = (g.kb + 1) / 2;
            if (zp_bytes < (int64_t)N * row_bytes)
                return fail(MNB_ERR_INVALID_ARGUMENT, "zero points truncated: %lld bytes, expected %lld",
                            (long long)zp_bytes, (long long)N * row_bytes);
            for (int64_t n = 0; n < N; ++n)
                for (int64_t b = 0; b < g.kb; ++b) {
                    const int64_t src = n * row_bytes * 2 + b;
                    const uint8_t v = (zero_points[src / 2] >> (4 * (src & 1))) & 0xF;
                    const int64_t dst = n * g.kb + b;
                    zp_flat[(size_t)(dst / 2)] |= (uint8_t)(v << (4 * (dst & 1)));
                }
        }
        g.has_zp = 1;
    } else {
        return fail(MNB_ERR_INVALID_ARGUMENT, "zp_layout=%d is not a known layout", zp_layout);
    }

    // scales: keep fp16 unless an fp32 value is not exactly representable
    std::vector<uint16_t> s16;
    const void *s_src = scales;
    size_t s_elem = 2;
    if (scale_type == MNB_F32) {
        const float *sf = (const float *)scales;
        bool exact = true;
        s16.resize((size_t)blocks);
        for (int64_t i = 0; i < blocks; ++i) {
            const uint16_t h = f32_to_f16_bits(sf[i]);
            const float back = f16_bits_to_f32(h);
            if (memcmp(&back, &sf[i], 4) != 0) { exact = false; break; }
            s16[(size_t)i] = h;
        }
        if (exact) {
            s_src = s16.data();
        } else {
            g.scale_f32 = 1;
            s_elem = 4;
            s16.clear();
        }
    }
    // the power of two the device copy of the scales carries (see mnb_internal.h)
    double max_abs_scale = 0.0;
    for (int64_t i = 0; i < blocks; ++i) {
        const double v = scale_type == MNB_F32 ? (double)((const float *)scales)[i]
                                               : (double)f16_bits_to_f32(((const uint16_t *)scales)[i]);
        if (std::fabs(v) > max_abs_scale || std::isnan(v)) max_abs_scale = std::isnan(v) ? NAN : std::fabs(v);
        if (std::isnan(max_abs_scale)) break;
    }
    g.fold_exp = mnb::fold_exponent(max_abs_scale);

    DeviceGuard guard(ctx->device);
    mnb_weight *w = new mnb_weight();
    w->ctx = ctx;
    w->g = g;
    const size_t tiles = (size_t)g.NT * g.ST;
    const size_t q_t_bytes = tiles * mnb::kTileBytes;
    const size_t s_t_bytes = tiles * mnb::kTileRows * g.SPS * s_elem;
    const size_t z_t_bytes = g.has_zp ? tiles * mnb::kTileRows * g.ZB : 0;
    void *q_nat = nullptr, *s_nat = nullptr, *z_nat = nullptr;
    hipError_t e = hipSuccess;
    auto cleanup_tmp = [&]() {
        if (q_nat) (void)hipFree(q_nat);
        if (s_nat) (void)hipFree(s_nat);
        if (z_nat) (void)hipFree(z_nat);
    };
    auto cleanup_all = [&]() {
        cleanup_tmp();
        if (w->q_t) (void)hipFree(w->q_t);
        if (w->s_t) (void)hipFree(w->s_t);
        if (w->zp_t) (void)hipFree(w->zp_t);
        delete w;
    };
    if ((e = dev_alloc(&w->q_t, q_t_bytes)) != hipSuccess ||
        (e = dev_alloc(&w->s_t, s_t_bytes)) != hipSuccess ||
        (g.has_zp && (e = dev_alloc(&w->zp_t, z_t_bytes)) != hipSuccess) ||
        (e = dev_alloc(&q_nat, (size_t)need_q)) != hipSuccess ||
        (e = dev_alloc(&s_nat, (size_t)blocks * s_elem)) != hipSuccess ||
        (g.has_zp && (e = dev_alloc(&z_nat, zp_flat.size())) != hipSuccess)) {
        cleanup_all();
        return hip_fail(e, "prepare");
    }
    if ((e = hipMemcpyAsync(q_nat, q, (size_t)need_q, hipMemcpyHostToDevice, ctx->stream)) != hipSuccess ||
        (e = hipMemcpyAsync(s_nat, s_src, (size_t)blocks * s_elem, hipMemcpyHostToDevice, ctx->stream)) != hipSuccess ||
        (g.has_zp && (e = hipMemcpyAsync(z_nat, zp_flat.data(), zp_flat.size(), hipMemcpyHostToDevice, ctx->stream)) != hipSuccess) ||
        (e = mnb::launch_repack(g, (const uint8_t *)q_nat, s_nat, (const uint8_t *)z_nat, w->q_t, w->s_t, w->zp_t,
                                ctx->stream)) != hipSuccess ||
        (e = hipStreamSynchronize(ctx->stream)) != hipSuccess) {
        cleanup_all();
        return hip_fail(e, "prepare");
    }
    cleanup_tmp();
    w->bytes = (int64_t)(q_t_bytes + s_t_bytes + z_t_bytes);
    ctx->live_weights++;
    *out = w;
    return ok();
}

int32_t mnb_weight_fuse_rows(mnb_context *ctx, const mnb_weight *const *parts, int32_t count, mnb_weight **out) {
    if (!out) return fail(MNB_ERR_INVALID_ARGUMENT, "out must not be null");
    *out = nullptr;
    if (!ctx) return fail(MNB_ERR_INVALID_STATE, "Kernel not prepared: no context");
    if (!parts || count < 1) return fail(MNB_ERR_INVALID_ARGUMENT, "count=%d: at least one part is needed", count);
    int64_t rows = 0;
    bool any_f32 = false, any_zp = false;
    for (int32_t i = 0; i < count; ++i) {
        const mnb_weight *p = parts[i];
        if (!p) return fail(MNB_ERR_INVALID_STATE, "Kernel not prepared: part %d", i);
        if (p->ctx != ctx) return fail(MNB_ERR_INVALID_ARGUMENT, "part %d belongs to another context", i);
        if (p->g.K != parts[0]->g.K || p->g.bs != parts[0]->g.bs)
            return fail(MNB_ERR_INVALID_ARGUMENT, "part %d has K=%d blockSize=%d but expected K=%d blockSize=%d", i,
                        p->g.K, p->g.bs, parts[0]->g.K, parts[0]->g.bs);
        rows += p->g.N;
        any_f32 |= p->g.scale_f32 != 0;
        any_zp |= p->g.has_zp != 0;
    }
    if (rows > std::numeric_limits<int32_t>::max())
        return fail(MNB_ERR_INVALID_ARGUMENT, "fused N=%lld exceeds the 32-bit row count", (long long)rows);
    WeightGeom g = mnb::make_geom((int32_t)rows, parts[0]->g.K, parts[0]->g.bs);
    g.scale_f32 = any_f32 ? 1 : 0;
    g.has_zp = any_zp ? 1 : 0;
    // the smallest exponent of the parts: every part's stored scales move
    // toward the caller's values, so none can overflow
    g.fold_exp = parts[0]->g.fold_exp;
    for (int32_t i = 1; i < count; ++i) g.fold_exp = std::min(g.fold_exp, parts[i]->g.fold_exp);

    DeviceGuard guard(ctx->device);
    mnb_weight *w = new mnb_weight();
    w->ctx = ctx;
    w->g = g;
    const size_t tiles = (size_t)g.NT * g.ST;
    const size_t q_t_bytes = tiles * mnb::kTileBytes;
    const size_t s_t_bytes = tiles * mnb::kTileRows * g.SPS * (g.scale_f32 ? 4 : 2);
    const size_t z_t_bytes = g.has_zp ? tiles * mnb::kTileRows * g.ZB : 0;
    hipError_t e = hipSuccess;
    if ((e = dev_alloc(&w->q_t, q_t_bytes)) != hipSuccess || (e = dev_alloc(&w->s_t, s_t_bytes)) != hipSuccess ||
        (g.has_zp && (e = dev_alloc(&w->zp_t, z_t_bytes)) != hipSuccess) ||
        (e = hipMemsetAsync(w->q_t, 0, q_t_bytes, ctx->stream)) != hipSuccess ||
        (e = hipMemsetAsync(w->s_t, 0, s_t_bytes, ctx->stream)) != hipSuccess ||
        (g.has_zp && (e = hipMemsetAsync(w->zp_t, 0, z_t_bytes, ctx->stream)) != hipSuccess)) {
        if (w->q_t) (void)hipFree(w->q_t);
        if (w->s_t) (void)hipFree(w->s_t);
        if (w->zp_t) (void)hipFree(w->zp_t);
        delete w;
        return hip_fail(e, "prepare");
    }
    int32_t row0 = 0;
    for (int32_t i = 0; i < count && e == hipSuccess; ++i) {
        const mnb_weight *p = parts[i];
        e = mnb::launch_copy_rows(p->g, p->q_t, p->s_t, p->zp_t, g, w->q_t, w->s_t, w->zp_t, row0, ctx->stream);
        row0 += p->g.N;
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        (void)hipFree(w->q_t);
        (void)hipFree(w->s_t);
        if (w->zp_t) (void)hipFree(w->zp_t);
        delete w;
        return hip_fail(e, "prepare");
    }
    w->bytes = (int64_t)(q_t_bytes + s_t_bytes + z_t_bytes);
    ctx->live_weights++;
    *out = w;
    return ok();
}

int32_t mnb_weight_quantize(mnb_context *ctx, const void *data, int32_t data_type, int32_t rows, int32_t cols,
                            int32_t block_size, uint32_t flags, mnb_weight **out) {
    if (!out) return fail(MNB_ERR_INVALID_ARGUMENT, "out must not be null");
    *out = nullptr;
    if (!ctx) return fail(MNB_ERR_INVALID_STATE, "Kernel not prepared: no context");
    if (flags & ~MNB_HOST_MEMORY) return fail(MNB_ERR_INVALID_ARGUMENT, "unknown flags 0x%x", flags);
    if (!data) return fail(MNB_ERR_INVALID_ARGUMENT, "data must not be null");
    if (data_type != MNB_F16 && data_type != MNB_F32)
        return fail(MNB_ERR_INVALID_ARGUMENT, "data_type=%d must be MNB_F16 or MNB_F32", data_type);
    if (rows < 1 || cols < 1) return fail(MNB_ERR_INVALID_ARGUMENT, "rows=%d and cols=%d must be positive", rows, cols);
    if (block_size == 0) {  // chooseTiedLmHeadBlockSize (Qwen2Weights.java:1339-1346)
        for (int c : {128, 64, 32, 16})
            if (cols % c == 0) {
                block_size = c;
                break;
            }
        if (block_size == 0)
            return fail(MNB_ERR_INVALID_ARGUMENT, "Cannot runtime-quantize: hidden size %d is not block-aligned", cols);
    }
    if (block_size != 16 && block_size != 32 && block_size != 64 && block_size != 128)
        return fail(MNB_ERR_INVALID_ARGUMENT, "block_size=%d must be 16, 32, 64 or 128", block_size);
    if (cols % block_size)
        return fail(MNB_ERR_INVALID_ARGUMENT, "cols=%d is not a multiple of block_size=%d", cols, block_size);
    if (!(flags & MNB_HOST_MEMORY) && ((uintptr_t)data & 15))
        return fail(MNB_ERR_INVALID_ARGUMENT, "device data must be 16-byte aligned");
    WeightGeom g = mnb::make_geom(rows, cols, block_size);
    g.scale_f32 = 1;
    g.has_zp = 1;

    DeviceGuard guard(ctx->device);
    const size_t data_bytes = (size_t)rows * cols * dtype_size(data_type);
    void *staged = nullptr;
    hipError_t e = hipSuccess;
    if (flags & MNB_HOST_MEMORY) {
        if ((e = dev_alloc(&staged, data_bytes)) != hipSuccess) return hip_fail(e, "prepare");
        if ((e = hipMemcpyAsync(staged, data, data_bytes, hipMemcpyHostToDevice, ctx->stream)) != hipSuccess) {
            (void)hipFree(staged);
            return hip_fail(e, "prepare");
        }
    }
    mnb_weight *w = new mnb_weight();
    w->ctx = ctx;
    w->g = g;
    const size_t tiles = (size_t)g.NT * g.ST;
    const size_t q_t_bytes = tiles * mnb::kTileBytes;
    const size_t s_t_bytes = tiles * mnb::kTileRows * g.SPS * 4;
    const size_t z_t_bytes = tiles * mnb::kTileRows * g.ZB;
    if ((e = dev_alloc(&w->q_t, q_t_bytes)) != hipSuccess || (e = dev_alloc(&w->s_t, s_t_bytes)) != hipSuccess ||
        (e = dev_alloc(&w->zp_t, z_t_bytes)) != hipSuccess ||
        (e = mnb::launch_quantize(g, staged ? staged : data, data_type, w->q_t, (float *)w->s_t,
                                  (uint8_t *)w->zp_t, ctx->stream)) != hipSuccess ||
        (e = hipStreamSynchronize(ctx->stream)) != hipSuccess) {
        if (staged) (void)hipFree(staged);
        if (w->q_t) (void)hipFree(w->q_t);
        if (w->s_t) (void)hipFree(w->s_t);
        if (w->zp_t) (void)hipFree(w->zp_t);
        delete w;
        return hip_fail(e, "prepare");
    }
    if (staged) (void)hipFree(staged);
    // the scales' power of two (see mnb_internal.h), from the quantized scales
    {
        std::vector<float> sh(s_t_bytes / 4);
        if ((e = hipMemcpy(sh.data(), w->s_t, s_t_bytes, hipMemcpyDeviceToHost)) == hipSuccess) {
            double max_abs_scale = 0.0;
            for (float v : sh) max_abs_scale = std::max(max_abs_scale, (double)std::fabs(v));
            w->g.fold_exp = mnb::fold_exponent(max_abs_scale);
            if (w->g.fold_exp != 0 &&
                (e = mnb::launch_scale_f32((float *)w->s_t, sh.size(), mnb::pow2f(w->g.fold_exp), ctx->stream)) ==
                    hipSuccess)
                e = hipStreamSynchronize(ctx->stream);
        }
        if (e != hipSuccess) {
            (void)hipFree(w->q_t);
            (void)hipFree(w->s_t);
            (void)hipFree(w->zp_t);
            delete w;
            return hip_fail(e, "prepare");
        }
    }
    w->bytes = (int64_t)(q_t_bytes + s_t_bytes + z_t_bytes);
    ctx->live_weights++;
    *out = w;
    return ok();
}

int32_t mnb_weight_read(mnb_context *ctx, const mnb_weight *w, uint8_t *q, int64_t q_cap, float *scales,
                        int64_t scale_cap, uint8_t *zero_points, int64_t zp_cap) {
    if (!ctx || !w) return fail(MNB_ERR_INVALID_STATE, "Kernel not prepared");
    if (w->ctx != ctx) return fail(MNB_ERR_INVALID_ARGUMENT, "weight belongs to another context");
    const WeightGeom &g = w->g;
    const int64_t blocks = (int64_t)g.N * g.kb, q_bytes = (int64_t)g.N * g.Kpad / 2, zp_bytes = (blocks + 1) / 2;
    if (!q || !scales || !zero_points) return fail(MNB_ERR_INVALID_ARGUMENT, "q, scales and zero_points must not be null");
    if (q_cap < q_bytes || scale_cap < blocks || zp_cap < zp_bytes)
        return fail(MNB_ERR_INVALID_ARGUMENT, "buffers too small: need q %lld bytes, %lld scales, %lld zero-point bytes",
                    (long long)q_bytes, (long long)blocks, (long long)zp_bytes);
    DeviceGuard guard(ctx->device);
    void *dq = nullptr, *ds = nullptr, *dz = nullptr;
    hipError_t e = hipSuccess;
    std::vector<uint8_t> zb((size_t)blocks);
    if ((e = dev_alloc(&dq, (size_t)q_bytes)) == hipSuccess && (e = dev_alloc(&ds, (size_t)blocks * 4)) == hipSuccess &&
        (e = dev_alloc(&dz, (size_t)blocks)) == hipSuccess &&
        (e = mnb::launch_unpack(w, (uint8_t *)dq, (float *)ds, (uint8_t *)dz, ctx->stream)) == hipSuccess &&
        (e = hipMemcpyAsync(q, dq, (size_t)q_bytes, hipMemcpyDeviceToHost, ctx->stream)) == hipSuccess &&
        (e = hipMemcpyAsync(scales, ds, (size_t)blocks * 4, hipMemcpyDeviceToHost, ctx->stream)) == hipSuccess &&
        (e = hipMemcpyAsync(zb.data(), dz, (size_t)blocks, hipMemcpyDeviceToHost, ctx->stream)) == hipSuccess)
        e = hipStreamSynchronize(ctx->stream);
    if (dq) (void)hipFree(dq);
    if (ds) (void)hipFree(ds);
    if (dz) (void)hipFree(dz);
    if (e != hipSuccess) return hip_fail(e, "read");
    if (!g.has_zp) {  // createDefaultZeroPoints: every byte 0x88, the unused last nibble included
        memset(zero_points, 0x88, (size_t)zp_bytes);
        return ok();
    }
    memset(zero_points, 0, (size_t)zp_bytes);
    for (int64_t i = 0; i < blocks; ++i) zero_points[i / 2] |= (uint8_t)((zb[(size_t)i] & 0xF) << (4 * (i & 1)));
    return ok();
}

int32_t mnb_weight_destroy(mnb_weight *w) {
    if (!w) return ok();
    DeviceGuard guard(w->ctx->device);
    hipError_t first = hipStreamSynchronize(w->ctx->stream);
    hipError_t e;
    if (w->q_t && (e = hipFree(w->q_t)) != hipSuccess && first == hipSuccess) first = e;
    if (w->s_t && (e = hipFree(w->s_t)) != hipSuccess && first == hipSuccess) first = e;
    if (w->zp_t && (e = hipFree(w->zp_t)) != hipSuccess && first == hipSuccess) first = e;
    w->ctx->live_weights--;
    delete w;
    if (first != hipSuccess) return hip_fail(first, "close");
    return ok();
}

int32_t mnb_weight_shape(const mnb_weight *w, int32_t *N, int32_t *K, int32_t *block_size) {
    if (!w) return fail(MNB_ERR_INVALID_STATE, "Kernel not prepared");
    if (N) *N = w->g.N;
    if (K) *K = w->g.K;
    if (block_size) *block_size = w->g.bs;
    return ok();
}

int64_t mnb_weight_device_bytes(const mnb_weight *w) { return w ? w->bytes : 0; }

int32_t mnb_supports_batch(const mnb_weight *w) { return w ? 1 : 0; }

int32_t mnb_matmul_plan(const mnb_context *ctx, const mnb_weight *w, int32_t M, mnb_plan_info *out) {
    if (!ctx || !w) return fail(MNB_ERR_INVALID_STATE, "Kernel not prepared");
    if (w->ctx != ctx) return fail(MNB_ERR_INVALID_ARGUMENT, "weight belongs to another context");
    if (!out) return fail(MNB_ERR_INVALID_ARGUMENT, "out must not be null");
    if (M < 1 || M > mnb_max_batch_rows()) return fail(MNB_ERR_INVALID_ARGUMENT, "M out of range [1, %d]: %d", mnb_max_batch_rows(), M);
    *out = mnb_plan_info{};
    const WeightGeom &g = w->g;
    if (M > mnb::kSkinnyMaxM && mnb::weight_over_4gib(g))
        return fail(MNB_ERR_UNSUPPORTED, "packed weights of 4 GiB or more run only with M <= 16 (M=%d)", M);
    if (M <= mnb::kSkinnyMaxM) {
        const mnb::KsPlan kp = mnb::ks_skinny_plan(g, M, ctx->cu_count);
        if (kp.wgs > 0) {
            out->kernel = MNB_KERNEL_KSLICE;
            out->order = MNB_ORDER_NONE;
            out->tile_rows = 16 * kp.c.mb;
            out->tile_cols = 16 * kp.c.ntw;
            out->workgroups = (int32_t)kp.wgs;
            return ok();
        }
        out->kernel = MNB_KERNEL_GEMV;
        out->tile_cols = mnb::kTileRows;
        out->workgroups = g.NT;
        return ok();
    }
    // the first chunk of x rows (see launch_prefill)
    const int32_t Mc = (int32_t)std::min<int64_t>(M, prefill_chunk_rows((g.K + 7) & ~7));
    const mnb::ProductPlan pp = mnb::product_plan(g, Mc, ctx->cu_count);
    if (pp.ks) {
        out->kernel = MNB_KERNEL_KSLICE;
        out->order = MNB_ORDER_NONE;
        out->tile_rows = 16 * pp.kc.mb;
        out->tile_cols = 16 * pp.kc.ntw;
        out->workgroups = (int32_t)mnb::ks_workgroups(Mc, g.NT, pp.kc);
        return ok();
    }
    const mnb::SinglePlan &p = pp.sp;
    out->kernel = MNB_KERNEL_GEMM;
    out->order = p.closed ? MNB_ORDER_TILE_LIST : MNB_ORDER_STREAM_K;
    out->tile_rows = 32 * p.fm;
    out->tile_cols = 128 * p.ntw;
    out->workgroups = p.closed ? std::min(p.G, mnb::sk_tiles(Mc, g.NT, p.ntw, p.fm)) : p.G;
    return ok();
}

int32_t mnb_max_batch_rows(void) { return std::numeric_limits<int32_t>::max() / 2; }

}  // extern "C"

mnb::ProductPlan mnb::product_plan(const WeightGeom &g, int32_t M, int32_t cu_count) {
    ProductPlan p;
    p.sp = sk_single_plan(M, g.NT, g.ST, g.scale_f32, g.SPS, cu_count);
    const KsPlan k = ks_single_plan(M, g.NT, g.ST, g.scale_f32, g.has_zp, g.SPS, cu_count);
    p.ks = k.wgs > 0 && k.est < p.sp.est;
    p.kc = k.c;
    return p;
}

size_t mnb::prefill_workspace_bytes(const WeightGeom &g, int32_t M, int32_t cu_count) {
    if (M <= kSkinnyMaxM) return 0;
    const int64_t chunk = std::min<int64_t>(M, prefill_chunk_rows((g.K + 7) & ~7));
    size_t need = 0;
    // every chunk but the last has `chunk` rows
    for (const int64_t rows : {chunk, (int64_t)M % chunk}) {
        if (rows <= 0) continue;
        const ProductPlan pp = product_plan(g, (int32_t)rows, cu_count);
        if (!pp.ks && !pp.sp.closed) need = std::max(need, sk_workspace_bytes(pp.sp.G));
    }
    return need;
}

// M > 16: per chunk of rows, the K-sliced kernel or the GEMM (stream-K over
// one persistent workgroup per CU, or a closed-form tile list), whichever the
// cost models expect to finish first.  ws (ws_bytes bytes: the context's
// workspace, allocated with it, or the fixed scratch array of
// mnb_matmul_noalloc) holds the GEMM's partial tiles of split tiles and their
// arrival counters; launch_gemm_sk refuses a grid it does not cover.  The
// kernels address x and the scales with 32-bit byte offsets: rows of x go in
// chunks of at most 2 GiB, and packed weights of 4 GiB or more are refused.
static hipError_t launch_prefill(const mnb_weight *w, int cu_count, const mnb::MatmulArgs &a, float *ws,
                                 size_t ws_bytes, hipStream_t s) {
    const mnb::WeightGeom &g = w->g;
    if ((uint64_t)g.NT * (uint64_t)g.ST * mnb::kTileBytes >= ((uint64_t)1 << 32)) return hipErrorInvalidValue;
    const int chunk = (int)std::min<int64_t>(a.M, prefill_chunk_rows(a.ldx));
    const size_t y_row = (size_t)g.N * (a.y_type == MNB_F16 ? 2 : 4);
    for (int m0 = 0; m0 < a.M; m0 += chunk) {
        mnb::MatmulArgs c = a;
        c.M = std::min(chunk, a.M - m0);
        c.x = a.x + (size_t)m0 * a.ldx;
        c.y = (unsigned char *)a.y + (size_t)m0 * y_row;
        const mnb::ProductPlan pp = mnb::product_plan(g, c.M, cu_count);
        const mnb::SinglePlan &plan = pp.sp;
        const hipError_t e = pp.ks       ? mnb::launch_gemm_ks(w, c, pp.kc, s)
                             : plan.closed ? mnb::launch_gemm_closed(w, c, plan.ntw, plan.fm, plan.G, s)
                                           : mnb::launch_gemm_sk(w, c, plan.G, ws, ws_bytes, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

int32_t mnb::check_matmul(const mnb_context *ctx, const mnb_weight *w, int32_t M, const void *x, int32_t x_type,
                          int64_t x_elems, const void *y, int32_t y_type, int64_t y_elems, uint32_t flags) {
    if (!ctx || !w) return fail(MNB_ERR_INVALID_STATE, "Kernel not prepared");
    if (w->ctx != ctx) return fail(MNB_ERR_INVALID_ARGUMENT, "weight belongs to another context");
    if (flags & ~(MNB_HOST_MEMORY | MNB_ACCUMULATE)) return fail(MNB_ERR_INVALID_ARGUMENT, "unknown flags 0x%x", flags);
    if ((x_type != MNB_F16 && x_type != MNB_F32) || (y_type != MNB_F16 && y_type != MNB_F32))
        return fail(MNB_ERR_INVALID_ARGUMENT, "x_type/y_type must be MNB_F16 or MNB_F32");
    const WeightGeom &g = w->g;
    if (M < 1 || M > mnb_max_batch_rows()) return fail(MNB_ERR_INVALID_ARGUMENT, "M out of range [1, %d]: %d", mnb_max_batch_rows(), M);
    if (!x || !y) return fail(MNB_ERR_INVALID_ARGUMENT, "x and y must not be null");
    const int64_t MK = (int64_t)M * g.K, MN = (int64_t)M * g.N;
    if (M == 1 && (flags & MNB_HOST_MEMORY) && x_elems != g.K)
        return fail(MNB_ERR_INVALID_ARGUMENT, "Input length %lld != K=%d", (long long)x_elems, g.K);
    if (x_elems < MK) return fail(MNB_ERR_INVALID_ARGUMENT, "xBatch too short: %lld < %lld", (long long)x_elems, (long long)MK);
    if (y_elems < MN) return fail(MNB_ERR_INVALID_ARGUMENT, "outBatch too short: %lld < %lld", (long long)y_elems, (long long)MN);
    if (M > mnb::kSkinnyMaxM && mnb::weight_over_4gib(g))
        return fail(MNB_ERR_UNSUPPORTED, "packed weights of 4 GiB or more run only with M <= 16 (M=%d)", M);
    return MNB_OK;
}

size_t mnb::stage_x_bytes(const mnb_weight *w, int32_t M, const void *x, int32_t x_type) {
    const WeightGeom &g = w->g;
    if (x_type == MNB_F16 && (g.K % 8) == 0 && ((uintptr_t)x & 15u) == 0) return 0;
    return (size_t)M * (size_t)((g.K + 7) & ~7) * 2;
}

hipError_t mnb::launch_product(const mnb_weight *w, int cu_count, int32_t M, const void *x, int32_t x_type, void *y,
                               int32_t y_type, bool accumulate, void *stage_x, void *sk_ws, size_t ws_bytes,
                               hipStream_t s) {
    const WeightGeom &g = w->g;
    const int32_t ldx_pad = (g.K + 7) & ~7;
    mnb::MatmulArgs a;
    a.x = (const _Float16 *)x;
    a.ldx = g.K;
    if (stage_x_bytes(w, M, x, x_type) != 0) {
        const hipError_t e = mnb::launch_stage_x(x, x_type, M, g.K, ldx_pad, (_Float16 *)stage_x, s);
        if (e != hipSuccess) return e;
        a.x = (const _Float16 *)stage_x;
        a.ldx = ldx_pad;
    }
    a.kx = ldx_pad;
    a.M = M;
    a.y = y;
    a.y_type = y_type;
    a.accumulate = accumulate ? 1 : 0;
    if (M > mnb::kSkinnyMaxM) return launch_prefill(w, cu_count, a, (float *)sk_ws, ws_bytes, s);
    // M <= 16: the K-sliced kernel where its cost model expects a clear gain
    // over the GEMV (9 <= M <= 16 and wide N)
    const mnb::KsPlan kp = mnb::ks_skinny_plan(g, M, cu_count);
    return kp.wgs > 0 ? mnb::launch_gemm_ks(w, a, kp.c, s) : mnb::launch_gemv(w, a, cu_count, s);
}

extern "C" {

int32_t mnb_matmul(mnb_context *ctx, const mnb_weight *w, int32_t M, const void *x, int32_t x_type, int64_t x_elems,
                   void *y, int32_t y_type, int64_t y_elems, uint32_t flags, void *stream) {
    const int32_t st = mnb::check_matmul(ctx, w, M, x, x_type, x_elems, y, y_type, y_elems, flags);
    if (st != MNB_OK) return st;
    const WeightGeom &g = w->g;
    const int64_t MK = (int64_t)M * g.K, MN = (int64_t)M * g.N;
    const char *op = M == 1 ? "matvec" : "matmulBatch";
    DeviceGuard guard(ctx->device);
    hipStream_t s = (flags & MNB_HOST_MEMORY) || !stream ? ctx->stream : (hipStream_t)stream;
    const bool host = (flags & MNB_HOST_MEMORY) != 0;
    hipError_t e;

    // host arrays: x goes to a device staging buffer as it is (fp16 rows
    // whose stride is a multiple of 8 land where the kernels read them)
    const void *xd = x;
    if (host) {
        void **buf = mnb::stage_x_bytes(w, M, ctx->stage_x, x_type) == 0 ? &ctx->stage_x : &ctx->stage_raw;
        size_t *cap = buf == &ctx->stage_x ? &ctx->stage_x_cap : &ctx->stage_raw_cap;
        const size_t bytes = (size_t)MK * dtype_size(x_type);
        if ((e = ensure(buf, cap, bytes)) != hipSuccess ||
            (e = hipMemcpyAsync(*buf, x, bytes, hipMemcpyHostToDevice, s)) != hipSuccess)
            return hip_fail(e, op);
        xd = *buf;
    }
    const size_t stage = mnb::stage_x_bytes(w, M, xd, x_type);
    if (stage && (e = ensure(&ctx->stage_x, &ctx->stage_x_cap, stage)) != hipSuccess) return hip_fail(e, op);

    void *yd = y;
    const size_t y_bytes = (size_t)MN * dtype_size(y_type);
    if (host) {
        if ((e = ensure(&ctx->stage_y, &ctx->stage_y_cap, y_bytes)) != hipSuccess) return hip_fail(e, op);
        yd = ctx->stage_y;
        if ((flags & MNB_ACCUMULATE) &&
            (e = hipMemcpyAsync(yd, y, y_bytes, hipMemcpyHostToDevice, s)) != hipSuccess)
            return hip_fail(e, op);
    }

    e = mnb::launch_product(w, ctx->cu_count, M, xd, x_type, yd, y_type, (flags & MNB_ACCUMULATE) != 0, ctx->stage_x,
                            ctx->sk_ws, ctx->sk_ws_cap, s);
    if (e != hipSuccess) return hip_fail(e, op);

    if (host) {
        if ((e = hipMemcpyAsync(y, yd, y_bytes, hipMemcpyDeviceToHost, s)) != hipSuccess ||
            (e = hipStreamSynchronize(s)) != hipSuccess)
            return hip_fail(e, op);
    }
    return ok();
}

int32_t mnb_dequantize(mnb_context *ctx, const mnb_weight *w, void *out, int32_t out_type, int64_t out_elems,
                       uint32_t flags, void *stream) {
    if (!ctx || !w) return fail(MNB_ERR_INVALID_STATE, "Kernel not prepared");
    if (w->ctx != ctx) return fail(MNB_ERR_INVALID_ARGUMENT, "weight belongs to another context");
    if (!out) return fail(MNB_ERR_INVALID_ARGUMENT, "out must not be null");
    if (out_type != MNB_F16 && out_type != MNB_F32) return fail(MNB_ERR_INVALID_ARGUMENT, "out_type must be MNB_F16 or MNB_F32");
    if (flags & ~MNB_HOST_MEMORY) return fail(MNB_ERR_INVALID_ARGUMENT, "unknown flags 0x%x", flags);
    const int64_t NK = (int64_t)w->g.N * w->g.K;
    if (out_elems < NK) return fail(MNB_ERR_INVALID_ARGUMENT, "out too short: %lld < N*K = %lld", (long long)out_elems, (long long)NK);
    DeviceGuard guard(ctx->device);
    const bool host = (flags & MNB_HOST_MEMORY) != 0;
    hipStream_t s = host || !stream ? ctx->stream : (hipStream_t)stream;
    const size_t bytes = (size_t)NK * dtype_size(out_type);
    hipError_t e;
    void *od = out;
    if (host) {
        if ((e = ensure(&ctx->stage_y, &ctx->stage_y_cap, bytes)) != hipSuccess) return hip_fail(e, "dequantizeInt4");
        od = ctx->stage_y;
    }
    if ((e = mnb::launch_dequant(w, od, out_type, s)) != hipSuccess) return hip_fail(e, "dequantizeInt4");
    if (host) {
        if ((e = hipMemcpyAsync(out, od, bytes, hipMemcpyDeviceToHost, s)) != hipSuccess ||
            (e = hipStreamSynchronize(s)) != hipSuccess)
            return hip_fail(e, "dequantizeInt4");
    }
    return ok();
}

}  // extern "C"

struct mnb_group {
    mnb_context *ctx = nullptr;
    mnb::GemvGroupPlan plan;        // items with M <= 16
    bool gemm = false;              // items with M > 16: one stream-K GEMM launch
    mnb::GemmGroupPlan gplan;
};

// Whole tiles per workgroup from which a GEMM group runs in tile-list order.
constexpr int kGemmListTilesPerWg = 4;
// Largest M of a group's items for 32-row tiles, and for 64-row tiles.
constexpr int kGemmSkinnyMaxM = 32, kGemmHalfMaxM = 64;
// Cost of a 64 x 512 stage in 128 x 256 stages: the same MFMA work and the
// same operand bytes (x and weights trade places), rounded up.
constexpr double kGemmHalfStageCost = 1.1;
// Cost of cutting a tile list into parts, in stages of the busiest
// workgroup: the reduce launch (~5 us against ~2.5 us per 64 x 512 stage) and
// the fp32 partial tiles written and read back.  The Qwen2.5-0.5B step at
// M = 64, whose parts take its busiest workgroup from 38 to 35 stages, ran
// 1-3% slower with them on two boxes and 2% faster on a third, so a cut must
// save more than 4 stages.
constexpr int64_t kGemmPartsReduceStages = 4;

// A group of products with M > 16: one launch over one workgroup per CU,
// the items' (tile, stage) iterations in stream-K order or, for many tiles,
// in a tile list.
static int32_t group_create_gemm(mnb_context *ctx, int32_t count, const mnb_group_item *items, mnb_group **out) {
    mnb::GemmGroupPlan plan;
    std::vector<mnb::MatmulArgs> args((size_t)count);
    for (int32_t i = 0; i < count; ++i) {
        const mnb_group_item &it = items[i];
        const WeightGeom &g = it.weight->g;
        if (i == 0) {
            plan.scale_f32 = g.scale_f32;
            plan.has_zp = g.has_zp;
            plan.sps = g.SPS;
        } else if (plan.scale_f32 != g.scale_f32 || plan.has_zp != g.has_zp || plan.sps != g.SPS) {
            return fail(MNB_ERR_UNSUPPORTED, "item %d: a group needs one weight variant and one M class", i);
        }
        if ((int64_t)it.M * g.K * 2 >= ((int64_t)1 << 31) || mnb::weight_over_4gib(g))
            return fail(MNB_ERR_UNSUPPORTED, "item %d: x of 2 GiB or packed weights of 4 GiB or more in a group", i);
        mnb::MatmulArgs &a = args[(size_t)i];
        a.x = (const _Float16 *)it.x;
        a.ldx = g.K;
        a.kx = g.K;
        a.M = it.M;
        a.y = it.y;
        a.y_type = it.y_type;
        a.accumulate = (it.flags & MNB_ACCUMULATE) ? 1 : 0;
    }
    // the items at tile width ntw; false when the launch would have 2^31
    // iterations or more
    int64_t tiles = 0;
    auto build = [&](int ntw, int fm = mnb::kGemmFM) {
        plan.ntw = ntw;
        plan.fm = fm;
        plan.host.resize((size_t)count);
        plan.iters = 0;
        tiles = 0;
        for (int32_t i = 0; i < count; ++i) {
            plan.host[(size_t)i] = mnb::sk_make_item(items[i].weight, args[(size_t)i], (int32_t)plan.iters, ntw, fm);
            plan.iters += (int64_t)plan.host[(size_t)i].T * plan.host[(size_t)i].ST;
            tiles += plan.host[(size_t)i].T;
            if (plan.iters >= ((int64_t)1 << 31)) return false;
        }
        return true;
    };
    if (!build(mnb::kGemmNTW)) return fail(MNB_ERR_INVALID_ARGUMENT, "group too large");
    plan.count = count;
    plan.G = (int32_t)std::min<int64_t>(mnb::sk_max_grid(ctx->cu_count), plan.iters);
    // Tile-list order once every workgroup gets several whole tiles: the
    // workgroups of one XCD then run tiles that share x rows and weight
    // columns side by side, and no tile is split, so the 512-column kernel
    // (half the LDS reads of x per MFMA) can run where the variant has one;
    // fewer tiles keep the stream-K split, which balances any tile count.
    // The width is the one whose busiest workgroup finishes first: a
    // 512-column stage has twice the flops of a 256-column one and costs
    // kGemmWideStageCost of them (a 16-21% gain measured on the Phi-3 groups),
    // but whole tiles balance worse when they are fewer.
    std::vector<mnb::SkTile> seq;
    std::vector<mnb::SkRange> wg;
    const int64_t min_tiles = (int64_t)kGemmListTilesPerWg * plan.G;
    auto busiest = [&](const std::vector<mnb::SkRange> &r) {
        int64_t m = 0;
        for (int32_t g = 0; g < plan.G; ++g) m = std::max<int64_t>(m, r[(size_t)g + 1].iter - r[(size_t)g].iter);
        return m;
    };
    // A tile longer than a workgroup's mean share of the stages sets the
    // busiest workgroup of a tile list (Qwen2.5-0.5B's down tiles at M = 64:
    // 38 stages against a mean of 31).  Where a tile's fp32 partial fits one
    // workspace slot (all but 128 x 512 tiles), the long tiles are cut along
    // K into parts, summed by a reduce launch after the GEMM, when that
    // shortens the busiest workgroup by more than the reduce costs; the
    // parts' partial tiles must fit the context's workspace.
    // Parts of about the mean, a half, a third or a quarter of it are
    // tried (parts near the mean pack unevenly: two of them on one
    // workgroup double it), and the cut whose busiest workgroup finishes
    // first is kept.
    auto try_parts = [&]() {
        plan.parts.n = 0;
        if (seq.empty() || 32 * plan.fm * 128 * plan.ntw > mnb::kSkPartialFloats) return;
        const int64_t mean = (plan.iters + plan.G - 1) / plan.G, b0 = busiest(wg);
        if (b0 <= mean + kGemmPartsReduceStages) return;
        int64_t best = b0 - kGemmPartsReduceStages;
        std::vector<mnb::SkTile> seq_p, seq_best;
        std::vector<mnb::SkRange> wg_p, wg_best;
        mnb::SkSplitList parts;
        for (int d = 1; d <= 4; ++d) {
            const int64_t split = (mean + d - 1) / d;
            if (split < 1 || !mnb::sk_tile_list_parts(plan.host, plan.G, split, seq_p, wg_p, parts) || parts.n == 0)
                continue;
            int n_parts = 0;
            for (int j = 0; j < parts.n; ++j) n_parts = std::max(n_parts, (int)parts.e[j].last + 1);
            if (n_parts > 2 * mnb::sk_max_grid(ctx->cu_count)) continue;
            const int64_t b = busiest(wg_p);
            if (b < best) {
                best = b;
                seq_best.swap(seq_p);
                wg_best.swap(wg_p);
                plan.parts = parts;
            }
        }
        if (plan.parts.n == 0) return;
        seq.swap(seq_best);
        wg.swap(wg_best);
    };
    // Rows of at most 32 (64) per item: 32-row (64-row) tiles of 512 columns
    // (128-row tiles would multiply by up to 8 (2) the MFMA work).
    int32_t max_m = 0;
    for (int32_t i = 0; i < count; ++i) max_m = std::max(max_m, items[i].M);
    const bool wide_ok = mnb::sk_wide_supported(plan.scale_f32, plan.sps);
    // 64-row tiles take half the stages of 128-row tiles at about the same
    // cost each; they need no split, so they run in tile-list order, chosen
    // when the busiest workgroup's stages beat the 128-row plan's average
    // (its best case); leaves the list in seq/wg when chosen
    auto half_wins = [&]() {
        int64_t narrow_iters = 0;
        for (int32_t i = 0; i < count; ++i) {
            const WeightGeom &g = items[i].weight->g;
            narrow_iters += (int64_t)mnb::sk_tiles(items[i].M, g.NT, mnb::kGemmNTW, mnb::kGemmFM) * g.ST;
        }
        mnb::sk_tile_list(plan.host, plan.G, seq, wg);
        try_parts();
        if ((double)busiest(wg) * kGemmHalfStageCost < (double)narrow_iters / plan.G) return true;
        seq.clear();
        wg.clear();
        plan.parts.n = 0;
        return false;
    };
    if (max_m <= kGemmSkinnyMaxM && wide_ok && build(mnb::kGemmWideNTW, mnb::kGemmSkinnyFM) && tiles >= min_tiles) {
        mnb::sk_tile_list(plan.host, plan.G, seq, wg);
        try_parts();
    } else if (max_m <= kGemmHalfMaxM && wide_ok && build(mnb::kGemmWideNTW, mnb::kGemmHalfFM) && tiles >= plan.G &&
               half_wins()) {
        // 64 x 512 tiles in tile-list order
    } else if (!build(mnb::kGemmNTW)) {
        return fail(MNB_ERR_INVALID_ARGUMENT, "group too large");
    } else if (tiles >= min_tiles) {
        mnb::sk_tile_list(plan.host, plan.G, seq, wg);
        if (mnb::sk_wide_supported(plan.scale_f32, plan.sps)) {
            const double narrow = (double)busiest(wg);
            std::vector<mnb::SkTile> seq_w;
            std::vector<mnb::SkRange> wg_w;
            if (build(mnb::kGemmWideNTW) && tiles >= min_tiles) {
                mnb::sk_tile_list(plan.host, plan.G, seq_w, wg_w);
                if ((double)busiest(wg_w) * mnb::kGemmWideStageCost < narrow) {
                    seq.swap(seq_w);
                    wg.swap(wg_w);
                } else {
                    build(mnb::kGemmNTW);
                }
            } else {
                build(mnb::kGemmNTW);
            }
        }
        if (plan.ntw == mnb::kGemmNTW) try_parts();
    }
    DeviceGuard guard(ctx->device);
    hipError_t e;
    if ((e = dev_alloc(&plan.items, plan.host.size() * sizeof(mnb::SkItem))) != hipSuccess ||
        (e = hipMemcpy(plan.items, plan.host.data(), plan.host.size() * sizeof(mnb::SkItem), hipMemcpyHostToDevice)) !=
            hipSuccess ||
        (!seq.empty() &&
         ((e = dev_alloc(&plan.seq, seq.size() * sizeof(mnb::SkTile))) != hipSuccess ||
          (e = dev_alloc(&plan.wg, wg.size() * sizeof(mnb::SkRange))) != hipSuccess ||
          (e = hipMemcpy(plan.seq, seq.data(), seq.size() * sizeof(mnb::SkTile), hipMemcpyHostToDevice)) != hipSuccess ||
          (e = hipMemcpy(plan.wg, wg.data(), wg.size() * sizeof(mnb::SkRange), hipMemcpyHostToDevice)) != hipSuccess))) {
        if (plan.items) (void)hipFree(plan.items);
        if (plan.seq) (void)hipFree(plan.seq);
        if (plan.wg) (void)hipFree(plan.wg);
        return hip_fail(e, "group");
    }
    mnb_group *grp = new mnb_group();
    grp->ctx = ctx;
    grp->gemm = true;
    grp->gplan = std::move(plan);
    ctx->live_weights++;   // a group keeps its context alive like a weight does
    *out = grp;
    return ok();
}

extern "C" {

int32_t mnb_group_create(mnb_context *ctx, int32_t count, const mnb_group_item *items, mnb_group **out) {
    if (!out) return fail(MNB_ERR_INVALID_ARGUMENT, "out must not be null");
    *out = nullptr;
    if (!ctx) return fail(MNB_ERR_INVALID_STATE, "Kernel not prepared: no context");
    if (count < 1 || count > 65535 || !items) return fail(MNB_ERR_INVALID_ARGUMENT, "count=%d must be in [1, 65535]", count);
    std::vector<mnb::GroupItem> host((size_t)count);
    mnb::GemvGroupPlan plan;
    int64_t wgs = 0;
    for (int32_t i = 0; i < count; ++i) {
        const mnb_group_item &it = items[i];
        const mnb_weight *w = it.weight;
        if (!w) return fail(MNB_ERR_INVALID_STATE, "item %d: Kernel not prepared", i);
        if (w->ctx != ctx) return fail(MNB_ERR_INVALID_ARGUMENT, "item %d: weight belongs to another context", i);
        const WeightGeom &g = w->g;
        if (it.M < 1) return fail(MNB_ERR_INVALID_ARGUMENT, "item %d: M=%d must be at least 1", i, it.M);
        if ((it.M > mnb::kSkinnyMaxM) != (items[0].M > mnb::kSkinnyMaxM))
            return fail(MNB_ERR_UNSUPPORTED, "item %d: a group needs one weight variant and one M class", i);
        if (it.x_type != MNB_F16 || (g.K % 8) != 0 || ((uintptr_t)it.x & 15u) || !it.x)
            return fail(MNB_ERR_UNSUPPORTED, "item %d: x must be 16-byte aligned fp16 with K a multiple of 8", i);
        if ((it.y_type != MNB_F16 && it.y_type != MNB_F32) || !it.y)
            return fail(MNB_ERR_INVALID_ARGUMENT, "item %d: y must be fp16 or fp32", i);
        if (it.flags & ~MNB_ACCUMULATE) return fail(MNB_ERR_INVALID_ARGUMENT, "item %d: unknown flags 0x%x", i, it.flags);
        if (it.x_elems < (int64_t)it.M * g.K || it.y_elems < (int64_t)it.M * g.N)
            return fail(MNB_ERR_INVALID_ARGUMENT, "item %d: x or y too short", i);
        const int m1 = it.M == 1;
        if (i == 0) {
            plan.scale_f32 = g.scale_f32;
            plan.has_zp = g.has_zp;
            plan.sps = g.SPS;
            plan.m1 = m1;
        } else if (plan.scale_f32 != g.scale_f32 || plan.has_zp != g.has_zp || plan.sps != g.SPS || plan.m1 != m1) {
            return fail(MNB_ERR_UNSUPPORTED, "item %d: a group needs one weight variant and one M class", i);
        }
        mnb::GemvParams &p = host[(size_t)i].p;
        p.q_t = w->q_t;
        p.s_t = w->s_t;
        p.zp_t = (const uint8_t *)w->zp_t;
        p.x = (const _Float16 *)it.x;
        p.ldx = g.K;
        p.kx = g.K;
        p.M = it.M;
        p.N = g.N;
        p.ST = g.ST;
        p.y = it.y;
        p.y_f16 = it.y_type == MNB_F16;
        p.accumulate = (it.flags & MNB_ACCUMULATE) ? 1 : 0;
        p.unfold = mnb::pow2f(-g.fold_exp);
        host[(size_t)i].first_wg = (int32_t)wgs;
        wgs += g.NT;
        const int stw = m1 ? 4 : mnb::kGemvRowsSTW;
        int waves = (g.ST + stw - 1) / stw;
        waves = std::min(waves, m1 ? mnb::kGemvMaxWaves : mnb::kGemvMaxWavesRows);
        if (waves > plan.waves) plan.waves = waves;
        plan.max_m = std::max(plan.max_m, it.M);
    }
    if (items[0].M > mnb::kSkinnyMaxM) return group_create_gemm(ctx, count, items, out);
    // M == 1, and 2 <= M <= 4 (small-batch decode): the persistent streaming
    // kernel with as many x rows per job as the group's largest M.  Its units
    // code the n-tile in 16 bits, so a group with an item of more than 65536
    // n-tiles (N > 1048576) runs on the GEMV group kernel instead.
    bool stream_ok = true;
    for (int32_t i = 0; i < count; ++i) stream_ok = stream_ok && items[i].weight->g.NT <= 65536;
    plan.stream_rows = !stream_ok ? 0 : plan.m1 ? 1 : plan.max_m <= 4 ? plan.max_m : 0;
    // 4 < M <= 16 with many 32 x 512 tiles: the GEMM's weight stream (x
    // shared by the workgroup's waves in LDS, persistent workgroups) beats one
    // workgroup per n-tile, whose waves each read their own x rows.
    if (plan.stream_rows == 0 && plan.max_m > 4 && mnb::sk_wide_supported(plan.scale_f32, plan.sps)) {
        int64_t skinny_tiles = 0;
        for (int32_t i = 0; i < count; ++i)
            skinny_tiles += mnb::sk_tiles(items[i].M, items[i].weight->g.NT, mnb::kGemmWideNTW, mnb::kGemmSkinnyFM);
        if (skinny_tiles >= (int64_t)kGemmListTilesPerWg * mnb::sk_max_grid(ctx->cu_count))
            return group_create_gemm(ctx, count, items, out);
    }
    if (wgs > std::numeric_limits<int32_t>::max()) return fail(MNB_ERR_INVALID_ARGUMENT, "group too large");
    std::vector<uint16_t> wg_item((size_t)wgs);
    for (int32_t i = 0; i < count; ++i) {
        const int32_t end = i + 1 < count ? host[(size_t)i + 1].first_wg : (int32_t)wgs;
        for (int32_t b = host[(size_t)i].first_wg; b < end; ++b) wg_item[(size_t)b] = (uint16_t)i;
    }
    plan.count = count;
    plan.total_wgs = (int32_t)wgs;
    DeviceGuard guard(ctx->device);

    // static schedule for the persistent streaming kernel (units dealt
    // longest first to the least loaded wave, mnb_sched.cpp)
    std::vector<uint32_t> units;
    std::vector<int32_t> wave_begin;
    if (plan.stream_rows > 0) {
        const int wpc = mnb::stream_kernel_waves_per_cu(plan.scale_f32, plan.has_zp, plan.sps, plan.stream_rows);
        const int64_t total_waves = (int64_t)ctx->cu_count * wpc;
        plan.stream_wgs = (int32_t)(total_waves / mnb::kStreamWavesPerBlock);
        std::vector<int32_t> nt((size_t)count), st((size_t)count);
        for (int32_t i = 0; i < count; ++i) {
            nt[(size_t)i] = items[i].weight->g.NT;
            st[(size_t)i] = items[i].weight->g.ST;
        }
        if (!mnb::stream_schedule(nt, st, (int64_t)plan.stream_wgs * mnb::kStreamWavesPerBlock, units, wave_begin))
            return fail(MNB_ERR_INVALID_ARGUMENT, "group too large");
    }

    hipError_t e;
    auto release = [&]() {
        if (plan.items) (void)hipFree(plan.items);
        if (plan.wg_item) (void)hipFree(plan.wg_item);
        if (plan.units) (void)hipFree(plan.units);
        if (plan.wave_begin) (void)hipFree(plan.wave_begin);
    };
    if ((e = dev_alloc(&plan.items, host.size() * sizeof(mnb::GroupItem))) != hipSuccess ||
        (e = dev_alloc(&plan.wg_item, wg_item.size() * sizeof(uint16_t))) != hipSuccess ||
        (e = hipMemcpy(plan.items, host.data(), host.size() * sizeof(mnb::GroupItem), hipMemcpyHostToDevice)) != hipSuccess ||
        (e = hipMemcpy(plan.wg_item, wg_item.data(), wg_item.size() * sizeof(uint16_t), hipMemcpyHostToDevice)) != hipSuccess ||
        (plan.stream_rows > 0 && ((e = dev_alloc(&plan.units, units.size() * sizeof(uint32_t))) != hipSuccess ||
                     (e = dev_alloc(&plan.wave_begin, wave_begin.size() * sizeof(int32_t))) != hipSuccess ||
                     (e = hipMemcpy(plan.units, units.data(), units.size() * sizeof(uint32_t), hipMemcpyHostToDevice)) != hipSuccess ||
                     (e = hipMemcpy(plan.wave_begin, wave_begin.data(), wave_begin.size() * sizeof(int32_t), hipMemcpyHostToDevice)) != hipSuccess))) {
        release();
        return hip_fail(e, "group");
    }
    mnb_group *grp = new mnb_group();
    grp->ctx = ctx;
    grp->plan = plan;
    ctx->live_weights++;   // a group keeps its context alive like a weight does
    *out = grp;
    return ok();
}

int32_t mnb_group_run(mnb_context *ctx, const mnb_group *group, void *stream) {
    if (!ctx || !group) return fail(MNB_ERR_INVALID_STATE, "Kernel not prepared");
    if (group->ctx != ctx) return fail(MNB_ERR_INVALID_ARGUMENT, "group belongs to another context");
    DeviceGuard guard(ctx->device);
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    if (group->gemm) {
        const hipError_t e = mnb::launch_gemm_group(group->gplan, (float *)ctx->sk_ws, ctx->sk_ws_cap, s);
        if (e != hipSuccess) return hip_fail(e, "matmulBatch");
        return ok();
    }
    hipError_t e = group->plan.stream_rows > 0 ? mnb::launch_gemv_stream(group->plan, s) : mnb::launch_gemv_group(group->plan, s);
    if (e != hipSuccess) return hip_fail(e, "matvec");
    return ok();
}

int32_t mnb_group_plan(const mnb_group *group, mnb_plan_info *out) {
    if (!group || !out) return fail(MNB_ERR_INVALID_ARGUMENT, "group and out must not be null");
    *out = mnb_plan_info{};
    if (group->gemm) {
        const mnb::GemmGroupPlan &g = group->gplan;
        out->kernel = MNB_KERNEL_GEMM;
        out->order = !g.seq ? MNB_ORDER_STREAM_K : g.parts.n > 0 ? MNB_ORDER_TILE_LIST_PARTS : MNB_ORDER_TILE_LIST;
        out->tile_rows = 32 * g.fm;
        out->tile_cols = 128 * g.ntw;
        out->workgroups = g.G;
    } else if (group->plan.stream_rows > 0) {
        out->kernel = MNB_KERNEL_STREAM;
        out->tile_rows = group->plan.stream_rows > 1 ? group->plan.stream_rows : 0;
        out->tile_cols = mnb::kTileRows;
        out->workgroups = group->plan.stream_wgs;
    } else {
        out->kernel = MNB_KERNEL_GEMV_GROUP;
        out->tile_cols = mnb::kTileRows;
        out->workgroups = group->plan.total_wgs;
    }
    return ok();
}

int32_t mnb_group_destroy(mnb_group *group) {
    if (!group) return ok();
    DeviceGuard guard(group->ctx->device);
    hipError_t first = hipStreamSynchronize(group->ctx->stream), e;
    if (group->gplan.items && (e = hipFree(group->gplan.items)) != hipSuccess && first == hipSuccess) first = e;
    if (group->gplan.seq && (e = hipFree(group->gplan.seq)) != hipSuccess && first == hipSuccess) first = e;
    if (group->gplan.wg && (e = hipFree(group->gplan.wg)) != hipSuccess && first == hipSuccess) first = e;
    if (group->plan.items && (e = hipFree(group->plan.items)) != hipSuccess && first == hipSuccess) first = e;
    if (group->plan.wg_item && (e = hipFree(group->plan.wg_item)) != hipSuccess && first == hipSuccess) first = e;
    if (group->plan.units && (e = hipFree(group->plan.units)) != hipSuccess && first == hipSuccess) first = e;
    if (group->plan.wave_begin && (e = hipFree(group->plan.wave_begin)) != hipSuccess && first == hipSuccess) first = e;
    group->ctx->live_weights--;
    delete group;
    if (first != hipSuccess) return hip_fail(first, "close");
    return ok();
}

int32_t mnb_device_alloc(mnb_context *ctx, int64_t bytes, void **out) {
    if (!ctx || !out) return fail(MNB_ERR_INVALID_ARGUMENT, "context and out must not be null");
    if (bytes < 0) return fail(MNB_ERR_INVALID_ARGUMENT, "negative size");
    DeviceGuard guard(ctx->device);
    hipError_t e = dev_alloc(out, (size_t)bytes);
    if (e != hipSuccess) return hip_fail(e, "alloc");
    return ok();
}

int32_t mnb_device_free(mnb_context *ctx, void *ptr) {
    if (!ctx) return fail(MNB_ERR_INVALID_ARGUMENT, "context must not be null");
    if (!ptr) return ok();
    DeviceGuard guard(ctx->device);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess) e = hipFree(ptr);
    if (e != hipSuccess) return hip_fail(e, "free");
    return ok();
}

int32_t mnb_memcpy(mnb_context *ctx, void *dst, const void *src, int64_t bytes, int32_t kind) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(MNB_ERR_INVALID_ARGUMENT, "null argument");
    if (bytes < 0) return fail(MNB_ERR_INVALID_ARGUMENT, "negative size");
    hipMemcpyKind k;
    switch (kind) {
        case MNB_COPY_H2D: k = hipMemcpyHostToDevice; break;
        case MNB_COPY_D2H: k = hipMemcpyDeviceToHost; break;
        case MNB_COPY_D2D: k = hipMemcpyDeviceToDevice; break;
        default: return fail(MNB_ERR_INVALID_ARGUMENT, "unknown copy kind %d", kind);
    }
    DeviceGuard guard(ctx->device);
    hipError_t e = hipMemcpyAsync(dst, src, (size_t)bytes, k, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "copy");
    return ok();
}

int32_t mnb_synchronize(mnb_context *ctx) {
    if (!ctx) return fail(MNB_ERR_INVALID_ARGUMENT, "context must not be null");
    DeviceGuard guard(ctx->device);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "synchronize");
    return ok();
}

}  // extern "C"
