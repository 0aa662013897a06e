// mnb_noalloc.hip -- mnb_matmul_noalloc: the device-pointer product of
// mnb_matmul with its two buffers beyond x and y -- the fp32 partial tiles of
// the stream-K GEMM's split tiles and the fp16 copy of x that the kernels read
// when x is fp32, unaligned or has K % 8 != 0 -- in a fixed device array of
// this file instead of buffers the context allocates and grows.  For callers
// that cannot allocate device memory while they run (HIP graph capture,
// serving loops that forbid allocation).
//
// `scratch` below is a host-side stand-in in host code: its device address is
// looked up with hipGetSymbolAddress once per device (at mnb_context_create,
// with the device current) and only that address is handed to kernels.  Every
// call on one device shares the array, and nothing in it has to start at zero
// (each partial tile and each staged row is written in full before it is
// read), so calls that overlap on one device race; calls on one stream, or
// ordered across streams, do not.
#include <mutex>
#include <vector>

#include "mnb_internal.h"

namespace {

// Partial tiles of the largest GEMM grid (kSkMaxGrid workgroups: two
// 128 x 256 fp32 tiles each, 64 MiB); staged x: 16 MiB of fp16.
constexpr size_t kWorkspaceBytes = mnb::sk_workspace_bytes(mnb::kSkMaxGrid);
constexpr size_t kStageBytes = (size_t)16 << 20;

}  // namespace

static __device__ __align__(256) unsigned char scratch[kWorkspaceBytes + kStageBytes];

namespace {

std::mutex g_mutex;
std::vector<void *> g_scratch;   // device address of `scratch`, per device

}  // namespace

hipError_t mnb::noalloc_scratch(int device, void **out) {
    *out = nullptr;
    if (device < 0) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mutex);
    if ((size_t)device >= g_scratch.size()) g_scratch.resize((size_t)device + 1, nullptr);
    if (!g_scratch[(size_t)device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch[(size_t)device] = p;
    }
    *out = g_scratch[(size_t)device];
    return hipSuccess;
}

extern "C" int32_t mnb_matmul_noalloc(mnb_context *ctx, const mnb_weight *w, int32_t M, const void *x,
                                      int32_t x_type, int64_t x_elems, void *y, int32_t y_type, int64_t y_elems,
                                      uint32_t flags, void *stream) {
    const int32_t st = mnb::check_matmul(ctx, w, M, x, x_type, x_elems, y, y_type, y_elems, flags);
    if (st != MNB_OK) return st;
    if (flags & MNB_HOST_MEMORY)
        return mnb::report(MNB_ERR_INVALID_ARGUMENT, "mnb_matmul_noalloc takes device pointers only (no MNB_HOST_MEMORY)");
    if (!ctx->scratch) return mnb::report(MNB_ERR_INVALID_STATE, "Kernel not prepared: no scratch array on this device");
    char msg[256];
    const size_t stage = mnb::stage_x_bytes(w, M, x, x_type);
    if (stage > kStageBytes) {
        snprintf(msg, sizeof msg,
                 "x needs %zu bytes of fp16 staging, more than the %zu of mnb_matmul_noalloc's scratch array "
                 "(16-byte aligned fp16 x with K a multiple of 8 needs none)",
                 stage, kStageBytes);
        return mnb::report(MNB_ERR_INVALID_ARGUMENT, msg);
    }
    // the workspace of the grids this call will launch (the plan of every row chunk)
    const size_t ws = mnb::prefill_workspace_bytes(w->g, M, ctx->cu_count);
    if (ws > kWorkspaceBytes) {
        snprintf(msg, sizeof msg, "the GEMM's partial tiles need %zu bytes, more than the %zu of mnb_matmul_noalloc's "
                 "scratch array", ws, kWorkspaceBytes);
        return mnb::report(MNB_ERR_UNSUPPORTED, msg);
    }
    mnb::DeviceGuard guard(ctx->device);
    hipStream_t s = stream ? (hipStream_t)stream : ctx->stream;
    unsigned char *base = (unsigned char *)ctx->scratch;
    const hipError_t e = mnb::launch_product(w, ctx->cu_count, M, x, x_type, y, y_type, (flags & MNB_ACCUMULATE) != 0,
                                             base + kWorkspaceBytes, base, kWorkspaceBytes, s);
    if (e != hipSuccess) {
        snprintf(msg, sizeof msg, "MatMulNBitsKernel.%s failed: %s (%s)", M == 1 ? "matvec" : "matmulBatch",
                 hipGetErrorString(e), hipGetErrorName(e));
        return mnb::report(MNB_ERR_DEVICE, msg);
    }
    return MNB_OK;
}
