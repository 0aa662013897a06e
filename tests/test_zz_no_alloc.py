"""mnb_matmul_noalloc against mnb_matmul, through the C ABI.

The allocation-free entry point runs the same kernels on the same grid as
mnb_matmul with device pointers (the GEMV, the K-sliced kernel or the GEMM,
by the same plan); only the GEMM's split-tile partial sums and the staged
fp16 x live in the library's fixed device array instead of context buffers.  Its outputs therefore equal mnb_matmul's bit for bit (a stronger bar
than the parity bound).  Each case runs two calls in a row, the second with a
smaller input, so the second call reads scratch contents the first one left
behind.  With every library allocation made to fail (MNB_FAULT_INJECT=alloc)
the entry point still succeeds where mnb_matmul, which must grow its staging
buffer, fails."""
import ctypes
import os

import numpy as np
import pytest

import mnb_hip
from mnb_hip import synth
import mnb_oracle as orc
from parity_util import assert_parity, oracle_matmul, say, upload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    orc.build()
    c = mnb_hip.Context(0)
    yield c
    c.close()


def _call(fn, ctx, w, x, y, accumulate=False, stream=None):
    import torch
    M = x.shape[0]
    code = {torch.float16: mnb_hip.MNB_F16, torch.float32: mnb_hip.MNB_F32}
    return fn(ctx.handle, w.handle, M, ctypes.c_void_p(x.data_ptr()), code[x.dtype], x.numel(),
              ctypes.c_void_p(y.data_ptr()), code[y.dtype], y.numel(),
              mnb_hip.MNB_ACCUMULATE if accumulate else 0, stream)


def _both(ctx, w, x, ydt, acc=False):
    """(mnb_matmul output, mnb_matmul_noalloc output) on fresh outputs."""
    import torch
    L = mnb_hip.load()
    M = x.shape[0]
    y0 = torch.randn((M, w.N), device="cuda").to(ydt)
    ya, yb = y0.clone(), y0.clone()
    torch.cuda.synchronize()     # the calls run on the context's own stream
    mnb_hip.check(_call(L.mnb_matmul, ctx, w, x, ya, acc))
    mnb_hip.check(_call(L.mnb_matmul_noalloc, ctx, w, x, yb, acc))
    torch.cuda.synchronize()
    return ya, yb


# (M, K, N, zero points, x dtype, unaligned x, y dtype, y +=): split GEMM
# tiles (stream-K partials in the scratch array), the K-sliced kernel (also
# with 16-row blocks at M <= 16), staged x (fp32, K % 8 != 0, a misaligned
# pointer), the M <= 16 kernels (the GEMV with one, two and four x row
# groups); each case is followed by a smaller one of the same kind.
CASES = [
    ((200, 8192, 9001, False, "f16", False, "f16", False), (150, 8192, 9001, False, "f16", False, "f16", False)),
    # both regions of the array in one call: staged x (fp32, then a misaligned
    # fp16 pointer) with split stream-K tiles
    ((200, 8192, 9001, True, "f32", False, "f32", False), (150, 8192, 9001, True, "f16", True, "f16", True)),
    ((200, 3072, 1000, False, "f16", False, "f16", False), (130, 3072, 1000, False, "f16", False, "f16", False)),
    ((300, 4096, 1001, True, "f32", False, "f32", True), (40, 4096, 1001, True, "f32", False, "f32", True)),
    ((64, 1001, 700, True, "f16", False, "f16", False), (33, 1001, 700, True, "f16", False, "f16", False)),
    ((129, 3072, 3072, False, "f16", True, "f16", False), (17, 3072, 3072, False, "f16", True, "f16", False)),
    ((1, 3072, 9216, False, "f32", False, "f16", False), (1, 3072, 3072, False, "f16", False, "f32", True)),
    ((16, 1003, 500, True, "f32", False, "f16", False), (5, 1003, 500, True, "f16", True, "f16", False)),
    ((16, 3001, 16000, True, "f32", False, "f16", False), (12, 3001, 16000, True, "f16", True, "f32", True)),
    ((8, 2000, 3000, False, "f32", False, "f16", False), (3, 2000, 3000, False, "f16", True, "f32", True)),
]


@pytest.mark.parametrize("pair", CASES, ids=lambda p: "M%d-K%d-N%d" % p[0][:3])
def test_noalloc_equals_matmul_twice(ctx, pair):
    import torch
    for ci, (M, K, N, zp, xdt, unaligned, ydt, acc) in enumerate(pair):
        label = "noalloc M=%d K=%d N=%d zp=%d x=%s unaligned=%d y=%s acc=%d" % (M, K, N, zp, xdt, unaligned, ydt, acc)
        say(label)
        t = synth.make_weight(7000 + M + K + N, N, K, 32, with_zp=zp)
        w = upload(ctx, t)
        try:
            x16 = synth.make_x(7100 + M + K, M, K)
            tdt = torch.float16 if xdt == "f16" else torch.float32
            xt = torch.from_numpy(x16).cuda().to(tdt)
            if unaligned:     # a view that starts one element into its buffer
                buf = torch.empty(M * K + 1, dtype=tdt, device="cuda")
                buf[1:].copy_(xt.reshape(-1))
                xt = buf[1:].view(M, K)
                assert xt.data_ptr() % 16 != 0
            ydt_t = torch.float16 if ydt == "f16" else torch.float32
            if (M, K, N) in ((200, 8192, 9001), (150, 8192, 9001)):
                assert w.plan(M).as_tuple() == (mnb_hip.MNB_KERNEL_GEMM, mnb_hip.MNB_ORDER_STREAM_K, 128, 256), label
            if (K, N) == (3001, 16000):
                assert w.plan(M).as_tuple() == (mnb_hip.MNB_KERNEL_KSLICE, mnb_hip.MNB_ORDER_NONE, 16, 64), label
            ya, yb = _both(ctx, w, xt, ydt_t, acc)
            assert torch.equal(ya.view(torch.int16 if ydt == "f16" else torch.int32),
                               yb.view(torch.int16 if ydt == "f16" else torch.int32)), label
            if not acc:
                cols = np.arange(N) if N <= 4096 else np.concatenate([np.arange(0, N, 37), np.arange(N - 16, N)])
                y_ref, _ = oracle_matmul(t, x16, cols, want_wmax=False)
                assert_parity(yb.cpu().numpy()[:, cols], y_ref, x16, t, None, ydt == "f16", label)
        finally:
            w.close()


def test_noalloc_allocates_nothing_and_checks_its_limit(ctx):
    """With every library allocation failing, mnb_matmul cannot stage an fp32
    x for a weight whose staging buffer has not been grown yet, while
    mnb_matmul_noalloc runs it from the fixed array; host pointers and a
    staging need above the array's 16 MiB are refused with clear errors."""
    import torch
    L = mnb_hip.load()
    t = synth.make_weight(7301, 1000, 3001, 32)
    w = upload(ctx, t)
    ctx2 = mnb_hip.Context(0)        # a fresh context: its staging buffer is empty
    w2 = upload(ctx2, t)
    try:
        x16 = synth.make_x(7302, 300, 3001)
        x32 = torch.from_numpy(x16).cuda().float()
        ya = torch.zeros((300, 1000), dtype=torch.float32, device="cuda")
        yb = torch.zeros_like(ya)
        torch.cuda.synchronize()
        os.environ["MNB_FAULT_INJECT"] = "alloc"
        try:
            rc = _call(L.mnb_matmul, ctx2, w2, x32, ya)
            assert rc == mnb_hip.MNB_ERR_OUT_OF_MEMORY, (rc, mnb_hip.last_error())
            mnb_hip.check(_call(L.mnb_matmul_noalloc, ctx2, w2, x32, yb))
            torch.cuda.synchronize()
        finally:
            del os.environ["MNB_FAULT_INJECT"]
        mnb_hip.check(_call(L.mnb_matmul, ctx2, w2, x32, ya))
        torch.cuda.synchronize()
        assert torch.equal(ya.view(torch.int32), yb.view(torch.int32))
        # host pointers are refused
        xh = np.zeros((2, 3001), np.float32)
        yh = np.zeros((2, 1000), np.float32)
        rc = L.mnb_matmul_noalloc(ctx.handle, w.handle, 2, xh.ctypes.data, mnb_hip.MNB_F32, xh.size, yh.ctypes.data,
                                  mnb_hip.MNB_F32, yh.size, mnb_hip.MNB_HOST_MEMORY, None)
        assert rc == mnb_hip.MNB_ERR_INVALID_ARGUMENT and "device pointers only" in mnb_hip.last_error()
        # staging beyond the array: 2800 rows x 3008 halves = 16.8 MB > 16 MiB
        big = torch.zeros((2800, 3001), dtype=torch.float32, device="cuda")
        ybig = torch.zeros((2800, 1000), dtype=torch.float16, device="cuda")
        torch.cuda.synchronize()
        rc = _call(L.mnb_matmul_noalloc, ctx, w, big, ybig)
        assert rc == mnb_hip.MNB_ERR_INVALID_ARGUMENT and "staging" in mnb_hip.last_error(), mnb_hip.last_error()
        # the same call within the limit, 2700 rows (16.2 MB)
        mnb_hip.check(_call(L.mnb_matmul_noalloc, ctx, w, big[:2700], ybig[:2700]))
        torch.cuda.synchronize()
    finally:
        w2.close()
        ctx2.close()
        w.close()
