"""Python binding of libmnb_hip.so (ctypes over the C ABI in include/mnb.h).

The classes mirror the reference's Java operator interface for int4
MatMulNBits (paths relative to the reference repository root):

* ``MatMulNBitsKernel`` -- directml-windows-bindings/src/main/java/com/aresstack/
  windirectml/windows/MatMulNBitsKernel.java (ctor :940-970, matvec
  :1847-1914, matmulBatch :2145-2263, supportsBatch :2128, maxBatchRows
  :2361, dequantizeInt4 :2674-2705, getN/getK :2803-2812, close :2740).
* ``QuantizedWeightMatrix`` -- Qwen2Weights.WeightMatrix (y += x W^T),
  directml-inference/.../qwen/Qwen2Weights.java:289-319.

Errors map as in the reference: ``IllegalArgumentException`` (a ValueError)
for bad arguments, ``IllegalStateException`` (a RuntimeError) for use after
close, ``MnbError`` (RuntimeError, "MatMulNBitsKernel.<op> failed") for native
failures.  There is no CPU fallback: without the built library or a gfx950
device every call fails loudly.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# MNB_HIP_LIBRARY points the binding at another build of the same library.
LIB_PATH = os.environ.get("MNB_HIP_LIBRARY") or os.path.join(_HERE, "libmnb_hip.so")
CONTRACT_TEST_PATH = os.path.join(_HERE, "mnb_contract_test")

MNB_OK = 0
MNB_ERR_INVALID_ARGUMENT = 1
MNB_ERR_INVALID_STATE = 2
MNB_ERR_OUT_OF_MEMORY = 3
MNB_ERR_DEVICE = 4
MNB_ERR_NO_DEVICE = 5
MNB_ERR_UNSUPPORTED = 6
MNB_ERR_IO = 7

MNB_F32 = 0
MNB_F16 = 1
MNB_ZP_NONE = 0
MNB_ZP_FLAT = 1
MNB_ZP_ROW_PADDED = 2
MNB_HOST_MEMORY = 0x1
MNB_ACCUMULATE = 0x2
MNB_COPY_H2D, MNB_COPY_D2H, MNB_COPY_D2D = 0, 1, 2
MNB_PACK_PHI3, MNB_PACK_QWEN2, MNB_PACK_ONNX, MNB_PACK_SAFETENSORS = 1, 2, 3, 4

# Every symbol include/mnb.h declares.
EXPORTED_SYMBOLS = (
    "mnb_version", "mnb_last_error", "mnb_context_create", "mnb_context_destroy", "mnb_context_info",
    "mnb_weight_create", "mnb_weight_fuse_rows", "mnb_weight_quantize", "mnb_weight_read", "mnb_weight_destroy", "mnb_weight_shape", "mnb_weight_device_bytes", "mnb_matmul", "mnb_matmul_noalloc",
    "mnb_dequantize", "mnb_supports_batch", "mnb_max_batch_rows", "mnb_device_alloc", "mnb_device_free",
    "mnb_memcpy", "mnb_synchronize", "mnb_group_create", "mnb_group_run", "mnb_group_destroy", "mnb_matmul_plan", "mnb_group_plan",
    "mnb_pack_open", "mnb_pack_close", "mnb_pack_kind", "mnb_pack_weight_count", "mnb_pack_weight_name",
    "mnb_pack_find_projection", "mnb_pack_weight_info", "mnb_pack_read_weight", "mnb_pack_weight_create",
    "mnb_pack_tensor_info", "mnb_pack_weight_quantize",
)


class MnbError(RuntimeError):
    """Native failure: the reference's RuntimeException("MatMulNBitsKernel.<op> failed")."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class IllegalArgumentException(ValueError):
    code = MNB_ERR_INVALID_ARGUMENT


class IllegalStateException(RuntimeError):
    code = MNB_ERR_INVALID_STATE


class IOException(OSError):
    """Weight-file failure: the reference's java.io.IOException, with its message."""
    code = MNB_ERR_IO


class DeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 64), ("arch", ctypes.c_char * 64), ("compute_units", ctypes.c_int32),
                ("clock_khz", ctypes.c_int32), ("memory_clock_khz", ctypes.c_int32),
                ("memory_bus_width", ctypes.c_int32), ("total_memory", ctypes.c_int64),
                ("l2_bytes", ctypes.c_int32), ("lds_bytes_per_block", ctypes.c_int32),
                ("wavefront_size", ctypes.c_int32), ("device", ctypes.c_int32)]


class TripletInfo(ctypes.Structure):
    _fields_ = [("N", ctypes.c_int32), ("K", ctypes.c_int32), ("block_size", ctypes.c_int32),
                ("blocks_per_row", ctypes.c_int32), ("q_bytes", ctypes.c_int64), ("scale_count", ctypes.c_int64),
                ("zp_bytes", ctypes.c_int64), ("zp_implicit", ctypes.c_int32), ("scale_dtype", ctypes.c_int32)]


MNB_KERNEL_GEMV, MNB_KERNEL_STREAM, MNB_KERNEL_GEMV_GROUP, MNB_KERNEL_GEMM, MNB_KERNEL_KSLICE = 1, 2, 3, 4, 5
MNB_ORDER_NONE, MNB_ORDER_STREAM_K, MNB_ORDER_TILE_LIST, MNB_ORDER_TILE_LIST_PARTS = 0, 1, 2, 3


class PlanInfo(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_int32), ("order", ctypes.c_int32), ("tile_rows", ctypes.c_int32),
                ("tile_cols", ctypes.c_int32), ("workgroups", ctypes.c_int32)]

    def as_tuple(self):
        """(kernel, order, tile_rows, tile_cols)"""
        return (self.kernel, self.order, self.tile_rows, self.tile_cols)


class GroupItem(ctypes.Structure):
    _fields_ = [("weight", ctypes.c_void_p), ("M", ctypes.c_int32), ("x", ctypes.c_void_p),
                ("x_type", ctypes.c_int32), ("x_elems", ctypes.c_int64), ("y", ctypes.c_void_p),
                ("y_type", ctypes.c_int32), ("y_elems", ctypes.c_int64), ("flags", ctypes.c_uint32)]


_lib: Optional[ctypes.CDLL] = None


def library_path() -> str:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load libmnb_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise MnbError(MNB_ERR_NO_DEVICE, "libmnb_hip.so is not built (run __graft_entry__.build())")
    # One HIP runtime per process: PyTorch-ROCm ships its own libamdhip64 (soname
    # libamdhip64.so.7) and loads it under another file name.  Loaded first, it
    # also satisfies this library's libamdhip64.so.7 dependency; loaded after
    # this library it would start a second runtime that sees no device.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    L = ctypes.CDLL(LIB_PATH)
    vp, i32, i64, u32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32
    sig = {
        "mnb_version": (i32, []),
        "mnb_last_error": (ctypes.c_char_p, []),
        "mnb_context_create": (i32, [i32, ctypes.POINTER(vp)]),
        "mnb_context_destroy": (i32, [vp]),
        "mnb_context_info": (i32, [vp, ctypes.POINTER(DeviceInfo)]),
        "mnb_weight_create": (i32, [vp, i32, i32, i32, i32, vp, i64, vp, i32, i64, vp, i64, i32, u32,
                                    ctypes.POINTER(vp)]),
        "mnb_weight_fuse_rows": (i32, [vp, ctypes.POINTER(vp), i32, ctypes.POINTER(vp)]),
        "mnb_weight_quantize": (i32, [vp, vp, i32, i32, i32, i32, u32, ctypes.POINTER(vp)]),
        "mnb_weight_read": (i32, [vp, vp, vp, i64, vp, i64, vp, i64]),
        "mnb_weight_destroy": (i32, [vp]),
        "mnb_weight_shape": (i32, [vp, ctypes.POINTER(i32), ctypes.POINTER(i32), ctypes.POINTER(i32)]),
        "mnb_weight_device_bytes": (i64, [vp]),
        "mnb_matmul": (i32, [vp, vp, i32, vp, i32, i64, vp, i32, i64, u32, vp]),
        "mnb_matmul_noalloc": (i32, [vp, vp, i32, vp, i32, i64, vp, i32, i64, u32, vp]),
        "mnb_dequantize": (i32, [vp, vp, vp, i32, i64, u32, vp]),
        "mnb_supports_batch": (i32, [vp]),
        "mnb_max_batch_rows": (i32, []),
        "mnb_device_alloc": (i32, [vp, i64, ctypes.POINTER(vp)]),
        "mnb_device_free": (i32, [vp, vp]),
        "mnb_memcpy": (i32, [vp, vp, vp, i64, i32]),
        "mnb_synchronize": (i32, [vp]),
        "mnb_group_create": (i32, [vp, i32, ctypes.POINTER(GroupItem), ctypes.POINTER(vp)]),
        "mnb_group_run": (i32, [vp, vp, vp]),
        "mnb_group_destroy": (i32, [vp]),
        "mnb_matmul_plan": (i32, [vp, vp, i32, ctypes.POINTER(PlanInfo)]),
        "mnb_group_plan": (i32, [vp, ctypes.POINTER(PlanInfo)]),
        "mnb_pack_open": (i32, [ctypes.c_char_p, ctypes.POINTER(vp)]),
        "mnb_pack_close": (i32, [vp]),
        "mnb_pack_kind": (i32, [vp, ctypes.POINTER(i32)]),
        "mnb_pack_weight_count": (i32, [vp, ctypes.POINTER(i32)]),
        "mnb_pack_weight_name": (i32, [vp, i32, ctypes.c_char_p, i64, ctypes.POINTER(i64)]),
        "mnb_pack_find_projection": (i32, [vp, i32, ctypes.c_char_p, ctypes.c_char_p, i64, ctypes.POINTER(i64)]),
        "mnb_pack_weight_info": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(TripletInfo)]),
        "mnb_pack_read_weight": (i32, [vp, ctypes.c_char_p, vp, i64, vp, i64, vp, i64]),
        "mnb_pack_weight_create": (i32, [vp, vp, ctypes.c_char_p, ctypes.POINTER(vp)]),
        "mnb_pack_tensor_info": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(i32), ctypes.POINTER(i64), i32,
                                       ctypes.POINTER(i32)]),
        "mnb_pack_weight_quantize": (i32, [vp, vp, ctypes.c_char_p, i32, i32, i32, ctypes.POINTER(vp)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def last_error() -> str:
    return load().mnb_last_error().decode("utf-8", "replace")


def check(rc: int, op: str = "call") -> None:
    if rc == MNB_OK:
        return
    msg = last_error()
    if rc == MNB_ERR_INVALID_ARGUMENT:
        raise IllegalArgumentException(msg)
    if rc == MNB_ERR_INVALID_STATE:
        raise IllegalStateException(msg)
    if rc == MNB_ERR_IO:
        raise IOException(msg)
    raise MnbError(rc, msg)


def _dtype_code(dt) -> int:
    dt = np.dtype(dt)
    if dt == np.float32:
        return MNB_F32
    if dt == np.float16:
        return MNB_F16
    raise IllegalArgumentException("unsupported dtype %s (float16 or float32)" % dt)


def _torch_dtype_code(t) -> int:
    import torch
    if t.dtype == torch.float32:
        return MNB_F32
    if t.dtype == torch.float16:
        return MNB_F16
    raise IllegalArgumentException("unsupported dtype %s (float16 or float32)" % t.dtype)


def _is_torch(a) -> bool:
    return type(a).__module__.startswith("torch")


class Context:
    """One device (the reference's WindowsBindings + its command queue)."""

    def __init__(self, device: int = 0):
        L = load()
        h = ctypes.c_void_p()
        check(L.mnb_context_create(device, ctypes.byref(h)), "init")
        self._h = h
        self.device = device

    @property
    def handle(self):
        if self._h is None:
            raise IllegalStateException("context is closed")
        return self._h

    def info(self) -> DeviceInfo:
        i = DeviceInfo()
        check(load().mnb_context_info(self.handle, ctypes.byref(i)), "info")
        return i

    def synchronize(self) -> None:
        check(load().mnb_synchronize(self.handle), "synchronize")

    def close(self) -> None:
        if self._h is not None:
            check(load().mnb_context_destroy(self._h), "close")
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class Weight:
    """A resident int4 weight triplet (one mnb_weight)."""

    def __init__(self, ctx: Context, N: int, K: int, block_size: int, q, scales, zero_points=None,
                 zp_layout: Optional[int] = None):
        L = load()
        q = np.ascontiguousarray(q, dtype=np.uint8).reshape(-1)
        scales = np.ascontiguousarray(scales)
        if scales.dtype == np.uint16:
            scales = scales.view(np.float16)
        st = _dtype_code(scales.dtype)
        scales = scales.reshape(-1)
        if zero_points is None:
            zp_layout = MNB_ZP_NONE
            zp_ptr, zp_len = None, 0
        else:
            zero_points = np.ascontiguousarray(zero_points, dtype=np.uint8).reshape(-1)
            zp_layout = MNB_ZP_FLAT if zp_layout is None else zp_layout
            zp_ptr, zp_len = zero_points.ctypes.data, zero_points.size
        h = ctypes.c_void_p()
        check(L.mnb_weight_create(ctx.handle, N, K, block_size, 4, q.ctypes.data, q.size, scales.ctypes.data, st,
                                  scales.size, zp_ptr, zp_len, zp_layout, 0, ctypes.byref(h)), "prepare")
        self._h = h
        self.ctx = ctx
        self.N, self.K, self.block_size = N, K, block_size

    @classmethod
    def _adopt(cls, ctx: Context, h: ctypes.c_void_p) -> "Weight":
        """Wrap a weight handle the library created (e.g. mnb_pack_weight_create)."""
        w = cls.__new__(cls)
        w._h, w.ctx = h, ctx
        n, k, bs = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        check(load().mnb_weight_shape(h, ctypes.byref(n), ctypes.byref(k), ctypes.byref(bs)), "prepare")
        w.N, w.K, w.block_size = n.value, k.value, bs.value
        return w

    @classmethod
    def fuse_rows(cls, ctx: Context, parts) -> "Weight":
        """Rows of parts[0], then parts[1], ... in one new weight (mnb_weight_fuse_rows):
        QwenGpuKernels.tryFuseQuantizedRowwise / Phi3GpuKernels.createFusedQKV."""
        arr = (ctypes.c_void_p * len(parts))(*[p.handle for p in parts])
        h = ctypes.c_void_p()
        check(load().mnb_weight_fuse_rows(ctx.handle, arr, len(parts), ctypes.byref(h)), "prepare")
        return cls._adopt(ctx, h)

    @classmethod
    def quantize(cls, ctx: Context, data, block_size: int = 0, rows: Optional[int] = None,
                 cols: Optional[int] = None) -> "Weight":
        """Dense [rows, cols] -> int4 weight on the device (mnb_weight_quantize):
        Qwen2Weights.quantizeDenseRowsToUInt4; block_size 0 = the reference's choice.
        numpy data is a host array; a torch CUDA tensor is used in place."""
        L = load()
        h = ctypes.c_void_p()
        if _is_torch(data):
            rows, cols = (rows, cols) if rows is not None else tuple(data.shape)
            check(L.mnb_weight_quantize(ctx.handle, data.data_ptr(), _torch_dtype_code(data), rows, cols, block_size,
                                        0, ctypes.byref(h)), "prepare")
        else:
            a = np.ascontiguousarray(data)
            rows, cols = (rows, cols) if rows is not None else a.shape
            check(L.mnb_weight_quantize(ctx.handle, a.ctypes.data, _dtype_code(a.dtype), rows, cols, block_size,
                                        MNB_HOST_MEMORY, ctypes.byref(h)), "prepare")
        return cls._adopt(ctx, h)

    def read(self):
        """(qWeight uint8 [N*kb*bs/2], scales float32 [N*kb], zeroPoints uint8 flat): the
        reference's QuantizedWeight arrays of this resident weight (mnb_weight_read)."""
        kb = -(-self.K // self.block_size)
        q = np.empty(self.N * kb * self.block_size // 2, np.uint8)
        s = np.empty(self.N * kb, np.float32)
        z = np.empty((self.N * kb + 1) // 2, np.uint8)
        check(load().mnb_weight_read(self.ctx.handle, self.handle, q.ctypes.data, q.size, s.ctypes.data, s.size,
                                     z.ctypes.data, z.size), "read")
        return q, s, z

    @property
    def handle(self):
        if self._h is None:
            raise IllegalStateException("Kernel not prepared")
        return self._h

    @property
    def device_bytes(self) -> int:
        return int(load().mnb_weight_device_bytes(self.handle))

    def matmul(self, x, y=None, accumulate: bool = False, out_dtype=np.float32, stream=None):
        """y (=|+=) x W^T.  numpy arrays -> host path (synchronous, returns y);
        torch CUDA tensors -> device path (asynchronous on ``stream``)."""
        L = load()
        flags = MNB_ACCUMULATE if accumulate else 0
        if _is_torch(x):
            if y is None:
                raise IllegalArgumentException("device calls need an output tensor")
            M = x.numel() // self.K if x.dim() == 1 else x.shape[0]
            st = stream if stream is not None else 0
            check(L.mnb_matmul(self.ctx.handle, self.handle, M, x.data_ptr(), _torch_dtype_code(x), x.numel(),
                               y.data_ptr(), _torch_dtype_code(y), y.numel(), flags, st or None),
                  "matmulBatch")
            return y
        x = np.ascontiguousarray(x)
        M = 1 if x.ndim == 1 else x.shape[0]
        if y is None:
            y = np.zeros((M, self.N) if x.ndim > 1 else (self.N,), dtype=out_dtype)
        if not y.flags.c_contiguous:
            raise IllegalArgumentException("y must be contiguous")
        check(L.mnb_matmul(self.ctx.handle, self.handle, M, x.ctypes.data, _dtype_code(x.dtype), x.size,
                           y.ctypes.data, _dtype_code(y.dtype), y.size, flags | MNB_HOST_MEMORY, None),
              "matvec" if M == 1 else "matmulBatch")
        return y

    def plan(self, M: int) -> PlanInfo:
        """How mnb_matmul runs this weight at M rows (mnb_matmul_plan)."""
        p = PlanInfo()
        check(load().mnb_matmul_plan(self.ctx.handle, self.handle, M, ctypes.byref(p)), "plan")
        return p

    def dequantize(self, dtype=np.float32, out=None, stream=None):
        """[N, K] dequantized weight; numpy (host) or a torch CUDA tensor ``out``."""
        L = load()
        if out is not None and _is_torch(out):
            check(L.mnb_dequantize(self.ctx.handle, self.handle, out.data_ptr(), _torch_dtype_code(out),
                                   out.numel(), 0, stream or None), "dequantizeInt4")
            return out
        out = np.empty((self.N, self.K), dtype=dtype)
        check(L.mnb_dequantize(self.ctx.handle, self.handle, out.ctypes.data, _dtype_code(dtype), out.size,
                               MNB_HOST_MEMORY, None), "dequantizeInt4")
        return out

    def close(self) -> None:
        if self._h is not None:
            check(load().mnb_weight_destroy(self._h), "close")
            self._h = None


class Group:
    """Independent products recorded once and run as one launch (device tensors).

    ``entries`` is a list of (Weight, x, y) with torch CUDA tensors; x is fp16
    [M, K], y fp16 or fp32 [M, N]; all items M == 1, all 1 < M <= 16, or all
    M > 16.  No item may read another item's output (they may run
    concurrently)."""

    def __init__(self, ctx: Context, entries, accumulate: bool = False):
        L = load()
        arr = (GroupItem * len(entries))()
        for i, (w, x, y) in enumerate(entries):
            M = x.numel() // w.K
            arr[i] = GroupItem(w.handle.value, M, x.data_ptr(), _torch_dtype_code(x), x.numel(), y.data_ptr(),
                               _torch_dtype_code(y), y.numel(), MNB_ACCUMULATE if accumulate else 0)
        h = ctypes.c_void_p()
        check(L.mnb_group_create(ctx.handle, len(entries), arr, ctypes.byref(h)), "group")
        self._h = h
        self.ctx = ctx
        self._keep = entries

    def plan(self) -> PlanInfo:
        """The kernel and work order recorded for this group (mnb_group_plan)."""
        if self._h is None:
            raise IllegalStateException("group is closed")
        p = PlanInfo()
        check(load().mnb_group_plan(self._h, ctypes.byref(p)), "plan")
        return p

    def run(self, stream=None) -> None:
        if self._h is None:
            raise IllegalStateException("group is closed")
        check(load().mnb_group_run(self.ctx.handle, self._h, stream or None), "matvec")

    def close(self) -> None:
        if self._h is not None:
            check(load().mnb_group_destroy(self._h), "close")
            self._h = None
            self._keep = None


class MatMulNBitsKernel:
    """The reference's MatMulNBitsKernel over the HIP library (fp32 host arrays)."""

    def __init__(self, ctx: Context, N: int, K: int, qWeight, scales, zeroPoints, blockSize: int):
        zp = None if zeroPoints is None else zeroPoints
        self._w = Weight(ctx, N, K, blockSize, qWeight, np.asarray(scales, dtype=np.float32), zp, MNB_ZP_FLAT)
        self.N, self.K = N, K

    def _weight(self) -> Weight:
        if self._w is None:
            raise IllegalStateException("Kernel not prepared")
        return self._w

    def matvec(self, x, out=None):
        x = np.asarray(x, dtype=np.float32)
        if x.size != self.K or x.ndim != 1:
            raise IllegalArgumentException("Input length %d != K=%d" % (x.size, self.K))
        y = np.empty(self.N, np.float32) if out is None else out
        self._weight().matmul(x, y)
        return y

    def matmulBatch(self, xBatch, outBatch, M: int):
        if M < 1:
            raise IllegalArgumentException("M out of range [1, %d]: %d" % (self.maxBatchRows(), M))
        x = np.asarray(xBatch, dtype=np.float32).reshape(-1)
        if x.size < M * self.K:
            raise IllegalArgumentException("xBatch too short: %d < %d" % (x.size, M * self.K))
        if outBatch.size < M * self.N:
            raise IllegalArgumentException("outBatch too short: %d < %d" % (outBatch.size, M * self.N))
        y = outBatch.reshape(-1)[: M * self.N].reshape(M, self.N)
        self._weight().matmul(x[: M * self.K].reshape(M, self.K), y)
        return outBatch

    def supportsBatch(self) -> bool:
        return self._w is not None and bool(load().mnb_supports_batch(self._w.handle))

    @staticmethod
    def maxBatchRows() -> int:
        return int(load().mnb_max_batch_rows())

    def getN(self) -> int:
        return self.N

    def getK(self) -> int:
        return self.K

    def dequantize(self) -> np.ndarray:
        return self._weight().dequantize(np.float32).reshape(-1)

    @staticmethod
    def dequantizeInt4(ctx: Context, qWeight, scales, zeroPoints, N: int, K: int, blockSize: int) -> np.ndarray:
        k = MatMulNBitsKernel(ctx, N, K, qWeight, scales, zeroPoints, blockSize)
        try:
            return k.dequantize()
        finally:
            k.close()

    def close(self) -> None:
        if self._w is not None:
            self._w.close()
            self._w = None


class QuantizedWeightMatrix:
    """Qwen2Weights.WeightMatrix semantics over the GPU: y += x W^T."""

    def __init__(self, kernel: MatMulNBitsKernel):
        self.kernel = kernel

    def matvec(self, x, y):
        self.kernel._weight().matmul(np.asarray(x, np.float32), y, accumulate=True)

    def matmul(self, x, y, seqLen: int):
        xs = np.asarray(x, np.float32).reshape(seqLen, self.kernel.K)
        self.kernel._weight().matmul(xs, y.reshape(seqLen, self.kernel.N), accumulate=True)

    def N(self) -> int:
        return self.kernel.N

    def K(self) -> int:
        return self.kernel.K


def _name_bytes(name: str) -> bytes:
    """Tensor and weight names are byte strings in the files; names that are
    not valid UTF-8 round-trip through surrogate escapes."""
    return name.encode("utf-8", "surrogateescape")


class Pack:
    """An opened weight file: a .wdmlpack package (Phi-3 roles or a Qwen
    runtimeGraph) or an ONNX model with MatMulNBits nodes (include/mnb.h,
    mnb_pack_*).  Mirrors Phi3RuntimePackage.open/weights and the quantized
    branch of Qwen2Weights loading: names are Phi-3 roles or MatMulNBits
    output names; failures raise ``IOException`` with the reference's text."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        check(load().mnb_pack_open(os.fsencode(path), ctypes.byref(h)), "open")
        self._h = h
        self.path = path

    @property
    def handle(self):
        if self._h is None:
            raise IllegalStateException("pack is closed")
        return self._h

    @property
    def kind(self) -> int:
        k = ctypes.c_int32()
        check(load().mnb_pack_kind(self.handle, ctypes.byref(k)))
        return k.value

    def names(self) -> list:
        L = load()
        n = ctypes.c_int32()
        check(L.mnb_pack_weight_count(self.handle, ctypes.byref(n)))
        out = []
        for i in range(n.value):
            ln = ctypes.c_int64()
            check(L.mnb_pack_weight_name(self.handle, i, None, 0, ctypes.byref(ln)))
            buf = ctypes.create_string_buffer(ln.value + 1)
            check(L.mnb_pack_weight_name(self.handle, i, buf, ln.value + 1, ctypes.byref(ln)))
            out.append(buf.value.decode("utf-8", "surrogateescape"))
        return out

    def find_projection(self, layer: int, projection: str) -> str:
        L = load()
        ln = ctypes.c_int64()
        check(L.mnb_pack_find_projection(self.handle, layer, _name_bytes(projection), None, 0, ctypes.byref(ln)))
        buf = ctypes.create_string_buffer(ln.value + 1)
        check(L.mnb_pack_find_projection(self.handle, layer, _name_bytes(projection), buf, ln.value + 1,
                                         ctypes.byref(ln)))
        return buf.value.decode("utf-8", "surrogateescape")

    def info(self, name: str) -> TripletInfo:
        i = TripletInfo()
        check(load().mnb_pack_weight_info(self.handle, _name_bytes(name), ctypes.byref(i)))
        return i

    def read(self, name: str):
        """(qWeight uint8, scales float32, zeroPoints uint8): the resolved triplet on the host."""
        i = self.info(name)
        q = np.empty(i.q_bytes, np.uint8)
        s = np.empty(i.scale_count, np.float32)
        z = np.empty(i.zp_bytes, np.uint8)
        check(load().mnb_pack_read_weight(self.handle, _name_bytes(name), q.ctypes.data, q.size, s.ctypes.data, s.size,
                                          z.ctypes.data if z.size else None, z.size))
        return q, s, z

    def tensor_info(self, name: str):
        """(ONNX element type, shape) of any tensor of the file (mnb_pack_tensor_info)."""
        dt, nd = ctypes.c_int32(), ctypes.c_int32()
        dims = (ctypes.c_int64 * 16)()
        check(load().mnb_pack_tensor_info(self.handle, _name_bytes(name), ctypes.byref(dt), dims, 16, ctypes.byref(nd)))
        return dt.value, tuple(dims[i] for i in range(min(nd.value, 16)))

    def quantize(self, ctx: Context, name: str, rows: int, cols: int, block_size: int = 0) -> Weight:
        """Dense [rows, cols] tensor -> int4 weight on the device (mnb_pack_weight_quantize): the
        reference's runtime-quantized tied lm_head read from the file."""
        h = ctypes.c_void_p()
        check(load().mnb_pack_weight_quantize(ctx.handle, self.handle, _name_bytes(name), rows, cols, block_size,
                                              ctypes.byref(h)), "prepare")
        return Weight._adopt(ctx, h)

    def weight(self, ctx: Context, name: str) -> Weight:
        """Upload one triplet to HBM (mnb_pack_weight_create)."""
        h = ctypes.c_void_p()
        check(load().mnb_pack_weight_create(ctx.handle, self.handle, _name_bytes(name), ctypes.byref(h)), "prepare")
        return Weight._adopt(ctx, h)

    def close(self) -> None:
        if self._h is not None:
            check(load().mnb_pack_close(self._h))
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
