"""numpy-facing wrapper of the CPU oracle (oracle/mnb_oracle.c).

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of bench.py may import this module; the product library
never does.  It restates the reference's Java CPU MatMulNBits path; each
function names the reference file:line it follows (paths relative to the
reference repository root; see the header of mnb_oracle.c for the short
names P3W, Q2W, MNK, QGK, SFO, VFO).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libmnb_oracle.so")
_lib = None

_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)


def build() -> str:
    """Compile the oracle with its own Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.mnb_ref_fp16_to_fp32.restype = ctypes.c_float
        L.mnb_ref_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.mnb_ref_fp32_to_fp16.restype = ctypes.c_uint16
        L.mnb_ref_fp32_to_fp16.argtypes = [ctypes.c_float]
        L.mnb_ref_scales_fp16_to_fp32.restype = None
        L.mnb_ref_scales_fp16_to_fp32.argtypes = [_u16p, _f32p, ctypes.c_int64]
        L.mnb_ref_dequantize.restype = None
        L.mnb_ref_dequantize.argtypes = [_u8p, _f32p, _u8p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _f32p]
        L.mnb_ref_dot_scalar.restype = ctypes.c_float
        L.mnb_ref_dot_scalar.argtypes = [_f32p, _f32p, ctypes.c_int32]
        L.mnb_ref_dot_lanes.restype = ctypes.c_float
        L.mnb_ref_dot_lanes.argtypes = [_f32p, _f32p, ctypes.c_int32, ctypes.c_int32]
        L.mnb_ref_matmul.restype = ctypes.c_int
        L.mnb_ref_matmul.argtypes = [_u8p, _f32p, _u8p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _f32p,
                                     _f32p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
        L.mnb_ref_matvec.restype = ctypes.c_int
        L.mnb_ref_matvec.argtypes = [_u8p, _f32p, _u8p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _f32p,
                                     _f32p, ctypes.c_int32, ctypes.c_int32]
        L.mnb_ref_matmul_f64.restype = ctypes.c_int
        L.mnb_ref_matmul_f64.argtypes = [_u8p, _f32p, _u8p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                         _f32p, _f64p, ctypes.c_int32]
        L.mnb_ref_pack_u4.restype = None
        L.mnb_ref_pack_u4.argtypes = [_u8p, ctypes.c_int64, ctypes.c_int]
        L.mnb_ref_java_round.restype = ctypes.c_int32
        L.mnb_ref_java_round.argtypes = [ctypes.c_float]
        L.mnb_ref_zp_default.restype = ctypes.c_int64
        L.mnb_ref_zp_default.argtypes = [ctypes.c_int64, _u8p]
        L.mnb_ref_zp_repack_row_padded.restype = ctypes.c_int64
        L.mnb_ref_zp_repack_row_padded.argtypes = [_u8p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, _u8p]
        L.mnb_ref_zp_pack_unpacked_u8.restype = ctypes.c_int64
        L.mnb_ref_zp_pack_unpacked_u8.argtypes = [_u8p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, _u8p]
        L.mnb_ref_zp_pack_unpacked_f32.restype = ctypes.c_int64
        L.mnb_ref_zp_pack_unpacked_f32.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, _u8p]
        L.mnb_ref_zp_normalize_raw.restype = ctypes.c_int64
        L.mnb_ref_zp_normalize_raw.argtypes = [_u8p, ctypes.c_int64, _i64p, ctypes.c_int32, ctypes.c_int32,
                                               ctypes.c_int32, _u8p]
        L.mnb_ref_choose_tied_block_size.restype = ctypes.c_int32
        L.mnb_ref_choose_tied_block_size.argtypes = [ctypes.c_int32]
        L.mnb_ref_quant_block_params.restype = None
        L.mnb_ref_quant_block_params.argtypes = [_f32p, ctypes.c_int32, _f32p, _i32p]
        L.mnb_ref_quantize_rows_u4.restype = ctypes.c_int
        L.mnb_ref_quantize_rows_u4.argtypes = [_f32p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _u8p, _f32p,
                                               _u8p]
        L.mnb_ref_fuse_rows.restype = ctypes.c_int32
        L.mnb_ref_fuse_rows.argtypes = [ctypes.c_int32, _i32p, _i32p, _i32p, ctypes.POINTER(_u8p),
                                        ctypes.POINTER(_f32p), ctypes.POINTER(_u8p), _u8p, _f32p, _u8p]
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# --------------------------------------------------------------------------
# fp16 conversions
# --------------------------------------------------------------------------

def fp16_bits_to_fp32(bits) -> np.ndarray:
    """P3W:665-683 fp16ToFp32 applied element-wise (loader conversion of scales,
    including the subnormal quirk)."""
    b = _c(bits, np.uint16).reshape(-1)
    out = np.empty(b.shape, np.float32)
    lib().mnb_ref_scales_fp16_to_fp32(_p(b, _u16p), _p(out, _f32p), b.size)
    return out.reshape(np.shape(bits))


def fp32_to_fp16_bits(values) -> np.ndarray:
    """IEEE binary32 -> binary16 RNE bit patterns (fixture generation)."""
    v = _c(values, np.float32).reshape(-1)
    f = lib().mnb_ref_fp32_to_fp16
    out = np.fromiter((f(float(x)) for x in v), dtype=np.uint16, count=v.size)
    return out.reshape(np.shape(values))


# --------------------------------------------------------------------------
# Dequantization and products
# --------------------------------------------------------------------------

def dequantize(q, scales, zp_flat, N: int, K: int, bs: int) -> np.ndarray:
    """MNK:2674-2705 dequantizeInt4 -> float32 [N, K] (K = padded reference K)."""
    q = _c(q, np.uint8).reshape(-1)
    s = _c(scales, np.float32).reshape(-1)
    z = _c(zp_flat, np.uint8).reshape(-1)
    _check_sizes(q, s, z, N, K, bs)
    out = np.empty((N, K), np.float32)
    lib().mnb_ref_dequantize(_p(q, _u8p), _p(s, _f32p), _p(z, _u8p), N, K, bs, _p(out, _f32p))
    return out


def _check_sizes(q, s, z, N, K, bs):
    if K % bs:
        raise ValueError("reference K must be a multiple of block_size")
    kb = K // bs
    if q.size < N * K // 2 or s.size < N * kb or z.size < (N * kb + 1) // 2:
        raise ValueError("buffer too small for N=%d K=%d bs=%d" % (N, K, bs))


def matmul(q, scales, zp_flat, N: int, K: int, bs: int, x, y: Optional[np.ndarray] = None,
           lanes: int = 0, threads: int = 1) -> np.ndarray:
    """P3W:157-192 QuantizedWeight.matmul: y += x @ W^T (accumulate), fp32.

    ``x`` is float32 [M, K] (K padded, as the reference requires).  ``y`` is
    updated in place when given, otherwise a zero array is used.  ``lanes``=0
    uses the scalar block dot (SFO:16-22), otherwise the Vector-API dot
    (VFO:47-68) with that many lanes.
    """
    q = _c(q, np.uint8).reshape(-1)
    s = _c(scales, np.float32).reshape(-1)
    z = _c(zp_flat, np.uint8).reshape(-1)
    _check_sizes(q, s, z, N, K, bs)
    x = _c(x, np.float32)
    M = x.size // K
    if x.size != M * K:
        raise ValueError("x size is not a multiple of K")
    if y is None:
        y = np.zeros((M, N), np.float32)
    if y.dtype != np.float32 or not y.flags.c_contiguous or y.size != M * N:
        raise ValueError("y must be a contiguous float32 array of M*N elements")
    rc = lib().mnb_ref_matmul(_p(q, _u8p), _p(s, _f32p), _p(z, _u8p), N, K, bs, _p(x, _f32p), _p(y, _f32p), M,
                              lanes, threads)
    if rc != 0:
        raise ValueError("mnb_ref_matmul rejected its arguments")
    return y


def matvec(q, scales, zp_flat, N, K, bs, x, y=None, lanes=0, threads=1) -> np.ndarray:
    """P3W:123-152 QuantizedWeight.matvec: y += x @ W^T for one row."""
    x = _c(x, np.float32).reshape(1, K)
    if y is not None:
        y2 = y.reshape(1, N)
        matmul(q, scales, zp_flat, N, K, bs, x, y2, lanes, threads)
        return y
    return matmul(q, scales, zp_flat, N, K, bs, x, None, lanes, threads).reshape(N)


def matmul_f64(q, scales, zp_flat, N, K, bs, x) -> np.ndarray:
    """Double-precision product of the dequantized weights (error analysis)."""
    q = _c(q, np.uint8).reshape(-1)
    s = _c(scales, np.float32).reshape(-1)
    z = _c(zp_flat, np.uint8).reshape(-1)
    _check_sizes(q, s, z, N, K, bs)
    x = _c(x, np.float32)
    M = x.size // K
    out = np.empty((M, N), np.float64)
    lib().mnb_ref_matmul_f64(_p(q, _u8p), _p(s, _f32p), _p(z, _u8p), N, K, bs, _p(x, _f32p), _p(out, _f64p), M)
    return out


def dot_scalar(a, b) -> float:
    a = _c(a, np.float32)
    b = _c(b, np.float32)
    return float(lib().mnb_ref_dot_scalar(_p(a, _f32p), _p(b, _f32p), a.size))


def dot_lanes(a, b, lanes: int) -> float:
    a = _c(a, np.float32)
    b = _c(b, np.float32)
    return float(lib().mnb_ref_dot_lanes(_p(a, _f32p), _p(b, _f32p), a.size, lanes))


def tolerance(K: int, x, w) -> float:
    """The parity bound 1e-3 * sqrt(K) * max|x| * max|w| (K = true K)."""
    return 1e-3 * float(np.sqrt(K)) * float(np.max(np.abs(x))) * float(np.max(np.abs(w)))


# --------------------------------------------------------------------------
# Zero-point layouts, quantizer, fusion
# --------------------------------------------------------------------------

def zp_default(block_count: int) -> np.ndarray:
    out = np.empty((block_count + 1) // 2, np.uint8)
    lib().mnb_ref_zp_default(block_count, _p(out, _u8p))
    return out


def zp_repack_row_padded(row_packed, rows: int, bpr: int) -> np.ndarray:
    """Q2W:1055-1075: ONNX [rows, ceil(bpr/2)] -> flat stream."""
    d = _c(row_packed, np.uint8).reshape(-1)
    out = np.empty((rows * bpr + 1) // 2, np.uint8)
    n = lib().mnb_ref_zp_repack_row_padded(_p(d, _u8p), d.size, rows, bpr, _p(out, _u8p))
    if n < 0:
        raise ValueError("zero-point tensor is truncated")
    return out


def zp_pack_unpacked_u8(vals, rows: int, bpr: int) -> np.ndarray:
    d = _c(vals, np.uint8).reshape(-1)
    out = np.empty((rows * bpr + 1) // 2, np.uint8)
    if lib().mnb_ref_zp_pack_unpacked_u8(_p(d, _u8p), d.size, rows, bpr, _p(out, _u8p)) < 0:
        raise ValueError("zero-point tensor is truncated")
    return out


def zp_pack_unpacked_f32(vals, rows: int, bpr: int) -> np.ndarray:
    d = _c(vals, np.float32).reshape(-1)
    out = np.empty((rows * bpr + 1) // 2, np.uint8)
    if lib().mnb_ref_zp_pack_unpacked_f32(_p(d, _f32p), d.size, rows, bpr, _p(out, _u8p)) < 0:
        raise ValueError("zero-point tensor is truncated")
    return out


def zp_normalize_raw(data, dims: Sequence[int], rows: int, bpr: int) -> np.ndarray:
    """Q2W:1023-1053 normalizeRawUInt4ZeroPoints."""
    d = _c(data, np.uint8).reshape(-1)
    dm = np.asarray(list(dims), np.int64)
    out = np.zeros(max(d.size, (rows * bpr + 1) // 2, 1), np.uint8)
    n = lib().mnb_ref_zp_normalize_raw(_p(d, _u8p), d.size, _p(dm, _i64p), dm.size, rows, bpr, _p(out, _u8p))
    if n < 0:
        raise ValueError("Unexpected zero-point layout")
    return out[:n].copy()


def java_round(v: float) -> int:
    return int(lib().mnb_ref_java_round(float(v)))


def choose_tied_block_size(hidden: int) -> int:
    return int(lib().mnb_ref_choose_tied_block_size(hidden))


def quant_block_params(block) -> tuple:
    b = _c(block, np.float32)
    s = ctypes.c_float()
    z = ctypes.c_int32()
    lib().mnb_ref_quant_block_params(_p(b, _f32p), b.size, ctypes.byref(s), ctypes.byref(z))
    return float(np.float32(s.value)), int(z.value)


def quantize_rows_u4(data, rows: int, cols: int, bs: int):
    """Q2W:1348-1398 quantizeDenseRowsToUInt4 -> (q, scales f32, zp flat)."""
    d = _c(data, np.float32).reshape(-1)
    q = np.empty(rows * cols // 2, np.uint8)
    s = np.empty(rows * (cols // bs), np.float32)
    z = np.empty((rows * (cols // bs) + 1) // 2, np.uint8)
    if lib().mnb_ref_quantize_rows_u4(_p(d, _f32p), rows, cols, bs, _p(q, _u8p), _p(s, _f32p), _p(z, _u8p)):
        raise ValueError("columns are not block-aligned")
    return q, s, z


def fuse_rows(parts):
    """QGK:243-315 tryFuseQuantizedRowwise over parts = [(q, scales, zp, N, K, bs)].
    Returns (q, scales, zp, fusedN) or None where the reference refuses."""
    n = len(parts)
    Ns = np.asarray([p[3] for p in parts], np.int32)
    Ks = np.asarray([p[4] for p in parts], np.int32)
    Bs = np.asarray([p[5] for p in parts], np.int32)
    qs = [_c(p[0], np.uint8).reshape(-1) for p in parts]
    ss = [_c(p[1], np.float32).reshape(-1) for p in parts]
    zs = [_c(p[2], np.uint8).reshape(-1) for p in parts]
    K, bs = int(Ks[0]), int(Bs[0])
    bpr = K // bs
    total = int(Ns.sum())
    outQ = np.zeros(total * K // 2, np.uint8)
    outS = np.zeros(total * bpr, np.float32)
    outZ = np.zeros((total * bpr + 1) // 2, np.uint8)
    qa = (_u8p * n)(*[_p(a, _u8p) for a in qs])
    sa = (_f32p * n)(*[_p(a, _f32p) for a in ss])
    za = (_u8p * n)(*[_p(a, _u8p) for a in zs])
    r = lib().mnb_ref_fuse_rows(n, _p(Ns, _i32p), _p(Ks, _i32p), _p(Bs, _i32p), qa, sa, za, _p(outQ, _u8p),
                                _p(outS, _f32p), _p(outZ, _u8p))
    if r < 0:
        return None
    return outQ, outS, outZ, int(r)
