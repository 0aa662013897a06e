"""Shared helpers of the GPU parity tests: oracle inputs in the reference's
form, the parity bound, and weight upload through the C ABI.

The bound is the one the product is held to: |y - y_oracle| <= 1e-3 *
sqrt(K) * max|x| * max|w| (K = true K, max|w| over the dequantized weights),
plus one fp16 ulp of |y_oracle| when the output is fp16.
"""
import os
import sys

import numpy as np

import mnb_hip
from mnb_hip import synth
import mnb_oracle as orc

THREADS = min(16, len(os.sched_getaffinity(0)))


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def fp16_ulp(v):
    a = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return 2.0 ** (e - 10)


def zp_blocks(t: synth.QuantTensor) -> np.ndarray:
    """Zero point of every block, [N * kb] (8 where the weight has none)."""
    kb = t.kb
    if t.zp_row_padded is None:
        return np.full(t.N * kb, 8, np.int16)
    nib = np.empty((t.N, 2 * t.zp_row_padded.shape[1]), np.int16)
    nib[:, 0::2] = t.zp_row_padded & 0xF
    nib[:, 1::2] = t.zp_row_padded >> 4
    return nib[:, :kb].reshape(-1)


def oracle_inputs(t: synth.QuantTensor, rows=None, scales=None):
    """Reference-form tensors: fp32 scales (loader widening, or `scales` [N*kb]
    fp32 as uploaded), flat zero points (runtime layout; 0x88 when absent),
    optionally restricted to `rows`."""
    kb, bs = t.kb, t.bs
    q = t.q.reshape(t.N, kb * bs // 2)
    if scales is not None:
        s = np.asarray(scales, np.float32).reshape(t.N, kb)
    else:
        s = orc.fp16_bits_to_fp32(t.scales_f16.view(np.uint16)).reshape(t.N, kb)
    if t.zp_row_padded is not None:
        zrp = t.zp_row_padded
    else:
        zrp = np.full((t.N, (kb + 1) // 2), 0x88, np.uint8)
    if rows is not None:
        q, s, zrp = q[rows], s[rows], zrp[rows]
    n = q.shape[0]
    z = synth.zp_row_padded_to_flat(zrp, n, kb)
    return q.reshape(-1), s.reshape(-1), z, n


def oracle_matmul(t: synth.QuantTensor, x16: np.ndarray, rows=None, want_wmax=True, scales=None):
    """The oracle's y = x W^T (fp32) for output columns `rows` (all when None),
    and max|w| when asked for and the dequantized weight is small enough to
    form (else None).  `scales`: fp32 scales [N*kb] uploaded instead of the
    tensor's fp16 ones."""
    q, s, z, n = oracle_inputs(t, rows, scales)
    kpad = t.kb * t.bs
    M = x16.shape[0]
    x = np.zeros((M, kpad), np.float32)
    x[:, : t.K] = x16.astype(np.float32)
    y = orc.matmul(q, s, z, n, kpad, t.bs, x, threads=THREADS)
    wmax = None
    if want_wmax and n * kpad <= 64 << 20:
        wmax = float(np.max(np.abs(orc.dequantize(q, s, z, n, kpad, t.bs))))
    return y, wmax


def max_abs_w(t: synth.QuantTensor, scales=None) -> float:
    """An upper bound of max|w|: max over blocks of |scale| (the tensor's fp16
    scales, or `scales`) times the largest |q - zp| the zero-point layout
    allows (15 with zero points, 8 without)."""
    s = t.scales_f16.astype(np.float32) if scales is None else np.asarray(scales, np.float32)
    return float(np.max(np.abs(s)) * 15.0) if t.zp_row_padded is not None else float(np.max(np.abs(s)) * 8.0)


def exact_max_abs_w(t: synth.QuantTensor) -> float:
    """max|w| over the dequantized weight, exactly, without forming it: the
    largest |scale| * max|q - zp| over the 4096 blocks of largest |scale|, then
    over every block whose |scale| times the largest possible |q - zp| could
    still beat it."""
    kb, bs = t.kb, t.bs
    s = np.abs(t.scales_f16.astype(np.float32)).reshape(-1)
    q = t.q.reshape(t.N * kb, bs // 2)
    zp = zp_blocks(t)
    bound = 15 if t.zp_row_padded is not None else 8

    def block_max(idx):
        best = 0.0
        for i in range(0, idx.size, 65536):
            b = idx[i:i + 65536]
            qb = q[b].astype(np.int16)
            z = zp[b][:, None]
            m = np.maximum(np.abs((qb & 0xF) - z).max(1), np.abs((qb >> 4) - z).max(1))
            best = max(best, float((s[b] * m).max()))
        return best

    k = min(4096, s.size)
    best = block_max(np.argpartition(-s, k - 1)[:k])
    rest = np.nonzero(s * bound > best)[0]
    return max(best, block_max(rest)) if rest.size else best


def parity_bound(K: int, x16: np.ndarray, wmax: float) -> float:
    return 1e-3 * np.sqrt(K) * float(np.max(np.abs(x16.astype(np.float32)))) * wmax


def assert_parity(y, y_ref, x16, t, wmax=None, fp16_out=False, label=""):
    wm = wmax if wmax is not None else max_abs_w(t)
    tol = parity_bound(t.K, x16, wm)
    allowed = tol + (fp16_ulp(y_ref) if fp16_out else 0.0)
    err = np.abs(y.astype(np.float64) - y_ref.astype(np.float64))
    worst = float(np.max(err - allowed))
    say("parity %s: max|err|=%.3e tol=%.3e" % (label, float(np.max(err)), tol))
    assert np.all(np.isfinite(y)), label
    assert worst <= 0.0, "%s: max|err| %.3e exceeds bound %.3e" % (label, float(np.max(err)), tol)


def upload(ctx, t: synth.QuantTensor, as_f32_scales=False):
    s = t.scales_f16.astype(np.float32) if as_f32_scales else t.scales_f16
    if t.zp_row_padded is not None:
        return mnb_hip.Weight(ctx, t.N, t.K, t.bs, t.q, s, t.zp_row_padded, mnb_hip.MNB_ZP_ROW_PADDED)
    return mnb_hip.Weight(ctx, t.N, t.K, t.bs, t.q, s)
