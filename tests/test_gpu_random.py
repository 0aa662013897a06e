"""Seeded random single products through every path the planners choose.

Each case draws M from one of the size classes (1; 2..8; 9..16; 17..64;
65..600; and 601..3000 in a test of its own), K from 8 to 6000 (mostly multiples of 8, else x is staged), N
from 1 to 40000, a block size from 16 to 256, zero points or not, and (a
quarter of the single-product cases) fp32 scales that fp16 cannot hold, and
checks mnb_matmul against the oracle on up to 256 sampled output columns:
fp32 y within the parity bound, fp16 y the rounded fp32 y, and y += equal
to y0 + y bit for bit.  The planners' choice (GEMV, K-sliced kernel, GEMM
in stream-K or tile-list order) is printed with each case."""
import numpy as np
import pytest

import mnb_hip
from mnb_hip import synth
import mnb_oracle as orc
from parity_util import assert_parity, max_abs_w, oracle_matmul, say, upload

pytestmark = pytest.mark.gpu

CASES_PER_SEED = 16


@pytest.fixture(scope="module")
def ctx():
    orc.build()
    c = mnb_hip.Context(0)
    yield c
    c.close()


def _draw(rng):
    cls = int(rng.integers(0, 5))
    M = [1, int(rng.integers(2, 9)), int(rng.integers(9, 17)), int(rng.integers(17, 65)), int(rng.integers(65, 601))][cls]
    bs = int(rng.choice([16, 32, 64, 128, 256]))
    K = int(rng.integers(8, 6001))
    if rng.random() < 0.7:
        K -= K % 8
    K = max(K, 8)
    N = [int(rng.integers(1, 64)), int(rng.integers(64, 4096)), int(rng.integers(4096, 40001))][int(rng.integers(0, 3))]
    zp = bool(rng.random() < 0.5)
    return M, K, N, bs, zp


def _upload(ctx, t, f32s):
    """The weight with its fp16 scales, or (f32s) with fp32 scales that fp16
    cannot hold (the device then keeps fp32 scales, as for the tied head's
    quantizer); returns the weight and the fp32 scales given (or None)."""
    if not f32s:
        return upload(ctx, t), None
    s = t.scales_f16.astype(np.float32) * np.float32(1.0 + 2.0 ** -14)
    if t.zp_row_padded is not None:
        return mnb_hip.Weight(ctx, t.N, t.K, t.bs, t.q, s, t.zp_row_padded, mnb_hip.MNB_ZP_ROW_PADDED), s
    return mnb_hip.Weight(ctx, t.N, t.K, t.bs, t.q, s), s


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_single_products(ctx, seed):
    rng = np.random.default_rng(70000 + seed)
    for case in range(CASES_PER_SEED):
        M, K, N, bs, zp = _draw(rng)
        f32s = bool(rng.random() < 0.25)
        t = synth.make_weight(71000 + 100 * seed + case, N, K, bs, with_zp=zp)
        w, s32 = _upload(ctx, t, f32s)
        try:
            label = "random seed=%d case=%d M=%d K=%d N=%d bs=%d zp=%d f32s=%d plan=%s" % (
                seed, case, M, K, N, bs, zp, f32s, w.plan(M).as_tuple())
            say(label)
            x16 = synth.make_x(72000 + 100 * seed + case, M, K)
            rows = np.sort(rng.choice(N, min(N, 256), replace=False))
            y_ref, wmax = oracle_matmul(t, x16, rows, scales=s32)
            if wmax is None and s32 is not None:
                wmax = max_abs_w(t, s32)
            y32 = w.matmul(x16).reshape(M, N)
            assert_parity(y32[:, rows], y_ref.reshape(M, -1), x16, t, wmax, False, label)
            y16 = w.matmul(x16, out_dtype=np.float16).reshape(M, N)
            assert np.array_equal(y16.view(np.uint16), y32.astype(np.float16).view(np.uint16)), label
            y0 = rng.standard_normal((M, N)).astype(np.float32)
            acc = w.matmul(x16, y=y0.copy(), accumulate=True).reshape(M, N)
            assert np.array_equal(acc.view(np.uint32), (y0 + y32).view(np.uint32)), label
        finally:
            w.close()


@pytest.mark.parametrize("seed", [0, 1])
def test_random_large_single_products(ctx, seed):
    rng = np.random.default_rng(73000 + seed)
    for case in range(4):
        M, K, N = int(rng.integers(601, 3001)), int(rng.integers(8, 6001)), int(rng.integers(1, 20001))
        bs, zp = int(rng.choice([16, 32, 64, 128, 256])), bool(rng.random() < 0.5)
        t = synth.make_weight(74000 + 100 * seed + case, N, K, bs, with_zp=zp)
        w = upload(ctx, t)
        try:
            label = "random large seed=%d case=%d M=%d K=%d N=%d bs=%d zp=%d plan=%s" % (
                seed, case, M, K, N, bs, zp, w.plan(M).as_tuple())
            say(label)
            x16 = synth.make_x(75000 + 100 * seed + case, M, K)
            rows = np.sort(rng.choice(N, min(N, 128), replace=False))
            y_ref, wmax = oracle_matmul(t, x16, rows)
            y32 = w.matmul(x16).reshape(M, N)
            assert_parity(y32[:, rows], y_ref.reshape(M, -1), x16, t, wmax, False, label)
            y16 = w.matmul(x16, out_dtype=np.float16).reshape(M, N)
            assert np.array_equal(y16.view(np.uint16), y32.astype(np.float16).view(np.uint16)), label
        finally:
            w.close()
