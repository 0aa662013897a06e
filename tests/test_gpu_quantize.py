"""Device quantizer (mnb_weight_quantize) and weight read-back (mnb_weight_read).

Bars:
* the quantized weight's arrays (read back with mnb_weight_read) equal, byte
  for byte and bit for bit, the oracle's restatement of the reference's
  quantizeDenseRowsToUInt4 (Qwen2Weights.java:1352-1422; pinned by the
  closed-form cases of tests/golden/quantizer.json in tests/test_oracle.py);
* block_size 0 picks what chooseTiedLmHeadBlockSize picks;
* mnb_weight_read returns the arrays a weight was created from (flat or
  row-padded zero points, the 0x88 fill for the implicit zero point, fp16
  scales widened exactly);
* the tied lm_head of Qwen2.5-0.5B ([151936, 896], bs 128) quantized on the
  device gives products within 1e-3 * sqrt(K) * max|x| * max|w| of the
  oracle's, at M = 1 and 64.
"""
import sys
import time

import numpy as np
import pytest

import mnb_hip
import mnb_oracle as orc
from mnb_hip import synth

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    orc.build()
    c = mnb_hip.Context(0)
    yield c
    c.close()


def special_rows(cols, bs, rng):
    """Rows whose blocks hit every branch of calculateUInt4QuantizationBlock."""
    rows = []
    blocks = cols // bs
    kinds = [
        lambda: np.zeros(bs),                                   # max == min, |max| < 1e-8
        lambda: np.full(bs, 3e-9),                              # max == min, tiny
        lambda: np.full(bs, 0.75),                              # max == min > 0
        lambda: np.full(bs, -0.3),                              # max == min < 0
        lambda: np.linspace(-1, 2, bs),                         # ramp
        lambda: np.where(np.arange(bs) == 5, 40.0, 0.01),       # one outlier
        lambda: rng.standard_normal(bs) * 1e-40,                # fp32 subnormal values
        lambda: np.arange(bs) * 0.5 - 3.0,                      # ties at .5 after scaling
        lambda: -np.abs(rng.standard_normal(bs)),               # all negative
        lambda: rng.standard_normal(bs) * 0.02,                 # embedding-like
    ]
    for i in range(len(kinds)):
        row = np.concatenate([kinds[(i + b) % len(kinds)]() for b in range(blocks)])
        rows.append(row)
    return np.asarray(rows, np.float32)


@pytest.mark.parametrize("rows,cols,bs", [(37, 896, 0), (40, 576, 0), (17, 96, 0), (21, 48, 16), (19, 256, 32),
                                          (16, 640, 64), (3, 128, 128)])
def test_quantizer_bytes_equal_reference(ctx, rows, cols, bs):
    rng = np.random.default_rng(rows * cols + bs)
    data = rng.standard_normal((rows, cols)).astype(np.float32) * np.float32(0.05)
    bs_eff = bs or orc.choose_tied_block_size(cols)
    data = np.concatenate([data, special_rows(cols, bs_eff, rng)])
    R = data.shape[0]
    w = mnb_hip.Weight.quantize(ctx, data, bs)
    try:
        assert (w.N, w.K, w.block_size) == (R, cols, bs_eff)
        q, s, z = w.read()
        rq, rs, rz = orc.quantize_rows_u4(data, R, cols, bs_eff)
        assert np.array_equal(q, rq), "q bytes differ"
        assert np.array_equal(s.view(np.uint32), rs.view(np.uint32)), "scales differ"
        assert np.array_equal(z, rz), "zero points differ"
        # and the weight dequantizes to the reference's values
        dq = w.dequantize(np.float32)
        assert np.array_equal(dq.view(np.uint32), orc.dequantize(rq, rs, rz, R, cols, bs_eff).view(np.uint32))
    finally:
        w.close()


def test_quantizer_fp16_input_and_device_pointer(ctx):
    import torch
    rows, cols = 64, 384
    rng = np.random.default_rng(5)
    d16 = (rng.standard_normal((rows, cols)) * 0.1).astype(np.float16)
    w_host = mnb_hip.Weight.quantize(ctx, d16)
    t = torch.from_numpy(d16).to("cuda:0")
    torch.cuda.synchronize()
    w_dev = mnb_hip.Weight.quantize(ctx, t)
    try:
        rq, rs, rz = orc.quantize_rows_u4(d16.astype(np.float32), rows, cols, 128)
        for w in (w_host, w_dev):
            q, s, z = w.read()
            assert np.array_equal(q, rq) and np.array_equal(s.view(np.uint32), rs.view(np.uint32))
            assert np.array_equal(z, rz)
    finally:
        w_host.close()
        w_dev.close()


def test_quantizer_errors(ctx):
    d = np.zeros((4, 100), np.float32)
    with pytest.raises(mnb_hip.IllegalArgumentException, match="hidden size 100 is not block-aligned"):
        mnb_hip.Weight.quantize(ctx, d)
    with pytest.raises(mnb_hip.IllegalArgumentException, match="block_size=256 must be 16, 32, 64 or 128"):
        mnb_hip.Weight.quantize(ctx, np.zeros((4, 256), np.float32), 256)
    with pytest.raises(mnb_hip.IllegalArgumentException, match="cols=96 is not a multiple of block_size=64"):
        mnb_hip.Weight.quantize(ctx, np.zeros((4, 96), np.float32), 64)


@pytest.mark.parametrize("layout", ["flat", "row_padded", "none", "f32_scales"])
def test_read_returns_the_created_arrays(ctx, layout):
    N, K, bs = 45, 576, 64
    t = synth.make_weight(9, N, K, bs, with_zp=layout != "none")
    kb = t.kb
    s16 = t.scales_f16
    if layout == "flat":
        z = synth.zp_row_padded_to_flat(t.zp_row_padded, N, kb)
        w = mnb_hip.Weight(ctx, N, K, bs, t.q, s16, z, mnb_hip.MNB_ZP_FLAT)
    elif layout == "row_padded":
        z = synth.zp_row_padded_to_flat(t.zp_row_padded, N, kb)
        w = mnb_hip.Weight(ctx, N, K, bs, t.q, s16, t.zp_row_padded, mnb_hip.MNB_ZP_ROW_PADDED)
    elif layout == "none":
        z = orc.zp_default(N * kb)
        w = mnb_hip.Weight(ctx, N, K, bs, t.q, s16)
    else:
        s32 = (s16.astype(np.float32) * np.float32(1 + 2 ** -18)).astype(np.float32)
        z = synth.zp_row_padded_to_flat(t.zp_row_padded, N, kb)
        w = mnb_hip.Weight(ctx, N, K, bs, t.q, s32, z, mnb_hip.MNB_ZP_FLAT)
    try:
        q, s, zz = w.read()
        assert np.array_equal(q, t.q)
        exp_s = s32 if layout == "f32_scales" else s16.astype(np.float32)
        assert np.array_equal(s.view(np.uint32), exp_s.view(np.uint32))
        assert np.array_equal(zz, z)
    finally:
        w.close()


@pytest.mark.parametrize("bs", [16, 256])
def test_read_other_block_sizes(ctx, bs):
    N, K = 20, 1024
    t = synth.make_weight(3, N, K, bs, with_zp=True)
    z = synth.zp_row_padded_to_flat(t.zp_row_padded, N, t.kb)
    w = mnb_hip.Weight(ctx, N, K, bs, t.q, t.scales_f16, z, mnb_hip.MNB_ZP_FLAT)
    try:
        q, s, zz = w.read()
        assert np.array_equal(q, t.q) and np.array_equal(zz, z)
        assert np.array_equal(s.view(np.uint32), t.scales_f16.astype(np.float32).view(np.uint32))
    finally:
        w.close()


def test_qwen_tied_lm_head_quantized_on_device(ctx):
    """Qwen2.5-0.5B tied lm_head: embed_tokens [151936, 896] quantized on the
    device with the reference's block size choice (128), bytes equal to the
    oracle's, products at M = 1 and 64 within tolerance."""
    V, H = 151936, 896
    rng = np.random.default_rng(151936)
    emb = (rng.standard_normal((V, H), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    import torch
    t = torch.from_numpy(emb).to("cuda:0")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    w = mnb_hip.Weight.quantize(ctx, t)
    dt = time.perf_counter() - t0
    say("quantize [151936, 896] fp32 on device: %.2f ms (incl. allocation), %.1f GB/s of input"
        % (dt * 1e3, emb.nbytes / dt / 1e9))
    del t
    try:
        assert w.block_size == 128
        q, s, z = w.read()
        t0 = time.perf_counter()
        rq, rs, rz = orc.quantize_rows_u4(emb, V, H, 128)
        say("oracle quantizer: %.2f s" % (time.perf_counter() - t0))
        assert np.array_equal(q, rq) and np.array_equal(s.view(np.uint32), rs.view(np.uint32))
        assert np.array_equal(z, rz)
        wref = orc.dequantize(rq, rs, rz, V, H, 128)
        for M in (1, 64):
            x16 = synth.make_x(M, M, H)
            x = x16.astype(np.float32)
            y = w.matmul(x16, out_dtype=np.float32).reshape(M, V)
            y_ref = orc.matmul(rq, rs, rz, V, H, 128, x, threads=16)
            tol = orc.tolerance(H, x, wref)
            err = float(np.max(np.abs(y - y_ref)))
            say("  M=%d max|err| %.3e tol %.3e" % (M, err, tol))
            assert err <= tol
    finally:
        w.close()
