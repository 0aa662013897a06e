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


def test_tied_lm_head_quantized_from_weight_files(ctx, tmp_path):
    """The runtime-quantized tied lm_head read from a file
    (mnb_pack_weight_quantize): a safetensors model.embed_tokens.weight in F32
    and in F16 (widened with the reference's fp16ToFp32, subnormal values
    included), and an ONNX model's FLOAT16 initializer in external data.  The
    weight's bytes equal the oracle's quantizeDenseRowsToUInt4 of the values
    the reference's embedding table holds; BF16 is refused as the reference
    refuses it, and a shape other than [vocab, hidden] fails with the
    reference's text."""
    import weightfiles as wf
    rows, cols = 300, 896
    rng = np.random.default_rng(11)
    emb = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    emb[3, :40] = rng.standard_normal(40).astype(np.float32) * 1e-6     # fp16 subnormals after rounding
    e16 = emb.astype(np.float16)
    e16_ref = orc.fp16_bits_to_fp32(e16.view(np.uint16))              # the reference's widening
    st = wf.write_safetensors(tmp_path / "model.safetensors",
                              [("model.embed_tokens.weight", "F32", (rows, cols), emb.tobytes()),
                               ("embed16", "F16", (rows, cols), e16.tobytes()),
                               ("emb_bf16", "BF16", (rows, cols), (emb.view(np.uint32) >> 16).astype(np.uint16).tobytes())])
    with mnb_hip.Pack(st) as pk:
        for name, ref in (("model.embed_tokens.weight", emb), ("embed16", e16_ref)):
            w = pk.quantize(ctx, name, rows, cols)
            try:
                bs = orc.choose_tied_block_size(cols)
                assert (w.N, w.K, w.block_size) == (rows, cols, bs)
                q, s, z = w.read()
                rq, rs, rz = orc.quantize_rows_u4(ref, rows, cols, bs)
                assert np.array_equal(q, rq) and np.array_equal(s.view(np.uint32), rs.view(np.uint32)), name
                assert np.array_equal(z, rz), name
            finally:
                w.close()
        with pytest.raises(mnb_hip.IOException, match=r"Unsupported inline tensor data for emb_bf16: BFLOAT16 \(16\)"):
            pk.quantize(ctx, "emb_bf16", rows, cols)
        with pytest.raises(mnb_hip.IOException,
                           match=r"Unexpected dimensions for embed16: \[300, 896\], expected \[151936, 896\]"):
            pk.quantize(ctx, "embed16", 151936, cols)
        with pytest.raises(mnb_hip.IOException, match="Tensor not found: lm_head"):
            pk.quantize(ctx, "lm_head", rows, cols)
    # an ONNX model with the embedding as an external FLOAT16 initializer
    b = wf.OnnxBuilder()
    b.tensor("model.embed_tokens.weight", 10, [rows, cols], e16.tobytes(), external=True)
    d = tmp_path / "onnx"
    d.mkdir()
    with mnb_hip.Pack(b.write(str(d))) as pk:
        w = pk.quantize(ctx, "model.embed_tokens.weight", rows, cols, 64)
        try:
            q, s, z = w.read()
            rq, rs, rz = orc.quantize_rows_u4(e16_ref, rows, cols, 64)
            assert np.array_equal(q, rq) and np.array_equal(s.view(np.uint32), rs.view(np.uint32))
            assert np.array_equal(z, rz)
        finally:
            w.close()
