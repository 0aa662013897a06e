"""GPU parity of libmnb_hip against the oracle, through the C ABI.

Bars (stated per test):
* dequantize: bit-exact to the reference's dequantizeInt4 (fp32), and fp16
  output = round-to-nearest-even of that fp32 value.
* matmul: |y - y_oracle| <= 1e-3 * sqrt(K) * max|x| * max|w| (K = true K),
  plus one fp16 ulp of |y_oracle| when the output is fp16.
* full-size shapes: the oracle on sampled output rows, and properties that
  hold bit-for-bit (power-of-two scaling, row independence of the skinny
  kernel, run-to-run determinism of the GEMM and the K-sliced kernel).
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

import mnb_hip
from mnb_hip import synth
import mnb_oracle as orc
from parity_util import (THREADS, assert_parity, fp16_ulp, max_abs_w, oracle_inputs, oracle_matmul, say,
                         upload)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    orc.build()
    c = mnb_hip.Context(0)
    i = c.info()
    say("device:", i.name.decode(), i.arch.decode(), "CUs", i.compute_units)
    yield c
    c.close()


# ------------------------------------------------------------ dequant -----

def test_dequant_bit_exact_on_golden_fixtures(ctx, golden_dir):
    d = np.load(os.path.join(golden_dir, "dequant_exact.npz"), allow_pickle=False)
    names = sorted({k.split("__")[0] for k in d.files})
    done = 0
    for n in names:
        N, K, bs = (int(v) for v in d[n + "__shape"])
        if bs < 16:
            continue    # MatMulNBits block sizes start at 16
        say("dequant golden", n)
        w_exp = d[n + "__w"]
        variants = [d[n + "__scales"]]
        if d[n + "__scales_f16"].size:
            variants.append(d[n + "__scales_f16"].view(np.float16))
        for s in variants:
            w = mnb_hip.Weight(ctx, N, K, bs, d[n + "__q"], s, d[n + "__zp"], mnb_hip.MNB_ZP_FLAT)
            got = w.dequantize(np.float32)
            assert np.array_equal(got.view(np.uint32), w_exp.view(np.uint32)), n
            got16 = w.dequantize(np.float16)
            assert np.array_equal(got16.view(np.uint16), w_exp.astype(np.float16).view(np.uint16)), n
            w.close()
            done += 1
    assert done >= 8


@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("K,N", synth.SMOL_SHAPES)
def test_dequant_config4_bit_exact(ctx, bs, K, N):
    say("dequant config4", K, N, bs)
    t = synth.make_weight(1000 + bs + K, N, K, bs, with_zp=True)
    q, s, z, n = oracle_inputs(t)
    kpad = t.kb * bs
    ref = orc.dequantize(q, s, z, n, kpad, bs)[:, :K]
    w = upload(ctx, t)
    got = w.dequantize(np.float32)
    assert np.array_equal(got.view(np.uint32), np.ascontiguousarray(ref).view(np.uint32))
    got16 = w.dequantize(np.float16)
    assert np.array_equal(got16.view(np.uint16), ref.astype(np.float16).view(np.uint16))
    w.close()


def test_dequant_reference_loader_subnormal_scales(ctx):
    """fp16 subnormal scales widened by the reference loader (m * 2^-150) and
    passed as fp32 must dequantize bit-exactly like the reference."""
    rng = np.random.default_rng(9)
    N, K, bs = 32, 256, 32
    q = rng.integers(0, 256, N * K // 2, dtype=np.uint8)
    bits = rng.integers(1, 0x400, N * K // bs).astype(np.uint16)          # subnormal fp16 patterns
    bits[::3] = rng.integers(0x0400, 0x7C00, bits[::3].size).astype(np.uint16)  # and normals
    s_ref = orc.fp16_bits_to_fp32(bits)
    z = orc.zp_pack_unpacked_u8(rng.integers(0, 16, N * K // bs), N, K // bs)
    ref = orc.dequantize(q, s_ref, z, N, K, bs)
    w = mnb_hip.Weight(ctx, N, K, bs, q, s_ref, z, mnb_hip.MNB_ZP_FLAT)
    assert np.array_equal(w.dequantize(np.float32).view(np.uint32), ref.view(np.uint32))
    w.close()


# ------------------------------------------------------------- matmul -----

def test_closed_form_kats(ctx, golden_dir):
    import json
    kat = json.load(open(os.path.join(golden_dir, "kat_closed_form.json")))
    for c in kat["matvec"]:
        say("kat", c["name"])
        N, K = c["N"], 128
        q = np.full(N * K // 2, (c["nibble"] & 0xF) * 0x11, np.uint8)
        s = np.full(N, c["scale"], np.float32)
        z = np.full((N + 1) // 2, (c["zp"] & 0xF) * 0x11, np.uint8)
        k = mnb_hip.MatMulNBitsKernel(ctx, N, K, q, s, z, 128)
        qm = mnb_hip.QuantizedWeightMatrix(k)
        y = np.array(c["y_init"], np.float32)
        qm.matvec(np.full(K, c["x"], np.float32), y)
        assert np.allclose(y, c["expected"], atol=c["atol"], rtol=0), c["name"]
        k.close()


def test_config0_decode_gemv(ctx):
    """M=1, K=3072, N=9216, bs=32, implicit zero point 8 (Phi-3 fused QKV)."""
    t = synth.make_weight(0, 9216, 3072, 32)
    x16 = synth.make_x(1, 1, 3072)
    y_ref, wmax = oracle_matmul(t, x16)
    w = upload(ctx, t)
    for out_dt in (np.float16, np.float32):
        y = w.matmul(x16, out_dtype=out_dt)
        assert_parity(y, y_ref, x16, t, wmax, out_dt == np.float16, "cfg0 out=%s" % np.dtype(out_dt).name)
    # the Java float[] contract: fp32 in, fp32 out
    y = w.matmul(x16.astype(np.float32), out_dtype=np.float32)
    assert_parity(y, y_ref, x16, t, wmax, False, "cfg0 f32->f32")
    w.close()


@pytest.mark.parametrize("M", [1, 7, 33])
@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("K,N", synth.SMOL_SHAPES)
def test_config4_asymmetric_tails(ctx, M, bs, K, N):
    say("config4", M, bs, K, N)
    t = synth.make_weight(2000 + M + bs + K, N, K, bs, with_zp=True)
    x16 = synth.make_x(3000 + M, M, K)
    y_ref, wmax = oracle_matmul(t, x16)
    w = upload(ctx, t)
    y = w.matmul(x16, out_dtype=np.float16)
    assert_parity(y, y_ref, x16, t, wmax, True, "cfg4 M=%d bs=%d K=%d N=%d" % (M, bs, K, N))
    w.close()


@pytest.mark.parametrize("M", [2, 3, 4, 6, 8, 9, 12, 16])
def test_multi_row_products_by_row_group(ctx, M):
    """Single products with 1 < M <= 16 load the x rows in XR groups of four
    (XR = 1 up to M = 4, 2 up to 8, 4 above) and MFMA row m reads x row
    m * XR / 4, so with M <= 4 a lane keeps one sum per output row, with
    M <= 8 two; rows past M repeat row M - 1 and are not stored.  Shapes:
    whole super-tiles, a K tail with zero points and fp32 scales, and
    K = 8192, where 12 waves loop over 32 K chunks."""
    cases = [(3072, 200, 32, False, False), (1000, 130, 128, True, True), (8192, 48, 64, False, False)]
    for ci, (K, N, bs, zp, f32) in enumerate(cases):
        t = synth.make_weight(6100 + 10 * M + ci, N, K, bs, with_zp=zp)
        x16 = synth.make_x(6200 + 10 * M + ci, M, K)
        y_ref, wmax = oracle_matmul(t, x16)
        w = upload(ctx, t, as_f32_scales=f32)
        label = "rows M=%d K=%d N=%d bs=%d zp=%d f32=%d" % (M, K, N, bs, zp, f32)
        say(label)
        y32 = w.matmul(x16)
        assert_parity(y32, y_ref, x16, t, wmax, False, label)
        y16 = w.matmul(x16, out_dtype=np.float16)
        assert np.array_equal(y16.view(np.uint16), y32.astype(np.float16).view(np.uint16)), label
        y0 = np.random.default_rng(M + ci).standard_normal((M, N)).astype(np.float32)
        acc = w.matmul(x16, y=y0.copy(), accumulate=True)
        assert np.array_equal(acc.view(np.uint32), (y0 + y32).view(np.uint32)), label
        w.close()


@pytest.mark.parametrize("bs", [16, 256])
def test_block_sizes_16_and_256(ctx, bs):
    t = synth.make_weight(77 + bs, 200, 1024, bs, with_zp=True)
    for M in (1, 3, 5, 40):
        x16 = synth.make_x(78 + M, M, 1024)
        y_ref, wmax = oracle_matmul(t, x16)
        w = upload(ctx, t)
        assert_parity(w.matmul(x16), y_ref, x16, t, wmax, False, "bs=%d M=%d" % (bs, M))
        w.close()


@pytest.mark.parametrize("M", [1, 64])
def test_config3_qwen_shapes(ctx, M):
    for li, (name, K, N) in enumerate(synth.QWEN_LAYER + [synth.QWEN_LM_HEAD]):
        say("config3", name, M)
        t = synth.make_weight(4000 + li, N, K, 32)
        x16 = synth.make_x(5000 + li + M, M, K)
        rows = None
        if N * M > 2_000_000:
            rows = np.random.default_rng(li).choice(N, 2048, replace=False)
            rows.sort()
        y_ref, _ = oracle_matmul(t, x16, rows)
        w = upload(ctx, t)
        y = w.matmul(x16, out_dtype=np.float16)
        ys = y if rows is None else y[:, rows] if y.ndim == 2 else y[rows]
        assert_parity(ys, y_ref.reshape(ys.shape), x16, t, None, True, "cfg3 %s M=%d" % (name, M))
        w.close()


@pytest.mark.parametrize("M", [16, 128, 512, 2048])
def test_config2_phi3_prefill_sampled_rows(ctx, M):
    for li, (name, K, N) in enumerate(synth.PHI3_LAYER):
        say("config2", name, M)
        t = synth.make_weight(6000 + li, N, K, 32)
        x16 = synth.make_x(7000 + li + M, M, K)
        nrow = max(64, min(N, 16_000_000 // (M * K) * 4))
        rows = np.sort(np.random.default_rng(M + li).choice(N, min(N, nrow), replace=False))
        y_ref, _ = oracle_matmul(t, x16, rows)
        w = upload(ctx, t)
        y = w.matmul(x16, out_dtype=np.float16)
        assert_parity(y[:, rows], y_ref, x16, t, None, True, "cfg2 %s M=%d" % (name, M))
        w.close()


# ------------------------------------------------ bitwise properties ------

def test_rows_are_independent_in_skinny_kernel(ctx):
    """On the GEMV a row's result does not depend on M (rows of an M = 16
    product equal M = 1 products bit for bit).  A wide product at M = 16 runs
    on 16 x 64 K-sliced blocks instead, whose K slices are summed in another
    order: its rows match the M = 1 products to the tolerance, and repeated
    calls are bitwise identical."""
    t = synth.make_weight(11, 3072, 3072, 32)
    w = upload(ctx, t)
    assert w.plan(16).kernel == mnb_hip.MNB_KERNEL_GEMV, w.plan(16).as_tuple()
    x16 = synth.make_x(12, 16, 3072)
    y16 = w.matmul(x16)
    for m in (0, 5, 15):
        y1 = w.matmul(x16[m])
        assert np.array_equal(y1.view(np.uint32), y16[m].view(np.uint32)), m
    w.close()
    t = synth.make_weight(16, 9216, 3072, 32)
    w = upload(ctx, t)
    assert w.plan(16).as_tuple() == (KSLICE, NO_ORDER, 16, 64), w.plan(16).as_tuple()
    y16 = w.matmul(x16)
    assert np.array_equal(w.matmul(x16).view(np.uint32), y16.view(np.uint32))
    tol = orc.tolerance(3072, x16.astype(np.float32), w.dequantize(np.float32))
    for m in (0, 5, 15):
        assert np.abs(w.matmul(x16[m]) - y16[m]).max() <= tol, m
    w.close()


def test_gemm_determinism_tiling_and_pow2_scaling(ctx):
    """The schedule, and for single products the kernel, depend on M, so a
    row's summation order depends on M: rows of an M=512 product (the GEMM)
    match an M=128 product of the same rows (the K-sliced kernel) to the
    tolerance, and repeated calls with the same M are bitwise identical
    (nothing is summed in an order that depends on timing)."""
    t = synth.make_weight(13, 9216, 3072, 32)
    w = upload(ctx, t)
    assert w.plan(512).kernel == GEMM and w.plan(128).kernel == KSLICE, (w.plan(512).as_tuple(), w.plan(128).as_tuple())
    x16 = synth.make_x(14, 512, 3072)
    y = w.matmul(x16)
    for _ in range(3):
        assert np.array_equal(w.matmul(x16).view(np.uint32), y.view(np.uint32))
    y_part = w.matmul(np.ascontiguousarray(x16[128:256]))
    tol = orc.tolerance(3072, x16.astype(np.float32),
                        w.dequantize(np.float32))
    assert np.abs(y[128:256] - y_part).max() <= tol
    y2 = w.matmul((x16.astype(np.float32) * 2).astype(np.float16))
    assert np.array_equal(y2.view(np.uint32), (y * 2).view(np.uint32))
    x1 = synth.make_x(15, 1, 3072)
    g1 = w.matmul(x1[0])
    g2 = w.matmul((x1[0].astype(np.float32) * 4).astype(np.float16))
    assert np.array_equal(g2.view(np.uint32), (g1 * 4).view(np.uint32))
    w.close()


def test_tall_single_row_product(ctx):
    """A tall M = 1 product (4376 n-tiles, more than the chip holds waves):
    N = 70001 leaves a partial last n-tile, K = 1000 a k tail inside a
    super-tile; zero points, fp16 and fp32 outputs, y += and row 0 of an M = 2
    product (the 16-row kernel variant) all agree."""
    N, K = 70001, 1000
    t = synth.make_weight(61, N, K, 32, with_zp=True)
    w = upload(ctx, t)
    try:
        x2 = synth.make_x(62, 2, K)
        x16 = np.ascontiguousarray(x2[:1])
        y_ref, _ = oracle_matmul(t, x16)
        y32 = w.matmul(x16[0])
        assert_parity(y32.reshape(1, N), y_ref, x16, t, None, False, "tall M=1")
        y16 = w.matmul(x16[0], out_dtype=np.float16)
        assert np.array_equal(y16.view(np.uint16), y32.astype(np.float16).view(np.uint16))
        y0 = np.random.default_rng(63).standard_normal(N).astype(np.float32)
        acc = w.matmul(x16[0], y=y0.copy(), accumulate=True)
        assert np.array_equal(acc.view(np.uint32), (y0 + y32).view(np.uint32))
        y_pair = w.matmul(x2)
        tol = 1e-3 * np.sqrt(K) * float(np.abs(x16.astype(np.float32)).max()) * max_abs_w(t)
        assert float(np.abs(y_pair[0] - y32).max()) <= tol
    finally:
        w.close()


@pytest.mark.parametrize("M,K,N", [(200, 8192, 9001), (250, 6144, 7001), (150, 8192, 10001)])
def test_gemm_split_tiles_tails_and_outputs(ctx, M, K, N):
    """Few 128 x 256 tiles for their K, so stream-K splits them across
    workgroups and the partial tiles go through the reduce kernel (shapes
    where the GEMM beats the K-sliced kernel).  M and N tails (N % 4 != 0
    falls back to per-element stores), fp16 and fp32 outputs, y += and a y
    that is not aligned for 4-element stores: within the tolerance of the
    oracle on sampled columns, bitwise repeatable, and y += equal to y0 + y."""
    import torch
    t = synth.make_weight(50 + M, N, K, 32, with_zp=True)
    w = upload(ctx, t)
    assert w.plan(M).as_tuple() == (GEMM, STREAM_K, 128, 256), w.plan(M).as_tuple()
    x16 = synth.make_x(51 + M, M, K)
    rng = np.random.default_rng(M + N)
    cols = np.sort(np.concatenate([rng.choice(N - 16, 240, replace=False), np.arange(N - 16, N)]))
    y_ref, _ = oracle_matmul(t, x16, cols, want_wmax=False)
    y32 = w.matmul(x16)
    assert_parity(y32[:, cols], y_ref, x16, t, None, False, "split f32 M=%d K=%d N=%d" % (M, K, N))
    assert np.array_equal(w.matmul(x16).view(np.uint32), y32.view(np.uint32))
    y16 = w.matmul(x16, out_dtype=np.float16)
    assert np.array_equal(y16.view(np.uint16), y32.astype(np.float16).view(np.uint16))
    y0 = np.random.default_rng(M).standard_normal((M, N)).astype(np.float32)
    acc = w.matmul(x16, y=y0.copy(), accumulate=True)
    assert np.array_equal(acc.view(np.uint32), (y0 + y32).view(np.uint32))
    # device output one element past an aligned address: per-element stores
    xd = torch.from_numpy(x16).cuda()
    buf = torch.zeros(M * N + 1, dtype=torch.float32, device="cuda")
    yd = buf[1:]
    w.matmul(xd, yd)
    torch.cuda.synchronize()
    assert np.array_equal(yd.cpu().numpy().reshape(M, N).view(np.uint32), y32.view(np.uint32))
    assert float(buf[0].item()) == 0.0
    w.close()


@pytest.mark.parametrize("case", [
    # M, K, N, bs, zero points, fp32 scales (not fp16-exact), output block
    (40, 1000, 300, 32, True, False, (32, 16)),
    (17, 3000, 1001, 32, False, True, (32, 16)),
    (129, 576, 1000, 64, True, False, (32, 32)),
    (48, 1536, 4000, 16, False, False, (32, 32)),
    (300, 4096, 1001, 128, True, False, (32, 64)),
    (130, 8192, 3072, 32, False, False, (32, 64)),
    (64, 3072, 9216, 32, False, False, (64, 64)),
    (250, 3072, 3070, 32, True, False, (64, 64)),
    # 9 <= M <= 16 with wide N: 16 x 64 blocks instead of the GEMV
    (16, 3072, 16384, 32, False, False, (16, 64)),
    (13, 2500, 16000, 64, True, False, (16, 64)),
    (14, 1500, 30000, 16, False, False, (16, 64)),
    (9, 3001, 20000, 128, True, False, (16, 64)),
    (11, 3000, 16001, 32, False, True, (16, 64)),
    # fp32 scales with zero points (the tied head's quantizer and subnormal
    # fp16 scales give such weights) at bs 16, 32 and 64
    (40, 1024, 600, 16, True, True, (32, 16)),
    (33, 1000, 300, 32, True, True, (32, 16)),
    (60, 3000, 2000, 64, True, True, (32, 16)),
    (48, 1536, 4000, 16, True, True, (32, 32))],
    ids=lambda c: "M%d-K%d-N%d-bs%d%s%s" % (c[0], c[1], c[2], c[3], "-zp" if c[4] else "", "-f32s" if c[5] else ""))
def test_single_products_k_sliced(ctx, case):
    """Single products where the GEMM would have few tiles run on the
    K-sliced kernel (workgroup = 16 MB rows x 16 NTW columns over the whole K,
    its waves' K slices summed in LDS in wave order): each of its four output
    blocks (and the 16-row block that replaces the GEMV for 9 <= M <= 16 with
    wide N), M, N and K tails (rows past M, n-tiles past N, a partial last
    super-tile, K % 8 != 0), zero points, bs 16 to 128, fp32 scales, fp16 and fp32
    outputs, y +=, a y not aligned for 4-column stores.  Within the tolerance
    of the oracle, bitwise repeatable, fp16 output = fp32 output rounded, and
    y += equal to y0 + y."""
    import torch
    M, K, N, bs, zp, f32s, block = case
    t = synth.make_weight(9100 + M + N, N, K, bs, with_zp=zp)
    s = None
    if f32s:    # scales that fp16 cannot hold: the device keeps fp32 scales
        s = t.scales_f16.astype(np.float32) * np.float32(1.0 + 2.0 ** -14)
        if zp:
            w = mnb_hip.Weight(ctx, N, K, bs, t.q, s, t.zp_row_padded, mnb_hip.MNB_ZP_ROW_PADDED)
        else:
            w = mnb_hip.Weight(ctx, N, K, bs, t.q, s)
    else:
        w = upload(ctx, t)
    try:
        p = w.plan(M)
        if f32s and not zp:
            assert p.kernel == KSLICE, p.as_tuple()
        else:
            assert p.as_tuple() == (KSLICE, NO_ORDER) + block, p.as_tuple()
        x16 = synth.make_x(9200 + M, M, K)
        y_ref, wmax = oracle_matmul(t, x16, scales=s)
        label = "k-sliced M=%d K=%d N=%d bs=%d" % (M, K, N, bs)
        y32 = w.matmul(x16)
        assert_parity(y32, y_ref, x16, t, wmax, False, label)
        assert np.array_equal(w.matmul(x16).view(np.uint32), y32.view(np.uint32))
        y16 = w.matmul(x16, out_dtype=np.float16)
        assert np.array_equal(y16.view(np.uint16), y32.astype(np.float16).view(np.uint16))
        y0 = np.random.default_rng(M + K).standard_normal((M, N)).astype(np.float32)
        acc = w.matmul(x16, y=y0.copy(), accumulate=True)
        assert np.array_equal(acc.view(np.uint32), (y0 + y32).view(np.uint32))
        # device output one element past an aligned address: per-element stores
        xd = torch.from_numpy(x16).cuda()
        buf = torch.zeros(M * N + 1, dtype=torch.float32, device="cuda")
        yd = buf[1:]
        w.matmul(xd, yd)
        torch.cuda.synchronize()
        assert np.array_equal(yd.cpu().numpy().reshape(M, N).view(np.uint32), y32.view(np.uint32))
        assert float(buf[0].item()) == 0.0
    finally:
        w.close()


def test_accumulate_and_dtypes_and_zp_layouts(ctx):
    t = synth.make_weight(21, 1536, 576, 64, with_zp=True)
    w_rp = upload(ctx, t)
    q, s, z, n = oracle_inputs(t)
    w_flat = mnb_hip.Weight(ctx, t.N, t.K, t.bs, t.q, t.scales_f16, z, mnb_hip.MNB_ZP_FLAT)
    for M in (1, 33):
        x16 = synth.make_x(22 + M, M, 576)
        a = w_rp.matmul(x16)
        b = w_flat.matmul(x16)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        c = w_rp.matmul(x16.astype(np.float32))        # fp32 activations are rounded to fp16 first
        assert np.array_equal(a.view(np.uint32), c.view(np.uint32))
        y0 = np.random.default_rng(M).standard_normal(a.shape).astype(np.float32)
        acc = w_rp.matmul(x16, y=y0.copy(), accumulate=True)
        assert np.array_equal(acc.view(np.uint32), (y0 + a).view(np.uint32))
    w_rp.close()
    w_flat.close()


def test_fp32_scales_not_fp16_exact(ctx):
    """Scales from the tied-lm_head quantizer are arbitrary fp32 values."""
    rng = np.random.default_rng(31)
    rows, cols, bs = 300, 896, 128
    dense = rng.standard_normal((rows, cols)).astype(np.float32) * 0.05
    q, s, z = orc.quantize_rows_u4(dense, rows, cols, bs)
    w = mnb_hip.Weight(ctx, rows, cols, bs, q, s, z, mnb_hip.MNB_ZP_FLAT)
    ref_w = orc.dequantize(q, s, z, rows, cols, bs)
    assert np.array_equal(w.dequantize(np.float32).view(np.uint32), ref_w.view(np.uint32))
    for M in (1, 64):
        x16 = synth.make_x(32 + M, M, cols)
        y_ref = orc.matmul(q, s, z, rows, cols, bs, x16.astype(np.float32), threads=THREADS)
        tol = 1e-3 * np.sqrt(cols) * float(np.max(np.abs(x16.astype(np.float32)))) * float(np.max(np.abs(ref_w)))
        err = float(np.max(np.abs(w.matmul(x16) - y_ref)))
        say("fp32 scales M=%d max|err|=%.3e tol=%.3e" % (M, err, tol))
        assert err <= tol
    w.close()


def test_device_pointers_match_host_path(ctx):
    import torch
    t = synth.make_weight(41, 9216, 3072, 32)
    w = upload(ctx, t)
    for M in (1, 64):
        x16 = synth.make_x(42 + M, M, 3072)
        host = w.matmul(x16, out_dtype=np.float16)
        st = torch.cuda.Stream()
        with torch.cuda.stream(st):
            xd = torch.from_numpy(x16).cuda()
            yd = torch.empty((M, t.N), dtype=torch.float16, device="cuda")
            w.matmul(xd, yd, stream=st.cuda_stream)
        torch.cuda.synchronize()
        assert np.array_equal(yd.cpu().numpy().view(np.uint16), host.view(np.uint16))
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        wd = torch.empty((t.N, t.K), dtype=torch.float16, device="cuda")
        w.dequantize(out=wd, stream=st.cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(wd.cpu().numpy().view(np.uint16), w.dequantize(np.float16).view(np.uint16))
    w.close()


# ---------------------------------------------------------- contract ------

def test_cpp_mirror_contract():
    """The C++ MatMulNBitsKernel mirror runs the reference's matvec KATs."""
    assert os.path.exists(mnb_hip.CONTRACT_TEST_PATH), "contract test not built"
    r = subprocess.run([mnb_hip.CONTRACT_TEST_PATH], capture_output=True, text=True, timeout=120)
    say(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


def test_error_paths(ctx):
    t = synth.make_weight(51, 64, 256, 32)
    k = mnb_hip.MatMulNBitsKernel(ctx, 64, 256, t.q, t.scales_f16.astype(np.float32), None, 32)
    with pytest.raises(mnb_hip.IllegalArgumentException, match="Input length 255 != K=256"):
        k.matvec(np.zeros(255, np.float32))
    with pytest.raises(mnb_hip.IllegalArgumentException):
        k.matmulBatch(np.zeros(256 * 2, np.float32), np.zeros(64, np.float32), 2)
    with pytest.raises(mnb_hip.IllegalArgumentException):
        mnb_hip.Weight(ctx, 64, 256, 48, t.q, t.scales_f16)      # block size not a power of two
    with pytest.raises(mnb_hip.IllegalArgumentException):
        mnb_hip.Weight(ctx, 64, 256, 32, t.q[:100], t.scales_f16)
    k.close()
    with pytest.raises(mnb_hip.IllegalStateException, match="Kernel not prepared"):
        k.matvec(np.zeros(256, np.float32))
    os.environ["MNB_FAULT_INJECT"] = "alloc"
    try:
        with pytest.raises(mnb_hip.MnbError) as ei:
            mnb_hip.Weight(ctx, 64, 256, 32, t.q, t.scales_f16)
        assert ei.value.code == mnb_hip.MNB_ERR_OUT_OF_MEMORY
    finally:
        del os.environ["MNB_FAULT_INJECT"]
    w = mnb_hip.Weight(ctx, 64, 256, 32, t.q, t.scales_f16)     # recovers after the injected failure
    # a weight of another context: the plan query refuses it like the product does
    ctx2 = mnb_hip.Context(0)
    try:
        info = mnb_hip.PlanInfo()
        rc = mnb_hip.load().mnb_matmul_plan(ctx2.handle, w.handle, 40, ctypes.byref(info))
        assert rc == mnb_hip.MNB_ERR_INVALID_ARGUMENT and "another context" in mnb_hip.last_error(), rc
    finally:
        ctx2.close()
    w.close()


def test_group_matches_oracle_and_single_launches(ctx):
    """Independent products recorded as one group launch."""
    import torch
    shapes = [(3072, 9216), (3072, 3072), (8192, 3072), (896, 1152), (3072, 3072)]
    entries, host = [], []
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        for i, (K, N) in enumerate(shapes):
            t = synth.make_weight(900 + i, N, K, 32)
            w = upload(ctx, t)
            x16 = synth.make_x(950 + i, 1, K)
            xd = torch.from_numpy(x16).cuda()
            yd = torch.empty((1, N), dtype=torch.float16, device="cuda")
            entries.append((w, xd, yd))
            host.append((t, x16))
    torch.cuda.synchronize()
    g = mnb_hip.Group(ctx, entries)
    assert g.plan().kernel == mnb_hip.MNB_KERNEL_STREAM and g.plan().order == mnb_hip.MNB_ORDER_NONE
    for rep in range(3):     # replays overwrite the same outputs
        g.run(st.cuda_stream)
        torch.cuda.synchronize()
        for (w, xd, yd), (t, x16) in zip(entries, host):
            rows = np.sort(np.random.default_rng(t.N).choice(t.N, min(t.N, 512), replace=False))
            y_ref, _ = oracle_matmul(t, x16, rows)
            y = yd.cpu().numpy()
            assert_parity(y[:, rows], y_ref, x16, t, None, True, "group K=%d N=%d rep=%d" % (t.K, t.N, rep))
            single = w.matmul(x16, out_dtype=np.float16)
            assert np.max(np.abs(single.astype(np.float32) - y.astype(np.float32))) <= 2 * fp16_ulp(
                np.abs(single.astype(np.float32)).max())
    g.close()
    with pytest.raises(mnb_hip.MnbError):       # mixed M classes are refused
        mnb_hip.Group(ctx, [entries[0], (entries[1][0], torch.zeros((2, 3072), dtype=torch.float16,
                                                                    device="cuda"),
                                         torch.zeros((2, 3072), dtype=torch.float16, device="cuda"))])
    for w, _, _ in entries:
        w.close()


GEMM, GEMV_GROUP, KSLICE = mnb_hip.MNB_KERNEL_GEMM, mnb_hip.MNB_KERNEL_GEMV_GROUP, mnb_hip.MNB_KERNEL_KSLICE
STREAM = mnb_hip.MNB_KERNEL_STREAM
STREAM_K, TILE_LIST, NO_ORDER = mnb_hip.MNB_ORDER_STREAM_K, mnb_hip.MNB_ORDER_TILE_LIST, mnb_hip.MNB_ORDER_NONE
PARTS = mnb_hip.MNB_ORDER_TILE_LIST_PARTS


def _check_prefill_group(ctx, specs, seed, bs=32, plan=None, f32_scales=False):
    """Records the products `specs` (M, K, N, y dtype, y +=) as groups (one
    per accumulate flag) and checks every item against the oracle on sampled
    rows and against its own single launch, with replays bitwise identical.
    `plan` (kernel, order, tile rows, tile columns) is the schedule every
    group must have recorded (mnb_group_plan); `f32_scales` uploads the
    scales as fp32 (the same values)."""
    import torch
    entries, host = [], []
    st = torch.cuda.Stream()
    for i, (M, K, N, ydt, acc) in enumerate(specs):
        t = synth.make_weight(seed + i, N, K, bs, with_zp=True)
        w = upload(ctx, t, as_f32_scales=f32_scales)
        x16 = synth.make_x(seed + 100 + i, M, K)
        y0 = np.random.default_rng(seed + 200 + i).standard_normal((M, N)).astype(ydt)
        entries.append((w, torch.from_numpy(x16).cuda(), torch.from_numpy(y0.copy()).cuda()))
        host.append((t, x16, y0, acc))
    torch.cuda.synchronize()
    for acc_group in (False, True):
        items = [e for e, h in zip(entries, host) if h[3] == acc_group]
        if not items:
            continue
        g = mnb_hip.Group(ctx, items, accumulate=acc_group)
        if plan is not None:
            assert g.plan().as_tuple() == plan, (g.plan().as_tuple(), plan)
        outs = []
        for rep in range(3):
            with torch.cuda.stream(st):
                for (w, xd, yd), (t, x16, y0, acc) in zip(entries, host):
                    if acc == acc_group:
                        yd.copy_(torch.from_numpy(y0).cuda())
                g.run(st.cuda_stream)
            torch.cuda.synchronize()
            outs.append([yd.cpu().numpy().copy() for (w, xd, yd) in items])
        for r in outs[1:]:
            for a, b in zip(outs[0], r):
                assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
        hs = [h for h in host if h[3] == acc_group]
        for (w, xd, yd), (t, x16, y0, acc), y in zip(items, hs, outs[0]):
            rows = np.sort(np.random.default_rng(t.N).choice(t.N, min(t.N, 512), replace=False))
            y_ref, _ = oracle_matmul(t, x16, rows)
            base = y0.astype(np.float32)[:, rows] if acc else 0.0
            label = "group M=%d K=%d N=%d acc=%d" % (x16.shape[0], t.K, t.N, acc)
            assert_parity(y.astype(np.float32)[:, rows] - base, y_ref, x16, t, None, y.dtype == np.float16, label)
            single = w.matmul(x16, y=y0.astype(np.float32).copy() if acc else None, accumulate=acc)
            tol = 1e-3 * np.sqrt(t.K) * float(np.abs(x16.astype(np.float32)).max()) * max_abs_w(t)
            err = np.abs(single - y.astype(np.float32))
            assert float(np.max(err - (fp16_ulp(single) if y.dtype == np.float16 else 0.0))) <= tol, label
        g.close()
    return entries


def test_group_of_prefill_products(ctx):
    """Independent products with M > 16 recorded as one group, few tiles: one
    stream-K launch whose workgroup ranges run across item boundaries
    (different K, so different stage counts per tile; M and N tails; fp16 and
    fp32 outputs; y +=)."""
    import torch
    specs = [(200, 3072, 1000, np.float16, False), (64, 8192, 3072, np.float32, False),
             (512, 3072, 9216, np.float16, False), (33, 1536, 577, np.float32, True),
             (300, 576, 1536, np.float16, False)]
    entries = _check_prefill_group(ctx, specs, 1200, plan=(GEMM, STREAM_K, 128, 256))
    with pytest.raises(mnb_hip.MnbError):       # M <= 16 and M > 16 do not mix
        mnb_hip.Group(ctx, [entries[0], (entries[1][0], torch.zeros((2, 8192), dtype=torch.float16, device="cuda"),
                                         torch.zeros((2, 3072), dtype=torch.float32, device="cuda"))])
    for w, _, _ in entries:
        w.close()


def test_group_of_prefill_products_in_tile_list_order(ctx):
    """A group with 1142 output tiles (more than four per workgroup on a
    256-CU device) runs in tile-list order: whole tiles per workgroup, blocks
    of tiles that share x rows and weight columns side by side on one XCD.
    Items cover one to 36 m-tiles, k tails (K = 200, 576), N tails and fp16
    and fp32 outputs; no tile is longer than a workgroup's mean share, so
    none is cut into parts."""
    specs = [(512, 3072, 9216, np.float16, False), (700, 576, 8000, np.float32, False),
             (2048, 1536, 3072, np.float16, False), (300, 2048, 5000, np.float16, False),
             (4500, 256, 1100, np.float32, False), (129, 3072, 16384, np.float16, False),
             (64, 200, 30000, np.float16, False), (1024, 1024, 4096, np.float32, False)]
    tiles = sum(((M + 127) // 128) * ((N + 255) // 256) for M, K, N, _, _ in specs)
    assert tiles == 1142
    # at 512 columns the group has 589 tiles, fewer than four per workgroup:
    # it runs with 256-column tiles
    assert sum(((M + 127) // 128) * ((N + 511) // 512) for M, K, N, _, _ in specs) < 1024
    for w, _, _ in _check_prefill_group(ctx, specs, 1500, plan=(GEMM, TILE_LIST, 128, 256)):
        w.close()


def test_group_of_prefill_products_with_wide_tiles(ctx):
    """A group with 1243 tiles of 512 columns runs the 512-column kernel (8
    waves of 128 x 64) in tile-list order: more than 32 m-tiles (M = 4500),
    N tails inside a 512-column tile (N = 8000, 30000), k tails (K = 200,
    576), fp16 and fp32 outputs, zero points."""
    specs = [(2048, 1536, 16384, np.float16, False), (4500, 256, 8000, np.float32, False),
             (700, 576, 8000, np.float16, False), (64, 200, 30000, np.float16, False)]
    assert sum(((M + 127) // 128) * ((N + 511) // 512) for M, K, N, _, _ in specs) == 1243
    for w, _, _ in _check_prefill_group(ctx, specs, 1700, plan=(GEMM, TILE_LIST, 128, 512)):
        w.close()


@pytest.mark.parametrize("bs", [64, 128])
def test_group_with_wide_tiles_other_block_sizes(ctx, bs):
    """The 512-column kernel for 2 and 1 scales per 128-k stage (bs 64 and
    128, with zero points): 2096 tiles, whole and ragged."""
    specs = [(4500, 256, 16000, np.float16, False), (2048, 256, 30000, np.float16, False)]
    assert sum(((M + 127) // 128) * ((N + 511) // 512) for M, K, N, _, _ in specs) == 2096
    for w, _, _ in _check_prefill_group(ctx, specs, 2100 + bs, bs, plan=(GEMM, TILE_LIST, 128, 512)):
        w.close()


@pytest.mark.parametrize("seed", [0, 1])
def test_random_prefill_groups(ctx, seed):
    """Random groups of prefill products (17 <= M <= 2000, K a multiple of 8
    up to 1024, 1 <= N <= 24000, random output type) with at least 1100
    256-column tiles, so they run in tile-list order, with 256- or 512-column
    tiles as the schedule chooses."""
    rng = np.random.default_rng(4200 + seed)
    specs, tiles = [], 0
    ydt = [np.float16, np.float32][int(rng.integers(0, 2))]
    while tiles < 1100:
        M, K, N = int(rng.integers(17, 2001)), 8 * int(rng.integers(1, 129)), int(rng.integers(1, 24001))
        specs.append((M, K, N, ydt, False))
        tiles += ((M + 127) // 128) * ((N + 255) // 256)
    for w, _, _ in _check_prefill_group(ctx, specs, 4300 + 100 * seed):
        w.close()


@pytest.mark.parametrize("rows", [32, 64, 128])
@pytest.mark.parametrize("seed", [0, 1])
def test_random_groups_with_parts(ctx, rows, seed):
    """Random tile-list groups whose long items (K 4096 to 8192: 32 to 64
    stages) are cut into parts among many short tiles (K up to 512): M up to
    32, 33 to 64 or 65 to 600 (32 x 512, 64 x 512 or 128 x 256 tiles), N and
    M tails, fp16 or fp32 y; every item against the oracle and its own single
    launch, replays bitwise equal."""
    rng = np.random.default_rng(9100 + 10 * seed + rows)
    lo, hi = {32: (17, 32), 64: (33, 64), 128: (65, 600)}[rows]
    bn = 256 if rows == 128 else 512
    specs, tiles = [], 0
    while tiles < 1100:
        M, K, N = int(rng.integers(lo, hi + 1)), 8 * int(rng.integers(8, 65)), int(rng.integers(1000, 40001))
        specs.append((M, K, N, [np.float16, np.float32][int(rng.integers(0, 2))], False))
        tiles += ((M + rows - 1) // rows) * ((N + bn - 1) // bn)
    for _ in range(int(rng.integers(1, 4))):
        M, K, N = int(rng.integers(lo, hi + 1)), 8 * int(rng.integers(512, 1025)), int(rng.integers(256, 3001))
        specs.append((M, K, N, [np.float16, np.float32][int(rng.integers(0, 2))], False))
    say("random parts group", rows, seed, [sp[:3] for sp in specs])
    for w, _, _ in _check_prefill_group(ctx, specs, 9200 + 10 * seed + rows, plan=(GEMM, PARTS, rows, bn)):
        w.close()


@pytest.mark.parametrize("cls", ["m1", "rows2to4", "rows5to16"])
@pytest.mark.parametrize("seed", [0, 1])
def test_random_small_groups(ctx, cls, seed):
    """Random groups of M <= 16 products: all M = 1 (the streaming kernel),
    2 <= M <= 4 (the streaming kernel with the group's largest M rows of x
    per job) or 5 <= M <= 16 (the GEMV over every item's n-tiles, or 32-row
    GEMM tiles when there are many); 3 to 10 items, K a multiple of 8 up to
    4096, N up to 12000, one block size per group, fp16 or fp32 y, y += or
    not; every item against the oracle and its own single launch."""
    ci = {"m1": 0, "rows2to4": 1, "rows5to16": 2}[cls]
    rng = np.random.default_rng(7300 + 10 * seed + ci)
    lo, hi = [(1, 1), (2, 4), (5, 16)][ci]
    bs = int(rng.choice([16, 32, 64, 128, 256]))
    specs = []
    for _ in range(int(rng.integers(3, 11))):
        M, K, N = int(rng.integers(lo, hi + 1)), 8 * int(rng.integers(1, 513)), int(rng.integers(1, 12001))
        specs.append((M, K, N, [np.float16, np.float32][int(rng.integers(0, 2))], bool(rng.random() < 0.3)))
    say("random small group", cls, seed, "bs", bs, [sp[:3] for sp in specs])
    for w, _, _ in _check_prefill_group(ctx, specs, 7400 + 10 * seed + ci, bs=bs):
        w.close()


@pytest.mark.parametrize("ms", [(6, 3), (13, 2, 8), (8, 5)])
def test_small_groups_of_multi_row_products(ctx, ms):
    """Groups with 4 < M <= 16 (largest M of the group) and few 32 x 512
    tiles run one workgroup per n-tile of each item; the x row groups loaded
    follow the largest M of the group (two groups of four rows up to M = 8,
    four above), and items with fewer rows still drop their rows past M.  K
    tails, N tails, fp16 and fp32 outputs, and a group with y +=."""
    shapes = [(3072, 3072, np.float16), (1000, 500, np.float32), (8192, 700, np.float16)]
    specs = [(M, K, N, ydt, False) for M, (K, N, ydt) in zip(ms, shapes)]
    specs.append((ms[0], 2048, 300, np.float32, True))   # M > 4: the GEMV group kernel
    assert sum((N + 511) // 512 for M, K, N, _, _ in specs) < 1024
    for w, _, _ in _check_prefill_group(ctx, specs, 2500 + sum(ms), plan=(GEMV_GROUP, NO_ORDER, 0, 16)):
        w.close()


@pytest.mark.parametrize("bs", [16, 32, 128])
@pytest.mark.parametrize("ms", [(2, 2, 2), (3, 2, 3), (4, 3, 2)])
def test_small_batch_groups_on_the_streaming_kernel(ctx, bs, ms):
    """Groups whose items all have 2 <= M <= 4 rows (small-batch decode) run
    the persistent streaming kernel with as many x rows per job as the
    group's largest M (rows past an item's M re-read its last row and are
    never stored): zero points, bs 16
    (two scale blocks per 32-k step), 32 and 128 (one scale per super-tile),
    a K tail inside the last super-tile and one inside the last 4-super-tile
    job, N tails, fp16 and fp32 outputs, and a group with y +=; each item
    against the oracle and its own single launch, replays bitwise identical."""
    rows = max(ms)
    shapes = [(3072, 1000, np.float16), (1000, 130, np.float32), (8192, 700, np.float16)]
    specs = [(M, K, N, ydt, False) for M, (K, N, ydt) in zip(ms, shapes)]
    specs += [(ms[0], 896, 1152, np.float16, True), (ms[-1], 2048, 300, np.float32, True)]
    for w, _, _ in _check_prefill_group(ctx, specs, 2900 + bs + sum(ms), bs=bs, plan=(STREAM, NO_ORDER, rows, 16)):
        w.close()


@pytest.mark.parametrize("ms", [(1, 1), (3, 2)])
def test_group_with_an_item_of_more_than_65536_n_tiles(ctx, ms):
    """The streaming kernel codes an item's n-tile in 16 bits, so a group of
    M <= 4 products with an item of N > 1048576 (65537 n-tiles) runs on the
    GEMV group kernel instead of failing: each item against the oracle on
    sampled columns and against its own single
    launch."""
    specs = [(ms[0], 64, 1048592, np.float32, False), (ms[1], 1000, 300, np.float16, False)]
    for w, _, _ in _check_prefill_group(ctx, specs, 9700 + sum(ms), plan=(GEMV_GROUP, NO_ORDER, 0, 16)):
        w.close()


def test_small_batch_group_with_fp32_scales(ctx):
    """The streaming kernel with 4 x rows per job on weights whose scales
    fp16 cannot hold (the device keeps fp32 scales): items of M = 3 and 4
    against the oracle with those scales."""
    import torch
    items, checks = [], []
    for i, (M, K, N) in enumerate([(3, 3072, 777), (4, 1024, 2048)]):
        t = synth.make_weight(9500 + i, N, K, 32)
        s32 = t.scales_f16.astype(np.float32) * np.float32(1.0 + 2.0 ** -14)
        w = mnb_hip.Weight(ctx, N, K, 32, t.q, s32)
        x16 = synth.make_x(9510 + i, M, K)
        y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        items.append((w, torch.from_numpy(x16).cuda(), y))
        checks.append((t, s32, x16))
    g = mnb_hip.Group(ctx, items)
    try:
        assert g.plan().as_tuple() == (STREAM, NO_ORDER, 4, 16), g.plan().as_tuple()
        g.run()
        torch.cuda.synchronize()
        for (w, xd, y), (t, s32, x16) in zip(items, checks):
            kb = t.kb
            z = synth.zp_row_padded_to_flat(np.full((t.N, (kb + 1) // 2), 0x88, np.uint8), t.N, kb)
            xp = np.zeros((x16.shape[0], kb * 32), np.float32)
            xp[:, :t.K] = x16.astype(np.float32)
            y_ref = orc.matmul(t.q, s32, z, t.N, kb * 32, 32, xp, threads=THREADS)
            wmax = float(np.abs(s32).max()) * 8.0
            assert_parity(y.cpu().numpy(), y_ref, x16, t, wmax, False, "stream rows fp32 scales M=%d" % x16.shape[0])
    finally:
        g.close()
        for w, _, _ in items:
            w.close()


def test_group_of_products_with_64_row_tiles(ctx):
    """A large group with 32 < M <= 64 (1115 tiles of 64 x 512) runs on the
    GEMM kernel with 64-row tiles in tile-list order: M of 64, 33, 48 and 40
    (rows past M clamped and dropped), k tails (K = 200, 1000), N tails, fp16
    and fp32 outputs; each item is also checked against its own single
    launch (128-row tiles)."""
    specs = [(64, 256, 200000, np.float16, False), (33, 200, 150001, np.float32, False),
             (48, 1000, 120000, np.float16, False), (40, 64, 100000, np.float16, False)]
    assert sum((N + 511) // 512 for M, K, N, _, _ in specs) == 1115
    for w, _, _ in _check_prefill_group(ctx, specs, 2700, plan=(GEMM, TILE_LIST, 64, 512)):
        w.close()


def test_group_of_skinny_products_as_weight_stream(ctx):
    """A large group with 1 < M <= 16 (1115 tiles of 32 x 512) runs on the
    GEMM kernel with 32-row tiles in tile-list order: M of 2, 7, 9 and 16
    (rows past M clamped and dropped), k tails (K = 200, 1000), N tails, fp16
    and fp32 outputs.  Each single launch runs the GEMV kernel, so the two
    paths check each other besides the oracle."""
    specs = [(16, 256, 200000, np.float16, False), (7, 200, 150001, np.float32, False),
             (2, 64, 100000, np.float16, False), (9, 1000, 120000, np.float16, False)]
    assert sum((N + 511) // 512 for M, K, N, _, _ in specs) == 1115
    for w, _, _ in _check_prefill_group(ctx, specs, 2300, plan=(GEMM, TILE_LIST, 32, 512)):
        w.close()


def test_group_of_short_products_with_32_row_tiles(ctx):
    """16 < M <= 32 in a large group (1173 tiles): 32-row tiles, with M = 32
    filling a whole tile (the staged epilogue) and M = 17, 24 ragged."""
    specs = [(32, 512, 150000, np.float16, False), (17, 256, 200000, np.float32, False),
             (24, 128, 250000, np.float16, False)]
    assert sum((N + 511) // 512 for M, K, N, _, _ in specs) == 1173
    for w, _, _ in _check_prefill_group(ctx, specs, 2400, plan=(GEMM, TILE_LIST, 32, 512)):
        w.close()


def test_group_with_long_tiles_cut_into_parts_64_row(ctx):
    """64-row tiles in a tile list whose long tiles (K = 4864: 38 stages,
    against a mean of 5 to 7 per workgroup) are cut along K into parts: the
    parts write fp32 partial tiles and the reduce launch sums them in K order
    into y; rows past M (M = 48, 40), N tails, fp16 and fp32 outputs, and y +=
    (the reduce adds y once).  The short items' whole tiles write y
    directly in the same launch."""
    specs = [(64, 512, 200000, np.float16, False), (48, 4864, 1000, np.float32, False),
             (64, 4864, 896, np.float16, False), (40, 4864, 1000, np.float16, True),
             (64, 512, 150000, np.float32, True)]
    for w, _, _ in _check_prefill_group(ctx, specs, 2800, plan=(GEMM, PARTS, 64, 512)):
        w.close()


def test_group_with_long_tiles_cut_into_parts_fp32_scales_bs128(ctx):
    """Parts of 64 x 512 tiles with the export format's block size (bs 128,
    one scale per row and stage) and fp32 scales with zero points: K = 4800
    (37.5 blocks: the last stage's block is half outside K) and 4864 items
    cut into parts among short tiles, rows past M, y +=."""
    specs = [(64, 512, 200000, np.float16, False), (48, 4800, 1000, np.float32, False),
             (64, 4864, 896, np.float16, False), (40, 4800, 1000, np.float16, True),
             (64, 512, 150000, np.float32, True)]
    for w, _, _ in _check_prefill_group(ctx, specs, 3100, bs=128, plan=(GEMM, PARTS, 64, 512), f32_scales=True):
        w.close()


def test_group_with_long_tiles_cut_into_parts_32_row(ctx):
    """32-row tiles (16 < M <= 32) with parts: K = 4864 and 8192 items (38 and
    64 stages) among 1172 two-stage tiles; M = 17 and 24 ragged."""
    specs = [(32, 256, 600000, np.float16, False), (17, 4864, 1000, np.float32, False),
             (24, 8192, 3072, np.float16, False)]
    for w, _, _ in _check_prefill_group(ctx, specs, 2900, plan=(GEMM, PARTS, 32, 512)):
        w.close()


def test_group_with_long_tiles_cut_into_parts_128_row(ctx):
    """128 x 256 tiles in a tile list with parts (fp32 scales at bs 16 have
    no 512-column kernel): K = 4864 and 8192 items with two m-tiles (M = 200,
    130: rows past M in the second) among 1024 two-stage tiles."""
    specs = [(128, 256, 262000, np.float16, False), (200, 4864, 1000, np.float32, False),
             (130, 8192, 512, np.float16, False)]
    assert sum(((M + 127) // 128) * ((N + 255) // 256) for M, K, N, _, _ in specs) == 1036
    for w, _, _ in _check_prefill_group(ctx, specs, 3000, bs=16, plan=(GEMM, PARTS, 128, 256), f32_scales=True):
        w.close()


def test_single_item_group_in_tile_list_order(ctx):
    """A group of one product with many tiles (1564 of 128 x 512): the item
    comes from the launch parameters rather than the table while the
    workgroups walk a tile list."""
    specs = [(512, 256, 200000, np.float16, False)]
    for w, _, _ in _check_prefill_group(ctx, specs, 2500, plan=(GEMM, TILE_LIST, 128, 512)):
        w.close()


def test_group_of_prefill_products_accumulating_in_tile_list_order(ctx):
    """y += in tile-list order (1412 tiles of 512 columns, enough per
    workgroup for the wide kernel): the epilogue's general path (read y, add,
    write) for whole and ragged tiles, N not a multiple of 4, fp16 and fp32
    outputs, 2, 3 and 5 stages per tile."""
    specs = [(2000, 384, 16001, np.float32, True), (1500, 256, 30000, np.float16, True),
             (900, 640, 12000, np.float16, True)]
    assert sum(((M + 127) // 128) * ((N + 511) // 512) for M, K, N, _, _ in specs) == 1412
    for w, _, _ in _check_prefill_group(ctx, specs, 1900, plan=(GEMM, TILE_LIST, 128, 512)):
        w.close()


# ------------------------------------------------ tiny scales, k tails ----

def _tiny_scale_weight(seed, N, K, bs, lo, hi, zp):
    """synth weight whose block scales are uniform in [lo, hi] (fp32, so not
    rounded to fp16) with random signs."""
    t = synth.make_weight(seed, N, K, bs, with_zp=zp)
    rng = np.random.default_rng(seed + 1)
    s = rng.uniform(lo, hi, t.N * t.kb).astype(np.float32) * rng.choice([-1.0, 1.0], t.N * t.kb).astype(np.float32)
    return t, s


def _oracle_f32_scales(t, s, x16):
    kb = t.kb
    zrp = t.zp_row_padded if t.zp_row_padded is not None else np.full((t.N, (kb + 1) // 2), 0x88, np.uint8)
    z = synth.zp_row_padded_to_flat(zrp, t.N, kb)
    kpad = kb * t.bs
    x = np.zeros((x16.shape[0], kpad), np.float32)
    x[:, : t.K] = x16.astype(np.float32)
    y = orc.matmul(t.q, s, z, t.N, kpad, t.bs, x, threads=THREADS)
    wmax = float(np.abs(orc.dequantize(t.q, s, z, t.N, kpad, t.bs)).max())
    return y, wmax


@pytest.mark.parametrize("lo,hi", [(1e-7, 1e-6), (2e-9, 3e-8), (1e-3, 4e-3)])
def test_tiny_block_scales_keep_the_bound(ctx, lo, hi):
    """Block scales far below fp16's normal range: products (q - zp) * s
    below 6.1e-5 would be fp16 subnormals (absolute error up to 2^-25 each)
    where a kernel folds the scale into its fp16 operand -- the GEMM at every
    M > 16 and the bs = 16 GEMV.  Each weight keeps a power-of-two exponent
    that lifts its largest |15 s| just below 65504 for that fold, undone
    exactly on the fp32 sums, so all paths stay within the bound; fp32 and
    subnormal fp16 scales, zero points or none, M = 1, 5, 40, 300, single
    launches and groups, and the dequantization stays bit-exact."""
    import torch
    cases = [(700, 1000, 32, True), (300, 2048, 16, False), (513, 384, 64, True)]
    for ci, (N, K, bs, zp) in enumerate(cases):
        t, s = _tiny_scale_weight(8100 + ci, N, K, bs, lo, hi, zp)
        zl = mnb_hip.MNB_ZP_ROW_PADDED if zp else None
        w32 = mnb_hip.Weight(ctx, N, K, bs, t.q, s, t.zp_row_padded, zl)
        s16 = s.astype(np.float16)          # fp16 scales: subnormal for most of these ranges
        w16 = mnb_hip.Weight(ctx, N, K, bs, t.q, s16, t.zp_row_padded, zl)
        try:
            for w, sv, tag in ((w32, s, "f32"), (w16, s16.astype(np.float32), "f16")):
                kb = t.kb
                zrp = t.zp_row_padded if zp else np.full((N, (kb + 1) // 2), 0x88, np.uint8)
                wd = w.dequantize(np.float32)
                w_ref = orc.dequantize(t.q, sv, synth.zp_row_padded_to_flat(zrp, N, kb), N, kb * bs, bs)[:, :K]
                assert np.array_equal(wd.view(np.uint32), np.ascontiguousarray(w_ref).view(np.uint32)), tag
                for M in (1, 5, 40, 300):
                    x16 = synth.make_x(8200 + M + ci, M, K)
                    y_ref, wmax = _oracle_f32_scales(t, sv, x16)
                    label = "tiny scales [%g, %g] %s N=%d K=%d bs=%d zp=%d M=%d" % (lo, hi, tag, N, K, bs, zp, M)
                    assert_parity(w.matmul(x16, out_dtype=np.float32), y_ref, x16, t, wmax, False, label)
                    if M > 1:     # one item of a group (the GEMM for M > 16, the 32-row GEMM or the GEMV group)
                        xd = torch.from_numpy(x16).cuda()
                        yd = torch.zeros((M, N), dtype=torch.float32, device="cuda")
                        g = mnb_hip.Group(ctx, [(w, xd, yd)])
                        torch.cuda.synchronize()     # the group runs on the context's stream
                        g.run()
                        torch.cuda.synchronize()
                        g.close()
                        assert_parity(yd.cpu().numpy(), y_ref, x16, t, wmax, False, label + " group")
        finally:
            w32.close()
            w16.close()


def test_single_product_with_x_beyond_2_gib(ctx):
    """x of one product larger than 2 GiB (M = 140000 rows at K = 8192, 2.29 GB
    on the device): the library runs it in row chunks of at most 2 GiB
    (131072 rows here), each planned on its own, with 32-bit offsets inside a
    chunk.  Rows on both sides of the chunk boundary, the first and the last
    match the oracle; the fp16 output equals the fp32 output rounded.  A group
    refuses the same item."""
    import torch
    M, K, N, bs = 140000, 8192, 64, 32
    t = synth.make_weight(9300, N, K, bs, with_zp=True)
    w = upload(ctx, t)
    try:
        say("x beyond 2 GiB: plan of the first chunk", w.plan(M).as_tuple())
        gen = torch.Generator(device="cuda").manual_seed(9301)
        xd = torch.randn(M, K, device="cuda", generator=gen, dtype=torch.float16)
        assert xd.numel() * 2 > (1 << 31)
        yd = torch.empty(M, N, device="cuda", dtype=torch.float32)
        w.matmul(xd, yd)
        yh = torch.empty(M, N, device="cuda", dtype=torch.float16)
        w.matmul(xd, yh)
        torch.cuda.synchronize()
        rows = torch.tensor([0, 1, 131070, 131071, 131072, 131073, 139998, 139999], device="cuda")
        x16 = xd[rows].cpu().numpy()
        y_ref, wmax = oracle_matmul(t, x16)
        assert_parity(yd[rows].cpu().numpy(), y_ref, x16, t, wmax, False, "x beyond 2 GiB")
        assert torch.isfinite(yd).all()
        assert torch.equal(yh.view(torch.int16), yd.half().view(torch.int16))
        # a group refuses such an item (its kernels take 32-bit x offsets)
        with pytest.raises(mnb_hip.MnbError, match="x of 2 GiB or packed weights of 4 GiB or more in a group"):
            mnb_hip.Group(ctx, [(w, xd, yd)])
        del xd, yd, yh
    finally:
        w.close()


def test_packed_weight_of_4_gib(ctx):
    """A weight of 4 GiB of packed nibbles (N = 524288, K = 16384, bs 32;
    4.5 GB resident with its scales): the repack and the M <= 16 kernels use
    64-bit offsets, so products at M = 1 and M = 4 match the oracle on output
    columns spread over the whole weight, the last ones lying past 4 GiB.  The
    GEMM and K-sliced kernels take 32-bit offsets into the scales: M > 16 is
    refused with MNB_ERR_UNSUPPORTED by mnb_matmul and mnb_matmul_plan, and
    9 <= M <= 16 stays on the GEMV."""
    import torch
    N, K, bs = 524288, 16384, 32
    t = synth.make_weight(9400, N, K, bs)
    assert t.q.nbytes == 4 << 30
    w = upload(ctx, t)
    try:
        say("4 GiB weight resident: %d bytes" % w.device_bytes)
        cols = np.concatenate([np.arange(0, N, 2053), np.arange(N - 40, N)])
        for M in (1, 4):
            x16 = synth.make_x(9401 + M, M, K)
            y = w.matmul(x16)
            y_ref, _ = oracle_matmul(t, x16, cols, want_wmax=False)
            assert_parity(y.reshape(M, N)[:, cols], y_ref, x16, t, None, False, "4 GiB weight M=%d" % M)
        assert w.plan(16).kernel == mnb_hip.MNB_KERNEL_GEMV, w.plan(16).as_tuple()
        x17 = torch.zeros(17, K, device="cuda", dtype=torch.float16)
        y17 = torch.zeros(17, N, device="cuda", dtype=torch.float16)
        with pytest.raises(mnb_hip.MnbError, match="packed weights of 4 GiB or more run only with M <= 16"):
            w.matmul(x17, y17)
        with pytest.raises(mnb_hip.MnbError, match="packed weights of 4 GiB or more run only with M <= 16"):
            w.plan(17)
        torch.cuda.synchronize()
        assert not torch.any(y17), "the refused call wrote y"
    finally:
        w.close()


@pytest.mark.parametrize("K", [1001, 203, 4099])
def test_single_products_with_a_k_tail_not_a_multiple_of_8(ctx, K):
    """K % 8 != 0: the kernels read x in 16-byte pieces, so x is first copied
    to fp16 rows padded to a multiple of 8 with zeros (host arrays, and device
    fp16 or fp32 x alike); M = 1, 7 (GEMV) and 40, 200 (the K-sliced kernel),
    zero points, bs 32 and 64."""
    import torch
    for bs in (32, 64):
        t = synth.make_weight(8300 + K + bs, 300, K, bs, with_zp=True)
        w = upload(ctx, t)
        try:
            for M in (1, 7, 40, 200):
                x16 = synth.make_x(8400 + M + K, M, K)
                y_ref, wmax = oracle_matmul(t, x16)
                label = "k tail K=%d bs=%d M=%d" % (K, bs, M)
                assert_parity(w.matmul(x16, out_dtype=np.float16), y_ref, x16, t, wmax, True, label + " host f16")
                for xdt in (torch.float16, torch.float32):
                    xd = torch.from_numpy(x16).cuda().to(xdt)
                    yd = torch.empty((M, 300), dtype=torch.float32, device="cuda")
                    torch.cuda.synchronize()
                    w.matmul(xd, yd)
                    torch.cuda.synchronize()
                    assert_parity(yd.cpu().numpy(), y_ref, x16, t, wmax, False, label + " device %s" % xdt)
        finally:
            w.close()


@pytest.mark.parametrize("N,K,bs,zp", [(1, 32, 32, False), (1, 8, 16, True), (17, 40, 32, True), (5, 136, 64, False),
                                        (33, 128, 128, True), (2, 264, 256, False)])
def test_tiny_shapes_on_every_path(ctx, N, K, bs, zp):
    """The smallest shapes: one output column (N = 1, a 16-row n-tile with 15
    padding rows, and 128- or 256-column GEMM tiles of one column), K below
    one 128-k super-tile or a block (K = 8 with bs 16, K = 40 with bs 32), a
    block larger than K; M from 1 to 130, so each single-product path the
    planners pick at these sizes runs (the GEMV with one, two and four x
    row groups, and the K-sliced kernel; groups of such products run the
    GEMM, in the test below).  fp32 y against the oracle, fp16 y as the
    rounded fp32 result, y += bitwise."""
    t = synth.make_weight(8700 + N + K + bs, N, K, bs, with_zp=zp)
    w = upload(ctx, t)
    try:
        for M in (1, 2, 3, 5, 8, 12, 16, 17, 40, 130):
            x16 = synth.make_x(8800 + M + K, M, K)
            y_ref, wmax = oracle_matmul(t, x16)
            label = "tiny N=%d K=%d bs=%d zp=%d M=%d plan=%s" % (N, K, bs, zp, M, w.plan(M).as_tuple())
            say(label)
            y32 = w.matmul(x16)
            assert_parity(y32, y_ref, x16, t, wmax, False, label)
            y16 = w.matmul(x16, out_dtype=np.float16)
            assert np.array_equal(y16.view(np.uint16), y32.astype(np.float16).view(np.uint16)), label
            y0 = np.random.default_rng(M + N).standard_normal(y32.shape).astype(np.float32)
            acc = w.matmul(x16, y=y0.copy(), accumulate=True)
            assert np.array_equal(acc.view(np.uint32), (y0 + y32).view(np.uint32)), label
    finally:
        w.close()


@pytest.mark.parametrize("ms", [(1, 1, 1, 1), (2, 3, 4, 2), (6, 5, 8, 6), (17, 130, 40, 33)],
                         ids=["m1-stream", "small-batch-stream", "gemv-group", "gemm"])
@pytest.mark.parametrize("bs,Ks", [(16, (8, 40, 136)), (32, (32, 40, 264))])
def test_tiny_shapes_in_groups(ctx, bs, Ks, ms):
    """The same small shapes recorded as groups of each M class: M = 1 and
    2 <= M <= 4 (the streaming kernel: units of one super-tile, so a job
    re-loads it for its missing tiles), 4 < M <= 8 with few tiles (the GEMV
    over every item's n-tiles) and M > 16 (the GEMM: one n-tile under a
    256- or 512-column tile); N = 1, K below a super-tile or a block, fp16
    and fp32 y, y +=; every item against the oracle and its own single
    launch, replays bitwise identical."""
    specs = [(ms[0], Ks[0], 1, np.float16, False), (ms[1], Ks[1], 17, np.float32, False),
             (ms[2], Ks[2], 5, np.float16, True), (ms[3], Ks[0], 33, np.float32, True)]
    for w, _, _ in _check_prefill_group(ctx, specs, 9100 + bs + sum(ms), bs=bs):
        w.close()


@pytest.mark.parametrize("case", [(500, 3000, 32001, 32, True, False, np.float32, False),
                                  (2048, 1024, 16384, 64, False, False, np.float16, True),
                                  (512, 3072, 32064, 128, False, True, np.float16, False)],
                         ids=["M500-K3000-N32001", "M2048-K1024-N16384-acc", "M512-K3072-N32064-f32scales"])
def test_single_products_in_closed_form_tile_order(ctx, case):
    """Single products with many 128 x 512 tiles run in tile-list order with
    the list computed in the kernel from the tile count (no table, so the call
    still allocates nothing): M, N and K tails, zero points, fp32 scales not
    fp16-exact (so kept fp32), fp16 and fp32 outputs, y +=.  Sampled outputs
    against the oracle, repeat calls bitwise identical."""
    import torch
    M, K, N, bs, zp, f32s, ydt, acc = case
    t = synth.make_weight(8600 + M + N, N, K, bs, with_zp=zp)
    w = upload(ctx, t, as_f32_scales=f32s)
    if f32s:    # scales that fp16 cannot hold: the device keeps fp32 scales
        s = t.scales_f16.astype(np.float32) * np.float32(1.0 + 2.0 ** -14)
        w.close()
        w = mnb_hip.Weight(ctx, N, K, bs, t.q, s)
    try:
        p = w.plan(M)
        assert p.as_tuple() == (GEMM, TILE_LIST, 128, 512), p.as_tuple()
        x16 = synth.make_x(8700 + M, M, K)
        y0 = np.random.default_rng(8800 + M).standard_normal((M, N)).astype(ydt)
        xd = torch.from_numpy(x16).cuda()
        outs = []
        for _ in range(2):
            yd = torch.from_numpy(y0.copy()).cuda()
            torch.cuda.synchronize()
            w.matmul(xd, yd, accumulate=acc)
            torch.cuda.synchronize()
            outs.append(yd.cpu().numpy())
        assert np.array_equal(outs[0].view(np.uint8), outs[1].view(np.uint8))
        rng = np.random.default_rng(8900 + M)
        rows = np.sort(np.concatenate([rng.choice(M, 40, replace=False), [M - 1]]))
        cols = np.sort(np.concatenate([rng.choice(N - 16, 48, replace=False), np.arange(N - 16, N)]))
        if f32s:
            kb = t.kb
            z = synth.zp_row_padded_to_flat(np.full((N, (kb + 1) // 2), 0x88, np.uint8), N, kb)
            q2 = t.q.reshape(N, -1)[cols].reshape(-1)
            sc = s.reshape(N, kb)[cols].reshape(-1)
            z2 = synth.zp_row_padded_to_flat(np.full((cols.size, (kb + 1) // 2), 0x88, np.uint8), cols.size, kb)
            xp = np.zeros((rows.size, kb * bs), np.float32)
            xp[:, :K] = x16[rows].astype(np.float32)
            y_ref = orc.matmul(q2, sc, z2, cols.size, kb * bs, bs, xp, threads=THREADS)
            wmax = float(np.abs(sc).max()) * 8.0
        else:
            y_ref, wmax = oracle_matmul(t, np.ascontiguousarray(x16[rows]), cols, want_wmax=False)
            wmax = None
        got = outs[0].astype(np.float32)[np.ix_(rows, cols)] - (y0.astype(np.float32)[np.ix_(rows, cols)] if acc else 0)
        assert_parity(got, y_ref, x16, t, wmax, ydt == np.float16 or acc,
                      "closed-form single M=%d K=%d N=%d bs=%d" % (M, K, N, bs))
    finally:
        w.close()


def test_matmul_plan_reports_the_single_product_schedule(ctx):
    """mnb_matmul_plan: the GEMV kernel up to M = 8, and up to 16 for
    narrow products (o_proj); 16 x 64 K-sliced blocks for wide products at
    M = 12 and 16 (qkv, gate_up); the K-sliced kernel where the GEMM would
    have few tiles for the chip (o_proj and down at M 32 to 512, qkv at 32
    and 64: 32 x 16 up to 64 x 64 output blocks);
    stream-K 128 x 256 tiles for the qkv shape at M = 512; closed-form
    128 x 512 tile lists for products with many tiles (the Phi-3 lm_head at
    M = 512 and gate_up at 2048)."""
    for (K, N, M), expect in [((3072, 9216, 1), (mnb_hip.MNB_KERNEL_GEMV, NO_ORDER, 0, 16)),
                              ((3072, 9216, 8), (mnb_hip.MNB_KERNEL_GEMV, NO_ORDER, 0, 16)),
                              ((3072, 3072, 16), (mnb_hip.MNB_KERNEL_GEMV, NO_ORDER, 0, 16)),
                              ((3072, 9216, 16), (KSLICE, NO_ORDER, 16, 64)),
                              ((3072, 16384, 12), (KSLICE, NO_ORDER, 16, 64)),
                              ((3072, 3072, 32), (KSLICE, NO_ORDER, 32, 16)),
                              ((3072, 3072, 64), (KSLICE, NO_ORDER, 32, 32)),
                              ((3072, 9216, 32), (KSLICE, NO_ORDER, 32, 64)),
                              ((3072, 9216, 64), (KSLICE, NO_ORDER, 64, 64)),
                              ((8192, 3072, 128), (KSLICE, NO_ORDER, 32, 64)),
                              ((3072, 3072, 512), (KSLICE, NO_ORDER, 64, 64)),
                              ((3072, 9216, 512), (GEMM, STREAM_K, 128, 256)),
                              ((3072, 32064, 512), (GEMM, TILE_LIST, 128, 512)),
                              ((3072, 16384, 2048), (GEMM, TILE_LIST, 128, 512))]:
        t = synth.make_weight(1, N, K, 32)
        w = upload(ctx, t)
        try:
            assert w.plan(M).as_tuple() == expect, (K, N, M, w.plan(M).as_tuple())
        finally:
            w.close()
