"""Pins the CPU oracle (oracle/mnb_oracle.c) before anything is compared to it.

Each check is chosen so that a plausible restatement mistake fails it: a
swapped nibble order, a wrong zero-point index, a dropped scale, a transposed
operand, a wrong fp16 widening, FMA contraction, or a changed accumulation
semantic (y += vs y =).
"""
import json
import math
import os

import numpy as np
import pytest

import mnb_oracle as orc


@pytest.fixture(scope="module", autouse=True)
def _built():
    orc.build()


def _load(golden_dir, name):
    return np.load(os.path.join(golden_dir, name), allow_pickle=False)


# ---------------------------------------------------------------- fp16 ----

def test_fp16_to_fp32_matches_reference_table_exhaustively(golden_dir):
    d = _load(golden_dir, "fp16_to_fp32_ref.npz")
    got = orc.fp16_bits_to_fp32(d["fp16_bits"]).view(np.uint32)
    assert np.array_equal(got, d["fp32_bits"])


def test_fp16_to_fp32_normals_equal_ieee_widening():
    bits = np.arange(65536, dtype=np.uint16)
    e = (bits >> 10) & 0x1F
    normal = (e > 0) & (e < 31)
    ieee = bits.view(np.float16).astype(np.float32)
    got = orc.fp16_bits_to_fp32(bits)
    assert np.array_equal(got[normal].view(np.uint32), ieee[normal].view(np.uint32))
    # the subnormal quirk: m * 2^-150 instead of m * 2^-24
    sub = (e == 0) & ((bits & 0x3FF) != 0)
    assert np.all(np.abs(got[sub]) < 2.0 ** -139)
    assert np.all(np.abs(ieee[sub]) >= 2.0 ** -24)


def test_fp32_to_fp16_rne_matches_numpy():
    rng = np.random.default_rng(1)
    v = np.concatenate([
        rng.standard_normal(4096).astype(np.float32),
        (rng.uniform(-1, 1, 2048) * 2.0 ** -20).astype(np.float32),       # fp16 subnormal range
        (rng.uniform(-1, 1, 2048) * 70000).astype(np.float32),            # overflow
        # exact ties between two fp16 values: (2k+1) * 2^-11 in [1, 2)
        ((2 * np.arange(1024) + 1) * 2.0 ** -11 + 1.0).astype(np.float32),
        ((2 * np.arange(1024) + 1) * 2.0 ** -25).astype(np.float32),       # subnormal ties
        np.array([0.0, -0.0, np.inf, -np.inf, 65504, 65520, 65519.99, 2.0 ** -25, 2.0 ** -26], np.float32),
    ])
    got = orc.fp32_to_fp16_bits(v)
    exp = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, exp)


# ------------------------------------------------------------- dequant ----

def _dequant_cases(golden_dir):
    d = _load(golden_dir, "dequant_exact.npz")
    names = sorted({k.split("__")[0] for k in d.files})
    for n in names:
        N, K, bs = (int(v) for v in d[n + "__shape"])
        yield n, d[n + "__q"], d[n + "__scales"], d[n + "__zp"], N, K, bs, d[n + "__w"]


def test_dequant_bit_exact_against_exact_rational(golden_dir):
    count = 0
    for name, q, s, z, N, K, bs, w in _dequant_cases(golden_dir):
        got = orc.dequantize(q, s, z, N, K, bs)
        assert np.array_equal(got.view(np.uint32), w.view(np.uint32)), name
        count += 1
    assert count >= 9


def test_dequant_nibble_order_and_signed_zero(golden_dir):
    cases = {c[0]: c for c in _dequant_cases(golden_dir)}
    _, q, s, z, N, K, bs, w = cases["nibble_order_0x21"]
    got = orc.dequantize(q, s, z, N, K, bs)
    assert got[0, 0] == 1.0 and got[0, 1] == 2.0          # low nibble first
    _, q, s, z, N, K, bs, w = cases["q_eq_zp_signed_zero"]
    got = orc.dequantize(q, s, z, N, K, bs)
    assert np.all(got == 0.0)
    signs = np.signbit(got).reshape(N, K // bs, bs)
    assert not signs[0, 0].any() and signs[0, 1].all()       # +scale -> +0, -scale -> -0


# ------------------------------------------------------------------ dot ---

def test_dot_closed_form_and_tail(golden_dir):
    kat = json.load(open(os.path.join(golden_dir, "kat_closed_form.json")))
    for c in kat["dot"]:
        assert abs(orc.dot_scalar(c["a"], c["b"]) - c["expected"]) <= c["atol"]
        assert abs(orc.dot_lanes(c["a"], c["b"], 8) - c["expected"]) <= c["atol"]
    # FloatMathOpsTest.java:33-42: 17 elements exercise the lane loop and the tail
    a = np.array([(i % 5) - 2.0 for i in range(17)], np.float32)
    b = np.array([0.25 * i - 1.0 for i in range(17)], np.float32)
    exact = math.fsum(float(x) * float(y) for x, y in zip(a, b))
    for lanes in (0, 4, 8, 16):
        got = orc.dot_scalar(a, b) if lanes == 0 else orc.dot_lanes(a, b, lanes)
        assert abs(got - exact) <= 1e-3


def test_dot_scalar_is_sequential_without_fma():
    # 1 + 2^-24 - 1 depends on the order and on contraction: a fused or
    # reordered sum would not reproduce the sequential binary32 result.
    a = np.array([1.0, 2.0 ** -24, -1.0], np.float32)
    b = np.array([1.0, 1.0, 1.0], np.float32)
    assert orc.dot_scalar(a, b) == 0.0      # (1 + 2^-24) rounds to 1, then - 1
    # products rounded before the add: (1+2^-12)^2 = 1 + 2^-11 + 2^-24 -> 1 + 2^-11
    e = np.float32(1.0 + 2.0 ** -12)
    got = orc.dot_scalar(np.array([e, -1.0], np.float32), np.array([e, 1.0], np.float32))
    assert got == np.float32(2.0 ** -11)


# --------------------------------------------------------- matvec / mm ----

def _uniform_weight(N, nibble, zp, scale, bs=128):
    K = bs
    q = np.full(N * K // 2, (nibble & 0xF) | ((nibble & 0xF) << 4), np.uint8)
    s = np.full(N, scale, np.float32)
    z = np.full((N + 1) // 2, (zp & 0xF) | ((zp & 0xF) << 4), np.uint8)
    return q, s, z, K


def test_matvec_closed_form_kats(golden_dir):
    kat = json.load(open(os.path.join(golden_dir, "kat_closed_form.json")))
    for c in kat["matvec"]:
        q, s, z, K = _uniform_weight(c["N"], c["nibble"], c["zp"], c["scale"])
        x = np.full(K, c["x"], np.float32)
        for lanes in (0, 8):
            y = np.array(c["y_init"], np.float32)
            orc.matvec(q, s, z, c["N"], K, 128, x, y, lanes=lanes)
            assert np.allclose(y, c["expected"], atol=c["atol"], rtol=0), (c["name"], lanes)


def test_matmul_equals_repeated_matvec_bitwise():
    rng = np.random.default_rng(5)
    N, K, bs, M = 9, 256, 32, 4
    q = rng.integers(0, 256, N * K // 2, dtype=np.uint8)
    s = rng.uniform(0.005, 0.02, N * K // bs).astype(np.float16).astype(np.float32)
    z = rng.integers(0, 256, (N * K // bs + 1) // 2, dtype=np.uint8)
    x = rng.standard_normal((M, K)).astype(np.float32)
    for lanes in (0, 8):
        yb = orc.matmul(q, s, z, N, K, bs, x, lanes=lanes, threads=3)
        for m in range(M):
            ym = orc.matvec(q, s, z, N, K, bs, x[m], lanes=lanes)
            assert np.array_equal(yb[m].view(np.uint32), ym.view(np.uint32))


def test_matmul_within_fp32_bound_of_exact(golden_dir):
    d = _load(golden_dir, "matmul_exact.npz")
    names = sorted({k.split("__")[0] for k in d.files})
    for n in names:
        N, K, bs, M = (int(v) for v in d[n + "__shape"])
        x = d[n + "__x"]
        y = orc.matmul(d[n + "__q"], d[n + "__scales"], d[n + "__zp"], N, K, bs, x)
        # sequential binary32 summation of K rounded terms: |err| <= gamma_K * sum|x*w|
        # with gamma_K = K u / (1 - K u), plus the rounding of each dequantized w.
        u = 2.0 ** -24
        bound = (K + 2) * u / (1 - (K + 2) * u) * d[n + "__abs_sum"] + 1e-30
        err = np.abs(y.astype(np.float64) - d[n + "__y_exact"])
        assert np.all(err <= bound), n
        y64 = orc.matmul_f64(d[n + "__q"], d[n + "__scales"], d[n + "__zp"], N, K, bs, x)
        assert np.all(np.abs(y64 - d[n + "__y_exact"]) <= 1e-12 * (1 + d[n + "__abs_sum"])), n


def test_matmul_linear_in_x_and_scale():
    rng = np.random.default_rng(7)
    N, K, bs = 5, 128, 32
    q = rng.integers(0, 256, N * K // 2, dtype=np.uint8)
    s = rng.uniform(0.005, 0.02, N * K // bs).astype(np.float32)
    z = np.full((N * K // bs + 1) // 2, 0x88, np.uint8)
    x = rng.standard_normal(K).astype(np.float32)
    y1 = orc.matvec(q, s, z, N, K, bs, x)
    y2 = orc.matvec(q, s * 2, z, N, K, bs, x)      # power-of-2 scaling is exact
    y3 = orc.matvec(q, s, z, N, K, bs, x * 4)
    assert np.array_equal(y2, 2 * y1) and np.array_equal(y3, 4 * y1)
    # a transposed / mis-indexed weight would not match an explicit dequant @ x
    w = orc.dequantize(q, s, z, N, K, bs).astype(np.float64)
    assert np.allclose(y1, w @ x.astype(np.float64), rtol=1e-5, atol=1e-5)


# ------------------------------------------------------- zero points ------

def test_zero_point_layouts(golden_dir):
    zk = json.load(open(os.path.join(golden_dir, "zero_points.json")))
    rows, bpr = zk["rows"], zk["blocks_per_row"]
    flat = np.array(zk["flat_bytes"], np.uint8)
    rp = np.array(zk["row_padded_bytes"], np.uint8)
    assert np.array_equal(orc.zp_repack_row_padded(rp, rows, bpr), flat)
    assert np.array_equal(orc.zp_normalize_raw(rp, [rows, (bpr + 1) // 2], rows, bpr), flat)
    assert np.array_equal(orc.zp_normalize_raw(rp, [rows * ((bpr + 1) // 2)], rows, bpr), flat)
    assert np.array_equal(orc.zp_normalize_raw(flat, [flat.size], rows, bpr), flat)
    un = np.array(zk["unpacked_u8"], np.uint8)
    assert np.array_equal(orc.zp_pack_unpacked_u8(un, rows, bpr), flat)
    assert np.array_equal(orc.zp_normalize_raw(un, [rows, bpr], rows, bpr), flat)
    f = np.array(zk["unpacked_f32"], np.float32)
    nib = zk["unpacked_f32_expected_nibbles"]
    packed = orc.zp_pack_unpacked_f32(f, rows, bpr)
    got = [(packed[i // 2] >> (4 * (i % 2))) & 0xF for i in range(rows * bpr)]
    assert got == nib
    assert list(orc.zp_default(zk["default_blocks"])) == zk["default_bytes"]
    with pytest.raises(ValueError):
        orc.zp_normalize_raw(np.zeros(7, np.uint8), [7], rows, bpr)


# --------------------------------------------------------- quantizer ------

def test_quantizer_closed_forms(golden_dir):
    qz = json.load(open(os.path.join(golden_dir, "quantizer.json")))
    for c in qz["cases"]:
        s, z = orc.quant_block_params(c["data"])
        assert s == np.float32(c["scale"]) and z == c["zp"], c["name"]
        q, sc, zp = orc.quantize_rows_u4(np.array(c["data"], np.float32), 1, 16, 16)
        nibs = [(q[i // 2] >> (4 * (i % 2))) & 0xF for i in range(16)]
        assert nibs == c["q"], c["name"]
        assert (zp[0] & 0xF) == c["zp"]
    for v, r in qz["java_round"]:
        assert orc.java_round(v) == r, v
    for h, b in qz["tied_block_size"]:
        assert orc.choose_tied_block_size(h) == b


def test_quantizer_roundtrip_error_bounded():
    rng = np.random.default_rng(11)
    rows, cols, bs = 8, 256, 64
    data = rng.standard_normal((rows, cols)).astype(np.float32)
    q, s, z = orc.quantize_rows_u4(data, rows, cols, bs)
    w = orc.dequantize(q, s, z, rows, cols, bs)
    # asymmetric min/max quantization: error <= scale/2 (+ the zp rounding of up to scale/2)
    smax = np.repeat(s.reshape(rows, cols // bs), bs, axis=1)
    assert np.all(np.abs(w - data) <= smax * 1.0 + 1e-6)


# ------------------------------------------------------------ fusion ------

def test_row_fusion_concatenates_and_refuses_odd_nibbles():
    rng = np.random.default_rng(3)
    K, bs = 96, 32
    parts = []
    for N in (4, 6, 3):
        q = rng.integers(0, 256, N * K // 2, dtype=np.uint8)
        s = rng.uniform(0.005, 0.02, N * K // bs).astype(np.float32)
        z = orc.zp_pack_unpacked_u8(rng.integers(0, 16, N * K // bs), N, K // bs)
        parts.append((q, s, z, N, K, bs))
    fq, fs, fz, fN = orc.fuse_rows(parts)
    assert fN == 13
    assert np.array_equal(fq, np.concatenate([p[0] for p in parts]))
    assert np.array_equal(fs, np.concatenate([p[1] for p in parts]))
    # fused dequant == stacked per-part dequant
    w = orc.dequantize(fq, fs, fz, fN, K, bs)
    ws = np.concatenate([orc.dequantize(p[0], p[1], p[2], p[3], K, bs) for p in parts])
    assert np.array_equal(w, ws)
    # N=3 with bpr=3 gives 9 nibbles: a non-last part ending mid-byte is refused
    assert orc.fuse_rows([parts[2], parts[0]]) is None
