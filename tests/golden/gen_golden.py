"""Generate the golden fixtures under tests/golden/.

The expected values here are computed WITHOUT the oracle: closed forms taken
from the reference's own tests, exact rational arithmetic (fractions.Fraction)
and the IEEE definitions.  The oracle (oracle/mnb_oracle.c) and the HIP
kernels are then checked against these files.

Reference tests whose cases are restated (paths relative to the reference
repository root):
  TQW = directml-inference/src/test/java/com/aresstack/windirectml/inference/qwen/QuantizedWeightMatvecTest.java
  TFM = directml-inference/src/test/java/com/aresstack/windirectml/inference/simd/FloatMathOpsTest.java
  TWP = directml-inference/src/test/java/com/aresstack/windirectml/inference/phi3/Phi3WdmlPackCompilerTest.java

Run:  python tests/golden/gen_golden.py   (rewrites the fixtures in place)
"""
from __future__ import annotations

import json
import os
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


# --------------------------------------------------------------------------
# exact helpers
# --------------------------------------------------------------------------

def f32(x) -> np.float32:
    return np.float32(x)


def frac_of_f32(v: np.float32) -> Fraction:
    return Fraction(float(v))   # a binary32 value is exactly a binary64 value


def rne_f32_of_fraction(r: Fraction) -> np.float32:
    """Round an exact rational to binary32, ties to even (only used where the
    value has <= 53 significant bits, so float(r) is exact)."""
    d = float(r)
    assert Fraction(d) == r, "value is not exact in binary64"
    return np.float32(d)


def fp16_ref_quirk_bits(h: int) -> int:
    """Expected binary32 bits of the reference's fp16ToFp32 for fp16 bits h
    (P3W:665-683).  Normal and inf/nan: IEEE.  Subnormal m: m * 2^-150
    rounded to the binary32 grid (2^-149), ties to even."""
    s = (h >> 15) & 1
    e = (h >> 10) & 0x1F
    m = h & 0x3FF
    if e == 0:
        if m == 0:
            return s << 31
        # m * 2^-150 = (m/2) * 2^-149 ; binary32 subnormal grid is 2^-149
        q, r = divmod(m, 2)
        if r == 1 and (q & 1) == 1:   # exact tie: round half to even
            q += 1
        return (s << 31) | q           # subnormal binary32 with mantissa q
    if e == 31:
        return (s << 31) | 0x7F800000 | (m << 13)
    return (s << 31) | ((e - 15 + 127) << 23) | (m << 13)


def unpack_nib(buf: bytes, idx: int) -> int:
    b = buf[idx // 2]
    return (b & 0xF) if idx % 2 == 0 else (b >> 4)


def exact_dequant(q: np.ndarray, scales: np.ndarray, zp: np.ndarray, N: int, K: int, bs: int) -> np.ndarray:
    """Exact w[n,k] = (nib - zp) * scale rounded once to binary32."""
    bpr = K // bs
    out = np.empty((N, K), np.float32)
    qb = q.tobytes()
    zb = zp.tobytes()
    for n in range(N):
        for blk in range(bpr):
            s = frac_of_f32(scales[n * bpr + blk])
            z = unpack_nib(zb, n * bpr + blk)
            for kk in range(bs):
                k = blk * bs + kk
                nib = unpack_nib(qb, n * K + k)   # row n has K/2 bytes; nibble index n*K + k
                v = rne_f32_of_fraction((nib - z) * s)
                if v == 0:
                    # IEEE sign of a zero product: float(nib - z) is +0 when nib == z
                    neg = ((nib - z) < 0) != bool(np.signbit(scales[n * bpr + blk]))
                    v = np.float32(-0.0) if neg else np.float32(0.0)
                out[n, k] = v
    return out


def exact_matmul(wq: np.ndarray, x: np.ndarray) -> tuple:
    """Exact y = x @ w^T over the binary32 values of w and x, and sum|x||w|
    (the scale of the fp32 summation-error bound).  Returned as float64."""
    M, K = x.shape
    N = wq.shape[0]
    y = np.empty((M, N), np.float64)
    mag = np.empty((M, N), np.float64)
    for m in range(M):
        xf = [frac_of_f32(v) for v in x[m]]
        for n in range(N):
            acc = Fraction(0)
            a = Fraction(0)
            for k in range(K):
                p = xf[k] * frac_of_f32(wq[n, k])
                acc += p
                a += abs(p)
            y[m, n] = float(acc)
            mag[m, n] = float(a)
    return y, mag


def pack_nibbles(vals) -> np.ndarray:
    vals = list(vals)
    out = bytearray((len(vals) + 1) // 2)
    for i, v in enumerate(vals):
        if i % 2 == 0:
            out[i // 2] = (out[i // 2] & 0xF0) | (v & 0xF)
        else:
            out[i // 2] = (out[i // 2] & 0x0F) | ((v & 0xF) << 4)
    return np.frombuffer(bytes(out), np.uint8).copy()


# --------------------------------------------------------------------------
# generators
# --------------------------------------------------------------------------

def twp_quant(n: int, k: int, bs: int, seed: int):
    """TWP:174-191 deterministic triplet generator: q[i]=(i*7+seed)&0xFF,
    scale[i]=(i+seed)*0.01f (Java int->float then float multiply),
    zp[i]=(i*3+seed)&0xFF."""
    bpr = k // bs
    qlen = n * bpr * (bs // 2)
    q = np.array([(i * 7 + seed) & 0xFF for i in range(qlen)], np.uint8)
    scales = np.array([f32(f32(i + seed) * f32(0.01)) for i in range(n * bpr)], np.float32)
    zp = np.array([(i * 3 + seed) & 0xFF for i in range((n * bpr + 1) // 2)], np.uint8)
    return q, scales, zp


def random_case(rng, N, K, bs, with_zp, neg_scales=False):
    bpr = K // bs
    q = rng.integers(0, 256, N * K // 2, dtype=np.uint8)
    s16 = rng.uniform(0.005, 0.02, N * bpr).astype(np.float32).astype(np.float16)
    if neg_scales:
        s16 = np.where(rng.integers(0, 2, s16.size) == 1, -s16, s16).astype(np.float16)
    scales = s16.astype(np.float32)   # IEEE widening == the reference's for normal fp16
    if with_zp:
        zp = pack_nibbles(rng.integers(0, 16, N * bpr))
    else:
        zp = np.full((N * bpr + 1) // 2, 0x88, np.uint8)
    return q, scales, s16.view(np.uint16), zp


def main():
    rng = np.random.default_rng(20261201)

    # ---- fp16 -> fp32 (reference loader conversion), all 65536 patterns ----
    bits = np.arange(65536, dtype=np.uint32)
    expect = np.array([fp16_ref_quirk_bits(int(h)) for h in bits], np.uint32)
    np.savez_compressed(os.path.join(HERE, "fp16_to_fp32_ref.npz"), fp16_bits=bits.astype(np.uint16),
                        fp32_bits=expect)

    # ---- closed-form KATs (TQW:86-195, TFM:20-48) ----
    kats = {
        "source": "QuantizedWeightMatvecTest.java:86-195 and FloatMathOpsTest.java:20-48",
        "block_size": 128,
        "matvec": [
            {"name": "allOnesNibbleZpZero", "N": 4, "nibble": 1, "zp": 0, "scale": 1.0, "x": 1.0,
             "y_init": [0, 0, 0, 0], "expected": [128.0] * 4, "atol": 1e-3},
            {"name": "nibble8Zp8ScaleOneGivesZero", "N": 4, "nibble": 8, "zp": 8, "scale": 1.0, "x": 5.0,
             "y_init": [0, 0, 0, 0], "expected": [0.0] * 4, "atol": 1e-6},
            {"name": "scalePropagates", "N": 2, "nibble": 2, "zp": 0, "scale": 0.5, "x": 1.0,
             "y_init": [0, 0], "expected": [128.0] * 2, "atol": 1e-3},
            {"name": "accumulatesIntoExistingY", "N": 2, "nibble": 1, "zp": 0, "scale": 1.0, "x": 1.0,
             "y_init": [10.0, 20.0], "expected": [138.0, 148.0], "atol": 1e-3},
        ],
        "dot": [
            {"a": [1, 2, 3], "b": [4, 5, 6], "expected": 32.0, "atol": 1e-5},
        ],
    }
    with open(os.path.join(HERE, "kat_closed_form.json"), "w") as f:
        json.dump(kats, f, indent=1)

    # ---- dequant fixtures (exact) ----
    cases = []
    # TWP deterministic generator, bs=4 exactly as the reference test, and bs=32
    for (n, k, bs, seed) in [(3, 16, 4, 2), (5, 64, 32, 3), (4, 96, 32, 7)]:
        q, s, z = twp_quant(n, k, bs, seed)
        cases.append(("twp_n%d_k%d_bs%d_s%d" % (n, k, bs, seed), q, s, None, z, n, k, bs))
    # random q4f16 with explicit zp, odd blocksPerRow (flat zp crosses byte boundaries)
    for (N, K, bs, wz, neg) in [(7, 96, 32, True, False),     # bpr=3 (odd)
                                (5, 192, 64, True, True),      # bpr=3, negative scales -> -0 cases
                                (3, 640, 128, True, False),    # bpr=5 (K=576 padded to 640)
                                (6, 256, 32, False, False),    # implicit zp 8
                                (4, 64, 16, True, False)]:     # bs=16
        q, s, s16, z = random_case(rng, N, K, bs, wz, neg)
        cases.append(("rand_n%d_k%d_bs%d_zp%d" % (N, K, bs, int(wz)), q, s, s16, z, N, K, bs))
    # q == zp everywhere (must give +0 for positive and -0 for negative scales)
    N, K, bs = 2, 64, 32
    q = np.full(N * K // 2, 0x55, np.uint8)
    z = pack_nibbles([5] * (N * K // bs))
    s = np.array([0.01, -0.01, 0.02, -0.02], np.float32).astype(np.float16).astype(np.float32)
    cases.append(("q_eq_zp_signed_zero", q, s, s.astype(np.float16).view(np.uint16), z, N, K, bs))
    # asymmetric nibbles: byte 0x21 -> k0=1, k1=2 (low nibble first), MNK:2697-2700
    N, K, bs = 1, 32, 32
    q = np.full(16, 0x21, np.uint8)
    z = pack_nibbles([0])
    s = np.array([1.0], np.float32)
    cases.append(("nibble_order_0x21", q, s, np.array([0x3C00], np.uint16), z, N, K, bs))

    dq = {}
    for (name, q, s, s16, z, N, K, bs) in cases:
        w = exact_dequant(q, s, z, N, K, bs)
        dq[name + "__q"] = q
        dq[name + "__scales"] = s
        dq[name + "__scales_f16"] = s16 if s16 is not None else np.zeros(0, np.uint16)
        dq[name + "__zp"] = z
        dq[name + "__shape"] = np.array([N, K, bs], np.int64)
        dq[name + "__w"] = w
    np.savez_compressed(os.path.join(HERE, "dequant_exact.npz"), **dq)

    # ---- matvec / matmul fixtures: exact products over binary32 values ----
    mm = {}
    for (name, N, K, bs, M, wz) in [("phi_block32", 6, 128, 32, 2, False),
                                    ("zp_bs64_oddbpr", 5, 192, 64, 3, True),
                                    ("bs128_pad", 4, 640, 128, 1, True)]:
        q, s, s16, z = random_case(rng, N, K, bs, wz)
        x = rng.standard_normal((M, K)).astype(np.float32).astype(np.float16).astype(np.float32)
        if name == "bs128_pad":
            x[:, 576:] = 0.0     # true K=576, padded to 640 as the reference requires
        w = exact_dequant(q, s, z, N, K, bs)
        y, mag = exact_matmul(w, x)
        for key, val in (("q", q), ("scales", s), ("scales_f16", s16), ("zp", z), ("x", x), ("y_exact", y),
                         ("abs_sum", mag), ("shape", np.array([N, K, bs, M], np.int64))):
            mm[name + "__" + key] = val
    np.savez_compressed(os.path.join(HERE, "matmul_exact.npz"), **mm)

    # ---- zero-point layout known answers (Q2W:1023-1075) ----
    # rows=3, bpr=3 (odd): row-padded bytes [3, 2]; nibble values row r, block b = 3r+b+1
    vals = [[3 * r + b + 1 for b in range(3)] for r in range(3)]
    row_padded = []
    for r in range(3):
        row = vals[r] + [0]       # pad to an even nibble count per row
        row_padded += list(pack_nibbles(row))
    flat = list(pack_nibbles([v for r in vals for v in r]))
    zpk = {
        "rows": 3, "blocks_per_row": 3,
        "row_padded_bytes": [int(b) for b in row_padded],
        "flat_bytes": [int(b) for b in flat],
        "unpacked_u8": [v | 0xA0 for r in vals for v in r],     # high bits must be masked off
        "unpacked_f32": [0.49, 1.5, 2.5, -0.7, 15.2, 16.0, 7.5, 8.49, -3.0],
        "unpacked_f32_expected_nibbles": [0, 2, 3, 0, 15, 15, 8, 8, 0],
        "default_blocks": 5, "default_bytes": [0x88, 0x88, 0x88],
    }
    with open(os.path.join(HERE, "zero_points.json"), "w") as f:
        json.dump(zpk, f, indent=1)

    # ---- tied quantizer closed forms (Q2W:1373-1398) ----
    ramp = [float(i) for i in range(16)]                 # min 0, max 15 -> scale 1, zp 0, q = i
    negramp = [float(i - 15) for i in range(16)]         # min -15, max 0 -> scale 1, zp 15, q = i
    qz = {
        "cases": [
            {"name": "zero_block", "data": [0.0] * 16, "scale": 1.0, "zp": 0, "q": [0] * 16},
            {"name": "const_pos", "data": [3.0] * 16, "scale": float(f32(3.0) / f32(15.0)), "zp": 0,
             "q": [15] * 16},
            {"name": "const_neg", "data": [-3.0] * 16, "scale": float(f32(3.0) / f32(15.0)), "zp": 15,
             "q": [0] * 16},
            {"name": "ramp", "data": ramp, "scale": 1.0, "zp": 0, "q": list(range(16))},
            {"name": "neg_ramp", "data": negramp, "scale": 1.0, "zp": 15, "q": list(range(16))},
        ],
        "java_round": [[0.5, 1], [-0.5, 0], [1.5, 2], [-1.5, -1], [2.5, 3], [-2.5, -2],
                       [0.49999997, 0], [-0.49999997, 0], [7.5, 8], [1e10, 2147483647],
                       [-1e10, -2147483648]],
        "tied_block_size": [[896, 128], [576, 64], [96, 32], [48, 16], [40, 0]],
    }
    with open(os.path.join(HERE, "quantizer.json"), "w") as f:
        json.dump(qz, f, indent=1)


if __name__ == "__main__":
    main()
