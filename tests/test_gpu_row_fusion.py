"""Row fusion on the device (mnb_weight_fuse_rows) against byte concatenation.

The reference fuses QKV / gate_up by concatenating the parts' triplets along
N (QwenGpuKernels.java:243-315; the oracle's fuse_rows restates it and is
pinned by the concatenation identity in tests/test_oracle.py).  Bars:
* the fused weight dequantizes bit-exactly to the row concatenation of the
  parts' dequantized rows, and to the weight created from the host-fused
  triplet;
* its products equal, bit for bit, those of the weight created from the
  host-fused triplet (same values, same kernels), and match the separate
  parts' products within 1e-3 * sqrt(K) * max|x| * max|w|
  (WarpDenseProjectionFusionParityTest.java:81-103 compares fused and
  separate outputs the same way).
"""
import sys

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


def make_part(ctx, seed, N, K, bs, zp=True, f32_scales=False):
    t = synth.make_weight(seed, N, K, bs, with_zp=zp)
    if f32_scales:  # fp32 scales that fp16 cannot hold: the device keeps fp32
        s = orc.fp16_bits_to_fp32(t.scales_f16.view(np.uint16)) * np.float32(1.0 + 2.0 ** -20)
        s = s.astype(np.float32)
    else:
        s = t.scales_f16
    w = mnb_hip.Weight(ctx, N, K, bs, t.q, s, t.zp_row_padded if zp else None,
                       mnb_hip.MNB_ZP_ROW_PADDED if zp else None)
    s32 = s if f32_scales else orc.fp16_bits_to_fp32(t.scales_f16.view(np.uint16))
    zflat = synth.zp_row_padded_to_flat(t.zp_row_padded, N, t.kb) if zp else orc.zp_default(N * t.kb)
    return w, (t.q.reshape(N, -1), np.asarray(s32, np.float32).reshape(N, -1), zflat, N, t.kb)


def nibbles(flat, count):
    b = np.asarray(flat, np.uint8)
    return np.stack([b & 0xF, b >> 4], axis=1).reshape(-1)[:count]


def pack_nibbles(nib):
    nib = np.asarray(nib, np.uint8)
    if nib.size % 2:
        nib = np.append(nib, 0)
    return (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)


def host_fused(ctx, arrays, K, bs, any_zp):
    """The concatenated triplet on the host (rows of q and scales, the flat
    zero-point streams joined nibble by nibble), uploaded with
    mnb_weight_create.  Where the reference's tryFuseQuantizedRowwise accepts
    the parts (every non-last N_i*kb even), the oracle's restatement of it
    must give the same arrays."""
    kb = arrays[0][4]
    N = sum(a[3] for a in arrays)
    fq = np.concatenate([a[0] for a in arrays]).reshape(-1)
    fs = np.concatenate([a[1] for a in arrays]).reshape(-1)
    fz = pack_nibbles(np.concatenate([nibbles(a[2], a[3] * kb) for a in arrays]))
    ref = orc.fuse_rows([(a[0], a[1], a[2], a[3], kb * bs, bs) for a in arrays])
    if all(a[3] * kb % 2 == 0 for a in arrays[:-1]):
        rq, rs, rz, rn = ref
        assert rn == N and np.array_equal(rq, fq) and np.array_equal(rs.view(np.uint32), fs.view(np.uint32))
        assert np.array_equal(rz, fz)
    else:
        assert ref is None  # the reference falls back to fp32 here
    w = mnb_hip.Weight(ctx, N, K, bs, fq, fs, fz if any_zp else None, mnb_hip.MNB_ZP_FLAT if any_zp else None)
    return w, (fq, fs, fz, N)


@pytest.mark.parametrize("case", [
    # (name, K, bs, [(N, zp, f32_scales)])
    ("phi3_qkv_bs32", 3072, 32, [(3072, False, False)] * 3),
    ("phi3_gate_up_bs128_zp", 3072, 128, [(8192, True, False)] * 2),
    ("qwen_qkv_odd_rows", 896, 64, [(896, True, False), (129, True, False), (127, True, False)]),
    ("odd_nibbles_k576_bs64", 576, 64, [(5, True, False), (7, True, False), (33, True, False)]),
    ("mixed_zp_and_scale_types", 1536, 32, [(48, True, False), (40, False, False), (24, True, True)]),
    ("tail_k576_bs128", 576, 128, [(17, True, False), (300, False, True)]),
])
def test_fused_rows_equal_concatenation(ctx, case):
    name, K, bs, spec = case
    say("case", name)
    parts, arrays = [], []
    try:
        for i, (N, zp, f32) in enumerate(spec):
            w, a = make_part(ctx, 100 * i + N, N, K, bs, zp, f32)
            parts.append(w)
            arrays.append(a)
        fused = mnb_hip.Weight.fuse_rows(ctx, parts)
        parts.append(fused)
        Nf = sum(a[3] for a in arrays)
        assert (fused.N, fused.K, fused.block_size) == (Nf, K, bs)
        # dequantize: bit-exact row concatenation of the parts
        dq = fused.dequantize(np.float32)
        cat = np.concatenate([p.dequantize(np.float32) for p in parts[:-1]])
        assert np.array_equal(dq.view(np.uint32), cat.view(np.uint32))
        # the same weight as the host-fused triplet
        any_zp = any(zp for _, zp, _ in spec)
        hf, (fq, fs, fz, _) = host_fused(ctx, arrays, K, bs, any_zp)
        parts.append(hf)
        assert np.array_equal(hf.dequantize(np.float32).view(np.uint32), dq.view(np.uint32))
        kp = arrays[0][4] * bs
        ref = orc.dequantize(fq, fs, fz, Nf, kp, bs)
        assert np.array_equal(dq.view(np.uint32), ref[:, :K].view(np.uint32))
        for M in (1, 40):
            x16 = synth.make_x(M, M, K)
            y = fused.matmul(x16, out_dtype=np.float32).reshape(M, Nf)
            y_hf = hf.matmul(x16, out_dtype=np.float32).reshape(M, Nf)
            assert np.array_equal(y.view(np.uint32), y_hf.view(np.uint32)), "fused != host-fused weight"
            tol = orc.tolerance(K, x16.astype(np.float32), dq)
            off = 0
            for p, a in zip(parts, arrays):
                ys = p.matmul(x16, out_dtype=np.float32).reshape(M, a[3])
                err = float(np.max(np.abs(ys - y[:, off:off + a[3]])))
                assert err <= tol, (M, err, tol)
                off += a[3]
            say("  M=%d fused == host-fused bitwise; parts within %.2e" % (M, tol))
    finally:
        for p in parts:
            p.close()


def test_fuse_errors(ctx):
    a, _ = make_part(ctx, 1, 16, 256, 32)
    b, _ = make_part(ctx, 2, 16, 288, 32)
    c, _ = make_part(ctx, 3, 16, 256, 64)
    try:
        with pytest.raises(mnb_hip.IllegalArgumentException,
                           match=r"^part 1 has K=288 blockSize=32 but expected K=256 blockSize=32$"):
            mnb_hip.Weight.fuse_rows(ctx, [a, b])
        with pytest.raises(mnb_hip.IllegalArgumentException, match=r"^part 2 has K=256 blockSize=64"):
            mnb_hip.Weight.fuse_rows(ctx, [a, a, c])
        with pytest.raises(mnb_hip.IllegalArgumentException, match="at least one part"):
            mnb_hip.Weight.fuse_rows(ctx, [])
        one = mnb_hip.Weight.fuse_rows(ctx, [a])  # a single part is a copy
        assert np.array_equal(one.dequantize().view(np.uint32), a.dequantize().view(np.uint32))
        one.close()
    finally:
        for w in (a, b, c):
            w.close()
