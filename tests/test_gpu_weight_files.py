"""GPU parity of weights loaded from files (mnb_pack_weight_create).

A triplet opened from a .wdmlpack package or an ONNX model and uploaded
straight from the file mapping must give the same device weight as the
reference's loaded QuantizedWeight: dequantize bit-exact to the oracle's
dequantizeInt4 over the reference-form arrays (fp32 scales after the
loader's fp16ToFp32, flat zero points), and matmul within
1e-3 * sqrt(K) * max|x| * max|w| of the oracle's fp32 product.
"""
import sys

import numpy as np
import pytest

import mnb_hip
import mnb_oracle as orc
import weightfiles as wf
from mnb_hip import Pack, synth

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


def check_weight(ctx, w, q, s, z, N, K, bs, Ms=(1, 33), seed=0, true_k=None):
    """Device weight vs the oracle on the same reference-form arrays."""
    say("  check N=%d K=%d bs=%d" % (N, K, bs))
    ref = orc.dequantize(q, s, z, N, K, bs)
    got = w.dequantize(np.float32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), "dequantize is not bit-exact"
    kt = true_k or K
    for M in Ms:
        x16 = synth.make_x(seed + M, M, K)
        x16[:, kt:] = 0
        x = x16.astype(np.float32)
        y = w.matmul(x16, out_dtype=np.float32).reshape(M, N)
        y_ref = orc.matmul(q, s, z, N, K, bs, x)
        tol = orc.tolerance(kt, x, ref)
        err = float(np.max(np.abs(y - y_ref)))
        say("    M=%d max|err| %.3e tol %.3e" % (M, err, tol))
        assert err <= tol


@pytest.mark.parametrize("bs", [32, 128])
def test_phi3_package_roles_upload_from_mapping(ctx, tmp_path, bs):
    """Phi-3 package triplets (fp32 scales, flat zero points, q dims [N,K,bs])
    at Phi-3 projection widths, uploaded role by role; the pack is closed
    before the weights are used (the host copy is released, the weights stay)."""
    roles = [("layers.0.qkv_proj", 192, 3072, 1), ("layers.0.down_proj", 96, 8192, 2), ("lm_head", 160, 3072, 3)]
    payload, expect = [], {}
    for role, N, K, seed in roles:
        t = synth.make_weight(seed, N, K, bs, with_zp=True)
        s32 = orc.fp16_bits_to_fp32(t.scales_f16.view(np.uint16))
        z = synth.zp_row_padded_to_flat(t.zp_row_padded, N, t.kb)
        payload += wf.phi3_triplet_tensors(role, t.q.tobytes(), N, K, bs, s32, z.tobytes())
        expect[role] = (t.q, s32, z, N, K)
    p = tmp_path / "model_phi3.wdmlpack"
    wf.write_wdmlpack(p, wf.phi3_manifest(), payload)
    pk = Pack(str(p))
    weights = {role: pk.weight(ctx, role) for role, *_ in roles}
    pk.close()
    try:
        for role, (q, s, z, N, K) in expect.items():
            say("role", role)
            w = weights[role]
            assert (w.N, w.K, w.block_size) == (N, K, bs)
            check_weight(ctx, w, q, s, z, N, K, bs, seed=N)
    finally:
        for w in weights.values():
            w.close()


@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("K,N", [(576, 1536), (1536, 576)])
def test_onnx_external_triplets_with_odd_block_counts(ctx, tmp_path, bs, K, N):
    """ONNX MatMulNBits, fp16 scales and row-padded zero points in
    model.onnx_data, at the odd-kb shapes (K=576: kb=9 at bs=64, kb=5 and
    K=640 at bs=128): the reference's K = kb*bs, x zero past the true K."""
    t = synth.make_weight(bs + K, N, K, bs, with_zp=True)
    b = wf.OnnxBuilder()
    b.matmul_nbits("/model/layers.3/mlp/down_proj/MatMul_output_0", N, K, bs, t.q.reshape(N, t.kb, bs // 2),
                   t.scales_f16.view(np.uint16), zp=t.zp_row_padded, external=True)
    with Pack(b.write(str(tmp_path))) as pk:
        name = pk.find_projection(3, "down_proj")
        w = pk.weight(ctx, name)
        q, s, z = pk.read(name)
    try:
        kp = t.kb * bs
        assert (w.N, w.K) == (N, kp)
        check_weight(ctx, w, q, s, z, N, kp, bs, Ms=(1, 7, 33), seed=K, true_k=K)
    finally:
        w.close()


def test_subnormal_scales_and_default_zero_points(ctx, tmp_path):
    """fp16 scales with subnormals widen to the reference's values (not fp16
    values: the device keeps fp32 scales); a missing zero-point input and an
    all-8 stored stream both give the implicit zero point."""
    N, K, bs = 64, 512, 32
    t = synth.make_weight(77, N, K, bs)
    s16 = t.scales_f16.view(np.uint16).copy()
    s16[::7] = np.arange(1, s16[::7].size + 1, dtype=np.uint16)  # subnormal fp16 patterns
    b = wf.OnnxBuilder()
    q3 = t.q.reshape(N, t.kb, bs // 2)
    b.matmul_nbits("sub", N, K, bs, q3, s16)
    b.matmul_nbits("all8", N, K, bs, q3, t.scales_f16.view(np.uint16),
                   zp=np.full((N, (t.kb + 1) // 2), 0x88, np.uint8))
    with Pack(b.write(str(tmp_path))) as pk:
        ws = {n: pk.weight(ctx, n) for n in ("sub", "all8")}
        arrays = {n: pk.read(n) for n in ("sub", "all8")}
    try:
        q, s, z = arrays["sub"]
        assert np.array_equal(s.view(np.uint32), orc.fp16_bits_to_fp32(s16).view(np.uint32))
        assert np.array_equal(z, orc.zp_default(N * t.kb))
        check_weight(ctx, ws["sub"], q, s, z, N, K, bs)
        q, s, z = arrays["all8"]
        check_weight(ctx, ws["all8"], q, s, z, N, K, bs)
    finally:
        for w in ws.values():
            w.close()


def test_upload_errors_name_the_weight(ctx, tmp_path):
    """A triplet the device path cannot take (block size 4, as in the
    reference's tiny package test) fails with the weight's name."""
    q, s, z = wf.reference_quant(6, 4, 4, 1)
    p = tmp_path / "m.wdmlpack"
    wf.write_wdmlpack(p, wf.phi3_manifest(), wf.phi3_triplet_tensors("lm_head", q.tobytes(), 6, 4, 4, s,
                                                                      z.tobytes()))
    with Pack(str(p)) as pk:
        with pytest.raises(mnb_hip.IllegalArgumentException, match=r"^lm_head: block_size=4 must be a power of two"):
            pk.weight(ctx, "lm_head")
