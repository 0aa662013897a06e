"""Weight files on the CPU: the loader in libmnb_hip.so (mnb_pack_*) opens
.wdmlpack packages and ONNX models and resolves MatMulNBits triplets the way
the reference loads them.  No device is used: these tests call only the
parsing entry points (mnb_pack_open / info / read_weight).

What pins the loader:
* byte-exact round trips of the reference test's deterministic triplets
  (Phi3WdmlPackCompilerTest.java:150-239: same generator, same config);
* scale widening checked against the oracle's restatement of the
  reference's fp16ToFp32 (pinned itself by tests/test_oracle.py), including
  subnormal scales;
* zero-point normalization checked against the oracle's
  normalizeRawUInt4ZeroPoints restatement (pinned by byte-level KATs in
  tests/test_oracle.py), over every layout branch (Q2W:1017-1048);
* the IOException texts of the reference for each failure it reports
  (WdmlPackWriter.java:143-177, 254-259; WdmlPackManifest.java:108-123;
  WdmlPackReader.java:67-96; Phi3RuntimePackage.java:35-46, 132-152;
  Qwen2Weights.java:936-976, 1017-1104, 2063-2117).
"""
import json
import os
import struct

import numpy as np
import pytest

import mnb_hip
import mnb_oracle as orc
import weightfiles as wf
from mnb_hip import IOException, Pack


def _err(path, match):
    with pytest.raises(IOException, match=match):
        Pack(str(path))


# ---------------------------------------------------------------------------
# Phi-3 packages
# ---------------------------------------------------------------------------

REF_LAYER_ROLES = [  # (role, N, K, seed) of Phi3WdmlPackCompilerTest.syntheticWeights, h=4, inter=8, bs=4
    ("lm_head", 6, 4, 1),
    ("layers.0.q_proj", 4, 4, 2), ("layers.0.k_proj", 4, 4, 3), ("layers.0.v_proj", 4, 4, 4),
    ("layers.0.o_proj", 4, 4, 5), ("layers.0.gate_up_proj", 16, 4, 6), ("layers.0.down_proj", 4, 8, 7),
]


def _ref_package(path, roles=REF_LAYER_ROLES, bs=4, manifest=None, drop=(), edit=None):
    payload = [("embed_tokens", wf.FLOAT, [24], np.arange(24, dtype="<f4").tobytes())]
    expect = {}
    for role, n, k, seed in roles:
        q, s, z = wf.reference_quant(n, k, bs, seed)
        expect[role] = (q, s, z, n, k)
        payload += wf.phi3_triplet_tensors(role, q.tobytes(), n, k, bs, s, z.tobytes())
    payload = [t for t in payload if t[0] not in drop]
    if edit:
        payload = [edit(t) for t in payload]
    wf.write_wdmlpack(path, manifest or wf.phi3_manifest(), payload)
    return expect


def test_phi3_reference_triplets_round_trip_byte_exact(tmp_path):
    """Phi3WdmlPackCompilerTest.syntheticWeightsRoundTripThroughPackage: every
    INT4 triplet comes back byte-exact (q, fp32 scales, zero points) with its
    N, K and block size."""
    p = tmp_path / "model_phi3.wdmlpack"
    expect = _ref_package(p)
    with Pack(str(p)) as pk:
        assert pk.kind == mnb_hip.MNB_PACK_PHI3
        assert pk.names() == [r for r, *_ in REF_LAYER_ROLES]
        for role, (q, s, z, n, k) in expect.items():
            i = pk.info(role)
            assert (i.N, i.K, i.block_size, i.blocks_per_row) == (n, k, 4, k // 4)
            assert i.zp_implicit == 0 and i.scale_dtype == wf.FLOAT
            gq, gs, gz = pk.read(role)
            assert np.array_equal(gq, q)
            assert np.array_equal(gs.view(np.uint32), s.view(np.uint32))
            assert np.array_equal(gz, z)


def test_phi3_package_layout_is_the_reference_writers(tmp_path):
    """The container the writer produces has the documented layout, so the
    reader is tested on what the reference writes: manifest at 64, payload at
    a 4096 boundary, tensors 64-byte aligned relative to the payload."""
    p = tmp_path / "a.wdmlpack"
    _ref_package(p)
    raw = p.read_bytes()
    assert raw[:8] == b"WDMLPACK"
    ver, flags, mo, ml, do, dl, po, pl = struct.unpack_from("<ii6q", raw, 8)
    assert (ver, flags, mo, do, dl) == (1, 0, 64, 0, 0)
    assert po % 4096 == 0 and po >= 64 + ml and po + pl == len(raw)
    m = json.loads(raw[mo:mo + ml])
    assert all(t["payloadOffset"] % 64 == 0 for t in m["tensors"])


def test_phi3_realistic_triplet_scales_match_fp16_widening(tmp_path):
    """A Phi-3 package stores the scales the compiler widened with fp16ToFp32
    (Phi3WdmlPackCompiler.java:270-285); the loader returns those fp32 values
    unchanged, and they equal the oracle's widening of the fp16 source."""
    N, K, bs = 48, 256, 32
    from mnb_hip import synth
    t = synth.make_weight(11, N, K, bs)
    s16 = t.scales_f16.view(np.uint16)
    s16 = s16.copy()
    s16[:4] = [0x0001, 0x03FF, 0x8200, 0x0000]  # subnormals and zero
    s32 = orc.fp16_bits_to_fp32(s16)
    zp = orc.zp_default(N * (K // bs))
    p = tmp_path / "m.wdmlpack"
    wf.write_wdmlpack(p, wf.phi3_manifest(), wf.phi3_triplet_tensors("layers.0.o_proj", t.q.tobytes(), N, K, bs,
                                                                    s32, zp.tobytes()))
    with Pack(str(p)) as pk:
        q, s, z = pk.read("layers.0.o_proj")
        assert np.array_equal(s.view(np.uint32), s32.view(np.uint32))
        assert np.array_equal(q, t.q) and np.array_equal(z, zp)


def test_wdmlpack_header_errors(tmp_path):
    p = tmp_path / "x.wdmlpack"
    p.write_bytes(b"WDMLPACK" + b"\0" * 10)
    _err(p, r"^Invalid wdmlpack: file is smaller than header: .*x\.wdmlpack$")
    wf.write_wdmlpack(p, wf.phi3_manifest(), header_override={"magic": b"WDMLPAKK"})
    _err(p, r"^Invalid wdmlpack magic: WDMLPAKK$")
    wf.write_wdmlpack(p, wf.phi3_manifest(), header_override={"version": 2})
    _err(p, r"^Unsupported wdmlpack version: 2$")
    wf.write_wdmlpack(p, wf.phi3_manifest(), header_override={"manifest_off": 10})
    size = p.stat().st_size
    _err(p, r"^Invalid wdmlpack manifest range: offset=10, length=\d+, fileSize=%d$" % size)
    wf.write_wdmlpack(p, wf.phi3_manifest(), header_override={"manifest_len": 1 << 40})
    _err(p, r"^Invalid wdmlpack manifest range: offset=64, length=1099511627776, fileSize=\d+$")
    wf.write_wdmlpack(p, wf.phi3_manifest(), header_override={"payload_off": 4096, "payload_len": 1 << 20})
    _err(p, r"^Invalid wdmlpack payload range: offset=4096, length=1048576, fileSize=\d+$")
    wf.write_wdmlpack(p, wf.phi3_manifest(), header_override={"payload_off": 0, "payload_len": -5})
    _err(p, r"^Invalid wdmlpack payload range: offset=0, length=-5")


def test_wdmlpack_manifest_errors(tmp_path):
    p = tmp_path / "x.wdmlpack"
    m = wf.phi3_manifest()
    m["format"] = "zip"
    wf.write_wdmlpack(p, m)
    _err(p, r"^Invalid wdmlpack manifest format: zip$")
    m = wf.phi3_manifest()
    del m["format"]
    wf.write_wdmlpack(p, m)
    _err(p, r"^Invalid wdmlpack manifest format: null$")
    m = wf.phi3_manifest(version=2)
    wf.write_wdmlpack(p, m)
    _err(p, r"^Unsupported wdmlpack manifest version: 2$")
    m = wf.phi3_manifest(version="1")  # WdmlPackManifest.intValue accepts numeric strings
    wf.write_wdmlpack(p, m, wf.phi3_triplet_tensors("lm_head", b"\x11" * 32, 2, 32, 32, [0.5, 0.25], b"\x88"))
    assert Pack(str(p)).names() == ["lm_head"]
    # payloadIncluded must agree with the container
    wf.write_wdmlpack(p, wf.phi3_manifest())
    _err(p, r"^wdmlpack manifest says payloadIncluded=true but the container header has no payload$")
    wf.write_wdmlpack(p, wf.phi3_manifest(payloadIncluded=False),
                      wf.phi3_triplet_tensors("lm_head", b"\x11" * 32, 2, 32, 32, [0.5, 0.25], b"\x88"))
    _err(p, r"^wdmlpack container has payload but manifest says payloadIncluded=false$")
    # a manifest-only flag makes the header payload-less
    wf.write_wdmlpack(p, wf.phi3_manifest(), wf.phi3_triplet_tensors("lm_head", b"\x11" * 32, 2, 32, 32,
                                                                      [0.5, 0.25], b"\x88"), flags=1)
    _err(p, r"^wdmlpack manifest says payloadIncluded=true but the container header has no payload$")
    # JSON syntax
    raw = bytearray(open(wf.write_wdmlpack(p, wf.phi3_manifest()), "rb").read())
    raw[64] = ord("[")
    p.write_bytes(bytes(raw))
    _err(p, r"^Invalid wdmlpack manifest JSON at byte \d+: ")


def test_phi3_package_errors(tmp_path):
    p = tmp_path / "x.wdmlpack"
    trip = wf.phi3_triplet_tensors("lm_head", b"\x11" * 32, 2, 32, 32, [0.5, 0.25], b"\x88")
    wf.write_wdmlpack(p, wf.phi3_manifest(runtimeLoadable=False), trip)
    _err(p, r"^Phi-3 wdmlpack is not a runtime-loadable payload package: .*x\.wdmlpack$")
    wf.write_wdmlpack(p, wf.phi3_manifest(architecture="llama"), trip)
    _err(p, r"^Unsupported wdmlpack architecture: llama")
    wf.write_wdmlpack(p, dict(wf.phi3_manifest(), tensors="none"), trip)
    _err(p, r"^Invalid wdmlpack: missing tensors directory$")
    # tensor range outside the payload
    m = wf.phi3_manifest()
    wf.write_wdmlpack(p, m, trip)
    raw = p.read_bytes()
    ml = struct.unpack_from("<q", raw, 24)[0]
    man = json.loads(raw[64:64 + ml])
    man["tensors"][1]["payloadOffset"] = 1 << 20
    wf.write_wdmlpack(p, dict(man), trip)
    _err(p, r"^Invalid wdmlpack tensor payload range for lm_head\.scales: offset=1048576, length=8$")
    # a missing zero-point tensor and a qweight with 2 dims
    _ref_package(p, drop=("layers.0.k_proj.zeropoints",))
    with Pack(str(p)) as pk:
        assert pk.info("layers.0.q_proj").N == 4
        with pytest.raises(IOException, match=r"^Phi-3 wdmlpack is missing payload tensor: "
                                              r"layers\.0\.k_proj\.zeropoints$"):
            pk.info("layers.0.k_proj")
        with pytest.raises(IOException, match=r"^Phi-3 wdmlpack is missing payload tensor: nope\.qweight$"):
            pk.read("nope")
    _ref_package(p, edit=lambda t: (t[0], t[1], t[2][:2], t[3]) if t[0] == "lm_head.qweight" else t)
    with Pack(str(p)) as pk:
        with pytest.raises(IOException, match=r"^Phi-3 qweight 'lm_head' must encode dims \[N,K,blockSize\], "
                                              r"got 2 dims$"):
            pk.info("lm_head")


# ---------------------------------------------------------------------------
# ONNX models
# ---------------------------------------------------------------------------

def _onnx_weight(seed, N, K, bs):
    from mnb_hip import synth
    t = synth.make_weight(seed, N, K, bs, with_zp=True)
    kb = t.kb
    q3 = t.q.reshape(N, kb, bs // 2)
    return t, q3, kb


@pytest.mark.parametrize("bs,K,N", [(32, 576, 40), (64, 576, 24), (128, 576, 17), (128, 1536, 12)])
@pytest.mark.parametrize("external", [False, True])
def test_onnx_matmulnbits_triplets_follow_qwen2weights(tmp_path, bs, K, N, external):
    """ONNX MatMulNBits with fp16 scales and row-padded zero points, the
    shapes of the odd-kb edge cases (K=576: kb=9 at bs=64, kb=5 at bs=128,
    where the reference pads K to 640): N, K=kb*bs and bs from the q dims,
    scales widened with fp16ToFp32, zero points repacked to the flat stream."""
    t, q3, kb = _onnx_weight(bs + K + N, N, K, bs)
    b = wf.OnnxBuilder()
    b.matmul_nbits("/model/layers.0/attn/q_proj/MatMul_output_0", N, K, bs, q3, t.scales_f16.view(np.uint16),
                   zp=t.zp_row_padded, external=external)
    path = b.write(str(tmp_path))
    with Pack(path) as pk:
        assert pk.kind == mnb_hip.MNB_PACK_ONNX
        name = pk.names()[0]
        i = pk.info(name)
        assert (i.N, i.K, i.block_size, i.blocks_per_row) == (N, kb * bs, bs, kb)
        assert i.scale_dtype == wf.FLOAT16 and i.zp_implicit == 0
        q, s, z = pk.read(name)
        assert np.array_equal(q, t.q)
        assert np.array_equal(s.view(np.uint32), orc.fp16_bits_to_fp32(t.scales_f16.view(np.uint16)).view(np.uint32))
        assert np.array_equal(z, orc.zp_normalize_raw(t.zp_row_padded, [N, (kb + 1) // 2], N, kb))
        assert np.array_equal(z, orc.zp_repack_row_padded(t.zp_row_padded, N, kb))


@pytest.mark.parametrize("layout", ["row_dims", "unpacked_dims", "row_flat_len", "flat_len", "unpacked_len"])
def test_onnx_zero_point_layout_branches(tmp_path, layout):
    """Every branch of normalizeRawUInt4ZeroPoints (Q2W:1017-1048), checked
    against the oracle's restatement of it."""
    N, K, bs = 6, 96, 32  # kb = 3 (odd): row-padded and flat streams differ
    t, q3, kb = _onnx_weight(5, N, K, bs)
    rng = np.random.default_rng(1)
    unpacked = rng.integers(0, 16, N * kb).astype(np.uint8)
    flat = orc.zp_pack_unpacked_u8(unpacked, N, kb)
    data, dims = {
        "row_dims": (t.zp_row_padded, [N, (kb + 1) // 2]),
        "unpacked_dims": (unpacked | 0xA0, [N, kb]),          # high nibbles are ignored
        "row_flat_len": (t.zp_row_padded, [t.zp_row_padded.size]),
        "flat_len": (flat, [flat.size]),
        "unpacked_len": (unpacked, [unpacked.size]),
    }[layout]
    b = wf.OnnxBuilder()
    b.matmul_nbits("w", N, K, bs, q3, t.scales_f16.view(np.uint16), zp=data, zp_dims=dims)
    with Pack(b.write(str(tmp_path))) as pk:
        _, _, z = pk.read("w")
    assert np.array_equal(z, orc.zp_normalize_raw(data, dims, N, kb))


def test_onnx_zero_point_errors(tmp_path):
    N, K, bs = 6, 96, 32
    t, q3, kb = _onnx_weight(5, N, K, bs)
    b = wf.OnnxBuilder()
    b.matmul_nbits("w", N, K, bs, q3, t.scales_f16.view(np.uint16), zp=np.zeros(7, np.uint8), zp_dims=[7])
    with Pack(b.write(str(tmp_path / "a"))) as pk:
        with pytest.raises(IOException, match=r"^Unexpected zero-point layout for w_zp: dims=\[7\], bytes=7, "
                                              r"expected packed row layout \[6, 2\], flat packed bytes 9, "
                                              r"or unpacked \[6, 3\]$"):
            pk.read("w")
    b = wf.OnnxBuilder()
    b.matmul_nbits("w", N, K, bs, q3, t.scales_f16.view(np.uint16), zp=np.zeros(5, np.uint8), zp_dims=[N, 2])
    with Pack(b.write(str(tmp_path / "b"))) as pk:
        with pytest.raises(IOException, match=r"^Zero-point tensor w_zp is truncated: 5 bytes, "
                                              r"expected at least 12$"):
            pk.read("w")
    b = wf.OnnxBuilder()
    b.matmul_nbits("w", N, K, bs, q3, t.scales_f16.view(np.uint16), zp=np.zeros(10, np.uint8), zp_dims=[N, kb])
    with Pack(b.write(str(tmp_path / "c"))) as pk:
        with pytest.raises(IOException, match=r"^Zero-point tensor w_zp is truncated: 10 values, expected 18$"):
            pk.read("w")


def test_onnx_missing_zero_points_are_eight(tmp_path):
    """No zero-point input (or an empty optional-input name): the default
    stream 0x88... (Q2W:1107-1112)."""
    N, K, bs = 5, 96, 32
    t, q3, kb = _onnx_weight(3, N, K, bs)
    b = wf.OnnxBuilder()
    b.matmul_nbits("a", N, K, bs, q3, t.scales_f16.view(np.uint16))
    b.matmul_nbits("b", N, K, bs, q3, t.scales_f16.view(np.uint16), prefix="b", zp_input="")
    with Pack(b.write(str(tmp_path))) as pk:
        for name in ("a", "b"):
            i = pk.info(name)
            assert i.zp_implicit == 1 and i.zp_bytes == (N * kb + 1) // 2
            assert np.array_equal(pk.read(name)[2], orc.zp_default(N * kb))


def test_onnx_fp32_scales_and_int32_data_encodings(tmp_path):
    """FLOAT scales are taken as stored; UINT8 and FLOAT16 tensors given as
    int32_data (one value per element) read like raw_data
    (OnnxModelReader.java:540-565)."""
    N, K, bs = 4, 64, 32
    t, q3, kb = _onnx_weight(9, N, K, bs)
    s32 = np.random.default_rng(2).uniform(-1, 1, N * kb).astype(np.float32)
    b = wf.OnnxBuilder()
    b.matmul_nbits("f32", N, K, bs, q3, s32, scale_dtype=wf.FLOAT)
    b.inits.append(wf.tensor_proto("i_Q4", wf.UINT8, [N, kb, bs // 2], int32_data=t.q.tolist()))
    b.inits.append(wf.tensor_proto("i_scales", wf.FLOAT16, [N, kb],
                                   int32_data=t.scales_f16.view(np.uint16).tolist()))
    b.inits.append(wf.tensor_proto("i_fd", wf.FLOAT, [N, kb], float_data=s32))
    b.nodes.append(wf.node_proto("MatMulNBits", ["x", "i_Q4", "i_scales"], ["i32"]))
    b.nodes.append(wf.node_proto("MatMulNBits", ["x", "i_Q4", "i_fd"], ["fd"]))
    with Pack(b.write(str(tmp_path))) as pk:
        assert pk.names() == ["f32", "i32", "fd"]
        q, s, _ = pk.read("f32")
        assert np.array_equal(s.view(np.uint32), s32.view(np.uint32)) and pk.info("f32").scale_dtype == wf.FLOAT
        q, s, _ = pk.read("i32")
        assert np.array_equal(q, t.q)
        assert np.array_equal(s.view(np.uint32), orc.fp16_bits_to_fp32(t.scales_f16.view(np.uint16)).view(np.uint32))
        assert np.array_equal(pk.read("fd")[1].view(np.uint32), s32.view(np.uint32))


def test_onnx_external_data_files(tmp_path):
    """External initializers resolve from model.onnx_data, else model.onnx.data,
    in the model's directory (QwenModelDirValidator.java:163-174); a raw_data
    stub longer than the file is skipped (OnnxModelReader.java:466-480)."""
    N, K, bs = 8, 64, 32
    t, q3, kb = _onnx_weight(4, N, K, bs)
    for data_name in ("model.onnx_data", "model.onnx.data"):
        d = tmp_path / data_name.replace(".", "_")
        b = wf.OnnxBuilder()
        b.matmul_nbits("w", N, K, bs, q3, t.scales_f16.view(np.uint16), zp=t.zp_row_padded, external=True,
                       data_file=data_name)
        with Pack(b.write(str(d), data_name=data_name)) as pk:
            q, _, _ = pk.read("w")
            assert np.array_equal(q, t.q)
    d = tmp_path / "missing"
    b = wf.OnnxBuilder()
    b.matmul_nbits("w", N, K, bs, q3, t.scales_f16.view(np.uint16), external=True)
    path = b.write(str(d))
    os.remove(os.path.join(str(d), "model.onnx_data"))
    _err(path, r"^Required file missing: model\.onnx_data \(or model\.onnx\.data\) \(looked in .*missing\)$")
    # an external tensor that also carries an oversized raw_data stub
    d = tmp_path / "stub"
    b = wf.OnnxBuilder()
    b.matmul_nbits("w", N, K, bs, q3, t.scales_f16.view(np.uint16), external=True)
    off = len(b.ext) - t.scales_f16.nbytes
    b.inits[1] = (wf.tensor_proto("w_scales", wf.FLOAT16, [N, kb], external=("model.onnx_data", off,
                                                                            t.scales_f16.nbytes))
                  + wf.key(9, 2) + wf.varint(1 << 40))
    with Pack(b.write(str(d))) as pk:
        assert np.array_equal(pk.read("w")[1].view(np.uint32),
                              orc.fp16_bits_to_fp32(t.scales_f16.view(np.uint16)).view(np.uint32))
    # out-of-range external reference
    d = tmp_path / "range"
    b = wf.OnnxBuilder()
    b.matmul_nbits("w", N, K, bs, q3, t.scales_f16.view(np.uint16), external=True)
    b.inits[0] = wf.tensor_proto("w_Q4", wf.UINT8, [N, kb, bs // 2], external=("model.onnx_data", 1 << 30, 128))
    with Pack(b.write(str(d))) as pk:
        with pytest.raises(IOException, match=r"^External tensor w_Q4 lies outside .*model\.onnx_data: "
                                              r"offset=1073741824, length=128, fileSize=\d+$"):
            pk.read("w")


def test_onnx_graph_errors(tmp_path):
    N, K, bs = 4, 64, 32
    t, q3, kb = _onnx_weight(6, N, K, bs)
    p = tmp_path / "empty.onnx"
    p.write_bytes(wf.vfield(1, 8))
    _err(p, r"^No graph found in ONNX model$")
    p.write_bytes(wf.model_proto(wf.graph_proto([wf.node_proto("MatMulNBits", ["x", "q", "s"], ["y"])], [])))
    _err(p, r"^No ONNX tensor initializers found in selected model file$")
    b = wf.OnnxBuilder()
    b.matmul_nbits("w", N, K, bs, q3, t.scales_f16.view(np.uint16))
    b.nodes.append(wf.node_proto("MatMulNBits", ["x", "nope", "w_scales"], ["v"]))
    _err(b.write(str(tmp_path / "a")), r"^Required quantized weight tensor not found: nope$")
    b = wf.OnnxBuilder()
    b.matmul_nbits("w", N, K, bs, q3, t.scales_f16.view(np.uint16))
    b.inits.append(wf.tensor_proto("bad", wf.INT32, [4], raw=b"\0" * 16))
    b.nodes.append(wf.node_proto("MatMulNBits", ["x", "w_Q4", "bad"], ["v"]))
    _err(b.write(str(tmp_path / "b")), r"^Tensor 'bad' has unsupported data type INT32 \(6\)$")
    b = wf.OnnxBuilder()
    b.inits.append(wf.tensor_proto("q2", wf.UINT8, [N, kb * bs // 2], raw=t.q.tobytes()))
    b.inits.append(wf.tensor_proto("s2", wf.FLOAT16, [N * kb], raw=t.scales_f16.tobytes()))
    b.inits.append(wf.tensor_proto("s3", wf.FLOAT16, [N * kb - 1], raw=t.scales_f16.tobytes()[:-2]))
    b.nodes.append(wf.node_proto("MatMulNBits", ["x", "q2", "s2"], ["dims2"]))
    b.matmul_nbits("w", N, K, bs, q3, t.scales_f16.view(np.uint16))
    b.nodes.append(wf.node_proto("MatMulNBits", ["x", "w_Q4", "s3"], ["short"]))
    with Pack(b.write(str(tmp_path / "c"))) as pk:
        with pytest.raises(IOException, match=r"^Unexpected dimensions for quantized weight q2: \[4, 32\], "
                                              r"expected \[N, blocks, packedBlock\]$"):
            pk.info("dims2")
        with pytest.raises(IOException, match=r"^Unexpected scale tensor size for s3: 7, expected 8 for "
                                              r"quantized weight w_Q4$"):
            pk.info("short")
        with pytest.raises(IOException, match=r"^Quantized weight not found: zzz$"):
            pk.info("zzz")
    p = tmp_path / "wire.onnx"
    p.write_bytes(wf.key(7, 3) + b"\0" * 8)
    _err(p, r"^Failed to parse ONNX model '.*wire\.onnx' at byte offset \d+ of 9 \(Unknown wire type: 3\)$")


def test_find_projection_mirrors_the_reference_lookup(tmp_path):
    """Q2W:800-815: the first MatMulNBits output (graph order) containing both
    "layers.<l>" and the projection name."""
    N, K, bs = 4, 64, 32
    t, q3, kb = _onnx_weight(6, N, K, bs)
    b = wf.OnnxBuilder()
    outs = ["/model/layers.%d/attn/%s/MatMul_output_0" % (l, p) for l in (0, 1, 10) for p in ("q_proj", "o_proj")]
    for o in outs:
        b.matmul_nbits(o, N, K, bs, q3, t.scales_f16.view(np.uint16))
    with Pack(b.write(str(tmp_path))) as pk:
        assert pk.names() == outs
        assert pk.find_projection(1, "o_proj") == outs[3]
        assert pk.find_projection(10, "q_proj") == outs[4]
        with pytest.raises(IOException, match=r"^Quantized weight not found for layer 2 q_proj$"):
            pk.find_projection(2, "q_proj")


# ---------------------------------------------------------------------------
# Qwen packages: payload (runtimeGraph) and manifest-only (source ONNX)
# ---------------------------------------------------------------------------

def _qwen_manifest(**kw):
    m = {"format": "wdmlpack", "version": 1, "mode": "payload", "payloadIncluded": True, "runtimeLoadable": True,
         "runtimeLoadMode": "qwen-native-payload", "model": {"architecture": "Qwen2", "hiddenSize": 64}}
    m.update(kw)
    return m


def test_qwen2_payload_package_resolves_runtime_graph(tmp_path):
    N, K, bs = 10, 192, 64
    t, q3, kb = _onnx_weight(21, N, K, bs)
    payload = [("lm_head_Q4", wf.UINT8, [N, kb, bs // 2], t.q.tobytes()),
               ("lm_head_scales", wf.FLOAT16, [N, kb], t.scales_f16.tobytes()),
               ("lm_head_zp", wf.UINT8, [N, (kb + 1) // 2], t.zp_row_padded.tobytes())]
    graph = {"nodes": [{"opType": "Add", "inputs": ["a", "b"], "outputs": ["c"]},
                       {"opType": "MatMulNBits", "inputs": ["x", "lm_head_Q4", "lm_head_scales", "lm_head_zp"],
                        "outputs": ["logits"]}]}
    p = tmp_path / "model_qwen.wdmlpack"
    wf.write_wdmlpack(p, _qwen_manifest(runtimeGraph=graph), payload)
    with Pack(str(p)) as pk:
        assert pk.kind == mnb_hip.MNB_PACK_QWEN2 and pk.names() == ["logits"]
        q, s, z = pk.read("logits")
        assert np.array_equal(q, t.q)
        assert np.array_equal(s.view(np.uint32), orc.fp16_bits_to_fp32(t.scales_f16.view(np.uint16)).view(np.uint32))
        assert np.array_equal(z, orc.zp_repack_row_padded(t.zp_row_padded, N, kb))
    wf.write_wdmlpack(p, _qwen_manifest(runtimeGraph=graph, runtimeLoadable=False,
                                        runtimeLoadMode="import-only"), payload)
    _err(p, r"^wdmlpack package is import-only and not runtime-loadable yet: import-only$")


def test_qwen2_manifest_only_package_opens_its_source_model(tmp_path):
    N, K, bs = 6, 64, 32
    t, q3, kb = _onnx_weight(22, N, K, bs)
    b = wf.OnnxBuilder()
    b.matmul_nbits("w", N, K, bs, q3, t.scales_f16.view(np.uint16), external=True)
    model = b.write(str(tmp_path))
    size = os.path.getsize(model)
    p = tmp_path / "model.wdmlpack"
    src = {"format": "onnx", "fileName": "model.onnx", "relativePath": "model.onnx", "sizeBytes": size}
    wf.write_wdmlpack(p, _qwen_manifest(payloadIncluded=False, mode="manifest", source=src), flags=1)
    with Pack(str(p)) as pk:
        assert pk.kind == mnb_hip.MNB_PACK_ONNX and pk.names() == ["w"]
        assert np.array_equal(pk.read("w")[0], t.q)
    wf.write_wdmlpack(p, _qwen_manifest(payloadIncluded=False, source=dict(src, sizeBytes=size + 1)), flags=1)
    _err(p, r"^wdmlpack source size mismatch for model\.onnx: manifest=%d, actual=%d$" % (size + 1, size))
    wf.write_wdmlpack(p, _qwen_manifest(payloadIncluded=False, source=dict(src, relativePath="../x.onnx")),
                      flags=1)
    _err(p, r"^Invalid wdmlpack source path escapes model directory: \.\./x\.onnx$")


def test_pack_handles_are_checked():
    import ctypes
    L = mnb_hip.load()
    h = ctypes.c_void_p()
    assert L.mnb_pack_open(None, ctypes.byref(h)) == mnb_hip.MNB_ERR_INVALID_ARGUMENT
    assert L.mnb_pack_close(None) == mnb_hip.MNB_OK
    n = ctypes.c_int32()
    assert L.mnb_pack_weight_count(None, ctypes.byref(n)) == mnb_hip.MNB_ERR_INVALID_ARGUMENT
    with pytest.raises(IOException, match="Cannot open"):
        Pack("/nonexistent/model.onnx")


def test_mutated_files_fail_cleanly(tmp_path):
    """Bit flips, truncations and overwritten bytes in valid files: the reader
    either opens the file or reports an IOException; reading every weight of
    what opens either succeeds or reports one.  (Run in-process: a crash or an
    out-of-range read would end the test run.)"""
    N, K, bs = 6, 192, 64
    t, q3, kb = _onnx_weight(3, N, K, bs)
    b = wf.OnnxBuilder()
    b.matmul_nbits("/model/layers.0/attn/q_proj/MatMul_output_0", N, K, bs, q3, t.scales_f16.view(np.uint16),
                   zp=t.zp_row_padded)
    b.matmul_nbits("w2", N, K, bs, q3, t.scales_f16.view(np.uint16))
    seeds = {"m.onnx": open(b.write(str(tmp_path / "src")), "rb").read()}
    pk_path = tmp_path / "p.wdmlpack"
    wf.write_wdmlpack(pk_path, wf.phi3_manifest(), wf.phi3_triplet_tensors(
        "lm_head", t.q.tobytes(), N, K, bs, np.ones(N * kb, np.float32), np.full(9, 0x88, np.uint8).tobytes()))
    seeds["m.wdmlpack"] = pk_path.read_bytes()
    rng = np.random.default_rng(7)
    opened = 0
    for fname, base in seeds.items():
        target = tmp_path / fname
        for _ in range(400):
            buf = bytearray(base)
            for _ in range(int(rng.integers(1, 4))):
                k = int(rng.integers(0, 3))
                i = int(rng.integers(0, len(buf)))
                if k == 0:
                    buf[i] ^= 1 << int(rng.integers(0, 8))
                elif k == 1:
                    buf[i] = int(rng.integers(0, 256))
                else:
                    del buf[i:]
                if not buf:
                    break
            target.write_bytes(bytes(buf))
            try:
                pk = Pack(str(target))
            except (IOException, mnb_hip.MnbError):
                continue
            opened += 1
            for name in pk.names():
                try:
                    pk.read(name)
                except (IOException, mnb_hip.MnbError):
                    pass
            pk.close()
    assert opened > 0


# ---------------------------------------------------------------------------
# The reference's real Phi-3 export
# ---------------------------------------------------------------------------

PHI3_EXPORT = "/root/reference/model/phi3-mini-directml-int4/directml/directml-int4-awq-block-128/model.onnx"


@pytest.mark.skipif(not os.path.exists(PHI3_EXPORT), reason="the reference checkout is not present")
def test_reference_phi3_export_resolves_every_matmulnbits_triplet(tmp_path):
    """The Phi-3-mini DirectML int4 AWQ export that the reference ships (its
    external weights are a download, model.onnx.data.url): the graph beside a
    sparse stand-in for model.onnx.data resolves 193 MatMulNBits triplets with
    the shapes of Phi-3-mini (32 layers of q, k, v, o 3072 -> 3072, gate
    3072 -> 16384 and down 8192 -> 3072, and the 3072 -> 32064 head), block
    size 128, explicit zero points and fp16 scales, as Qwen2Weights'
    MatMulNBits loading would (Q2W:534-545, 936-976); the layer lookup of
    loadQuantizedProjection (Q2W:800-815) finds each projection."""
    import collections
    import shutil
    model = tmp_path / "model.onnx"
    shutil.copyfile(PHI3_EXPORT, model)
    with open(tmp_path / "model.onnx.data", "wb") as f:
        f.truncate(4 << 30)          # sparse: every tensor range lies inside, read as zeros
    with Pack(str(model)) as pk:
        assert pk.kind == mnb_hip.MNB_PACK_ONNX
        names = pk.names()
        assert len(names) == 193
        shapes = collections.Counter()
        for n in names:
            i = pk.info(n)
            assert i.block_size == 128 and i.zp_implicit == 0 and i.scale_dtype == 10, n
            kb = i.K // 128
            assert i.blocks_per_row == kb and i.q_bytes == i.N * kb * 64 and i.scale_count == i.N * kb, n
            assert i.zp_bytes == (i.N * kb + 1) // 2, n
            shapes[(i.K, i.N)] += 1
        assert shapes == {(3072, 3072): 128, (3072, 16384): 32, (8192, 3072): 32, (3072, 32064): 1}
        for layer in (0, 17, 31):
            for proj in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "down_proj"):
                name = pk.find_projection(layer, proj)
                assert "layers.%d/" % layer in name and proj in name
                K, N = (pk.info(name).K, pk.info(name).N)
                assert (K, N) == {"down_proj": (8192, 3072), "gate_proj": (3072, 16384)}.get(proj, (3072, 3072))
        assert pk.info("logits").N == 32064
        q, s, z = pk.read(pk.find_projection(0, "q_proj"))
        assert q.size == 3072 * 24 * 64 and s.size == 3072 * 24 and z.size == 3072 * 24 // 2


# ---------------------------------------------------------------------------
# SafeTensors files (SafeTensorsReader.java:84-277)
# ---------------------------------------------------------------------------

def test_safetensors_reference_case_parses_header_and_payload(tmp_path):
    """SafeTensorsReaderTest.parsesHeaderAndMmapBackedPayload: an F16 [2, 2]
    embedding with metadata; dtype code 10 (toOnnxDataType), shape, bytes."""
    header = ('{"model.embed_tokens.weight":{"dtype":"F16","shape":[2,2],"data_offsets":[0,8]},'
              '"__metadata__":{"format":"pt"}}')
    p = wf.write_safetensors(tmp_path / "model.safetensors", [], header=header, tail=bytes(range(1, 9)))
    with Pack(p) as pk:
        assert pk.kind == mnb_hip.MNB_PACK_SAFETENSORS
        assert pk.names() == ["model.embed_tokens.weight"]
        assert pk.tensor_info("model.embed_tokens.weight") == (10, (2, 2))
        with pytest.raises(IOException, match="Quantized weight not found for layer 0 q_proj"):
            pk.find_projection(0, "q_proj")
        with pytest.raises(IOException, match="Quantized weight not found: model.embed_tokens.weight"):
            pk.info("model.embed_tokens.weight")


def test_safetensors_reference_case_rejects_invalid_byte_length(tmp_path):
    """SafeTensorsReaderTest.rejectsInvalidByteLength: F32 [2] in 4 bytes."""
    header = '{"x":{"dtype":"F32","shape":[2],"data_offsets":[0,4]}}'
    p = wf.write_safetensors(tmp_path / "bad.safetensors", [], header=header, tail=struct.pack("<i", 1234))
    _err(p, "SafeTensors byte length mismatch for x in bad.safetensors: expected 8 bytes from dtype/shape, got 4")


def test_safetensors_directory_order_dtypes_and_shapes(tmp_path):
    """Tensors in directory order (every dtype the reader knows, with its
    ONNX code), lower-case dtypes upper-cased, a repeated name keeping its
    first position and last value, empty and scalar shapes."""
    ts = [("b.f32", "F32", (3, 2), bytes(24)), ("a.bf16", "bf16", (4,), bytes(8)), ("c.u8", "U8", (), bytes(1)),
          ("d.i64", "I64", (0, 5), b""), ("e.bool", "BOOL", (2,), bytes(2)), ("f.f64", "F64", (1,), bytes(8)),
          ("g.i16", "I16", (1,), bytes(2)), ("h.u16", "U16", (1,), bytes(2)), ("i.u32", "U32", (1,), bytes(4)),
          ("j.u64", "U64", (1,), bytes(8)), ("k.i8", "I8", (1,), bytes(1)), ("l.i32", "I32", (1,), bytes(4)),
          ("m.f16", "F16", (2, 1), bytes(4))]
    p = wf.write_safetensors(tmp_path / "m.safetensors", ts, metadata={"format": "pt"})
    codes = {"F32": 1, "BF16": 16, "U8": 2, "I64": 7, "BOOL": 9, "F64": 11, "I16": 5, "U16": 4, "U32": 12, "U64": 13,
             "I8": 3, "I32": 6, "F16": 10}
    with Pack(p) as pk:
        assert pk.names() == [t[0] for t in ts]
        for name, dt, shape, _ in ts:
            assert pk.tensor_info(name) == (codes[dt.upper()], tuple(shape)), name
    dup = '{"x":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},"y":{"dtype":"U8","shape":[1],"data_offsets":[4,5]},' \
          '"x":{"dtype":"F16","shape":[2],"data_offsets":[0,4]}}'
    with Pack(wf.write_safetensors(tmp_path / "d.safetensors", [], header=dup, tail=bytes(5))) as pk:
        assert pk.names() == ["x", "y"] and pk.tensor_info("x") == (10, (2,))
    with Pack(wf.write_safetensors(tmp_path / "a.safetensors", [], header="[1, 2]", tail=b"")) as pk:
        assert pk.names() == []        # a directory that is not an object lists no tensors


@pytest.mark.parametrize("header,tail,match", [
    ('{"x":5}', b"", "Invalid SafeTensors tensor entry for x in e.safetensors"),
    ('{"x":{"shape":[1],"data_offsets":[0,4]}}', bytes(4), "Invalid SafeTensors tensor x in e.safetensors: missing textual dtype"),
    ('{"x":{"dtype":7,"shape":[1],"data_offsets":[0,4]}}', bytes(4), "missing textual dtype"),
    ('{"x":{"dtype":"F32","data_offsets":[0,4]}}', bytes(4), "Invalid SafeTensors tensor x in e.safetensors: missing array shape"),
    ('{"x":{"dtype":"F32","shape":[1]}}', bytes(4), "missing array data_offsets"),
    ('{"x":{"dtype":"F32","shape":["1"],"data_offsets":[0,4]}}', bytes(4), "Invalid SafeTensors tensor x in e.safetensors: non-integer shape"),
    ('{"x":{"dtype":"F32","shape":[1],"data_offsets":[0,true]}}', bytes(4), "non-integer data_offsets"),
    ('{"x":{"dtype":"F32","shape":[1],"data_offsets":[0,4,8]}}', bytes(8), "Invalid SafeTensors data_offsets for x in e.safetensors"),
    ('{"x":{"dtype":"F32","shape":[1],"data_offsets":[-4,0]}}', bytes(4), r"Invalid SafeTensors data range for x: \[-4, 0\]"),
    ('{"x":{"dtype":"F32","shape":[1],"data_offsets":[8,4]}}', bytes(8), r"Invalid SafeTensors data range for x: \[8, 4\]"),
    ('{"x":{"dtype":"F32","shape":[1],"data_offsets":[0,8]}}', bytes(4),
     r"SafeTensors data range for x escapes file bounds: \[0, 8\] fileSize="),
    ('{"x":{"dtype":"F32","shape":[-1],"data_offsets":[0,4]}}', bytes(4),
     "Invalid negative dimension for SafeTensors tensor x in e.safetensors: -1"),
    ('{"x":{"dtype":"Q4","shape":[1],"data_offsets":[0,4]}}', bytes(4), "Unsupported SafeTensors dtype: Q4"),
    ('{"x":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}', bytes(4), "Invalid SafeTensors header JSON"),
])
def test_safetensors_entry_errors(tmp_path, header, tail, match):
    _err(wf.write_safetensors(tmp_path / "e.safetensors", [], header=header, tail=tail), match)


def test_safetensors_container_errors(tmp_path):
    small = tmp_path / "s.safetensors"
    small.write_bytes(b"\x01\x02\x03")
    _err(small, "Invalid SafeTensors file: too small: " + str(small))
    for hl, name in ((1, "h1"), (100, "h2"), (-5, "h3")):
        p = tmp_path / (name + ".safetensors")
        p.write_bytes(struct.pack("<q", hl) + b"{}" + bytes(4))
        _err(p, "Invalid SafeTensors header length for %s.safetensors: %d" % (name, hl))


def test_dense_tensor_quantize_checks_before_any_device_work(tmp_path):
    """mnb_pack_weight_quantize reads and checks the dense matrix on the host
    first: an unknown name, a shape other than the expected [rows, cols]
    (Qwen2Weights.validateMatrixShape's text) and a BF16 tensor (which the
    reference's embedding table refuses) fail with MNB_ERR_IO before the
    context is used; a good tensor then needs a context."""
    import ctypes
    L = mnb_hip.load()
    p = wf.write_safetensors(tmp_path / "model.safetensors",
                             [("model.embed_tokens.weight", "F32", (6, 32), bytes(6 * 32 * 4)),
                              ("b", "BF16", (6, 32), bytes(6 * 32 * 2))])
    with Pack(p) as pk:
        h = ctypes.c_void_p()
        cases = [(b"nope", 6, 32, mnb_hip.MNB_ERR_IO, "Tensor not found: nope"),
                 (b"model.embed_tokens.weight", 7, 32, mnb_hip.MNB_ERR_IO,
                  "Unexpected dimensions for model.embed_tokens.weight: [6, 32], expected [7, 32]"),
                 (b"b", 6, 32, mnb_hip.MNB_ERR_IO, "Unsupported inline tensor data for b: BFLOAT16 (16)"),
                 (b"model.embed_tokens.weight", 6, 32, mnb_hip.MNB_ERR_INVALID_STATE, "Kernel not prepared")]
        for name, r, c, code, msg in cases:
            rc = L.mnb_pack_weight_quantize(None, pk.handle, name, r, c, 0, ctypes.byref(h))
            assert rc == code and msg in mnb_hip.last_error(), (name, rc, mnb_hip.last_error())
