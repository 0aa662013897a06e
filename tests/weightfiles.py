"""Writers of the weight files the loader reads, used by the tests.

* ``.wdmlpack`` containers laid out as the reference writes them: a 64-byte
  little-endian header (magic "WDMLPACK", int32 version 1, int32 flags, then
  int64 manifest offset/length, tensor-directory offset/length (0/0) and
  payload offset/length), the JSON manifest at byte 64, the payload at the
  next 4096-byte boundary, and each tensor at a 64-byte aligned offset
  relative to the payload base (WdmlPackWriter.java:100-111, 184-213;
  Phi3WdmlPackCompiler.java:154-213; WDMLPACK_FORMAT.md:58-77).
* ONNX models encoded field by field in the protobuf wire format with the
  onnx.proto field numbers (ModelProto.graph 7; GraphProto node 1, name 2,
  initializer 5; NodeProto input 1, output 2, name 3, op_type 4, attribute 5,
  domain 7; TensorProto dims 1, data_type 2, float_data 4, int32_data 5,
  name 8, raw_data 9, external_data 13, data_location 14).

Also the reference test's deterministic triplet generator
(Phi3WdmlPackCompilerTest.java:222-239).
"""
import json
import os
import struct

import numpy as np

FLOAT, UINT8, INT8, INT32, FLOAT16 = 1, 2, 3, 6, 10


def align(v: int, a: int) -> int:
    return (v + a - 1) // a * a


# ---------------------------------------------------------------------------
# .wdmlpack
# ---------------------------------------------------------------------------

def write_wdmlpack(path, manifest: dict, payload=(), flags: int = 0, header_override=None):
    """Write a container.  ``payload`` is a list of (name, dataType, dims, bytes);
    their directory entries are appended to manifest["tensors"] unless the
    manifest already holds a "tensors" key.  ``header_override`` maps header
    field names to values written instead of the computed ones."""
    dir_entries, chunks, cursor = [], [], 0
    for name, dtype, dims, data in payload:
        cursor = align(cursor, 64)
        dir_entries.append({"name": name, "dataType": dtype, "dims": [int(d) for d in dims],
                            "byteLength": len(data), "payloadOffset": cursor, "payloadLength": len(data)})
        chunks.append((cursor, bytes(data)))
        cursor += len(data)
    m = dict(manifest)
    if "tensors" not in m:
        m["tensors"] = dir_entries
    js = json.dumps(m).encode("utf-8")
    payload_len = cursor
    payload_off = align(64 + len(js), 4096) if payload_len > 0 else 0
    h = {"magic": b"WDMLPACK", "version": 1, "flags": flags, "manifest_off": 64, "manifest_len": len(js),
         "dir_off": 0, "dir_len": 0, "payload_off": payload_off, "payload_len": payload_len}
    h.update(header_override or {})
    hdr = h["magic"][:8].ljust(8, b"\0") + struct.pack("<ii6q", h["version"], h["flags"], h["manifest_off"],
                                                         h["manifest_len"], h["dir_off"], h["dir_len"],
                                                         h["payload_off"], h["payload_len"])
    body = bytearray(hdr + js)
    if payload_len > 0:
        body.extend(b"\0" * (payload_off - len(body)))
        base = len(body)
        body.extend(b"\0" * payload_len)
        for off, data in chunks:
            body[base + off:base + off + len(data)] = data
    with open(path, "wb") as f:
        f.write(bytes(body))
    return path


def phi3_manifest(hidden=4, heads=2, layers=1, kv_heads=2, vocab=6, max_pos=8, inter=8, **extra) -> dict:
    """Root keys of a Phi-3 payload package (Phi3WdmlPackCompiler.java:179-213)."""
    m = {"format": "wdmlpack", "version": 1, "createdAt": "2026-01-01T00:00:00Z", "architecture": "phi3",
         "mode": "payload", "payloadIncluded": True, "runtimeLoadable": True,
         "runtimeLoadMode": "phi3-native-payload", "payloadAlignment": 4096, "payloadBytes": 0,
         "tokenizer": "tokenizer.json", "tokenizerPresentAtCompile": False,
         "model": {"hiddenSize": hidden, "numAttentionHeads": heads, "numHiddenLayers": layers,
                   "numKeyValueHeads": kv_heads, "vocabSize": vocab, "maxPositionEmbeddings": max_pos,
                   "intermediateSize": inter, "rmsNormEps": 1.0e-5, "ropeTheta": 10000.0},
         "cache": {"compiler": "Phi3WdmlPackCompiler", "compilerVersion": 1, "createdBy": "win-directml-java"}}
    m.update(extra)
    return m


def phi3_triplet_tensors(role, q: bytes, N: int, K: int, bs: int, scales_f32, zp: bytes):
    """<role>.qweight UINT8 [N,K,bs], <role>.scales FLOAT [count], <role>.zeropoints UINT8 [len]
    (Phi3WdmlPackCompiler.java:256-264)."""
    s = np.asarray(scales_f32, np.float32).reshape(-1)
    return [(role + ".qweight", UINT8, [N, K, bs], bytes(q)),
            (role + ".scales", FLOAT, [s.size], s.astype("<f4").tobytes()),
            (role + ".zeropoints", UINT8, [len(zp)], bytes(zp))]


def reference_quant(n: int, k: int, bs: int, seed: int):
    """Phi3WdmlPackCompilerTest.quant: q[i] = (7i+seed) & 0xFF, scales[i] =
    float(i+seed) * 0.01f, zp[i] = (3i+seed) & 0xFF."""
    kb = k // bs
    q = ((np.arange(n * kb * (bs // 2), dtype=np.int64) * 7 + seed) & 0xFF).astype(np.uint8)
    scales = ((np.arange(n * kb, dtype=np.int64) + seed).astype(np.float32) * np.float32(0.01)).astype(np.float32)
    zp = ((np.arange((n * kb + 1) // 2, dtype=np.int64) * 3 + seed) & 0xFF).astype(np.uint8)
    return q, scales, zp


# ---------------------------------------------------------------------------
# ONNX protobuf
# ---------------------------------------------------------------------------

def varint(n: int) -> bytes:
    n &= (1 << 64) - 1
    out = bytearray()
    while True:
        b = n & 0x7F
        n >>= 7
        if n:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def key(field: int, wt: int) -> bytes:
    return varint(field << 3 | wt)


def ld(field: int, payload: bytes) -> bytes:
    return key(field, 2) + varint(len(payload)) + payload


def sfield(field: int, s: str) -> bytes:
    return ld(field, s.encode("utf-8"))


def vfield(field: int, n: int) -> bytes:
    return key(field, 0) + varint(n)


def tensor_proto(name, dtype, dims, raw=None, float_data=None, int32_data=None, external=None,
                 packed_dims=False, raw_len_override=None) -> bytes:
    """TensorProto.  ``external`` = (location, offset, length) writes the
    external_data entries and data_location EXTERNAL.  ``raw_len_override``
    writes a raw_data length prefix that differs from the bytes that follow
    (the external-data stubs of some exporters)."""
    b = ld(1, b"".join(varint(int(d)) for d in dims)) if packed_dims else b"".join(vfield(1, int(d)) for d in dims)
    b += vfield(2, dtype)
    if float_data is not None:
        b += ld(4, np.asarray(float_data, "<f4").tobytes())
    if int32_data is not None:
        b += ld(5, b"".join(varint(int(v)) for v in int32_data))
    b += sfield(8, name)
    if raw is not None:
        if raw_len_override is not None:
            b += key(9, 2) + varint(raw_len_override) + bytes(raw)
        else:
            b += ld(9, bytes(raw))
    if external is not None:
        loc, off, length = external
        for k, v in (("location", loc), ("offset", str(off)), ("length", str(length))):
            b += ld(13, sfield(1, k) + sfield(2, v))
        b += vfield(14, 1)
    return b


def attribute_int(name: str, value: int) -> bytes:
    return sfield(1, name) + vfield(3, value) + vfield(20, 2)  # AttributeProto.i, type INT


def node_proto(op_type, inputs, outputs, name="", attrs=None, domain="") -> bytes:
    b = b"".join(sfield(1, i) for i in inputs) + b"".join(sfield(2, o) for o in outputs)
    b += sfield(3, name) + sfield(4, op_type)
    for k, v in (attrs or {}).items():
        b += ld(5, attribute_int(k, v))
    if domain:
        b += sfield(7, domain)
    return b


def graph_proto(nodes, initializers, name="g") -> bytes:
    return b"".join(ld(1, n) for n in nodes) + sfield(2, name) + b"".join(ld(5, t) for t in initializers)


def model_proto(graph: bytes) -> bytes:
    opset = sfield(1, "") + vfield(2, 17)
    ms = sfield(1, "com.microsoft") + vfield(2, 1)
    return vfield(1, 8) + ld(8, opset) + ld(8, ms) + ld(7, graph)


class OnnxBuilder:
    """Collects MatMulNBits nodes and initializers; tensors go inline or into
    an external data file (offsets in the order written)."""

    def __init__(self):
        self.nodes, self.inits, self.ext = [], [], bytearray()

    def tensor(self, name, dtype, dims, data: bytes, external=False, data_file="model.onnx_data"):
        if external:
            off = len(self.ext)
            self.ext.extend(data)
            self.inits.append(tensor_proto(name, dtype, dims, external=(data_file, off, len(data))))
        else:
            self.inits.append(tensor_proto(name, dtype, dims, raw=data))

    def matmul_nbits(self, out, N, K, bs, q, scales, zp=None, external=False, scale_dtype=FLOAT16,
                     zp_dims=None, prefix=None, zp_input=None, data_file="model.onnx_data"):
        """q: uint8 [N, kb, bs/2]; scales: fp16 bit patterns (uint16) or float32 [N*kb];
        zp: uint8 bytes (row-padded [N, ceil(kb/2)] unless zp_dims says otherwise)."""
        p = prefix or out.replace("/", "_")
        kb = q.shape[1]
        self.tensor(p + "_Q4", UINT8, list(q.shape), np.ascontiguousarray(q, np.uint8).tobytes(), external, data_file)
        s = np.asarray(scales)
        sdata = s.astype("<u2").tobytes() if scale_dtype == FLOAT16 else s.astype("<f4").tobytes()
        self.tensor(p + "_scales", scale_dtype, [N, kb], sdata, external, data_file)
        inputs = ["x", p + "_Q4", p + "_scales"]
        if zp is not None:
            zb = np.asarray(zp, np.uint8).reshape(-1)
            self.tensor(p + "_zp", UINT8, zp_dims if zp_dims is not None else [N, (kb + 1) // 2], zb.tobytes(),
                        external, data_file)
            inputs.append(p + "_zp")
        elif zp_input is not None:
            inputs.append(zp_input)
        self.nodes.append(node_proto("MatMulNBits", inputs, [out], name=p,
                                     attrs={"K": K, "N": N, "bits": 4, "block_size": bs}, domain="com.microsoft"))

    def write(self, directory, model_name="model.onnx", data_name="model.onnx_data"):
        os.makedirs(directory, exist_ok=True)
        path = os.path.join(directory, model_name)
        with open(path, "wb") as f:
            f.write(model_proto(graph_proto(self.nodes, self.inits)))
        if self.ext:
            with open(os.path.join(directory, data_name), "wb") as f:
                f.write(bytes(self.ext))
        return path


# ---------------------------------------------------------------------------
# SafeTensors files (the container SafeTensorsReader.java:84-277 reads)
# ---------------------------------------------------------------------------

def write_safetensors(path, tensors, metadata=None, header=None, tail=b""):
    """tensors: list of (name, dtype str, shape, payload bytes) laid out in
    order; `header` (a str) replaces the generated JSON directory."""
    import json as _json
    import struct as _struct
    directory, blobs, off = {}, [], 0
    for name, dtype, shape, data in tensors:
        directory[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(data)]}
        blobs.append(data)
        off += len(data)
    if metadata is not None:
        directory["__metadata__"] = metadata
    text = header if header is not None else _json.dumps(directory)
    hb = text.encode("utf-8")
    with open(path, "wb") as f:
        f.write(_struct.pack("<q", len(hb)) + hb + b"".join(blobs) + tail)
    return str(path)
