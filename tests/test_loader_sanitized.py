"""The weight-file readers under AddressSanitizer and UndefinedBehaviorSanitizer.

tests/loader_sanitized.cpp is built with the reader's source
(win-directml-java_amd/csrc/mnb_pack.cpp) and -fsanitize=address,undefined
(host code only: no device code is compiled), then run over random mutations
of valid files of every kind the reader opens: an ONNX model with inline
initializers and one with external data (the model or its data file
mutated), a Phi-3 .wdmlpack package, a Qwen2 payload package and a
safetensors file.  Mutations flip bits, overwrite, insert or truncate bytes.
Any out-of-bounds access, use after free, leak or undefined behaviour ends
the driver with a sanitizer report and a non-zero status; the test requires
a clean exit, and that some mutants still open and read (so the reading code
runs, not only the header checks).  test_weight_files.py checks the texts of
the errors the reader reports; this test checks that no input makes it touch
memory it does not own."""
import os
import shutil
import subprocess

import numpy as np
import pytest

import weightfiles as wf
from mnb_hip import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLANG = "/opt/rocm/llvm/bin/clang++"


def _mutate(rng, base):
    buf = bytearray(base)
    for _ in range(int(rng.integers(1, 5))):
        k, j = int(rng.integers(0, 4)), int(rng.integers(0, len(buf)))
        if k == 0:
            buf[j] ^= 1 << int(rng.integers(0, 8))
        elif k == 1:
            buf[j] = int(rng.integers(0, 256))
        elif k == 2:
            del buf[j:]
        else:
            buf[j:j] = rng.integers(0, 256, int(rng.integers(1, 9))).astype(np.uint8).tobytes()
        if not buf:
            break
    return bytes(buf)


def _seeds(d):
    """(path of a valid file, extension) of each kind, and the path of an ONNX model with external data."""
    N, K, bs = 6, 192, 64
    t = synth.make_weight(3, N, K, bs, with_zp=True)
    q3 = t.q.reshape(N, t.kb, bs // 2)
    b = wf.OnnxBuilder()
    b.matmul_nbits("/model/layers.0/attn/q_proj/MatMul_output_0", N, K, bs, q3, t.scales_f16.view(np.uint16),
                   zp=t.zp_row_padded)
    b.matmul_nbits("w2", N, K, bs, q3, t.scales_f16.view(np.uint16))
    seeds = [(b.write(os.path.join(d, "inline")), ".onnx")]
    pk = os.path.join(d, "phi3.wdmlpack")
    payload = [("embed_tokens", wf.FLOAT, [24], np.arange(24, dtype="<f4").tobytes())]
    for role, n, k, seed in [("lm_head", 6, 4, 1), ("layers.0.q_proj", 4, 4, 2), ("layers.0.down_proj", 4, 8, 7)]:
        q, s, z = wf.reference_quant(n, k, 4, seed)
        payload += wf.phi3_triplet_tensors(role, q.tobytes(), n, k, 4, s, z.tobytes())
    wf.write_wdmlpack(pk, wf.phi3_manifest(), payload)
    seeds.append((pk, ".wdmlpack"))
    N, K, bs = 10, 192, 64
    t = synth.make_weight(21, N, K, bs, with_zp=True)
    kb = t.kb
    graph = {"nodes": [{"opType": "MatMulNBits", "inputs": ["x", "h_Q4", "h_scales", "h_zp"], "outputs": ["logits"]}]}
    man = {"format": "wdmlpack", "version": 1, "mode": "payload", "payloadIncluded": True, "runtimeLoadable": True,
           "runtimeLoadMode": "qwen-native-payload", "model": {"architecture": "Qwen2", "hiddenSize": 64},
           "runtimeGraph": graph}
    qp = os.path.join(d, "qwen.wdmlpack")
    wf.write_wdmlpack(qp, man, [("h_Q4", wf.UINT8, [N, kb, bs // 2], t.q.tobytes()),
                                ("h_scales", wf.FLOAT16, [N, kb], t.scales_f16.tobytes()),
                                ("h_zp", wf.UINT8, [N, (kb + 1) // 2], t.zp_row_padded.tobytes())])
    seeds.append((qp, ".wdmlpack"))
    st = wf.write_safetensors(os.path.join(d, "m.safetensors"), [
        ("model.embed_tokens.weight", "F16", [4, 8], np.arange(32, dtype="<f2").tobytes()),
        ("a", "F32", [3], np.ones(3, "<f4").tobytes()), ("b", "BF16", [2, 2], bytes(8))], metadata={"format": "pt"})
    seeds.append((st, ".safetensors"))
    N, K, bs = 8, 64, 32
    t = synth.make_weight(4, N, K, bs, with_zp=True)
    b = wf.OnnxBuilder()
    b.matmul_nbits("w", N, K, bs, t.q.reshape(N, t.kb, bs // 2), t.scales_f16.view(np.uint16), zp=t.zp_row_padded,
                   external=True)
    ext = b.write(os.path.join(d, "external"))
    return seeds, ext


def test_readers_under_sanitizers(tmp_path):
    if not os.path.exists(CLANG):
        pytest.skip("clang++ of the ROCm toolchain is not present")
    exe = str(tmp_path / "loader_sanitized")
    cmd = [CLANG, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=undefined", "-I" + os.path.join(ROOT, "include"),
           "-I" + os.path.join(ROOT, "win-directml-java_amd", "csrc"), "-I/opt/rocm/include",
           "-D__HIP_PLATFORM_AMD__", os.path.join(ROOT, "tests", "loader_sanitized.cpp"),
           os.path.join(ROOT, "win-directml-java_amd", "csrc", "mnb_pack.cpp"), "-o", exe]
    subprocess.run(cmd, check=True, capture_output=True, timeout=300)
    seeds, ext = _seeds(str(tmp_path))
    rng = np.random.default_rng(2026)
    files = [p for p, _ in seeds] + [ext]
    mut = tmp_path / "mutants"
    mut.mkdir()
    for si, (path, suffix) in enumerate(seeds):
        base = open(path, "rb").read()
        for i in range(300):
            f = mut / ("s%d_%03d%s" % (si, i, suffix))
            f.write_bytes(_mutate(rng, base))
            files.append(str(f))
    model, data = open(ext, "rb").read(), open(os.path.join(os.path.dirname(ext), "model.onnx_data"), "rb").read()
    for i in range(200):
        d = mut / ("ext_%03d" % i)
        d.mkdir()
        (d / "model.onnx").write_bytes(_mutate(rng, model) if i % 2 == 0 else model)
        (d / "model.onnx_data").write_bytes(data if i % 2 == 0 else _mutate(rng, data))
        files.append(str(d / "model.onnx"))
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe] + files, capture_output=True, text=True, timeout=600, env=env)
    assert r.returncode == 0, r.stderr[-4000:]
    opened, reads = [int(v) for v in r.stdout.split()[3::2]]
    assert opened > len(seeds) and reads > len(seeds), r.stdout
    shutil.rmtree(str(mut), ignore_errors=True)
