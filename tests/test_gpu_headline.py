"""The benchmarked workloads, checked against the oracle at full size.

Every timed workload of bench.py is run here with the bench's weight seeds and
shapes (activations from their own seeds) and compared with the oracle, the
restatement of the reference's CPU MatMulNBits (Phi3Weights.QuantizedWeight.
matmul, directml-inference/.../phi3/Phi3Weights.java:123-192):

* the Phi-3-mini decode step at M = 1 as ONE group launch (the headline
  figure; 129 products, 65,492 (item, n-tile) units on a few thousand waves,
  so every wave's pipeline runs across many unit boundaries), every output of
  every product against the oracle;
* the same 129 products as separate launches (the dependent-chain form; this
  includes gate_up 3072 -> 16384 and lm_head 3072 -> 32064 at M = 1), every
  output against the oracle;
* the prefill step at M in {16, 128, 512, 2048} as one group launch: every
  output of every product against that product's own single launch (another
  kernel schedule), and sampled rows and columns against the oracle;
* the Qwen2.5-0.5B step at M = 1 and 64 as one group launch;
* the Phi-3-mini step with M = 2 and 4 rows per product (small-batch decode)
  as one group launch, sampled outputs of every product against the oracle.

Each group output buffer is filled with NaN before the launch, so a unit or
tile that the schedule skipped shows up as NaN; a second launch must
reproduce the first bit for bit.  Bound: |y - y_oracle| <= 1e-3 * sqrt(K) *
max|x| * max|w| (max|w| exact, over the dequantized weight) plus one fp16 ulp;
a group output and the single launch of the same product, each within that
bound of the oracle, may differ by twice the bound plus two fp16 ulps.
"""
import numpy as np
import pytest

import mnb_hip
from mnb_hip import synth
import mnb_oracle as orc
from parity_util import assert_parity, exact_max_abs_w, oracle_matmul, parity_bound, say, upload

pytestmark = pytest.mark.gpu

BS = 32
PHI3_SEED, QWEN_SEED = 10_000, 20_000    # weight seeds of bench.py


@pytest.fixture(scope="module")
def ctx():
    orc.build()
    c = mnb_hip.Context(0)
    yield c
    c.close()


def _step(ctx, projs, seed):
    host, ws = [], []
    for i, (_, _, K, N) in enumerate(projs):
        t = synth.make_weight(seed + i, N, K, BS)
        host.append(t)
        ws.append(upload(ctx, t))
    wmax = [exact_max_abs_w(t) for t in host]
    return host, ws, wmax


@pytest.fixture(scope="module")
def phi3(ctx):
    projs = synth.phi3_decode_step()
    say("uploading the Phi-3-mini decode step (%d products)" % len(projs))
    host, ws, wmax = _step(ctx, projs, PHI3_SEED)
    yield projs, host, ws, wmax
    for w in ws:
        w.close()


@pytest.fixture(scope="module")
def qwen(ctx):
    projs = synth.qwen_decode_step()
    host, ws, wmax = _step(ctx, projs, QWEN_SEED)
    yield projs, host, ws, wmax
    for w in ws:
        w.close()


def _run_group_twice(ctx, entries, stream):
    """Records the group and runs it twice on NaN-filled outputs; checks that
    the second run reproduces the first bit for bit and returns the outputs
    (device tensors)."""
    import torch
    g = mnb_hip.Group(ctx, entries)
    first = []
    try:
        for rep in range(2):
            for _, _, y in entries:
                y.fill_(float("nan"))
            torch.cuda.synchronize()
            g.run(stream.cuda_stream)
            torch.cuda.synchronize()
            if rep == 0:
                first = [y.clone() for _, _, y in entries]
    finally:
        g.close()
    for i, ((_, _, y), y0) in enumerate(zip(entries, first)):
        assert torch.equal(y.view(torch.int16), y0.view(torch.int16)), "item %d: the replay differs" % i
    del first
    return [y for _, _, y in entries]


def _decode_inputs(projs, seed):
    import torch
    x16 = [synth.make_x(seed + i, 1, K) for i, (_, _, K, _) in enumerate(projs)]
    xd = [torch.from_numpy(x).cuda() for x in x16]
    yd = [torch.empty((1, N), dtype=torch.float16, device="cuda") for (_, _, _, N) in projs]
    return x16, xd, yd


def _check_decode_outputs(projs, host, wmax, ys, x16, what):
    for i, ((name, layer, K, N), t, yd, x) in enumerate(zip(projs, host, ys, x16)):
        y = yd.cpu().numpy()
        assert not np.isnan(y).any(), "%s item %d (%s layer %d): outputs never written" % (what, i, name, layer)
        y_ref, _ = oracle_matmul(t, x, want_wmax=False)
        assert_parity(y, y_ref, x, t, wmax[i], True, "%s item %d %s.%d" % (what, i, name, layer))


def test_config1_decode_step_as_one_group_launch(ctx, phi3):
    """The headline workload: the 129 M = 1 products of a Phi-3-mini decode
    step recorded as one group and run as one launch of the streaming kernel;
    every output of every product against the oracle."""
    import torch
    projs, host, ws, wmax = phi3
    x16, xd, yd = _decode_inputs(projs, 30_000)
    ys = _run_group_twice(ctx, list(zip(ws, xd, yd)), torch.cuda.Stream())
    _check_decode_outputs(projs, host, wmax, ys, x16, "decode group")


@pytest.mark.parametrize("M", [2, 4])
def test_small_batch_decode_step_as_one_group_launch(ctx, phi3, M):
    """The 129 products of the Phi-3-mini step with M = 2 and 4 rows each
    (small-batch decode) as one group launch of the streaming kernel with M x
    rows per job: every row of 512 sampled outputs of every product against
    the oracle, every output written, the replay bitwise identical."""
    import torch
    projs, host, ws, wmax = phi3
    x16 = [synth.make_x(32_000 + 200 * M + i, M, K) for i, (_, _, K, _) in enumerate(projs)]
    xd = [torch.from_numpy(x).cuda() for x in x16]
    yd = [torch.empty((M, N), dtype=torch.float16, device="cuda") for (_, _, _, N) in projs]
    g = mnb_hip.Group(ctx, list(zip(ws, xd, yd)))
    plan = g.plan().as_tuple()
    g.close()
    assert plan == (mnb_hip.MNB_KERNEL_STREAM, mnb_hip.MNB_ORDER_NONE, M, 16), plan
    ys = _run_group_twice(ctx, list(zip(ws, xd, yd)), torch.cuda.Stream())
    for i, ((name, layer, K, N), t, yg, x) in enumerate(zip(projs, host, ys, x16)):
        y = yg.cpu().numpy()
        assert not np.isnan(y).any(), "item %d (%s layer %d): outputs never written" % (i, name, layer)
        cols = np.sort(np.random.default_rng(i).choice(N, min(N, 512), replace=False))
        y_ref, _ = oracle_matmul(t, x, cols, want_wmax=False)
        assert_parity(y[:, cols], y_ref, x, t, wmax[i], True, "M=%d group item %d %s.%d" % (M, i, name, layer))


def test_config1_decode_step_as_separate_launches(ctx, phi3):
    """The same 129 products as stream-ordered single launches with device
    pointers (bench decode_step_sequential), fp16 outputs, every output
    against the oracle; gate_up 3072 -> 16384 and lm_head 3072 -> 32064 also
    with fp32 outputs through the host-array path (the reference's float[]
    matvec contract, MatMulNBitsKernel.java:1847-1914)."""
    import torch
    projs, host, ws, wmax = phi3
    x16, xd, yd = _decode_inputs(projs, 31_000)
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        for w, x, y in zip(ws, xd, yd):
            y.fill_(float("nan"))
            w.matmul(x, y, stream=st.cuda_stream)
    torch.cuda.synchronize()
    _check_decode_outputs(projs, host, wmax, yd, x16, "single launch")
    for i, ((name, layer, K, N), t, x, w) in enumerate(zip(projs, host, x16, ws)):
        if (name == "gate_up" and layer == 0) or name == "lm_head":
            y_ref, _ = oracle_matmul(t, x, want_wmax=False)
            y32 = w.matmul(x[0].astype(np.float32), out_dtype=np.float32)
            assert_parity(y32.reshape(1, N), y_ref, x, t, wmax[i], False, "%s f32 host path" % name)


def _sample(rng, n, k):
    """Sorted indices below n: the first and the last 16 and k random others."""
    base = set(range(min(n, 16))) | set(range(max(0, n - 16), n))
    extra = rng.choice(n, min(n, k), replace=False)
    return np.array(sorted(base | set(int(v) for v in extra)))


def _check_prefill_group(ctx, projs, host, ws, wmax, M, seed, mrows, ncols):
    """The products at M rows (one activation per K, as bench.py) as one group
    launch: every output against the product's own single launch on the
    device, sampled outputs against the oracle."""
    import torch
    xs = {}
    for (_, _, K, _) in projs:
        if K not in xs:
            xs[K] = synth.make_x(seed + K, M, K)
    xd = {K: torch.from_numpy(x).cuda() for K, x in xs.items()}
    yd = [torch.empty((M, N), dtype=torch.float16, device="cuda") for (_, _, _, N) in projs]
    st = torch.cuda.Stream()
    ys = _run_group_twice(ctx, [(w, xd[K], y) for w, (_, _, K, _), y in zip(ws, projs, yd)], st)
    rng = np.random.default_rng(seed)
    for i, ((name, layer, K, N), t, y, w) in enumerate(zip(projs, host, ys, ws)):
        label = "M=%d group item %d %s.%d" % (M, i, name, layer)
        assert not bool(torch.isnan(y).any()), label + ": outputs never written"
        x = xs[K]
        tol = parity_bound(K, x, wmax[i])
        single = torch.empty((M, N), dtype=torch.float16, device="cuda")
        with torch.cuda.stream(st):
            w.matmul(xd[K], single, stream=st.cuda_stream)
        torch.cuda.synchronize()
        a = single.float()
        ulp = torch.exp2(torch.floor(torch.log2(a.abs().clamp_min(2.0 ** -14))) - 10)
        excess = ((y.float() - a).abs() - (2 * tol + 2 * ulp)).max().item()
        assert excess <= 0.0, "%s: group vs single launch exceeds 2x the bound %.3e by %.3e" % (label, tol, excess)
        del single, a, ulp
        rows = _sample(rng, M, mrows)
        cols = _sample(rng, N, ncols)
        yh = y[torch.from_numpy(rows).cuda()][:, torch.from_numpy(cols).cuda()].cpu().numpy()
        y_ref, _ = oracle_matmul(t, np.ascontiguousarray(x[rows]), cols, want_wmax=False)
        assert_parity(yh, y_ref, x, t, wmax[i], True, label)


@pytest.mark.parametrize("M", [16, 128, 512, 2048])
def test_config2_prefill_step_as_one_group_launch(ctx, phi3, M):
    """The bench's prefill groups (M = 512 is prefill_m512; 16, 128 and 2048
    its sweep): the 129 Phi-3 products, each with its own output."""
    projs, host, ws, wmax = phi3
    say("prefill group M=%d" % M)
    _check_prefill_group(ctx, projs, host, ws, wmax, M, 40_000 + M, 8, 48)


def test_config3_qwen_step_as_one_group_launch(ctx, qwen):
    """The Qwen2.5-0.5B step with a quantized lm_head (97 products, bench
    qwen_step): M = 1 with every output against the oracle, and M = 64
    (64-row GEMM tiles) against single launches and the oracle on samples."""
    import torch
    projs, host, ws, wmax = qwen
    x16, xd, yd = _decode_inputs(projs, 50_000)
    ys = _run_group_twice(ctx, list(zip(ws, xd, yd)), torch.cuda.Stream())
    _check_decode_outputs(projs, host, wmax, ys, x16, "qwen M=1")
    _check_prefill_group(ctx, projs, host, ws, wmax, 64, 51_000, 8, 48)
