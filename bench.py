#!/usr/bin/env python3
"""Benchmark of the int4 MatMulNBits library on one MI355X.

Workload (the headline metric "int4 MatMulNBits GB/s at M=1 and TFLOP/s at
M=512, Phi-3-mini shapes"):

* step = one Phi-3-mini decode step at M=1: every quantized projection of 32
  layers (qkv 3072->9216, o_proj 3072->3072, gate_up 3072->16384,
  down 8192->3072) plus lm_head 3072->32064, block size 32, no zero-point
  tensor (implicit 8), run back to back.  About 2.1 GB of packed int4 weights
  and fp16 scales stay resident in HBM; each projection has its own fp16
  activation (N(0,1)) and fp16 output buffer.  Weights are random (seeded);
  there is no checkpoint.  The step is captured once in a HIP graph and
  replayed; inputs are resident before the timed region starts.
* value = algorithmic bytes per step / wall time per step, in GB/s.
* prefill: the same 129 projections at M = 512 (and a sweep over
  M = 16, 128, 2048), reported as TFLOP/s (2*M*N*K flops): recorded as one
  group and run as one launch (like the decode step), and as 129 launches in
  stream order.
* roofline: per-launch HIP-event timing of the dominant kernel (the M=1
  kernel) and of the M=512 kernel, against 8 TB/s HBM and 2.5 PFLOP/s fp16.
* small_batch_decode: the same 129 projections with 2 and 4 rows each (a
  decode step of 2 or 4 sequences) as one group launch.
* config0: the single qkv product (M=1) as back-to-back launches over 17
  weight copies (each launch reads from HBM).
* qwen: the Qwen2.5-0.5B tied lm_head (quantized on the device, M=1) and the
  Qwen step with a quantized lm_head (97 projections, bs 32) as one group
  launch at M=1 and M=64.
* phi3_export_variant: the same 129 Phi-3 projections in the weight format
  of the reference's DirectML int4 export (block size 128, explicit uint8
  zero points, fp16 scales) as one group launch at M=1 and at M=512.
* ceilings: what the matrix cores sustain (an MFMA-only kernel at the GEMM's
  occupancy, libmnb_probe.so) and hipBLASLt's dense fp16 GEMM of the same
  129 projections as 129 launches, reference points for the prefill lines.
* cpu_baseline: the oracle's restatement of the reference's Java CPU path
  (8-lane FMA block dot, one thread per core) on a bounded sample of the
  same decode step.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5]
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "win-directml-java_amd"), os.path.join(ROOT, "oracle")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
RIDGE_FLOP_PER_BYTE = FP16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)
BLOCK = 32


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                   help="untimed GPU work before the warm-up steps of each timed phase (clock ramp after idle)")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="bounded CPU-baseline sample (M=1)")
    p.add_argument("--cpu-m512-seconds", type=float, default=15.0, help="bounded CPU-baseline sample (M=512)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-sweep", action="store_true")
    p.add_argument("--eager", action="store_true", help="launch directly instead of via HIP graphs (counter runs)")
    p.add_argument("--phase", choices=("all", "decode", "chain", "prefill", "qwen", "config0", "export", "ceilings"),
                   default="all",
                   help="decode: only the M=1 group launch and the copy calibration; chain: only the 129 M=1 "
                        "launches in stream order (a HIP graph); prefill: only the M=512 launches (both for "
                        "counter runs); qwen: only the Qwen2.5-0.5B step at M=1 and 64; config0: only the single "
                        "qkv product at M=1; export: only the Phi-3 step in the export's weight format; "
                        "ceilings: only the MFMA ceiling and the dense fp16 GEMM reference points")
    p.add_argument("--prefill-group", action="store_true",
                   help="with --phase prefill: the 129 projections as one group launch instead of 129 launches")
    p.add_argument("--prefill-m", type=int, default=512, help="with --phase prefill: rows M of the prefill step")
    return p.parse_args()


class Launcher:
    """Direct C-ABI calls for a fixed list of (weight, x, y) triples."""

    def __init__(self, ctx, weights, xs, ys, M, stream):
        import mnb_hip
        self.lib = mnb_hip.load()
        self.calls = []
        for w, x, y in zip(weights, xs, ys):
            self.calls.append((ctx.handle, w.handle, M, ctypes.c_void_p(x.data_ptr()), mnb_hip.MNB_F16,
                               x.numel(), ctypes.c_void_p(y.data_ptr()), mnb_hip.MNB_F16, y.numel(), 0,
                               ctypes.c_void_p(stream.cuda_stream)))

    def run(self, idx=None):
        import mnb_hip
        f = self.lib.mnb_matmul
        for a in (self.calls if idx is None else [self.calls[i] for i in idx]):
            rc = f(*a)
            if rc != 0:
                raise mnb_hip.MnbError(rc, mnb_hip.last_error())


SETTLE_MS = 200.0


def settle(torch, graph, stream, ms):
    """Untimed replays for about `ms` of GPU time before any warm-up step.
    After an idle period the MI355X ramps its clocks for tens of milliseconds
    (the decode launch then drifts from 363 to 510 us and back to ~375 us over
    ~25 launches); measurements are taken on the settled chip."""
    if ms <= 0:
        return
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        graph.replay()
    torch.cuda.synchronize()
    one = max(time.perf_counter() - t0, 1e-5)
    n = int(min(10000, max(1, ms * 1e-3 / one)))
    with torch.cuda.stream(stream):
        for _ in range(n):
            graph.replay()
    torch.cuda.synchronize()


def time_graph(torch, graph, stream, steps, warmup, settle_ms=0.0):
    settle(torch, graph, stream, settle_ms)
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            graph.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        ev0.record(stream)
        for _ in range(steps):
            graph.replay()
        ev1.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    gpu = ev0.elapsed_time(ev1) / 1e3 / steps
    return wall, gpu


class _Direct:
    """A step launched directly (counter runs: one dispatch per step, no graph)."""

    def __init__(self, run):
        self.replay = run


def time_steps(torch, run, stream, steps, warmup, settle_ms=0.0, eager=False):
    """Wall and GPU time per step of `run` (one step: its launches in stream
    order).  The timed region is one replay of a HIP graph holding exactly
    `steps` steps back to back, bracketed by two synchronizations and by HIP
    events on the launch stream, so no host launch latency sits between two
    steps (a graph of one short step replayed per step would time the host's
    graph-launch rate, not the device).  Before it: `settle_ms` of untimed
    replays of that graph and `warmup` single steps.  With eager, the steps are
    launched directly (for counter runs)."""
    with torch.cuda.stream(stream):
        run()                   # eager run first (validates every call)
    torch.cuda.synchronize()
    if eager:
        return time_graph(torch, _Direct(run), stream, steps, warmup, settle_ms)
    gk = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gk, stream=stream):
        for _ in range(steps):
            run()
    torch.cuda.synchronize()
    settle(torch, gk, stream, settle_ms)
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            run()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        ev0.record(stream)
        gk.replay()
        ev1.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    gpu = ev0.elapsed_time(ev1) / 1e3 / steps
    del gk
    return wall, gpu


def per_launch_times(torch, launcher, stream, reps=3):
    """Kernel duration of every launch (mean over reps), from a HIP event pair
    around it on the launch stream.  The stream is first held by a GPU sleep so
    that all launches are queued before the first one starts (no host gaps
    inside a bracket)."""
    n = len(launcher.calls)
    durs = np.zeros((reps, n))
    for r in range(reps):
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
        with torch.cuda.stream(stream):
            if hasattr(torch.cuda, "_sleep"):
                torch.cuda._sleep(int(40e6))
            for i in range(n):
                evs[i][0].record(stream)
                launcher.run([i])
                evs[i][1].record(stream)
        torch.cuda.synchronize()
        durs[r] = [a.elapsed_time(b) / 1e3 for a, b in evs]
    return durs.mean(axis=0)


def group_launch_times(torch, grp, stream, reps=20):
    """Duration of each of reps back-to-back launches of a recorded group (HIP
    event pairs on the launch stream).  Called right after the timed graph
    replays, on the settled chip; a launch takes far longer than enqueuing
    the next one, so no host gap falls inside a bracket."""
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    with torch.cuda.stream(stream):
        for a, b in evs:
            a.record(stream)
            grp.run(stream.cuda_stream)
            b.record(stream)
    torch.cuda.synchronize()
    return np.array([a.elapsed_time(b) / 1e3 for a, b in evs])


def capture(torch, launcher, stream):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        launcher.run()          # eager run first (validates every call)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=stream):
        launcher.run()
    torch.cuda.synchronize()
    return g


def copy_bandwidth(torch, stream):
    n = 1 << 30
    a = torch.empty(n, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    with torch.cuda.stream(stream):
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(10):
            b.copy_(a)
        e1.record(stream)
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) / 1e3 / 10
    del a, b
    return 2 * n / t / 1e9


def torch_read_bandwidth(torch, stream):
    """Read rate of torch's fastest whole-buffer reduction found here (an
    int64 sum over 4 GiB): a reference point for reads, like the copy
    figure, not a ceiling."""
    n = 4 << 30
    a = torch.ones(n // 8, dtype=torch.int64, device="cuda")
    with torch.cuda.stream(stream):
        for _ in range(3):
            a.sum()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(10):
            a.sum()
        e1.record(stream)
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) / 1e3 / 10
    del a
    return n / t / 1e9


def measured_traffic(kernel_profile, key="traffic_bytes_per_launch"):
    """HBM bytes of a kernel from its committed rocprofv3 counter summary
    (FETCH_SIZE + WRITE_SIZE, copy-calibrated)."""
    path = os.path.join(ROOT, "profiles", kernel_profile)
    try:
        for line in open(path):
            if line.startswith(key):
                return int(line.split("=")[1])
    except OSError:
        pass
    return None


def cpu_baseline(host, projs, seconds, m512_seconds):
    """Oracle restatement of the reference CPU path on bounded samples.

    M = 1: decode-step projections in step order for about `seconds` (GB/s of
    algorithmic bytes, the headline unit).  M = 512: one projection of each
    Phi-3 shape (qkv, o_proj, gate_up, down, lm_head) with 512 fp32 activation
    rows through the reference's matmul loop (QuantizedWeight.matmul,
    Phi3Weights.java:157-192, which dequantizes every block again for each
    row), TFLOP/s over those five; a shape whose estimated time would pass
    `m512_seconds` in total runs on a prefix of its rows instead (the rate is
    per row).  Threads: one per core the process may use, at most 16.  No JDK
    is probed for beyond PATH: with one, the reference's own Java path could
    be timed; without, the C restatement is (kind "port")."""
    import shutil
    import mnb_oracle as orc
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    orc.build()
    rng = np.random.default_rng(99)
    done_bytes = 0
    done = 0
    t_total = 0.0
    while t_total < seconds:
        (name, layer, K, N), t = projs[done % len(projs)], host[done % len(projs)]
        s32 = orc.fp16_bits_to_fp32(t.scales_f16.view(np.uint16))
        z = np.full((N * t.kb + 1) // 2, 0x88, np.uint8)
        x = rng.standard_normal(K).astype(np.float16).astype(np.float32)
        y = np.zeros(N, np.float32)
        t0 = time.perf_counter()
        orc.matvec(t.q, s32, z, N, K, BLOCK, x, y, lanes=8, threads=threads)
        t_total += time.perf_counter() - t0
        done_bytes += t.algorithmic_bytes(1)
        done += 1
    # M = 512: one projection per shape, rows capped by the time budget
    shapes, flops, secs, rows_done = {}, 0.0, 0.0, {}
    for (name, layer, K, N), t in zip(projs, host):
        if name not in shapes:
            shapes[name] = t
    rate = None     # flop/s measured so far, to size the later shapes
    for name, t in shapes.items():
        M = 512
        if rate is not None:
            left = max(0.5, m512_seconds - secs) / max(1, len(shapes) - len(rows_done))
            M = max(8, min(512, int(left * rate / (2.0 * t.N * t.K))))
        s32 = orc.fp16_bits_to_fp32(t.scales_f16.view(np.uint16))
        z = np.full((t.N * t.kb + 1) // 2, 0x88, np.uint8)
        x = rng.standard_normal((M, t.K)).astype(np.float16).astype(np.float32)
        t0 = time.perf_counter()
        orc.matmul(t.q, s32, z, t.N, t.K, BLOCK, x, lanes=8, threads=threads)
        dt = time.perf_counter() - t0
        secs += dt
        flops += 2.0 * M * t.N * t.K
        rate = flops / secs
        rows_done[name] = M
    jdk = shutil.which("java")
    return {"value": round(done_bytes / t_total / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "host_cpus": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)), "jdk": jdk,
            "sample": "%d decode-step projections at M=1 in step order (%.2f GB of weights, %.2f steps), fp32 "
                      "activations, 8-lane FMA block dot, %d threads, %.1f s" % (
                          done, done_bytes / 1e9, done / len(projs), threads, t_total),
            "m512": {"value": round(flops / secs / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
                     "rows": rows_done, "seconds": round(secs, 2),
                     "sample": "one projection per Phi-3 shape with 512 fp32 activation rows (fewer where the "
                               "time budget ran out: rows listed), the reference's matmul loop that dequantizes "
                               "every block again per row, 8-lane FMA block dot, %d threads" % threads}}


def qwen_tied_lm_head(torch, mnb_hip, ctx, stream, args):
    """Qwen2.5-0.5B tied lm_head: embed_tokens [151936, 896] (fp32, N(0, 0.02))
    quantized on the device to int4 (bs 128, fp32 scales, zero points), then
    the tall-skinny M=1 product.  Four copies of the quantized head (292 MB,
    more than the 256 MB MALL, as a decode step that runs the whole model
    between two heads would see it) are used in turn by 40 back-to-back
    launches, captured in a HIP graph; one event pair brackets each replay, so
    the per-launch time excludes event overhead."""
    V, H = 151936, 896
    gen = torch.Generator(device="cuda").manual_seed(151936)
    emb = torch.randn(V, H, device="cuda", generator=gen) * 0.02
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    w = mnb_hip.Weight.quantize(ctx, emb)
    quant_ms = (time.perf_counter() - t0) * 1e3
    ws = [w] + [mnb_hip.Weight.quantize(ctx, emb) for _ in range(3)]
    del emb
    x = torch.randn(H, device="cuda", generator=gen).half()
    y = torch.empty(V, device="cuda", dtype=torch.float16)
    per_replay = 40
    la = Launcher(ctx, [ws[i % len(ws)] for i in range(per_replay)], [x] * per_replay, [y] * per_replay, 1, stream)
    g = capture(torch, la, stream)
    wall, gpu = time_graph(torch, g, stream, args.steps, args.warmup, args.settle_ms)
    us = gpu / per_replay * 1e6
    kb = H // 128
    nbytes = V * H // 2 + V * kb * 4 + (V * kb + 1) // 2 + H * 2 + V * 2
    del g
    for w in ws:
        w.close()
    gbs = nbytes / us / 1e3
    log("qwen tied lm_head: quantize %.2f ms, M=1 product %.2f us, %.1f GB/s" % (quant_ms, us, gbs))
    return {"shape": [V, H], "block_size": 128, "quantize_ms_incl_alloc": round(quant_ms, 3),
            "m1_avg_launch_us": round(us, 3), "m1_bytes_per_launch": nbytes, "m1_gbs": round(gbs, 1),
            "m1_frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "kernel": "mnb::gemv_kernel (fp32 scales, zero points, bs 128)",
            "timing": "GPU time of graph replays of 40 back-to-back launches over 4 copies of the head / 40",
            "note": "bytes = packed int4 + fp32 scales + zero points + fp16 x and y"}


def config0_qkv(torch, mnb_hip, ctx, stream, args):
    """The single MatMulNBits op of the reference's CPU case: M=1, K=3072,
    N=9216 (Phi-3-mini fused qkv), bs 32, fp16 scales, no zero points, fp16
    x and y.  17 device copies of the weight (272 MB, more than the 256 MB
    MALL) are used in turn by 68 back-to-back launches captured in a HIP
    graph, so each launch reads its weight from HBM; the per-launch time is
    the graph's GPU time / 68."""
    from mnb_hip import synth
    N, K, copies, per_replay = 9216, 3072, 17, 68
    t = synth.make_weight(0, N, K, BLOCK)
    ws = [mnb_hip.Weight(ctx, N, K, BLOCK, t.q, t.scales_f16) for _ in range(copies)]
    gen = torch.Generator(device="cuda").manual_seed(3072)
    x = torch.randn(K, device="cuda", generator=gen).half()
    y = torch.empty(N, device="cuda", dtype=torch.float16)
    la = Launcher(ctx, [ws[i % copies] for i in range(per_replay)], [x] * per_replay, [y] * per_replay, 1, stream)
    g = capture(torch, la, stream)
    wall, gpu = time_graph(torch, g, stream, args.steps, args.warmup, args.settle_ms)
    del g
    for w in ws:
        w.close()
    us = gpu / per_replay * 1e6
    nbytes = t.algorithmic_bytes(1)
    gbs = nbytes / us / 1e3
    log("config 0 (qkv 3072->9216, M=1, single launches from HBM): %.2f us, %.1f GB/s" % (us, gbs))
    return {"shape": [N, K], "block_size": BLOCK, "avg_launch_us": round(us, 3), "bytes_per_launch": nbytes,
            "gbs": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "kernel": "mnb::gemv_kernel (one launch per product)",
            "timing": "GPU time of graph replays of 68 back-to-back launches over 17 weight copies (272 MB) / 68"}


def phi3_export_variant(torch, mnb_hip, ctx, stream, args):
    """The Phi-3-mini step in the weight format of the reference's DirectML
    int4 export (model/phi3-mini-directml-int4/directml/
    directml-int4-awq-block-128: block size 128, explicit uint8 zero points
    in the ONNX row-padded layout, fp16 scales), seeded random weights: the
    129 projections as one group launch at M=1 (GB/s of algorithmic bytes,
    zero points included) and at M=512 (TFLOP/s)."""
    from mnb_hip import synth
    bs = 128
    projs = synth.phi3_decode_step()
    host, ws = [], []
    for i, (_, _, K, N) in enumerate(projs):
        t = synth.make_weight(30_000 + i, N, K, bs, with_zp=True)
        host.append(t)
        ws.append(mnb_hip.Weight(ctx, N, K, bs, t.q, t.scales_f16, t.zp_row_padded, mnb_hip.MNB_ZP_ROW_PADDED))
    gen = torch.Generator(device="cuda").manual_seed(128)
    out = {"projections": len(projs), "block_size": bs, "zero_points": "explicit, uint8 row-padded (ONNX layout)"}
    for M in (1, 512):
        if M == 1:
            xs = [torch.randn(K, device="cuda", generator=gen).half() for (_, _, K, _) in projs]
        else:
            xk = {K: torch.randn(M, K, device="cuda", generator=gen).half() for (_, _, K, _) in projs}
            xs = [xk[K] for (_, _, K, _) in projs]
        ys = [torch.empty(M, N, device="cuda", dtype=torch.float16) for (_, _, _, N) in projs]
        grp = mnb_hip.Group(ctx, list(zip(ws, xs, ys)))
        wall, gpu = time_steps(torch, lambda: grp.run(stream.cuda_stream), stream, args.steps, args.warmup,
                               args.settle_ms, args.eager)
        grp.close()
        if M == 1:
            nbytes = sum(t.algorithmic_bytes(1) for t in host)
            e = {"us_per_step": round(wall * 1e6, 2), "gpu_us_per_step": round(gpu * 1e6, 2), "bytes_per_step": nbytes,
                 "gbs": round(nbytes / wall / 1e9, 1), "frac_hbm_peak": round(nbytes / wall / 1e9 / HBM_PEAK_GBS, 4),
                 "kernel": "mnb::gemv_stream_kernel (one launch per step)"}
            log("export-format step M=1 as one group launch: %.1f us, %.1f GB/s" % (wall * 1e6, e["gbs"]))
        else:
            flops = sum(2.0 * M * N * K for (_, _, K, N) in projs)
            e = {"us_per_step": round(wall * 1e6, 2), "gpu_us_per_step": round(gpu * 1e6, 2),
                 "tflops": round(flops / wall / 1e12, 2), "frac_fp16_peak": round(flops / wall / 1e12 / FP16_PEAK_TFLOPS, 4),
                 "kernel": "mnb::gemm_sk_kernel (one group launch per step)"}
            log("export-format step M=512 as one group launch: %.1f us, %.1f TFLOP/s" % (wall * 1e6, e["tflops"]))
        out["m%d" % M] = e
        del xs, ys
        torch.cuda.empty_cache()
    for w in ws:
        w.close()
    return out


def qwen_step(torch, mnb_hip, ctx, stream, args):
    """Qwen2.5-0.5B-shaped q4f16 step with a quantized lm_head: 24 layers x
    {qkv 896->1152, o 896->896, gate_up 896->9728, down 4864->896} + lm_head
    896->151936, bs 32, fp16 scales in [0.005, 0.02], no zero points.  The 97
    projections are recorded as one group and replayed in a HIP graph, at
    M=1 (each with its own activation; GB/s of algorithmic bytes) and at
    M=64 (one activation per K, one output per projection; TFLOP/s)."""
    from mnb_hip import synth
    projs = synth.qwen_decode_step()
    host, ws = [], []
    for i, (_, _, K, N) in enumerate(projs):
        t = synth.make_weight(20_000 + i, N, K, BLOCK)
        host.append(t)
        ws.append(mnb_hip.Weight(ctx, N, K, BLOCK, t.q, t.scales_f16))
    gen = torch.Generator(device="cuda").manual_seed(896)
    out = {"projections": len(projs), "block_size": BLOCK}
    for M in (1, 64):
        if M == 1:
            xs = [torch.randn(K, device="cuda", generator=gen).half() for (_, _, K, _) in projs]
        else:
            xk = {K: torch.randn(M, K, device="cuda", generator=gen).half() for (_, _, K, _) in projs}
            xs = [xk[K] for (_, _, K, _) in projs]
        ys = [torch.empty(M, N, device="cuda", dtype=torch.float16) for (_, _, _, N) in projs]
        grp = mnb_hip.Group(ctx, list(zip(ws, xs, ys)))
        wall, gpu = time_steps(torch, lambda: grp.run(stream.cuda_stream), stream, args.steps, args.warmup,
                               args.settle_ms, args.eager)
        grp.close()
        nbytes = sum(t.algorithmic_bytes(M) for t in host)
        flops = sum(2.0 * M * N * K for (_, _, K, N) in projs)
        e = {"us_per_step": round(wall * 1e6, 2), "gpu_us_per_step": round(gpu * 1e6, 2), "bytes_per_step": nbytes,
             "gbs": round(nbytes / wall / 1e9, 1), "tflops": round(flops / wall / 1e12, 2)}
        # the roofline that bounds the step: HBM below the ridge (2.5 PFLOP/s /
        # 8 TB/s = 312.5 flop per byte), MFMA above it; both fractions reported
        e["flop_per_byte"] = round(flops / nbytes, 1)
        e["bound"] = "hbm" if flops / nbytes < RIDGE_FLOP_PER_BYTE else "mfma"
        e["frac_hbm_peak"] = round(nbytes / wall / 1e9 / HBM_PEAK_GBS, 4)
        e["frac_fp16_peak"] = round(flops / wall / 1e12 / FP16_PEAK_TFLOPS, 4)
        if M == 1:
            e["kernel"] = "mnb::gemv_stream_kernel (one launch per step)"
        else:
            e["kernel"] = "mnb::gemm_sk_kernel (one group launch per step)"
        out["m%d" % M] = e
        log("qwen step M=%d as one group launch: %.1f us, %.1f GB/s, %.1f TFLOP/s" % (M, wall * 1e6, e["gbs"],
                                                                                    e["tflops"]))
        del xs, ys
    for w in ws:
        w.close()
    return out


def mfma_ceiling(torch, stream, settle_ms, launches=20):
    """What the matrix cores sustain at the GEMM's occupancy: TFLOP/s of
    libmnb_probe.so's MFMA-only kernel (v_mfma_f32_32x32x16_f16 on operands
    drawn like the GEMM's, 256 workgroups of 8 waves, no memory traffic in
    its loop), timed with HIP events on the launch stream after `settle_ms`
    of untimed launches."""
    lib = ctypes.CDLL(os.path.join(ROOT, "win-directml-java_amd", "mnb_hip", "libmnb_probe.so"))
    lib.mnb_probe_mfma.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p]
    lib.mnb_probe_mfma.restype = ctypes.c_int32
    lib.mnb_probe_mfma_flops.argtypes = [ctypes.c_int32, ctypes.c_int32]
    lib.mnb_probe_mfma_flops.restype = ctypes.c_double
    wgs, iters = 256, 600
    out = torch.empty(wgs * 512, dtype=torch.float32, device="cuda")
    run = lambda n: lib.mnb_probe_mfma(wgs, iters, n, ctypes.c_void_p(out.data_ptr()),
                                       ctypes.c_void_p(stream.cuda_stream))
    assert run(1) == 0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    assert run(4) == 0
    torch.cuda.synchronize()
    one = (time.perf_counter() - t0) / 4
    assert run(int(max(1, settle_ms * 1e-3 / one))) == 0
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    assert run(launches) == 0
    e1.record(stream)
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) * 1e-3 / launches
    return lib.mnb_probe_mfma_flops(wgs, iters) / sec / 1e12, sec * 1e6


def dense_fp16_gemm(torch, stream, projs, M, steps, warmup, settle_ms):
    """The same projections as dense fp16 products through torch (hipBLASLt):
    one fp16 weight [N, K] per projection (random, about 2 bytes per weight
    where the int4 path streams about 0.56), x [M, K] fp16 per K, y fp16 per
    N, 129 launches in stream order captured in a HIP graph; TFLOP/s of the
    wall time per step.  A reference point for the single-product int4 path,
    not part of it."""
    gen = torch.Generator(device="cuda").manual_seed(4096)
    ws = [torch.randn(N, K, device="cuda", dtype=torch.float16, generator=gen) * 0.05 for (_, _, K, N) in projs]
    xs = {K: torch.randn(M, K, device="cuda", dtype=torch.float16, generator=gen) for (_, _, K, _) in projs}
    ys = {N: torch.empty(M, N, device="cuda", dtype=torch.float16) for (_, _, _, N) in projs}
    order = [(xs[K], w, ys[N]) for (_, _, K, N), w in zip(projs, ws)]

    def run():
        for x, w, y in order:
            torch.mm(x, w.t(), out=y)
    with torch.cuda.stream(stream):
        run()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        run()
    torch.cuda.synchronize()
    wall, _ = time_graph(torch, g, stream, steps, warmup, settle_ms)
    del g, ws, xs, ys, order
    torch.cuda.empty_cache()
    return sum(2.0 * M * N * K for (_, _, K, N) in projs) / wall / 1e12


def ceilings(torch, stream, args):
    """Reference points for the prefill GEMM's roofline fraction: the MFMA
    ceiling the chip sustains, and hipBLASLt's dense fp16 GEMM of the same
    129 Phi-3 projections as 129 launches (the single-product int4 path's
    counterpart)."""
    from mnb_hip import synth
    tf, us = mfma_ceiling(torch, stream, args.settle_ms)
    log("MFMA-only ceiling: %.1f TFLOP/s (%.1f us per launch)" % (tf, us))
    projs = synth.phi3_decode_step()
    dense = {}
    for M in (512, 2048):
        dense[str(M)] = round(dense_fp16_gemm(torch, stream, projs, M, max(3, args.steps // 4), 2, args.settle_ms), 1)
        log("dense fp16 GEMM (hipBLASLt) of the 129 projections at M=%d as 129 launches: %.1f TFLOP/s" % (
            M, dense[str(M)]))
    return {"mfma_ceiling_tflops": round(tf, 1), "mfma_ceiling_frac_fp16_peak": round(tf / FP16_PEAK_TFLOPS, 4),
            "mfma_ceiling_us_per_launch": round(us, 1),
            "dense_fp16_gemm_tflops": dense,
            "note": "mfma_ceiling: libmnb_probe.so, v_mfma_f32_32x32x16_f16 only, 256 workgroups of 8 waves; "
                    "dense_fp16_gemm: torch.mm (hipBLASLt) of the same 129 Phi-3 projections with dense fp16 "
                    "weights as 129 launches in a HIP graph"}


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py measures one GPU; this build has no multi-GPU path (requested --gpus %d)" % args.gpus,
              file=sys.stderr)
        sys.exit(2)
    import torch
    import mnb_hip
    from mnb_hip import synth

    ctx = mnb_hip.Context(0)
    info = ctx.info()
    log("device %s %s, %d CUs" % (info.name.decode(), info.arch.decode(), info.compute_units))
    stream = torch.cuda.Stream()
    if args.phase == "qwen":
        print(json.dumps({"phase": "qwen", "qwen_step": qwen_step(torch, mnb_hip, ctx, stream, args)}), flush=True)
        ctx.close()
        return
    if args.phase == "export":
        print(json.dumps({"phase": "export", "phi3_export_variant": phi3_export_variant(torch, mnb_hip, ctx, stream, args)}),
              flush=True)
        ctx.close()
        return
    if args.phase == "ceilings":
        print(json.dumps({"phase": "ceilings", "ceilings": ceilings(torch, stream, args)}), flush=True)
        ctx.close()
        return
    if args.phase == "config0":
        print(json.dumps({"phase": "config0", "config0_single_qkv": config0_qkv(torch, mnb_hip, ctx, stream, args)}),
              flush=True)
        ctx.close()
        return

    projs = synth.phi3_decode_step()
    host, weights = [], []
    t0 = time.perf_counter()
    for i, (name, layer, K, N) in enumerate(projs):
        t = synth.make_weight(10_000 + i, N, K, BLOCK)
        host.append(t)
        weights.append(mnb_hip.Weight(ctx, N, K, BLOCK, t.q, t.scales_f16))
    log("uploaded %d weights (%.2f GB resident) in %.1f s" % (
        len(weights), sum(w.device_bytes for w in weights) / 1e9, time.perf_counter() - t0))
    bytes_step = sum(t.algorithmic_bytes(1) for t in host)

    # ---------------- decode step, M = 1 ----------------
    gen = torch.Generator(device="cuda").manual_seed(5)

    # prefill-shaped products: the same 129 projections at M rows, either one
    # launch each in stream order (group=False; projections of equal N share
    # one output buffer) or recorded as one group and run as one launch
    # (group=True; each projection has its own output, as group items may run
    # concurrently)
    def prefill(M, group=False):
        xs_m, ys_m = {}, []
        for (_, _, K, N) in projs:
            if K not in xs_m:
                xs_m[K] = torch.randn(M, K, device="cuda", generator=gen).half()
        xs_l = [xs_m[K] for (_, _, K, _) in projs]
        ybuf = {}
        for (_, _, K, N) in projs:
            if group:
                ys_m.append(torch.empty(M, N, device="cuda", dtype=torch.float16))
                continue
            if N not in ybuf:
                ybuf[N] = torch.empty(M, N, device="cuda", dtype=torch.float16)
            ys_m.append(ybuf[N])
        if group:
            la = mnb_hip.Group(ctx, list(zip(weights, xs_l, ys_m)))
            run = lambda: la.run(stream.cuda_stream)
        else:
            la = Launcher(ctx, weights, xs_l, ys_m, M, stream)
            run = la.run
        steps = max(3, args.steps // 4) if M >= 512 and not group else args.steps
        wall_m, gpu_m = time_steps(torch, run, stream, steps, 2, args.settle_ms, args.eager)
        flops = sum(2.0 * M * N * K for (_, _, K, N) in projs)
        if group:
            la.close()
            la = None
        return la, flops, wall_m, gpu_m


    if args.phase == "prefill":
        _, fl, w_m, g_m = prefill(args.prefill_m, group=args.prefill_group)
        print(json.dumps({"phase": "prefill", "M": args.prefill_m, "group": args.prefill_group,
                          "tflops": round(fl / w_m / 1e12, 2),
                          "us_per_step": round(w_m * 1e6, 1), "gpu_us_per_step": round(g_m * 1e6, 1),
                          "flops_per_step": fl}), flush=True)
        for w in weights:
            w.close()
        ctx.close()
        return

    xs = [torch.randn(K, device="cuda", generator=gen).half() for (_, _, K, _) in projs]
    ys = [torch.empty(N, device="cuda", dtype=torch.float16) for (_, _, _, N) in projs]

    if args.phase == "chain":
        dec = Launcher(ctx, weights, xs, ys, 1, stream)
        wall_seq, gpu_seq = time_steps(torch, dec.run, stream, args.steps, args.warmup, args.settle_ms, args.eager)
        print(json.dumps({"phase": "chain", "gbs": round(bytes_step / wall_seq / 1e9, 2),
                          "us_per_step": round(wall_seq * 1e6, 2), "gpu_us_per_step": round(gpu_seq * 1e6, 2),
                          "launches_per_step": len(projs), "bytes_per_step": bytes_step}), flush=True)
        for w in weights:
            w.close()
        ctx.close()
        return

    # (1) headline: the 129 projections (each with its own activation, no
    #     dependence between them) recorded once as a group and run as one
    #     launch of the streaming kernel.
    grp = mnb_hip.Group(ctx, list(zip(weights, xs, ys)))
    wall, gpu = time_steps(torch, lambda: grp.run(stream.cuda_stream), stream, args.steps, args.warmup,
                           args.settle_ms, args.eager)
    value = bytes_step / wall / 1e9
    kern = group_launch_times(torch, grp, stream, reps=args.steps).mean()   # one launch per step
    achieved_gbs = bytes_step / kern / 1e9
    log("decode step as one group launch: %.1f us per step, %.1f us per launch (event brackets), %.1f GB/s" % (
        wall * 1e6, kern * 1e6, value))
    grp.close()

    if args.phase == "decode":
        copy_gbs = copy_bandwidth(torch, stream)
        print(json.dumps({"phase": "decode", "group_gbs": round(value, 2), "kernel_us": round(kern * 1e6, 2),
                          "bytes_per_step": bytes_step, "device_copy_gbs": round(copy_gbs, 1),
                          "copy_bytes_per_launch": 2 << 30}), flush=True)
        for w in weights:
            w.close()
        ctx.close()
        return

    # (2) the same projections as 129 separate launches in stream order (each
    #     launch waits for the previous one, as in a dependent decode chain).
    dec = Launcher(ctx, weights, xs, ys, 1, stream)
    wall_seq, gpu_seq = time_steps(torch, dec.run, stream, args.steps, args.warmup, args.settle_ms, args.eager)
    log("decode step as 129 launches: %.1f us wall, %.1f GB/s" % (wall_seq * 1e6, bytes_step / wall_seq / 1e9))
    d1 = per_launch_times(torch, dec, stream)
    per_shape = {}
    for (name, layer, K, N), t, d in zip(projs, host, d1):
        e = per_shape.setdefault(name, {"K": K, "N": N, "bytes": t.algorithmic_bytes(1), "us": []})
        e["us"].append(d * 1e6)
    for name, e in per_shape.items():
        us = float(np.mean(e.pop("us")))
        e["avg_us"] = round(us, 3)
        e["gbs"] = round(e["bytes"] / us / 1e3, 1)
    log("per-launch (event brackets): " + json.dumps(per_shape))

    # ---------------- prefill, M = 512 (+ sweep) ----------------
    # (1) the 129 projections recorded as one group: one stream-K launch over
    #     all their tiles (plus the split-tile reduce)
    _, flops512, wall512, gpu512 = prefill(512, group=True)
    tflops512 = flops512 / wall512 / 1e12
    # a replay is the GEMM launch and its reduce back to back, so the GPU time
    # per replay is the kernel time of one step
    kernel_tflops512 = flops512 / gpu512 / 1e12
    log("prefill M=512 as one group launch: %.1f us per step, %.1f us GPU time, %.1f TFLOP/s (kernel time %.1f)" % (
        wall512 * 1e6, gpu512 * 1e6, tflops512, kernel_tflops512))
    torch.cuda.empty_cache()
    # (2) the same projections as 129 launches in stream order
    la512, _, wall512s, gpu512s = prefill(512)
    tflops512s = flops512 / wall512s / 1e12
    kernel_tflops512s = flops512 / gpu512s / 1e12
    log("prefill M=512 as 129 launches: %.1f us per step, %.1f us GPU time, %.1f TFLOP/s (kernel time %.1f)" % (
        wall512s * 1e6, gpu512s * 1e6, tflops512s, kernel_tflops512s))
    del la512
    sweep, sweep_seq = {}, {}
    # both fractions per M (M = 128 sits near the ridge of the two rooflines)
    frac, frac_seq = {}, {}

    def fractions(M, fl, w_m):
        nb = sum(t.algorithmic_bytes(M) for t in host)
        return {"tflops": round(fl / w_m / 1e12, 2), "frac_fp16_peak": round(fl / w_m / 1e12 / FP16_PEAK_TFLOPS, 4),
                "gbs": round(nb / w_m / 1e9, 1), "frac_hbm_peak": round(nb / w_m / 1e9 / HBM_PEAK_GBS, 4),
                "flop_per_byte": round(fl / nb, 1)}

    if not args.no_sweep:
        for M in (16, 128, 2048):
            _, fl, w_m, _ = prefill(M, group=True)
            sweep[str(M)] = round(fl / w_m / 1e12, 2)
            frac[str(M)] = fractions(M, fl, w_m)
            torch.cuda.empty_cache()
            _, fl, w_m, _ = prefill(M)
            sweep_seq[str(M)] = round(fl / w_m / 1e12, 2)
            frac_seq[str(M)] = fractions(M, fl, w_m)
            torch.cuda.empty_cache()
            log("prefill M=%d: %.1f TFLOP/s as one group launch, %.1f as 129 launches" % (
                M, sweep[str(M)], sweep_seq[str(M)]))
    # small-batch decode: the 129 projections with 2 and 4 rows each as one
    # group launch (the streaming kernel with M activation rows per job)
    small_batch = {}
    for M in (2, 4):
        _, fl, w_m, _ = prefill(M, group=True)
        nb = sum(t.algorithmic_bytes(M) for t in host)
        small_batch[str(M)] = {"us_per_step": round(w_m * 1e6, 1), "gbs": round(nb / w_m / 1e9, 1),
                               "bytes_per_step": nb, "tflops": round(fl / w_m / 1e12, 2)}
        torch.cuda.empty_cache()
        log("small-batch decode M=%d as one group launch: %.1f us, %.1f GB/s" % (M, w_m * 1e6, nb / w_m / 1e9))

    copy_gbs = copy_bandwidth(torch, stream)
    log("device copy bandwidth: %.0f GB/s" % copy_gbs)
    read_gbs = torch_read_bandwidth(torch, stream)
    log("torch int64 sum read rate: %.0f GB/s" % read_gbs)

    for w in weights:
        w.close()
    del weights
    torch.cuda.empty_cache()
    cfg0 = config0_qkv(torch, mnb_hip, ctx, stream, args)
    qwen_head = qwen_tied_lm_head(torch, mnb_hip, ctx, stream, args)
    qwen = qwen_step(torch, mnb_hip, ctx, stream, args)
    torch.cuda.empty_cache()
    export = phi3_export_variant(torch, mnb_hip, ctx, stream, args)
    torch.cuda.empty_cache()
    ceil = ceilings(torch, stream, args)
    ctx.close()

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(host, projs, args.cpu_seconds, args.cpu_m512_seconds)
        log("cpu baseline: %s" % json.dumps(cpu))

    result = {
        "metric": "int4 MatMulNBits GB/s at M=1 (Phi-3-mini decode step)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": args.settle_ms,
        "ms_per_step": round(wall * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded random int4 weights, fp16 scales in [0.005,0.02], fp16 N(0,1) activations)",
        "config": {"workload": "phi3-mini int4 decode step: 32 x {qkv 3072->9216, o 3072->3072, "
                               "gate_up 3072->16384, down 8192->3072} + lm_head 3072->32064, M=1, bs=32, "
                               "implicit zero point 8, each projection with its own activation; "
                               "the 129 projections recorded as one group and run as one launch",
                   "M": 1, "block_size": BLOCK, "projections": len(projs), "bytes_per_step": bytes_step},
        "roofline": {"bound": "hbm", "achieved": round(achieved_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("gemv_stream_phi3_decode_step.md"),
                     "traffic_source": "profiles/gemv_stream_phi3_decode_step.md (rocprofv3 FETCH_SIZE + WRITE_SIZE)",
                     "kernel": "mnb::gemv_stream_kernel (one launch per step)",
                     "avg_launch_us": round(kern * 1e6, 2)},
        "decode_step_sequential": {"gbs": round(bytes_step / wall_seq / 1e9, 2),
                                   "ms_per_step": round(wall_seq * 1e3, 4),
                                   "gpu_ms_per_step": round(gpu_seq * 1e3, 4),
                                   "frac_hbm_peak": round(bytes_step / wall_seq / 1e9 / HBM_PEAK_GBS, 4),
                                   "note": "the same 129 projections as 129 stream-ordered launches "
                                           "(mnb::gemv_kernel, HIP graph); gpu_ms_per_step is the span of "
                                           "HIP events around the replays on the launch stream",
                                   "per_shape": per_shape},
        "prefill_m512": {"tflops": round(tflops512, 2), "ms_per_step": round(wall512 * 1e3, 4),
                         "flops_per_step": flops512, "frac_fp16_peak": round(tflops512 / FP16_PEAK_TFLOPS, 4),
                         "note": "the 129 projections at M=512 (fp16 x and y, each projection with its own "
                                 "output) recorded as one group and run as one launch, like the decode step",
                         "roofline": {"bound": "mfma", "achieved": round(kernel_tflops512, 2),
                                      "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                      "frac": round(kernel_tflops512 / FP16_PEAK_TFLOPS, 4),
                                      "kernel": "mnb::gemm_sk_kernel (one group launch per step: 128x512 tiles in tile-list order)",
                                      "avg_launch_us": round(gpu512 * 1e6, 2),
                                      "traffic": measured_traffic("gemm_sk_phi3_prefill_m512_group.md",
                                                                  "traffic_bytes_per_step"),
                                      "traffic_unit": "HBM bytes per step (one launch)",
                                      "traffic_source": "profiles/gemm_sk_phi3_prefill_m512_group.md "
                                                        "(rocprofv3 FETCH_SIZE + WRITE_SIZE)"},
                         "sweep_tflops": sweep, "sweep_fractions": frac},
        "prefill_m512_sequential": {
                         "tflops": round(tflops512s, 2), "ms_per_step": round(wall512s * 1e3, 4),
                         "frac_fp16_peak": round(tflops512s / FP16_PEAK_TFLOPS, 4),
                         "note": "the same projections as 129 stream-ordered launches (HIP graph)",
                         "roofline": {"bound": "mfma", "achieved": round(kernel_tflops512s, 2),
                                      "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                      "frac": round(kernel_tflops512s / FP16_PEAK_TFLOPS, 4),
                                      "kernel": "mnb::gemm_sk_kernel, mnb::gemm_ks_kernel for o_proj (M=512, one launch per projection)",
                                      "avg_launch_us": round(gpu512s / len(projs) * 1e6, 2),
                                      "traffic": measured_traffic("gemm_sk_phi3_prefill_m512.md",
                                                                  "traffic_bytes_per_step"),
                                      "traffic_unit": "HBM bytes per step (129 launches)",
                                      "traffic_source": "profiles/gemm_sk_phi3_prefill_m512.md "
                                                        "(rocprofv3 FETCH_SIZE + WRITE_SIZE)"},
                         "sweep_tflops": sweep_seq, "sweep_fractions": frac_seq},
        "small_batch_decode": dict(small_batch, note="the 129 projections with M rows each recorded as one group "
                                                     "(mnb::gemv_stream_kernel with M activation rows per job)"),
        "device_copy_gbs": round(copy_gbs, 1),
        "torch_read_gbs": round(read_gbs, 1),
        "config0_single_qkv": cfg0,
        "qwen_tied_lm_head": qwen_head,
        "qwen_step": qwen,
        "phi3_export_variant": export,
        "ceilings": ceil,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
