"""Schedules of group launches (win-directml-java_amd/csrc/mnb_sched.cpp),
checked on the CPU: the tile list of a grouped prefill GEMM
(mnb::sk_tile_list) and the static unit lists of the M = 1 streaming kernel
(mnb::stream_schedule).

The grouped launch replaces a sequence of the reference's batched GEMM
dispatches (INT4_MATMUL_BATCH_TILED_HLSL, MatMulNBitsKernel.java:732-820,
one per projection); the reference has no counterpart of this schedule, so
what is pinned here are its invariants: every output tile of every item is
computed exactly once, each workgroup's iteration range equals the stages of
its own tiles, the ranges tile the launch, and the per-workgroup work is
balanced; a tile list with parts covers each cut tile's stages exactly once,
in K order, with the partial tiles the reduce list names."""
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "win-directml-java_amd", "csrc")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("sched") / "sched_check")
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Werror", "-I" + CSRC, "-o", exe,
                    os.path.join(ROOT, "tests", "sched_check.cpp"), os.path.join(CSRC, "mnb_sched.cpp")],
                   check=True)
    return exe


def run(checker, G, items):
    """items: (MT, NG, ST) per item.  Returns the checker's figures."""
    inp = "%d\n" % G + "\n".join("%d %d %d" % t for t in items) + "\n"
    r = subprocess.run([checker], input=inp, capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout
    return {k: float(v) for k, v in re.findall(r"(\w+)=([\d.]+)", r.stdout)}


def phi3(M):
    """The Phi-3-mini decode step's 129 projections at M rows: (MT, NG, ST)."""
    MT = (M + 127) // 128
    layer = [(3072, 9216), (3072, 3072), (3072, 16384), (8192, 3072)]
    return [(MT, (N + 255) // 256, (K + 127) // 128) for _ in range(32) for K, N in layer] + \
        [(MT, (32064 + 255) // 256, 24)]


@pytest.mark.parametrize("M", [128, 512, 2048])
def test_phi3_step_groups(checker, M):
    f = run(checker, 256, phi3(M))
    assert f["imbalance"] < (0.06 if M == 128 else 0.01)
    # side by side on one XCD: a few x row blocks (blocks of at most 4
    # m-tiles by 8 n-groups), not one per workgroup
    assert f["x_blocks"] <= {128: 4, 512: 6, 2048: 6}[M]


def test_tile_list_group_of_the_gpu_test(checker):
    specs = [(512, 3072, 9216), (700, 576, 8000), (2048, 1536, 3072), (300, 2048, 5000), (4500, 256, 1100),
             (129, 3072, 16384), (64, 200, 30000), (1024, 1024, 4096)]
    items = [((M + 127) // 128, (N + 255) // 256, (((K + 31) // 32) * 32 + 127) // 128) for M, K, N in specs]
    f = run(checker, 256, items)
    assert f["tiles"] == 1142


@pytest.mark.parametrize("seed", range(40))
def test_random_groups(checker, seed):
    rng = np.random.default_rng(seed)
    G = int(rng.choice([1, 3, 8, 64, 80, 104, 256]))
    n = int(rng.integers(1, 40))
    items = [(int(rng.integers(1, 41)), int(rng.integers(1, 131)), int(rng.integers(1, 71))) for _ in range(n)]
    run(checker, G, items)


def run_parts(checker, lines):
    """lines: (G, split_above, [(MT, NG, ST), ...]) per case.  Returns the
    checker's output lines (one per case, then a summary)."""
    inp = "parts\n" + "".join("%d %d " % (G, split) + " ".join("%d %d %d" % t for t in items) + "\n"
                              for G, split, items in lines)
    r = subprocess.run([checker], input=inp, capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    return r.stdout.splitlines()


def qwen_m64():
    """The Qwen2.5-0.5B step's 97 projections at M = 64 in 64 x 512 tiles."""
    layer = [(896, 1152), (896, 896), (896, 9728), (4864, 896)]
    return [(1, (N + 511) // 512, (K + 127) // 128) for _ in range(24) for K, N in layer] + \
        [(1, (151936 + 511) // 512, 7)]


def test_tile_list_parts_of_the_qwen_step_at_m64(checker):
    """The down tiles (38 stages) against a mean of 31 stages per workgroup:
    cut into two parts each, the busiest workgroup falls from 38 to 35 stages
    (the rest is the 7-stage tiles' granularity)."""
    items = qwen_m64()
    iters = sum(a * b * c for a, b, c in items)
    mean = -(-iters // 256)
    out = run_parts(checker, [(256, 0, items), (256, mean, items)])
    whole = dict(re.findall(r"(\w+)=([\d.]+)", out[0]))
    cut = dict(re.findall(r"(\w+)=([\d.]+)", out[1]))
    assert int(whole["busiest"]) == 38 and int(whole["cut"]) == 0
    assert int(cut["cut"]) == 48 and int(cut["busiest"]) <= 35


@pytest.mark.parametrize("seed", range(30))
def test_tile_list_parts_random(checker, seed):
    """Random groups and cut lengths: coverage of every tile's stages by its
    parts in K order, consecutive partial indices named by the reduce list,
    workgroup ranges, balance; or a refusal when the parts would exceed the
    workspace's partial tiles or the list."""
    rng = np.random.default_rng(1000 + seed)
    cases = []
    for _ in range(4):
        G = int(rng.choice([1, 8, 40, 128, 256]))
        n = int(rng.integers(1, 12))
        items = [(int(rng.integers(1, 5)), int(rng.integers(1, 60)), int(rng.integers(1, 90))) for _ in range(n)]
        cases.append((G, int(rng.integers(0, 40)), items))
    out = run_parts(checker, cases)
    assert out[-1] == "ok parts cases=%d" % len(cases)
    assert all(l.startswith("ok parts busiest=") or l.startswith("refused") for l in out[:-1])


def test_tile_list_parts_refused_beyond_the_list(checker):
    """More than 256 partial tiles (300 or 129 tiles of 2 parts, 64 tiles of
    10): refused, so the planner keeps whole tiles; 128 tiles of 2 parts fit."""
    out = run_parts(checker, [(256, 10, [(1, 300, 20)]), (256, 10, [(1, 128, 20)]), (256, 2, [(1, 64, 20)]),
                              (256, 10, [(1, 129, 20)])])
    assert out[0].startswith("refused") and out[1].startswith("ok parts") and out[2].startswith("refused")
    assert out[3].startswith("refused")


def test_more_workgroups_than_tiles(checker):
    f = run(checker, 256, [(1, 3, 24), (2, 1, 5)])
    assert f["tiles"] == 5


# ------------------------------------------------ M = 1 streaming schedule

def run_stream(checker, waves, items):
    """items: (NT, ST) per item.  Returns the checker's figures (None when refused)."""
    inp = "stream\n%d\n" % waves + "\n".join("%d %d" % t for t in items) + "\n"
    r = subprocess.run([checker], input=inp, capture_output=True, text=True)
    assert r.returncode == 0, r.stdout
    if r.stdout.startswith("refused"):
        return None
    assert r.stdout.startswith("ok"), r.stdout
    return {k: float(v) for k, v in re.findall(r"(\w+)=([\d.]+)", r.stdout)}


def phi3_stream_items():
    """The Phi-3-mini decode step's 129 M = 1 products: (n-tiles, super-tiles)."""
    layer = [(3072, 9216), (3072, 3072), (3072, 16384), (8192, 3072)]
    return [((N + 15) // 16, (K + 127) // 128) for _ in range(32) for K, N in layer] + [((32064 + 15) // 16, 24)]


@pytest.mark.parametrize("waves", [256 * 8, 256 * 12, 256 * 16, 1000])
def test_stream_schedule_of_the_phi3_decode_step(checker, waves):
    """The headline decode group: 32 x {qkv, o, gate_up, down} + lm_head, 65,492
    units, far more than the waves, so every wave's pipeline carries across
    many unit boundaries; every unit is listed once and the busiest wave is
    within one unit of the mean."""
    f = run_stream(checker, waves, phi3_stream_items())
    assert f["units"] == 65492
    assert f["busy"] == waves
    assert f["imbalance"] < 0.05


def test_stream_schedule_fewer_units_than_waves(checker):
    f = run_stream(checker, 4096, [(576, 24), (192, 24), (192, 64), (3, 7)])
    assert f["units"] == 963 and f["busy"] == 963


def test_stream_schedule_refuses_oversized_items(checker):
    assert run_stream(checker, 64, [(65537, 1)]) is None
    assert run_stream(checker, 64, [(65536, 1)]) is not None


@pytest.mark.parametrize("seed", range(30))
def test_stream_schedule_random_groups(checker, seed):
    rng = np.random.default_rng(100 + seed)
    waves = int(rng.choice([1, 7, 64, 1024, 3072]))
    items = [(int(rng.integers(1, 3000)), int(rng.integers(1, 80))) for _ in range(int(rng.integers(1, 60)))]
    run_stream(checker, waves, items)


# ------------------------------------------- single items in closed form

def test_closed_form_equals_the_table_of_a_single_item(checker):
    """A single product runs in tile-list order without a device table: the
    kernel computes its workgroup's tiles from the tile count (mnb::sk_cf_*).
    For every grid and shape here the closed form gives each workgroup the
    same tiles, in the same order, as sk_tile_list builds for that item: the
    Phi-3 and Qwen products at M in {16, 64, 128, 512, 2048} with 128-, 64-
    and 32-row and 256- and 512-column tiles, and random shapes and grids
    (grids not a multiple of 8, fewer tiles than workgroups, one m-tile,
    ragged m-chunks of 1 to 3 m-tiles)."""
    rng = np.random.default_rng(7)
    lines = []
    for M in (16, 64, 128, 512, 2048):
        for K, N in [(3072, 9216), (3072, 3072), (3072, 16384), (8192, 3072), (3072, 32064), (896, 1152),
                     (4864, 896), (896, 151936)]:
            for bm, bn in ((128, 256), (128, 512), (64, 512), (32, 512)):
                MT, NG, ST = -(-M // bm), -(-N // bn), -(-K // 128)
                for G in (256, 248, min(256, MT * NG)):
                    lines.append("%d %d %d %d" % (G, MT, NG, ST))
    for _ in range(400):
        lines.append("%d %d %d %d" % (int(rng.integers(1, 257)), int(rng.integers(1, 40)), int(rng.integers(1, 300)),
                                      int(rng.integers(1, 70))))
    r = subprocess.run([checker], input="closed\n" + "\n".join(lines) + "\n", capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.startswith("ok closed cases=%d" % len(lines)), r.stdout


def test_planner_grids_fit_the_workspace(checker):
    """sk_grid and sk_single_plan (the single-product GEMM planner) never pick
    more workgroups than sk_max_grid(cu_count) <= 256 nor more than the
    launch's iterations, for devices of 1 to 1024 CUs, so the partial tiles of
    every plan fit the workspace of the largest grid -- the context's
    workspace and the fixed scratch array of mnb_matmul_noalloc
    (mnb_noalloc.hip), whose size check uses the same plan."""
    rng = np.random.default_rng(17)
    lines = []
    for cu in (1, 7, 32, 80, 104, 200, 240, 255, 256, 257, 304, 512, 1024):
        for M, NT, ST in [(512, 576, 24), (512, 192, 24), (512, 1024, 24), (512, 192, 64), (512, 2004, 24),
                          (17, 1, 1), (2048, 9496, 7), (140000, 192, 64)]:
            lines.append("%d %d %d %d 0 4" % (cu, M, NT, ST))
        for _ in range(40):
            lines.append("%d %d %d %d %d %d" % (cu, rng.integers(17, 5000), rng.integers(1, 3000), rng.integers(1, 120),
                                                rng.integers(0, 2), 2 ** rng.integers(0, 4)))
    r = subprocess.run([checker], input="grid\n" + "\n".join(lines) + "\n", capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.startswith("ok grid cases=%d" % len(lines)), r.stdout


def test_reduce_split_list_matches_the_gemms_partial_tiles(checker):
    """The split tiles the reduce launch sums (mnb::sk_split_list, built by the
    host at launch time) are exactly the tiles the stream-K GEMM writes as
    partial tiles, with the same contributors in the same order and the slot
    each contributor writes: over the Phi-3 single products at M = 128, 512
    and 2048 on the grids the planner picks, and 3000 random launches of 1 to
    6 items on 1 to 256 workgroups."""
    rng = np.random.default_rng(29)
    lines = []
    for M in (128, 512, 2048):
        MT = (M + 127) // 128
        for K, N in [(3072, 9216), (3072, 3072), (3072, 16384), (8192, 3072), (3072, 32064)]:
            T, ST = MT * ((N + 255) // 256), (K + 127) // 128
            for G in (T, min(256, T * ST), 240, 192, 144):
                if 1 <= G <= min(256, T * ST):
                    lines.append("%d %d %d" % (G, ST, T))
    for _ in range(3000):
        items = [(int(rng.integers(1, 71)), int(rng.integers(1, 61))) for _ in range(int(rng.integers(1, 7)))]
        iters = sum(st * t for st, t in items)
        G = int(rng.integers(1, min(256, iters) + 1))
        lines.append("%d %s" % (G, " ".join("%d %d" % it for it in items)))
    r = subprocess.run([checker], input="split\n" + "\n".join(lines) + "\n", capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.startswith("ok split cases=%d" % len(lines)), r.stdout


def ksplan(checker, queries):
    """mnb::ks_single_plan for (M, K, N, scale_f32, has_zp, bs) queries:
    [(mb, ntw, est, workgroups)]."""
    lines = []
    for M, K, N, f32, zp, bs in queries:
        kpad = -(-K // bs) * bs
        lines.append("%d %d %d %d %d %d" % (M, -(-N // 16), -(-kpad // 128), f32, zp, 128 // bs))
    r = subprocess.run([checker], input="ksplan\n" + "\n".join(lines) + "\n", capture_output=True, text=True)
    assert r.returncode == 0, r.stdout
    out = [tuple(float(v) for v in line.split()) for line in r.stdout.strip().splitlines()]
    assert len(out) == len(queries)
    return [(int(a), int(b), c, int(d)) for a, b, c, d in out]


def test_k_sliced_blocks_are_the_fastest_measured(checker):
    """The K-sliced planner's block for single products, against the fastest
    of its four blocks measured on MI355X with each block forced (fp16
    scales, bs 32; the Phi-3 and Qwen2.5-0.5B projections at M = 32 to 512 and
    random shapes; times in us, same box): with 6 or more super-tiles the
    block comes from the fit with a per-round cost (the Qwen K = 896 rows,
    where the first model's 32 x 32 blocks measured 17-19% slower), with
    fewer (K = 512) from the first model."""
    cases = [  # (M, K, N) -> (mb, ntw)                       fastest measured block (us)
        ((256, 896, 1152), (2, 4)),     # 32x64 6.09; 32x32 7.44
        ((512, 896, 1152), (4, 4)),     # 64x64 8.46; 32x32 10.21
        ((512, 896, 896), (2, 4)),      # 32x64 6.08; 32x32 7.54
        ((32, 896, 9728), (2, 4)),      # 32x64 6.07; 32x32 7.41
        ((64, 896, 9728), (4, 4)),      # 64x64 8.44; 32x32 10.39
        ((32, 3072, 3072), (2, 1)),     # 32x16 6.26
        ((64, 3072, 3072), (2, 2)),     # 32x32 7.39
        ((128, 3072, 3072), (2, 4)),    # 32x64 9.75
        ((32, 3072, 9216), (2, 4)),     # 32x64 10.29
        ((64, 3072, 9216), (4, 4)),     # 64x64 14.68
        ((128, 8192, 3072), (2, 4)),    # 32x64 19.12
        ((137, 4096, 9850), (4, 4)),    # 64x64 34.56; 32x64 41.92
        ((78, 8192, 7050), (4, 4)),     # 64x64 27.86; 32x64 34.70
        ((231, 512, 1760), (2, 2)),     # 32x32 4.72; 32x64 5.12 (K = 512: the first model)
        ((80, 512, 6023), (2, 2)),      # 32x32 5.62; 64x64 7.49 (K = 512: the first model)
    ]
    got = ksplan(checker, [(M, K, N, 0, 0, 32) for (M, K, N), _ in cases])
    for ((M, K, N), want), (mb, ntw, _, wgs) in zip(cases, got):
        assert (mb, ntw) == want, (M, K, N, (mb, ntw), want)
        assert wgs == -(-N // (16 * ntw)) * -(-M // (16 * mb))


def test_k_sliced_plan_respects_supported_blocks(checker):
    """Over random shapes and every weight variant the planner returns a
    block the kernel is compiled for (no 64 x 64 block with bs 16 or with
    fp32 scales and zero points) and its workgroup count."""
    rng = np.random.default_rng(41)
    queries = []
    for _ in range(3000):
        queries.append((int(rng.integers(17, 2049)), int(rng.integers(8, 20000)), int(rng.integers(1, 200000)),
                        int(rng.integers(0, 2)), int(rng.integers(0, 2)), int(rng.choice([16, 32, 64, 128]))))
    for (M, K, N, f32, zp, bs), (mb, ntw, est, wgs) in zip(queries, ksplan(checker, queries)):
        assert mb in (2, 4) and est > 0
        if mb == 4:
            assert bs != 16 and not (f32 and zp), (M, K, N, f32, zp, bs)
