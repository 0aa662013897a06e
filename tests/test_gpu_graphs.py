"""Resident activations and graph capture (the record-into semantics of
MatMulNBitsKernel.recordResidentInto / recordIntoGpuResident,
directml-windows-bindings/.../windows/MatMulNBitsKernel.java:1687-1832,
and the batched recording of WarpExecutionContext.java:131-160).

Products on device pointers allocate nothing and record only kernel launches,
so a sequence of them -- single-row products, a prefill product whose tiles
are split over workgroups (GEMM plus its reduce kernel), a prefill product
on the K-sliced kernel, and group launches (M = 1, and a 3-row group on the
streaming kernel) -- is captured into a HIP graph on
a fresh context, with no eager call first.
Each replay, with new activations written by eager work between replays,
equals the eager calls bit for bit."""
import numpy as np
import pytest

import mnb_hip
from mnb_hip import synth

pytestmark = pytest.mark.gpu


def _weight(ctx, seed, N, K, bs=32, zp=False):
    t = synth.make_weight(seed, N, K, bs, with_zp=zp)
    if zp:
        return mnb_hip.Weight(ctx, N, K, bs, t.q, t.scales_f16, t.zp_row_padded, mnb_hip.MNB_ZP_ROW_PADDED)
    return mnb_hip.Weight(ctx, N, K, bs, t.q, t.scales_f16)


def test_graph_capture_replays_match_eager():
    import torch
    ctx = mnb_hip.Context(0)
    try:
        dev = "cuda"
        w_o = _weight(ctx, 1, 3072, 3072)                  # decode o_proj
        w_gu = _weight(ctx, 2, 16384, 3072)                # decode gate_up
        w_pf = _weight(ctx, 3, 9001, 8192, zp=True)        # prefill product with split tiles
        w_ks = _weight(ctx, 4, 1000, 3072, zp=True)        # prefill product on the K-sliced kernel
        w_k16 = _weight(ctx, 5, 16384, 3072)               # M = 12 product on 16 x 64 K-sliced blocks
        assert w_pf.plan(200).as_tuple() == (mnb_hip.MNB_KERNEL_GEMM, mnb_hip.MNB_ORDER_STREAM_K, 128, 256)
        assert w_ks.plan(200).kernel == mnb_hip.MNB_KERNEL_KSLICE
        assert w_k16.plan(12).as_tuple() == (mnb_hip.MNB_KERNEL_KSLICE, mnb_hip.MNB_ORDER_NONE, 16, 64)
        w_g = [_weight(ctx, 10 + i, 1536, 576, 64, zp=True) for i in range(3)]
        gen = torch.Generator(device=dev).manual_seed(7)
        x1 = torch.empty(3072, device=dev, dtype=torch.float16)
        xp = torch.empty(200, 8192, device=dev, dtype=torch.float16)
        xk = torch.empty(200, 3072, device=dev, dtype=torch.float16)
        x12 = torch.empty(12, 3072, device=dev, dtype=torch.float16)
        xg = [torch.empty(576, device=dev, dtype=torch.float16) for _ in w_g]
        xg3 = [torch.empty(3, 576, device=dev, dtype=torch.float16) for _ in w_g]   # small-batch group, 3 rows
        y_o = torch.empty(3072, device=dev, dtype=torch.float16)
        y_gu = torch.empty(16384, device=dev, dtype=torch.float32)
        y_pf = torch.empty(200, 9001, device=dev, dtype=torch.float16)
        y_ks = torch.empty(200, 1000, device=dev, dtype=torch.float32)
        y_k16 = torch.empty(12, 16384, device=dev, dtype=torch.float16)
        y_g = [torch.empty(1536, device=dev, dtype=torch.float16) for _ in w_g]
        y_g3 = [torch.empty(3, 1536, device=dev, dtype=torch.float32) for _ in w_g]
        st = torch.cuda.Stream()

        def fill():
            x1.copy_(torch.randn(3072, device=dev, generator=gen).half())
            xp.copy_(torch.randn(200, 8192, device=dev, generator=gen).half())
            xk.copy_(torch.randn(200, 3072, device=dev, generator=gen).half())
            x12.copy_(torch.randn(12, 3072, device=dev, generator=gen).half())
            for x in xg:
                x.copy_(torch.randn(576, device=dev, generator=gen).half())
            for x in xg3:
                x.copy_(torch.randn(3, 576, device=dev, generator=gen).half())

        with torch.cuda.stream(st):
            fill()
        torch.cuda.synchronize()
        group = mnb_hip.Group(ctx, list(zip(w_g, xg, y_g)))
        group3 = mnb_hip.Group(ctx, list(zip(w_g, xg3, y_g3)))
        assert group3.plan().as_tuple() == (mnb_hip.MNB_KERNEL_STREAM, mnb_hip.MNB_ORDER_NONE, 3, 16)

        def record():
            w_o.matmul(x1, y_o, stream=st.cuda_stream)
            w_gu.matmul(x1, y_gu, stream=st.cuda_stream)
            w_pf.matmul(xp, y_pf, stream=st.cuda_stream)
            w_ks.matmul(xk, y_ks, stream=st.cuda_stream)
            w_k16.matmul(x12, y_k16, stream=st.cuda_stream)
            group.run(st.cuda_stream)
            group3.run(st.cuda_stream)

        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=st):
            record()
        torch.cuda.synchronize()

        outs = [y_o, y_gu, y_pf, y_ks, y_k16] + y_g + y_g3
        for rep in range(4):
            with torch.cuda.stream(st):
                fill()
                for y in outs:
                    y.fill_(float("nan"))
                graph.replay()
            torch.cuda.synchronize()
            got = [y.clone() for y in outs]
            with torch.cuda.stream(st):
                for y in outs:
                    y.fill_(float("nan"))
                record()
            torch.cuda.synchronize()
            for i, (a, b) in enumerate(zip(got, outs)):
                assert torch.isfinite(a).all(), (rep, i)
                assert torch.equal(a.view(torch.int16) if a.dtype == torch.float16 else a.view(torch.int32),
                                   b.view(torch.int16) if b.dtype == torch.float16 else b.view(torch.int32)), (rep, i)
        group.close()
        group3.close()
        for w in [w_o, w_gu, w_pf, w_ks, w_k16] + w_g:
            w.close()
        del graph
    finally:
        torch.cuda.synchronize()
        ctx.close()


def test_graph_capture_of_tile_list_groups():
    """Group launches in tile-list order (a prefill group with 512-column
    tiles, a 32 < M <= 64 group on 64-row tiles and a 1 < M <= 16 group on
    32-row tiles) captured into one HIP graph; every replay, with new
    activations written between replays, equals the eager launches bit for
    bit."""
    import torch
    ctx = mnb_hip.Context(0)
    try:
        dev = "cuda"
        gen = torch.Generator(device=dev).manual_seed(11)
        groups, xs, ys, ws = [], [], [], []
        # 1344 tiles of 128 x 512, 316 of 64 x 512 (K = 896: 7 stages each, fewer
        # than 4 per workgroup) and 1075 of 32 x 512: all run in tile-list order
        for gi, (M, shapes) in enumerate([(512, [(3072, 16384), (3072, 9216), (8192, 3072)] * 6),
                                           (48, [(896, 151936), (896, 9728)]),
                                           (8, [(256, 200000), (512, 200000), (128, 150000)])]):
            items = []
            for i, (K, N) in enumerate(shapes):
                w = _weight(ctx, 100 * gi + i, N, K)
                x = torch.empty(M, K, device=dev, dtype=torch.float16)
                y = torch.empty(M, N, device=dev, dtype=torch.float16)
                ws.append(w)
                xs.append(x)
                ys.append(y)
                items.append((w, x, y))
            groups.append(mnb_hip.Group(ctx, items))
        st = torch.cuda.Stream()

        def fill():
            for x in xs:
                x.copy_(torch.randn(x.shape, device=dev, generator=gen).half())

        def record():
            for g in groups:
                g.run(st.cuda_stream)

        with torch.cuda.stream(st):
            fill()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=st):
            record()
        torch.cuda.synchronize()
        for rep in range(3):
            with torch.cuda.stream(st):
                fill()
                for y in ys:
                    y.fill_(float("nan"))
                graph.replay()
            torch.cuda.synchronize()
            got = [y.clone() for y in ys]
            with torch.cuda.stream(st):
                for y in ys:
                    y.fill_(float("nan"))
                record()
            torch.cuda.synchronize()
            for i, (a, b) in enumerate(zip(got, ys)):
                assert torch.isfinite(a).all(), (rep, i)
                assert torch.equal(a.view(torch.int16), b.view(torch.int16)), (rep, i)
        for g in groups:
            g.close()
        for w in ws:
            w.close()
        del graph
    finally:
        torch.cuda.synchronize()
        ctx.close()
