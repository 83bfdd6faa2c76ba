"""GPU: the hot-path entry points captured into HIP graphs.

The reference's benchmark captures sparse_int8_gemm into a CUDA graph (bench_int8_sparse.cu:60-63),
so every launcher must be capturable: no synchronisation, allocation, attribute or device query
inside the capture, and no memset nodes (the split-K workspace is cleared by a kernel). Each graph
is replayed several times with eager work and synchronisations between the replays, and every
replay is compared bit-for-bit with the eager result of the same calls."""
import os

import numpy as np
import pytest

from helpers import fp16_normal, int8_uniform, say, to_dev

pytestmark = pytest.mark.gpu


def _replay_check(dev, calls, outputs, replays=4):
    """Eager results of `calls`, then a captured graph of the same calls replayed `replays`
    times; every output tensor must match the eager bits after each replay."""
    import torch
    for c in calls:
        c()
    torch.cuda.synchronize()
    want = [o.clone() for o in outputs]
    for o in outputs:
        o.view(torch.uint8).fill_(0x7B)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for c in calls:          # warm-up on the capture stream (first-call attributes etc.)
            c()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for c in calls:
            c()
    scratch = torch.empty((1 << 20,), dtype=torch.int32, device=dev)
    for r in range(replays):
        for o in outputs:
            o.view(torch.uint8).fill_(0x5A)
        scratch.fill_(r)                           # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for o, w in zip(outputs, want):
            assert torch.equal(o.view(torch.uint8), w.view(torch.uint8)), f"replay {r} differs"


def test_graph_int8_linear(dev):
    """configs[1]-style fused linear (quantize + dequantizing GEMM), plus decode shapes; (16, 4096,
    1024) and (40, 8192, 512) split K across workgroups (on the capture's own sum slot)."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(21)
    for (M, K, N) in [(512, 1024, 768), (16, 4096, 1024), (3, 1152, 96), (40, 8192, 512)]:
        say(f"graph int8_linear M={M} K={K} N={N}")
        x = to_dev(fp16_normal(rng, (M, K)), dev)
        w = to_dev(int8_uniform(rng, (N, K)), dev)
        ws = to_dev(rng.uniform(1e-3, 1e-2, N).astype(np.float16), dev)
        b = to_dev(fp16_normal(rng, (N,), 0.1), dev)
        q = torch.empty((M, K), dtype=torch.int8, device=dev)
        s = torch.empty((M,), dtype=torch.float32, device=dev)
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        c32 = torch.empty((M, N), dtype=torch.int32, device=dev)
        calls = [lambda: ops.int8_linear(x, w, ws, b, q, s, out=y),
                 lambda: ops.int8_gemm_s32(q, w, out=c32)]
        _replay_check(dev, calls, [q, s, y, c32])


def test_graph_ksplit_slot_keys(dev):
    """Decode K split inside graphs: a capture records split launches on a slot of its own,
    distinct from the eager slot of the capture stream and from another capture's slot; replays
    interleaved with eager split work on the capture stream (its own slot) all give the eager
    bits; forge_ksplit_reset leaves the slots usable."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(26)
    M, K, N = 16, 4096, 1024
    x = to_dev(fp16_normal(rng, (M, K)), dev)
    w = to_dev(int8_uniform(rng, (N, K)), dev)
    x2 = to_dev(fp16_normal(rng, (M, K)), dev)
    w2 = to_dev(int8_uniform(rng, (N, K)), dev)
    ws = to_dev(rng.uniform(1e-3, 1e-2, N).astype(np.float16), dev)
    b = to_dev(fp16_normal(rng, (N,), 0.1), dev)
    q, q2 = (torch.empty((M, K), dtype=torch.int8, device=dev) for _ in range(2))
    s, s2 = (torch.empty((M,), dtype=torch.float32, device=dev) for _ in range(2))
    y, y2, y3 = (torch.empty((M, N), dtype=torch.float16, device=dev) for _ in range(3))
    say("graph ksplit slots: eager")
    ops.int8_linear(x, w, ws, b, q, s, out=y)
    slot_e, kp_e = ops.ksplit_last()
    assert slot_e >= 0 and kp_e > 1, (slot_e, kp_e)
    ops.int8_linear(x2, w2, ws, b, q2, s2, out=y2)
    torch.cuda.synchronize()
    ref, ref2 = y.clone(), y2.clone()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        ops.int8_linear(x2, w2, ws, b, q2, s2, out=y2)
        slot_ce, _ = ops.ksplit_last()
    torch.cuda.current_stream().wait_stream(cap)
    torch.cuda.synchronize()
    assert slot_ce >= 0 and slot_ce != slot_e
    say("graph ksplit slots: capture")
    g1, g2 = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1, stream=cap):
        ops.int8_linear(x, w, ws, b, q, s, out=y)
        slot_g1, kp_g1 = ops.ksplit_last()
    with torch.cuda.graph(g2, stream=cap):
        ops.int8_linear(x, w, ws, b, q, s, out=y3)
        slot_g2, kp_g2 = ops.ksplit_last()
    assert kp_g1 > 1 and kp_g2 > 1, (kp_g1, kp_g2)
    assert len({slot_e, slot_ce, slot_g1, slot_g2}) == 4 and min(slot_g1, slot_g2) >= 0
    for r in range(4):
        if r == 2:
            ops.ksplit_reset()
        y.view(torch.uint8).fill_(0x5A)
        y2.view(torch.uint8).fill_(0x5A)
        y3.view(torch.uint8).fill_(0x5A)
        torch.cuda.synchronize()
        say(f"graph ksplit slots: replay {r}")
        g1.replay()
        cap.wait_stream(torch.cuda.current_stream()) if r == 3 else None
        with torch.cuda.stream(cap):
            for _ in range(3):
                ops.int8_linear(x2, w2, ws, b, q2, s2, out=y2)
        g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.uint8), ref.view(torch.uint8)), f"replay {r}: graph 1 differs"
        assert torch.equal(y3.view(torch.uint8), ref.view(torch.uint8)), f"replay {r}: graph 2 differs"
        assert torch.equal(y2.view(torch.uint8), ref2.view(torch.uint8)), f"replay {r}: eager work differs"


def test_graph_sparse_splitk(dev):
    """2:4 sparse GEMM with split-K (workspace cleared by a kernel, integer atomics, finalize),
    the unsplit path and the decode shape."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(22)
    for (M, K, N, split) in [(256, 2048, 512, 4), (256, 2048, 512, 1), (8, 2048, 256, 1)]:
        say(f"graph sparse M={M} K={K} N={N} split={split}")
        W = to_dev(int8_uniform(rng, (N, K)), dev)
        comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
        raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
        meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
        ops.prune_compress_24(W, comp, raw, N, K)
        ops.pack_metadata(raw, meta, N, K)
        x = to_dev(int8_uniform(rng, (M, K)), dev)
        act = to_dev(rng.uniform(1e-3, 5e-2, M).astype(np.float32), dev)
        ws = to_dev(rng.uniform(1e-3, 1e-2, N).astype(np.float16), dev)
        b = to_dev(fp16_normal(rng, (N,), 0.1), dev)
        wsp = torch.empty((M * N,), dtype=torch.float32, device=dev)
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        calls = [lambda: ops.sparse_int8_gemm(comp, x, meta, act, ws, b, splitk_workspace=wsp, split_k=split,
                                              out=y)]
        _replay_check(dev, calls, [y])


def test_graph_tail_splits(dev):
    """The one-launch tail splits of the 256 x 256 engines (whole tile waves, then one wave of
    192-row tiles): dense over weight columns (512 x 1024 x 35000: 128 x 2 + 9 x 3 tiles) and
    2:4 sparse (512 x 4096 x 35008), INT32 and FP16 out."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(31)
    M, K, N = 512, 1024, 35000
    say(f"graph dense column tail M={M} K={K} N={N}")
    A = to_dev(int8_uniform(rng, (M, K)), dev)
    B = to_dev(int8_uniform(rng, (N, K)), dev)
    act = to_dev(rng.uniform(1e-3, 5e-2, M).astype(np.float32), dev)
    ws = to_dev(rng.uniform(1e-3, 1e-2, N).astype(np.float16), dev)
    b = to_dev(fp16_normal(rng, (N,), 0.1), dev)
    c = torch.empty((M, N), dtype=torch.int32, device=dev)
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    calls = [lambda: ops.int8_gemm_s32(A, B, out=c), lambda: ops.int8_gemm_dequant(A, B, act, ws, b, out=y)]
    _replay_check(dev, calls, [c, y])
    assert ops.last_route() == "dma256x256+tail192"
    M, K, N = 512, 4096, 35008
    say(f"graph sparse tail M={M} K={K} N={N}")
    W = to_dev(int8_uniform(rng, (N, K)), dev)
    comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
    raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
    meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
    ops.prune_compress_24(W, comp, raw, N, K)
    ops.pack_metadata(raw, meta, N, K)
    x = to_dev(int8_uniform(rng, (M, K)), dev)
    act = to_dev(rng.uniform(1e-3, 5e-2, M).astype(np.float32), dev)
    ws = to_dev(rng.uniform(1e-3, 1e-2, N).astype(np.float16), dev)
    b = to_dev(fp16_normal(rng, (N,), 0.1), dev)
    c = torch.empty((M, N), dtype=torch.int32, device=dev)
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    calls = [lambda: ops.sparse_int8_gemm_s32(comp, x, meta, out=c),
             lambda: ops.sparse_int8_gemm(comp, x, meta, act, ws, b, split_k=0, out=y)]
    _replay_check(dev, calls, [c, y])
    assert ops.last_route() == "dma256x256+tail192"


def test_graph_sparse_fq(dev):
    """The fused quantize + sparse linear with its weight-packing launch: the capture packs into
    a slot of its own (distinct from the eager slot of the capture stream)."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(29)
    M, K, N = 200, 1280, 320
    say(f"graph fused sparse linear M={M} K={K} N={N}")
    W = to_dev(int8_uniform(rng, (N, K)), dev)
    comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
    raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
    meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
    ops.prune_compress_24(W, comp, raw, N, K)
    ops.pack_metadata(raw, meta, N, K)
    x = to_dev(fp16_normal(rng, (M, K)), dev)
    ws = to_dev(rng.uniform(1e-3, 1e-2, N).astype(np.float16), dev)
    b = to_dev(fp16_normal(rng, (N,), 0.1), dev)
    q = torch.empty((M, K), dtype=torch.int8, device=dev)
    s = torch.empty((M,), dtype=torch.float32, device=dev)
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    calls = [lambda: ops.sparse_int8_linear(x, comp, meta, ws, b, q, s, None, 1, 1, out=y)]
    _replay_check(dev, calls, [y])
    assert ops.last_route() == "fused-quantize packed"


def test_graph_conv(dev):
    """NHWC conv on the DMA gather (C % 128 == 0) and on the register engine (C = 48)."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(23)
    for (N, H, W, C, Co) in [(2, 64, 64, 128, 256), (2, 9, 11, 48, 40)]:
        say(f"graph conv N={N} H={H} W={W} C={C} Co={Co}")
        x = to_dev(int8_uniform(rng, (N, H, W, C)), dev)
        w = to_dev(int8_uniform(rng, (Co, 3, 3, C)), dev)
        out = torch.empty((N, H, W, Co), dtype=torch.int32, device=dev)
        calls = [lambda: ops.int8_conv2d_nhwc_s32(x, w, (1, 1), out=out)]
        _replay_check(dev, calls, [out])


def test_graph_conv_special(dev):
    """Depthwise conv (tile and direct kernels) and the k2s2 transposed conv (pixel quantizer
    + scatter GEMM, two images per chunk)."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(24)
    x = to_dev(rng.uniform(-1, 1, (2, 8, 33, 40)).astype(np.float16), dev)
    w = to_dev(int8_uniform(rng, (8, 9)), dev)
    ws = to_dev(rng.uniform(0.005, 0.05, 8).astype(np.float16), dev)
    b = to_dev(rng.uniform(-0.5, 0.5, 8).astype(np.float16), dev)
    y1 = torch.empty((2, 8, 33, 40), dtype=torch.float16, device=dev)
    y2 = torch.empty((2, 8, 17, 20), dtype=torch.float16, device=dev)
    wt = to_dev(int8_uniform(rng, (4 * 12, 8)), dev)
    wts = to_dev(rng.uniform(0.005, 0.05, 12).astype(np.float16), dev)
    bt = to_dev(rng.uniform(-0.5, 0.5, 12).astype(np.float16), dev)
    nbytes = ops.int8_conv_transpose2d_k2s2_workspace_size(8, 33, 40, 12)
    wsp = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
    y3 = torch.empty((2, 12, 66, 80), dtype=torch.float16, device=dev)
    say("graph depthwise + conv_transpose")
    calls = [lambda: ops.int8_depthwise_conv2d_forward(x, w, ws, b, 3, 3, (1, 1), out=y1),
             lambda: ops.int8_depthwise_conv2d_forward(x, w, ws, b, 3, 3, (1, 1), (2, 2), out=y2),
             lambda: ops.int8_conv_transpose2d_k2s2_forward(x, wt, wts, bt, workspace=wsp, out=y3)]
    _replay_check(dev, calls, [y1, y2, y3])


def test_graph_weight_prep(dev):
    """The one-pass sparse weight preparation and the dense weight quantizer."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(25)
    w = to_dev((rng.standard_normal((96, 512)) * 0.05).astype(np.float32), dev)
    comp = torch.empty((96, 256), dtype=torch.int8, device=dev)
    meta = torch.empty((96, 16), dtype=torch.int32, device=dev)
    sc = torch.empty((96,), dtype=torch.float16, device=dev)
    q = torch.empty((96, 512), dtype=torch.int8, device=dev)
    qs = torch.empty((96,), dtype=torch.float16, device=dev)

    def prep():
        c, m, s = ops.prepare_sparse_weight(w)
        comp.copy_(c)
        meta.copy_(m)
        sc.copy_(s)

    say("graph weight prep")
    calls = [prep, lambda: ops.quantize_weight_rows(w, q, qs)]
    _replay_check(dev, calls, [comp, meta, sc, q, qs])


def _fresh_process(mode):
    """Runs tests/fresh_process_checks.py MODE in a child process (it needs the library's
    per-process slot and no-alloc state untouched) and returns its JSON line."""
    import json
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    say(f"fresh process check: {mode}")
    r = subprocess.run([sys.executable, os.path.join(here, "fresh_process_checks.py"), mode], capture_output=True,
                       text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-3000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


def test_graph_slot_exhaustion():
    """The K-split slots are held for good by the first 32 launch keys (streams for eager
    launches, captures for graph launches). In a fresh process the eager stream takes one, 31
    captures of a K-split decode record split launches on 31 more distinct slots, and the next
    capture -- the 33rd key -- records the unsplit decode (no slot); forge_slots_in_use then
    reports all 32 held. Every replay is bit-identical to eager."""
    r = _fresh_process("slots")
    assert r["eager"][0] >= 0 and r["eager"][1] == 8, r["eager"]
    total, rec = r["total"], r["recorded"]
    assert total == 32 and len(rec) == total - r["used0"] + 1
    split = rec[:-1]
    assert all(s >= 0 and p == 8 for s, p in split), split
    assert len({s for s, _ in split}) == len(split)
    assert rec[-1] == [-1, 1], rec[-1]
    assert r["after"][0] == total and r["after"][1] == total
    assert all(r["equal"])
