"""GPU parity: 2:4 prune/compress, gfx950 metadata pack, and the SMFMAC sparse GEMM.

Bar: compressed values, raw nibbles and packed words bit-exact (tests/test_prune_compress.cu,
tests/test_pack_metadata.cu); INT32 GEMM bit-exact; FP16 outputs bit-exact to the oracle's
epilogue for every tile x split the planner can run (tests/test_int8_sparse_gemm.cu:140-155),
with poisoned output and workspace; split-K bit-identical to unsplit (exact INT32
reduction); sparse_int8_linear paths bit-identical (:222-230)."""
import numpy as np
import pytest

from conftest import golden
from helpers import fp16_normal, int8_uniform, poison, say, to_dev, to_host

pytestmark = pytest.mark.gpu


def _prep(dev, W):
    import torch
    from forge_amd import ops
    N, K = W.shape
    comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
    raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
    meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
    ops.prune_compress_24(to_dev(W, dev), comp, raw, N, K)
    ops.pack_metadata(raw, meta, N, K)
    return comp, raw, meta


def test_prune_golden(dev):
    import torch
    from forge_amd import ops
    g = golden("prune")
    N, K = g["W"].shape
    say("prune golden")
    comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
    raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
    ops.prune_compress_24(to_dev(g["W"], dev), comp, raw, N, K)
    assert np.array_equal(to_host(comp), g["comp"]) and np.array_equal(to_host(raw), g["nibbles"])



def test_prune_every_tie_pattern(dev, orc):
    """Every group of 4 drawn from a tie-rich alphabet (magnitudes 0-3, 127 and 128 with both
    signs: 10^4 groups) through the vector and the exported per-group kernels, against the
    oracle's restatement of the reference's strict-< scan (prune_compress.cu:39-50)."""
    import itertools
    import torch
    from forge_amd import ops
    vals = [-128, -127, -3, -2, -1, 0, 1, 2, 3, 127]
    groups = np.array(list(itertools.product(vals, repeat=4)), dtype=np.int8)    # 10,000 x 4
    W = groups.reshape(625, 64)                                                   # K % 16 == 0
    comp_ref, nib_ref = orc.prune_compress_24(W)
    say("prune every tie pattern 625x64")
    N, K = W.shape
    comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
    raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
    ops.prune_compress_24(to_dev(W, dev), comp, raw, N, K)
    assert np.array_equal(to_host(comp), comp_ref) and np.array_equal(to_host(raw), nib_ref)
    W2 = groups                                                                   # K = 4: per-group kernel
    comp_ref2, nib_ref2 = orc.prune_compress_24(W2)
    comp2 = torch.empty((10000, 2), dtype=torch.int8, device=dev)
    raw2 = torch.empty((10000,), dtype=torch.uint8, device=dev)
    ops.prune_compress_24(to_dev(W2, dev), comp2, raw2, 10000, 4)
    assert np.array_equal(to_host(comp2), comp_ref2) and np.array_equal(to_host(raw2), nib_ref2)


@pytest.mark.parametrize("N,K", [(32, 128), (11008, 4096), (7, 20), (48, 1040)])
def test_prune_random(dev, orc, N, K):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(N + K)
    W = rng.integers(-128, 128, (N, K)).astype(np.int8)
    W[:, :8] = rng.integers(-2, 3, (N, 8))          # ties
    cr, mr = orc.prune_compress_24(W)
    say(f"prune N={N} K={K}")
    comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
    raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
    ops.prune_compress_24(to_dev(W, dev), comp, raw, N, K)
    assert np.array_equal(to_host(comp), cr) and np.array_equal(to_host(raw), mr)


@pytest.mark.parametrize("which", ["", "_ragged"])
def test_pack_golden_and_roundtrip(dev, which):
    import torch
    from forge_amd import ops
    g = golden("pack")
    raw = g["raw" + which]
    N, K = (16, 128) if not which else (20, 96)
    say(f"pack golden {which}")
    meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
    ops.pack_metadata(to_dev(raw, dev), meta, N, K)
    assert np.array_equal(to_host(meta).view(np.uint32), g["gfx950" + which])
    back = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
    ops.unpack_metadata(meta, back, N, K)
    assert np.array_equal(to_host(back), raw)


@pytest.mark.parametrize("N,K", [(37, 4096), (11008, 256), (5, 32)])
def test_pack_random_vs_oracle(dev, orc, N, K):
    """Random raw nibbles (one byte per group, values 0-15) packed into the gfx950 word order;
    (37, 4096): two whole 16-row blocks and a 5-row one; (5, 32): one partial block."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(N * 3 + K)
    raw = rng.integers(0, 16, N * K // 4).astype(np.uint8)
    say(f"pack random N={N} K={K}")
    meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
    poison(meta, 0x7B)
    ops.pack_metadata(to_dev(raw, dev), meta, N, K)
    assert np.array_equal(to_host(meta).view(np.uint32), orc.pack_metadata_gfx950(raw, N, K))


# tests/test_int8_sparse_gemm.cu:275-284
REF_SHAPES = [(1, 64, 16), (32, 128, 64), (37, 192, 208), (100, 640, 272), (300, 1280, 384),
              (1000, 1536, 512), (2050, 512, 400), (129, 4096, 96)]


@pytest.mark.parametrize("M,K,N", REF_SHAPES)
def test_sparse_int32_all_tiles(dev, orc, M, K, N):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M * 13 + K + N)
    W = int8_uniform(rng, (N, K))
    x = int8_uniform(rng, (M, K))
    cr, mr = orc.prune_compress_24(W)
    ref = orc.sparse_gemm_s32(cr, x, mr, N, K)
    comp, raw, meta = _prep(dev, W)
    xd = to_dev(x, dev)
    say(f"sparse s32 M={M} K={K} N={N}")
    C = to_host(ops.sparse_int8_gemm_s32(comp, xd, meta))
    assert np.array_equal(C, ref)


@pytest.mark.parametrize("M,K,N", REF_SHAPES)
def test_sparse_fp16_tiles_and_splits(dev, orc, M, K, N):
    """Every tile x split (1,2,3,4,6,7, ksteps+1), poisoned output and workspace."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M + K * 5 + N)
    W = int8_uniform(rng, (N, K))
    x = int8_uniform(rng, (M, K))
    act = rng.uniform(0.001, 0.05, M).astype(np.float32)
    ws = rng.uniform(0.001, 0.05, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16)
    cr, mr = orc.prune_compress_24(W)
    acc = orc.sparse_gemm_s32(cr, x, mr, N, K)
    ref_b = orc.dequant_epilogue(acc, act, ws, b).view(np.uint16)
    ref_nb = orc.dequant_epilogue(acc, act, ws, None).view(np.uint16)
    comp, raw, meta = _prep(dev, W)
    xd, actd, wsd, bd = to_dev(x, dev), to_dev(act, dev), to_dev(ws, dev), to_dev(b, dev)
    out = torch.empty((M, N), dtype=torch.float16, device=dev)
    wsp = torch.empty((M, N), dtype=torch.float32, device=dev)
    ksteps = K // 64
    for tile in range(3):
        for split in (1, 2, 3, 4, 6, 7, ksteps + 1):
            use_bias = split % 2 == 1
            poison(out, 0x7B)
            poison(wsp, 0x5A)
            say(f"sparse fp16 M={M} K={K} N={N} tile={tile} split={split}")
            ops.sparse_int8_gemm(comp, xd, meta, actd, wsd, bd if use_bias else None, splitk_workspace=wsp,
                                 split_k=split, tile=tile, out=out)
            got = to_host(out).view(np.uint16)
            assert np.array_equal(got, ref_b if use_bias else ref_nb), (tile, split)
    for split, use_ws in [(0, True), (0, False), (1, False), (4, False)]:
        poison(out, 0x7B)
        say(f"sparse fp16 auto split={split} ws={use_ws}")
        ops.sparse_int8_gemm(comp, xd, meta, actd, wsd, bd, splitk_workspace=wsp if use_ws else None,
                             split_k=split, out=out)
        assert np.array_equal(to_host(out).view(np.uint16), ref_b)


@pytest.mark.parametrize("M,K,N", [(37, 64, 16), (5000, 1024, 336), (70, 1280, 320), (16, 8192, 1024)])
def test_sparse_linear_paths(dev, orc, M, K, N):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M + K + N)
    W = int8_uniform(rng, (N, K))
    x = rng.uniform(-2.0, 2.0, (M, K)).astype(np.float16)
    ws = rng.uniform(0.001, 0.05, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16)
    cr, mr = orc.prune_compress_24(W)
    qr, sr = orc.quantize_rows(x)
    ref = orc.dequant_epilogue(orc.sparse_gemm_s32(cr, qr, mr, N, K), sr, ws, b).view(np.uint16)
    comp, raw, meta = _prep(dev, W)
    xd, wsd, bd = to_dev(x, dev), to_dev(ws, dev), to_dev(b, dev)
    sq = torch.empty((M, K), dtype=torch.int8, device=dev)
    ss = torch.empty((M,), dtype=torch.float32, device=dev)
    outs = []
    for path, split in [(0, 1), (1, 1), (-1, 0), (-1, 3)]:
        say(f"sparse linear M={M} K={K} N={N} path={path} split={split}")
        outs.append(to_host(ops.sparse_int8_linear(xd, comp, meta, wsd, bd, sq, ss, None, split, path)).view(np.uint16))
    for o in outs:
        assert np.array_equal(o, ref)


def test_config3_full_size(dev, orc):
    """W (11008, 4096) pruned 2:4, A (4096, 4096); every INT32 output bit-exact
    against the oracle (threaded loop over the decompressed weights)."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(3)
    N, K, M = 11008, 4096, 4096
    W = int8_uniform(rng, (N, K))
    x = int8_uniform(rng, (M, K))
    cr, mr = orc.prune_compress_24(W)
    ref = orc.sparse_gemm_s32(cr, x, mr, N, K, threads=orc.cpu_threads())
    comp, raw, meta = _prep(dev, W)
    assert np.array_equal(to_host(comp), cr) and np.array_equal(to_host(raw), mr)
    say("config3 sparse 4096x11008x4096")
    out = torch.empty((M, N), dtype=torch.int32, device=dev)
    poison(out, 0x7B)
    C = to_host(ops.sparse_int8_gemm_s32(comp, to_dev(x, dev), meta, out=out))
    assert ops.last_route() == "wide256 tile2"
    bad = int((C != ref).sum())
    assert bad == 0, f"{bad} of {C.size} outputs differ"


# Plans on each unsplit DMA engine, chosen by the engine model (tile -1) or forced to the
# reference's 256 x 128 tile (0): the 64 x 64 ring engine (narrow N or few token tiles with deep
# K; partial last token tile), the 128 x 128 engine (one and several rounds of tiles per CU,
# partial last weight and token tiles), the 256 x 128 engine and the 256 x 256 one. The INT32
# call always plans itself.
ENGINE_SHAPES = [
    (200, 2048, 256, -1, "ring64x64"),     # 4 token tiles (last 8 rows), 4 weight tiles
    (1024, 6144, 1536, -1, "ring64x64"),   # the reference benchmark's narrow deep-K layer
    (100, 256, 144, -1, "dma128x128"),     # 2 stages, last weight tile 16 of 128 rows, M < 128
    (1024, 1536, 6144, -1, "dma128x128"),
    (40000, 640, 320, -1, "dma128x128"),   # 4 tiles on the busiest CU, ragged token and weight tiles
    (512, 128, 2048, 0, "dma256x128"),     # one stage
    (4000, 4096, 4096, -1, "dma256x256"),  # ragged token tile
]


@pytest.mark.parametrize("M,K,N,tile,engine", ENGINE_SHAPES)
def test_sparse_auto_engines(dev, orc, M, K, N, tile, engine):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M + 3 * K + 7 * N)
    W = int8_uniform(rng, (N, K))
    x = int8_uniform(rng, (M, K))
    act = rng.uniform(0.001, 0.05, M).astype(np.float32)
    ws = rng.uniform(0.001, 0.05, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16)
    rows = np.unique(np.r_[0:17, M // 2, M - 70:M])
    rows = rows[rows < M]
    cr, mr = orc.prune_compress_24(W)
    acc = orc.sparse_gemm_s32(cr, x[rows], mr, N, K)
    comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
    raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
    meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
    ops.prune_compress_24(to_dev(W, dev), comp, raw, N, K)
    ops.pack_metadata(raw, meta, N, K)
    say(f"sparse auto engine M={M} K={K} N={N}")
    xd = to_dev(x, dev)
    C = torch.empty((M, N), dtype=torch.int32, device=dev)
    poison(C, 0x7B)
    assert np.array_equal(to_host(ops.sparse_int8_gemm_s32(comp, xd, meta, out=C))[rows], acc)
    Y = torch.empty((M, N), dtype=torch.float16, device=dev)
    poison(Y, 0x7B)
    ops.sparse_int8_gemm(comp, xd, meta, to_dev(act, dev), to_dev(ws, dev), to_dev(b, dev), split_k=0, tile=tile,
                         out=Y)
    assert ops.last_route() == engine
    ref = orc.dequant_epilogue(acc, act[rows], ws, b).view(np.uint16)
    assert np.array_equal(to_host(Y)[rows].view(np.uint16), ref)


# The tail split of the 256 x 256 engines: whole waves of 256 x 256 tiles over the first weight
# blocks, then the remaining weight blocks as one wave of 192-token tiles (one launch). (1000,
# 4096, 17904): 280 tiles = 256 + 6 weight blocks x 6 token tiles of 192 (the last 40 rows, the
# last weight block 240 rows); (512, 4096, 35008): 128 blocks x 2 + 9 x 3. INT32 (256-deep weight
# stages) and FP16 (128-deep) outputs, every one against the oracle. With K % 512 == 0 the INT32
# output takes the wide-tile engine instead (its per-CU plan applies at both shapes); K = 3840
# keeps the 256 x 256 tail split for INT32 too.
@pytest.mark.parametrize("M,K,N,route32", [(1000, 4096, 17904, "wide256 tile1"), (512, 4096, 35008, "wide256 tile1"),
                                           (1000, 3840, 17904, "dma256x256+tail192")])
def test_sparse_256x256_tail_split(dev, orc, M, K, N, route32):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M + K + N + 1)
    W = int8_uniform(rng, (N, K))
    x = int8_uniform(rng, (M, K))
    act = rng.uniform(0.001, 0.05, M).astype(np.float32)
    ws = rng.uniform(0.001, 0.05, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16)
    cr, mr = orc.prune_compress_24(W)
    ref = orc.sparse_gemm_s32(cr, x, mr, N, K, threads=orc.cpu_threads())
    comp, raw, meta = _prep(dev, W)
    say(f"sparse 256x256 tail split M={M} K={K} N={N}")
    xd = to_dev(x, dev)
    C = torch.empty((M, N), dtype=torch.int32, device=dev)
    poison(C, 0x7B)
    got = to_host(ops.sparse_int8_gemm_s32(comp, xd, meta, out=C))
    assert ops.last_route() == route32
    bad = int((got != ref).sum())
    assert bad == 0, f"INT32: {bad} of {got.size} outputs differ"
    Y = torch.empty((M, N), dtype=torch.float16, device=dev)
    poison(Y, 0x7B)
    ops.sparse_int8_gemm(comp, xd, meta, to_dev(act, dev), to_dev(ws, dev), to_dev(b, dev), split_k=0, out=Y)
    assert ops.last_route() == "dma256x256+tail192"
    refy = orc.dequant_epilogue(ref, act, ws, b).view(np.uint16)
    bad = int((to_host(Y).view(np.uint16) != refy).sum())
    assert bad == 0, f"FP16: {bad} of {Y.numel()} outputs differ"
    poison(Y, 0x5A)
    ops.sparse_int8_gemm(comp, xd, meta, to_dev(act, dev), to_dev(ws, dev), None, split_k=0, out=Y)
    assert ops.last_route() == "dma256x256+tail192"
    refy = orc.dequant_epilogue(ref, act, ws, None).view(np.uint16)
    bad = int((to_host(Y).view(np.uint16) != refy).sum())
    assert bad == 0, f"FP16 without bias: {bad} of {Y.numel()} outputs differ"


# The 256 x 256 SMFMAC engine with 256-deep weight stages (INT32 out, K % 256 == 0): one and
# three weight double-stages, ragged token and weight tiles; every output against the oracle.
# The grid is large enough that the engine choice takes 256 x 256 tiles (checked by route).
@pytest.mark.parametrize("M,K,N", [(4040, 256, 8112), (4096, 768, 8192), (3000, 512, 8208)])
def test_sparse_256x256_int32_whole(dev, orc, M, K, N):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M + K + N)
    W = int8_uniform(rng, (N, K))
    x = int8_uniform(rng, (M, K))
    cr, mr = orc.prune_compress_24(W)
    ref = orc.sparse_gemm_s32(cr, x, mr, N, K, threads=orc.cpu_threads())
    comp, raw, meta = _prep(dev, W)
    say(f"sparse 256x256 INT32 M={M} K={K} N={N}")
    C = torch.empty((M, N), dtype=torch.int32, device=dev)
    poison(C, 0x7B)
    got = to_host(ops.sparse_int8_gemm_s32(comp, to_dev(x, dev), meta, out=C))
    assert ops.last_route() == "dma256x256"
    bad = int((got != ref).sum())
    assert bad == 0, f"{bad} of {got.size} outputs differ"
