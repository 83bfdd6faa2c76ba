"""GPU parity: decode-shape GEMMs (M <= 16 tokens) on the weight-streaming decode kernel,
dense and 2:4 sparse, against the oracle; and 16 < M <= 64 on the same kernels with several
16-token blocks per weight fragment.

Bar: INT32 bit-exact; FP16 bit-exact to the oracle's epilogue. Shapes exercise the kernel's
K split over 8 wavefronts (K = 128: one wave works; K = 1152: 9 stages, uneven slices and
idle waves), ragged N (not a multiple of the 32-row workgroup tile), M from 1 to 16 (the
sparse register kernel with K % 256 == 0, the DMA-ring kernel otherwise), and
configs[3] at full size (M = 16, 4 and 1, N = K = 8192; every output column); narrow N with K
split across workgroups (exact INT32 hand-off), repeated and on two streams at once."""
import numpy as np
import pytest

from helpers import fp16_normal, int8_uniform, poison, say, to_dev, to_host

pytestmark = pytest.mark.gpu

DENSE = [(1, 128, 32), (3, 1152, 96), (16, 2048, 50), (7, 4096, 200), (16, 1024, 8)]
# K % 256 == 0 runs the register kernel; K % 256 == 128 the DMA-ring kernel.
SPARSE = [(1, 128, 32), (5, 1152, 48), (16, 2048, 208), (9, 4096, 1024), (16, 1024, 16),
          (1, 256, 32), (5, 1280, 48), (8, 2048, 208), (3, 768, 16), (4, 8192, 1024),
          (12, 1152, 48), (16, 640, 64), (13, 256, 80), (3, 1024, 48), (15, 3072, 96), (2, 2048, 64)]


@pytest.mark.parametrize("M,K,N", DENSE)
def test_decode_dense(dev, orc, M, K, N):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M * 31 + K + N)
    A = int8_uniform(rng, (M, K))
    B = int8_uniform(rng, (N, K))
    act = rng.uniform(0.001, 0.05, M).astype(np.float32)
    ws = rng.uniform(0.001, 0.05, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16)
    acc = orc.gemm_s32(A, B)
    say(f"decode dense M={M} K={K} N={N}")
    C = torch.empty((M, N), dtype=torch.int32, device=dev)
    poison(C, 0x7B)
    assert np.array_equal(to_host(ops.int8_gemm_s32(to_dev(A, dev), to_dev(B, dev), out=C)), acc)
    Y = torch.empty((M, N), dtype=torch.float16, device=dev)
    poison(Y, 0x7B)
    ops.int8_gemm_dequant(to_dev(A, dev), to_dev(B, dev), to_dev(act, dev), to_dev(ws, dev), to_dev(b, dev), out=Y)
    assert np.array_equal(to_host(Y).view(np.uint16), orc.dequant_epilogue(acc, act, ws, b).view(np.uint16))


@pytest.mark.parametrize("M,K,N", SPARSE)
def test_decode_sparse(dev, orc, M, K, N):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M * 17 + K * 3 + N)
    W = int8_uniform(rng, (N, K))
    x = int8_uniform(rng, (M, K))
    act = rng.uniform(0.001, 0.05, M).astype(np.float32)
    ws = rng.uniform(0.001, 0.05, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16)
    cr, mr = orc.prune_compress_24(W)
    acc = orc.sparse_gemm_s32(cr, x, mr, N, K)
    comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
    raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
    meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
    ops.prune_compress_24(to_dev(W, dev), comp, raw, N, K)
    ops.pack_metadata(raw, meta, N, K)
    say(f"decode sparse M={M} K={K} N={N}")
    xd = to_dev(x, dev)
    C = torch.empty((M, N), dtype=torch.int32, device=dev)
    poison(C, 0x7B)
    assert np.array_equal(to_host(ops.sparse_int8_gemm_s32(comp, xd, meta, out=C)), acc)
    Y = torch.empty((M, N), dtype=torch.float16, device=dev)
    for split in (1, 4):
        poison(Y, 0x7B)
        ops.sparse_int8_gemm(comp, xd, meta, to_dev(act, dev), to_dev(ws, dev), to_dev(b, dev), split_k=split, out=Y)
        assert np.array_equal(to_host(Y).view(np.uint16), orc.dequant_epilogue(acc, act, ws, b).view(np.uint16))


@pytest.mark.parametrize("M", [16, 4, 1])
def test_config4_full_size(dev, orc, M):
    """M = 1, 4 and 16 tokens, N = K = 8192, dense and 2:4, FP16 tokens quantized
    per token, dequant + bias. Every output column against the oracle, through the whole
    int8_linear / sparse_int8_linear and through the GEMM alone on the quantized tokens
    (int8_gemm_dequant / sparse_int8_gemm), with poisoned outputs."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(4 + M)
    K, N = 8192, 8192
    T = orc.cpu_threads()
    W = int8_uniform(rng, (N, K))
    x = fp16_normal(rng, (M, K))
    ws = rng.uniform(1e-3, 1e-2, N).astype(np.float16)
    b = fp16_normal(rng, (N,), 0.1)
    q, s = orc.quantize_rows(x)
    ref_d = orc.gemm_dequant(q, W, s, ws, b, threads=T).view(np.uint16)
    cr, mr = orc.prune_compress_24(W)
    Wp = orc.decompress_24(cr, mr, N, K)
    ref_s = orc.gemm_dequant(q, Wp, s, ws, b, threads=T).view(np.uint16)
    xd, Wd, wsd, bd = to_dev(x, dev), to_dev(W, dev), to_dev(ws, dev), to_dev(b, dev)
    sq = torch.empty((M, K), dtype=torch.int8, device=dev)
    ss = torch.empty((M,), dtype=torch.float32, device=dev)
    y = torch.empty((M, N), dtype=torch.float16, device=dev)

    def check(what, ref):
        got = to_host(y).view(np.uint16)
        bad = int((got != ref).sum())
        assert bad == 0, f"{what}: {bad} of {got.size} outputs differ"

    say(f"config4 dense int8_linear {M}x8192x8192")
    poison(y, 0x7B)
    ops.int8_linear(xd, Wd, wsd, bd, sq, ss, out=y)
    check("int8_linear", ref_d)
    assert np.array_equal(to_host(sq), q) and np.array_equal(to_host(ss), s)
    say(f"config4 dense gemm {M}x8192x8192")
    poison(y, 0x7B)
    ops.int8_gemm_dequant(sq, Wd, ss, wsd, bd, out=y)
    check("int8_gemm_dequant", ref_d)
    comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
    raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
    meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
    ops.prune_compress_24(Wd, comp, raw, N, K)
    ops.pack_metadata(raw, meta, N, K)
    say(f"config4 sparse sparse_int8_linear {M}x8192x8192")
    poison(y, 0x7B)
    ops.sparse_int8_linear(xd, comp, meta, wsd, bd, sq, ss, out=y)
    check("sparse_int8_linear", ref_s)
    ops.fused_quantize_activation(xd, M, K, out=sq, scales=ss)
    say(f"config4 sparse gemm {M}x8192x8192")
    poison(y, 0x7B)
    ops.sparse_int8_gemm(comp, sq, meta, ss, wsd, bd, out=y)
    check("sparse_int8_gemm", ref_s)


# 16 < M <= 64: two (M <= 32) or four token blocks, partial last block; K covering every padded
# per-wave stage count (idle waves at small K, padding stages at 640 / 1152 / 5120); N ragged,
# odd (element stores), and >= 4096 (32-row workgroups instead of 16).
# Dense from K = 4096 on (K % 256 == 0, 16-row workgroups fewer than the CUs) runs the dense
# token-block kernel, with 2 or 4 K parts where N is narrow enough: (40, 5120, 64), (64, 8192, 32),
# (64, 6144, 1536), (33, 8192, 1000), (20, 4096, 2047) (odd N: element stores), and unsplit at
# (64, 8192, 4000) and (48, 4352, 300) (17 segments); the rest run the tile engine.
TB_DENSE = [(17, 128, 48), (32, 384, 200), (33, 640, 201), (48, 1152, 96), (64, 1536, 4160),
            (40, 5120, 64), (64, 8192, 32), (25, 2048, 4112), (64, 6144, 1536), (33, 8192, 1000),
            (20, 4096, 2047), (64, 8192, 4000), (48, 4352, 300)]
# From K = 4096 on, narrow N (16-row workgroups fewer than the CUs) splits K over 2 or 4
# workgroups per row block: (40, 5120, 64), (64, 8192, 32), (64, 6144, 1536), (64, 8192, 1024),
# (30, 4096, 1008). 32-row workgroups (N >= 4096) run 8 waves for K <= 4096 and N < 8192
# ((64, 1536, 4160), (25, 3072, 4112), (64, 256, 4096): 7 idle waves, (20, 4096, 4112)), else 4
# ((64, 5120, 4096), (40, 1024, 8208)).
TB_SPARSE = [(17, 256, 48), (32, 768, 208), (33, 1280, 16), (48, 2048, 96), (64, 1536, 4160),
             (40, 5120, 64), (64, 8192, 32), (25, 3072, 4112), (64, 6144, 1536), (64, 8192, 1024),
             (30, 4096, 1008), (64, 256, 4096), (20, 4096, 4112), (64, 5120, 4096), (40, 1024, 8208)]


def _check_cols(N):
    """Every output column (the oracle runs on the host's cores)."""
    return np.arange(N)


@pytest.mark.parametrize("M,K,N", TB_DENSE)
def test_token_blocks_dense(dev, orc, M, K, N):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M * 13 + K + N)
    A = int8_uniform(rng, (M, K))
    B = int8_uniform(rng, (N, K))
    act = rng.uniform(0.001, 0.05, M).astype(np.float32)
    ws = rng.uniform(0.001, 0.05, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16)
    cols = _check_cols(N)
    acc = orc.gemm_s32(A, B[cols], threads=orc.cpu_threads())
    say(f"token-block dense M={M} K={K} N={N}")
    Ad, Bd = to_dev(A, dev), to_dev(B, dev)
    C = torch.empty((M, N), dtype=torch.int32, device=dev)
    poison(C, 0x7B)
    C1 = to_host(ops.int8_gemm_s32(Ad, Bd, out=C))
    assert np.array_equal(C1[:, cols], acc)
    Y = torch.empty((M, N), dtype=torch.float16, device=dev)
    poison(Y, 0x7B)
    ops.int8_gemm_dequant(Ad, Bd, to_dev(act, dev), to_dev(ws, dev), to_dev(b, dev), out=Y)
    ref = orc.dequant_epilogue(acc, act, ws[cols], b[cols]).view(np.uint16)
    assert np.array_equal(to_host(Y).view(np.uint16)[:, cols], ref)
    # repeat run: identical bits
    assert np.array_equal(to_host(ops.int8_gemm_s32(Ad, Bd, out=C)), C1)


@pytest.mark.parametrize("M,K,N", TB_SPARSE)
def test_token_blocks_sparse(dev, orc, M, K, N):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M * 7 + K * 5 + N)
    W = int8_uniform(rng, (N, K))
    x = int8_uniform(rng, (M, K))
    act = rng.uniform(0.001, 0.05, M).astype(np.float32)
    ws = rng.uniform(0.001, 0.05, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16)
    cols = _check_cols(N)
    cr, mr = orc.prune_compress_24(W)
    Wp = orc.decompress_24(cr, mr, N, K)
    acc = orc.gemm_s32(x, Wp[cols], threads=orc.cpu_threads())
    comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
    raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
    meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
    ops.prune_compress_24(to_dev(W, dev), comp, raw, N, K)
    ops.pack_metadata(raw, meta, N, K)
    say(f"token-block sparse M={M} K={K} N={N}")
    xd = to_dev(x, dev)
    C = torch.empty((M, N), dtype=torch.int32, device=dev)
    poison(C, 0x7B)
    assert np.array_equal(to_host(ops.sparse_int8_gemm_s32(comp, xd, meta, out=C))[:, cols], acc)
    ref = orc.dequant_epilogue(acc, act, ws[cols], b[cols]).view(np.uint16)
    Y = torch.empty((M, N), dtype=torch.float16, device=dev)
    wsp = torch.empty((M, N), dtype=torch.float32, device=dev)
    # automatic plan (the token-block kernel) and a forced split (the split-K engine): same bits
    for split in (0, 1, 2):
        poison(Y, 0x7B)
        ops.sparse_int8_gemm(comp, xd, meta, to_dev(act, dev), to_dev(ws, dev), to_dev(b, dev),
                             splitk_workspace=wsp, split_k=split, out=Y)
        assert np.array_equal(to_host(Y).view(np.uint16)[:, cols], ref)


# Narrow N with K >= 4096: the dense decode splits K over 2, 4 or 8 workgroups per row block and
# hands the INT32 sums over through per-stream device slots. Ragged and odd N, 16- and 32-row
# blocks. Every shape runs twice with new operands: the hand-off must leave its sums and
# counters at zero for the next launch.
KSPLIT_DENSE = [(16, 8192, 1000), (1, 8192, 520), (4, 8192, 2048), (12, 4096, 4100), (2, 6144, 777),
                (9, 8192, 33), (16, 4096, 2047), (7, 4096, 200)]


@pytest.mark.parametrize("M,K,N", KSPLIT_DENSE)
def test_decode_dense_ksplit(dev, orc, M, K, N):
    import torch
    from forge_amd import ops
    for rep in range(2):
        rng = np.random.default_rng(M * 19 + K + N + 1000 * rep)
        A = int8_uniform(rng, (M, K))
        B = int8_uniform(rng, (N, K))
        act = rng.uniform(0.001, 0.05, M).astype(np.float32)
        ws = rng.uniform(0.001, 0.05, N).astype(np.float16)
        b = rng.uniform(-0.5, 0.5, N).astype(np.float16)
        acc = orc.gemm_s32(A, B)
        say(f"decode dense K split M={M} K={K} N={N} rep={rep}")
        Ad, Bd = to_dev(A, dev), to_dev(B, dev)
        C = torch.empty((M, N), dtype=torch.int32, device=dev)
        poison(C, 0x7B)
        assert np.array_equal(to_host(ops.int8_gemm_s32(Ad, Bd, out=C)), acc)
        Y = torch.empty((M, N), dtype=torch.float16, device=dev)
        poison(Y, 0x7B)
        ops.int8_gemm_dequant(Ad, Bd, to_dev(act, dev), to_dev(ws, dev), to_dev(b, dev), out=Y)
        assert np.array_equal(to_host(Y).view(np.uint16), orc.dequant_epilogue(acc, act, ws, b).view(np.uint16))


def test_decode_dense_ksplit_two_streams(dev, orc):
    """Split launches queued on two streams at once, without synchronising between them: each
    stream has its own sum slots, so every output matches the oracle."""
    import torch
    from forge_amd import ops
    M, K, N, n = 16, 8192, 1000, 6
    rng = np.random.default_rng(77)
    xs = [int8_uniform(rng, (M, K)) for _ in range(n)]
    B = int8_uniform(rng, (N, K))
    Bd = to_dev(B, dev)
    Ad = [to_dev(x, dev) for x in xs]
    outs = [torch.empty((M, N), dtype=torch.int32, device=dev) for _ in range(n)]
    for o in outs:
        poison(o, 0x7B)
    streams = [torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)]
    torch.cuda.synchronize(dev)
    say("decode dense K split on two streams")
    for i in range(n):
        with torch.cuda.stream(streams[i % 2]):
            ops.int8_gemm_s32(Ad[i], Bd, out=outs[i])
    torch.cuda.synchronize(dev)
    for i in range(n):
        assert np.array_equal(to_host(outs[i]), orc.gemm_s32(xs[i], B))


# Sparse register kernel (M <= 8) at K = 8192 with narrow N: 2 or 4 K parts; the LDS-ring kernel
# (9-16 tokens) from K = 6144 on: 2 or 4 parts.
KSPLIT_SPARSE = [(8, 8192, 1008), (1, 8192, 4096), (5, 8192, 2000), (3, 8192, 48),
                 (16, 8192, 4096), (12, 8192, 1008), (9, 6144, 2048), (16, 6144, 48)]


@pytest.mark.parametrize("M,K,N", KSPLIT_SPARSE)
def test_decode_sparse_ksplit(dev, orc, M, K, N):
    import torch
    from forge_amd import ops
    for rep in range(2):
        rng = np.random.default_rng(M * 23 + K + N + 1000 * rep)
        W = int8_uniform(rng, (N, K))
        x = int8_uniform(rng, (M, K))
        act = rng.uniform(0.001, 0.05, M).astype(np.float32)
        ws = rng.uniform(0.001, 0.05, N).astype(np.float16)
        b = rng.uniform(-0.5, 0.5, N).astype(np.float16)
        cr, mr = orc.prune_compress_24(W)
        acc = orc.sparse_gemm_s32(cr, x, mr, N, K)
        comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
        raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
        meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
        ops.prune_compress_24(to_dev(W, dev), comp, raw, N, K)
        ops.pack_metadata(raw, meta, N, K)
        say(f"decode sparse K split M={M} K={K} N={N} rep={rep}")
        xd = to_dev(x, dev)
        C = torch.empty((M, N), dtype=torch.int32, device=dev)
        poison(C, 0x7B)
        assert np.array_equal(to_host(ops.sparse_int8_gemm_s32(comp, xd, meta, out=C)), acc)
        Y = torch.empty((M, N), dtype=torch.float16, device=dev)
        poison(Y, 0x7B)
        ops.sparse_int8_gemm(comp, xd, meta, to_dev(act, dev), to_dev(ws, dev), to_dev(b, dev), out=Y)
        assert np.array_equal(to_host(Y).view(np.uint16), orc.dequant_epilogue(acc, act, ws, b).view(np.uint16))
