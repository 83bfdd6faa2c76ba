"""GPU parity: dense INT8 GEMM (INT32 and dequantized FP16) and int8_linear vs the oracle.

Bar: INT32 bit-exact; FP16 bit-exact to the oracle's epilogue fma((float)acc, as*ws, b)
(and therefore within the 1-ulp budget against the reference's wmma epilogue,
src/gemm/int8_dense.cu:171-174); int8_linear's quantized activation bit-exact.
Shapes cover configs[0] (golden), the reference test's shapes (tests/test_int8_dense_gemm.cu:13,
tests/test_int8_dp4a_gemm.cu:180-196 incl. K=7 and K=28), ragged edges, every tile
configuration, the skinny decode kernel, and configs[1] at full size (sampled rows)."""
import numpy as np
import pytest

from conftest import golden
from helpers import fp16_normal, int8_uniform, poison, say, to_dev, to_host

pytestmark = pytest.mark.gpu


def test_c1_golden_int32(dev):
    from forge_amd import ops
    g = golden("c1_gemm")
    say("gemm c1 golden")
    C = ops.int8_gemm_s32(to_dev(g["A"], dev), to_dev(g["B"], dev))
    assert np.array_equal(to_host(C), g["C"])


SHAPES = [
    (1, 1, 1), (6, 7, 40), (33, 28, 17), (32, 128, 64), (4, 64, 100), (16, 8192, 64), (1, 8192, 48),
    (17, 256, 33), (128, 512, 256), (130, 520, 260), (300, 1000, 700), (1024, 1024, 1024),
    (2048, 640, 2048), (4096, 256, 4096),
]


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_gemm_int32(dev, orc, M, K, N):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M * 7 + K * 3 + N)
    A = int8_uniform(rng, (M, K))
    B = int8_uniform(rng, (N, K))
    rows = np.unique(np.linspace(0, M - 1, min(M, 64)).astype(int))
    ref = orc.gemm_s32(A[rows], B)
    say(f"gemm s32 M={M} K={K} N={N}")
    out = torch.empty((M, N), dtype=torch.int32, device=dev)
    poison(out, 0x7B)
    C = to_host(ops.int8_gemm_s32(to_dev(A, dev), to_dev(B, dev), out=out))
    assert np.array_equal(C[rows], ref)
    if M <= 1024:
        assert np.array_equal(C, orc.gemm_s32(A, B))


@pytest.mark.parametrize("M,K,N", [(32, 128, 64), (6, 7, 40), (16, 8192, 256), (130, 520, 260), (512, 1024, 768)])
@pytest.mark.parametrize("bias", [True, False])
def test_gemm_dequant(dev, orc, M, K, N, bias):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M + K + N + bias)
    A = int8_uniform(rng, (M, K))
    B = int8_uniform(rng, (N, K))
    act = rng.uniform(0.001, 0.05, M).astype(np.float32)
    ws = rng.uniform(0.001, 0.05, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16) if bias else None
    ref = orc.gemm_dequant(A, B, act, ws, b)
    say(f"gemm dequant M={M} K={K} N={N} bias={bias}")
    out = torch.empty((M, N), dtype=torch.float16, device=dev)
    poison(out, 0x7B)
    Y = ops.int8_gemm_dequant(to_dev(A, dev), to_dev(B, dev), to_dev(act, dev), to_dev(ws, dev),
                              None if b is None else to_dev(b, dev), out=out)
    assert np.array_equal(to_host(Y).view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("M,K,N", [(1, 8192, 512), (4, 8192, 512), (16, 8192, 512), (37, 640, 300)])
def test_int8_linear(dev, orc, M, K, N):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M + N)
    x = fp16_normal(rng, (M, K))
    W = int8_uniform(rng, (N, K))
    ws = rng.uniform(1e-3, 1e-2, N).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float16)
    ref, qr, sr = orc.linear(x, W, ws, b)
    say(f"int8_linear M={M} K={K} N={N}")
    sq = torch.empty((M, K), dtype=torch.int8, device=dev)
    ss = torch.empty((M,), dtype=torch.float32, device=dev)
    Y = ops.int8_linear(to_dev(x, dev), to_dev(W, dev), to_dev(ws, dev), to_dev(b, dev), sq, ss)
    assert np.array_equal(to_host(sq), qr) and np.array_equal(to_host(ss), sr)
    assert np.array_equal(to_host(Y).view(np.uint16), ref.view(np.uint16))


def test_config2_full_size(dev, orc):
    """W8A8 linear 4096^3, outlier channels; every quantized activation, scale and
    FP16 output compared bit-exactly with the oracle (threaded loop); repeat run bit-identical."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(2)
    M = N = K = 4096
    x = rng.standard_normal((M, K), dtype=np.float32)
    x[:, rng.choice(K, 8, replace=False)] *= 20
    x = x.astype(np.float16)
    W = int8_uniform(rng, (N, K))
    ws = rng.uniform(1e-3, 1e-2, N).astype(np.float32).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float16)
    ref, qr, sr = orc.linear(x, W, ws, b, threads=orc.cpu_threads())
    say("config2 4096^3 linear")
    sq = torch.empty((M, K), dtype=torch.int8, device=dev)
    ss = torch.empty((M,), dtype=torch.float32, device=dev)
    xd, Wd, wsd, bd = to_dev(x, dev), to_dev(W, dev), to_dev(ws, dev), to_dev(b, dev)
    out = torch.empty((M, N), dtype=torch.float16, device=dev)
    poison(out, 0x7B)
    Y1 = to_host(ops.int8_linear(xd, Wd, wsd, bd, sq, ss, out=out))
    assert np.array_equal(to_host(sq), qr) and np.array_equal(to_host(ss), sr)
    bad = int((Y1.view(np.uint16) != ref.view(np.uint16)).sum())
    assert bad == 0, f"{bad} of {Y1.size} outputs differ"
    Y2 = to_host(ops.int8_linear(xd, Wd, wsd, bd, sq, ss))
    assert np.array_equal(Y1.view(np.uint16), Y2.view(np.uint16))


def test_4096_cube_int32(dev, orc):
    """4096^3 INT32 (the headline GEMM shape without the epilogue): every output bit-exact."""
    from forge_amd import ops
    rng = np.random.default_rng(4096)
    A = int8_uniform(rng, (4096, 4096))
    B = int8_uniform(rng, (4096, 4096))
    ref = orc.gemm_s32(A, B, threads=orc.cpu_threads())
    say("gemm s32 4096^3")
    C = to_host(ops.int8_gemm_s32(to_dev(A, dev), to_dev(B, dev)))
    bad = int((C != ref).sum())
    assert bad == 0, f"{bad} of {C.size} outputs differ"


@pytest.mark.parametrize("N", [256, 200])
def test_gemm_tail_split(dev, orc, N):
    """M = 70,000 rows in one column of 256x256 tiles: 274 tiles, the second wave 7 % full, so
    the first 65,536 rows run as 256-row tiles and the rest as 192-row tiles in a second
    launch. Rows on both sides of the boundary and the last rows bit-exact (INT32 and FP16);
    every column's sum over all rows equals (sum of A's rows) . B (exact in int64)."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(70000 + N)
    M, K = 70000, 256
    A = int8_uniform(rng, (M, K))
    B = int8_uniform(rng, (N, K))
    rows = np.array([0, 255, 65535, 65536, 65537, 65727, 65728, 69887, 69888, 69999])
    ref = orc.gemm_s32(A[rows], B)
    say(f"gemm tail split M={M} K={K} N={N}")
    Ad, Bd = to_dev(A, dev), to_dev(B, dev)
    out = torch.empty((M, N), dtype=torch.int32, device=dev)
    poison(out, 0x7B)
    C = to_host(ops.int8_gemm_s32(Ad, Bd, out=out))
    assert np.array_equal(C[rows], ref)
    assert np.array_equal(C.astype(np.int64).sum(axis=0), A.astype(np.int64).sum(axis=0) @ B.astype(np.int64).T)
    act = rng.uniform(0.001, 0.05, M).astype(np.float32)
    ws = rng.uniform(0.001, 0.05, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16)
    Y = torch.empty((M, N), dtype=torch.float16, device=dev)
    poison(Y, 0x7B)
    ops.int8_gemm_dequant(Ad, Bd, to_dev(act, dev), to_dev(ws, dev), to_dev(b, dev), out=Y)
    refy = orc.dequant_epilogue(ref, act[rows], ws, b)
    assert np.array_equal(to_host(Y)[rows].view(np.uint16), refy.view(np.uint16))


@pytest.mark.parametrize("M,K,N", [(1000, 1024, 17900), (512, 1024, 35000), (4096, 4096, 11008)])
def test_gemm_column_tail_split(dev, orc, M, K, N):
    """Grids of several 256-column tiles that are more than one wave but not whole waves: whole
    waves of 256 x 256 tiles over the first tile columns, the remaining columns as one wave of
    192-row tiles, in one launch. (1000, 1024, 17900): 280 tiles = 64 columns x 4 + 6 x 6
    (ragged rows and last column); (512, 1024, 35000): 128 x 2 + 9 x 3; (4096, 4096, 11008):
    configs[2]'s shape, 32 x 16 + 11 x 22. Every INT32 and FP16 output against the oracle."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M + K + N + 3)
    A = int8_uniform(rng, (M, K))
    B = int8_uniform(rng, (N, K))
    ref = orc.gemm_s32(A, B, threads=orc.cpu_threads())
    say(f"gemm column tail split M={M} K={K} N={N}")
    Ad, Bd = to_dev(A, dev), to_dev(B, dev)
    out = torch.empty((M, N), dtype=torch.int32, device=dev)
    poison(out, 0x7B)
    C = to_host(ops.int8_gemm_s32(Ad, Bd, out=out))
    assert ops.last_route() == "dma256x256+tail192"
    bad = int((C != ref).sum())
    assert bad == 0, f"INT32: {bad} of {C.size} outputs differ"
    act = rng.uniform(0.001, 0.05, M).astype(np.float32)
    ws = rng.uniform(0.001, 0.05, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16)
    Y = torch.empty((M, N), dtype=torch.float16, device=dev)
    poison(Y, 0x7B)
    ops.int8_gemm_dequant(Ad, Bd, to_dev(act, dev), to_dev(ws, dev), to_dev(b, dev), out=Y)
    assert ops.last_route() == "dma256x256+tail192"
    refy = orc.dequant_epilogue(ref, act, ws, b).view(np.uint16)
    bad = int((to_host(Y).view(np.uint16) != refy).sum())
    assert bad == 0, f"FP16: {bad} of {Y.numel()} outputs differ"
    poison(Y, 0x5A)
    ops.int8_gemm_dequant(Ad, Bd, to_dev(act, dev), to_dev(ws, dev), None, out=Y)
    refy = orc.dequant_epilogue(ref, act, ws, None).view(np.uint16)
    bad = int((to_host(Y).view(np.uint16) != refy).sum())
    assert bad == 0, f"FP16 without bias: {bad} of {Y.numel()} outputs differ"
