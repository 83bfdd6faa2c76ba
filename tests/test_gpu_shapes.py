"""GPU parity over a seeded sweep of shapes, through every dispatch branch.

The dense GEMM picks between the decode kernels (M <= 16, K % 128 == 0, K <= 8192), the skinny
kernel (other M <= 16), the DMA engine with 256- or 128-row tiles (K % 128 == 0, grid large
enough), the register-staged engine (other K % 16 == 0 with aligned rows) and the byte-gather
engine (anything else, e.g. misaligned views). The sparse GEMM picks between the decode kernels,
the DMA tiles, the register-staged kernel and split-K. Each case is checked bit-exactly against
the oracle (INT32, and FP16 through the dequant epilogue)."""
import numpy as np
import pytest

from helpers import int8_uniform, say, to_dev, to_host

pytestmark = pytest.mark.gpu


def _cases_dense():
    rng = np.random.default_rng(1234)
    cases = []
    for i in range(28):
        kind = i % 7
        if kind == 0:       # decode / skinny
            M = int(rng.integers(1, 17))
            K = int(rng.choice([128, 384, 1152, 2048, 4096, 8192, 8320, 208, 16 * int(rng.integers(1, 60))]))
            N = int(rng.integers(1, 300))
        elif kind == 1:     # DMA engine, 128-row tiles
            M, N, K = int(rng.integers(700, 1300)), int(rng.integers(1500, 2600)), 128 * int(rng.integers(1, 9))
        elif kind == 2:     # DMA engine, 256-row tiles, ragged edges
            M, N, K = int(rng.integers(3000, 4200)), int(rng.integers(3000, 4200)), 128 * int(rng.integers(1, 4))
        elif kind == 3:     # register-staged (K % 16 == 0, K % 128 != 0)
            M, N, K = int(rng.integers(17, 600)), int(rng.integers(1, 700)), 16 * int(rng.integers(1, 80))
        elif kind == 4:     # odd K: byte gathers
            M, N, K = int(rng.integers(1, 300)), int(rng.integers(1, 300)), int(rng.integers(1, 700))
        elif kind == 5:     # misaligned A (offset view): byte gathers
            M, N, K = int(rng.integers(1, 400)), int(rng.integers(1, 400)), 16 * int(rng.integers(1, 40))
        else:               # small everything
            M, N, K = int(rng.integers(1, 80)), int(rng.integers(1, 80)), int(rng.integers(1, 300))
        cases.append((i, kind, M, N, K))
    return cases


def _offset_view(a: np.ndarray, dev, off: int):
    """A device copy of `a` whose data pointer is `off` bytes past a 256-byte boundary."""
    import torch
    flat = torch.zeros((a.nbytes + 256,), dtype=torch.int8, device=dev)
    v = flat[off:off + a.size].view(a.shape)
    v.copy_(torch.from_numpy(np.ascontiguousarray(a)).to(dev))
    return v


@pytest.mark.parametrize("i,kind,M,N,K", _cases_dense())
def test_dense_sweep(dev, orc, i, kind, M, N, K):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(100 + i)
    A = int8_uniform(rng, (M, K))
    B = int8_uniform(rng, (N, K))
    act = rng.uniform(1e-3, 5e-2, M).astype(np.float32)
    ws = rng.uniform(1e-3, 5e-2, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16) if i % 2 else None
    acc = orc.gemm_s32(A, B)
    say(f"dense sweep {i} kind={kind} M={M} N={N} K={K}")
    Ad = _offset_view(A, dev, 1 + (i % 15)) if kind == 5 else to_dev(A, dev)
    Bd = to_dev(B, dev)
    C = torch.empty((M, N), dtype=torch.int32, device=dev)
    C.view(torch.uint8).fill_(0x7B)
    assert np.array_equal(to_host(ops.int8_gemm_s32(Ad, Bd, out=C)), acc)
    Y = torch.empty((M, N), dtype=torch.float16, device=dev)
    Y.view(torch.uint8).fill_(0x7B)
    ops.int8_gemm_dequant(Ad, Bd, to_dev(act, dev), to_dev(ws, dev), None if b is None else to_dev(b, dev), out=Y)
    assert np.array_equal(to_host(Y).view(np.uint16), orc.dequant_epilogue(acc, act, ws, b).view(np.uint16))


def _cases_sparse():
    rng = np.random.default_rng(4321)
    cases = []
    for i in range(16):
        kind = i % 4
        if kind == 0:       # decode shapes
            M, K = int(rng.integers(1, 17)), 64 * int(rng.integers(1, 100))
            N = 16 * int(rng.integers(1, 40))
        elif kind == 1:     # DMA tiles
            M, K, N = int(rng.integers(65, 700)), 128 * int(rng.integers(1, 12)), 16 * int(rng.integers(20, 120))
        elif kind == 2:     # K % 128 == 64: register-staged
            M, K, N = int(rng.integers(1, 400)), 64 + 128 * int(rng.integers(0, 10)), 16 * int(rng.integers(1, 60))
        else:               # split-K through the caller's workspace
            M, K, N = int(rng.integers(1, 300)), 128 * int(rng.integers(2, 20)), 16 * int(rng.integers(1, 50))
        cases.append((i, kind, M, N, K))
    return cases


@pytest.mark.parametrize("i,kind,M,N,K", _cases_sparse())
def test_sparse_sweep(dev, orc, i, kind, M, N, K):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(200 + i)
    W = int8_uniform(rng, (N, K))
    x = int8_uniform(rng, (M, K))
    act = rng.uniform(1e-3, 5e-2, M).astype(np.float32)
    ws = rng.uniform(1e-3, 5e-2, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16)
    cr, mr = orc.prune_compress_24(W)
    acc = orc.sparse_gemm_s32(cr, x, mr, N, K)
    say(f"sparse sweep {i} kind={kind} M={M} N={N} K={K}")
    comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
    raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
    meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
    ops.prune_compress_24(to_dev(W, dev), comp, raw, N, K)
    ops.pack_metadata(raw, meta, N, K)
    xd = to_dev(x, dev)
    C = torch.empty((M, N), dtype=torch.int32, device=dev)
    C.view(torch.uint8).fill_(0x7B)
    assert np.array_equal(to_host(ops.sparse_int8_gemm_s32(comp, xd, meta, out=C)), acc)
    Y = torch.empty((M, N), dtype=torch.float16, device=dev)
    want = orc.dequant_epilogue(acc, act, ws, b).view(np.uint16)
    wsp = torch.empty((M * N,), dtype=torch.float32, device=dev)
    for split in ((1, 3) if kind == 3 else (1,)):
        Y.view(torch.uint8).fill_(0x7B)
        wsp.view(torch.uint8).fill_(0x5A)
        ops.sparse_int8_gemm(comp, xd, meta, to_dev(act, dev), to_dev(ws, dev), to_dev(b, dev),
                             splitk_workspace=wsp if split > 1 else None, split_k=split, out=Y)
        assert np.array_equal(to_host(Y).view(np.uint16), want)


def _cases_conv():
    rng = np.random.default_rng(777)
    cases = []
    for i in range(8):
        C = int(rng.choice([16, 32, 48, 128, 256, 24]))
        k = int(rng.choice([1, 3, 5]))
        pad = int(rng.integers(0, k // 2 + 2))
        stride = int(rng.integers(1, 3))
        dil = int(rng.integers(1, 3))
        H, W = int(rng.integers(k * dil, 40)), int(rng.integers(k * dil, 40))
        N, Co = int(rng.integers(1, 4)), int(rng.integers(1, 300))
        cases.append((i, N, H, W, C, Co, k, pad, stride, dil))
    return cases


@pytest.mark.parametrize("i,N,H,W,C,Co,k,pad,stride,dil", _cases_conv())
def test_conv_sweep(dev, orc, i, N, H, W, C, Co, k, pad, stride, dil):
    from forge_amd import ops
    rng = np.random.default_rng(300 + i)
    x = int8_uniform(rng, (N, H, W, C))
    w = int8_uniform(rng, (Co, k, k, C))
    ref = orc.conv2d_nhwc_s32(x, w, (pad, pad), (stride, stride), (dil, dil))
    say(f"conv sweep {i} N={N} H={H} W={W} C={C} Co={Co} k={k} p={pad} s={stride} d={dil}")
    out = ops.int8_conv2d_nhwc_s32(to_dev(x, dev), to_dev(w, dev), (pad, pad), (stride, stride), (dil, dil))
    assert np.array_equal(to_host(out), ref)
