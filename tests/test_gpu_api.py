"""GPU: the entry points of the reference API that no other test reaches.

- forge_get_compute_capability / forge_has_int8_matrix_cores (the reference's
  get_compute_capability / has_wmma_int8, src/gemm/int8_gemm.cu:12-24): 950 and 1 on MI355X.
- forge_int8_gemm (the reference's capability dispatch, int8_gemm.cu:26-46): bit-identical to
  forge_int8_gemm_dequant, and to the oracle's GEMM + epilogue.
- forge_splitk_reduce (int8_sparse.cu:99-111, :945-958): an FP32 workspace plus FP16 bias to
  FP16, bit-exact against the oracle, with and without bias, on ragged sizes.
"""
import numpy as np
import pytest

from helpers import int8_uniform, poison, say, to_dev, to_host

pytestmark = pytest.mark.gpu


def test_compute_capability(dev):
    from forge_amd import ops
    say("compute capability")
    assert ops.get_compute_capability(0) == 950
    assert ops.has_int8_matrix_cores(0) is True


def test_compute_capability_bad_device(dev):
    from forge_amd import _lib
    import ctypes
    v = ctypes.c_int(-7)
    st = _lib.load().forge_get_compute_capability(1 << 20, ctypes.addressof(v))
    assert st != _lib.FORGE_OK and v.value == -7
    assert _lib.load().forge_get_compute_capability(0, None) == _lib.FORGE_EINVAL


@pytest.mark.parametrize("M,K,N,bias", [(64, 512, 192, True), (1, 8192, 520, False), (300, 1000, 700, True),
                                        (4096, 4096, 256, True)])
def test_int8_gemm_dispatch(dev, orc, M, K, N, bias):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M + 5 * K + N)
    A = int8_uniform(rng, (M, K))
    B = int8_uniform(rng, (N, K))
    act = rng.uniform(0.001, 0.05, M).astype(np.float32)
    ws = rng.uniform(0.001, 0.05, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16) if bias else None
    ref = orc.gemm_dequant(A, B, act, ws, b, threads=orc.cpu_threads()).view(np.uint16)
    say(f"int8_gemm M={M} K={K} N={N} bias={bias}")
    Ad, Bd, actd, wsd = to_dev(A, dev), to_dev(B, dev), to_dev(act, dev), to_dev(ws, dev)
    bd = None if b is None else to_dev(b, dev)
    y1 = torch.empty((M, N), dtype=torch.float16, device=dev)
    y2 = torch.empty((M, N), dtype=torch.float16, device=dev)
    poison(y1, 0x7B)
    poison(y2, 0x5A)
    ops.int8_gemm(Ad, Bd, actd, wsd, bd, out=y1)
    ops.int8_gemm_dequant(Ad, Bd, actd, wsd, bd, out=y2)
    g1, g2 = to_host(y1).view(np.uint16), to_host(y2).view(np.uint16)
    assert np.array_equal(g1, g2)
    assert np.array_equal(g1, ref)


@pytest.mark.parametrize("M,N,bias", [(1, 16, True), (37, 1000, True), (37, 1000, False), (513, 4112, True),
                                      (7, 1002, True)])
def test_splitk_reduce(dev, orc, M, N, bias):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M * 3 + N)
    ws = (rng.standard_normal((M, N)) * 40).astype(np.float32)
    ws.flat[:3] = [65520.0, -70000.0, 3e-8]      # overflow to +-inf and an fp16 subnormal
    b = (rng.standard_normal(N) * 2).astype(np.float16) if bias else None
    ref = orc.splitk_reduce(ws, b).view(np.uint16)
    say(f"splitk_reduce M={M} N={N} bias={bias}")
    out = torch.empty((M, N), dtype=torch.float16, device=dev)
    poison(out, 0x7B)
    ops.splitk_reduce(to_dev(ws, dev), None if b is None else to_dev(b, dev), M, N, out=out)
    assert np.array_equal(to_host(out).view(np.uint16), ref)
