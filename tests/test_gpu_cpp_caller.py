"""GPU: a compiled C++ caller of the drop-in API (tests/cpp/forge_caller.hip), loaded into this
process with ctypes. It includes only include/forge/**.h and calls forge::quant::* and
forge::gemm::* by the reference's names and default arguments, and launches the exported
forge::quant::fused_quantize_activation_kernel with <<<M, threads>>> as the reference's
tests/test_quantize.cu:50-55 does. Results are checked bit-exactly against the oracle."""
import ctypes
import os

import numpy as np
import pytest

from helpers import fp16_normal, int8_uniform, poison, say, special_fp16_rows, to_dev, to_host

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
CALLER = os.path.join(HERE, "cpp", "lib", "libforge_caller.so")
_P, _I = ctypes.c_void_p, ctypes.c_int


@pytest.fixture(scope="module")
def caller(dev):
    if not os.path.exists(CALLER):
        raise RuntimeError(f"{CALLER} is not built (python tests/cpp/build.py)")
    lib = ctypes.CDLL(CALLER)
    sigs = {
        "caller_quantize_kernel": [_P, _P, _P, _I, _I, _I, _P],
        "caller_quantize": [_P, _P, _P, _I, _I, _P],
        "caller_dequantize_bias": [_P, _P, _P, _P, _P, _I, _I, _P],
        "caller_int8_linear": [_P, _P, _P, _P, _P, _I, _I, _I, _P, _P, _P],
        "caller_sparse_int8_linear": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _P],
        "caller_dp4a_gemm_dequant": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _P],
        "caller_dp4a_linear": [_P, _P, _P, _P, _P, _I, _I, _I, _P, _P, _P],
        "caller_last_error_after_bad_call": [],
    }
    for name, args in sigs.items():
        getattr(lib, name).argtypes = args
        getattr(lib, name).restype = _I
    return lib


def _stream():
    import torch
    return torch.cuda.current_stream().cuda_stream


def _p(t):
    return None if t is None else t.data_ptr()


@pytest.mark.parametrize("M,K,threads", [(37, 1000, 256), (8, 4096, 64), (5, 333, 1024), (3, 64, 1)])
def test_cpp_quantize_kernel_launch(dev, orc, caller, M, K, threads):
    import torch
    rng = np.random.default_rng(M + K + threads)
    x = special_fp16_rows(rng, M, K) if M >= 8 else fp16_normal(rng, (M, K))
    q_ref, s_ref = orc.quantize_rows(x)
    xd = to_dev(x, dev)
    q = torch.empty((M, K), dtype=torch.int8, device=dev)
    s = torch.empty((M,), dtype=torch.float32, device=dev)
    poison(q, 0x7B)
    poison(s, 0x5A)
    say(f"C++ <<<{M}, {threads}>>> quantize kernel K={K}")
    assert caller.caller_quantize_kernel(_p(xd), _p(q), _p(s), M, K, threads, _stream()) == 0
    assert np.array_equal(to_host(q), q_ref)
    assert np.array_equal(to_host(s).view(np.uint32), s_ref.view(np.uint32))
    q2 = torch.empty_like(q)
    s2 = torch.empty_like(s)
    assert caller.caller_quantize(_p(xd), _p(q2), _p(s2), M, K, _stream()) == 0
    assert np.array_equal(to_host(q2), q_ref)
    assert np.array_equal(to_host(s2).view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("M,K,N", [(1, 8192, 512), (16, 4096, 1000), (300, 640, 260), (1024, 1024, 1024)])
def test_cpp_int8_linear(dev, orc, caller, M, K, N):
    import torch
    rng = np.random.default_rng(M * 5 + N)
    x = fp16_normal(rng, (M, K))
    W = int8_uniform(rng, (N, K))
    ws = rng.uniform(1e-3, 1e-2, N).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float16)
    ref, qr, sr = orc.linear(x, W, ws, b, threads=orc.cpu_threads())
    say(f"C++ forge::gemm::int8_linear M={M} K={K} N={N}")
    xd, Wd, wsd, bd = to_dev(x, dev), to_dev(W, dev), to_dev(ws, dev), to_dev(b, dev)
    sq = torch.empty((M, K), dtype=torch.int8, device=dev)
    ss = torch.empty((M,), dtype=torch.float32, device=dev)
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    poison(y, 0x7B)
    assert caller.caller_int8_linear(_p(xd), _p(Wd), _p(wsd), _p(bd), _p(y), M, K, N, _p(sq), _p(ss),
                                     _stream()) == 0
    assert np.array_equal(to_host(y).view(np.uint16), ref.view(np.uint16))
    assert np.array_equal(to_host(sq), qr)


# The reference's dp4a test shapes include K = 7 and K = 28 (tests/test_int8_dp4a_gemm.cu:180-196);
# here the dp4a names forward to the matrix-core path, which must give the oracle's bits.
@pytest.mark.parametrize("M,K,N", [(5, 7, 9), (33, 28, 40), (64, 256, 96), (129, 1000, 300), (4, 4096, 512)])
def test_cpp_dp4a_forwards(dev, orc, caller, M, K, N):
    import torch
    rng = np.random.default_rng(M * 3 + K + N)
    A = int8_uniform(rng, (M, K))
    W = int8_uniform(rng, (N, K))
    act = rng.uniform(1e-3, 5e-2, M).astype(np.float32)
    ws = rng.uniform(1e-3, 1e-2, N).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float16)
    say(f"C++ forge::gemm::int8_dp4a_gemm_dequant / int8_dp4a_linear M={M} K={K} N={N}")
    Ad, Wd, actd, wsd, bd = to_dev(A, dev), to_dev(W, dev), to_dev(act, dev), to_dev(ws, dev), to_dev(b, dev)
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    poison(y, 0x7B)
    assert caller.caller_dp4a_gemm_dequant(_p(Ad), _p(Wd), _p(actd), _p(wsd), _p(bd), _p(y), M, K, N,
                                           _stream()) == 0
    ref = orc.gemm_dequant(A, W, act, ws, b, threads=orc.cpu_threads())
    assert np.array_equal(to_host(y).view(np.uint16), ref.view(np.uint16))
    x = fp16_normal(rng, (M, K))
    ref2, qr, sr = orc.linear(x, W, ws, b, threads=orc.cpu_threads())
    xd = to_dev(x, dev)
    sq = torch.empty((M, K), dtype=torch.int8, device=dev)
    ss = torch.empty((M,), dtype=torch.float32, device=dev)
    poison(y, 0x7B)
    assert caller.caller_dp4a_linear(_p(xd), _p(Wd), _p(wsd), _p(bd), _p(y), M, K, N, _p(sq), _p(ss),
                                     _stream()) == 0
    assert np.array_equal(to_host(y).view(np.uint16), ref2.view(np.uint16))
    assert np.array_equal(to_host(sq), qr)
    assert np.array_equal(to_host(ss).view(np.uint32), sr.view(np.uint32))


@pytest.mark.parametrize("M,K,N", [(1, 8192, 1024), (16, 2048, 208), (600, 1024, 512)])
def test_cpp_sparse_int8_linear_defaults(dev, orc, caller, M, K, N):
    """forge::gemm::sparse_int8_linear with the header's default trailing arguments, on the
    null stream (torch's default stream in this test)."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M * 7 + K + N)
    x = fp16_normal(rng, (M, K))
    W = int8_uniform(rng, (N, K))
    ws = rng.uniform(1e-3, 1e-2, N).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float16)
    cr, mr = orc.prune_compress_24(W)
    qr, sr = orc.quantize_rows(x)
    ref = orc.dequant_epilogue(orc.sparse_gemm_s32(cr, qr, mr, N, K, threads=orc.cpu_threads()), sr, ws, b)
    comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
    raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
    meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
    ops.prune_compress_24(to_dev(W, dev), comp, raw, N, K)
    ops.pack_metadata(raw, meta, N, K)
    xd, wsd, bd = to_dev(x, dev), to_dev(ws, dev), to_dev(b, dev)
    sq = torch.empty((M, K), dtype=torch.int8, device=dev)
    ss = torch.empty((M,), dtype=torch.float32, device=dev)
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    poison(y, 0x7B)
    assert torch.cuda.current_stream().cuda_stream == 0
    torch.cuda.synchronize()
    say(f"C++ forge::gemm::sparse_int8_linear M={M} K={K} N={N}")
    assert caller.caller_sparse_int8_linear(_p(xd), _p(comp), _p(meta), _p(wsd), _p(bd), _p(y), M, K, N,
                                            _p(sq), _p(ss)) == 0
    assert np.array_equal(to_host(y).view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("M,N,bias", [(7, 300, True), (64, 4096, False)])
def test_cpp_dequantize_bias(dev, orc, caller, M, N, bias):
    import torch
    rng = np.random.default_rng(M + N)
    acc = rng.integers(-(1 << 24), 1 << 24, (M, N)).astype(np.int32)
    act = rng.uniform(1e-3, 5e-2, M).astype(np.float32)
    ws = rng.uniform(1e-3, 1e-2, N).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float16) if bias else None
    ref = orc.dequantize_bias(acc, act, ws, b)
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    poison(y, 0x7B)
    accd, actd, wsd = to_dev(acc, dev), to_dev(act, dev), to_dev(ws, dev)
    bd = None if b is None else to_dev(b, dev)
    say(f"C++ forge::quant::fused_dequantize_bias M={M} N={N}")
    assert caller.caller_dequantize_bias(_p(accd), _p(actd), _p(wsd), _p(bd), _p(y), M, N, _stream()) == 0
    assert np.array_equal(to_host(y).view(np.uint16), ref.view(np.uint16))


def test_cpp_last_error(dev, caller):
    from forge_amd import _lib
    assert caller.caller_last_error_after_bad_call() == _lib.FORGE_EINVAL
