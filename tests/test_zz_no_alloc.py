"""GPU: forge_int8_linear_noalloc (the no-allocation form of forge_int8_linear, whose quantized
activations live in the library's per-GPU device array) against forge_int8_linear with caller
scratch and against the oracle, through the C ABI: two calls in a row, the second with a smaller
input, bit-identical outputs; sizes beyond the array's limits are rejected with FORGE_ERANGE before any launch."""
import ctypes

import numpy as np
import pytest

from helpers import fp16_normal, int8_uniform, poison, say, to_dev, to_host

pytestmark = pytest.mark.gpu


def _call_noalloc(lib, x, w, ws, b, out, M, K, N, stream):
    return lib.forge_int8_linear_noalloc(x.data_ptr(), w.data_ptr(), ws.data_ptr(),
                                         None if b is None else b.data_ptr(), out.data_ptr(), M, K, N, stream)


def test_noalloc_matches_int8_linear(dev, orc):
    import torch
    from forge_amd import _lib, ops
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    rng = np.random.default_rng(77)
    # the second call is smaller than the first (fewer rows, shorter K), so it reads only what
    # it wrote itself; the third runs the decode path with the quantize fused into the GEMM
    for M, K, N, bias in [(1024, 2048, 768, True), (37, 512, 264, False), (2, 8192, 512, True)]:
        x = to_dev(fp16_normal(rng, (M, K)), dev)
        w = to_dev(int8_uniform(rng, (N, K)), dev)
        ws = to_dev(rng.uniform(1e-3, 1e-2, N).astype(np.float16), dev)
        b = to_dev(fp16_normal(rng, (N,), 0.1), dev) if bias else None
        q = torch.empty((M, K), dtype=torch.int8, device=dev)
        s = torch.empty((M,), dtype=torch.float32, device=dev)
        want = torch.empty((M, N), dtype=torch.float16, device=dev)
        ops.int8_linear(x, w, ws, b, q, s, out=want)
        got = torch.empty((M, N), dtype=torch.float16, device=dev)
        poison(got, 0x7B)
        say(f"int8_linear_noalloc M={M} K={K} N={N} bias={bias}")
        assert _call_noalloc(lib, x, w, ws, b, got, M, K, N, stream) == _lib.FORGE_OK
        assert np.array_equal(to_host(got).view(np.uint16), to_host(want).view(np.uint16))
        # and against the oracle's quantize + INT32 GEMM + epilogue directly
        ref, _, _ = orc.linear(to_host(x), to_host(w), to_host(ws), None if b is None else to_host(b),
                               threads=orc.cpu_threads())
        assert np.array_equal(to_host(got).view(np.uint16), ref.view(np.uint16))


def test_noalloc_limits(dev):
    import torch
    from forge_amd import _lib
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    x = torch.empty((8,), dtype=torch.float16, device=dev)
    w = torch.empty((8,), dtype=torch.int8, device=dev)
    ws = torch.empty((8,), dtype=torch.float16, device=dev)
    out = torch.empty((8,), dtype=torch.float16, device=dev)
    # shapes only: nothing is launched for a rejected size, so the tiny buffers are never read
    assert _call_noalloc(lib, x, w, ws, None, out, 4097, 4096, 16, stream) == _lib.FORGE_ERANGE
    assert _call_noalloc(lib, x, w, ws, None, out, 65537, 16, 16, stream) == _lib.FORGE_ERANGE
    assert lib.forge_int8_linear_noalloc(None, None, None, None, None, 4, 64, 16, stream) == _lib.FORGE_EINVAL


def test_noalloc_graph_capture(dev):
    """Under graph capture (in a process of its own, so that forge_init has not run yet): a
    first call inside a capture is rejected with FORGE_EINVAL (the array's address is resolved
    outside captures); after forge_init, two calls of different shapes captured into one graph
    replay three times, with eager work in between, to the bits of eager forge_int8_linear."""
    import json
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    say("fresh process check: noalloc under graph capture")
    r = subprocess.run([sys.executable, os.path.join(here, "fresh_process_checks.py"), "noalloc"],
                       capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-3000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["before_init"] == out["EINVAL"]
    assert out["init"] == out["OK"]
    assert out["statuses"] == [out["OK"], out["OK"]]
    assert all(all(e) for e in out["equal"]), out["equal"]
