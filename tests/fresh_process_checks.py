"""GPU checks that need a process of their own (run by the -m gpu tests as a child process,
one at a time): they depend on the library's per-process state -- which launch keys hold the
static device slots, and whether forge_init has resolved the no-alloc array -- so they must not
share a process with the other tests.

    python tests/fresh_process_checks.py slots      # the 33rd graph capture of a K-split decode
    python tests/fresh_process_checks.py noalloc    # no-alloc entry point captured before/after init

Prints one JSON line with what it saw; the calling test asserts on it."""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, HERE)


def _capture(torch, fn):
    """fn() recorded into a graph on a side stream; returns (graph, fn's return value)."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        r = fn()
    return g, r


def slots():
    """Each graph capture is a launch key of its own, so a K-split decode launch recorded into
    32 captures takes the 32 K-split slots; the 33rd capture records the unsplit decode. Every
    replay must equal the eager result bit for bit."""
    import torch
    from forge_amd import _lib, ops
    from helpers import fp16_normal, int8_uniform
    dev = torch.device("cuda:0")
    lib = _lib.load()
    assert lib.forge_init() == _lib.FORGE_OK
    rng = np.random.default_rng(5)
    M, K, N = 16, 8192, 1024          # 32 row blocks: the decode splits K in 8 parts
    x = torch.from_numpy(int8_uniform(rng, (M, K))).to(dev)
    W = torch.from_numpy(int8_uniform(rng, (N, K))).to(dev)
    act = torch.from_numpy(rng.uniform(1e-3, 5e-2, M).astype(np.float32)).to(dev)
    ws = torch.from_numpy(rng.uniform(1e-3, 1e-2, N).astype(np.float16)).to(dev)
    b = torch.from_numpy(fp16_normal(rng, (N,), 0.1)).to(dev)
    ref = torch.empty((M, N), dtype=torch.float16, device=dev)
    ops.int8_gemm_dequant(x, W, act, ws, b, out=ref)
    eager = ops.ksplit_last()
    used0, total, _, _ = ops.slots_in_use()
    torch.cuda.synchronize()
    graphs, outs, recorded = [], [], []
    for _ in range(total - used0 + 1):
        y = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
        g, _ = _capture(torch, lambda y=y: ops.int8_gemm_dequant(x, W, act, ws, b, out=y))
        recorded.append(list(ops.ksplit_last()))
        graphs.append(g)
        outs.append(y)
    after = list(ops.slots_in_use())
    equal = []
    for rep in range(3):
        for g in graphs:
            g.replay()
        ops.int8_gemm_dequant(x, W, act, ws, b, out=ref)   # eager work between replays
        torch.cuda.synchronize()
        equal.append(all(bool(torch.equal(y.view(torch.int16), ref.view(torch.int16))) for y in outs))
    print(json.dumps({"eager": list(eager), "used0": used0, "total": total, "recorded": recorded,
                      "after": after, "equal": equal}))


def noalloc():
    """forge_int8_linear_noalloc captured before forge_init is rejected (FORGE_EINVAL: the
    array's address cannot be resolved inside a capture); after forge_init two calls of
    different shapes captured into one graph replay to the bits of eager forge_int8_linear."""
    import ctypes
    import torch
    from forge_amd import _lib, ops
    from helpers import fp16_normal, int8_uniform
    dev = torch.device("cuda:0")
    lib = _lib.load()
    rng = np.random.default_rng(9)
    shapes = [(512, 2048, 768), (33, 1024, 264)]   # the second smaller than the first
    ins = []
    for M, K, N in shapes:
        x = torch.from_numpy(fp16_normal(rng, (M, K))).to(dev)
        w = torch.from_numpy(int8_uniform(rng, (N, K))).to(dev)
        ws = torch.from_numpy(rng.uniform(1e-3, 1e-2, N).astype(np.float16)).to(dev)
        b = torch.from_numpy(fp16_normal(rng, (N,), 0.1)).to(dev)
        ins.append((M, K, N, x, w, ws, b))
    refs = []
    for M, K, N, x, w, ws, b in ins:
        q = torch.empty((M, K), dtype=torch.int8, device=dev)
        s = torch.empty((M,), dtype=torch.float32, device=dev)
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        ops.int8_linear(x, w, ws, b, q, s, out=y)
        refs.append(y)
    torch.cuda.synchronize()

    def call(M, K, N, x, w, ws, b, y):
        stream = torch.cuda.current_stream().cuda_stream
        return lib.forge_int8_linear_noalloc(x.data_ptr(), w.data_ptr(), ws.data_ptr(), b.data_ptr(),
                                             y.data_ptr(), M, K, N, ctypes.c_void_p(stream))

    M, K, N, x, w, ws, b = ins[0]
    y0 = torch.empty((M, N), dtype=torch.float16, device=dev)
    _, before_init = _capture(torch, lambda: call(M, K, N, x, w, ws, b, y0))
    init = lib.forge_init()
    outs = [torch.full((M, N), float("nan"), dtype=torch.float16, device=dev) for (M, K, N, *_r) in ins]
    statuses = []
    g, _ = _capture(torch, lambda: statuses.extend(call(*a[:7], y) for a, y in zip(ins, outs)))
    equal = []
    for rep in range(3):
        g.replay()
        for (M, K, N, x, w, ws, b), r in zip(ins, refs):   # eager work between replays
            q = torch.empty((M, K), dtype=torch.int8, device=dev)
            s = torch.empty((M,), dtype=torch.float32, device=dev)
            ops.int8_linear(x, w, ws, b, q, s, out=r)
        torch.cuda.synchronize()
        equal.append([bool(torch.equal(y.view(torch.int16), r.view(torch.int16))) for y, r in zip(outs, refs)])
    print(json.dumps({"before_init": before_init, "init": init, "statuses": statuses, "equal": equal,
                      "EINVAL": _lib.FORGE_EINVAL, "OK": _lib.FORGE_OK}))


if __name__ == "__main__":
    {"slots": slots, "noalloc": noalloc}[sys.argv[1]]()
