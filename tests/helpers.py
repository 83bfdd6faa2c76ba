"""Shared helpers for the GPU parity tests (host<->device copies, fp16 ulp distance)."""
import sys

import numpy as np


def say(*a):
    """Names the case before a GPU step (flushed, so a fault still leaves the name)."""
    print(*a, flush=True)
    sys.stdout.flush()


def to_dev(a: np.ndarray, dev):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.float16)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a).to(dev)


def to_host(t) -> np.ndarray:
    import torch
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def ulp_diff16(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a).view(np.uint16).astype(np.int32)
    b = np.ascontiguousarray(b).view(np.uint16).astype(np.int32)
    a = np.where(a & 0x8000, 0x8000 - (a & 0x7FFF), 0x8000 + a)
    b = np.where(b & 0x8000, 0x8000 - (b & 0x7FFF), 0x8000 + b)
    return np.abs(a - b)


def int8_uniform(rng, shape):
    return rng.integers(-127, 128, size=shape, dtype=np.int64).astype(np.int8)


def fp16_normal(rng, shape, scale=1.0):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float16)


def poison(t, byte: int):
    """Fills a device tensor's bytes with a garbage pattern (the reference tests use 0x7B/0x5A)."""
    import torch
    t.view(torch.uint8).fill_(byte)


def special_fp16_rows(rng, M, K, inf=True):
    """fp16 rows for the quantizers' edge cases (bit patterns): NaNs with various payloads
    (quiet, the signalling pattern, negative, all ones) among normal values, a row of NaNs, a
    NaN where the row's largest magnitude would be, a row of subnormals with +-0, a row of
    -0, exact ties after scaling (absmax 127 makes the scale 1: 2.5 -> 2, 3.5 -> 4, ...), the
    fp16 maximum, and optionally +inf and -inf rows (scale inf, every value quantized to 0).
    Special rows sit at the start and at the end of the matrix."""
    x = (rng.standard_normal((M, K), dtype=np.float32)).astype(np.float16).view(np.uint16).copy()
    nan_bits = np.array([0x7E00, 0x7C01, 0xFE00, 0x7D55, 0xFFFF], np.uint16)

    def r(i):
        return i % M if i >= 0 else (M + i) % M

    n = min(K, 7)
    x[r(0), rng.choice(K, n, replace=False)] = rng.choice(nan_bits, n)
    x[r(1)] = rng.choice(np.array([0x0001, 0x8001, 0x03FF, 0x83FF, 0x0200, 0x8000, 0x0000], np.uint16), K)
    x[r(2)] = 0x8000
    ties = np.array([127.0, 2.5, 3.5, -2.5, 0.5, -0.5, 1.5, -126.5], np.float16).view(np.uint16)
    x[r(3)] = 0
    x[r(3), :min(K, 8)] = ties[:min(K, 8)]
    x[r(4)] = np.float16(65504).view(np.uint16)
    x[r(4), ::3] = np.float16(-65504).view(np.uint16)
    big = int(np.argmax(np.abs(x[r(5)].view(np.float16).astype(np.float32))))
    x[r(5), big] = 0x7E00
    x[r(-1)] = 0x7E00
    x[r(-2), rng.choice(K, n, replace=False)] = rng.choice(nan_bits, n)
    if inf:
        x[r(6), K // 2] = 0x7C00
        x[r(-3), 0] = 0xFC00
    return x.view(np.float16)
