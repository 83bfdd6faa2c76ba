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
