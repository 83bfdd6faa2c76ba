"""Writes the golden fixtures under tests/golden/ (inputs + expected outputs).

Expected outputs are computed here with library routines independent of the oracle
(numpy int64 matmul, numpy IEEE float32 arithmetic and rint, torch float64 conv2d,
a brute-force key formulation of the 2:4 selection), so a test comparing the oracle
or the GPU against these files checks them against an independent derivation.

Inputs:
  c1_gemm      configs[0] of BASELINE.json: A (128,512), B (256,512) int8 in [-127,127]
  quantize     hand-built rows: zero row, one nonzero, exact .5 ties at scale 1.0 and 2.0,
               outlier columns, random N(0,1) rows (fp16)
  prune        tie-heavy int8 groups including -128 / 127
  pack         the reference test's own input: std::mt19937(42), rng() & 0xF, N=16, K=128
               (tests/test_pack_metadata.cu:118-126 of the reference)
  dequant      the reference test's ranges (tests/test_dequantize.cu:13-31)
  conv         NHWC int8 convolutions with padding, stride and dilation
  sparse       pruned weights x activations (INT32)

Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def mt19937(seed: int, count: int) -> np.ndarray:
    """MT19937 (Matsumoto & Nishimura) with std::mt19937's seeding (init_genrand)."""
    mt = [0] * 624
    mt[0] = seed & 0xFFFFFFFF
    for i in range(1, 624):
        mt[i] = (1812433253 * (mt[i - 1] ^ (mt[i - 1] >> 30)) + i) & 0xFFFFFFFF
    out, idx = [], 624
    for _ in range(count):
        if idx >= 624:
            for i in range(624):
                y = (mt[i] & 0x80000000) | (mt[(i + 1) % 624] & 0x7FFFFFFF)
                mt[i] = mt[(i + 397) % 624] ^ (y >> 1) ^ (0x9908B0DF if y & 1 else 0)
            idx = 0
        y = mt[idx]
        idx += 1
        y ^= y >> 11
        y ^= (y << 7) & 0x9D2C5680
        y ^= (y << 15) & 0xEFC60000
        y ^= y >> 18
        out.append(y & 0xFFFFFFFF)
    return np.array(out, dtype=np.uint32)


def int8_uniform(rng: np.random.Generator, shape) -> np.ndarray:
    return rng.integers(-127, 128, size=shape, dtype=np.int64).astype(np.int8)


def quantize_np(x16: np.ndarray):
    """IEEE float32 per-row quantization with numpy scalar/array float32 operations."""
    x = x16.astype(np.float32)
    amax = np.max(np.abs(x), axis=1).astype(np.float32)
    scale = (np.maximum(amax, np.float32(1e-8)) / np.float32(127.0)).astype(np.float32)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    v = (x * inv[:, None]).astype(np.float32)
    q = np.clip(np.rint(v), -128, 127).astype(np.int8)
    return q, scale


def prune_keys(w: np.ndarray):
    """Keep the two largest (|v|, index) keys of every group of 4 along K."""
    N, K = w.shape
    comp = np.empty((N, K // 2), np.int8)
    nib = np.empty((N, K // 4), np.uint8)
    for n in range(N):
        for g in range(K // 4):
            v = [int(t) for t in w[n, 4 * g: 4 * g + 4]]
            order = sorted(range(4), key=lambda i: (abs(v[i]), i))
            keep = sorted(order[2:])
            comp[n, 2 * g] = v[keep[0]]
            comp[n, 2 * g + 1] = v[keep[1]]
            nib[n, g] = keep[0] | (keep[1] << 2)
    return comp, nib.ravel()


def pack_ref_np(nib: np.ndarray, N: int, K: int) -> np.ndarray:
    n = nib.reshape(N, K // 32, 8).astype(np.uint32) & 0xF
    return np.bitwise_or.reduce(n << (4 * np.arange(8, dtype=np.uint32)), axis=2).astype(np.uint32)


def pack_gfx950_np(words: np.ndarray, N: int, K: int) -> np.ndarray:
    cpr = K // 32
    out = np.empty(N * cpr, np.uint32)
    for n in range(N):
        blk = n // 16
        rows = min(16, N - 16 * blk)
        for c in range(cpr):
            out[blk * cpr * 16 + c * rows + n % 16] = words[n, c]
    return out


def main() -> None:
    rng = np.random.default_rng(20261201)

    # --- c1 GEMM ---------------------------------------------------
    A = int8_uniform(np.random.default_rng(1), (128, 512))
    B = int8_uniform(np.random.default_rng(2), (256, 512))
    C = (A.astype(np.int64) @ B.astype(np.int64).T).astype(np.int32)
    np.savez_compressed(os.path.join(HERE, "c1_gemm.npz"), A=A, B=B, C=C)

    # --- quantize -----------------------------------------------------------------
    K = 40
    rows = []
    rows.append(np.zeros(K, np.float32))                                  # all zero
    r = np.zeros(K, np.float32); r[7] = -3.25; rows.append(r)             # single nonzero
    r = np.zeros(K, np.float32); r[:8] = [127, 2.5, 3.5, -2.5, 0.5, 1.5, -0.5, 126.5]; rows.append(r)  # scale 1.0
    r = np.zeros(K, np.float32); r[:6] = [254, 5, 7, -5, 1, 3]; rows.append(r)                  # scale 2.0
    r = rng.standard_normal(K).astype(np.float32); r[[3, 17]] *= 20; rows.append(r)              # outliers
    for _ in range(3):
        rows.append(rng.standard_normal(K).astype(np.float32))
    r = np.full(K, 1e-9, np.float32); rows.append(r)                      # below the 1e-8 floor (fp16: 0)
    r = (rng.standard_normal(K) * 60000).clip(-65504, 65504).astype(np.float32); rows.append(r)  # fp16 range
    X = np.stack(rows).astype(np.float16)
    q, s = quantize_np(X)
    np.savez_compressed(os.path.join(HERE, "quantize.npz"), X=X, q=q, scales=s)

    # --- prune ----------------------------------------------------------------------
    Wp = rng.integers(-3, 4, size=(16, 64)).astype(np.int8)
    Wp[0, :4] = [5, 5, 5, 5]
    Wp[0, 4:8] = [0, 0, 0, 0]
    Wp[1, :4] = [-128, 127, -127, 1]
    Wp[1, 4:8] = [1, -5, 3, 0]
    Wp[2, :8] = [-128, -128, 127, 127, 2, -2, 2, -2]
    comp, nib = prune_keys(Wp)
    np.savez_compressed(os.path.join(HERE, "prune.npz"), W=Wp, comp=comp, nibbles=nib)

    # --- pack (the reference test's input vectors) ------------------------------------
    Np, Kp = 16, 128
    raw = (mt19937(42, Np * Kp // 4) & 0xF).astype(np.uint8)
    words = pack_ref_np(raw, Np, Kp)
    # a ragged N for the gfx950 layout as well
    Nr, Kr = 20, 96
    raw_r = (mt19937(7, Nr * Kr // 4) & 0xF).astype(np.uint8)
    words_r = pack_ref_np(raw_r, Nr, Kr)
    np.savez_compressed(os.path.join(HERE, "pack.npz"), raw=raw, words=words,
                        gfx950=pack_gfx950_np(words, Np, Kp), raw_ragged=raw_r,
                        words_ragged=words_r, gfx950_ragged=pack_gfx950_np(words_r, Nr, Kr),
                        mt19937_5489_10000=mt19937(5489, 10000)[-1:])

    # --- dequant ----------------------------------------------------------------------
    M, N = 16, 64
    acc = rng.integers(-50000, 50001, size=(M, N)).astype(np.int32)
    act = rng.uniform(0.001, 0.1, M).astype(np.float32)
    ws = rng.uniform(0.001, 0.1, N).astype(np.float16)
    bias = rng.uniform(-0.5, 0.5, N).astype(np.float16)
    a64 = acc.astype(np.float64)
    # standalone dequant ((acc*as)*ws + b) and GEMM epilogue (acc*(as*ws) + b), in float64
    deq = ((a64 * act[:, None].astype(np.float64)) * ws.astype(np.float64) + bias.astype(np.float64)).astype(np.float16)
    s32 = (act[:, None] * ws.astype(np.float32)[None, :]).astype(np.float32)
    epi = (a64 * s32.astype(np.float64) + bias.astype(np.float64)).astype(np.float16)
    np.savez_compressed(os.path.join(HERE, "dequant.npz"), acc=acc, act_scale=act, w_scale=ws, bias=bias,
                        out_standalone=deq, out_epilogue=epi)

    # --- conv (torch float64 conv2d; exact for these integer sums) ---------------------
    import torch
    cases = {}
    for name, (n, h, w, c, co, k, pad, stride, dil) in {
        "3x3_p1": (2, 7, 7, 16, 8, 3, 1, 1, 1),
        "2x2_s2": (1, 8, 8, 32, 16, 2, 0, 2, 1),
        "3x3_d2": (1, 9, 9, 16, 8, 3, 2, 1, 2),
    }.items():
        x = int8_uniform(rng, (n, h, w, c))
        wt = int8_uniform(rng, (co, k, k, c))
        ref = torch.nn.functional.conv2d(torch.from_numpy(x).permute(0, 3, 1, 2).double(),
                                         torch.from_numpy(wt).permute(0, 3, 1, 2).double(),
                                         stride=stride, padding=pad, dilation=dil)
        cases[name + "_x"] = x
        cases[name + "_w"] = wt
        cases[name + "_cfg"] = np.array([pad, stride, dil], np.int32)
        cases[name + "_out"] = ref.permute(0, 2, 3, 1).numpy().astype(np.int32)
    np.savez_compressed(os.path.join(HERE, "conv.npz"), **cases)

    # --- sparse ------------------------------------------------------------------------
    Ws = int8_uniform(rng, (32, 128))
    comp_s, nib_s = prune_keys(Ws)
    keep = np.zeros_like(Ws)
    nb = nib_s.reshape(32, 32)
    for n in range(32):
        for g in range(32):
            keep[n, 4 * g + (nb[n, g] & 3)] = 1
            keep[n, 4 * g + (nb[n, g] >> 2)] = 1
    Wpr = (Ws * keep).astype(np.int8)
    xs = int8_uniform(rng, (8, 128))
    Cs = (xs.astype(np.int64) @ Wpr.astype(np.int64).T).astype(np.int32)
    np.savez_compressed(os.path.join(HERE, "sparse.npz"), W=Ws, comp=comp_s, nibbles=nib_s, x=xs, C=Cs)


if __name__ == "__main__":
    main()
