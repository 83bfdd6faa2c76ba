"""GPU parity: per-token quantization and standalone dequantization vs the oracle.

Bar: INT8 outputs and FP32 scales bit-exact; the single-pass (one wavefront per row)
and exported two-pass kernels bit-identical, as the reference requires
(tests/test_quantize.cu:82-84, :96); FP16 dequant bit-exact to the oracle's association
and within 1 ulp of the float64 golden value."""
import numpy as np
import pytest

from conftest import golden
from helpers import fp16_normal, poison, say, special_fp16_rows, to_dev, to_host, ulp_diff16

pytestmark = pytest.mark.gpu

# tests/test_quantize.cu:103-113: vector path VPT 1..4, K > 8192, K % 8 != 0, misaligned,
# and an input larger than L2.
# The last four (M >= 2048, K <= 2048) run the wave-per-row kernel (1, 2 and 4 vectors per lane,
# a ragged last workgroup).
REF_CASES = [(32, 256, 0), (7, 8, 0), (64, 2056, 0), (16, 6144, 0), (16, 8192, 0), (5, 8200, 0),
             (9, 100, 0), (9, 256, 1), (8192, 5120, 0),
             (2048, 1280, 0), (3001, 2048, 0), (2050, 8, 0), (4096, 1000, 0)]


@pytest.mark.parametrize("M,K,offset", REF_CASES)
def test_quantize_reference_cases(dev, orc, M, K, offset):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(42 + M + K)
    x = rng.uniform(-3.0, 3.0, (M, K)).astype(np.float16)
    qr, sr = orc.quantize_rows(x)
    say(f"quantize M={M} K={K} offset={offset}")
    buf = torch.empty(M * K + offset, dtype=torch.float16, device=dev)
    buf[offset:] = to_dev(x.ravel(), dev)
    xin = buf[offset:]
    q, s = ops.fused_quantize_activation(xin, M, K)
    threads = min(256, (K + 31) // 32 * 32)
    q2, s2 = ops.fused_quantize_activation_twopass(xin, M, K, threads)
    q, s, q2, s2 = to_host(q), to_host(s), to_host(q2), to_host(s2)
    assert np.array_equal(s.view(np.uint32), sr.view(np.uint32))
    assert np.array_equal(q, qr)
    assert np.array_equal(q, q2) and np.array_equal(s.view(np.uint32), s2.view(np.uint32))


def test_quantize_golden(dev):
    from forge_amd import ops
    g = golden("quantize")
    M, K = g["X"].shape
    say("quantize golden")
    q, s = ops.fused_quantize_activation(to_dev(g["X"], dev), M, K)
    assert np.array_equal(to_host(s).view(np.uint32), g["scales"].view(np.uint32))
    assert np.array_equal(to_host(q), g["q"])


@pytest.mark.parametrize("threads", [1, 32, 64, 100, 256, 1024])
def test_twopass_any_block_size(dev, orc, threads):
    from forge_amd import ops
    rng = np.random.default_rng(threads)
    M, K = 13, 777
    x = fp16_normal(rng, (M, K), 4.0)
    qr, sr = orc.quantize_rows(x)
    say(f"twopass threads={threads}")
    q, s = ops.fused_quantize_activation_twopass(to_dev(x, dev), M, K, threads)
    assert np.array_equal(to_host(q), qr) and np.array_equal(to_host(s), sr)


def test_quantize_outlier_rows_and_ties(dev, orc):
    """configs[1]'s activation statistics (N(0,1), 8 outlier channels x20) at a small M."""
    from forge_amd import ops
    rng = np.random.default_rng(7)
    M, K = 64, 4096
    x = rng.standard_normal((M, K), dtype=np.float32)
    x[:, rng.choice(K, 8, replace=False)] *= 20
    x = x.astype(np.float16)
    x[3] = 0
    x[4, :] = 0
    x[4, :5] = [127, 2.5, 3.5, -2.5, 0.5]
    qr, sr = orc.quantize_rows(x)
    say("quantize outliers/ties")
    q, s = ops.fused_quantize_activation(to_dev(x, dev), M, K)
    assert np.array_equal(to_host(q), qr) and np.array_equal(to_host(s), sr)


# Shapes reaching each kernel: block kernel VPT 1 / 2 / 8, wave kernel VPT 1 / 2 / 4 (ragged
# last workgroup at 2050 rows), and the scalar kernel (K % 8 != 0).
SPECIAL_CASES = [(9, 1024), (16, 4096), (4, 16384), (2050, 8), (2048, 1000), (2051, 2048), (6, 1003),
                 (2049, 3072), (2048, 4096)]   # wave-per-row kernel with 6 and 8 vectors per lane


@pytest.mark.parametrize("M,K", SPECIAL_CASES)
def test_quantize_special_values(dev, orc, M, K):
    """NaN payloads, a NaN at the largest magnitude, NaN-only rows, subnormals, +-0, ties after
    scaling, the fp16 maximum and +-inf rows: INT8 and scales bit-exact against the oracle
    (which follows the reference's fmaxf, skipping NaN, and its NaN -> 0 conversion), for the
    main kernels and the exported two-pass kernel."""
    from forge_amd import ops
    rng = np.random.default_rng(M * 7 + K)
    x = special_fp16_rows(rng, M, K)
    qr, sr = orc.quantize_rows(x)
    say(f"quantize special values M={M} K={K}")
    q, s = ops.fused_quantize_activation(to_dev(x, dev), M, K)
    assert np.array_equal(to_host(s).view(np.uint32), sr.view(np.uint32))
    assert np.array_equal(to_host(q), qr)
    q2, s2 = ops.fused_quantize_activation_twopass(to_dev(x, dev), M, K, 256)
    assert np.array_equal(to_host(s2).view(np.uint32), sr.view(np.uint32))
    assert np.array_equal(to_host(q2), qr)


def test_dequant_golden(dev, orc):
    from forge_amd import ops
    g = golden("dequant")
    M, N = g["acc"].shape
    say("dequant golden")
    out = to_host(ops.fused_dequantize_bias(to_dev(g["acc"], dev), to_dev(g["act_scale"], dev),
                                            to_dev(g["w_scale"], dev), to_dev(g["bias"], dev), M, N))
    assert ulp_diff16(out, g["out_standalone"]).max() <= 1
    ref = orc.dequantize_bias(g["acc"], g["act_scale"], g["w_scale"], g["bias"])
    assert np.array_equal(out.view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("M,N,bias", [(16, 64, True), (16, 64, False), (33, 63, True), (5, 1000, False),
                                      (257, 4100, True)])
def test_dequant_random(dev, orc, M, N, bias):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M * N)
    acc = rng.integers(-50000, 50001, (M, N)).astype(np.int32)
    act = rng.uniform(0.001, 0.1, M).astype(np.float32)
    ws = rng.uniform(0.001, 0.1, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16) if bias else None
    ref = orc.dequantize_bias(acc, act, ws, b)
    say(f"dequant M={M} N={N} bias={bias}")
    out = ops.fused_dequantize_bias(to_dev(acc, dev), to_dev(act, dev), to_dev(ws, dev),
                                    None if b is None else to_dev(b, dev), M, N)
    assert np.array_equal(to_host(out).view(np.uint16), ref.view(np.uint16))
