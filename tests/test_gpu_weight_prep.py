"""GPU parity: weight preparation (python/forge/nn/linear.py:168-173, :231-249) on the device.

forge_quantize_weight_rows (QuantizedLinear.quantize_weight) and forge_prepare_sparse_weight
(SparseLinear.from_dense_weight: quantize + 2:4 prune + compress + gfx950 pack in one pass) are
compared bit-for-bit with the oracle (whose weight quantization is pinned to the reference's own
torch expression), for fp32 and fp16 weights, odd shapes, ragged 16-row blocks of the packed
index words, and the configs[2] weight (11008 x 4096); at that size also against the library's
separate prune_compress_24 + pack_metadata launches (the reference's two-step sequence)."""
import numpy as np
import pytest

from helpers import say, to_dev, to_host

pytestmark = pytest.mark.gpu


def _weights(rng, N, K, f16):
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    w[:, rng.choice(K, min(4, K), replace=False)] *= 30
    return w.astype(np.float16) if f16 else w


@pytest.mark.parametrize("N,K,f16", [(64, 256, False), (33, 100, False), (7, 4097, True), (128, 1024, True),
                                     (11, 4096, False), (9, 4112, True), (5, 48, True)])
def test_quantize_weight_rows(dev, orc, N, K, f16):
    from forge_amd import ops
    rng = np.random.default_rng(N * 7 + K)
    w = _weights(rng, N, K, f16)
    q, s16, _ = orc.quantize_weight_rows(w.astype(np.float32))
    say(f"quantize_weight_rows N={N} K={K} fp16={f16}")
    gq, gs = ops.quantize_weight_rows(to_dev(w, dev))
    assert np.array_equal(to_host(gq), q)
    assert np.array_equal(to_host(gs).view(np.uint16), s16.view(np.uint16))


@pytest.mark.parametrize("N,K,f16", [(48, 256, False), (16, 64, True), (37, 1280, False), (5, 8192, True),
                                     (300, 96, False), (3, 16384, False), (2, 8256, True), (256, 1024, False),
                                     (1152, 4096, True)])
def test_prepare_sparse_weight(dev, orc, N, K, f16):
    from forge_amd import ops
    rng = np.random.default_rng(N * 5 + K)
    w = _weights(rng, N, K, f16)
    comp, meta, s16 = orc.prepare_sparse_weight(w.astype(np.float32))
    say(f"prepare_sparse_weight N={N} K={K} fp16={f16}")
    gc, gm, gs = ops.prepare_sparse_weight(to_dev(w, dev))
    assert np.array_equal(to_host(gc), comp)
    assert np.array_equal(to_host(gm).reshape(-1).view(np.uint32), meta)
    assert np.array_equal(to_host(gs).view(np.uint16), s16.view(np.uint16))


def test_prepare_sparse_weight_full_size(dev):
    """configs[2]'s weight shape: the one-pass prep equals quantize_weight_rows followed by the
    separate prune_compress_24 and pack_metadata launches."""
    import torch
    from forge_amd import ops
    N, K = 11008, 4096
    g = torch.Generator(device=dev)
    g.manual_seed(9)
    w = torch.randn((N, K), generator=g, device=dev) * 0.02
    say("prepare_sparse_weight 11008x4096")
    gc, gm, gs = ops.prepare_sparse_weight(w)
    q, s = ops.quantize_weight_rows(w)
    comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
    raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
    meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
    ops.prune_compress_24(q, comp, raw, N, K)
    ops.pack_metadata(raw, meta, N, K)
    torch.cuda.synchronize()
    assert torch.equal(gc, comp)
    assert torch.equal(gm.reshape(-1), meta)
    assert torch.equal(gs.view(torch.int16), s.view(torch.int16))
