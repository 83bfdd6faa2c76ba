"""GPU: the PyTorch modules (reference python/forge/nn/linear.py:115-254) against the oracle.

QuantizedLinear / SparseLinear: weight quantization formula, forward bit-exact to the oracle's
composition (per-token quantize -> INT32 GEMM on the (pruned) weights -> dequant epilogue),
state_dict round trip, QuantizedLinear's backward (input and bias gradients through the
dequantized FP16 weight), and the w_meta conversion to and from the reference's row-major words
(oracle pack_metadata_ref, pack_metadata.cu:23-29)."""
import numpy as np
import pytest

from helpers import fp16_normal, say, to_dev, to_host

pytestmark = pytest.mark.gpu


def _np_weight_quant(w32):
    """The oracle's restatement of linear.py:168-173 (pinned to the reference's torch
    expression in test_oracle.py)."""
    from oracle import oracle
    q, s16, _ = oracle.quantize_weight_rows(w32)
    return q, s16


@pytest.mark.parametrize("M,K,N,bias", [(7, 256, 96, True), (64, 1024, 320, False), (300, 512, 200, True)])
def test_quantized_linear(dev, orc, M, K, N, bias):
    import torch
    from forge_amd.nn import QuantizedLinear
    rng = np.random.default_rng(M + K + N)
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    x = fp16_normal(rng, (M, K))
    say(f"QuantizedLinear M={M} K={K} N={N}")
    m = QuantizedLinear(K, N, bias=bias).to(dev)
    m.quantize_weight(torch.from_numpy(w).to(dev))
    q, s = _np_weight_quant(w)
    assert np.array_equal(to_host(m.w_int8), q)
    assert np.array_equal(to_host(m.w_scale).view(np.uint16), s.view(np.uint16))
    b = None
    if bias:
        b = (rng.standard_normal(N) * 0.1).astype(np.float16)
        m.bias.data.copy_(torch.from_numpy(b).to(dev))
    y = to_host(m(to_dev(x, dev)))
    ref, _, _ = orc.linear(x, q, s, b)
    assert np.array_equal(y.view(np.uint16), ref.view(np.uint16))
    # state_dict round trip into a fresh module
    m2 = QuantizedLinear(K, N, bias=bias).to(dev)
    m2.load_state_dict(m.state_dict())
    assert np.array_equal(to_host(m2(to_dev(x, dev))).view(np.uint16), ref.view(np.uint16))


def test_quantized_linear_backward(dev):
    import torch
    from forge_amd.nn import QuantizedLinear
    rng = np.random.default_rng(5)
    M, K, N = 32, 256, 64
    m = QuantizedLinear(K, N).to(dev)
    m.quantize_weight(torch.from_numpy((rng.standard_normal((N, K)) * 0.05).astype(np.float32)).to(dev))
    x = to_dev(fp16_normal(rng, (M, K)), dev).requires_grad_(True)
    say("QuantizedLinear backward")
    y = m(x)
    g = torch.from_numpy(fp16_normal(rng, (M, N))).to(dev)
    y.backward(g)
    w16 = (m.w_int8.float() * m.w_scale.float().unsqueeze(1)).cpu()
    gx_ref = g.float().cpu() @ w16
    assert x.grad.shape == (M, K) and x.grad.dtype == torch.float16
    assert torch.allclose(x.grad.float().cpu(), gx_ref, rtol=2e-2, atol=2e-2)
    assert torch.allclose(m.bias.grad.float().cpu(), g.float().sum(0).cpu(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("M,K,N,bias", [(5, 256, 64, True), (200, 1280, 320, True), (129, 512, 96, False)])
def test_sparse_linear(dev, orc, M, K, N, bias):
    import torch
    from forge_amd.nn import SparseLinear
    rng = np.random.default_rng(M * 3 + K + N)
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    x = fp16_normal(rng, (M, K))
    say(f"SparseLinear M={M} K={K} N={N}")
    m = SparseLinear(K, N, bias=bias).to(dev)
    m.from_dense_weight(torch.from_numpy(w).to(dev))
    q, s = _np_weight_quant(w)
    comp, raw = orc.prune_compress_24(q)
    assert np.array_equal(to_host(m.W_comp), comp)
    assert np.array_equal(to_host(m.w_meta).reshape(-1).view(np.uint32),
                          orc.pack_metadata_gfx950(raw, N, K).reshape(-1))
    b = None
    if bias:
        b = (rng.standard_normal(N) * 0.1).astype(np.float16)
        m.bias.data.copy_(torch.from_numpy(b).to(dev))
    y = to_host(m(to_dev(x, dev)))
    qx, sx = orc.quantize_rows(x)
    ref = orc.dequant_epilogue(orc.sparse_gemm_s32(comp, qx, raw, N, K), sx, s, b)
    assert np.array_equal(y.view(np.uint16), ref.view(np.uint16))
    m2 = SparseLinear(K, N, bias=bias).to(dev)
    m2.load_state_dict(m.state_dict())
    assert np.array_equal(to_host(m2(to_dev(x, dev))).view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("N,K", [(16, 64), (48, 1024), (320, 1280)])
def test_w_meta_conversion(dev, orc, N, K):
    import torch
    from forge_amd.nn import w_meta_from_reference, w_meta_to_reference
    rng = np.random.default_rng(N + K)
    q = rng.integers(-127, 128, (N, K)).astype(np.int8)
    _, raw = orc.prune_compress_24(q)
    ref_words = orc.pack_metadata_ref(raw, N, K)                 # reference layout (uint32)
    gfx_words = orc.pack_metadata_gfx950(raw, N, K).reshape(N, K // 32)
    say(f"w_meta conversion N={N} K={K}")
    got = w_meta_from_reference(to_dev(ref_words.view(np.int32), dev))
    assert np.array_equal(to_host(got).view(np.uint32), gfx_words)
    back = w_meta_to_reference(to_dev(gfx_words.view(np.int32), dev))
    assert np.array_equal(to_host(back).view(np.uint32), ref_words)


@pytest.mark.parametrize("M,K,N", [(9, 512, 64), (300, 1280, 320)])
def test_sparse_linear_loads_reference_state_dict(dev, orc, M, K, N):
    """A state_dict laid out as the reference's SparseLinear saves it (w_meta in its row-major
    word order, module version 1) loads into a module on the device and computes the oracle's
    outputs for those weights."""
    import collections
    import torch
    from forge_amd.nn import SparseLinear
    rng = np.random.default_rng(M + 2 * K + N)
    q = rng.integers(-127, 128, (N, K)).astype(np.int8)
    comp, raw = orc.prune_compress_24(q)
    ws = rng.uniform(1e-3, 1e-2, N).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float16)
    sd = collections.OrderedDict()
    sd["W_comp"] = torch.from_numpy(comp)
    sd["w_meta"] = torch.from_numpy(orc.pack_metadata_ref(raw, N, K).view(np.int32).copy())
    sd["w_scale"] = torch.from_numpy(ws)
    sd["bias"] = torch.from_numpy(b)
    sd._metadata = collections.OrderedDict({"": {"version": 1}})
    x = fp16_normal(rng, (M, K))
    say(f"SparseLinear reference state_dict M={M} K={K} N={N}")
    m = SparseLinear(K, N).to(dev)
    m.load_state_dict(sd)
    y = to_host(m(to_dev(x, dev)))
    qx, sx = orc.quantize_rows(x)
    ref = orc.dequant_epilogue(orc.sparse_gemm_s32(comp, qx, raw, N, K), sx, ws, b)
    assert np.array_equal(y.view(np.uint16), ref.view(np.uint16))
