"""GPU parity: the fused quantize + 2:4 sparse linear path (the reference's FQ path,
src/gemm/int8_sparse.cu:250-335, chosen at :1022-1033).

Forced (path 1) over every weight-blocks-per-wave variant (N = 16 .. 528, including a second
pass with a partial block set), ragged token counts and K from 128 to the 2048 limit (2, 3 and 4
row vectors per producer lane, each at its largest K and below), each
bit-exact against the oracle's two-pass composition (quantize rows -> sparse INT32 GEMM ->
dequant epilogue) and against the library's own two-pass path; the scratch buffers stay
untouched, as the reference documents (int8_sparse.cuh:87-89), with the weights packed into
fragment order in the library's own slot or, beyond a slot, read in place; and the automatic choice takes
the fused kernel for the reference's own example layer (1280 -> 320 at M = 147,456), where its
output equals the two-pass output bit for bit."""
import numpy as np
import pytest

from helpers import int8_uniform, say, special_fp16_rows, to_dev, to_host

pytestmark = pytest.mark.gpu


def _prep(dev, W):
    import torch
    from forge_amd import ops
    N, K = W.shape
    comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
    raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
    meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
    ops.prune_compress_24(to_dev(W, dev), comp, raw, N, K)
    ops.pack_metadata(raw, meta, N, K)
    return comp, meta


@pytest.mark.parametrize("M,K,N,bias", [(65, 128, 16, True), (1, 512, 96, True), (200, 1280, 176, False),
                                        (130, 2048, 256, True), (97, 384, 384, True), (257, 256, 528, True),
                                        (64, 1280, 320, True), (129, 1152, 64, True), (70, 1536, 112, False)])
def test_fq_forced_parity(dev, orc, M, K, N, bias):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M * 3 + K + N)
    W = int8_uniform(rng, (N, K))
    x = rng.uniform(-2.0, 2.0, (M, K)).astype(np.float16)
    x[:, rng.choice(K, 2, replace=False)] *= 8
    ws = rng.uniform(0.001, 0.05, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16) if bias else None
    cr, mr = orc.prune_compress_24(W)
    qr, sr = orc.quantize_rows(x)
    ref = orc.dequant_epilogue(orc.sparse_gemm_s32(cr, qr, mr, N, K), sr, ws, b).view(np.uint16)
    comp, meta = _prep(dev, W)
    xd, wsd = to_dev(x, dev), to_dev(ws, dev)
    bd = None if b is None else to_dev(b, dev)
    sq = torch.empty((M, K), dtype=torch.int8, device=dev)
    ss = torch.empty((M,), dtype=torch.float32, device=dev)
    sq.fill_(0x5A)
    ss.view(torch.int32).fill_(0x5A5A5A5A)
    say(f"fused sparse linear M={M} K={K} N={N} bias={bias}")
    y = ops.sparse_int8_linear(xd, comp, meta, wsd, bd, sq, ss, None, 1, 1)
    assert ops.last_route() in ("fused-quantize packed", "decode+quantize")
    assert np.array_equal(to_host(y).view(np.uint16), ref)
    # the scratch buffers are not touched on the fused path
    assert bool((sq == 0x5A).all()) and bool((ss.view(torch.int32) == 0x5A5A5A5A).all())
    y2 = ops.sparse_int8_linear(xd, comp, meta, wsd, bd, sq, ss, None, 1, 0)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))


def test_fq_weights_in_place(dev, orc):
    """Weights beyond a packed-weight slot (N * K / 2 > 1 MiB: 1040 x 2048) are read from W_comp
    in place, with several passes of weight blocks per consumer wave: bit-exact against the
    oracle and the two-pass path, scratch untouched."""
    import torch
    from forge_amd import ops
    M, K, N = 100, 2048, 1040
    rng = np.random.default_rng(1040)
    W = int8_uniform(rng, (N, K))
    x = rng.uniform(-2.0, 2.0, (M, K)).astype(np.float16)
    ws = rng.uniform(0.001, 0.05, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16)
    cr, mr = orc.prune_compress_24(W)
    qr, sr = orc.quantize_rows(x)
    ref = orc.dequant_epilogue(orc.sparse_gemm_s32(cr, qr, mr, N, K), sr, ws, b).view(np.uint16)
    comp, meta = _prep(dev, W)
    xd, wsd, bd = to_dev(x, dev), to_dev(ws, dev), to_dev(b, dev)
    sq = torch.full((M, K), 0x5A, dtype=torch.int8, device=dev)
    ss = torch.empty((M,), dtype=torch.float32, device=dev)
    ss.view(torch.int32).fill_(0x5A5A5A5A)
    say(f"fused sparse linear, weights in place M={M} K={K} N={N}")
    y = ops.sparse_int8_linear(xd, comp, meta, wsd, bd, sq, ss, None, 1, 1)
    assert ops.last_route() == "fused-quantize"
    assert np.array_equal(to_host(y).view(np.uint16), ref)
    assert bool((sq == 0x5A).all()) and bool((ss.view(torch.int32) == 0x5A5A5A5A).all())
    y2 = ops.sparse_int8_linear(xd, comp, meta, wsd, bd, sq, ss, None, 1, 0)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))


def test_fq_output_8_byte_aligned(dev, orc):
    """An output 8 but not 16 bytes aligned (a view 4 halves into a buffer) takes the per-lane
    stores instead of the LDS-staged 16-byte row runs: bit-exact against the oracle, and the
    halves around the view untouched."""
    import torch
    from forge_amd import ops
    M, K, N = 150, 1280, 320
    rng = np.random.default_rng(808)
    W = int8_uniform(rng, (N, K))
    x = rng.uniform(-2.0, 2.0, (M, K)).astype(np.float16)
    ws = rng.uniform(0.001, 0.05, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16)
    cr, mr = orc.prune_compress_24(W)
    qr, sr = orc.quantize_rows(x)
    ref = orc.dequant_epilogue(orc.sparse_gemm_s32(cr, qr, mr, N, K), sr, ws, b).view(np.uint16)
    comp, meta = _prep(dev, W)
    sq = torch.empty((M, K), dtype=torch.int8, device=dev)
    ss = torch.empty((M,), dtype=torch.float32, device=dev)
    buf = torch.full((M * N + 8,), 0x5A5A, dtype=torch.int16, device=dev)
    out = buf[4:4 + M * N].view(torch.float16).view(M, N)
    assert out.data_ptr() % 16 == 8
    say(f"fused sparse linear, 8-byte aligned output M={M} K={K} N={N}")
    ops.sparse_int8_linear(to_dev(x, dev), comp, meta, to_dev(ws, dev), to_dev(b, dev), sq, ss, None, 1, 1, out=out)
    assert ops.last_route().startswith("fused-quantize")
    assert np.array_equal(to_host(out).view(np.uint16), ref)
    h = to_host(buf).view(np.uint16)
    assert (h[:4] == 0x5A5A).all() and (h[4 + M * N:] == 0x5A5A).all()


@pytest.mark.parametrize("M,K,N", [(64, 1280, 320), (101, 512, 96), (48, 2048, 64)])
def test_fq_special_values(dev, orc, M, K, N):
    """The fused kernel's on-chip quantization on NaN payloads (skipped by the absmax, quantized
    to 0), NaN-only rows, subnormals, +-0, ties after scaling and the fp16 maximum: outputs
    bit-exact against the oracle's two-pass composition and the library's two-pass path. (No
    inf rows: their scale is inf and the dequantized outputs NaN, whose sign bit the host
    arithmetic of the oracle need not share.)"""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(M + K + N)
    W = int8_uniform(rng, (N, K))
    x = special_fp16_rows(rng, M, K, inf=False)
    ws = rng.uniform(0.001, 0.05, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16)
    cr, mr = orc.prune_compress_24(W)
    qr, sr = orc.quantize_rows(x)
    ref = orc.dequant_epilogue(orc.sparse_gemm_s32(cr, qr, mr, N, K), sr, ws, b).view(np.uint16)
    comp, meta = _prep(dev, W)
    xd, wsd, bd = to_dev(x, dev), to_dev(ws, dev), to_dev(b, dev)
    sq = torch.empty((M, K), dtype=torch.int8, device=dev)
    ss = torch.empty((M,), dtype=torch.float32, device=dev)
    say(f"fused sparse linear special values M={M} K={K} N={N}")
    y = ops.sparse_int8_linear(xd, comp, meta, wsd, bd, sq, ss, None, 1, 1)
    assert np.array_equal(to_host(y).view(np.uint16), ref)
    y2 = ops.sparse_int8_linear(xd, comp, meta, wsd, bd, sq, ss, None, 1, 0)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))


def test_fq_auto_on_reference_layer(dev, orc):
    """1280 -> 320 at M = 147,456 (int8_sparse.cuh:82): auto takes the fused kernel and its
    output equals the two-pass output; sampled rows against the oracle."""
    import torch
    from forge_amd import ops
    M, K, N = 147456, 1280, 320
    assert ops.sparse_int8_linear_fused(M, K, N)
    assert not ops.sparse_int8_linear_fused(4096, K, N)
    # measured two-pass wins: M*K below 50M, N over 640 at K = 2048, N over 1024
    assert not ops.sparse_int8_linear_fused(65536, 640, 320)
    assert not ops.sparse_int8_linear_fused(M, 2048, 1024)
    assert not ops.sparse_int8_linear_fused(M, 1024, 2048)
    rng = np.random.default_rng(7)
    W = int8_uniform(rng, (N, K))
    comp, meta = _prep(dev, W)
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    xd = torch.randn((M, K), generator=g, device=dev).half()
    wsd = to_dev(rng.uniform(0.001, 0.05, N).astype(np.float16), dev)
    bd = to_dev(rng.uniform(-0.5, 0.5, N).astype(np.float16), dev)
    sq = torch.empty((M, K), dtype=torch.int8, device=dev)
    ss = torch.empty((M,), dtype=torch.float32, device=dev)
    say("fused sparse linear 147456x1280->320 auto vs two-pass")
    y_auto = ops.sparse_int8_linear(xd, comp, meta, wsd, bd, sq, ss, None, 1, -1)
    assert ops.last_route() == "fused-quantize packed"
    y_two = ops.sparse_int8_linear(xd, comp, meta, wsd, bd, sq, ss, None, 1, 0)
    torch.cuda.synchronize()
    assert torch.equal(y_auto.view(torch.int16), y_two.view(torch.int16))
    rows = np.array([0, 63, 64, 70001, M - 1])
    x_rows = to_host(xd[torch.from_numpy(rows).to(dev)])
    cr, mr = orc.prune_compress_24(W)
    qr, sr = orc.quantize_rows(x_rows)
    ref = orc.dequant_epilogue(orc.sparse_gemm_s32(cr, qr, mr, N, K), sr, to_host(wsd), to_host(bd)).view(np.uint16)
    assert np.array_equal(to_host(y_auto)[rows].view(np.uint16), ref)
