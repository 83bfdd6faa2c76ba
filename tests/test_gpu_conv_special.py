"""GPU parity: INT8 depthwise conv2d and ConvTranspose2d (kernel 2, stride 2), NCHW FP16.

Every output is compared bit-for-bit with the oracle (oracle/forge_oracle.c), which restates
src/nn/int8_depthwise_conv2d.cu:25-103 and src/nn/int8_conv_transpose2d.cu:70-191 and is
pinned against torch float64 convolutions in tests/test_oracle.py. The reference test's own
cases (tests/test_int8_special_conv.cu:266-279) are included with its float criterion.
Branches covered: the depthwise rolling-window kernel (every kernel size and padding it
takes, several strips and column waves, ragged and unaligned stores, non-finite taps), the
LDS tile kernel (the other stride-1 shapes; its masked loop for non-finite taps) and the
direct kernel (strides, dilations, wide kernels); the transposed conv's fused single-pass
kernel (partial pixel tiles and column blocks, rows that span image rows) and its two-kernel
path: the pixel quantizer (4-byte and byte rows, LDS stash and re-read), the three GEMM
engines under the scatter epilogue (16-byte groups and element stores), image chunking; and
the full-size shapes."""
import numpy as np
import pytest

from helpers import int8_uniform, say, to_dev, to_host

pytestmark = pytest.mark.gpu


def _bits_equal(got: np.ndarray, want: np.ndarray) -> bool:
    """fp16 bit equality, with any NaN equal to any NaN (payloads are not specified)."""
    g = np.ascontiguousarray(got).view(np.uint16)
    w = np.ascontiguousarray(want).view(np.uint16)
    gn = np.isnan(got.astype(np.float32))
    wn = np.isnan(want.astype(np.float32))
    return bool(np.array_equal(gn, wn) and np.array_equal(g[~gn], w[~wn]))


# ---- depthwise ---------------------------------------------------------------------

def _dw_inputs(rng, N, C, H, W, kH, kW, bias):
    x = rng.uniform(-1, 1, (N, C, H, W)).astype(np.float16)
    w = int8_uniform(rng, (C, kH, kW))
    ws = rng.uniform(0.005, 0.05, C).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, C).astype(np.float16) if bias else None
    return x, w, ws, b


DW_CASES = [
    # N, C, H, W, kH, kW, pad, stride, dil, bias
    (1, 16, 16, 16, 3, 3, (1, 1), (1, 1), (1, 1), True),     # reference test cases
    (1, 32, 32, 32, 3, 3, (1, 1), (1, 1), (1, 1), True),
    (1, 64, 8, 8, 3, 3, (1, 1), (1, 1), (1, 1), False),
    (2, 5, 37, 70, 3, 3, (1, 1), (1, 1), (1, 1), True),      # ragged tiles, element stores
    (1, 3, 64, 128, 5, 5, (2, 2), (1, 1), (1, 1), True),     # full tiles, 16-byte stores
    (2, 4, 40, 33, 7, 1, (3, 0), (1, 1), (1, 1), True),
    (1, 2, 9, 100, 1, 9, (0, 4), (1, 1), (1, 1), False),
    (1, 3, 50, 20, 16, 2, (0, 1), (1, 1), (1, 1), True),     # tallest kernel of the tile path
    (1, 6, 12, 12, 3, 3, (3, 3), (1, 1), (1, 1), True),      # padding wider than the kernel
    (2, 3, 30, 41, 3, 3, (1, 1), (2, 2), (1, 1), True),      # direct kernel: stride
    (1, 4, 25, 26, 3, 3, (2, 2), (1, 1), (2, 2), True),      # direct kernel: dilation
    (1, 2, 20, 30, 3, 11, (1, 5), (1, 1), (1, 1), True),     # direct kernel: kW > 9
    (1, 1, 1, 1, 1, 1, (0, 0), (1, 1), (1, 1), True),
    # rolling-window kernel (W % 8 == 0, square 1/3/5/7, column pad (k-1)/2 or 0)
    (2, 3, 40, 64, 7, 7, (3, 3), (1, 1), (1, 1), True),
    (1, 2, 21, 32, 7, 7, (0, 0), (1, 1), (1, 1), True),     # valid conv, Wo % 8 != 0
    (1, 5, 33, 48, 5, 5, (1, 0), (1, 1), (1, 1), False),    # row pad != column pad
    (3, 4, 17, 16, 1, 1, (0, 0), (1, 1), (1, 1), True),
    (1, 2, 100, 1024, 3, 3, (1, 1), (1, 1), (1, 1), True),  # 3 column waves, many strips
    (1, 3, 9, 24, 3, 3, (2, 0), (1, 1), (1, 1), True),      # row pad 2, column pad 0
    (1, 2, 5, 8, 5, 5, (2, 2), (1, 1), (1, 1), True),       # kernel taller than the image
]


@pytest.mark.parametrize("N,C,H,W,kH,kW,pad,stride,dil,bias", DW_CASES)
def test_depthwise_parity(dev, orc, N, C, H, W, kH, kW, pad, stride, dil, bias):
    from forge_amd import ops
    rng = np.random.default_rng(N * 1000 + C * 10 + kH)
    x, w, ws, b = _dw_inputs(rng, N, C, H, W, kH, kW, bias)
    want = orc.depthwise_conv2d(x, w, ws, b, pad, stride, dil)
    say(f"depthwise N={N} C={C} H={H} W={W} k={kH}x{kW} pad={pad} stride={stride} dil={dil}")
    y = to_host(ops.int8_depthwise_conv2d_forward(to_dev(x, dev), to_dev(w, dev), to_dev(ws, dev),
                                                  None if b is None else to_dev(b, dev), kH, kW, pad, stride, dil))
    assert y.shape == want.shape
    assert _bits_equal(y, want)
    if (C, H, W) in [(16, 16, 16), (32, 32, 32), (64, 8, 8)]:
        # test_int8_special_conv.cu:128-131: max |gpu - float reference| < 0.01
        import torch
        wf = (w.astype(np.float32) * ws.astype(np.float32)[:, None, None]).astype(np.float64)
        ref = torch.nn.functional.conv2d(torch.from_numpy(x.astype(np.float64)), torch.from_numpy(wf)[:, None],
                                         padding=pad, groups=C).numpy()
        if b is not None:
            ref += b.astype(np.float64)[None, :, None, None]
        assert np.abs(y.astype(np.float64) - ref).max() < 0.01


def test_depthwise_nonfinite_tap_skips_padding(dev, orc):
    """A channel whose scale is inf: its taps are +-inf (q != 0) or NaN (q == 0). Out-of-image
    taps must be skipped, not multiplied by a zero pad, so border outputs match the oracle."""
    from forge_amd import ops
    rng = np.random.default_rng(77)
    x, w, ws, b = _dw_inputs(rng, 1, 4, 20, 24, 3, 3, True)
    ws[1] = np.float16(np.inf)
    w[2, 0, 0] = 0
    ws[2] = np.float16(np.inf)
    want = orc.depthwise_conv2d(x, w, ws, b, (1, 1))
    say("depthwise non-finite taps")
    y = to_host(ops.int8_depthwise_conv2d_forward(to_dev(x, dev), to_dev(w, dev), to_dev(ws, dev), to_dev(b, dev),
                                                  3, 3, (1, 1)))
    assert _bits_equal(y, want)


def test_depthwise_nonfinite_tap_tile_kernel(dev, orc):
    """As above through the LDS tile kernel (W % 8 != 0): its masked loop."""
    from forge_amd import ops
    rng = np.random.default_rng(78)
    x, w, ws, b = _dw_inputs(rng, 1, 3, 19, 26, 3, 3, True)
    ws[0] = np.float16(-np.inf)
    want = orc.depthwise_conv2d(x, w, ws, b, (1, 1))
    say("depthwise non-finite taps, tile kernel")
    y = to_host(ops.int8_depthwise_conv2d_forward(to_dev(x, dev), to_dev(w, dev), to_dev(ws, dev), to_dev(b, dev),
                                                  3, 3, (1, 1)))
    assert _bits_equal(y, want)


def test_depthwise_full_size(dev, orc):
    """The measured workload: (1, 64, 540, 960), 3x3, pad 1, bias."""
    from forge_amd import ops
    rng = np.random.default_rng(540)
    x, w, ws, b = _dw_inputs(rng, 1, 64, 540, 960, 3, 3, True)
    want = orc.depthwise_conv2d(x, w, ws, b, (1, 1))
    say("depthwise full size (1,64,540,960) 3x3")
    y = to_host(ops.int8_depthwise_conv2d_forward(to_dev(x, dev), to_dev(w, dev), to_dev(ws, dev), to_dev(b, dev),
                                                  3, 3, (1, 1)))
    assert _bits_equal(y, want)


def test_depthwise_unaligned_output(dev, orc):
    """An output view 2 bytes past a 16-byte boundary takes the element stores."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(3)
    x, w, ws, b = _dw_inputs(rng, 1, 2, 16, 64, 3, 3, True)
    want = orc.depthwise_conv2d(x, w, ws, b, (1, 1))
    buf = torch.zeros((want.size + 8,), dtype=torch.float16, device=dev)
    out = buf[1:1 + want.size].view(want.shape)
    say("depthwise unaligned output")
    ops.int8_depthwise_conv2d_forward(to_dev(x, dev), to_dev(w, dev), to_dev(ws, dev), to_dev(b, dev), 3, 3, (1, 1),
                                      out=out)
    assert _bits_equal(to_host(out), want)


# ---- ConvTranspose2d k2s2 ----------------------------------------------------------

def _ct_inputs(rng, N, C_in, H, W, C_out, bias):
    x = rng.uniform(-1, 1, (N, C_in, H, W)).astype(np.float16)
    w = int8_uniform(rng, (4 * C_out, C_in))
    ws = rng.uniform(0.005, 0.05, C_out).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, C_out).astype(np.float16) if bias else None
    return x, w, ws, b


CT_CASES = [
    # N, C_in, H, W, C_out, bias
    (1, 32, 16, 16, 64, True),      # reference test cases (the first two take the fused kernel)
    (1, 64, 8, 8, 32, True),
    (1, 16, 32, 32, 16, False),
    # fused single-pass kernel: C_in in {32, 64, 128, 256}, H*W % 8 == 0
    (1, 128, 32, 64, 64, True),
    (2, 256, 24, 36, 96, False),
    (2, 64, 6, 12, 5, True),        # partial pixel tile, C_out % 8 != 0 (partial column block)
    (1, 32, 3, 8, 33, True),        # 5 column blocks over 4 waves
    (1, 128, 8, 3, 16, True),       # odd W: a 32-pixel block spans image rows
    (2, 64, 10, 20, 24, True),      # 8-pixel last tile per image, 3 waves of MFMA items
    (1, 256, 16, 24, 8, False),     # C_in = 256, one column block (waves without an item)
    # two-kernel path: pixel quantizer + GEMM with the scatter epilogue
    (3, 24, 7, 5, 10, True),        # W % 4 != 0: element stores; chunked images
    (2, 13, 6, 8, 5, True),         # C_in % 4 != 0: byte rows, byte-gather GEMM
    (1, 640, 4, 8, 8, True),        # C_in > 512: the quantizer re-reads x
    (1, 384, 16, 16, 40, True),     # C_in % 128 == 0: DMA engine
    (2, 192, 24, 36, 96, False),    # register-staged engine
    (1, 48, 1, 1, 7, True),         # one pixel
    (5, 8, 3, 4, 3, True),          # many small images in one chunk
]


@pytest.mark.parametrize("N,C_in,H,W,C_out,bias", CT_CASES)
def test_conv_transpose_parity(dev, orc, N, C_in, H, W, C_out, bias):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(N * 7 + C_in * 3 + W)
    x, w, ws, b = _ct_inputs(rng, N, C_in, H, W, C_out, bias)
    want = orc.conv_transpose2d_k2s2(x, w, ws, b)
    say(f"conv_transpose N={N} C_in={C_in} H={H} W={W} C_out={C_out} bias={bias}")
    nbytes = ops.int8_conv_transpose2d_k2s2_workspace_size(C_in, H, W, C_out)
    wsp = torch.empty((nbytes,), dtype=torch.uint8, device=dev)
    wsp.fill_(0x5A)
    out = torch.empty(want.shape, dtype=torch.float16, device=dev)
    out.view(torch.uint8).fill_(0x7B)
    ops.int8_conv_transpose2d_k2s2_forward(to_dev(x, dev), to_dev(w, dev), to_dev(ws, dev),
                                           None if b is None else to_dev(b, dev), workspace=wsp, out=out)
    y = to_host(out)
    assert _bits_equal(y, want)
    if N == 1 and (C_in, H, W, C_out) in [(32, 16, 16, 64), (64, 8, 8, 32), (16, 32, 32, 16)]:
        # test_int8_special_conv.cu:245-249: max < 0.5 and mean < 0.1 against the float conv
        w4 = w.reshape(C_out, 2, 2, C_in).transpose(3, 0, 1, 2).astype(np.float64) \
            * ws.astype(np.float64)[None, :, None, None]
        ref = torch.nn.functional.conv_transpose2d(torch.from_numpy(x.astype(np.float64)), torch.from_numpy(w4),
                                                   bias=None if b is None else torch.from_numpy(b.astype(np.float64)),
                                                   stride=2).numpy()
        d = np.abs(y.astype(np.float64) - ref)
        assert d.max() < 0.5 and d.mean() < 0.1


def test_conv_transpose_unaligned_output(dev, orc):
    """An output view 2 bytes past a 16-byte boundary takes the element stores."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(12)
    x, w, ws, b = _ct_inputs(rng, 1, 32, 8, 16, 16, True)
    want = orc.conv_transpose2d_k2s2(x, w, ws, b)
    buf = torch.zeros((want.size + 8,), dtype=torch.float16, device=dev)
    out = buf[1:1 + want.size].view(want.shape)
    say("conv_transpose unaligned output")
    ops.int8_conv_transpose2d_k2s2_forward(to_dev(x, dev), to_dev(w, dev), to_dev(ws, dev), to_dev(b, dev), out=out)
    assert _bits_equal(to_host(out), want)


def test_conv_transpose_full_size(dev, orc):
    """The measured workload: (1, 64, 270, 480) -> (1, 32, 540, 960), bias."""
    from forge_amd import ops
    rng = np.random.default_rng(270)
    x, w, ws, b = _ct_inputs(rng, 1, 64, 270, 480, 32, True)
    want = orc.conv_transpose2d_k2s2(x, w, ws, b)
    say("conv_transpose full size (1,64,270,480)->(1,32,540,960)")
    y = to_host(ops.int8_conv_transpose2d_k2s2_forward(to_dev(x, dev), to_dev(w, dev), to_dev(ws, dev),
                                                       to_dev(b, dev)))
    assert _bits_equal(y, want)


@pytest.mark.parametrize("C_in", [32, 64, 256])
def test_conv_transpose_special_pixels(dev, orc, C_in):
    """Pixels holding the quantizer's edge cases -- a NaN among finite channels (several
    payloads), an all-NaN pixel, +-inf, subnormals with +-0, exact ties after scaling (absmax
    127 gives scale 1), the fp16 maximum -- through the fused kernel (aligned output) and the
    two-kernel path (an output view 2 bytes off a 4-byte boundary), both against the oracle."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(C_in)
    N, H, W, C_out = 1, 12, 16, 24
    x, w, ws, b = _ct_inputs(rng, N, C_in, H, W, C_out, True)
    xb = x.view(np.uint16)
    px = lambda p: (p // W, p % W)
    for p, bits in [(0, 0x7E00), (3, 0x7C01), (9, 0xFE00), (17, 0x7D55)]:   # one NaN channel
        h, wc = px(p)
        xb[0, rng.integers(C_in), h, wc] = bits
    h, wc = px(20)
    xb[0, :, h, wc] = 0x7E00                                                # all NaN
    h, wc = px(24)
    xb[0, 5 % C_in, h, wc] = 0x7C00                                         # +inf
    h, wc = px(33)
    xb[0, 7 % C_in, h, wc] = 0xFC00                                         # -inf
    h, wc = px(40)
    xb[0, :, h, wc] = rng.choice(np.array([0x0001, 0x8001, 0x03FF, 0x0200, 0x8000, 0x0000], np.uint16), C_in)
    h, wc = px(47)
    xb[0, :, h, wc] = 0
    xb[0, :8, h, wc] = np.array([127.0, 2.5, 3.5, -2.5, 0.5, -0.5, 1.5, -126.5], np.float16).view(np.uint16)
    h, wc = px(58)
    xb[0, :, h, wc] = np.float16(-65504).view(np.uint16)
    xb[0, ::3, h, wc] = np.float16(65504).view(np.uint16)
    want = orc.conv_transpose2d_k2s2(x, w, ws, b)
    say(f"conv_transpose special pixels C_in={C_in}")
    xd, wd, wsd, bd = to_dev(x, dev), to_dev(w, dev), to_dev(ws, dev), to_dev(b, dev)
    y1 = to_host(ops.int8_conv_transpose2d_k2s2_forward(xd, wd, wsd, bd))
    assert _bits_equal(y1, want)
    buf = torch.zeros((want.size + 8,), dtype=torch.float16, device=dev)
    out = buf[1:1 + want.size].view(want.shape)
    ops.int8_conv_transpose2d_k2s2_forward(xd, wd, wsd, bd, out=out)
    assert _bits_equal(to_host(out), want)
