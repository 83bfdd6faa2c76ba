"""GPU parity: INT8 conv2d.

NHWC implicit GEMM: INT32 bit-exact vs the oracle's direct convolution (golden cases from
torch float64 conv2d, padding / stride / dilation, C % 16 != 0 byte path, the DMA gather for
C % 128 == 0 at 128- and 256-row tiles, configs[4] at its full spatial size); FP16 dequant bit-exact to the oracle epilogue. NCHW FP16 API
(src/nn/int8_conv2d.cu:126-223): bit-exact to the oracle composition im2col -> per-row
quantize -> GEMM dequant -> NCHW, and within the reference test's float tolerance
(tests/test_int8_conv2d.cu:166-176) of a float convolution."""
import numpy as np
import pytest

from conftest import golden
from helpers import int8_uniform, poison, say, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["3x3_p1", "2x2_s2", "3x3_d2"])
def test_conv_golden(dev, name):
    from forge_amd import ops
    g = golden("conv")
    pad, stride, dil = (int(v) for v in g[name + "_cfg"])
    say(f"conv golden {name}")
    out = ops.int8_conv2d_nhwc_s32(to_dev(g[name + "_x"], dev), to_dev(g[name + "_w"], dev),
                                   (pad, pad), (stride, stride), (dil, dil))
    assert np.array_equal(to_host(out), g[name + "_out"])


@pytest.mark.parametrize("N,H,W,C,Co,k,pad,stride,dil", [
    (1, 5, 5, 8, 4, 3, 1, 1, 1),       # C % 16 != 0: byte gather path
    (2, 9, 11, 48, 40, 3, 1, 2, 1),
    (1, 14, 14, 64, 96, 1, 0, 1, 1),   # pointwise
    (1, 12, 12, 32, 300, 5, 2, 1, 1),
])
def test_conv_random(dev, orc, N, H, W, C, Co, k, pad, stride, dil):
    from forge_amd import ops
    rng = np.random.default_rng(N * H * C + Co)
    x = int8_uniform(rng, (N, H, W, C))
    w = int8_uniform(rng, (Co, k, k, C))
    ref = orc.conv2d_nhwc_s32(x, w, (pad, pad), (stride, stride), (dil, dil))
    say(f"conv N={N} H={H} W={W} C={C} Co={Co} k={k}")
    out = ops.int8_conv2d_nhwc_s32(to_dev(x, dev), to_dev(w, dev), (pad, pad), (stride, stride), (dil, dil))
    assert np.array_equal(to_host(out), ref)


# C % 128 == 0 with grids large enough for the DMA engine (128- and 256-row tiles): the
# implicit-im2col gather by DMA, padding read from the zero line, ragged last tile.
@pytest.mark.parametrize("N,H,W,C,Co,k,pad,stride,dil,check", [
    (2, 64, 64, 128, 256, 3, 1, 1, 1, "all"),      # 128x128 tiles, padding
    (2, 63, 61, 128, 384, 3, 1, 1, 1, "all"),      # ragged rows (7686)
    (8, 130, 130, 128, 256, 3, 2, 2, 2, "ends"),   # 256x256 tiles, stride 2, dilation 2
    (4, 40, 40, 256, 256, 1, 0, 1, 1, "all"),      # pointwise, two stages per tap
])
def test_conv_dma_gather(dev, orc, N, H, W, C, Co, k, pad, stride, dil, check):
    from forge_amd import ops
    rng = np.random.default_rng(H * W + C + Co)
    x = int8_uniform(rng, (N, H, W, C))
    w = int8_uniform(rng, (Co, k, k, C))
    say(f"conv dma N={N} H={H} W={W} C={C} Co={Co} k={k} p={pad} s={stride} d={dil}")
    out = to_host(ops.int8_conv2d_nhwc_s32(to_dev(x, dev), to_dev(w, dev), (pad, pad), (stride, stride),
                                           (dil, dil)))
    imgs = range(N) if check == "all" else (0, N - 1)
    for n in imgs:
        ref = orc.conv2d_nhwc_s32(x[n:n + 1], w, (pad, pad), (stride, stride), (dil, dil))
        assert np.array_equal(out[n:n + 1], ref)


# Stride-1 convs with C % 128 == 0 and Co % 256 == 0 whose tiles are whole output rows of 224 or
# 256 pixels: the window-fed tile (input window in LDS once per 128-channel chunk, every tap's
# fragment read at its shift), with the 2-slot weight ring and two window buffers or the 3-slot
# ring and one. Padding on every side, no padding, 5x5, dilation along W, 1-3 channel chunks,
# two column tiles; INT32 and FP16 (with and without bias) against the oracle.
@pytest.mark.parametrize("N,H,W,C,Co,k,pad,dil,route", [
    (2, 56, 56, 128, 256, 3, 1, (1, 1), "conv-window224"),
    (2, 32, 14, 256, 256, 3, 1, (1, 1), "conv-window224"),
    (1, 16, 28, 128, 512, 5, 2, (1, 1), "conv-window224"),
    (2, 34, 30, 384, 256, 3, 0, (1, 1), "conv-window224"),
    (1, 16, 34, 128, 256, 3, 1, (1, 2), "conv-window256"),
    (2, 16, 32, 256, 256, 3, 1, (1, 1), "conv-window256"),
    (2, 17, 33, 128, 256, 2, 0, (1, 1), "conv-window256"),       # odd tap reach: padded window rows
    (1, 4, 56, 128, 256, 3, 1, (1, 1), "conv-window224"),
    (2, 64, 64, 256, 256, 3, 1, (1, 1), "conv-window256 ring3"),  # two windows do not fit
    (1, 8, 56, 512, 768, 3, 1, (1, 1), "conv-window224"),         # 4 channel chunks, 3 column tiles
    (1, 16, 28, 128, 256, 3, 2, (2, 2), "conv-window224"),        # dilation 2 on both axes
])
def test_conv_window(dev, orc, N, H, W, C, Co, k, pad, dil, route):
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(H * W + C + Co + k)
    x = int8_uniform(rng, (N, H, W, C))
    w = int8_uniform(rng, (Co, k, k, C))
    ref = orc.conv2d_nhwc_s32(x, w, (pad, pad), (1, 1), dil, threads=orc.cpu_threads())
    say(f"conv window N={N} H={H} W={W} C={C} Co={Co} k={k} p={pad} d={dil}")
    xd, wd = to_dev(x, dev), to_dev(w, dev)
    o32 = torch.empty(ref.shape, dtype=torch.int32, device=dev)
    poison(o32, 0x7B)
    out = to_host(ops.int8_conv2d_nhwc_s32(xd, wd, (pad, pad), (1, 1), dil, out=o32))
    assert ops.last_route() == route, ops.last_route()
    bad = int((out != ref).sum())
    assert bad == 0, f"{bad} of {out.size} INT32 outputs differ"
    M = ref.size // Co
    act = rng.uniform(0.01, 0.03, M).astype(np.float32)
    ws = rng.uniform(1e-3, 1e-2, Co).astype(np.float16)
    b = (rng.standard_normal(Co) * 0.1).astype(np.float16)
    for bias in (b, None):
        o16 = torch.empty(ref.shape, dtype=torch.float16, device=dev)
        poison(o16, 0x7B)
        y = to_host(ops.int8_conv2d_nhwc_dequant(xd, wd, to_dev(act, dev), to_dev(ws, dev),
                                                 None if bias is None else to_dev(bias, dev), (pad, pad), (1, 1),
                                                 dil, out=o16))
        assert ops.last_route() == route, ops.last_route()
        refy = orc.dequant_epilogue(ref.reshape(-1, Co), act, ws, bias)
        bad = int((y.reshape(-1, Co).view(np.uint16) != refy.view(np.uint16)).sum())
        assert bad == 0, f"{bad} of {y.size} FP16 outputs differ (bias={bias is not None})"


def test_config5_full_size(dev, orc):
    """NHWC (32,56,56,256) x (256,3,3,256), stride 1, pad 1; every INT32 output of
    all 32 images bit-exact against the oracle's direct convolution (threaded), and every FP16
    output of the per-channel dequant + bias epilogue against the oracle's epilogue on it."""
    import torch
    from forge_amd import ops
    rng = np.random.default_rng(5)
    x = int8_uniform(rng, (32, 56, 56, 256))
    w = int8_uniform(rng, (256, 3, 3, 256))
    ref = orc.conv2d_nhwc_s32(x, w, (1, 1), threads=orc.cpu_threads())
    say("config5 conv 32x56x56x256")
    xd, wd = to_dev(x, dev), to_dev(w, dev)
    o32 = torch.empty((32, 56, 56, 256), dtype=torch.int32, device=dev)
    poison(o32, 0x7B)
    out = to_host(ops.int8_conv2d_nhwc_s32(xd, wd, (1, 1), out=o32))
    assert ops.last_route() == "conv-window224", ops.last_route()
    bad = int((out != ref).sum())
    assert bad == 0, f"{bad} of {out.size} INT32 outputs differ"
    M = 32 * 56 * 56
    act = rng.uniform(0.01, 0.03, M).astype(np.float32)
    ws = rng.uniform(1e-3, 1e-2, 256).astype(np.float16)
    b = (rng.standard_normal(256) * 0.1).astype(np.float16)
    say("config5 conv dequant")
    o16 = torch.empty((32, 56, 56, 256), dtype=torch.float16, device=dev)
    poison(o16, 0x7B)
    y = to_host(ops.int8_conv2d_nhwc_dequant(xd, wd, to_dev(act, dev), to_dev(ws, dev), to_dev(b, dev), (1, 1),
                                             out=o16))
    refy = orc.dequant_epilogue(ref.reshape(-1, 256), act, ws, b)
    bad = int((y.reshape(-1, 256).view(np.uint16) != refy.view(np.uint16)).sum())
    assert bad == 0, f"{bad} of {y.size} FP16 outputs differ"


def _im2col_nchw(x, kH, kW, pad, stride, dil):
    C, H, W = x.shape
    Ho = (H + 2 * pad[0] - dil[0] * (kH - 1) - 1) // stride[0] + 1
    Wo = (W + 2 * pad[1] - dil[1] * (kW - 1) - 1) // stride[1] + 1
    xp = np.zeros((C, H + 2 * pad[0], W + 2 * pad[1]), x.dtype)
    xp[:, pad[0]:pad[0] + H, pad[1]:pad[1] + W] = x
    cols = np.empty((Ho * Wo, C, kH, kW), x.dtype)
    for kh in range(kH):
        for kw in range(kW):
            sl = xp[:, kh * dil[0]: kh * dil[0] + stride[0] * (Ho - 1) + 1: stride[0],
                    kw * dil[1]: kw * dil[1] + stride[1] * (Wo - 1) + 1: stride[1]]
            cols[:, :, kh, kw] = sl.reshape(C, -1).T
    return cols.reshape(Ho * Wo, -1), Ho, Wo


# tests/test_int8_conv2d.cu:203-255
NCHW_CASES = [(8, 16, 16, 16, 3, 1, 1, 1, True), (16, 8, 8, 32, 1, 0, 1, 1, True),
              (7, 32, 32, 16, 2, 0, 2, 1, True), (4, 12, 12, 8, 3, 1, 1, 1, False),
              (16, 64, 64, 32, 3, 1, 1, 1, True), (8, 16, 16, 8, 3, 2, 1, 2, True)]


@pytest.mark.parametrize("C,H,W,Co,k,pad,stride,dil,bias", NCHW_CASES)
def test_conv_nchw_api(dev, orc, C, H, W, Co, k, pad, stride, dil, bias):
    from forge_amd import ops
    rng = np.random.default_rng(C * H + Co)
    N = 2
    x = rng.uniform(-1, 1, (N, C, H, W)).astype(np.float16)
    w = int8_uniform(rng, (Co, C * k * k))
    ws = rng.uniform(0.005, 0.05, Co).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, Co).astype(np.float16) if bias else None
    say(f"conv nchw C={C} H={H} Co={Co} k={k} s={stride} d={dil}")
    y = to_host(ops.int8_conv2d_forward(to_dev(x, dev), to_dev(w, dev), to_dev(ws, dev),
                                        None if b is None else to_dev(b, dev), k, k, (pad, pad), (stride, stride),
                                        (dil, dil)))
    for n in range(N):
        cols, Ho, Wo = _im2col_nchw(x[n], k, k, (pad, pad), (stride, stride), (dil, dil))
        q, s = orc.quantize_rows(cols)
        ref = orc.gemm_dequant(q, w, s, ws, b)                  # (Ho*Wo, Co)
        assert np.array_equal(y[n].reshape(Co, -1).T.copy().view(np.uint16), ref.view(np.uint16))
        # the reference test's float check: dequantized weights, unquantized activations
        fref = cols.astype(np.float64) @ (w.astype(np.float64) * ws.astype(np.float64)[:, None]).T
        if b is not None:
            fref += b.astype(np.float64)
        err = np.abs(y[n].reshape(Co, -1).T.astype(np.float64) - fref)
        assert err.max() < 0.5 and err.mean() < 0.1


def _nchw_check(orc, y, x, w, ws, b, k, pad, stride, dil):
    """Every output of every image against the reference pipeline composed on the oracle."""
    N, Co = y.shape[0], y.shape[1]
    for n in range(N):
        cols, Ho, Wo = _im2col_nchw(x[n], k, k, (pad, pad), (stride, stride), (dil, dil))
        assert y.shape[2:] == (Ho, Wo)
        q, s = orc.quantize_rows(cols)
        ref = orc.gemm_dequant(q, w, s, ws, b)
        got = y[n].reshape(Co, -1).T.copy().view(np.uint16)
        bad = int((got != ref.view(np.uint16)).sum())
        assert bad == 0, f"image {n}: {bad} of {got.size} outputs differ"


def _nchw_run(dev, x, w, ws, b, k, pad, stride, dil):
    import torch
    from forge_amd import ops
    N, _, H, W = x.shape
    Co = w.shape[0]
    Ho = (H + 2 * pad - dil * (k - 1) - 1) // stride + 1
    Wo = (W + 2 * pad - dil * (k - 1) - 1) // stride + 1
    out = torch.empty((N, Co, Ho, Wo), dtype=torch.float16, device=dev)
    poison(out, 0x7B)
    y = to_host(ops.int8_conv2d_forward(to_dev(x, dev), to_dev(w, dev), to_dev(ws, dev),
                                        None if b is None else to_dev(b, dev), k, k, (pad, pad), (stride, stride),
                                        (dil, dil), out=out))
    return y, ops.last_route()


# The one-launch NCHW paths. "conv-nchw-cl": channel-last window (W % 8 == 0, C_out <= 128,
# LDS <= 80 KB), tiles of 32 output pixels per wave (8 waves: "tile256", else 4: "tile128"),
# weights permuted to the (kh, kw, c) order in LDS; with the next tile's window loads in flight
# ("prefetch") when each wave has at most one load instruction per tile. "conv-nchw-fused":
# NCHW window, 64-pixel tiles (K % 16 == 0).
# Cases: 64 x 4 tiles; C = 24 (channels padded to 32 with zeros) with C_out = 48 (two
# 32-channel blocks, the second partial); C = 16 (odd chunk count: the last 32-deep step half
# past the patch) at stride 2 with C_out = 64 and Wo = 24 (pixel blocks across output rows);
# C = 8 with a dilated 5x5 and C_out = 96 (4 waves: the 8-wave window does not fit); RGB input
# (C = 3); pointwise 1x1 with Wo = 24, a partial last pixel block and C_out = 128; C = 64 (4
# waves, five load instructions: no prefetch); the NCHW-window kernel at W % 8 != 0 (several
# rows per tile at Wo = 10, K % 32 == 16, 1x1) and at C_out > 128 (a dilated 5x5).
FUSED_CASES = [(32, 64, 64, 32, 3, 1, 1, 1, True, "conv-nchw-cl prefetch tile256"),
               (24, 20, 72, 48, 3, 1, 1, 1, True, "conv-nchw-cl prefetch tile256"),
               (16, 30, 48, 64, 3, 1, 2, 1, False, "conv-nchw-cl prefetch tile256"),
               (8, 33, 40, 96, 5, 4, 1, 2, True, "conv-nchw-cl prefetch tile128"),
               (3, 32, 32, 16, 3, 1, 1, 1, True, "conv-nchw-cl prefetch tile256"),
               (48, 17, 24, 128, 1, 0, 1, 1, True, "conv-nchw-cl prefetch tile256"),
               (64, 40, 96, 32, 3, 1, 1, 1, True, "conv-nchw-cl tile128"),
               (32, 45, 70, 48, 3, 1, 1, 1, True, "conv-nchw-fused"),
               (16, 20, 20, 24, 3, 1, 2, 1, False, "conv-nchw-fused"),
               (32, 24, 40, 160, 5, 4, 1, 2, True, "conv-nchw-fused"),
               (48, 17, 33, 16, 3, 1, 1, 1, True, "conv-nchw-fused"),
               (64, 33, 33, 128, 1, 0, 1, 1, True, "conv-nchw-fused")]


@pytest.mark.parametrize("C,H,W,Co,k,pad,stride,dil,bias,route", FUSED_CASES)
def test_conv_nchw_fused(dev, orc, C, H, W, Co, k, pad, stride, dil, bias, route):
    rng = np.random.default_rng(C * W + Co + k)
    N = 3
    x = rng.uniform(-1, 1, (N, C, H, W)).astype(np.float16)
    w = int8_uniform(rng, (Co, C * k * k))
    ws = rng.uniform(0.005, 0.05, Co).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, Co).astype(np.float16) if bias else None
    say(f"conv nchw one-launch C={C} H={H} W={W} Co={Co} k={k} s={stride} d={dil} ({route})")
    y, got_route = _nchw_run(dev, x, w, ws, b, k, pad, stride, dil)
    assert got_route == route if route.startswith("conv-nchw-cl") else got_route.startswith(route), got_route
    _nchw_check(orc, y, x, w, ws, b, k, pad, stride, dil)


# Shapes with more tiles than the persistent grid holds (each workgroup walks several tiles):
# the channel-last kernel with and without the next tile's loads in flight; the NCHW-window
# kernel with 16-byte loads and prefetch (C_out > 128), 16-byte loads without (a window of
# more than 16 load rounds at C = 128) and 2-byte loads (W % 8 != 0).
PERSISTENT_CASES = [(4, 16, 256, 512, 16, "conv-nchw-cl prefetch tile256"), (2, 64, 256, 256, 32, "conv-nchw-cl tile128"),
                    (2, 16, 256, 512, 160, "conv-nchw-fused prefetch"), (2, 128, 64, 256, 32, "conv-nchw-fused"),
                    (3, 16, 200, 250, 24, "conv-nchw-fused")]


@pytest.mark.parametrize("N,C,H,W,Co,route", PERSISTENT_CASES)
def test_conv_nchw_fused_persistent(dev, orc, N, C, H, W, Co, route):
    rng = np.random.default_rng(N * C + W)
    x = rng.uniform(-1, 1, (N, C, H, W)).astype(np.float16)
    w = int8_uniform(rng, (Co, C * 9))
    ws = rng.uniform(0.005, 0.05, Co).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, Co).astype(np.float16)
    say(f"conv nchw one-launch persistent N={N} C={C} H={H} W={W} Co={Co} ({route})")
    y, got_route = _nchw_run(dev, x, w, ws, b, 3, 1, 1, 1)
    assert got_route == route, got_route
    _nchw_check(orc, y, x, w, ws, b, 3, 1, 1, 1)


@pytest.mark.parametrize("W,Co,route", [(80, 32, "conv-nchw-cl prefetch tile256"), (84, 32, "conv-nchw-fused"),
                                        (80, 160, "conv-nchw-fused prefetch")])
def test_conv_nchw_fused_special_values(dev, orc, W, Co, route):
    """Patches holding NaN, +-inf, subnormals and all-zero windows through the one-launch paths:
    the same bits as quantize_rows on the reference's im2col rows, then its GEMM epilogue."""
    from helpers import special_fp16_rows
    rng = np.random.default_rng(77)
    N, C, H = 2, 16, 12
    x = special_fp16_rows(rng, N * C * H, W).reshape(N, C, H, W)
    x[1, :, 4:7, 10:20] = 0
    w = int8_uniform(rng, (Co, C * 9))
    ws = rng.uniform(0.005, 0.05, Co).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, Co).astype(np.float16)
    say(f"conv nchw one-launch special values W={W} Co={Co} ({route})")
    y, got_route = _nchw_run(dev, x, w, ws, b, 3, 1, 1, 1)
    assert got_route == route, got_route
    _nchw_check(orc, y, x, w, ws, b, 3, 1, 1, 1)
