"""Pins the CPU oracle (oracle/forge_oracle.c) before it is trusted as the checker.

Each oracle function is checked against something independent of its own formula:
numpy/torch library routines, the golden fixtures (computed by tests/golden/make_golden.py
with those routines), closed-form special cases, invariants, and brute force -- chosen so
that a plausible mistake (dropped term, wrong sign or index, transposed operand, wrong
rounding mode) fails at least one check.
"""
import itertools

import numpy as np
import pytest

from conftest import golden


# ---- fp16 conversions -------------------------------------------------------------

def test_f16_to_f32_all_halves(orc):
    L = orc.lib()
    bits = np.arange(65536, dtype=np.uint32)
    ref = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([L.orc_f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne_matches_numpy(orc):
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(1000),
        rng.standard_normal(20000).astype(np.float32) * np.float32(1e-5),   # subnormal halves
        np.array([65504, 65519.99, 65520, 65536, -65520, 2 ** -24, 2 ** -25, 3 * 2 ** -26,
                  2 ** -25 * 1.0000001, 0.0, -0.0, np.inf, -np.inf, 1.0 + 2 ** -11,
                  1.0 + 3 * 2 ** -11, 2049.0, 2051.0], np.float32),
    ])
    # every halfway point between consecutive halves (ties) in the normal range
    h = np.arange(0x0400, 0x7BFF, 37, dtype=np.uint16).view(np.float16).astype(np.float64)
    h2 = np.arange(0x0401, 0x7C00, 37, dtype=np.uint16).view(np.float16).astype(np.float64)
    n = min(len(h), len(h2))
    ties = ((h[:n] + h2[:n]) / 2).astype(np.float32)
    vals = np.concatenate([vals, ties, -ties])
    got = orc.f32_to_f16_bits(vals)
    ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


# ---- quantize ----------------------------------------------------------------------

def test_quantize_golden(orc):
    g = golden("quantize")
    q, s = orc.quantize_rows(g["X"])
    assert np.array_equal(s.view(np.uint32), g["scales"].view(np.uint32))
    assert np.array_equal(q, g["q"])


def test_quantize_closed_forms(orc):
    K = 16
    x = np.zeros((4, K), np.float16)
    x[1, 3] = -3.25                         # single nonzero -> -127
    x[2, :6] = [127, 2.5, 3.5, -2.5, 0.5, 1.5]   # scale exactly 1.0: RNE ties
    x[3, :4] = [254, 5, 7, -3]              # scale exactly 2.0: 2.5 -> 2, 3.5 -> 4, -1.5 -> -2
    q, s = orc.quantize_rows(x)
    assert s[0] == np.float32(1e-8) / np.float32(127.0) and not q[0].any()
    assert q[1, 3] == -127 and np.count_nonzero(q[1]) == 1
    assert s[2] == 1.0 and list(q[2, :6]) == [127, 2, 4, -2, 0, 2]
    assert s[3] == 2.0 and list(q[3, :4]) == [127, 2, 4, -2]


def test_quantize_invariants(orc):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((64, 300)) * rng.uniform(0.01, 100, (64, 1))).astype(np.float16)
    q, s = orc.quantize_rows(x)
    xf = x.astype(np.float32)
    amax = np.abs(xf).max(axis=1)
    assert np.all(np.abs(q.astype(np.int32)) <= 127)
    # the absmax element maps to +-127 with its sign
    idx = np.abs(xf).argmax(axis=1)
    assert np.all(q[np.arange(64), idx] == np.sign(xf[np.arange(64), idx]) * 127)
    # reconstruction error at most half a step (plus float slack)
    err = np.abs(xf - q.astype(np.float32) * s[:, None])
    assert np.all(err <= s[:, None] * 0.5 * (1 + 1e-5))
    # scale = amax / 127 up to one rounding
    assert np.allclose(s, amax / 127.0, rtol=2e-7)
    # sign preserved and monotone within a row
    assert np.all(np.sign(q) * np.sign(xf) >= 0)


def test_quantize_matches_numpy_float32(orc):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((40, 1000)).astype(np.float16)
    x[:, rng.choice(1000, 8, replace=False)] *= 20
    q, s = orc.quantize_rows(x)
    xf = x.astype(np.float32)
    sc = (np.maximum(np.abs(xf).max(axis=1), np.float32(1e-8)) / np.float32(127)).astype(np.float32)
    inv = (np.float32(1) / sc).astype(np.float32)
    qr = np.clip(np.rint((xf * inv[:, None]).astype(np.float32)), -128, 127).astype(np.int8)
    assert np.array_equal(s, sc) and np.array_equal(q, qr)


def test_quantize_special_values_match_numpy(orc):
    """NaN of every kind (quiet, signalling pattern, negative, payloads) is skipped by the
    absmax, as the reference's GPU fmaxf does, and quantizes to 0; a NaN-only row has amax 0;
    an inf row has scale inf and quantizes everything to 0 (x * 0, or inf * 0 = NaN -> 0);
    subnormals, -0, ties and the fp16 maximum follow the float32 formula. Checked against
    numpy's nanmax and float32 arithmetic, element by element."""
    from helpers import special_fp16_rows
    rng = np.random.default_rng(11)
    for M, K in [(9, 64), (12, 1003), (16, 4096)]:
        x = special_fp16_rows(rng, M, K)
        q, s = orc.quantize_rows(x)
        xf = x.astype(np.float32)
        with np.errstate(invalid="ignore"):
            a = np.abs(xf)
            amax = np.where(np.isnan(a).all(axis=1), np.float32(0), np.nanmax(np.where(np.isnan(a), -1, a), axis=1))
            sc = (np.maximum(amax.astype(np.float32), np.float32(1e-8)) / np.float32(127)).astype(np.float32)
            inv = (np.float32(1) / sc).astype(np.float32)
            v = np.rint((xf * inv[:, None]).astype(np.float32))
        qr = np.where(np.isnan(v), 0, np.clip(np.nan_to_num(v, nan=0.0), -128, 127)).astype(np.int8)
        assert np.array_equal(s.view(np.uint32), sc.view(np.uint32))
        assert np.array_equal(q, qr)
        assert np.isinf(s).any() and not q[np.isinf(s)].any()


# ---- dequant ----------------------------------------------------------------------

def _ulp_diff(a16, b16):
    a = a16.view(np.uint16).astype(np.int32)
    b = b16.view(np.uint16).astype(np.int32)
    # map sign-magnitude to a monotone integer line
    a = np.where(a & 0x8000, 0x8000 - (a & 0x7FFF), 0x8000 + a)
    b = np.where(b & 0x8000, 0x8000 - (b & 0x7FFF), 0x8000 + b)
    return np.abs(a - b)


def test_dequant_golden(orc):
    g = golden("dequant")
    out = orc.dequantize_bias(g["acc"], g["act_scale"], g["w_scale"], g["bias"])
    assert _ulp_diff(out, g["out_standalone"]).max() <= 1
    epi = orc.dequant_epilogue(g["acc"], g["act_scale"], g["w_scale"], g["bias"])
    assert _ulp_diff(epi, g["out_epilogue"]).max() <= 1
    # the two associations really are different functions (and both are exercised)
    nob = orc.dequant_epilogue(g["acc"], g["act_scale"], g["w_scale"], None)
    ref = (g["acc"].astype(np.float64) * (g["act_scale"][:, None] * g["w_scale"].astype(np.float32)[None, :])
           .astype(np.float64)).astype(np.float16)
    assert _ulp_diff(nob, ref).max() <= 1


def test_dequant_bias_and_sign(orc):
    acc = np.array([[0, 1, -1, 1000]], np.int32)
    out = orc.dequant_epilogue(acc, np.array([0.5], np.float32), np.array([2.0] * 4, np.float16),
                               np.array([0.25, 0.25, 0.25, -1.0], np.float16))
    assert list(out.astype(np.float32)[0]) == [0.25, 1.25, -0.75, 999.0]


# ---- GEMM ---------------------------------------------------------------------------

def test_gemm_c1_golden(orc):
    g = golden("c1_gemm")
    assert np.array_equal(orc.gemm_s32(g["A"], g["B"]), g["C"])


def test_gemm_numpy_and_closed_forms(orc):
    rng = np.random.default_rng(5)
    for M, K, N in [(1, 1, 1), (7, 7, 5), (33, 28, 17), (16, 8192, 4)]:
        A = rng.integers(-128, 128, (M, K)).astype(np.int8)
        B = rng.integers(-128, 128, (N, K)).astype(np.int8)
        assert np.array_equal(orc.gemm_s32(A, B), (A.astype(np.int64) @ B.astype(np.int64).T).astype(np.int32))
    K = 8192
    ones = np.ones((2, K), np.int8)
    assert np.all(orc.gemm_s32(ones, -ones) == -K)
    ext = np.full((1, K), -128, np.int8)
    assert orc.gemm_s32(ext, ext)[0, 0] == 128 * 128 * K          # 2^27, no overflow
    # transposition check: C = A B^T, not A^T B or B A^T
    A = np.array([[1, 2], [3, 4], [5, 6]], np.int8)
    B = np.array([[1, 0], [0, 1]], np.int8)
    assert np.array_equal(orc.gemm_s32(A, B), A.astype(np.int32))


# ---- prune / pack ---------------------------------------------------------------------

def test_prune_golden(orc):
    g = golden("prune")
    comp, meta = orc.prune_compress_24(g["W"])
    assert np.array_equal(comp, g["comp"]) and np.array_equal(meta, g["nibbles"])


def test_prune_known_answers(orc):
    cases = {
        (5, 5, 5, 5): ((5, 5), 2 | 3 << 2),         # all equal: lower indices pruned -> keep {2,3}
        (0, 0, 0, 0): ((0, 0), 2 | 3 << 2),
        (1, -5, 3, 0): ((-5, 3), 1 | 2 << 2),
        (-128, 127, -127, 1): ((-128, -127), 0 | 2 << 2),   # |127| tie: index 1 pruned
        (2, 1, 1, 0): ((2, 1), 0 | 2 << 2),          # tie between 1 and 2: index 1 pruned
        (0, 0, 0, 9): ((0, 9), 2 | 3 << 2),
        (7, 0, 0, 0): ((7, 0), 0 | 3 << 2),
    }
    for vals, (kept, nib) in cases.items():
        comp, meta = orc.prune_compress_24(np.array([vals], np.int8))
        assert tuple(comp[0]) == kept and meta[0] == nib, vals


def test_prune_brute_force(orc):
    values = [-128, -3, -1, 0, 1, 3, 127]
    groups = np.array(list(itertools.product(values, repeat=4)), np.int8)      # 2401 groups
    comp, meta = orc.prune_compress_24(groups.reshape(1, -1))
    comp = comp.reshape(-1, 2)
    for g, c, m in zip(groups, comp, meta):
        order = sorted(range(4), key=lambda i: (abs(int(g[i])), i))
        keep = sorted(order[2:])
        assert m == (keep[0] | keep[1] << 2)
        assert c[0] == g[keep[0]] and c[1] == g[keep[1]]
    # decompress round trip
    dense = orc.decompress_24(comp.reshape(1, -1), meta, 1, groups.size)
    for g, d in zip(groups, dense.reshape(-1, 4)):
        order = sorted(range(4), key=lambda i: (abs(int(g[i])), i))
        exp = g.copy()
        exp[order[0]] = 0
        exp[order[1]] = 0
        assert np.array_equal(d, exp)


def test_mt19937_standard_answer(orc):
    # C++ [rand.predef]: the 10000th invocation of a default-constructed mt19937 is 4123659995
    assert orc.mt19937(5489, 10000)[-1] == 4123659995
    assert orc.mt19937(5489, 10000)[-1] == golden("pack")["mt19937_5489_10000"][0]


def test_pack_reference_vectors(orc):
    g = golden("pack")
    raw = g["raw"]
    # the reference test's input: std::mt19937(42) & 0xF (tests/test_pack_metadata.cu:124-126)
    assert np.array_equal((orc.mt19937(42, raw.size) & 0xF).astype(np.uint8), raw)
    words = orc.pack_metadata_ref(raw, 16, 128)
    assert np.array_equal(words, g["words"])
    gfx = orc.pack_metadata_gfx950(raw, 16, 128)
    assert np.array_equal(gfx, g["gfx950"])
    assert np.array_equal(orc.unpack_metadata_gfx950(gfx, 16, 128), raw)
    # the gfx950 buffer is a permutation of the reference words
    assert np.array_equal(np.sort(gfx), np.sort(words.ravel()))


def test_pack_ragged_rows(orc):
    g = golden("pack")
    raw = g["raw_ragged"]
    gfx = orc.pack_metadata_gfx950(raw, 20, 96)
    assert np.array_equal(gfx, g["gfx950_ragged"])
    assert np.array_equal(orc.unpack_metadata_gfx950(gfx, 20, 96), raw)


def test_sparse_gemm_golden_and_dense_equivalence(orc):
    g = golden("sparse")
    comp, meta = orc.prune_compress_24(g["W"])
    assert np.array_equal(comp, g["comp"]) and np.array_equal(meta, g["nibbles"])
    C = orc.sparse_gemm_s32(comp, g["x"], meta, 32, 128)
    assert np.array_equal(C, g["C"])
    # sparse == dense GEMM of the decompressed weights, computed by numpy
    rng = np.random.default_rng(9)
    W = rng.integers(-127, 128, (48, 256)).astype(np.int8)
    x = rng.integers(-127, 128, (5, 256)).astype(np.int8)
    comp, meta = orc.prune_compress_24(W)
    dense = orc.decompress_24(comp, meta, 48, 256)
    assert np.array_equal(orc.sparse_gemm_s32(comp, x, meta, 48, 256),
                          (x.astype(np.int64) @ dense.astype(np.int64).T).astype(np.int32))
    # exactly two nonzeros survive per group of 4 when the weights have no zeros
    Wn = np.where(W == 0, 1, W).astype(np.int8)
    comp, meta = orc.prune_compress_24(Wn)
    d = orc.decompress_24(comp, meta, 48, 256).reshape(48, 64, 4)
    assert np.all((d != 0).sum(axis=2) == 2)


# ---- conv -----------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["3x3_p1", "2x2_s2", "3x3_d2"])
def test_conv_golden(orc, name):
    g = golden("conv")
    pad, stride, dil = (int(v) for v in g[name + "_cfg"])
    out = orc.conv2d_nhwc_s32(g[name + "_x"], g[name + "_w"], (pad, pad), (stride, stride), (dil, dil))
    assert np.array_equal(out, g[name + "_out"])


def test_conv_matches_torch_asymmetric(orc):
    import torch
    rng = np.random.default_rng(11)
    x = rng.integers(-127, 128, (2, 9, 6, 16)).astype(np.int8)
    w = rng.integers(-127, 128, (5, 3, 2, 16)).astype(np.int8)
    out = orc.conv2d_nhwc_s32(x, w, (1, 0), (2, 1), (1, 2))
    ref = torch.nn.functional.conv2d(torch.from_numpy(x).permute(0, 3, 1, 2).double(),
                                     torch.from_numpy(w).permute(0, 3, 1, 2).double(),
                                     stride=(2, 1), padding=(1, 0), dilation=(1, 2))
    assert np.array_equal(out, ref.permute(0, 2, 3, 1).numpy().astype(np.int32))


# ---- depthwise conv2d (src/nn/int8_depthwise_conv2d.cu) -------------------------------

def _ulp16(v):
    """Spacing of fp16 values at |v| (subnormal spacing below the normal range)."""
    a = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return 2.0 ** (e - 10)


def _dw_case(rng, N, C, H, W, k, bias=True):
    x = rng.uniform(-1, 1, (N, C, H, W)).astype(np.float16)
    w = rng.integers(-127, 128, (C,) + k).astype(np.int8)
    ws = rng.uniform(0.005, 0.05, C).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, C).astype(np.float16) if bias else None
    return x, w, ws, b


def _dw_torch64(x, w, ws, b, pad, stride, dil):
    """float64 depthwise conv (groups = C) with the weights dequantized as the reference does
    ((float)q * scale, one fp32 product), plus the bias, and sum |terms| for the error bound."""
    import torch
    wf = (w.astype(np.float32) * ws.astype(np.float32)[:, None, None]).astype(np.float64)
    C = w.shape[0]
    xt = torch.from_numpy(x.astype(np.float64))
    y = torch.nn.functional.conv2d(xt, torch.from_numpy(wf)[:, None], stride=stride, padding=pad,
                                   dilation=dil, groups=C)
    s = torch.nn.functional.conv2d(xt.abs(), torch.from_numpy(np.abs(wf))[:, None], stride=stride,
                                   padding=pad, dilation=dil, groups=C)
    if b is not None:
        bb = torch.from_numpy(b.astype(np.float64))[None, :, None, None]
        y = y + bb
        s = s + bb.abs()
    return y.numpy(), s.numpy()


@pytest.mark.parametrize("N,C,H,W,k,pad,stride,dil", [
    (1, 16, 16, 16, (3, 3), (1, 1), (1, 1), (1, 1)),
    (2, 5, 9, 13, (3, 2), (2, 0), (2, 1), (1, 2)),
    (1, 3, 20, 7, (5, 5), (2, 3), (1, 2), (2, 1)),
    (3, 4, 6, 6, (1, 1), (0, 0), (1, 1), (1, 1)),
    (1, 2, 11, 17, (7, 1), (3, 0), (3, 1), (1, 1)),
])
def test_depthwise_matches_torch_float64(orc, N, C, H, W, k, pad, stride, dil):
    rng = np.random.default_rng(N * 100 + C)
    x, w, ws, b = _dw_case(rng, N, C, H, W, k, bias=(C % 2 == 0))
    y = orc.depthwise_conv2d(x, w, ws, b, pad, stride, dil).astype(np.float64)
    ref, s = _dw_torch64(x, w, ws, b, pad, stride, dil)
    assert y.shape == ref.shape
    taps = k[0] * k[1] + 1
    bound = _ulp16(ref) / 2 + 2.0 ** -23 * taps * s + 2.0 ** -25
    assert np.all(np.abs(y - ref) <= bound)


@pytest.mark.parametrize("C,H,W,bias", [(16, 16, 16, True), (32, 32, 32, True), (64, 8, 8, False)])
def test_depthwise_reference_test_shapes(orc, C, H, W, bias):
    """The reference test's depthwise cases and criterion (test_int8_special_conv.cu:71-141,
    269-271: max |gpu - float ref| < 0.01), against the float64 reference."""
    rng = np.random.default_rng(C)
    x, w, ws, b = _dw_case(rng, 1, C, H, W, (3, 3), bias)
    y = orc.depthwise_conv2d(x, w, ws, b, (1, 1)).astype(np.float64)
    ref, _ = _dw_torch64(x, w, ws, b, (1, 1), (1, 1), (1, 1))
    assert np.abs(y - ref).max() < 0.01


def test_depthwise_closed_forms(orc):
    # A 1x1 kernel is one rounded fp32 product, then the fp32 bias add and fp16 rounding.
    rng = np.random.default_rng(5)
    x, w, ws, b = _dw_case(rng, 2, 6, 5, 7, (1, 1))
    y = orc.depthwise_conv2d(x, w, ws, b)
    wf = w[:, 0, 0].astype(np.float32) * ws.astype(np.float32)
    want = (x.astype(np.float32) * wf[None, :, None, None] + b.astype(np.float32)[None, :, None, None])
    assert np.array_equal(y.view(np.uint16), want.astype(np.float16).view(np.uint16))
    # Taps outside the image are skipped: with pad = k - 1 the corner output of a 2x2
    # kernel sees only the image's corner pixel, times the kernel's opposite corner tap.
    xs = np.ones((1, 1, 4, 4), np.float16)
    wk = np.array([[[1, 2], [3, 4]]], np.int8)
    y = orc.depthwise_conv2d(xs, wk, np.array([1.0], np.float16), None, (1, 1)).astype(np.float32)
    assert y[0, 0, 0, 0] == 4 and y[0, 0, 0, 1] == 7 and y[0, 0, 1, 1] == 10 and y[0, 0, 4, 4] == 1


def test_depthwise_accumulates_with_fma(orc):
    """Each tap is one fused multiply-add into the running sum (nvcc contracts
    `sum += inp * w` by default): with taps x*w and (-x)*w the exact sum is 0, an unfused
    sum gives 0, and the fused one leaves the rounding error of fl(x*w), which is not 0."""
    x = np.array([[[[1001.0, -1001.0]]]], np.float16)
    wk = np.array([[[127, 127]]], np.int8)
    ws = np.array([7.99], np.float16)
    y = orc.depthwise_conv2d(x, wk, ws, None).astype(np.float64)
    wf = np.float32(127) * np.float32(ws[0])
    exact = np.float64(x[0, 0, 0, 0]) * np.float64(wf)
    resid = np.float64(np.float32(exact)) - exact       # fl(x*w) - x*w, in exact arithmetic
    assert resid != 0
    assert y[0, 0, 0, 0] == np.float64(np.float16(resid))


# ---- ConvTranspose2d k=2 s=2 (src/nn/int8_conv_transpose2d.cu) ----------------------

def _ct_case(rng, N, C_in, H, W, C_out, bias=True):
    x = rng.uniform(-1, 1, (N, C_in, H, W)).astype(np.float16)
    w = rng.integers(-127, 128, (4 * C_out, C_in)).astype(np.int8)
    ws = rng.uniform(0.005, 0.05, C_out).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, C_out).astype(np.float16) if bias else None
    return x, w, ws, b


def _ct_weight4(w_rep, C_in, C_out):
    """Repacked rows (co*4 + kh*2 + kw, ci) back to the (C_in, C_out, 2, 2) ConvTranspose2d
    weight (int8_conv_transpose2d.cuh:13-16)."""
    return w_rep.reshape(C_out, 2, 2, C_in).transpose(3, 0, 1, 2)


@pytest.mark.parametrize("N,C_in,H,W,C_out", [(1, 32, 6, 5, 8), (2, 7, 3, 4, 3), (1, 64, 4, 4, 16)])
def test_conv_transpose_int32_stage_matches_torch(orc, N, C_in, H, W, C_out):
    import torch
    rng = np.random.default_rng(C_in + H)
    x, w, ws, b = _ct_case(rng, N, C_in, H, W, C_out)
    y, acc = orc.conv_transpose2d_k2s2(x, w, ws, b, with_acc=True)
    # Per-pixel quantization through the (separately pinned) row quantizer.
    rows = x.transpose(0, 2, 3, 1).reshape(-1, C_in)
    q, s = orc.quantize_rows(rows)
    qn = q.reshape(N, H, W, C_in).transpose(0, 3, 1, 2).astype(np.float64)
    w4 = _ct_weight4(w, C_in, C_out).astype(np.float64)
    ref = torch.nn.functional.conv_transpose2d(torch.from_numpy(qn), torch.from_numpy(w4), stride=2).numpy()
    assert np.array_equal(acc, ref.astype(np.int32))
    # FP16 output: float64 of the dequantized operands, within the two fp16 roundings.
    sn = s.reshape(N, 1, H, W).astype(np.float64)
    ref16 = torch.nn.functional.conv_transpose2d(torch.from_numpy(qn * sn),
                                                 torch.from_numpy(w4 * ws.astype(np.float64)[None, :, None, None]),
                                                 bias=torch.from_numpy(b.astype(np.float64)), stride=2).numpy()
    # Two fp16 roundings: of the GEMM value g = y - bias, then of g + bias.
    g = ref16 - b.astype(np.float64)[None, :, None, None]
    bound = _ulp16(g) / 2 + _ulp16(ref16) / 2 + 2.0 ** -21 * np.abs(g) + 2.0 ** -25
    assert np.all(np.abs(y.astype(np.float64) - ref16) <= bound)


@pytest.mark.parametrize("C_in,H,W,C_out,bias", [(32, 16, 16, 64, True), (64, 8, 8, 32, True),
                                                 (16, 32, 32, 16, False)])
def test_conv_transpose_reference_test_shapes(orc, C_in, H, W, C_out, bias):
    """The reference test's cases and criterion (test_int8_special_conv.cu:146-257, 275-279:
    max |gpu - float ref| < 0.5 and mean < 0.1 against the unquantized float conv)."""
    import torch
    rng = np.random.default_rng(C_in * 7 + C_out)
    x, w, ws, b = _ct_case(rng, 1, C_in, H, W, C_out, bias)
    y = orc.conv_transpose2d_k2s2(x, w, ws, b).astype(np.float64)
    w4 = _ct_weight4(w, C_in, C_out).astype(np.float64) * ws.astype(np.float64)[None, :, None, None]
    ref = torch.nn.functional.conv_transpose2d(torch.from_numpy(x.astype(np.float64)), torch.from_numpy(w4),
                                               bias=None if b is None else torch.from_numpy(b.astype(np.float64)),
                                               stride=2).numpy()
    d = np.abs(y - ref)
    assert d.max() < 0.5 and d.mean() < 0.1


def test_conv_transpose_bias_after_rounding(orc):
    """The bias is added to the already-rounded FP16 GEMM value (the scatter step,
    int8_conv_transpose2d.cu:99-101): output == half(half(acc * as * ws) + bias)."""
    rng = np.random.default_rng(9)
    x, w, ws, b = _ct_case(rng, 1, 16, 3, 3, 4)
    y0 = orc.conv_transpose2d_k2s2(x, w, ws, None)
    y1 = orc.conv_transpose2d_k2s2(x, w, ws, b)
    want = (y0.astype(np.float32) + b.astype(np.float32)[None, :, None, None]).astype(np.float16)
    assert np.array_equal(y1.view(np.uint16), want.view(np.uint16))


# ---- weight quantization (python/forge/nn/linear.py:168-173, :235-238) --------------

def _torch_weight_quant(w):
    """The reference's own expression (linear.py:168-173), run by torch on the CPU."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(w)).to(torch.float32)
    scale = t.abs().amax(dim=1).clamp(min=1e-8) / 127.0
    q = (t / scale.unsqueeze(1)).round().clamp(-127, 127).to(torch.int8)
    return q.numpy(), scale.to(torch.float16).numpy(), scale.numpy()


@pytest.mark.parametrize("N,K,dist", [(64, 256, "normal"), (33, 100, "uniform"), (8, 4096, "outlier"),
                                      (5, 7, "normal")])
def test_weight_quant_matches_reference_expression(orc, N, K, dist):
    rng = np.random.default_rng(N + K)
    if dist == "normal":
        w = rng.standard_normal((N, K)).astype(np.float32) * 0.02
    elif dist == "uniform":
        w = rng.uniform(-3, 3, (N, K)).astype(np.float32)
    else:
        w = rng.standard_normal((N, K)).astype(np.float32)
        w[:, rng.choice(K, 4, replace=False)] *= 50
    q, s16, s32 = orc.quantize_weight_rows(w)
    tq, ts16, ts32 = _torch_weight_quant(w)
    assert np.array_equal(q, tq)
    assert np.array_equal(s16.view(np.uint16), ts16.view(np.uint16))
    assert np.array_equal(s32.view(np.uint32), ts32.view(np.uint32))


def test_weight_quant_closed_forms(orc):
    # the absmax element maps to +-127; a zero row gets scale 1e-8/127 and q = 0; half-way
    # quotients round to even (w = 2.5 * scale with scale = 1 -> 2).
    w = np.array([[0.5, -1.0, 0.25, 0.0], [0, 0, 0, 0], [127.0, 2.5, -3.5, 0.5]], np.float32)
    q, s16, s32 = orc.quantize_weight_rows(w)
    assert q[0, 1] == -127 and q[0, 0] == 64 and q[0, 2] == 32       # 63.5 -> 64, 31.75 -> 32
    assert s32[1] == np.float32(np.float32(1e-8) / np.float32(127)) and not q[1].any()
    assert s32[2] == 1.0 and list(q[2]) == [127, 2, -4, 0]           # RNE: 2.5 -> 2, -3.5 -> -4, 0.5 -> 0


def test_sparse_weight_prep_is_the_composition(orc):
    """prepare_sparse_weight == quantize rows, then the (separately pinned) prune + gfx950 pack;
    decompressing gives the 2:4-pruned quantized weights."""
    rng = np.random.default_rng(11)
    w = rng.standard_normal((48, 256)).astype(np.float32)
    comp, meta, s16 = orc.prepare_sparse_weight(w)
    q, s16b, _ = orc.quantize_weight_rows(w)
    assert np.array_equal(s16.view(np.uint16), s16b.view(np.uint16))
    raw = orc.unpack_metadata_gfx950(meta, 48, 256)
    d = orc.decompress_24(comp, raw, 48, 256).reshape(48, 64, 4)
    qg = q.reshape(48, 64, 4)
    kept = d != 0
    assert np.all(kept.sum(axis=2) <= 2)
    assert np.array_equal(d[kept], qg[kept])


@pytest.mark.parametrize("threads", [2, 3, 7])
def test_threaded_forms_equal_single_thread(orc, threads):
    """The threaded loops used for whole-output comparisons at full size give the single-threaded
    functions' bits, also where the rows do not divide evenly among the threads."""
    rng = np.random.default_rng(threads)
    M, K, N = 37, 96, 53
    A = rng.integers(-127, 128, (M, K)).astype(np.int8)
    B = rng.integers(-127, 128, (N, K)).astype(np.int8)
    assert np.array_equal(orc.gemm_s32(A, B, threads=threads), orc.gemm_s32(A, B))
    act = rng.uniform(1e-3, 5e-2, M).astype(np.float32)
    ws = rng.uniform(1e-3, 5e-2, N).astype(np.float16)
    b = rng.uniform(-0.5, 0.5, N).astype(np.float16)
    for bias in (b, None):
        assert np.array_equal(orc.gemm_dequant(A, B, act, ws, bias, threads=threads).view(np.uint16),
                              orc.gemm_dequant(A, B, act, ws, bias).view(np.uint16))
    Wd = rng.integers(-127, 128, (48, 128)).astype(np.int8)
    comp, raw = orc.prune_compress_24(Wd)
    x = rng.integers(-127, 128, (29, 128)).astype(np.int8)
    assert np.array_equal(orc.sparse_gemm_s32(comp, x, raw, 48, 128, threads=threads),
                          orc.sparse_gemm_s32(comp, x, raw, 48, 128))
    xc = rng.integers(-127, 128, (3, 9, 7, 16)).astype(np.int8)
    wc = rng.integers(-127, 128, (5, 3, 2, 16)).astype(np.int8)
    for pad, stride, dil in (((1, 1), (1, 1), (1, 1)), ((0, 1), (2, 1), (1, 2))):
        assert np.array_equal(orc.conv2d_nhwc_s32(xc, wc, pad, stride, dil, threads=threads),
                              orc.conv2d_nhwc_s32(xc, wc, pad, stride, dil))


def test_splitk_reduce_matches_numpy(orc):
    """ws + bias in float32, then float16 RNE (numpy's conversion is IEEE RNE, pinned above);
    without bias a plain conversion. Values near fp16 ties, overflow to inf and subnormals."""
    rng = np.random.default_rng(8)
    ws = (rng.standard_normal((23, 41)) * 50).astype(np.float32)
    ws[0, :4] = [65520.0, -65520.0, 1e-6, 2049.0]
    b = (rng.standard_normal(41) * 3).astype(np.float16)
    got = orc.splitk_reduce(ws, b)
    ref = (ws + b.astype(np.float32)[None, :]).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    assert np.array_equal(orc.splitk_reduce(ws).view(np.uint16), ws.astype(np.float16).view(np.uint16))
    assert np.isinf(got[0, 0]) or abs(float(ws[0, 0]) + float(b[0])) < 65520
