"""numpy front end of the CPU oracle (oracle/forge_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker. The product (forge_amd) never
imports it. fp16 arrays are passed as uint16 bit patterns (np.float16 views).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "lib", "liboracle.so")
_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I = ctypes.c_int


def _declare(L: ctypes.CDLL) -> None:
    L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_f16_to_f32.restype = ctypes.c_float
    L.orc_f32_to_f16.argtypes = [ctypes.c_float]
    L.orc_f32_to_f16.restype = ctypes.c_uint16
    L.orc_quantize_rows.argtypes = [_P, _P, _P, _I, _I]
    L.orc_dequantize_bias.argtypes = [_P, _P, _P, _P, _P, _I, _I]
    L.orc_gemm_s32.argtypes = [_P, _P, _P, _I, _I, _I]
    L.orc_splitk_reduce.argtypes = [_P, _P, _P, _I, _I]
    L.orc_gemm_s32_rows.argtypes = [_P, _P, _P, _I, _I, _I, _I]
    L.orc_dequant_epilogue.argtypes = [_P, _P, _P, _P, _P, _I, _I]
    L.orc_gemm_dequant.argtypes = [_P, _P, _P, _P, _P, _P, _I, _I, _I]
    L.orc_linear.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I]
    L.orc_prune_compress_24.argtypes = [_P, _P, _P, _I, _I]
    L.orc_decompress_24.argtypes = [_P, _P, _P, _I, _I]
    L.orc_pack_metadata_ref.argtypes = [_P, _P, _I, _I]
    L.orc_pack_metadata_gfx950.argtypes = [_P, _P, _I, _I]
    L.orc_unpack_metadata_gfx950.argtypes = [_P, _P, _I, _I]
    L.orc_sparse_gemm_s32.argtypes = [_P, _P, _P, _P, _I, _I, _I]
    L.orc_conv_out_size.argtypes = [_I, _I, _I, _I, _I]
    L.orc_conv_out_size.restype = _I
    L.orc_conv2d_nhwc_s32.argtypes = [_P, _P, _P] + [_I] * 13
    L.orc_depthwise_conv2d.argtypes = [_P] * 5 + [_I] * 12
    L.orc_quantize_weight_rows.argtypes = [_P] * 4 + [_I] * 2
    L.orc_conv_transpose2d_k2s2.argtypes = [_P] * 6 + [_I] * 5
    L.orc_mt19937_seed.argtypes = [_P, ctypes.c_uint32]
    L.orc_mt19937_next.argtypes = [_P]
    L.orc_mt19937_next.restype = ctypes.c_uint32
    L.orc_time_gemm_dequant_rows.argtypes = [_P, _P, _P, _P, _P, _P, _I, _I, _I]
    L.orc_time_gemm_dequant_rows.restype = ctypes.c_double
    L.orc_time_gemm_dequant_rows_mt.argtypes = [_P] * 6 + [_I] * 4
    L.orc_time_gemm_dequant_rows_mt.restype = ctypes.c_double
    L.orc_gemm_s32_mt.argtypes = [_P, _P, _P, _I, _I, _I, _I]
    L.orc_gemm_dequant_mt.argtypes = [_P] * 6 + [_I] * 4
    L.orc_sparse_gemm_s32_mt.argtypes = [_P] * 4 + [_I] * 4
    L.orc_conv2d_nhwc_s32_mt.argtypes = [_P, _P, _P] + [_I] * 14


def cpu_threads() -> int:
    """Threads for the oracle's threaded loops: the host's cores, at most 16 (a GPU box's
    CPU share per GPU)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _u16(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint16) if a.dtype == np.float16 else a.astype(np.uint16)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    L = lib()
    return np.array([L.orc_f32_to_f16(float(v)) for v in x], dtype=np.uint16)


def quantize_rows(x16: np.ndarray):
    x = _u16(x16)
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    s = np.empty((M,), np.float32)
    lib().orc_quantize_rows(_p(x), _p(q), _p(s), M, K)
    return q, s


def dequantize_bias(acc, act_scale, w_scale16, bias16=None):
    acc = np.ascontiguousarray(acc, np.int32)
    M, N = acc.shape
    as_ = np.ascontiguousarray(act_scale, np.float32)
    ws = _u16(w_scale16)
    b = None if bias16 is None else _u16(bias16)
    out = np.empty((M, N), np.uint16)
    lib().orc_dequantize_bias(_p(acc), _p(as_), _p(ws), _p(b), _p(out), M, N)
    return out.view(np.float16)


def splitk_reduce(ws, bias16=None):
    """fp32 (M, N) split-K workspace [+ fp16 bias] -> fp16 (int8_sparse.cu:99-111)."""
    ws = np.ascontiguousarray(ws, np.float32)
    M, N = ws.shape
    b = None if bias16 is None else _u16(bias16)
    out = np.empty((M, N), np.uint16)
    lib().orc_splitk_reduce(_p(ws), _p(b), _p(out), M, N)
    return out.view(np.float16)


def gemm_s32(A, B, threads: int = 1):
    A = np.ascontiguousarray(A, np.int8)
    B = np.ascontiguousarray(B, np.int8)
    M, K = A.shape
    N = B.shape[0]
    C = np.empty((M, N), np.int32)
    if threads > 1:
        lib().orc_gemm_s32_mt(_p(A), _p(B), _p(C), M, K, N, threads)
    else:
        lib().orc_gemm_s32(_p(A), _p(B), _p(C), M, K, N)
    return C


def dequant_epilogue(acc, act_scale, w_scale16, bias16=None):
    acc = np.ascontiguousarray(acc, np.int32)
    M, N = acc.shape
    as_ = np.ascontiguousarray(act_scale, np.float32)
    ws = _u16(w_scale16)
    b = None if bias16 is None else _u16(bias16)
    out = np.empty((M, N), np.uint16)
    lib().orc_dequant_epilogue(_p(acc), _p(as_), _p(ws), _p(b), _p(out), M, N)
    return out.view(np.float16)


def gemm_dequant(A, B, act_scale, w_scale16, bias16=None, threads: int = 1):
    if threads <= 1:
        return dequant_epilogue(gemm_s32(A, B), act_scale, w_scale16, bias16)
    A = np.ascontiguousarray(A, np.int8)
    B = np.ascontiguousarray(B, np.int8)
    M, K = A.shape
    N = B.shape[0]
    as_ = np.ascontiguousarray(act_scale, np.float32)
    ws = _u16(w_scale16)
    b = None if bias16 is None else _u16(bias16)
    out = np.empty((M, N), np.uint16)
    lib().orc_gemm_dequant_mt(_p(A), _p(B), _p(as_), _p(ws), _p(b), _p(out), M, K, N, threads)
    return out.view(np.float16)


def linear(x16, W, w_scale16, bias16=None, threads: int = 1):
    q, s = quantize_rows(x16)
    return gemm_dequant(q, W, s, w_scale16, bias16, threads=threads), q, s


def prune_compress_24(w):
    w = np.ascontiguousarray(w, np.int8)
    N, K = w.shape
    comp = np.empty((N, K // 2), np.int8)
    meta = np.empty((N * (K // 4),), np.uint8)
    lib().orc_prune_compress_24(_p(w), _p(comp), _p(meta), N, K)
    return comp, meta


def decompress_24(comp, meta_raw, N, K):
    comp = np.ascontiguousarray(comp, np.int8)
    meta = np.ascontiguousarray(meta_raw, np.uint8)
    w = np.empty((N, K), np.int8)
    lib().orc_decompress_24(_p(comp), _p(meta), _p(w), N, K)
    return w


def pack_metadata_ref(meta_raw, N, K):
    meta = np.ascontiguousarray(meta_raw, np.uint8)
    out = np.empty((N, K // 32), np.uint32)
    lib().orc_pack_metadata_ref(_p(meta), _p(out), N, K)
    return out


def pack_metadata_gfx950(meta_raw, N, K):
    meta = np.ascontiguousarray(meta_raw, np.uint8)
    out = np.empty((N * (K // 32),), np.uint32)
    lib().orc_pack_metadata_gfx950(_p(meta), _p(out), N, K)
    return out


def unpack_metadata_gfx950(packed, N, K):
    packed = np.ascontiguousarray(packed, np.uint32)
    out = np.empty((N * (K // 4),), np.uint8)
    lib().orc_unpack_metadata_gfx950(_p(packed), _p(out), N, K)
    return out


def sparse_gemm_s32(W_comp, x, meta_raw, N, K, threads: int = 1):
    W_comp = np.ascontiguousarray(W_comp, np.int8)
    x = np.ascontiguousarray(x, np.int8)
    meta = np.ascontiguousarray(meta_raw, np.uint8)
    M = x.shape[0]
    C = np.empty((M, N), np.int32)
    if threads > 1:
        lib().orc_sparse_gemm_s32_mt(_p(W_comp), _p(x), _p(meta), _p(C), M, K, N, threads)
    else:
        lib().orc_sparse_gemm_s32(_p(W_comp), _p(x), _p(meta), _p(C), M, K, N)
    return C


def conv_out_size(i, pad, dil, k, stride):
    return lib().orc_conv_out_size(i, pad, dil, k, stride)


def conv2d_nhwc_s32(x, w, pad=(0, 0), stride=(1, 1), dil=(1, 1), threads: int = 1):
    x = np.ascontiguousarray(x, np.int8)
    w = np.ascontiguousarray(w, np.int8)
    N, H, W, C = x.shape
    Co, kH, kW, C2 = w.shape
    assert C2 == C
    Ho = conv_out_size(H, pad[0], dil[0], kH, stride[0])
    Wo = conv_out_size(W, pad[1], dil[1], kW, stride[1])
    out = np.empty((N, Ho, Wo, Co), np.int32)
    args = (N, H, W, C, Co, kH, kW, pad[0], pad[1], stride[0], stride[1], dil[0], dil[1])
    if threads > 1:
        lib().orc_conv2d_nhwc_s32_mt(_p(x), _p(w), _p(out), *args, threads)
    else:
        lib().orc_conv2d_nhwc_s32(_p(x), _p(w), _p(out), *args)
    return out


def quantize_weight_rows(w):
    """w (N, K) float (converted to fp32 as the reference does) -> (q int8 (N, K),
    scale fp16 (N,), scale fp32 (N,))."""
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    q = np.empty((N, K), np.int8)
    s16 = np.empty(N, np.uint16)
    s32 = np.empty(N, np.float32)
    lib().orc_quantize_weight_rows(_p(w), _p(q), _p(s16), _p(s32), N, K)
    return q, s16.view(np.float16), s32


def prepare_sparse_weight(w):
    """SparseLinear.from_dense_weight (linear.py:231-249): quantize rows, prune 2:4, compress,
    pack the index words in the gfx950 layout. -> (W_comp (N, K/2) int8, w_meta (N*K/32,)
    uint32, w_scale fp16 (N,))."""
    q, s16, _ = quantize_weight_rows(w)
    N, K = q.shape
    comp, raw = prune_compress_24(q)
    return comp, pack_metadata_gfx950(raw, N, K), s16


def depthwise_conv2d(x16, w, w_scale16, bias16=None, pad=(0, 0), stride=(1, 1), dil=(1, 1)):
    """x16 (N, C, H, W) fp16, w (C, kH, kW) int8 -> (N, C, Ho, Wo) fp16."""
    x = _u16(x16)
    w = np.ascontiguousarray(w, np.int8)
    N, C, H, W = x.shape
    C2, kH, kW = w.shape
    assert C2 == C
    Ho = conv_out_size(H, pad[0], dil[0], kH, stride[0])
    Wo = conv_out_size(W, pad[1], dil[1], kW, stride[1])
    out = np.zeros((N, C, max(Ho, 0), max(Wo, 0)), np.uint16)
    ws = _u16(w_scale16)
    b = None if bias16 is None else _u16(bias16)
    lib().orc_depthwise_conv2d(_p(x), _p(w), _p(ws), _p(b), _p(out), N, C, H, W, kH, kW,
                               pad[0], pad[1], stride[0], stride[1], dil[0], dil[1])
    return out.view(np.float16)


def conv_transpose2d_k2s2(x16, w_rep, w_scale16, bias16=None, with_acc=False):
    """x16 (N, C_in, H, W) fp16, w_rep (4*C_out, C_in) int8 (row co*4 + kh*2 + kw) ->
    (N, C_out, 2H, 2W) fp16, and the INT32 GEMM stage in the same layout if with_acc."""
    x = _u16(x16)
    w = np.ascontiguousarray(w_rep, np.int8)
    N, C_in, H, W = x.shape
    C_out = w.shape[0] // 4
    assert w.shape == (4 * C_out, C_in)
    out = np.empty((N, C_out, 2 * H, 2 * W), np.uint16)
    acc = np.empty((N, C_out, 2 * H, 2 * W), np.int32) if with_acc else None
    ws = _u16(w_scale16)
    b = None if bias16 is None else _u16(bias16)
    lib().orc_conv_transpose2d_k2s2(_p(x), _p(w), _p(ws), _p(b), _p(out), _p(acc), N, C_in, H, W, C_out)
    return (out.view(np.float16), acc) if with_acc else out.view(np.float16)


def mt19937(seed: int, count: int) -> np.ndarray:
    state = ctypes.create_string_buffer(624 * 4 + 8)
    L = lib()
    L.orc_mt19937_seed(ctypes.addressof(state), seed)
    return np.array([L.orc_mt19937_next(ctypes.addressof(state)) for _ in range(count)],
                    dtype=np.uint32)


def time_gemm_dequant_rows_mt(A, B, act_scale, w_scale16, bias16, rows, threads):
    """time_gemm_dequant_rows split over output rows on `threads` POSIX threads."""
    A = np.ascontiguousarray(A, np.int8)
    B = np.ascontiguousarray(B, np.int8)
    K = A.shape[1]
    N = B.shape[0]
    as_ = np.ascontiguousarray(act_scale, np.float32)
    ws = _u16(w_scale16)
    b = None if bias16 is None else _u16(bias16)
    out = np.empty((rows, N), np.uint16)
    secs = lib().orc_time_gemm_dequant_rows_mt(_p(A), _p(B), _p(as_), _p(ws), _p(b), _p(out), rows, K, N, threads)
    return secs, out.view(np.float16)


def time_gemm_dequant_rows(A, B, act_scale, w_scale16, bias16, rows):
    A = np.ascontiguousarray(A, np.int8)
    B = np.ascontiguousarray(B, np.int8)
    K = A.shape[1]
    N = B.shape[0]
    as_ = np.ascontiguousarray(act_scale, np.float32)
    ws = _u16(w_scale16)
    b = None if bias16 is None else _u16(bias16)
    out = np.empty((rows, N), np.uint16)
    secs = lib().orc_time_gemm_dequant_rows(_p(A), _p(B), _p(as_), _p(ws), _p(b), _p(out),
                                            rows, K, N)
    return secs, out.view(np.float16)
