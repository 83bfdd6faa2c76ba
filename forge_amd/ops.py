"""PyTorch-facing operators over the C-ABI.

Names and argument meaning follow the reference's pybind module for this path
(python/forge/csrc/bindings.cpp:446-576, registered at :1120-1142): tensors in,
tensors out, launched on torch's current HIP stream. Extensions (INT32-output GEMMs,
NHWC conv, the sparse planner) follow the C-ABI names in include/forge_amd.h.
torch supplies device memory and the stream only; every computation runs in
libforge_amd.so.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib

_lib_check = _lib.check


def _p(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _need(t: torch.Tensor, dtype: torch.dtype, name: str, numel: Optional[int] = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if numel is not None and t.numel() < numel:
        raise ValueError(f"{name} holds {t.numel()} elements, needs {numel}")


def _call(name: str, *args) -> None:
    _lib_check(getattr(_lib.load(), name)(*args), name)


# ---- quantization (bindings.cpp:448-476) -----------------------------------------

def fused_quantize_activation(input: torch.Tensor, M: int, K: int, out: Optional[torch.Tensor] = None,
                              scales: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """bindings.cpp:448-461 (allocating); `out` / `scales` may be passed to reuse buffers."""
    _need(input, torch.float16, "input", M * K)
    if out is None:
        out = torch.empty((M, K), dtype=torch.int8, device=input.device)
    if scales is None:
        scales = torch.empty((M,), dtype=torch.float32, device=input.device)
    _need(out, torch.int8, "out", M * K)
    _need(scales, torch.float32, "scales", M)
    _call("forge_quantize_activation", _p(input), _p(out), _p(scales), M, K, _stream())
    return out, scales


def fused_quantize_activation_twopass(input: torch.Tensor, M: int, K: int, threads: int = 256):
    """The exported two-pass kernel launched with `threads` per row (quantize.cuh:17-21)."""
    _need(input, torch.float16, "input", M * K)
    out = torch.empty((M, K), dtype=torch.int8, device=input.device)
    scales = torch.empty((M,), dtype=torch.float32, device=input.device)
    _call("forge_quantize_activation_twopass", _p(input), _p(out), _p(scales), M, K, threads, _stream())
    return out, scales


def fused_dequantize_bias(input: torch.Tensor, act_scale: torch.Tensor, w_scale: torch.Tensor,
                          bias: Optional[torch.Tensor], M: int, N: int) -> torch.Tensor:
    _need(input, torch.int32, "input", M * N)
    _need(act_scale, torch.float32, "act_scale", M)
    _need(w_scale, torch.float16, "w_scale", N)
    if bias is not None:
        _need(bias, torch.float16, "bias", N)
    out = torch.empty((M, N), dtype=torch.float16, device=input.device)
    _call("forge_dequantize_bias", _p(input), _p(act_scale), _p(w_scale), _p(bias), _p(out), M, N, _stream())
    return out


# ---- decode K-split slots (extension) ---------------------------------------------

def ksplit_last() -> Tuple[int, int]:
    """(slot, K parts) of this thread's last decode launch: slot -1 = no slot (unsplit)."""
    import ctypes
    slot, parts = ctypes.c_int(), ctypes.c_int()
    _call("forge_ksplit_last", ctypes.addressof(slot), ctypes.addressof(parts))
    return slot.value, parts.value


def last_route() -> str:
    """The engine of this thread's last GEMM launch (forge_last_route)."""
    return _lib.load().forge_last_route().decode()


def ksplit_reset() -> None:
    """Zeroes every decode K-split slot of the current device on torch's current stream."""
    _call("forge_ksplit_reset", _stream())


def slots_in_use() -> Tuple[int, int, int, int]:
    """(K-split slots held, K-split slots, packed-weight slots held, packed-weight slots) of
    the current device (forge_slots_in_use). Slots are never released; once all are held, a
    new stream or graph capture runs the unsplit decode / in-place fused path (same bits)."""
    import ctypes
    v = [ctypes.c_int() for _ in range(4)]
    _call("forge_slots_in_use", *[ctypes.addressof(x) for x in v])
    return tuple(x.value for x in v)


# ---- device queries (int8_gemm.cuh:18-24) ----------------------------------------

def get_compute_capability(device: int = 0) -> int:
    """forge_get_compute_capability: 100 * major + 10 * minor of the HIP device (gfx950 -> 950)."""
    import ctypes
    v = ctypes.c_int()
    _call("forge_get_compute_capability", device, ctypes.addressof(v))
    return v.value


def has_int8_matrix_cores(device: int = 0) -> bool:
    """forge_has_int8_matrix_cores (the reference's has_wmma_int8): INT8 MFMA / SMFMAC present."""
    import ctypes
    v = ctypes.c_int()
    _call("forge_has_int8_matrix_cores", device, ctypes.addressof(v))
    return bool(v.value)


# ---- dense GEMM (bindings.cpp:498-519) -------------------------------------------

def int8_linear(x: torch.Tensor, w_int8: torch.Tensor, w_scale: torch.Tensor, bias: Optional[torch.Tensor],
                scratch_a_int8: torch.Tensor, scratch_a_scale: torch.Tensor,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """int8_dense.cuh:37-48; `out` may be passed to reuse an (M, N) FP16 buffer."""
    M, K = x.shape
    N = w_int8.shape[0]
    _need(x, torch.float16, "x")
    _need(w_int8, torch.int8, "w_int8", N * K)
    _need(w_scale, torch.float16, "w_scale", N)
    if bias is not None:
        _need(bias, torch.float16, "bias", N)
    _need(scratch_a_int8, torch.int8, "scratch_a_int8", M * K)
    _need(scratch_a_scale, torch.float32, "scratch_a_scale", M)
    if out is None:
        out = torch.empty((M, N), dtype=torch.float16, device=x.device)
    _need(out, torch.float16, "out", M * N)
    _call("forge_int8_linear", _p(x), _p(w_int8), _p(w_scale), _p(bias), _p(out), M, K, N,
          _p(scratch_a_int8), _p(scratch_a_scale), _stream())
    return out


def int8_gemm_dequant(A: torch.Tensor, B: torch.Tensor, act_scale: torch.Tensor, w_scale: torch.Tensor,
                      bias: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    M, K = A.shape
    N = B.shape[0]
    _need(A, torch.int8, "A")
    _need(B, torch.int8, "B", N * K)
    _need(act_scale, torch.float32, "act_scale", M)
    _need(w_scale, torch.float16, "w_scale", N)
    if bias is not None:
        _need(bias, torch.float16, "bias", N)
    if out is None:
        out = torch.empty((M, N), dtype=torch.float16, device=A.device)
    _need(out, torch.float16, "out", M * N)
    _call("forge_int8_gemm_dequant", _p(A), _p(B), _p(act_scale), _p(w_scale), _p(bias), _p(out),
          M, K, N, _stream())
    return out


def int8_gemm(A: torch.Tensor, B: torch.Tensor, act_scale: torch.Tensor, w_scale: torch.Tensor,
              bias: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The reference's capability-dispatching int8_gemm (int8_gemm.cu:26-46): on gfx950 always the
    matrix-core GEMM, so it equals int8_gemm_dequant."""
    M, K = A.shape
    N = B.shape[0]
    _need(A, torch.int8, "A")
    _need(B, torch.int8, "B", N * K)
    _need(act_scale, torch.float32, "act_scale", M)
    _need(w_scale, torch.float16, "w_scale", N)
    if bias is not None:
        _need(bias, torch.float16, "bias", N)
    if out is None:
        out = torch.empty((M, N), dtype=torch.float16, device=A.device)
    _need(out, torch.float16, "out", M * N)
    _call("forge_int8_gemm", _p(A), _p(B), _p(act_scale), _p(w_scale), _p(bias), _p(out), M, K, N, _stream())
    return out


def int8_gemm_s32(A: torch.Tensor, B: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    M, K = A.shape
    N = B.shape[0]
    _need(A, torch.int8, "A")
    _need(B, torch.int8, "B", N * K)
    if out is None:
        out = torch.empty((M, N), dtype=torch.int32, device=A.device)
    _need(out, torch.int32, "out", M * N)
    _call("forge_int8_gemm_s32", _p(A), _p(B), _p(out), M, K, N, _stream())
    return out


# ---- sparsity (bindings.cpp:558-575) ------------------------------------------------

def prune_compress_24(weight: torch.Tensor, compressed: torch.Tensor, metadata_raw: torch.Tensor,
                      N: int, K: int) -> None:
    _need(weight, torch.int8, "weight", N * K)
    _need(compressed, torch.int8, "compressed", N * K // 2)
    _need(metadata_raw, torch.uint8, "metadata_raw", N * K // 4)
    _call("forge_prune_compress_24", _p(weight), _p(compressed), _p(metadata_raw), N, K, _stream())


def pack_metadata(meta_raw: torch.Tensor, meta_packed: torch.Tensor, N: int, K: int) -> None:
    _need(meta_raw, torch.uint8, "meta_raw", N * K // 4)
    _need(meta_packed, torch.int32, "meta_packed", N * K // 32)
    _call("forge_pack_metadata", _p(meta_raw), _p(meta_packed), N, K, _stream())


def unpack_metadata(meta_packed: torch.Tensor, meta_raw: torch.Tensor, N: int, K: int) -> None:
    _need(meta_packed, torch.int32, "meta_packed", N * K // 32)
    _need(meta_raw, torch.uint8, "meta_raw", N * K // 4)
    _call("forge_unpack_metadata", _p(meta_packed), _p(meta_raw), N, K, _stream())


# ---- sparse GEMM (bindings.cpp:521-556) -----------------------------------------------

def sparse_int8_gemm_plan(M: int, K: int, N_out: int, split_k: int = 0, have_workspace: bool = True,
                          tile: int = -1) -> Tuple[int, int]:
    import ctypes
    t, s = ctypes.c_int(), ctypes.c_int()
    _call("forge_sparse_int8_gemm_plan", M, K, N_out, split_k, 1 if have_workspace else 0, tile,
          ctypes.addressof(t), ctypes.addressof(s))
    return t.value, s.value


def sparse_int8_gemm(W_comp: torch.Tensor, x_int8: torch.Tensor, w_meta: torch.Tensor, act_scale: torch.Tensor,
                     w_scale: torch.Tensor, bias: Optional[torch.Tensor] = None,
                     splitk_workspace: Optional[torch.Tensor] = None, split_k: int = 1, tile: int = -1,
                     out: Optional[torch.Tensor] = None) -> torch.Tensor:
    M, K = x_int8.shape
    N = W_comp.shape[0]
    _need(W_comp, torch.int8, "W_comp", N * K // 2)
    _need(x_int8, torch.int8, "x_int8")
    _need(w_meta, torch.int32, "w_meta", N * K // 32)
    _need(act_scale, torch.float32, "act_scale", M)
    _need(w_scale, torch.float16, "w_scale", N)
    if bias is not None:
        _need(bias, torch.float16, "bias", N)
    if splitk_workspace is not None:
        _need(splitk_workspace, torch.float32, "splitk_workspace", M * N)
    if out is None:
        out = torch.empty((M, N), dtype=torch.float16, device=x_int8.device)
    _need(out, torch.float16, "out", M * N)
    _call("forge_sparse_int8_gemm", _p(W_comp), _p(x_int8), _p(w_meta), _p(act_scale), _p(w_scale), _p(bias),
          _p(out), M, K, N, _p(splitk_workspace), split_k, _stream(), tile)
    return out


def sparse_int8_gemm_s32(W_comp: torch.Tensor, x_int8: torch.Tensor, w_meta: torch.Tensor,
                         out: Optional[torch.Tensor] = None) -> torch.Tensor:
    M, K = x_int8.shape
    N = W_comp.shape[0]
    _need(W_comp, torch.int8, "W_comp", N * K // 2)
    _need(x_int8, torch.int8, "x_int8")
    _need(w_meta, torch.int32, "w_meta", N * K // 32)
    if out is None:
        out = torch.empty((M, N), dtype=torch.int32, device=x_int8.device)
    _need(out, torch.int32, "out", M * N)
    _call("forge_sparse_int8_gemm_s32", _p(W_comp), _p(x_int8), _p(w_meta), _p(out), M, K, N, _stream())
    return out


def sparse_int8_linear_fused(M: int, K: int, N_out: int) -> bool:
    import ctypes
    f = ctypes.c_int()
    _call("forge_sparse_int8_linear_fused", M, K, N_out, ctypes.addressof(f))
    return bool(f.value)


def sparse_int8_linear(x: torch.Tensor, W_comp: torch.Tensor, w_meta: torch.Tensor, w_scale: torch.Tensor,
                       bias: Optional[torch.Tensor], scratch_x_int8: torch.Tensor, scratch_x_scale: torch.Tensor,
                       splitk_workspace: Optional[torch.Tensor] = None, split_k: int = 1,
                       path: int = -1, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """int8_sparse.cuh:92-105; `out` may be passed to reuse an (M, N) FP16 buffer."""
    M, K = x.shape
    N = W_comp.shape[0]
    _need(x, torch.float16, "x")
    _need(W_comp, torch.int8, "W_comp", N * K // 2)
    _need(w_meta, torch.int32, "w_meta", N * K // 32)
    _need(w_scale, torch.float16, "w_scale", N)
    if bias is not None:
        _need(bias, torch.float16, "bias", N)
    _need(scratch_x_int8, torch.int8, "scratch_x_int8", M * K)
    _need(scratch_x_scale, torch.float32, "scratch_x_scale", M)
    ws = splitk_workspace
    # As the reference binding (bindings.cpp:531-537): an automatic split without a caller
    # workspace gets one allocated here when the planner splits.
    if ws is None and split_k <= 0 and sparse_int8_gemm_plan(M, K, N, split_k, True)[1] > 1:
        ws = torch.empty((M, N), dtype=torch.float32, device=x.device)
    if ws is not None:
        _need(ws, torch.float32, "splitk_workspace", M * N)
    if out is None:
        out = torch.empty((M, N), dtype=torch.float16, device=x.device)
    _need(out, torch.float16, "out", M * N)
    _call("forge_sparse_int8_linear", _p(x), _p(W_comp), _p(w_meta), _p(w_scale), _p(bias), _p(out), M, K, N,
          _p(scratch_x_int8), _p(scratch_x_scale), _p(ws), split_k, _stream(), path)
    return out


def splitk_reduce(workspace: torch.Tensor, bias: Optional[torch.Tensor], M: int, N: int,
                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """int8_sparse.cuh:107-114: FP32 (M, N) workspace [+ bias] -> FP16."""
    _need(workspace, torch.float32, "workspace", M * N)
    if bias is not None:
        _need(bias, torch.float16, "bias", N)
    if out is None:
        out = torch.empty((M, N), dtype=torch.float16, device=workspace.device)
    _need(out, torch.float16, "out", M * N)
    _call("forge_splitk_reduce", _p(workspace), _p(bias), _p(out), M, N, _stream())
    return out


# ---- conv ------------------------------------------------------------------------

def conv_out_size(i: int, pad: int, dil: int, k: int, stride: int) -> int:
    return (i + 2 * pad - dil * (k - 1) - 1) // stride + 1


def int8_conv2d_workspace_size(C_in, H, W, C_out, kH, kW, padH, padW, strideH, strideW, dilH=1, dilW=1) -> int:
    return _lib.load().forge_int8_conv2d_workspace_size(C_in, H, W, C_out, kH, kW, padH, padW, strideH, strideW,
                                                        dilH, dilW)


def int8_conv2d_forward(input: torch.Tensor, weight: torch.Tensor, w_scale: torch.Tensor,
                        bias: Optional[torch.Tensor], kH: int, kW: int, pad=(0, 0), stride=(1, 1), dil=(1, 1),
                        workspace: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """int8_conv2d.cuh:33-53; `out` may be passed to reuse an (N, C_out, H_out, W_out) FP16 buffer."""
    N, C, H, W = input.shape
    Co = weight.shape[0]
    _need(input, torch.float16, "input")
    _need(weight, torch.int8, "weight", Co * C * kH * kW)
    _need(w_scale, torch.float16, "w_scale", Co)
    if bias is not None:
        _need(bias, torch.float16, "bias", Co)
    Ho = conv_out_size(H, pad[0], dil[0], kH, stride[0])
    Wo = conv_out_size(W, pad[1], dil[1], kW, stride[1])
    nbytes = int8_conv2d_workspace_size(C, H, W, Co, kH, kW, pad[0], pad[1], stride[0], stride[1], dil[0], dil[1])
    if workspace is None:
        workspace = torch.empty((nbytes,), dtype=torch.uint8, device=input.device)
    if workspace.numel() * workspace.element_size() < nbytes:
        raise ValueError(f"workspace needs {nbytes} bytes")
    if out is None:
        out = torch.empty((N, Co, Ho, Wo), dtype=torch.float16, device=input.device)
    _need(out, torch.float16, "out", N * Co * Ho * Wo)
    _call("forge_int8_conv2d_forward", _p(input), _p(weight), _p(w_scale), _p(bias), _p(out), N, C, H, W, Co, kH, kW,
          pad[0], pad[1], stride[0], stride[1], dil[0], dil[1], _p(workspace), _stream())
    return out


def int8_conv2d_nhwc_s32(x: torch.Tensor, w: torch.Tensor, pad=(0, 0), stride=(1, 1), dil=(1, 1),
                         out: Optional[torch.Tensor] = None) -> torch.Tensor:
    N, H, W, C = x.shape
    Co, kH, kW, C2 = w.shape
    if C2 != C:
        raise ValueError("channel mismatch")
    _need(x, torch.int8, "x")
    _need(w, torch.int8, "w")
    Ho = conv_out_size(H, pad[0], dil[0], kH, stride[0])
    Wo = conv_out_size(W, pad[1], dil[1], kW, stride[1])
    if out is None:
        out = torch.empty((N, Ho, Wo, Co), dtype=torch.int32, device=x.device)
    _need(out, torch.int32, "out", N * Ho * Wo * Co)
    _call("forge_int8_conv2d_nhwc_s32", _p(x), _p(w), _p(out), N, H, W, C, Co, kH, kW, pad[0], pad[1],
          stride[0], stride[1], dil[0], dil[1], _stream())
    return out


def int8_conv2d_nhwc_dequant(x: torch.Tensor, w: torch.Tensor, act_scale: torch.Tensor, w_scale: torch.Tensor,
                             bias: Optional[torch.Tensor], pad=(0, 0), stride=(1, 1), dil=(1, 1),
                             out: Optional[torch.Tensor] = None) -> torch.Tensor:
    N, H, W, C = x.shape
    Co, kH, kW, C2 = w.shape
    if C2 != C:
        raise ValueError("channel mismatch")
    _need(x, torch.int8, "x")
    _need(w, torch.int8, "w")
    Ho = conv_out_size(H, pad[0], dil[0], kH, stride[0])
    Wo = conv_out_size(W, pad[1], dil[1], kW, stride[1])
    _need(act_scale, torch.float32, "act_scale", N * Ho * Wo)
    _need(w_scale, torch.float16, "w_scale", Co)
    if bias is not None:
        _need(bias, torch.float16, "bias", Co)
    if out is None:
        out = torch.empty((N, Ho, Wo, Co), dtype=torch.float16, device=x.device)
    _need(out, torch.float16, "out", N * Ho * Wo * Co)
    _call("forge_int8_conv2d_nhwc_dequant", _p(x), _p(w), _p(act_scale), _p(w_scale), _p(bias), _p(out), N, H, W,
          C, Co, kH, kW, pad[0], pad[1], stride[0], stride[1], dil[0], dil[1], _stream())
    return out


def int8_conv_transpose2d_k2s2_workspace_size(C_in: int, H: int, W: int, C_out: int) -> int:
    return _lib.load().forge_int8_conv_transpose2d_k2s2_workspace_size(C_in, H, W, C_out)


def int8_conv_transpose2d_k2s2_forward(input: torch.Tensor, weight: torch.Tensor, w_scale: torch.Tensor,
                                       bias: Optional[torch.Tensor], workspace: Optional[torch.Tensor] = None,
                                       out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """ConvTranspose2d, kernel 2, stride 2 (int8_conv_transpose2d.cuh:37-46): input (N, C_in, H, W)
    fp16, weight (4*C_out, C_in) int8 repacked (row co*4 + kh*2 + kw = weight[ci, co, kh, kw])."""
    N, C_in, H, W = input.shape
    Ng = weight.shape[0]
    if Ng % 4 != 0 or weight.dim() != 2 or weight.shape[1] != C_in:
        raise ValueError("weight must be (4*C_out, C_in)")
    C_out = Ng // 4
    _need(input, torch.float16, "input")
    _need(weight, torch.int8, "weight")
    _need(w_scale, torch.float16, "w_scale", C_out)
    if bias is not None:
        _need(bias, torch.float16, "bias", C_out)
    nbytes = int8_conv_transpose2d_k2s2_workspace_size(C_in, H, W, C_out)
    if workspace is None:
        workspace = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=input.device)
    if workspace.numel() * workspace.element_size() < nbytes:
        raise ValueError(f"workspace needs {nbytes} bytes")
    if out is None:
        out = torch.empty((N, C_out, 2 * H, 2 * W), dtype=torch.float16, device=input.device)
    _need(out, torch.float16, "out", N * C_out * 4 * H * W)
    _call("forge_int8_conv_transpose2d_k2s2_forward", _p(input), _p(weight), _p(w_scale), _p(bias), _p(out),
          N, C_in, H, W, C_out, _p(workspace), _stream())
    return out


def int8_depthwise_conv2d_forward(input: torch.Tensor, weight: torch.Tensor, w_scale: torch.Tensor,
                                  bias: Optional[torch.Tensor], kH: int, kW: int, pad=(0, 0), stride=(1, 1),
                                  dil=(1, 1), out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Depthwise conv2d (int8_depthwise_conv2d.cuh:28-41): input (N, C, H, W) fp16, weight
    (C, kH*kW) int8 (any shape holding C*kH*kW values), per-channel w_scale and bias."""
    N, C, H, W = input.shape
    _need(input, torch.float16, "input")
    _need(weight, torch.int8, "weight", C * kH * kW)
    _need(w_scale, torch.float16, "w_scale", C)
    if bias is not None:
        _need(bias, torch.float16, "bias", C)
    Ho = conv_out_size(H, pad[0], dil[0], kH, stride[0])
    Wo = conv_out_size(W, pad[1], dil[1], kW, stride[1])
    if out is None:
        out = torch.empty((N, C, max(Ho, 0), max(Wo, 0)), dtype=torch.float16, device=input.device)
    _need(out, torch.float16, "out", N * C * max(Ho, 0) * max(Wo, 0))
    _call("forge_int8_depthwise_conv2d_forward", _p(input), _p(weight), _p(w_scale), _p(bias), _p(out), N, C, H, W,
          kH, kW, pad[0], pad[1], stride[0], stride[1], dil[0], dil[1], _stream())
    return out


# ---- weight preparation ------------------------------------------------------------

def _weight_arg(w: torch.Tensor):
    if w.dtype not in (torch.float32, torch.float16):
        raise TypeError(f"weight must be float32 or float16, got {w.dtype}")
    if not w.is_cuda or not w.is_contiguous() or w.dim() != 2:
        raise ValueError("weight must be a contiguous 2-D device tensor")
    return 1 if w.dtype == torch.float16 else 0


def quantize_weight_rows(w: torch.Tensor, w_int8: Optional[torch.Tensor] = None,
                         w_scale: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """QuantizedLinear.quantize_weight (linear.py:168-173) on the device: (N, K) fp32/fp16 ->
    (w_int8 (N, K) int8, w_scale (N,) fp16)."""
    f16 = _weight_arg(w)
    N, K = w.shape
    if w_int8 is None:
        w_int8 = torch.empty((N, K), dtype=torch.int8, device=w.device)
    if w_scale is None:
        w_scale = torch.empty((N,), dtype=torch.float16, device=w.device)
    _need(w_int8, torch.int8, "w_int8", N * K)
    _need(w_scale, torch.float16, "w_scale", N)
    _call("forge_quantize_weight_rows", _p(w), f16, _p(w_int8), _p(w_scale), N, K, _stream())
    return w_int8, w_scale


def prepare_sparse_weight(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """SparseLinear.from_dense_weight (linear.py:231-249) in one device pass: (N, K) fp32/fp16 ->
    (W_comp (N, K/2) int8, w_meta (N, K/32) int32 in the gfx950 order, w_scale (N,) fp16)."""
    f16 = _weight_arg(w)
    N, K = w.shape
    comp = torch.empty((N, K // 2), dtype=torch.int8, device=w.device)
    meta = torch.empty((N, K // 32), dtype=torch.int32, device=w.device)
    scale = torch.empty((N,), dtype=torch.float16, device=w.device)
    _call("forge_prepare_sparse_weight", _p(w), f16, _p(comp), _p(meta), _p(scale), N, K, _stream())
    return comp, meta, scale
