"""PyTorch modules of the INT8 path, shaped like the reference's python/forge/nn/linear.py:115-254.

QuantizedLinear and SparseLinear keep the reference's parameter and buffer names, shapes and
dtypes, so a reference state_dict loads as is:
- QuantizedLinear: w_int8 (N, K) int8 buffer, w_scale (N) fp16, bias (N) fp16 or None;
- SparseLinear: W_comp (N, K/2) int8 buffer, w_meta (N, K/32) int32 buffer, w_scale, bias.
The one stored difference is the order of the 2:4 index words in w_meta: here the gfx950 SMFMAC
order (forge_pack_metadata). w_meta_from_reference / w_meta_to_reference convert a whole tensor
between the reference's row-major words (pack_metadata.cu:23-29) and this layout; the word values
and the raw nibbles are the same.

Forward runs the library (forge_int8_linear / forge_sparse_int8_linear); there is no other path.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import nn

from . import ops


def _prep_device(module_tensor: torch.Tensor) -> torch.device:
    """Weight preparation runs on the module's device, or cuda:0 for a CPU module."""
    return module_tensor.device if module_tensor.is_cuda else torch.device("cuda", 0)


def _as_weight(weight_fp: torch.Tensor, dev: torch.device) -> torch.Tensor:
    """The reference converts any float weight to float32 (linear.py:169, :234); fp16 and fp32
    go to the device as they are (the kernel widens fp16 exactly), other dtypes as float32."""
    w = weight_fp if weight_fp.dtype in (torch.float16, torch.float32) else weight_fp.to(torch.float32)
    return w.to(dev).contiguous()


class _Int8LinearFn(torch.autograd.Function):
    """Forward on the INT8 path; backward through the dequantized FP16 weight, returning the
    input and bias gradients (the reference's _Int8LinearFn, linear.py:115-132)."""

    @staticmethod
    def forward(ctx, x, w_int8, w_scale, bias, scratch_a, scratch_s):
        ctx.save_for_backward(w_int8, w_scale)
        ctx.has_bias = bias is not None
        return ops.int8_linear(x, w_int8, w_scale, bias, scratch_a, scratch_s)

    @staticmethod
    def backward(ctx, grad_output):
        w_int8, w_scale = ctx.saved_tensors
        g = grad_output.to(torch.float16)
        w16 = w_int8.to(torch.float16) * w_scale.unsqueeze(1)
        grad_x = g @ w16
        grad_bias = grad_output.sum(dim=0).to(torch.float16) if ctx.has_bias else None
        return grad_x, None, None, grad_bias, None, None


class QuantizedLinear(nn.Module):
    """INT8 linear layer: y = dequant(quantize_per_token(x) @ w_int8^T) + bias, FP16 in and out
    (linear.py:135-184)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.register_buffer("w_int8", torch.zeros(out_features, in_features, dtype=torch.int8))
        self.w_scale = nn.Parameter(torch.ones(out_features, dtype=torch.float16))
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features, dtype=torch.float16))
        else:
            self.register_parameter("bias", None)
        self._scratch_a: Optional[torch.Tensor] = None
        self._scratch_s: Optional[torch.Tensor] = None

    def _scratch(self, M: int, K: int, device):
        a = self._scratch_a
        if a is None or a.shape[0] < M or a.shape[1] != K or a.device != device:
            self._scratch_a = torch.empty(M, K, dtype=torch.int8, device=device)
            self._scratch_s = torch.empty(M, dtype=torch.float32, device=device)
        return self._scratch_a[:M], self._scratch_s[:M]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        M, K = x.shape
        a, s = self._scratch(M, K, x.device)
        return _Int8LinearFn.apply(x, self.w_int8, self.w_scale, self.bias, a, s)

    @torch.no_grad()
    def quantize_weight(self, weight_fp: torch.Tensor) -> None:
        """Per-output-row symmetric quantization (linear.py:167-173) on the device:
        scale = max(amax|w|, 1e-8) / 127, w_int8 = clamp(round(w / scale), -127, 127) (round half
        to even, IEEE division), scale stored as FP16."""
        q, scale = ops.quantize_weight_rows(_as_weight(weight_fp, _prep_device(self.w_int8)))
        self.w_int8.copy_(q)
        self.w_scale.data.copy_(scale)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, bias={self.bias is not None}"


class _SparseInt8LinearFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, W_comp, w_meta, w_scale, bias, scratch_q, scratch_s):
        # split_k = 0: the planner's automatic tile and split, as the reference module asks
        # (linear.py:191-193); every plan gives the same bits.
        return ops.sparse_int8_linear(x, W_comp, w_meta, w_scale, bias, scratch_q, scratch_s, split_k=0)

    @staticmethod
    def backward(ctx, grad_output):
        raise NotImplementedError("SparseLinear has no backward (as in the reference, linear.py:201-203)")


class SparseLinear(nn.Module):
    """2:4 structured-sparse INT8 linear layer (linear.py:206-254). in_features % 64 == 0 and
    out_features % 16 == 0."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True):
        super().__init__()
        if in_features % 64 != 0 or out_features % 16 != 0:
            raise ValueError("SparseLinear needs in_features % 64 == 0 and out_features % 16 == 0")
        self.in_features = in_features
        self.out_features = out_features
        self.register_buffer("W_comp", torch.zeros(out_features, in_features // 2, dtype=torch.int8))
        self.register_buffer("w_meta", torch.zeros(out_features, in_features // 32, dtype=torch.int32))
        self.w_scale = nn.Parameter(torch.ones(out_features, dtype=torch.float16))
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features, dtype=torch.float16))
        else:
            self.register_parameter("bias", None)
        self._scratch_q: Optional[torch.Tensor] = None
        self._scratch_s: Optional[torch.Tensor] = None

    def _scratch(self, M: int, K: int, device):
        q = self._scratch_q
        if q is None or q.shape[0] < M or q.shape[1] != K or q.device != device:
            self._scratch_q = torch.empty(M, K, dtype=torch.int8, device=device)
            self._scratch_s = torch.empty(M, dtype=torch.float32, device=device)
        return self._scratch_q[:M], self._scratch_s[:M]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        M, K = x.shape
        q, s = self._scratch(M, K, x.device)
        return _SparseInt8LinearFn.apply(x, self.W_comp, self.w_meta, self.w_scale, self.bias, q, s)

    @torch.no_grad()
    def from_dense_weight(self, weight_fp: torch.Tensor) -> None:
        """linear.py:231-249 in one device pass (forge_prepare_sparse_weight): quantize per row
        as QuantizedLinear does, prune 2:4 (the lower-magnitude pair of each group of 4),
        compress, and write the index words in the gfx950 order."""
        comp, meta, scale = ops.prepare_sparse_weight(_as_weight(weight_fp, _prep_device(self.W_comp)))
        self.W_comp.copy_(comp)
        self.w_meta.copy_(meta)
        self.w_scale.data.copy_(scale)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, sparse=2:4")


def w_meta_from_reference(w_meta_ref: torch.Tensor) -> torch.Tensor:
    """The reference's (N, K/32) int32 index words (word (n, c) = sum_g nib[n, 8c+g] << 4g,
    pack_metadata.cu:23-29) -> the same words in the gfx950 order, on the tensor's device."""
    N, W = w_meta_ref.shape
    K = W * 32
    words = w_meta_ref.contiguous().view(torch.int32)
    shifts = torch.arange(0, 32, 4, device=words.device, dtype=torch.int32)
    nibs = torch.bitwise_and(torch.bitwise_right_shift(words.unsqueeze(-1), shifts), 0xF).to(torch.uint8)
    raw = nibs.reshape(-1).contiguous()
    out = torch.empty(N, W, dtype=torch.int32, device=words.device)
    ops.pack_metadata(raw, out, N, K)
    return out


def w_meta_to_reference(w_meta: torch.Tensor) -> torch.Tensor:
    """Inverse of w_meta_from_reference: gfx950-order words -> the reference's row-major words."""
    N, W = w_meta.shape
    K = W * 32
    raw = torch.empty(N * K // 4, dtype=torch.uint8, device=w_meta.device)
    ops.unpack_metadata(w_meta.contiguous(), raw, N, K)
    nibs = raw.view(N, W, 8).to(torch.int32)
    shifts = torch.arange(0, 32, 4, device=w_meta.device, dtype=torch.int32)
    return torch.bitwise_left_shift(nibs, shifts).sum(dim=-1, dtype=torch.int64).to(torch.int32)
