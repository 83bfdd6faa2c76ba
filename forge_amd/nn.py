"""PyTorch modules of the INT8 path, shaped like the reference's python/forge/nn/linear.py:115-254.

QuantizedLinear and SparseLinear keep the reference's parameter and buffer names, shapes and
dtypes:
- QuantizedLinear: w_int8 (N, K) int8 buffer, w_scale (N) fp16, bias (N) fp16 or None;
- SparseLinear: W_comp (N, K/2) int8 buffer, w_meta (N, K/32) int32 buffer, w_scale, bias.
The one stored difference is the order of the 2:4 index words in w_meta: here the gfx950 SMFMAC
order (forge_pack_metadata), in the reference the row-major order (pack_metadata.cu:23-29); the
word values and the raw nibbles are the same. SparseLinear's state_dict carries layout version 2
in its metadata (torch's per-module `version`); load_state_dict converts w_meta from the
reference order when the version is lower or absent (a reference checkpoint: the reference
module has torch's default version 1), so a reference state_dict loads as is and computes the
reference's outputs. w_meta_from_reference / w_meta_to_reference convert a whole tensor on any
device.

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
    out_features % 16 == 0.

    State-dict layout version 2: w_meta in the gfx950 word order. Loading a state_dict whose
    metadata says version 1 or nothing (the reference's own modules save version 1) converts
    w_meta from the reference's row-major order first."""

    _version = 2

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

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                              error_msgs):
        version = local_metadata.get("version", None) if local_metadata else None
        key = prefix + "w_meta"
        if (version is None or version < 2) and key in state_dict:
            meta = state_dict[key]
            if meta.dim() != 2 or meta.shape[1] * 32 != self.in_features or meta.shape[0] != self.out_features:
                error_msgs.append(f"{key}: expected a ({self.out_features}, {self.in_features // 32}) tensor of the "
                                  f"reference's index words, got {tuple(meta.shape)}")
                return
            state_dict = dict(state_dict)
            state_dict[key] = w_meta_from_reference(meta.to(torch.int32))
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                                      error_msgs)

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


def _gfx950_word_positions(N: int, W: int, device) -> torch.Tensor:
    """Position in the gfx950 layout of reference word (n, c) (row-major index n * W + c):
    (n / 16) * W * 16 + c * R + n % 16, R = the rows of n's 16-row block (16, or fewer in a
    ragged last block), as forge_pack_metadata stores them."""
    n = torch.arange(N, device=device, dtype=torch.int64).unsqueeze(1)
    c = torch.arange(W, device=device, dtype=torch.int64).unsqueeze(0)
    blk = n // 16
    rows = torch.clamp(N - 16 * blk, max=16)
    return (blk * W * 16 + c * rows + n % 16).reshape(-1)


def w_meta_from_reference(w_meta_ref: torch.Tensor) -> torch.Tensor:
    """The reference's (N, K/32) int32 index words (word (n, c) = sum_g nib[n, 8c+g] << 4g,
    pack_metadata.cu:23-29) -> the same words in the gfx950 order, on the tensor's device."""
    N, W = w_meta_ref.shape
    src = w_meta_ref.contiguous().view(torch.int32).reshape(-1)
    out = torch.empty(N * W, dtype=torch.int32, device=src.device)
    out[_gfx950_word_positions(N, W, src.device)] = src
    return out.view(N, W)


def w_meta_to_reference(w_meta: torch.Tensor) -> torch.Tensor:
    """Inverse of w_meta_from_reference: gfx950-order words -> the reference's row-major words."""
    N, W = w_meta.shape
    src = w_meta.contiguous().view(torch.int32).reshape(-1)
    return src[_gfx950_word_positions(N, W, src.device)].view(N, W).clone()
