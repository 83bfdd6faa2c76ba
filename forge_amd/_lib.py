"""ctypes binding of the C-ABI in include/forge_amd.h (libforge_amd.so).

Loading fails loudly when the library has not been built: there is no CPU or
PyTorch fallback for any operator of this package.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libforge_amd.so")

FORGE_OK = 0
FORGE_EINVAL = -1
FORGE_ENODEV = -2
FORGE_ERANGE = -3

_P = ctypes.c_void_p
_I = ctypes.c_int

# name -> (restype, argtypes); mirrors include/forge_amd.h one to one.
SIGNATURES = {
    "forge_status_string": (ctypes.c_char_p, [_I]),
    "forge_init": (_I, []),
    "forge_ksplit_last": (_I, [_P, _P]),
    "forge_ksplit_reset": (_I, [_P]),
    "forge_slots_in_use": (_I, [_P, _P, _P, _P]),
    "forge_last_route": (ctypes.c_char_p, []),
    "forge_get_compute_capability": (_I, [_I, _P]),
    "forge_has_int8_matrix_cores": (_I, [_I, _P]),
    "forge_quantize_activation": (_I, [_P, _P, _P, _I, _I, _P]),
    "forge_quantize_activation_twopass": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "forge_dequantize_bias": (_I, [_P, _P, _P, _P, _P, _I, _I, _P]),
    "forge_int8_gemm_dequant": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "forge_int8_gemm": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "forge_int8_linear": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _P, _P, _P]),
    "forge_int8_gemm_s32": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "forge_int8_linear_noalloc": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "forge_prune_compress_24": (_I, [_P, _P, _P, _I, _I, _P]),
    "forge_pack_metadata": (_I, [_P, _P, _I, _I, _P]),
    "forge_unpack_metadata": (_I, [_P, _P, _I, _I, _P]),
    "forge_sparse_int8_gemm_plan": (_I, [_I, _I, _I, _I, _I, _I, _P, _P]),
    "forge_sparse_int8_gemm": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _I, _P, _I]),
    "forge_sparse_int8_gemm_s32": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "forge_sparse_int8_linear_fused": (_I, [_I, _I, _I, _P]),
    "forge_sparse_int8_linear": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _P, _P, _I, _P, _I]),
    "forge_splitk_reduce": (_I, [_P, _P, _P, _I, _I, _P]),
    "forge_int8_conv2d_workspace_size": (ctypes.c_size_t, [_I] * 12),
    "forge_int8_conv2d_forward": (_I, [_P, _P, _P, _P, _P] + [_I] * 13 + [_P, _P]),
    "forge_int8_conv2d_nhwc_s32": (_I, [_P, _P, _P] + [_I] * 13 + [_P]),
    "forge_int8_conv2d_nhwc_dequant": (_I, [_P, _P, _P, _P, _P, _P] + [_I] * 13 + [_P]),
    "forge_quantize_weight_rows": (_I, [_P, _I, _P, _P, _I, _I, _P]),
    "forge_prepare_sparse_weight": (_I, [_P, _I, _P, _P, _P, _I, _I, _P]),
    "forge_int8_conv_transpose2d_k2s2_workspace_size": (ctypes.c_size_t, [_I] * 4),
    "forge_int8_conv_transpose2d_k2s2_forward": (_I, [_P] * 5 + [_I] * 5 + [_P, _P]),
    "forge_int8_depthwise_conv2d_forward": (_I, [_P] * 5 + [_I] * 12 + [_P]),
}

_lib = None


class ForgeError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Returns the loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ForgeError(
                f"forge_amd native library not found at {LIB_PATH}; "
                "build it with `python -m forge_amd.build` (hipcc, gfx950)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(status: int, what: str = "") -> None:
    if status != FORGE_OK:
        msg = load().forge_status_string(status)
        raise ForgeError(f"{what}: status {status} ({msg.decode() if msg else '?'})")
