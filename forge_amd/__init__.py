"""forge_amd: the reference's INT8 quantized-inference path (forge::quant, forge::gemm,
forge::sparsity, forge::nn int8 conv) as a gfx950-native HIP library.

The product is libforge_amd.so (C-ABI in include/forge_amd.h, C++ API in
include/forge/). This package builds it (forge_amd.build), binds it with ctypes
(forge_amd._lib) and exposes torch-tensor operators (forge_amd.ops).
"""
from ._lib import ForgeError, LIB_PATH, load  # noqa: F401

__all__ = ["ForgeError", "LIB_PATH", "load", "ops"]


def __getattr__(name):
    # importlib (not `from . import ops`): the from-import would probe this hook again
    # through hasattr() before the submodule is bound, and recurse.
    if name == "ops":
        import importlib
        return importlib.import_module(".ops", __name__)
    raise AttributeError(name)
