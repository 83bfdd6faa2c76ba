"""CPU checks of the C-ABI library: it loads, exports every symbol include/forge_amd.h
declares (and the C++ API symbols of include/forge/), and rejects invalid arguments
before touching a device. No compute calls are made here."""
import ctypes
import os
import re
import subprocess

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "forge_amd.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(forge_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    import forge_amd
    return forge_amd.load()


def test_header_declares_the_path():
    syms = declared_symbols()
    for s in ["forge_quantize_activation", "forge_dequantize_bias", "forge_int8_gemm_dequant",
              "forge_int8_linear", "forge_int8_gemm", "forge_sparse_int8_gemm", "forge_sparse_int8_linear",
              "forge_sparse_int8_gemm_plan", "forge_prune_compress_24", "forge_pack_metadata",
              "forge_splitk_reduce", "forge_int8_conv2d_forward", "forge_int8_conv2d_workspace_size",
              "forge_int8_conv_transpose2d_k2s2_forward", "forge_int8_conv_transpose2d_k2s2_workspace_size",
              "forge_int8_depthwise_conv2d_forward", "forge_quantize_weight_rows",
              "forge_prepare_sparse_weight"]:
        assert s in syms


def test_library_exports_every_declared_symbol(lib):
    from forge_amd import _lib
    for name in declared_symbols():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} missing from the ctypes table"


def test_cpp_api_symbols_exported():
    from forge_amd import LIB_PATH
    out = subprocess.run(["nm", "-DC", "--defined-only", LIB_PATH], capture_output=True, text=True).stdout
    for sym in ["forge::quant::fused_quantize_activation(", "forge::quant::fused_dequantize_bias(",
                "forge::quant::fused_quantize_activation_kernel(", "forge::quant::fused_dequantize_bias_kernel(",
                "forge::gemm::int8_gemm_dequant(", "forge::gemm::int8_linear(", "forge::gemm::int8_gemm(",
                "forge::gemm::get_compute_capability(", "forge::gemm::has_wmma_int8(",
                "forge::gemm::int8_dp4a_gemm_dequant(", "forge::gemm::int8_dp4a_linear(",
                "forge::gemm::sparse_int8_gemm_plan(", "forge::gemm::sparse_int8_gemm(",
                "forge::gemm::sparse_int8_linear(", "forge::gemm::sparse_int8_linear_fused(",
                "forge::gemm::splitk_reduce(", "forge::sparsity::prune_compress_24(",
                "forge::sparsity::pack_metadata(", "forge::sparsity::prune_compress_kernel(",
                "forge::sparsity::pack_metadata_kernel(", "forge::nn::int8_conv2d_forward(",
                "forge::nn::int8_conv2d_workspace_size(", "forge::nn::int8_conv_transpose2d_k2s2_forward(",
                "forge::nn::int8_conv_transpose2d_k2s2_workspace_size(", "forge::nn::int8_depthwise_conv2d_forward(",
                "forge::last_error("]:
        assert sym in out, sym


def test_status_strings(lib):
    assert lib.forge_status_string(0) == b"ok"
    assert b"invalid" in lib.forge_status_string(-1)


def test_nonpositive_dims_are_noops(lib):
    # reference launchers return early on M, N or K <= 0 (src/gemm/int8_dense.cu:195)
    assert lib.forge_int8_gemm_dequant(None, None, None, None, None, None, 0, 16, 16, None) == 0
    assert lib.forge_quantize_activation(None, None, None, 0, 8, None) == 0
    assert lib.forge_sparse_int8_gemm(None, None, None, None, None, None, None, 4, -1, 16, None, 1, None, -1) == 0
    assert lib.forge_prune_compress_24(None, None, None, 0, 0, None) == 0


def test_invalid_arguments_rejected_without_device(lib):
    fake = ctypes.c_void_p(4096)   # never dereferenced: validation fails first
    assert lib.forge_int8_gemm_dequant(None, fake, fake, fake, None, fake, 4, 16, 16, None) == -1
    assert lib.forge_quantize_activation(fake, None, fake, 4, 8, None) == -1
    assert lib.forge_quantize_activation_twopass(fake, fake, fake, 4, 8, 0, None) == -1
    assert lib.forge_quantize_activation_twopass(fake, fake, fake, 4, 8, 2048, None) == -1
    # sparse contract: K % 64 == 0 and N % 16 == 0 (include/forge/gemm/int8_sparse.cuh:12)
    assert lib.forge_sparse_int8_gemm(fake, fake, fake, fake, fake, None, fake, 4, 96, 16, None, 1, None, -1) == -1
    assert lib.forge_sparse_int8_gemm(fake, fake, fake, fake, fake, None, fake, 4, 128, 24, None, 1, None, -1) == -1
    assert lib.forge_sparse_int8_linear(fake, fake, fake, fake, None, fake, 4, 96, 16, fake, fake, None, 1, None,
                                        -1) == -1
    # misaligned compressed weights
    assert lib.forge_sparse_int8_gemm(ctypes.c_void_p(4097), fake, fake, fake, fake, None, fake, 4, 128, 16, None,
                                      1, None, -1) == -1
    assert lib.forge_prune_compress_24(fake, fake, fake, 4, 6, None) == -1     # K % 4
    assert lib.forge_pack_metadata(fake, fake, 4, 48, None) == -1             # K % 32
    out = ctypes.c_int()
    assert lib.forge_sparse_int8_gemm_plan(4, 64, 16, 1, 1, -1, None, ctypes.byref(out)) == -1


def test_conv_workspace_size(lib):
    # [col fp16 | col int8 | act_scale | gemm_out] for one sample, 256-byte aligned regions
    n = lib.forge_int8_conv2d_workspace_size(8, 16, 16, 16, 3, 3, 1, 1, 1, 1, 1, 1)
    M, K = 16 * 16, 8 * 9
    up = lambda b: (b + 255) // 256 * 256
    assert n == up(M * K * 2) + up(M * K) + up(M * 4) + up(M * 16 * 2)
    assert n >= M * K * 2 + M * K + M * 4 + M * 16 * 2     # at least the reference's size


def test_weight_prep_argument_checks(lib):
    fake = ctypes.c_void_p(4096)   # never dereferenced: validation fails first
    assert lib.forge_prepare_sparse_weight(fake, 0, fake, fake, fake, 4, 48, None) == -1      # K % 32
    assert lib.forge_prepare_sparse_weight(ctypes.c_void_p(4100), 0, fake, fake, fake, 4, 64, None) == -1
    assert lib.forge_quantize_weight_rows(fake, 0, None, fake, 4, 64, None) == -1
    assert lib.forge_quantize_weight_rows(None, 0, None, None, 0, 64, None) == 0


def test_conv_transpose_workspace_size(lib):
    # int8_conv_transpose2d.cu:107-123: col fp16 + col int8 + act_scale + w_scale_rep + gemm_out
    M, K, Ng = 16 * 16, 32, 4 * 64
    assert lib.forge_int8_conv_transpose2d_k2s2_workspace_size(32, 16, 16, 64) == \
        M * K * 2 + M * K + M * 4 + Ng * 2 + M * Ng * 2
    assert lib.forge_int8_conv_transpose2d_k2s2_workspace_size(0, 16, 16, 64) == 0


def test_special_conv_argument_checks(lib):
    fake = ctypes.c_void_p(4096)   # never dereferenced: validation fails first
    # N, C_in or C_out <= 0 returns early, as the reference does (int8_conv_transpose2d.cu:139)
    assert lib.forge_int8_conv_transpose2d_k2s2_forward(None, None, None, None, None, 0, 8, 4, 4, 8, None, None) == 0
    assert lib.forge_int8_conv_transpose2d_k2s2_forward(fake, fake, fake, None, fake, 1, 8, 4, 4, 8, None, None) == -1
    assert lib.forge_int8_depthwise_conv2d_forward(None, None, None, None, None, 1, 0, 4, 4, 3, 3, 1, 1, 1, 1, 1, 1,
                                                   None) == 0
    assert lib.forge_int8_depthwise_conv2d_forward(fake, fake, None, None, fake, 1, 4, 4, 4, 3, 3, 1, 1, 1, 1, 1, 1,
                                                   None) == -1
    assert lib.forge_int8_depthwise_conv2d_forward(fake, fake, fake, None, fake, 1, 4, 4, 4, 3, 3, 1, 1, 0, 1, 1, 1,
                                                   None) == -1
    # an empty output (kernel larger than the padded input) launches nothing
    assert lib.forge_int8_depthwise_conv2d_forward(fake, fake, fake, None, fake, 1, 4, 2, 2, 5, 5, 0, 0, 1, 1, 1, 1,
                                                   None) == 0


def test_ops_module_imports_like_the_gpu_tests():
    """`from forge_amd import ops` (the form every GPU test uses) resolves on the CPU."""
    import forge_amd
    from forge_amd import ops
    assert ops is forge_amd.ops
    assert callable(ops.int8_linear) and callable(ops.sparse_int8_gemm)


def test_nn_modules_match_reference_state_dict_layout():
    """QuantizedLinear / SparseLinear expose the reference's parameter and buffer names,
    shapes and dtypes (python/forge/nn/linear.py:135-154, :206-226), so its state_dict loads."""
    import torch
    from forge_amd.nn import QuantizedLinear, SparseLinear
    q = QuantizedLinear(256, 96)
    sd = q.state_dict()
    assert set(sd) == {"w_int8", "w_scale", "bias"}
    assert sd["w_int8"].shape == (96, 256) and sd["w_int8"].dtype == torch.int8
    assert sd["w_scale"].shape == (96,) and sd["w_scale"].dtype == torch.float16
    assert sd["bias"].dtype == torch.float16
    assert "bias" not in QuantizedLinear(256, 96, bias=False).state_dict()
    s = SparseLinear(256, 96)
    sd = s.state_dict()
    assert set(sd) == {"W_comp", "w_meta", "w_scale", "bias"}
    assert sd["W_comp"].shape == (96, 128) and sd["W_comp"].dtype == torch.int8
    assert sd["w_meta"].shape == (96, 8) and sd["w_meta"].dtype == torch.int32
    import pytest
    with pytest.raises(ValueError):
        SparseLinear(100, 96)


def test_cpp_caller_links_and_reports_errors(lib):
    """The test suite's C++ caller of include/forge/**.h (tests/cpp) loads against the library
    (every forge:: symbol it uses resolves) and sees forge::last_error() = FORGE_EINVAL for a
    call with null operands, which the C ABI rejects before any device work."""
    from forge_amd import _lib
    path = os.path.join(ROOT, "tests", "cpp", "lib", "libforge_caller.so")
    if not os.path.exists(path):
        pytest.skip("tests/cpp caller not built (python tests/cpp/build.py)")
    caller = ctypes.CDLL(path)
    caller.caller_last_error_after_bad_call.restype = ctypes.c_int
    assert caller.caller_last_error_after_bad_call() == _lib.FORGE_EINVAL


def test_probe_library_loads_and_checks_arguments():
    """libforge_probes.so (the measurement probes behind bench.py --probes) is a separate
    library: it exports the three probes, rejects bad arguments before any launch, and the
    product library does not carry them."""
    from forge_amd import build
    if not os.path.exists(build.PROBE_LIB):
        pytest.skip("probe library not built")
    P = ctypes.CDLL(build.PROBE_LIB)
    fake = ctypes.c_void_p(4096)
    P.probe_stream.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    P.probe_dma.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                            ctypes.c_void_p, ctypes.c_void_p]
    assert P.probe_mfma_lds(None, fake, fake, 4, 4, 1, 1, None) == -1
    assert P.probe_mfma_lds(fake, fake, fake, 0, 4, 1, 1, None) == -1
    assert P.probe_stream(fake, 1000, 4, fake, None) == -1                      # not a multiple of 16 * wgs
    assert P.probe_dma(fake, 1 << 30, 8192, 3, 0, 0, fake, None) == -1          # share not a power of two <= 32
    assert P.probe_dma(fake, 1 << 20, 8192, 1, 0, 0, fake, None) == -1          # rows do not fit in `bytes`
    assert P.probe_dma(fake, 1 << 30, 8000, 1, 0, 0, fake, None) == -1          # K % 128
    import forge_amd
    assert not hasattr(forge_amd.load(), "probe_mfma_lds")
