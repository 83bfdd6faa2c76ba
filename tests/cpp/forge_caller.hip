// A C++ caller of the drop-in API, written the way the reference's own C++ tests call it:
// it includes only include/forge/**.h, calls forge::quant / forge::gemm by their reference
// names, and launches the exported quantize kernel with <<<M, threads>>> as
// tests/test_quantize.cu:50-55 does. Linked against libforge_amd.so; the Python tests load
// it with ctypes and compare its results with the oracle. Each entry returns the call's
// status (forge::last_error(), or the launch's hipError_t).
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "forge/status.h"
#include "forge/quant/quantize.h"
#include "forge/quant/dequantize.h"
#include "forge/gemm/int8_dense.h"
#include "forge/gemm/int8_dp4a.h"
#include "forge/gemm/int8_sparse.h"

extern "C" int caller_quantize_kernel(const void* x, void* q, float* scales, int M, int K, int threads,
                                      void* stream)
{
    // The reference test launches the exported kernel directly: grid = rows, any block size.
    forge::quant::fused_quantize_activation_kernel<<<M, threads, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const __half*>(x), static_cast<int8_t*>(q), scales, K);
    return static_cast<int>(hipGetLastError());
}

extern "C" int caller_quantize(const void* x, void* q, float* scales, int M, int K, void* stream)
{
    forge::quant::fused_quantize_activation(static_cast<const __half*>(x), static_cast<int8_t*>(q), scales, M, K,
                                            static_cast<hipStream_t>(stream));
    return forge::last_error();
}

extern "C" int caller_dequantize_bias(const int32_t* acc, const float* act_scale, const void* w_scale,
                                      const void* bias, void* out, int M, int N, void* stream)
{
    forge::quant::fused_dequantize_bias(acc, act_scale, static_cast<const __half*>(w_scale),
                                        static_cast<const __half*>(bias), static_cast<__half*>(out), M, N,
                                        static_cast<hipStream_t>(stream));
    return forge::last_error();
}

extern "C" int caller_int8_linear(const void* x, const int8_t* w, const void* w_scale, const void* bias, void* out,
                                  int M, int K, int N, int8_t* scratch_q, float* scratch_s, void* stream)
{
    forge::gemm::int8_linear(static_cast<const __half*>(x), w, static_cast<const __half*>(w_scale),
                             static_cast<const __half*>(bias), static_cast<__half*>(out), M, K, N, scratch_q,
                             scratch_s, static_cast<hipStream_t>(stream));
    return forge::last_error();
}

// The dp4a entry points (the reference's fallback for GPUs without INT8 tensor cores); here they
// forward to the matrix-core path, so their results must equal the oracle's.
extern "C" int caller_dp4a_gemm_dequant(const int8_t* A, const int8_t* B, const float* act_scale, const void* w_scale,
                                        const void* bias, void* out, int M, int K, int N, void* stream)
{
    forge::gemm::int8_dp4a_gemm_dequant(A, B, act_scale, static_cast<const __half*>(w_scale),
                                        static_cast<const __half*>(bias), static_cast<__half*>(out), M, K, N,
                                        static_cast<hipStream_t>(stream));
    return forge::last_error();
}

extern "C" int caller_dp4a_linear(const void* x, const int8_t* w, const void* w_scale, const void* bias, void* out,
                                  int M, int K, int N, int8_t* scratch_q, float* scratch_s, void* stream)
{
    forge::gemm::int8_dp4a_linear(static_cast<const __half*>(x), w, static_cast<const __half*>(w_scale),
                                  static_cast<const __half*>(bias), static_cast<__half*>(out), M, K, N, scratch_q,
                                  scratch_s, static_cast<hipStream_t>(stream));
    return forge::last_error();
}

// Called with the header's default arguments for everything after the scratch buffers
// (no split-K workspace, split_k = 1, the null stream, the automatic path), as a reference
// caller that passes only the required arguments would; the test runs it on torch's default
// stream, which is the null stream.
extern "C" int caller_sparse_int8_linear(const void* x, const int8_t* W_comp, const uint32_t* w_meta,
                                         const void* w_scale, const void* bias, void* out, int M, int K, int N,
                                         int8_t* scratch_q, float* scratch_s)
{
    forge::gemm::sparse_int8_linear(static_cast<const __half*>(x), W_comp, w_meta,
                                    static_cast<const __half*>(w_scale), static_cast<const __half*>(bias),
                                    static_cast<__half*>(out), M, K, N, scratch_q, scratch_s);
    return forge::last_error();
}

extern "C" int caller_last_error_after_bad_call()
{
    // A misuse the reference leaves undefined: forge::last_error() reports it.
    forge::gemm::int8_linear(nullptr, nullptr, nullptr, nullptr, nullptr, 4, 64, 16, nullptr, nullptr);
    return forge::last_error();
}
