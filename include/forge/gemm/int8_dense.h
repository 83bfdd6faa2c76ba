// forge::gemm dense INT8 GEMM for MI355X (gfx950 MFMA v_mfma_i32_32x32x32_i8).
// Drop-in for include/forge/gemm/int8_dense.cuh of the reference.
//
// Y[m,n] = half(fma(sum_k A[m,k] * B[n,k], act_scale[m] * w_scale[n], bias[n]))
// A: (M, K) row-major int8; B: (N, K) row-major int8 ("NT"); Y: (M, N) fp16.
// Any M, N, K >= 1 (the reference's K % 64 / N % 16 note is not required here).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>

namespace forge { namespace gemm {

/// int8_dense.cuh:24-34.
void int8_gemm_dequant(
    const int8_t* A,            // (M, K) device
    const int8_t* B,            // (N, K) device
    const float*  act_scale,    // (M,) device
    const __half* w_scale,      // (N,) device
    const __half* bias,         // (N,) device, or nullptr
    __half*       output,       // (M, N) device
    int           M,
    int           K,
    int           N,
    hipStream_t   stream = nullptr);

/// int8_dense.cuh:37-48: quantize activation + GEMM + dequant.
void int8_linear(
    const __half* x,            // (M, K) fp16 device
    const int8_t* w_int8,       // (N, K) int8 device (pre-quantized weight)
    const __half* w_scale,      // (N,) fp16 device
    const __half* bias,         // (N,) fp16 device or nullptr
    __half*       output,       // (M, N) fp16 device
    int           M,
    int           K,
    int           N,
    int8_t*       scratch_a_int8,  // (M, K) int8 workspace
    float*        scratch_a_scale, // (M,) float workspace
    hipStream_t   stream = nullptr);

/// Extension: exact INT32 output, C (M, N) = A x B^T.
void int8_gemm_s32(
    const int8_t* A, const int8_t* B, int32_t* C, int M, int K, int N,
    hipStream_t stream = nullptr);

}} // namespace forge::gemm
