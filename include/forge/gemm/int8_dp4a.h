// forge::gemm dp4a entry points for MI355X. Drop-in for include/forge/gemm/int8_dp4a.cuh.
// The dp4a kernel is dropped: gfx950 always has INT8 MFMA, so these forward to the MFMA
// path (same math, any K) and keep existing callers linking.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>

namespace forge { namespace gemm {

/// int8_dp4a.cuh:25-35 (forwards to int8_gemm_dequant).
void int8_dp4a_gemm_dequant(
    const int8_t* A, const int8_t* B, const float* act_scale, const __half* w_scale,
    const __half* bias, __half* output, int M, int K, int N, hipStream_t stream = nullptr);

/// int8_dp4a.cuh:38-49 (forwards to int8_linear).
void int8_dp4a_linear(
    const __half* x, const int8_t* w_int8, const __half* w_scale, const __half* bias,
    __half* output, int M, int K, int N, int8_t* scratch_a_int8, float* scratch_a_scale,
    hipStream_t stream = nullptr);

}} // namespace forge::gemm
