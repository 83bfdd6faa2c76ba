// forge::quant fused dequantization + bias for MI355X (gfx950).
// Drop-in for include/forge/quant/dequantize.cuh of the reference.
//
// out[m,n] = half((float)acc[m,n] * act_scale[m] * w_scale[n] + bias[n]).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>

namespace forge { namespace quant {

/// dequantize.cuh:14-20: launch with grid = M rows and any block size.
__global__ void fused_dequantize_bias_kernel(
    const int32_t* __restrict__ input,
    const float* __restrict__   act_scale,
    const __half* __restrict__  w_scale,
    const __half* __restrict__  bias,
    __half* __restrict__        output,
    int                         N);

/// dequantize.cuh:22-30.
void fused_dequantize_bias(
    const int32_t* input,       // (M, N) device
    const float*   act_scale,   // (M,) device
    const __half*  w_scale,     // (N,) device
    const __half*  bias,        // (N,) device, nullptr for no bias
    __half*        output,      // (M, N) device
    int            M,
    int            N,
    hipStream_t    stream = nullptr);

}} // namespace forge::quant
