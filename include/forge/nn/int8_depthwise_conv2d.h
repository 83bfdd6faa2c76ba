// forge::nn INT8-weight depthwise conv2d for MI355X. Drop-in for
// include/forge/nn/int8_depthwise_conv2d.cuh.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>

namespace forge { namespace nn {

/// int8_depthwise_conv2d.cuh:28-41. groups = C_in = C_out; FP16 NCHW in and out, INT8
/// weights (C, kH*kW) with a per-channel FP16 scale, float arithmetic, no workspace.
void int8_depthwise_conv2d_forward(
    const __half* input,       // [N, C, H, W]
    const int8_t* weight,      // [C, kH*kW]
    const __half* w_scale,     // [C]
    const __half* bias,        // [C] or nullptr
    __half*       output,      // [N, C, H_out, W_out]
    int N, int C, int H, int W,
    int kH, int kW,
    int padH, int padW,
    int strideH  = 1,
    int strideW  = 1,
    int dilH     = 1,
    int dilW     = 1,
    hipStream_t stream = nullptr);

}} // namespace forge::nn
