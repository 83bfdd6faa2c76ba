// forge::nn INT8 conv2d for MI355X. Drop-in for include/forge/nn/int8_conv2d.cuh, plus
// NHWC implicit-GEMM extensions on the same MFMA tile as the dense GEMM.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstddef>
#include <cstdint>

namespace forge { namespace nn {

/// int8_conv2d.cuh:23-29.
size_t int8_conv2d_workspace_size(
    int C_in, int H, int W,
    int C_out, int kH, int kW,
    int padH, int padW,
    int strideH, int strideW,
    int dilH  = 1,
    int dilW  = 1);

/// int8_conv2d.cuh:41-53. NCHW fp16 in/out, weight (C_out, C_in*kH*kW) int8.
void int8_conv2d_forward(
    const __half* input,       // [N, C_in, H, W]
    const int8_t* weight,      // [C_out, C_in*kH*kW]
    const __half* w_scale,     // [C_out]
    const __half* bias,        // [C_out] or nullptr
    __half*       output,      // [N, C_out, H_out, W_out]
    int N, int C_in, int H, int W,
    int C_out, int kH, int kW,
    int padH, int padW,
    int strideH, int strideW,
    int dilH, int dilW,
    void*         workspace,
    hipStream_t   stream = nullptr);

/// Extension: NHWC int8 input, OHWI int8 weight, INT32 NHWC output.
void int8_conv2d_nhwc_s32(
    const int8_t* x, const int8_t* w, int32_t* out,
    int N, int H, int W, int C, int Co, int kH, int kW,
    int padH, int padW, int strideH, int strideW, int dilH, int dilW,
    hipStream_t stream = nullptr);

/// Extension: as int8_conv2d_nhwc_s32 with the dequant + bias epilogue (fp16 NHWC out).
void int8_conv2d_nhwc_dequant(
    const int8_t* x, const int8_t* w, const float* act_scale, const __half* w_scale,
    const __half* bias, __half* out,
    int N, int H, int W, int C, int Co, int kH, int kW,
    int padH, int padW, int strideH, int strideW, int dilH, int dilW,
    hipStream_t stream = nullptr);

}} // namespace forge::nn
