// forge::nn INT8 ConvTranspose2d (kernel 2, stride 2) for MI355X. Drop-in for
// include/forge/nn/int8_conv_transpose2d.cuh.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstddef>
#include <cstdint>

namespace forge { namespace nn {

/// int8_conv_transpose2d.cuh:25-27. The reference's byte count (one image's buffers).
size_t int8_conv_transpose2d_k2s2_workspace_size(
    int C_in, int H, int W, int C_out);

/// int8_conv_transpose2d.cuh:37-46.
/// Input FP16 [N, C_in, H, W]; weight INT8 [4*C_out, C_in], row co*4 + kh*2 + kw holding
/// ConvTranspose2d weight[ci, co, kh, kw]; w_scale [C_out]; bias [C_out] or nullptr, added
/// after the FP16 rounding of the GEMM value; output FP16 [N, C_out, 2H, 2W].
void int8_conv_transpose2d_k2s2_forward(
    const __half* input,       // [N, C_in, H, W]
    const int8_t* weight,      // [4*C_out, C_in] (repacked)
    const __half* w_scale,     // [C_out]
    const __half* bias,        // [C_out] or nullptr
    __half*       output,      // [N, C_out, 2*H, 2*W]
    int N, int C_in, int H, int W,
    int C_out,
    void*         workspace,
    hipStream_t   stream = nullptr);

}} // namespace forge::nn
