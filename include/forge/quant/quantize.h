// forge::quant per-token activation quantization for MI355X (gfx950).
// Drop-in for include/forge/quant/quantize.cuh of the reference (same names and
// argument meaning, hipStream_t in place of cudaStream_t).
//
// Fused per-token activation quantization: FP16 (M, K) -> INT8 (M, K) + scales (M,).
// scale = max(absmax, 1e-8) / 127, q = clamp(rne(x * (1/scale)), -128, 127).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>

namespace forge { namespace quant {

/// Two-pass kernel (quantize.cuh:17-21): launch with grid = M rows and any block size
/// (1..1024 threads). Bit-identical to fused_quantize_activation.
__global__ void fused_quantize_activation_kernel(
    const __half* __restrict__ input,
    int8_t* __restrict__       output,
    float* __restrict__        scales,
    int                        K);

/// quantize.cuh:23-29.
void fused_quantize_activation(
    const __half* input,        // (M, K) device
    int8_t*       output,       // (M, K) device
    float*        scales,       // (M,) device
    int           M,
    int           K,
    hipStream_t   stream = nullptr);

}} // namespace forge::quant
