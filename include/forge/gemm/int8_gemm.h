// forge::gemm INT8 GEMM entry for MI355X. Drop-in for include/forge/gemm/int8_gemm.cuh.
// gfx950 has one INT8 path (MFMA); there is no runtime backend dispatch.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>

namespace forge { namespace gemm {

/// int8_gemm.cuh:18-19: returns the gfx IP version (950 on MI355X).
int get_compute_capability(int device = 0);

/// int8_gemm.cuh:22-23: true on gfx94x/gfx950 (INT8 matrix cores).
bool has_wmma_int8(int device = 0);

/// int8_gemm.cuh:26-35: same as int8_gemm_dequant.
void int8_gemm(
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

}} // namespace forge::gemm
