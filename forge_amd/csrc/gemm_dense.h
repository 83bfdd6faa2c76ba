// Internal interfaces between the GEMM translation units.
#pragma once

#include "common.h"

namespace forge_amd {

// Output of a GEMM: exactly one of c32 (INT32) or c16 (dequantized FP16) is non-null.
struct GemmEpilogue {
    int32_t* c32;
    uint16_t* c16;
    const float* act_scale;     // (M,)  FP16 mode only
    const uint16_t* w_scale;    // (N,)
    const uint16_t* bias;       // (N,) or nullptr
    int M, N;
};

// Rows at or below which the weight-streaming skinny kernel serves the dense GEMM.
constexpr int kSkinnyMaxM = 16;

int launch_quantize(const uint16_t* x, int8_t* q, float* scales, int M, int K, hipStream_t s);

// Dense C = A (M,K) x B (N,K)^T; writes out16 (dequant) if non-null, else out32.
int gemm_dense(const int8_t* A, const int8_t* B, const float* act_scale, const uint16_t* w_scale,
               const uint16_t* bias, uint16_t* out16, int32_t* out32, int M, int K, int N,
               hipStream_t s);

// Skinny (M <= kSkinnyMaxM) weight-streaming GEMM; needs K % 16 == 0 and 16-byte bases.
int launch_gemm_skinny(const int8_t* A, const int8_t* B, const GemmEpilogue& ep, int M, int K, int N,
                       hipStream_t s);

template <bool DEQUANT, class ALoader>
int launch_gemm_tiles(const ALoader& la, const struct RowMajorLoader& lb, const GemmEpilogue& ep,
                      int M, int N, int K, bool vec, hipStream_t s);

}  // namespace forge_amd
