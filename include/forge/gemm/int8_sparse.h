// forge::gemm 2:4 structured-sparse INT8 GEMM for MI355X (gfx950 SMFMAC
// v_smfmac_i32_16x16x128_i8). Drop-in for include/forge/gemm/int8_sparse.cuh.
//
// W_comp: (N_out, K/2) compressed weight (2:4 structured sparsity)
// x_int8: (M, K) quantized activation
// w_meta: (N_out, K/32) uint32 metadata in the gfx950 index layout written by
//         forge::sparsity::pack_metadata
// Requires: K % 64 == 0, N_out % 16 == 0.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>

#define FORGE_SPARSE_GEMM_API_VERSION 3

namespace forge { namespace gemm {

/// Workgroup tile configurations (weight rows x tokens per tile), int8_sparse.cuh:26-31.
constexpr int kSparseTileAuto    = -1;
constexpr int kSparseTile256x128 = 0;
constexpr int kSparseTile128x128 = 1;
constexpr int kSparseTile128x64  = 2;
constexpr int kSparseNumTiles    = 3;

/// int8_sparse.cuh:33-37.
struct SparseGemmPlan {
    int tile;      // kSparseTile256x128 / kSparseTile128x128 / kSparseTile128x64
    int split_k;   // >= 1
};

/// int8_sparse.cuh:39-50: (tile, split-K) from an MI355X wave-aware cost model.
///   split_k <= 0: choose split-K too (only with a workspace); split_k >= 1: use it
///   (1 if !have_workspace). tile < 0: choose; 0..2: force.
SparseGemmPlan sparse_int8_gemm_plan(
    int  M,
    int  K,
    int  N_out,
    int  split_k        = 0,
    bool have_workspace = true,
    int  tile           = kSparseTileAuto);

/// int8_sparse.cuh:52-71. splitk_workspace: (M, N_out) 4-byte elements, overwritten; split-K
/// partial sums are exact INT32, so every split gives the same bits as split_k = 1.
void sparse_int8_gemm(
    const int8_t*   W_comp,     // (N_out, K/2) device
    const int8_t*   x_int8,     // (M, K) device
    const uint32_t* w_meta,     // (N_out, K/32) device
    const float*    act_scale,  // (M,) device
    const __half*   w_scale,    // (N_out,) device
    const __half*   bias,       // (N_out,) device or nullptr
    __half*         output,     // (M, N_out) device
    int             M,
    int             K,
    int             N_out,
    float*          splitk_workspace = nullptr,
    int             split_k = 1,
    hipStream_t     stream  = nullptr,
    int             tile    = kSparseTileAuto);

/// int8_sparse.cuh:73-76.
constexpr int kSparseLinearAuto    = -1;
constexpr int kSparseLinearTwoPass = 0;
constexpr int kSparseLinearFused   = 1;

/// int8_sparse.cuh:78-83.
bool sparse_int8_linear_fused(int M, int K, int N_out);

/// int8_sparse.cuh:85-105. Outputs are bit-identical across paths.
void sparse_int8_linear(
    const __half*   x,           // (M, K) fp16 device
    const int8_t*   W_comp,      // (N_out, K/2) int8 device
    const uint32_t* w_meta,      // (N_out, K/32) device
    const __half*   w_scale,     // (N_out,) fp16 device
    const __half*   bias,        // (N_out,) fp16 device or nullptr
    __half*         output,      // (M, N_out) fp16 device
    int             M,
    int             K,
    int             N_out,
    int8_t*         scratch_x_int8,
    float*          scratch_x_scale,
    float*          splitk_workspace = nullptr,
    int             split_k = 1,
    hipStream_t     stream  = nullptr,
    int             path    = kSparseLinearAuto);

/// int8_sparse.cuh:107-114: fp32 workspace + bias -> fp16.
void splitk_reduce(
    const float*  workspace,    // (M, N_out) fp32 device
    const __half* bias,         // (N_out,) device or nullptr
    __half*       output,       // (M, N_out) fp16 device
    int           M,
    int           N_out,
    hipStream_t   stream = nullptr);

/// Extension: exact INT32 output, C (M, N_out) = x x decompress(W)^T.
void sparse_int8_gemm_s32(
    const int8_t* W_comp, const int8_t* x_int8, const uint32_t* w_meta, int32_t* C,
    int M, int K, int N_out, hipStream_t stream = nullptr);

}} // namespace forge::gemm
