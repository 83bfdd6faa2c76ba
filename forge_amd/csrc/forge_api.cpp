// C++ API with the reference's namespaces and signatures (include/forge/...), as thin
// wrappers over the C-ABI (include/forge_amd.h). The reference's launchers return void;
// these keep void and record the C-ABI status for forge::last_error().
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "forge_amd.h"
#include "forge/status.h"
#include "forge/quant/quantize.h"
#include "forge/quant/dequantize.h"
#include "forge/gemm/int8_dense.h"
#include "forge/gemm/int8_gemm.h"
#include "forge/gemm/int8_dp4a.h"
#include "forge/gemm/int8_sparse.h"
#include "forge/sparsity/prune_compress.h"
#include "forge/sparsity/pack_metadata.h"
#include "forge/nn/int8_conv2d.h"
#include "forge/nn/int8_conv_transpose2d.h"
#include "forge/nn/int8_depthwise_conv2d.h"

namespace {
thread_local int t_status = FORGE_OK;
inline void rec(int st) { t_status = st; }
inline const uint16_t* hb(const __half* p) { return reinterpret_cast<const uint16_t*>(p); }
inline uint16_t* hb(__half* p) { return reinterpret_cast<uint16_t*>(p); }
inline void* S(hipStream_t s) { return reinterpret_cast<void*>(s); }
}  // namespace

namespace forge {

int last_error() { return t_status; }

namespace quant {

void fused_quantize_activation(const __half* input, int8_t* output, float* scales, int M, int K,
                               hipStream_t stream) {
    rec(forge_quantize_activation(hb(input), output, scales, M, K, S(stream)));
}

void fused_dequantize_bias(const int32_t* input, const float* act_scale, const __half* w_scale,
                           const __half* bias, __half* output, int M, int N, hipStream_t stream) {
    rec(forge_dequantize_bias(input, act_scale, hb(w_scale), hb(bias), hb(output), M, N, S(stream)));
}

}  // namespace quant

namespace gemm {

int get_compute_capability(int device) {
    int cc = 0;
    rec(forge_get_compute_capability(device, &cc));
    return cc;
}

bool has_wmma_int8(int device) {
    int f = 0;
    rec(forge_has_int8_matrix_cores(device, &f));
    return f != 0;
}

void int8_gemm_dequant(const int8_t* A, const int8_t* B, const float* act_scale, const __half* w_scale,
                       const __half* bias, __half* output, int M, int K, int N, hipStream_t stream) {
    rec(forge_int8_gemm_dequant(A, B, act_scale, hb(w_scale), hb(bias), hb(output), M, K, N, S(stream)));
}

void int8_gemm(const int8_t* A, const int8_t* B, const float* act_scale, const __half* w_scale,
               const __half* bias, __half* output, int M, int K, int N, hipStream_t stream) {
    rec(forge_int8_gemm(A, B, act_scale, hb(w_scale), hb(bias), hb(output), M, K, N, S(stream)));
}

void int8_linear(const __half* x, const int8_t* w_int8, const __half* w_scale, const __half* bias,
                 __half* output, int M, int K, int N, int8_t* scratch_a_int8, float* scratch_a_scale,
                 hipStream_t stream) {
    rec(forge_int8_linear(hb(x), w_int8, hb(w_scale), hb(bias), hb(output), M, K, N, scratch_a_int8,
                          scratch_a_scale, S(stream)));
}

void int8_gemm_s32(const int8_t* A, const int8_t* B, int32_t* C, int M, int K, int N, hipStream_t stream) {
    rec(forge_int8_gemm_s32(A, B, C, M, K, N, S(stream)));
}

void int8_dp4a_gemm_dequant(const int8_t* A, const int8_t* B, const float* act_scale, const __half* w_scale,
                            const __half* bias, __half* output, int M, int K, int N, hipStream_t stream) {
    int8_gemm_dequant(A, B, act_scale, w_scale, bias, output, M, K, N, stream);
}

void int8_dp4a_linear(const __half* x, const int8_t* w_int8, const __half* w_scale, const __half* bias,
                      __half* output, int M, int K, int N, int8_t* scratch_a_int8, float* scratch_a_scale,
                      hipStream_t stream) {
    int8_linear(x, w_int8, w_scale, bias, output, M, K, N, scratch_a_int8, scratch_a_scale, stream);
}

SparseGemmPlan sparse_int8_gemm_plan(int M, int K, int N_out, int split_k, bool have_workspace, int tile) {
    SparseGemmPlan p{kSparseTile128x128, 1};
    rec(forge_sparse_int8_gemm_plan(M, K, N_out, split_k, have_workspace ? 1 : 0, tile, &p.tile, &p.split_k));
    return p;
}

void sparse_int8_gemm(const int8_t* W_comp, const int8_t* x_int8, const uint32_t* w_meta, const float* act_scale,
                      const __half* w_scale, const __half* bias, __half* output, int M, int K, int N_out,
                      float* splitk_workspace, int split_k, hipStream_t stream, int tile) {
    rec(forge_sparse_int8_gemm(W_comp, x_int8, w_meta, act_scale, hb(w_scale), hb(bias), hb(output), M, K, N_out,
                               splitk_workspace, split_k, S(stream), tile));
}

bool sparse_int8_linear_fused(int M, int K, int N_out) {
    int f = 0;
    rec(forge_sparse_int8_linear_fused(M, K, N_out, &f));
    return f != 0;
}

void sparse_int8_linear(const __half* x, const int8_t* W_comp, const uint32_t* w_meta, const __half* w_scale,
                        const __half* bias, __half* output, int M, int K, int N_out, int8_t* scratch_x_int8,
                        float* scratch_x_scale, float* splitk_workspace, int split_k, hipStream_t stream,
                        int path) {
    rec(forge_sparse_int8_linear(hb(x), W_comp, w_meta, hb(w_scale), hb(bias), hb(output), M, K, N_out,
                                 scratch_x_int8, scratch_x_scale, splitk_workspace, split_k, S(stream), path));
}

void splitk_reduce(const float* workspace, const __half* bias, __half* output, int M, int N_out,
                   hipStream_t stream) {
    rec(forge_splitk_reduce(workspace, hb(bias), hb(output), M, N_out, S(stream)));
}

void sparse_int8_gemm_s32(const int8_t* W_comp, const int8_t* x_int8, const uint32_t* w_meta, int32_t* C,
                          int M, int K, int N_out, hipStream_t stream) {
    rec(forge_sparse_int8_gemm_s32(W_comp, x_int8, w_meta, C, M, K, N_out, S(stream)));
}

}  // namespace gemm

namespace sparsity {

void prune_compress_24(const int8_t* weight, int8_t* compressed, uint8_t* metadata_raw, int N, int K,
                       hipStream_t stream) {
    rec(forge_prune_compress_24(weight, compressed, metadata_raw, N, K, S(stream)));
}

void pack_metadata(const uint8_t* meta_raw, uint32_t* meta_packed, int N, int K, hipStream_t stream) {
    rec(forge_pack_metadata(meta_raw, meta_packed, N, K, S(stream)));
}

void unpack_metadata(const uint32_t* meta_packed, uint8_t* meta_raw, int N, int K, hipStream_t stream) {
    rec(forge_unpack_metadata(meta_packed, meta_raw, N, K, S(stream)));
}

}  // namespace sparsity

namespace nn {

size_t int8_conv2d_workspace_size(int C_in, int H, int W, int C_out, int kH, int kW, int padH, int padW,
                                  int strideH, int strideW, int dilH, int dilW) {
    return forge_int8_conv2d_workspace_size(C_in, H, W, C_out, kH, kW, padH, padW, strideH, strideW, dilH, dilW);
}

void int8_conv2d_forward(const __half* input, const int8_t* weight, const __half* w_scale, const __half* bias,
                         __half* output, int N, int C_in, int H, int W, int C_out, int kH, int kW, int padH,
                         int padW, int strideH, int strideW, int dilH, int dilW, void* workspace,
                         hipStream_t stream) {
    rec(forge_int8_conv2d_forward(hb(input), weight, hb(w_scale), hb(bias), hb(output), N, C_in, H, W, C_out, kH, kW,
                                  padH, padW, strideH, strideW, dilH, dilW, workspace, S(stream)));
}

void int8_conv2d_nhwc_s32(const int8_t* x, const int8_t* w, int32_t* out, int N, int H, int W, int C, int Co,
                          int kH, int kW, int padH, int padW, int strideH, int strideW, int dilH, int dilW,
                          hipStream_t stream) {
    rec(forge_int8_conv2d_nhwc_s32(x, w, out, N, H, W, C, Co, kH, kW, padH, padW, strideH, strideW, dilH, dilW,
                                   S(stream)));
}

void int8_conv2d_nhwc_dequant(const int8_t* x, const int8_t* w, const float* act_scale, const __half* w_scale,
                              const __half* bias, __half* out, int N, int H, int W, int C, int Co, int kH, int kW,
                              int padH, int padW, int strideH, int strideW, int dilH, int dilW,
                              hipStream_t stream) {
    rec(forge_int8_conv2d_nhwc_dequant(x, w, act_scale, hb(w_scale), hb(bias), hb(out), N, H, W, C, Co, kH, kW, padH,
                                       padW, strideH, strideW, dilH, dilW, S(stream)));
}

size_t int8_conv_transpose2d_k2s2_workspace_size(int C_in, int H, int W, int C_out) {
    return forge_int8_conv_transpose2d_k2s2_workspace_size(C_in, H, W, C_out);
}

void int8_conv_transpose2d_k2s2_forward(const __half* input, const int8_t* weight, const __half* w_scale,
                                        const __half* bias, __half* output, int N, int C_in, int H, int W,
                                        int C_out, void* workspace, hipStream_t stream) {
    rec(forge_int8_conv_transpose2d_k2s2_forward(hb(input), weight, hb(w_scale), hb(bias), hb(output), N, C_in, H, W,
                                                 C_out, workspace, S(stream)));
}

void int8_depthwise_conv2d_forward(const __half* input, const int8_t* weight, const __half* w_scale,
                                   const __half* bias, __half* output, int N, int C, int H, int W, int kH, int kW,
                                   int padH, int padW, int strideH, int strideW, int dilH, int dilW,
                                   hipStream_t stream) {
    rec(forge_int8_depthwise_conv2d_forward(hb(input), weight, hb(w_scale), hb(bias), hb(output), N, C, H, W, kH, kW,
                                            padH, padW, strideH, strideW, dilH, dilW, S(stream)));
}

}  // namespace nn
}  // namespace forge
