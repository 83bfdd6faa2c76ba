// Internal interfaces between the GEMM translation units.
#pragma once

#include "common.h"
#include "mfma_tile.h"

namespace forge_amd {

// Rows at or below which the weight-streaming skinny kernel serves the dense GEMM.
constexpr int kSkinnyMaxM = 16;

int launch_quantize(const uint16_t* x, int8_t* q, float* scales, int M, int K, hipStream_t s);
// Per-pixel rows of NCHW FP16 images: q (images*HW, C) int8 and scales (images*HW,).
int launch_quantize_pixels_nchw(const uint16_t* x, int8_t* q, float* scales, int images, int C, int HW,
                                hipStream_t s);

// Dense C = A (M,K) x B (N,K)^T; writes out16 (dequant) if non-null, else out32.
int gemm_dense(const int8_t* A, const int8_t* B, const float* act_scale, const uint16_t* w_scale,
               const uint16_t* bias, uint16_t* out16, int32_t* out32, int M, int K, int N,
               hipStream_t s);

// The tile engines only (no decode or skinny kernels): every GemmEpilogue mode, including
// the upsample scatter, which the decode and skinny kernels do not implement.
int gemm_tiles(const int8_t* A, const int8_t* B, const GemmEpilogue& ep, int M, int K, int N, hipStream_t s);

// Skinny (M <= kSkinnyMaxM) weight-streaming GEMM; needs K % 16 == 0 and 16-byte bases.
int launch_gemm_skinny(const int8_t* A, const int8_t* B, const GemmEpilogue& ep, int M, int K, int N,
                       hipStream_t s);

// Decode GEMM (M <= kDecodeMaxM tokens, K % 128 == 0): weights W (N,K) dense or W_comp (N,K/2) +
// gfx950 index words (sparse), tokens X (M,K) int8; 16-byte aligned operands.
constexpr int kDecodeMaxM = 16;
constexpr int kDecodeMaxK = 8192;   // dense: 4 waves x 16 stages of 128; sparse: 8 waves x 8 stages
// Decode with the per-token quantize fused into the kernel (FP16 tokens in): up to this many
// tokens each workgroup quantizes the whole token block itself. Measured against quantize kernel
// + decode GEMM replayed in a graph (N = K = 8192, 6 rotating weight copies): dense 13.4-14.2 vs
// 14.8-15.1 us at M = 1-2, sparse 10.6-11.1 vs 11.3-11.5 us; a 4-row prologue was level with the
// two launches at 3-4 tokens (sparse 0.2-0.7 us behind), so those keep the quantize kernel.
constexpr int kDecodeFqMaxM = 2;
bool decode_supported(int M, int K);
// int8_linear / sparse_int8_linear at M <= kDecodeFqMaxM on the decode kernels with the per-token
// quantize fused in (dense K % 128 == 0, sparse K % 256 == 0, K <= kDecodeMaxK; x, W, W_comp and
// the index words 16-byte aligned, q_scratch 8-byte aligned). Same bits as quantize + GEMM; with
// q_scratch non-null the quantized rows and scales are also left in the scratch buffers.
bool decode_fq_supported(int M, int K, bool sparse);
int launch_decode_fq(const uint16_t* x, const int8_t* W, const uint32_t* meta, const uint16_t* w_scale,
                     const uint16_t* bias, uint16_t* out, int8_t* q_scratch, float* scale_scratch, int M, int K,
                     int N, bool sparse, hipStream_t s);
int launch_decode(const int8_t* W, const uint32_t* meta, const int8_t* X, const GemmEpilogue& ep, int K,
                  bool sparse, hipStream_t s);

// Sparse GEMM at 16 < M <= kSkinnyTbMaxM tokens on the sparse register decode kernel with
// several 16-token blocks per weight fragment: K % 256 == 0, K <= kDecodeMaxK, 16-byte aligned
// operands (W_comp, gfx950 index words, tokens). Narrow N splits K over 2 or 4 workgroups per
// row block (exact INT32 hand-off); kp forces the parts (1, 2, 4; 0 = chosen by shape).
// Resolves the decode K-split slot arrays on the current device (forge_init calls it, so that a
// first split launch inside a graph capture needs no symbol lookup).
int ksplit_prepare();
// Resolves the fused sparse linear's packed-weight slots on the current device (forge_init).
int fq_pack_prepare();
// Resolves the device address of forge_int8_linear_noalloc's array on the current device.
int noalloc_prepare();
// Slots of device dev held by launch keys: the decode K split's (of kKSplitSlotCount) and the
// fused sparse linear's packed-weight slots (of kFqPackSlotCount).
constexpr int kKSplitSlotCount = 32;
constexpr int kFqPackSlotCount = 32;
int ksplit_slots_used(int dev);
int fq_pack_slots_used(int dev);

constexpr int kSkinnyTbMaxM = 64;
bool skinny_tb_supported(int M, int K);
// Dense 16 < M <= 64 with K >= 4096 (K % 256 == 0, K <= kDecodeMaxK) and N narrow enough that
// 16-row workgroups are fewer than the CUs: token blocks + K split (kp as launch_skinny_tb).
bool dense_tb_supported(int M, int K, int N, int cu);
int launch_dense_tb(const int8_t* W, const int8_t* X, const GemmEpilogue& ep, int K, int cu, hipStream_t s,
                    int kp = 0);
int launch_skinny_tb(const int8_t* W, const uint32_t* meta, const int8_t* X, const GemmEpilogue& ep, int K, int cu,
                     hipStream_t s, int kp = 0);

// Wide-tile 2:4 sparse GEMM with INT32 output (gemm_sparse_wide.hip): 256 tokens x 8-11 32-row
// weight blocks per tile, every CU the same number of weight blocks per 256-token block, as T
// tiles. The plan: TB token blocks, c CUs per token block, q blocks per CU (q + 1 for the first r),
// XCD grouping gt token blocks x gc block runs per XCD (gc = 0: none). Needs K % 512 == 0,
// N % 16 == 0, M * K, N * K / 2 and M * N * 4 < 2^31, 16-byte aligned operands.
struct SpWidePlan {
    int TB, c, q, r, T, gc, gt;
};
bool sparse_wide_plan(int M, int N, int K, int cu, SpWidePlan* out);
int launch_sparse_wide_s32(const int8_t* W_comp, const int8_t* x, const uint32_t* meta, int32_t* C, int M, int K,
                           int N, const SpWidePlan& p, hipStream_t s);

// NHWC conv, stride 1, C % 128 == 0, Co % 256 == 0, on the window-fed tile (conv_window.hip):
// returns -1 when the shape is not one it takes.
int launch_conv_window(const ConvGeom& g, const int8_t* w, const GemmEpilogue& ep, int Co, hipStream_t s);

// Implicit-GEMM NHWC conv through the dense tile engine (conv.hip supplies the geometry).
int launch_conv_gemm(const ConvGeom& g, const int8_t* w, const GemmEpilogue& ep, int Co, bool vec,
                     hipStream_t s);

}  // namespace forge_amd
