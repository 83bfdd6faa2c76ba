/*
 * forge_oracle.h -- CPU restatement of the reference's INT8 quantized-inference
 * path (WizardsForgeGames/Forge, src/quant, src/gemm, src/sparsity, src/nn).
 *
 * TEST INFRASTRUCTURE ONLY. This code is the checker for the HIP library: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product path (forge_amd/) never links, loads or calls it.
 *
 * Every function cites the reference file:line whose arithmetic it restates.
 * Pinning (what each function is checked against, so a plausible mistake fails):
 *   orc_f32_to_f16 / orc_f16_to_f32   numpy float16 conversions (IEEE-754 RNE), all 65536 halves
 *   orc_quantize_rows                 closed-form special cases (zero row, single nonzero, exact
 *                                     .5 ties with scale 1.0 / 2.0), invariants (|q|<=127, absmax
 *                                     element -> +-127, |x - q*scale| <= scale/2), numpy fp32 path
 *   orc_dequantize_bias               float64 evaluation of the same expression (<= 1 fp16 ulp)
 *   orc_splitk_reduce                 numpy float32 addition + float16 conversion; the bias-less
 *                                     case as a plain RNE conversion
 *   orc_gemm_s32                      numpy int64 matmul; all-ones and identity closed forms
 *   orc_gemm_dequant                  float64 evaluation (<= 1 fp16 ulp)
 *   orc_prune_compress_24             hand-derived known answers; exhaustive brute force over all
 *                                     4-tuples of a tie-heavy value set against the independent
 *                                     "keep the two largest (|v|, index) keys" formulation
 *   orc_pack_metadata_ref             the reference test's mt19937(42) nibble vectors, unpack
 *                                     round trip
 *   orc_pack/unpack_metadata_gfx950   round trip to raw nibbles; permutation of the reference words
 *   orc_sparse_gemm_s32               dense GEMM of the decompressed weights == dense GEMM of the
 *                                     pruned weights (numpy)
 *   orc_conv2d_nhwc_s32               torch.nn.functional.conv2d in float64 (exact for these ints)
 *   orc_quantize_weight_rows          the reference's own torch float32 expression run on the CPU
 *                                     (bit-identical), closed forms (|q| max 127 at the absmax,
 *                                     zero row, the -127 clamp)
 *   orc_depthwise_conv2d              torch conv2d (groups = C) in float64 on the dequantized weights
 *                                     (<= 1 fp16 ulp + fp32 sum error); 1x1 kernels as one rounded
 *                                     product; the reference test's three shapes at its tolerance
 *   orc_conv_transpose2d_k2s2         INT32 stage == torch conv_transpose2d in float64 on the
 *                                     quantized integers (exact), with the (C_in, C_out, 2, 2)
 *                                     weight rebuilt from the repacked rows; FP16 output vs the
 *                                     float64 dequantized conv_transpose2d (<= 2 fp16 ulps);
 *                                     the quantize stage is orc_quantize_rows (pinned above)
 *   orc_mt19937                       the C++ standard's 10000th-output check (4123659995)
 *   orc_*_mt (threaded forms)         bit-identical to the single-threaded functions above on
 *                                     shapes whose row count does not divide the thread count
 */
#ifndef FORGE_ORACLE_H
#define FORGE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

float    orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);

void orc_quantize_rows(const uint16_t* x, int8_t* q, float* scales, int M, int K);
void orc_dequantize_bias(const int32_t* acc, const float* act_scale, const uint16_t* w_scale,
                         const uint16_t* bias, uint16_t* out, int M, int N);
void orc_splitk_reduce(const float* ws, const uint16_t* bias, uint16_t* out, int M, int N);
void orc_gemm_s32(const int8_t* A, const int8_t* B, int32_t* C, int M, int K, int N);
void orc_gemm_s32_rows(const int8_t* A, const int8_t* B, int32_t* C, int m0, int m1, int K, int N);
void orc_dequant_epilogue(const int32_t* acc, const float* act_scale, const uint16_t* w_scale,
                          const uint16_t* bias, uint16_t* out, int M, int N);
void orc_gemm_dequant(const int8_t* A, const int8_t* B, const float* act_scale,
                      const uint16_t* w_scale, const uint16_t* bias, uint16_t* out,
                      int M, int K, int N);
void orc_linear(const uint16_t* x, const int8_t* W, const uint16_t* w_scale,
                const uint16_t* bias, uint16_t* out, int M, int K, int N);

void orc_prune_compress_24(const int8_t* w, int8_t* comp, uint8_t* meta_raw, int N, int K);
void orc_decompress_24(const int8_t* comp, const uint8_t* meta_raw, int8_t* w, int N, int K);
void orc_pack_metadata_ref(const uint8_t* meta_raw, uint32_t* packed, int N, int K);
void orc_pack_metadata_gfx950(const uint8_t* meta_raw, uint32_t* packed, int N, int K);
void orc_unpack_metadata_gfx950(const uint32_t* packed, uint8_t* meta_raw, int N, int K);
void orc_sparse_gemm_s32(const int8_t* W_comp, const int8_t* x, const uint8_t* meta_raw,
                         int32_t* C, int M, int K, int N);

int  orc_conv_out_size(int in, int pad, int dil, int k, int stride);
void orc_conv2d_nhwc_s32(const int8_t* x, const int8_t* w, int32_t* out,
                         int N, int H, int W, int C, int Co, int kH, int kW,
                         int padH, int padW, int strideH, int strideW, int dilH, int dilW);

void orc_quantize_weight_rows(const float* w, int8_t* q, uint16_t* scale16, float* scale32, int N, int K);
void orc_depthwise_conv2d(const uint16_t* in, const int8_t* w, const uint16_t* w_scale,
                          const uint16_t* bias, uint16_t* out, int N, int C, int H, int W,
                          int kH, int kW, int padH, int padW, int strideH, int strideW,
                          int dilH, int dilW);
void orc_conv_transpose2d_k2s2(const uint16_t* in, const int8_t* w, const uint16_t* w_scale,
                               const uint16_t* bias, uint16_t* out, int32_t* acc32,
                               int N, int C_in, int H, int W, int C_out);

typedef struct { uint32_t mt[624]; int idx; } orc_mt19937_t;
void     orc_mt19937_seed(orc_mt19937_t* s, uint32_t seed);
uint32_t orc_mt19937_next(orc_mt19937_t* s);

double orc_time_gemm_dequant_rows_mt(const int8_t* A, const int8_t* B, const float* act_scale,
                                     const uint16_t* w_scale, const uint16_t* bias, uint16_t* out,
                                     int rows, int K, int N, int threads);
double orc_time_gemm_dequant_rows(const int8_t* A, const int8_t* B, const float* act_scale,
                                  const uint16_t* w_scale, const uint16_t* bias, uint16_t* out,
                                  int rows, int K, int N);

/* The same functions split over output rows (conv: output pixel rows) on `threads` POSIX
 * threads, so full-size results can be compared whole; each output is computed by exactly
 * the single-threaded code on its own row range, so the bits are those of the functions above. */
void orc_gemm_s32_mt(const int8_t* A, const int8_t* B, int32_t* C, int M, int K, int N, int threads);
void orc_gemm_dequant_mt(const int8_t* A, const int8_t* B, const float* act_scale,
                         const uint16_t* w_scale, const uint16_t* bias, uint16_t* out,
                         int M, int K, int N, int threads);
void orc_sparse_gemm_s32_mt(const int8_t* W_comp, const int8_t* x, const uint8_t* meta_raw,
                            int32_t* C, int M, int K, int N, int threads);
void orc_conv2d_nhwc_s32_mt(const int8_t* x, const int8_t* w, int32_t* out,
                            int N, int H, int W, int C, int Co, int kH, int kW,
                            int padH, int padW, int strideH, int strideW, int dilH, int dilW, int threads);

#ifdef __cplusplus
}
#endif
#endif
