/*
 * forge_amd.h -- C-ABI of the MI355X (gfx950) INT8 quantized-inference library.
 *
 * This is the drop-in boundary for the reference's forge::quant, forge::gemm,
 * forge::sparsity and forge::nn INT8 entry points (WizardsForgeGames/Forge). Every
 * entry point is extern "C", takes plain device pointers, sizes and a hipStream_t
 * (passed as void*; NULL = the legacy null stream), allocates nothing and is
 * asynchronous on the stream. The C++ API in include/forge/ and any FFI
 * (ctypes, pybind, JNI, cgo) bind these symbols.
 *
 * Types at the boundary:
 *   int8 tensors        int8_t*     row-major
 *   fp16 tensors        uint16_t*   IEEE binary16 bit patterns (HIP __half)
 *   per-token scales    float*
 *   accumulators        int32_t*
 *
 * Return value: FORGE_OK (0); FORGE_EINVAL (-1) for arguments the path cannot run
 * (null pointer, shape or alignment outside the documented contract); FORGE_ENODEV
 * (-2) when no HIP device is present; otherwise the positive hipError_t reported by
 * the launch. Non-positive M, N or K return FORGE_OK without launching, as the
 * reference's launchers return early (src/gemm/int8_dense.cu:195,
 * src/gemm/int8_sparse.cu:976, src/quant/quantize.cu:170).
 */
#ifndef FORGE_AMD_H
#define FORGE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FORGE_OK      0
#define FORGE_EINVAL  (-1)
#define FORGE_ENODEV  (-2)
#define FORGE_ERANGE  (-3)   /* size beyond a fixed limit of forge_int8_linear_noalloc */

/* Sparse tile configurations (weight rows x tokens per workgroup tile).
 * Reference: include/forge/gemm/int8_sparse.cuh:26-31. */
#define FORGE_SPARSE_TILE_AUTO     (-1)
#define FORGE_SPARSE_TILE_256x128  0
#define FORGE_SPARSE_TILE_128x128  1
#define FORGE_SPARSE_TILE_128x64   2
#define FORGE_SPARSE_NUM_TILES     3

/* sparse_int8_linear paths. Reference: include/forge/gemm/int8_sparse.cuh:73-76. */
#define FORGE_SPARSE_LINEAR_AUTO     (-1)
#define FORGE_SPARSE_LINEAR_TWO_PASS 0
#define FORGE_SPARSE_LINEAR_FUSED    1

/* Mirrors FORGE_SPARSE_GEMM_API_VERSION of include/forge/gemm/int8_sparse.cuh:19-22. */
#define FORGE_AMD_SPARSE_GEMM_API_VERSION 3

/* ---- library ---------------------------------------------------------------- */

/* Human-readable text for a status code. */
const char* forge_status_string(int status);

/* One-time per-device setup (device properties, the device addresses of the decode K-split
 * sum slots). Called implicitly by every entry point; calling it before graph capture keeps
 * captured calls free of device queries (a capture that starts before any split launch on
 * the device otherwise records the decode launches unsplit: same bits, slower). */
int forge_init(void);

/* Decode K-split slots (no counterpart in the reference, whose split-K takes a caller
 * workspace). Decode launches for narrow N split K over several workgroups that hand exact
 * INT32 partial sums over through static device slots, one slot per (stream, graph capture)
 * key. forge_ksplit_last reports the calling thread's last decode launch: the slot it used
 * (-1: none) and its K parts (1: unsplit; 0: no decode launch yet on this thread).
 * forge_ksplit_reset zeroes every slot of the current device, in stream order on `stream`;
 * call it only when no decode launch is in flight on the device (a launch is left
 * unfinished only by a device fault or an aborted graph). */
int forge_ksplit_last(int* slot, int* parts);
int forge_ksplit_reset(void* stream);

/* Extension, no counterpart in the reference: how many of the current device's static slots
 * are held, and how many there are -- the decode K split's (forge_ksplit_last) and the fused
 * sparse linear's packed-weight slots. Each slot belongs for the rest of the process to the
 * first key that takes it (a stream for eager launches, a stream + capture for launches
 * recorded into a graph); once all are held, launches of a new key run the path that needs
 * none (unsplit decode, W_comp read in place), with the same results. For serving stacks
 * that capture many graphs: they can see when captures start recording those paths. */
int forge_slots_in_use(int* ksplit_used, int* ksplit_total, int* fq_pack_used, int* fq_pack_total);

/* The engine of the calling thread's last GEMM launch made through this library (no
 * counterpart in the reference; its benchmark prints the plan it computes itself,
 * benchmarks/bench_int8_sparse.cu:164-170): e.g. "dma256x256", "dma256x256+tail192"
 * (whole waves of 256 x 256 tiles, then one wave of 192-row tiles, in one launch),
 * "ring64x64", "decode", "decode+quantize", "token-block", "fused-quantize", "regstaged tile1 s3"
 * (tile = the reference's kSparseTile* index, s = split-K parts). "none" before any launch.
 * The string belongs to the library and stays valid until the thread's next GEMM call. */
const char* forge_last_route(void);

/* Replaces forge::gemm::get_compute_capability / has_wmma_int8
 * (include/forge/gemm/int8_gemm.cuh:18-23). On gfx950 the "compute capability"
 * is the gfx IP version 950 and INT8 matrix cores are always present. */
int forge_get_compute_capability(int device, int* out_cc);
int forge_has_int8_matrix_cores(int device, int* out_flag);

/* ---- quantization ------------------------------------------------------------ */

/* Replaces forge::quant::fused_quantize_activation (include/forge/quant/quantize.cuh:23-29).
 * x (M,K) fp16 -> q (M,K) int8 and scales (M) fp32: scale = max(absmax,1e-8)/127,
 * q = clamp(rne(x * (1/scale)), -128, 127). Any K >= 1 and any alignment. */
int forge_quantize_activation(const uint16_t* x, int8_t* q, float* scales,
                              int M, int K, void* stream);

/* Launches the exported two-pass kernel forge::quant::fused_quantize_activation_kernel
 * with grid M and `threads` threads per block, as include/forge/quant/quantize.cuh:17-21
 * lets callers do (tests/test_quantize.cu:54-55). Output is bit-identical to
 * forge_quantize_activation. threads in [1, 1024]. */
int forge_quantize_activation_twopass(const uint16_t* x, int8_t* q, float* scales,
                                      int M, int K, int threads, void* stream);

/* Replaces forge::quant::fused_dequantize_bias (include/forge/quant/dequantize.cuh:22-30).
 * out[m,n] = half(((float)acc[m,n] * as[m]) * ws[n] + bias[n]); bias may be NULL. */
int forge_dequantize_bias(const int32_t* acc, const float* act_scale, const uint16_t* w_scale,
                          const uint16_t* bias, uint16_t* out, int M, int N, void* stream);

/* ---- dense INT8 GEMM ------------------------------------------------------------ */

/* Replaces forge::gemm::int8_gemm_dequant (include/forge/gemm/int8_dense.cuh:24-34).
 * out[m,n] = half(fma((float)sum_k A[m,k]*B[n,k], as[m]*ws[n], bias[n])).
 * A (M,K), B (N,K) row-major int8; any M, N, K >= 1. */
int forge_int8_gemm_dequant(const int8_t* A, const int8_t* B, const float* act_scale,
                            const uint16_t* w_scale, const uint16_t* bias, uint16_t* out,
                            int M, int K, int N, void* stream);

/* Replaces forge::gemm::int8_gemm (include/forge/gemm/int8_gemm.cuh:26-35): one MFMA
 * path on gfx950, so identical to forge_int8_gemm_dequant. */
int forge_int8_gemm(const int8_t* A, const int8_t* B, const float* act_scale,
                    const uint16_t* w_scale, const uint16_t* bias, uint16_t* out,
                    int M, int K, int N, void* stream);

/* Replaces forge::gemm::int8_linear (include/forge/gemm/int8_dense.cuh:37-48): quantize x
 * into the caller's scratch (M,K) int8 + (M) fp32, then the dequantizing GEMM. */
int forge_int8_linear(const uint16_t* x, const int8_t* w, const uint16_t* w_scale,
                      const uint16_t* bias, uint16_t* out, int M, int K, int N,
                      int8_t* scratch_q, float* scratch_scale, void* stream);

/* No counterpart in the reference. forge_int8_linear for callers that cannot allocate
 * device memory (code under graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): the same computation and bits, with the quantized activations and scales in
 * a fixed per-GPU device array of the library instead of caller scratch. Limits: M * K <=
 * FORGE_NOALLOC_MAX_QBYTES and M <= FORGE_NOALLOC_MAX_ROWS, else FORGE_ERANGE (nothing is
 * launched). Allocates nothing. Every call on one GPU shares the array: calls that overlap
 * in time on one GPU race and must not be made. The array's address is resolved by
 * forge_init or by the first call on a device; a first call inside a graph capture returns
 * FORGE_EINVAL (call forge_init before capturing). */
#define FORGE_NOALLOC_MAX_QBYTES (16u << 20)
#define FORGE_NOALLOC_MAX_ROWS   65536
int forge_int8_linear_noalloc(const uint16_t* x, const int8_t* w, const uint16_t* w_scale,
                              const uint16_t* bias, uint16_t* out, int M, int K, int N, void* stream);

/* Extension (no reference counterpart: the reference GEMMs always dequantize):
 * C (M,N) int32 = A (M,K) x B (N,K)^T, exact INT32 accumulation. */
int forge_int8_gemm_s32(const int8_t* A, const int8_t* B, int32_t* C,
                        int M, int K, int N, void* stream);

/* ---- 2:4 sparsity ------------------------------------------------------------ */

/* Replaces forge::sparsity::prune_compress_24 (include/forge/sparsity/prune_compress.cuh:
 * 16-29). w (N,K) -> comp (N,K/2) + meta_raw (N*K/4) nibbles keep0|keep1<<2, bit-identical
 * to the reference (lower index pruned among equal magnitudes). K % 4 == 0. */
int forge_prune_compress_24(const int8_t* w, int8_t* comp, uint8_t* meta_raw,
                            int N, int K, void* stream);

/* Replaces forge::sparsity::pack_metadata (include/forge/sparsity/pack_metadata.cuh:15-26).
 * Same (N, K/32) uint32 buffer; words are emitted in the gfx950 SMFMAC index layout:
 * the reference word (n, c) = sum_g nib[n,8c+g] << 4g is stored at
 * (n/16)*(K/32)*16 + c*R + n%16, R = rows in n's 16-row block (16 unless N%16 != 0).
 * K % 32 == 0. */
int forge_pack_metadata(const uint8_t* meta_raw, uint32_t* meta_packed,
                        int N, int K, void* stream);

/* Extension: inverse of forge_pack_metadata (gfx950 words -> raw nibbles); converts
 * legacy checkpoints via unpack(reference layout) -> repack. */
int forge_unpack_metadata(const uint32_t* meta_packed, uint8_t* meta_raw,
                          int N, int K, void* stream);

/* ---- 2:4 sparse INT8 GEMM ------------------------------------------------------- */

/* Replaces forge::gemm::sparse_int8_gemm_plan (include/forge/gemm/int8_sparse.cuh:39-50).
 * Pure host arithmetic over an MI355X cost model; honours a forced tile (0..2) and a
 * forced split (>= 1, 1 without a workspace). */
int forge_sparse_int8_gemm_plan(int M, int K, int N_out, int split_k, int have_workspace,
                                int tile, int* out_tile, int* out_split_k);

/* Replaces forge::gemm::sparse_int8_gemm (include/forge/gemm/int8_sparse.cuh:57-71).
 * out (M,N_out) = half(fma(sum_k x[m,k]*Wp[n,k], as[m]*ws[n], bias[n])), Wp the 2:4
 * weights given by W_comp (N_out,K/2) and the gfx950-layout w_meta (N_out*K/32).
 * K % 64 == 0, N_out % 16 == 0. splitk_workspace: (M,N_out) 4-byte elements, used as
 * INT32 partial sums (exact, deterministic: every split gives the unsplit bits). */
int forge_sparse_int8_gemm(const int8_t* W_comp, const int8_t* x, const uint32_t* w_meta,
                           const float* act_scale, const uint16_t* w_scale,
                           const uint16_t* bias, uint16_t* out, int M, int K, int N_out,
                           float* splitk_workspace, int split_k, void* stream, int tile);

/* Extension: C (M,N_out) int32 = x (M,K) x Wp^T, exact. Same shape contract. */
int forge_sparse_int8_gemm_s32(const int8_t* W_comp, const int8_t* x, const uint32_t* w_meta,
                               int32_t* C, int M, int K, int N_out, void* stream);

/* Replaces forge::gemm::sparse_int8_linear_fused (include/forge/gemm/int8_sparse.cuh:83). */
int forge_sparse_int8_linear_fused(int M, int K, int N_out, int* out_flag);

/* Replaces forge::gemm::sparse_int8_linear (include/forge/gemm/int8_sparse.cuh:90-105).
 * Outputs are bit-identical across paths. */
int forge_sparse_int8_linear(const uint16_t* x, const int8_t* W_comp, const uint32_t* w_meta,
                             const uint16_t* w_scale, const uint16_t* bias, uint16_t* out,
                             int M, int K, int N_out, int8_t* scratch_q, float* scratch_scale,
                             float* splitk_workspace, int split_k, void* stream, int path);

/* Replaces forge::gemm::splitk_reduce (include/forge/gemm/int8_sparse.cuh:108-114):
 * out = half(ws[m,n] + bias[n]) from an fp32 (M,N_out) workspace. */
int forge_splitk_reduce(const float* workspace, const uint16_t* bias, uint16_t* out,
                        int M, int N_out, void* stream);

/* ---- weight preparation ------------------------------------------------------------- */

/* Extension: the reference quantizes weights with torch float32 ops in Python
 * (python/forge/nn/linear.py:168-173, QuantizedLinear.quantize_weight); this is that
 * computation as one device pass: per row scale = max(amax|w|, 1e-8) / 127 (fp32),
 * w_int8 = clamp(round_half_even(w / scale), -127, 127), w_scale = fp16(scale).
 * w: (N, K) row-major fp32, or fp16 when w_fp16 != 0 (widened exactly, as .to(float32) does). */
int forge_quantize_weight_rows(const void* w, int w_fp16, int8_t* w_int8, uint16_t* w_scale,
                               int N, int K, void* stream);

/* Extension: SparseLinear.from_dense_weight (python/forge/nn/linear.py:231-249) in one device
 * pass: the quantization above, then 2:4 prune + compress (forge_prune_compress_24's rule) and
 * the index words in the gfx950 layout (forge_pack_metadata's), with no dense INT8 or raw-nibble
 * buffer. W_comp (N, K/2) int8, w_meta (N*K/32) uint32, w_scale (N) fp16.
 * K % 32 == 0; w and W_comp 16-byte aligned. */
int forge_prepare_sparse_weight(const void* w, int w_fp16, int8_t* W_comp, uint32_t* w_meta,
                                uint16_t* w_scale, int N, int K, void* stream);

/* ---- INT8 conv2d ------------------------------------------------------------------- */

/* Replaces forge::nn::int8_conv2d_workspace_size (include/forge/nn/int8_conv2d.cuh:23-29). */
size_t forge_int8_conv2d_workspace_size(int C_in, int H, int W, int C_out, int kH, int kW,
                                        int padH, int padW, int strideH, int strideW,
                                        int dilH, int dilW);

/* Replaces forge::nn::int8_conv2d_forward (include/forge/nn/int8_conv2d.cuh:41-53):
 * NCHW fp16 input, weight (C_out, C_in*kH*kW) int8, per-patch-row activation
 * quantization, dequant + bias, NCHW fp16 output. */
int forge_int8_conv2d_forward(const uint16_t* input, const int8_t* weight,
                              const uint16_t* w_scale, const uint16_t* bias, uint16_t* output,
                              int N, int C_in, int H, int W, int C_out, int kH, int kW,
                              int padH, int padW, int strideH, int strideW, int dilH, int dilW,
                              void* workspace, void* stream);

/* Extension: implicit-GEMM conv, NHWC int8 input (N,H,W,C), OHWI int8 weights
 * (Co,kH,kW,C), INT32 NHWC output (N,Ho,Wo,Co). */
int forge_int8_conv2d_nhwc_s32(const int8_t* x, const int8_t* w, int32_t* out,
                               int N, int H, int W, int C, int Co, int kH, int kW,
                               int padH, int padW, int strideH, int strideW,
                               int dilH, int dilW, void* stream);

/* Extension: as forge_int8_conv2d_nhwc_s32 with the GEMM dequant epilogue:
 * out (N,Ho,Wo,Co) fp16 = half(fma(acc, act_scale[pixel]*w_scale[co], bias[co])). */
int forge_int8_conv2d_nhwc_dequant(const int8_t* x, const int8_t* w, const float* act_scale,
                                   const uint16_t* w_scale, const uint16_t* bias,
                                   uint16_t* out, int N, int H, int W, int C, int Co,
                                   int kH, int kW, int padH, int padW, int strideH,
                                   int strideW, int dilH, int dilW, void* stream);

/* ---- INT8 ConvTranspose2d (kernel 2, stride 2) and depthwise conv2d ------------------ */

/* Replaces forge::nn::int8_conv_transpose2d_k2s2_workspace_size
 * (include/forge/nn/int8_conv_transpose2d.cuh:25-27, src/nn/int8_conv_transpose2d.cu:107-123):
 * the same byte count as the reference's formula; 0 for a non-positive dimension. */
size_t forge_int8_conv_transpose2d_k2s2_workspace_size(int C_in, int H, int W, int C_out);

/* Replaces forge::nn::int8_conv_transpose2d_k2s2_forward
 * (include/forge/nn/int8_conv_transpose2d.cuh:37-46, src/nn/int8_conv_transpose2d.cu:128-191):
 * input (N,C_in,H,W) fp16, weight (4*C_out, C_in) int8 with row co*4 + kh*2 + kw holding
 * ConvTranspose2d weight[ci, co, kh, kw], w_scale (C_out) fp16, bias (C_out) fp16 or NULL,
 * output (N,C_out,2H,2W) fp16; workspace of at least the size above. Per-pixel activation
 * quantization; output = half(half(acc * as * w_scale[co]) + bias[co]). */
int forge_int8_conv_transpose2d_k2s2_forward(const uint16_t* input, const int8_t* weight,
                                             const uint16_t* w_scale, const uint16_t* bias,
                                             uint16_t* output, int N, int C_in, int H, int W,
                                             int C_out, void* workspace, void* stream);

/* Replaces forge::nn::int8_depthwise_conv2d_forward
 * (include/forge/nn/int8_depthwise_conv2d.cuh:28-41, src/nn/int8_depthwise_conv2d.cu:72-103):
 * input (N,C,H,W) fp16, weight (C, kH*kW) int8, w_scale (C) fp16, bias (C) fp16 or NULL,
 * output (N,C,H_out,W_out) fp16; no workspace. Float arithmetic, no activation quantization. */
int forge_int8_depthwise_conv2d_forward(const uint16_t* input, const int8_t* weight,
                                        const uint16_t* w_scale, const uint16_t* bias,
                                        uint16_t* output, int N, int C, int H, int W,
                                        int kH, int kW, int padH, int padW, int strideH,
                                        int strideW, int dilH, int dilW, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* FORGE_AMD_H */
