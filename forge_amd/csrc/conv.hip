// INT8 conv2d for gfx950.
//
// NHWC implicit GEMM (the MI355X form of config-5 shapes): output pixels are GEMM rows
// (M = N*Ho*Wo), output channels GEMM columns, K = kH*kW*C in (kh, kw, c) order so
// OHWI weights are already the (Co, K) row-major B operand. The A tile is gathered
// straight from the NHWC image by ConvOperand (16 contiguous channels per chunk, zero
// outside the padded image) into the same LDS-staged MFMA tile as the dense GEMM; no
// im2col buffer is written. Integer sums do not depend on K order, so the INT32 stage
// equals the reference's im2col GEMM (src/nn/int8_conv2d.cu:151-223, K order
// ci*kH*kW + kh*kW + kw) on the same integers.
//
// NCHW FP16 API (src/nn/int8_conv2d.cu:126-223): per sample, the patch matrix
// [Ho*Wo, C_in*kH*kW] is gathered to FP16 in the caller's workspace, quantized per patch
// row, multiplied with the dequant epilogue, and transposed to NCHW -- the reference's
// workspace contract (one sample's buffers) fixes that per-sample structure.
#include "common.h"
#include "gemm_dense.h"
#include "mfma_tile.h"
#include "forge/nn/int8_conv2d.h"

#include <algorithm>

namespace forge_amd {

static int conv_out(int in, int pad, int dil, int k, int stride) {
    return (in + 2 * pad - dil * (k - 1) - 1) / stride + 1;
}

static int conv_nhwc(const int8_t* x, const int8_t* w, const float* act_scale, const uint16_t* w_scale,
                     const uint16_t* bias, uint16_t* out16, int32_t* out32, int N, int H, int W, int C,
                     int Co, int kH, int kW, int padH, int padW, int strideH, int strideW, int dilH,
                     int dilW, hipStream_t s)
{
    if (N <= 0 || C <= 0 || Co <= 0 || H <= 0 || W <= 0) return FORGE_OK;
    if (!x || !w || (!out16 && !out32) || kH <= 0 || kW <= 0 || strideH <= 0 || strideW <= 0 ||
        dilH <= 0 || dilW <= 0 || padH < 0 || padW < 0)
        return FORGE_EINVAL;
    if (out16 && (!act_scale || !w_scale)) return FORGE_EINVAL;
    const int Ho = conv_out(H, padH, dilH, kH, strideH), Wo = conv_out(W, padW, dilW, kW, strideW);
    if (Ho <= 0 || Wo <= 0) return FORGE_OK;
    const long long rows = static_cast<long long>(N) * Ho * Wo;
    const long long K = static_cast<long long>(kH) * kW * C;
    if (rows > 0x7FFFFFFFLL || K > 0x7FFFFFFFLL) return FORGE_EINVAL;
    const bool vec = (C % 16 == 0) && aligned(x, 16) && aligned(w, 16);
    ConvGeom g{x, static_cast<int>(rows), static_cast<int>(K), H, W, C, Ho, Wo, kW,
               padH, padW, strideH, strideW, dilH, dilW};
    const int vec_out = out16 ? (aligned(out16, 16) && Co % 8 == 0) : (aligned(out32, 16) && Co % 4 == 0);
    GemmEpilogue ep{out32, out16, act_scale, w_scale, bias, static_cast<int>(rows), Co, vec_out ? 1 : 0};
    return launch_conv_gemm(g, w, ep, Co, vec, s);
}

// Patch gather for the NCHW API: col[p][k], p = ho*Wo + wo, k = ci*kH*kW + kh*kW + kw
// (the reference's im2col order, src/nn/int8_conv2d.cu:59-75), FP16, zero padding.
__global__ __launch_bounds__(256) void im2col_nchw_kernel(
    const uint16_t* __restrict__ in, uint16_t* __restrict__ col, int C, int H, int W, int kH, int kW,
    int padH, int padW, int strideH, int strideW, int dilH, int dilW, int Ho, int Wo)
{
    const int K = C * kH * kW;
    const long long total = static_cast<long long>(Ho) * Wo * K;
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < total; i += stride) {
        const int k = static_cast<int>(i % K);
        const int p = static_cast<int>(i / K);
        const int ho = p / Wo, wo = p % Wo;
        const int kw = k % kW, t = k / kW, kh = t % kH, c = t / kH;
        const int hi = ho * strideH + kh * dilH - padH, wi = wo * strideW + kw * dilW - padW;
        col[i] = (hi >= 0 && hi < H && wi >= 0 && wi < W) ? in[(static_cast<size_t>(c) * H + hi) * W + wi] : 0;
    }
}

// [P, Co] -> [Co, P] through a 32x33 LDS tile.
__global__ __launch_bounds__(256) void transpose_f16_kernel(const uint16_t* __restrict__ src,
                                                           uint16_t* __restrict__ dst, int P, int Co)
{
    __shared__ uint16_t t[32][33];
    const int p0 = blockIdx.x * 32, c0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int r = ty; r < 32; r += 8) {
        const int p = p0 + r, c = c0 + tx;
        if (p < P && c < Co) t[r][tx] = src[static_cast<size_t>(p) * Co + c];
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const int c = c0 + r, p = p0 + tx;
        if (p < P && c < Co) dst[static_cast<size_t>(c) * P + p] = t[tx][r];
    }
}

}  // namespace forge_amd

using namespace forge_amd;

extern "C" size_t forge_int8_conv2d_workspace_size(int C_in, int H, int W, int C_out, int kH, int kW,
                                                   int padH, int padW, int strideH, int strideW,
                                                   int dilH, int dilW)
{
    const int Ho = conv_out(H, padH, dilH, kH, strideH), Wo = conv_out(W, padW, dilW, kW, strideW);
    if (Ho <= 0 || Wo <= 0) return 0;
    const size_t M = static_cast<size_t>(Ho) * Wo, K = static_cast<size_t>(C_in) * kH * kW;
    // [col fp16 | col int8 | act_scale | gemm_out fp16], each region 256-byte aligned.
    auto up = [](size_t b) { return (b + 255) & ~static_cast<size_t>(255); };
    return up(M * K * 2) + up(M * K) + up(M * 4) + up(M * static_cast<size_t>(C_out) * 2);
}

extern "C" int forge_int8_conv2d_forward(const uint16_t* input, const int8_t* weight,
                                         const uint16_t* w_scale, const uint16_t* bias, uint16_t* output,
                                         int N, int C_in, int H, int W, int C_out, int kH, int kW,
                                         int padH, int padW, int strideH, int strideW, int dilH, int dilW,
                                         void* workspace, void* stream)
{
    if (N <= 0 || C_in <= 0 || C_out <= 0) return FORGE_OK;
    if (!input || !weight || !w_scale || !output || !workspace) return FORGE_EINVAL;
    const int Ho = conv_out(H, padH, dilH, kH, strideH), Wo = conv_out(W, padW, dilW, kW, strideW);
    if (Ho <= 0 || Wo <= 0) return FORGE_OK;
    const int M = Ho * Wo, K = C_in * kH * kW;
    auto up = [](size_t b) { return (b + 255) & ~static_cast<size_t>(255); };
    char* ws = static_cast<char*>(workspace);
    uint16_t* col16 = reinterpret_cast<uint16_t*>(ws);
    int8_t* col8 = reinterpret_cast<int8_t*>(ws + up(static_cast<size_t>(M) * K * 2));
    float* as = reinterpret_cast<float*>(reinterpret_cast<char*>(col8) + up(static_cast<size_t>(M) * K));
    uint16_t* gout = reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(as) + up(static_cast<size_t>(M) * 4));
    hipStream_t s = as_stream(stream);
    const long long total = static_cast<long long>(M) * K;
    const int blocks = static_cast<int>(std::min<long long>(divupll(total, 256), 16384));
    const dim3 tgrid(divup(M, 32), divup(C_out, 32));
    for (int n = 0; n < N; n++) {
        const uint16_t* in_n = input + static_cast<size_t>(n) * C_in * H * W;
        uint16_t* out_n = output + static_cast<size_t>(n) * C_out * M;
        im2col_nchw_kernel<<<blocks, 256, 0, s>>>(in_n, col16, C_in, H, W, kH, kW, padH, padW, strideH,
                                                   strideW, dilH, dilW, Ho, Wo);
        int st = launch_status();
        if (st != FORGE_OK) return st;
        if ((st = launch_quantize(col16, col8, as, M, K, s)) != FORGE_OK) return st;
        if ((st = gemm_dense(col8, weight, as, w_scale, bias, gout, nullptr, M, K, C_out, s)) != FORGE_OK)
            return st;
        transpose_f16_kernel<<<tgrid, 256, 0, s>>>(gout, out_n, M, C_out);
        if ((st = launch_status()) != FORGE_OK) return st;
    }
    return FORGE_OK;
}

extern "C" int forge_int8_conv2d_nhwc_s32(const int8_t* x, const int8_t* w, int32_t* out, int N, int H, int W,
                                          int C, int Co, int kH, int kW, int padH, int padW, int strideH,
                                          int strideW, int dilH, int dilW, void* stream)
{
    return conv_nhwc(x, w, nullptr, nullptr, nullptr, nullptr, out, N, H, W, C, Co, kH, kW, padH, padW, strideH,
                     strideW, dilH, dilW, as_stream(stream));
}

extern "C" int forge_int8_conv2d_nhwc_dequant(const int8_t* x, const int8_t* w, const float* act_scale,
                                              const uint16_t* w_scale, const uint16_t* bias, uint16_t* out,
                                              int N, int H, int W, int C, int Co, int kH, int kW, int padH,
                                              int padW, int strideH, int strideW, int dilH, int dilW,
                                              void* stream)
{
    return conv_nhwc(x, w, act_scale, w_scale, bias, out, nullptr, N, H, W, C, Co, kH, kW, padH, padW, strideH,
                     strideW, dilH, dilW, as_stream(stream));
}
