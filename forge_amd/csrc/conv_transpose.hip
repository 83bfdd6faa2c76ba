// INT8 ConvTranspose2d, kernel 2, stride 2, for gfx950.
//
// Reference: src/nn/int8_conv_transpose2d.cu:107-191. With stride == kernel every input
// pixel owns one 2x2 output block, so the layer is a GEMM of the per-pixel quantized input
// rows (H*W, C_in) with the repacked weights (4*C_out, C_in), row co*4 + kh*2 + kw, followed
// by a scatter to NCHW. The reference runs transpose -> quantize -> GEMM to an FP16 buffer
// -> scatter + bias, one image at a time. Here:
//   1. quantize_pixels_nchw reads the NCHW image once and writes the INT8 pixel rows and
//      their scales (no FP16 transpose buffer);
//   2. the dense tile engine runs the GEMM with the upsample-scatter epilogue: each wave's
//      FP16 tile (act_scale * w_scale[co], no bias, rounded to FP16 as the reference's GEMM
//      output is) gets the bias added in fp32, is rounded again, and is stored straight into
//      the NCHW output as 16-byte runs of 4 pixels x (kw = 0, 1) -- the (M, 4*C_out) FP16
//      intermediate is never written.
// Images are processed in chunks as large as the caller's workspace allows (its size is the
// reference's formula, of which one image needs only the INT8 rows and scales), so small
// images do not cost two launches each. Every per-pixel result is independent of the chunk.
#include "common.h"
#include "gemm_dense.h"
#include "mfma_tile.h"

#include <algorithm>

namespace forge_amd {

static size_t up256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

}  // namespace forge_amd

using namespace forge_amd;

extern "C" size_t forge_int8_conv_transpose2d_k2s2_workspace_size(int C_in, int H, int W, int C_out)
{
    // int8_conv_transpose2d.cu:107-123: col fp16 + col int8 + act_scale + w_scale_rep + gemm_out.
    if (C_in <= 0 || H <= 0 || W <= 0 || C_out <= 0) return 0;
    const size_t M = static_cast<size_t>(H) * W, K = static_cast<size_t>(C_in), Ng = 4 * static_cast<size_t>(C_out);
    return M * K * 2 + M * K + M * 4 + Ng * 2 + M * Ng * 2;
}

extern "C" int forge_int8_conv_transpose2d_k2s2_forward(const uint16_t* input, const int8_t* weight,
                                                        const uint16_t* w_scale, const uint16_t* bias,
                                                        uint16_t* output, int N, int C_in, int H, int W,
                                                        int C_out, void* workspace, void* stream)
{
    if (N <= 0 || C_in <= 0 || C_out <= 0 || H <= 0 || W <= 0) return FORGE_OK;
    if (!input || !weight || !w_scale || !output || !workspace) return FORGE_EINVAL;
    const long long HW = static_cast<long long>(H) * W;
    if (HW > 0x7FFFFFFFLL || 4LL * C_out > 0x7FFFFFFFLL) return FORGE_EINVAL;
    const size_t per_image = up256(static_cast<size_t>(HW) * C_in) + up256(static_cast<size_t>(HW) * 4);
    const size_t ws_bytes = forge_int8_conv_transpose2d_k2s2_workspace_size(C_in, H, W, C_out);
    long long chunk = static_cast<long long>(ws_bytes / per_image);
    chunk = std::max(1LL, std::min<long long>(chunk, N));
    chunk = std::min<long long>(chunk, 0x7FFFFFFFLL / HW);       // GEMM rows stay in int range
    hipStream_t s = as_stream(stream);
    const int Ng = 4 * C_out;
    const size_t in_img = static_cast<size_t>(C_in) * HW, out_img = static_cast<size_t>(Ng) * HW;
    for (long long n0 = 0; n0 < N; n0 += chunk) {
        const int cnt = static_cast<int>(std::min<long long>(chunk, N - n0));
        const int M = static_cast<int>(cnt * HW);
        int8_t* q = static_cast<int8_t*>(workspace);
        float* as = reinterpret_cast<float*>(static_cast<char*>(workspace) + up256(static_cast<size_t>(M) * C_in));
        int st = launch_quantize_pixels_nchw(input + n0 * in_img, q, as, cnt, C_in, static_cast<int>(HW), s);
        if (st != FORGE_OK) return st;
        uint16_t* out = output + n0 * out_img;
        GemmEpilogue ep{};
        ep.c16 = out;
        ep.act_scale = as;
        ep.w_scale = w_scale;
        ep.bias = nullptr;
        ep.M = M;
        ep.N = Ng;
        ep.vec_out = (W % 4 == 0 && aligned(out, 16)) ? 1 : 0;
        ep.up_w = W;
        ep.up_hw = static_cast<int>(HW);
        ep.post_bias = bias;
        if ((st = gemm_tiles(q, weight, ep, M, C_in, Ng, s)) != FORGE_OK) return st;
    }
    return FORGE_OK;
}
