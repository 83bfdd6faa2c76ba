// INT8-weight depthwise conv2d for gfx950: FP16 NCHW in and out, weights (C, kH*kW) int8 with
// a per-channel FP16 scale.
//
// Reference: src/nn/int8_depthwise_conv2d.cu:25-103 -- one thread per output, taps in
// (kh, kw) order, out-of-image taps skipped, w = (float)q * scale, sum += inp * w (one fused
// multiply-add per tap, as nvcc contracts it), + bias, round to FP16. Both kernels here keep
// exactly that per-output sequence, so their results are bit-identical to it.
//
// The layer is HBM-bound (2 bytes in and 2 bytes out per pixel at stride 1), so the MI355X
// design is about reading the input once:
//   depthwise_tile_kernel (stride 1, dilation 1, kW <= 9, kH <= 16): a workgroup computes a
//     32 x 64 output tile of one channel plane from a (32 + kH - 1) x (64 + kW - 1) input
//     tile staged in LDS with coalesced 128-byte row reads; each lane computes 8 adjacent
//     outputs of one row from two 16-byte LDS reads per tap row, with the channel's
//     dequantized taps broadcast from LDS, and writes them as one 16-byte store.
//     Zero-filled padding gives the same sums as skipped taps (fma(0, w, s) == s for finite w,
//     and the sum starts at +0 so it is never -0); a channel with a non-finite tap weight
//     takes the masked loop, which skips out-of-image taps exactly as the reference does.
//   depthwise_direct_kernel: every other geometry, one output per lane, the reference's loop.
#include "common.h"

#include <algorithm>

namespace forge_amd {

constexpr int kDwTileH = 32, kDwTileW = 64, kDwPer = 8;
constexpr int kDwMaxKH = 16, kDwMaxKW = 9;
constexpr int kDwPitch = 72;   // halves per staged row (>= kDwTileW + kDwMaxKW - 1, 16-byte multiple)

static int dw_out(int in, int pad, int dil, int k, int stride) {
    return (in + 2 * pad - dil * (k - 1) - 1) / stride + 1;
}

template <bool MASK>
__device__ __forceinline__ void dw_rows(const uint16_t* tile, const float* wf, float (&acc)[kDwPer], int ty, int tx,
                                        int kH, int kW, int hi0, int H, uint32_t colmask)
{
    for (int kh = 0; kh < kH; kh++) {
        const uint16_t* row = tile + (ty + kh) * kDwPitch + tx * kDwPer;
        const uint4 a = *reinterpret_cast<const uint4*>(row);
        const uint4 b = *reinterpret_cast<const uint4*>(row + 8);
        const uint32_t u[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        float v[16];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            v[2 * i] = h2f(static_cast<uint16_t>(u[i] & 0xFFFFu));
            v[2 * i + 1] = h2f(static_cast<uint16_t>(u[i] >> 16));
        }
        const bool row_ok = !MASK || static_cast<unsigned>(hi0 + kh) < static_cast<unsigned>(H);
#pragma unroll
        for (int kw = 0; kw < kDwMaxKW; kw++) {
            if (kw < kW) {             // a guard, not a break: the loop stays unrolled
                const float wk = wf[kh * kW + kw];
#pragma unroll
                for (int j = 0; j < kDwPer; j++) {
                    if constexpr (MASK) {
                        if (row_ok && ((colmask >> (j + kw)) & 1u)) acc[j] = __builtin_fmaf(v[j + kw], wk, acc[j]);
                    } else {
                        acc[j] = __builtin_fmaf(v[j + kw], wk, acc[j]);
                    }
                }
            }
        }
    }
}

__global__ __launch_bounds__(256) void depthwise_tile_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ w, const uint16_t* __restrict__ w_scale,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int C, int H, int W, int kH, int kW, int padH,
    int padW, int Ho, int Wo, int tiles_h, int tiles_w, int vec_out)
{
    __shared__ __align__(16) uint16_t tile[(kDwTileH + kDwMaxKH - 1) * kDwPitch];
    __shared__ float wf[kDwMaxKH * kDwMaxKW];
    const int t = threadIdx.x;
    const int per_plane = tiles_h * tiles_w;
    const int plane = blockIdx.x / per_plane;          // n * C + c
    const int rem = blockIdx.x - plane * per_plane;
    const int th = rem / tiles_w, tw = rem - th * tiles_w;
    const int c = plane % C;
    const int ho0 = th * kDwTileH, wo0 = tw * kDwTileW;
    const int hi0 = ho0 - padH, wi0 = wo0 - padW;

    // The channel's taps, dequantized once: (float)q * scale.
    bool finite = true;
    if (t < kH * kW) {
        const float v = static_cast<float>(w[static_cast<size_t>(c) * kH * kW + t]) * h2f(w_scale[c]);
        wf[t] = v;
        finite = __builtin_isfinite(v);
    }
    // Input tile with zero padding outside the image. Every load is issued before the first
    // LDS write (fixed trip counts, guarded), so a wave has all of its rows in flight at once:
    // the main 64 columns as one 128-byte row per wave instruction, and the at most 8 halo
    // columns of 8 rows per instruction.
    const uint16_t* xp = x + static_cast<size_t>(plane) * H * W;
    const int rows = kDwTileH + kH - 1, cols = kDwTileW + kW - 1;
    constexpr int kMainIters = (kDwTileH + kDwMaxKH - 1 + 3) / 4;
    constexpr int kHaloIters = ((kDwTileH + kDwMaxKH - 1) * 8 + 255) / 256;
    const int lane = t & 63, wv = t >> 6;
    uint16_t mv[kMainIters], hv[kHaloIters];
#pragma unroll
    for (int k = 0; k < kMainIters; k++) {
        const int r = wv + 4 * k, hi = hi0 + r, wi = wi0 + lane;
        uint16_t v = 0;
        if (r < rows && static_cast<unsigned>(hi) < static_cast<unsigned>(H) &&
            static_cast<unsigned>(wi) < static_cast<unsigned>(W))
            v = xp[static_cast<size_t>(hi) * W + wi];
        mv[k] = v;
    }
#pragma unroll
    for (int k = 0; k < kHaloIters; k++) {
        const int e = t + 256 * k, r = e >> 3, cl = kDwTileW + (e & 7);
        const int hi = hi0 + r, wi = wi0 + cl;
        uint16_t v = 0;
        if (r < rows && cl < cols && static_cast<unsigned>(hi) < static_cast<unsigned>(H) &&
            static_cast<unsigned>(wi) < static_cast<unsigned>(W))
            v = xp[static_cast<size_t>(hi) * W + wi];
        hv[k] = v;
    }
#pragma unroll
    for (int k = 0; k < kMainIters; k++) {
        const int r = wv + 4 * k;
        if (r < rows) tile[r * kDwPitch + lane] = mv[k];
    }
#pragma unroll
    for (int k = 0; k < kHaloIters; k++) {
        const int e = t + 256 * k, r = e >> 3, cl = kDwTileW + (e & 7);
        if (r < rows && cl < cols) tile[r * kDwPitch + cl] = hv[k];
    }
    const bool all_finite = __syncthreads_and(finite);

    const int tx = t & 7, ty = t >> 3;
    float acc[kDwPer];
#pragma unroll
    for (int j = 0; j < kDwPer; j++) acc[j] = 0.0f;
    if (all_finite) {
        dw_rows<false>(tile, wf, acc, ty, tx, kH, kW, 0, 0, 0u);
    } else {
        // Bit i: input column wo + i - padW of this lane's first output wo is inside the image.
        uint32_t colmask = 0;
        const int wb = wi0 + tx * kDwPer;
        for (int i = 0; i < kDwPer + kDwMaxKW - 1; i++)
            if (static_cast<unsigned>(wb + i) < static_cast<unsigned>(W)) colmask |= 1u << i;
        dw_rows<true>(tile, wf, acc, ty, tx, kH, kW, hi0 + ty, H, colmask);
    }

    const int ho = ho0 + ty, wo = wo0 + tx * kDwPer;
    if (ho >= Ho || wo >= Wo) return;
    const bool has_bias = bias != nullptr;
    const float b = has_bias ? h2f(bias[c]) : 0.0f;
    uint16_t h[kDwPer];
#pragma unroll
    for (int j = 0; j < kDwPer; j++) h[j] = f2h(has_bias ? acc[j] + b : acc[j]);
    uint16_t* yp = y + (static_cast<size_t>(plane) * Ho + ho) * Wo + wo;
    if (vec_out && wo + kDwPer <= Wo) {
        *reinterpret_cast<uint4*>(yp) = make_uint4(h[0] | (static_cast<uint32_t>(h[1]) << 16),
                                                   h[2] | (static_cast<uint32_t>(h[3]) << 16),
                                                   h[4] | (static_cast<uint32_t>(h[5]) << 16),
                                                   h[6] | (static_cast<uint32_t>(h[7]) << 16));
    } else {
#pragma unroll
        for (int j = 0; j < kDwPer; j++)
            if (wo + j < Wo) yp[j] = h[j];
    }
}

__global__ __launch_bounds__(256) void depthwise_direct_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ w, const uint16_t* __restrict__ w_scale,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int C, int H, int W, int kH, int kW, int padH,
    int padW, int strideH, int strideW, int dilH, int dilW, int Ho, int Wo, long long total)
{
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int wo = static_cast<int>(i % Wo);
        const long long t = i / Wo;
        const int ho = static_cast<int>(t % Ho);
        const long long plane = t / Ho;
        const int c = static_cast<int>(plane % C);
        const float scale = h2f(w_scale[c]);
        const int8_t* wc = w + static_cast<size_t>(c) * kH * kW;
        const uint16_t* xp = x + static_cast<size_t>(plane) * H * W;
        float sum = 0.0f;
        for (int kh = 0; kh < kH; kh++) {
            const int hi = ho * strideH + kh * dilH - padH;
            if (hi < 0 || hi >= H) continue;
            for (int kw = 0; kw < kW; kw++) {
                const int wi = wo * strideW + kw * dilW - padW;
                if (wi < 0 || wi >= W) continue;
                const float wk = static_cast<float>(wc[kh * kW + kw]) * scale;
                sum = __builtin_fmaf(h2f(xp[static_cast<size_t>(hi) * W + wi]), wk, sum);
            }
        }
        if (bias) sum = sum + h2f(bias[c]);
        y[i] = f2h(sum);
    }
}

}  // namespace forge_amd

using namespace forge_amd;

extern "C" int forge_int8_depthwise_conv2d_forward(const uint16_t* input, const int8_t* weight,
                                                   const uint16_t* w_scale, const uint16_t* bias,
                                                   uint16_t* output, int N, int C, int H, int W, int kH,
                                                   int kW, int padH, int padW, int strideH, int strideW,
                                                   int dilH, int dilW, void* stream)
{
    if (N <= 0 || C <= 0) return FORGE_OK;
    if (!input || !weight || !w_scale || !output) return FORGE_EINVAL;
    if (kH <= 0 || kW <= 0 || strideH <= 0 || strideW <= 0 || dilH <= 0 || dilW <= 0 || padH < 0 || padW < 0)
        return FORGE_EINVAL;
    if (H <= 0 || W <= 0) return FORGE_OK;
    const int Ho = dw_out(H, padH, dilH, kH, strideH), Wo = dw_out(W, padW, dilW, kW, strideW);
    if (Ho <= 0 || Wo <= 0) return FORGE_OK;
    const long long planes = static_cast<long long>(N) * C;
    hipStream_t s = as_stream(stream);
    if (strideH == 1 && strideW == 1 && dilH == 1 && dilW == 1 && kH <= kDwMaxKH && kW <= kDwMaxKW) {
        const int tiles_h = divup(Ho, kDwTileH), tiles_w = divup(Wo, kDwTileW);
        const long long blocks = planes * tiles_h * tiles_w;
        if (blocks <= 0x7FFFFFFFLL) {
            const int vec = (Wo % kDwPer == 0 && aligned(output, 16)) ? 1 : 0;
            depthwise_tile_kernel<<<static_cast<unsigned>(blocks), 256, 0, s>>>(
                input, weight, w_scale, bias, output, C, H, W, kH, kW, padH, padW, Ho, Wo, tiles_h, tiles_w, vec);
            return launch_status();
        }
    }
    const long long total = planes * Ho * Wo;
    const int blocks = static_cast<int>(std::min<long long>(divupll(total, 256), 65536));
    depthwise_direct_kernel<<<blocks, 256, 0, s>>>(input, weight, w_scale, bias, output, C, H, W, kH, kW, padH, padW,
                                                   strideH, strideW, dilH, dilW, Ho, Wo, total);
    return launch_status();
}
