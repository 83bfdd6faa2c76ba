// INT8-weight depthwise conv2d for gfx950: FP16 NCHW in and out, weights (C, kH*kW) int8 with
// a per-channel FP16 scale.
//
// Reference: src/nn/int8_depthwise_conv2d.cu:25-103 -- one thread per output, taps in
// (kh, kw) order, out-of-image taps skipped, w = (float)q * scale, sum += inp * w (one fused
// multiply-add per tap, as nvcc contracts it), + bias, round to FP16. Both kernels here keep
// exactly that per-output sequence, so their results are bit-identical to it.
//
// The layer is HBM-bound (2 bytes in and 2 bytes out per pixel at stride 1), so the MI355X
// design is about reading the input once, with few instructions per byte:
//   depthwise_rows_kernel (stride 1, dilation 1, square 1/3/5/7 kernels, column padding
//     (k-1)/2 or 0, W % 8 == 0): the barrier-free rolling window described at the kernel.
//     (1, 64, 540, 960) 3x3: 31.9 us, 4.2 TB/s; the LDS tile kernel below took 54 us there --
//     its load / barrier / compute / store life per 32 x 64 tile kept a wave alive ~5 us
//     for ~700 instructions.
//   depthwise_tile_kernel (other stride-1 shapes, kW <= 9, kH <= 16): a workgroup computes a
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
#include <climits>

namespace forge_amd {

constexpr int kDwTileH = 32, kDwTileW = 64, kDwPer = 8;
constexpr int kDwMaxKH = 16, kDwMaxKW = 9;
constexpr int kDwPitch = 72;   // halves per staged row (>= kDwTileW + kDwMaxKW - 1, 16-byte multiple)

// Output size (int8_depthwise_conv2d.cu's formula, C's truncating division) in 64 bits, INT_MAX
// where it passes the int range; the caller has checked k, stride, dil > 0 and pad >= 0.
static int dw_out(int in, int pad, int dil, int k, int stride) {
    const long long o = (static_cast<long long>(in) + 2LL * pad - static_cast<long long>(dil) * (k - 1) - 1) / stride + 1;
    return o > INT_MAX ? INT_MAX : static_cast<int>(o);
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
    const int tid = xcd_contiguous(blockIdx.x, gridDim.x);
    const int plane = tid / per_plane;                 // n * C + c
    const int rem = tid - plane * per_plane;
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

// Rolling-window kernel (stride 1, dilation 1, compile-time KH x KW, W % 8 == 0,
// 0 <= padW <= KW - 1): no LDS and no barrier. Lane l of a wave owns output columns
// [8c, 8c + 8) with c = 62 * cw + l - 1 (lanes 0 and 63 only lend their columns as the
// halo); every input row of the wave's strip is read once, as one 16-byte load per lane, and
// the padW columns on the left / KW - 1 - padW on the right come from the neighbouring lanes
// through DPP wave shifts. The wave walks the input rows of a strip of R output rows top to
// bottom, keeping the KH partial output rows in registers: input row hi adds its taps to the
// rows it reaches (kh ascending over time, kw ascending within a row -- the reference's
// per-output order), then the oldest row, now complete, is rounded and stored. Loads run
// kDwAhead rows ahead of the arithmetic. Rows outside the image are skipped like the
// reference's taps; columns outside it load as zeros, which is exact for finite taps
// (a channel with a non-finite tap runs the reference loop for its outputs instead).
constexpr int kDwAhead = 4;

__device__ __forceinline__ float half_of(const uint32_t (&u)[4], int i) {
    return h2f(static_cast<uint16_t>((i & 1) ? (u[i >> 1] >> 16) : (u[i >> 1] & 0xFFFFu)));
}

template <int KH, int KW, int PW>
__global__ __launch_bounds__(256) void depthwise_rows_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ w, const uint16_t* __restrict__ w_scale,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int C, int H, int W, int padH, int Ho,
    int Wo, int col_waves, int strips, int R, int total_waves, int vec_out)
{
    static_assert(KW - 1 <= 8 && PW >= 0 && PW <= KW - 1, "halo must fit a neighbour lane's 8 columns");
    constexpr int padW = PW;
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = xcd_contiguous(blockIdx.x, gridDim.x) * 4 + static_cast<int>(threadIdx.x / kWave);
    if (wid >= total_waves) return;
    const int per_plane = col_waves * strips;
    const int plane = wid / per_plane;
    const int rem = wid - plane * per_plane;
    const int cw = rem / strips, strip = rem - cw * strips;
    const int c = plane % C;
    const int chunk = 62 * cw + lane - 1;
    const int wo0 = 8 * chunk;
    const bool own = lane >= 1 && lane <= 62 && chunk >= 0 && wo0 < Wo;
    const bool in_cols = chunk >= 0 && wo0 < W;          // W % 8 == 0: a chunk is all in or all out
    const int ho0 = strip * R, ho_end = min(ho0 + R, Ho);

    float wt[KH * KW];
    bool finite = true;
    const float scale = h2f(w_scale[c]);
#pragma unroll
    for (int t = 0; t < KH * KW; t++) {
        wt[t] = static_cast<float>(w[static_cast<size_t>(c) * KH * KW + t]) * scale;
        finite = finite && __builtin_isfinite(wt[t]);
    }
    const bool has_bias = bias != nullptr;
    const float bv = has_bias ? h2f(bias[c]) : 0.0f;
    const uint16_t* xp = x + static_cast<size_t>(plane) * H * W;
    uint16_t* yp = y + static_cast<size_t>(plane) * Ho * Wo;

    if (!finite) {
        // The reference loop, for this lane's outputs of the strip.
        if (!own) return;
        for (int ho = ho0; ho < ho_end; ho++)
            for (int j = 0; j < 8; j++) {
                const int wo = wo0 + j;
                if (wo >= Wo) break;
                float sum = 0.0f;
                for (int kh = 0; kh < KH; kh++) {
                    const int hi = ho + kh - padH;
                    if (hi < 0 || hi >= H) continue;
                    for (int kw = 0; kw < KW; kw++) {
                        const int wi = wo + kw - padW;
                        if (wi < 0 || wi >= W) continue;
                        sum = __builtin_fmaf(h2f(xp[static_cast<size_t>(hi) * W + wi]), wt[kh * KW + kw], sum);
                    }
                }
                yp[static_cast<size_t>(ho) * Wo + wo] = f2h(has_bias ? sum + bv : sum);
            }
        return;
    }

    const int hi_first = ho0 - padH;
    const int rows = (ho_end - ho0) + KH - 1;             // input rows hi_first .. hi_first + rows - 1
    auto load_row = [&](int hi) -> uint4 {
        if (in_cols && static_cast<unsigned>(hi) < static_cast<unsigned>(H))
            return *reinterpret_cast<const uint4*>(xp + static_cast<size_t>(hi) * W + wo0);
        return make_uint4(0u, 0u, 0u, 0u);
    };
    float acc[KH][8];
#pragma unroll
    for (int s = 0; s < KH; s++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[s][j] = 0.0f;

    // Rows in flight. For 3x3 it is 3 (= KH): the unrolled rows then map each output offset s to
    // the partial-row slot (s + d) % KH at compile time, so slots are renamed instead of shifted
    // every row, and the kernel keeps 6 waves per SIMD (74 VGPRs; 4 rows with shifting: 81 VGPRs,
    // 5 waves, 30.6-30.9 vs 29.1-29.2 us at (1,64,540,960)).
    constexpr int kAhead = KH == 3 ? 3 : kDwAhead;
    constexpr bool kRename = kAhead % KH == 0;
    uint4 nxt[kAhead];
#pragma unroll
    for (int d = 0; d < kAhead; d++) nxt[d] = load_row(hi_first + d);

    for (int r0 = 0; r0 < rows; r0 += kAhead) {
        uint4 cur[kAhead];
#pragma unroll
        for (int d = 0; d < kAhead; d++) {
            cur[d] = nxt[d];
            nxt[d] = load_row(hi_first + r0 + kAhead + d);
        }
#pragma unroll
        for (int d = 0; d < kAhead; d++) {
            const int r = r0 + d;
            if (r >= rows) break;
            const int hi = hi_first + r;
            if (static_cast<unsigned>(hi) < static_cast<unsigned>(H)) {
                // The row window: padW halves from lane - 1, 8 own, KW - 1 - padW from lane + 1.
                const uint32_t own_w[4] = {cur[d].x, cur[d].y, cur[d].z, cur[d].w};
                uint32_t lft[4], rgt[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    lft[k] = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(own_w[k]), 0x138, 0xF, 0xF, false));
                    rgt[k] = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(own_w[k]), 0x130, 0xF, 0xF, false));
                }
                float v[8 + KW - 1];
#pragma unroll
                for (int i = 0; i < 8 + KW - 1; i++) {
                    // window index i is input column wo0 + i - PW (compile-time source lane and half)
                    const int col = i - PW;
                    v[i] = col < 0 ? half_of(lft, 8 + col) : (col < 8 ? half_of(own_w, col) : half_of(rgt, col - 8));
                }
                // Output offset s (row hi + padH - (KH - 1) + s, in slot (s + d) % KH when renamed,
                // else slot s) takes tap row kh = KH - 1 - s.
#pragma unroll
                for (int s = 0; s < KH; s++) {
                    const int kh = KH - 1 - s;
#pragma unroll
                    for (int kw = 0; kw < KW; kw++) {
                        const float wk = wt[kh * KW + kw];
#pragma unroll
                        for (int j = 0; j < 8; j++) {
                            const int sl = kRename ? (s + d) % KH : s;
                            acc[sl][j] = __builtin_fmaf(v[j + kw], wk, acc[sl][j]);
                        }
                    }
                }
            }
            // Offset 0 (output row hi + padH - KH + 1) has seen all its tap rows.
            const int o = hi + padH - (KH - 1);
            if (own && o >= ho0 && o < ho_end) {
                uint16_t h[8];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float a0 = acc[kRename ? d % KH : 0][j];
                    h[j] = f2h(has_bias ? a0 + bv : a0);
                }
                uint16_t* dst = yp + static_cast<size_t>(o) * Wo + wo0;
                if (vec_out && wo0 + 8 <= Wo) {
                    const v4i o4 = v4i{static_cast<int>(h[0] | (static_cast<uint32_t>(h[1]) << 16)),
                                       static_cast<int>(h[2] | (static_cast<uint32_t>(h[3]) << 16)),
                                       static_cast<int>(h[4] | (static_cast<uint32_t>(h[5]) << 16)),
                                       static_cast<int>(h[6] | (static_cast<uint32_t>(h[7]) << 16))};
                    __builtin_nontemporal_store(o4, reinterpret_cast<v4i*>(dst));
                } else {
#pragma unroll
                    for (int j = 0; j < 8; j++)
                        if (wo0 + j < Wo) dst[j] = h[j];
                }
            }
            if constexpr (kRename) {
#pragma unroll
                for (int j = 0; j < 8; j++) acc[d % KH][j] = 0.0f;   // the stored slot starts a new output row
            } else {
#pragma unroll
                for (int s = 0; s + 1 < KH; s++)
#pragma unroll
                    for (int j = 0; j < 8; j++) acc[s][j] = acc[s + 1][j];
#pragma unroll
                for (int j = 0; j < 8; j++) acc[KH - 1][j] = 0.0f;
            }
        }
    }
}

template <int KH, int KW, int PW>
static int launch_dw_rows(const uint16_t* input, const int8_t* weight, const uint16_t* w_scale,
                          const uint16_t* bias, uint16_t* output, long long planes, int C, int H, int W,
                          int padH, int Ho, int Wo, hipStream_t s)
{
    const int chunks = divup(Wo, 8);
    const int col_waves = divup(chunks, 62);
    // Strip height: the tallest of 32 / 16 / 8 rows that still gives >= 4 waves per SIMD.
    int R = 32;
    while (R > 8 && planes * col_waves * divup(Ho, R) < 4096) R >>= 1;
    const int strips = divup(Ho, R);
    const long long waves = planes * col_waves * strips;
    if (waves > 0x7FFFFFFFLL - 3) return FORGE_EINVAL;
    const unsigned blocks = static_cast<unsigned>(divupll(waves, 4));
    const int vec = (Wo % 8 == 0 && aligned(output, 16)) ? 1 : 0;
    depthwise_rows_kernel<KH, KW, PW><<<blocks, 256, 0, s>>>(input, weight, w_scale, bias, output, C, H, W, padH,
                                                             Ho, Wo, col_waves, strips, R, static_cast<int>(waves), vec);
    return launch_status();
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
    if (static_cast<long long>(H) * W > INT_MAX || static_cast<long long>(Ho) * Wo > INT_MAX) return FORGE_EINVAL;
    const long long planes = static_cast<long long>(N) * C;
    hipStream_t s = as_stream(stream);
    const bool unit = strideH == 1 && strideW == 1 && dilH == 1 && dilW == 1;
    // Rolling-window kernel: square 1/3/5/7 kernels with "same" (k-1)/2 or zero column padding.
    if (unit && W % 8 == 0 && aligned(input, 16) && kH == kW && (padW == (kW - 1) / 2 || padW == 0)) {
        const bool same = padW == (kW - 1) / 2;
#define FORGE_DW_ROWS(K) \
        return same ? launch_dw_rows<K, K, (K - 1) / 2>(input, weight, w_scale, bias, output, planes, C, H, W, padH, Ho, Wo, s) \
                    : launch_dw_rows<K, K, 0>(input, weight, w_scale, bias, output, planes, C, H, W, padH, Ho, Wo, s)
        switch (kH) {
            case 1: FORGE_DW_ROWS(1);
            case 3: FORGE_DW_ROWS(3);
            case 5: FORGE_DW_ROWS(5);
            case 7: FORGE_DW_ROWS(7);
            default: break;
        }
#undef FORGE_DW_ROWS
    }
    if (unit && kH <= kDwMaxKH && kW <= kDwMaxKW) {
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
