// INT8 ConvTranspose2d, kernel 2, stride 2, for gfx950.
//
// Reference: src/nn/int8_conv_transpose2d.cu:107-191. With stride == kernel every input
// pixel owns one 2x2 output block, so the layer is a GEMM of the per-pixel quantized input
// rows (H*W, C_in) with the repacked weights (4*C_out, C_in), row co*4 + kh*2 + kw, followed
// by a scatter to NCHW. The reference runs transpose -> quantize -> GEMM to an FP16 buffer
// -> scatter + bias, one image at a time. Here, for C_in in {32, 64, 128, 256} and
// H*W % 8 == 0, convt_fused_kernel does all of it in one pass per 32-pixel tile (described at
// the kernel): input read once, INT8 activations kept in LDS, output written once, one launch
// for all images, no workspace traffic. Every other shape takes two kernels:
//   1. quantize_pixels_nchw reads the NCHW image once and writes the INT8 pixel rows and
//      their scales (no FP16 transpose buffer);
//   2. the dense tile engine runs the GEMM with the upsample-scatter epilogue: each wave's
//      FP16 tile (act_scale * w_scale[co], no bias, rounded to FP16 as the reference's GEMM
//      output is) gets the bias added in fp32, is rounded again, and is stored straight into
//      the NCHW output as 16-byte runs of 4 pixels x (kw = 0, 1) -- the (M, 4*C_out) FP16
//      intermediate is never written.
//    Images are processed in chunks as large as the caller's workspace allows (its size is
//    the reference's formula, of which one image needs only the INT8 rows and scales), so
//    small images do not cost two launches each.
// Every per-pixel result is independent of the path and the chunking.
#include "common.h"
#include "gemm_dense.h"
#include "mfma_tile.h"

#include <algorithm>

namespace forge_amd {

static size_t up256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

// Single-pass kernel for C_in = 32 * KC (KC = 1, 2, 4, 8), H*W % 8 == 0: one workgroup (2 waves)
// takes 32 consecutive pixels of one image and writes their whole (C_out, 2x2) output, so the
// INT8 activations never leave the chip and the input is read once. Tiles of 32 pixels (one MFMA
// row block) rather than 64 give twice the workgroups, whose load, compute and store phases then
// overlap across a CU's workgroups instead of running in step (measured (1,64,270,480) -> 32:
// 22.5 -> 21.1 us; (2,128,128,128) -> 64: 16.0 -> 14.4 us); 128-pixel tiles were slower still.
//   1. Thread t loads pixels 8*(t%4) .. +8 of channels t/4 + 32k as 16-byte rows (KC loads
//      in flight; the wave's first MFMA item's weight rows and scales load behind them, later
//      items one item ahead), takes the per-pixel absmax over its channels on fp16 bit patterns
//      (one packed u16 maximum per two pixels; the fp32 maximum for a pixel holding a NaN),
//      then over the wave's 16 channel groups (lane shuffles) and the 2 waves (LDS): the row
//      arithmetic of quantize_rows on each pixel's C_in values.
//   2. The quantized pixels form the A tile in LDS (32 x C_in bytes, 16-byte chunks swizzled
//      by row so the MFMA row reads spread over the banks).
//   3. Work items (n-block j of 32 GEMM columns for the tile's 32 pixels) go round-robin to the
//      2 waves; B fragments are the weight rows, read from L2 straight into registers; K is
//      KC steps of v_mfma_i32_32x32x32_i8.
//   4. A lane's accumulators are one pixel x 4 consecutive columns n = co*4 + (kh, kw): the
//      2x2 output block of one channel, so the dequant (act_scale * w_scale[co], no bias,
//      rounded to FP16), the bias (added in fp32 and rounded again) and two 4-byte stores
//      (rows 2h and 2h + 1) happen in registers; adjacent lanes are adjacent pixels, so each
//      store instruction writes 128-byte runs.
// Up to 64 input channels the kernel is asked for 6 waves per SIMD: the compiler then keeps the
// 16 accumulators in VGPRs beside the rest (67 at C_in = 64, 7 waves; 86 registers and 5 waves
// otherwise), (1,64,270,480)->32 20.5 -> 19.0-19.1 us, (1,32,540,960)->16 33 -> 29.7-30.3 us. At 128
// and 256 channels that limit spills, so those keep the default.
template <int KC>
constexpr int convt_min_waves() { return KC <= 2 ? 6 : 1; }

template <int KC>
__global__ __launch_bounds__(128, convt_min_waves<KC>()) void convt_fused_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ w, const uint16_t* __restrict__ w_scale,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int HW, int W, int C_out, int tiles)
{
    constexpr int C = 32 * KC;
    constexpr int kNch = C / 16;
    constexpr int PT = 32;                           // pixels per tile
    constexpr int kNW = PT / 16;                     // waves: 4 * PT threads
    constexpr int kPG = PT / 8;                      // 8-pixel groups per tile
    constexpr int kMB = PT / 32;                     // 32-pixel MFMA row blocks
    static_assert((kNch & (kNch - 1)) == 0, "row swizzle needs a power-of-two chunk count");
    __shared__ __align__(16) int8_t As[PT * C];
    __shared__ float red[kNW][PT];
    __shared__ uint32_t redb[kNW][PT];
    __shared__ int nan_px[PT];
    __shared__ float ascale[PT];
    __shared__ float sinv[PT];
    const int t = threadIdx.x, lane = t & (kWave - 1), wave = t >> 6;
    const int img = blockIdx.x / tiles;
    const int p0 = (blockIdx.x - img * tiles) * PT;
    const int np = min(PT, HW - p0);                 // a multiple of 8

    // 1. loads and per-pixel absmax
    const int po = t % kPG, cg = t / kPG;
    const bool pin = 8 * po < np;
    const uint16_t* xi = x + static_cast<size_t>(img) * C * HW + p0 + 8 * po;
    uint4 v[KC];
#pragma unroll
    for (int k = 0; k < KC; k++)
        v[k] = pin ? *reinterpret_cast<const uint4*>(xi + static_cast<size_t>(cg + 32 * k) * HW)
                   : make_uint4(0u, 0u, 0u, 0u);

    // The wave's first MFMA item's weight fragments and scales load now, behind the input loads
    // (they do not depend on them); later items load one item ahead.
    const int N = 4 * C_out;
    const int items = kMB * ((N + 31) / 32);
    const int l31 = lane & 31, hi = lane >> 5;
    const bool has_bias = bias != nullptr;
    struct Item { v4i fb[KC]; uint16_t ws[4], b[4]; };
    auto load_item = [&](int it, Item& I) {
        const int j = it / kMB;
        const int n = 32 * j + l31;
        const int nc = n < N ? n : N - 1;
#pragma unroll
        for (int ks = 0; ks < KC; ks++)
            I.fb[ks] = *reinterpret_cast<const v4i*>(w + static_cast<size_t>(nc) * C + 16 * (2 * ks + hi));
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int co = min(8 * j + 2 * g + hi, C_out - 1);
            I.ws[g] = w_scale[co];
            I.b[g] = has_bias ? bias[co] : static_cast<uint16_t>(0);
        }
    };
    Item cur;
    if (wave < items) load_item(wave, cur);

    // Per-pixel absmax on fp16 bit patterns: lane word q holds pixels 2q, 2q + 1 of one channel,
    // so one packed u16 maximum covers two pixels (magnitude bits order as the magnitudes); a
    // pixel whose maximum pattern is a NaN takes the fp32 maximum (fmaxf skips NaN).
    uint32_t mb[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int k = 0; k < KC; k++) {
        mb[0] = pk_max_u16(mb[0], v[k].x & 0x7FFF7FFFu);
        mb[1] = pk_max_u16(mb[1], v[k].y & 0x7FFF7FFFu);
        mb[2] = pk_max_u16(mb[2], v[k].z & 0x7FFF7FFFu);
        mb[3] = pk_max_u16(mb[3], v[k].w & 0x7FFF7FFFu);
    }
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int off = kPG; off < kWave; off <<= 1)
            mb[q] = pk_max_u16(mb[q], static_cast<uint32_t>(__shfl_xor(static_cast<int>(mb[q]), off, kWave)));
    if (lane < kPG) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            redb[wave][8 * po + 2 * q] = mb[q] & 0xFFFFu;
            redb[wave][8 * po + 2 * q + 1] = mb[q] >> 16;
        }
    }
    __syncthreads();
    if (t < PT) {
        uint32_t bits = redb[0][t];
#pragma unroll
        for (int wv = 1; wv < kNW; wv++) bits = max(bits, redb[wv][t]);
        nan_px[t] = bits > kHalfInfBits ? 1 : 0;
        ascale[t] = h2f(static_cast<uint16_t>(bits));
    }
    __syncthreads();
    if (__builtin_amdgcn_readfirstlane(__syncthreads_or(t < PT && nan_px[t]))) {
        // rare: some pixel holds a NaN -- its fp32 maximum over the channels
        float m[8];
#pragma unroll
        for (int e = 0; e < 8; e++) m[e] = 0.0f;
#pragma unroll
        for (int k = 0; k < KC; k++) {
            const uint32_t u[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
            for (int e = 0; e < 8; e++)
                m[e] = fmaxf(m[e], fabsf(h2f(static_cast<uint16_t>((e & 1) ? (u[e >> 1] >> 16) : (u[e >> 1] & 0xFFFFu)))));
        }
#pragma unroll
        for (int e = 0; e < 8; e++)
#pragma unroll
            for (int off = kPG; off < kWave; off <<= 1) m[e] = fmaxf(m[e], __shfl_xor(m[e], off, kWave));
        if (lane < kPG) {
#pragma unroll
            for (int e = 0; e < 8; e++) red[wave][8 * po + e] = m[e];
        }
        __syncthreads();
        if (t < PT && nan_px[t]) {
            float a = red[0][t];
#pragma unroll
            for (int wv = 1; wv < kNW; wv++) a = fmaxf(a, red[wv][t]);
            ascale[t] = a;
        }
        __syncthreads();
    }
    if (t < PT) {
        const float scale = row_scale(ascale[t]);
        ascale[t] = scale;
        sinv[t] = 1.0f / scale;
    }
    __syncthreads();

    // 2. quantize into the A tile: As[p][c] at chunk (c / 16) ^ (p % kNch). qrow_bits gives the
    //    byte of clamp(rne(x * inv)) for a value of the pixel whose absmax gave inv.
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const int p = 8 * po + e;
        const float inv = sinv[p];
#pragma unroll
        for (int k = 0; k < KC; k++) {
            const int c = cg + 32 * k;
            const uint32_t word = (e & 1) ? ((&v[k].x)[e >> 1] >> 16) : ((&v[k].x)[e >> 1] & 0xFFFFu);
            As[p * C + ((((c >> 4) ^ (p & (kNch - 1)))) << 4) + (c & 15)] =
                static_cast<int8_t>(qrow_bits(static_cast<uint16_t>(word), inv) & 0xFFu);
        }
    }
    __syncthreads();

    // 3./4. MFMA items and the in-register scatter, stored through a buffer resource over this
    // image's output (under 2^31 bytes, checked by the host) with 32-bit byte offsets.
    const uint32_t plane_b = 8u * static_cast<uint32_t>(HW);     // bytes of one output channel
    const uint32_t row_b = 4u * static_cast<uint32_t>(W);        // bytes of one output row
    const __amdgpu_buffer_rsrc_t yr =
        buf_rsrc(y + static_cast<size_t>(img) * C_out * 4 * static_cast<size_t>(HW), plane_b * static_cast<uint32_t>(C_out));
    for (int it = wave; it < items; it += kNW) {
        const int i = it % kMB, j = it / kMB;
        v4i fb[KC];
#pragma unroll
        for (int ks = 0; ks < KC; ks++) fb[ks] = cur.fb[ks];
        float wsv[4];
        uint32_t bbits[4];
#pragma unroll
        for (int g = 0; g < 4; g++) {
            wsv[g] = h2f(cur.ws[g]);
            bbits[g] = cur.b[g];
        }
        if (it + kNW < items) load_item(it + kNW, cur);
        v16i acc;
#pragma unroll
        for (int e = 0; e < 16; e++) acc[e] = 0;
        const int row = 32 * i + l31;
#pragma unroll
        for (int ks = 0; ks < KC; ks++) {
            const int c = 2 * ks + hi;
            const v4i fa = *reinterpret_cast<const v4i*>(As + row * C + ((c ^ (row & (kNch - 1))) << 4));
            acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(fb[ks], fa, acc, 0, 0, 0);
        }
        if (row < np) {
            const int p = p0 + row, h = p / W, wc = p - h * W;
            const float as = ascale[row];
            const uint32_t pix_b = 2u * static_cast<uint32_t>(h) * row_b + 4u * static_cast<uint32_t>(wc);
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int co = 8 * j + 2 * g + hi;     // columns 4co .. 4co + 3
                if (co >= C_out) continue;
                // dequant_gemm without a bias, (kw 0, 1) pairs rounded to fp16 by one
                // v_cvt_pk_f16_f32 (round to nearest even, kw 0 in the low half), then the bias by
                // one v_pk_add_f16: an fp16 sum rounded once equals the sum taken in fp32 and
                // rounded to fp16 (when fp32 cannot hold the exact sum, the smaller term is below
                // a quarter of the larger's fp16 ulp, and both round to the larger)
                const float sc = as * wsv[g];
                float pq[4];
#pragma unroll
                for (int q = 0; q < 4; q++) pq[q] = static_cast<float>(acc[4 * g + q]) * sc;
                uint32_t h01, h23;
                asm("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(h01) : "v"(pq[0]), "v"(pq[1]));
                asm("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(h23) : "v"(pq[2]), "v"(pq[3]));
                if (has_bias) {
                    const uint32_t b2 = bbits[g] | (bbits[g] << 16);
                    asm("v_pk_add_f16 %0, %1, %2" : "=v"(h01) : "v"(h01), "v"(b2));
                    asm("v_pk_add_f16 %0, %1, %2" : "=v"(h23) : "v"(h23), "v"(b2));
                }
                const uint32_t off = pix_b + static_cast<uint32_t>(co) * plane_b;
                __builtin_amdgcn_raw_buffer_store_b32(h01, yr, off, 0, 0);          // kh = 0
                __builtin_amdgcn_raw_buffer_store_b32(h23, yr, off + row_b, 0, 0);  // kh = 1
            }
        }
    }
}

template <int KC>
static int launch_convt_fused(const uint16_t* input, const int8_t* weight, const uint16_t* w_scale,
                              const uint16_t* bias, uint16_t* output, int N, int HW, int W, int C_out,
                              hipStream_t s)
{
    const int tiles = divup(HW, 32);
    const long long blocks = static_cast<long long>(N) * tiles;
    if (blocks > 0x7FFFFFFFLL) return FORGE_EINVAL;
    convt_fused_kernel<KC><<<static_cast<unsigned>(blocks), 128, 0, s>>>(input, weight, w_scale, bias, output, HW, W,
                                                                        C_out, tiles);
    return launch_status();
}

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
    hipStream_t s = as_stream(stream);
    if (HW % 8 == 0 && 8LL * C_out * HW < (1LL << 31) && aligned(input, 16) && aligned(weight, 16) &&
        aligned(output, 4)) {
        const int hw = static_cast<int>(HW);
        switch (C_in) {
            case 32:  return launch_convt_fused<1>(input, weight, w_scale, bias, output, N, hw, W, C_out, s);
            case 64:  return launch_convt_fused<2>(input, weight, w_scale, bias, output, N, hw, W, C_out, s);
            case 128: return launch_convt_fused<4>(input, weight, w_scale, bias, output, N, hw, W, C_out, s);
            case 256: return launch_convt_fused<8>(input, weight, w_scale, bias, output, N, hw, W, C_out, s);
            default: break;
        }
    }
    const size_t per_image = up256(static_cast<size_t>(HW) * C_in) + up256(static_cast<size_t>(HW) * 4);
    const size_t ws_bytes = forge_int8_conv_transpose2d_k2s2_workspace_size(C_in, H, W, C_out);
    long long chunk = static_cast<long long>(ws_bytes / per_image);
    chunk = std::max(1LL, std::min<long long>(chunk, N));
    chunk = std::min<long long>(chunk, 0x7FFFFFFFLL / HW);       // GEMM rows stay in int range
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
