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
#include <climits>
#include <mutex>

namespace forge_amd {

// Output size (int8_conv2d.cu:29-31): (in + 2 pad - dil (k - 1) - 1) / stride + 1 with C's
// truncating division, evaluated in 64 bits; 0 for a geometry no convolution has (kernel, stride
// or dilation <= 0, negative padding), INT_MAX where the size passes the int range.
static int conv_out(int in, int pad, int dil, int k, int stride) {
    if (k <= 0 || stride <= 0 || dil <= 0 || pad < 0) return 0;
    const long long o = (static_cast<long long>(in) + 2LL * pad - static_cast<long long>(dil) * (k - 1) - 1) / stride + 1;
    return o > INT_MAX ? INT_MAX : static_cast<int>(o);
}
static bool conv_geom_ok(int kH, int kW, int padH, int padW, int strideH, int strideW, int dilH, int dilW) {
    return kH > 0 && kW > 0 && strideH > 0 && strideW > 0 && dilH > 0 && dilW > 0 && padH >= 0 && padW >= 0;
}

static int conv_nhwc(const int8_t* x, const int8_t* w, const float* act_scale, const uint16_t* w_scale,
                     const uint16_t* bias, uint16_t* out16, int32_t* out32, int N, int H, int W, int C,
                     int Co, int kH, int kW, int padH, int padW, int strideH, int strideW, int dilH,
                     int dilW, hipStream_t s)
{
    if (N <= 0 || C <= 0 || Co <= 0 || H <= 0 || W <= 0) return FORGE_OK;
    if (!x || !w || (!out16 && !out32) || !conv_geom_ok(kH, kW, padH, padW, strideH, strideW, dilH, dilW))
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

// ---- NCHW FP16 conv in one launch (implicit GEMM with per-patch-row quantization) ------
//
// The reference's int8_conv2d_forward (src/nn/int8_conv2d.cu:151-223) runs, per image, an FP16
// im2col into the workspace, the per-row quantize of that patch matrix, the dequantizing GEMM
// and a transpose to NCHW: 4 launches and ~3 passes over a K-times-inflated buffer per image.
// conv_nchw_fused_kernel does all of it in one pass for every image of the call: a workgroup
// owns a tile of up to 64 output pixels (R output rows x Wt columns of one image) and all
// output channels.
//   1. It loads the input window of the tile -- C x IH x IW FP16 values, zero outside the
//      image -- into LDS once (coalesced along W).
//   2. Per pixel, the absmax over its patch (C x kH x kW taps, the reference's im2col row,
//      padding included as zeros) is a max over LDS (fmaxf, which skips NaN as the reference
//      quantizer's reduction does), giving scale = max(absmax, 1e-8) / 127 and 1 / scale.
//   3. The patch rows are quantized into an INT8 A tile in LDS (64 rows x Kp bytes, K in the
//      reference's c*kH*kW + kh*kW + kw order, zero from K to Kp; row pitch Kp + 16 bytes so
//      the 16 rows of a ds_read_b128 phase fall on distinct banks).
//   4. v_mfma_i32_32x32x32_i8 items (32 output channels x 32 pixels) go round-robin to the 4
//      waves; weight fragments (the reference's (C_out, K) rows, K % 16 == 0) come from L2.
//   5. The accumulators are dequantized as the reference's GEMM epilogue does
//      (fma((float)acc, act_scale * w_scale, bias), one FP16 rounding) and stored straight to
//      NCHW: 32 adjacent pixels of one channel per store instruction.
// Every output equals the reference pipeline's on the same input: the INT8 rows and scales are
// those of quantize_rows on the im2col rows, the INT32 sums are exact, the epilogue identical.
struct ConvNchwArgs {
    const uint16_t* x;
    const int8_t* w;
    const uint16_t* w_scale;
    const uint16_t* bias;
    uint16_t* y;
    int C, H, W, Co, kH, kW, padH, padW, sH, sW, dH, dW, Ho, Wo;
    int K, Kp, pitch;          // patch length, padded to 32, A row pitch (bytes)
    int R, Wt, IH, IW;         // tile rows / columns, input window rows / columns
    int P, G;                  // window row pitch (values); 8-value groups per row (vector loads)
    int tiles_h, tiles_w, tiles, N;
    int xin_bytes;             // LDS bytes of the input window (16-byte multiple)
    int Cop;                   // Co rounded up to 32 (w_scale / bias strips in LDS)
    int rpi, ninst, step_c, step_ih;   // vector loads: rows per instruction, instructions, 4 rpi rows as (c, ih)
    uint32_t mg_khw, mg_kw, mg_ih, mg_wt, mg_g;   // udiv_magic multipliers
    uint32_t x_bytes, y_bytes; // bytes of one image of x / of y (buffer-resource ranges)
};

constexpr int kCnPix = 64;     // output pixels per workgroup tile

// A persistent workgroup runs tiles start, start + stride, ... of its XCD's contiguous range
// (xcd_contiguous's split of the tiles over the 8 XCDs), so the workgroups of one XCD work on
// neighbouring tiles together and share their window halos in that XCD's L2.
struct ConvTileWalk {
    int next, end, stride;
};
__device__ __forceinline__ ConvTileWalk conv_tile_walk(int total)
{
    constexpr int kXcd = 8;
    const int b = blockIdx.x, grid = gridDim.x;
    const int x = b % kXcd, j = b / kXcd;
    const int q = total / kXcd, r = total % kXcd;
    const int gq = grid / kXcd, gr = grid % kXcd;
    const int start = x * q + min(x, r);
    return {start + j, start + q + (x < r ? 1 : 0), gq + (x < gr ? 1 : 0)};
}

// VEC (W % 8 == 0, 16-byte-aligned input): window rows start at the 8-aligned column at or
// before the window's first one (shift s0 = 0..7) and load as 16-byte buffer loads, several rows
// per instruction, whose out-of-image groups read as zeros (offsets past the buffer's range);
// with PF the next tile's loads are in flight while the current tile computes (a.ninst <=
// 4 kPF). Otherwise 2-byte loads, one row per instruction and lane.
constexpr int kPF = 4;   // prefetched 16-byte loads per lane (4 workgroups per CU keep 128 VGPRs)
template <bool VEC, bool PF>
__global__ __launch_bounds__(256, 4) void conv_nchw_fused_kernel(ConvNchwArgs a)
{
    extern __shared__ __align__(16) int8_t lds[];
    uint16_t* xin = reinterpret_cast<uint16_t*>(lds);
    int8_t* At = lds + a.xin_bytes;
    float* s_scale = reinterpret_cast<float*>(At + kCnPix * a.pitch);
    float* s_inv = s_scale + kCnPix;
    float* s_m1 = s_inv + kCnPix;                         // per window position: channel absmax
    int* koff = reinterpret_cast<int*>(s_m1 + ((a.IH * a.P + 3) & ~3));   // per k: window offset of tap k
    float* s_ws = reinterpret_cast<float*>(koff + a.K);   // Cop entries each, zero past Co
    float* s_b = s_ws + a.Cop;

    const int t = threadIdx.x, lane = t & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int l31 = lane & 31, hi = lane >> 5;
    const int P = a.P;
    const int HW = a.H * a.W;
    const int IHP = a.IH * P;
    const int ksteps = a.Kp >> 5;
    const int items = ((a.Co + 31) >> 5) * 2;
    const int rows = a.C * a.IH;
    const int npix = a.R * a.Wt;
    const uint32_t plane2 = 2u * static_cast<uint32_t>(a.Ho * a.Wo);
    const bool has_bias = a.bias != nullptr;

    // weight fragments: kG in flight per wave
    constexpr int kG = 4;
    v4i fw[kG];
    auto load_w = [&](int it, int ks0) {
        const int co_l = min((it >> 1) * 32 + l31, a.Co - 1);
        const int8_t* wr = a.w + static_cast<size_t>(co_l) * a.K;
#pragma unroll
        for (int g = 0; g < kG; g++) {
            const int kk = 32 * (ks0 + g) + 16 * hi;
            fw[g] = *reinterpret_cast<const v4i*>(wr + (ks0 + g < ksteps && kk < a.K ? kk : 0));
        }
    };

    // 0. tap offsets into the window (k = c kH kW + kh kW + kw, the reference's im2col order)
    //    and the w_scale / bias strips as floats, once per workgroup
    for (int k = t; k < a.K; k += 256) {
        const int c = udiv_magic(k, a.mg_khw), r = k - c * (a.kH * a.kW);
        const int kh = udiv_magic(r, a.mg_kw), kw = r - kh * a.kW;
        koff[k] = c * IHP + kh * a.dH * P + kw * a.dW;
    }
    for (int c = t; c < a.Cop; c += 256) {
        s_ws[c] = c < a.Co ? h2f(a.w_scale[c]) : 0.0f;
        s_b[c] = c < a.Co && a.bias ? h2f(a.bias[c]) : 0.0f;
    }

    // Tile geometry
    struct Geo {
        int n, ho0, wo0, hb, a0, s0;
    };
    auto geo_of = [&](int tile) {
        Geo g;
        g.n = tile / a.tiles;
        const int rem = tile - g.n * a.tiles;
        const int th = rem / a.tiles_w, tw = rem - th * a.tiles_w;
        g.ho0 = th * a.R;
        g.wo0 = tw * a.Wt;
        g.hb = g.ho0 * a.sH - a.padH;
        const int wb = g.wo0 * a.sW - a.padW;
        g.a0 = VEC ? (wb & ~7) : wb;                     // global column of window value 0
        g.s0 = wb - g.a0;                                // window column iw sits at iw + s0
        return g;
    };

    // 1. input window (C x IH rows, zero outside the image), VEC form: lane l of an instruction
    //    takes 8-value group l % G of window row slot l / G; the wave's instructions i = wave,
    //    wave + 4, ... cover rows [i rpi, i rpi + rpi), stepping (c, ih) by 4 rpi rows. W % 8 == 0,
    //    so a group lies wholly inside the image or wholly outside it. The window holds
    //    ninst * rpi rows (rows past C IH are zeros and never read).
    const int slot = VEC ? udiv_magic(lane, a.mg_g) : 0, grp = lane - slot * a.G;
    const bool lok = VEC && slot < a.rpi;
    const int r_first = wave * a.rpi + slot;
    const int c_first = VEC ? udiv_magic(r_first, a.mg_ih) : 0, ih_first = r_first - c_first * a.IH;
    const int dgoff = a.step_c * HW + a.step_ih * a.W, wrap = HW - a.IH * a.W;
    // issues the loads of instructions i0, i0 + 4, ... (kIB of them) of tile g into v
    auto issue_vec = [&](const Geo& g, int& r, int& ih, int& goff, v4i* v, int kIB) {
        const __amdgpu_buffer_rsrc_t rx = buf_rsrc(a.x + static_cast<size_t>(g.n) * a.C * HW, a.x_bytes);
        const int col = g.a0 + 8 * grp;
        const bool cok = col >= 0 && col < a.W;
        for (int q = 0; q < kIB; q++) {
            const bool ok = cok && r < rows && static_cast<unsigned>(g.hb + ih) < static_cast<unsigned>(a.H);
            v[q] = __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? 2u * static_cast<uint32_t>(goff + col) : 0x80000000u,
                                                         0, 0);
            r += 4 * a.rpi;
            ih += a.step_ih;
            goff += dgoff;
            if (ih >= a.IH) {
                ih -= a.IH;
                goff += wrap;
            }
        }
    };
    auto goff_first = [&](const Geo& g) { return c_first * HW + (g.hb + ih_first) * a.W; };

    v4i pf[PF ? kPF : 1];
    auto prefetch = [&](const Geo& g) {
        int r = r_first, ih = ih_first, goff = goff_first(g);
#pragma unroll
        for (int q = 0; q < (PF ? kPF : 1); q++) {
            if (PF && wave + 4 * q < a.ninst) issue_vec(g, r, ih, goff, &pf[q], 1);
        }
    };
    auto store_prefetched = [&]() {
        if (lok) {
#pragma unroll
            for (int q = 0; q < (PF ? kPF : 1); q++)
                if (PF && wave + 4 * q < a.ninst)
                    *reinterpret_cast<v4i*>(xin + (r_first + 4 * q * a.rpi) * P + 8 * grp) = pf[q];
        }
    };
    auto load_window_sync = [&](const Geo& g) {
        if constexpr (VEC) {
            int r = r_first, ih = ih_first, goff = goff_first(g);
            constexpr int kIB = 4;
            for (int i0 = wave; i0 < a.ninst; i0 += 4 * kIB) {
                v4i v[kIB];
                const int rb = r;
#pragma unroll
                for (int q = 0; q < kIB; q++) issue_vec(g, r, ih, goff, &v[q], 1);
                if (lok) {
#pragma unroll
                    for (int q = 0; q < kIB; q++)
                        if (i0 + 4 * q < a.ninst) *reinterpret_cast<v4i*>(xin + (rb + 4 * q * a.rpi) * P + 8 * grp) = v[q];
                }
            }
        } else {
            // Row (c, ih) of wave c % 4; up to kRB rows per batch, loads issued together.
            const uint16_t* xn = a.x + static_cast<size_t>(g.n) * a.C * HW;
            const int nu = a.IW > kWave ? 2 : 1;   // the plan keeps IW <= 128 here
            bool cok[2];
            int wi[2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int iw = lane + kWave * u;
                wi[u] = g.a0 + iw;
                cok[u] = u < nu && iw < a.IW && wi[u] >= 0 && wi[u] < a.W;
            }
            const int nrw = ((a.C - wave + 3) / 4) * a.IH;   // rows of this wave
            constexpr int kRB = 16;
            int cc0 = 0, ih0 = 0;
            for (int i0 = 0; i0 < nrw; i0 += kRB) {
                uint16_t v[kRB][2];
                int cc = cc0, ih = ih0;
#pragma unroll
                for (int q = 0; q < kRB; q++) {
                    const int c = wave + 4 * cc;
                    const int h_ = g.hb + ih;
                    const bool rok = i0 + q < nrw && h_ >= 0 && h_ < a.H;
                    const uint16_t* xr = xn + static_cast<size_t>(c) * HW + static_cast<size_t>(h_) * a.W;
#pragma unroll
                    for (int u = 0; u < 2; u++) v[q][u] = (rok && cok[u]) ? xr[wi[u]] : static_cast<uint16_t>(0);
                    if (++ih == a.IH) {
                        ih = 0;
                        cc++;
                    }
                }
                cc = cc0;
                ih = ih0;
#pragma unroll
                for (int q = 0; q < kRB; q++) {
                    uint16_t* dst = xin + ((wave + 4 * cc) * a.IH + ih) * P;
#pragma unroll
                    for (int u = 0; u < 2; u++)
                        if (i0 + q < nrw && u < nu && lane + kWave * u < a.IW) dst[lane + kWave * u] = v[q][u];
                    if (++ih == a.IH) {
                        ih = 0;
                        cc++;
                    }
                }
                cc0 = cc;
                ih0 = ih;
            }
        }
    };

    ConvTileWalk walk = conv_tile_walk(a.tiles * a.N);
    if (walk.next >= walk.end) return;
    Geo cur = geo_of(walk.next);
    if constexpr (PF) prefetch(cur);

    while (true) {
        // the window of the current tile into LDS (the previous tile's readers of xin and At
        // are past the barrier at the end of the loop)
        if constexpr (PF) store_prefetched();
        else load_window_sync(cur);
        if (wave < items) load_w(wave, 0);   // the first item's first weight fragments
        const int nxt = walk.next + walk.stride;
        const bool has_next = nxt < walk.end;
        Geo ng = cur;
        if (has_next) ng = geo_of(nxt);
        __syncthreads();
        if constexpr (PF) {
            if (has_next) prefetch(ng);   // in flight while this tile computes
        }

        // 2. per window position the absmax over the channels on fp16 magnitude bit patterns
        //    (they order as the magnitudes; a pattern above 0x7C00 is a NaN, and such a position
        //    takes the fp32 maximum, which skips NaN as the reference quantizer's reduction does),
        //    then per pixel the max over its kH x kW positions: the absmax of its im2col row
        //    (padding taps are zeros). s_m1 has the window's layout (IH rows of pitch P).
        if constexpr (VEC) {
            // two adjacent positions per thread, as packed u16 maxima of 4-byte reads
            const int npairs = a.IH * (P >> 1);
            const uint32_t* x32 = reinterpret_cast<const uint32_t*>(xin);
            for (int j = t; j < npairs; j += 256) {
                const uint32_t* xp = x32 + j;
                uint32_t mb = 0u;
                int c = 0;
                for (; c + 8 <= a.C; c += 8) {
                    uint32_t h[8];
#pragma unroll
                    for (int u = 0; u < 8; u++) h[u] = xp[(c + u) * npairs];
#pragma unroll
                    for (int u = 0; u < 8; u++) mb = pk_max_u16(mb, h[u] & 0x7FFF7FFFu);
                }
                for (; c < a.C; c++) mb = pk_max_u16(mb, xp[c * npairs] & 0x7FFF7FFFu);
                float m[2];
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const uint32_t b = (mb >> (16 * u)) & 0xFFFFu;
                    m[u] = h2f(static_cast<uint16_t>(b));
                    if (b > kHalfInfBits) {
                        m[u] = 0.0f;
                        for (int c2 = 0; c2 < a.C; c2++) m[u] = fmaxf(m[u], fabsf(h2f(xin[2 * j + u + c2 * IHP])));
                    }
                }
                *reinterpret_cast<float2*>(s_m1 + 2 * j) = make_float2(m[0], m[1]);
            }
        } else {
            const int IHW = a.IH * a.IW;
            for (int pos = t; pos < IHW; pos += 256) {
                const int ih = pos / a.IW, iw = pos - ih * a.IW;
                const uint16_t* xp = xin + ih * P + iw;
                uint32_t mb = 0u;
                int c = 0;
                for (; c + 8 <= a.C; c += 8) {
                    uint32_t h[8];
#pragma unroll
                    for (int u = 0; u < 8; u++) h[u] = xp[(c + u) * IHP];
#pragma unroll
                    for (int u = 0; u < 8; u++) mb = max(mb, h[u] & 0x7FFFu);
                }
                for (; c < a.C; c++) mb = max(mb, static_cast<uint32_t>(xp[c * IHP]) & 0x7FFFu);
                float m = h2f(static_cast<uint16_t>(mb));
                if (mb > kHalfInfBits) {
                    m = 0.0f;
                    for (int c2 = 0; c2 < a.C; c2++) m = fmaxf(m, fabsf(h2f(xp[c2 * IHP])));
                }
                s_m1[ih * P + iw] = m;
            }
        }
        __syncthreads();
        if (t < kCnPix) {
            const int p = t < npix ? t : npix - 1;
            const int pr = udiv_magic(p, a.mg_wt), pc = p - pr * a.Wt;
            float m = 0.0f;
            for (int kh = 0; kh < a.kH; kh++)
                for (int kw = 0; kw < a.kW; kw++)
                    m = fmaxf(m, s_m1[(pr * a.sH + kh * a.dH) * P + pc * a.sW + kw * a.dW + cur.s0]);
            const float scale = row_scale(m);
            s_scale[t] = scale;
            s_inv[t] = 1.0f / scale;
        }
        __syncthreads();

        // 3. quantized A tile: lane = pixel, a wave takes 16-byte chunks ch = wave, wave + 4, ...;
        //    a chunk's 16 tap offsets are uniform LDS reads, its 16 window reads issue together
        //    (adjacent pixels read adjacent window values). K % 16 == 0, so a chunk is all taps or
        //    all padding (zeros).
        {
            const int p = lane < npix ? lane : npix - 1;
            const int pr = udiv_magic(p, a.mg_wt), pc = p - pr * a.Wt;
            const int base = pr * a.sH * P + pc * a.sW + cur.s0;
            const float inv = s_inv[lane];
            const int nch = a.Kp >> 4, nkc = a.K >> 4;
            for (int ch = wave; ch < nch; ch += 4) {
                uint4 qv = make_uint4(0u, 0u, 0u, 0u);
                if (ch < nkc) {
                    const int k0 = ch * 16;
                    int o[16];
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const int4 v = *reinterpret_cast<const int4*>(koff + k0 + 4 * q);
                        o[4 * q] = v.x;
                        o[4 * q + 1] = v.y;
                        o[4 * q + 2] = v.z;
                        o[4 * q + 3] = v.w;
                    }
                    uint32_t h[16];
#pragma unroll
                    for (int j = 0; j < 16; j++) h[j] = xin[base + o[j]];
                    float pr[16];
#pragma unroll
                    for (int j = 0; j < 16; j++) pr[j] = fma_mix_lo(h[j], inv);
                    qv = pack16_rint_sdwa(pr);
                }
                *reinterpret_cast<uint4*>(At + lane * a.pitch + 16 * ch) = qv;
            }
        }
        __syncthreads();

        // 4./5. MFMA items (32 channels x 32 pixels) and the NCHW epilogue: 2-byte buffer stores at
        //    32-bit offsets within image n's output, whose channels past Co and pixels outside the
        //    tile carry offsets past the range (dropped)
        const __amdgpu_buffer_rsrc_t ry =
            buf_rsrc(a.y + static_cast<size_t>(cur.n) * a.Co * (plane2 >> 1), a.y_bytes);
        for (int it = wave; it < items; it += 4) {
            const int cb = it >> 1, pb = it & 1;
            const int8_t* ar = At + (pb * 32 + l31) * a.pitch;
            v16i acc;
#pragma unroll
            for (int e = 0; e < 16; e++) acc[e] = 0;
            for (int ks0 = 0; ks0 < ksteps; ks0 += kG) {
                if (ks0 > 0) load_w(it, ks0);
#pragma unroll
                for (int g = 0; g < kG; g++) {
                    if (ks0 + g < ksteps) {
                        const v4i fa = *reinterpret_cast<const v4i*>(ar + 16 * (2 * (ks0 + g) + hi));
                        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(fw[g], fa, acc, 0, 0, 0);
                    }
                }
            }
            if (it + 4 < items) load_w(it + 4, 0);   // the next item's first fragments
            const int p = pb * 32 + l31;
            const int pr = udiv_magic(p, a.mg_wt), pc = p - pr * a.Wt;
            const int ho = cur.ho0 + pr, wo = cur.wo0 + pc;
            const bool pok = p < npix && ho < a.Ho && wo < a.Wo;
            const int co0 = cb * 32 + 4 * hi;
            const uint32_t vo = pok ? 2u * static_cast<uint32_t>(ho * a.Wo + wo) + static_cast<uint32_t>(co0) * plane2
                                    : 0x80000000u;
            const float as = s_scale[p < npix ? p : 0];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const float4 ws4 = *reinterpret_cast<const float4*>(s_ws + co0 + 8 * g);
                const float4 b4 = *reinterpret_cast<const float4*>(s_b + co0 + 8 * g);
                const float wsv[4] = {ws4.x, ws4.y, ws4.z, ws4.w}, bv[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint16_t yv = dequant_gemm(acc[4 * g + e], as, wsv[e], bv[e], has_bias);
                    __builtin_amdgcn_raw_buffer_store_b16(yv, ry, vo + static_cast<uint32_t>(8 * g + e) * plane2, 0, 0);
                }
            }
        }
        if (!has_next) break;
        walk.next = nxt;
        cur = ng;
        __syncthreads();   // xin, s_m1, s_scale and At are free for the next tile
    }
}

// Workgroups of fn with lds bytes resident per CU (the persistent grid is CUs times this), or
// minus a HIP error. Sets the 160 KB dynamic-LDS limit on first use of each kernel.
static int conv_nchw_fused_residency(const void* fn, size_t lds)
{
    static std::once_flag once[3];
    static hipError_t attr[3];
    static const void* fns[3] = {reinterpret_cast<const void*>(&conv_nchw_fused_kernel<true, true>),
                                 reinterpret_cast<const void*>(&conv_nchw_fused_kernel<true, false>),
                                 reinterpret_cast<const void*>(&conv_nchw_fused_kernel<false, false>)};
    int i = 0;
    while (i < 3 && fns[i] != fn) i++;
    if (i == 3) return -static_cast<int>(hipErrorInvalidDeviceFunction);
    std::call_once(once[i], [&] {
        attr[i] = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    });
    if (attr[i] != hipSuccess) return -static_cast<int>(attr[i]);
    int blocks = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, 256, lds);
    if (e != hipSuccess) return -static_cast<int>(e);
    return blocks > 0 ? blocks : 1;
}

// Geometry of the one-launch path, or false when it does not apply (the per-image pipeline
// runs instead): K % 16 == 0 with 16-byte-aligned weights (weight fragments are 16-byte
// loads), the input window and A tile within LDS, the weights small enough to re-read per tile.
static bool conv_nchw_fused_plan(ConvNchwArgs& a, int N, size_t* lds_bytes, bool* vec)
{
    if (a.K % 16 != 0 || !aligned(a.w, 16)) return false;
    a.Kp = (a.K + 31) & ~31;
    if (a.Kp > 2048 || static_cast<long long>(a.Co) * a.Kp > (128 << 10) || a.Co > 4096) return false;
    // buffer-resource offsets of one image stay 32-bit: valid ones below 2^30, and an invalid
    // 0x80000000 plus a channel offset (channels up to Co rounded to 32) below 2^32
    a.Cop = (a.Co + 31) & ~31;
    const long long xb = 2LL * a.C * a.H * a.W, yb = 2LL * a.Co * a.Ho * a.Wo;
    if (xb >= (1LL << 30) || 2LL * a.Cop * a.Ho * a.Wo >= (1LL << 31)) return false;
    a.x_bytes = static_cast<uint32_t>(xb);
    a.y_bytes = static_cast<uint32_t>(yb);
    *vec = a.W % 8 == 0 && aligned(a.x, 16);
    a.pitch = a.Kp + 16;
    a.Wt = a.Wo < kCnPix ? a.Wo : kCnPix;
    a.R = kCnPix / a.Wt;
    if (a.R > a.Ho) a.R = a.Ho;
    a.IH = (a.R - 1) * a.sH + (a.kH - 1) * a.dH + 1;
    a.IW = (a.Wt - 1) * a.sW + (a.kW - 1) * a.dW + 1;
    long long xrows = static_cast<long long>(a.C) * a.IH;
    if (*vec) {
        // a window row spans the 8-aligned groups from the one holding its first value
        a.G = (a.IW + 7 + 7) / 8;
        if (a.G > kWave) return false;
        a.P = 8 * a.G;
        a.rpi = kWave / a.G;
        a.ninst = static_cast<int>((xrows + a.rpi - 1) / a.rpi);
        xrows = static_cast<long long>(a.ninst) * a.rpi;
        a.step_c = 4 * a.rpi / a.IH;
        a.step_ih = 4 * a.rpi - a.step_c * a.IH;
        a.mg_g = udiv_multiplier(a.G);
        a.mg_ih = udiv_multiplier(a.IH);
        if (xrows * a.IH >= (1LL << 32)) return false;   // udiv_magic range (row / IH)
    } else {
        if (a.IW > 2 * kWave) return false;
        a.G = a.rpi = a.ninst = a.step_c = a.step_ih = 0;
        a.mg_g = a.mg_ih = 0;
        a.P = a.IW;
    }
    a.mg_khw = udiv_multiplier(a.kH * a.kW);
    a.mg_kw = udiv_multiplier(a.kW);
    a.mg_wt = udiv_multiplier(a.Wt);
    const long long xin = (2LL * xrows * a.P + 15) & ~15LL;
    const long long bytes = xin + static_cast<long long>(kCnPix) * a.pitch + 2 * kCnPix * 4 +
                            4LL * ((a.IH * a.P + 3) & ~3) + 4LL * a.K + 8LL * a.Cop;
    if (bytes > 160 * 1024) return false;
    a.xin_bytes = static_cast<int>(xin);
    a.tiles_h = divup(a.Ho, a.R);
    a.tiles_w = divup(a.Wo, a.Wt);
    const long long tiles = static_cast<long long>(a.tiles_h) * a.tiles_w;
    if (tiles * N > 0x7FFFFFFFLL) return false;
    a.tiles = static_cast<int>(tiles);
    a.N = N;
    *lds_bytes = static_cast<size_t>(bytes);
    return true;
}

// ---- NCHW FP16 conv on a channel-last window (one launch, 128-pixel tiles) --------------
//
// conv_nchw_cl_kernel gives the same bits as conv_nchw_fused_kernel (the reference pipeline's:
// per-patch-row quantize of the im2col rows, exact INT32 sums, the GEMM's dequant epilogue),
// with the work spread evenly over the four waves and fewer instructions per tap:
//   * The input window is kept channel-last in LDS ([window row][column][channel], channels
//     padded to Cp = 16k with zeros), so the 16 channels of one tap are 32 contiguous bytes:
//     two ds_read_b128 give a lane 16 taps, where the NCHW window needs 16 ds_read_u16 and
//     16 address adds. Window rows load as 16-byte buffer loads of 8 columns, 8 channels per
//     lane (zeros outside the image and past C), transposed in registers by v_perm.
//   * The GEMM's K order is free (the INT32 sums are exact in any order), so the patch row is
//     taken as k' = (kh kW + kw) Cp + c; each workgroup holds its weights permuted to that
//     order in LDS once (zero for padded channels and rows), where the reference's (C_out, K)
//     rows have k = c kH kW + kh kW + kw.
//   * Wave w owns pixels 32w .. 32w + 31 of the tile. Lane l quantizes taps 16 (2 ks + l / 32)
//     .. + 15 of pixel l % 32 for K step ks: exactly its B fragment of
//     v_mfma_i32_32x32x32_i8, which it feeds straight to the MFMA (no INT8 tile in LDS, no
//     barrier between quantize and MFMA), for every 32-channel block of C_out.
//   * The per-pixel scale is the max over the pixel's kH x kW window positions of each
//     position's channel absmax (fp16 magnitude bit patterns, as the one-launch NCHW kernel
//     takes them), which the lanes that write the window take over their 8 channels in
//     registers and merge per position with LDS atomic maxima (no pass of its own).
// A tile is R output rows x Wt columns (R Wt <= 128); workgroups are persistent and walk their
// XCD's contiguous range of tiles, with the next tile's window loads in flight during the
// current tile (when a wave has at most one load instruction per tile).
struct ConvClArgs {
    const uint16_t* x;
    const int8_t* w;
    const uint16_t* w_scale;
    const uint16_t* bias;
    uint16_t* y;
    int C, H, W, Co, kH, kW, padH, padW, sH, sW, dH, dW, Ho, Wo, K;
    int Cp, CQ, nch, ksteps;   // channels padded to 16, 16-channel chunks per tap, chunks, 32-deep K steps
    int R, Wt, npix, IH, IW;   // tile rows / columns / pixels; window rows / columns read
    int G, IWr, Pp;            // 8-column load groups per window row; LDS row pitch (positions); position bytes
    int rpi, nrows, ninst;     // load rows (8 channels of one window row) per instruction; rows; instructions
    int KWp;                   // row pitch of the permuted weights (bytes)
    int w_off, m1_off, koff_off, ws_off;   // LDS offsets (bytes)
    int tiles_h, tiles_w, tiles, N;
    int nw;                    // waves per workgroup (32 output pixels each)
    uint32_t mg_wt, mg_rpi, mg_ih, mg_iw;  // udiv_magic multipliers
    uint32_t mg_tiles, mg_tw;              // tile -> (image, tile row, tile column)
    uint32_t mg_c;                         // weight fill: (output, input channel) pair -> output channel
    int wpad;                              // the permuted weight block has padding
    uint32_t x_bytes, y_bytes;
};


// 16 fp16 taps (8 dwords, two per dword, lower address in the low half) -> 16 INT8 values:
// per tap one v_fma_mix_f32 (the rounded product) and one SDWA add (pack16_rint_sdwa).
__device__ __forceinline__ v4i quant16_cl(uint4 h0, uint4 h1, float inv) {
    const uint32_t w[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
    float p[16];
#pragma unroll
    for (int d = 0; d < 8; d++) {
        p[2 * d] = fma_mix_lo(w[d], inv);
        p[2 * d + 1] = fma_mix_hi(w[d], inv);
    }
    return __builtin_bit_cast(v4i, pack16_rint_sdwa(p));
}

template <int NCB, bool PF, int NW>
__global__ __launch_bounds__(64 * NW, (NCB == 1 ? 16 : NCB == 2 ? 12 : 8) / NW) void conv_nchw_cl_kernel(
    ConvClArgs a)
{
    constexpr int kThr = 64 * NW;
    extern __shared__ __align__(16) int8_t lds[];
    int8_t* win = lds;
    int8_t* wl = lds + a.w_off;
    // the tile's channel maxima (tagged), IH x IW entries
    uint32_t* s_m1u = reinterpret_cast<uint32_t*>(lds + a.m1_off);
    int* koff = reinterpret_cast<int*>(lds + a.koff_off);
    float* s_ws = reinterpret_cast<float*>(lds + a.ws_off);
    float* s_b = s_ws + 32 * NCB;
    constexpr int kCop = 32 * NCB;

    const int t = threadIdx.x, lane = t & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int l31 = lane & 31, hi = lane >> 5;
    const int HW = a.H * a.W;
    const int khw = a.kH * a.kW;
    const int m1n = a.IH * a.IW;
    const uint32_t plane2 = 2u * static_cast<uint32_t>(a.Ho * a.Wo);
    const bool has_bias = a.bias != nullptr;

    ConvTileWalk walk = conv_tile_walk(a.tiles * a.N);
    if (walk.next >= walk.end) return;

    struct Geo {
        int n, ho0, wo0, hb, a0, s0;
    };
    auto geo_of = [&](int tile) {
        Geo g;
        g.n = udiv_magic(tile, a.mg_tiles);
        const int rem = tile - g.n * a.tiles;
        const int th = udiv_magic(rem, a.mg_tw), tw = rem - th * a.tiles_w;
        g.ho0 = th * a.R;
        g.wo0 = tw * a.Wt;
        g.hb = g.ho0 * a.sH - a.padH;
        const int wb = g.wo0 * a.sW - a.padW;
        g.a0 = wb & ~7;                                  // 8-aligned global column of window position 0
        g.s0 = wb - g.a0;                                // the first column read sits at position s0
        return g;
    };

    // 1. window loads: lane l of an instruction takes load row i rpi + l % rpi, 8-column
    //    group l / rpi (lanes past rpi G idle); load row r holds channels 8 (r / IH) .. + 7 of
    //    window row r % IH. W % 8 == 0, so a group is wholly inside or outside the image;
    //    offsets past the buffer's range read as zeros (outside the image, channels past C).
    //    The row runs fastest over the lanes for the LDS writes: a lane writes 8 positions of
    //    its group, and lanes of different groups (8 positions apart) would hit the same banks,
    //    while different rows (channel groups, window rows of odd pitch) spread over them.
    const int grp = udiv_magic(lane, a.mg_rpi), slot = lane - grp * a.rpi;
    const bool lok = grp < a.G;
    auto issue_rows = [&](const Geo& g, int i, v4i* v) {
        const __amdgpu_buffer_rsrc_t rx = buf_rsrc(a.x + static_cast<size_t>(g.n) * a.C * HW, a.x_bytes);
        const int r = i * a.rpi + slot;
        const int cg = udiv_magic(r, a.mg_ih), ih = r - cg * a.IH;
        const int col = g.a0 + 8 * grp, h = g.hb + ih;
        // (bitwise &, not &&: selects rather than branches)
        const bool ok = lok & (r < a.nrows) & (col >= 0) & (col < a.W) &
                        (static_cast<unsigned>(h) < static_cast<unsigned>(a.H));
        const int cleft = a.C - 8 * cg;   // channels of this load row inside the image
        const uint32_t base = 2u * static_cast<uint32_t>(8 * cg * HW + h * a.W + col);
#pragma unroll
        for (int u = 0; u < 8; u++)
            v[u] = __builtin_amdgcn_raw_buffer_load_b128(
                rx, (ok & (u < cleft)) ? base + static_cast<uint32_t>(2 * u * HW) : 0x80000000u, 0, 0);
    };
    // the 8 x 8 block transposed by v_perm into 8 positions of 8 channels (16 bytes each); and
    // per position read by the tile (columns s0 .. s0 + IW - 1) the maximum of the 8 channels'
    // fp16 magnitude bit patterns, merged into the tile's channel maxima by LDS atomic maxima
    // of (tag << 15 | bits): a tile's tag exceeds every earlier tile's, so its first merge
    // replaces an entry left by an earlier tile (no zeroing between tiles)
    auto write_rows = [&](int i, const v4i* v, int s0, uint32_t tag) {
        const int r = i * a.rpi + slot;
        if (!lok || r >= a.nrows) return;
        const int cg = udiv_magic(r, a.mg_ih), ih = r - cg * a.IH;
        int8_t* dst = win + (ih * a.IWr + 8 * grp) * a.Pp + 16 * cg;
#pragma unroll
        for (int jj = 0; jj < 8; jj++) {
            const int d = jj >> 1;
            const uint32_t sel = (jj & 1) ? 0x07060302u : 0x05040100u;
            uint4 o;
            o.x = __builtin_amdgcn_perm(static_cast<uint32_t>(v[1][d]), static_cast<uint32_t>(v[0][d]), sel);
            o.y = __builtin_amdgcn_perm(static_cast<uint32_t>(v[3][d]), static_cast<uint32_t>(v[2][d]), sel);
            o.z = __builtin_amdgcn_perm(static_cast<uint32_t>(v[5][d]), static_cast<uint32_t>(v[4][d]), sel);
            o.w = __builtin_amdgcn_perm(static_cast<uint32_t>(v[7][d]), static_cast<uint32_t>(v[6][d]), sel);
            *reinterpret_cast<uint4*>(dst + jj * a.Pp) = o;
        }
        if constexpr (!PF) return;   // without prefetch a pass of its own takes the maxima
        const int iw0 = 8 * grp - s0;   // window column of this group's first position
        uint32_t* mrow = s_m1u + ih * a.IW + iw0;
        const uint32_t tg = tag << 15;
#pragma unroll
        for (int d = 0; d < 4; d++) {
            uint32_t cm = static_cast<uint32_t>(v[0][d]) & 0x7FFF7FFFu;
#pragma unroll
            for (int u = 1; u < 8; u++) cm = pk_max_u16(cm, static_cast<uint32_t>(v[u][d]) & 0x7FFF7FFFu);
            if (static_cast<unsigned>(iw0 + 2 * d) < static_cast<unsigned>(a.IW))
                __hip_atomic_fetch_max(mrow + 2 * d, tg | (cm & 0xFFFFu), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            if (static_cast<unsigned>(iw0 + 2 * d + 1) < static_cast<unsigned>(a.IW))
                __hip_atomic_fetch_max(mrow + 2 * d + 1, tg | (cm >> 16), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    };

    Geo cur = geo_of(walk.next);
    v4i pf[PF ? 8 : 1];
    if constexpr (PF) {
        if (wave < a.ninst) issue_rows(cur, wave, pf);   // in flight during the set-up
    }

    // 0. once per workgroup, while the first tile's window loads are in flight: the weights
    //    in the k' order; the window offset of each 16-channel chunk (chunks past the patch
    //    point at offset 0: their weights are zero); w_scale / bias.
    //    The weights: zeros first where the permuted block has padding (channels past C, rows
    //    past C_out, the half step past the last chunk), then per (output, input channel) pair
    //    of the reference's rows its kH kW contiguous bytes (k = c kH kW + tap) scattered to
    //    k' = tap Cp + c (taps past kH kW re-read the pair's last byte and store nothing).
    {
        if (a.wpad) {
            for (int i = t; i < (kCop * a.KWp) >> 4; i += kThr)
                *reinterpret_cast<uint4*>(wl + 16 * i) = make_uint4(0u, 0u, 0u, 0u);
            __syncthreads();
        }
        // up to 9 taps: the reads of 4 pairs in flight together; more taps: per pair, 9 at a time
        constexpr int kTapB = 9, kPairB = 4;
        {
            const int8_t* wsrc = a.w;
            const int np = a.Co * a.C;
            if (khw <= kTapB) {
                for (int p0 = t; p0 < np; p0 += kPairB * kThr) {
                    int8_t v[kPairB][kTapB];
                    int dofs[kPairB];
#pragma unroll
                    for (int q = 0; q < kPairB; q++) {
                        const int pi = min(p0 + kThr * q, np - 1);
                        const int co = udiv_magic(pi, a.mg_c), c = pi - co * a.C;
                        const int8_t* src = wsrc + static_cast<size_t>(co) * a.K + c * khw;
                        dofs[q] = co * a.KWp + c;
#pragma unroll
                        for (int u = 0; u < kTapB; u++) v[q][u] = src[min(u, khw - 1)];
                    }
#pragma unroll
                    for (int q = 0; q < kPairB; q++) {
                        if (p0 + kThr * q >= np) break;
#pragma unroll
                        for (int u = 0; u < kTapB; u++)
                            if (u < khw) wl[dofs[q] + u * a.Cp] = v[q][u];
                    }
                }
            } else {
                for (int pi = t; pi < np; pi += kThr) {
                    const int co = udiv_magic(pi, a.mg_c), c = pi - co * a.C;
                    const int8_t* src = wsrc + static_cast<size_t>(co) * a.K + c * khw;
                    int8_t* dst = wl + co * a.KWp + c;
                    for (int tp0 = 0; tp0 < khw; tp0 += kTapB) {
                        int8_t v[kTapB];
#pragma unroll
                        for (int u = 0; u < kTapB; u++) v[u] = src[min(tp0 + u, khw - 1)];
#pragma unroll
                        for (int u = 0; u < kTapB; u++)
                            if (tp0 + u < khw) dst[(tp0 + u) * a.Cp] = v[u];
                    }
                }
            }
        }
        for (int j = t; j < 2 * a.ksteps + 4; j += kThr) {
            int off = 0;
            if (j < a.nch) {
                const int tap = j / a.CQ, cc = j - tap * a.CQ;
                const int kh = tap / a.kW, kw = tap - kh * a.kW;
                off = (kh * a.dH * a.IWr + kw * a.dW) * a.Pp + 32 * cc;
            }
            koff[j] = off;
        }
        // Without a bias the strip holds -0: fma(acc, s, -0) is acc * s rounded once, zeros'
        // signs included, i.e. the reference epilogue's product.
        for (int c = t; c < kCop; c += kThr) {
            s_ws[c] = c < a.Co ? h2f(a.w_scale[c]) : 0.0f;
            s_b[c] = c < a.Co && has_bias ? h2f(a.bias[c]) : -0.0f;
        }
        for (int i = t; i < m1n; i += kThr) s_m1u[i] = 0u;
        __syncthreads();   // zeroed (tag 0) before the first tile's atomics
    }

    constexpr uint32_t kTagMax = 0x1FFFFu;   // 17 tag bits above the 15 magnitude bits
    uint32_t tag = 1;
    while (true) {
        // the current tile's window into LDS and its channel maxima (the previous tile's readers
        // are past the barrier at the end of the loop); after kTagMax tiles the maxima start
        // over from zero
        if (tag > kTagMax) {
            for (int i = t; i < m1n; i += kThr) s_m1u[i] = 0u;
            __syncthreads();
            tag = 1;
        }
        if constexpr (PF) {
            if (wave < a.ninst) write_rows(wave, pf, cur.s0, tag);
        } else {
            for (int i = wave; i < a.ninst; i += NW) {
                v4i v[8];
                issue_rows(cur, i, v);
                write_rows(i, v, cur.s0, tag);
            }
        }
        const int nxt = walk.next + walk.stride;
        const bool has_next = nxt < walk.end;
        __syncthreads();
        if constexpr (PF) {
            if (has_next && wave < a.ninst) issue_rows(geo_of(nxt), wave, pf);   // in flight while this tile computes
        } else {
            // the channel maxima by a pass over the window positions, spread over all threads
            // (the loading lanes hold more than one load instruction's data here)
            for (int q = t; q < m1n; q += kThr) {
                const int ih = udiv_magic(q, a.mg_iw), iw = q - ih * a.IW;
                const int8_t* src = win + (ih * a.IWr + cur.s0 + iw) * a.Pp;
                uint32_t mb = 0u;
                for (int c8 = 0; c8 < a.Cp; c8 += 16) {   // Cp % 16 == 0: two 16-byte reads in flight
                    const uint4 v0 = *reinterpret_cast<const uint4*>(src + 2 * c8);
                    const uint4 v1 = *reinterpret_cast<const uint4*>(src + 2 * c8 + 16);
                    mb = absbits8(v1, absbits8(v0, mb));
                }
                s_m1u[q] = (tag << 15) | max(mb & 0xFFFFu, mb >> 16);
            }
            __syncthreads();
        }

        // 3./4./5. per wave: 32 pixels' scales, the quantized B fragments fed to the MFMAs,
        //    the dequant epilogue stored to NCHW (2-byte buffer stores; pixels outside the
        //    image and channels past C_out carry offsets past the range and are dropped)
        if (32 * wave < a.npix) {
            const int p0 = 32 * wave + l31;
            const int p = p0 < a.npix ? p0 : a.npix - 1;
            const int pr = udiv_magic(p, a.mg_wt), pc = p - pr * a.Wt;
            // the pixel's kH x kW window positions (tagged channel maxima, fp16 magnitude bit
            // patterns), three reads in flight; a read past the last tap takes tap (0, 0) again,
            // which leaves the maximum as it is. A maximum above 0x7C00 is a NaN: the pixel then
            // takes the fp32 maximum over its taps, which skips NaN as the reference quantizer's
            // reduction does.
            const uint32_t* mr = s_m1u + pr * a.sH * a.IW + pc * a.sW;
            uint32_t mu = 0u;
            int kh = 0, kw = 0;
            for (int tp = 0; tp < khw; tp += 3) {
                uint32_t v[3];
#pragma unroll
                for (int u = 0; u < 3; u++) {
                    const int off = tp + u < khw ? kh * a.dH * a.IW + kw * a.dW : 0;
                    v[u] = mr[off];
                    if (++kw == a.kW) {
                        kw = 0;
                        kh++;
                    }
                }
                mu = max(mu, max(v[0], max(v[1], v[2])));
            }
            mu &= 0x7FFFu;   // the tag (the same for all of this tile's entries) off
            float m = h2f(static_cast<uint16_t>(mu));
            if (mu > kHalfInfBits) {
                m = 0.0f;
                for (int kh2 = 0; kh2 < a.kH; kh2++)
                    for (int kw2 = 0; kw2 < a.kW; kw2++) {
                        const uint16_t* xp = reinterpret_cast<const uint16_t*>(
                            win + ((pr * a.sH + kh2 * a.dH) * a.IWr + cur.s0 + pc * a.sW + kw2 * a.dW) * a.Pp);
                        for (int c = 0; c < a.Cp; c++) m = fmaxf(m, fabsf(h2f(xp[c])));
                    }
            }
            const float scale = row_scale(m);
            const float inv = 1.0f / scale;

            const int8_t* pix = win + (pr * a.sH * a.IWr + cur.s0 + pc * a.sW) * a.Pp;
            const int8_t* wrow = wl + l31 * a.KWp + 16 * hi;
            v16i acc[NCB];
#pragma unroll
            for (int cb = 0; cb < NCB; cb++)
#pragma unroll
                for (int e = 0; e < 16; e++) acc[cb][e] = 0;
            // one step ahead: the window taps and weight fragments of step ks + 1 and the
            // chunk offset of step ks + 2 are read while step ks is quantized (the offset
            // table is padded with zeros past the last step, so the reads stay in the window)
            int off_n = koff[2 + hi];
            uint4 h0 = *reinterpret_cast<const uint4*>(pix + koff[hi]);
            uint4 h1 = *reinterpret_cast<const uint4*>(pix + koff[hi] + 16);
            v4i wf[NCB];
#pragma unroll
            for (int cb = 0; cb < NCB; cb++) wf[cb] = *reinterpret_cast<const v4i*>(wrow + cb * 32 * a.KWp);
            for (int ks = 0; ks < a.ksteps; ks++) {
                const uint4 c0 = h0, c1 = h1;
                v4i wc[NCB];
#pragma unroll
                for (int cb = 0; cb < NCB; cb++) wc[cb] = wf[cb];
                h0 = *reinterpret_cast<const uint4*>(pix + off_n);
                h1 = *reinterpret_cast<const uint4*>(pix + off_n + 16);
                off_n = koff[2 * ks + 4 + hi];
                const int kn = ks + 1 < a.ksteps ? 32 * (ks + 1) : 0;
#pragma unroll
                for (int cb = 0; cb < NCB; cb++) wf[cb] = *reinterpret_cast<const v4i*>(wrow + cb * 32 * a.KWp + kn);
                // (an empty asm that may write memory: the compiler otherwise folds the
                // loop-carried loads back into loads at the top of the step, waited on at once)
                asm volatile("" ::: "memory");
                const v4i fb = quant16_cl(c0, c1, inv);
#pragma unroll
                for (int cb = 0; cb < NCB; cb++) acc[cb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wc[cb], fb, acc[cb], 0, 0, 0);
            }

            // the epilogue as dequant_gemm: half(fma((float)acc, as * ws, bias)), with -0 as
            // the bias without one; 2-byte buffer stores at 32-bit offsets, where pixels
            // outside the image and channels past C_out fall past the range and are dropped
            const __amdgpu_buffer_rsrc_t ry =
                buf_rsrc(a.y + static_cast<size_t>(cur.n) * a.Co * (plane2 >> 1), a.y_bytes);
            const int ho = cur.ho0 + pr, wo = cur.wo0 + pc;
            const bool pok = p0 < a.npix && ho < a.Ho && wo < a.Wo;
            const uint32_t vo = pok ? 2u * static_cast<uint32_t>(ho * a.Wo + wo) : 0x80000000u;
#pragma unroll
            for (int cb = 0; cb < NCB; cb++) {
                const int co0 = cb * 32 + 4 * hi;
                const uint32_t vc = vo + static_cast<uint32_t>(co0) * plane2;
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const float4 ws4 = *reinterpret_cast<const float4*>(s_ws + co0 + 8 * g);
                    const float4 b4 = *reinterpret_cast<const float4*>(s_b + co0 + 8 * g);
                    const float wsv[4] = {ws4.x, ws4.y, ws4.z, ws4.w}, bv[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const uint16_t yv =
                            f2h(__builtin_fmaf(static_cast<float>(acc[cb][4 * g + e]), scale * wsv[e], bv[e]));
                        __builtin_amdgcn_raw_buffer_store_b16(yv, ry, vc + static_cast<uint32_t>(8 * g + e) * plane2, 0,
                                                              0);
                    }
                }
            }
        }
        if (!has_next) break;
        walk.next = nxt;
        cur = geo_of(nxt);   // (decoded again rather than kept live across the tile)
        tag++;
        __syncthreads();   // the window and the maxima are free for the next tile
    }
}

// Workgroups of conv_nchw_cl_kernel<NCB, PF, NW> with lds bytes resident per CU, or minus a
// HIP error (sets the 160 KB dynamic-LDS limit on first use).
template <int NCB, bool PF, int NW>
static int conv_nchw_cl_residency(size_t lds)
{
    static std::once_flag once;
    static hipError_t attr;
    const void* fn = reinterpret_cast<const void*>(&conv_nchw_cl_kernel<NCB, PF, NW>);
    std::call_once(once, [&] { attr = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024); });
    if (attr != hipSuccess) return -static_cast<int>(attr);
    int blocks = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, 64 * NW, lds);
    if (e != hipSuccess) return -static_cast<int>(e);
    return blocks > 0 ? blocks : 1;
}

template <int NCB, bool PF, int NW>
static int conv_nchw_cl_launch(const ConvClArgs& a, size_t lds, hipStream_t s)
{
    int st = FORGE_OK;
    const DeviceInfo& dinfo = device_info(&st);
    if (st != FORGE_OK) return st;
    const int per_cu = conv_nchw_cl_residency<NCB, PF, NW>(lds);
    if (per_cu < 0) return -per_cu;
    const long long total = static_cast<long long>(a.tiles) * a.N;
    const long long cap = static_cast<long long>(dinfo.cu_count) * per_cu;
    const unsigned grid = static_cast<unsigned>(total < cap ? total : cap);
    note_route(PF ? "conv-nchw-cl prefetch" : "conv-nchw-cl", 32 * NW);
    conv_nchw_cl_kernel<NCB, PF, NW><<<grid, 64 * NW, lds, s>>>(a);
    return launch_status();
}

// Geometry of the channel-last path, or false when it does not apply (16-byte window loads
// need W % 8 == 0 and an aligned input; C_out <= 128; window, weights and tables within 80 KB
// of LDS so that two workgroups share a CU). The tile is Wt = 64 or 32 columns (fewer when the
// output is narrower) by R = 128 / Wt rows, whichever loads fewer window positions per pixel.
static bool conv_nchw_cl_plan(ConvClArgs& a, size_t* lds_bytes, int nw)
{
    const int npix_max = 32 * nw;
    if (a.W % 8 != 0 || !aligned(a.x, 16) || a.Co > 128) return false;
    a.Cp = (a.C + 15) & ~15;
    a.CQ = a.Cp / 16;
    const long long nch = static_cast<long long>(a.kH) * a.kW * a.CQ;
    if (nch > 512) return false;
    a.nch = static_cast<int>(nch);
    a.ksteps = (a.nch + 1) / 2;
    a.Pp = 2 * a.Cp + 16;
    a.KWp = 32 * a.ksteps + 16;
    const int cop = 32 * ((a.Co + 31) / 32);
    const long long xb = 2LL * a.C * a.H * a.W;
    if (xb >= (1LL << 30) || 2LL * cop * a.Ho * a.Wo >= (1LL << 31)) return false;
    auto up16 = [](long long b) { return (b + 15) & ~15LL; };
    long long best_bytes = -1;
    double best_cost = 0.0;
    for (const int wt_c : {64, 32}) {
        const int Wt = a.Wo < wt_c ? a.Wo : wt_c;
        const int R = std::min(npix_max / Wt, a.Ho);
        const long long IH = static_cast<long long>(R - 1) * a.sH + static_cast<long long>(a.kH - 1) * a.dH + 1;
        const long long IW = static_cast<long long>(Wt - 1) * a.sW + static_cast<long long>(a.kW - 1) * a.dW + 1;
        const long long G = (IW + 7 + 7) / 8;   // the first column read sits at position 0..7
        if (G > kWave) continue;
        const long long win = IH * (8 * G + 1) * a.Pp;
        const long long w_off = win, m1_off = w_off + static_cast<long long>(cop) * a.KWp;
        const long long koff_off = m1_off + up16(4 * IH * IW), ws_off = koff_off + up16(4LL * (2 * a.ksteps + 4));
        const long long bytes = ws_off + 8LL * cop;
        if (bytes > 80 * 1024) continue;
        const double cost = static_cast<double>(IH * 8 * G) / (R * Wt);
        if (best_bytes < 0 || cost < best_cost) {
            best_bytes = bytes;
            best_cost = cost;
            a.Wt = Wt;
            a.R = R;
            a.IH = static_cast<int>(IH);
            a.IW = static_cast<int>(IW);
            a.G = static_cast<int>(G);
            a.w_off = static_cast<int>(w_off);
            a.m1_off = static_cast<int>(m1_off);
            a.koff_off = static_cast<int>(koff_off);
            a.ws_off = static_cast<int>(ws_off);
        }
    }
    if (best_bytes < 0) return false;
    a.nw = nw;
    a.npix = a.R * a.Wt;
    a.IWr = 8 * a.G + 1;   // odd: the 8 positions a lane writes per row fall on different banks per row
    a.rpi = kWave / a.G;
    a.nrows = (a.Cp / 8) * a.IH;
    a.ninst = (a.nrows + a.rpi - 1) / a.rpi;
    a.mg_wt = udiv_multiplier(a.Wt);
    a.mg_rpi = udiv_multiplier(a.rpi);
    a.mg_ih = udiv_multiplier(a.IH);
    a.mg_iw = udiv_multiplier(a.IW);
    a.x_bytes = static_cast<uint32_t>(xb);
    a.y_bytes = static_cast<uint32_t>(2LL * a.Co * a.Ho * a.Wo);
    a.tiles_h = divup(a.Ho, a.R);
    a.tiles_w = divup(a.Wo, a.Wt);
    const long long tiles = static_cast<long long>(a.tiles_h) * a.tiles_w;
    if (tiles * a.N > 0x7FFFFFFFLL) return false;
    a.tiles = static_cast<int>(tiles);
    // udiv_magic ranges of the tile decode and the weight fill (larger calls take the
    // NCHW-window kernel)
    if (tiles * a.N * tiles >= (1LL << 32) || tiles * a.tiles_w >= (1LL << 32)) return false;
    if (1LL * a.Co * a.C * a.C >= (1LL << 32)) return false;
    a.mg_c = udiv_multiplier(a.C);
    a.wpad = a.C != a.Cp || a.Co % 32 != 0 || a.nch % 2 != 0;

    a.mg_tiles = udiv_multiplier(a.tiles);
    a.mg_tw = udiv_multiplier(a.tiles_w);
    *lds_bytes = static_cast<size_t>(best_bytes);
    return true;
}

template <int NW>
static int conv_nchw_cl_nw(const ConvClArgs& a, size_t lds, hipStream_t s)
{
    // each wave holds at most one load instruction's data (the 8-wave plan guarantees it)
    const bool pf = NW == 8 || a.ninst <= NW;
    switch ((a.Co + 31) / 32) {
        case 1: return pf ? conv_nchw_cl_launch<1, true, NW>(a, lds, s) : conv_nchw_cl_launch<1, NW == 8, NW>(a, lds, s);
        case 2: return pf ? conv_nchw_cl_launch<2, true, NW>(a, lds, s) : conv_nchw_cl_launch<2, NW == 8, NW>(a, lds, s);
        case 3: return pf ? conv_nchw_cl_launch<3, true, NW>(a, lds, s) : conv_nchw_cl_launch<3, NW == 8, NW>(a, lds, s);
        default: return pf ? conv_nchw_cl_launch<4, true, NW>(a, lds, s) : conv_nchw_cl_launch<4, NW == 8, NW>(a, lds, s);
    }
}
static int conv_nchw_cl(const ConvClArgs& a, size_t lds, hipStream_t s)
{
    return a.nw == 8 ? conv_nchw_cl_nw<8>(a, lds, s) : conv_nchw_cl_nw<4>(a, lds, s);
}

}  // namespace forge_amd

using namespace forge_amd;

extern "C" size_t forge_int8_conv2d_workspace_size(int C_in, int H, int W, int C_out, int kH, int kW,
                                                   int padH, int padW, int strideH, int strideW,
                                                   int dilH, int dilW)
{
    if (C_in <= 0 || C_out <= 0 || !conv_geom_ok(kH, kW, padH, padW, strideH, strideW, dilH, dilW)) return 0;
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
    if (!conv_geom_ok(kH, kW, padH, padW, strideH, strideW, dilH, dilW)) return FORGE_EINVAL;
    const int Ho = conv_out(H, padH, dilH, kH, strideH), Wo = conv_out(W, padW, dilW, kW, strideW);
    if (Ho <= 0 || Wo <= 0) return FORGE_OK;
    if (static_cast<long long>(Ho) * Wo > INT_MAX || static_cast<long long>(C_in) * kH * kW > INT_MAX ||
        static_cast<long long>(H) * W > INT_MAX)
        return FORGE_EINVAL;
    const int M = Ho * Wo, K = C_in * kH * kW;
    hipStream_t s = as_stream(stream);
    {
        ConvClArgs a{};
        a.x = input;
        a.w = weight;
        a.w_scale = w_scale;
        a.bias = bias;
        a.y = output;
        a.C = C_in;
        a.H = H;
        a.W = W;
        a.Co = C_out;
        a.kH = kH;
        a.kW = kW;
        a.padH = padH;
        a.padW = padW;
        a.sH = strideH;
        a.sW = strideW;
        a.dH = dilH;
        a.dW = dilW;
        a.Ho = Ho;
        a.Wo = Wo;
        a.K = K;
        a.N = N;
        size_t lds = 0;
        if (conv_nchw_cl_plan(a, &lds, 8) || conv_nchw_cl_plan(a, &lds, 4)) return conv_nchw_cl(a, lds, s);
    }
    {
        ConvNchwArgs a{input, weight, w_scale, bias, output, C_in, H, W, C_out, kH, kW, padH, padW, strideH, strideW,
                       dilH, dilW, Ho, Wo, K};
        size_t lds = 0;
        bool vec = false;
        if (conv_nchw_fused_plan(a, N, &lds, &vec)) {
            const bool pf = vec && a.ninst <= 4 * kPF;
            const void* fn = vec ? (pf ? reinterpret_cast<const void*>(&conv_nchw_fused_kernel<true, true>)
                                       : reinterpret_cast<const void*>(&conv_nchw_fused_kernel<true, false>))
                                 : reinterpret_cast<const void*>(&conv_nchw_fused_kernel<false, false>);
            int st = FORGE_OK;
            const DeviceInfo& dinfo = device_info(&st);
            if (st != FORGE_OK) return st;
            const int per_cu = conv_nchw_fused_residency(fn, lds);
            if (per_cu < 0) return -per_cu;
            const long long total = static_cast<long long>(a.tiles) * N;
            const long long cap = static_cast<long long>(dinfo.cu_count) * per_cu;
            const unsigned grid = static_cast<unsigned>(total < cap ? total : cap);
            note_route(pf ? "conv-nchw-fused prefetch" : "conv-nchw-fused");
            if (pf) conv_nchw_fused_kernel<true, true><<<grid, 256, lds, s>>>(a);
            else if (vec) conv_nchw_fused_kernel<true, false><<<grid, 256, lds, s>>>(a);
            else conv_nchw_fused_kernel<false, false><<<grid, 256, lds, s>>>(a);
            return launch_status();
        }
    }
    note_route("conv-nchw-per-image");
    auto up = [](size_t b) { return (b + 255) & ~static_cast<size_t>(255); };
    char* ws = static_cast<char*>(workspace);
    uint16_t* col16 = reinterpret_cast<uint16_t*>(ws);
    int8_t* col8 = reinterpret_cast<int8_t*>(ws + up(static_cast<size_t>(M) * K * 2));
    float* as = reinterpret_cast<float*>(reinterpret_cast<char*>(col8) + up(static_cast<size_t>(M) * K));
    uint16_t* gout = reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(as) + up(static_cast<size_t>(M) * 4));
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
