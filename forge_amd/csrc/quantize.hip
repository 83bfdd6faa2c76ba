// Per-token FP16 -> INT8 activation quantization and INT32 -> FP16 dequantization
// for gfx950.
//
// Reference behaviour: src/quant/quantize.cu:8-191 and src/quant/dequantize.cu:8-45.
//   scale[m] = max(absmax(x[m,:]), 1e-8f) / 127.0f      (IEEE division)
//   q[m,k]   = clamp(rne(x[m,k] * (1.0f / scale[m])), -128, 127)
//
// MI355X design: the main kernel gives each row to one 256-thread workgroup (short rows at
// large M: one wavefront per row, 4 rows per workgroup). A lane holds VPT 16-byte vectors of
// its row in VGPRs, so x is read from HBM once; the row absmax is a packed u16 maximum of the
// fp16 magnitude bit patterns reduced across the wave by DPP (plus a 4-entry LDS max), with
// the fp32 maximum for a row that holds a NaN; then each lane writes 8 int8 per vector. The
// exported two-pass kernel (any K, any alignment, any block size) reduces through LDS in
// fp32. All compute the same max (exact) and the same IEEE-rounded arithmetic, so their
// outputs are bit-identical.
#include "common.h"
#include "forge/quant/quantize.h"
#include "forge/quant/dequantize.h"

namespace forge_amd {

// One 256-thread workgroup per row; K % 8 == 0, K <= VPT * 2048, x 16-byte and q 8-byte
// aligned. Thread t holds 16-byte vectors t, t + 256, ... of its row in VGPRs (x is read
// once) and every lane writes 8 int8 per vector. Spreading a row over 4 waves keeps
// decode-size calls (a handful of rows) from serialising one wave's loads.
//
// All of a lane's loads are issued before any is used, unconditionally: a lane past the row
// end re-reads the row's last vector, which cannot change a maximum (a load inside
// `if (idx < nvec)` next to its use compiled to load -> wait -> use, one memory latency per
// vector). The absmax runs on fp16 bit patterns (absbits8: one packed u16 max per two values,
// DPP across the wave, 4 entries through LDS); a row holding a NaN takes the fp32 maximum,
// which skips NaN as fmaxf does. Values are quantized by quant8_row, bit-equal to quant8
// for a row's own scale.
template <int VPT>
__global__ __launch_bounds__(256) void quantize_rows_block_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ scales, int K)
{
    __shared__ uint32_t wbits[4];
    __shared__ float wmax[4];
    const int row = blockIdx.x;
    const int t = threadIdx.x, lane = t & (kWave - 1), wave = t / kWave;
    const int nvec = K >> 3;
    const uint4* src = reinterpret_cast<const uint4*>(x + static_cast<size_t>(row) * K);
    uint2* dst = reinterpret_cast<uint2*>(q + static_cast<size_t>(row) * K);
    uint4 v[VPT];
#pragma unroll
    for (int i = 0; i < VPT; i++) v[i] = src[min(t + i * 256, nvec - 1)];
    uint32_t m = 0u;
#pragma unroll
    for (int i = 0; i < VPT; i++) m = absbits8(v[i], m);
    m = wave_max_pk_u16(pk_max_u16(m, m >> 16)) & 0xFFFFu;
    if (lane == 0) wbits[wave] = m;
    __syncthreads();
    const uint32_t bits = max(max(wbits[0], wbits[1]), max(wbits[2], wbits[3]));
    float amax;
    if (bits > kHalfInfBits) {               // the row holds a NaN (uniform over the workgroup)
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < VPT; i++) a = absmax8(v[i], a);
        a = wave_max(a);
        if (lane == 0) wmax[wave] = a;
        __syncthreads();
        amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    } else {
        amax = h2f(static_cast<uint16_t>(bits));
    }
    const float scale = row_scale(amax);
    const float inv = 1.0f / scale;
    if (t == 0) scales[row] = scale;
#pragma unroll
    for (int i = 0; i < VPT; i++) {
        const int idx = t + i * 256;
        if (idx < nvec) dst[idx] = quant8_row(v[i], inv);
    }
}

// Rows up to K = 4096 at large M: one wavefront per row, 4 rows per workgroup, so a workgroup
// moves 4 rows, needs no barrier, and the grid is M/4 workgroups instead of M (at M = 147,456,
// K = 1280 the per-row workgroups ran at 3.6 TB/s; configs[1], 4096 x 4096: 9.3 -> 8.3 us,
// 6.06 TB/s of 50.3 MB). Lane t holds vectors t, t + 64,
// ... of its row; loads, absmax and quantization as in the kernel above, the absmax reduced
// within the wave by DPP.
template <int VPT>
__global__ __launch_bounds__(256) void quantize_rows_wave_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ scales, int M, int K)
{
    const int lane = threadIdx.x & (kWave - 1);
    const int row = blockIdx.x * 4 + static_cast<int>(threadIdx.x / kWave);
    if (row >= M) return;                    // whole waves leave: the DPP reduction sees 64 lanes
    const int nvec = K >> 3;
    const uint4* src = reinterpret_cast<const uint4*>(x + static_cast<size_t>(row) * K);
    uint2* dst = reinterpret_cast<uint2*>(q + static_cast<size_t>(row) * K);
    uint4 v[VPT];
#pragma unroll
    for (int i = 0; i < VPT; i++) v[i] = src[min(lane + i * kWave, nvec - 1)];
    uint32_t m = 0u;
#pragma unroll
    for (int i = 0; i < VPT; i++) m = absbits8(v[i], m);
    const uint32_t bits = wave_max_pk_u16(pk_max_u16(m, m >> 16)) & 0xFFFFu;
    float amax;
    if (bits > kHalfInfBits) {               // the row holds a NaN (uniform over the wave)
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < VPT; i++) a = absmax8(v[i], a);
        amax = wave_max(a);
    } else {
        amax = h2f(static_cast<uint16_t>(bits));
    }
    const float scale = row_scale(amax);
    const float inv = 1.0f / scale;
    if (lane == 0) scales[row] = scale;
#pragma unroll
    for (int i = 0; i < VPT; i++) {
        const int idx = lane + i * kWave;
        if (idx < nvec) dst[idx] = quant8_row(v[i], inv);
    }
}

// Per-pixel quantization of NCHW FP16 images (the transposed conv's input rows): pixel p of
// image i is the row x[i, :, p] (C channels at stride HW), quantized with the row arithmetic
// above and written as row i*HW + p of q (C contiguous int8) with its scale. A workgroup
// takes 64 consecutive pixels of one image: each wave reads every 4th channel as 128-byte
// coalesced runs (x is read from HBM once), the four partial absmaxes meet in LDS, and the
// 64 rows -- one contiguous block of q -- are written G channels (4 bytes or 1) per lane.
// STASH keeps the tile in LDS (64 x (C + 4) halves; the +4 pad spreads the column writes
// over the banks and keeps 8-byte row reads aligned); without it the second pass re-reads x.
constexpr int kPixTile = 64;
constexpr int kPixStashMaxC = 512;

template <int G, bool STASH>
__global__ __launch_bounds__(256) void quantize_pixels_nchw_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ scales, int C, int HW,
    int tiles)
{
    extern __shared__ __align__(16) uint16_t stash[];
    __shared__ float red[4][kPixTile];
    __shared__ float sinv[kPixTile];
    const int img = blockIdx.x / tiles;
    const int p0 = (blockIdx.x - img * tiles) * kPixTile;
    const int np = min(kPixTile, HW - p0);
    const int t = threadIdx.x, pl = t & (kPixTile - 1), cg = t >> 6;
    const int pitch = C + 4;
    const uint16_t* xi = x + static_cast<size_t>(img) * C * HW + p0;
    float amax = 0.0f;
    if (pl < np) {
        // kBatch channel loads in flight per lane before the first use.
        constexpr int kBatch = 16;
        for (int c0 = cg; c0 < C; c0 += 4 * kBatch) {
            uint16_t v[kBatch];
#pragma unroll
            for (int j = 0; j < kBatch; j++) {
                const int c = c0 + 4 * j;
                v[j] = c < C ? xi[static_cast<size_t>(c) * HW + pl] : static_cast<uint16_t>(0);
            }
#pragma unroll
            for (int j = 0; j < kBatch; j++) {
                const int c = c0 + 4 * j;
                if (c < C) {
                    amax = fmaxf(amax, fabsf(h2f(v[j])));
                    if constexpr (STASH) stash[pl * pitch + c] = v[j];
                }
            }
        }
    }
    red[cg][pl] = amax;
    __syncthreads();
    if (t < kPixTile) {
        const float a = fmaxf(fmaxf(red[0][t], red[1][t]), fmaxf(red[2][t], red[3][t]));
        const float scale = row_scale(a);
        sinv[t] = 1.0f / scale;
        if (t < np) scales[static_cast<size_t>(img) * HW + p0 + t] = scale;
    }
    __syncthreads();
    int8_t* qb = q + (static_cast<size_t>(img) * HW + p0) * C;
    const int items = np * (C / G);
    for (int i = t; i < items; i += 256) {
        const int e = i * G;
        const int p = e / C, c = e - p * C;
        const float inv = sinv[p];
        if constexpr (G == 4) {
            uint16_t v[4];
            if constexpr (STASH) {
                const uint2 w = *reinterpret_cast<const uint2*>(stash + p * pitch + c);
                v[0] = static_cast<uint16_t>(w.x & 0xFFFFu); v[1] = static_cast<uint16_t>(w.x >> 16);
                v[2] = static_cast<uint16_t>(w.y & 0xFFFFu); v[3] = static_cast<uint16_t>(w.y >> 16);
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) v[j] = xi[static_cast<size_t>(c + j) * HW + p];
            }
            uint32_t packed = 0;
#pragma unroll
            for (int j = 0; j < 4; j++)
                packed |= (static_cast<uint32_t>(quant1(h2f(v[j]), inv)) & 0xFFu) << (8 * j);
            *reinterpret_cast<uint32_t*>(qb + e) = packed;
        } else {
            const uint16_t v = STASH ? stash[p * pitch + c] : xi[static_cast<size_t>(c) * HW + p];
            qb[e] = static_cast<int8_t>(quant1(h2f(v), inv));
        }
    }
}

// Two-pass body shared by the exported kernel: any K, any alignment, any blockDim.
__device__ void quantize_row_twopass(const uint16_t* __restrict__ in_row, int8_t* __restrict__ out_row,
                                     float* __restrict__ scale_out, int K)
{
    __shared__ float red[1024];
    const int t = threadIdx.x, nt = blockDim.x;
    float m = 0.0f;
    for (int k = t; k < K; k += nt) m = fmaxf(m, fabsf(h2f(in_row[k])));
    red[t] = m;
    __syncthreads();
    // Tree over the next power of two >= blockDim (missing entries read as 0).
    int p = 1;
    while (p < nt) p <<= 1;
    for (int s = p >> 1; s > 0; s >>= 1) {
        if (t < s && t + s < nt) red[t] = fmaxf(red[t], red[t + s]);
        __syncthreads();
    }
    const float scale = row_scale(red[0]);
    const float inv = 1.0f / scale;
    if (t == 0) *scale_out = scale;
    for (int k = t; k < K; k += nt) out_row[k] = static_cast<int8_t>(quant1(h2f(in_row[k]), inv));
}

// Dequant of src/quant/dequantize.cu:22-26: ((float)acc * as) * ws [+ bias].
__device__ __forceinline__ uint16_t dequant_standalone(int acc, float as, float ws, float b, bool has_bias) {
    const float p = static_cast<float>(acc) * as;
    return f2h(has_bias ? __builtin_fmaf(p, ws, b) : p * ws);
}

// Vectorised launcher kernel: 4 outputs per thread, grid-stride over the (M,N) range.
// Four columns per thread: 16 bytes of INT32 sums, the columns' w_scale and bias as one 8-byte
// load each (N % 4 == 0, 8-byte-aligned vectors), 8 bytes of FP16 out; 32-bit indices
// (M * N / 4 < 2^31, checked by the host). The index is unsigned: with total4 < 2^31 and a
// stride of at most 2^22 (16384 workgroups of 256), i + stride stays below 2^32, so the last
// increment cannot wrap into the range again.
__global__ __launch_bounds__(256) void dequantize_vec4_kernel(
    const int4* __restrict__ acc, const float* __restrict__ act_scale,
    const uint16_t* __restrict__ w_scale, const uint16_t* __restrict__ bias,
    uint2* __restrict__ out, uint32_t n4, uint32_t total4)
{
    // total4 < 2^31 and stride <= 16384 * 256 = 2^22 (host guards), so i + stride < 2^32: the
    // unsigned counter never wraps.
    const uint32_t stride = gridDim.x * 256u;
    for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < total4; i += stride) {
        const uint32_t m = i / n4;
        const uint32_t n = (i - m * n4) * 4;
        const int4 a = acc[i];
        const float as = act_scale[m];
        const uint2 wv = *reinterpret_cast<const uint2*>(w_scale + n);
        const uint2 bv = bias ? *reinterpret_cast<const uint2*>(bias + n) : make_uint2(0u, 0u);
        const int av[4] = {a.x, a.y, a.z, a.w};
        const uint32_t wr[4] = {wv.x & 0xFFFFu, wv.x >> 16, wv.y & 0xFFFFu, wv.y >> 16};
        const uint32_t br[4] = {bv.x & 0xFFFFu, bv.x >> 16, bv.y & 0xFFFFu, bv.y >> 16};
        uint16_t h[4];
#pragma unroll
        for (int j = 0; j < 4; j++)
            h[j] = dequant_standalone(av[j], as, h2f(static_cast<uint16_t>(wr[j])),
                                      bias ? h2f(static_cast<uint16_t>(br[j])) : 0.0f, bias != nullptr);
        out[i] = make_uint2(h[0] | (static_cast<uint32_t>(h[1]) << 16),
                            h[2] | (static_cast<uint32_t>(h[3]) << 16));
    }
}

}  // namespace forge_amd

// ---- exported kernels (reference symbols) ----------------------------------------

namespace forge { namespace quant {

// include/forge/quant/quantize.cuh:17-21: grid = M rows, any block size.
__global__ void fused_quantize_activation_kernel(const __half* __restrict__ input,
                                                 int8_t* __restrict__ output,
                                                 float* __restrict__ scales, int K)
{
    const size_t row = blockIdx.x;
    forge_amd::quantize_row_twopass(reinterpret_cast<const uint16_t*>(input) + row * K,
                                    output + row * K, scales + row, K);
}

// include/forge/quant/dequantize.cuh:14-20: grid = M rows, any block size.
__global__ void fused_dequantize_bias_kernel(const int32_t* __restrict__ input,
                                             const float* __restrict__ act_scale,
                                             const __half* __restrict__ w_scale,
                                             const __half* __restrict__ bias,
                                             __half* __restrict__ output, int N)
{
    const size_t row = blockIdx.x;
    const float as = act_scale[row];
    const uint16_t* ws = reinterpret_cast<const uint16_t*>(w_scale);
    const uint16_t* b = reinterpret_cast<const uint16_t*>(bias);
    uint16_t* out = reinterpret_cast<uint16_t*>(output) + row * N;
    for (int n = threadIdx.x; n < N; n += blockDim.x)
        out[n] = forge_amd::dequant_standalone(input[row * N + n], as, forge_amd::h2f(ws[n]),
                                               b ? forge_amd::h2f(b[n]) : 0.0f, b != nullptr);
}

}}  // namespace forge::quant

// ---- C-ABI -----------------------------------------------------------------------

using namespace forge_amd;

namespace forge_amd {

// Rows per launch from which the wave-per-row kernel takes short rows: below it the grid is
// small and a whole workgroup per row spreads each row's loads wider.
constexpr int kWaveRowsMinM = 2048;

int launch_quantize(const uint16_t* x, int8_t* q, float* scales, int M, int K, hipStream_t s)
{
    const bool vec_ok = (K % 8 == 0) && K <= 8 * 2048 && aligned(x, 16) && aligned(q, 8);
    if (vec_ok && K <= 4096 && M >= kWaveRowsMinM) {
        const int vpt = divup(K, 8 * kWave);
        const unsigned grid = static_cast<unsigned>(divup(M, 4));
        if (vpt <= 1)      quantize_rows_wave_kernel<1><<<grid, 256, 0, s>>>(x, q, scales, M, K);
        else if (vpt <= 2) quantize_rows_wave_kernel<2><<<grid, 256, 0, s>>>(x, q, scales, M, K);
        else if (vpt <= 4) quantize_rows_wave_kernel<4><<<grid, 256, 0, s>>>(x, q, scales, M, K);
        else               quantize_rows_wave_kernel<8><<<grid, 256, 0, s>>>(x, q, scales, M, K);
        return launch_status();
    }
    if (vec_ok) {
        const int vpt = divup(K, 2048);
        if (vpt <= 1)      quantize_rows_block_kernel<1><<<M, 256, 0, s>>>(x, q, scales, K);
        else if (vpt <= 2) quantize_rows_block_kernel<2><<<M, 256, 0, s>>>(x, q, scales, K);
        else if (vpt <= 4) quantize_rows_block_kernel<4><<<M, 256, 0, s>>>(x, q, scales, K);
        else               quantize_rows_block_kernel<8><<<M, 256, 0, s>>>(x, q, scales, K);
    } else {
        forge::quant::fused_quantize_activation_kernel<<<M, 256, 0, s>>>(
            reinterpret_cast<const __half*>(x), q, scales, K);
    }
    return launch_status();
}

int launch_quantize_pixels_nchw(const uint16_t* x, int8_t* q, float* scales, int images, int C, int HW,
                                hipStream_t s)
{
    const int tiles = divup(HW, kPixTile);
    const long long blocks = static_cast<long long>(images) * tiles;
    if (blocks > 0x7FFFFFFFLL) return FORGE_EINVAL;
    const bool g4 = (C % 4 == 0) && aligned(q, 4);
    const bool stash = C <= kPixStashMaxC;
    const size_t lds = stash ? static_cast<size_t>(kPixTile) * (C + 4) * sizeof(uint16_t) : 0;
    const unsigned grid = static_cast<unsigned>(blocks);
    if (stash) {
        // At most 64 x 516 halves = 66 KB: above the default 64 KB, so raise the limit once.
        static const hipError_t a4 = hipFuncSetAttribute(
            reinterpret_cast<const void*>(quantize_pixels_nchw_kernel<4, true>),
            hipFuncAttributeMaxDynamicSharedMemorySize, kPixTile * (kPixStashMaxC + 4) * 2);
        static const hipError_t a1 = hipFuncSetAttribute(
            reinterpret_cast<const void*>(quantize_pixels_nchw_kernel<1, true>),
            hipFuncAttributeMaxDynamicSharedMemorySize, kPixTile * (kPixStashMaxC + 4) * 2);
        if (a4 != hipSuccess) return static_cast<int>(a4);
        if (a1 != hipSuccess) return static_cast<int>(a1);
        if (g4) quantize_pixels_nchw_kernel<4, true><<<grid, 256, lds, s>>>(x, q, scales, C, HW, tiles);
        else    quantize_pixels_nchw_kernel<1, true><<<grid, 256, lds, s>>>(x, q, scales, C, HW, tiles);
    } else {
        if (g4) quantize_pixels_nchw_kernel<4, false><<<grid, 256, 0, s>>>(x, q, scales, C, HW, tiles);
        else    quantize_pixels_nchw_kernel<1, false><<<grid, 256, 0, s>>>(x, q, scales, C, HW, tiles);
    }
    return launch_status();
}

}  // namespace forge_amd

extern "C" int forge_quantize_activation(const uint16_t* x, int8_t* q, float* scales,
                                         int M, int K, void* stream)
{
    if (M <= 0 || K <= 0) return FORGE_OK;
    if (!x || !q || !scales) return FORGE_EINVAL;
    return launch_quantize(x, q, scales, M, K, as_stream(stream));
}

extern "C" int forge_quantize_activation_twopass(const uint16_t* x, int8_t* q, float* scales,
                                                 int M, int K, int threads, void* stream)
{
    if (M <= 0 || K <= 0) return FORGE_OK;
    if (!x || !q || !scales || threads < 1 || threads > 1024) return FORGE_EINVAL;
    forge::quant::fused_quantize_activation_kernel<<<M, threads, 0, as_stream(stream)>>>(
        reinterpret_cast<const __half*>(x), q, scales, K);
    return launch_status();
}

extern "C" int forge_dequantize_bias(const int32_t* acc, const float* act_scale,
                                     const uint16_t* w_scale, const uint16_t* bias, uint16_t* out,
                                     int M, int N, void* stream)
{
    if (M <= 0 || N <= 0) return FORGE_OK;
    if (!acc || !act_scale || !w_scale || !out) return FORGE_EINVAL;
    hipStream_t s = as_stream(stream);
    const long long total4 = static_cast<long long>(M) * (N / 4);
    if (N % 4 == 0 && total4 < (1LL << 31) && aligned(acc, 16) && aligned(out, 8) && aligned(w_scale, 8) &&
        (!bias || aligned(bias, 8))) {
        const int blocks = static_cast<int>(std::min<long long>(divupll(total4, 256), 16384));
        dequantize_vec4_kernel<<<blocks, 256, 0, s>>>(reinterpret_cast<const int4*>(acc), act_scale,
                                                     w_scale, bias, reinterpret_cast<uint2*>(out),
                                                     static_cast<uint32_t>(N / 4), static_cast<uint32_t>(total4));
    } else {
        forge::quant::fused_dequantize_bias_kernel<<<M, 256, 0, s>>>(
            acc, act_scale, reinterpret_cast<const __half*>(w_scale),
            reinterpret_cast<const __half*>(bias), reinterpret_cast<__half*>(out), N);
    }
    return launch_status();
}
