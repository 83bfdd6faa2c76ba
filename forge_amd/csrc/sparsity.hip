// 2:4 prune + compress and metadata packing for gfx950.
//
// prune: src/sparsity/prune_compress.cu:24-68 -- per group of 4 along K keep the two
// largest magnitudes; the two smallest are found with strict '<' comparisons seeded
// from positions (0, 1), so among equal magnitudes the lower index is pruned. Kept
// positions are ascending; nibble = keep0 | keep1 << 2. Values and nibbles are
// bit-identical to the reference.
//
// pack: src/sparsity/pack_metadata.cu:23-29 builds word (n, c) = sum_g nib[n,8c+g] << 4g.
// The same words are emitted here in the gfx950 SMFMAC layout: position
//     (n/16) * (K/32) * 16 + c * R + n%16,  R = min(16, N - 16*(n/16))
// For a full 16-row block, the 64 lanes of one v_smfmac_i32_16x16x128_i8 (lane =
// row%16 + 16*chunk) then read their index words as one contiguous 256-byte run.
#include "common.h"
#include "forge/sparsity/prune_compress.h"
#include "forge/sparsity/pack_metadata.h"

namespace forge_amd {

__host__ __device__ __forceinline__ size_t meta_pos(int n, int c, int N, int cpr) {
    const int blk = n >> 4;
    const int rows = (N - (blk << 4)) < 16 ? (N - (blk << 4)) : 16;
    return static_cast<size_t>(blk) * cpr * 16 + static_cast<size_t>(c) * rows + (n & 15);
}

// Prune one group of 4 (abs of int8 fits in int; abs(-128) = 128). The reference
// (prune_compress.cu:39-50) scans for the two smallest |v| with strict `<`, so on equal
// magnitudes the earlier position counts as the smaller: it prunes the two smallest keys
// |v_i| * 4 + i (distinct) and keeps the two largest, which a min/max network finds without
// branches or indexed register selects (checked against the scan on all 2^32 groups).
// c0, c1 = the kept values in ascending position, nib = k0 | k1 << 2.
__device__ __forceinline__ void prune4(const int8_t v[4], int8_t& c0, int8_t& c1, uint8_t& nib) {
    int key[4];
#pragma unroll
    for (int i = 0; i < 4; i++) key[i] = abs(static_cast<int>(v[i])) * 4 + i;
    const int a = max(key[0], key[1]), b = min(key[0], key[1]);
    const int c = max(key[2], key[3]), d = min(key[2], key[3]);
    const int m1 = max(a, c), m2 = max(min(a, c), max(b, d));   // the largest two keys
    const int i1 = m1 & 3, i2 = m2 & 3;
    const int k0 = min(i1, i2), k1 = max(i1, i2);
    c0 = v[k0];
    c1 = v[k1];
    nib = static_cast<uint8_t>(k0 | (k1 << 2));
}

// Vectorised launcher kernel: one thread per 4 groups (16 weights -> 8 compressed bytes and
// 4 nibbles); needs K % 16 == 0 and 16/8/4-byte aligned buffers.
__global__ __launch_bounds__(256) void prune_compress_vec_kernel(
    const int4* __restrict__ w, uint2* __restrict__ comp, uint32_t* __restrict__ meta, long long n16)
{
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < n16;
         i += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int4 v = w[i];
        const int8_t* b = reinterpret_cast<const int8_t*>(&v);
        uint32_t cw[2] = {0u, 0u};
        uint32_t mw = 0;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            int8_t c0, c1;
            uint8_t nib;
            prune4(b + 4 * g, c0, c1, nib);
            const uint32_t pair = (static_cast<uint32_t>(static_cast<uint8_t>(c0))) |
                                  (static_cast<uint32_t>(static_cast<uint8_t>(c1)) << 8);
            cw[g >> 1] |= pair << (16 * (g & 1));
            mw |= static_cast<uint32_t>(nib) << (8 * g);
        }
        comp[i] = make_uint2(cw[0], cw[1]);
        meta[i] = mw;
    }
}

// forge_pack_metadata's kernel: one thread per packed word in output order, so each store
// instruction writes 256 contiguous bytes (the gfx950 layout interleaves 16 rows, and walking it
// in input order scatters 4-byte stores 64 bytes apart). Word o of 16-row block b is chunk
// c = o' / rows of row 16b + o' % rows (o' = o - 16 b cpr; rows = 16 except in a last partial
// block); its 8 nibble bytes are one 8-byte load. N * K / 32 < 2^31 (the host checks).
__global__ __launch_bounds__(256) void pack_metadata_out_kernel(const uint8_t* __restrict__ raw,
                                                                uint32_t* __restrict__ packed, int N, int K)
{
    const int cpr = K / 32;
    const int total = N * cpr;
    const int o = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
    if (o >= total) return;
    const int per_blk = 16 * cpr;
    const int blk = o / per_blk;
    const int rows = min(16, N - 16 * blk);
    const int oi = o - blk * per_blk;
    const int c = oi / rows, n = 16 * blk + (oi - c * rows);
    const uint2 r = *reinterpret_cast<const uint2*>(raw + static_cast<size_t>(n) * (K / 4) + static_cast<size_t>(c) * 8);
    uint32_t w = 0;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        w |= ((r.x >> (8 * g)) & 0xFu) << (4 * g);
        w |= ((r.y >> (8 * g)) & 0xFu) << (4 * (g + 4));
    }
    packed[o] = w;
}

__global__ __launch_bounds__(256) void unpack_metadata_kernel(
    const uint32_t* __restrict__ packed, uint8_t* __restrict__ raw, int N, int K)
{
    const int cpr = K / 32;
    const long long total = static_cast<long long>(N) * cpr;
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int n = static_cast<int>(i / cpr), c = static_cast<int>(i % cpr);
        const uint32_t w = packed[meta_pos(n, c, N, cpr)];
        uint8_t* dst = raw + static_cast<size_t>(n) * (K / 4) + static_cast<size_t>(c) * 8;
#pragma unroll
        for (int g = 0; g < 8; g++) dst[g] = static_cast<uint8_t>((w >> (4 * g)) & 0xFu);
    }
}

// ---- weight preparation ------------------------------------------------------------
// python/forge/nn/linear.py:168-173 and :231-249 quantize a weight matrix with torch float32
// ops (scale = clamp(amax|w|, 1e-8) / 127, q = clamp(round(w / scale), -127, 127), scale
// stored as FP16), then SparseLinear launches prune_compress and pack_metadata through a raw
// nibble buffer. Here one workgroup per weight row does all of it: the row absmax (first read),
// then per 32-value chunk (second read, from L2) the IEEE division, round-half-even and clamp,
// the 2:4 prune of its 8 groups (prune4, the reference's tie rule), one 16-byte store of the
// compressed bytes and one index word at its gfx950 position. No dense INT8 or raw-nibble
// intermediate exists. The dense variant (QuantizedLinear) writes the INT8 row instead.

template <bool F16>
__device__ __forceinline__ float wload(const void* w, size_t i) {
    if constexpr (F16) return h2f(static_cast<const uint16_t*>(w)[i]);
    else return static_cast<const float*>(w)[i];
}

// 32 consecutive values from element offset off (a multiple of 32; 16-byte aligned base).
template <bool F16>
__device__ __forceinline__ void wload32(const void* w, size_t off, float (&v)[32]) {
    if constexpr (F16) {
        const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(w) + off);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint4 u = p[j];
            const uint32_t ws[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                v[8 * j + 2 * e] = h2f(static_cast<uint16_t>(ws[e] & 0xFFFFu));
                v[8 * j + 2 * e + 1] = h2f(static_cast<uint16_t>(ws[e] >> 16));
            }
        }
    } else {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(w) + off);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float4 f = p[j];
            v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
        }
    }
}

__device__ __forceinline__ int8_t quant_weight(float x, float scale) {
    const float r = fminf(fmaxf(__builtin_rintf(x / scale), -127.0f), 127.0f);
    return static_cast<int8_t>(static_cast<int>(r));
}

// Row absmax over the workgroup (256 threads), the reference's scale, and its FP16 copy.
__device__ __forceinline__ float block_row_scale(float amax, uint16_t* w_scale, int n) {
    __shared__ float red[4];
    amax = wave_max(amax);
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float scale = row_scale(amax);
    if (threadIdx.x == 0) w_scale[n] = f2h(scale);
    return scale;
}

// Chunk c (32 values) of weight row n: quantized with the row's scale, pruned 2:4, its 16
// compressed bytes and gfx950 index word stored.
__device__ __forceinline__ void prep_chunk(int8_t* __restrict__ comp, uint32_t* __restrict__ meta, int n, int c,
                                           int N, int K, const float (&v)[32], float scale)
{
    const int cpr = K / 32;
    uint32_t cw[4] = {0u, 0u, 0u, 0u};
    uint32_t word = 0;
#pragma unroll
    for (int g = 0; g < 8; g++) {
        int8_t q[4];
#pragma unroll
        for (int i = 0; i < 4; i++) q[i] = quant_weight(v[4 * g + i], scale);
        int8_t c0, c1;
        uint8_t nib;
        prune4(q, c0, c1, nib);
        const uint32_t pair = static_cast<uint32_t>(static_cast<uint8_t>(c0)) |
                              (static_cast<uint32_t>(static_cast<uint8_t>(c1)) << 8);
        cw[g >> 1] |= pair << (16 * (g & 1));
        word |= static_cast<uint32_t>(nib) << (4 * g);
    }
    *reinterpret_cast<uint4*>(comp + static_cast<size_t>(n) * (K / 2) + 16 * static_cast<size_t>(c)) =
        make_uint4(cw[0], cw[1], cw[2], cw[3]);
    meta[meta_pos(n, c, N, cpr)] = word;
}

template <bool F16>
__global__ __launch_bounds__(256) void prepare_sparse_weight_kernel(
    const void* __restrict__ w, int8_t* __restrict__ comp, uint32_t* __restrict__ meta,
    uint16_t* __restrict__ w_scale, int N, int K)
{
    const int n = blockIdx.x, t = threadIdx.x;
    const int cpr = K / 32;
    const size_t row = static_cast<size_t>(n) * K;
    float amax = 0.0f;
    if (cpr <= 256) {
        // At most one chunk per thread (K <= 8192): it stays in registers between the row
        // absmax and the quantization, so the row is read once.
        float v[32];
        if (t < cpr) {
            wload32<F16>(w, row + 32 * static_cast<size_t>(t), v);
#pragma unroll
            for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
        }
        const float scale = block_row_scale(amax, w_scale, n);
        if (t < cpr) prep_chunk(comp, meta, n, t, N, K, v, scale);
        return;
    }
    for (int c = t; c < cpr; c += 256) {
        float v[32];
        wload32<F16>(w, row + 32 * static_cast<size_t>(c), v);
#pragma unroll
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    }
    const float scale = block_row_scale(amax, w_scale, n);
    for (int c = t; c < cpr; c += 256) {
        float v[32];
        wload32<F16>(w, row + 32 * static_cast<size_t>(c), v);
        prep_chunk(comp, meta, n, c, N, K, v, scale);
    }
}

// Rows of at most 128 chunks (K <= 4096): two rows per workgroup, 128 threads (two waves) per
// row, one chunk per thread held in registers between the row absmax and the quantization.
template <bool F16>
__global__ __launch_bounds__(256) void prepare_sparse_weight2_kernel(
    const void* __restrict__ w, int8_t* __restrict__ comp, uint32_t* __restrict__ meta,
    uint16_t* __restrict__ w_scale, int N, int K)
{
    __shared__ float red[4];
    const int t = threadIdx.x, wave = t / kWave, c = t & 127;
    // Row pair of this workgroup. With N % 128 == 0 the 8 pairs of each 16-row block go to
    // workgroups of one XCD (workgroup ids are dealt round-robin over the 8 XCDs), so the
    // block's interleaved index words (16 rows per 256-byte group) meet in one L2.
    int pair = static_cast<int>(blockIdx.x);
    if (N % 128 == 0) {
        const int xcd = pair & 7, k = pair >> 3;
        pair = 8 * (8 * (k >> 3) + xcd) + (k & 7);
    }
    const int n = 2 * pair + (t >> 7);
    const int cpr = K / 32;
    const bool on = n < N && c < cpr;
    float v[32];
    float amax = 0.0f;
    if (on) {
        wload32<F16>(w, static_cast<size_t>(n) * K + 32 * static_cast<size_t>(c), v);
#pragma unroll
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    }
    amax = wave_max(amax);
    if ((t & (kWave - 1)) == 0) red[wave] = amax;
    __syncthreads();
    const float scale = row_scale(fmaxf(red[wave & ~1], red[wave | 1]));
    if (c == 0 && n < N) w_scale[n] = f2h(scale);
    if (on) prep_chunk(comp, meta, n, c, N, K, v, scale);
}

// Rows with K <= 4096, K % 16 == 0 and 16-byte-aligned rows: thread t holds values
// [16t, 16t + 16) of its row in registers between the row absmax and the quantization (the row
// is read once, in 16-byte loads) and stores its 16 INT8 values as one 16-byte store.
template <bool F16>
__global__ __launch_bounds__(256) void quantize_weight_rows_vec_kernel(
    const void* __restrict__ w, int8_t* __restrict__ q, uint16_t* __restrict__ w_scale, int K)
{
    const int n = blockIdx.x, t = threadIdx.x;
    const size_t off = static_cast<size_t>(n) * K + 16 * static_cast<size_t>(t);
    const bool on = 16 * t < K;
    float v[16];
    float amax = 0.0f;
    if (on) {
        if constexpr (F16) {
            const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(w) + off);
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const uint4 u = p[j];
                const uint32_t ws[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    v[8 * j + 2 * e] = h2f(static_cast<uint16_t>(ws[e] & 0xFFFFu));
                    v[8 * j + 2 * e + 1] = h2f(static_cast<uint16_t>(ws[e] >> 16));
                }
            }
        } else {
            const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(w) + off);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float4 f = p[j];
                v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
            }
        }
#pragma unroll
        for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(v[i]));
    }
    const float scale = block_row_scale(amax, w_scale, n);
    if (!on) return;
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        o[j] = 0u;
#pragma unroll
        for (int e = 0; e < 4; e++)
            o[j] |= static_cast<uint32_t>(static_cast<uint8_t>(quant_weight(v[4 * j + e], scale))) << (8 * e);
    }
    *reinterpret_cast<uint4*>(q + off) = make_uint4(o[0], o[1], o[2], o[3]);
}

template <bool F16>
__global__ __launch_bounds__(256) void quantize_weight_rows_kernel(
    const void* __restrict__ w, int8_t* __restrict__ q, uint16_t* __restrict__ w_scale, int K)
{
    const int n = blockIdx.x, t = threadIdx.x;
    const size_t row = static_cast<size_t>(n) * K;
    float amax = 0.0f;
    for (int k = t; k < K; k += 256) amax = fmaxf(amax, fabsf(wload<F16>(w, row + k)));
    const float scale = block_row_scale(amax, w_scale, n);
    for (int k = t; k < K; k += 256) q[row + k] = quant_weight(wload<F16>(w, row + k), scale);
}

}  // namespace forge_amd

namespace forge { namespace sparsity {

__global__ void prune_compress_kernel(const int8_t* __restrict__ weight,
                                      int8_t* __restrict__ compressed,
                                      uint8_t* __restrict__ metadata_raw, int N, int K)
{
    const long long idx = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    const int gpr = K / 4;
    if (idx >= static_cast<long long>(N) * gpr) return;
    const long long row = idx / gpr, g = idx % gpr;
    const int8_t* src = weight + row * K + g * 4;
    const int8_t v[4] = {src[0], src[1], src[2], src[3]};
    int8_t c0, c1;
    uint8_t nib;
    forge_amd::prune4(v, c0, c1, nib);
    compressed[row * (K / 2) + g * 2 + 0] = c0;
    compressed[row * (K / 2) + g * 2 + 1] = c1;
    metadata_raw[idx] = nib;
}

__global__ void pack_metadata_kernel(const uint8_t* __restrict__ meta_raw,
                                     uint32_t* __restrict__ meta_packed, int N, int K)
{
    const long long idx = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    const int cpr = K / 32;
    if (idx >= static_cast<long long>(N) * cpr) return;
    const int n = static_cast<int>(idx / cpr), c = static_cast<int>(idx % cpr);
    const uint8_t* src = meta_raw + static_cast<size_t>(n) * (K / 4) + static_cast<size_t>(c) * 8;
    uint32_t w = 0;
#pragma unroll
    for (int g = 0; g < 8; g++) w |= (static_cast<uint32_t>(src[g]) & 0xFu) << (4 * g);
    meta_packed[forge_amd::meta_pos(n, c, N, cpr)] = w;
}

}}  // namespace forge::sparsity

using namespace forge_amd;

extern "C" int forge_prune_compress_24(const int8_t* w, int8_t* comp, uint8_t* meta_raw,
                                       int N, int K, void* stream)
{
    if (N <= 0 || K <= 0) return FORGE_OK;
    if (!w || !comp || !meta_raw || K % 4 != 0) return FORGE_EINVAL;
    hipStream_t s = as_stream(stream);
    const long long groups = static_cast<long long>(N) * (K / 4);
    if (K % 16 == 0 && aligned(w, 16) && aligned(comp, 8) && aligned(meta_raw, 4)) {
        const long long n16 = groups / 4;
        const int blocks = static_cast<int>(std::min<long long>(divupll(n16, 256), 16384));
        prune_compress_vec_kernel<<<blocks, 256, 0, s>>>(reinterpret_cast<const int4*>(w),
                                                        reinterpret_cast<uint2*>(comp),
                                                        reinterpret_cast<uint32_t*>(meta_raw), n16);
    } else {
        forge::sparsity::prune_compress_kernel<<<static_cast<unsigned>(divupll(groups, 256)), 256, 0, s>>>(
            w, comp, meta_raw, N, K);
    }
    return launch_status();
}

extern "C" int forge_pack_metadata(const uint8_t* meta_raw, uint32_t* meta_packed, int N, int K,
                                   void* stream)
{
    if (N <= 0 || K <= 0) return FORGE_OK;
    if (!meta_raw || !meta_packed || K % 32 != 0) return FORGE_EINVAL;
    const long long total = static_cast<long long>(N) * (K / 32);
    if (total < (1LL << 31) && aligned(meta_raw, 8)) {
        pack_metadata_out_kernel<<<static_cast<unsigned>(divupll(total, 256)), 256, 0, as_stream(stream)>>>(
            meta_raw, meta_packed, N, K);
    } else {
        forge::sparsity::pack_metadata_kernel<<<static_cast<unsigned>(divupll(total, 256)), 256, 0,
                                                as_stream(stream)>>>(meta_raw, meta_packed, N, K);
    }
    return launch_status();
}

extern "C" int forge_unpack_metadata(const uint32_t* meta_packed, uint8_t* meta_raw, int N, int K,
                                     void* stream)
{
    if (N <= 0 || K <= 0) return FORGE_OK;
    if (!meta_raw || !meta_packed || K % 32 != 0) return FORGE_EINVAL;
    const long long total = static_cast<long long>(N) * (K / 32);
    const int blocks = static_cast<int>(std::min<long long>(divupll(total, 256), 16384));
    unpack_metadata_kernel<<<blocks, 256, 0, as_stream(stream)>>>(meta_packed, meta_raw, N, K);
    return launch_status();
}

extern "C" int forge_quantize_weight_rows(const void* w, int w_fp16, int8_t* w_int8, uint16_t* w_scale, int N, int K,
                                          void* stream)
{
    if (N <= 0 || K <= 0) return FORGE_OK;
    if (!w || !w_int8 || !w_scale) return FORGE_EINVAL;
    hipStream_t s = as_stream(stream);
    if (K % 16 == 0 && K <= 4096 && aligned(w, 16) && aligned(w_int8, 16)) {
        if (w_fp16) quantize_weight_rows_vec_kernel<true><<<N, 256, 0, s>>>(w, w_int8, w_scale, K);
        else        quantize_weight_rows_vec_kernel<false><<<N, 256, 0, s>>>(w, w_int8, w_scale, K);
    } else if (w_fp16) {
        quantize_weight_rows_kernel<true><<<N, 256, 0, s>>>(w, w_int8, w_scale, K);
    } else {
        quantize_weight_rows_kernel<false><<<N, 256, 0, s>>>(w, w_int8, w_scale, K);
    }
    return launch_status();
}

extern "C" int forge_prepare_sparse_weight(const void* w, int w_fp16, int8_t* W_comp, uint32_t* w_meta,
                                           uint16_t* w_scale, int N, int K, void* stream)
{
    if (N <= 0 || K <= 0) return FORGE_OK;
    if (!w || !W_comp || !w_meta || !w_scale || K % 32 != 0 || !aligned(w, 16) || !aligned(W_comp, 16) ||
        !aligned(w_meta, 4))
        return FORGE_EINVAL;
    hipStream_t s = as_stream(stream);
    if (K / 32 <= 128) {
        const unsigned g2 = static_cast<unsigned>((N + 1) / 2);
        if (w_fp16) prepare_sparse_weight2_kernel<true><<<g2, 256, 0, s>>>(w, W_comp, w_meta, w_scale, N, K);
        else        prepare_sparse_weight2_kernel<false><<<g2, 256, 0, s>>>(w, W_comp, w_meta, w_scale, N, K);
    } else if (w_fp16) {
        prepare_sparse_weight_kernel<true><<<N, 256, 0, s>>>(w, W_comp, w_meta, w_scale, N, K);
    } else {
        prepare_sparse_weight_kernel<false><<<N, 256, 0, s>>>(w, W_comp, w_meta, w_scale, N, K);
    }
    return launch_status();
}
