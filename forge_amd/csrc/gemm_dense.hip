// Dense INT8 GEMM for gfx950: C = A (M,K) x B (N,K)^T with exact INT32 accumulation on
// v_mfma_i32_32x32x32_i8, and the fused dequant + bias epilogue to FP16.
//
// Reference: src/gemm/int8_dense.cu:26-232 (wmma 16x16x16, 128x64 / 128x128 tiles,
// unpipelined global->smem loads) and src/gemm/int8_gemm.cu:12-46 (dispatch). The
// epilogue arithmetic follows int8_dense.cu:171-174:
//     Y[m,n] = half(fma((float)acc, act_scale[m] * w_scale[n], bias[n]))
// The tile engine (mfma_tile.h) stages 64-byte K slices through swizzled LDS with one
// barrier per stage; tiles are mapped XCD-aware. Skinny M (decode) goes to gemm_skinny.
#include "common.h"
#include "mfma_tile.h"
#include "gemm_dense.h"
#include "forge/gemm/int8_dense.h"
#include "forge/gemm/int8_gemm.h"
#include "forge/gemm/int8_dp4a.h"

#include <algorithm>

namespace forge_amd {

template <int BM, int BN, int WM, int WN, bool DEQUANT, class ALoader>
__global__ __launch_bounds__(WM * WN * kWave) void gemm_tile_kernel(
    ALoader la, RowMajorLoader lb, GemmEpilogue ep, int tiles_m, int tiles_n, int K, int vec)
{
    extern __shared__ __align__(16) int8_t lds[];
    using Tile = MfmaTile<BM, BN, WM, WN>;
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    Tile t;
    t.run(la, lb, m0, n0, K, vec != 0, lds);

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int wm = m0 + (wave / WN) * (BM / WM);
    const int wn = n0 + (wave % WN) * (BN / WN);
#pragma unroll
    for (int j = 0; j < Tile::kTN; j++) {
        const int col = wn + 32 * j + acc_col(lane);
        if (col >= ep.N) continue;
        float ws = 0.0f, b = 0.0f;
        if constexpr (DEQUANT) {
            ws = h2f(ep.w_scale[col]);
            if (ep.bias) b = h2f(ep.bias[col]);
        }
#pragma unroll
        for (int i = 0; i < Tile::kTM; i++) {
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int row = wm + 32 * i + acc_row(e, lane);
                if (row >= ep.M) continue;
                const size_t o = static_cast<size_t>(row) * ep.N + col;
                if constexpr (DEQUANT)
                    ep.c16[o] = dequant_gemm(t.acc[i][j][e], ep.act_scale[row], ws, b, ep.bias != nullptr);
                else
                    ep.c32[o] = t.acc[i][j][e];
            }
        }
    }
}

template <int BM, int BN, int WM, int WN, bool DEQUANT, class ALoader>
static int launch_tile(const ALoader& la, const RowMajorLoader& lb, const GemmEpilogue& ep,
                       int M, int N, int K, bool vec, hipStream_t s)
{
    using Tile = MfmaTile<BM, BN, WM, WN>;
    const int tiles_m = divup(M, BM), tiles_n = divup(N, BN);
    const long long total = static_cast<long long>(tiles_m) * tiles_n;
    if (total > 0x7FFFFFFFLL) return FORGE_EINVAL;
    gemm_tile_kernel<BM, BN, WM, WN, DEQUANT, ALoader>
        <<<static_cast<unsigned>(total), Tile::kThreads, Tile::kLdsBytes, s>>>(
            la, lb, ep, tiles_m, tiles_n, K, vec ? 1 : 0);
    return launch_status();
}

// Picks the largest tile that still gives every CU a workgroup.
template <bool DEQUANT, class ALoader>
int launch_gemm_tiles(const ALoader& la, const RowMajorLoader& lb, const GemmEpilogue& ep,
                      int M, int N, int K, bool vec, hipStream_t s)
{
    int st = FORGE_OK;
    const DeviceInfo& d = device_info(&st);
    if (st != FORGE_OK) return st;
    const long long t256 = static_cast<long long>(divup(M, 256)) * divup(N, 256);
    const long long t128 = static_cast<long long>(divup(M, 128)) * divup(N, 128);
    if (t256 >= d.cu_count)
        return launch_tile<256, 256, 2, 2, DEQUANT>(la, lb, ep, M, N, K, vec, s);
    if (t128 >= d.cu_count / 2)
        return launch_tile<128, 128, 2, 2, DEQUANT>(la, lb, ep, M, N, K, vec, s);
    return launch_tile<64, 64, 2, 2, DEQUANT>(la, lb, ep, M, N, K, vec, s);
}

template int launch_gemm_tiles<true, ConvLoader>(const ConvLoader&, const RowMajorLoader&,
                                                 const GemmEpilogue&, int, int, int, bool, hipStream_t);
template int launch_gemm_tiles<false, ConvLoader>(const ConvLoader&, const RowMajorLoader&,
                                                  const GemmEpilogue&, int, int, int, bool, hipStream_t);

int gemm_dense(const int8_t* A, const int8_t* B, const float* act_scale, const uint16_t* w_scale,
               const uint16_t* bias, uint16_t* out16, int32_t* out32, int M, int K, int N,
               hipStream_t s)
{
    const bool vec = (K % 16 == 0) && aligned(A, 16) && aligned(B, 16);
    GemmEpilogue ep{out32, out16, act_scale, w_scale, bias, M, N};
    if (M <= kSkinnyMaxM && vec)
        return launch_gemm_skinny(A, B, ep, M, K, N, s);
    RowMajorLoader la{A, M, K}, lb{B, N, K};
    if (out16) return launch_gemm_tiles<true>(la, lb, ep, M, N, K, vec, s);
    return launch_gemm_tiles<false>(la, lb, ep, M, N, K, vec, s);
}

}  // namespace forge_amd

using namespace forge_amd;

extern "C" int forge_int8_gemm_dequant(const int8_t* A, const int8_t* B, const float* act_scale,
                                       const uint16_t* w_scale, const uint16_t* bias, uint16_t* out,
                                       int M, int K, int N, void* stream)
{
    if (M <= 0 || K <= 0 || N <= 0) return FORGE_OK;
    if (!A || !B || !act_scale || !w_scale || !out) return FORGE_EINVAL;
    return gemm_dense(A, B, act_scale, w_scale, bias, out, nullptr, M, K, N, as_stream(stream));
}

extern "C" int forge_int8_gemm(const int8_t* A, const int8_t* B, const float* act_scale,
                               const uint16_t* w_scale, const uint16_t* bias, uint16_t* out,
                               int M, int K, int N, void* stream)
{
    return forge_int8_gemm_dequant(A, B, act_scale, w_scale, bias, out, M, K, N, stream);
}

extern "C" int forge_int8_gemm_s32(const int8_t* A, const int8_t* B, int32_t* C,
                                   int M, int K, int N, void* stream)
{
    if (M <= 0 || K <= 0 || N <= 0) return FORGE_OK;
    if (!A || !B || !C) return FORGE_EINVAL;
    return gemm_dense(A, B, nullptr, nullptr, nullptr, nullptr, C, M, K, N, as_stream(stream));
}

extern "C" int forge_int8_linear(const uint16_t* x, const int8_t* w, const uint16_t* w_scale,
                                 const uint16_t* bias, uint16_t* out, int M, int K, int N,
                                 int8_t* scratch_q, float* scratch_scale, void* stream)
{
    if (M <= 0 || K <= 0 || N <= 0) return FORGE_OK;
    if (!x || !w || !w_scale || !out || !scratch_q || !scratch_scale) return FORGE_EINVAL;
    hipStream_t s = as_stream(stream);
    int st = launch_quantize(x, scratch_q, scratch_scale, M, K, s);
    if (st != FORGE_OK) return st;
    return gemm_dense(scratch_q, w, scratch_scale, w_scale, bias, out, nullptr, M, K, N, s);
}
