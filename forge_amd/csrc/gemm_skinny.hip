// Decode-shape (M <= 16) dense INT8 GEMM for gfx950: weight streaming at HBM rate.
//
// The reference runs these shapes through the same 128-row wmma tile as large M
// (src/gemm/int8_dense.cu:200-210), wasting 7/8 of each tile. Here a workgroup owns 16
// weight rows and the whole K range; its 4 wavefronts split K (an intra-workgroup
// split-K, reduced exactly in INT32 through LDS, so no workspace and no atomics).
// v_mfma_i32_16x16x64_i8 takes the (<= 16) activation rows as operand A and 16 weight
// rows as operand B: lane l supplies row l%16 and the 32 K-bytes [32*(l/16), +32) of a
// 128-deep step, split over two MFMAs (bytes 0-15, then 16-31). A and B use the same
// (lane, byte) -> k assignment, so the dot products are exact whatever order the
// hardware uses inside a lane. Each lane keeps kUnroll steps of weight loads in flight.
// Accumulator layout of a 16x16 block (lane l, register e): row 4*(l/16)+e, col l%16.
#include "common.h"
#include "gemm_dense.h"

namespace forge_amd {

constexpr int kSkWaves = 4;
constexpr int kSkUnroll = 4;
constexpr int kSkStep = 128;   // K bytes per wave step

// 16 bytes at row[k], or zeros when k >= K (K % 16 == 0, so a chunk is all in or all out).
__device__ __forceinline__ int4 ld16_guard(const int8_t* row, int k, int K) {
    return (k < K) ? *reinterpret_cast<const int4*>(row + k) : make_int4(0, 0, 0, 0);
}

__device__ __forceinline__ v4i as_v4i(int4 v) {
    v4i r;
    r[0] = v.x; r[1] = v.y; r[2] = v.z; r[3] = v.w;
    return r;
}

template <bool DEQUANT>
__global__ __launch_bounds__(kSkWaves * kWave) void gemm_skinny_kernel(
    const int8_t* __restrict__ A, const int8_t* __restrict__ B, GemmEpilogue ep, int K)
{
    __shared__ v4i red[kSkWaves - 1][kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int n0 = blockIdx.x * 16;
    const int r = lane & 15;
    const int kq = 32 * (lane >> 4);
    const int M = ep.M, N = ep.N;
    const bool arow = r < M;
    const bool brow = (n0 + r) < N;
    const int8_t* pa = A + static_cast<size_t>(arow ? r : 0) * K;
    const int8_t* pb = B + static_cast<size_t>(brow ? n0 + r : n0) * K;

    v4i acc = {0, 0, 0, 0};
    const int steps = (K + kSkStep - 1) / kSkStep;
    for (int s0 = wave * kSkUnroll; s0 < steps; s0 += kSkWaves * kSkUnroll) {
        int4 wb[kSkUnroll][2], xa[kSkUnroll][2];
#pragma unroll
        for (int u = 0; u < kSkUnroll; u++) {
            const int kl = (s0 + u) * kSkStep + kq;
            wb[u][0] = brow ? ld16_guard(pb, kl, K) : make_int4(0, 0, 0, 0);
            wb[u][1] = brow ? ld16_guard(pb, kl + 16, K) : make_int4(0, 0, 0, 0);
            xa[u][0] = arow ? ld16_guard(pa, kl, K) : make_int4(0, 0, 0, 0);
            xa[u][1] = arow ? ld16_guard(pa, kl + 16, K) : make_int4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < kSkUnroll; u++) {
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_v4i(xa[u][0]), as_v4i(wb[u][0]), acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(as_v4i(xa[u][1]), as_v4i(wb[u][1]), acc, 0, 0, 0);
        }
    }

    if (wave > 0) red[wave - 1][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < kSkWaves - 1; w++) acc += red[w][lane];

    const int col = n0 + (lane & 15);
    if (col >= N) return;
    float ws = 0.0f, b = 0.0f;
    if constexpr (DEQUANT) {
        ws = h2f(ep.w_scale[col]);
        if (ep.bias) b = h2f(ep.bias[col]);
    }
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int row = 4 * (lane >> 4) + e;
        if (row >= M) continue;
        const size_t o = static_cast<size_t>(row) * N + col;
        if constexpr (DEQUANT)
            ep.c16[o] = dequant_gemm(acc[e], ep.act_scale[row], ws, b, ep.bias != nullptr);
        else
            ep.c32[o] = acc[e];
    }
}

int launch_gemm_skinny(const int8_t* A, const int8_t* B, const GemmEpilogue& ep, int M, int K, int N,
                       hipStream_t s)
{
    if (M > kSkinnyMaxM) return FORGE_EINVAL;
    const unsigned grid = static_cast<unsigned>(divup(N, 16));
    if (ep.c16)
        gemm_skinny_kernel<true><<<grid, kSkWaves * kWave, 0, s>>>(A, B, ep, K);
    else
        gemm_skinny_kernel<false><<<grid, kSkWaves * kWave, 0, s>>>(A, B, ep, K);
    return launch_status();
}

}  // namespace forge_amd
