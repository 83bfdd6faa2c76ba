// 2:4 structured-sparse INT8 GEMM for gfx950 on v_smfmac_i32_16x16x128_i8.
//
// Reference: src/gemm/int8_sparse.cu (persistent-CTA mma.sp.m16n8k64, 3-stage cp.async
// pipeline, FP32-atomic split-K, RTX-4090 cost model). Computes
//     Y[m,n] = half(fma(sum_k x[m,k] * Wp[n,k], act_scale[m] * w_scale[n], bias[n]))
// (int8_sparse.cu:659-661), Wp = the 2:4 weights given by W_comp (N,K/2) and w_meta.
//
// Operand roles: the SMFMAC sparse operand A is the compressed weight (16 weight rows x
// 128 dense K per instruction), operand B the activations (128 K x 16 tokens). The
// accumulator block is C[n][m]; lane l holds rows n = 4*(l/16)+e (e = 0..3) of token
// column m = l%16, i.e. 4 consecutive outputs of one row of Y -> one 8-byte FP16 (or
// 16-byte INT32) store.
// Lane operand ownership per 128-deep K step (lane l, g = l/16), as measured on gfx950 with
// one-hot operands:
//   A: 16 compressed bytes of weight row l%16 covering dense K [32g, 32g+32); compressed
//      byte pair q is the q-th group of 4 of that range
//   index: the lane's own VGPR, the reference metadata word (row l%16, 32-K chunk 4s+g):
//          nibble q (bits 4q..4q+3) holds the two kept positions of the q-th group
//   B: 32 bytes of token row l%16: bytes 0-15 = K [16g, 16g+16), bytes 16-31 =
//      K [64+16g, 64+16g+16) (two 64-deep halves, each in the dense 16x16x64 layout)
// pack_metadata stores exactly these words so that a wave's 64 index words are one
// contiguous 256-byte run (sparsity.hip).
//
// Split-K: each split adds its exact INT32 partial sum into the caller's (M,N)
// workspace with integer atomics (order-independent), then a finalize kernel applies
// the epilogue -- every split yields the same bits as split_k = 1 (the reference's
// FP32-atomic split-K is not deterministic, int8_sparse.cu:610-632).
#include "common.h"
#include "gemm_dense.h"
#include "mfma_tile.h"
#include "stream_slots.h"
#include "forge/gemm/int8_sparse.h"

#include <algorithm>
#include <mutex>
#include <cmath>
#include <type_traits>

namespace forge_amd {

constexpr int kSpStep = 128;        // dense K per stage
constexpr int kSpARow = 64;         // compressed bytes per weight row per stage
constexpr int kSpBRow = 128;        // activation bytes per token row per stage

// A rows: 64 B (4 chunks), same swizzle as the dense engine. B rows: 128 B (8 chunks),
// chunk position c ^ ((r ^ (r >> 3)) & 7): conflict free for the 16-row, same-chunk reads.
__device__ __forceinline__ int sp_a_off(int r, int c) { return r * kSpARow + ((c ^ (((r >> 1) ^ (r >> 3)) & 3)) << 4); }
__device__ __forceinline__ int sp_b_off(int r, int c) { return r * kSpBRow + ((c ^ ((r ^ (r >> 3)) & 7)) << 4); }

struct SparseArgs {
    const int8_t* W_comp;     // (N, K/2)
    const int8_t* x;          // (M, K)
    const uint32_t* meta;     // gfx950 layout
    const float* act_scale;
    const uint16_t* w_scale;
    const uint16_t* bias;
    uint16_t* out16;          // direct FP16 output (split == 1)
    int32_t* out32;           // direct INT32 output, or the split-K workspace
    int M, K, N;
    int split_k, steps_per_split;
    int tiles_n, tiles_m;
    int atomic;               // accumulate into out32 with atomics (split-K)
};

template <int BNW, int BMT, int WN, int WM>
struct SparseCfg {
    static constexpr int kThreads = WN * WM * kWave;
    static constexpr int kTN = BNW / WN / 16;   // 16-row weight blocks per wave
    static constexpr int kTM = BMT / WM / 16;   // 16-token blocks per wave
    static constexpr int kAChunks = BNW * 4 / kThreads;
    static constexpr int kBChunks = BMT * 8 / kThreads;
    static constexpr int kMetaInt4 = BNW;               // BNW/16 blocks x 16 int4 (64 words)
    static constexpr int kMChunks = (kMetaInt4 + kThreads - 1) / kThreads;
    static constexpr int kStageBytes = BNW * kSpARow + BMT * kSpBRow + BNW * 16;
    static constexpr int kLdsBytes = 2 * kStageBytes;
    static_assert(BNW * 4 % kThreads == 0 && BMT * 8 % kThreads == 0, "stage split");
};

template <int BNW, int BMT, int WN, int WM>
__global__ __launch_bounds__(WN * WM * kWave) void sparse_gemm_kernel(SparseArgs p)
{
    using Cfg = SparseCfg<BNW, BMT, WN, WM>;
    extern __shared__ __align__(16) int8_t lds[];
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;

    const int spatial = p.tiles_n * p.tiles_m;
    const int split = blockIdx.x / spatial;
    int tn, tm;
    tile_coords(blockIdx.x - split * spatial, p.tiles_n, p.tiles_m, tn, tm);
    const int n0 = tn * BNW, m0 = tm * BMT;
    const int steps_total = (p.K + kSpStep - 1) / kSpStep;
    const int s_begin = split * p.steps_per_split;
    const int s_end = min(s_begin + p.steps_per_split, steps_total);
    const int wn = (wave / WM) * (BNW / WN);
    const int wm = (wave % WM) * (BMT / WM);
    const int K = p.K, N = p.N, M = p.M;
    const int Kc = K >> 1, cpr = K >> 5;

    v4i acc[Cfg::kTN][Cfg::kTM];
#pragma unroll
    for (int i = 0; i < Cfg::kTN; i++)
#pragma unroll
        for (int j = 0; j < Cfg::kTM; j++) acc[i][j] = v4i{0, 0, 0, 0};

    if (s_begin < s_end) {
        int4 ra[Cfg::kAChunks], rb[Cfg::kBChunks], rm[Cfg::kMChunks];
        auto gload = [&](int s) {
            const int kd = s * kSpStep;          // dense K of this stage
            const int kc = kd >> 1;              // compressed K
#pragma unroll
            for (int i = 0; i < Cfg::kAChunks; i++) {
                const int id = tid + i * Cfg::kThreads;
                const int r = id >> 2, c = id & 3;
                const int n = n0 + r, k = kc + (c << 4);
                ra[i] = (n < N && k < Kc) ? *reinterpret_cast<const int4*>(p.W_comp + static_cast<size_t>(n) * Kc + k)
                                          : make_int4(0, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < Cfg::kBChunks; i++) {
                const int id = tid + i * Cfg::kThreads;
                const int r = id >> 3, c = id & 7;
                const int m = m0 + r, k = kd + (c << 4);
                rb[i] = (m < M && k < K) ? *reinterpret_cast<const int4*>(p.x + static_cast<size_t>(m) * K + k)
                                         : make_int4(0, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < Cfg::kMChunks; i++) {
                const int id = tid + i * Cfg::kThreads;     // int4 index within the stage
                const int blk = id >> 4, q = id & 15;       // 16 int4 = 64 words per 16-row block
                const int c = (kd >> 5) + (q >> 2);         // 32-K chunk of these 4 words
                const int n = n0 + blk * 16;
                rm[i] = (id < Cfg::kMetaInt4 && n < N && c < cpr)
                            ? *reinterpret_cast<const int4*>(p.meta + static_cast<size_t>(n >> 4) * cpr * 16 +
                                                             static_cast<size_t>(kd >> 5) * 16 + q * 4)
                            : make_int4(0, 0, 0, 0);
            }
        };
        auto lstore = [&](int buf) {
            int8_t* base = lds + buf * Cfg::kStageBytes;
            int8_t* As = base;
            int8_t* Bs = base + BNW * kSpARow;
            int8_t* Ms = Bs + BMT * kSpBRow;
#pragma unroll
            for (int i = 0; i < Cfg::kAChunks; i++) {
                const int id = tid + i * Cfg::kThreads;
                *reinterpret_cast<int4*>(As + sp_a_off(id >> 2, id & 3)) = ra[i];
            }
#pragma unroll
            for (int i = 0; i < Cfg::kBChunks; i++) {
                const int id = tid + i * Cfg::kThreads;
                *reinterpret_cast<int4*>(Bs + sp_b_off(id >> 3, id & 7)) = rb[i];
            }
#pragma unroll
            for (int i = 0; i < Cfg::kMChunks; i++) {
                const int id = tid + i * Cfg::kThreads;
                if (id < Cfg::kMetaInt4) *reinterpret_cast<int4*>(Ms + id * 16) = rm[i];
            }
        };

        gload(s_begin);
        lstore(0);
        __syncthreads();
        const int g = lane >> 4;
        const int r16 = lane & 15;
        for (int s = s_begin; s < s_end; s++) {
            const int cur = (s - s_begin) & 1;
            const bool more = (s + 1) < s_end;
            if (more) gload(s + 1);
            const int8_t* base = lds + cur * Cfg::kStageBytes;
            const int8_t* As = base;
            const int8_t* Bs = base + BNW * kSpARow;
            const uint32_t* Ms = reinterpret_cast<const uint32_t*>(Bs + BMT * kSpBRow);
            v4i fa[Cfg::kTN];
            int fi[Cfg::kTN];
#pragma unroll
            for (int i = 0; i < Cfg::kTN; i++) {
                const int r = wn + 16 * i + r16;
                fa[i] = *reinterpret_cast<const v4i*>(As + sp_a_off(r, g));
                fi[i] = static_cast<int>(Ms[((wn >> 4) + i) * 64 + lane]);
            }
#pragma unroll
            for (int j = 0; j < Cfg::kTM; j++) {
                const int r = wm + 16 * j + r16;
                const v4i b0 = *reinterpret_cast<const v4i*>(Bs + sp_b_off(r, g));
                const v4i b1 = *reinterpret_cast<const v4i*>(Bs + sp_b_off(r, g + 4));
                const v8i fb = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
#pragma unroll
                for (int i = 0; i < Cfg::kTN; i++)
                    acc[i][j] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(fa[i], fb, acc[i][j], fi[i], 0, 0);
            }
            if (more) lstore(cur ^ 1);
            __syncthreads();
        }
    }

    // Epilogue: lane holds C[n0+wn+16i+4*(l/16)+e][m0+wm+16j+l%16], e = 0..3.
    const int nq = 4 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < Cfg::kTM; j++) {
        const int m = m0 + wm + 16 * j + (lane & 15);
        if (m >= M) continue;
        const float as = p.out16 ? p.act_scale[m] : 0.0f;
#pragma unroll
        for (int i = 0; i < Cfg::kTN; i++) {
            const int n = n0 + wn + 16 * i + nq;
            if (n >= N) continue;                      // N % 16 == 0: 4 rows in or out together
            const size_t o = static_cast<size_t>(m) * N + n;
            if (p.atomic) {
#pragma unroll
                for (int e = 0; e < 4; e++) atomicAdd(p.out32 + o + e, acc[i][j][e]);
            } else if (p.out16) {
                float ws4[4], b4[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    ws4[e] = h2f(p.w_scale[n + e]);
                    b4[e] = p.bias ? h2f(p.bias[n + e]) : -0.0f;   // dequant4_pk: -0 without a bias
                }
                *reinterpret_cast<uint2*>(p.out16 + o) =
                    dequant4_pk(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3], as, ws4, b4);
            } else {
                *reinterpret_cast<int4*>(p.out32 + o) = make_int4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
            }
        }
    }
}

// Zero fill (graph-capture safe: a kernel, not a memset node).
__global__ __launch_bounds__(256) void zero_i32_kernel(int4* __restrict__ p, long long n4, int32_t* tail, int ntail)
{
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < n4; i += stride)
        p[i] = make_int4(0, 0, 0, 0);
    if (blockIdx.x == 0 && threadIdx.x < ntail) tail[threadIdx.x] = 0;
}

// Split-K finalize: INT32 sums -> FP16 with the GEMM epilogue.
__global__ __launch_bounds__(256) void splitk_finalize_kernel(
    const int32_t* __restrict__ ws, const float* __restrict__ act_scale, const uint16_t* __restrict__ w_scale,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int N, long long total)
{
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < total; i += stride) {
        const int m = static_cast<int>(i / N), n = static_cast<int>(i % N);
        out[i] = dequant_gemm(ws[i], act_scale[m], h2f(w_scale[n]), bias ? h2f(bias[n]) : 0.0f, bias != nullptr);
    }
}

// Reference splitk_reduce (int8_sparse.cu:99-111): fp32 workspace + bias -> fp16.
__global__ __launch_bounds__(256) void splitk_reduce_f32_kernel(
    const float* __restrict__ ws, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int N, long long total)
{
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < total; i += stride) {
        float v = ws[i];
        if (bias) v += h2f(bias[i % N]);
        out[i] = f2h(v);
    }
}

// Four columns per thread (N % 4 == 0, 16-byte workspace, 8-byte out and bias, M * N / 4 <
// 2^31): the same sums as splitk_reduce_f32_kernel, one 16-byte load, one 8-byte bias load and
// one 8-byte store per thread. Unsigned index: total4 < 2^31 plus a stride of at most 2^22
// stays below 2^32, so the last increment cannot wrap.
__global__ __launch_bounds__(256) void splitk_reduce_vec4_kernel(
    const float4* __restrict__ ws, const uint16_t* __restrict__ bias, uint2* __restrict__ out, uint32_t n4,
    uint32_t total4)
{
    // total4 < 2^31 and stride <= 16384 * 256 = 2^22 (host guards), so i + stride < 2^32: the
    // unsigned counter never wraps.
    const uint32_t stride = gridDim.x * 256u;
    for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < total4; i += stride) {
        const float4 f = ws[i];
        float v[4] = {f.x, f.y, f.z, f.w};
        if (bias) {
            const uint32_t n = (i - (i / n4) * n4) * 4;
            const uint2 bv = *reinterpret_cast<const uint2*>(bias + n);
            const uint32_t br[4] = {bv.x & 0xFFFFu, bv.x >> 16, bv.y & 0xFFFFu, bv.y >> 16};
#pragma unroll
            for (int j = 0; j < 4; j++) v[j] += h2f(static_cast<uint16_t>(br[j]));
        }
        out[i] = make_uint2(f2h(v[0]) | (static_cast<uint32_t>(f2h(v[1])) << 16),
                            f2h(v[2]) | (static_cast<uint32_t>(f2h(v[3])) << 16));
    }
}

// ---- DMA-fed sparse engine (256 weight rows x BMT tokens, 128-deep dense K stages) -------
//
// The operands stream into a 2-slot LDS ring with global_load_lds_dwordx4 (mfma_tile.h):
//   W: 256 weight rows x 64 compressed bytes (4 chunks; chunk c of row r at c ^ lds_swz4(r))
//   X: BMT token rows x 128 bytes (one cache line; chunk c of row r at c ^ lds_swz8(r))
//   I: 16 blocks x 64 index words, word (32-K chunk g, row r) of block b at b*64 + g*16 + r --
//      the order pack_metadata stores them in HBM, so the DMA copies them verbatim and lane
//      l of every SMFMAC reads word l of its block.
// Each wave owns 128 weight rows x BMT/2 tokens: 8 x (BMT/32) blocks of
// v_smfmac_i32_16x16x128_i8 (one per block per stage). A stage's token blocks are split in
// two halves: the second half's operands are read while the first half's SMFMACs run, and
// the next stage's weights, indices and first-half tokens while the second half runs, on the
// far side of the barrier that publishes the next stage.

// The sparse GEMM operands as buffer resources: compressed weights (N x K/2 bytes), tokens
// (M x K) and index words (N x K/8 bytes). The host keeps every size under 2^31.
struct SpBufs {
    __amdgpu_buffer_rsrc_t w, x, i;
};
__device__ __forceinline__ SpBufs sp_bufs(const int8_t* W, const int8_t* X, const uint32_t* meta, int M, int N, int K)
{
    const uint32_t n = static_cast<uint32_t>(N), m = static_cast<uint32_t>(M), k = static_cast<uint32_t>(K);
    return SpBufs{buf_rsrc(W, n * (k / 2)), buf_rsrc(X, m * k), buf_rsrc(meta, n * (k / 8))};
}

template <int BMT, int BNW_ = 256>
struct SpDmaTile {
    static constexpr int BNW = BNW_;                   // 256, or 128 for twice the tiles
    static constexpr int kTN = BNW / 2 / 16;           // weight blocks per wave
    static constexpr int kTM = BMT / 2 / 16;           // token blocks per wave
    static constexpr int kTH = kTM / 2;                // token blocks per half
    static constexpr int kWBytes = BNW * 64;
    static constexpr int kXBytes = BMT * 128;
    static constexpr int kIBytes = BNW / 16 * 256;
    static constexpr int kSlotBytes = kWBytes + kXBytes + kIBytes;
    static constexpr int kLdsBytes = 2 * kSlotBytes;
    static constexpr int kWIns = BNW * 4 / kWave / 4;   // 1 KB DMA instructions per wave per stage
    static constexpr int kXIns = BMT * 8 / kWave / 4;
    static constexpr int kILanes = kIBytes / 16 / 4;    // lanes of a wave copying 16 index bytes each
    static_assert(BNW == 128 || BNW == 256, "weight rows per tile");
    static_assert(kILanes == 32 || kILanes == 64, "one index DMA instruction per wave");
    static_assert(kTH >= 1, "tile too small");

    v4i acc[kTN][kTM];   // acc[i][j]: C[n: 16i + 4*(l/16) + e][m: 16j + l%16]

    struct WFrag { v4i a[kTN]; int idx[kTN]; };
    struct XFrag { v8i b[kTH]; };

    __device__ __forceinline__ void run(const int8_t* W, const int8_t* X, const uint32_t* meta, int M, int N,
                                        int K, int n0, int m0, int8_t* lds) {
        const int lane = threadIdx.x & (kWave - 1);
        const int wave = threadIdx.x / kWave;
        const int wn = (wave >> 1) * (BNW / 2);
        const int wm = (wave & 1) * (BMT / 2);
        const int r16 = lane & 15, g = lane >> 4;
        const int Kc = K >> 1, cpr = K >> 5;

#pragma unroll
        for (int i = 0; i < kTN; i++)
#pragma unroll
            for (int j = 0; j < kTM; j++) acc[i][j] = v4i{0, 0, 0, 0};

        // The three operands as buffer resources (sizes < 2^31, checked by the host): a lane's
        // offsets are fixed, a stage's K offset is the scalar offset of its DMAs.
        const SpBufs bf = sp_bufs(W, X, meta, M, N, K);
        uint32_t ow[kWIns], ox[kXIns];
#pragma unroll
        for (int q = 0; q < kWIns; q++) {
            const int s = (wave * kWIns + q) * kWave + lane;
            const int r = s >> 2, c = (s & 3) ^ lds_swz4(r);
            const int gr = (n0 + r) < N ? (n0 + r) : N - 1;
            ow[q] = static_cast<uint32_t>(gr) * Kc + 16 * c;
        }
#pragma unroll
        for (int q = 0; q < kXIns; q++) {
            const int s = (wave * kXIns + q) * kWave + lane;
            const int r = s >> 3, c = (s & 7) ^ lds_swz8(r);
            const int gr = (m0 + r) < M ? (m0 + r) : M - 1;
            ox[q] = static_cast<uint32_t>(gr) * K + 16 * c;
        }
        uint32_t oi;
        {
            const int s = wave * kILanes + (lane & (kILanes - 1));   // 16-byte chunk of the stage's index area
            int b = (n0 >> 4) + (s >> 4);
            b = b < (N >> 4) ? b : (N >> 4) - 1;
            oi = static_cast<uint32_t>(b) * cpr * 64 + 16 * (s & 15);
        }
        const int nst = K / 128;
        auto issue = [&](int st) {
            int8_t* slot = lds + (st & 1) * kSlotBytes;
            const uint32_t sc = st < nst ? st : nst - 1;  // past the end: re-read (dead slot)
#pragma unroll
            for (int q = 0; q < kWIns; q++) dma16_buf(bf.w, ow[q], sc * 64, slot + (wave * kWIns + q) * 1024);
#pragma unroll
            for (int q = 0; q < kXIns; q++) dma16_buf(bf.x, ox[q], sc * 128, slot + kWBytes + (wave * kXIns + q) * 1024);
            if (kILanes == kWave || lane < kILanes)
                dma16_buf(bf.i, oi, sc * 256, slot + kWBytes + kXBytes + wave * (16 * kILanes));
        };
        auto load_w = [&](int st, WFrag& F) {
            const int8_t* Ws = lds + (st & 1) * kSlotBytes;
            const uint32_t* Is = reinterpret_cast<const uint32_t*>(Ws + kWBytes + kXBytes);
#pragma unroll
            for (int i = 0; i < kTN; i++) {
                const int r = wn + 16 * i + r16;
                F.a[i] = *reinterpret_cast<const v4i*>(Ws + lds_off64(r, g));
                F.idx[i] = static_cast<int>(Is[((wn >> 4) + i) * 64 + lane]);
            }
        };
        auto load_x = [&](int st, int half, XFrag& F) {
            const int8_t* Xs = lds + (st & 1) * kSlotBytes + kWBytes;
#pragma unroll
            for (int j = 0; j < kTH; j++) {
                const int r = wm + 16 * (half * kTH + j) + r16;
                const v4i lo = *reinterpret_cast<const v4i*>(Xs + lds_off128(r, g));
                const v4i hi = *reinterpret_cast<const v4i*>(Xs + lds_off128(r, g + 4));
                F.b[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
            }
        };
        auto smfmacs = [&](const WFrag& Wf, const XFrag& Xf, int half) {
#pragma unroll
            for (int j = 0; j < kTH; j++)
#pragma unroll
                for (int i = 0; i < kTN; i++)
                    acc[i][half * kTH + j] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(
                        Wf.a[i], Xf.b[j], acc[i][half * kTH + j], Wf.idx[i], 0, 0);
        };
        constexpr int kMf = kTN * kTH;
        constexpr int kRdW = 2 * kTN, kRdX = 2 * kTH, kVm = kWIns + kXIns + 1;
        // One stage: first half with (Wc, Xlo), second half with (Wc, Xhi) after the barrier
        // that publishes stage kt+1, whose operands (Wn, Xlo) load meanwhile.
        auto stage = [&](int kt, WFrag& Wc, WFrag& Wn, XFrag& Xlo, XFrag& Xhi) {
            load_x(kt, 1, Xhi);
            smfmacs(Wc, Xlo, 0);
            sched_interleave<kMf, kRdX, 0>();
            wait_vm_lgkm0();
            lds_barrier();
            issue(kt + 2);
            load_w(kt + 1, Wn);
            load_x(kt + 1, 0, Xlo);
            smfmacs(Wc, Xhi, 1);
            sched_interleave<kMf / 2, 0, kVm>();
            sched_interleave<kMf / 2, kRdW + kRdX, 0>();
        };

        issue(0);
        wait_vm_lgkm0();
        lds_barrier();
        issue(1);
        WFrag W0, W1;
        XFrag Xlo, Xhi;
        load_w(0, W0);
        load_x(0, 0, Xlo);
        int kt = 0;
        for (; kt + 2 < nst; kt += 2) {
            stage(kt, W0, W1, Xlo, Xhi);
            stage(kt + 1, W1, W0, Xlo, Xhi);
        }
        if (kt + 1 < nst) {                  // two stages left: kt, kt+1
            stage(kt, W0, W1, Xlo, Xhi);
            load_x(kt + 1, 1, Xhi);
            smfmacs(W1, Xlo, 0);
            smfmacs(W1, Xhi, 1);
        } else {                             // one stage left: kt
            load_x(kt, 1, Xhi);
            smfmacs(W0, Xlo, 0);
            smfmacs(W0, Xhi, 1);
        }
        wait_vm_lgkm0();
        lds_barrier();
    }
};

// Same ring, v_smfmac_i32_32x32x64_i8 (256 weight rows x 256 tokens per workgroup; each wave
// 128 tokens x 128 weight rows = 4 x 4 blocks of 32x32 INT32 accumulators, the dense engine's
// layout, so the dense epilogue store_tile writes it). Lane layout measured on gfx950 with
// one-hot operands: A lane l holds compressed bytes of weight row l%32 covering dense K
// [32*(l/32), +32) of the 64-deep step, pair q = group q, indexed by nibble q of the lane's
// own word; B lane l holds token l%32, bytes 0-15 = K [16*(l/32), +16) and bytes 16-31 =
// K [32 + 16*(l/32), +16); the accumulator is the 32x32 MFMA layout (row = weight).
// BMT_ (tokens per tile) is 256, or 192 for the tail wave of sparse_dma32_tail_kernel.
template <int BMT_>
struct SpDmaTile32B {
    static constexpr int BNW = 256, BMT = BMT_;
    static_assert(BMT % 64 == 0, "two waves of 32-token blocks");
    static constexpr int kTN = 4, kTM = BMT / 64;      // 32-row weight / 32-token blocks per wave
    static constexpr int kWBytes = BNW * 64;
    static constexpr int kXBytes = BMT * 128;
    static constexpr int kIBytes = BNW / 16 * 256;
    static constexpr int kSlotBytes = kWBytes + kXBytes + kIBytes;
    static constexpr int kLdsBytes = 2 * kSlotBytes;
    static constexpr int kWIns = BNW * 4 / kWave / 4;
    static constexpr int kXIns = BMT * 8 / kWave / 4;

    v16i acc[kTN][kTM];   // acc[j][i]: D[n: 32j + row(e, l)][m: 32i + l%32]

    struct Frags { v4i a[kTN]; int idx[kTN]; v8i b[kTM]; };

    __device__ __forceinline__ void run(const int8_t* W, const int8_t* X, const uint32_t* meta, int M, int N,
                                        int K, int n0, int m0, int8_t* lds) {
        const int lane = threadIdx.x & (kWave - 1);
        const int wave = threadIdx.x / kWave;
        const int wm = (wave >> 1) * (BMT / 2);        // token offset (dense engine's wave layout)
        const int wn = (wave & 1) * (BNW / 2);         // weight offset
        const int l31 = lane & 31, g = lane >> 5;
        const int Kc = K >> 1, cpr = K >> 5;

#pragma unroll
        for (int j = 0; j < kTN; j++)
#pragma unroll
            for (int i = 0; i < kTM; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) acc[j][i][e] = 0;

        const SpBufs bf = sp_bufs(W, X, meta, M, N, K);
        uint32_t ow[kWIns], ox[kXIns];
#pragma unroll
        for (int q = 0; q < kWIns; q++) {
            const int s = (wave * kWIns + q) * kWave + lane;
            const int r = s >> 2, c = (s & 3) ^ lds_swz4(r);
            const int gr = (n0 + r) < N ? (n0 + r) : N - 1;
            ow[q] = static_cast<uint32_t>(gr) * Kc + 16 * c;
        }
#pragma unroll
        for (int q = 0; q < kXIns; q++) {
            const int s = (wave * kXIns + q) * kWave + lane;
            const int r = s >> 3, c = (s & 7) ^ lds_swz8(r);
            const int gr = (m0 + r) < M ? (m0 + r) : M - 1;
            ox[q] = static_cast<uint32_t>(gr) * K + 16 * c;
        }
        // Index words: LDS chunk position s (16 blocks x 16 chunks of 4 words) takes chunk
        // (s % 16) ^ 12 of its block in odd blocks (read below as word w ^ 48). The 16-lane
        // groups of an index read (block parity x g) then start at banks {0, 48, 16, 32}
        // (+32 for the odd step): distinct over all 64 lanes and within each 32-lane half.
        uint32_t oi;
        {
            const int s = wave * kWave + lane;
            int b = (n0 >> 4) + (s >> 4);
            b = b < (N >> 4) ? b : (N >> 4) - 1;
            const int k = (s & 15) ^ (((s >> 4) & 1) * 12);
            oi = static_cast<uint32_t>(b) * cpr * 64 + 16 * k;
        }
        const int nst = K / 128;
        auto issue = [&](int st) {
            int8_t* slot = lds + (st & 1) * kSlotBytes;
            const uint32_t sc = st < nst ? st : nst - 1;
#pragma unroll
            for (int q = 0; q < kWIns; q++) dma16_buf(bf.w, ow[q], sc * 64, slot + (wave * kWIns + q) * 1024);
#pragma unroll
            for (int q = 0; q < kXIns; q++) dma16_buf(bf.x, ox[q], sc * 128, slot + kWBytes + (wave * kXIns + q) * 1024);
            dma16_buf(bf.i, oi, sc * 256, slot + kWBytes + kXBytes + wave * 1024);
        };
        // Sub-step h (dense K [64h, 64h+64) of the stage).
        auto load = [&](int st, int h, Frags& F) {
            const int8_t* Ws = lds + (st & 1) * kSlotBytes;
            const int8_t* Xs = Ws + kWBytes;
            const uint32_t* Is = reinterpret_cast<const uint32_t*>(Xs + kXBytes);
#pragma unroll
            for (int j = 0; j < kTN; j++) {
                const int r = wn + 32 * j + l31;
                F.a[j] = *reinterpret_cast<const v4i*>(Ws + lds_off64(r, 2 * h + g));
                const int w = ((2 * h + g) * 16 + (r & 15)) ^ (((r >> 4) & 1) * 48);
                F.idx[j] = static_cast<int>(Is[(r >> 4) * 64 + w]);
            }
#pragma unroll
            for (int i = 0; i < kTM; i++) {
                const int r = wm + 32 * i + l31;
                const v4i lo = *reinterpret_cast<const v4i*>(Xs + lds_off128(r, 4 * h + g));
                const v4i hi = *reinterpret_cast<const v4i*>(Xs + lds_off128(r, 4 * h + 2 + g));
                F.b[i] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
            }
        };
        auto smfmacs = [&](const Frags& F) {
#pragma unroll
            for (int j = 0; j < kTN; j++)
#pragma unroll
                for (int i = 0; i < kTM; i++)
                    acc[j][i] = __builtin_amdgcn_smfmac_i32_32x32x64_i8(F.a[j], F.b[i], acc[j][i], F.idx[j], 0, 0);
        };
        constexpr int kMf = kTN * kTM, kRd = 2 * kTN + 2 * kTM, kVm = kWIns + kXIns + 1;
        // Stage kt: sub-step 0 with F0 while sub-step 1 loads into F1; barrier publishing
        // stage kt+1; sub-step 1 with F1 while stage kt+1's sub-step 0 loads into F0.
        auto stage = [&](int kt, Frags& F0, Frags& F1) {
            load(kt, 1, F1);
            smfmacs(F0);
            sched_interleave<kMf, kRd, 0>();
            wait_vm_lgkm0();
            lds_barrier();
            issue(kt + 2);
            load(kt + 1, 0, F0);
            smfmacs(F1);
            sched_interleave<kMf / 2, 0, kVm>();
            sched_interleave<kMf / 2, kRd, 0>();
        };
        issue(0);
        wait_vm_lgkm0();
        lds_barrier();
        issue(1);
        Frags F0, F1;
        load(0, 0, F0);
        for (int kt = 0; kt + 1 < nst; kt++) stage(kt, F0, F1);
        load(nst - 1, 1, F1);
        smfmacs(F0);
        smfmacs(F1);
        wait_vm_lgkm0();
        lds_barrier();
    }
};

// SpDmaTile32 with 256-deep weight stages (K % 256 == 0): each compressed weight row's 128
// bytes covering two dense 128-deep stages arrive as one full cache line (one 128-byte
// request instead of two 64-byte ones), every other stage, into a 2-slot weight ring of its
// own; tokens and index words keep their per-stage 2-slot rings. A stage's L2 requests go from
// 256 (tokens) + 256 (weights, 64 B) + 32 (index) to 256 + 128 + 32 on average. Weight rows use
// the token rows' 128-byte swizzle (lds_off128), the half of stage kt being chunks 4 (kt & 1) ..
// 4 (kt & 1) + 3. Slot reuse: the weights of stages (kt + 2, kt + 3) are issued at stage kt's
// barrier (kt even); their slot held stages (kt - 2, kt - 1), last read before stage kt - 1's
// barrier.
template <int BMT_>
struct SpDmaTile32WB {
    static constexpr int BNW = 256, BMT = BMT_;
    static_assert(BMT % 64 == 0, "two waves of 32-token blocks");
    static constexpr int kTN = 4, kTM = BMT / 64;
    static constexpr int kWBytes = BNW * 128;          // one weight slot: two stages
    static constexpr int kXBytes = BMT * 128;
    static constexpr int kIBytes = BNW / 16 * 256;
    static constexpr int kXOff = 2 * kWBytes;
    static constexpr int kIOff = kXOff + 2 * kXBytes;
    static constexpr int kLdsBytes = kIOff + 2 * kIBytes;
    static constexpr int kWIns = BNW * 8 / kWave / 4;   // 1 KB DMA instructions per wave per weight slot
    static constexpr int kXIns = BMT * 8 / kWave / 4;

    v16i acc[kTN][kTM];   // acc[j][i]: D[n: 32j + row(e, l)][m: 32i + l%32]

    struct Frags { v4i a[kTN]; int idx[kTN]; v8i b[kTM]; };

    __device__ __forceinline__ void run(const int8_t* W, const int8_t* X, const uint32_t* meta, int M, int N,
                                        int K, int n0, int m0, int8_t* lds) {
        const int lane = threadIdx.x & (kWave - 1);
        const int wave = threadIdx.x / kWave;
        const int wm = (wave >> 1) * (BMT / 2);
        const int wn = (wave & 1) * (BNW / 2);
        const int l31 = lane & 31, g = lane >> 5;
        const int Kc = K >> 1, cpr = K >> 5;

#pragma unroll
        for (int j = 0; j < kTN; j++)
#pragma unroll
            for (int i = 0; i < kTM; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) acc[j][i][e] = 0;

        // 32-bit byte offsets into buffer resources (the launcher checks N * K / 2 and M * K
        // < 2^31): one VGPR per load instead of a 64-bit address, which the 256 accumulators
        // leave no room for; the stage offset goes in the instruction's scalar offset.
        uint32_t ow[kWIns], ox[kXIns];
#pragma unroll
        for (int q = 0; q < kWIns; q++) {
            const int s = (wave * kWIns + q) * kWave + lane;
            const int r = s >> 3, c = (s & 7) ^ lds_swz8(r);
            const int gr = (n0 + r) < N ? (n0 + r) : N - 1;
            ow[q] = static_cast<uint32_t>(gr) * static_cast<uint32_t>(Kc) + 16 * c;
        }
#pragma unroll
        for (int q = 0; q < kXIns; q++) {
            const int s = (wave * kXIns + q) * kWave + lane;
            const int r = s >> 3, c = (s & 7) ^ lds_swz8(r);
            const int gr = (m0 + r) < M ? (m0 + r) : M - 1;
            ox[q] = static_cast<uint32_t>(gr) * static_cast<uint32_t>(K) + 16 * c;
        }
        uint32_t oi;
        {
            const int s = wave * kWave + lane;
            int b = (n0 >> 4) + (s >> 4);
            b = b < (N >> 4) ? b : (N >> 4) - 1;
            const int k = (s & 15) ^ (((s >> 4) & 1) * 12);
            oi = static_cast<uint32_t>(b) * static_cast<uint32_t>(cpr) * 64u + 16u * k;
        }
        const __amdgpu_buffer_rsrc_t rw = buf_rsrc(W, static_cast<uint32_t>(N) * static_cast<uint32_t>(Kc));
        const __amdgpu_buffer_rsrc_t rx = buf_rsrc(X, static_cast<uint32_t>(M) * static_cast<uint32_t>(K));
        const __amdgpu_buffer_rsrc_t ri = buf_rsrc(meta, static_cast<uint32_t>(N) * static_cast<uint32_t>(cpr) * 4u);
        const int nst = K / 128;   // even
        // Stage st's tokens and index words; at even st also the weights of st and st + 1.
        auto issue = [&](int st, bool with_w) {
            const int sc = st < nst ? st : nst - 1;       // past the end: re-read (dead slot)
            if (with_w) {
                const int sw = st < nst ? st : nst - 2;
                int8_t* wslot = lds + ((st >> 1) & 1) * kWBytes;
#pragma unroll
                for (int q = 0; q < kWIns; q++)
                    dma16_buf(rw, ow[q], static_cast<uint32_t>(sw * 64), wslot + (wave * kWIns + q) * 1024);
            }
            int8_t* xslot = lds + kXOff + (st & 1) * kXBytes;
#pragma unroll
            for (int q = 0; q < kXIns; q++)
                dma16_buf(rx, ox[q], static_cast<uint32_t>(sc * 128), xslot + (wave * kXIns + q) * 1024);
            dma16_buf(ri, oi, static_cast<uint32_t>(sc * 256), lds + kIOff + (st & 1) * kIBytes + wave * 1024);
        };
        auto load = [&](int st, int h, Frags& F) {
            const int8_t* Ws = lds + ((st >> 1) & 1) * kWBytes;
            const int8_t* Xs = lds + kXOff + (st & 1) * kXBytes;
            const uint32_t* Is = reinterpret_cast<const uint32_t*>(lds + kIOff + (st & 1) * kIBytes);
            const int wc = 4 * (st & 1) + 2 * h + g;
#pragma unroll
            for (int j = 0; j < kTN; j++) {
                const int r = wn + 32 * j + l31;
                F.a[j] = *reinterpret_cast<const v4i*>(Ws + lds_off128(r, wc));
                const int w = ((2 * h + g) * 16 + (r & 15)) ^ (((r >> 4) & 1) * 48);
                F.idx[j] = static_cast<int>(Is[(r >> 4) * 64 + w]);
            }
#pragma unroll
            for (int i = 0; i < kTM; i++) {
                const int r = wm + 32 * i + l31;
                const v4i lo = *reinterpret_cast<const v4i*>(Xs + lds_off128(r, 4 * h + g));
                const v4i hi = *reinterpret_cast<const v4i*>(Xs + lds_off128(r, 4 * h + 2 + g));
                F.b[i] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
            }
        };
        auto smfmacs = [&](const Frags& F) {
#pragma unroll
            for (int j = 0; j < kTN; j++)
#pragma unroll
                for (int i = 0; i < kTM; i++)
                    acc[j][i] = __builtin_amdgcn_smfmac_i32_32x32x64_i8(F.a[j], F.b[i], acc[j][i], F.idx[j], 0, 0);
        };
        constexpr int kMf = kTN * kTM, kRd = 2 * kTN + 2 * kTM;
        // Stage kt as in SpDmaTile32; EVEN: kt is even, so the weights of kt + 2, kt + 3 are
        // issued with the tokens of kt + 2.
        auto stage = [&](int kt, Frags& F0, Frags& F1, auto even) {
            constexpr bool EVEN = decltype(even)::value;
            constexpr int kVm = kXIns + 1 + (EVEN ? kWIns : 0);
            load(kt, 1, F1);
            smfmacs(F0);
            sched_interleave<kMf, kRd, 0>();
            wait_vm_lgkm0();
            lds_barrier();
            issue(kt + 2, EVEN);
            load(kt + 1, 0, F0);
            smfmacs(F1);
            sched_interleave<kMf / 2, 0, kVm>();
            sched_interleave<kMf / 2, kRd, 0>();
        };
        issue(0, true);
        wait_vm_lgkm0();
        lds_barrier();
        issue(1, false);
        Frags F0, F1;
        load(0, 0, F0);
        int kt = 0;
        for (; kt + 2 < nst; kt += 2) {
            stage(kt, F0, F1, std::true_type{});
            stage(kt + 1, F0, F1, std::false_type{});
        }
        stage(kt, F0, F1, std::true_type{});   // kt = nst - 2
        load(nst - 1, 1, F1);
        smfmacs(F0);
        smfmacs(F1);
        wait_vm_lgkm0();
        lds_barrier();
    }
};

using SpDmaTile32 = SpDmaTile32B<256>;
using SpDmaTile32W = SpDmaTile32WB<256>;

template <bool DEQUANT, class Tile>
__global__ __launch_bounds__(256) void sparse_dma32_kernel(const int8_t* __restrict__ W, const int8_t* __restrict__ X,
                                                           const uint32_t* __restrict__ meta, GemmEpilogue ep,
                                                           int tiles_n, int tiles_m, int K)
{
    extern __shared__ __align__(16) int8_t lds[];
    int tn, tm;
    tile_coords(blockIdx.x, tiles_n, tiles_m, tn, tm);
    const int n0 = tn * 256, m0 = tm * 256;
    Tile t;
    t.run(W, X, meta, ep.M, ep.N, K, n0, m0, lds);
    store_tile<256, 256, DEQUANT>(t.acc, ep, m0, n0, lds);
}

template <bool DEQUANT, class Tile>
static int launch_sparse_dma32_tile(const int8_t* W, const int8_t* X, const uint32_t* meta, const GemmEpilogue& ep,
                                    int K, hipStream_t s)
{
    constexpr int epi = epilogue_lds_bytes<256, 256, DEQUANT>();
    constexpr int lds = Tile::kLdsBytes > epi ? Tile::kLdsBytes : epi;
    const int tiles_n = divup(ep.N, 256), tiles_m = divup(ep.M, 256);
    const long long total = static_cast<long long>(tiles_n) * tiles_m;
    if (total > 0x7FFFFFFFLL) return FORGE_EINVAL;
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&sparse_dma32_kernel<DEQUANT, Tile>), hipFuncAttributeMaxDynamicSharedMemorySize,
        lds);
    if (attr != hipSuccess) return static_cast<int>(attr);
    sparse_dma32_kernel<DEQUANT, Tile><<<static_cast<unsigned>(total), 256, lds, s>>>(W, X, meta, ep, tiles_n, tiles_m,
                                                                                      K);
    return launch_status();
}

// The tail split in one launch: workgroups [0, n1) run the whole waves as 256 x 256 tiles over
// the first nb1 weight blocks, the rest the remaining weight blocks as one wave of 192-token
// tiles. configs[2] (4096 x 11008 x 4096): 688 tiles on 256 CUs are 2.69 waves, of which the
// third runs 69 % full; as 512 tiles + 242 tiles of 192 tokens it takes 2 + ~0.85 tile times.
template <bool DEQUANT, int BMT2, template <int> class TileT>
__global__ __launch_bounds__(256) void sparse_dma32_tail_kernel(const int8_t* __restrict__ W,
                                                                const int8_t* __restrict__ X,
                                                                const uint32_t* __restrict__ meta, GemmEpilogue ep,
                                                                int n1, int nb1, int tiles_n, int tiles_m,
                                                                int tiles_m2, int K)
{
    extern __shared__ __align__(16) int8_t lds[];
    int tn, tm;
    if (static_cast<int>(blockIdx.x) < n1) {
        tile_coords(blockIdx.x, nb1, tiles_m, tn, tm);
        TileT<256> t;
        t.run(W, X, meta, ep.M, ep.N, K, tn * 256, tm * 256, lds);
        store_tile<256, 256, DEQUANT>(t.acc, ep, tm * 256, tn * 256, lds);
    } else {
        tile_coords(static_cast<int>(blockIdx.x) - n1, tiles_n - nb1, tiles_m2, tn, tm);
        const int n0 = (nb1 + tn) * 256, m0 = tm * BMT2;
        TileT<BMT2> t;
        t.run(W, X, meta, ep.M, ep.N, K, n0, m0, lds);
        store_tile<BMT2, 256, DEQUANT>(t.acc, ep, m0, n0, lds);
    }
}

// Runs the tail split when the grid is more than one wave, not whole waves, its token tiles
// divide the CU count (so whole waves are whole weight blocks) and the remaining weight blocks
// fit one wave of 192-token tiles; -1 otherwise.
template <bool DEQUANT, template <int> class TileT>
static int launch_sparse_dma32_tail(const int8_t* W, const int8_t* X, const uint32_t* meta, const GemmEpilogue& ep,
                                    int K, hipStream_t s)
{
    constexpr int kTail = 192;
    int st = FORGE_OK;
    const int cu = device_info(&st).cu_count;
    if (st != FORGE_OK || cu <= 0) return -1;
    const int tiles_n = divup(ep.N, 256), tiles_m = divup(ep.M, 256);
    const long long tiles = static_cast<long long>(tiles_n) * tiles_m;
    if (tiles <= cu || tiles % cu == 0 || cu % tiles_m != 0 || ep.M < kTail) return -1;
    const int nb1 = static_cast<int>((tiles / cu) * cu / tiles_m);
    const int tiles_m2 = divup(ep.M, kTail);
    const long long tail = static_cast<long long>(tiles_n - nb1) * tiles_m2;
    if (nb1 <= 0 || nb1 >= tiles_n || tail > cu) return -1;
    constexpr int e1 = epilogue_lds_bytes<256, 256, DEQUANT>(), e2 = epilogue_lds_bytes<kTail, 256, DEQUANT>();
    constexpr int l1 = TileT<256>::kLdsBytes > e1 ? TileT<256>::kLdsBytes : e1;
    constexpr int l2 = TileT<kTail>::kLdsBytes > e2 ? TileT<kTail>::kLdsBytes : e2;
    constexpr int lds = l1 > l2 ? l1 : l2;
    auto kern = sparse_dma32_tail_kernel<DEQUANT, kTail, TileT>;
    static const hipError_t attr =
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (attr != hipSuccess) return static_cast<int>(attr);
    const int n1 = nb1 * tiles_m;
    kern<<<static_cast<unsigned>(n1 + tail), 256, lds, s>>>(W, X, meta, ep, n1, nb1, tiles_n, tiles_m, tiles_m2, K);
    note_route("dma256x256+tail192");
    return launch_status();
}

// 256 x 256 SMFMAC engine: 256-deep weight stages (full 128-byte lines) for INT32 outputs when
// K % 256 == 0 (configs[2]: 175 -> 160 us, measured in one run); the FP16 epilogue's registers
// do not fit beside them (the kernel spills), so dequantizing outputs keep 128-deep stages.
template <bool DEQUANT>
static int launch_sparse_dma32(const int8_t* W, const int8_t* X, const uint32_t* meta, const GemmEpilogue& ep,
                               int K, hipStream_t s)
{
    if constexpr (!DEQUANT) {
        if (K % 256 == 0 && static_cast<long long>(ep.N) * (K / 2) < (1LL << 31) &&
            static_cast<long long>(ep.M) * K < (1LL << 31) && static_cast<long long>(ep.N) * (K / 32) * 4 < (1LL << 31)) {
            const int r = launch_sparse_dma32_tail<DEQUANT, SpDmaTile32WB>(W, X, meta, ep, K, s);
            if (r != -1) return r;
            return launch_sparse_dma32_tile<DEQUANT, SpDmaTile32W>(W, X, meta, ep, K, s);
        }
    }
    const int r = launch_sparse_dma32_tail<DEQUANT, SpDmaTile32B>(W, X, meta, ep, K, s);
    if (r != -1) return r;
    return launch_sparse_dma32_tile<DEQUANT, SpDmaTile32>(W, X, meta, ep, K, s);
}

// Epilogue of a SpDmaTile: lane l of block (i, j) holds outputs (m = 16j + l%16, n = 16i +
// 4*(l/16) + e), 4 consecutive columns. FP16: the wave's whole (BMT/2) x 128 tile is staged in
// LDS; INT32: one 16-row strip per token block. Rows are flushed with 16-byte stores.
template <int BMT, bool DEQUANT, int BNW = 256>
__device__ __forceinline__ void sp_store_tile(const v4i (&acc)[BNW / 32][BMT / 32], const GemmEpilogue& ep, int n0,
                                              int m0, int8_t* lds) {
    constexpr int kTN = BNW / 32, kTM = BMT / 32;
    constexpr int kWN = BNW / 2;                             // output columns per wave
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int wn = n0 + (wave >> 1) * kWN;
    const int wm = m0 + (wave & 1) * (BMT / 2);
    const int r16 = lane & 15, q = lane >> 4;
    const int M = ep.M, N = ep.N;
    if constexpr (DEQUANT) {
        constexpr int kU = kWN / 8, kRowBytes = 2 * kWN;     // kWN FP16 columns per staged row
        int8_t* stage = lds + wave * ((BMT / 2) * kRowBytes);
        const bool has_bias = ep.bias != nullptr;
        float as[kTM];
#pragma unroll
        for (int j = 0; j < kTM; j++) {
            const int m = wm + 16 * j + r16;
            as[j] = ep.act_scale[m < M ? m : M - 1];
        }
        // The wave's kWN w_scale / bias halves go through a wave-private LDS strip (one load
        // per lane and 64 columns, in flight together) instead of one memory latency per
        // column group; the bias strip holds w_scale when there is no bias (ignored by
        // dequant_gemm).
        uint16_t* wsl = reinterpret_cast<uint16_t*>(lds + 4 * (BMT / 2) * kRowBytes) + wave * 256;
        uint16_t* bl = wsl + 128;
        {
            const uint16_t* bsrc = has_bias ? ep.bias : ep.w_scale;
            uint16_t w[kWN / 64], bb[kWN / 64];
#pragma unroll
            for (int h = 0; h < kWN / 64; h++) {
                const int nc = min(wn + 64 * h + lane, N - 1);
                w[h] = ep.w_scale[nc];
                bb[h] = bsrc[nc];
            }
#pragma unroll
            for (int h = 0; h < kWN / 64; h++) {
                wsl[64 * h + lane] = w[h];
                bl[64 * h + lane] = bb[h];
            }
        }
#pragma unroll
        for (int i = 0; i < kTN; i++) {
            const uint2 w2 = *reinterpret_cast<const uint2*>(wsl + 16 * i + 4 * q);
            const uint2 b2 = *reinterpret_cast<const uint2*>(bl + 16 * i + 4 * q);
            const uint32_t wr[4] = {w2.x & 0xFFFFu, w2.x >> 16, w2.y & 0xFFFFu, w2.y >> 16};
            const uint32_t br[4] = {b2.x & 0xFFFFu, b2.x >> 16, b2.y & 0xFFFFu, b2.y >> 16};
            float ws[4], b[4];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                ws[t] = h2f(static_cast<uint16_t>(wr[t]));
                b[t] = has_bias ? h2f(static_cast<uint16_t>(br[t])) : -0.0f;   // dequant4_pk: -0 without a bias
            }
            const int u = 2 * i + (q >> 1), half = q & 1;
#pragma unroll
            for (int j = 0; j < kTM; j++) {
                const int r = 16 * j + r16;
                *reinterpret_cast<uint2*>(stage + r * kRowBytes + ((u ^ (r & (kU - 1))) << 4) + 8 * half) =
                    dequant4_pk(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3], as[j], ws, b);
            }
        }
        flush_rows<kU, 2, true, false, BMT / 2>(stage, ep, wm, wn);
    } else {
        constexpr int kU = kWN / 4, kRowBytes = 4 * kWN;     // kWN INT32 columns per staged row
        int8_t* strip = lds + wave * (16 * kRowBytes);
#pragma unroll
        for (int j = 0; j < kTM; j++) {
#pragma unroll
            for (int i = 0; i < kTN; i++) {
                const int u = 4 * i + q;
                *reinterpret_cast<int4*>(strip + r16 * kRowBytes + ((u ^ (r16 & (kU - 1))) << 4)) =
                    make_int4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
            }
            flush_rows<kU, 4, false, true, 16>(strip, ep, wm + 16 * j, wn);
        }
    }
}

template <int BMT, bool DEQUANT, int BNW = 256>
constexpr int sp_dma_lds_bytes() {
    constexpr int epi = DEQUANT ? 4 * (BMT / 2) * BNW + 4 * 512 : 4 * 16 * (2 * BNW);
    return SpDmaTile<BMT, BNW>::kLdsBytes > epi ? SpDmaTile<BMT, BNW>::kLdsBytes : epi;
}

template <int BMT, bool DEQUANT, int BNW = 256>
__global__ __launch_bounds__(256) void sparse_dma_kernel(const int8_t* __restrict__ W, const int8_t* __restrict__ X,
                                                         const uint32_t* __restrict__ meta, GemmEpilogue ep,
                                                         int tiles_n, int tiles_m, int K)
{
    extern __shared__ __align__(16) int8_t lds[];
    int tn, tm;
    tile_coords(blockIdx.x, tiles_n, tiles_m, tn, tm);
    const int n0 = tn * BNW, m0 = tm * BMT;
    SpDmaTile<BMT, BNW> t;
    t.run(W, X, meta, ep.M, ep.N, K, n0, m0, lds);
    sp_store_tile<BMT, DEQUANT, BNW>(t.acc, ep, n0, m0, lds);
}

template <int BMT, bool DEQUANT, int BNW = 256>
static int launch_sparse_dma(const int8_t* W, const int8_t* X, const uint32_t* meta, const GemmEpilogue& ep,
                             int K, hipStream_t s)
{
    constexpr int lds = sp_dma_lds_bytes<BMT, DEQUANT, BNW>();
    const int tiles_n = divup(ep.N, BNW), tiles_m = divup(ep.M, BMT);
    const long long total = static_cast<long long>(tiles_n) * tiles_m;
    if (total > 0x7FFFFFFFLL) return FORGE_EINVAL;
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&sparse_dma_kernel<BMT, DEQUANT, BNW>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (attr != hipSuccess) return static_cast<int>(attr);
    sparse_dma_kernel<BMT, DEQUANT, BNW>
        <<<static_cast<unsigned>(total), 256, lds, s>>>(W, X, meta, ep, tiles_n, tiles_m, K);
    return launch_status();
}

// ---- DMA ring engine for small tiles: 128 weight rows x 64 tokens -------------------
// For shapes whose 256-row tiles leave most CUs idle (narrow N, deep K: the reference
// benchmark's 6144x1536 and 5120x1280 at M = 1024 give 48 and 40 such tiles). A stage is small
// (18 KB: 128 compressed rows x 64 B, 64 token rows x 128 B, 8 blocks x 64 index words, the
// layouts of SpDmaTile), so one stage of lead cannot cover the load latency; D slots give
// D - 1 stages in flight. One barrier per stage publishes stage kt (every wave waited for its
// own DMAs of it) and marks stage kt - 1's slot read by every wave, which then receives stage
// kt + D - 1. Waves in a 2 x 2 grid own 64 weight rows x 32 tokens: 4 x 2 blocks of
// v_smfmac_i32_16x16x128_i8 per stage.
// BNW = 64 (64 weight rows x 64 tokens, 13 KB stages): twice the tiles, and with a shallower
// ring two or three workgroups per CU, for the shapes whose 128-row tiles leave CUs idle.
template <int D, int BNW_ = 128>
struct SpRingTile {
    static constexpr int BNW = BNW_, BMT = 64;
    static constexpr int kTN = BNW / 32, kTM = 2;
    static constexpr int kWBytes = BNW * 64, kXBytes = BMT * 128, kIBytes = BNW / 16 * 256;
    static constexpr int kSlotBytes = kWBytes + kXBytes + kIBytes;
    static constexpr int kLdsBytes = D * kSlotBytes;
    static constexpr int kWIns = kWBytes / 1024 / 4;    // 1 KB DMA instructions per wave per stage
    static constexpr int kXIns = kXBytes / 1024 / 4;
    static constexpr int kVm = kWIns + kXIns + 1;       // + one partial-wave index DMA
    static constexpr int kILanes = kIBytes / 4 / 16;    // lanes of a wave copying 16 index bytes each
    static_assert(BNW == 64 || BNW == 128, "ring tile rows");
    static_assert(kWIns >= 1 && kILanes >= 1 && kILanes <= 32, "ring stage split over 4 waves");
    static_assert(D >= 2 && (D - 2) * kVm < 64, "ring depth");

    v4i acc[kTN][kTM];

    __device__ __forceinline__ void run(const int8_t* W, const int8_t* X, const uint32_t* meta, int M, int N, int K,
                                        int n0, int m0, int8_t* lds) {
        const int lane = threadIdx.x & (kWave - 1);
        const int wave = threadIdx.x / kWave;
        const int wn = (wave >> 1) * (BNW / 2);
        const int wm = (wave & 1) * (BMT / 2);
        const int r16 = lane & 15, g = lane >> 4;
        const int Kc = K >> 1, cpr = K >> 5;
#pragma unroll
        for (int i = 0; i < kTN; i++)
#pragma unroll
            for (int j = 0; j < kTM; j++) acc[i][j] = v4i{0, 0, 0, 0};

        const SpBufs bf = sp_bufs(W, X, meta, M, N, K);
        uint32_t ow[kWIns], ox[kXIns];
#pragma unroll
        for (int q = 0; q < kWIns; q++) {
            const int s = (wave * kWIns + q) * kWave + lane;
            const int r = s >> 2, c = (s & 3) ^ lds_swz4(r);
            const int gr = (n0 + r) < N ? (n0 + r) : N - 1;
            ow[q] = static_cast<uint32_t>(gr) * Kc + 16 * c;
        }
#pragma unroll
        for (int q = 0; q < kXIns; q++) {
            const int s = (wave * kXIns + q) * kWave + lane;
            const int r = s >> 3, c = (s & 7) ^ lds_swz8(r);
            const int gr = (m0 + r) < M ? (m0 + r) : M - 1;
            ox[q] = static_cast<uint32_t>(gr) * K + 16 * c;
        }
        uint32_t oi;
        {
            const int s = wave * kILanes + (lane & (kILanes - 1));   // 16-byte chunk of the stage's index area
            int b = (n0 >> 4) + (s >> 4);
            b = b < (N >> 4) ? b : (N >> 4) - 1;
            oi = static_cast<uint32_t>(b) * cpr * 64 + 16 * (s & 15);
        }
        const int nst = K / 128;
        auto slot_of = [&](int st) { return lds + (st % D) * kSlotBytes; };
        auto issue = [&](int st) {
            int8_t* slot = slot_of(st);
            const uint32_t su = static_cast<uint32_t>(st);
#pragma unroll
            for (int q = 0; q < kWIns; q++) dma16_buf(bf.w, ow[q], su * 64, slot + (wave * kWIns + q) * 1024);
#pragma unroll
            for (int q = 0; q < kXIns; q++) dma16_buf(bf.x, ox[q], su * 128, slot + kWBytes + (wave * kXIns + q) * 1024);
            if (lane < kILanes) dma16_buf(bf.i, oi, su * 256, slot + kWBytes + kXBytes + wave * (16 * kILanes));
        };
        // Waits for this wave's DMAs of stage kt when `later` stages were issued after it.
        auto wait_stage = [&](int later) {
            switch (later) {
            case 0: wait_vmcnt<0>(); break;
            case 1: wait_vmcnt<kVm>(); break;
            case 2: wait_vmcnt<2 * kVm>(); break;
            case 3: wait_vmcnt<3 * kVm>(); break;
            case 4: wait_vmcnt<4 * kVm>(); break;
            case 5: wait_vmcnt<5 * kVm>(); break;
            default: wait_vmcnt<(D - 2) * kVm>(); break;
            }
        };
        for (int d = 0; d < D - 1; d++)
            if (d < nst) issue(d);
        for (int kt = 0; kt < nst; kt++) {
            const int later = (nst - 1 - kt) < (D - 2) ? (nst - 1 - kt) : (D - 2);
            wait_stage(later);
            lds_barrier();
            if (kt + D - 1 < nst) issue(kt + D - 1);
            const int8_t* Ws = slot_of(kt);
            const int8_t* Xs = Ws + kWBytes;
            const uint32_t* Is = reinterpret_cast<const uint32_t*>(Xs + kXBytes);
            v4i a[kTN];
            int idx[kTN];
            v8i b[kTM];
#pragma unroll
            for (int i = 0; i < kTN; i++) {
                a[i] = *reinterpret_cast<const v4i*>(Ws + lds_off64(wn + 16 * i + r16, g));
                idx[i] = static_cast<int>(Is[((wn >> 4) + i) * 64 + lane]);
            }
#pragma unroll
            for (int j = 0; j < kTM; j++) {
                const int r = wm + 16 * j + r16;
                const v4i lo = *reinterpret_cast<const v4i*>(Xs + lds_off128(r, g));
                const v4i hi = *reinterpret_cast<const v4i*>(Xs + lds_off128(r, g + 4));
                b[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
            }
#pragma unroll
            for (int j = 0; j < kTM; j++)
#pragma unroll
                for (int i = 0; i < kTN; i++)
                    acc[i][j] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(a[i], b[j], acc[i][j], idx[i], 0, 0);
        }
    }
};

constexpr int kSpRingSlots = 8;

// Lane l of block (i, j) holds outputs (m = 16 j + l % 16, n = 16 i + 4 (l / 16) + e): one
// 8-byte FP16 or 16-byte INT32 store each (N % 16 == 0, so the 4 columns are in or out together).
template <bool DEQUANT, int BNW = 128, int D = kSpRingSlots>
__global__ __launch_bounds__(256) void sparse_ring_kernel(const int8_t* __restrict__ W, const int8_t* __restrict__ X,
                                                          const uint32_t* __restrict__ meta, GemmEpilogue ep,
                                                          int tiles_n, int tiles_m, int K)
{
    using T = SpRingTile<D, BNW>;
    extern __shared__ __align__(16) int8_t lds[];
    int tn, tm;
    tile_coords(blockIdx.x, tiles_n, tiles_m, tn, tm);
    const int n0 = tn * T::BNW, m0 = tm * T::BMT;
    T t;
    t.run(W, X, meta, ep.M, ep.N, K, n0, m0, lds);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int wn = n0 + (wave >> 1) * (T::BNW / 2), wm = m0 + (wave & 1) * (T::BMT / 2);
    const int M = ep.M, N = ep.N;
#pragma unroll
    for (int j = 0; j < T::kTM; j++) {
        const int m = wm + 16 * j + (lane & 15);
        if (m >= M) continue;
        const float as = DEQUANT ? ep.act_scale[m] : 0.0f;
#pragma unroll
        for (int i = 0; i < T::kTN; i++) {
            const int n = wn + 16 * i + 4 * (lane >> 4);
            if (n >= N) continue;
            const size_t o = static_cast<size_t>(m) * N + n;
            if constexpr (DEQUANT) {
                float ws4[4], b4[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    ws4[e] = h2f(ep.w_scale[n + e]);
                    b4[e] = ep.bias ? h2f(ep.bias[n + e]) : -0.0f;   // dequant4_pk: -0 without a bias
                }
                *reinterpret_cast<uint2*>(ep.c16 + o) =
                    dequant4_pk(t.acc[i][j][0], t.acc[i][j][1], t.acc[i][j][2], t.acc[i][j][3], as, ws4, b4);
            } else {
                *reinterpret_cast<int4*>(ep.c32 + o) =
                    make_int4(t.acc[i][j][0], t.acc[i][j][1], t.acc[i][j][2], t.acc[i][j][3]);
            }
        }
    }
}

template <bool DEQUANT, int BNW = 128, int D = kSpRingSlots>
static int launch_sparse_ring(const int8_t* W, const int8_t* X, const uint32_t* meta, const GemmEpilogue& ep, int K,
                              hipStream_t s)
{
    using T = SpRingTile<D, BNW>;
    constexpr int lds = T::kLdsBytes;
    const int tiles_n = divup(ep.N, T::BNW), tiles_m = divup(ep.M, T::BMT);
    const long long total = static_cast<long long>(tiles_n) * tiles_m;
    if (total > 0x7FFFFFFFLL) return FORGE_EINVAL;
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&sparse_ring_kernel<DEQUANT, BNW, D>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (attr != hipSuccess) return static_cast<int>(attr);
    sparse_ring_kernel<DEQUANT, BNW, D>
        <<<static_cast<unsigned>(total), 256, lds, s>>>(W, X, meta, ep, tiles_n, tiles_m, K);
    return launch_status();
}

// ---- tile configurations ----------------------------------------------------------

constexpr int kSpTileBW[FORGE_SPARSE_NUM_TILES] = {256, 128, 128};
constexpr int kSpTileBC[FORGE_SPARSE_NUM_TILES] = {128, 128, 64};

template <int BNW, int BMT, int WN, int WM>
static void sparse_set_attr() {
    using Cfg = SparseCfg<BNW, BMT, WN, WM>;
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&sparse_gemm_kernel<BNW, BMT, WN, WM>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, Cfg::kLdsBytes);
}

static void sparse_init_attrs() {
    static std::once_flag once;
    std::call_once(once, [] {
        sparse_set_attr<256, 128, 2, 2>();
        sparse_set_attr<128, 128, 2, 2>();
        sparse_set_attr<128, 64, 2, 2>();
        (void)hipGetLastError();
    });
}

template <int BNW, int BMT, int WN, int WM>
static int sparse_launch_cfg(SparseArgs p, hipStream_t s)
{
    using Cfg = SparseCfg<BNW, BMT, WN, WM>;
    p.tiles_n = divup(p.N, BNW);
    p.tiles_m = divup(p.M, BMT);
    const long long grid = static_cast<long long>(p.tiles_n) * p.tiles_m * p.split_k;
    if (grid > 0x7FFFFFFFLL) return FORGE_EINVAL;
    sparse_gemm_kernel<BNW, BMT, WN, WM><<<static_cast<unsigned>(grid), Cfg::kThreads, Cfg::kLdsBytes, s>>>(p);
    return launch_status();
}

static int sparse_launch(int tile, const SparseArgs& p, hipStream_t s)
{
    sparse_init_attrs();
    switch (tile) {
    case 0: return sparse_launch_cfg<256, 128, 2, 2>(p, s);
    case 1: return sparse_launch_cfg<128, 128, 2, 2>(p, s);
    default: return sparse_launch_cfg<128, 64, 2, 2>(p, s);
    }
}

// ---- planner ------------------------------------------------------------------------
// Wave-aware cost model with the reference's form (int8_sparse.cu:875-920):
//   t(tile, s) = waves * (a_tile * ceil(steps / s) + b_tile) + [s > 1] (c0 + (c1 + c2 s) MN/1e6)
//   waves      = ceil(tiles(tile) * s / CUs)
// a_tile: time of one 128-deep K step of a tile at the SMFMAC rate (dense-equivalent
// 2*BW*BC*128 ops at 2 x 5.0 POPS / 256 CUs per CU), inflated for LDS/issue overhead;
// b_tile: per-tile fixed cost (fill + epilogue). Times in microseconds.
double sparse_plan_cost(int M, int K, int N, int split_k, bool have_ws, int tile, int cu, int* out_tile,
                        int* out_split)
{
    static const double kA[FORGE_SPARSE_NUM_TILES] = {0.110, 0.058, 0.032};   // us per K step per tile
    static const double kB[FORGE_SPARSE_NUM_TILES] = {1.60, 1.10, 0.80};      // us per tile
    const double kC0 = 2.0, kC1 = 0.60, kC2 = 0.25;                     // split-K launch / zero+finalize / atomics
    static const int kAutoSplits[] = {1, 2, 3, 4, 6};
    if (tile >= FORGE_SPARSE_NUM_TILES) tile = -1;
    if (split_k > 1 && !have_ws) split_k = 1;
    const int steps = divup(K, kSpStep);
    const bool auto_split = split_k <= 0;
    int best_t = 1, best_s = 1;
    double best = 1e300;
    for (int t = 0; t < FORGE_SPARSE_NUM_TILES; t++) {
        if (tile >= 0 && t != tile) continue;
        const long long tiles = static_cast<long long>(divup(N, kSpTileBW[t])) * divup(M, kSpTileBC[t]);
        const int ncand = auto_split ? (have_ws ? 5 : 1) : 1;
        for (int c = 0; c < ncand; c++) {
            const int sp = auto_split ? kAutoSplits[c] : split_k;
            if (auto_split && sp > 1 && sp > steps / 2) continue;
            // in double: a forced split times the tile count can pass 2^63 (exact below 2^53)
            const double waves = std::ceil(static_cast<double>(tiles) * sp / cu);
            const int ks = divup(steps, sp);
            double cost = waves * (kA[t] * ks + kB[t]);
            if (sp > 1) cost += kC0 + (kC1 + kC2 * sp) * (static_cast<double>(M) * N * 1e-6);
            if (cost < best) { best = cost; best_t = t; best_s = sp; }
        }
    }
    *out_tile = best_t;
    *out_split = best_s;
    return best;
}

static int cu_count_or_default() {
    int st = FORGE_OK;
    const DeviceInfo& d = device_info(&st);
    return (st == FORGE_OK && d.cu_count > 0) ? d.cu_count : default_cu_count();
}

// Unsplit DMA engine choice (automatic plans, M > 64, K % 128 == 0): 256 weight rows x 256
// tokens (sparse_dma32, M > 128), 128 x 128 (sparse_dma<128, 128>: 52 KB of LDS, two
// workgroups per CU by registers), or the 64 x 64 ring engine (sparse_ring, 4 slots, three
// workgroups per CU). Each engine's time is modelled from the tiles on the busiest CU (w) and
// the 128-deep stages (steps), with coefficients fitted on MI355X timings of every engine on 30
// shapes (the reference sweep at M = 1024 / 4096 / 8192, its narrow layers at M up to 147,456,
// the engine tests' shapes, configs[2] with FP16 out, deep-K layers at M = 256-2048), in us:
//   256 x 256: w (0.88 steps + 10.0)
//   128 x 128: 0.48 steps + 3.7 for one tile per CU, else ceil(w / 2) (0.71 steps + 5.2)
//   ring:      steps (0.175 ceil(w / 3) + 0.123 w) + 4.6, only up to one round (w <= 3)
// The pick is the fastest engine on 28 of the 30 shapes and within 8 % on the other two (the
// 256 x 128 engine, kept for the reference's forced 256x128 tile, was never the fastest there).
// Examples (us): 1536x6144 at M = 1024 128x128 13.5 (256x256 19.3, 256x128 15.1); 6144x1536 at
// M = 1024 ring 24.0 (128x128 32.3); 640x320 at M = 147,456 128x128 53.5 (256x256 71.6);
// configs[2] on 256x256.
enum class SpEngine { k256x256, k256x128, k128x128, kRing };
constexpr int kSpRingRows = 64, kSpRingDepth = 4, kSpRingPerCu = 3;

static SpEngine sparse_pick_engine(int M, int N, int K, int cu)
{
    const double steps = static_cast<double>(divup(K, kSpStep));
    const long long w128 = divupll(static_cast<long long>(divup(N, 128)) * divup(M, 128), cu);
    const long long wr = divupll(static_cast<long long>(divup(N, kSpRingRows)) * divup(M, 64), cu);
    double best = w128 == 1 ? 0.48 * steps + 3.7 : static_cast<double>(divupll(w128, 2)) * (0.71 * steps + 5.2);
    SpEngine e = SpEngine::k128x128;
    if (M > 128) {
        const double w256 = static_cast<double>(divupll(static_cast<long long>(divup(N, 256)) * divup(M, 256), cu));
        const double t = w256 * (0.88 * steps + 10.0);
        if (t < best) { best = t; e = SpEngine::k256x256; }
    }
    if (wr <= kSpRingPerCu) {
        const double t = steps * (0.175 * static_cast<double>(divupll(wr, kSpRingPerCu)) + 0.123 * static_cast<double>(wr)) + 4.6;
        if (t < best) e = SpEngine::kRing;
    }
    return e;
}

// Whether the wide-tile engine's plan beats 256 x 256 tiles, by bytes streamed per CU (both
// engines run at the same LDS-DMA byte rate): a 256-token tile of NJ 32-row blocks moves 32 KB
// of tokens + 2.5 KB per block each 128-deep stage, a 256 x 256 tile 52 KB; the 256 x 256 grid
// takes whole tile waves, the last one a 192-token tail wave (~0.85 of a tile) where
// launch_sparse_dma32_tail applies. Measured at configs[2] (4096 x 11008 x 4096): 2 x 11-block
// tiles 115 us vs 2.85 tile times of 256 x 256 126 us; at exact 256 x 256 waves with 8-block
// wide tiles (4096 x 8192) the two are level by bytes, so the 256 x 256 engine keeps them.
static bool sparse_wide_pays(int M, int N, int cu, const SpWidePlan& p)
{
    const int nbmax = p.q + (p.r > 0 ? 1 : 0);
    const int njmax = divup(nbmax, p.T);
    const double wide = p.T * (32.0 + 2.5 * njmax) / 52.0;
    const int tiles_m = divup(M, 256);
    const long long tiles = static_cast<long long>(divup(N, 256)) * tiles_m;
    const long long waves = divupll(tiles, cu);
    const bool tail = tiles > cu && tiles % cu != 0 && cu % tiles_m == 0 && M >= 192;
    const double d256 = static_cast<double>(waves) - (tail ? 0.15 : 0.0);
    return wide < 0.95 * d256;
}

int sparse_gemm(const int8_t* W_comp, const int8_t* x, const uint32_t* meta, const float* act_scale,
                const uint16_t* w_scale, const uint16_t* bias, uint16_t* out16, int32_t* out32, int M,
                int K, int N, int32_t* ws, int split_k, int tile, hipStream_t s)
{
    if (K % 64 != 0 || N % 16 != 0) return FORGE_EINVAL;
    if (!aligned(W_comp, 16) || !aligned(x, 16) || !aligned(meta, 16)) return FORGE_EINVAL;
    if (out16 && !aligned(out16, 8)) return FORGE_EINVAL;
    if (out32 && !aligned(out32, 16)) return FORGE_EINVAL;
    int st = FORGE_OK;
    device_info(&st);
    if (st != FORGE_OK) return st;

    // Decode shapes stream the weights once on the decode kernel (any tile / split request
    // gives the same bits, so those hints do not apply here).
    if (decode_supported(M, K)) {
        void* o = out16 ? static_cast<void*>(out16) : static_cast<void*>(out32);
        GemmEpilogue ep{out32, out16, act_scale, w_scale, bias, M, N, aligned(o, 16) ? 1 : 0};
        note_route("decode");
        return launch_decode(W_comp, meta, x, ep, K, true, s);
    }
    // 16 < M <= 64 in automatic mode: the same weight-streaming kernel with several token blocks
    // (a forced tile or split runs the engine it names).
    if (skinny_tb_supported(M, K) && tile == FORGE_SPARSE_TILE_AUTO && split_k <= 1) {
        void* o = out16 ? static_cast<void*>(out16) : static_cast<void*>(out32);
        GemmEpilogue ep{out32, out16, act_scale, w_scale, bias, M, N, aligned(o, 16) ? 1 : 0};
        note_route("token-block");
        return launch_skinny_tb(W_comp, meta, x, ep, K, cu_count_or_default(), s);
    }
    int pt = 1, ps = 1;
    sparse_plan_cost(M, K, N, out32 ? 1 : split_k, out32 ? false : ws != nullptr, tile,
                     cu_count_or_default(), &pt, &ps);
    const int steps = divup(K, kSpStep);
    SparseArgs p{};
    p.W_comp = W_comp; p.x = x; p.meta = meta; p.act_scale = act_scale; p.w_scale = w_scale;
    p.bias = bias; p.M = M; p.K = K; p.N = N;
    if (ps > 1 && ws) {
        p.split_k = ps;
        p.steps_per_split = divup(steps, ps);
        p.out16 = nullptr;
        p.out32 = ws;
        p.atomic = 1;
        const long long total = static_cast<long long>(M) * N;
        const int blocks = static_cast<int>(std::min<long long>(divupll(total / 4, 256) + 1, 8192));
        zero_i32_kernel<<<blocks, 256, 0, s>>>(reinterpret_cast<int4*>(ws), total / 4, ws + (total / 4) * 4,
                                               static_cast<int>(total % 4));
        if ((st = launch_status()) != FORGE_OK) return st;
        note_route("regstaged", pt, ps);
        if ((st = sparse_launch(pt, p, s)) != FORGE_OK) return st;
        const int fblocks = static_cast<int>(std::min<long long>(divupll(total, 256), 8192));
        splitk_finalize_kernel<<<fblocks, 256, 0, s>>>(ws, act_scale, w_scale, bias, out16, N, total);
        return launch_status();
    }
    // Unsplit plans on 128-deep K stages run on the DMA-fed engines: chosen by tile waves when
    // the planner chose freely, 256 weight rows x 128 tokens for the reference's 256x128 tile.
    const bool dma_fits = static_cast<long long>(M) * K < (1LL << 31) && static_cast<long long>(N) * K < (1LL << 32);
    if (dma_fits && K % 128 == 0 && M > 64 && (tile == FORGE_SPARSE_TILE_AUTO || pt == FORGE_SPARSE_TILE_256x128) &&
        (tile == FORGE_SPARSE_TILE_AUTO || tile == FORGE_SPARSE_TILE_256x128)) {
        void* o = out16 ? static_cast<void*>(out16) : static_cast<void*>(out32);
        GemmEpilogue ep{out32, out16, act_scale, w_scale, bias, M, N, aligned(o, 16) ? 1 : 0};
        const SpEngine e = tile == FORGE_SPARSE_TILE_AUTO ? sparse_pick_engine(M, N, K, cu_count_or_default())
                                                          : SpEngine::k256x128;
        note_route(e == SpEngine::k256x256 ? "dma256x256"
                   : e == SpEngine::kRing  ? "ring64x64"
                   : e == SpEngine::k128x128 ? "dma128x128"
                                             : "dma256x128");
        // INT32 output where 256 x 256 tiles would run: the wide-tile engine when its per-CU
        // plan applies (fewer token bytes per output, every CU the same weight blocks).
        SpWidePlan wp;
        if (e == SpEngine::k256x256 && !out16 && tile == FORGE_SPARSE_TILE_AUTO &&
            sparse_wide_plan(M, N, K, cu_count_or_default(), &wp) && sparse_wide_pays(M, N, cu_count_or_default(), wp)) {
            note_route("wide256", wp.T);
            return launch_sparse_wide_s32(W_comp, x, meta, out32, M, K, N, wp, s);
        }
        if (e == SpEngine::k256x256)
            return out16 ? launch_sparse_dma32<true>(W_comp, x, meta, ep, K, s)
                         : launch_sparse_dma32<false>(W_comp, x, meta, ep, K, s);
        if (e == SpEngine::kRing)
            return out16 ? launch_sparse_ring<true, kSpRingRows, kSpRingDepth>(W_comp, x, meta, ep, K, s)
                         : launch_sparse_ring<false, kSpRingRows, kSpRingDepth>(W_comp, x, meta, ep, K, s);
        if (e == SpEngine::k128x128)
            return out16 ? launch_sparse_dma<128, true, 128>(W_comp, x, meta, ep, K, s)
                         : launch_sparse_dma<128, false, 128>(W_comp, x, meta, ep, K, s);
        return out16 ? launch_sparse_dma<128, true>(W_comp, x, meta, ep, K, s)
                     : launch_sparse_dma<128, false>(W_comp, x, meta, ep, K, s);
    }
    p.split_k = 1;
    p.steps_per_split = steps;
    p.out16 = out16;
    p.out32 = out32;
    p.atomic = 0;
    note_route("regstaged", pt, 1);
    return sparse_launch(pt, p, s);
}

// ---- fused quantize + sparse linear (the reference's FQ path) ------------------------
// src/gemm/int8_sparse.cu:250-335 (and :1022-1033): for narrow layers at large M the int8
// copy of the activations costs a DRAM round trip (write M*K, read it back) that the fused
// path avoids by quantizing each block of token rows on the chip. MI355X form: a persistent
// 512-thread workgroup (2 waves per SIMD) with a double-buffered LDS token tile of BT rows:
//   - producer waves 4..7 quantize tile t+1 (BT/4 rows each) into one buffer -- K/128 slabs
//     of BT rows x 128 bytes in the two-pass engine's conflict-free B layout (sp_b_off) --
//     and its row scales. kFqRowsInFlight rows form a batch whose 16-byte loads issue
//     together, before the previous batch is quantized; the last batch of a tile fetches the
//     first batch of the next, across the barrier. Row absmax on fp16 bit patterns (one
//     packed u16 max per two values, DPP across the wave, two rows per reduction), values by
//     quant8_rows2 (two rows at a time, SDWA byte inserts): the arithmetic of quantize_rows.
//   - consumer waves 0..3 run tile t from the other buffer: each owns NBW consecutive 16-row
//     weight blocks per pass, streams their compressed bytes and index words straight from
//     L2 into registers (kFqAhead K steps ahead, in the SMFMAC lane layout), reads the
//     step's 16-token B fragments from LDS once for all NBW blocks
//     (v_smfmac_i32_16x16x128_i8, A = weights), and writes each lane's 4 consecutive outputs
//     of one token row as one 8-byte store with the GEMM dequant epilogue (w_scale and bias
//     staged in LDS once).
// The two kinds of waves run separate loops with one LDS-only barrier per tile (so the
// producer's prefetch stays in flight across it). A producer's quantize (VALU) and a
// consumer's SMFMACs share every SIMD. The scratch buffers and the split-K workspace are not
// touched (as in the reference). Every output equals the two-pass path's bits: same
// quantization, exact INT32 sums, same epilogue. Measured at 147,456 x 1280 -> 320: 210 us
// (two-pass 229); the consumer side bounds it -- weight-fragment loads (16 half cache lines
// per instruction) and LDS reads with one consumer wave per SIMD keep the matrix core ~11 %
// busy.
constexpr int kFqMaxK = 2048;
constexpr int kFqRowsInFlight = 4;   // token rows per producer wave whose loads are in flight together
constexpr int kFqAhead = 3;          // K steps of weight fragments in flight per consumer wave
constexpr int kFqLds = 160 * 1024;

// PACKED: W_comp is in fragment order (fq_pack_weights_kernel): a consumer's weight fragment
// of one block and K step is one contiguous 1 KB load instead of 16 half cache lines, 64 bytes
// in each of 16 rows -- adjacent lanes then read adjacent 16-byte units, which the texture
// unit serves several times faster (measured at 147,456 x 1280 -> 320: consumer waves alone
// 104 -> 64 us).
// NV: 16-byte vectors per lane per token row, at least K / 512 (rows of K / 8 vectors over the
// 64 lanes of a producer wave): lanes past the row end hold no data but still cost a load slot
// and registers, so NV follows K (at K = 1280, 3 rather than 4: 147,456 x 1280 -> 320 155 ->
// 142 us).
template <int NBW, int BT, bool PACKED, int NV>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void sparse_fq_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ W_comp, const uint32_t* __restrict__ meta,
    const uint16_t* __restrict__ w_scale, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out,
    int M, int K, int N, int tiles, int stg)
{
    constexpr int kTB = BT / 16;                 // 16-token blocks per tile
    constexpr int kRowsPerProducer = BT / 4;
    static_assert(BT % 16 == 0 && kRowsPerProducer % kFqRowsInFlight == 0 && kFqRowsInFlight % 2 == 0,
                  "tile rows must split evenly");
    constexpr int kSlab = BT * kSpBRow;
    extern __shared__ __align__(16) int8_t lds[];
    const int tileBytes = BT * K;
    float* sscale = reinterpret_cast<float*>(lds + 2 * tileBytes);          // [2][BT]
    uint16_t* sws = reinterpret_cast<uint16_t*>(sscale + 2 * BT);          // N
    uint16_t* sbias = sws + N;                                              // N
    // stg: each consumer wave's outputs of a pass go through its own LDS strip (BT rows x NBW
    // blocks of 16 columns) and leave as 16-byte stores of whole row runs: stored from the
    // accumulators directly, a lane quad writes 4 different rows, which costs the texture unit
    // several times the cycles of a contiguous quad (147,456 x 1280 -> 320: the output stores
    // took 15-17 us of the kernel).
    constexpr int kStgPitch = NBW * 16 + 8;   // halves per staged row (+16 bytes: rows spread over the banks)
    uint16_t* sstg = reinterpret_cast<uint16_t*>(lds + ((2 * tileBytes + 8 * BT + 4 * N + 15) & ~15));
    const int t = threadIdx.x, lane = t & (kWave - 1), wave = t >> 6;
    const int KS = K / kSpStep, Kc = K / 2, cpr = K / 32, NB = N / 16;
    const bool has_bias = bias != nullptr;
    const int nvec = K / 8;
    for (int n = t; n < N; n += 512) {
        sws[n] = w_scale[n];
        sbias[n] = has_bias ? bias[n] : static_cast<uint16_t>(0x8000);   // -0: dequant4_pk without a bias
    }

    // Producer: rows pw*BT/4 .. +BT/4 of `tile` into buffer `buf`, kFqRowsInFlight rows per
    // batch, the next batch's loads issued before this one is used. Loads are unconditional:
    // lanes past the row end re-read its last vector (one coalesced request; a repeated value
    // leaves the maximum unchanged), since a load inside `if (idx < nvec)` together with its
    // use compiled to load -> wait -> use, one memory latency per vector.
    constexpr int kR = kFqRowsInFlight;
    constexpr int kBatches = kRowsPerProducer / kR;
    auto load_batch = [&](int ln, int m0, int r0, uint4 (&v)[kR][NV]) {
#pragma unroll
        for (int u = 0; u < kR; u++) {
            const int row = min(m0 + r0 + u, M - 1);
            const uint4* src = reinterpret_cast<const uint4*>(x + static_cast<size_t>(row) * K);
#pragma unroll
            for (int i = 0; i < NV; i++) v[u][i] = src[min(ln + kWave * i, nvec - 1)];
        }
    };
    auto quantize_batch = [&](int ln, int r0, const uint4 (&v)[kR][NV], int8_t* Xs, float* sc) {
        uint32_t mb[kR];
#pragma unroll
        for (int u = 0; u < kR; u++) {
            mb[u] = 0u;
#pragma unroll
            for (int i = 0; i < NV; i++) mb[u] = absbits8(v[u][i], mb[u]);
        }
        uint32_t abits[kR];
#pragma unroll
        for (int u = 0; u < kR; u += 2) {
            const uint32_t r2 = wave_max_pk_u16(pk_rows2(mb[u], mb[u + 1]));
            abits[u] = r2 & 0xFFFFu;
            abits[u + 1] = r2 >> 16;
        }
        float inv[kR];
#pragma unroll
        for (int u = 0; u < kR; u++) {
            float amax;
            if (abits[u] > kHalfInfBits) {       // the row holds a NaN: fp32 max skipping it
                float a = 0.0f;
#pragma unroll
                for (int i = 0; i < NV; i++) a = absmax8(v[u][i], a);
                amax = wave_max(a);
            } else {
                amax = h2f(static_cast<uint16_t>(abits[u]));
            }
            const float scale = row_scale(amax);
            inv[u] = 1.0f / scale;
            if (ln == 0) sc[r0 + u] = scale;
        }
        // two rows' vectors at a time: quant8_rows2's SDWA byte inserts need 4 dwords to cycle over
#pragma unroll
        for (int u = 0; u < kR; u += 2) {
#pragma unroll
            for (int i = 0; i < NV; i++) {
                const int idx = ln + kWave * i;
                uint2 qa, qb;
                quant8_rows2(v[u][i], inv[u], v[u + 1][i], inv[u + 1], qa, qb);
                if (idx < nvec) {
                    const int k = 8 * idx;
                    int8_t* xk = Xs + (k >> 7) * kSlab + (k & 8);
                    *reinterpret_cast<uint2*>(xk + sp_b_off(r0 + u, (k >> 4) & 7)) = qa;
                    *reinterpret_cast<uint2*>(xk + sp_b_off(r0 + u + 1, (k >> 4) & 7)) = qb;
                }
            }
        }
    };
    // Producer tile: the first batch of `tile` is in v[E] on entry (loaded during the previous
    // tile); the last batch's successor load fetches the first batch of tile `after` (a valid
    // tile in any case) into v[(E + kBatches) & 1], so every batch's loads, a tile's first
    // included, are in flight while the batch before it is quantized.
    auto quantize_tile = [&](auto E, int tile, int buf, int after, int ln, int rp, uint4 (&v)[2][kR][NV]) {
        constexpr int e = decltype(E)::value;
        asm volatile("" : "+v"(ln));             // re-made opaque per tile: nothing lane-derived is hoisted
        int8_t* Xs = lds + buf * tileBytes;
        float* sc = sscale + buf * BT;
        const int m0 = tile * BT;
#pragma unroll
        for (int bt = 0; bt < kBatches; bt++) {
            const int cur = (bt + e) & 1;
            if (bt + 1 < kBatches) load_batch(ln, m0, rp + (bt + 1) * kR, v[cur ^ 1]);
            else load_batch(ln, min(after, tiles - 1) * BT, rp, v[cur ^ 1]);
            quantize_batch(ln, rp + bt * kR, v[cur], Xs, sc);
        }
    };

    // Consumer wave cw: every output of `tile` from buffer `buf`. Workgroups walk K from
    // different starting steps (integer sums do not depend on the order), so the CUs reading
    // the same weight rows at the same time spread over different addresses.
    auto compute_tile = [&](int tile, int buf, int cw) {
        int ln = lane;                           // opaque, as in the producer
        asm volatile("" : "+v"(ln));
        const int r16 = ln & 15, g = ln >> 4;
        const int8_t* Xs = lds + buf * tileBytes;
        const float* sc = sscale + buf * BT;
        const int m0 = tile * BT;
        const int rot = (blockIdx.x + tile) % KS;
        for (int p0 = 0; p0 < NB; p0 += 4 * NBW) {
            const int wb0 = p0 + cw * NBW;
            if (wb0 >= NB) continue;
            v4i acc[NBW][kTB];
#pragma unroll
            for (int i = 0; i < NBW; i++)
#pragma unroll
                for (int j = 0; j < kTB; j++) acc[i][j] = v4i{0, 0, 0, 0};
            v4i fa[kFqAhead][NBW];
            int fi[kFqAhead][NBW];
            // Blocks past NB (a ragged last pass) re-read block NB-1; their accumulators are never
            // stored. (Zeroing the fragment instead put a use right behind each load, which made
            // the compiler wait for the whole prefetch ring at once.)
            auto aload = [&](int s, v4i (&a)[NBW], int (&ix)[NBW]) {
                const int sr = s + rot < KS ? s + rot : s + rot - KS;
#pragma unroll
                for (int i = 0; i < NBW; i++) {
                    const int b = min(wb0 + i, NB - 1);
                    if constexpr (PACKED)
                        a[i] = *reinterpret_cast<const v4i*>(W_comp + (static_cast<size_t>(b) * KS + sr) * 1024 +
                                                             16 * ln);
                    else
                        a[i] = *reinterpret_cast<const v4i*>(W_comp + static_cast<size_t>(16 * b + r16) * Kc +
                                                             kSpARow * sr + 16 * g);
                    ix[i] = static_cast<int>(meta[static_cast<size_t>(b) * cpr * 16 + (4 * sr + g) * 16 + r16]);
                }
            };
            // One K step: the step's kTB token fragments are read from LDS together, so their
            // latency overlaps the first block's SMFMACs instead of preceding each block's.
            auto step = [&](int s, const v4i (&a)[NBW], const int (&ix)[NBW]) {
                const int8_t* slab = Xs + (s + rot < KS ? s + rot : s + rot - KS) * kSlab;
                v8i fb[kTB];
#pragma unroll
                for (int j = 0; j < kTB; j++) {
                    const int r = 16 * j + r16;
                    const v4i b0 = *reinterpret_cast<const v4i*>(slab + sp_b_off(r, g));
                    const v4i b1 = *reinterpret_cast<const v4i*>(slab + sp_b_off(r, g + 4));
                    fb[j] = v8i{b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
                }
#pragma unroll
                for (int j = 0; j < kTB; j++)
#pragma unroll
                    for (int i = 0; i < NBW; i++)
                        acc[i][j] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(a[i], fb[j], acc[i][j], ix[i], 0, 0);
            };
            // The fragment ring: kFqAhead K steps in flight. The main loop is branch-free (every
            // step loads its successor), so the compiler's wait before a step counts only that
            // step's loads; loads under a condition made it wait for the whole ring. Steps past
            // KS in the prologue re-read step KS-1 and go unused.
#pragma unroll
            for (int d = 0; d < kFqAhead; d++) aload(min(d, KS - 1), fa[d], fi[d]);
            int s0 = 0;
            for (; s0 + 2 * kFqAhead <= KS; s0 += kFqAhead) {
#pragma unroll
                for (int d = 0; d < kFqAhead; d++) {
                    step(s0 + d, fa[d], fi[d]);
                    aload(s0 + d + kFqAhead, fa[d], fi[d]);
                }
            }
#pragma unroll
            for (int d = 0; d < kFqAhead; d++) {         // fewer than 2 * kFqAhead steps remain
                if (s0 + d < KS) {
                    step(s0 + d, fa[d], fi[d]);
                    if (s0 + d + kFqAhead < KS) aload(s0 + d + kFqAhead, fa[d], fi[d]);
                }
            }
#pragma unroll
            for (int d = 0; d < kFqAhead; d++)
                if (s0 + kFqAhead + d < KS) step(s0 + kFqAhead + d, fa[d], fi[d]);
            // epilogue: lane holds C[16 blk + 4 g + e][16 j + r16]
            if (stg && wb0 + NBW <= NB) {
                uint16_t* sw = sstg + cw * (BT * kStgPitch);
#pragma unroll
                for (int i = 0; i < NBW; i++) {
                    const int n = 16 * (wb0 + i) + 4 * g;
                    float ws[4], bv[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        ws[e] = h2f(sws[n + e]);
                        bv[e] = h2f(sbias[n + e]);
                    }
#pragma unroll
                    for (int j = 0; j < kTB; j++) {
                        const float as = sc[16 * j + r16];
                        *reinterpret_cast<uint2*>(sw + (16 * j + r16) * kStgPitch + 16 * i + 4 * g) =
                            dequant4_pk(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3], as, ws, bv);
                    }
                }
                // The strip is this wave's own and a wave's LDS accesses complete in order, so
                // the rows can be read back without a barrier.
                constexpr int kCpr = 2 * NBW;    // 16-byte chunks per staged row
                for (int q = ln; q < BT * kCpr; q += kWave) {
                    const int r = q / kCpr, c = q - r * kCpr;
                    if (m0 + r < M)
                        *reinterpret_cast<uint4*>(out + static_cast<size_t>(m0 + r) * N + 16 * wb0 + 8 * c) =
                            *reinterpret_cast<const uint4*>(sw + r * kStgPitch + 8 * c);
                }
                continue;
            }
#pragma unroll
            for (int i = 0; i < NBW; i++) {
                const int blk = wb0 + i;
                if (blk >= NB) continue;
                const int n = 16 * blk + 4 * g;
                float ws[4], bv[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    ws[e] = h2f(sws[n + e]);
                    bv[e] = h2f(sbias[n + e]);
                }
#pragma unroll
                for (int j = 0; j < kTB; j++) {
                    const int m = m0 + 16 * j + r16;
                    if (m >= M) continue;
                    const float as = sc[16 * j + r16];
                    *reinterpret_cast<uint2*>(out + static_cast<size_t>(m) * N + n) =
                        dequant4_pk(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3], as, ws, bv);
                }
            }
        }
    };

    // Producer and consumer waves run separate tile loops with the same number of barriers
    // (one before the first tile, one after each tile), so each side's registers and hoisted
    // addresses stay its own. The barrier waits for LDS traffic only: the producer's prefetch
    // loads stay in flight across it.
    auto barrier = [] {
        __builtin_amdgcn_s_waitcnt(0xC07F);      // lgkmcnt(0)
        lds_barrier();
    };
    const int grid = static_cast<int>(gridDim.x);
    int tile = blockIdx.x;
    if (wave >= 4) {
        const int rp = (wave - 4) * kRowsPerProducer;
        // The lane id passes through an opaque copy at every tile, so the per-lane load and LDS
        // store offsets are derived per tile rather than hoisted out of the loop as
        // 4 x kRowsPerProducer live registers.
        int ln = lane;
        uint4 v[2][kR][NV];
        // Tile i of this workgroup uses buffer i & 1 and enters with parity (i * kBatches) & 1;
        // the loop is unrolled by two so both are compile-time.
        using P0 = std::integral_constant<int, 0>;
        using P1 = std::integral_constant<int, kBatches & 1>;
        load_batch(ln, tile * BT, rp, v[0]);
        quantize_tile(P0{}, tile, 0, tile + grid, ln, rp, v);
        barrier();
        while (tile < tiles) {
            int next = tile + grid;
            if (next < tiles) quantize_tile(P1{}, next, 1, next + grid, ln, rp, v);
            barrier();
            tile = next;
            if (tile >= tiles) break;
            next = tile + grid;
            if (next < tiles) quantize_tile(P0{}, next, 0, next + grid, ln, rp, v);
            barrier();
            tile = next;
        }
    } else {
        barrier();
        for (int it = 0; tile < tiles; it++, tile += grid) {
            compute_tile(tile, it & 1, wave);
            barrier();                           // buffer it&1 is free, buffer (it+1)&1 is complete
        }
    }
}

// The fused kernel's weights in fragment order: for 16-row block b and 128-deep step s, the
// 1 KB at (b * KS + s) * 1024 holds the SMFMAC A operand in lane order, lane 16 g + r at byte
// 16 (16 g + r): row 16 b + r, compressed bytes 64 s + 16 g .. + 15 of W_comp (N, K/2). One
// thread per 16-byte unit, read in W_comp's order.
__global__ __launch_bounds__(256) void fq_pack_weights_kernel(const int8_t* __restrict__ W_comp, int8_t* __restrict__ dst,
                                                              int N, int K)
{
    const int upr = K / 32;                      // 16-byte units per row
    const long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= static_cast<long long>(N) * upr) return;
    const int row = static_cast<int>(i / upr), u = static_cast<int>(i % upr);
    const int s = u >> 2, g = u & 3;
    const size_t o = (static_cast<size_t>(row >> 4) * (K / kSpStep) + s) * 64 + 16 * g + (row & 15);
    reinterpret_cast<uint4*>(dst)[o] = reinterpret_cast<const uint4*>(W_comp)[i];
}

// Packed weights live in static device slots owned per launch key (stream_slots.h), so the
// fused path allocates nothing and leaves the caller's scratch buffers untouched (the
// reference's contract for it). A launch without a slot, or with weights beyond a slot, reads
// W_comp in place (same bits).
constexpr int kFqPackSlots = kFqPackSlotCount;   // one per stream and per graph capture, as the decode K split's
constexpr size_t kFqPackBytes = size_t(1) << 20;   // N * K / 2: 1280 x 1638, 2048 x 1024
static __device__ __align__(16) int8_t g_fq_pack[kFqPackSlots * kFqPackBytes];

namespace {
std::mutex g_fq_mu;
int8_t* g_fq_pack_dev[kSlotMaxDev];
SlotOwners<kFqPackSlots> g_fq_slots;

// Resolves the pack array of device dev (g_fq_mu held); false if it cannot be resolved.
bool fq_pack_resolve(int dev)
{
    if (g_fq_pack_dev[dev]) return true;
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_fq_pack)) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    g_fq_pack_dev[dev] = static_cast<int8_t*>(p);
    return true;
}

// The pack slot of the launch key of s on the current device, or nullptr (no packing): every
// slot held by other keys, a key that cannot be formed, or the array not resolved yet while s
// captures a graph (forge_init resolves it outside any capture).
int8_t* fq_pack_slot(hipStream_t s)
{
    int dev = 0;
    SlotKey key{};
    if (!slot_device(&dev) || !slot_key(s, &key)) return nullptr;
    std::lock_guard<std::mutex> lock(g_fq_mu);
    if (!g_fq_pack_dev[dev] && (key.capture != 0 || !fq_pack_resolve(dev))) return nullptr;
    const int slot = g_fq_slots.take(dev, key);
    return slot < 0 ? nullptr : g_fq_pack_dev[dev] + static_cast<size_t>(slot) * kFqPackBytes;
}
}  // namespace

int fq_pack_slots_used(int dev)
{
    std::lock_guard<std::mutex> lock(g_fq_mu);
    return g_fq_slots.used(dev);
}

int fq_pack_prepare()
{
    int dev = 0;
    if (!slot_device(&dev)) return FORGE_ENODEV;
    std::lock_guard<std::mutex> lock(g_fq_mu);
    return fq_pack_resolve(dev) ? FORGE_OK : FORGE_ENODEV;
}

// Token rows per tile: the tallest of 64 / 48 / 32 whose two buffers and the scale strips fit.
static int fq_bt(int K, int N) {
    for (int bt : {64, 48, 32}) {
        const size_t need = 2 * static_cast<size_t>(bt) * K + 2 * bt * sizeof(float) + 4 * static_cast<size_t>(N);
        if (need <= static_cast<size_t>(kFqLds)) return bt;
    }
    return 0;
}

static size_t fq_lds_bytes(int K, int N, int bt) {
    return 2 * static_cast<size_t>(bt) * K + 2 * bt * sizeof(float) + 4 * static_cast<size_t>(N);
}

// Whether the fused kernel applies: K a multiple of the 128-deep step and at most kFqMaxK, a
// token tile that fits twice in LDS, 16-byte aligned activations and weights, 8-byte aligned
// output.
static bool fq_fits(const void* x, const void* W_comp, const void* out, int K, int N) {
    return K % kSpStep == 0 && K <= kFqMaxK && fq_bt(K, N) > 0 && aligned(x, 16) && aligned(W_comp, 16) &&
           aligned(out, 8);
}

// Automatic path choice (the role of the reference's sp_use_fused, int8_sparse.cu:926-938).
// The two-pass path writes an INT8 copy of x and reads it back (2*M*K extra DRAM bytes once
// x and its copy, 3*M*K, outgrow the 256 MB MALL); the fused kernel instead re-streams the
// packed weights (N*K*5/8 bytes with the index words) from L2 for every tile of token rows, so
// its consumer work grows with N. Fitted to 160 measured shapes on MI355X (M = 65,536 ..
// 262,144; K = 640 .. 2048; N = 128 .. 1024; fused vs two-pass, us): fused for N <= 640 once
// M*K >= 50M (147,456 x 1280 -> 320: 147 vs 196; 147,456 x 1024 -> 256: 106 vs 144; below the
// threshold two-pass wins, 65,536 x 640 -> 320: 46 vs 53), and for N up to 1024 at K <= 1536
// once M*K >= 150M (147,456 x 1024 -> 1024: 251 vs 264; 98,304 x 1280 -> 1024: 221 vs 201 and
// every K = 2048, N = 1024 shape go two-pass). Over the sweep this rule is 0.16 % slower in total
// than the faster path at every shape (7 shapes more than 2 % off).
static bool fq_pays(int M, int K, int N) {
    if (K % kSpStep != 0 || K > kFqMaxK || fq_bt(K, N) == 0) return false;
    const double mk = static_cast<double>(M) * K;
    if (N <= 640) return mk >= 50e6;
    return N <= 1024 && K <= 1536 && mk >= 150e6;
}

template <int NBW, int BT, bool PACKED, int NV>
static int launch_fq_kernel(const uint16_t* x, const int8_t* W, const uint32_t* meta, const uint16_t* w_scale,
                            const uint16_t* bias, uint16_t* out, int M, int K, int N, int cu, hipStream_t s)
{
    // The output staging strips from K = 1024 on, when they fit beside the token tiles and the
    // output takes 16-byte stores. Measured at M = 147,456 (without -> with, us): 1280 -> 320
    // 141 -> 136, 2048 -> 256 180 -> 177, 1024 -> 320 even; at K = 640, where the producer's
    // share of each tile is largest, they cost time (640 -> 320 97.5 -> 99, 640 -> 480 at
    // M = 98,304 66.4 -> 70.5).
    const size_t base = (fq_lds_bytes(K, N, BT) + 15) & ~static_cast<size_t>(15);
    const size_t strips = 4 * static_cast<size_t>(BT) * (NBW * 16 + 8) * sizeof(uint16_t);
    const int stg = K >= 1024 && aligned(out, 16) && base + strips <= static_cast<size_t>(kFqLds) ? 1 : 0;
    const size_t lds = stg ? base + strips : fq_lds_bytes(K, N, BT);
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&sparse_fq_kernel<NBW, BT, PACKED, NV>), hipFuncAttributeMaxDynamicSharedMemorySize,
        kFqLds);
    if (attr != hipSuccess) return static_cast<int>(attr);
    const int tiles = divup(M, BT);
    const int grid = std::min(tiles, cu);     // one 8-wave workgroup per CU
    sparse_fq_kernel<NBW, BT, PACKED, NV><<<grid, 512, lds, s>>>(x, W, meta, w_scale, bias, out, M, K, N, tiles, stg);
    return launch_status();
}

template <int NBW, int BT, int NV>
static int launch_fq(const uint16_t* x, const int8_t* W_comp, const uint32_t* meta, const uint16_t* w_scale,
                     const uint16_t* bias, uint16_t* out, int M, int K, int N, hipStream_t s)
{
    int st = FORGE_OK;
    const int cu = device_info(&st).cu_count;
    if (st != FORGE_OK) return st;
    int8_t* pk = static_cast<size_t>(N) * K / 2 <= kFqPackBytes ? fq_pack_slot(s) : nullptr;
    if (!pk) {
        note_route("fused-quantize");
        return launch_fq_kernel<NBW, BT, false, NV>(x, W_comp, meta, w_scale, bias, out, M, K, N, cu, s);
    }
    note_route("fused-quantize packed");
    const long long units = static_cast<long long>(N) * (K / 32);
    fq_pack_weights_kernel<<<static_cast<unsigned>(divupll(units, 256)), 256, 0, s>>>(W_comp, pk, N, K);
    if ((st = launch_status()) != FORGE_OK) return st;
    return launch_fq_kernel<NBW, BT, true, NV>(x, pk, meta, w_scale, bias, out, M, K, N, cu, s);
}

template <int BT, int NV>
static int launch_fq_nbw(const uint16_t* x, const int8_t* W_comp, const uint32_t* meta, const uint16_t* w_scale,
                         const uint16_t* bias, uint16_t* out, int M, int K, int N, hipStream_t s)
{
    // Weight blocks per consumer wave per pass: all of N in one pass up to kMax blocks per wave,
    // several passes of kMax beyond. kMax keeps the accumulators (NBW x BT/16 blocks) and the
    // fragment ring within the 256 registers of a wave at 2 waves per SIMD (no spills).
    constexpr int kMax = BT == 64 ? 4 : (BT == 48 ? 5 : 6);
    const int per_wave = divup(N / 16, 4);
    if (per_wave <= 1) return launch_fq<1, BT, NV>(x, W_comp, meta, w_scale, bias, out, M, K, N, s);
    if (per_wave <= 2) return launch_fq<2, BT, NV>(x, W_comp, meta, w_scale, bias, out, M, K, N, s);
    if (per_wave <= 3) return launch_fq<3, BT, NV>(x, W_comp, meta, w_scale, bias, out, M, K, N, s);
    if (per_wave <= 4 || kMax == 4) return launch_fq<4, BT, NV>(x, W_comp, meta, w_scale, bias, out, M, K, N, s);
    if constexpr (kMax >= 5) {
        if (per_wave <= 5 || kMax == 5)
            return launch_fq<5, BT, NV>(x, W_comp, meta, w_scale, bias, out, M, K, N, s);
    }
    if constexpr (kMax >= 6) return launch_fq<6, BT, NV>(x, W_comp, meta, w_scale, bias, out, M, K, N, s);
    return FORGE_EINVAL;
}

// Vectors per lane (NV) from K: 2 up to K = 1024, 3 up to 1536, 4 up to the 2048 limit. The
// 64-row tile exists only for K <= 1152 (two tiles in LDS) and the 32-row tile in practice only
// near K = 2048, so those build the NV values they can meet (a larger NV is always correct).
template <int BT>
static int launch_fq_bt(const uint16_t* x, const int8_t* W_comp, const uint32_t* meta, const uint16_t* w_scale,
                        const uint16_t* bias, uint16_t* out, int M, int K, int N, hipStream_t s)
{
    const int nv = K <= 1024 ? 2 : (K <= 1536 ? 3 : 4);
    if constexpr (BT != 32) {
        if (nv == 2) return launch_fq_nbw<BT, 2>(x, W_comp, meta, w_scale, bias, out, M, K, N, s);
        if (nv == 3) return launch_fq_nbw<BT, 3>(x, W_comp, meta, w_scale, bias, out, M, K, N, s);
    }
    if constexpr (BT != 64) return launch_fq_nbw<BT, 4>(x, W_comp, meta, w_scale, bias, out, M, K, N, s);
    return FORGE_EINVAL;                         // unreachable: two 64-row tiles need K <= 1152
}

static int launch_sparse_fq(const uint16_t* x, const int8_t* W_comp, const uint32_t* meta, const uint16_t* w_scale,
                            const uint16_t* bias, uint16_t* out, int M, int K, int N, hipStream_t s)
{
    switch (fq_bt(K, N)) {
        case 64: return launch_fq_bt<64>(x, W_comp, meta, w_scale, bias, out, M, K, N, s);
        case 48: return launch_fq_bt<48>(x, W_comp, meta, w_scale, bias, out, M, K, N, s);
        case 32: return launch_fq_bt<32>(x, W_comp, meta, w_scale, bias, out, M, K, N, s);
        default: return FORGE_EINVAL;
    }
}

}  // namespace forge_amd

using namespace forge_amd;

extern "C" int forge_sparse_int8_gemm_plan(int M, int K, int N_out, int split_k, int have_workspace,
                                           int tile, int* out_tile, int* out_split_k)
{
    if (!out_tile || !out_split_k) return FORGE_EINVAL;
    sparse_plan_cost(std::max(M, 1), std::max(K, 1), std::max(N_out, 1), split_k, have_workspace != 0, tile,
                     cu_count_or_default(), out_tile, out_split_k);
    return FORGE_OK;
}

extern "C" int forge_sparse_int8_gemm(const int8_t* W_comp, const int8_t* x, const uint32_t* w_meta,
                                      const float* act_scale, const uint16_t* w_scale,
                                      const uint16_t* bias, uint16_t* out, int M, int K, int N_out,
                                      float* splitk_workspace, int split_k, void* stream, int tile)
{
    if (M <= 0 || K <= 0 || N_out <= 0) return FORGE_OK;
    if (!W_comp || !x || !w_meta || !act_scale || !w_scale || !out) return FORGE_EINVAL;
    if (splitk_workspace && !aligned(splitk_workspace, 16)) return FORGE_EINVAL;
    return sparse_gemm(W_comp, x, w_meta, act_scale, w_scale, bias, out, nullptr, M, K, N_out,
                       reinterpret_cast<int32_t*>(splitk_workspace), split_k, tile, as_stream(stream));
}

extern "C" int forge_sparse_int8_gemm_s32(const int8_t* W_comp, const int8_t* x, const uint32_t* w_meta,
                                          int32_t* C, int M, int K, int N_out, void* stream)
{
    if (M <= 0 || K <= 0 || N_out <= 0) return FORGE_OK;
    if (!W_comp || !x || !w_meta || !C) return FORGE_EINVAL;
    return sparse_gemm(W_comp, x, w_meta, nullptr, nullptr, nullptr, nullptr, C, M, K, N_out, nullptr, 1,
                       -1, as_stream(stream));
}

// Whether the automatic path of sparse_int8_linear (with no split-K asked for, and aligned
// operands) takes a fused quantize + GEMM kernel at this shape (reference sp_use_fused,
// int8_sparse.cu:926-938): the decode kernel with its quantize prologue at decode shapes, the
// persistent fused kernel where the MI355X chooser fq_pays says so.
extern "C" int forge_sparse_int8_linear_fused(int M, int K, int N_out, int* out_flag)
{
    if (!out_flag) return FORGE_EINVAL;
    const bool ok = M > 0 && N_out > 0 && N_out % 16 == 0 && K > 0 && K % 64 == 0;
    *out_flag = (ok && (decode_fq_supported(M, K, true) || fq_pays(M, K, N_out))) ? 1 : 0;
    return FORGE_OK;
}

extern "C" int forge_sparse_int8_linear(const uint16_t* x, const int8_t* W_comp, const uint32_t* w_meta,
                                        const uint16_t* w_scale, const uint16_t* bias, uint16_t* out,
                                        int M, int K, int N_out, int8_t* scratch_q, float* scratch_scale,
                                        float* splitk_workspace, int split_k, void* stream, int path)
{
    if (M <= 0 || K <= 0 || N_out <= 0) return FORGE_OK;
    if (!x || !W_comp || !w_meta || !w_scale || !out || !scratch_q || !scratch_scale) return FORGE_EINVAL;
    if (K % 64 != 0 || N_out % 16 != 0) return FORGE_EINVAL;
    hipStream_t s = as_stream(stream);
    // int8_sparse.cu:1022-1033: the fused kernel when forced (path 1) or, on auto (-1) with no
    // split-K asked for, when it pays; it needs its shape and alignment, else two-pass. Every
    // path gives the same bits.
    // Decode shapes on the fused path: the decode kernel quantizes the few token rows in its
    // prologue (one kernel instead of two); like the reference's fused path it leaves the scratch
    // buffers untouched (int8_sparse.cuh:87-89).
    if ((path == 1 || (path == -1 && split_k <= 1)) && decode_fq_supported(M, K, true) && aligned(x, 16) &&
        aligned(W_comp, 16) && aligned(w_meta, 16)) {
        note_route("decode+quantize");
        return launch_decode_fq(x, W_comp, w_meta, w_scale, bias, out, nullptr, nullptr, M, K, N_out, true, s);
    }
    if (fq_fits(x, W_comp, out, K, N_out) &&
        (path == 1 || (path == -1 && split_k <= 1 && fq_pays(M, K, N_out)))) {
        return launch_sparse_fq(x, W_comp, w_meta, w_scale, bias, out, M, K, N_out, s);
    }
    int st = launch_quantize(x, scratch_q, scratch_scale, M, K, s);
    if (st != FORGE_OK) return st;
    return sparse_gemm(W_comp, scratch_q, w_meta, scratch_scale, w_scale, bias, out, nullptr, M, K, N_out,
                       reinterpret_cast<int32_t*>(splitk_workspace), split_k, -1, s);
}

extern "C" int forge_splitk_reduce(const float* workspace, const uint16_t* bias, uint16_t* out, int M,
                                   int N_out, void* stream)
{
    if (M <= 0 || N_out <= 0) return FORGE_OK;
    if (!workspace || !out) return FORGE_EINVAL;
    const long long total = static_cast<long long>(M) * N_out;
    if (N_out % 4 == 0 && total / 4 < (1LL << 31) && aligned(workspace, 16) && aligned(out, 8) &&
        (!bias || aligned(bias, 8))) {
        const long long total4 = total / 4;
        const int blocks = static_cast<int>(std::min<long long>(divupll(total4, 256), 16384));
        splitk_reduce_vec4_kernel<<<blocks, 256, 0, as_stream(stream)>>>(
            reinterpret_cast<const float4*>(workspace), bias, reinterpret_cast<uint2*>(out),
            static_cast<uint32_t>(N_out / 4), static_cast<uint32_t>(total4));
        return launch_status();
    }
    const int blocks = static_cast<int>(std::min<long long>(divupll(total, 256), 8192));
    splitk_reduce_f32_kernel<<<blocks, 256, 0, as_stream(stream)>>>(workspace, bias, out, N_out, total);
    return launch_status();
}
