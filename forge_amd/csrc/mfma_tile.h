// LDS-staged INT8 MFMA tile engine for gfx950 (v_mfma_i32_32x32x32_i8).
//
// One workgroup computes a BM x BN INT32 tile of C = A (rows, K) x B (cols, K)^T with
// both operands K-contiguous ("NT", the layout of the reference's int8 GEMMs:
// include/forge/gemm/int8_dense.cuh:9-11). WM x WN wavefronts each own a
// (BM/WM) x (BN/WN) sub-tile of 32x32 MFMA blocks held in accumulator registers.
//
// K advances in 64-byte stages. A and B stages live in LDS as rows of 64 bytes (four
// 16-byte chunks); chunk c of row r is stored at chunk position c ^ swz(r), with
// swz(r) = ((r >> 1) ^ (r >> 3)) & 3. An MFMA operand read (lane l -> row l%32,
// chunk 2*ks + l/32, one ds_read_b128) then touches 8 (or 16) distinct 16-byte bank
// groups per 8-lane (16-lane) phase: bank-conflict free for 32 or 64 banks, and the
// 16-byte ds_write_b128 stores of a stage are conflict free as well.
//
// Two LDS buffers and register prefetch: the global loads of stage k+1 are issued
// before the MFMAs of stage k and written to the other buffer after them, so one
// barrier per stage orders everything.
//
// Operand K mapping: for MFMA operands A (32 rows x 32 K) and B (32 cols x 32 K) each
// lane supplies 16 bytes; lanes l and l+32 cover the two 16-byte halves of the 32-K
// sub-step. A and B use the same (lane, byte) -> k assignment, and an integer dot
// product is invariant under a common permutation of k, so results are exact whatever
// order the hardware uses inside a lane.
// Accumulator layout of a 32x32 block (lane l, register e = 0..15):
//     row = 8*(e/4) + 4*(l/32) + (e%4),  col = l%32.
#pragma once

#include "common.h"

namespace forge_amd {

constexpr int kBK = 64;   // K bytes per pipeline stage

__device__ __forceinline__ int lds_swz(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }
__device__ __forceinline__ int lds_off(int r, int c) { return r * kBK + ((c ^ lds_swz(r)) << 4); }

__device__ __forceinline__ int acc_row(int e, int lane) { return 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3); }
__device__ __forceinline__ int acc_col(int lane) { return lane & 31; }

// ---- operand loaders: fetch one 16-byte chunk (row r of the tile, chunk c of stage k0) ----

// Row-major (rows, K) int8 matrix; vector path needs K % 16 == 0 and a 16-byte base.
struct RowMajorLoader {
    const int8_t* p;
    int rows;   // valid rows
    int K;
    __device__ __forceinline__ int4 load(int row, int k, bool vec) const {
        if (row >= rows || k >= K) return make_int4(0, 0, 0, 0);
        const int8_t* src = p + static_cast<size_t>(row) * K + k;
        if (vec) return *reinterpret_cast<const int4*>(src);
        int4 v = make_int4(0, 0, 0, 0);
        int8_t* b = reinterpret_cast<int8_t*>(&v);
        const int n = (K - k) < 16 ? (K - k) : 16;
        for (int i = 0; i < n; i++) b[i] = src[i];
        return v;
    }
};

// Implicit im2col of an NHWC int8 image: row = output pixel (n, ho, wo), k = (kh*kW+kw)*C + c.
// Vector path needs C % 16 == 0 (a chunk never straddles two taps) and a 16-byte base.
struct ConvLoader {
    const int8_t* x;
    int rows;   // N * Ho * Wo
    int K;      // kH * kW * C
    int H, W, C, Ho, Wo, kW;
    int padH, padW, strideH, strideW, dilH, dilW;
    __device__ __forceinline__ int4 load(int row, int k, bool vec) const {
        int4 v = make_int4(0, 0, 0, 0);
        if (row >= rows || k >= K) return v;
        const int wo = row % Wo;
        const int t0 = row / Wo;
        const int ho = t0 % Ho;
        const int n = t0 / Ho;
        if (vec) {
            const int tap = k / C, c = k - tap * C;
            const int kh = tap / kW, kw = tap - kh * kW;
            const int hi = ho * strideH + kh * dilH - padH;
            const int wi = wo * strideW + kw * dilW - padW;
            if (hi < 0 || hi >= H || wi < 0 || wi >= W) return v;
            return *reinterpret_cast<const int4*>(x + ((static_cast<size_t>(n) * H + hi) * W + wi) * C + c);
        }
        int8_t* b = reinterpret_cast<int8_t*>(&v);
        for (int i = 0; i < 16 && k + i < K; i++) {
            const int kk = k + i;
            const int tap = kk / C, c = kk - tap * C;
            const int kh = tap / kW, kw = tap - kh * kW;
            const int hi = ho * strideH + kh * dilH - padH;
            const int wi = wo * strideW + kw * dilW - padW;
            if (hi >= 0 && hi < H && wi >= 0 && wi < W)
                b[i] = x[((static_cast<size_t>(n) * H + hi) * W + wi) * C + c];
        }
        return v;
    }
};

// ---- the tile engine -------------------------------------------------------------

template <int BM, int BN, int WM, int WN>
struct MfmaTile {
    static constexpr int kThreads = WM * WN * kWave;
    static constexpr int kTM = BM / WM / 32;       // 32x32 blocks per wave along rows
    static constexpr int kTN = BN / WN / 32;       // ... along cols
    static constexpr int kAChunks = BM * 4 / kThreads;   // 16-byte chunks per thread per stage
    static constexpr int kBChunks = BN * 4 / kThreads;
    static constexpr int kLdsBytes = 2 * (BM + BN) * kBK;
    static_assert(kTM >= 1 && kTN >= 1, "wave tile must hold a 32x32 block");
    static_assert(BM * 4 % kThreads == 0 && BN * 4 % kThreads == 0, "stage must split evenly");

    v16i acc[kTM][kTN];

    // Runs the K loop for the tile whose first row/col are (m0, n0); ALoader/BLoader are
    // addressed with tile-relative rows offset by m0/n0.
    template <class ALoader, class BLoader>
    __device__ __forceinline__ void run(const ALoader& la, const BLoader& lb, int m0, int n0,
                                        int K, bool vec, int8_t* lds) {
        const int tid = threadIdx.x;
        const int lane = tid & (kWave - 1);
        const int wave = tid / kWave;
        const int wm = (wave / WN) * (BM / WM);
        const int wn = (wave % WN) * (BN / WN);
        int8_t* As = lds;
        int8_t* Bs = lds + 2 * BM * kBK;

#pragma unroll
        for (int i = 0; i < kTM; i++)
#pragma unroll
            for (int j = 0; j < kTN; j++)
#pragma unroll
                for (int e = 0; e < 16; e++) acc[i][j][e] = 0;

        int4 ra[kAChunks], rb[kBChunks];
        auto gload = [&](int k0) {
#pragma unroll
            for (int i = 0; i < kAChunks; i++) {
                const int id = tid + i * kThreads;
                ra[i] = la.load(m0 + (id >> 2), k0 + ((id & 3) << 4), vec);
            }
#pragma unroll
            for (int i = 0; i < kBChunks; i++) {
                const int id = tid + i * kThreads;
                rb[i] = lb.load(n0 + (id >> 2), k0 + ((id & 3) << 4), vec);
            }
        };
        auto lstore = [&](int buf) {
            int8_t* a = As + buf * BM * kBK;
            int8_t* b = Bs + buf * BN * kBK;
#pragma unroll
            for (int i = 0; i < kAChunks; i++) {
                const int id = tid + i * kThreads;
                *reinterpret_cast<int4*>(a + lds_off(id >> 2, id & 3)) = ra[i];
            }
#pragma unroll
            for (int i = 0; i < kBChunks; i++) {
                const int id = tid + i * kThreads;
                *reinterpret_cast<int4*>(b + lds_off(id >> 2, id & 3)) = rb[i];
            }
        };

        const int kt_total = divup_dev(K, kBK);
        gload(0);
        lstore(0);
        __syncthreads();
        for (int kt = 0; kt < kt_total; kt++) {
            const int cur = kt & 1;
            const bool more = (kt + 1) < kt_total;
            if (more) gload((kt + 1) * kBK);
            const int8_t* a = As + cur * BM * kBK;
            const int8_t* b = Bs + cur * BN * kBK;
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                const int c = 2 * ks + (lane >> 5);
                v4i fa[kTM], fb[kTN];
#pragma unroll
                for (int i = 0; i < kTM; i++)
                    fa[i] = *reinterpret_cast<const v4i*>(a + lds_off(wm + 32 * i + (lane & 31), c));
#pragma unroll
                for (int j = 0; j < kTN; j++)
                    fb[j] = *reinterpret_cast<const v4i*>(b + lds_off(wn + 32 * j + (lane & 31), c));
#pragma unroll
                for (int i = 0; i < kTM; i++)
#pragma unroll
                    for (int j = 0; j < kTN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
            }
            if (more) lstore(cur ^ 1);
            __syncthreads();
        }
    }

    __device__ static __forceinline__ int divup_dev(int a, int b) { return (a + b - 1) / b; }
};

// Tile index -> (tile_m, tile_n): consecutive workgroups land on different XCDs
// (dispatch is round-robin over the 8 XCDs), so the linear id is first regrouped so each
// XCD receives a contiguous run, then runs are rasterised in groups of kGroupM tile-rows:
// an XCD's L2 then holds a few A row-blocks and B col-blocks instead of all of them.
__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
    constexpr int kXcd = 8, kGroupM = 4;
    const int total = tiles_m * tiles_n;
    int t = bid;
    if (total % kXcd == 0) t = (bid % kXcd) * (total / kXcd) + bid / kXcd;
    const int per_group = kGroupM * tiles_n;
    const int group = t / per_group;
    const int first_m = group * kGroupM;
    const int gm = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
    const int r = t - group * per_group;
    tm = first_m + r % gm;
    tn = r / gm;
}

}  // namespace forge_amd
