// Decode-shape (M <= 16 tokens) INT8 GEMMs for gfx950, dense and 2:4 sparse: weight
// streaming at HBM rate.
//
// Reference shapes: configs[3] of the reference's decode use (sparse_int8_linear / int8_linear
// with a handful of tokens, src/gemm/int8_sparse.cu:1005-1043, src/gemm/int8_dense.cu:213-232),
// where the weights are read once per call and every other operand is tiny.
//
// Dense (decode_dense_kernel): a workgroup owns 32 weight rows (16 for up to 4 tokens) and all
// of K; its wavefronts (8 with 32 rows, 4 with 16) split K into contiguous slices of 128-deep
// stages.
// Operands are loaded straight into registers with coalesced 8-row x 128-byte instructions
// (non-temporal for the weights, which are read once), rearranged into the matrix-core layout
// by one DPP lane swap, and fed to v_mfma_i32_16x16x64_i8. Measured on MI355X, this streams a
// 64 MB weight matrix from HBM faster than staging it through LDS: coalesced register loads at
// this shape reach ~6 TB/s in isolation, LDS DMA rings of any shape stay under 4.8 TB/s.
//
// Sparse with K % 256 == 0 (decode_sparse_reg_kernel): the dense kernel's structure on 256-deep
// segments of compressed rows, with a K permutation that keeps the SMFMAC operands consistent
// (described at the kernel). The same kernel serves 16 < M <= 64 tokens of the sparse GEMM with
// TB = 2 or 4 token blocks per weight fragment (launch_skinny_tb).
//
// Sparse with K % 256 == 128 (decode_sparse_kernel): a 512-thread workgroup owns 32 weight rows and all of K; its 8
// wavefronts split K into 128-deep stages, each wave streaming its slice of the compressed
// rows, index words and token rows through a PRIVATE LDS ring with global_load_lds_dwordx4,
// so only the wave's own vmcnt orders the ring -- no barrier in the K loop (4 slots of
// 4.5 KB, 3 stages in flight per wave). Stages feed 2 v_smfmac_i32_16x16x128_i8 (compressed
// weights + index words as A, lane layout as in gemm_sparse.hip).
//
// Both: the per-wave INT32 partials are summed exactly through LDS, then the dequant epilogue
// writes the outputs. Each wave's stage count is padded to S in {1, 2, 4, 8, 16} (K <= 8192):
// padding stages re-read the wave's last real stage and multiply it by zero tokens, and the
// per-wave stage sequence is unrolled, so it has no branches, constant ring slots and exact
// waits.
#include "common.h"
#include "gemm_dense.h"
#include "mfma_tile.h"
#include "stream_slots.h"

#include <mutex>

namespace forge_amd {

// Sparse decode geometry.
constexpr int kDecRows = 32;       // weight rows per workgroup
constexpr int kDecWaves = 8;
constexpr int kDecTokRows = 16;    // token rows staged per stage (the MFMA's 16 columns)
// Dense decode geometry: 16-row blocks per workgroup, waves (K split), stages in flight.
constexpr int kDecDenseBlocks = 2;
constexpr int kDecDenseOneBlockMaxM = 4;   // one 16-row block per workgroup up to this many tokens
constexpr int kDecDenseWaves = 4;
constexpr int kDecDenseWavesTwoBlock = 8;   // 8 tokens and more: measured 17.96 -> 17.47 us at M = 16
                                            // (graph-replayed int8_linear); 4 waves stay faster at M <= 4
constexpr int kDecDenseAhead = 6;
constexpr int kDecSparseRegMaxM = 16;   // register sparse kernel up to this many tokens

struct SparseDecodeCfg {
    // Per-wave ring slot: 32 rows x 64 compressed bytes, 2 x 64 index words, then the stage's
    // 16 token rows x 128 B.
    static constexpr int kWBytes = kDecRows * 64;
    static constexpr int kIBytes = 2 * 256;
    static constexpr int kXBytes = kDecTokRows * 128;
    static constexpr int kSlotBytes = kWBytes + kIBytes + kXBytes;
    static constexpr int kSlots = 4;                             // ring depth: 144 KB of LDS
    static constexpr int kWIns = kWBytes / 1024;                 // 1 KB DMA instructions per stage
    static constexpr int kVmPerStage = kWIns + 1 + kXBytes / 1024;
    static_assert(kDecWaves * kSlots * kSlotBytes <= 160 * 1024, "ring fits in LDS");
    static_assert(kDecWaves * 2 * 64 * 16 <= kDecWaves * kSlotBytes, "reduction area fits in slot 0");
};

// LDS byte offset of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p)
{
    using lds_ptr = const __attribute__((address_space(3))) int8_t*;
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr)(p)));
}

// Reads of a ring slot, complete on return. Each is one asm block, so the compiler sees no
// LDS read that might alias a DMA in flight (it would wait for all of them) and no register
// written asynchronously; the ring's own vmcnt waits order the reads after the slot's DMA.
__device__ __forceinline__ void lds_read4(const int8_t* p0, const int8_t* p1, const int8_t* p2, const int8_t* p3,
                                          v4i& a0, v4i& a1, v4i& a2, v4i& a3)
{
    asm volatile("ds_read_b128 %0, %4\n\tds_read_b128 %1, %5\n\tds_read_b128 %2, %6\n\tds_read_b128 %3, %7\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(a0), "=&v"(a1), "=&v"(a2), "=&v"(a3)
                 : "v"(lds_addr(p0)), "v"(lds_addr(p1)), "v"(lds_addr(p2)), "v"(lds_addr(p3))
                 : "memory");
}
__device__ __forceinline__ void lds_read_idx(const uint32_t* q0, const uint32_t* q1, int& i0, int& i1)
{
    asm volatile("ds_read_b32 %0, %2\n\tds_read_b32 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(i0), "=&v"(i1) : "v"(lds_addr(q0)), "v"(lds_addr(q1)) : "memory");
}

// S: stages per wave after padding (1, 2, 4 or 8). The per-wave stage sequence is
// straight-line code with constant ring slots; every load in it is a DMA into LDS, so the only
// vmcnt waits are the ring's own (whole stages, counted from the end).
// K split across the workgroups of one row block: acc holds gridDim.x x RB x 256 INT32 sums
// (16 x 16 outputs per 16-row block), cnt one arrival counter per row block; both are zero
// between launches (the last workgroup of a row block leaves them so).
struct KSplit {
    int* acc;
    unsigned* cnt;
};

// Exact INT32 hand-off between the KP workgroups of a row block, through device-scope atomics
// only (no cache write-back or invalidate fences, which stall every workgroup on the XCD):
// every workgroup adds its lane partials (per thread NQ 16 x 16 output blocks; block i when
// has[i], at sum slot blk[i]) into the row block's sums, waits for the adds to complete, and one thread counts the arrival with
// atomicInc(cnt, KP - 1), which wraps the counter back to 0 on the last arrival. Workgroups
// that arrive earlier return false; the last one takes the sums with atomicExch(..., 0), which
// clears them for the next launch, and returns true. No workgroup waits for another, so the
// hand-off cannot stall on a workgroup that is not resident. INT32 addition is associative, so
// the result is exact in any arrival order.
template <int KP, int NQ>
__device__ bool ksplit_handoff(const KSplit& ks, v4i (&sum)[NQ], const bool (&has)[NQ], const int (&blk)[NQ], int lane)
{
    __shared__ int s_last;
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        if (!has[i]) continue;
        int* slot = ks.acc + static_cast<size_t>(blk[i]) * 4 * kWave + lane;
#pragma unroll
        for (int e = 0; e < 4; e++) atomicAdd(slot + e * kWave, sum[i][e]);
    }
    wait_vmcnt<0>();
    __syncthreads();
    if (threadIdx.x == 0) s_last = atomicInc(ks.cnt + blockIdx.x, KP - 1) == KP - 1;
    __syncthreads();
    if (!s_last) return false;
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        if (!has[i]) continue;
        int* slot = ks.acc + static_cast<size_t>(blk[i]) * 4 * kWave + lane;
#pragma unroll
        for (int e = 0; e < 4; e++) sum[i][e] = atomicExch(slot + e * kWave, 0);
    }
    return true;
}

// KP > 1: K split over the KP workgroups blockIdx.y of a row block (ksplit_handoff).
template <bool DEQUANT, int S, int KP = 1>
__global__ __launch_bounds__(kDecWaves * kWave) void decode_sparse_kernel(
    const int8_t* __restrict__ W, const uint32_t* __restrict__ meta, const int8_t* __restrict__ X,
    GemmEpilogue ep, int K, KSplit ks)
{
    using Cfg = SparseDecodeCfg;
    constexpr int D = Cfg::kSlots;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    // One LDS array per ring slot (all waves' copies of that slot): distinct arrays carry
    // distinct alias scopes.
    __shared__ __align__(16) int8_t slot0[kDecWaves * Cfg::kSlotBytes];
    __shared__ __align__(16) int8_t slot1[kDecWaves * Cfg::kSlotBytes];
    __shared__ __align__(16) int8_t slot2[kDecWaves * Cfg::kSlotBytes];
    __shared__ __align__(16) int8_t slot3[kDecWaves * Cfg::kSlotBytes];
    auto slot_base = [&](int slot) -> int8_t* {
        int8_t* b = slot == 0 ? slot0 : slot == 1 ? slot1 : slot == 2 ? slot2 : slot3;
        return b + wave * Cfg::kSlotBytes;
    };
    const int n0 = blockIdx.x * kDecRows;
    const int M = ep.M, N = ep.N;
    const int r16 = lane & 15, g = lane >> 4;

    const int kp = KP > 1 ? static_cast<int>(blockIdx.y) : 0;
    const int k0 = kp * (K / KP);   // whole 128-deep stages: k0 / 2 compressed bytes, k0 / 2 index words

    // This wave's stages [s0, s0 + ns), ns <= S; stages ns..S-1 are padding.
    const int nst = K / KP / 128;
    const int s0 = wave * S < nst ? wave * S : nst;
    const int ns = (s0 + S < nst ? s0 + S : nst) - s0;

    // DMA sources at K stage 0. Lane s of a 1 KB instruction fills LDS bytes [16 s, +16) of
    // its part of the slot: compressed row s >> 2 or token row s >> 3, at the swizzled chunk
    // position.
    const int8_t* pw[Cfg::kWIns];
#pragma unroll
    for (int q = 0; q < Cfg::kWIns; q++) {
        const int s = q * kWave + lane;
        const int r = s >> 2;
        const int c = (s & 3) ^ lds_swz4(r);
        const int gr = (n0 + r) < N ? (n0 + r) : N - 1;
        pw[q] = W + static_cast<size_t>(gr) * (K / 2) + k0 / 2 + 16 * c;
    }
    const int8_t* px[2];
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const int s = q * kWave + lane;
        const int r = s >> 3;
        const int c = (s & 7) ^ lds_swz8(r);
        px[q] = X + static_cast<size_t>(r < M ? r : M - 1) * K + k0 + 16 * c;   // rows >= M: zeroed on read
    }
    // 2 blocks of 16 rows x 64 index words per stage; lanes 0..31 each copy 16 bytes.
    int blk = (n0 >> 4) + ((lane & 31) >> 4);
    blk = blk < (N >> 4) ? blk : (N >> 4) - 1;
    const int8_t* pi = reinterpret_cast<const int8_t*>(meta + static_cast<size_t>(blk) * (K / 2) + k0 / 2) + 16 * (lane & 15);

    auto issue = [&](int t, int slot) {
        const int st = s0 + (t < ns ? t : ns - 1);
        int8_t* dst = slot_base(slot);
#pragma unroll
        for (int q = 0; q < Cfg::kWIns; q++) dma16(pw[q] + st * 64, dst + q * 1024);
        if (lane < 32) dma16(pi + st * 256, dst + Cfg::kWBytes);
#pragma unroll
        for (int q = 0; q < 2; q++) dma16(px[q] + st * 128, dst + Cfg::kWBytes + Cfg::kIBytes + q * 1024);
        // Keep the stages' DMAs in stage order for the counted waits.
        asm volatile("" ::: "memory");
    };

    const bool tok = r16 < M;
    v4i acc[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
    auto compute = [&](int slot, bool real) {
        const int8_t* src = slot_base(slot);
        const int8_t* xs = src + Cfg::kWBytes + Cfg::kIBytes;
        // B: token row r16, K [16g, +16) and [64 + 16g, +16); A: compressed rows, chunk g.
        v4i a0, a1, xlo, xhi;
        lds_read4(src + lds_off64(r16, g), src + lds_off64(16 + r16, g), xs + lds_off128(r16, g),
                  xs + lds_off128(r16, 4 + g), a0, a1, xlo, xhi);
        int i0, i1;
        const uint32_t* idx = reinterpret_cast<const uint32_t*>(src + Cfg::kWBytes);
        lds_read_idx(idx + lane, idx + 64 + lane, i0, i1);
        if (!(tok && real)) {
            xlo = v4i{0, 0, 0, 0};
            xhi = v4i{0, 0, 0, 0};
        }
        const v8i b = __builtin_shufflevector(xlo, xhi, 0, 1, 2, 3, 4, 5, 6, 7);
        acc[0] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(a0, b, acc[0], i0, 0, 0);
        acc[1] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(a1, b, acc[1], i1, 0, 0);
    };

    // Ring of D slots: stage t lives in slot t % D; issuing stage t + D - 1 reuses the slot of
    // stage t - 1, whose reads completed in the previous step. Before computing stage t, the
    // later issued stages (at most D - 1) may still be in flight.
    if (ns > 0) {
#pragma unroll
        for (int t = 0; t < D - 1 && t < S; t++) issue(t, t);
#pragma unroll
        for (int t = 0; t < S; t++) {
            if (t + D - 1 < S) issue(t + D - 1, (t + D - 1) % D);
            const int later = (S - 1 - t) < (D - 1) ? (S - 1 - t) : (D - 1);
            if (later >= 3) wait_vmcnt<3 * Cfg::kVmPerStage>();
            else if (later == 2) wait_vmcnt<2 * Cfg::kVmPerStage>();
            else if (later == 1) wait_vmcnt<Cfg::kVmPerStage>();
            else wait_vmcnt<0>();
            compute(t % D, t < ns);
        }
    }

    // Sum the 8 waves' partials exactly (INT32) through LDS, then the epilogue: lane l of
    // block b holds rows n0 + 16b + 4*(l/16) + e of token l % 16.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    v4i* red = reinterpret_cast<v4i*>(slot0);
    red[(wave * 2 + 0) * kWave + lane] = acc[0];
    red[(wave * 2 + 1) * kWave + lane] = acc[1];
    __syncthreads();
    const int b = threadIdx.x / kWave;
    v4i sum = v4i{0, 0, 0, 0};
    if (threadIdx.x < 2 * kWave) {
#pragma unroll
        for (int w = 0; w < kDecWaves; w++) sum += red[(w * 2 + b) * kWave + lane];
    }
    if constexpr (KP > 1) {
        v4i sums[1] = {sum};
        const bool has[1] = {threadIdx.x < 2 * kWave};
        const int blk[1] = {static_cast<int>(blockIdx.x) * 2 + b};
        if (!ksplit_handoff<KP, 1>(ks, sums, has, blk, lane)) return;
        sum = sums[0];
    }
    if (threadIdx.x < 2 * kWave) {
        const int m = r16;
        if (m < M) {
            const int nb = n0 + 16 * b + 4 * g;
            const float as = DEQUANT ? ep.act_scale[m] : 0.0f;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int n = nb + e;
                if (n >= N) continue;
                const size_t o = static_cast<size_t>(m) * N + n;
                if constexpr (DEQUANT) {
                    const float bv = ep.bias ? h2f(ep.bias[n]) : 0.0f;
                    ep.c16[o] = dequant_gemm(sum[e], as, h2f(ep.w_scale[n]), bv, ep.bias != nullptr);
                } else {
                    ep.c32[o] = sum[e];
                }
            }
        }
    }
}

template <typename T>
__device__ __forceinline__ T ld_stream(const void* p)
{
    return __builtin_nontemporal_load(reinterpret_cast<const T*>(p));
}

// 16 rows x 128 K of a row-major int8 matrix, loaded as two coalesced instructions (rows
// 0..7 and 8..15; lane l reads row l % 8, 16-byte chunk l / 8, so each lane quad covers 64
// contiguous bytes), then rearranged with one 8-lane swap (DPP row_ror:8) into the matrix-core
// layout: lane l = 16 G + 8 b + i holds row l % 16 = 8 b + i, K chunks 2 G (step 0) and
// 2 G + 1 (step 1). Both operands of the 16x16x64 product use this K order, so the dot
// products are unchanged.
__device__ __forceinline__ void swap8_rows(v4i own0, v4i own1, bool hi, v4i& h0, v4i& h1)
{
    const v4i x = hi ? own0 : own1;   // lanes of the low half send rows 8..15, the high half rows 0..7
    v4i y;
#pragma unroll
    for (int k = 0; k < 4; k++) y[k] = __builtin_amdgcn_mov_dpp(x[k], 0x128, 0xF, 0xF, false);
    h0 = hi ? y : own0;
    h1 = hi ? own1 : y;
}

// Fused quantize prologue of the decode kernels (M <= kDecodeFqMaxM = 2 tokens, the
// int8_linear / sparse_int8_linear entry points): the workgroup quantizes the FP16 token rows
// (fq.x, (M, K), K % 8 == 0, 16-byte aligned) into LDS rows of stride K + kFqPad, with the
// arithmetic of quantize_rows_block_kernel -- the row absmax as a packed u16 maximum of fp16
// magnitude bit patterns (two rows per DPP wave reduction), the fp32 maximum for a row that
// holds a NaN, quant8_row -- so the INT8 tokens and scales are bit-identical to the quantize
// kernel's. Thread t holds vectors t, t + 256, ... (VPR per row) of every row, loaded before any
// use; loads past the row end re-read its last vector, rows past M re-read row M - 1 (neither
// changes a result). When fq.q is set, workgroup 0 also writes the INT8 rows and the scales to
// the caller's scratch, as the two-pass path leaves them there (int8_linear); the sparse fused
// path leaves the scratch untouched, as the reference's does. The 128-byte row padding puts the two token
// rows of a 16-lane LDS read phase in different bank halves.
struct FqArgs {
    const uint16_t* x;   // (M, K) FP16 tokens
    int8_t* q;           // (M, K) INT8 scratch, 8-byte aligned, or null (not written)
    float* scale;        // (M,) scratch (written with q)
};

constexpr int kFqPad = 128;
constexpr int kFqTokAhead = 2;   // token stages read from LDS ahead of their MFMAs
constexpr int kFqTokBytes = kDecodeFqMaxM * (kDecodeMaxK + kFqPad);

// The prologue in two parts: the token loads (issued before the kernel's first weight loads, so
// that waiting for them does not wait for the weights: loads retire in issue order), then the
// rest once the weights are in flight.
template <int VPR>
__device__ __forceinline__ void fq_load_tokens(const FqArgs& fq, int M, int K, uint4 (&v)[kDecodeFqMaxM][VPR])
{
    const int t = threadIdx.x;
    const int nvec = K >> 3;
#pragma unroll
    for (int r = 0; r < kDecodeFqMaxM; r++) {
        const uint4* src = reinterpret_cast<const uint4*>(fq.x + static_cast<size_t>(r < M ? r : M - 1) * K);
#pragma unroll
        for (int i = 0; i < VPR; i++) v[r][i] = src[min(t + i * 256, nvec - 1)];
    }
}

template <int VPR>
__device__ __forceinline__ void fq_quantize_tokens(const FqArgs& fq, int M, int K, const uint4 (&v)[kDecodeFqMaxM][VPR],
                                                   int8_t* tok, float* sscale, uint32_t* sbits, float* smax)
{
    constexpr int MT = kDecodeFqMaxM;
    static_assert(MT == 2, "one packed row pair");
    const int t = threadIdx.x, lane = t & (kWave - 1), wave = t / kWave;
    const int nvec = K >> 3;
    const int ld = K + kFqPad;
    uint32_t m[MT];
#pragma unroll
    for (int r = 0; r < MT; r++) {
        m[r] = 0u;
#pragma unroll
        for (int i = 0; i < VPR; i++) m[r] = absbits8(v[r][i], m[r]);
    }
    const uint32_t p01 = wave_max_pk_u16(pk_rows2(m[0], m[1]));
    if (lane == 0) {
        sbits[wave * MT + 0] = p01 & 0xFFFFu;
        sbits[wave * MT + 1] = p01 >> 16;
    }
    __syncthreads();
    uint32_t bits[MT];
    bool nan_row = false;
#pragma unroll
    for (int r = 0; r < MT; r++) {
        bits[r] = max(max(sbits[r], sbits[MT + r]), max(sbits[2 * MT + r], sbits[3 * MT + r]));
        nan_row |= r < M && bits[r] > kHalfInfBits;
    }
    float amax[MT];
#pragma unroll
    for (int r = 0; r < MT; r++) amax[r] = h2f(static_cast<uint16_t>(bits[r]));
    if (nan_row) {                  // uniform: a row holding a NaN takes the fp32 maximum
#pragma unroll
        for (int r = 0; r < MT; r++) {
            float a = 0.0f;
#pragma unroll
            for (int i = 0; i < VPR; i++) a = absmax8(v[r][i], a);
            a = wave_max(a);
            if (lane == 0) smax[wave * MT + r] = a;
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < MT; r++)
            if (bits[r] > kHalfInfBits)
                amax[r] = fmaxf(fmaxf(smax[r], smax[MT + r]), fmaxf(smax[2 * MT + r], smax[3 * MT + r]));
    }
    const bool out = blockIdx.x == 0 && blockIdx.y == 0 && fq.q != nullptr;
#pragma unroll
    for (int r = 0; r < MT; r++) {
        if (r >= M) break;
        const float scale = row_scale(amax[r]);
        const float inv = 1.0f / scale;
        if (t == 0) {
            sscale[r] = scale;
            if (out) fq.scale[r] = scale;
        }
#pragma unroll
        for (int i = 0; i < VPR; i++) {
            const int idx = t + i * 256;
            if (idx >= nvec) continue;
            const uint2 q = quant8_row(v[r][i], inv);
            *reinterpret_cast<uint2*>(tok + r * ld + idx * 8) = q;
            if (out) *reinterpret_cast<uint2*>(fq.q + static_cast<size_t>(r) * K + idx * 8) = q;
        }
    }
    __syncthreads();
}

// Epilogue of the register kernels with several token blocks: red holds each wave's INT32
// partials, block (b, tb) of wave w at ((w * RB + b) * TB + tb) * 64 + lane; lane l holds
// rows n0 + 16 b + 4 (l / 16) + e of token 16 tb + l % 16. Waves take the RB x TB blocks in
// turn, sum the WV partials exactly and store each lane's 4 consecutive outputs of one token
// row together (8-byte FP16 or 16-byte INT32 stores when the rows allow it).
template <int RB, int TB, int WV>
__device__ __forceinline__ v4i decode_block_sum(const v4i* red, int q, int lane)
{
    const int b = q / TB, tb = q - b * TB;
    v4i sum = red[(b * TB + tb) * kWave + lane];
#pragma unroll
    for (int w = 1; w < WV; w++) sum += red[((w * RB + b) * TB + tb) * kWave + lane];
    return sum;
}

// Stores block q = b * TB + tb of a row block (rows n0 + 16 b + 4 g + e, token 16 tb + lane % 16).
template <bool DEQUANT, int TB>
__device__ __forceinline__ void decode_store_block(const GemmEpilogue& ep, const v4i& sum, int n0, int q, int lane)
{
    const int M = ep.M, N = ep.N;
    const int r16 = lane & 15, g = lane >> 4;
    const int b = q / TB, tb = q - b * TB;
    const int m = 16 * tb + r16;
    const int nb = n0 + 16 * b + 4 * g;
    if (m >= M || nb >= N) return;
    const size_t o = static_cast<size_t>(m) * N + nb;
    const bool whole = ep.vec_out && nb + 4 <= N;
    if constexpr (DEQUANT) {
        const float as = ep.act_scale[m];
        uint16_t h[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int n = nb + e < N ? nb + e : N - 1;
            const float bv = ep.bias ? h2f(ep.bias[n]) : 0.0f;
            h[e] = dequant_gemm(sum[e], as, h2f(ep.w_scale[n]), bv, ep.bias != nullptr);
        }
        if (whole) {
            *reinterpret_cast<uint2*>(ep.c16 + o) =
                make_uint2(h[0] | (static_cast<uint32_t>(h[1]) << 16), h[2] | (static_cast<uint32_t>(h[3]) << 16));
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (nb + e < N) ep.c16[o + e] = h[e];
        }
    } else {
        if (whole) {
            *reinterpret_cast<int4*>(ep.c32 + o) = make_int4(sum[0], sum[1], sum[2], sum[3]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (nb + e < N) ep.c32[o + e] = sum[e];
        }
    }
}

template <bool DEQUANT, int RB, int TB, int WV>
__device__ __forceinline__ void decode_epilogue_blocks(const v4i* red, const GemmEpilogue& ep, int n0, int wave,
                                                       int lane)
{
    for (int q = wave; q < RB * TB; q += WV)
        decode_store_block<DEQUANT, TB>(ep, decode_block_sum<RB, TB, WV>(red, q, lane), n0, q, lane);
}

// VPR > 0: fused quantize (fq_quantize_tokens with VPR vectors per thread per row); the tokens
// are then read from LDS instead of X.
// KP > 1: the KP workgroups blockIdx.y = 0..KP-1 of a row block each take one contiguous K/KP
// range and hand their INT32 partials over through ks (ksplit_handoff), so that a row block
// can be taller (each workgroup reads 16 token rows per 16 x RB weight rows) at the same
// number of workgroups.
template <bool DEQUANT, int S, int RB, int WV, int AH, int VPR = 0, int KP = 1>
__global__ __launch_bounds__(WV * kWave) __attribute__((amdgpu_waves_per_eu(1, 2))) void decode_dense_kernel(
    const int8_t* __restrict__ W, const int8_t* __restrict__ X, GemmEpilogue ep, int K, FqArgs fq, KSplit ks)
{
    constexpr bool FQ = VPR > 0;
    __shared__ v4i red[WV * RB * kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int n0 = blockIdx.x * 16 * RB;
    const int M = ep.M, N = ep.N;
    const int r16 = lane & 15, g = lane >> 4;
    const bool hi = (lane >> 3) & 1;
    const int kp = KP > 1 ? static_cast<int>(blockIdx.y) : 0;
    const int k0 = kp * (K / KP);

    const int nst = K / KP / 128;
    const int s0 = wave * S < nst ? wave * S : nst;
    const int ns = (s0 + S < nst ? s0 + S : nst) - s0;

    // Load addresses: instruction j of block b reads row 16 b + 8 j + (lane % 8), chunk lane / 8.
    const int8_t* pw[RB][2];
#pragma unroll
    for (int b = 0; b < RB; b++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int r = n0 + 16 * b + 8 * j + (lane & 7);
            pw[b][j] = W + static_cast<size_t>(r < N ? r : N - 1) * K + k0 + 16 * (lane >> 3);
        }
    [[maybe_unused]] int8_t* ftok = nullptr;
    [[maybe_unused]] float* fscale = nullptr;
    if constexpr (FQ) {
        __shared__ __align__(16) int8_t s_tok[kFqTokBytes];
        __shared__ float s_scale[kDecodeFqMaxM];
        ftok = s_tok;
        fscale = s_scale;
    }
    const int8_t* px[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int r = 8 * j + (lane & 7);
        if constexpr (FQ) px[j] = ftok + (r < M ? r : M - 1) * (K + kFqPad) + k0 + 16 * (lane >> 3);
        else px[j] = X + static_cast<size_t>(r < M ? r : M - 1) * K + k0 + 16 * (lane >> 3);
    }
    const bool tok = r16 < M;   // after the swap, lane l holds token row l % 16

    // Epilogue operands of waves 0..RB-1 (block b = wave: rows n0 + 16 b + 4 g + e, token
    // r16), fetched before the K loop so that their latency hides behind it (the act scale
    // comes from the fused prologue when it runs).
    float e_as = 0.0f, e_ws[4] = {0.0f, 0.0f, 0.0f, 0.0f}, e_b[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (DEQUANT && wave < RB) {
        if constexpr (!FQ) e_as = ep.act_scale[tok ? r16 : 0];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int n = n0 + 16 * wave + 4 * g + e;
            const int nc = n < N ? n : N - 1;
            e_ws[e] = h2f(ep.w_scale[nc]);
            e_b[e] = ep.bias ? h2f(ep.bias[nc]) : 0.0f;
        }
    }

    struct Stage { v4i w[RB][2], x[2]; };
    auto load_w = [&](int t, Stage& f) {
        const int st = s0 + (t < ns ? t : ns - 1);
#pragma unroll
        for (int b = 0; b < RB; b++)
#pragma unroll
            for (int j = 0; j < 2; j++) f.w[b][j] = ld_stream<v4i>(pw[b][j] + st * 128);
    };
    auto load_x = [&](int t, Stage& f) {
        const int st = s0 + (t < ns ? t : ns - 1);
#pragma unroll
        for (int j = 0; j < 2; j++) f.x[j] = *reinterpret_cast<const v4i*>(px[j] + st * 128);
    };
    auto load = [&](int t, Stage& f) {
        load_w(t, f);
        load_x(t, f);
    };

    v4i acc[RB];
#pragma unroll
    for (int b = 0; b < RB; b++) acc[b] = v4i{0, 0, 0, 0};
    auto compute = [&](Stage& f, bool real) {
        v4i x0, x1;
        swap8_rows(f.x[0], f.x[1], hi, x0, x1);
        if (!(tok && real)) {
            x0 = v4i{0, 0, 0, 0};
            x1 = v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int b = 0; b < RB; b++) {
            v4i a0, a1;
            swap8_rows(f.w[b][0], f.w[b][1], hi, a0, a1);
            acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, x0, acc[b], 0, 0, 0);
            acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, x1, acc[b], 0, 0, 0);
        }
    };

    // Fused: the first A weight stages are issued before the prologue (issuing all of them
    // measured slower); the token stages then come from LDS kFqTokAhead ahead.
    constexpr int A = AH < S ? AH : S;
    constexpr int AX = FQ ? (kFqTokAhead < S ? kFqTokAhead : S) : A;
    Stage f[S];
    if constexpr (FQ) {
        // The first weight stages stream in while the workgroup quantizes its tokens (every wave
        // takes part in the prologue, idle K slices included).
        uint4 xv[kDecodeFqMaxM][VPR];
        fq_load_tokens<VPR>(fq, M, K, xv);
        if (ns > 0) {
#pragma unroll
            for (int t = 0; t < A; t++) load_w(t, f[t]);
        }
        __shared__ uint32_t s_bits[4 * kDecodeFqMaxM];
        __shared__ float s_max[4 * kDecodeFqMaxM];
        fq_quantize_tokens<VPR>(fq, M, K, xv, ftok, fscale, s_bits, s_max);
        if (DEQUANT && wave < RB) e_as = fscale[tok ? r16 : 0];
        if (ns > 0) {
#pragma unroll
            for (int t = 0; t < AX; t++) load_x(t, f[t]);
        }
    } else if (ns > 0) {
#pragma unroll
        for (int t = 0; t < A; t++) load(t, f[t]);
    }
    if (ns > 0) {
#pragma unroll
        for (int t = 0; t < S; t++) {
            if (t + A < S) load_w(t + A, f[t + A]);
            if (t + AX < S) load_x(t + AX, f[t + AX]);
            compute(f[t], t < ns);
        }
    }

#pragma unroll
    for (int b = 0; b < RB; b++) red[(wave * RB + b) * kWave + lane] = acc[b];
    __syncthreads();
    v4i sum = v4i{0, 0, 0, 0};
    if (wave < RB) {
        sum = red[wave * kWave + lane];
#pragma unroll
        for (int w = 1; w < WV; w++) sum += red[(w * RB + wave) * kWave + lane];
    }
    if constexpr (KP > 1) {
        v4i sums[1] = {sum};
        const bool has[1] = {wave < RB};
        const int blk[1] = {static_cast<int>(blockIdx.x) * RB + wave};
        if (!ksplit_handoff<KP, 1>(ks, sums, has, blk, lane)) return;
        sum = sums[0];
    }
    if (wave < RB) {
        const int b = wave;
        const int m = r16;
        if (m < M) {
            const int nb = n0 + 16 * b + 4 * g;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int n = nb + e;
                if (n >= N) continue;
                const size_t o = static_cast<size_t>(m) * N + n;
                if constexpr (DEQUANT)
                    ep.c16[o] = dequant_gemm(sum[e], e_as, e_ws[e], e_b[e], ep.bias != nullptr);
                else
                    ep.c32[o] = sum[e];
            }
        }
    }
}

// 2:4 sparse decode on coalesced register loads. A stage is a 256-deep dense K segment:
// per 16-row block, two coalesced instructions read 8 compressed rows x 128 bytes each (the
// segment's 2 x 64 compressed bytes per row), and the 8-lane swap leaves lane l = 16 G + 8 b + i
// with row l % 16 and compressed chunks 2 G and 2 G + 1. SMFMAC step h (0, 1) takes chunk
// 2 G + h in lane group G, i.e. the dense K range [32 (2 G + h), +32) of the segment stands in
// for the instruction's K range [32 G, +32) of its 128-deep step. Whole 4-groups move, so the
// index nibbles stay valid: the lane's index word is the packed word of 32-K chunk
// 8 seg + 2 G + h, and the token operand is gathered with the same permutation.
// VPR > 0 (one token block only): fused quantize, as in decode_dense_kernel.
template <bool DEQUANT, int S, int RB, int WV, int AH, int TB = 1, int VPR = 0, int KP = 1>
__global__ __launch_bounds__(WV * kWave) __attribute__((amdgpu_waves_per_eu(1, 2))) void decode_sparse_reg_kernel(
    const int8_t* __restrict__ W, const uint32_t* __restrict__ meta, const int8_t* __restrict__ X,
    GemmEpilogue ep, int K, FqArgs fq, KSplit ks)
{
    constexpr bool FQ = VPR > 0;
    static_assert(!FQ || TB == 1, "the fused prologue serves one token block");
    __shared__ v4i red[WV * RB * TB * kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int n0 = blockIdx.x * 16 * RB;
    const int M = ep.M, N = ep.N;
    const int r16 = lane & 15, g = lane >> 4;
    const bool hi = (lane >> 3) & 1;
    const int kp = KP > 1 ? static_cast<int>(blockIdx.y) : 0;
    const int k0 = kp * (K / KP);   // a multiple of 256: k0 / 2 compressed bytes, k0 / 2 index words

    const int nseg = K / KP / 256;
    const int s0 = wave * S < nseg ? wave * S : nseg;
    const int ns = (s0 + S < nseg ? s0 + S : nseg) - s0;

    // Compressed rows (K/2 bytes): instruction j of block b reads row 16 b + 8 j + lane % 8,
    // chunk lane / 8 of the segment's 128 bytes.
    const int8_t* pw[RB][2];
    const uint32_t* pi[RB][2];
#pragma unroll
    for (int b = 0; b < RB; b++) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int r = n0 + 16 * b + 8 * j + (lane & 7);
            pw[b][j] = W + static_cast<size_t>(r < N ? r : N - 1) * (K / 2) + k0 / 2 + 16 * (lane >> 3);
        }
        // Packed index words of block b: stage s (128 dense K) holds 64 words, the word of
        // (row r, 32-K chunk 4 s + q) at 16 q + r. Chunk 8 seg + 2 g + h lies in stage
        // 2 seg + (2 g + h) / 4 at q = (2 g + h) % 4.
        const int blk = (n0 >> 4) + b < (N >> 4) ? (n0 >> 4) + b : (N >> 4) - 1;
        const uint32_t* base = meta + static_cast<size_t>(blk) * (K / 2) + k0 / 2 + r16;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int c = 2 * g + h;
            pi[b][h] = base + (c >> 2) * 64 + 16 * (c & 3);
        }
    }
    // Tokens of block tb: row 16 tb + r16 (clamped; rows >= M are zeroed). Step h reads the
    // segment's dense bytes [64 (g >> 1) + 32 h + 16 (g & 1), +16) and the same + 128.
    [[maybe_unused]] int8_t* ftok = nullptr;
    [[maybe_unused]] float* fscale = nullptr;
    if constexpr (FQ) {
        __shared__ __align__(16) int8_t s_tok[kFqTokBytes];
        __shared__ float s_scale[kDecodeFqMaxM];
        ftok = s_tok;
        fscale = s_scale;
    }
    bool tok[TB];
    const int8_t* px[TB];
#pragma unroll
    for (int tb = 0; tb < TB; tb++) {
        const int r = 16 * tb + r16;
        tok[tb] = r < M;
        const int rr = tok[tb] ? r : M - 1;
        if constexpr (FQ) px[tb] = ftok + rr * (K + kFqPad) + k0 + 64 * (g >> 1) + 16 * (g & 1);
        else px[tb] = X + static_cast<size_t>(rr) * K + k0 + 64 * (g >> 1) + 16 * (g & 1);
    }

    struct Stage { v4i w[RB][2], x[TB][4]; int ix[RB][2]; };
    auto load_w = [&](int t, Stage& f) {
        const int sg = s0 + (t < ns ? t : ns - 1);
#pragma unroll
        for (int b = 0; b < RB; b++) {
#pragma unroll
            for (int j = 0; j < 2; j++) f.w[b][j] = ld_stream<v4i>(pw[b][j] + sg * 128);
#pragma unroll
            for (int h = 0; h < 2; h++) f.ix[b][h] = static_cast<int>(ld_stream<uint32_t>(pi[b][h] + sg * 128));
        }
    };
    auto load_x = [&](int t, Stage& f) {
        const int sg = s0 + (t < ns ? t : ns - 1);
#pragma unroll
        for (int tb = 0; tb < TB; tb++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                f.x[tb][2 * h] = *reinterpret_cast<const v4i*>(px[tb] + sg * 256 + 32 * h);
                f.x[tb][2 * h + 1] = *reinterpret_cast<const v4i*>(px[tb] + sg * 256 + 32 * h + 128);
            }
    };
    auto load = [&](int t, Stage& f) {
        load_w(t, f);
        load_x(t, f);
    };

    v4i acc[RB][TB];
#pragma unroll
    for (int b = 0; b < RB; b++)
#pragma unroll
        for (int tb = 0; tb < TB; tb++) acc[b][tb] = v4i{0, 0, 0, 0};
    auto compute = [&](Stage& f, bool real) {
        v4i a[RB][2];
#pragma unroll
        for (int b = 0; b < RB; b++) swap8_rows(f.w[b][0], f.w[b][1], hi, a[b][0], a[b][1]);
#pragma unroll
        for (int tb = 0; tb < TB; tb++) {
            const bool live = tok[tb] && real;
            v8i xb[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const v4i lo = live ? f.x[tb][2 * h] : v4i{0, 0, 0, 0};
                const v4i hi4 = live ? f.x[tb][2 * h + 1] : v4i{0, 0, 0, 0};
                xb[h] = __builtin_shufflevector(lo, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
            }
#pragma unroll
            for (int b = 0; b < RB; b++) {
                acc[b][tb] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(a[b][0], xb[0], acc[b][tb], f.ix[b][0], 0, 0);
                acc[b][tb] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(a[b][1], xb[1], acc[b][tb], f.ix[b][1], 0, 0);
            }
        }
    };

    // Fused: the first A weight stages are issued before the prologue (issuing all of them
    // measured slower); the token stages then come from LDS kFqTokAhead ahead.
    constexpr int A = AH < S ? AH : S;
    constexpr int AX = FQ ? (kFqTokAhead < S ? kFqTokAhead : S) : A;
    Stage f[S];
    if constexpr (FQ) {
        uint4 xv[kDecodeFqMaxM][VPR];
        fq_load_tokens<VPR>(fq, M, K, xv);
        if (ns > 0) {
#pragma unroll
            for (int t = 0; t < A; t++) load_w(t, f[t]);
        }
        __shared__ uint32_t s_bits[4 * kDecodeFqMaxM];
        __shared__ float s_max[4 * kDecodeFqMaxM];
        fq_quantize_tokens<VPR>(fq, M, K, xv, ftok, fscale, s_bits, s_max);
        if (ns > 0) {
#pragma unroll
            for (int t = 0; t < AX; t++) load_x(t, f[t]);
        }
    } else if (ns > 0) {
#pragma unroll
        for (int t = 0; t < A; t++) load(t, f[t]);
    }
    if (ns > 0) {
#pragma unroll
        for (int t = 0; t < S; t++) {
            if (t + A < S) load_w(t + A, f[t + A]);
            if (t + AX < S) load_x(t + AX, f[t + AX]);
            compute(f[t], t < ns);
        }
    }

#pragma unroll
    for (int b = 0; b < RB; b++)
#pragma unroll
        for (int tb = 0; tb < TB; tb++) red[((wave * RB + b) * TB + tb) * kWave + lane] = acc[b][tb];
    __syncthreads();
    if constexpr (TB > 1) {
        if constexpr (KP == 1) {
            decode_epilogue_blocks<DEQUANT, RB, TB, WV>(red, ep, n0, wave, lane);
        } else {
            // Wave w reduces blocks q = w, w + WV, ...; the sums are handed over, then stored.
            constexpr int NQ = (RB * TB + WV - 1) / WV;
            v4i sums[NQ];
            bool has[NQ];
            int blk[NQ];
#pragma unroll
            for (int i = 0; i < NQ; i++) {
                const int q = wave + i * WV;
                has[i] = q < RB * TB;
                blk[i] = static_cast<int>(blockIdx.x) * RB * TB + q;
                sums[i] = has[i] ? decode_block_sum<RB, TB, WV>(red, q, lane) : v4i{0, 0, 0, 0};
            }
            if (!ksplit_handoff<KP, NQ>(ks, sums, has, blk, lane)) return;
#pragma unroll
            for (int i = 0; i < NQ; i++)
                if (has[i]) decode_store_block<DEQUANT, TB>(ep, sums[i], n0, wave + i * WV, lane);
        }
        return;
    }
    v4i sum = v4i{0, 0, 0, 0};
    if (wave < RB) {
        sum = red[wave * kWave + lane];
#pragma unroll
        for (int w = 1; w < WV; w++) sum += red[(w * RB + wave) * kWave + lane];
    }
    if constexpr (KP > 1) {
        v4i sums[1] = {sum};
        const bool has[1] = {wave < RB};
        const int blk[1] = {static_cast<int>(blockIdx.x) * RB + wave};
        if (!ksplit_handoff<KP, 1>(ks, sums, has, blk, lane)) return;
        sum = sums[0];
    }
    if (wave < RB) {
        const int b = wave;
        const int m = r16;
        if (m < M) {
            const int nb = n0 + 16 * b + 4 * g;
            float as = 0.0f;
            if constexpr (DEQUANT) as = FQ ? fscale[m] : ep.act_scale[m];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int n = nb + e;
                if (n >= N) continue;
                const size_t o = static_cast<size_t>(m) * N + n;
                if constexpr (DEQUANT) {
                    const float bv = ep.bias ? h2f(ep.bias[n]) : 0.0f;
                    ep.c16[o] = dequant_gemm(sum[e], as, h2f(ep.w_scale[n]), bv, ep.bias != nullptr);
                } else {
                    ep.c32[o] = sum[e];
                }
            }
        }
    }
}

// K split for narrow N (row blocks fewer than CUs): the KP workgroups of a row block each take
// K / KP and hand their sums over (ksplit_handoff). The sums and counters live in static device
// slots, zero when the code object loads and left zero by every launch, so nothing is
// allocated; a slot belongs to one launch key (stream_slots.h), and with every slot taken a
// launch runs unsplit (same bits, no split).
// Measured at M = 16, K = 8192 (128 and 32 row blocks of 32 rows): N = 4096
// 13.6 -> 9.9 us, N = 1000 13.2 -> 8.8 us. Where the row blocks already fill the chip the split
// only adds the hand-off (N = 8192: 14.4 -> 15.2 us), so it is not used there.
constexpr int kKSplitSlots = kKSplitSlotCount;
constexpr int kKSplitMaxBlocks = 512;   // 16-row blocks per slot (N <= 8192)
constexpr int kKSplitMaxParts = 8;
constexpr size_t kKSplitAccPerSlot = static_cast<size_t>(kKSplitMaxBlocks) * 4 * kWave;
static __device__ int g_ksplit_acc[kKSplitSlots * kKSplitAccPerSlot];
static __device__ unsigned g_ksplit_cnt[kKSplitSlots * kKSplitMaxBlocks];

namespace {
std::mutex g_ks_mu;
int* g_ks_acc_dev[kSlotMaxDev];
unsigned* g_ks_cnt_dev[kSlotMaxDev];
SlotOwners<kKSplitSlots> g_ks_slots;
thread_local int t_ks_last_slot = -1;   // the calling thread's last decode launch: slot (-1: none)
thread_local int t_ks_last_kp = 0;      // and its K parts (1: unsplit; 0: no decode launch yet)

// Resolves the slot arrays of device dev (g_ks_mu held); false if they cannot be resolved.
bool ksplit_resolve(int dev)
{
    if (g_ks_acc_dev[dev]) return true;
    void* a = nullptr;
    void* c = nullptr;
    if (hipGetSymbolAddress(&a, HIP_SYMBOL(g_ksplit_acc)) != hipSuccess ||
        hipGetSymbolAddress(&c, HIP_SYMBOL(g_ksplit_cnt)) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    g_ks_acc_dev[dev] = static_cast<int*>(a);
    g_ks_cnt_dev[dev] = static_cast<unsigned*>(c);
    return true;
}

}  // namespace

int ksplit_slots_used(int dev)
{
    std::lock_guard<std::mutex> lock(g_ks_mu);
    return g_ks_slots.used(dev);
}

int ksplit_prepare()
{
    int dev = 0;
    if (!slot_device(&dev)) return FORGE_ENODEV;
    std::lock_guard<std::mutex> lock(g_ks_mu);
    return ksplit_resolve(dev) ? FORGE_OK : FORGE_ENODEV;
}

// The K-split slot of the key (s, capture id of s or 0) on the current device, or {} (no split)
// when every slot is held by other keys, for hipStreamPerThread (one handle for many host
// threads' streams), when the capture state of s cannot be read, or when the slot arrays are
// not resolved yet and s is capturing a graph (forge_init resolves them outside any capture).
static KSplit ksplit_slot(hipStream_t s, int* slot_out)
{
    *slot_out = -1;
    int dev = 0;
    SlotKey key{};
    if (!slot_device(&dev) || !slot_key(s, &key)) return {};
    std::lock_guard<std::mutex> lock(g_ks_mu);
    if (!g_ks_acc_dev[dev] && (key.capture != 0 || !ksplit_resolve(dev))) return {};
    const int slot = g_ks_slots.take(dev, key);
    if (slot < 0) return {};
    *slot_out = slot;
    return {g_ks_acc_dev[dev] + static_cast<size_t>(slot) * kKSplitAccPerSlot,
            g_ks_cnt_dev[dev] + static_cast<size_t>(slot) * kKSplitMaxBlocks};
}

// The K split of one decode launch: kp > 1 takes the slot of the launch's key; without one
// the launch runs unsplit (kp = 1). Records the decision for forge_ksplit_last.
static KSplit ksplit_take(hipStream_t s, int& kp)
{
    KSplit ks{};
    int slot = -1;
    if (kp > 1) {
        ks = ksplit_slot(s, &slot);
        if (!ks.acc) kp = 1;
    }
    t_ks_last_slot = slot;
    t_ks_last_kp = kp;
    return ks;
}

__global__ __launch_bounds__(256) void ksplit_clear_kernel(int* acc, size_t n_acc, unsigned* cnt, size_t n_cnt)
{
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n_acc; i += stride) acc[i] = 0;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n_cnt; i += stride) cnt[i] = 0;
}

// K parts for a dense decode launch: doubled while twice the workgroups still fit 1.25 waves
// of CUs and each part stays at least 1024 deep in whole 128-deep stages; no split below
// K = 4096, where one launch is already near its fixed cost. Measured (K = 8192, M = 16 / 1):
// N = 4096 13.5 -> 9.9 us (2 parts), N = 2048 13.5 -> 7.5 us (4), N = 1024 13.3 / 7.2 -> 6.6 /
// 5.9 us (8 / 4); K = 2048 splits measured slower at every N.
constexpr int kKSplitMinK = 4096;
constexpr int kKSplitMinPartK = 1024;

static int decode_dense_kparts(int N, int K, int rb, int cu)
{
    const int g = divup(N, 16 * rb);
    if (K < kKSplitMinK || g * rb > kKSplitMaxBlocks) return 1;
    int kp = 1;
    while (kp < kKSplitMaxParts && 2 * g * kp * 4 <= 5 * cu && K % (256 * kp) == 0 && K / (2 * kp) >= kKSplitMinPartK)
        kp *= 2;
    return kp;
}

template <bool DEQUANT, int RB, int WV, int AH, int KP>
static int launch_decode_dense_kp(const int8_t* W, const int8_t* X, const GemmEpilogue& ep, int K, const KSplit& ks,
                                  hipStream_t s)
{
    const dim3 grid(static_cast<unsigned>(divup(ep.N, 16 * RB)), KP);
    const int per = divup(K / KP / 128, WV);
    // Largest per-wave stage count K <= kDecodeMaxK can need at this KP (no larger S is built).
    constexpr int SM = kDecodeMaxK / 128 / KP / WV > 1 ? kDecodeMaxK / 128 / KP / WV : 1;
    constexpr int S2 = 2 < SM ? 2 : SM, S4 = 4 < SM ? 4 : SM, S8 = 8 < SM ? 8 : SM, S16 = 16 < SM ? 16 : SM;
#define FORGE_DEC_DENSE(SS) \
    decode_dense_kernel<DEQUANT, SS, RB, WV, AH, 0, KP><<<grid, WV * kWave, 0, s>>>(W, X, ep, K, FqArgs{}, ks)
    if (per <= 1) FORGE_DEC_DENSE(1);
    else if (per <= 2) FORGE_DEC_DENSE(S2);
    else if (per <= 4) FORGE_DEC_DENSE(S4);
    else if (per <= 8) FORGE_DEC_DENSE(S8);
    else FORGE_DEC_DENSE(S16);
#undef FORGE_DEC_DENSE
    return launch_status();
}

// kp = 0: choose the K parts (decode_dense_kparts); otherwise that many (1, 2, 4 or 8; the
// caller checks K % (128 kp) == 0). Without a free slot the launch is not split.
template <bool DEQUANT, int RB, int WV, int AH>
static int launch_decode_dense(const int8_t* W, const int8_t* X, const GemmEpilogue& ep, int K, hipStream_t s,
                               int kp = 0)
{
    if (kp == 0) {
        int st = FORGE_OK;
        const DeviceInfo& di = device_info(&st);
        if (st != FORGE_OK) return st;
        kp = decode_dense_kparts(ep.N, K, RB, di.cu_count);
    }
    const KSplit ks = ksplit_take(s, kp);
    switch (kp) {
    case 2: return launch_decode_dense_kp<DEQUANT, RB, WV, AH, 2>(W, X, ep, K, ks, s);
    case 4: return launch_decode_dense_kp<DEQUANT, RB, WV, AH, 4>(W, X, ep, K, ks, s);
    case 8: return launch_decode_dense_kp<DEQUANT, RB, WV, AH, 8>(W, X, ep, K, ks, s);
    default: return launch_decode_dense_kp<DEQUANT, RB, WV, AH, 1>(W, X, ep, K, ks, s);
    }
}

template <bool DEQUANT, int RB, int WV, int AH, int KP>
static int launch_decode_sparse_reg_kp(const int8_t* W, const uint32_t* meta, const int8_t* X, const GemmEpilogue& ep,
                                       int K, const KSplit& ks, hipStream_t s)
{
    const dim3 grid(static_cast<unsigned>(divup(ep.N, 16 * RB)), KP);
    const int per = divup(K / KP / 256, WV);
    constexpr int SM = kDecodeMaxK / 256 / KP / WV > 1 ? kDecodeMaxK / 256 / KP / WV : 1;
    constexpr int S2 = 2 < SM ? 2 : SM, S4 = 4 < SM ? 4 : SM, S8 = 8 < SM ? 8 : SM;
#define FORGE_DEC_SPREG(SS) \
    decode_sparse_reg_kernel<DEQUANT, SS, RB, WV, AH, 1, 0, KP><<<grid, WV * kWave, 0, s>>>(W, meta, X, ep, K, FqArgs{}, ks)
    if (per <= 1) FORGE_DEC_SPREG(1);
    else if (per <= 2) FORGE_DEC_SPREG(S2);
    else if (per <= 4) FORGE_DEC_SPREG(S4);
    else FORGE_DEC_SPREG(S8);
#undef FORGE_DEC_SPREG
    return launch_status();
}

// K parts for the sparse register kernel: as decode_dense_kparts, in whole 256-deep segments;
// up to 8 tokens from K = 8192 on with parts at least 2048 deep (a launch streams half the dense
// bytes per K), 9-16 tokens (twice the token bytes per weight byte) from K = 6144 on with parts
// at least 1536 deep. Measured (M = 8 / 1, K = 8192): N = 4096 9.7 / 8.4 -> 8.2 / 7.7 us,
// N = 1024 9.5 / 8.1 -> 6.3 / 5.8 us; at K = 4096 splits moved times by -0.45 to +0.4 us.
static int decode_sparse_kparts(int N, int K, int rb, int cu, int M)
{
    const int min_k = M > 8 ? 6144 : 8192, min_part = M > 8 ? 1536 : 2048;
    const int g = divup(N, 16 * rb);
    if (K < min_k || g * rb > kKSplitMaxBlocks) return 1;
    int kp = 1;
    while (kp < kKSplitMaxParts && 2 * g * kp * 4 <= 5 * cu && K % (512 * kp) == 0 && K / (2 * kp) >= min_part)
        kp *= 2;
    return kp;
}

// kp = 0: choose (decode_sparse_kparts); otherwise that many parts (K % (256 kp) == 0).
template <bool DEQUANT, int RB, int WV, int AH>
static int launch_decode_sparse_reg(const int8_t* W, const uint32_t* meta, const int8_t* X, const GemmEpilogue& ep,
                                    int K, hipStream_t s, int kp = 0)
{
    if (kp == 0) {
        int st = FORGE_OK;
        const DeviceInfo& di = device_info(&st);
        if (st != FORGE_OK) return st;
        kp = decode_sparse_kparts(ep.N, K, RB, di.cu_count, ep.M);
    }
    const KSplit ks = ksplit_take(s, kp);
    switch (kp) {
    case 2: return launch_decode_sparse_reg_kp<DEQUANT, RB, WV, AH, 2>(W, meta, X, ep, K, ks, s);
    case 4: return launch_decode_sparse_reg_kp<DEQUANT, RB, WV, AH, 4>(W, meta, X, ep, K, ks, s);
    case 8: return launch_decode_sparse_reg_kp<DEQUANT, RB, WV, AH, 8>(W, meta, X, ep, K, ks, s);
    default: return launch_decode_sparse_reg_kp<DEQUANT, RB, WV, AH, 1>(W, meta, X, ep, K, ks, s);
    }
}

// Dense with several 16-token blocks (16 < M <= 64) at narrow N and deep K, where the tile
// engine has too few tiles to fill the chip: one 16-row weight block per workgroup, each weight
// fragment reused for TB token blocks (the dense decode kernel's loads, swap and
// v_mfma_i32_16x16x64_i8), K split over KP workgroups per row block with the exact hand-off.
template <bool DEQUANT, int S, int WV, int AH, int TB, int KP>
__global__ __launch_bounds__(WV * kWave) __attribute__((amdgpu_waves_per_eu(1, 2))) void decode_dense_tb_kernel(
    const int8_t* __restrict__ W, const int8_t* __restrict__ X, GemmEpilogue ep, int K, KSplit ks)
{
    __shared__ v4i red[WV * TB * kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int n0 = blockIdx.x * 16;
    const int M = ep.M, N = ep.N;
    const int r16 = lane & 15;
    const bool hi = (lane >> 3) & 1;
    const int kp = KP > 1 ? static_cast<int>(blockIdx.y) : 0;
    const int k0 = kp * (K / KP);
    const int nst = K / KP / 128;
    const int s0 = wave * S < nst ? wave * S : nst;
    const int ns = (s0 + S < nst ? s0 + S : nst) - s0;

    const int8_t* pw[2];
    const int8_t* px[TB][2];
    bool tok[TB];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int r = n0 + 8 * j + (lane & 7);
        pw[j] = W + static_cast<size_t>(r < N ? r : N - 1) * K + k0 + 16 * (lane >> 3);
    }
#pragma unroll
    for (int tb = 0; tb < TB; tb++) {
        tok[tb] = 16 * tb + r16 < M;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int r = 16 * tb + 8 * j + (lane & 7);
            px[tb][j] = X + static_cast<size_t>(r < M ? r : M - 1) * K + k0 + 16 * (lane >> 3);
        }
    }

    struct Stage { v4i w[2], x[TB][2]; };
    auto load = [&](int t, Stage& f) {
        const int st = s0 + (t < ns ? t : ns - 1);
#pragma unroll
        for (int j = 0; j < 2; j++) f.w[j] = ld_stream<v4i>(pw[j] + st * 128);
#pragma unroll
        for (int tb = 0; tb < TB; tb++)
#pragma unroll
            for (int j = 0; j < 2; j++) f.x[tb][j] = *reinterpret_cast<const v4i*>(px[tb][j] + st * 128);
    };
    v4i acc[TB];
#pragma unroll
    for (int tb = 0; tb < TB; tb++) acc[tb] = v4i{0, 0, 0, 0};
    auto compute = [&](Stage& f, bool real) {
        v4i a0, a1;
        swap8_rows(f.w[0], f.w[1], hi, a0, a1);
#pragma unroll
        for (int tb = 0; tb < TB; tb++) {
            v4i x0, x1;
            swap8_rows(f.x[tb][0], f.x[tb][1], hi, x0, x1);
            if (!(tok[tb] && real)) {
                x0 = v4i{0, 0, 0, 0};
                x1 = v4i{0, 0, 0, 0};
            }
            acc[tb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, x0, acc[tb], 0, 0, 0);
            acc[tb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, x1, acc[tb], 0, 0, 0);
        }
    };
    constexpr int A = AH < S ? AH : S;
    Stage f[S];
    if (ns > 0) {
#pragma unroll
        for (int t = 0; t < A; t++) load(t, f[t]);
#pragma unroll
        for (int t = 0; t < S; t++) {
            if (t + A < S) load(t + A, f[t + A]);
            compute(f[t], t < ns);
        }
    }
#pragma unroll
    for (int tb = 0; tb < TB; tb++) red[(wave * TB + tb) * kWave + lane] = acc[tb];
    __syncthreads();
    if constexpr (KP == 1) {
        decode_epilogue_blocks<DEQUANT, 1, TB, WV>(red, ep, n0, wave, lane);
    } else {
        constexpr int NQ = (TB + WV - 1) / WV;
        v4i sums[NQ];
        bool has[NQ];
        int blk[NQ];
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            const int q = wave + i * WV;
            has[i] = q < TB;
            blk[i] = static_cast<int>(blockIdx.x) * TB + q;
            sums[i] = has[i] ? decode_block_sum<1, TB, WV>(red, q, lane) : v4i{0, 0, 0, 0};
        }
        if (!ksplit_handoff<KP, NQ>(ks, sums, has, blk, lane)) return;
#pragma unroll
        for (int i = 0; i < NQ; i++)
            if (has[i]) decode_store_block<DEQUANT, TB>(ep, sums[i], n0, wave + i * WV, lane);
    }
}

constexpr int kDenseTbWaves = 4;
constexpr int kDenseTbAhead = 2;

template <bool DEQUANT, int TB, int KP>
static int launch_dense_tb_kp(const int8_t* W, const int8_t* X, const GemmEpilogue& ep, int K, const KSplit& ks,
                              hipStream_t s)
{
    constexpr int WV = kDenseTbWaves;
    const dim3 grid(static_cast<unsigned>(divup(ep.N, 16)), KP);
    const int per = divup(K / KP / 128, WV);
    constexpr int SM = kDecodeMaxK / 128 / KP / WV;
#define FORGE_DENSE_TB(SS) \
    decode_dense_tb_kernel<DEQUANT, (SS <= SM ? SS : SM), WV, kDenseTbAhead, TB, KP><<<grid, WV * kWave, 0, s>>>(W, X, ep, K, ks)
    if (per <= 1) FORGE_DENSE_TB(1);
    else if (per <= 2) FORGE_DENSE_TB(2);
    else if (per <= 4) FORGE_DENSE_TB(4);
    else if (per <= 8) FORGE_DENSE_TB(8);
    else FORGE_DENSE_TB(16);
#undef FORGE_DENSE_TB
    return launch_status();
}

// kp: 0 = as skinny_tb_kparts (defined with the sparse token-block path), else 1, 2 or 4.
template <bool DEQUANT, int TB>
static int launch_dense_tb_tb(const int8_t* W, const int8_t* X, const GemmEpilogue& ep, int K, int cu, hipStream_t s,
                              int kp);

template <bool DEQUANT, int KP>
static int launch_decode_sparse_kp(const int8_t* W, const uint32_t* meta, const int8_t* X, const GemmEpilogue& ep,
                                   int K, const KSplit& ks, hipStream_t s)
{
    const dim3 grid(static_cast<unsigned>(divup(ep.N, kDecRows)), KP);
    const int per = divup(K / KP / 128, kDecWaves);
    constexpr int SM = kDecodeMaxK / 128 / KP / kDecWaves;
#define FORGE_DEC_SPARSE(SS) \
    decode_sparse_kernel<DEQUANT, (SS <= SM ? SS : SM), KP><<<grid, kDecWaves * kWave, 0, s>>>(W, meta, X, ep, K, ks)
    if (per <= 1) FORGE_DEC_SPARSE(1);
    else if (per <= 2) FORGE_DEC_SPARSE(2);
    else if (per <= 4) FORGE_DEC_SPARSE(4);
    else FORGE_DEC_SPARSE(8);
#undef FORGE_DEC_SPARSE
    return launch_status();
}

// K parts for the LDS-ring kernel (K % 256 == 128, 32-row workgroups, 128-deep stages): as
// decode_dense_kparts from K = 6144 on, up to 4 parts of at least 1536. Measured (M = 16):
// K = 8192 N = 4096 11.0 -> 9.6 us, N = 2048 10.1 -> 7.7 us, N = 1024 8.2 -> 6.2 us; K = 6144
// N = 2048 8.7 -> 7.1 us.
static int decode_ring_kparts(int N, int K, int cu)
{
    const int g = divup(N, kDecRows);
    if (K < 6144 || g * (kDecRows / 16) > kKSplitMaxBlocks) return 1;
    int kp = 1;
    while (kp < 4 && 2 * g * kp * 4 <= 5 * cu && K % (256 * kp) == 0 && K / (2 * kp) >= 1536) kp *= 2;
    return kp;
}

// K % 256 == 128: the LDS-ring kernel (kp = 0 chooses the K parts, otherwise 1, 2 or 4).
template <bool DEQUANT>
static int launch_decode_sparse(const int8_t* W, const uint32_t* meta, const int8_t* X, const GemmEpilogue& ep,
                                int K, hipStream_t s, int kp = 0)
{
    if (kp == 0) {
        int st = FORGE_OK;
        const DeviceInfo& di = device_info(&st);
        if (st != FORGE_OK) return st;
        kp = decode_ring_kparts(ep.N, K, di.cu_count);
    }
    const KSplit ks = ksplit_take(s, kp);
    switch (kp) {
    case 2: return launch_decode_sparse_kp<DEQUANT, 2>(W, meta, X, ep, K, ks, s);
    case 4: return launch_decode_sparse_kp<DEQUANT, 4>(W, meta, X, ep, K, ks, s);
    default: return launch_decode_sparse_kp<DEQUANT, 1>(W, meta, X, ep, K, ks, s);
    }
}

// Sparse with several token blocks (16 < M <= 64): the register kernel with each weight
// fragment and index word reused for TB = 2 or 4 token blocks. Each wave's segment count is
// padded to the next value of {1, 2, 3, 4, 6, 8}. Workgroups own 32 weight rows when that still
// gives half the chip's CUs one each, else 16 (each workgroup reads the whole token block, so
// fewer, taller workgroups read less). Measured on the reference benchmark's M = 64 shapes:
// 1536x6144 14.7 -> 7.1 us, 6144x1536 33.9 -> 15.1 us against the register-staged tile engine.
// (The dense GEMM keeps its tile engine at these M: the same structure measured slower there.)
constexpr int kSkinnyTbAheadSparse = 2;

static int pad_stages(int per)
{
    static const int kSparse[] = {1, 2, 3, 4, 6, 8};
    for (int c : kSparse)
        if (per <= c) return c;
    return -1;
}

template <bool DEQUANT, int RB, int TB, int KP, int WV = kDecDenseWaves>
static int launch_tb_sparse(const int8_t* W, const uint32_t* meta, const int8_t* X, const GemmEpilogue& ep, int K,
                            const KSplit& ks, hipStream_t s)
{
    constexpr int AH = kSkinnyTbAheadSparse;
    const dim3 grid(static_cast<unsigned>(divup(ep.N, 16 * RB)), KP);
    const int S = pad_stages(divup(K / KP / 256, WV));
    // Largest per-wave segment count K <= kDecodeMaxK can need at this KP.
    constexpr int SM = (kDecodeMaxK / 256 / KP + WV - 1) / WV;
#define FORGE_TB_SPARSE(SS) \
    decode_sparse_reg_kernel<DEQUANT, (SS <= SM ? SS : SM), RB, WV, AH, TB, 0, KP><<<grid, WV * kWave, 0, s>>>(W, meta, X, ep, K, FqArgs{}, ks)
    switch (S) {
    case 1: FORGE_TB_SPARSE(1); break;
    case 2: FORGE_TB_SPARSE(2); break;
    case 3: FORGE_TB_SPARSE(3); break;
    case 4: FORGE_TB_SPARSE(4); break;
    case 6: FORGE_TB_SPARSE(6); break;
    case 8: FORGE_TB_SPARSE(8); break;
    default: return FORGE_EINVAL;
    }
#undef FORGE_TB_SPARSE
    return launch_status();
}

bool skinny_tb_supported(int M, int K)
{
    return M > kDecodeMaxM && M <= kSkinnyTbMaxM && K <= kDecodeMaxK && K % 256 == 0;
}

// K parts for the token-block kernel with 16-row workgroups: as decode_dense_kparts, in whole
// 256-deep segments, parts at least kKSplitMinPartKTb deep, the sums of RB x TB blocks per
// workgroup within a slot.
constexpr int kKSplitMinPartKTb = 1024;

static int skinny_tb_kparts(int N, int K, int blocks, int cu)
{
    const int g = divup(N, 16);
    if (K < kKSplitMinK || g * blocks > kKSplitMaxBlocks) return 1;
    int kp = 1;
    while (kp < 4 && 2 * g * kp * 4 <= 5 * cu && K % (512 * kp) == 0 && K / (2 * kp) >= kKSplitMinPartKTb) kp *= 2;
    return kp;
}

template <bool DEQUANT, int TB>
static int launch_tb_sparse_narrow(const int8_t* W, const uint32_t* meta, const int8_t* X, const GemmEpilogue& ep,
                                   int K, int cu, hipStream_t s, int kp)
{
    if (kp == 0) kp = skinny_tb_kparts(ep.N, K, TB, cu);
    const KSplit ks = ksplit_take(s, kp);
    switch (kp) {
    case 2: return launch_tb_sparse<DEQUANT, 1, TB, 2>(W, meta, X, ep, K, ks, s);
    case 4: return launch_tb_sparse<DEQUANT, 1, TB, 4>(W, meta, X, ep, K, ks, s);
    default: return launch_tb_sparse<DEQUANT, 1, TB, 1>(W, meta, X, ep, K, ks, s);
    }
}

// kp: 0 chooses the K parts for 16-row workgroups (skinny_tb_kparts); otherwise 1, 2 or 4
// (K % (256 kp) == 0).
int launch_skinny_tb(const int8_t* W, const uint32_t* meta, const int8_t* X, const GemmEpilogue& ep, int K, int cu,
                     hipStream_t s, int kp)
{
    if (!skinny_tb_supported(ep.M, K)) return FORGE_EINVAL;
    const bool tall = 2 * divup(ep.N, 32) >= cu;
    // 8 waves (each fewer 256-deep segments) where K is short and N moderate; measured (us, 4 ->
    // 8 waves): M = 64 1536x6144 7.0 -> 6.4, 1280x5120 7.0 -> 5.9, 4096x4096 13.0 -> 12.3;
    // M = 32 1280x5120 4.75 -> 4.5; but 4096x11008 at M = 64 22.7 -> 23.2 and 8192x8192 at
    // M = 32 14.8 -> 16.0.
    const bool w8 = K <= 4096 && ep.N < 8192;
    const bool dq = ep.c16 != nullptr;
    if (ep.M <= 32) {
        if (tall && w8)
            return dq ? launch_tb_sparse<true, 2, 2, 1, 8>(W, meta, X, ep, K, KSplit{}, s)
                      : launch_tb_sparse<false, 2, 2, 1, 8>(W, meta, X, ep, K, KSplit{}, s);
        if (tall)
            return dq ? launch_tb_sparse<true, 2, 2, 1>(W, meta, X, ep, K, KSplit{}, s)
                      : launch_tb_sparse<false, 2, 2, 1>(W, meta, X, ep, K, KSplit{}, s);
        return dq ? launch_tb_sparse_narrow<true, 2>(W, meta, X, ep, K, cu, s, kp)
                  : launch_tb_sparse_narrow<false, 2>(W, meta, X, ep, K, cu, s, kp);
    }
    if (tall && w8)
        return dq ? launch_tb_sparse<true, 2, 4, 1, 8>(W, meta, X, ep, K, KSplit{}, s)
                  : launch_tb_sparse<false, 2, 4, 1, 8>(W, meta, X, ep, K, KSplit{}, s);
    if (tall)
        return dq ? launch_tb_sparse<true, 2, 4, 1>(W, meta, X, ep, K, KSplit{}, s)
                  : launch_tb_sparse<false, 2, 4, 1>(W, meta, X, ep, K, KSplit{}, s);
    return dq ? launch_tb_sparse_narrow<true, 4>(W, meta, X, ep, K, cu, s, kp)
              : launch_tb_sparse_narrow<false, 4>(W, meta, X, ep, K, cu, s, kp);
}

template <bool DEQUANT, int TB>
static int launch_dense_tb_tb(const int8_t* W, const int8_t* X, const GemmEpilogue& ep, int K, int cu, hipStream_t s,
                              int kp)
{
    if (kp == 0) kp = skinny_tb_kparts(ep.N, K, TB, cu);
    const KSplit ks = ksplit_take(s, kp);
    switch (kp) {
    case 2: return launch_dense_tb_kp<DEQUANT, TB, 2>(W, X, ep, K, ks, s);
    case 4: return launch_dense_tb_kp<DEQUANT, TB, 4>(W, X, ep, K, ks, s);
    default: return launch_dense_tb_kp<DEQUANT, TB, 1>(W, X, ep, K, ks, s);
    }
}

bool dense_tb_supported(int M, int K, int N, int cu)
{
    return M > kDecodeMaxM && M <= kSkinnyTbMaxM && K >= kKSplitMinK && K <= kDecodeMaxK && K % 256 == 0 &&
           divup(N, 16) < cu;
}

int launch_dense_tb(const int8_t* W, const int8_t* X, const GemmEpilogue& ep, int K, int cu, hipStream_t s, int kp)
{
    if (!dense_tb_supported(ep.M, K, ep.N, cu)) return FORGE_EINVAL;
    const bool dq = ep.c16 != nullptr;
    if (ep.M <= 32)
        return dq ? launch_dense_tb_tb<true, 2>(W, X, ep, K, cu, s, kp) : launch_dense_tb_tb<false, 2>(W, X, ep, K, cu, s, kp);
    return dq ? launch_dense_tb_tb<true, 4>(W, X, ep, K, cu, s, kp) : launch_dense_tb_tb<false, 4>(W, X, ep, K, cu, s, kp);
}

bool decode_supported(int M, int K) { return M <= kDecodeMaxM && K % 128 == 0 && K <= kDecodeMaxK; }

bool decode_fq_supported(int M, int K, bool sparse)
{
    return M <= kDecodeFqMaxM && K <= kDecodeMaxK && K % (sparse ? 256 : 128) == 0;
}

// The fused path takes the same K split as the two-pass decode launches (every workgroup of a
// row block quantizes the whole token rows in its prologue, then reads its K part from LDS);
// 2 or 4 parts.
template <int VPR, int KP>
static int launch_decode_fq_kp(const int8_t* W, const uint32_t* meta, const GemmEpilogue& ep, int K, bool sparse,
                               const FqArgs& fq, const KSplit& ks, hipStream_t s)
{
    if (sparse) {
        constexpr int RB = 2, WV = 4, AH = 4;
        const dim3 grid(static_cast<unsigned>(divup(ep.N, 16 * RB)), KP);
        const int per = divup(K / KP / 256, WV);
        constexpr int SM = kDecodeMaxK / 256 / KP / WV;
#define FORGE_DEC_FQ_SP(SS)                                                                              \
    decode_sparse_reg_kernel<true, (SS <= SM ? SS : SM), RB, WV, AH, 1, VPR, KP><<<grid, WV * kWave, 0, s>>>( \
        W, meta, nullptr, ep, K, fq, ks)
        if (per <= 1) FORGE_DEC_FQ_SP(1);
        else if (per <= 2) FORGE_DEC_FQ_SP(2);
        else if (per <= 4) FORGE_DEC_FQ_SP(4);
        else FORGE_DEC_FQ_SP(8);
#undef FORGE_DEC_FQ_SP
        return launch_status();
    }
    constexpr int RB = 1, WV = kDecDenseWaves, AH = kDecDenseAhead;
    const dim3 grid(static_cast<unsigned>(divup(ep.N, 16 * RB)), KP);
    const int per = divup(K / KP / 128, WV);
    constexpr int SM = kDecodeMaxK / 128 / KP / WV;
#define FORGE_DEC_FQ_DENSE(SS) \
    decode_dense_kernel<true, (SS <= SM ? SS : SM), RB, WV, AH, VPR, KP><<<grid, WV * kWave, 0, s>>>(W, nullptr, ep, K, fq, ks)
    if (per <= 1) FORGE_DEC_FQ_DENSE(1);
    else if (per <= 2) FORGE_DEC_FQ_DENSE(2);
    else if (per <= 4) FORGE_DEC_FQ_DENSE(4);
    else if (per <= 8) FORGE_DEC_FQ_DENSE(8);
    else FORGE_DEC_FQ_DENSE(16);
#undef FORGE_DEC_FQ_DENSE
    return launch_status();
}

template <int VPR>
static int launch_decode_fq_vpr(const int8_t* W, const uint32_t* meta, const GemmEpilogue& ep, int K, bool sparse,
                                const FqArgs& fq, hipStream_t s)
{
    int st = FORGE_OK;
    const DeviceInfo& di = device_info(&st);
    if (st != FORGE_OK) return st;
    int kp = sparse ? decode_sparse_kparts(ep.N, K, 2, di.cu_count, ep.M) : decode_dense_kparts(ep.N, K, 1, di.cu_count);
    kp = kp < 4 ? kp : 4;
    const KSplit ks = ksplit_take(s, kp);
    switch (kp) {
    case 2: return launch_decode_fq_kp<VPR, 2>(W, meta, ep, K, sparse, fq, ks, s);
    case 4: return launch_decode_fq_kp<VPR, 4>(W, meta, ep, K, sparse, fq, ks, s);
    default: return launch_decode_fq_kp<VPR, 1>(W, meta, ep, K, sparse, fq, ks, s);
    }
}

int launch_decode_fq(const uint16_t* x, const int8_t* W, const uint32_t* meta, const uint16_t* w_scale,
                     const uint16_t* bias, uint16_t* out, int8_t* q_scratch, float* scale_scratch, int M, int K,
                     int N, bool sparse, hipStream_t s)
{
    if (!decode_fq_supported(M, K, sparse) || !aligned(x, 16) || (q_scratch && !aligned(q_scratch, 8)))
        return FORGE_EINVAL;
    const GemmEpilogue ep{nullptr, out, nullptr, w_scale, bias, M, N, 0};
    const FqArgs fq{x, q_scratch, scale_scratch};
    const int vpr = divup(K, 8 * 256);
    if (vpr <= 1) return launch_decode_fq_vpr<1>(W, meta, ep, K, sparse, fq, s);
    if (vpr <= 2) return launch_decode_fq_vpr<2>(W, meta, ep, K, sparse, fq, s);
    return launch_decode_fq_vpr<4>(W, meta, ep, K, sparse, fq, s);
}

int launch_decode(const int8_t* W, const uint32_t* meta, const int8_t* X, const GemmEpilogue& ep, int K,
                  bool sparse, hipStream_t s)
{
    if (!decode_supported(ep.M, K)) return FORGE_EINVAL;
    // Sparse: the register kernel wherever K % 256 == 0 (measured with the weights rotated
    // past the MALL, N = K = 8192: M = 16 13.6 -> 12.0 us, M = 9 12.6 -> 10.6 us against the
    // DMA ring, whose LDS-DMA stream tops out lower); the ring takes K % 256 == 128.
    if (sparse && K % 256 == 0 && ep.M <= kDecSparseRegMaxM)
        return ep.c16 ? launch_decode_sparse_reg<true, 2, 4, 4>(W, meta, X, ep, K, s)
                      : launch_decode_sparse_reg<false, 2, 4, 4>(W, meta, X, ep, K, s);
    if (sparse) return ep.c16 ? launch_decode_sparse<true>(W, meta, X, ep, K, s) : launch_decode_sparse<false>(W, meta, X, ep, K, s);
    // Up to 4 tokens the token stream is light and 16-row workgroups (twice as many) stream
    // the weights faster; from 8 tokens on, two blocks sharing the token registers win.
    if (ep.M <= kDecDenseOneBlockMaxM)
        return ep.c16 ? launch_decode_dense<true, 1, kDecDenseWaves, kDecDenseAhead>(W, X, ep, K, s)
                      : launch_decode_dense<false, 1, kDecDenseWaves, kDecDenseAhead>(W, X, ep, K, s);
    return ep.c16 ? launch_decode_dense<true, kDecDenseBlocks, kDecDenseWavesTwoBlock, kDecDenseAhead>(W, X, ep, K, s)
                  : launch_decode_dense<false, kDecDenseBlocks, kDecDenseWavesTwoBlock, kDecDenseAhead>(W, X, ep, K, s);
}

}  // namespace forge_amd

using namespace forge_amd;

extern "C" int forge_ksplit_last(int* slot, int* parts)
{
    if (!slot || !parts) return FORGE_EINVAL;
    *slot = t_ks_last_slot;
    *parts = t_ks_last_kp;
    return FORGE_OK;
}

extern "C" int forge_slots_in_use(int* ksplit_used, int* ksplit_total, int* fq_pack_used, int* fq_pack_total)
{
    if (!ksplit_used || !ksplit_total || !fq_pack_used || !fq_pack_total) return FORGE_EINVAL;
    int dev = 0;
    if (!slot_device(&dev)) return FORGE_ENODEV;
    *ksplit_used = ksplit_slots_used(dev);
    *ksplit_total = kKSplitSlotCount;
    *fq_pack_used = fq_pack_slots_used(dev);
    *fq_pack_total = kFqPackSlotCount;
    return FORGE_OK;
}

extern "C" int forge_ksplit_reset(void* stream)
{
    int dev = 0;
    if (!slot_device(&dev)) return FORGE_ENODEV;
    int* acc = nullptr;
    unsigned* cnt = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_ks_mu);
        if (!ksplit_resolve(dev)) return FORGE_ENODEV;
        acc = g_ks_acc_dev[dev];
        cnt = g_ks_cnt_dev[dev];
    }
    ksplit_clear_kernel<<<1024, 256, 0, as_stream(stream)>>>(acc, kKSplitSlots * kKSplitAccPerSlot, cnt,
                                                             static_cast<size_t>(kKSplitSlots) * kKSplitMaxBlocks);
    return launch_status();
}
