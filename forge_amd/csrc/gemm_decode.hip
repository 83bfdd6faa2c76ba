// Decode-shape (M <= 16 tokens) INT8 GEMMs for gfx950, dense and 2:4 sparse: weight
// streaming at HBM rate.
//
// Reference shapes: configs[3] of the reference's decode use (sparse_int8_linear / int8_linear
// with a handful of tokens, src/gemm/int8_sparse.cu:1005-1043, src/gemm/int8_dense.cu:213-232),
// where the weights are read once per call and every other operand is tiny.
//
// One 512-thread workgroup owns 32 weight rows and all of K; its 8 wavefronts split K into
// contiguous slices of 128-deep stages. Each wave streams its slice of the 32 weight rows
// through a PRIVATE LDS ring with global_load_lds_dwordx4 (full 128-byte lines per row: the
// fastest load path into a CU), so only the wave's own vmcnt orders the ring -- no barrier in
// the K loop. The stage's 16 token rows ride in the same slot, also by DMA. Dense: 3 slots of
// 6 KB, 2 stages in flight per wave; sparse: 4 slots of 4.5 KB, 3 in flight (144 KB of LDS,
// one workgroup per CU). Dense stages feed
// 2 x 2 v_mfma_i32_16x16x64_i8 (weights as the A operand); sparse stages feed 2
// v_smfmac_i32_16x16x128_i8 (compressed weights + index words as A, lane layout as in
// gemm_sparse.hip). The 8 per-wave INT32 partials are summed exactly through LDS, then the
// dequant epilogue writes the outputs.
//
// Each wave's stage count is padded to S in {1, 2, 4, 8} (K <= 8192): padding stages
// re-read the last real weights (into a slot never read again) and multiply them by zero
// tokens, and the whole per-wave sequence is unrolled, so it has no branches, constant ring
// indices and exact waits.
#include "common.h"
#include "gemm_dense.h"
#include "mfma_tile.h"

namespace forge_amd {

constexpr int kDecRows = 32;       // weight rows per workgroup
constexpr int kDecWaves = 8;
constexpr int kDecTokRows = 16;    // token rows staged per stage (the MFMA's 16 columns)

template <bool SPARSE>
struct DecodeCfg {
    // Per-wave ring slot: weights (dense 32 rows x 128 B; sparse 32 rows x 64 compressed B and
    // 2 x 64 index words), then the stage's 16 token rows x 128 B.
    static constexpr int kWBytes = SPARSE ? kDecRows * 64 : kDecRows * 128;
    static constexpr int kIBytes = SPARSE ? 2 * 256 : 0;
    static constexpr int kXBytes = kDecTokRows * 128;
    static constexpr int kSlotBytes = kWBytes + kIBytes + kXBytes;
    static constexpr int kSlots = SPARSE ? 4 : 3;                // ring depth: 144 KB of LDS either way
    static constexpr int kWIns = kWBytes / 1024;                 // 1 KB DMA instructions per stage
    static constexpr int kVmPerStage = kWIns + (SPARSE ? 1 : 0) + kXBytes / 1024;
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
__device__ __forceinline__ void lds_read2(const int8_t* p0, const int8_t* p1, v4i& a0, v4i& a1)
{
    asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(a0), "=&v"(a1) : "v"(lds_addr(p0)), "v"(lds_addr(p1)) : "memory");
}
__device__ __forceinline__ void lds_read_idx(const uint32_t* q0, const uint32_t* q1, int& i0, int& i1)
{
    asm volatile("ds_read_b32 %0, %2\n\tds_read_b32 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(i0), "=&v"(i1) : "v"(lds_addr(q0)), "v"(lds_addr(q1)) : "memory");
}

// S: stages per wave after padding (1, 2, 4 or 8). The per-wave stage sequence is
// straight-line code with constant ring slots; every load in it is a DMA into LDS, so the only
// vmcnt waits are the ring's own (whole stages, counted from the end).
template <bool SPARSE, bool DEQUANT, int S>
__global__ __launch_bounds__(kDecWaves * kWave) void decode_kernel(
    const int8_t* __restrict__ W, const uint32_t* __restrict__ meta, const int8_t* __restrict__ X,
    GemmEpilogue ep, int K)
{
    using Cfg = DecodeCfg<SPARSE>;
    constexpr int D = Cfg::kSlots;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    // One LDS array per ring slot (all waves' copies of that slot).
    __shared__ __align__(16) int8_t slot0[kDecWaves * Cfg::kSlotBytes];
    __shared__ __align__(16) int8_t slot1[kDecWaves * Cfg::kSlotBytes];
    __shared__ __align__(16) int8_t slot2[kDecWaves * Cfg::kSlotBytes];
    __shared__ __align__(16) int8_t slot3[SPARSE ? kDecWaves * Cfg::kSlotBytes : 16];
    auto slot_base = [&](int slot) -> int8_t* {
        int8_t* b = slot == 0 ? slot0 : slot == 1 ? slot1 : slot == 2 ? slot2 : slot3;
        return b + wave * Cfg::kSlotBytes;
    };
    const int n0 = blockIdx.x * kDecRows;
    const int M = ep.M, N = ep.N;
    const int r16 = lane & 15, g = lane >> 4;

    // This wave's stages [s0, s0 + ns), ns <= S; stages ns..S-1 are padding.
    const int nst = K / 128;
    const int s0 = wave * S < nst ? wave * S : nst;
    const int ns = (s0 + S < nst ? s0 + S : nst) - s0;

    // DMA sources at K stage 0. Lane s of a 1 KB instruction fills LDS bytes [16 s, +16) of
    // its part of the slot: row s >> 3 (dense, tokens) or s >> 2 (sparse weights), at the
    // swizzled chunk position.
    const int8_t* pw[Cfg::kWIns];
    const int wrow_bytes = SPARSE ? K / 2 : K;
#pragma unroll
    for (int q = 0; q < Cfg::kWIns; q++) {
        const int s = q * kWave + lane;
        const int r = SPARSE ? (s >> 2) : (s >> 3);
        const int c = SPARSE ? ((s & 3) ^ lds_swz4(r)) : ((s & 7) ^ lds_swz8(r));
        const int gr = (n0 + r) < N ? (n0 + r) : N - 1;
        pw[q] = W + static_cast<size_t>(gr) * wrow_bytes + 16 * c;
    }
    const int8_t* px[2];
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const int s = q * kWave + lane;
        const int r = s >> 3;
        const int c = (s & 7) ^ lds_swz8(r);
        px[q] = X + static_cast<size_t>(r < M ? r : M - 1) * K + 16 * c;   // rows >= M: zeroed on read
    }
    const int8_t* pi = nullptr;
    if constexpr (SPARSE) {
        // 2 blocks of 16 rows x 64 words per stage; lanes 0..31 each copy 16 bytes.
        const int cpr = K / 32;
        int b = (n0 >> 4) + ((lane & 31) >> 4);
        b = b < (N >> 4) ? b : (N >> 4) - 1;
        pi = reinterpret_cast<const int8_t*>(meta + static_cast<size_t>(b) * cpr * 16) + 16 * (lane & 15);
    }

    auto issue = [&](int t, int slot) {
        const int st = s0 + (t < ns ? t : ns - 1);
        int8_t* dst = slot_base(slot);
        const int wk = SPARSE ? st * 64 : st * 128;
#pragma unroll
        for (int q = 0; q < Cfg::kWIns; q++) dma16(pw[q] + wk, dst + q * 1024);
        if constexpr (SPARSE) {
            if (lane < 32) dma16(pi + st * 256, dst + Cfg::kWBytes);
        }
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
        const bool live = tok && real;
        if constexpr (SPARSE) {
            // B: token row r16, K [16g, +16) and [64 + 16g, +16); A: compressed rows, chunk g.
            v4i a0, a1, xlo, xhi;
            lds_read4(src + lds_off64(r16, g), src + lds_off64(16 + r16, g), xs + lds_off128(r16, g),
                      xs + lds_off128(r16, 4 + g), a0, a1, xlo, xhi);
            int i0, i1;
            const uint32_t* idx = reinterpret_cast<const uint32_t*>(src + Cfg::kWBytes);
            lds_read_idx(idx + lane, idx + 64 + lane, i0, i1);
            if (!live) {
                xlo = v4i{0, 0, 0, 0};
                xhi = v4i{0, 0, 0, 0};
            }
            const v8i b = __builtin_shufflevector(xlo, xhi, 0, 1, 2, 3, 4, 5, 6, 7);
            acc[0] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(a0, b, acc[0], i0, 0, 0);
            acc[1] = __builtin_amdgcn_smfmac_i32_16x16x128_i8(a1, b, acc[1], i1, 0, 0);
        } else {
            // Two 16x16x64 steps h = 0, 1 over K [64h, +64): lane chunk g of each half.
            v4i xlo, xhi, a00, a01, a10, a11;
            lds_read4(src + lds_off128(r16, g), src + lds_off128(r16, 4 + g), src + lds_off128(16 + r16, g),
                      src + lds_off128(16 + r16, 4 + g), a00, a01, a10, a11);
            lds_read2(xs + lds_off128(r16, g), xs + lds_off128(r16, 4 + g), xlo, xhi);
            if (!live) {
                xlo = v4i{0, 0, 0, 0};
                xhi = v4i{0, 0, 0, 0};
            }
            acc[0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a00, xlo, acc[0], 0, 0, 0);
            acc[0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a01, xhi, acc[0], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a10, xlo, acc[1], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a11, xhi, acc[1], 0, 0, 0);
        }
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
    if (threadIdx.x < 2 * kWave) {
        const int blk = threadIdx.x / kWave;
        v4i s = v4i{0, 0, 0, 0};
#pragma unroll
        for (int w = 0; w < kDecWaves; w++) s += red[(w * 2 + blk) * kWave + lane];
        const int m = r16;
        if (m < M) {
            const int nb = n0 + 16 * blk + 4 * g;
            const float as = DEQUANT ? ep.act_scale[m] : 0.0f;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int n = nb + e;
                if (n >= N) continue;
                const size_t o = static_cast<size_t>(m) * N + n;
                if constexpr (DEQUANT) {
                    const float b = ep.bias ? h2f(ep.bias[n]) : 0.0f;
                    ep.c16[o] = dequant_gemm(s[e], as, h2f(ep.w_scale[n]), b, ep.bias != nullptr);
                } else {
                    ep.c32[o] = s[e];
                }
            }
        }
    }
}

template <bool SPARSE, bool DEQUANT, int S>
static int launch_decode_s(const int8_t* W, const uint32_t* meta, const int8_t* X, const GemmEpilogue& ep, int K,
                           hipStream_t s)
{
    const unsigned grid = static_cast<unsigned>(divup(ep.N, kDecRows));
    decode_kernel<SPARSE, DEQUANT, S><<<grid, kDecWaves * kWave, 0, s>>>(W, meta, X, ep, K);
    return launch_status();
}

template <bool SPARSE, bool DEQUANT>
static int launch_decode_t(const int8_t* W, const uint32_t* meta, const int8_t* X, const GemmEpilogue& ep, int K,
                           hipStream_t s)
{
    const int per = divup(K / 128, kDecWaves);
    if (per <= 1) return launch_decode_s<SPARSE, DEQUANT, 1>(W, meta, X, ep, K, s);
    if (per <= 2) return launch_decode_s<SPARSE, DEQUANT, 2>(W, meta, X, ep, K, s);
    if (per <= 4) return launch_decode_s<SPARSE, DEQUANT, 4>(W, meta, X, ep, K, s);
    return launch_decode_s<SPARSE, DEQUANT, 8>(W, meta, X, ep, K, s);
}

bool decode_supported(int M, int K) { return M <= kDecodeMaxM && K % 128 == 0 && K <= kDecodeMaxK; }

int launch_decode(const int8_t* W, const uint32_t* meta, const int8_t* X, const GemmEpilogue& ep, int K,
                  bool sparse, hipStream_t s)
{
    if (!decode_supported(ep.M, K)) return FORGE_EINVAL;
    if (sparse) return ep.c16 ? launch_decode_t<true, true>(W, meta, X, ep, K, s) : launch_decode_t<true, false>(W, meta, X, ep, K, s);
    return ep.c16 ? launch_decode_t<false, true>(W, meta, X, ep, K, s) : launch_decode_t<false, false>(W, meta, X, ep, K, s);
}

}  // namespace forge_amd
