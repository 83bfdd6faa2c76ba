// Wide-tile 2:4 sparse INT8 GEMM with INT32 output for gfx950 (v_smfmac_i32_32x32x64_i8).
//
// Reference: the 2:4 sparse GEMM of src/gemm/int8_sparse.cu:139-736 (mma.sp tiles, persistent
// CTAs); this engine computes the same INT32 sums sum_k x[m,k] * Wp[n,k] (Wp from W_comp and the
// gfx950 index words, int8_sparse.cu:116-120) for the INT32-output extension symbol.
//
// Why a wider tile. A 256 x 256 tile streams per 256-deep slice of K 64 KB of tokens, 32 KB of
// compressed weights and 8 KB of index words through the CU: tokens are most of the bytes, and
// 2:4 sparsity does not touch them. A tile of 256 tokens x W weight rows moves 64 KB + W * 160 B
// per slice for 256 W outputs; at W = 352 that is 20 % fewer bytes per output (measured: the
// DMA-only loop of configs[2], 89 -> 71 us). A workgroup's tiles are planned per CU so that every
// CU gets the same number of 32-row weight blocks (configs[2], 4096 x 11008: 16 CUs per 256-token
// block, 21 or 22 blocks each, as two tiles of 10 or 11 blocks: two tile times, where 256 x 256
// tiles need 2.69 (2.85 with their 192-token tail wave)).
//
// Layout. Four waves, each owning 64 tokens (two 32-token blocks) and all NJ 32-row weight blocks:
// 2 x NJ blocks of 32 x 32 INT32 accumulators per wave (352 registers at NJ = 11, held in the AGPRs
// and the VGPRs). LDS per stage of 128 dense K:
//   tokens: one slot per wave (64 rows x 128 B = one cache line each), filled by DMA and read into
//           registers once per stage; the registers are double-buffered, so a single slot
//           suffices and the weight ring below fits;
//   weights: a 2-slot ring of 256-deep pairs (each compressed row one full 128-byte line per two
//           stages: half-line rows measured 3.5x slower per byte through the LDS DMA);
//   index words: a 2-slot ring of 128-deep stages (the gfx950 word layout, 256-byte runs per
//           16-row block; odd blocks' chunks XOR 12 so a wave's index read hits distinct banks).
// Rows of 128 bytes use the chunk swizzle swzJ below, whose period of 32 rows makes every
// fragment address one per-lane base register plus an immediate (block j: + 4096 j), which keeps
// the 352 accumulators from pushing the addresses into scratch.
//
// Schedule per stage: SMFMACs over (64-deep half h, weight block j) with the A fragment and its
// index word read three steps ahead; 8 steps before the end the wave reads the next stage's
// tokens from its slot into the other register buffer and then refills the slot by DMA (almost
// two stages of lead); at the end, one barrier publishes the next stage's weights/indices and the
// slots this stage used take the stage after next.
//
// Epilogue: each wave stages 32 tokens x 64 columns at a time in LDS and writes whole 16-byte row
// units with cached buffer stores (measured on configs[2]: 116 us cached vs 121.5 us with the
// non-temporal stores of the other engines; direct stores from the accumulator layout write
// 32-byte pieces of 32 rows per instruction: 125 us cached, 315 us non-temporal).
#include "common.h"
#include "gemm_dense.h"
#include "mfma_tile.h"

#include <type_traits>

namespace forge_amd {

namespace {

// s_waitcnt vmcnt(N) lgkmcnt(0) (expcnt unconstrained).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm(void) {
    static_assert(N >= 0 && N < 64, "vmcnt immediate");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4));
}
// s_waitcnt lgkmcnt(N) only.
template <int N>
__device__ __forceinline__ void wait_lgkm(void) {
    static_assert(N >= 0 && N < 16, "lgkmcnt immediate");
    __builtin_amdgcn_s_waitcnt(0xC07F | (N << 8));
}

// Chunk swizzle of 128-byte LDS rows with a period of 32 rows: swzJ(r) = (r ^ (r >> 3)) & 7 for
// r < 32, the swizzle of the other engines' 128-byte rows (bank-conflict free for the 32-row
// fragment reads of the 32x32 matrix-core layouts), repeated every 32 rows.
__device__ __forceinline__ int swzJ(int r) { return ((r ^ (r >> 3)) & 3) ^ (r & 4); }

constexpr int kWidePD = 3;        // A fragments read this many (h, j) steps ahead
constexpr int kWideTokAhead = 8;  // steps before a stage's end at which the next tokens are read

template <int NJ>
struct SpWideTile {
    static constexpr int W = 32 * NJ;
    static constexpr int kWSlot = W * 128;      // compressed rows of one 256-deep stage pair
    static constexpr int kISlot = W * 16;       // index words of one 128-deep stage
    static constexpr int kXWave = 64 * 128;     // a wave's 64 token rows of one stage
    static constexpr int kXOff = 0;
    static constexpr int kIOff = 4 * kXWave;
    static constexpr int kWOff = kIOff + 2 * kISlot;
    static constexpr int kLdsBytes = kWOff + 2 * kWSlot;
    static constexpr int kIIns = (W + 63) / 64;  // index DMA instructions per stage (workgroup)
    static_assert(kIIns <= 8, "two index DMA instructions per wave at most");

    v16i acc[NJ][2];   // acc[j][i]: D[n: 32j + row(e, l)][m: 64 wave + 32i + l%32]

    __device__ __forceinline__ void run(const int8_t* Wc, const int8_t* X, const uint32_t* meta, int M, int N, int K,
                                        int n0, int m0, int8_t* lds) {
        const int lane = threadIdx.x & (kWave - 1);
        const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
        const int l31 = lane & 31, g = lane >> 5;
        const int Kc = K >> 1, cpr = K >> 5;

#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) acc[j][i][e] = 0;

        // DMA lane offsets, formed per issue from a few registers: chunk s = q * 64 + lane of a
        // stage area is row 8 q + lane / 8 (after the wave's first row), and its physical chunk
        // s % 8 receives logical chunk (s % 8) ^ swzJ(row). Rows past the matrix read zeros
        // through the buffer range (their per-lane offset alone lies past it).
        const int lr = lane >> 3;
        const uint32_t wrow0 = static_cast<uint32_t>(n0 + 8 * wave * NJ + lr) * static_cast<uint32_t>(Kc);
        const uint32_t xrow0 = static_cast<uint32_t>(m0 + 64 * wave + lr) * static_cast<uint32_t>(K);
        const int wq0 = wave * NJ;
        auto chunk_of = [&](int q) {   // q: the row's 8-row group, swzJ depends on q % 4 and lr
            return static_cast<uint32_t>((lane & 7) ^ (((lr ^ q) & 3) ^ (lr & 4)));
        };
        uint32_t oi[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int s = (wave + 4 * t) * kWave + lane;      // 16-byte chunk of the stage's index area
            int b = (n0 >> 4) + (s >> 4);
            b = b < (N >> 4) ? b : (N >> 4) - 1;
            const int k = (s & 15) ^ (((s >> 4) & 1) * 12);
            oi[t] = static_cast<uint32_t>(b) * static_cast<uint32_t>(cpr) * 64u + 16u * k;
        }
        const __amdgpu_buffer_rsrc_t rw = buf_rsrc(Wc, static_cast<uint32_t>(N) * static_cast<uint32_t>(Kc));
        const __amdgpu_buffer_rsrc_t rx = buf_rsrc(X, static_cast<uint32_t>(M) * static_cast<uint32_t>(K));
        const __amdgpu_buffer_rsrc_t ri = buf_rsrc(meta, static_cast<uint32_t>(N) * static_cast<uint32_t>(cpr) * 4u);
        const int nst = K / 128;   // a multiple of 4
        int8_t* xs = lds + kXOff + wave * kXWave;

        auto issue_x = [&](int st) {
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const uint32_t o = xrow0 + static_cast<uint32_t>(8 * q) * static_cast<uint32_t>(K) + 16u * chunk_of(q);
                dma16_buf(rx, o, static_cast<uint32_t>(st * 128), xs + q * 1024);
            }
        };
        // The index words of stage st and, for even st, the weight pair (st, st + 1).
        auto issue_wi = [&](int st, auto with_w) {
            constexpr bool WW = decltype(with_w)::value;
            if constexpr (WW) {
                int8_t* wslot = lds + kWOff + ((st >> 1) & 1) * kWSlot;
#pragma unroll
                for (int q = 0; q < NJ; q++) {
                    const uint32_t o = wrow0 + static_cast<uint32_t>(8 * q) * static_cast<uint32_t>(Kc) +
                                       16u * chunk_of(wq0 + q);
                    dma16_buf(rw, o, static_cast<uint32_t>(st * 64), wslot + (wave * NJ + q) * 1024);
                }
            }
            int8_t* islot = lds + kIOff + (st & 1) * kISlot;
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const int q = wave + 4 * t;
                if (q < kIIns && (q * kWave + 64 <= W || lane < (W & 63)))
                    dma16_buf(ri, oi[t], static_cast<uint32_t>(st * 256), islot + q * 1024);
            }
        };
        // Per-lane parts of the fragment addresses (bytes into lds): tokens [h][lo/hi half],
        // weights [slot][half of the pair][h], index words [half][h]; blocks add immediates.
        const int swl = swzJ(l31);
        uint32_t xb[2][2], wb[2][2][2], ib[2][2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
#pragma unroll
            for (int p = 0; p < 2; p++)
                xb[h][p] = kXOff + wave * kXWave + l31 * 128 + (((4 * h + 2 * p + g) ^ swl) << 4);
#pragma unroll
            for (int sl = 0; sl < 2; sl++)
#pragma unroll
                for (int hf = 0; hf < 2; hf++)
                    wb[sl][hf][h] = kWOff + sl * kWSlot + l31 * 128 + (((4 * hf + 2 * h + g) ^ swl) << 4);
            const int w = ((2 * h + g) * 16 + (l31 & 15)) ^ (((l31 >> 4) & 1) * 48);
#pragma unroll
            for (int hf = 0; hf < 2; hf++) ib[hf][h] = kIOff + hf * kISlot + 4 * ((l31 >> 4) * 64 + w);
        }
        // The B operand of token block i, half h: bytes 0-15 = K [16g, +16), 16-31 = K [32 + 16g, +16)
        // of the 64-deep half (the 32x32x64 SMFMAC B layout).
        auto read_x = [&](v8i (&B)[2][2]) {
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const v4i lo = *reinterpret_cast<const v4i*>(lds + xb[h][0] + 4096 * i);
                    const v4i hi = *reinterpret_cast<const v4i*>(lds + xb[h][1] + 4096 * i);
                    B[i][h] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                }
        };

        v8i B0[2][2], B1[2][2];
        // Prologue: tokens of stage 0 into B0, stage 1 into the slot; weights pair 0, indices 0, 1.
        issue_x(0);
        issue_wi(0, std::true_type{});
        issue_wi(1, std::false_type{});
        wait_vm_lgkm0();
        read_x(B0);
        wait_lgkm<0>();
        issue_x(1);
        wait_vm_lgkm0();
        lds_barrier();

        constexpr int kSteps = 2 * NJ;
        constexpr int PD = kWidePD, RING = PD + 1;
        constexpr int TB = kSteps - kWideTokAhead;   // step reading the next stage's tokens
        constexpr int TD = TB + 3;                   // step after which the slot is refilled
        static_assert(TB > 0 && TD < kSteps && 2 * PD < 16, "stage schedule");
        // One stage st (SL = weight slot, HF = half of the weight pair): Bc holds its tokens.
        auto stage = [&](int st, v8i (&Bc)[2][2], v8i (&Bn)[2][2], auto slc, auto hfc) {
            constexpr int SL = decltype(slc)::value, HF = decltype(hfc)::value;
            auto read_a = [&](int t, v4i& av, int& iv) {
                const int h = t / NJ, j = t % NJ;
                av = *reinterpret_cast<const v4i*>(lds + wb[SL][HF][h] + 4096 * j);
                iv = *reinterpret_cast<const int*>(lds + ib[HF][h] + 512 * j);
            };
            v4i a[RING];
            int ix[RING];
#pragma unroll
            for (int t = 0; t < PD; t++) read_a(t, a[t], ix[t]);
#pragma unroll
            for (int t = 0; t < kSteps; t++) {
                const int h = t / NJ, j = t % NJ;
                if (t == TB) {
                    // The tokens of st+1 (DMA issued in stage st-1) have landed once only the
                    // indices (and, HF == 1, weights) of st+1 issued after them may be in flight:
                    // 1 (+ NJ) instructions per wave at least. Past the end nothing was issued
                    // (the buffer is read but not used).
                    wait_vmcnt<HF == 1 ? NJ + 1 : 1>();
                    read_x(Bn);
                }
                if (t + PD < kSteps) read_a(t + PD, a[(t + PD) % RING], ix[(t + PD) % RING]);
                acc[j][0] = __builtin_amdgcn_smfmac_i32_32x32x64_i8(a[t % RING], Bc[0][h], acc[j][0], ix[t % RING],
                                                                    0, 0);
                acc[j][1] = __builtin_amdgcn_smfmac_i32_32x32x64_i8(a[t % RING], Bc[1][h], acc[j][1], ix[t % RING],
                                                                    0, 0);
                if (t == TD) {
                    // LDS reads return in order and the token reads precede the 2 PD operations
                    // issued since: once at most those are outstanding, the slot is free.
                    wait_lgkm<2 * PD>();
                    if (st + 2 < nst) issue_x(st + 2);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            // The indices (and weights) of st+1, issued at the end of st-1, must land; the 8
            // token DMAs of st+2 issued above may stay in flight (if they were issued).
            if (st + 2 < nst) wait_vm_lgkm<8>();
            else wait_vm_lgkm0();
            lds_barrier();   // also: every wave is done with the slots stage st used
            if (st + 2 < nst) issue_wi(st + 2, std::integral_constant<bool, HF == 0>{});
        };
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        for (int st = 0; st < nst; st += 4) {
            stage(st, B0, B1, I0{}, I0{});
            stage(st + 1, B1, B0, I0{}, I1{});
            stage(st + 2, B0, B1, I1{}, I0{});
            stage(st + 3, B1, B0, I1{}, I1{});
        }
        wait_vm_lgkm0();
        lds_barrier();
    }

    // INT32 epilogue: per wave, strips of 32 tokens x 64 weight columns (16 units of 16 bytes a
    // row, unit u of row r at slot u ^ (r % 16)) staged in LDS, read back as whole row units and
    // written with buffer stores at 32-bit offsets (M * N * 4 < 2^31, checked by the host); rows
    // past M and columns past N are not stored.
    __device__ __forceinline__ void store_s32(int32_t* C, int M, int N, int m0, int n0, int8_t* lds) {
        const int lane = threadIdx.x & (kWave - 1);
        const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
        const int l31 = lane & 31, hi = lane >> 5;
        const __amdgpu_buffer_rsrc_t rc = buf_rsrc(C, static_cast<uint32_t>(M) * static_cast<uint32_t>(N) * 4u);
        int8_t* strip = lds + wave * (32 * 256);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int row0 = m0 + 64 * wave + 32 * i;
#pragma unroll
            for (int jp = 0; jp < NJ; jp += 2) {
                const int nb = (jp + 1 < NJ) ? 2 : 1;          // 32-column blocks in this strip
#pragma unroll
                for (int jj = 0; jj < 2; jj++) {
                    if (jj < nb) {
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            const int u = 8 * jj + 2 * q + hi;
                            const v16i& A = acc[jp + jj][i];
                            *reinterpret_cast<int4*>(strip + l31 * 256 + ((u ^ (l31 & 15)) << 4)) =
                                make_int4(A[4 * q], A[4 * q + 1], A[4 * q + 2], A[4 * q + 3]);
                        }
                    }
                }
                int4 v[8];
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const int idx = lane + 64 * k, r = idx >> 4, u = idx & 15;
                    v[k] = *reinterpret_cast<const int4*>(strip + r * 256 + ((u ^ (r & 15)) << 4));
                }
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const int idx = lane + 64 * k, r = idx >> 4, u = idx & 15;
                    const int row = row0 + r, col = n0 + 32 * jp + 4 * u;
                    if (row < M && u < 8 * nb && col < N) {
                        const uint32_t off =
                            (static_cast<uint32_t>(row) * static_cast<uint32_t>(N) + static_cast<uint32_t>(col)) * 4u;
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, v[k]), rc, off, 0, 0);
                    }
                }
            }
        }
    }
};

template <int NJ>
__device__ __forceinline__ void wide_tile(const int8_t* Wc, const int8_t* X, const uint32_t* meta, int32_t* C, int M,
                                          int N, int K, int n0, int m0, int8_t* lds) {
    SpWideTile<NJ> T;
    T.run(Wc, X, meta, M, N, K, n0, m0, lds);
    T.store_s32(C, M, N, m0, n0, lds);
}

}  // namespace

// Grid = T x S workgroups; workgroup b runs tile k = b / S of CU slot b % S. Each slot is a
// 256-token block tb and a run of weight blocks ci: the first r CUs of a token block take q + 1
// blocks, the rest q, as T tiles of 8-11 blocks. XCD grouping: workgroups go round-robin over the
// 8 XCDs (b % 8), and with gc > 0 the 32 slots of an XCD are gt token blocks x gc block runs, so
// that their tokens and weights meet in one L2.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void sparse_wide_s32_kernel(
    const int8_t* __restrict__ Wc, const int8_t* __restrict__ X, const uint32_t* __restrict__ meta,
    int32_t* __restrict__ C, int M, int N, int K, SpWidePlan p)
{
    extern __shared__ __align__(16) int8_t lds[];
    const int S = p.TB * p.c;
    const int bid = static_cast<int>(blockIdx.x);
    const int k = bid / S, slot = bid - k * S;
    int tb, ci;
    if (p.gc > 0) {
        const int x = slot & 7, local = slot >> 3;
        const int cg = p.c / p.gc;
        tb = (x / cg) * p.gt + local / p.gc;
        ci = (x % cg) * p.gc + local % p.gc;
    } else {
        tb = slot / p.c;
        ci = slot - tb * p.c;
    }
    const int nb = p.q + (ci < p.r ? 1 : 0);
    const int b0 = ci * p.q + (ci < p.r ? ci : p.r);
    const int base = nb / p.T, extra = nb % p.T;
    const int nj = base + (k < extra ? 1 : 0);
    const int n0 = (b0 + k * base + (k < extra ? k : extra)) * 32, m0 = tb * 256;
    switch (nj) {
        case 11: wide_tile<11>(Wc, X, meta, C, M, N, K, n0, m0, lds); break;
        case 10: wide_tile<10>(Wc, X, meta, C, M, N, K, n0, m0, lds); break;
        case 9: wide_tile<9>(Wc, X, meta, C, M, N, K, n0, m0, lds); break;
        default: wide_tile<8>(Wc, X, meta, C, M, N, K, n0, m0, lds); break;
    }
}

bool sparse_wide_plan(int M, int N, int K, int cu, SpWidePlan* out)
{
    if (M <= 0 || N <= 0 || K < 512 || K % 512 != 0 || N % 16 != 0 || cu < 8) return false;
    if (static_cast<long long>(M) * K >= (1LL << 31) || static_cast<long long>(N) * (K / 2) >= (1LL << 31) ||
        static_cast<long long>(M) * N * 4 >= (1LL << 31))
        return false;
    SpWidePlan p{};
    p.TB = divup(M, 256);
    if (p.TB > cu / 8) return false;
    p.c = cu / p.TB;
    const int NB = divup(N, 32);
    p.q = NB / p.c;
    p.r = NB % p.c;
    const int nbmax = p.q + (p.r > 0 ? 1 : 0);
    p.T = divup(nbmax, 11);
    if (p.T < 1 || p.T > 4 || p.q / p.T < 8) return false;
    p.gc = 0;
    p.gt = 0;
    if (p.TB * p.c == cu && cu == 256) {
        for (int gc : {4, 8, 2, 16, 1, 32}) {
            const int gt = 32 / gc;
            if (p.c % gc == 0 && p.TB % gt == 0 && (p.TB / gt) * (p.c / gc) == 8) {
                p.gc = gc;
                p.gt = gt;
                break;
            }
        }
    }
    *out = p;
    return true;
}

int launch_sparse_wide_s32(const int8_t* W_comp, const int8_t* x, const uint32_t* meta, int32_t* C, int M, int K,
                           int N, const SpWidePlan& p, hipStream_t s)
{
    constexpr int lds = SpWideTile<11>::kLdsBytes;
    static_assert(SpWideTile<11>::kLdsBytes >= 4 * 32 * 256, "epilogue strips fit the tile's LDS");
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&sparse_wide_s32_kernel),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (attr != hipSuccess) return static_cast<int>(attr);
    const long long grid = static_cast<long long>(p.T) * p.TB * p.c;
    sparse_wide_s32_kernel<<<static_cast<unsigned>(grid), 256, lds, s>>>(W_comp, x, meta, C, M, N, K, p);
    return launch_status();
}

}  // namespace forge_amd
