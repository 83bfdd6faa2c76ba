// NHWC INT8 conv2d, stride 1, as a window-fed MFMA tile (configs[4]-class shapes: C % 128 == 0,
// Co % 256 == 0, a few image rows per tile).
//
// The implicit GEMM of the dense engine (mfma_tile.h DmaConv) gathers a patch row per output
// pixel and tap, so a 3x3 conv moves every input byte through the LDS DMA nine times per tile.
// Here a tile is R whole output rows of one image (TW = R * Wo = 32 NI pixels) x 256 output
// channels: the input window those rows touch (R + (kH-1) dilH rows x Wo + (kW-1) dilW columns,
// zeros where it leaves the image) is loaded into LDS once per 128-channel chunk, and every tap's
// A fragment is read from it at the tap's pixel shift. Only the weights stream per tap
// (256 rows x 128 bytes a stage: the dense engine's 2-slot ring with a double-buffered window,
// or, where two windows do not fit, a 3-slot ring with one). For configs[4] (56 x 56 x 256 ->
// 256, 3x3): 224-pixel tiles move 89 KB of window + 576 KB of weights instead of 2 x 590 KB.
//
// Integer sums do not depend on the order of K, so the INT32 result equals the reference's
// im2col GEMM (src/nn/int8_conv2d.cu:151-223) on the same integers, and the FP16 epilogue is
// the dense GEMM's (int8_dense.cu:171-174).
#include "common.h"
#include "mfma_tile.h"
#include "gemm_dense.h"

namespace forge_amd {

namespace {

constexpr int kWinMaxQ = 16;          // window DMA instructions per wave (<= 512 pixels)
constexpr int kWinLds = 160 * 1024;   // LDS per workgroup

struct ConvWinArgs {
    const int8_t* x;          // NHWC image
    const int8_t* w;          // OHWI weights = (Co, K) row-major, K = kH kW C in (kh, kw, c) order
    GemmEpilogue ep;
    uint32_t x_bytes;
    int H, W, C, K, kW, T;    // T = kH kW taps
    int padH, padW, dilH, dilW;
    int Ho, Wo, WC, nwin;     // window columns WC (row stride), window pixels nwin
    int nc, nqw, win_bytes;   // 128-channel chunks, window DMA instructions per wave, bytes per window
    int R, tiles_h;           // output rows per tile (32 NI pixels), tiles per image
    int tiles_m, tiles_n;     // row tiles, 256-channel column tiles
};

// s_waitcnt vmcnt(N) lgkmcnt(0) (expcnt unconstrained; gfx9 splits the 6-bit vmcnt over bits
// [3:0] and [15:14]).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm() {
    static_assert(N >= 0 && N < 64, "vmcnt immediate");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4));
}

// Wave-uniform position of stage st = ch * T + tap.
struct StagePos {
    int ch, tap, kh, kw;
    __device__ __forceinline__ void next(int T, int kW) {
        if (++tap == T) {
            tap = 0;
            kh = 0;
            kw = 0;
            ch++;
        } else if (++kw == kW) {
            kw = 0;
            kh++;
        }
    }
};

}  // namespace

// One tile per workgroup (4 waves) of R output rows from row ho0 of image img (32 NI pixels) x
// 256 output channels from n0: wave w owns channels [64 w, +64) of all the tile's pixels,
// 2 x NI accumulator blocks of v_mfma_i32_32x32x32_i8. Tiles map to workgroups XCD-aware.
template <int NI, int SLOTS, bool DEQUANT>
__global__ __launch_bounds__(kGemmThreads) void conv_window_kernel(ConvWinArgs a)
{
    extern __shared__ __align__(16) int8_t lds[];
    int tm, tn;
    tile_coords(static_cast<int>(blockIdx.x), a.tiles_m, a.tiles_n, tm, tn);
    const int img = tm / a.tiles_h;
    const int ho0 = (tm - img * a.tiles_h) * a.R;
    const int n0 = tn * 256;
    constexpr int kBN = 256;                   // tile channels
    constexpr int kSlot = kBN * kBK;           // weight ring slot bytes
    constexpr int kBI = kBN / 32;              // weight DMA instructions per wave per stage
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int l31 = lane & 31, hi = lane >> 5;
    const int m0 = (img * a.Ho + ho0) * a.Wo;  // pixel index of the tile's first pixel
    const int h0 = ho0 - a.padH;               // input row of window row 0

    // FP16 out: the rows' activation scales are loaded first: a load issued after the epilogue's
    // stores would be waited for together with them (one counter covers both).
    [[maybe_unused]] float asv[NI];
    if constexpr (DEQUANT) {
#pragma unroll
        for (int i = 0; i < NI; i++) asv[i] = a.ep.act_scale[m0 + 32 * i + l31];
    }

    int8_t* ring = lds;
    int8_t* win = lds + SLOTS * kSlot;

    // Weight DMA lanes: instruction q of this wave fills ring chunks s = (kBI wave + q) 64 + lane,
    // row s / 8, physical chunk s % 8 = logical chunk (s % 8) ^ swz(row).
    uint32_t lb[kBI];
#pragma unroll
    for (int q = 0; q < kBI; q++) {
        const int s = (wave * kBI + q) * kWave + lane;
        const int r = s >> 3, c = (s & 7) ^ lds_swz8(r);
        lb[q] = static_cast<uint32_t>(n0 + r) * static_cast<uint32_t>(a.K) + 16u * c;
    }
    // Window DMA lanes: chunk s = (nqw wave + q) 64 + lane is window pixel wp = s / 8 (row
    // wr = wp / WC, column wc), physical chunk s % 8 = logical 16-channel group
    // (s % 8) ^ ((v / 2) % 8) with v = wr Wo + wc. A fragment read's 16-lane groups take 16
    // consecutive output pixels, whose v are 16 consecutive integers across a row wrap too, and
    // WC - Wo is even (the host pads WC), so wp % 2 = v % 2: the 16 reads fill the 16 16-byte
    // slots of a 256-byte bank row once each. Offsets outside the image (padding, or past the
    // window) read as zeros.
    uint32_t vo[kWinMaxQ];
#pragma unroll
    for (int q = 0; q < kWinMaxQ; q++) {
        const int s = (wave * a.nqw + q) * kWave + lane;
        const int wp = s >> 3;
        const int wr = wp / a.WC, wc = wp - wr * a.WC;
        const int cj = (s & 7) ^ (((wr * a.Wo + wc) >> 1) & 7);
        const int hin = h0 + wr, win_c = wc - a.padW;
        const bool ok = q < a.nqw && wp < a.nwin && hin >= 0 && hin < a.H && win_c >= 0 && win_c < a.W;
        vo[q] = ok ? static_cast<uint32_t>(((img * a.H + hin) * a.W + win_c) * a.C + 16 * cj) : 0x80000000u;
    }
    // Window pixel of tile pixel p = 32 i + l31 at tap (0, 0).
    int wp0[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int p = 32 * i + l31;
        const int r = p / a.Wo;
        wp0[i] = r * a.WC + (p - r * a.Wo);
    }

    const __amdgpu_buffer_rsrc_t xres = buf_rsrc(a.x, a.x_bytes);
    const __amdgpu_buffer_rsrc_t wres = buf_rsrc(a.w, static_cast<uint32_t>(a.tiles_n * kBN) * static_cast<uint32_t>(a.K));
    const int nst = a.nc * a.T;

    auto issue_w = [&](int st, const StagePos& P) {
        int8_t* slot = ring + (st % SLOTS) * kSlot;
        const uint32_t soff = static_cast<uint32_t>(P.tap * a.C + P.ch * kBK);
#pragma unroll
        for (int q = 0; q < kBI; q++) dma16_buf(wres, lb[q], soff, slot + (wave * kBI + q) * 1024);
    };
    // With 2 ring slots the window is double-buffered by chunk parity; with 3, single.
    auto win_buf = [&](int ch) { return win + (SLOTS == 2 ? (ch & 1) * a.win_bytes : 0); };
    auto issue_win = [&](int ch) {
        int8_t* buf = win_buf(ch);
#pragma unroll
        for (int q = 0; q < kWinMaxQ; q++)
            if (q < a.nqw) dma16_buf(xres, vo[q] + static_cast<uint32_t>(ch * kBK), 0, buf + (wave * a.nqw + q) * 1024);
    };

    struct Frags {
        v4i a[NI];
        v4i b[2];
    };
    v16i acc[2][NI];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[j][i][e] = 0;

    auto load_frags = [&](int st, const StagePos& P, int ks, Frags& F) {
        const int8_t* wb = win_buf(P.ch);
        const int8_t* bs = ring + (st % SLOTS) * kSlot;
        const int tp = P.kh * a.dilH * a.WC + P.kw * a.dilW;       // window pixel shift
        const int tv = P.kh * a.dilH * a.Wo + P.kw * a.dilW;       // its v shift
        const int c = 2 * ks + hi;
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int sw = ((32 * i + l31 + tv) >> 1) & 7;
            F.a[i] = *reinterpret_cast<const v4i*>(wb + ((wp0[i] + tp) << 7) + ((c ^ sw) << 4));
        }
#pragma unroll
        for (int j = 0; j < 2; j++)
            F.b[j] = *reinterpret_cast<const v4i*>(bs + lds_off128(64 * wave + 32 * j + l31, c));
    };
    auto mfmas = [&](const Frags& F) {
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int i = 0; i < NI; i++)
                acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(F.b[j], F.a[i], acc[j][i], 0, 0, 0);
    };

    // Fragments are read two sub-steps ahead of their MFMAs, as in the dense engine.
    // SLOTS = 2: the dense engine's ring (the weight DMA of stage kt+2 after the barrier of stage
    // kt, into its slot), and the window of chunk ch+1 is issued at the first stage of chunk ch
    // into the other window buffer (which last served chunk ch-1, whose reads ended before this
    // barrier); it has landed by the barrier that publishes chunk ch+1's first stage (T >= 2).
    // SLOTS = 3: the DMA of stage kt+3 goes out after the barrier of stage kt (into stage kt's
    // slot), so each stage's weights have two stages of lead, and the wait before a barrier
    // leaves the kBI DMAs of the next stage in flight (vector-memory loads return in issue
    // order); the one window buffer is reloaded after the barrier that ends the last reads of a
    // chunk, and the workgroup waits for it.
    constexpr int kMf = 2 * NI, kRd = NI + 2, kVm = kBI / 2;
    Frags F0, F1, F2, F3;
    StagePos P0{0, 0, 0, 0};                   // stage kt
    StagePos P1 = P0;                          // stage kt + 1
    P1.next(a.T, a.kW);
    StagePos P2 = P1;                          // stage kt + 2
    P2.next(a.T, a.kW);
    StagePos P3 = P2;                          // stage kt + 3
    P3.next(a.T, a.kW);
    issue_win(0);
    issue_w(0, P0);
    issue_w(1, P1);
    if constexpr (SLOTS == 3) {
        issue_w(2, P2);
        wait_vm_lgkm<2 * kBI>();               // window and stage 0
    } else {
        wait_vm_lgkm<kBI>();
    }
    lds_barrier();
    load_frags(0, P0, 0, F0);
    load_frags(0, P0, 1, F1);
    for (int kt = 0; kt + 1 < nst; kt++) {
        load_frags(kt, P0, 2, F2);
        mfmas(F0);
        sched_interleave<kMf, kRd, 0>();
        load_frags(kt, P0, 3, F3);
        mfmas(F1);
        sched_interleave<kMf, kRd, 0>();
        if constexpr (SLOTS == 3) {
            wait_vm_lgkm<kBI>();               // stage kt+1 landed; stage kt+2 may be in flight
            lds_barrier();
            if (P1.tap == 0) {                 // stage kt+1 opens chunk P1.ch
                issue_win(P1.ch);
                wait_vm_lgkm<0>();
                lds_barrier();
            }
            issue_w(kt + 3, P3);               // into stage kt's slot; past the end: unused re-reads
        } else {
            wait_vm_lgkm<0>();                 // stage kt+1 (and a window issued one stage ago)
            lds_barrier();
            if (P0.tap == 0 && P0.ch + 1 < a.nc) issue_win(P0.ch + 1);
            issue_w(kt + 2, P2);               // into stage kt's slot; past the end: unused re-reads
        }
        load_frags(kt + 1, P1, 0, F0);
        mfmas(F2);
        load_frags(kt + 1, P1, 1, F1);
        mfmas(F3);
        sched_interleave<kMf, 0, 2 * kVm>();
        sched_interleave<kMf, 2 * kRd, 0>();
        P0 = P1;
        P1 = P2;
        P2 = P3;
        P3.next(a.T, a.kW);
    }
    load_frags(nst - 1, P0, 2, F2);
    mfmas(F0);
    load_frags(nst - 1, P0, 3, F3);
    mfmas(F1);
    mfmas(F2);
    mfmas(F3);
    wait_vm_lgkm0();
    lds_barrier();

    // Epilogue: per 32-pixel block, the wave's 32 x 64 outputs go through a wave-private LDS
    // strip (16-byte units XOR-swizzled by row) and out as coalesced 16-byte row stores.
    const GemmEpilogue& ep = a.ep;
    const int rm = m0;                         // the wave's first pixel
    const int cn = n0 + 64 * wave;             // the wave's first channel
    if constexpr (DEQUANT) {
        constexpr int kU = 8;                  // 64 FP16 columns = 8 units of 16 bytes
        int8_t* strip = lds + wave * (32 * kU * 16);
        uint16_t* wsl = reinterpret_cast<uint16_t*>(lds + 4 * 32 * kU * 16) + wave * 128;
        uint16_t* bl = wsl + 64;
        const bool has_bias = ep.bias != nullptr;
        wsl[lane] = ep.w_scale[cn + lane];
        bl[lane] = has_bias ? ep.bias[cn + lane] : static_cast<uint16_t>(0);
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const float as = asv[i];
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const int nl = 32 * j + 8 * g + 4 * hi;
                    const uint2 w2 = *reinterpret_cast<const uint2*>(wsl + nl);
                    const uint2 b2 = *reinterpret_cast<const uint2*>(bl + nl);
                    const uint32_t wv[4] = {w2.x & 0xFFFFu, w2.x >> 16, w2.y & 0xFFFFu, w2.y >> 16};
                    const uint32_t bv[4] = {b2.x & 0xFFFFu, b2.x >> 16, b2.y & 0xFFFFu, b2.y >> 16};
                    float ws[4], b[4];
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        ws[t] = h2f(static_cast<uint16_t>(wv[t]));
                        b[t] = has_bias ? h2f(static_cast<uint16_t>(bv[t])) : -0.0f;
                    }
                    const int u = 4 * j + g;
                    *reinterpret_cast<uint2*>(strip + l31 * (kU * 16) + ((u ^ (l31 & (kU - 1))) << 4) + 8 * hi) =
                        dequant4_pk(acc[j][i][4 * g], acc[j][i][4 * g + 1], acc[j][i][4 * g + 2], acc[j][i][4 * g + 3],
                                    as, ws, b);
                }
            flush_rows<kU, 2, true, true, 32>(strip, ep, rm + 32 * i, cn);
        }
    } else {
        constexpr int kU = 16;                 // 64 INT32 columns = 16 units of 16 bytes
        int8_t* strip = lds + wave * (32 * kU * 16);
#pragma unroll
        for (int i = 0; i < NI; i++) {
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const int u = 8 * j + 2 * g + hi;
                    *reinterpret_cast<int4*>(strip + l31 * (kU * 16) + ((u ^ (l31 & (kU - 1))) << 4)) =
                        make_int4(acc[j][i][4 * g], acc[j][i][4 * g + 1], acc[j][i][4 * g + 2], acc[j][i][4 * g + 3]);
                }
            flush_rows<kU, 4, false, true, 32>(strip, ep, rm + 32 * i, cn);
        }
    }
}

// The kernel's dynamic-LDS limit is raised once to the largest window (host-side attribute).
template <int NI, int SLOTS, bool DEQUANT>
static int launch_win(const ConvWinArgs& a, unsigned grid, int lds, hipStream_t s)
{
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(conv_window_kernel<NI, SLOTS, DEQUANT>),
        hipFuncAttributeMaxDynamicSharedMemorySize, kWinLds);
    if (attr != hipSuccess) return static_cast<int>(attr);
    conv_window_kernel<NI, SLOTS, DEQUANT><<<grid, kGemmThreads, lds, s>>>(a);
    return launch_status();
}

// Returns -1 when the shape is not one the window kernel takes.
int launch_conv_window(const ConvGeom& g, const int8_t* w, const GemmEpilogue& ep, int Co, hipStream_t s)
{
    const int N = g.rows / (g.Ho * g.Wo);
    const int kH = g.K / (g.C * g.kW), T = kH * g.kW;
    if (g.strideH != 1 || g.strideW != 1 || g.C % kBK != 0 || Co % 256 != 0 || T < 2 || g.r0 != 0 ||
        !ep.vec_out || ep.up_w != 0 || !aligned(g.x, 16) || !aligned(w, 16))
        return -1;
    const long long x_bytes = static_cast<long long>(N) * g.H * g.W * g.C;
    if (x_bytes >= (1LL << 31) || static_cast<long long>(Co) * g.K >= (1LL << 31)) return -1;
    // Tile height: R whole output rows with R Wo = 256 or 224 pixels (8 or 7 row blocks).
    int NI = 0, R = 0;
    for (int ni : {8, 7}) {
        if ((32 * ni) % g.Wo == 0 && g.Ho % ((32 * ni) / g.Wo) == 0) {
            NI = ni;
            R = 32 * ni / g.Wo;
            break;
        }
    }
    if (NI == 0) return -1;
    const int tn = Co / 256;
    // Window row stride: the columns the taps reach, padded to keep WC - Wo even (the swizzle).
    long long WC = g.Wo + static_cast<long long>(g.kW - 1) * g.dilW;
    WC += (WC - g.Wo) & 1;
    const long long WR = R + static_cast<long long>(kH - 1) * g.dilH;
    const long long nwin = WR * WC;
    const long long nqw = (nwin * 8 + 4 * kWave - 1) / (4 * kWave);
    // 2 ring slots + two window buffers where they fit (measured faster on configs[4]), else
    // 3 slots + one window buffer.
    const int slots = 2 * 256 * kBK + 2 * nqw * 4 * 1024 <= kWinLds ? 2 : 3;
    const long long lds = static_cast<long long>(slots) * 256 * kBK + (4 - slots) * nqw * 4 * 1024;
    if (nqw > kWinMaxQ || lds > kWinLds) return -1;
    const long long tiles_m = static_cast<long long>(N) * (g.Ho / R);
    if (tiles_m * tn > 0x7FFFFFFFLL) return -1;

    ConvWinArgs a;
    a.x = g.x;
    a.w = w;
    a.ep = ep;
    a.x_bytes = static_cast<uint32_t>(x_bytes);
    a.H = g.H;
    a.W = g.W;
    a.C = g.C;
    a.K = g.K;
    a.kW = g.kW;
    a.T = T;
    a.padH = g.padH;
    a.padW = g.padW;
    a.dilH = g.dilH;
    a.dilW = g.dilW;
    a.Ho = g.Ho;
    a.Wo = g.Wo;
    a.WC = static_cast<int>(WC);
    a.nwin = static_cast<int>(nwin);
    a.nc = g.C / kBK;
    a.nqw = static_cast<int>(nqw);
    a.win_bytes = static_cast<int>(nqw) * 4 * 1024;
    a.R = R;
    a.tiles_h = g.Ho / R;
    a.tiles_m = static_cast<int>(tiles_m);
    a.tiles_n = tn;
    const unsigned grid = static_cast<unsigned>(tiles_m * tn);
    const int l = static_cast<int>(lds);
    const bool o16 = ep.c16 != nullptr;
    note_route(NI == 8 ? (slots == 2 ? "conv-window256" : "conv-window256 ring3")
                       : (slots == 2 ? "conv-window224" : "conv-window224 ring3"));
    if (slots == 2) {
        if (NI == 8) return o16 ? launch_win<8, 2, true>(a, grid, l, s) : launch_win<8, 2, false>(a, grid, l, s);
        return o16 ? launch_win<7, 2, true>(a, grid, l, s) : launch_win<7, 2, false>(a, grid, l, s);
    }
    if (NI == 8) return o16 ? launch_win<8, 3, true>(a, grid, l, s) : launch_win<8, 3, false>(a, grid, l, s);
    return o16 ? launch_win<7, 3, true>(a, grid, l, s) : launch_win<7, 3, false>(a, grid, l, s);
}

}  // namespace forge_amd
