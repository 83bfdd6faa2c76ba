// Dense INT8 GEMM for gfx950: C = A (M,K) x B (N,K)^T with exact INT32 accumulation on
// v_mfma_i32_32x32x32_i8, and the fused dequant + bias epilogue to FP16.
//
// Reference: src/gemm/int8_dense.cu:26-232 (wmma 16x16x16, 128x64 / 128x128 tiles,
// unpipelined global->smem loads) and src/gemm/int8_gemm.cu:12-46 (dispatch). The
// epilogue arithmetic follows int8_dense.cu:171-174:
//     Y[m,n] = half(fma((float)acc, act_scale[m] * w_scale[n], bias[n]))
// Row-major operands with K % 128 == 0 run on the DMA engine (global_load_lds into a
// 2-slot LDS ring); other shapes and the conv gather on the register-staged engine
// (mfma_tile.h).
// Tiles are mapped XCD-aware. Skinny M (decode) goes to gemm_skinny.
#include "common.h"
#include "mfma_tile.h"
#include "gemm_dense.h"
#include "forge/gemm/int8_dense.h"
#include "forge/gemm/int8_gemm.h"
#include "forge/gemm/int8_dp4a.h"

#include <algorithm>
#include <type_traits>

namespace forge_amd {

// LDS bytes a tile needs: its K loop or the epilogue staging, whichever is larger.
template <class Tile, int BM, int BN, bool DEQUANT>
constexpr int tile_lds_bytes() {
    constexpr int epi = epilogue_lds_bytes<BM, BN, DEQUANT>();
    return Tile::kLdsBytes > epi ? Tile::kLdsBytes : epi;
}

// Register-staged engine: any operand type (row-major, conv gather, byte gathers).
template <int BM, int BN, bool EVEN_K, bool DEQUANT, class OpA, class OpB>
__global__ __launch_bounds__(kGemmThreads) void gemm_nt_kernel(
    OpA opa, OpB opb, GemmEpilogue ep, int tiles_m, int tiles_n, int K)
{
    extern __shared__ __align__(16) int8_t lds[];
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    NtTile<BM, BN> t;
    t.template run<EVEN_K>(opa, opb, m0, n0, K, lds);
    store_tile<BM, BN, DEQUANT>(t.acc, ep, m0, n0, lds);
}

// DMA engine: K % 128 == 0, 16-byte aligned; OpA is a row-major matrix or the NHWC im2col
// gather (DmaRowMajor / DmaConv), OpB the row-major weights.
template <int BM, int BN, bool DEQUANT, class OpA = DmaRowMajor>
__global__ __launch_bounds__(kGemmThreads) void gemm_dma_kernel(
    OpA opa, DmaRowMajor opb, GemmEpilogue ep, int tiles_m, int tiles_n, int K)
{
    extern __shared__ __align__(16) int8_t lds[];
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    DmaTile<BM, BN> t;
    t.run(opa, opb, K, m0, n0, lds);
    store_tile<BM, BN, DEQUANT>(t.acc, ep, m0, n0, lds);
}

// The tail split in one launch: workgroups [0, n1) run the 256-row tiles of the first rows
// (opa, ep), the rest the 192-row tiles of the remaining rows (opa2, ep2). Workgroups start in
// index order, so each CU takes a 192-row tile as soon as its 256-row tile ends, while other CUs
// still run their epilogues -- no launch boundary between the two tile sizes.
template <bool DEQUANT, class OpA>
__global__ __launch_bounds__(kGemmThreads) void gemm_dma_tail_kernel(
    OpA opa, OpA opa2, DmaRowMajor opb, GemmEpilogue ep, GemmEpilogue ep2, int n1, int tiles_m1, int tiles_m2,
    int tiles_n, int K)
{
    extern __shared__ __align__(16) int8_t lds[];
    int tm, tn;
    if (static_cast<int>(blockIdx.x) < n1) {
        tile_coords(blockIdx.x, tiles_m1, tiles_n, tm, tn);
        DmaTile<256, 256> t;
        t.run(opa, opb, K, tm * 256, tn * 256, lds);
        store_tile<256, 256, DEQUANT>(t.acc, ep, tm * 256, tn * 256, lds);
    } else {
        tile_coords(blockIdx.x - n1, tiles_m2, tiles_n, tm, tn);
        DmaTile<192, 256> t;
        t.run(opa2, opb, K, tm * 192, tn * 256, lds);
        store_tile<192, 256, DEQUANT>(t.acc, ep2, tm * 192, tn * 256, lds);
    }
}

// Raises a kernel's dynamic-LDS limit once (host-side attribute; safe under graph capture).
template <class Kern>
static int allow_lds(Kern kern, int bytes) {
    if (bytes <= 65536) return FORGE_OK;
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    return e == hipSuccess ? FORGE_OK : static_cast<int>(e);
}

template <int BM, int BN, bool EVEN_K, bool DEQUANT, class OpA, class OpB>
static int launch_tile(const OpA& opa, const OpB& opb, const GemmEpilogue& ep, int M, int N, int K,
                       hipStream_t s)
{
    constexpr int lds = tile_lds_bytes<NtTile<BM, BN>, BM, BN, DEQUANT>();
    const int tiles_m = divup(M, BM), tiles_n = divup(N, BN);
    const long long total = static_cast<long long>(tiles_m) * tiles_n;
    if (total > 0x7FFFFFFFLL) return FORGE_EINVAL;
    auto kern = gemm_nt_kernel<BM, BN, EVEN_K, DEQUANT, OpA, OpB>;
    static const int attr = allow_lds(kern, lds);
    if (attr != FORGE_OK) return attr;
    gemm_nt_kernel<BM, BN, EVEN_K, DEQUANT, OpA, OpB>
        <<<static_cast<unsigned>(total), kGemmThreads, lds, s>>>(opa, opb, ep, tiles_m, tiles_n, K);
    return launch_status();
}

template <int BM, int BN, bool DEQUANT, class OpA>
static int launch_dma(const OpA& opa, const DmaRowMajor& opb, const GemmEpilogue& ep, int M, int N, int K,
                      hipStream_t s)
{
    constexpr int lds = tile_lds_bytes<DmaTile<BM, BN>, BM, BN, DEQUANT>();
    const int tiles_m = divup(M, BM), tiles_n = divup(N, BN);
    const long long total = static_cast<long long>(tiles_m) * tiles_n;
    if (total > 0x7FFFFFFFLL) return FORGE_EINVAL;
    auto kern = gemm_dma_kernel<BM, BN, DEQUANT, OpA>;
    static const int attr = allow_lds(kern, lds);
    if (attr != FORGE_OK) return attr;
    gemm_dma_kernel<BM, BN, DEQUANT, OpA>
        <<<static_cast<unsigned>(total), kGemmThreads, lds, s>>>(opa, opb, ep, tiles_m, tiles_n, K);
    return launch_status();
}


// Tile choice: the largest tile whose grid still covers the chip's CUs; smaller tiles
// trade MFMA efficiency (operand reuse) for parallelism.
enum class TileCfg { k256, k128, k64 };

static TileCfg pick_tile(int M, int N, int cu) {
    const long long t256 = static_cast<long long>(divup(M, 256)) * divup(N, 256);
    const long long t128 = static_cast<long long>(divup(M, 128)) * divup(N, 128);
    // A side of 128 or less would leave half of a 256 tile (two of its four waves) idle.
    if (t256 * 2 >= cu && M > 128 && N > 128) return TileCfg::k256;
    if (t128 * 2 >= cu) return TileCfg::k128;
    return TileCfg::k64;
}

static int cu_count(int* st) {
    const DeviceInfo& d = device_info(st);
    return d.cu_count;
}

// DMA engine with the tile chosen for the grid (256 or 128; smaller grids take the
// register-staged engine): returns -1 when the DMA engine does not apply.
// The rows from m1 on, as an operand of their own (a second launch over them).
static DmaRowMajor rows_from(const DmaRowMajor& a, int m1) {
    return DmaRowMajor{a.p + static_cast<size_t>(m1) * a.K, a.rows - m1, a.K};
}
static DmaConv rows_from(const DmaConv& a, int m1) {
    DmaConv b = a;
    b.r0 += m1;
    return b;
}

// A single column of 256x256 tiles whose last tile wave is under 3/4 full (configs[4]: 392
// tiles on 256 CUs, the second wave 53 % full): the first full waves run as 256-row tiles, the
// remaining rows as one wave of 192-row tiles (3/4 of a tile's work each), 1.75 tile times
// instead of 2 there. Returns -1 when the split does not apply.
template <bool DEQUANT, class OpA>
static int launch_dma_tail_split(const OpA& opa, const DmaRowMajor& opb, const GemmEpilogue& ep, int M, int N, int K,
                                 int cu, hipStream_t s)
{
    const long long tiles = divup(M, 256);
    if (N > 256 || ep.up_w != 0 || tiles <= cu) return -1;
    const long long waves = divupll(tiles, cu);
    const long long last = tiles - (waves - 1) * cu;
    const long long m1 = (waves - 1) * cu * 256;
    if (4 * last >= 3LL * cu || m1 >= M || divup(M - static_cast<int>(m1), 192) > cu) return -1;
    const int M1 = static_cast<int>(m1), M2 = M - M1;
    GemmEpilogue ep1 = ep, ep2 = ep;
    ep1.M = M1;
    ep2.M = M2;
    if (ep.c16) ep2.c16 = ep.c16 + static_cast<size_t>(M1) * N;
    if (ep.c32) ep2.c32 = ep.c32 + static_cast<size_t>(M1) * N;
    if (ep.act_scale) ep2.act_scale = ep.act_scale + M1;
    // 16-byte row stores stay aligned: M1 * N * elem is a multiple of 256 * 16.
    constexpr int l1 = tile_lds_bytes<DmaTile<256, 256>, 256, 256, DEQUANT>();
    constexpr int l2 = tile_lds_bytes<DmaTile<192, 256>, 192, 256, DEQUANT>();
    constexpr int lds = l1 > l2 ? l1 : l2;
    const int tiles_n = divup(N, 256), tiles_m1 = M1 / 256, tiles_m2 = divup(M2, 192);
    const long long n1 = static_cast<long long>(tiles_m1) * tiles_n;
    const long long total = n1 + static_cast<long long>(tiles_m2) * tiles_n;
    if (total > 0x7FFFFFFFLL) return FORGE_EINVAL;
    auto kern = gemm_dma_tail_kernel<DEQUANT, OpA>;
    static const int attr = allow_lds(kern, lds);
    if (attr != FORGE_OK) return attr;
    gemm_dma_tail_kernel<DEQUANT, OpA><<<static_cast<unsigned>(total), kGemmThreads, lds, s>>>(
        opa, rows_from(opa, M1), opb, ep1, ep2, static_cast<int>(n1), tiles_m1, tiles_m2, tiles_n, K);
    return launch_status();
}

// The tail split over weight columns in one launch, for grids of several 256-column tiles
// (configs[2]: 16 x 43 = 688 tiles, 2.69 waves): workgroups [0, n1) run whole waves of 256 x
// 256 tiles over the first nb1 tile columns (every row tile of them), the rest the remaining
// columns as one wave of 192-row tiles (3/4 of a tile's work each, ~0.85 of its time): 2.85
// tile times instead of 3 there. Workgroups start in index order, so each CU takes a 192-row
// tile as soon as its last 256-row tile ends.
template <bool DEQUANT>
__global__ __launch_bounds__(kGemmThreads) void gemm_dma_coltail_kernel(
    DmaRowMajor opa, DmaRowMajor opb, GemmEpilogue ep, int n1, int nb1, int tiles_m, int tiles_m2, int tiles_n,
    int K)
{
    extern __shared__ __align__(16) int8_t lds[];
    int tm, tn;
    const int bid = static_cast<int>(blockIdx.x);
    if (bid < n1) {
        tile_coords(bid, tiles_m, nb1, tm, tn);
        DmaTile<256, 256> t;
        t.run(opa, opb, K, tm * 256, tn * 256, lds);
        store_tile<256, 256, DEQUANT>(t.acc, ep, tm * 256, tn * 256, lds);
    } else {
        tile_coords(bid - n1, tiles_m2, tiles_n - nb1, tm, tn);
        const int n0 = (nb1 + tn) * 256;
        DmaTile<192, 256> t;
        t.run(opa, opb, K, tm * 192, n0, lds);
        store_tile<192, 256, DEQUANT>(t.acc, ep, tm * 192, n0, lds);
    }
}

// Runs the column tail split when the grid is more than one wave, not whole waves, its row
// tiles divide the CU count (so the first columns make whole waves) and the remaining columns'
// 192-row tiles fit one wave. Returns -1 when it does not apply.
template <bool DEQUANT>
static int launch_dma_col_tail(const DmaRowMajor& opa, const DmaRowMajor& opb, const GemmEpilogue& ep, int M, int N,
                               int K, int cu, hipStream_t s)
{
    const int tiles_m = divup(M, 256), tiles_n = divup(N, 256);
    const long long tiles = static_cast<long long>(tiles_m) * tiles_n;
    if (tiles <= cu || tiles % cu == 0 || cu % tiles_m != 0 || M < 192 || ep.up_w != 0) return -1;
    const int nb1 = static_cast<int>(tiles / cu * cu / tiles_m);
    const int tiles_m2 = divup(M, 192);
    if (nb1 >= tiles_n || static_cast<long long>(tiles_n - nb1) * tiles_m2 > cu) return -1;
    const int n1 = nb1 * tiles_m;
    const int total = n1 + (tiles_n - nb1) * tiles_m2;
    constexpr int l1 = tile_lds_bytes<DmaTile<256, 256>, 256, 256, DEQUANT>();
    constexpr int l2 = tile_lds_bytes<DmaTile<192, 256>, 192, 256, DEQUANT>();
    constexpr int lds = l1 > l2 ? l1 : l2;
    auto kern = gemm_dma_coltail_kernel<DEQUANT>;
    static const int attr = allow_lds(kern, lds);
    if (attr != FORGE_OK) return attr;
    gemm_dma_coltail_kernel<DEQUANT><<<static_cast<unsigned>(total), kGemmThreads, lds, s>>>(
        opa, opb, ep, n1, nb1, tiles_m, tiles_m2, tiles_n, K);
    return launch_status();
}

template <class OpA>
static int dispatch_dma(const OpA& opa, const DmaRowMajor& opb, const GemmEpilogue& ep, int M, int N, int K,
                        hipStream_t s)
{
    int st = FORGE_OK;
    const int cu = cu_count(&st);
    if (st != FORGE_OK) return st;
    // Both operands as buffer resources with 32-bit offsets. A row-major A is addressed over
    // M * K bytes; the conv operand over its image, whose size the caller has checked.
    if (static_cast<long long>(opb.rows) * K >= (1LL << 31)) return -1;
    if constexpr (std::is_same<OpA, DmaRowMajor>::value) {
        if (static_cast<long long>(M) * K >= (1LL << 31)) return -1;
    }
    const TileCfg t = pick_tile(M, N, cu);
    const bool out16 = ep.c16 != nullptr;
    if (t == TileCfg::k256) {
        note_route("dma256x256+tail192");
        int r = out16 ? launch_dma_tail_split<true>(opa, opb, ep, M, N, K, cu, s)
                      : launch_dma_tail_split<false>(opa, opb, ep, M, N, K, cu, s);
        if (r != -1) return r;
        if constexpr (std::is_same<OpA, DmaRowMajor>::value) {
            r = out16 ? launch_dma_col_tail<true>(opa, opb, ep, M, N, K, cu, s)
                      : launch_dma_col_tail<false>(opa, opb, ep, M, N, K, cu, s);
            if (r != -1) return r;
        }
        note_route("dma256x256");
        return out16 ? launch_dma<256, 256, true>(opa, opb, ep, M, N, K, s) : launch_dma<256, 256, false>(opa, opb, ep, M, N, K, s);
    }
    if (t == TileCfg::k128) {
        note_route("dma128x128");
        return out16 ? launch_dma<128, 128, true>(opa, opb, ep, M, N, K, s) : launch_dma<128, 128, false>(opa, opb, ep, M, N, K, s);
    }
    return -1;
}

// MAX256: whether the 256 x 256 tile may be used (the byte-gather operands of odd shapes
// would spill registers at that size).
template <bool EVEN_K, bool DEQUANT, bool MAX256 = true, class OpA, class OpB>
static int dispatch_tiles(const OpA& opa, const OpB& opb, const GemmEpilogue& ep, int M, int N, int K,
                          hipStream_t s)
{
    int st = FORGE_OK;
    const int cu = cu_count(&st);
    if (st != FORGE_OK) return st;
    TileCfg t = pick_tile(M, N, cu);
    note_route(t == TileCfg::k256 && MAX256 ? "regstaged256" : t == TileCfg::k64 ? "regstaged64" : "regstaged128");
    if constexpr (MAX256) {
        if (t == TileCfg::k256) return launch_tile<256, 256, EVEN_K, DEQUANT>(opa, opb, ep, M, N, K, s);
    } else {
        if (t == TileCfg::k256) t = TileCfg::k128;
    }
    if (t == TileCfg::k128) return launch_tile<128, 128, EVEN_K, DEQUANT>(opa, opb, ep, M, N, K, s);
    return launch_tile<64, 64, EVEN_K, DEQUANT>(opa, opb, ep, M, N, K, s);
}

template <bool DEQUANT, class OpA, class OpB>
static int dispatch_k(const OpA& opa, const OpB& opb, const GemmEpilogue& ep, int M, int N, int K,
                      bool even_k, hipStream_t s)
{
    if (even_k) return dispatch_tiles<true, DEQUANT>(opa, opb, ep, M, N, K, s);
    return dispatch_tiles<false, DEQUANT>(opa, opb, ep, M, N, K, s);
}

int launch_conv_gemm(const ConvGeom& g, const int8_t* w, const GemmEpilogue& ep, int Co, bool vec,
                     hipStream_t s)
{
    const int M = g.rows, K = g.K;
    if (vec) {
        const int r = launch_conv_window(g, w, ep, Co, s);
        if (r != -1) return r;
    }
    // DMA engine when every 128-deep stage of a patch row is one pixel's contiguous channels
    // (and the image fits one buffer resource, the taps one 32-bit mask).
    const long long img_bytes = static_cast<long long>(g.rows / (g.Ho * g.Wo)) * g.H * g.W * g.C;
    const int taps = g.K / g.C;
    // The stage split st -> (tap, channel run) divides by the magic multipliers, exact while
    // stages * cps < 2^32 (udiv_magic's range).
    if (vec && g.C % kBK == 0 && aligned(w, 16) && img_bytes < (1LL << 31) && taps <= 32 &&
        static_cast<long long>(K / kBK) * (g.C / kBK) < (1LL << 32)) {
        DmaConv a;
        static_cast<ConvGeom&>(a) = g;
        a.x_bytes = static_cast<uint32_t>(img_bytes);
        a.cps = g.C / kBK;
        a.mg_cps = udiv_multiplier(a.cps);
        a.mg_kw = udiv_multiplier(g.kW);
        const int r = dispatch_dma(a, DmaRowMajor{w, Co, K}, ep, M, Co, K, s);
        if (r != -1) return r;
    }
    if (vec) {
        ConvOperand a;
        static_cast<ConvGeom&>(a) = g;
        RowMajorOperand b{w, Co, K};
        const bool even = K % kBK == 0;
        return ep.c16 ? dispatch_k<true>(a, b, ep, M, Co, K, even, s)
                      : dispatch_k<false>(a, b, ep, M, Co, K, even, s);
    }
    ConvBytes a;
    static_cast<ConvGeom&>(a) = g;
    RowMajorBytes b{w, Co, K};
    return ep.c16 ? dispatch_tiles<false, true, false>(a, b, ep, M, Co, K, s)
                  : dispatch_tiles<false, false, false>(a, b, ep, M, Co, K, s);
}

// Whether 16-byte row stores of the output are possible.
static int out_vec(const void* out, int N, int esz) {
    return aligned(out, 16) && (static_cast<long long>(N) * esz) % 16 == 0 ? 1 : 0;
}

int gemm_dense(const int8_t* A, const int8_t* B, const float* act_scale, const uint16_t* w_scale,
               const uint16_t* bias, uint16_t* out16, int32_t* out32, int M, int K, int N,
               hipStream_t s)
{
    const bool vec = (K % 16 == 0) && aligned(A, 16) && aligned(B, 16);
    GemmEpilogue ep{out32, out16, act_scale, w_scale, bias, M, N,
                    out16 ? out_vec(out16, N, 2) : out_vec(out32, N, 4)};
    if (vec && decode_supported(M, K)) {
        note_route("decode");
        return launch_decode(B, nullptr, A, ep, K, false, s);
    }
    if (M <= kSkinnyMaxM && vec) {
        note_route("skinny");
        return launch_gemm_skinny(A, B, ep, M, K, N, s);
    }
    if (vec && M <= kSkinnyTbMaxM) {
        // 16 < M <= 64, narrow N, deep K: the tile engine has too few tiles (M = 64, K = 6144,
        // N = 1536: 29.4 us on 64 x 64 tiles, 11.6 us on token blocks with K split in two).
        int st = FORGE_OK;
        const DeviceInfo& di = device_info(&st);
        if (st != FORGE_OK) return st;
        if (dense_tb_supported(M, K, N, di.cu_count)) {
            note_route("token-block");
            return launch_dense_tb(B, A, ep, K, di.cu_count, s);
        }
    }
    return gemm_tiles(A, B, ep, M, K, N, s);
}

int gemm_tiles(const int8_t* A, const int8_t* B, const GemmEpilogue& ep, int M, int K, int N, hipStream_t s)
{
    const bool vec = (K % 16 == 0) && aligned(A, 16) && aligned(B, 16);
    const bool out16 = ep.c16 != nullptr;
    if (vec && K % kBK == 0) {
        const int r = dispatch_dma(DmaRowMajor{A, M, K}, DmaRowMajor{B, N, K}, ep, M, N, K, s);
        if (r != -1) return r;
    }
    if (vec) {
        RowMajorOperand a{A, M, K}, b{B, N, K};
        const bool even = K % kBK == 0;
        return out16 ? dispatch_k<true>(a, b, ep, M, N, K, even, s) : dispatch_k<false>(a, b, ep, M, N, K, even, s);
    }
    RowMajorBytes a{A, M, K}, b{B, N, K};
    return out16 ? dispatch_tiles<false, true, false>(a, b, ep, M, N, K, s)
                 : dispatch_tiles<false, false, false>(a, b, ep, M, N, K, s);
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
    // Decode shapes: one kernel, the quantize fused into the decode GEMM's prologue (each
    // workgroup quantizes the few token rows itself while its first weight stages stream in).
    if (decode_fq_supported(M, K, false) && aligned(x, 16) && aligned(w, 16) && aligned(scratch_q, 8)) {
        note_route("decode+quantize");
        return launch_decode_fq(x, w, nullptr, w_scale, bias, out, scratch_q, scratch_scale, M, K, N, false, s);
    }
    int st = launch_quantize(x, scratch_q, scratch_scale, M, K, s);
    if (st != FORGE_OK) return st;
    return gemm_dense(scratch_q, w, scratch_scale, w_scale, bias, out, nullptr, M, K, N, s);
}
