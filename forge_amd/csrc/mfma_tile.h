// LDS-staged INT8 MFMA GEMM engines for gfx950 (v_mfma_i32_32x32x32_i8).
//
// One 256-thread workgroup (4 wavefronts in a 2 x 2 grid) computes a BM x BN INT32 tile of
// C = A (rows, K) x B (cols, K)^T with both operands K-contiguous ("NT", the layout of the
// reference's int8 GEMMs: include/forge/gemm/int8_dense.cuh:9-11). Each wavefront owns a
// (BM/2) x (BN/2) sub-tile of 32x32 MFMA blocks whose accumulators stay in registers for
// the whole K loop.
//
// Operand roles: the MFMA computes D[n][m] = sum_k B[n][k] A[m][k] (B rows are the MFMA's
// A operand). Its accumulator layout (lane l, register e = 0..15: row 8*(e/4) + 4*(l/32) +
// e%4, col l%32) then gives every lane FOUR CONSECUTIVE OUTPUT COLUMNS n of one output row
// m per register quad: 8 contiguous bytes of FP16 or 16 of INT32 per store.
//
// Operand K mapping: for each 32-K sub-step, lane l supplies 16 bytes of row l%32 at K
// offset 16*(l/32); both operands use the same (lane, byte) -> k assignment, so every
// INT32 dot product is exact.
//
// Two K-loop engines share that layout and the epilogue:
//
// DmaTile (K % 128 == 0, 16-byte aligned row-major operands; the hot path): 128-byte K
// stages in two LDS slots, filled by gfx950's LDS-DMA loads (buffer_load_dwordx4 ... lds
// through a buffer resource per operand: each lane's 16 bytes land at M0 + 16*lane, no VGPR
// staging, 32-bit offsets, the stage's K offset in the scalar offset). Every row of a stage is one full 128-byte
// cache line read by 8 consecutive lanes; on gfx950 this sustains ~30 B/clk per CU into
// LDS, against ~26 B/clk for 64-byte half-line rows, whatever the number of stages in
// flight. Stage kt+1 streams in while stage kt is multiplied; MFMA fragments are read two
// 32-deep sub-steps ahead of use into 4 register buffers, and the barrier that publishes
// stage kt+1 sits in the middle of stage kt, so the LDS latency never reaches the MFMA
// pipe. Synchronisation is explicit: one s_waitcnt vmcnt(0) lgkmcnt(0) (this wave's DMAs
// landed, its reads of the old slot done) and one s_barrier per stage.
// LDS rows are 8 chunks with the (r ^ (r >> 3)) & 7 swizzle below; the DMA lanes are
// assigned (row, chunk) pairs so that each 1 KB DMA write lands exactly in that layout.
//
// NtTile (any K % 16 == 0 operand, including the implicit-im2col conv gather with zero
// padding, and the byte-gather operands of odd shapes): 128-byte K stages through two LDS
// buffers with one stage of register staging; rows of 8 chunks, swizzle (r ^ (r >> 3)) & 7.
//
// Edges: operand rows beyond the matrix are clamped to its last row (their products land in
// accumulator entries that are never stored); the epilogue masks rows and columns.
#pragma once

#include "common.h"

namespace forge_amd {

constexpr int kGemmThreads = 256;

__device__ __forceinline__ int4 zero4() { return make_int4(0, 0, 0, 0); }

// Compiler-only memory fence: keeps LDS accesses on their side of a barrier, emits nothing.
__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

// s_waitcnt vmcnt(N) only (expcnt and lgkmcnt left unconstrained). gfx9 encodes the 6-bit
// vmcnt as bits [3:0] and [15:14] of the immediate.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt immediate");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// 16-byte global -> LDS DMA (global_load_lds_dwordx4): this lane's 16 bytes at `src` land at
// lds_base + 16 * lane; lds_base must be wave-uniform (it goes to M0). A plain __device__
// function, so the host pass never sees the device-only builtin inside kernel templates.
__device__ __forceinline__ void dma16(const int8_t* src, int8_t* lds_base) {
    __builtin_amdgcn_global_load_lds(src, lds_base, 16, 0, 0);
}

// The same DMA through a buffer resource (buffer_load_dwordx4 ... lds): this lane's 16 bytes
// at byte offset voff + soff of the resource land at lds_base + 16 * lane. The offsets are
// 32-bit (voff per lane, soff wave-uniform), so no 64-bit address is formed per load, and a
// read past the resource's size returns zeros instead of touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, int8_t* lds_base) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_base, 16, voff, soff, 0,
                                             0);
}

// Instruction-scheduling pattern for one MFMA sub-step: NMFMA MFMAs with NDS LDS reads and
// NVM vector-memory (DMA) instructions spread evenly between them, in issue order. Without
// it the scheduler clusters the loads behind the MFMAs.
template <int G, int NG, int NMFMA, int NDS, int NVM>
__device__ __forceinline__ void sched_groups() {
    if constexpr (G < NG) {
        // Group G takes its even share (rounded so the shares sum exactly) of each kind.
        constexpr int mf = NMFMA * (G + 1) / NG - NMFMA * G / NG;
        constexpr int ds = NDS * (G + 1) / NG - NDS * G / NG;
        constexpr int vm = NVM * (G + 1) / NG - NVM * G / NG;
        if constexpr (mf > 0) __builtin_amdgcn_sched_group_barrier(0x008, mf, 0);   // MFMA
        if constexpr (ds > 0) __builtin_amdgcn_sched_group_barrier(0x100, ds, 0);   // LDS read
        if constexpr (vm > 0) __builtin_amdgcn_sched_group_barrier(0x010, vm, 0);   // VMEM
        sched_groups<G + 1, NG, NMFMA, NDS, NVM>();
    }
}

template <int NMFMA, int NDS, int NVM>
__device__ __forceinline__ void sched_interleave() {
    constexpr int kLoads = NDS > NVM ? NDS : NVM;
    constexpr int kGroups = NMFMA < kLoads ? NMFMA : (kLoads > 0 ? kLoads : 1);
    sched_groups<0, kGroups, NMFMA, NDS, NVM>();
}

// Workgroup barrier without the memory fence of __syncthreads (which would also drain the
// LDS DMAs still in flight for later stages).
__device__ __forceinline__ void lds_barrier() {
    compiler_fence();
    __builtin_amdgcn_s_barrier();
    compiler_fence();
}

// ---- operands of the register-staged engine: per-thread row state + 16-byte chunk loads ----

// Row-major (rows, K) int8 matrix; needs K % 16 == 0 and a 16-byte aligned base.
struct RowMajorOperand {
    const int8_t* p;
    int rows;
    int K;
    struct Row { const int8_t* base; };
    __device__ __forceinline__ Row row(int r) const {
        r = r < rows ? r : rows - 1;
        return Row{p + static_cast<size_t>(r) * K};
    }
    // Chunk [k, k+16) of the row; zeros when k >= K (only possible when K % 128 != 0).
    template <bool EVEN_K>
    __device__ __forceinline__ int4 load(const Row& rw, int k) const {
        if constexpr (EVEN_K) {
            return *reinterpret_cast<const int4*>(rw.base + k);
        } else {
            const int4 v = *reinterpret_cast<const int4*>(rw.base + (k < K ? k : K - 16));
            return k < K ? v : zero4();
        }
    }
};

// Row-major (rows, K) int8 matrix of any K and alignment (byte gathers; odd shapes only).
struct RowMajorBytes {
    const int8_t* p;
    int rows;
    int K;
    struct Row { const int8_t* base; };
    __device__ __forceinline__ Row row(int r) const {
        r = r < rows ? r : rows - 1;
        return Row{p + static_cast<size_t>(r) * K};
    }
    template <bool EVEN_K>
    __device__ __forceinline__ int4 load(const Row& rw, int k) const {
        uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t b = (k + i < K) ? static_cast<uint8_t>(rw.base[k + i]) : 0u;
            w[i >> 2] |= b << (8 * (i & 3));
        }
        return make_int4(static_cast<int>(w[0]), static_cast<int>(w[1]), static_cast<int>(w[2]),
                         static_cast<int>(w[3]));
    }
};

// Implicit im2col of an NHWC int8 image: operand row = output pixel (n, ho, wo), k =
// (kh*kW + kw)*C + c.
struct ConvGeom {
    const int8_t* x;
    int rows;   // N * Ho * Wo
    int K;      // kH * kW * C
    int H, W, C, Ho, Wo, kW;
    int padH, padW, strideH, strideW, dilH, dilW;
    int r0 = 0; // operand row r is output pixel r0 + r (a launch over the rows from r0 on)
};

// Needs C % 16 == 0 (a chunk never straddles two taps) and a 16-byte aligned image.
struct ConvOperand : ConvGeom {
    struct Row { const int8_t* img; int hb, wb; };
    __device__ __forceinline__ Row row(int r) const {
        r = r < rows ? r : rows - 1;
        const int wo = r % Wo;
        const int t = r / Wo;
        const int ho = t % Ho;
        const int n = t / Ho;
        return Row{x + static_cast<size_t>(n) * H * W * C, ho * strideH - padH, wo * strideW - padW};
    }
    template <bool EVEN_K>
    __device__ __forceinline__ int4 load(const Row& rw, int k) const {
        const int tap = k / C, c = k - tap * C;
        const int kh = tap / kW, kw = tap - kh * kW;
        const int hi = rw.hb + kh * dilH, wi = rw.wb + kw * dilW;
        const bool ok = (EVEN_K || k < K) && hi >= 0 && hi < H && wi >= 0 && wi < W;
        const size_t off = ok ? (static_cast<size_t>(hi) * W + wi) * C + c : 0;
        const int4 v = *reinterpret_cast<const int4*>(rw.img + off);
        return ok ? v : zero4();
    }
};

// Same geometry, any C and alignment (byte gathers; odd shapes only).
struct ConvBytes : ConvGeom {
    struct Row { const int8_t* img; int hb, wb; };
    __device__ __forceinline__ Row row(int r) const {
        r = r < rows ? r : rows - 1;
        const int wo = r % Wo;
        const int t = r / Wo;
        const int ho = t % Ho;
        const int n = t / Ho;
        return Row{x + static_cast<size_t>(n) * H * W * C, ho * strideH - padH, wo * strideW - padW};
    }
    template <bool EVEN_K>
    __device__ __forceinline__ int4 load(const Row& rw, int k) const {
        uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int kk = k + i;
            const int tap = kk / C, c = kk - tap * C;
            const int kh = tap / kW, kw = tap - kh * kW;
            const int hi = rw.hb + kh * dilH, wi = rw.wb + kw * dilW;
            const bool ok = kk < K && hi >= 0 && hi < H && wi >= 0 && wi < W;
            const uint32_t b = ok ? static_cast<uint8_t>(rw.img[(static_cast<size_t>(hi) * W + wi) * C + c]) : 0u;
            w[i >> 2] |= b << (8 * (i & 3));
        }
        return make_int4(static_cast<int>(w[0]), static_cast<int>(w[1]), static_cast<int>(w[2]),
                         static_cast<int>(w[3]));
    }
};

// ---- register-staged engine (128-byte stages, two LDS buffers) -------------------------

constexpr int kBK = 128;

__device__ __forceinline__ int lds_swz8(int r) { return (r ^ (r >> 3)) & 7; }
__device__ __forceinline__ int lds_off128(int r, int c) { return r * kBK + ((c ^ lds_swz8(r)) << 4); }

// 64-byte LDS rows (4 chunks): chunk c of row r at c ^ (((r >> 1) ^ (r >> 4)) & 3). Measured
// bank-conflict free (SQ_LDS_BANK_CONFLICT = 0) on gfx950 for ds_read_b128 in both matrix-core
// operand orders over 64-byte rows: lane l -> row l % 32, chunk 2h + l / 32 (32x32 SMFMAC) and
// lane l -> row l % 16, chunk l / 16 (16x16 SMFMAC); ((r >> 1) ^ (r >> 3)) & 3 is 2-way there.
__device__ __forceinline__ int lds_swz4(int r) { return ((r >> 1) ^ (r >> 4)) & 3; }
__device__ __forceinline__ int lds_off64(int r, int c) { return r * 64 + ((c ^ lds_swz4(r)) << 4); }

template <int BM, int BN>
struct NtTile {
    static constexpr int kTM = BM / 2 / 32;            // 32x32 blocks per wave along rows (m)
    static constexpr int kTN = BN / 2 / 32;            // ... along cols (n)
    static constexpr int kAPass = BM * (kBK / 16) / kGemmThreads;   // A chunks per thread per stage
    static constexpr int kBPass = BN * (kBK / 16) / kGemmThreads;
    static constexpr int kRowsPerPass = kGemmThreads / (kBK / 16); // 32
    static constexpr int kStageBytes = (BM + BN) * kBK;
    static constexpr int kLdsBytes = 2 * kStageBytes;
    static_assert(kTM >= 1 && kTN >= 1, "wave tile must hold a 32x32 block");
    static_assert(kAPass >= 1 && kBPass >= 1, "stage must split evenly");

    v16i acc[kTN][kTM];   // acc[j][i]: D[n][m] of block (n: 32j.., m: 32i..)

    template <bool EVEN_K, class OpA, class OpB>
    __device__ __forceinline__ void run(const OpA& opa, const OpB& opb, int m0, int n0, int K,
                                        int8_t* lds) {
        const int tid = threadIdx.x;
        const int lane = tid & (kWave - 1);
        const int wave = tid / kWave;
        const int wm = (wave >> 1) * (BM / 2);
        const int wn = (wave & 1) * (BN / 2);
        const int cc = tid & 7;        // chunk column this thread stages
        const int rr = tid >> 3;       // first row this thread stages

#pragma unroll
        for (int j = 0; j < kTN; j++)
#pragma unroll
            for (int i = 0; i < kTM; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) acc[j][i][e] = 0;

        typename OpA::Row ra[kAPass];
        typename OpB::Row rb[kBPass];
#pragma unroll
        for (int i = 0; i < kAPass; i++) ra[i] = opa.row(m0 + rr + kRowsPerPass * i);
#pragma unroll
        for (int i = 0; i < kBPass; i++) rb[i] = opb.row(n0 + rr + kRowsPerPass * i);

        int4 sa[kAPass], sb[kBPass];
        auto gload = [&](int kt) {
            const int k = kt * kBK + 16 * cc;
#pragma unroll
            for (int i = 0; i < kAPass; i++) sa[i] = opa.template load<EVEN_K>(ra[i], k);
#pragma unroll
            for (int i = 0; i < kBPass; i++) sb[i] = opb.template load<EVEN_K>(rb[i], k);
        };
        auto lstore = [&](int buf) {
            int8_t* As = lds + buf * kStageBytes;
            int8_t* Bs = As + BM * kBK;
#pragma unroll
            for (int i = 0; i < kAPass; i++)
                *reinterpret_cast<int4*>(As + lds_off128(rr + kRowsPerPass * i, cc)) = sa[i];
#pragma unroll
            for (int i = 0; i < kBPass; i++)
                *reinterpret_cast<int4*>(Bs + lds_off128(rr + kRowsPerPass * i, cc)) = sb[i];
        };

        const int kt_total = (K + kBK - 1) / kBK;
        gload(0);
        lstore(0);
        if (kt_total > 1) gload(1);
        __syncthreads();
        const int l31 = lane & 31;
        const int hi = lane >> 5;
        for (int kt = 0; kt < kt_total; kt++) {
            const int cur = kt & 1;
            const int8_t* As = lds + cur * kStageBytes;
            const int8_t* Bs = As + BM * kBK;
#pragma unroll
            for (int ks = 0; ks < kBK / 32; ks++) {
                const int c = 2 * ks + hi;
                v4i fa[kTM], fb[kTN];
#pragma unroll
                for (int i = 0; i < kTM; i++)
                    fa[i] = *reinterpret_cast<const v4i*>(As + lds_off128(wm + 32 * i + l31, c));
#pragma unroll
                for (int j = 0; j < kTN; j++)
                    fb[j] = *reinterpret_cast<const v4i*>(Bs + lds_off128(wn + 32 * j + l31, c));
#pragma unroll
                for (int j = 0; j < kTN; j++)
#pragma unroll
                    for (int i = 0; i < kTM; i++)
                        acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fb[j], fa[i], acc[j][i], 0, 0, 0);
            }
            if (kt + 1 < kt_total) {
                lstore(cur ^ 1);
                if (kt + 2 < kt_total) gload(kt + 2);
            }
            __syncthreads();
        }
    }
};

// ---- DMA engine (128-byte stages, 2-slot LDS ring, global_load_lds) ---------------------

// s_waitcnt vmcnt(0) lgkmcnt(0) (expcnt unconstrained).
__device__ __forceinline__ void wait_vm_lgkm0() { __builtin_amdgcn_s_waitcnt(0x7 << 4); }

// DMA operand policies: where lane chunk c (16 bytes) of tile row r comes from at 128-deep
// stage st. lane() runs once per DMA instruction; src() once per stage.

// Row-major (rows, K) matrix, K % 128 == 0; rows past the end are clamped (never stored).
// A row-major INT8 matrix as one buffer resource (rows * K < 2^31, checked by the host): a lane's
// chunk offset is fixed, the stage's K offset is the uniform scalar offset of the buffer load,
// so a stage's DMAs need no per-lane address arithmetic.
struct DmaRowMajor {
    const int8_t* p;
    int rows, K;
    using Lane = uint32_t;
    __device__ __forceinline__ Lane lane(int r, int c) const {
        return static_cast<uint32_t>(r < rows ? r : rows - 1) * static_cast<uint32_t>(K) + 16u * c;
    }
    using Stage = uint32_t;
    __device__ __forceinline__ Stage stage(int st) const { return static_cast<uint32_t>(st) * kBK; }
    __device__ __forceinline__ void dma(const Lane& l, Stage soff, int8_t* dst) const {
        dma16_buf(buf_rsrc(p, static_cast<uint32_t>(rows) * static_cast<uint32_t>(K)), l, soff, dst);
    }
};

// Implicit im2col of an NHWC image, K order (kh, kw, c): with C % 128 == 0 a 128-deep stage of a
// patch row is one contiguous run of one input pixel's channels, or padding. The image is one
// buffer resource (x_bytes < 2^31, set by the host with the magic multipliers), and a stage's
// DMA is a buffer load at a 32-bit offset: the row's pixel offset (fixed per lane) plus the
// stage's tap offset (uniform: (kh dilH W + kw dilW) C + c0). A row keeps a bit per tap saying
// whether that tap lies inside the image; a padding tap gets an offset past the range, which
// the hardware reads as zeros. Needs a 16-byte aligned image and kH kW <= 32.
struct DmaConv : ConvGeom {
    uint32_t x_bytes;            // bytes of the whole NHWC input
    int cps;                     // 128-deep stages per tap (C / 128)
    uint32_t mg_cps, mg_kw;      // udiv_magic multipliers for / cps and / kW
    struct Lane {
        int off;                 // byte offset of pixel (n, hb, wb) + 16 * chunk (may be negative)
        uint32_t taps;           // bit kh kW + kw: tap inside the image
    };
    __device__ __forceinline__ Lane lane(int r, int c) const {
        r += r0;
        r = r < rows ? r : rows - 1;
        const int wo = r % Wo;
        const int t = r / Wo;
        const int ho = t % Ho;
        const int n = t / Ho;
        const int hb = ho * strideH - padH, wb = wo * strideW - padW;
        const int kH = K / (C * kW);
        uint32_t taps = 0u;
        for (int kh = 0; kh < kH; kh++)
            for (int kw = 0; kw < kW; kw++) {
                const int hi = hb + kh * dilH, wi = wb + kw * dilW;
                if (hi >= 0 && hi < H && wi >= 0 && wi < W) taps |= 1u << (kh * kW + kw);
            }
        return Lane{((n * H + hb) * W + wb) * C + 16 * c, taps};
    }
    struct Stage {
        int soff;                // (kh dilH W + kw dilW) C + c0
        int tap;                 // kh kW + kw
    };
    __device__ __forceinline__ Stage stage(int st) const {
        const int tap = udiv_magic(st, mg_cps), c0 = (st - tap * cps) * kBK;
        const int kh = udiv_magic(tap, mg_kw), kw = tap - kh * kW;
        return Stage{(kh * dilH * W + kw * dilW) * C + c0, tap};
    }
    __device__ __forceinline__ void dma(const Lane& l, const Stage& S, int8_t* dst) const {
        const uint32_t voff = (l.taps >> S.tap) & 1u ? static_cast<uint32_t>(l.off + S.soff) : 0x80000000u;
        dma16_buf(buf_rsrc(x, x_bytes), voff, 0, dst);
    }
};

template <int BM, int BN>
struct DmaTile {
    static constexpr int kTM = BM / 2 / 32;
    static constexpr int kTN = BN / 2 / 32;
    static constexpr int kAIns = BM * (kBK / 16) / kWave / 4;   // 1 KB DMA instructions per wave per stage
    static constexpr int kBIns = BN * (kBK / 16) / kWave / 4;
    static constexpr int kSlotBytes = (BM + BN) * kBK;
    static constexpr int kLdsBytes = 2 * kSlotBytes;
    static_assert(kTM >= 1 && kTN >= 1 && kAIns >= 1 && kBIns >= 1, "tile too small");

    // MFMA operand fragments of one 32-deep sub-step.
    struct Frags {
        v4i a[kTM];
        v4i b[kTN];
    };

    v16i acc[kTN][kTM];

    template <class OpA, class OpB>
    __device__ __forceinline__ void run(const OpA& opa, const OpB& opb, int K, int m0, int n0, int8_t* lds) {
        const int lane = threadIdx.x & (kWave - 1);
        const int wave = threadIdx.x / kWave;
        const int wm = (wave >> 1) * (BM / 2);
        const int wn = (wave & 1) * (BN / 2);
        const int l31 = lane & 31;
        const int hi = lane >> 5;

#pragma unroll
        for (int j = 0; j < kTN; j++)
#pragma unroll
            for (int i = 0; i < kTM; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) acc[j][i][e] = 0;

        // DMA instruction q of this wave fills slot chunks s = (wave*kIns + q)*64 + lane:
        // row s/8 (8 lanes read one 128-byte line), physical chunk s%8 = logical chunk
        // (s%8) ^ swz(row) of that row.
        typename OpA::Lane la[kAIns];
        typename OpB::Lane lb[kBIns];
#pragma unroll
        for (int q = 0; q < kAIns; q++) {
            const int s = (wave * kAIns + q) * kWave + lane;
            const int r = s >> 3, c = (s & 7) ^ lds_swz8(r);
            la[q] = opa.lane(m0 + r, c);
        }
#pragma unroll
        for (int q = 0; q < kBIns; q++) {
            const int s = (wave * kBIns + q) * kWave + lane;
            const int r = s >> 3, c = (s & 7) ^ lds_swz8(r);
            lb[q] = opb.lane(n0 + r, c);
        }
        const int nst = K / kBK;
        // Stage st into slot st % 2; stages past the end re-read the last one (their slot is
        // never read again), so the issue needs no branch.
        auto issue = [&](int st) {
            int8_t* slot = lds + (st & 1) * kSlotBytes;
            const int sc = st < nst ? st : nst - 1;
            const typename OpA::Stage sa = opa.stage(sc);
            const typename OpB::Stage sb = opb.stage(sc);
#pragma unroll
            for (int q = 0; q < kAIns; q++) opa.dma(la[q], sa, slot + (wave * kAIns + q) * 1024);
#pragma unroll
            for (int q = 0; q < kBIns; q++) opb.dma(lb[q], sb, slot + BM * kBK + (wave * kBIns + q) * 1024);
        };
        auto load_frags = [&](int st, int ks, Frags& F) {
            const int8_t* As = lds + (st & 1) * kSlotBytes;
            const int8_t* Bs = As + BM * kBK;
            const int c = 2 * ks + hi;
#pragma unroll
            for (int i = 0; i < kTM; i++)
                F.a[i] = *reinterpret_cast<const v4i*>(As + lds_off128(wm + 32 * i + l31, c));
#pragma unroll
            for (int j = 0; j < kTN; j++)
                F.b[j] = *reinterpret_cast<const v4i*>(Bs + lds_off128(wn + 32 * j + l31, c));
        };
        auto mfmas = [&](const Frags& F) {
#pragma unroll
            for (int j = 0; j < kTN; j++)
#pragma unroll
                for (int i = 0; i < kTM; i++)
                    acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(F.b[j], F.a[i], acc[j][i], 0, 0, 0);
        };
        // Fragments are read two 32-deep sub-steps ahead of their MFMAs (4 register buffers,
        // one rotation per stage), the reads and DMAs spread between the MFMAs (the scheduler
        // would otherwise cluster them and expose the LDS latency). The barrier that
        // publishes stage kt+1 sits after sub-step 1 of stage kt, once all of stage kt's
        // reads are done, so sub-steps 2-3 can already read stage kt+1 and refill stage kt's
        // slot with stage kt+2.
        constexpr int kMf = kTM * kTN, kRd = kTM + kTN, kVm = (kAIns + kBIns) / 2;
        Frags F0, F1, F2, F3;
        issue(0);
        wait_vm_lgkm0();
        lds_barrier();
        issue(1);
        load_frags(0, 0, F0);
        load_frags(0, 1, F1);
        for (int kt = 0; kt + 1 < nst; kt++) {
            load_frags(kt, 2, F2);
            mfmas(F0);
            sched_interleave<kMf, kRd, 0>();
            load_frags(kt, 3, F3);
            mfmas(F1);
            sched_interleave<kMf, kRd, 0>();
            // Stage kt+1 landed (own DMAs) and this wave's reads of stage kt are complete.
            wait_vm_lgkm0();
            lds_barrier();
            issue(kt + 2);                         // into stage kt's slot
            load_frags(kt + 1, 0, F0);
            mfmas(F2);
            load_frags(kt + 1, 1, F1);
            mfmas(F3);
            // The DMAs first (spread over sub-step 2), then the reads (over sub-step 3): a
            // global_load_lds also matches the LDS-read group, so the two are not mixed.
            sched_interleave<kMf, 0, 2 * kVm>();
            sched_interleave<kMf, 2 * kRd, 0>();
        }
        load_frags(nst - 1, 2, F2);
        mfmas(F0);
        load_frags(nst - 1, 3, F3);
        mfmas(F1);
        mfmas(F2);
        mfmas(F3);
        // Every wave is done with the ring (and no DMA is in flight) before the epilogue.
        wait_vm_lgkm0();
        lds_barrier();
    }
};

// ---- shared epilogue -------------------------------------------------------------------

// Output of a GEMM: exactly one of c32 (INT32) or c16 (dequantized FP16) is non-null.
struct GemmEpilogue {
    int32_t* c32;
    uint16_t* c16;
    const float* act_scale;     // (M,)  FP16 mode only
    const uint16_t* w_scale;    // (N,), or (N/4,) in the upsample scatter
    const uint16_t* bias;       // (N,) or nullptr
    int M, N;
    int vec_out;                // 16-byte row stores allowed (N * elem % 16 == 0, base aligned);
                                // in the upsample scatter: W % 4 == 0 and c16 16-byte aligned
    // ConvTranspose2d kernel-2 stride-2 scatter (FP16 only; up_w == 0 = plain (M, N) rows):
    // row m is pixel (img, h, w) of img * up_hw + h * up_w + w, column n = co*4 + kh*2 + kw,
    // and the value goes to c16[img][co][2h + kh][2w + kw] (NCHW, (2H) x (2W) planes). The
    // scale is w_scale[co]; the GEMM value is rounded to FP16, then post_bias[co] (if any) is
    // added in fp32 and rounded again (src/nn/int8_conv_transpose2d.cu:70-102, 174-189).
    int up_w, up_hw;
    const uint16_t* post_bias;
};

// Copies kRows x kU 16-byte units of a wave-private staging area (rows of kRowBytes, unit u
// of row r at slot u ^ (r % kU)) to the output with coalesced 16-byte row stores. The units
// go in batches of kB per lane: all kB LDS reads are issued before the first store, so the
// LDS latency is paid once per batch rather than once per unit (a loop of read -> wait ->
// store left the epilogue latency-bound). NT: non-temporal stores, used for both output
// types (measured: INT32 4096^2 2.5 us faster; FP16 4096^2 0.8 us and M = 129,600 x 128,
// K = 64 2 us faster than cached stores).
template <int kU, int kEsz, bool DEQUANT, bool NT = false, int kRows>
__device__ __forceinline__ void flush_rows(const int8_t* stage, const GemmEpilogue& ep, int row0, int col0) {
    constexpr int kPer = 16 / kEsz;
    constexpr int kRowBytes = kU * 16;
    constexpr int kUnits = kRows * kU;
    static_assert(kUnits % kWave == 0, "staged units must fill whole wave passes");
    constexpr int kIters = kUnits / kWave;
    constexpr int kB = kIters < 8 ? kIters : 8;
    static_assert(kIters % kB == 0, "batch must divide the passes");
    const int lane = threadIdx.x & (kWave - 1);
    const int M = ep.M, N = ep.N;
#pragma unroll 1
    for (int it = 0; it < kIters; it += kB) {
        int4 v[kB];
#pragma unroll
        for (int b = 0; b < kB; b++) {
            const int idx = lane + (it + b) * kWave;
            const int r = idx / kU, u = idx % kU;
            v[b] = *reinterpret_cast<const int4*>(stage + r * kRowBytes + ((u ^ (r & (kU - 1))) << 4));
        }
#pragma unroll
        for (int b = 0; b < kB; b++) {
            const int idx = lane + (it + b) * kWave;
            const int r = idx / kU, u = idx % kU;
            const int row = row0 + r;
            const int col = col0 + u * kPer;
            if (row >= M || col >= N) continue;
            const size_t o = static_cast<size_t>(row) * N + col;
            if (ep.vec_out && col + kPer <= N) {
                if constexpr (NT) {
                    const v4i w = v4i{v[b].x, v[b].y, v[b].z, v[b].w};
                    if constexpr (DEQUANT) __builtin_nontemporal_store(w, reinterpret_cast<v4i*>(ep.c16 + o));
                    else __builtin_nontemporal_store(w, reinterpret_cast<v4i*>(ep.c32 + o));
                } else {
                    if constexpr (DEQUANT) *reinterpret_cast<int4*>(ep.c16 + o) = v[b];
                    else *reinterpret_cast<int4*>(ep.c32 + o) = v[b];
                }
            } else {
                // Ragged or unaligned rows: element stores (constant register indices).
                const int n_ok = N - col;
                const uint32_t w[4] = {static_cast<uint32_t>(v[b].x), static_cast<uint32_t>(v[b].y),
                                       static_cast<uint32_t>(v[b].z), static_cast<uint32_t>(v[b].w)};
#pragma unroll
                for (int t = 0; t < kPer; t++) {
                    if (t >= n_ok) break;
                    if constexpr (DEQUANT)
                        ep.c16[o + t] = static_cast<uint16_t>(w[t >> 1] >> (16 * (t & 1)));
                    else
                        ep.c32[o + t] = static_cast<int32_t>(w[t]);
                }
            }
        }
    }
}

// Adds an fp16 bias to both halves of a packed pair, each in fp32 and rounded again.
__device__ __forceinline__ uint32_t add_bias_pair(uint32_t d, float b) {
    const uint32_t lo = f2h(h2f(static_cast<uint16_t>(d & 0xFFFFu)) + b);
    const uint32_t hi = f2h(h2f(static_cast<uint16_t>(d >> 16)) + b);
    return lo | (hi << 16);
}

// The upsample scatter of a wave's staged FP16 tile (kRows pixels x kU*8 columns, same
// staging layout as flush_rows). Column pair (co, kh) with kw = 0, 1 is one 4-byte LDS word,
// and the two kw values of a pixel are adjacent in the output row 2h + kh. vec_out: groups
// of 4 pixels (one image row, since W % 4 == 0) become one 16-byte store of 8 halves, and
// each lane keeps one group across its loop, so the pixel coordinates are computed once.
// pbias: the wave's LDS strip of post_bias[co] per wave-local column.
template <int kU, int kRows>
__device__ __forceinline__ void flush_up2x2(const int8_t* stage, const uint16_t* pbias, const GemmEpilogue& ep,
                                            int row0, int col0) {
    constexpr int kRowBytes = kU * 16;
    constexpr int kPairs = kU * 4;                   // (co, kh) column pairs in the wave tile
    const int lane = threadIdx.x & (kWave - 1);
    const int M = ep.M, N = ep.N, W = ep.up_w, HW = ep.up_hw;
    const int Co = N >> 2;
    const size_t plane = 4 * static_cast<size_t>(HW);
    const size_t W2 = 2 * static_cast<size_t>(W);
    const bool has_bias = ep.post_bias != nullptr;
    auto word = [&](int r, int cw) {
        return *reinterpret_cast<const uint32_t*>(stage + r * kRowBytes + (((cw >> 3) ^ (r & (kU - 1))) << 4) +
                                                  (cw & 7) * 2);
    };
    if (ep.vec_out) {
        constexpr int kQuads = kRows / 4;
        static_assert(kWave % kQuads == 0, "quads per wave tile must divide the wave");
        const int g = lane % kQuads;
        const int m = row0 + 4 * g;
        if (m >= M) return;                          // M % 4 == 0: a group is all in or all out
        const int img = m / HW, p = m - img * HW, h = p / W, w = p - h * W;
        uint16_t* base = ep.c16 + static_cast<size_t>(img) * Co * plane + 2 * h * W2 + 2 * w;
        // Column pairs j = lane / kQuads + k * (kWave / kQuads), in batches of kB whose LDS
        // words are all read before the first store.
        constexpr int kStep = kWave / kQuads, kIters = kPairs / kStep;
        constexpr int kB = kIters < 4 ? kIters : 4;
        static_assert(kPairs % kStep == 0 && kIters % kB == 0, "pairs must split evenly");
#pragma unroll 1
        for (int k0 = 0; k0 < kIters; k0 += kB) {
            uint32_t d[kB][4];
#pragma unroll
            for (int b = 0; b < kB; b++) {
                const int cw = 2 * (lane / kQuads + (k0 + b) * kStep);
#pragma unroll
                for (int t = 0; t < 4; t++) d[b][t] = word(4 * g + t, cw);
            }
#pragma unroll
            for (int b = 0; b < kB; b++) {
                const int cw = 2 * (lane / kQuads + (k0 + b) * kStep), n = col0 + cw;
                if (n >= N) continue;
                const int co = n >> 2, kh = (n >> 1) & 1;
                if (has_bias) {
                    const float bf = h2f(pbias[cw]);
#pragma unroll
                    for (int t = 0; t < 4; t++) d[b][t] = add_bias_pair(d[b][t], bf);
                }
                __builtin_nontemporal_store(v4i{static_cast<int>(d[b][0]), static_cast<int>(d[b][1]),
                                                static_cast<int>(d[b][2]), static_cast<int>(d[b][3])},
                                            reinterpret_cast<v4i*>(base + co * plane + kh * W2));
            }
        }
    } else {
        for (int r = lane; r < kRows; r += kWave) {
            const int m = row0 + r;
            if (m >= M) break;
            const int img = m / HW, p = m - img * HW, h = p / W, w = p - h * W;
            uint16_t* base = ep.c16 + static_cast<size_t>(img) * Co * plane + 2 * h * W2 + 2 * w;
            for (int j = 0; j < kPairs; j++) {
                const int cw = 2 * j, n = col0 + cw;
                if (n >= N) break;
                const int co = n >> 2, kh = (n >> 1) & 1;
                uint32_t d = word(r, cw);
                if (has_bias) d = add_bias_pair(d, h2f(pbias[cw]));
                uint16_t* o = base + co * plane + kh * W2;
                o[0] = static_cast<uint16_t>(d & 0xFFFFu);
                o[1] = static_cast<uint16_t>(d >> 16);
            }
        }
    }
}

// LDS bytes the epilogue needs: FP16 stages the whole wave tile, INT32 one 32-row strip.
template <int BM, int BN, bool DEQUANT>
constexpr int epilogue_lds_bytes() {
    // FP16: 4 wave tiles, then each wave's w_scale and bias strips (BN/2 halves each).
    return DEQUANT ? BM * BN * 2 + 4 * BN * 2 : 4 * 32 * (BN / 2) * 4;
}

// Writes the wave's (BM/2) x (BN/2) tile through a wave-private LDS staging area: each lane
// deposits its 4-column groups (8 bytes FP16 / 16 bytes INT32), then the wave reads back
// 16-byte row chunks for coalesced stores. FP16: the whole tile at once, loops ordered so
// only 4 columns' w_scale/bias are live at a time. INT32: one 32-row strip at a time.
// The caller's K loop must be finished with the LDS.
template <int BM, int BN, bool DEQUANT>
__device__ __forceinline__ void store_tile(const v16i (&acc)[BN / 64][BM / 64], const GemmEpilogue& ep,
                                           int m0, int n0, int8_t* lds) {
    constexpr int kTM = BM / 64, kTN = BN / 64;
    constexpr int kEsz = DEQUANT ? 2 : 4;
    constexpr int kCols = BN / 2;
    constexpr int kU = kCols * kEsz / 16;            // 16-byte units per staged row
    constexpr int kPer = 16 / kEsz;                  // elements per unit
    constexpr int kRowBytes = kCols * kEsz;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int wm = m0 + (wave >> 1) * (BM / 2);
    const int wn = n0 + (wave & 1) * (BN / 2);
    const int l31 = lane & 31, hi = lane >> 5;
    const int M = ep.M, N = ep.N;

    if constexpr (DEQUANT) {
        int8_t* stage = lds + wave * ((BM / 2) * kRowBytes);
        float as[kTM];
#pragma unroll
        for (int i = 0; i < kTM; i++) {
            const int m = wm + 32 * i + l31;
            as[i] = ep.act_scale[m < M ? m : M - 1];
        }
        const bool has_bias = ep.bias != nullptr;
        // The w_scale / bias halves of the wave's BN/2 columns are staged in a wave-private LDS
        // strip first (one or two coalesced loads per lane, all in flight together), then read
        // 4 columns at a time. Loading them per column group inside the loop below cost one
        // memory latency per group (the FP16 epilogue of a K = 64 GEMM ran at a third of the
        // INT32 one's rate); prefetching them into registers spilled the 256 x 256 tile.
        // Without a bias the bias strip holds w_scale (in range, and ignored by dequant_gemm),
        // so no load sits behind a branch; the upsample scatter has one scale per 4 columns.
        uint16_t* wsl = reinterpret_cast<uint16_t*>(lds + BM * BN * 2) + wave * BN;
        uint16_t* bl = wsl + BN / 2;
        const uint16_t* bsrc = has_bias ? ep.bias : ep.w_scale;
        {
            constexpr int kIt = (BN / 2 + kWave - 1) / kWave;
            uint16_t wv[kIt], bw[kIt];
            // The upsample scatter's bias strip holds post_bias[co] per column instead (its
            // GEMM value has no bias); without a post_bias it reads w_scale (ignored).
            const uint16_t* psrc = ep.post_bias ? ep.post_bias : ep.w_scale;
#pragma unroll
            for (int k = 0; k < kIt; k++) {
                const int n = min(wn + lane + kWave * k, N - 1);
                wv[k] = ep.w_scale[ep.up_w ? n >> 2 : n];
                bw[k] = ep.up_w ? psrc[n >> 2] : bsrc[n];
            }
#pragma unroll
            for (int k = 0; k < kIt; k++) {
                const int c = lane + kWave * k;
                if (c < BN / 2) {
                    wsl[c] = wv[k];
                    bl[c] = bw[k];
                }
            }
        }
#pragma unroll
        for (int j = 0; j < kTN; j++) {
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int nl = 32 * j + 8 * g + 4 * hi;     // first of this lane's 4 columns
                const uint2 w2 = *reinterpret_cast<const uint2*>(wsl + nl);
                const uint2 b2 = *reinterpret_cast<const uint2*>(bl + nl);
                const uint32_t wr[4] = {w2.x & 0xFFFFu, w2.x >> 16, w2.y & 0xFFFFu, w2.y >> 16};
                const uint32_t br[4] = {b2.x & 0xFFFFu, b2.x >> 16, b2.y & 0xFFFFu, b2.y >> 16};
                // dequant4_pk: b = -0 without a bias
                float ws[4], b[4];
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    ws[t] = h2f(static_cast<uint16_t>(wr[t]));
                    b[t] = has_bias ? h2f(static_cast<uint16_t>(br[t])) : -0.0f;
                }
                const int u = nl / kPer;                   // unit of 8 columns; half = hi
#pragma unroll
                for (int i = 0; i < kTM; i++) {
                    const int r = 32 * i + l31;
                    *reinterpret_cast<uint2*>(stage + r * kRowBytes + ((u ^ (r & (kU - 1))) << 4) + 8 * hi) =
                        dequant4_pk(acc[j][i][4 * g], acc[j][i][4 * g + 1], acc[j][i][4 * g + 2], acc[j][i][4 * g + 3],
                                    as[i], ws, b);
                }
            }
        }
        // The upsample scatter (4-pixel groups across the wave) exists for tile heights whose
        // wave tile splits into such groups; other heights never take it (the caller checks).
        if constexpr (kWave % ((BM / 2) / 4) == 0) {
            if (ep.up_w) flush_up2x2<kU, BM / 2>(stage, bl, ep, wm, wn);
            else flush_rows<kU, kEsz, true, true, BM / 2>(stage, ep, wm, wn);
        } else {
            flush_rows<kU, kEsz, true, true, BM / 2>(stage, ep, wm, wn);
        }
    } else {
        int8_t* strip = lds + wave * (32 * kRowBytes);
#pragma unroll
        for (int i = 0; i < kTM; i++) {
#pragma unroll
            for (int j = 0; j < kTN; j++) {
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const int u = (32 * j + 8 * g + 4 * hi) / kPer;   // unit of 4 columns
                    *reinterpret_cast<int4*>(strip + l31 * kRowBytes + ((u ^ (l31 & (kU - 1))) << 4)) =
                        make_int4(acc[j][i][4 * g], acc[j][i][4 * g + 1], acc[j][i][4 * g + 2], acc[j][i][4 * g + 3]);
                }
            }
            flush_rows<kU, kEsz, false, true, 32>(strip, ep, wm + 32 * i, wn);
        }
    }
}

// Tile index -> (tile_m, tile_n): consecutive workgroups land on different XCDs
// (dispatch is round-robin over the 8 XCDs), so the linear id is first regrouped so each
// XCD receives a contiguous run (xcd_contiguous, a bijection for any tile count; a tail
// grid whose first id is not a multiple of 8 shifts which XCD gets which run, not the
// grouping), then runs are rasterised in groups of kGroupM tile-rows: an XCD's L2 then
// holds a few A row-blocks and B col-blocks instead of all of them.
__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
    constexpr int kGroupM = 4;
    const int total = tiles_m * tiles_n;
    const int t = xcd_contiguous(bid, total);
    const int per_group = kGroupM * tiles_n;
    const int group = t / per_group;
    const int first_m = group * kGroupM;
    const int gm = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
    const int r = t - group * per_group;
    tm = first_m + r % gm;
    tn = r / gm;
}

}  // namespace forge_amd
