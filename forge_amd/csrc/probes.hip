// Measurement probes (libforge_probes.so, not part of libforge_amd.so): the microbenchmarks
// behind the ceilings the design rests on, run by `bench.py --probes` and, one at a time, by
// `bench.py --probe NAME` under rocprofv3 --pmc.
//
//   probe_mfma_lds: the dense 256 x 256 engine's inner loop (4 waves, 4 x 4 blocks of
//     v_mfma_i32_32x32x32_i8 per wave, fragments read from LDS in the engine's swizzled layout)
//     on one 64 KB stage loaded once, so no DMA runs: with random operands it shows the
//     sustained clock and MFMA rate under the matrix cores' own power draw. reads = 0 keeps the
//     fragments in registers (MFMA only).
//   probe_stream: a plain streaming read (16-byte non-temporal loads, 8 in flight per lane),
//     the ceiling of a weight-streaming decode GEMM.
//   probe_dma: 32 KB stages of rows streamed into a 2-slot LDS ring with buffer_load ... lds (the
//     GEMM engines' DMA), one barrier per stage; `share` workgroups of an XCD read the same rows
//     (L2 reuse), `half` streams 64-byte rows instead of 128-byte lines, `ldsr` adds the engines'
//     ratio of LDS reads (two bytes read per byte written).
#include "common.h"
#include "mfma_tile.h"

namespace forge_amd {
namespace {

template <bool READS>
__global__ __launch_bounds__(256) void probe_mfma_lds_kernel(const int8_t* __restrict__ A, const int8_t* __restrict__ B,
                                                             int* __restrict__ out, int nst, int tiles_a)
{
    extern __shared__ __align__(16) int8_t lds[];
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int wm = (wave >> 1) * 128, wn = (wave & 1) * 128;
    const int l31 = lane & 31, hi = lane >> 5;
    // one stage: A rows (tile-local 0..255) then B rows, 128 bytes each, chunk swizzle of DmaTile
    const int8_t* a = A + static_cast<size_t>(blockIdx.x % tiles_a) * 256 * 128;
    const int8_t* b = B + static_cast<size_t>(blockIdx.x % tiles_a) * 256 * 128;
    for (int s = threadIdx.x; s < 2 * 256 * 8; s += 256) {
        const int r = (s >> 3) & 255, c = s & 7, isb = s >> 11;
        const int4 v = *reinterpret_cast<const int4*>((isb ? b : a) + r * 128 + c * 16);
        *reinterpret_cast<int4*>(lds + isb * 256 * 128 + lds_off128(r, c)) = v;
    }
    __syncthreads();
    v16i acc[4][4];
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[j][i][e] = 0;
    v4i fa[4][4], fb[4][4];   // [ks][block]
    auto read = [&](int ks) {
        const int c = 2 * ks + hi;
#pragma unroll
        for (int i = 0; i < 4; i++) fa[ks][i] = *reinterpret_cast<const v4i*>(lds + lds_off128(wm + 32 * i + l31, c));
#pragma unroll
        for (int j = 0; j < 4; j++)
            fb[ks][j] = *reinterpret_cast<const v4i*>(lds + 256 * 128 + lds_off128(wn + 32 * j + l31, c));
    };
    if constexpr (!READS) {
#pragma unroll
        for (int ks = 0; ks < 4; ks++) read(ks);
    }
    for (int st = 0; st < nst; st++) {
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            if constexpr (READS) read(ks);
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fb[ks][j], fa[ks][i], acc[j][i], 0, 0, 0);
        }
        if constexpr (READS) {
            // keep the next stage's reads after this stage's MFMAs (as in the engine's loop)
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    int x = 0;
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int e = 0; e < 16; e++) x ^= acc[j][i][e];
    if (x == 0x12345678) out[blockIdx.x] = x;   // keeps the MFMAs live; practically never stored
}

__global__ __launch_bounds__(256) void probe_stream_kernel(const v4i* __restrict__ p, size_t n_per_wg, int* __restrict__ out)
{
    const v4i* base = p + blockIdx.x * n_per_wg;
    v4i acc = {0, 0, 0, 0};
    constexpr int U = 8;
    for (size_t i = threadIdx.x; i < n_per_wg; i += 256 * U) {
        v4i v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            size_t j = i + u * 256;
            j = j < n_per_wg ? j : n_per_wg - 1;
            v[u] = __builtin_nontemporal_load(base + j);
        }
#pragma unroll
        for (int u = 0; u < U; u++) acc += v[u];
    }
    const int s = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    if (s == 0x12345678) out[blockIdx.x] = s;
}

template <bool HALF, bool LDSR>
__global__ __launch_bounds__(256) void probe_dma_kernel(const int8_t* __restrict__ src, uint32_t bytes, int K, int share,
                                                        int* __restrict__ out)
{
    extern __shared__ __align__(16) int8_t lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int xcd = blockIdx.x % 8, member = blockIdx.x / 8;
    const int grp = xcd * (32 / share) + member / share;   // distinct row group
    constexpr int kRows = HALF ? 512 : 256, kRowB = HALF ? 64 : 128, kCh = kRowB / 16;
    const __amdgpu_buffer_rsrc_t r = buf_rsrc(src, bytes);
    uint32_t off[8];
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const int s = (wave * 8 + q) * 64 + lane;
        off[q] = static_cast<uint32_t>(grp * kRows + s / kCh) * static_cast<uint32_t>(K) + 16u * (s % kCh);
    }
    const int nst = K / kRowB;
    auto issue = [&](int st) {
        int8_t* slot = lds + (st & 1) * 32768;
        const int sc = st < nst ? st : nst - 1;
#pragma unroll
        for (int q = 0; q < 8; q++) dma16_buf(r, off[q], static_cast<uint32_t>(sc * kRowB), slot + (wave * 8 + q) * 1024);
    };
    issue(0);
    int acc = 0;
    for (int st = 0; st < nst; st++) {
        issue(st + 1);
        wait_vmcnt<8>();   // stage st landed; st + 1 may stay in flight
        __builtin_amdgcn_s_barrier();
        if constexpr (LDSR) {
            v4i a = {0, 0, 0, 0};
#pragma unroll
            for (int q = 0; q < 16; q++)
                a ^= *reinterpret_cast<const v4i*>(lds + (st & 1) * 32768 + ((q * 64 + lane) * 16 + wave * 4096) % 32768);
            acc ^= a[0] ^ a[1] ^ a[2] ^ a[3];
        } else {
            acc ^= *reinterpret_cast<const int*>(lds + (st & 1) * 32768 + threadIdx.x * 16);
        }
        __builtin_amdgcn_s_barrier();
    }
    wait_vmcnt<0>();
    if (acc == 0x12345678) out[blockIdx.x] = acc;
}

}  // namespace
}  // namespace forge_amd

using namespace forge_amd;

// A, B: tiles_a x (256 x 128) int8 each; grid of `wgs` workgroups, nst stages each.
extern "C" int probe_mfma_lds(const int8_t* A, const int8_t* B, int* out, int wgs, int nst, int tiles_a, int reads,
                              void* stream)
{
    if (!A || !B || !out || wgs <= 0 || nst <= 0 || tiles_a <= 0) return FORGE_EINVAL;
    constexpr int lds = 2 * 256 * 128;
    hipStream_t s = as_stream(stream);
    if (reads) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&probe_mfma_lds_kernel<true>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        probe_mfma_lds_kernel<true><<<wgs, 256, lds, s>>>(A, B, out, nst, tiles_a);
    } else {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&probe_mfma_lds_kernel<false>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        probe_mfma_lds_kernel<false><<<wgs, 256, lds, s>>>(A, B, out, nst, tiles_a);
    }
    return launch_status();
}

// Reads `bytes` (a multiple of 16 * wgs) once with wgs workgroups, each a contiguous chunk.
extern "C" int probe_stream(const void* buf, size_t bytes, int wgs, int* out, void* stream)
{
    if (!buf || !out || wgs <= 0 || bytes % (16 * static_cast<size_t>(wgs)) != 0) return FORGE_EINVAL;
    probe_stream_kernel<<<wgs, 256, 0, as_stream(stream)>>>(static_cast<const v4i*>(buf), bytes / 16 / wgs, out);
    return launch_status();
}

// 256 workgroups (one per CU); src holds 256 * (half ? 512 : 256) rows of K bytes (bytes < 2^31).
extern "C" int probe_dma(const void* src, uint32_t bytes, int K, int share, int half, int ldsr, int* out, void* stream)
{
    if (!src || !out || (share != 1 && share != 2 && share != 4 && share != 8 && share != 16 && share != 32) ||
        K % 128 != 0 || static_cast<uint64_t>(256) * (half ? 512 : 256) * static_cast<uint64_t>(K) > bytes ||
        bytes >= (1u << 31))
        return FORGE_EINVAL;
    constexpr int lds = 2 * 32768;
    hipStream_t s = as_stream(stream);
    const int8_t* p = static_cast<const int8_t*>(src);
#define FORGE_PROBE_DMA(H, R)                                                                                    \
    do {                                                                                                         \
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&probe_dma_kernel<H, R>),                        \
                                  hipFuncAttributeMaxDynamicSharedMemorySize, lds);                              \
        probe_dma_kernel<H, R><<<256, 256, lds, s>>>(p, bytes, K, share, static_cast<int*>(out));                \
    } while (0)
    if (half) {
        if (ldsr) FORGE_PROBE_DMA(true, true);
        else FORGE_PROBE_DMA(true, false);
    } else {
        if (ldsr) FORGE_PROBE_DMA(false, true);
        else FORGE_PROBE_DMA(false, false);
    }
#undef FORGE_PROBE_DMA
    return launch_status();
}
