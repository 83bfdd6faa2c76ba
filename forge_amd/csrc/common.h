// Internal helpers shared by the gfx950 kernels and their launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstddef>
#include <cstdint>

#include "forge_amd.h"

namespace forge_amd {

typedef int   v4i  __attribute__((ext_vector_type(4)));
typedef int   v8i  __attribute__((ext_vector_type(8)));
typedef int   v16i __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// Per-device properties, queried once per device (thread-safe).
struct DeviceInfo {
    int cu_count = 0;        // compute units (256 on MI355X)
    int l2_bytes = 0;        // L2 per XCD as reported by HIP
    int lds_per_block = 0;   // max LDS per workgroup
    int gfx = 0;             // gfx IP version, 950 on MI355X
    bool valid = false;
};

// Returns info for the current device; *status receives FORGE_ENODEV if none.
const DeviceInfo& device_info(int* status);
// Host-only default used where no device exists (planner, CPU tests).
int default_cu_count();
// Records the engine of the calling thread's last GEMM launch ("dma256x256", "decode", ...;
// tile/split appended when >= 0 / > 0), read back by forge_last_route.
void note_route(const char* engine, int tile = -1, int split = 0);

inline int divup(int a, int b) { return static_cast<int>((static_cast<long long>(a) + b - 1) / b); }
inline long long divupll(long long a, long long b) { return (a + b - 1) / b; }

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Status of the last launch on this thread (hipGetLastError semantics).
inline int launch_status() {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? FORGE_OK : static_cast<int>(e);
}

inline bool aligned(const void* p, size_t a) {
    return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

// ---- device-side helpers --------------------------------------------------------

// fp16 bits -> fp32 (exact widening) and fp32 -> fp16 bits (round to nearest even).
__device__ __forceinline__ float h2f(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}
// The empty asm makes f an opaque, already-rounded fp32 register value: without it the
// backend may fuse the multiply or add that produced f into the conversion
// (v_fma_mixlo_f16), which rounds a*b (+c) to fp16 once -- measured to differ from the
// reference's fp32-then-fp16 rounding when the fp32 result is an fp16 tie.
__device__ __forceinline__ uint16_t f2h(float f) {
    asm("" : "+v"(f));
    return __half_as_ushort(__float2half_rn(f));
}

// Per-row activation quantization (src/quant/quantize.cu:49-56, 112-126): the row scale from
// its absmax, and one value with the reciprocal scale, rounded to nearest even and clamped.
__device__ __forceinline__ float row_scale(float amax) {
    return fmaxf(amax, 1e-8f) / 127.0f;
}

__device__ __forceinline__ int quant1(float x, float inv) {
    const float r = __builtin_rintf(x * inv);
    // NaN -> 0 (as a float->int conversion of NaN gives on both vendors), then clamp.
    int q = (r == r) ? static_cast<int>(fminf(fmaxf(r, -128.0f), 127.0f)) : 0;
    return q;
}

// 8 halves (one uint4) -> 8 int8 packed into a uint2.
__device__ __forceinline__ uint2 quant8(uint4 v, float inv) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t out[2] = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int q0 = quant1(h2f(static_cast<uint16_t>(w[j] & 0xFFFFu)), inv);
        const int q1 = quant1(h2f(static_cast<uint16_t>(w[j] >> 16)), inv);
        out[j >> 1] |= ((static_cast<uint32_t>(q0) & 0xFFu) << (16 * (j & 1))) |
                       ((static_cast<uint32_t>(q1) & 0xFFu) << (16 * (j & 1) + 8));
    }
    return make_uint2(out[0], out[1]);
}

__device__ __forceinline__ float absmax8(uint4 v, float m) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
        m = fmaxf(m, fabsf(h2f(static_cast<uint16_t>(w[j] & 0xFFFFu))));
        m = fmaxf(m, fabsf(h2f(static_cast<uint16_t>(w[j] >> 16))));
    }
    return m;
}

// ---- row quantization on fp16 bit patterns (the same results as absmax8/quant8) -------
// With the sign bit cleared, fp16 bit patterns order exactly as their magnitudes (zero,
// subnormals, normals, inf), so the row absmax is a packed u16 maximum, one v_pk_max_u16 per
// two values. NaN patterns (above 0x7C00) sort above inf; a row whose maximum is one holds a
// NaN and takes the fp32 maximum instead, which skips NaN as fmaxf does.
__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
    typedef unsigned short us2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(us2, a),
                                                                  __builtin_bit_cast(us2, b)));
}
__device__ __forceinline__ uint32_t absbits8(uint4 v, uint32_t m) {
    m = pk_max_u16(m, v.x & 0x7FFF7FFFu);
    m = pk_max_u16(m, v.y & 0x7FFF7FFFu);
    m = pk_max_u16(m, v.z & 0x7FFF7FFFu);
    return pk_max_u16(m, v.w & 0x7FFF7FFFu);
}
// Two rows' packed maxima (lo, hi halves each) -> (max of row a, max of row b).
__device__ __forceinline__ uint32_t pk_rows2(uint32_t a, uint32_t b) {
    return pk_max_u16(__builtin_amdgcn_perm(b, a, 0x05040100u), __builtin_amdgcn_perm(b, a, 0x07060302u));
}
// Wave-wide packed u16 maximum by DPP (no LDS traffic): quad swaps and row rotations give
// every lane its 16-lane row's maximum, row_bcast:15/31 fold the four rows into lane 63, whose
// value is returned to all lanes. Needs all 64 lanes active.
__device__ __forceinline__ uint32_t wave_max_pk_u16(uint32_t v) {
    const int x = static_cast<int>(v);
    v = pk_max_u16(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(x, x, 0xB1, 0xF, 0xF, false)));
    int y = static_cast<int>(v);
    v = pk_max_u16(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(y, y, 0x4E, 0xF, 0xF, false)));
    y = static_cast<int>(v);
    v = pk_max_u16(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(y, y, 0x124, 0xF, 0xF, false)));
    y = static_cast<int>(v);
    v = pk_max_u16(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(y, y, 0x128, 0xF, 0xF, false)));
    y = static_cast<int>(v);
    v = pk_max_u16(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(y, y, 0x142, 0xA, 0xF, false)));
    y = static_cast<int>(v);
    v = pk_max_u16(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(y, y, 0x143, 0xC, 0xF, false)));
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}
constexpr uint32_t kHalfInfBits = 0x7C00u;

// One value of a row quantized with inv = 1 / row_scale(absmax of that row), as the byte of
// clamp(rne(x * inv), -128, 127). |x| <= absmax bounds |x * inv| by 127 plus a few ulp, so the
// clamp acts only on NaN (x NaN, or an inf row's inf * 0): fl(x * inv) + 1.5 * 2^23 rounds
// the product to an integer held in the low mantissa bits (round to nearest even, as rintf,
// for |v| < 2^22), whose low byte is the two's complement int8; a NaN's low byte is 0 (fp16
// NaN payloads land 13 bits up; the default NaN is 0x7FC00000). The asm keeps the product
// rounded on its own (a fused multiply-add would round once). The product is taken as
// fma(x, inv, +0), which rounds x * inv once just as the plain product does (only the sign of a
// zero result can differ, and the add erases it): with the fp16 operand widened inside, that is
// one v_fma_mix_f32 in place of a conversion and a multiply.
__device__ __forceinline__ uint32_t qrow_bits(uint16_t h, float inv) {
    float p = __builtin_fmaf(__half2float(__ushort_as_half(h)), inv, 0.0f);
    asm("" : "+v"(p));
    return __float_as_uint(p + 12582912.0f);
}
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
    return __builtin_amdgcn_perm(b1, b0, 0x0C0C0400u) | __builtin_amdgcn_perm(b3, b2, 0x04000C0Cu);
}
// 8 halves of a row -> 8 int8, equal to quant8(v, inv) when inv comes from the row's absmax.
__device__ __forceinline__ uint2 quant8_row(uint4 v, float inv) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t b[8];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        b[2 * j] = qrow_bits(static_cast<uint16_t>(w[j] & 0xFFFFu), inv);
        b[2 * j + 1] = qrow_bits(static_cast<uint16_t>(w[j] >> 16), inv);
    }
    return make_uint2(pack_low_bytes(b[0], b[1], b[2], b[3]), pack_low_bytes(b[4], b[5], b[6], b[7]));
}

// fl(h * inv) for the fp16 in the low / high half of h, as one v_fma_mix_f32 (the widening
// inside, fma(x, inv, +0) rounds the product once as the multiply does; only a zero's sign can
// differ, which the rounding add below erases).
__device__ __forceinline__ float fma_mix_lo(uint32_t h, float inv) {
    float p;
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(p) : "v"(h), "v"(inv));
    return p;
}
__device__ __forceinline__ float fma_mix_hi(uint32_t h, float inv) {
    float p;
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(p) : "v"(h), "v"(inv));
    return p;
}
// 16 rounded products -> 16 INT8 bytes (byte k of dword d from p[4 d + k]), the bytes of
// qrow_bits: one SDWA add of 1.5 * 2^23 per value whose low result byte goes straight into its
// byte of the dword (dst_sel:BYTE_k; a dword's first write zero-pads it, the others keep the
// bytes already there), in place of an add and a quarter of a 3-instruction pack. The adds
// cycle over the 4 dwords, so no add reads a dword the instruction just before it wrote (a
// byte-select write read by the next VALU instruction needs a wait state on this
// architecture), and the block ends with one for the instruction that reads the dwords.
__device__ __forceinline__ uint4 pack16_rint_sdwa(const float (&p)[16]) {
    const float magic = 12582912.0f;
    uint32_t q0, q1, q2, q3;
    asm("v_add_f32_sdwa %0, %4, %20 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:DWORD\n\t"
        "v_add_f32_sdwa %1, %8, %20 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:DWORD\n\t"
        "v_add_f32_sdwa %2, %12, %20 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:DWORD\n\t"
        "v_add_f32_sdwa %3, %16, %20 dst_sel:BYTE_0 dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:DWORD\n\t"
        "v_add_f32_sdwa %0, %5, %20 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD\n\t"
        "v_add_f32_sdwa %1, %9, %20 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD\n\t"
        "v_add_f32_sdwa %2, %13, %20 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD\n\t"
        "v_add_f32_sdwa %3, %17, %20 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD\n\t"
        "v_add_f32_sdwa %0, %6, %20 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD\n\t"
        "v_add_f32_sdwa %1, %10, %20 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD\n\t"
        "v_add_f32_sdwa %2, %14, %20 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD\n\t"
        "v_add_f32_sdwa %3, %18, %20 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD\n\t"
        "v_add_f32_sdwa %0, %7, %20 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD\n\t"
        "v_add_f32_sdwa %1, %11, %20 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD\n\t"
        "v_add_f32_sdwa %2, %15, %20 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD\n\t"
        "v_add_f32_sdwa %3, %19, %20 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD\n\t"
        "s_nop 0"
        : "=&v"(q0), "=&v"(q1), "=&v"(q2), "=&v"(q3)
        : "v"(p[0]), "v"(p[1]), "v"(p[2]), "v"(p[3]), "v"(p[4]), "v"(p[5]), "v"(p[6]), "v"(p[7]), "v"(p[8]),
          "v"(p[9]), "v"(p[10]), "v"(p[11]), "v"(p[12]), "v"(p[13]), "v"(p[14]), "v"(p[15]), "v"(magic));
    return make_uint4(q0, q1, q2, q3);
}
// Two rows' 8 halves each -> their 8 INT8 values (qa from a with inv_a, qb from b with inv_b),
// each equal to quant8_row of that row.
__device__ __forceinline__ void quant8_rows2(uint4 a, float inv_a, uint4 b, float inv_b, uint2& qa, uint2& qb) {
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    float p[16];
#pragma unroll
    for (int d = 0; d < 8; d++) {
        const float inv = d < 4 ? inv_a : inv_b;
        p[2 * d] = fma_mix_lo(w[d], inv);
        p[2 * d + 1] = fma_mix_hi(w[d], inv);
    }
    const uint4 q = pack16_rint_sdwa(p);
    qa = make_uint2(q.x, q.y);
    qb = make_uint2(q.z, q.w);
}

// GEMM dequant epilogue: half(fma((float)acc, as*ws, bias)), or acc*(as*ws) without bias.
__device__ __forceinline__ uint16_t dequant_gemm(int acc, float as, float ws, float b, bool has_bias) {
    const float s = as * ws;
    const float a = static_cast<float>(acc);
    return f2h(has_bias ? __builtin_fmaf(a, s, b) : a * s);
}

// dequant_gemm of 4 consecutive columns of one row as their 8 bytes of fp16:
// fma((float)acc, as * ws, b), where the caller passes b = -0 without a bias (fma(a, s, -0) is
// a * s rounded once, zeros' signs included, so one form serves both), rounded in column pairs
// by v_cvt_pk_f16_f32 (round to nearest even, the first column in the low half).
__device__ __forceinline__ uint2 dequant4_pk(int a0, int a1, int a2, int a3, float as, const float (&ws)[4],
                                             const float (&b)[4]) {
    const float p0 = __builtin_fmaf(static_cast<float>(a0), as * ws[0], b[0]);
    const float p1 = __builtin_fmaf(static_cast<float>(a1), as * ws[1], b[1]);
    const float p2 = __builtin_fmaf(static_cast<float>(a2), as * ws[2], b[2]);
    const float p3 = __builtin_fmaf(static_cast<float>(a3), as * ws[3], b[3]);
    uint32_t h01, h23;
    asm("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(h01) : "v"(p0), "v"(p1));
    asm("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(h23) : "v"(p2), "v"(p3));
    return make_uint2(h01, h23);
}

// n / d for 0 <= n with n * d < 2^32, with m = ceil(2^32 / d) (m = 0 stands for d = 1): n m / 2^32
// exceeds n / d by n (m d - 2^32) / (d 2^32) < 1 / d, which cannot carry it past the next integer.
__device__ __forceinline__ int udiv_magic(int n, uint32_t m) {
    return m ? static_cast<int>(__umulhi(static_cast<uint32_t>(n), m)) : n;
}
inline uint32_t udiv_multiplier(int d) {
    return d == 1 ? 0u : static_cast<uint32_t>(((1ULL << 32) + d - 1) / d);
}

// Workgroup id -> logical tile id such that each of the 8 XCDs (which receive workgroups
// round-robin by id) runs one contiguous range of tiles: neighbouring tiles, which share
// halo lines, then meet in the same L2. A bijection on [0, total) for any total.
__device__ __forceinline__ int xcd_contiguous(int bid, int total) {
    constexpr int kXcd = 8;
    const int q = total / kXcd, r = total % kXcd;
    const int x = bid % kXcd, i = bid / kXcd;
    return x * q + min(x, r) + i;
}

// Wave-wide max over 64 lanes (every lane receives the result).
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
        v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

}  // namespace forge_amd
