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

inline int divup(int a, int b) { return (a + b - 1) / b; }
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

// GEMM dequant epilogue: half(fma((float)acc, as*ws, bias)), or acc*(as*ws) without bias.
__device__ __forceinline__ uint16_t dequant_gemm(int acc, float as, float ws, float b, bool has_bias) {
    const float s = as * ws;
    const float a = static_cast<float>(acc);
    return f2h(has_bias ? __builtin_fmaf(a, s, b) : a * s);
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
