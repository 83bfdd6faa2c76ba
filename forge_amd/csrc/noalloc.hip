// forge_int8_linear_noalloc: forge_int8_linear for callers that cannot allocate device memory
// (code under graph capture, tight serving loops, harnesses that forbid hipMalloc). The
// quantized activations and their per-token scales -- the scratch that forge_int8_linear takes
// from its caller -- live in a file-scope device array here, one copy per GPU, so the call
// takes only inputs and outputs and allocates nothing.
//
// Layout of the array for one call: the INT8 rows (M*K bytes) from offset 0, the FP32 scales
// (M floats) from the next 256-byte boundary. Every call on a GPU uses that GPU's array and
// leaves its contents behind; each call overwrites all of what it reads (the quantize writes
// every row and scale before the GEMM reads them), so nothing needs clearing. Calls that
// overlap in time on one GPU (different streams with no ordering between them) race on the
// array and must not be made.
#include "common.h"
#include "gemm_dense.h"
#include "forge_amd.h"

#include <mutex>

namespace forge_amd {

constexpr size_t kNoAllocMaxQBytes = size_t{16} << 20;   // M * K quantized bytes
constexpr int kNoAllocMaxRows = 65536;                    // M (FP32 scales: 256 KiB)
constexpr size_t kNoAllocScalesOffset = kNoAllocMaxQBytes;
constexpr size_t kNoAllocBytes = kNoAllocMaxQBytes + static_cast<size_t>(kNoAllocMaxRows) * sizeof(float);
static_assert(FORGE_NOALLOC_MAX_QBYTES == kNoAllocMaxQBytes && FORGE_NOALLOC_MAX_ROWS == kNoAllocMaxRows,
              "header limits match");

static __device__ __align__(256) int8_t scratch[kNoAllocBytes];

namespace {
constexpr int kNoAllocMaxDev = 64;
std::mutex g_na_mu;
int8_t* g_na_ptr[kNoAllocMaxDev];   // device address of `scratch` on each device, once resolved

// The device address of `scratch` on the current device, resolved once per device with that
// device current (hipGetSymbolAddress); nullptr when it cannot be resolved. A first call made
// while `stream` captures a graph does not resolve it (forge_init does, outside any capture).
int8_t* scratch_ptr(hipStream_t stream, int* status)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kNoAllocMaxDev) {
        (void)hipGetLastError();
        *status = FORGE_ENODEV;
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_na_mu);
    if (g_na_ptr[dev]) return g_na_ptr[dev];
    if (stream) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cs) != hipSuccess) {
            (void)hipGetLastError();
            *status = FORGE_ENODEV;
            return nullptr;
        }
        if (cs != hipStreamCaptureStatusNone) {
            *status = FORGE_EINVAL;   // call forge_init (or the entry point) once before capturing
            return nullptr;
        }
    }
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        *status = FORGE_ENODEV;
        return nullptr;
    }
    g_na_ptr[dev] = static_cast<int8_t*>(p);
    return g_na_ptr[dev];
}
}  // namespace

int noalloc_prepare()
{
    int st = FORGE_OK;
    return scratch_ptr(nullptr, &st) ? FORGE_OK : st;
}

}  // namespace forge_amd

using namespace forge_amd;

extern "C" int forge_int8_linear_noalloc(const uint16_t* x, const int8_t* w, const uint16_t* w_scale,
                                         const uint16_t* bias, uint16_t* out, int M, int K, int N, void* stream)
{
    if (M <= 0 || K <= 0 || N <= 0) return FORGE_OK;
    if (!x || !w || !w_scale || !out) return FORGE_EINVAL;
    if (M > kNoAllocMaxRows || static_cast<size_t>(M) * static_cast<size_t>(K) > kNoAllocMaxQBytes)
        return FORGE_ERANGE;
    int st = FORGE_OK;
    int8_t* base = scratch_ptr(as_stream(stream), &st);
    if (!base) return st;
    int8_t* q = base;
    float* scales = reinterpret_cast<float*>(base + kNoAllocScalesOffset);
    return forge_int8_linear(x, w, w_scale, bias, out, M, K, N, q, scales, stream);
}
