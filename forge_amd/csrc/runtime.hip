// Library-level entry points: status strings, per-device property cache, init.
//
// The reference caches device attributes in unsynchronised function-level statics
// (src/gemm/int8_gemm.cu:13-20, src/quant/quantize.cu:138-147,
// src/gemm/int8_sparse.cu:757-772); here each device is queried once under
// std::call_once, so concurrent first calls are safe and a call made before graph
// capture (forge_init) keeps captured calls free of device queries.
#include "common.h"
#include "gemm_dense.h"

#include <cstdio>
#include <mutex>

namespace forge_amd {

namespace {
constexpr int kMaxDevices = 64;
DeviceInfo g_info[kMaxDevices];
std::once_flag g_once[kMaxDevices];

void query(int dev) {
    DeviceInfo& d = g_info[dev];
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return;
    d.cu_count = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : default_cu_count();
    d.l2_bytes = prop.l2CacheSize > 0 ? prop.l2CacheSize : (4 << 20);
    d.lds_per_block = static_cast<int>(prop.sharedMemPerBlock);
    d.gfx = prop.major * 100 + prop.minor * 10;   // gfx950 reports major 9, minor 5
    d.valid = true;
}
}  // namespace

int default_cu_count() { return 256; }

namespace {
thread_local char t_route[48] = "none";
}

void note_route(const char* engine, int tile, int split)
{
    if (tile >= 0 && split > 0) snprintf(t_route, sizeof t_route, "%s tile%d s%d", engine, tile, split);
    else if (tile >= 0) snprintf(t_route, sizeof t_route, "%s tile%d", engine, tile);
    else snprintf(t_route, sizeof t_route, "%s", engine);
}

const char* last_route() { return t_route; }

const DeviceInfo& device_info(int* status) {
    static DeviceInfo none;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        if (status) *status = FORGE_ENODEV;
        return none;
    }
    std::call_once(g_once[dev], query, dev);
    if (!g_info[dev].valid) {
        if (status) *status = FORGE_ENODEV;
        return none;
    }
    if (status) *status = FORGE_OK;
    return g_info[dev];
}

}  // namespace forge_amd

using namespace forge_amd;

extern "C" const char* forge_status_string(int status) {
    if (status == FORGE_OK) return "ok";
    if (status == FORGE_EINVAL) return "invalid argument (shape, alignment or null pointer)";
    if (status == FORGE_ENODEV) return "no HIP device";
    if (status == FORGE_ERANGE)
        return "size beyond the no-allocation limit (M * K <= 16 MiB of quantized activations, M <= 65536)";
    return hipGetErrorString(static_cast<hipError_t>(status));
}

extern "C" const char* forge_last_route(void) { return last_route(); }

extern "C" int forge_init(void) {
    int st = FORGE_OK;
    device_info(&st);
    if (st != FORGE_OK) return st;
    if ((st = ksplit_prepare()) != FORGE_OK) return st;
    if ((st = fq_pack_prepare()) != FORGE_OK) return st;
    return noalloc_prepare();
}

extern "C" int forge_get_compute_capability(int device, int* out_cc) {
    if (!out_cc) return FORGE_EINVAL;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
        (void)hipGetLastError();
        return FORGE_ENODEV;
    }
    *out_cc = prop.major * 100 + prop.minor * 10;
    return FORGE_OK;
}

extern "C" int forge_has_int8_matrix_cores(int device, int* out_flag) {
    if (!out_flag) return FORGE_EINVAL;
    int cc = 0;
    const int st = forge_get_compute_capability(device, &cc);
    if (st != FORGE_OK) return st;
    *out_flag = cc >= 940 ? 1 : 0;   // gfx94x/gfx950: INT8 MFMA and SMFMAC
    return FORGE_OK;
}
