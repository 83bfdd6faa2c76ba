// Ownership of static device buffers ("slots") by launch key, for kernels that need device
// memory beyond their operands without allocating it (the decode K-split sums, the fused
// sparse linear's packed weights). Two launches must never use one slot at the same time, so a
// slot belongs to one key: (stream, 0) for launches made outside graph capture, whose launches
// on that stream run in order, and (stream, capture id) for launches recorded into a graph,
// which run in order within each replay of that graph. No key is shared between eager work and
// a capture, or between two captures; a graph must not be replayed while another replay of the
// same graph is still running (as for any graph whose nodes share memory). A slot stays with
// its key until the process ends; a launch that finds every slot held by other keys takes the
// path that needs none.
#pragma once

#include <hip/hip_runtime.h>

namespace forge_amd {

constexpr int kSlotMaxDev = 64;

// The current device, or false (error cleared) when it cannot be read or is out of range.
inline bool slot_device(int* dev)
{
    if (hipGetDevice(dev) != hipSuccess || *dev < 0 || *dev >= kSlotMaxDev) {
        (void)hipGetLastError();
        return false;
    }
    return true;
}

struct SlotKey {
    hipStream_t stream;
    unsigned long long capture;   // 0: eager launches; otherwise the capture's id
};

// The key of a launch on s; false for hipStreamPerThread (one handle for many host threads'
// streams), for an invalidated capture, and when the capture state cannot be read.
inline bool slot_key(hipStream_t s, SlotKey* key)
{
    if (s == hipStreamPerThread) return false;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    unsigned long long cid = 0;
    if (hipStreamGetCaptureInfo(s, &cs, &cid) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    if (cs == hipStreamCaptureStatusInvalidated) return false;
    *key = SlotKey{s, cs == hipStreamCaptureStatusActive ? (cid ? cid : ~0ull) : 0ull};
    return true;
}

// Owners of kN slots on each device. Not locked: the caller serialises take() with its own
// mutex (the one that also guards its slot addresses).
template <int kN>
class SlotOwners {
public:
    // The key's slot on device dev (taking a free one on its first launch), or -1 when all kN
    // are held by other keys.
    int take(int dev, const SlotKey& key)
    {
        for (int i = 0; i < used_[dev]; i++)
            if (owner_[dev][i].stream == key.stream && owner_[dev][i].capture == key.capture) return i;
        if (used_[dev] == kN) return -1;
        owner_[dev][used_[dev]] = key;
        return used_[dev]++;
    }

    // Slots of device dev held by some key (they are never released).
    int used(int dev) const { return used_[dev]; }

private:
    SlotKey owner_[kSlotMaxDev][kN] = {};
    int used_[kSlotMaxDev] = {};
};

}  // namespace forge_amd
