// forge::sparsity metadata pack for MI355X. Drop-in for
// include/forge/sparsity/pack_metadata.cuh: same (N, K/32) uint32 buffer, words in the
// gfx950 SMFMAC index layout (word (n, c) of the reference at
// (n/16)*(K/32)*16 + c*R + n%16, R = rows of n's 16-row block).
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace forge { namespace sparsity {

/// pack_metadata.cuh:15-19: one thread per output word; grid covers N*K/32 threads.
__global__ void pack_metadata_kernel(
    const uint8_t* __restrict__ meta_raw,
    uint32_t* __restrict__      meta_packed,
    int                         N,
    int                         K);

/// pack_metadata.cuh:21-26.
void pack_metadata(
    const uint8_t* meta_raw,    // (N * K/4) device
    uint32_t*      meta_packed, // (N * K/32) device
    int            N,
    int            K,
    hipStream_t    stream = nullptr);

/// Extension: gfx950 words -> raw nibbles (inverse of pack_metadata).
void unpack_metadata(
    const uint32_t* meta_packed, uint8_t* meta_raw, int N, int K, hipStream_t stream = nullptr);

}} // namespace forge::sparsity
