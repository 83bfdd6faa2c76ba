// forge::sparsity 2:4 prune + compress for MI355X. Drop-in for
// include/forge/sparsity/prune_compress.cuh. Bit-identical values and nibbles.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace forge { namespace sparsity {

/// prune_compress.cuh:16-21: one thread per group of 4; grid covers N*K/4 threads.
__global__ void prune_compress_kernel(
    const int8_t* __restrict__  weight,
    int8_t* __restrict__        compressed,
    uint8_t* __restrict__       metadata_raw,
    int                         N,
    int                         K);

/// prune_compress.cuh:23-29.
void prune_compress_24(
    const int8_t* weight,       // (N, K) device
    int8_t*       compressed,   // (N, K/2) device
    uint8_t*      metadata_raw, // (N * K/4) device
    int           N,
    int           K,
    hipStream_t   stream = nullptr);

}} // namespace forge::sparsity
