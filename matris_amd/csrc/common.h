// Shared helpers for the MatRIS gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/matris_hip.h"

#define MATRIS_D 128  // feature width of every node / bond / angle row

#define MATRIS_CHECK_LAUNCH()                          \
    do {                                               \
        hipError_t _e = hipGetLastError();             \
        if (_e != hipSuccess) return (int)_e;          \
    } while (0)

static inline int matris_blocks(int64_t work, int per_block) {
    int64_t b = (work + per_block - 1) / per_block;
    return (int)(b < 1 ? 1 : b);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Sum over the 32 lanes sharing lane/32 (one half of a wave).
__device__ __forceinline__ float half_sum(float v) {
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Count of set bits below this lane in a 64-bit ballot.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
    int lane = threadIdx.x & 63;
    uint64_t below = lane == 0 ? 0ull : (mask & ((~0ull) >> (64 - lane)));
    return __popcll(below);
}
