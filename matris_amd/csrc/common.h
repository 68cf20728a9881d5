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

// The current device's status word (defined in gmlp.hip; MATRIS_STATUS_* bits), nullptr
// on failure.
unsigned *matris_range_flag();

static inline int matris_blocks(int64_t work, int per_block) {
    int64_t b = (work + per_block - 1) / per_block;
    return (int)(b < 1 ? 1 : b);
}

// The work-group's place in the grid with each XCD given one contiguous range: the
// hardware deals work-groups to the 8 XCDs round-robin (group b to XCD b % 8), so
// neighbouring groups -- which read neighbouring segments' rows and the rows those share
// -- would otherwise sit behind eight different L2s.  A bijection of [0, gridDim.x).
__device__ __forceinline__ int64_t xcd_block() {
    const int64_t nb = gridDim.x, b = blockIdx.x;
    const int64_t q = nb >> 3, r = nb & 7, x = b & 7;
    return x * q + (x < r ? x : r) + (b >> 3);
}

// Work-group barrier that orders LDS only: the fences are scoped to the local address
// space, so the barrier waits for this wave's LDS operations but leaves global loads
// (prefetches) in flight, where __syncthreads() would drain them all.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Sum over the 16 lanes of a DPP row (lanes 16r .. 16r+15), returned in all of them:
// quad swaps, then the half-row and row mirrors, as four VALU ops with DPP operands.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    v += dpp_f<0x140>(v);  // row_mirror
    return v;
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

// e^-x = 2^t, t = -x log2(e), on v_exp_f32 (1 ulp).  The rounding error of the product
// (recovered exactly by an FMA, plus the fp32 representation error of log2 e) is applied
// as the first-order factor 1 + err ln 2, so the result is within ~2 ulp of e^-x
// instead of degrading with |t| ulp.  Overflow gives +inf (the product form keeps
// inf * 1 = inf), underflow 0.  x must be finite (an infinite x makes the error term
// inf - inf).
__device__ __forceinline__ float exp_neg_f(float x) {
    constexpr float kL2e = 1.44269502162933349609375f;  // fp32(log2 e)
    constexpr float kL2eLo = 1.9259629911266175e-08f;   // log2 e - kL2e
    constexpr float kLn2 = 0.693147180559945309f;
    const float t = -x * kL2e;
    const float err = fmaf(-x, kL2eLo, fmaf(-x, kL2e, -t));
    return __builtin_amdgcn_exp2f(t) * (1.0f + err * kLn2);
}

// Count of set bits below this lane in a 64-bit ballot.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
    int lane = threadIdx.x & 63;
    uint64_t below = lane == 0 ? 0ull : (mask & ((~0ull) >> (64 - lane)));
    return __popcll(below);
}
