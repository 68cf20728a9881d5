// MFMA building blocks shared by the fused GEMM kernels (gmlp.hip, mlp.hip): fp32
// and split-bf16 32x32 MFMA tiles fed from LDS / global row-major operands.
#pragma once
#include "common.h"

typedef float v16f __attribute__((ext_vector_type(16)));

#define BM 64
#define BK 32
#define LDX 36   // LDS row stride (floats) of the X chunk
#define LDW 36   // LDS row stride of the W1 chunk
#define LDH 260  // LDS row stride of the [64, 256] h / gradient tiles

__device__ __forceinline__ v16f mfma32(float a, float b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float sigm_f(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float dsilu_f(float x) {
    float s = sigm_f(x);
    return s * (1.0f + x * (1.0f - s));
}

// Row of accumulator register i of a 32x32 tile for lane half h.
__device__ __forceinline__ int acc_row(int i, int h) { return (i >> 2) * 8 + h * 4 + (i & 3); }

// ------------------------------------------------------------------------------------
// MFMA precision modes.  MODE 0: fp32 operands on v_mfma_f32_32x32x2f32.  MODE 3 / 6:
// each fp32 operand is split exactly into bf16 parts x = hi + mid + lo (hi = bf16(x),
// mid = bf16(x - hi), lo = bf16(x - hi - mid)) and the product is accumulated in fp32 on
// v_mfma_f32_32x32x16_bf16 from 3 (hi*hi + hi*mid + mid*hi) or 6 (+ hi*lo + mid*mid +
// lo*hi) partial products.  MODE 6 carries ~24 significant bits per operand, i.e. fp32
// GEMM accuracy, at 6 x 32 cycles per 32x32x16 block instead of 8 x 64 for MODE 0.
//
// Operand fragments of one 32-wide K chunk: per 32-row tile the lane holds 16 values as
// 4 float4 at columns col4(q): MODE 0 uses columns 16h + 4q (step q*4+c consumes column
// 16h+4q+c); the bf16 modes use 16(q>>1) + 8h + 4(q&1) (sub-step s consumes the 8
// columns 16s + 8h .. +7, the k layout of the 32x32x16 instruction).  A and B always use
// the same permutation of K, so the sum over the chunk is unchanged.
// ------------------------------------------------------------------------------------
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

template <int MODE>
__device__ __forceinline__ int col4(int q, int h) {
    return MODE == 0 ? 16 * h + 4 * q : 16 * (q >> 1) + 8 * h + 4 * (q & 1);
}

template <int MODE>
__device__ __forceinline__ void split8(const float4 &u, const float4 &v, v8bf &hi, v8bf &mid, v8bf &lo) {
    const float x[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const __bf16 a = (__bf16)x[j];
        const float r = x[j] - (float)a;
        const __bf16 b = (__bf16)r;
        hi[j] = a;
        mid[j] = b;
        if (MODE == 6) lo[j] = (__bf16)(r - (float)b);
    }
}

__device__ __forceinline__ v16f mfma_bf16(const v8bf &a, const v8bf &b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// acc[rt][ct] += A-tile[rt] * B-tile[ct] for one K chunk given the fragments.
template <int MODE, int NRT, int NCT>
__device__ __forceinline__ void chunk_mma(v16f (&acc)[NRT][NCT], const float4 (&a)[NRT][4],
                                          const float4 (&b)[NCT][4]) {
    if constexpr (MODE == 0) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
                for (int ct = 0; ct < NCT; ++ct) {
                    acc[rt][ct] = mfma32(a[rt][q].x, b[ct][q].x, acc[rt][ct]);
                    acc[rt][ct] = mfma32(a[rt][q].y, b[ct][q].y, acc[rt][ct]);
                    acc[rt][ct] = mfma32(a[rt][q].z, b[ct][q].z, acc[rt][ct]);
                    acc[rt][ct] = mfma32(a[rt][q].w, b[ct][q].w, acc[rt][ct]);
                }
    } else {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            v8bf ah[NRT], am[NRT], al[NRT], bh[NCT], bm[NCT], bl[NCT];
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt) split8<MODE>(a[rt][2 * s], a[rt][2 * s + 1], ah[rt], am[rt], al[rt]);
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) split8<MODE>(b[ct][2 * s], b[ct][2 * s + 1], bh[ct], bm[ct], bl[ct]);
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
                for (int ct = 0; ct < NCT; ++ct) {
                    if constexpr (MODE == 6) {
                        acc[rt][ct] = mfma_bf16(al[rt], bh[ct], acc[rt][ct]);
                        acc[rt][ct] = mfma_bf16(am[rt], bm[ct], acc[rt][ct]);
                        acc[rt][ct] = mfma_bf16(ah[rt], bl[ct], acc[rt][ct]);
                    }
                    acc[rt][ct] = mfma_bf16(am[rt], bh[ct], acc[rt][ct]);
                    acc[rt][ct] = mfma_bf16(ah[rt], bm[ct], acc[rt][ct]);
                    acc[rt][ct] = mfma_bf16(ah[rt], bh[ct], acc[rt][ct]);
                }
        }
    }
}

// Fragments of NT 32-row tiles of a row-major array (rows t*32 + l32, row stride ld).
template <int MODE, int NT>
__device__ __forceinline__ void load_frag(float4 (&f)[NT][4], const float *base, int64_t ld, int lane) {
    const int h = lane >> 5, l32 = lane & 31;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q)
            f[t][q] = *reinterpret_cast<const float4 *>(base + (int64_t)(t * 32 + l32) * ld + col4<MODE>(q, h));
}

// acc[rt][ct] += A[rt*32.., k] * B[k, ct*32..] for a 32-wide K chunk; A rows at
// a_base + row * lda (LDS), B as rows n of a [n][k] array at b_base + n * ldb.
template <int MODE, int NRT, int NCT>
__device__ __forceinline__ void mfma_chunk(v16f (&acc)[NRT][NCT], const float *a_base, int lda, const float *b_base,
                                           int ldb, int lane) {
    float4 a[NRT][4], b[NCT][4];
    load_frag<MODE, NRT>(a, a_base, lda, lane);
    load_frag<MODE, NCT>(b, b_base, ldb, lane);
    chunk_mma<MODE, NRT, NCT>(acc, a, b);
}

// acc += A[:, 0:KD] (LDS) * B[0:KD, :] with B read from global as rows of a [n][k]
// array, the next chunk's B fragments prefetched while the current one is consumed.
template <int MODE, int NRT, int NCT, int KD>
__device__ __forceinline__ void gemm_lds_a_global_b(v16f (&acc)[NRT][NCT], const float *a_base, int lda,
                                                    const float *__restrict__ b_base, int ldb, int lane) {
    float4 cur[NCT][4], nxt[NCT][4];
    load_frag<MODE, NCT>(cur, b_base, ldb, lane);
#pragma unroll 1
    for (int kc = 0; kc < KD; kc += BK) {
        if (kc + BK < KD) load_frag<MODE, NCT>(nxt, b_base + kc + BK, ldb, lane);
        float4 a[NRT][4];
        load_frag<MODE, NRT>(a, a_base + kc, lda, lane);
        chunk_mma<MODE, NRT, NCT>(acc, a, cur);
        if (kc + BK < KD) {
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
                for (int q = 0; q < 4; ++q) cur[ct][q] = nxt[ct][q];
        }
    }
}

template <int NRT, int NCT>
__device__ __forceinline__ void zero_acc(v16f (&acc)[NRT][NCT]) {
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[rt][ct][i] = 0.f;
}

