// The readout of MatRIS (model.py:238-244, readout.py:18-133) on N node rows, fused:
//   n   = x * rsqrt(mean(x^2) + eps) * wn                            RMSNorm (readout_norm)
//   e   = w3 . SiLU(W2 SiLU(W1 n + b1) + b2) + b3                     EnergyHead MLP(128, (128, 128), 1)
//   m   = | w5 . SiLU(W4 n + b4) + b5 |                               MagmomHead MLP(128, 256, 1)
// and the backward of the energy branch to x (the forces' path; the magmom head is not
// differentiated):  g_x = RMSNorm'(x)^T W1^T (SiLU'(a1) * W2^T (SiLU'(a2) * w3 g_e)).
// The backward recomputes the forward's pre-activations of its rows instead of reading
// saved ones.  Every sum runs in fp32 FMAs in a fixed order (no atomics).
//
// A work-group of 256 threads takes RB = 8 rows (a launch of N = 864 rows is latency-bound,
// so more work-groups beat more reuse): the rows' vectors live in LDS, and each output
// column of a layer belongs to one thread (two for the 128-wide layers, each with half the
// rows), which streams its weight column from global memory (weights transposed, [K][C]:
// consecutive threads read consecutive floats), 32 weights in flight, and reuses every
// weight for its rows.
#include "mma.h"  // sigm_f / silu_f / dsilu_f

#define RB 8

// out[r][c] = b[c] + sum_k wt[k][c] in[r][k] for the thread's rows r0 .. r0+nr-1 (nr <= 8
// per thread), K a multiple of 4, in / out LDS rows of stride K / C.
template <int NR>
__device__ __forceinline__ void ro_layer(const float *in, int K, const float *__restrict__ wt, int C,
                                         const float *__restrict__ b, int c, int r0, float (&acc)[NR]) {
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = b ? b[c] : 0.f;
#pragma unroll 8
    for (int k = 0; k < K; k += 4) {
        const float w0 = wt[(k + 0) * C + c], w1 = wt[(k + 1) * C + c];
        const float w2 = wt[(k + 2) * C + c], w3 = wt[(k + 3) * C + c];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const float4 v = *reinterpret_cast<const float4 *>(in + (r0 + r) * K + k);
            acc[r] = fmaf(w0, v.x, acc[r]);
            acc[r] = fmaf(w1, v.y, acc[r]);
            acc[r] = fmaf(w2, v.z, acc[r]);
            acc[r] = fmaf(w3, v.w, acc[r]);
        }
    }
}

struct ReadoutW {
    const float *wn;                 // [128] RMSNorm weight
    const float *w1t, *b1;           // W1^T [128][128], b1 [128]
    const float *w2t, *b2, *w2;      // W2^T [128][128], b2 [128]; W2 [128][128] (backward)
    const float *w3, *b3;            // [128], [1]
    const float *w1;                 // W1 [128][128] (backward)
    const float *w4t, *b4, *w5, *b5;  // W4^T [128][256], b4 [256], w5 [256], b5 [1]
    float eps;
};

// LDS row vectors of the block's RB rows: x / n [RB][128], h1 [RB][128], a second
// [RB][256] buffer (h2 or the magmom hidden layer), row scalars.
struct RoSmem {
    float x[RB * 128];
    float n[RB * 128];
    float h1[RB * 128];
    float t[RB * 256];
    float rinv[RB];
    float red[RB][8];
};

// rows of the block into LDS, their RMS scale, n = x rinv wn
__device__ __forceinline__ void ro_norm(RoSmem &S, const float *__restrict__ x, int64_t r0, int64_t N,
                                       const ReadoutW &W) {
    const int tid = threadIdx.x;
    for (int q = tid; q < RB * 32; q += 256) {  // float4 units
        const int r = q >> 5, c4 = (q & 31) * 4;
        const int64_t row = r0 + r < N ? r0 + r : N - 1;
        *reinterpret_cast<float4 *>(S.x + r * 128 + c4) = *reinterpret_cast<const float4 *>(x + row * 128 + c4);
    }
    __syncthreads();
    if (tid < RB * 8) {  // 8 threads per row, then a fixed-order sum of the 8 partials
        const int r = tid >> 3, p = tid & 7;
        float s = 0.f;
        for (int k = p * 16; k < p * 16 + 16; ++k) s = fmaf(S.x[r * 128 + k], S.x[r * 128 + k], s);
        S.red[r][p] = s;
    }
    __syncthreads();
    if (tid < RB) {
        float s = 0.f;
        for (int p = 0; p < 8; ++p) s += S.red[tid][p];
        S.rinv[tid] = rsqrtf(s * (1.0f / 128.0f) + W.eps);
    }
    __syncthreads();
    for (int q = tid; q < RB * 128; q += 256) {
        const int r = q >> 7, c = q & 127;
        S.n[q] = S.x[q] * S.rinv[r] * W.wn[c];
    }
    __syncthreads();
}

// a1, h1 = SiLU(a1) (h1 to LDS; a1 kept by the caller when asked), then a2 (returned per
// thread: column c = tid & 127, rows (RB / 2) (tid >> 7) .. +RB/2-1)
__device__ __forceinline__ void ro_energy_layers(RoSmem &S, const ReadoutW &W, float (&a1)[RB / 2],
                                                 float (&a2)[RB / 2]) {
    const int tid = threadIdx.x, c = tid & 127, rh = (tid >> 7) * (RB / 2);
    ro_layer<RB / 2>(S.n, 128, W.w1t, 128, W.b1, c, rh, a1);
#pragma unroll
    for (int r = 0; r < RB / 2; ++r) S.h1[(rh + r) * 128 + c] = silu_f(a1[r]);
    __syncthreads();
    ro_layer<RB / 2>(S.h1, 128, W.w2t, 128, W.b2, c, rh, a2);
}

__global__ __launch_bounds__(256) void readout_fwd_kernel(int64_t N, const float *__restrict__ x, ReadoutW W,
                                                          float *__restrict__ e, float *__restrict__ m) {
    __shared__ RoSmem S;
    const int tid = threadIdx.x, c = tid & 127, rh = (tid >> 7) * (RB / 2);
    const int64_t r0 = (int64_t)blockIdx.x * RB;
    ro_norm(S, x, r0, N, W);
    float a1[RB / 2], a2[RB / 2];
    ro_energy_layers(S, W, a1, a2);
    // e = w3 . SiLU(a2) + b3: products to LDS, then a fixed-order row sum
#pragma unroll
    for (int r = 0; r < RB / 2; ++r) S.t[(rh + r) * 128 + c] = silu_f(a2[r]) * W.w3[c];
    __syncthreads();
    if (tid < RB * 8) {
        const int r = tid >> 3, p = tid & 7;
        float s = 0.f;
        for (int k = p * 16; k < p * 16 + 16; ++k) s += S.t[r * 128 + k];
        S.red[r][p] = s;
    }
    __syncthreads();
    if (tid < RB && r0 + tid < N) {
        float s = W.b3[0];
        for (int p = 0; p < 8; ++p) s += S.red[tid][p];
        e[r0 + tid] = s;
    }
    __syncthreads();
    // magmom: hidden 256 (thread tid = column), then | w5 . SiLU(.) + b5 |
    float am[RB];
    ro_layer<RB>(S.n, 128, W.w4t, 256, W.b4, tid, 0, am);
#pragma unroll
    for (int r = 0; r < RB; ++r) S.t[r * 256 + tid] = silu_f(am[r]) * W.w5[tid];
    __syncthreads();
    if (tid < RB * 8) {
        const int r = tid >> 3, p = tid & 7;
        float s = 0.f;
        for (int k = p * 32; k < p * 32 + 32; ++k) s += S.t[r * 256 + k];
        S.red[r][p] = s;
    }
    __syncthreads();
    if (tid < RB && r0 + tid < N) {
        float s = W.b5[0];
        for (int p = 0; p < 8; ++p) s += S.red[tid][p];
        m[r0 + tid] = fabsf(s);
    }
}

// g_e [N]: the gradient of each row's energy; g_x [N][128] written (or added to when
// accumulate).
__global__ __launch_bounds__(256) void readout_bwd_kernel(int64_t N, const float *__restrict__ x, ReadoutW W,
                                                          const float *__restrict__ g_e, int accumulate,
                                                          float *__restrict__ g_x) {
    __shared__ RoSmem S;
    const int tid = threadIdx.x, c = tid & 127, rh = (tid >> 7) * (RB / 2);
    const int64_t r0 = (int64_t)blockIdx.x * RB;
    ro_norm(S, x, r0, N, W);
    float a1[RB / 2], a2[RB / 2];
    ro_energy_layers(S, W, a1, a2);
    // g_a2 = g_e w3 SiLU'(a2)  -> S.t (stride 128)
#pragma unroll
    for (int r = 0; r < RB / 2; ++r) {
        const int64_t row = r0 + rh + r;
        const float ge = row < N ? g_e[row] : 0.f;
        S.t[(rh + r) * 128 + c] = ge * W.w3[c] * dsilu_f(a2[r]);
    }
    __syncthreads();
    // g_a1 = (W2^T g_a2) SiLU'(a1): column c of W2^T g_a2 is sum_j W2[j][c] g_a2[j]
    float g1[RB / 2];
    ro_layer<RB / 2>(S.t, 128, W.w2, 128, nullptr, c, rh, g1);
    __syncthreads();  // every thread is done reading S.t
#pragma unroll
    for (int r = 0; r < RB / 2; ++r) S.h1[(rh + r) * 128 + c] = g1[r] * dsilu_f(a1[r]);
    __syncthreads();
    // g_n = W1^T g_a1
    float gn[RB / 2];
    ro_layer<RB / 2>(S.h1, 128, W.w1, 128, nullptr, c, rh, gn);
    // RMSNorm backward: g_x = rinv (wn g_n) - x rinv^3 mean(wn g_n x)
#pragma unroll
    for (int r = 0; r < RB / 2; ++r) S.t[(rh + r) * 128 + c] = gn[r] * W.wn[c];
    __syncthreads();
    if (tid < RB * 8) {
        const int r = tid >> 3, p = tid & 7;
        float s = 0.f;
        for (int k = p * 16; k < p * 16 + 16; ++k) s = fmaf(S.t[r * 128 + k], S.x[r * 128 + k], s);
        S.red[r][p] = s;
    }
    __syncthreads();
    if (tid < RB) {
        float s = 0.f;
        for (int p = 0; p < 8; ++p) s += S.red[tid][p];
        S.red[tid][0] = s * (1.0f / 128.0f);
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < RB / 2; ++r) {
        const int rr = rh + r;
        const int64_t row = r0 + rr;
        if (row >= N) break;
        const float ri = S.rinv[rr];
        float v = ri * S.t[rr * 128 + c] - S.x[rr * 128 + c] * ri * ri * ri * S.red[rr][0];
        if (accumulate) v += g_x[row * 128 + c];
        g_x[row * 128 + c] = v;
    }
}

static ReadoutW readout_w(const float *wn, const float *w1t, const float *b1, const float *w1, const float *w2t,
                          const float *b2, const float *w2, const float *w3, const float *b3, const float *w4t,
                          const float *b4, const float *w5, const float *b5, float eps) {
    ReadoutW W;
    W.wn = wn; W.w1t = w1t; W.b1 = b1; W.w1 = w1; W.w2t = w2t; W.b2 = b2; W.w2 = w2; W.w3 = w3; W.b3 = b3;
    W.w4t = w4t; W.b4 = b4; W.w5 = w5; W.b5 = b5; W.eps = eps;
    return W;
}

extern "C" int matris_readout_fwd(int64_t n, const float *x, const float *wn, const float *w1t, const float *b1,
                                  const float *w2t, const float *b2, const float *w3, const float *b3,
                                  const float *w4t, const float *b4, const float *w5, const float *b5, float eps,
                                  float *e, float *m, void *stream) {
    if (n < 0) return MATRIS_E_ARG;
    if (n == 0) return 0;
    if (!x || !wn || !w1t || !b1 || !w2t || !b2 || !w3 || !b3 || !w4t || !b4 || !w5 || !b5 || !e || !m ||
        ((uintptr_t)x & 15))
        return MATRIS_E_ARG;
    const ReadoutW W = readout_w(wn, w1t, b1, nullptr, w2t, b2, nullptr, w3, b3, w4t, b4, w5, b5, eps);
    readout_fwd_kernel<<<matris_blocks(n, RB), 256, 0, (hipStream_t)stream>>>(n, x, W, e, m);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_readout_bwd(int64_t n, const float *x, const float *wn, const float *w1t, const float *b1,
                                  const float *w1, const float *w2t, const float *b2, const float *w2,
                                  const float *w3, float eps, const float *g_e, int accumulate, float *g_x,
                                  void *stream) {
    if (n < 0) return MATRIS_E_ARG;
    if (n == 0) return 0;
    if (!x || !wn || !w1t || !b1 || !w1 || !w2t || !b2 || !w2 || !w3 || !g_e || !g_x || ((uintptr_t)x & 15))
        return MATRIS_E_ARG;
    const ReadoutW W = readout_w(wn, w1t, b1, w1, w2t, b2, w2, w3, nullptr, nullptr, nullptr, nullptr, nullptr, eps);
    readout_bwd_kernel<<<matris_blocks(n, RB), 256, 0, (hipStream_t)stream>>>(n, x, W, g_e, accumulate, g_x);
    MATRIS_CHECK_LAUNCH();
    return 0;
}
