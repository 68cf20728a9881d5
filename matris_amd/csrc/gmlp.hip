// Fused gated MLP (GatedMLP with RMSNorm, SiLU core, sigmoid gate) on gfx950 MFMA.
//
//   x    = concat_j src_j[idx_j[m]]                         [BM, K]   (gathered on load)
//   p    = x W1^T + b1                                      [BM, 256] (core | gate)
//   h    = SiLU(p)
//   z    = [h_c W2c^T + b2c | h_g W2g^T + b2g]              [BM, 256]
//   out  = SiLU(RMS(z_c) * w_c) * sigmoid(RMS(z_g) * w_g)   [BM, 128]
//
// Work-group = 4 wave64s, BM = 64 rows.  GEMM1 streams K in 32-wide chunks through LDS
// (X chunk gathered row by row, W1 chunk), register-prefetching the next chunk while
// the current one feeds v_mfma_f32_32x32x2f32; each wave owns 64 output columns (a 2x2
// grid of 32x32 tiles).  The [64, 256] result tile goes through LDS: p is copied out
// with 16-byte row stores, h = SiLU(p) stays in LDS as GEMM2's A operand, z returns to
// LDS, is copied out, and a row-per-wave epilogue applies RMSNorm, SiLU, sigmoid and
// the product with 512-byte row stores.  p and z are written for the backward.
//
// Backward (input gradients only) recomputes the norm/activation Jacobians row-wise
// from z, then runs g_h = g_z W2 and g_x = (g_h * SiLU'(p)) W1 through the same MFMA
// tiling, with the transposed weights as B operands.
#include "mma.h"

struct GmlpSrc {
    const float *ptr[4];
    const int32_t *idx[4];
};

// ------------------------------------------------------------------------------------
// forward
// ------------------------------------------------------------------------------------
// Copy a [BM, 256] LDS tile (row stride LDH) to global rows of 256 floats with 16-byte
// stores: consecutive threads cover consecutive 16 B of a row (1 KB per row).
__device__ __forceinline__ void store_tile256(const float *tile, float *__restrict__ dst, int64_t m0, int64_t M,
                                              int tid) {
#pragma unroll
    for (int it = 0; it < (BM * 64) / 256; ++it) {
        const int q = it * 256 + tid;  // float4 index within the tile
        const int row = q >> 6, c4 = (q & 63) * 4;
        if (m0 + row < M)
            *reinterpret_cast<float4 *>(dst + (m0 + row) * 256 + c4) =
                *reinterpret_cast<const float4 *>(tile + row * LDH + c4);
    }
}

template <int MODE>
__global__ __launch_bounds__(256, 2) void gmlp_fwd_kernel(int64_t M, int nsrc, GmlpSrc src,
                                                          const float *__restrict__ W1, const float *__restrict__ b1,
                                                          const float *__restrict__ W2, const float *__restrict__ b2,
                                                          const float *__restrict__ norm_c,
                                                          const float *__restrict__ norm_g, float eps,
                                                          float *__restrict__ out, float *__restrict__ save_p,
                                                          float *__restrict__ save_z) {
    __shared__ __align__(16) float smem[BM * LDH];
    float *Xs = smem;
    float *Ws = smem + BM * LDX;
    float *Ts = smem;  // [BM, 256] tile: p, then h, then z

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int h = lane >> 5, l32 = lane & 31;
    const int64_t m0 = (int64_t)blockIdx.x * BM;
    const int K = nsrc * MATRIS_D;

    // gather assignment: thread -> (row xr, 8 columns at xc) of each X chunk
    const int xr = tid >> 2, xc = (tid & 3) * 8;
    const int64_t grow = m0 + xr;
    const bool xvalid = grow < M;
    int64_t sr0 = 0, sr1 = 0, sr2 = 0, sr3 = 0;
    if (xvalid) {
        sr0 = src.idx[0] ? (int64_t)src.idx[0][grow] : grow;
        if (nsrc > 1) sr1 = src.idx[1] ? (int64_t)src.idx[1][grow] : grow;
        if (nsrc > 2) sr2 = src.idx[2] ? (int64_t)src.idx[2][grow] : grow;
        if (nsrc > 3) sr3 = src.idx[3] ? (int64_t)src.idx[3][grow] : grow;
    }
    const float *__restrict__ wrow = W1 + (int64_t)tid * K;  // W1 row `tid` feeds LDS row `tid`

    float4 x0, x1, w0, w1, w2, w3, w4, w5, w6, w7;
#define GMLP_LOAD(kc)                                                                                    \
    do {                                                                                                 \
        const int j_ = (kc) >> 7, cc_ = (kc) & 127;                                                      \
        const float *sp_ = j_ == 0 ? src.ptr[0] + sr0 * MATRIS_D                                         \
                         : j_ == 1 ? src.ptr[1] + sr1 * MATRIS_D                                         \
                         : j_ == 2 ? src.ptr[2] + sr2 * MATRIS_D                                         \
                                   : src.ptr[3] + sr3 * MATRIS_D;                                        \
        if (xvalid) {                                                                                    \
            const float4 *xp_ = reinterpret_cast<const float4 *>(sp_ + cc_ + xc);                        \
            x0 = xp_[0];                                                                                 \
            x1 = xp_[1];                                                                                 \
        } else {                                                                                         \
            x0 = x1 = make_float4(0.f, 0.f, 0.f, 0.f);                                                   \
        }                                                                                                \
        const float4 *wp_ = reinterpret_cast<const float4 *>(wrow + (kc));                               \
        w0 = wp_[0]; w1 = wp_[1]; w2 = wp_[2]; w3 = wp_[3];                                              \
        w4 = wp_[4]; w5 = wp_[5]; w6 = wp_[6]; w7 = wp_[7];                                              \
    } while (0)

    v16f acc[2][2];
    zero_acc(acc);
    GMLP_LOAD(0);
    for (int kc = 0; kc < K; kc += BK) {
        __syncthreads();
        float4 *xs = reinterpret_cast<float4 *>(Xs + xr * LDX + xc);
        xs[0] = x0;
        xs[1] = x1;
        float4 *ws = reinterpret_cast<float4 *>(Ws + tid * LDW);
        ws[0] = w0; ws[1] = w1; ws[2] = w2; ws[3] = w3;
        ws[4] = w4; ws[5] = w5; ws[6] = w6; ws[7] = w7;
        __syncthreads();
        if (kc + BK < K) GMLP_LOAD(kc + BK);
        mfma_chunk<MODE, 2, 2>(acc, Xs, LDX, Ws + (wave * 64) * LDW, LDW, lane);
    }
#undef GMLP_LOAD
    __syncthreads();  // all waves are done with Xs / Ws before the tile overwrites them

    // p = acc + b1 -> LDS; copy p out with wide stores; h = SiLU(p) in place
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        const int col = wave * 64 + ct * 32 + l32;
        const float bias = b1[col];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int i = 0; i < 16; ++i) Ts[(rt * 32 + acc_row(i, h)) * LDH + col] = acc[rt][ct][i] + bias;
    }
    __syncthreads();
    if (save_p) store_tile256(Ts, save_p, m0, M, tid);
#pragma unroll
    for (int it = 0; it < (BM * 64) / 256; ++it) {
        const int q = it * 256 + tid;
        float4 *t = reinterpret_cast<float4 *>(Ts + (q >> 6) * LDH + (q & 63) * 4);
        float4 v = *t;
        v.x = silu_f(v.x); v.y = silu_f(v.y); v.z = silu_f(v.z); v.w = silu_f(v.w);
        *t = v;
    }
    __syncthreads();

    // GEMM2: wave w -> z columns [64w, 64w+64); block = w/2 (0 core, 1 gate)
    const int blk = wave >> 1;
    zero_acc(acc);
    gemm_lds_a_global_b<MODE, 2, 2, MATRIS_D>(acc, Ts + blk * MATRIS_D, LDH, W2 + (int64_t)(wave * 64) * MATRIS_D,
                                        MATRIS_D, lane);
    __syncthreads();  // every wave is done reading h
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        const int col = wave * 64 + ct * 32 + l32;
        const float bias = b2[col];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int i = 0; i < 16; ++i) Ts[(rt * 32 + acc_row(i, h)) * LDH + col] = acc[rt][ct][i] + bias;
    }
    __syncthreads();
    if (save_z) store_tile256(Ts, save_z, m0, M, tid);

    // row epilogue: wave w -> rows [16w, 16w+16); lane -> columns 2l, 2l+1 of each half
    const float2 wc = *reinterpret_cast<const float2 *>(norm_c + 2 * lane);
    const float2 wg = *reinterpret_cast<const float2 *>(norm_g + 2 * lane);
    for (int rr = 0; rr < BM / 4; ++rr) {
        const int row = wave * (BM / 4) + rr;
        const float2 zc = *reinterpret_cast<const float2 *>(Ts + row * LDH + 2 * lane);
        const float2 zg = *reinterpret_cast<const float2 *>(Ts + row * LDH + MATRIS_D + 2 * lane);
        const float rc = rsqrtf(wave_sum(zc.x * zc.x + zc.y * zc.y) * (1.0f / MATRIS_D) + eps);
        const float rg = rsqrtf(wave_sum(zg.x * zg.x + zg.y * zg.y) * (1.0f / MATRIS_D) + eps);
        float2 o;
        o.x = silu_f(zc.x * rc * wc.x) * sigm_f(zg.x * rg * wg.x);
        o.y = silu_f(zc.y * rc * wc.y) * sigm_f(zg.y * rg * wg.y);
        if (m0 + row < M) *reinterpret_cast<float2 *>(out + (m0 + row) * MATRIS_D + 2 * lane) = o;
    }
}

// ------------------------------------------------------------------------------------
// backward
// ------------------------------------------------------------------------------------
template <int MODE>
__global__ __launch_bounds__(256, 2) void gmlp_bwd_kernel(int64_t M, int K, const float *__restrict__ g_out,
                                                          const float *__restrict__ P, const float *__restrict__ Z,
                                                          const float *__restrict__ W1t,
                                                          const float *__restrict__ W2t,
                                                          const float *__restrict__ norm_c,
                                                          const float *__restrict__ norm_g, float eps,
                                                          float *__restrict__ g_x) {
    __shared__ __align__(16) float G[BM * LDH];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int h = lane >> 5, l32 = lane & 31;
    const int64_t m0 = (int64_t)blockIdx.x * BM;

    // phase 1: row-wise Jacobian of out = SiLU(RMS(z_c) w_c) * sigmoid(RMS(z_g) w_g).
    // Wave w owns rows [16w, 16w+16); lane owns columns (2l, 2l+1) of the core and gate
    // halves.  The next row's z / g_out are loaded before the current row is processed.
    const float2 wc = *reinterpret_cast<const float2 *>(norm_c + 2 * lane);
    const float2 wg = *reinterpret_cast<const float2 *>(norm_g + 2 * lane);
    const float2 zero2 = make_float2(0.f, 0.f);
    auto ld_row = [&](int rr, float2 &zc, float2 &zg, float2 &go) {
        const int64_t m = m0 + wave * (BM / 4) + rr;
        if (m < M) {
            zc = *reinterpret_cast<const float2 *>(Z + m * 256 + 2 * lane);
            zg = *reinterpret_cast<const float2 *>(Z + m * 256 + MATRIS_D + 2 * lane);
            go = *reinterpret_cast<const float2 *>(g_out + m * MATRIS_D + 2 * lane);
        } else {
            zc = zg = go = zero2;
        }
    };
    float2 zc, zg, go, zc_n, zg_n, go_n;
    ld_row(0, zc, zg, go);
#pragma unroll 1
    for (int rr = 0; rr < BM / 4; ++rr) {
        if (rr + 1 < BM / 4) ld_row(rr + 1, zc_n, zg_n, go_n);
        const int row = wave * (BM / 4) + rr;
        const float rc = rsqrtf(wave_sum(zc.x * zc.x + zc.y * zc.y) * (1.0f / MATRIS_D) + eps);
        const float rg = rsqrtf(wave_sum(zg.x * zg.x + zg.y * zg.y) * (1.0f / MATRIS_D) + eps);
        const float nc0 = zc.x * rc, nc1 = zc.y * rc, ng0 = zg.x * rg, ng1 = zg.y * rg;
        const float ac0 = nc0 * wc.x, ac1 = nc1 * wc.y, ag0 = ng0 * wg.x, ag1 = ng1 * wg.y;
        const float sc0 = sigm_f(ac0), sc1 = sigm_f(ac1);
        const float core0 = ac0 * sc0, core1 = ac1 * sc1;
        const float gate0 = sigm_f(ag0), gate1 = sigm_f(ag1);
        const float gnc0 = go.x * gate0 * (sc0 * (1.f + ac0 * (1.f - sc0))) * wc.x;
        const float gnc1 = go.y * gate1 * (sc1 * (1.f + ac1 * (1.f - sc1))) * wc.y;
        const float gng0 = go.x * core0 * (gate0 * (1.f - gate0)) * wg.x;
        const float gng1 = go.y * core1 * (gate1 * (1.f - gate1)) * wg.y;
        const float dc = wave_sum(gnc0 * nc0 + gnc1 * nc1) * (1.0f / MATRIS_D);
        const float dg = wave_sum(gng0 * ng0 + gng1 * ng1) * (1.0f / MATRIS_D);
        *reinterpret_cast<float2 *>(G + row * LDH + 2 * lane) = make_float2((gnc0 - nc0 * dc) * rc, (gnc1 - nc1 * dc) * rc);
        *reinterpret_cast<float2 *>(G + row * LDH + MATRIS_D + 2 * lane) =
            make_float2((gng0 - ng0 * dg) * rg, (gng1 - ng1 * dg) * rg);
        zc = zc_n; zg = zg_n; go = go_n;
    }
    __syncthreads();

    // phase 2: g_h = g_z W2 (block diagonal); wave w -> columns [64w, 64w+64)
    const int blk = wave >> 1;
    v16f acc[2][2];
    zero_acc(acc);
    gemm_lds_a_global_b<MODE, 2, 2, MATRIS_D>(acc, G + blk * MATRIS_D, LDH,
                                        W2t + (int64_t)((wave & 1) * 64) * 256 + blk * MATRIS_D, 256, lane);
    // g_p = g_h * SiLU'(p)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        const int col = wave * 64 + ct * 32 + l32;
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int row = rt * 32 + acc_row(i, h);
                const float p = (m0 + row < M) ? P[(m0 + row) * 256 + col] : 0.f;
                acc[rt][ct][i] *= dsilu_f(p);
            }
    }
    __syncthreads();  // every wave is done reading g_z
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        const int col = wave * 64 + ct * 32 + l32;
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int i = 0; i < 16; ++i) G[(rt * 32 + acc_row(i, h)) * LDH + col] = acc[rt][ct][i];
    }
    __syncthreads();

    // phase 3: g_x = g_p W1 over 128-column blocks; wave w -> 32 columns of each block
    for (int cb = 0; cb < K; cb += MATRIS_D) {
        v16f a2[2][1];
        zero_acc(a2);
        const int col0 = cb + wave * 32;
        gemm_lds_a_global_b<MODE, 2, 1, 256>(a2, G, LDH, W1t + (int64_t)col0 * 256, 256, lane);
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int row = rt * 32 + acc_row(i, h);
                if (m0 + row < M) g_x[(m0 + row) * K + col0 + l32] = a2[rt][0][i];
            }
    }
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

extern "C" int matris_gmlp_fwd(int64_t m, int n_src, const float *const *src_host,
                               const int32_t *const *src_idx_host, const float *w1, const float *b1, const float *w2,
                               const float *b2, const float *norm_c, const float *norm_g, float eps, float *out,
                               float *save_p, float *save_z, int mode, void *stream) {
    if (mode != 0 && mode != 3 && mode != 6) return MATRIS_E_ARG;
    if (m < 0 || n_src < 1 || n_src > 4 || !src_host || !w1 || !b1 || !w2 || !b2 || !norm_c || !norm_g || !out)
        return MATRIS_E_ARG;
    if (m == 0) return 0;
    GmlpSrc s;
    for (int j = 0; j < 4; ++j) {
        s.ptr[j] = j < n_src ? src_host[j] : nullptr;
        s.idx[j] = (j < n_src && src_idx_host) ? src_idx_host[j] : nullptr;
        if (j < n_src && (!s.ptr[j] || !aligned16(s.ptr[j]))) return MATRIS_E_ARG;
    }
    if (!aligned16(w1) || !aligned16(w2)) return MATRIS_E_ARG;
    const dim3 grid(matris_blocks(m, BM));
    hipStream_t st = (hipStream_t)stream;
    if (mode == 0)
        gmlp_fwd_kernel<0><<<grid, 256, 0, st>>>(m, n_src, s, w1, b1, w2, b2, norm_c, norm_g, eps, out, save_p, save_z);
    else if (mode == 3)
        gmlp_fwd_kernel<3><<<grid, 256, 0, st>>>(m, n_src, s, w1, b1, w2, b2, norm_c, norm_g, eps, out, save_p, save_z);
    else
        gmlp_fwd_kernel<6><<<grid, 256, 0, st>>>(m, n_src, s, w1, b1, w2, b2, norm_c, norm_g, eps, out, save_p, save_z);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_gmlp_bwd(int64_t m, int k, const float *g_out, const float *p, const float *z, const float *w1t,
                               const float *w2t, const float *norm_c, const float *norm_g, float eps, float *g_x,
                               int mode, void *stream) {
    if (mode != 0 && mode != 3 && mode != 6) return MATRIS_E_ARG;
    if (m < 0 || k < MATRIS_D || k > 4 * MATRIS_D || (k % MATRIS_D) || !g_out || !p || !z || !w1t || !w2t ||
        !norm_c || !norm_g || !g_x)
        return MATRIS_E_ARG;
    if (m == 0) return 0;
    if (!aligned16(w1t) || !aligned16(w2t)) return MATRIS_E_ARG;
    const dim3 grid(matris_blocks(m, BM));
    hipStream_t st = (hipStream_t)stream;
    if (mode == 0)
        gmlp_bwd_kernel<0><<<grid, 256, 0, st>>>(m, k, g_out, p, z, w1t, w2t, norm_c, norm_g, eps, g_x);
    else if (mode == 3)
        gmlp_bwd_kernel<3><<<grid, 256, 0, st>>>(m, k, g_out, p, z, w1t, w2t, norm_c, norm_g, eps, g_x);
    else
        gmlp_bwd_kernel<6><<<grid, 256, 0, st>>>(m, k, g_out, p, z, w1t, w2t, norm_c, norm_g, eps, g_x);
    MATRIS_CHECK_LAUNCH();
    return 0;
}
