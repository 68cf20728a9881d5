// Fused gated MLP (GatedMLP with RMSNorm, SiLU core, sigmoid gate) on gfx950 MFMA.
//
//   x    = concat_j src_j[idx_j[m]]                         [BM, K]   (gathered on load)
//   p    = x W1^T + b1                                      [BM, 256] (core | gate)
//   h    = SiLU(p)
//   z    = [h_c W2c^T + b2c | h_g W2g^T + b2g]              [BM, 256]
//   out  = SiLU(RMS(z_c) * w_c) * sigmoid(RMS(z_g) * w_g)   [BM, 128]
//
// Work-group = 4 wave64s, BM = 64 rows.  GEMM1 streams K in 32-wide chunks: each thread
// gathers 8 values of one row of the next chunk, converts them once into an operand
// fragment (mma.h) and writes it to a double-buffered LDS chunk, so one barrier per
// chunk suffices and no wave converts A values itself; the pre-packed W1 fragments come
// straight from global (L2) one k-block ahead.  Each wave owns 64 output columns (2x2
// grid of 32x32 tiles).  The [64, 256] result tile goes through LDS: p is copied out
// with 16-byte row stores, h = SiLU(p) stays in LDS as GEMM2's A operand, z returns to
// LDS, is copied out, and a row-per-wave epilogue applies RMSNorm, SiLU, sigmoid and
// the product with 512-byte row stores.  p and z are written for the backward.
//
// Backward (input gradients only) recomputes the norm/activation Jacobians row-wise
// from z, then runs g_h = g_z W2 and g_x = (g_h * SiLU'(p)) W1 through the same MFMA
// tiling, with packed transposed weights as B operands.
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
                                                          const uint4 *__restrict__ W1, const float *__restrict__ b1,
                                                          const uint4 *__restrict__ W2, const float *__restrict__ b2,
                                                          const float *__restrict__ norm_c,
                                                          const float *__restrict__ norm_g, float eps,
                                                          float *__restrict__ out, float *__restrict__ save_p,
                                                          float *__restrict__ save_z,
                                                          const float *__restrict__ res_src,
                                                          const float *__restrict__ res_w,
                                                          float *__restrict__ res_out) {
    constexpr int NPL = Npl<MODE>::v;
    constexpr int CHUNK = 2 * 2 * NPL * 64;  // uint4 per LDS chunk: [rt 2][kb 2][plane][lane]
    __shared__ __align__(16) float smem[BM * LDH];
    uint4 *Xp = reinterpret_cast<uint4 *>(smem);  // two chunk buffers (<= 24 KB)
    float *Ts = smem;                             // [BM, 256] tile: p, then h, then z

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int64_t m0 = (int64_t)blockIdx.x * BM;
    const int KB = nsrc * (MATRIS_D / 16);  // k-blocks of W1
    const int nchunk = nsrc * (MATRIS_D / 32);

    // gather assignment: thread -> (row xr, 8 columns at 8*xq) of each 32-wide chunk,
    // which is exactly the fragment (tile xr/32, k-block xq/2, lane xr%32 + 32*(xq&1)).
    const int xr = tid >> 2, xq = tid & 3, xc = xq * 8;
    const int xslot = ((xr >> 5) * 2 + (xq >> 1)) * NPL * 64 + (xr & 31) + 32 * (xq & 1);
    // Rows past M read row M-1 (their results are never stored), so every prefetch load
    // below is unconditional and the compiler can count outstanding loads exactly
    // instead of draining them all (a conditional load forces s_waitcnt vmcnt(0)).
    const int64_t grow = min(m0 + xr, M - 1);
    int64_t sr0 = 0, sr1 = 0, sr2 = 0, sr3 = 0;
    sr0 = src.idx[0] ? (int64_t)src.idx[0][grow] : grow;
    if (nsrc > 1) sr1 = src.idx[1] ? (int64_t)src.idx[1][grow] : grow;
    if (nsrc > 2) sr2 = src.idx[2] ? (int64_t)src.idx[2][grow] : grow;
    if (nsrc > 3) sr3 = src.idx[3] ? (int64_t)src.idx[3][grow] : grow;

    float4 x0, x1;
#define GMLP_LOADX(kc)                                                                                   \
    do {                                                                                                 \
        const int j_ = (kc) >> 7, cc_ = (kc) & 127;                                                      \
        const float *sp_ = j_ == 0 ? src.ptr[0] + sr0 * MATRIS_D                                         \
                         : j_ == 1 ? src.ptr[1] + sr1 * MATRIS_D                                         \
                         : j_ == 2 ? src.ptr[2] + sr2 * MATRIS_D                                         \
                                   : src.ptr[3] + sr3 * MATRIS_D;                                        \
        const float4 *xp_ = reinterpret_cast<const float4 *>(sp_ + cc_ + xc);                            \
        x0 = xp_[0];                                                                                     \
        x1 = xp_[1];                                                                                     \
    } while (0)
#define GMLP_STOREX(buf)                                                                                 \
    do {                                                                                                 \
        Frag<MODE> f_;                                                                                   \
        make_frag<MODE>(f_, x0, x1);                                                                     \
        _Pragma("unroll") for (int pl_ = 0; pl_ < NPL; ++pl_) Xp[(buf) * CHUNK + xslot + pl_ * 64] = f_.p[pl_]; \
    } while (0)

    v16f acc[2][2];
    zero_acc(acc);
    Frag<MODE> bcur[2], bnxt[2];
    load_bfrags<MODE, 2>(bcur, W1, 2 * wave, KB, 0, lane);
    GMLP_LOADX(0);
    GMLP_STOREX(0);
    __syncthreads();
#pragma unroll 1
    for (int c = 0; c < nchunk; ++c) {
        GMLP_LOADX(min(c + 1, nchunk - 1) * 32);  // the last iteration reloads its own chunk
        const uint4 *xb = Xp + (c & 1) * CHUNK;
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            const int kb = 2 * c + sub;
            load_bfrags<MODE, 2>(bnxt, W1, 2 * wave, KB, min(kb + 1, KB - 1), lane);
            __builtin_amdgcn_sched_barrier(0);  // issue the prefetches before this step's MFMAs
            Frag<MODE> a[2];
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                for (int pl = 0; pl < NPL; ++pl) a[rt].p[pl] = xb[((rt * 2 + sub) * NPL + pl) * 64 + lane];
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) mma_frag<MODE>(acc[rt][ct], a[rt], bcur[ct]);
            bcur[0] = bnxt[0];
            bcur[1] = bnxt[1];
        }
        GMLP_STOREX((c + 1) & 1);  // unread after the last chunk
        __syncthreads();
    }
#undef GMLP_LOADX
#undef GMLP_STOREX

    // p = acc + b1 -> LDS; copy p out with wide stores; h = SiLU(p) in place
    acc_to_lds<2>(acc, Ts, LDH, wave * 64, lane, b1);
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
    gemm_lds_packed<MODE, 2, 2, MATRIS_D / 16>(acc, Ts + blk * MATRIS_D, LDH, W2, 2 * wave, MATRIS_D / 16, 0, lane);
    __syncthreads();  // every wave is done reading h
    acc_to_lds<2>(acc, Ts, LDH, wave * 64, lane, b2);
    __syncthreads();
    if (save_z) store_tile256(Ts, save_z, m0, M, tid);

    // row epilogue: wave w -> rows [16w, 16w+16); lane -> columns 2l, 2l+1 of each half;
    // optional residual output res_out = out + res_w * res_src
    const float2 wc = *reinterpret_cast<const float2 *>(norm_c + 2 * lane);
    const float2 wg = *reinterpret_cast<const float2 *>(norm_g + 2 * lane);
    const float2 rw = res_out ? *reinterpret_cast<const float2 *>(res_w + 2 * lane) : make_float2(0.f, 0.f);
    for (int rr = 0; rr < BM / 4; ++rr) {
        const int row = wave * (BM / 4) + rr;
        const float2 zc = *reinterpret_cast<const float2 *>(Ts + row * LDH + 2 * lane);
        const float2 zg = *reinterpret_cast<const float2 *>(Ts + row * LDH + MATRIS_D + 2 * lane);
        const float rc = rsqrtf(wave_sum(zc.x * zc.x + zc.y * zc.y) * (1.0f / MATRIS_D) + eps);
        const float rg = rsqrtf(wave_sum(zg.x * zg.x + zg.y * zg.y) * (1.0f / MATRIS_D) + eps);
        float2 o;
        o.x = silu_f(zc.x * rc * wc.x) * sigm_f(zg.x * rg * wg.x);
        o.y = silu_f(zc.y * rc * wc.y) * sigm_f(zg.y * rg * wg.y);
        if (m0 + row < M) {
            *reinterpret_cast<float2 *>(out + (m0 + row) * MATRIS_D + 2 * lane) = o;
            if (res_out) {
                const float2 x = *reinterpret_cast<const float2 *>(res_src + (m0 + row) * MATRIS_D + 2 * lane);
                *reinterpret_cast<float2 *>(res_out + (m0 + row) * MATRIS_D + 2 * lane) =
                    make_float2(o.x + rw.x * x.x, o.y + rw.y * x.y);
            }
        }
    }
}

// ------------------------------------------------------------------------------------
// backward
// ------------------------------------------------------------------------------------
// Store a wave's [64, 32*NCT] accumulators to rows of dst (row stride ld) at column
// col + ct*32 + lane%32, rows below nrows only.
template <int NCT>
__device__ __forceinline__ void store_acc_rows(const v16f (&acc)[2][NCT], float *__restrict__ dst, int ld, int col,
                                               int nrows, int lane) {
    const int h = lane >> 5, l32 = lane & 31;
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int row = rt * 32 + acc_row(i, h);
                if (row < nrows) dst[row * ld + col + ct * 32 + l32] = acc[rt][ct][i];
            }
}

template <int MODE>
__global__ __launch_bounds__(256, 2) void gmlp_bwd_kernel(int64_t M, int K, const float *__restrict__ g_out,
                                                          const float *__restrict__ P, const float *__restrict__ Z,
                                                          const uint4 *__restrict__ W1t,
                                                          const uint4 *__restrict__ W2t,
                                                          const float *__restrict__ norm_c,
                                                          const float *__restrict__ norm_g, float eps,
                                                          float *__restrict__ g_x, float *__restrict__ g_x0,
                                                          int acc0, const float *__restrict__ res_w) {
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

    // phase 2: g_h = g_z W2 (block diagonal); wave w -> columns [64w, 64w+64).  W2t is
    // packed from [W2c^T ; W2g^T] ([256, 128]), so output tile nt reads block nt / 4.
    const int blk = wave >> 1;
    v16f acc[2][2];
    zero_acc(acc);
    gemm_lds_packed<MODE, 2, 2, MATRIS_D / 16>(acc, G + blk * MATRIS_D, LDH, W2t, 2 * wave, MATRIS_D / 16, 0, lane);
    // g_p = g_h * SiLU'(p); rows past M read row 0 of the tile (their results are unused)
    const int nrows = (int)min((int64_t)BM, M - m0);
    const float *__restrict__ Pt = P + m0 * 256;
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        const int col = wave * 64 + ct * 32 + l32;
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int row = rt * 32 + acc_row(i, h);
                acc[rt][ct][i] *= dsilu_f(Pt[(row < nrows ? row : 0) * 256 + col]);
            }
    }
    __syncthreads();  // every wave is done reading g_z
    acc_to_lds<2>(acc, G, LDH, wave * 64, lane);
    __syncthreads();

    // phase 3: g_x = g_p W1.  W1t is W1^T ([K, 256]) packed: output tile nt = column / 32,
    // 16 k-blocks.  Passes of 256 columns (wave w -> 64 columns, 2 tiles, so each A
    // fragment conversion feeds two tiles) and, if K % 256, one 128-column pass (32 per
    // wave), in descending column order so that the pass holding source 0 (columns
    // [0, 128)) ends the kernel.  Source 0's gradient goes to g_x0 when given (added to
    // its contents if acc0) and gains res_w * g_out when res_w is given; that epilogue
    // runs row-wise through LDS once G is no longer read.  Other columns go straight to
    // g_x (row stride K - 128 with g_x0, K without).
    const int coff = g_x0 ? MATRIS_D : 0;
    const int ldr = K - coff;
    float *__restrict__ gxr = g_x ? g_x + m0 * ldr : nullptr;
    const bool epi0 = g_x0 != nullptr || res_w != nullptr;
    if (K % 256) {
        const int cb = K - MATRIS_D;
        v16f a2[2][1];
        zero_acc(a2);
        const int col0 = cb + wave * 32;
        gemm_lds_packed<MODE, 2, 1, 256 / 16>(a2, G, LDH, W1t, col0 / 32, 256 / 16, 0, lane);
        if (cb > 0 || !epi0) store_acc_rows<1>(a2, gxr, ldr, col0 - coff, nrows, lane);
        if (cb == 0 && epi0) {  // K == 128: every wave holds source-0 columns
            __syncthreads();
            acc_to_lds<1>(a2, G, LDH, col0, lane);
        }
    }
    for (int cb = (K / 256 - 1) * 256; cb >= 0; cb -= 256) {
        v16f a2[2][2];
        zero_acc(a2);
        const int col0 = cb + wave * 64;
        gemm_lds_packed<MODE, 2, 2, 256 / 16>(a2, G, LDH, W1t, col0 / 32, 256 / 16, 0, lane);
        if (col0 >= MATRIS_D || !epi0) store_acc_rows<2>(a2, gxr, ldr, col0 - coff, nrows, lane);
        if (cb == 0 && epi0) {
            __syncthreads();  // all waves are done reading G
            if (col0 < MATRIS_D) acc_to_lds<2>(a2, G, LDH, col0, lane);
        }
    }
    if (epi0) {
        __syncthreads();
        float *__restrict__ gx0 = g_x0 ? g_x0 + m0 * MATRIS_D : gxr;
        const int ld0 = g_x0 ? MATRIS_D : ldr;
        const float *__restrict__ got = g_out + m0 * MATRIS_D;
#pragma unroll
        for (int it = 0; it < (BM * 32) / 256; ++it) {
            const int q = it * 256 + tid;
            const int r = q >> 5, c4 = (q & 31) * 4;
            if (r < nrows) {
                float4 v = *reinterpret_cast<const float4 *>(G + r * LDH + c4);
                if (res_w) {
                    const float4 w = *reinterpret_cast<const float4 *>(res_w + c4);
                    const float4 x = *reinterpret_cast<const float4 *>(got + r * MATRIS_D + c4);
                    v.x += w.x * x.x; v.y += w.y * x.y; v.z += w.z * x.z; v.w += w.w * x.w;
                }
                float4 *o = reinterpret_cast<float4 *>(gx0 + r * ld0 + c4);
                if (acc0) {
                    const float4 p0 = *o;
                    v.x += p0.x; v.y += p0.y; v.z += p0.z; v.w += p0.w;
                }
                *o = v;
            }
        }
    }
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

extern "C" int matris_gmlp_fwd(int64_t m, int n_src, const float *const *src_host,
                               const int32_t *const *src_idx_host, const void *w1p, const float *b1, const void *w2p,
                               const float *b2, const float *norm_c, const float *norm_g, float eps, float *out,
                               float *save_p, float *save_z, const float *res_src, const float *res_w,
                               float *res_out, int mode, void *stream) {
    if (mode != 0 && mode != 3 && mode != 6) return MATRIS_E_ARG;
    if (m < 0 || n_src < 1 || n_src > 4 || !src_host || !w1p || !b1 || !w2p || !b2 || !norm_c || !norm_g || !out)
        return MATRIS_E_ARG;
    if (m == 0) return 0;
    GmlpSrc s;
    for (int j = 0; j < 4; ++j) {
        s.ptr[j] = j < n_src ? src_host[j] : nullptr;
        s.idx[j] = (j < n_src && src_idx_host) ? src_idx_host[j] : nullptr;
        if (j < n_src && (!s.ptr[j] || !aligned16(s.ptr[j]))) return MATRIS_E_ARG;
    }
    if (!aligned16(w1p) || !aligned16(w2p)) return MATRIS_E_ARG;
    if (res_out && (!res_src || !res_w)) return MATRIS_E_ARG;
    const dim3 grid(matris_blocks(m, BM));
    hipStream_t st = (hipStream_t)stream;
    const uint4 *w1 = (const uint4 *)w1p, *w2 = (const uint4 *)w2p;
    if (mode == 0)
        gmlp_fwd_kernel<0><<<grid, 256, 0, st>>>(m, n_src, s, w1, b1, w2, b2, norm_c, norm_g, eps, out, save_p, save_z,
                                                 res_src, res_w, res_out);
    else if (mode == 3)
        gmlp_fwd_kernel<3><<<grid, 256, 0, st>>>(m, n_src, s, w1, b1, w2, b2, norm_c, norm_g, eps, out, save_p, save_z,
                                                 res_src, res_w, res_out);
    else
        gmlp_fwd_kernel<6><<<grid, 256, 0, st>>>(m, n_src, s, w1, b1, w2, b2, norm_c, norm_g, eps, out, save_p, save_z,
                                                 res_src, res_w, res_out);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_gmlp_bwd(int64_t m, int k, const float *g_out, const float *p, const float *z, const void *w1tp,
                               const void *w2tp, const float *norm_c, const float *norm_g, float eps, float *g_x,
                               float *g_x0, int acc0, const float *res_w, int mode, void *stream) {
    if (mode != 0 && mode != 3 && mode != 6) return MATRIS_E_ARG;
    if (m < 0 || k < MATRIS_D || k > 4 * MATRIS_D || (k % MATRIS_D) || !g_out || !p || !z || !w1tp || !w2tp ||
        !norm_c || !norm_g || (!g_x && !(g_x0 && k == MATRIS_D)))
        return MATRIS_E_ARG;
    if (m == 0) return 0;
    if (!aligned16(w1tp) || !aligned16(w2tp)) return MATRIS_E_ARG;
    if (acc0 && !g_x0) return MATRIS_E_ARG;
    const dim3 grid(matris_blocks(m, BM));
    hipStream_t st = (hipStream_t)stream;
    const uint4 *w1t = (const uint4 *)w1tp, *w2t = (const uint4 *)w2tp;
    if (mode == 0)
        gmlp_bwd_kernel<0><<<grid, 256, 0, st>>>(m, k, g_out, p, z, w1t, w2t, norm_c, norm_g, eps, g_x, g_x0,
                                                 acc0, res_w);
    else if (mode == 3)
        gmlp_bwd_kernel<3><<<grid, 256, 0, st>>>(m, k, g_out, p, z, w1t, w2t, norm_c, norm_g, eps, g_x, g_x0,
                                                 acc0, res_w);
    else
        gmlp_bwd_kernel<6><<<grid, 256, 0, st>>>(m, k, g_out, p, z, w1t, w2t, norm_c, norm_g, eps, g_x, g_x0,
                                                 acc0, res_w);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

// ------------------------------------------------------------------------------------
// weight packing: [n, k] row-major fp32 (rows = output columns of the GEMM) -> fragment
// planes, one thread per (tile, k-block, lane)
// ------------------------------------------------------------------------------------
template <int MODE>
__global__ void pack_b_kernel(int64_t n, int64_t k, const float *__restrict__ w, uint4 *__restrict__ out) {
    constexpr int NPL = Npl<MODE>::v;
    const int64_t KB = k / 16;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // (nt * KB + kb) * 64 + lane
    if (t >= n / 32 * KB * 64) return;
    const int lane = (int)(t & 63);
    const int64_t ntkb = t >> 6, nt = ntkb / KB, kb = ntkb % KB;
    const float *r = w + (nt * 32 + (lane & 31)) * k + kb * 16 + (lane >> 5) * 8;
    Frag<MODE> f;
    make_frag<MODE>(f, *reinterpret_cast<const float4 *>(r), *reinterpret_cast<const float4 *>(r + 4));
#pragma unroll
    for (int pl = 0; pl < NPL; ++pl) out[(ntkb * NPL + pl) * 64 + lane] = f.p[pl];
}

extern "C" size_t matris_pack_b_bytes(int64_t n, int64_t k, int mode) { return packed_b_bytes(n, k, mode); }

extern "C" int matris_pack_b(int64_t n, int64_t k, const float *w, int mode, void *out, void *stream) {
    if (mode != 0 && mode != 3 && mode != 6) return MATRIS_E_ARG;
    if (n < 0 || k < 0 || (n % 32) || (k % 16) || !w || !out || !aligned16(w) || !aligned16(out)) return MATRIS_E_ARG;
    const int64_t threads = n / 32 * (k / 16) * 64;
    if (threads == 0) return 0;
    const dim3 grid(matris_blocks(threads, 256));
    hipStream_t st = (hipStream_t)stream;
    if (mode == 0)
        pack_b_kernel<0><<<grid, 256, 0, st>>>(n, k, w, (uint4 *)out);
    else if (mode == 3)
        pack_b_kernel<3><<<grid, 256, 0, st>>>(n, k, w, (uint4 *)out);
    else
        pack_b_kernel<6><<<grid, 256, 0, st>>>(n, k, w, (uint4 *)out);
    MATRIS_CHECK_LAUNCH();
    return 0;
}
