// Segmented reductions, gathers and the fused segment attention (softmax by target and
// by source, alpha * e', both segment sums) for gfx950.
//
// All of these are HBM-bound.  Layout: one 64-lane wavefront per segment (or per row),
// each lane owning two adjacent columns of a 128-wide fp32 row, so every row access is
// one coalesced 512-byte transaction.  Reductions run in CSR order inside the wave:
// deterministic, no float atomics.
#include "common.h"

#define WAVES_PER_BLOCK 4

__device__ __forceinline__ float2 ld2(const float *p) { return *reinterpret_cast<const float2 *>(p); }
__device__ __forceinline__ void st2(float *p, float2 v) { *reinterpret_cast<float2 *>(p) = v; }

// ------------------------------------------------------------------------------------
// segment sum (CSR)
// ------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void seg_sum_kernel(const float *__restrict__ x, int64_t ldx, int64_t col_off,
                                                      const int32_t *__restrict__ rowptr,
                                                      const int32_t *__restrict__ perm, int64_t n_seg, float scale,
                                                      int accumulate, float *__restrict__ out) {
    int64_t s = (int64_t)blockIdx.x * WAVES_PER_BLOCK + (threadIdx.x >> 6);
    if (s >= n_seg) return;
    const int c = 2 * (threadIdx.x & 63);
    const int b = rowptr[s], e = rowptr[s + 1];
    const float *xc = x + col_off + c;
    float2 acc = make_float2(0.f, 0.f);
    int i = b;
    for (; i + 4 <= e; i += 4) {
        int64_t r0 = perm ? perm[i] : i, r1 = perm ? perm[i + 1] : i + 1;
        int64_t r2 = perm ? perm[i + 2] : i + 2, r3 = perm ? perm[i + 3] : i + 3;
        float2 v0 = ld2(xc + r0 * ldx), v1 = ld2(xc + r1 * ldx);
        float2 v2 = ld2(xc + r2 * ldx), v3 = ld2(xc + r3 * ldx);
        acc.x += v0.x; acc.y += v0.y;
        acc.x += v1.x; acc.y += v1.y;
        acc.x += v2.x; acc.y += v2.y;
        acc.x += v3.x; acc.y += v3.y;
    }
    for (; i < e; ++i) {
        int64_t r = perm ? perm[i] : i;
        float2 v = ld2(xc + r * ldx);
        acc.x += v.x; acc.y += v.y;
    }
    acc.x *= scale;
    acc.y *= scale;
    float *o = out + s * MATRIS_D + c;
    if (accumulate) {
        float2 p = ld2(o);
        acc.x += p.x;
        acc.y += p.y;
    }
    st2(o, acc);
}

extern "C" int matris_seg_sum(const float *x, int64_t ldx, int64_t col_off, const int32_t *rowptr,
                              const int32_t *perm, int64_t n_seg, float scale, int accumulate, float *out,
                              void *stream) {
    if (n_seg < 0 || !rowptr || !out || ldx < MATRIS_D || col_off < 0 || col_off + MATRIS_D > ldx ||
        (ldx % 2) || (col_off % 2))
        return MATRIS_E_ARG;
    if (n_seg == 0) return 0;
    seg_sum_kernel<<<matris_blocks(n_seg, WAVES_PER_BLOCK), 256, 0, (hipStream_t)stream>>>(
        x, ldx, col_off, rowptr, perm, n_seg, scale, accumulate, out);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

// ------------------------------------------------------------------------------------
// row gather
// ------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gather_rows_kernel(const float *__restrict__ src,
                                                          const int32_t *__restrict__ idx, int64_t n_rows,
                                                          float scale, int accumulate, float *__restrict__ out) {
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // one float4 per thread
    int64_t r = t >> 5;
    if (r >= n_rows) return;
    int q = (int)(t & 31) * 4;
    int64_t sr = idx ? idx[r] : r;
    float4 v = *reinterpret_cast<const float4 *>(src + sr * MATRIS_D + q);
    v.x *= scale; v.y *= scale; v.z *= scale; v.w *= scale;
    float4 *o = reinterpret_cast<float4 *>(out + r * MATRIS_D + q);
    if (accumulate) {
        float4 p = *o;
        v.x += p.x; v.y += p.y; v.z += p.z; v.w += p.w;
    }
    *o = v;
}

extern "C" int matris_gather_rows(const float *src, const int32_t *idx, int64_t n_rows, float scale,
                                  int accumulate, float *out, void *stream) {
    if (n_rows < 0 || !src || !out) return MATRIS_E_ARG;
    if (n_rows == 0) return 0;
    gather_rows_kernel<<<matris_blocks(n_rows * 32, 256), 256, 0, (hipStream_t)stream>>>(src, idx, n_rows, scale,
                                                                                      accumulate, out);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

// ------------------------------------------------------------------------------------
// segment attention forward: one wave per (segment, side); online softmax per column
// ------------------------------------------------------------------------------------
__device__ __forceinline__ void online_update(float2 a, float2 ev, float2 &m, float2 &s, float2 &acc) {
    float mx = fmaxf(m.x, a.x), my = fmaxf(m.y, a.y);
    float cx = expf(m.x - mx), cy = expf(m.y - my);  // 0 on the first row (m = -inf)
    float wx = expf(a.x - mx), wy = expf(a.y - my);
    s.x = s.x * cx + wx;
    s.y = s.y * cy + wy;
    acc.x = acc.x * cx + wx * ev.x;
    acc.y = acc.y * cy + wy * ev.y;
    m.x = mx;
    m.y = my;
}

// HAS_AIDX distinguishes the atom-graph launch (alpha rows read through d2u) from the
// line-graph launch, and gives them separate kernel symbols in profiles.
template <bool HAS_AIDX>
__global__ __launch_bounds__(256) void attn_fwd_kernel(int64_t n_seg, const float *__restrict__ alpha_t,
                                                       const float *__restrict__ alpha_s, int64_t lda,
                                                       const int32_t *__restrict__ aidx,
                                                       const float *__restrict__ e, const int32_t *__restrict__ t_ptr,
                                                       const int32_t *__restrict__ t_perm,
                                                       const int32_t *__restrict__ s_ptr,
                                                       const int32_t *__restrict__ s_perm, float *__restrict__ y_t,
                                                       float *__restrict__ y_s, float *__restrict__ lse_t,
                                                       float *__restrict__ lse_s) {
    int64_t w = (int64_t)blockIdx.x * WAVES_PER_BLOCK + (threadIdx.x >> 6);
    if (w >= 2 * n_seg) return;
    const bool src_side = w >= n_seg;
    const int64_t seg = src_side ? w - n_seg : w;
    const int32_t *ptr = src_side ? s_ptr : t_ptr;
    const int32_t *perm = src_side ? s_perm : t_perm;
    const float *alpha = src_side ? alpha_s : alpha_t;
    const int c = 2 * (threadIdx.x & 63);
    const int b = ptr[seg], end = ptr[seg + 1];
    float2 m = make_float2(-INFINITY, -INFINITY), s = make_float2(0.f, 0.f), acc = make_float2(0.f, 0.f);
    int i = b;
    for (; i + 2 <= end; i += 2) {
        int64_t r0 = perm ? perm[i] : i, r1 = perm ? perm[i + 1] : i + 1;
        int64_t a0 = HAS_AIDX ? aidx[r0] : r0, a1 = HAS_AIDX ? aidx[r1] : r1;
        float2 x0 = ld2(alpha + a0 * lda + c), x1 = ld2(alpha + a1 * lda + c);
        float2 e0 = ld2(e + r0 * MATRIS_D + c), e1 = ld2(e + r1 * MATRIS_D + c);
        online_update(x0, e0, m, s, acc);
        online_update(x1, e1, m, s, acc);
    }
    if (i < end) {
        int64_t r0 = perm ? perm[i] : i;
        int64_t a0 = HAS_AIDX ? aidx[r0] : r0;
        online_update(ld2(alpha + a0 * lda + c), ld2(e + r0 * MATRIS_D + c), m, s, acc);
    }
    float2 y = make_float2(0.f, 0.f), l = make_float2(0.f, 0.f);
    if (end > b) {
        y = make_float2(acc.x / s.x, acc.y / s.y);
        l = make_float2(m.x + logf(s.x), m.y + logf(s.y));
    }
    st2((src_side ? y_s : y_t) + seg * MATRIS_D + c, y);
    st2((src_side ? lse_s : lse_t) + seg * MATRIS_D + c, l);
}

extern "C" int matris_attn_fwd(int64_t n_rows, int64_t n_seg, const float *alpha_t, const float *alpha_s,
                               int64_t lda, const int32_t *alpha_idx, const float *e, const int32_t *t_ptr,
                               const int32_t *t_perm, const int32_t *s_ptr, const int32_t *s_perm, float *y_t,
                               float *y_s, float *lse_t, float *lse_s, void *stream) {
    if (n_rows < 0 || n_seg < 0 || lda < MATRIS_D || (lda % 2) || !t_ptr || !s_ptr || !y_t || !y_s || !lse_t ||
        !lse_s)
        return MATRIS_E_ARG;
    if (n_seg == 0) return 0;
    if (alpha_idx)
        attn_fwd_kernel<true><<<matris_blocks(2 * n_seg, WAVES_PER_BLOCK), 256, 0, (hipStream_t)stream>>>(
            n_seg, alpha_t, alpha_s, lda, alpha_idx, e, t_ptr, t_perm, s_ptr, s_perm, y_t, y_s, lse_t, lse_s);
    else
        attn_fwd_kernel<false><<<matris_blocks(2 * n_seg, WAVES_PER_BLOCK), 256, 0, (hipStream_t)stream>>>(
            n_seg, alpha_t, alpha_s, lda, nullptr, e, t_ptr, t_perm, s_ptr, s_perm, y_t, y_s, lse_t, lse_s);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

// ------------------------------------------------------------------------------------
// segment attention backward: one wave per row
//   p = exp(alpha - lse[seg]);  g_e = p_t g_yt + p_s g_ys;
//   g_alpha = p g_y (e - y)      (column-wise softmax Jacobian)
// ------------------------------------------------------------------------------------
template <bool HAS_AIDX>
__global__ __launch_bounds__(256) void attn_bwd_kernel(
    int64_t n_rows, const float *__restrict__ alpha_t, const float *__restrict__ alpha_s, int64_t lda,
    const int32_t *__restrict__ aidx, const float *__restrict__ e, const int32_t *__restrict__ t_idx,
    const int32_t *__restrict__ s_idx, const float *__restrict__ y_t, const float *__restrict__ y_s,
    const float *__restrict__ lse_t, const float *__restrict__ lse_s, const float *__restrict__ g_yt,
    const float *__restrict__ g_ys, int64_t ldgy, float *__restrict__ g_alpha_t, float *__restrict__ g_alpha_s,
    float *__restrict__ g_e, const float *__restrict__ g_e_base) {
    int64_t r = (int64_t)blockIdx.x * WAVES_PER_BLOCK + (threadIdx.x >> 6);
    if (r >= n_rows) return;
    const int c = 2 * (threadIdx.x & 63);
    const int64_t a = HAS_AIDX ? aidx[r] : r;
    const int64_t t = t_idx[r], s = s_idx[r];
    float2 at = ld2(alpha_t + a * lda + c), as = ld2(alpha_s + a * lda + c);
    float2 ev = ld2(e + r * MATRIS_D + c);
    float2 lt = ld2(lse_t + t * MATRIS_D + c), ls = ld2(lse_s + s * MATRIS_D + c);
    float2 gt = ld2(g_yt + t * ldgy + c), gs = ld2(g_ys + s * ldgy + c);
    float2 yt = ld2(y_t + t * MATRIS_D + c), ys = ld2(y_s + s * MATRIS_D + c);
    float ptx = expf(at.x - lt.x), pty = expf(at.y - lt.y);
    float psx = expf(as.x - ls.x), psy = expf(as.y - ls.y);
    float2 ge = make_float2(ptx * gt.x + psx * gs.x, pty * gt.y + psy * gs.y);
    if (g_e_base) {
        const float2 b0 = ld2(g_e_base + r * MATRIS_D + c);
        ge.x += b0.x;
        ge.y += b0.y;
    }
    st2(g_e + r * MATRIS_D + c, ge);
    st2(g_alpha_t + r * MATRIS_D + c, make_float2(ptx * gt.x * (ev.x - yt.x), pty * gt.y * (ev.y - yt.y)));
    st2(g_alpha_s + r * MATRIS_D + c, make_float2(psx * gs.x * (ev.x - ys.x), psy * gs.y * (ev.y - ys.y)));
}

extern "C" int matris_attn_bwd(int64_t n_rows, int64_t n_seg, const float *alpha_t, const float *alpha_s,
                               int64_t lda, const int32_t *alpha_idx, const float *e, const int32_t *t_idx,
                               const int32_t *s_idx, const float *y_t, const float *y_s, const float *lse_t,
                               const float *lse_s, const float *g_yt, const float *g_ys, int64_t ldgy,
                               float *g_alpha_t, float *g_alpha_s, float *g_e, const float *g_e_base, void *stream) {
    if (n_rows < 0 || n_seg < 0 || lda < MATRIS_D || (lda % 2) || ldgy < MATRIS_D || (ldgy % 2) || !t_idx ||
        !s_idx || !g_alpha_t || !g_alpha_s || !g_e)
        return MATRIS_E_ARG;
    if (n_rows == 0) return 0;
    if (alpha_idx)
        attn_bwd_kernel<true><<<matris_blocks(n_rows, WAVES_PER_BLOCK), 256, 0, (hipStream_t)stream>>>(
            n_rows, alpha_t, alpha_s, lda, alpha_idx, e, t_idx, s_idx, y_t, y_s, lse_t, lse_s, g_yt, g_ys, ldgy,
            g_alpha_t, g_alpha_s, g_e, g_e_base);
    else
        attn_bwd_kernel<false><<<matris_blocks(n_rows, WAVES_PER_BLOCK), 256, 0, (hipStream_t)stream>>>(
            n_rows, alpha_t, alpha_s, lda, nullptr, e, t_idx, s_idx, y_t, y_s, lse_t, lse_s, g_yt, g_ys, ldgy,
            g_alpha_t, g_alpha_s, g_e, g_e_base);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

// ------------------------------------------------------------------------------------
// envelope-weighted aggregation of the line-graph refinement (interaction_block.py:243-258):
//   agg[b] = sum_{a: tgt[a] = b} h[a] * env[src[a]] * env[tgt[a]] = env[b] * S[b],
//   S[b]   = sum_{a: tgt[a] = b} h[a] * env[src[a]]
// Backward:  g_h[a]   (+)= (g_agg * env)[tgt[a]] * env[src[a]]
//            g_env[b]  = g_agg[b] * S[b] + sum_{a: src[a] = b} (g_agg * env)[tgt[a]] * h[a]
// ------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void env_agg_fwd_kernel(int64_t n_seg, const float *__restrict__ h,
                                                          const float *__restrict__ env,
                                                          const int32_t *__restrict__ t_ptr,
                                                          const int32_t *__restrict__ t_perm,
                                                          const int32_t *__restrict__ s_idx, float *__restrict__ S,
                                                          float *__restrict__ agg) {
    const int64_t seg = (int64_t)blockIdx.x * WAVES_PER_BLOCK + (threadIdx.x >> 6);
    if (seg >= n_seg) return;
    const int c = 2 * (threadIdx.x & 63);
    const int b = t_ptr[seg], end = t_ptr[seg + 1];
    float2 acc = make_float2(0.f, 0.f);
    int i = b;
    for (; i + 2 <= end; i += 2) {
        const int64_t r0 = t_perm ? t_perm[i] : i, r1 = t_perm ? t_perm[i + 1] : i + 1;
        const int64_t s0 = s_idx[r0], s1 = s_idx[r1];
        const float2 h0 = ld2(h + r0 * MATRIS_D + c), h1 = ld2(h + r1 * MATRIS_D + c);
        const float2 w0 = ld2(env + s0 * MATRIS_D + c), w1 = ld2(env + s1 * MATRIS_D + c);
        acc.x += h0.x * w0.x; acc.y += h0.y * w0.y;
        acc.x += h1.x * w1.x; acc.y += h1.y * w1.y;
    }
    if (i < end) {
        const int64_t r0 = t_perm ? t_perm[i] : i;
        const float2 h0 = ld2(h + r0 * MATRIS_D + c), w0 = ld2(env + (int64_t)s_idx[r0] * MATRIS_D + c);
        acc.x += h0.x * w0.x; acc.y += h0.y * w0.y;
    }
    const float2 et = ld2(env + seg * MATRIS_D + c);
    st2(S + seg * MATRIS_D + c, acc);
    st2(agg + seg * MATRIS_D + c, make_float2(et.x * acc.x, et.y * acc.y));
}

__global__ __launch_bounds__(256) void env_agg_bwd_rows_kernel(int64_t n_rows, const float *__restrict__ g_agg,
                                                               const float *__restrict__ env,
                                                               const int32_t *__restrict__ t_idx,
                                                               const int32_t *__restrict__ s_idx, int accumulate,
                                                               float *__restrict__ g_h) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // one float4 per thread
    const int64_t r = t >> 5;
    if (r >= n_rows) return;
    const int q = (int)(t & 31) * 4;
    const int64_t tr = t_idx[r], sr = s_idx[r];
    const float4 g = *reinterpret_cast<const float4 *>(g_agg + tr * MATRIS_D + q);
    const float4 et = *reinterpret_cast<const float4 *>(env + tr * MATRIS_D + q);
    const float4 es = *reinterpret_cast<const float4 *>(env + sr * MATRIS_D + q);
    float4 v = make_float4(g.x * et.x * es.x, g.y * et.y * es.y, g.z * et.z * es.z, g.w * et.w * es.w);
    float4 *o = reinterpret_cast<float4 *>(g_h + r * MATRIS_D + q);
    if (accumulate) {
        const float4 p = *o;
        v.x += p.x; v.y += p.y; v.z += p.z; v.w += p.w;
    }
    *o = v;
}

__global__ __launch_bounds__(256) void env_agg_bwd_env_kernel(int64_t n_seg, const float *__restrict__ h,
                                                              const float *__restrict__ env,
                                                              const float *__restrict__ g_agg,
                                                              const float *__restrict__ S,
                                                              const int32_t *__restrict__ s_ptr,
                                                              const int32_t *__restrict__ s_perm,
                                                              const int32_t *__restrict__ t_idx,
                                                              float *__restrict__ g_env) {
    const int64_t seg = (int64_t)blockIdx.x * WAVES_PER_BLOCK + (threadIdx.x >> 6);
    if (seg >= n_seg) return;
    const int c = 2 * (threadIdx.x & 63);
    const int b = s_ptr[seg], end = s_ptr[seg + 1];
    float2 acc = make_float2(0.f, 0.f);
    for (int i = b; i < end; ++i) {
        const int64_t r = s_perm ? s_perm[i] : i;
        const int64_t tr = t_idx[r];
        const float2 hv = ld2(h + r * MATRIS_D + c);
        const float2 g = ld2(g_agg + tr * MATRIS_D + c), et = ld2(env + tr * MATRIS_D + c);
        acc.x += g.x * et.x * hv.x;
        acc.y += g.y * et.y * hv.y;
    }
    const float2 gs = ld2(g_agg + seg * MATRIS_D + c), sv = ld2(S + seg * MATRIS_D + c);
    st2(g_env + seg * MATRIS_D + c, make_float2(gs.x * sv.x + acc.x, gs.y * sv.y + acc.y));
}

extern "C" int matris_env_agg_fwd(int64_t n_seg, const float *h, const float *env, const int32_t *t_ptr,
                                  const int32_t *t_perm, const int32_t *s_idx, float *S, float *agg, void *stream) {
    if (n_seg < 0 || !h || !env || !t_ptr || !s_idx || !S || !agg) return MATRIS_E_ARG;
    if (n_seg == 0) return 0;
    env_agg_fwd_kernel<<<matris_blocks(n_seg, WAVES_PER_BLOCK), 256, 0, (hipStream_t)stream>>>(
        n_seg, h, env, t_ptr, t_perm, s_idx, S, agg);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_env_agg_bwd(int64_t n_rows, int64_t n_seg, const float *h, const float *env,
                                  const float *g_agg, const float *S, const int32_t *t_idx, const int32_t *s_idx,
                                  const int32_t *s_ptr, const int32_t *s_perm, int accumulate, float *g_h,
                                  float *g_env, void *stream) {
    if (n_rows < 0 || n_seg < 0 || !h || !env || !g_agg || !S || !t_idx || !s_idx || !s_ptr || !g_h || !g_env)
        return MATRIS_E_ARG;
    hipStream_t st = (hipStream_t)stream;
    if (n_rows > 0) {
        env_agg_bwd_rows_kernel<<<matris_blocks(n_rows * 32, 256), 256, 0, st>>>(n_rows, g_agg, env, t_idx, s_idx,
                                                                               accumulate, g_h);
        MATRIS_CHECK_LAUNCH();
    }
    if (n_seg > 0) {
        env_agg_bwd_env_kernel<<<matris_blocks(n_seg, WAVES_PER_BLOCK), 256, 0, st>>>(n_seg, h, env, g_agg, S, s_ptr,
                                                                                    s_perm, t_idx, g_env);
        MATRIS_CHECK_LAUNCH();
    }
    return 0;
}

extern "C" const char *matris_version(void) { return "matris_hip 0.1 gfx950"; }
