// Radial and three-body basis functions of the embeddings (rows E2, E3) on gfx950, with
// their input gradients.  Thread per row; the forward mirrors the reference's fp32
// evaluation order (matris/model/basis_function.py), the backward is the analytic
// derivative.
//
//   E2  Bessel x polynomial envelope (basis_function.py:8-50, 116-186):
//       out[i, n] = env(d_i / rc) * (sqrt(2/rc) sin(f_n d_i / rc) / d_i),
//       env(x) = 1 + a x^p + b x^(p+1) + c x^(p+2) for x < 1, else 0,
//       a = -(p+1)(p+2)/2, b = p(p+2), c = -p(p+1)/2
//   E3  spherical three-body basis (feature_embed.py:183-201, basis_function.py:53-77,
//       222-338): for angle row a with directed edges t = de_t[a] (i->j) and
//       s = de_s[a] (j->k) and unit vectors u:
//       cos = (u_t . u_s) (1 - 1e-6), theta = acos(cos), x = |u_s| / rc,
//       basis[a, 4n + j] = factor R_{n,j}(x) Y_n(cos theta),  n, j = 0..3
//       with R the spherical-Bessel root expansions of the coefficient table below and
//       Y_l the m = 0 real spherical harmonics.
#include "common.h"
#include "bessel.h"

// No FMA contraction in this file: products and sums round separately, as the
// reference's elementwise torch ops do.
#pragma clang fp contract(off)

// Coefficients of R_{n,j} (basis_function.py:241-274 / SphericalExpansion.coef):
// n = 0: sin(k0 x) / x; n = 1..3: the spherical Bessel j_n(k x) in closed form at the
// first four roots k of j_n, with the normalisation folded into the coefficients.
__constant__ float kSbf0[4] = {3.14159274101257f, 6.28318548202515f, 9.42477798461914f, 12.5663709640503f};
__constant__ float kSbf1[4][4] = {
    {-1.02446483277785f, -1.00834335996107f, -1.00419641763893f, -1.00252381898662f},
    {4.49340963363647f, 7.7252516746521f, 10.9041213989258f, 14.0661935806274f},
    {0.22799275301076f, 0.130525632358311f, 0.092093290316619f, 0.0712718627992818f},
    {4.49340963363647f, 7.7252516746521f, 10.9041213989258f, 14.0661935806274f}};
__constant__ float kSbf2[6][4] = {
    {-1.04807944170731f, -1.01861796359391f, -1.01002272174988f, -1.00628955560036f},
    {5.76345920562744f, 9.09501171112061f, 12.322940826416f, 15.5146026611328f},
    {0.545547077361439f, 0.335992298618515f, 0.245888396928293f, 0.194582402961821f},
    {5.76345920562744f, 9.09501171112061f, 12.322940826416f, 15.5146026611328f},
    {0.0946561878721665f, 0.0369424811413594f, 0.0199537107571916f, 0.0125418876146463f},
    {5.76345920562744f, 9.09501171112061f, 12.322940826416f, 15.5146026611328f}};
__constant__ float kSbf3[8][4] = {
    {1.06942831392075f, 1.0292173312802f, 1.01650804843248f, 1.01069656069999f},
    {6.9879322052002f, 10.4171180725098f, 13.6980228424072f, 16.9236221313477f},
    {0.918235852195231f, 0.592803493701152f, 0.445250264272671f, 0.358326327374518f},
    {6.9879322052002f, 10.4171180725098f, 13.6980228424072f, 16.9236221313477f},
    {0.328507713452024f, 0.142266673367543f, 0.0812617757677838f, 0.0529328657590962f},
    {6.9879322052002f, 10.4171180725098f, 13.6980228424072f, 16.9236221313477f},
    {0.0470107184508114f, 0.0136570088173405f, 0.0059323726279831f, 0.00312775039221944f},
    {6.9879322052002f, 10.4171180725098f, 13.6980228424072f, 16.9236221313477f}};

// real spherical harmonics Y_l(c), l = 0..3 (basis_function.py:56-73) and dY_l/dc
__device__ __forceinline__ void sph_y(float c, float y[4], float dy[4]) {
    const float k0 = 0.5641895835477563f;   // sqrt(1 / pi)
    const float k1 = 0.4886025119029199f;   // sqrt(3 / (4 pi))
    const float k2 = 0.31539156525252005f;  // sqrt(5 / (16 pi))
    const float k3 = 0.37317633259011546f;  // sqrt(7 / (16 pi))
    const float c2 = c * c;
    y[0] = 0.5f * k0;
    y[1] = k1 * c;
    y[2] = k2 * (3.0f * c2 - 1.0f);
    y[3] = k3 * c * (5.0f * c2 - 3.0f);
    dy[0] = 0.f;
    dy[1] = k1;
    dy[2] = k2 * 6.0f * c;
    dy[3] = k3 * (15.0f * c2 - 3.0f);
}

// R_{n,j}(x) (times factor) for all 16 (n, j) and, when D, dR/dx.
template <bool D>
__device__ __forceinline__ void sph_r(float x, float factor, float r[16], float dr[16]) {
    const float x2 = x * x, x3 = x * x * x, x4 = powf(x, 4.0f);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float a = kSbf0[j];
        const float s = sinf(a * x);
        r[j] = s / x * factor;
        if (D) dr[j] = (a * cosf(a * x) / x - s / x2) * factor;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float c0 = kSbf1[0][j], c1 = kSbf1[1][j], c2 = kSbf1[2][j], c3 = kSbf1[3][j];
        const float cs1 = cosf(c1 * x), sn3 = sinf(c3 * x);
        const float num = c0 * x * cs1 + c2 * sn3;
        r[4 + j] = num / x2 * factor;
        if (D) {
            const float dnum = c0 * cs1 - c0 * c1 * x * sinf(c1 * x) + c2 * c3 * cosf(c3 * x);
            dr[4 + j] = (dnum / x2 - 2.0f * num / x3) * factor;
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float c0 = kSbf2[0][j], c1 = kSbf2[1][j], c2 = kSbf2[2][j], c3 = kSbf2[3][j], c4 = kSbf2[4][j],
                    c5 = kSbf2[5][j];
        const float sn1 = sinf(c1 * x), cs3 = cosf(c3 * x), sn5 = sinf(c5 * x);
        const float num = c0 * x2 * sn1 - c2 * x * cs3 + c4 * sn5;
        r[8 + j] = num / x3 * factor;
        if (D) {
            const float dnum = 2.0f * c0 * x * sn1 + c0 * c1 * x2 * cosf(c1 * x) - c2 * cs3 +
                               c2 * c3 * x * sinf(c3 * x) + c4 * c5 * cosf(c5 * x);
            dr[8 + j] = (dnum / x3 - 3.0f * num / x4) * factor;
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float c0 = kSbf3[0][j], c1 = kSbf3[1][j], c2 = kSbf3[2][j], c3 = kSbf3[3][j], c4 = kSbf3[4][j],
                    c5 = kSbf3[5][j], c6 = kSbf3[6][j], c7 = kSbf3[7][j];
        const float cs1 = cosf(c1 * x), sn3 = sinf(c3 * x), cs5 = cosf(c5 * x), sn7 = sinf(c7 * x);
        const float num = c0 * x3 * cs1 - c2 * x2 * sn3 - c4 * x * cs5 + c6 * sn7;
        r[12 + j] = num / x4 * factor;
        if (D) {
            const float dnum = 3.0f * c0 * x2 * cs1 - c0 * c1 * x3 * sinf(c1 * x) - 2.0f * c2 * x * sn3 -
                               c2 * c3 * x2 * cosf(c3 * x) - c4 * cs5 + c4 * c5 * x * sinf(c5 * x) +
                               c6 * c7 * cosf(c7 * x);
            dr[12 + j] = (dnum / x4 - 4.0f * num / (x4 * x)) * factor;
        }
    }
}

struct SbfGeom {
    float c, ct, dct_dc, x, len;
};

// cos(theta) as in the reference: c = (u_t . u_s) (1 - 1e-6), theta = acos(c),
// ct = cos(theta); x = |u_s| / rc
__device__ __forceinline__ SbfGeom sbf_geom(const float *ut, const float *us, float rc) {
    SbfGeom g;
    const float dot = ut[0] * us[0] + ut[1] * us[1] + ut[2] * us[2];
    g.c = dot * 0.999999f;
    const float th = acosf(g.c);
    g.ct = cosf(th);
    g.dct_dc = sinf(th) / sqrtf(1.0f - g.c * g.c);  // d cos(acos c) / dc (= 1 up to rounding)
    g.len = sqrtf(us[0] * us[0] + us[1] * us[1] + us[2] * us[2]);
    g.x = g.len / rc;
    return g;
}

__global__ __launch_bounds__(256) void sbf_fwd_kernel(int64_t n, const float *__restrict__ unit,
                                                      const int32_t *__restrict__ de_t,
                                                      const int32_t *__restrict__ de_s, float rc, float factor,
                                                      float *__restrict__ out) {
    const int64_t a = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (a >= n) return;
    const float *ut = unit + 3 * (int64_t)de_t[a], *us = unit + 3 * (int64_t)de_s[a];
    const SbfGeom g = sbf_geom(ut, us, rc);
    float r[16], y[4], dy[4];
    sph_r<false>(g.x, factor, r, nullptr);
    sph_y(g.ct, y, dy);
    float4 *o = reinterpret_cast<float4 *>(out + 16 * a);
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = make_float4(r[4 * q] * y[q], r[4 * q + 1] * y[q], r[4 * q + 2] * y[q], r[4 * q + 3] * y[q]);
}

// dL/dc and dL/dx of one angle row from its basis gradient g[16]
__device__ __forceinline__ void sbf_row_grad(const SbfGeom &g, const float *__restrict__ gb, float &g_c, float &g_x) {
    float r[16], dr[16], y[4], dy[4];
    sph_r<true>(g.x, 1.0f, r, dr);
    sph_y(g.ct, y, dy);
    float sc = 0.f, sx = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        sc += gb[k] * r[k] * dy[k >> 2];
        sx += gb[k] * dr[k] * y[k >> 2];
    }
    g_c = sc * g.dct_dc;
    g_x = sx;
}

// Thread per directed edge d: the gradient of its unit vector collects every angle row
// that reads it as u_t (target CSR) or as u_s (source CSR), in CSR order.
// Backward, first pass: thread per angle row, the row's gradient into unit[t] and into
// unit[s] (work [n, 6]); every row's geometry and derivatives are evaluated once.
__global__ __launch_bounds__(256) void sbf_bwd_row_kernel(int64_t n, const float *__restrict__ unit,
                                                          const int32_t *__restrict__ de_t,
                                                          const int32_t *__restrict__ de_s,
                                                          const float *__restrict__ g_basis, float rc, float factor,
                                                          float *__restrict__ work) {
    const int64_t a = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (a >= n) return;
    const float *ut = unit + 3 * (int64_t)de_t[a], *us = unit + 3 * (int64_t)de_s[a];
    const SbfGeom g = sbf_geom(ut, us, rc);
    float gb[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) gb[k] = g_basis[16 * a + k] * factor;
    float g_c, g_x;
    sbf_row_grad(g, gb, g_c, g_x);
    const float w = g_c * 0.999999f, v = g_x / (rc * g.len);
    float *o = work + 6 * a;
    // unit[t]: dc/du_t = u_s (1 - 1e-6); unit[s]: dc/du_s = u_t (1 - 1e-6), dx/du_s = u_s / (rc |u_s|)
    o[0] = w * us[0];
    o[1] = w * us[1];
    o[2] = w * us[2];
    o[3] = w * ut[0] + v * us[0];
    o[4] = w * ut[1] + v * us[1];
    o[5] = w * ut[2] + v * us[2];
}

// Second pass: thread per directed edge d, the rows that read unit[d] as t, then as s, in
// CSR order (deterministic).
__global__ __launch_bounds__(256) void sbf_bwd_edge_kernel(int64_t n_edges, const int32_t *__restrict__ t_ptr,
                                                           const int32_t *__restrict__ t_perm,
                                                           const int32_t *__restrict__ s_ptr,
                                                           const int32_t *__restrict__ s_perm,
                                                           const float *__restrict__ work, int accumulate,
                                                           float *__restrict__ g_unit) {
    const int64_t d = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= n_edges) return;
    float gx = 0.f, gy = 0.f, gz = 0.f;
    for (int i = t_ptr[d]; i < t_ptr[d + 1]; ++i) {
        const float *o = work + 6 * (int64_t)(t_perm ? t_perm[i] : i);
        gx += o[0];
        gy += o[1];
        gz += o[2];
    }
    for (int i = s_ptr[d]; i < s_ptr[d + 1]; ++i) {
        const float *o = work + 6 * (int64_t)(s_perm ? s_perm[i] : i);
        gx += o[3];
        gy += o[4];
        gz += o[5];
    }
    float *o = g_unit + 3 * d;
    if (accumulate) {
        gx += o[0];
        gy += o[1];
        gz += o[2];
    }
    o[0] = gx;
    o[1] = gy;
    o[2] = gz;
}

__global__ __launch_bounds__(256) void bessel_fwd_kernel(int64_t n, int nr, const float *__restrict__ dist,
                                                         const float *__restrict__ freq, BesselParams P,
                                                         float rc, float *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    bessel_row(dist[i], nr, freq, P, rc, out + i * nr);
}

__global__ __launch_bounds__(256) void bessel_bwd_kernel(int64_t n, int nr, const float *__restrict__ dist,
                                                         const float *__restrict__ freq, BesselParams P,
                                                         float rc, const float *__restrict__ g_out, int accumulate,
                                                         float *__restrict__ g_dist) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float acc = bessel_row_grad(dist[i], nr, freq, P, rc, g_out + i * nr);
    g_dist[i] = accumulate ? g_dist[i] + acc : acc;
}

extern "C" int matris_bessel_fwd(int64_t n, int num_radial, const float *dist, const float *freq, double cutoff,
                                 double envelope_exponent, float *out, void *stream) {
    if (n < 0 || num_radial < 1 || !(cutoff > 0) || !(envelope_exponent > 0) || !dist || !freq || !out)
        return MATRIS_E_ARG;
    if (n == 0) return 0;
    bessel_fwd_kernel<<<matris_blocks(n, 256), 256, 0, (hipStream_t)stream>>>(
        n, num_radial, dist, freq, bessel_params(cutoff, envelope_exponent), (float)cutoff, out);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_bessel_bwd(int64_t n, int num_radial, const float *dist, const float *freq, double cutoff,
                                 double envelope_exponent, const float *g_out, int accumulate, float *g_dist,
                                 void *stream) {
    if (n < 0 || num_radial < 1 || !(cutoff > 0) || !(envelope_exponent > 0) || !dist || !freq || !g_out || !g_dist)
        return MATRIS_E_ARG;
    if (n == 0) return 0;
    bessel_bwd_kernel<<<matris_blocks(n, 256), 256, 0, (hipStream_t)stream>>>(
        n, num_radial, dist, freq, bessel_params(cutoff, envelope_exponent), (float)cutoff, g_out, accumulate,
        g_dist);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

static float sbf_factor(double cutoff) { return sqrtf((float)(2.0 / (cutoff * cutoff * cutoff))); }

extern "C" int matris_sbf_fwd(int64_t n_angles, const float *unit, const int32_t *de_t, const int32_t *de_s,
                              double cutoff, float *out, void *stream) {
    if (n_angles < 0 || !(cutoff > 0) || !unit || !de_t || !de_s || !out) return MATRIS_E_ARG;
    if (n_angles == 0) return 0;
    sbf_fwd_kernel<<<matris_blocks(n_angles, 256), 256, 0, (hipStream_t)stream>>>(
        n_angles, unit, de_t, de_s, (float)cutoff, sbf_factor(cutoff), out);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_sbf_bwd(int64_t n_edges, int64_t n_angles, const float *unit, const int32_t *de_t,
                              const int32_t *de_s, const float *g_basis, const int32_t *t_ptr, const int32_t *t_perm,
                              const int32_t *s_ptr, const int32_t *s_perm, double cutoff, int accumulate,
                              float *work, float *g_unit, void *stream) {
    if (n_edges < 0 || n_angles < 0 || !(cutoff > 0) || !unit || !t_ptr || !s_ptr || !g_unit ||
        (n_angles > 0 && (!de_t || !de_s || !g_basis || !work)))
        return MATRIS_E_ARG;
    if (n_edges == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    if (n_angles > 0) {
        sbf_bwd_row_kernel<<<matris_blocks(n_angles, 256), 256, 0, st>>>(n_angles, unit, de_t, de_s, g_basis,
                                                                         (float)cutoff, sbf_factor(cutoff), work);
        MATRIS_CHECK_LAUNCH();
    }
    sbf_bwd_edge_kernel<<<matris_blocks(n_edges, 256), 256, 0, st>>>(n_edges, t_ptr, t_perm, s_ptr, s_perm, work,
                                                                     accumulate, g_unit);
    MATRIS_CHECK_LAUNCH();
    return 0;
}
