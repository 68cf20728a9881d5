// Bessel basis with the polynomial envelope (basis_function.py:8-50, 116-186), per
// distance, shared by the basis kernels and the fused edge embedding:
//   rbf_n(d) = env(d / rc) * (sqrt(2/rc) sin(f_n d / rc) / d),
//   env(x) = 1 + a x^p + b x^(p+1) + c x^(p+2) for x < 1, else 0,
//   a = -(p+1)(p+2)/2, b = p(p+2), c = -p(p+1)/2.
// No FMA contraction inside these functions: products and sums round separately, as the
// reference's elementwise torch ops do, wherever they are inlined.
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>

struct BesselParams {
    float inv_rc, norm, a, b, c, p;
};

static inline BesselParams bessel_params(double cutoff, double p) {
    BesselParams P;
    P.inv_rc = (float)(1.0 / cutoff);
    P.norm = (float)std::sqrt(2.0 / cutoff);
    P.a = (float)(-(p + 1) * (p + 2) / 2);
    P.b = (float)(p * (p + 2));
    P.c = (float)(-p * (p + 1) / 2);
    P.p = (float)p;
    return P;
}

// out[k] = rbf_k(d), k < nr
__device__ __forceinline__ void bessel_row(float d, int nr, const float *__restrict__ freq, const BesselParams &P,
                                           float rc, float *out) {
#pragma clang fp contract(off)
    const float x = d / rc;
    float sf = 0.f;
    if (x < 1.0f) sf = 1.0f + P.a * powf(x, P.p) + P.b * powf(x, P.p + 1.0f) + P.c * powf(x, P.p + 2.0f);
    const float dic = d * P.inv_rc;
    for (int k = 0; k < nr; ++k) out[k] = sf * (P.norm * sinf(freq[k] * dic) / d);
}

// sum_k g[k] d rbf_k / d d
__device__ __forceinline__ float bessel_row_grad(float d, int nr, const float *__restrict__ freq,
                                                 const BesselParams &P, float rc, const float *g) {
#pragma clang fp contract(off)
    const float x = d / rc;
    float sf = 0.f, dsf = 0.f;
    if (x < 1.0f) {
        sf = 1.0f + P.a * powf(x, P.p) + P.b * powf(x, P.p + 1.0f) + P.c * powf(x, P.p + 2.0f);
        dsf = (P.a * P.p * powf(x, P.p - 1.0f) + P.b * (P.p + 1.0f) * powf(x, P.p) +
               P.c * (P.p + 2.0f) * powf(x, P.p + 1.0f)) / rc;
    }
    const float dic = d * P.inv_rc;
    float acc = 0.f;
    for (int k = 0; k < nr; ++k) {
        const float f = freq[k];
        const float s = sinf(f * dic), c = cosf(f * dic);
        const float base = P.norm * s / d;
        const float dbase = P.norm * (f * P.inv_rc * c / d - s / (d * d));
        acc += g[k] * (dsf * base + sf * dbase);
    }
    return acc;
}
