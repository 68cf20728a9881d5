// SiLU derivative ops of the reference's torch op library (matris/model/op: the
// matris_op::fuse_silu_bwd / fuse_silu_grad_bwd schemas of RegisterOp.cpp:9-13, with the
// arithmetic of fused_silu_op.py:5-28):
//   silu_bwd:      out = dgrad * s'(x),            s'(x) = sig(x) (1 + x (1 - sig(x)))
//   silu_grad_bwd: ggo = ggi * s'(x),  gx = ggi * go * s''(x),
//                  s''(x) = sig(x) (1 - sig(x)) (2 + x (1 - 2 sig(x)))
// (the first and second derivatives of SiLU(x) = x sig(x)).  Element-wise and HBM-bound:
// 16-byte vectors when every pointer is aligned, grid-stride, a scalar tail.
#include "mma.h"

__device__ __forceinline__ float silu_d1(float x) {
    const float s = sigm_f(x);
    return s * (1.f + x * (1.f - s));
}

__device__ __forceinline__ void silu_d12(float x, float &d1, float &d2) {
    const float s = sigm_f(x);
    d1 = s * (1.f + x * (1.f - s));
    d2 = s * (1.f - s) * (2.f + x * (1.f - 2.f * s));
}

__global__ __launch_bounds__(256) void silu_bwd_kernel(int64_t n, const float *__restrict__ dgrad,
                                                       const float *__restrict__ x, float *__restrict__ out,
                                                       int vec) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (vec) {
        const int64_t n4 = n >> 2;
        for (; i < n4; i += stride) {
            const float4 g = reinterpret_cast<const float4 *>(dgrad)[i], v = reinterpret_cast<const float4 *>(x)[i];
            reinterpret_cast<float4 *>(out)[i] =
                make_float4(g.x * silu_d1(v.x), g.y * silu_d1(v.y), g.z * silu_d1(v.z), g.w * silu_d1(v.w));
        }
        i = (n4 << 2) + ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
    }
    for (; i < n; i += stride) out[i] = dgrad[i] * silu_d1(x[i]);
}

__global__ __launch_bounds__(256) void silu_grad_bwd_kernel(int64_t n, const float *__restrict__ ggi,
                                                            const float *__restrict__ go,
                                                            const float *__restrict__ x, float *__restrict__ ggo,
                                                            float *__restrict__ gx, int vec) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (vec) {
        const int64_t n4 = n >> 2;
        for (; i < n4; i += stride) {
            const float4 a = reinterpret_cast<const float4 *>(ggi)[i], g = reinterpret_cast<const float4 *>(go)[i];
            const float4 v = reinterpret_cast<const float4 *>(x)[i];
            float4 o1, o2;
            float d1, d2;
            silu_d12(v.x, d1, d2); o1.x = a.x * d1; o2.x = a.x * g.x * d2;
            silu_d12(v.y, d1, d2); o1.y = a.y * d1; o2.y = a.y * g.y * d2;
            silu_d12(v.z, d1, d2); o1.z = a.z * d1; o2.z = a.z * g.z * d2;
            silu_d12(v.w, d1, d2); o1.w = a.w * d1; o2.w = a.w * g.w * d2;
            reinterpret_cast<float4 *>(ggo)[i] = o1;
            reinterpret_cast<float4 *>(gx)[i] = o2;
        }
        i = (n4 << 2) + ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
    }
    for (; i < n; i += stride) {
        float d1, d2;
        silu_d12(x[i], d1, d2);
        ggo[i] = ggi[i] * d1;
        gx[i] = ggi[i] * go[i] * d2;
    }
}

static bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// Work-groups for an element-wise pass over n floats: enough to fill the chip several
// times over, each thread then looping.
static dim3 ew_grid(int64_t n) {
    const int64_t want = (n / 4 + 255) / 256;
    return dim3((unsigned)std::max<int64_t>(1, std::min<int64_t>(want, 8192)));
}

extern "C" int matris_silu_bwd(int64_t n, const float *dgrad, const float *x, float *out, void *stream) {
    if (n < 0 || (n > 0 && (!dgrad || !x || !out))) return MATRIS_E_ARG;
    if (n == 0) return 0;
    const int vec = al16(dgrad) && al16(x) && al16(out);
    silu_bwd_kernel<<<ew_grid(n), 256, 0, (hipStream_t)stream>>>(n, dgrad, x, out, vec);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_silu_grad_bwd(int64_t n, const float *ggi, const float *go, const float *x, float *ggo,
                                    float *gx, void *stream) {
    if (n < 0 || (n > 0 && (!ggi || !go || !x || !ggo || !gx))) return MATRIS_E_ARG;
    if (n == 0) return 0;
    const int vec = al16(ggi) && al16(go) && al16(x) && al16(ggo) && al16(gx);
    silu_grad_bwd_kernel<<<ew_grid(n), 256, 0, (hipStream_t)stream>>>(n, ggi, go, x, ggo, gx, vec);
    MATRIS_CHECK_LAUNCH();
    return 0;
}
