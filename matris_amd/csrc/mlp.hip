// Fused dense layers on gfx950 MFMA for the 128-wide feature rows of the interaction
// blocks (same fp32 / split-bf16 / split-fp16 modes as the gated MLP, see mma.h):
//
//   FFN     out = W2 SiLU(W1 x)            node_FFN / edge_FFN of Refinement
//           (MLP(hidden=int, bias=False), matris/model/functions.py:198-205,
//            interaction_block.py:198-210, 269-270)
//   PAIR    (out0, out1) = (x W0^T, x W1^T) source / target attention projections
//           (interaction_block.py:33-38, 110-111), one [M,128]x[128,256] product
//
// and their input-gradient kernels.  Work-group = 4 wave64s over BM = 64 rows; the
// [64, 128] input tile is staged once in one LDS tile (K = 128 needs no K loop) -- in the
// two-plane modes already split into fragment units, so no wave converts an operand --
// weights are pre-packed fragments (mma.h) read from global ahead of use, and
// intermediate tiles (g_p) stay in LDS.  The GEMMs run transposed (weight fragment as
// the MFMA A operand, rows in lanes), so results reach LDS with 16-byte writes.  Outputs
// leave through LDS with 16-byte row stores.  The FFN forward of the two-plane modes is
// weight-stationary and persistent instead (ffn_fwd_ws_kernel).
#include <algorithm>
#include <initializer_list>

#include "mma.h"
#include "bessel.h"

// Copy rows [m0, m0+64) x 128 columns of a row-major [*, ld] array into LDS (zeros past M).
__device__ __forceinline__ void stage_tile128(float *dst, const float *__restrict__ src, int64_t ld, int64_t m0,
                                              int64_t M, int tid) {
#pragma unroll
    for (int it = 0; it < (BM * 32) / 256; ++it) {
        const int q = it * 256 + tid;
        const int r = q >> 5, c4 = (q & 31) * 4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (m0 + r < M) v = *reinterpret_cast<const float4 *>(src + (m0 + r) * ld + c4);
        *reinterpret_cast<float4 *>(dst + r * LDT + c4) = v;
    }
}

// Copy an LDS tile out to rows of dst; with res non-NULL, dst = tile + res_w * res (rows of
// 128, per-column weight res_w); with accumulate, dst's previous contents are added last.
__device__ __forceinline__ void store_tile128(const float *tile, float *__restrict__ dst, int64_t ld, int64_t m0,
                                              int64_t M, int tid, const float *__restrict__ res = nullptr,
                                              const float *__restrict__ res_w = nullptr, int accumulate = 0) {
#pragma unroll
    for (int it = 0; it < (BM * 32) / 256; ++it) {
        const int q = it * 256 + tid;
        const int r = q >> 5, c4 = (q & 31) * 4;
        if (m0 + r < M) {
            float4 v = *reinterpret_cast<const float4 *>(tile + r * LDT + c4);
            if (res) {
                const float4 x = *reinterpret_cast<const float4 *>(res + (m0 + r) * MATRIS_D + c4);
                const float4 w = *reinterpret_cast<const float4 *>(res_w + c4);
                v.x += w.x * x.x; v.y += w.y * x.y; v.z += w.z * x.z; v.w += w.w * x.w;
            }
            float4 *o = reinterpret_cast<float4 *>(dst + (m0 + r) * ld + c4);
            if (accumulate) {
                const float4 a = *o;
                v.x += a.x; v.y += a.y; v.z += a.z; v.w += a.w;
            }
            *o = v;
        }
    }
}

// dst rows = w * tile (per-column weight w).
__device__ __forceinline__ void store_tile128_scaled(const float *tile, float *__restrict__ dst,
                                                     const float *__restrict__ w, int64_t m0, int64_t M, int tid) {
#pragma unroll
    for (int it = 0; it < (BM * 32) / 256; ++it) {
        const int q = it * 256 + tid;
        const int r = q >> 5, c4 = (q & 31) * 4;
        if (m0 + r < M) {
            const float4 v = *reinterpret_cast<const float4 *>(tile + r * LDT + c4);
            const float4 s = *reinterpret_cast<const float4 *>(w + c4);
            *reinterpret_cast<float4 *>(dst + (m0 + r) * MATRIS_D + c4) = make_float4(s.x * v.x, s.y * v.y, s.z * v.z, s.w * v.w);
        }
    }
}

// A thread's share of rows m0 .. m0+63 of a [*, 128] array: row tid/4, 8-column groups
// q, q+4, q+8, q+12 for q = tid%4 (zeros past M).
struct Rows128 {
    float4 u[4], v[4];
};
__device__ __forceinline__ void load_rows128(Rows128 &x, const float *__restrict__ src, int64_t m0, int64_t M,
                                             int tid) {
    const int r = tid >> 2, q = tid & 3;
    const bool in = m0 + r < M;
    const float4 *p = reinterpret_cast<const float4 *>(src + (m0 + r) * MATRIS_D);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int g = q + 4 * i;
        x.u[i] = in ? p[2 * g] : make_float4(0.f, 0.f, 0.f, 0.f);
        x.v[i] = in ? p[2 * g + 1] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

// max |x| over the row (the 4 threads that hold it)
__device__ __forceinline__ float rows128_absmax(const Rows128 &x) {
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) m = abs_max4(abs_max4(m, x.u[i]), x.v[i]);
    return group4_max(m);
}

// g_res = res_w * rows (the FFN backward's residual gradient), rows below M
__device__ __forceinline__ void store_res128(const Rows128 &x, float *__restrict__ g_res,
                                             const float *__restrict__ res_w, int64_t m0, int64_t M, int tid) {
    const int r = tid >> 2, q = tid & 3;
    if (m0 + r >= M) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int g = q + 4 * i;
        const float4 wu = *reinterpret_cast<const float4 *>(res_w + 8 * g);
        const float4 wv = *reinterpret_cast<const float4 *>(res_w + 8 * g + 4);
        float4 *o = reinterpret_cast<float4 *>(g_res + (m0 + r) * MATRIS_D + 8 * g);
        o[0] = make_float4(wu.x * x.u[i].x, wu.y * x.u[i].y, wu.z * x.u[i].z, wu.w * x.u[i].w);
        o[1] = make_float4(wv.x * x.v[i].x, wv.y * x.v[i].y, wv.z * x.v[i].z, wv.w * x.v[i].w);
    }
}

// The envelope term of the line refinement's hidden-row gradient, the backward of
// agg[b] = sum_{a: t[a] = b} h[a] * env[s[a]] * env[t[a]] (interaction_block.py:243-258):
//   add[a] = ge[t[a]] * env[s[a]],  ge = g_agg * env (per bond, written beforehand by
//   matris_env_agg_bwd_env)                    (ge == nullptr: no term)
struct EnvTerm {
    const float *ge, *env;
    const int32_t *t, *s;
};

__device__ __forceinline__ float4 env_term4(const EnvTerm &e, int64_t tr, int64_t sr, int col) {
    const float4 g = *reinterpret_cast<const float4 *>(e.ge + tr * MATRIS_D + col);
    const float4 b = *reinterpret_cast<const float4 *>(e.env + sr * MATRIS_D + col);
    return make_float4(g.x * b.x, g.y * b.y, g.z * b.z, g.w * b.w);
}

// store_tile128 of a [*, 128] output plus the envelope term of each row.
__device__ __forceinline__ void store_tile128_env(const float *tile, float *__restrict__ dst, int64_t m0, int64_t M,
                                                  int tid, const EnvTerm &et) {
#pragma unroll
    for (int it = 0; it < (BM * 32) / 256; ++it) {
        const int q = it * 256 + tid;
        const int r = q >> 5, c4 = (q & 31) * 4;
        if (m0 + r < M) {
            float4 v = *reinterpret_cast<const float4 *>(tile + r * LDT + c4);
            if (et.ge) {
                const float4 a = env_term4(et, et.t[m0 + r], et.s[m0 + r], c4);
                v.x += a.x; v.y += a.y; v.z += a.z; v.w += a.w;
            }
            *reinterpret_cast<float4 *>(dst + (m0 + r) * MATRIS_D + c4) = v;
        }
    }
}

// Stage the rows, times s, into LDS pre-split into fragment units [rt 2][kb 8][plane 2][64
// lanes] (two-plane modes), each value converted once.
template <int MODE>
__device__ __forceinline__ float stage_rows128(uint4 *buf, const Rows128 &x, int tid, float amax, float s = 1.f) {
    const int r = tid >> 2, q = tid & 3;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int g = q + 4 * i;
        const float4 u = s == 1.f ? x.u[i] : mul4(x.u[i], s), v = s == 1.f ? x.v[i] : mul4(x.v[i], s);
        amax = frag_amax<MODE>(amax, u, v);
        frag_put8<MODE>(buf, (r >> 5) * 8 + (g >> 1), (r & 31) + 32 * (g & 1), u, v);
    }
    return amax;
}

template <int MODE>
__device__ __forceinline__ float stage_frag128(uint4 *buf, const float *__restrict__ src, int64_t m0, int64_t M,
                                               int tid, float amax) {
    Rows128 x;
    load_rows128(x, src, m0, M, tid);
    return stage_rows128<MODE>(buf, x, tid, amax);
}

// MODE 2: the row scale of a gradient tile (2^k, recorded as 2^-k in rinv by one of the
// row's threads); 1 in the other modes.
// MODE 2: multiply transposed accumulators (rows in lanes: row rt*32 + l32) by their rows'
// 2^-k.
template <int MODE, int NCT>
__device__ __forceinline__ void unscale_rows_t(v16f (&acc)[2][NCT], const float *rinv, int l32) {
    if constexpr (MODE == 2) {
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const float r = rinv[rt * 32 + l32];
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) acc[rt][ct] *= r;
        }
    }
}

template <int MODE>
__device__ __forceinline__ float tile_row_scale(float row_absmax, float *rinv, int tid) {
    if constexpr (MODE == 2) {
        const RowScale rs = row_scale(row_absmax);
        if ((tid & 3) == 0) rinv[tid >> 2] = rs.inv;
        return rs.s;
    } else {
        return 1.f;
    }
}

// ------------------------------------------------------------------------------------
// FFN forward: p = x W1^T (saved), out = SiLU(p) W2^T
// ------------------------------------------------------------------------------------
// One [64, 128] LDS tile per work-group (three work-groups per CU): x, then p / h, then
// out pass through it.  Both GEMMs run transposed (rows in lanes, mma.h), so results go
// to the tile as 16-byte writes; one pass saves p and applies SiLU in place.
template <int MODE>
__global__ __launch_bounds__(256, 3) void ffn_fwd_kernel(int64_t M, const float *__restrict__ x,
                                                         const uint4 *__restrict__ W1, const uint4 *__restrict__ W2,
                                                         float *__restrict__ out, float *__restrict__ save_p,
                                                         const float *__restrict__ res,
                                                         const float *__restrict__ res_w, unsigned *range_flag) {
    __shared__ __align__(16) float T[BM * LDT];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int64_t m0 = (int64_t)blockIdx.x * BM;
    const float w1s = take_wscale<MODE>(W1), w2s = take_wscale<MODE>(W2);
    stage_tile128(T, x, MATRIS_D, m0, M, tid);
    __syncthreads();
    v16f acc[2][1];
    zero_acc(acc);
    float amax = gemm_lds_packed<MODE, 2, 1, MATRIS_D / 16, true>(acc, T, LDT, W1, wave, MATRIS_D / 16, 0, lane);
    scale_acc<MODE>(acc, w1s);
    __syncthreads();  // every wave is done reading x
    acc_t_to_lds<2, 1>(acc, T, LDT, wave * 32, lane);
    __syncthreads();
#pragma unroll
    for (int it = 0; it < (BM * 32) / 256; ++it) {
        const int q = it * 256 + tid;
        const int r = q >> 5, c4 = (q & 31) * 4;
        float4 *t = reinterpret_cast<float4 *>(T + r * LDT + c4);
        float4 v = *t;
        if (save_p && m0 + r < M) *reinterpret_cast<float4 *>(save_p + (m0 + r) * MATRIS_D + c4) = v;
        v.x = silu_f(v.x); v.y = silu_f(v.y); v.z = silu_f(v.z); v.w = silu_f(v.w);
        *t = v;
    }
    __syncthreads();
    zero_acc(acc);
    amax = fmaxf(amax, gemm_lds_packed<MODE, 2, 1, MATRIS_D / 16, true>(acc, T, LDT, W2, wave, MATRIS_D / 16, 0, lane));
    scale_acc<MODE>(acc, w2s);
    __syncthreads();  // every wave is done reading h
    acc_t_to_lds<2, 1>(acc, T, LDT, wave * 32, lane);
    __syncthreads();
    store_tile128(T, out, MATRIS_D, m0, M, tid, res, res_w);
    report_range<MODE>(amax, range_flag);
}

// ------------------------------------------------------------------------------------
// Weight-stationary persistent forms (modes with two fragment planes: 0, 2, 3)
// ------------------------------------------------------------------------------------
// The weights are small (128 x 128 per layer), so each wave keeps its 32 output columns
// of both layers in registers for the whole launch (8 k-blocks x 2 planes x 2 layers =
// 128 VGPRs) and the work-groups loop over 64-row tiles.  The next tile's rows are
// loaded into registers while the current tile computes; a tile is staged into LDS
// already split into fragment planes, once; outputs leave straight from the transposed
// accumulators (lane = row, 16-byte column runs).  With no weight loads inside the loop,
// no load waits behind the previous tile's stores (vmcnt counts both).

// Resident weight fragments of output tile nt (8 k-blocks, two planes) of a packed
// [*, 128] weight.
__device__ __forceinline__ void load_wres(uint4 (&w)[8][2], const uint4 *__restrict__ W, int nt, int lane) {
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
        for (int pl = 0; pl < 2; ++pl) w[kb][pl] = W[((nt * 8 + kb) * 2 + pl) * 64 + lane];
}

// acc += (W tile) * (row tile rt of a fragment buffer)^T over one k-block, W resident.
template <int MODE, int KB>
__device__ __forceinline__ void gemm_res_kb(v16f &acc, const uint4 (&w)[8][2], const uint4 *buf, int rt, int lane) {
    Frag<MODE> wf, a;
    wf.p[0] = w[KB][0];
    wf.p[1] = w[KB][1];
    // MODE 2's derived plane is loop-invariant; made opaque here, it is recomputed at use
    // instead of being hoisted out of the tile loop (64 more live VGPRs)
    if constexpr (MODE == 2) asm volatile("" : "+v"(wf.p[0].x), "+v"(wf.p[0].y), "+v"(wf.p[0].z), "+v"(wf.p[0].w));
    prep_w<MODE>(wf);
    a.p[0] = buf[((rt * 8 + KB) * 2 + 0) * 64 + lane];
    a.p[1] = buf[((rt * 8 + KB) * 2 + 1) * 64 + lane];
    mma_wx<MODE>(acc, wf, a);
}

// The 8 k-blocks, unrolled by hand (constant register indices for the resident weights).
template <int MODE>
__device__ __forceinline__ void gemm_res(v16f &acc, const uint4 (&w)[8][2], const uint4 *buf, int rt, int lane) {
    gemm_res_kb<MODE, 0>(acc, w, buf, rt, lane);
    gemm_res_kb<MODE, 1>(acc, w, buf, rt, lane);
    gemm_res_kb<MODE, 2>(acc, w, buf, rt, lane);
    gemm_res_kb<MODE, 3>(acc, w, buf, rt, lane);
    gemm_res_kb<MODE, 4>(acc, w, buf, rt, lane);
    gemm_res_kb<MODE, 5>(acc, w, buf, rt, lane);
    gemm_res_kb<MODE, 6>(acc, w, buf, rt, lane);
    gemm_res_kb<MODE, 7>(acc, w, buf, rt, lane);
}

// FFN forward, weight-stationary: 512 threads = 8 waves; wave w owns output columns
// [32 (w%4), +32) of both layers and rows [32 (w/4), +32) of each 64-row tile.
template <int MODE>
__global__ __launch_bounds__(512, 1) void ffn_fwd_ws_kernel(int64_t M, const float *__restrict__ x,
                                                            const uint4 *__restrict__ W1,
                                                            const uint4 *__restrict__ W2, float *__restrict__ out,
                                                            float *__restrict__ save_p, const float *__restrict__ res,
                                                            const float *__restrict__ res_w, unsigned *range_flag) {
    static_assert(Npl<MODE>::v == 2, "two-plane modes only");
    __shared__ uint4 Xf[2 * 8 * 2 * 64];  // x tile as fragment planes (32 KB)
    __shared__ uint4 Hf[2 * 8 * 2 * 64];  // h = SiLU(p) tile, the same layout
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
    const int ct = wave & 3, rt = wave >> 2;
    const float w1s = take_wscale<MODE>(W1), w2s = take_wscale<MODE>(W2);
    uint4 w1[8][2], w2[8][2];
    load_wres(w1, W1, ct, lane);
    load_wres(w2, W2, ct, lane);
    const int64_t ntiles = (M + BM - 1) / BM;
    float amax = 0.f;
    float4 xr[4];
    int64_t tile = blockIdx.x;
    load_rows4(xr, x, tile * BM, M, tid);
#pragma unroll 1
    for (; tile < ntiles; tile += gridDim.x) {
        const int64_t m0 = tile * BM;
        amax = stage_rows4<MODE>(Xf, xr, tid, amax);
        __syncthreads();  // x staged; every wave is past the previous tile's GEMM2
        load_rows4(xr, x, min(tile + (int64_t)gridDim.x, ntiles - 1) * BM, M, tid);  // next tile
        v16f acc;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = 0.f;
        gemm_res<MODE>(acc, w1, Xf, rt, lane);
        // p (saved) and h = SiLU(p) into the second fragment buffer: lane (row l32, half h)
        // holds columns 32 ct + 8 j + 4 h .. +3, i.e. half h of fragment unit
        // (rt, k-block 2 ct + j/2), lane l32 + 32 (j%2)
        const int64_t row = m0 + rt * 32 + l32;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float4 v = make_float4(acc[4 * j] * w1s, acc[4 * j + 1] * w1s, acc[4 * j + 2] * w1s, acc[4 * j + 3] * w1s);
            if (save_p && row < M)
                *reinterpret_cast<float4 *>(save_p + row * MATRIS_D + ct * 32 + 8 * j + 4 * h) = v;
            v.x = silu_f(v.x); v.y = silu_f(v.y); v.z = silu_f(v.z); v.w = silu_f(v.w);
            amax = frag_amax<MODE>(amax, v, v);
            frag_put4<MODE>(Hf, rt * 8 + ct * 2 + (j >> 1), l32 + 32 * (j & 1), h, v);
        }
        __syncthreads();  // h complete; every wave is past GEMM1 (Xf free)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = 0.f;
        gemm_res<MODE>(acc, w2, Hf, rt, lane);
        if (row < M) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int col = ct * 32 + 8 * j + 4 * h;
                float4 v = make_float4(acc[4 * j] * w2s, acc[4 * j + 1] * w2s, acc[4 * j + 2] * w2s,
                                       acc[4 * j + 3] * w2s);
                if (res) {
                    const float4 r = *reinterpret_cast<const float4 *>(res + row * MATRIS_D + col);
                    const float4 rw = *reinterpret_cast<const float4 *>(res_w + col);
                    v.x += rw.x * r.x; v.y += rw.y * r.y; v.z += rw.z * r.z; v.w += rw.w * r.w;
                }
                *reinterpret_cast<float4 *>(out + row * MATRIS_D + col) = v;
            }
        }
    }
    report_range<MODE>(amax, range_flag);
}

// x W^T for W of 256 gridDim.y rows, weight-stationary (the projection pair, and
// matris_gmlp_project's column blocks): work-group (x, y) keeps W rows 256y .. 256y+255
// resident (wave w: the 32 columns 32 w .. +31, 64 VGPRs) and loops over 64-row tiles.
// Columns 256y + c go to out0 + 256y + c (c < 128) or out1 + 256y + c - 128, row stride ldo.
template <int MODE>
__global__ __launch_bounds__(512, 1) void proj_ws_kernel(int64_t M, const float *__restrict__ x,
                                                         const uint4 *__restrict__ W, float *__restrict__ out0,
                                                         float *__restrict__ out1, int64_t ldo, unsigned *range_flag) {
    static_assert(Npl<MODE>::v == 2, "two-plane modes only");
    __shared__ uint4 Xf[2 * 8 * 2 * 64];  // x tile as fragment planes (32 KB)
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
    const float ws = take_wscale<MODE>(W);
    uint4 w[8][2];
    load_wres(w, W, 8 * blockIdx.y + wave, lane);
    float *out = (wave < 4 ? out0 + 32 * wave : out1 + 32 * (wave - 4)) + 256 * blockIdx.y + 4 * h;
    const int64_t ntiles = (M + BM - 1) / BM;
    float amax = 0.f;
    float4 xr[4];
    int64_t tile = blockIdx.x;
    load_rows4(xr, x, tile * BM, M, tid);
#pragma unroll 1
    for (; tile < ntiles; tile += gridDim.x) {
        const int64_t m0 = tile * BM;
        amax = stage_rows4<MODE>(Xf, xr, tid, amax);
        __syncthreads();  // x staged
        load_rows4(xr, x, min(tile + (int64_t)gridDim.x, ntiles - 1) * BM, M, tid);  // next tile
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            v16f acc;
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[i] = 0.f;
            gemm_res<MODE>(acc, w, Xf, rt, lane);
            const int64_t row = m0 + rt * 32 + l32;
            if (row < M) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    *reinterpret_cast<float4 *>(out + row * ldo + 8 * j) =
                        make_float4(acc[4 * j] * ws, acc[4 * j + 1] * ws, acc[4 * j + 2] * ws, acc[4 * j + 3] * ws);
            }
        }
        __syncthreads();  // every wave is done reading Xf
    }
    report_range<MODE>(amax, range_flag);
}

// FFN backward, weight-stationary like ffn_fwd_ws_kernel: g_x = ((g W2) * SiLU'(p)) W1 with
// w1t, w2t = packs of W1^T, W2^T resident (wave w: columns 32 (w%4) .. +31 of both, rows
// 32 (w/4) .. +31 of each tile); g_res (optional) = res_w * g, written while g is staged;
// the envelope term (optional) is added to g_x, its rows loaded before the second GEMM.
template <int MODE>
__global__ __launch_bounds__(512, 1) void ffn_bwd_ws_kernel(int64_t M, const float *__restrict__ g,
                                                            const float *__restrict__ P,
                                                            const uint4 *__restrict__ W1t,
                                                            const uint4 *__restrict__ W2t, float *__restrict__ g_x,
                                                            float *__restrict__ g_res,
                                                            const float *__restrict__ res_w, EnvTerm et,
                                                            unsigned *range_flag) {
    static_assert(Npl<MODE>::v == 2, "two-plane modes only");
    __shared__ uint4 Xf[2 * 8 * 2 * 64];  // g tile as fragment planes (32 KB)
    __shared__ uint4 Hf[2 * 8 * 2 * 64];  // g_p tile, the same layout
    __shared__ float rinv[BM];            // MODE 2: 2^-k of each row's g / g_p scaling
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
    const int ct = wave & 3, rt = wave >> 2;
    const float w1s = take_wscale<MODE>(W1t), w2s = take_wscale<MODE>(W2t);
    uint4 w1[8][2], w2[8][2];
    load_wres(w1, W1t, ct, lane);
    load_wres(w2, W2t, ct, lane);
    const int64_t ntiles = (M + BM - 1) / BM;
    float amax = 0.f;
    float4 xr[4];
    int64_t tile = blockIdx.x;
    load_rows4(xr, g, tile * BM, M, tid);
#pragma unroll 1
    for (; tile < ntiles; tile += gridDim.x) {
        const int64_t m0 = tile * BM;
        if (g_res && m0 + (tid >> 3) < M) {  // the thread's row: columns 8 q .. +7 and 64 + 8 q .. +7
            const int q = (tid & 7) * 8;
            float *o = g_res + (m0 + (tid >> 3)) * MATRIS_D;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int col = q + 4 * (i & 1) + 64 * (i >> 1);
                const float4 rw = *reinterpret_cast<const float4 *>(res_w + col);
                *reinterpret_cast<float4 *>(o + col) =
                    make_float4(rw.x * xr[i].x, rw.y * xr[i].y, rw.z * xr[i].z, rw.w * xr[i].w);
            }
        }
        scale_rows4<MODE>(xr, rinv, tid);
        amax = stage_rows4<MODE>(Xf, xr, tid, amax);
        __syncthreads();  // g staged; every wave is past the previous tile's second GEMM
        const float ri = MODE == 2 ? rinv[rt * 32 + l32] : 1.f;  // read before the next tile's staging
        load_rows4(xr, g, min(tile + (int64_t)gridDim.x, ntiles - 1) * BM, M, tid);  // next tile
        v16f acc;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = 0.f;
        gemm_res<MODE>(acc, w2, Xf, rt, lane);
        // g_p = (g W2) * SiLU'(p) into Hf: lane (row l32, half h) holds columns
        // 32 ct + 8 j + 4 h .. +3, half h of unit (rt, k-block 2 ct + j/2), lane l32 + 32 (j%2)
        const int64_t row = m0 + rt * 32 + l32;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = ct * 32 + 8 * j + 4 * h;
            const float4 p = row < M ? *reinterpret_cast<const float4 *>(P + row * MATRIS_D + col)
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
            const float4 v = make_float4(acc[4 * j] * w2s * dsilu_f(p.x), acc[4 * j + 1] * w2s * dsilu_f(p.y),
                                         acc[4 * j + 2] * w2s * dsilu_f(p.z), acc[4 * j + 3] * w2s * dsilu_f(p.w));
            amax = frag_amax<MODE>(amax, v, v);
            frag_put4<MODE>(Hf, rt * 8 + ct * 2 + (j >> 1), l32 + 32 * (j & 1), h, v);
        }
        __syncthreads();  // g_p complete; every wave is past the first GEMM (Xf free)
        float4 ev[4];
        if (et.ge) {
            const int64_t rr = min(row, M - 1);
            const int64_t tr = et.t[rr], sr = et.s[rr];
#pragma unroll
            for (int j = 0; j < 4; ++j) ev[j] = env_term4(et, tr, sr, ct * 32 + 8 * j + 4 * h);
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = 0.f;
        gemm_res<MODE>(acc, w1, Hf, rt, lane);
        if (row < M) {
            const float sc = w1s * ri;  // both powers of two
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float4 v = make_float4(acc[4 * j] * sc, acc[4 * j + 1] * sc, acc[4 * j + 2] * sc, acc[4 * j + 3] * sc);
                if (et.ge) {
                    v.x += ev[j].x; v.y += ev[j].y; v.z += ev[j].z; v.w += ev[j].w;
                }
                *reinterpret_cast<float4 *>(g_x + row * MATRIS_D + ct * 32 + 8 * j + 4 * h) = v;
            }
        }
    }
    report_range<MODE>(amax, range_flag);
}

// ------------------------------------------------------------------------------------
// Three-body embedding (feature_embed.py:151-203 with functions.py:70-95):
//   tb = SiLU(Ws u),  u = Wa b        b = [M, 16] angle basis, Wa [128, 16], Ws [128, 128]
// and its input gradient g_b = Wa^T (Ws^T (g_tb * SiLU'(z))), z = Ws u.  Weight-stationary
// and persistent like ffn_fwd_ws_kernel: u is computed in fp32 while a tile is staged
// (16 FMAs per value, Wa in LDS) and written as fragment units; the backward recomputes u
// and z instead of reading saved activations (the basis is 64 B per row).
// ------------------------------------------------------------------------------------
#define TB_K 16  // basis width: max_n * max_l
// Wa in LDS: row r at r * 16 + (r / 16) * 8 floats, so the 8 lanes that read rows 16 q + c
// (q = 0..7) at one time hit 8 different banks
#define TB_WA_LDS (128 * TB_K + 8 * 8)
__device__ __forceinline__ int tb_wa_row(int r) { return r * TB_K + (r >> 4) * 8; }

__device__ __forceinline__ void stage_wa(float *Wa, const float *__restrict__ wa, int tid) {
    for (int i = tid; i < 128 * TB_K; i += 512) Wa[tb_wa_row(i / TB_K) + i % TB_K] = wa[i];
}

// Basis rows of tile m0 (rows past M read row M-1): thread (row tid/8, all 16 values).
__device__ __forceinline__ void load_basis(float4 (&br)[4], const float *__restrict__ b, int64_t m0, int64_t M,
                                           int tid) {
    const int64_t row = min(m0 + (tid >> 3), M - 1);
    const float4 *p = reinterpret_cast<const float4 *>(b + row * TB_K);
#pragma unroll
    for (int i = 0; i < 4; ++i) br[i] = p[i];
}

// u columns 16 q .. 16 q + 15 (q = tid % 8) of the thread's row, as fragment unit k-block q
// (both halves) of the tile buffer.
template <int MODE>
__device__ __forceinline__ float stage_u(uint4 *buf, const float4 (&br)[4], const float *Wa, int tid, float amax) {
    const int r = tid >> 3, q = tid & 7;
    const float bv[TB_K] = {br[0].x, br[0].y, br[0].z, br[0].w, br[1].x, br[1].y, br[1].z, br[1].w,
                            br[2].x, br[2].y, br[2].z, br[2].w, br[3].x, br[3].y, br[3].z, br[3].w};
    float u[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) {
        const float *w = Wa + tb_wa_row(16 * q + c);
        float t = 0.f;
#pragma unroll
        for (int j = 0; j < TB_K; ++j) t = fmaf(w[j], bv[j], t);
        u[c] = t;
    }
    const int unit = (r >> 5) * 8 + q;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        const float4 a = make_float4(u[8 * hh], u[8 * hh + 1], u[8 * hh + 2], u[8 * hh + 3]);
        const float4 c = make_float4(u[8 * hh + 4], u[8 * hh + 5], u[8 * hh + 6], u[8 * hh + 7]);
        amax = frag_amax<MODE>(amax, a, c);
        frag_put8<MODE>(buf, unit, (r & 31) + 32 * hh, a, c);
    }
    return amax;
}

template <int MODE>
__global__ __launch_bounds__(512, 1) void tb_embed_fwd_kernel(int64_t M, const float *__restrict__ basis,
                                                              const float *__restrict__ wa,
                                                              const uint4 *__restrict__ Ws, float *__restrict__ out,
                                                              unsigned *range_flag) {
    static_assert(Npl<MODE>::v == 2, "two-plane modes only");
    __shared__ uint4 Uf[2 * 8 * 2 * 64];  // u tile as fragment units (32 KB)
    __shared__ __align__(16) float Wa[TB_WA_LDS];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
    const int ct = wave & 3, rt = wave >> 2;
    const float ss = take_wscale<MODE>(Ws);
    stage_wa(Wa, wa, tid);
    uint4 w[8][2];
    load_wres(w, Ws, ct, lane);
    const int64_t ntiles = (M + BM - 1) / BM;
    float amax = 0.f;
    float4 br[4];
    int64_t tile = blockIdx.x;
    load_basis(br, basis, tile * BM, M, tid);
    __syncthreads();  // Wa staged
#pragma unroll 1
    for (; tile < ntiles; tile += gridDim.x) {
        const int64_t m0 = tile * BM;
        amax = stage_u<MODE>(Uf, br, Wa, tid, amax);
        __syncthreads();  // u staged; every wave is past the previous tile's GEMM
        load_basis(br, basis, min(tile + (int64_t)gridDim.x, ntiles - 1) * BM, M, tid);  // next tile
        v16f acc;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = 0.f;
        gemm_res<MODE>(acc, w, Uf, rt, lane);
        const int64_t row = m0 + rt * 32 + l32;
        if (row < M) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 v = make_float4(silu_f(acc[4 * j] * ss), silu_f(acc[4 * j + 1] * ss),
                                             silu_f(acc[4 * j + 2] * ss), silu_f(acc[4 * j + 3] * ss));
                *reinterpret_cast<float4 *>(out + row * MATRIS_D + ct * 32 + 8 * j + 4 * h) = v;
            }
        }
        __syncthreads();  // every wave is done reading Uf
    }
    report_range<MODE>(amax, range_flag);
}

template <int MODE>
__global__ __launch_bounds__(512, 1) void tb_embed_bwd_kernel(int64_t M, const float *__restrict__ basis,
                                                              const float *__restrict__ g_tb,
                                                              const float *__restrict__ wa,
                                                              const uint4 *__restrict__ Ws,
                                                              const uint4 *__restrict__ Wst,
                                                              float *__restrict__ g_basis, unsigned *range_flag) {
    static_assert(Npl<MODE>::v == 2, "two-plane modes only");
    __shared__ uint4 Uf[2 * 8 * 2 * 64];    // u, then g_z, as fragment units (32 KB)
    __shared__ __align__(16) float Wa[TB_WA_LDS];
    __shared__ float part[4][BM][TB_K + 1];  // g_b partial sums per column block (17 KB)
    __shared__ float pmax[4][BM];            // MODE 2: per column block, max |g_z| of each row
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
    const int ct = wave & 3, rt = wave >> 2;
    const float ss = take_wscale<MODE>(Ws), sst = take_wscale<MODE>(Wst);
    stage_wa(Wa, wa, tid);
    uint4 w[8][2], wt[8][2];
    load_wres(w, Ws, ct, lane);
    load_wres(wt, Wst, ct, lane);
    const int64_t ntiles = (M + BM - 1) / BM;
    float amax = 0.f;
    float4 br[4];
    int64_t tile = blockIdx.x;
    load_basis(br, basis, tile * BM, M, tid);
    __syncthreads();  // Wa staged
#pragma unroll 1
    for (; tile < ntiles; tile += gridDim.x) {
        const int64_t m0 = tile * BM;
        amax = stage_u<MODE>(Uf, br, Wa, tid, amax);
        __syncthreads();  // u staged
        load_basis(br, basis, min(tile + (int64_t)gridDim.x, ntiles - 1) * BM, M, tid);  // next tile
        v16f acc;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = 0.f;
        gemm_res<MODE>(acc, w, Uf, rt, lane);  // z (recomputed)
        // g_z = g_tb * SiLU'(z): lane (row rt*32 + l32, half h), columns 32 ct + 8 j + 4 h .. +3
        const int64_t row = m0 + rt * 32 + l32;
        float4 gz[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 g = row < M ? *reinterpret_cast<const float4 *>(g_tb + row * MATRIS_D + ct * 32 + 8 * j + 4 * h)
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
            gz[j] = make_float4(g.x * dsilu_f(acc[4 * j] * ss), g.y * dsilu_f(acc[4 * j + 1] * ss),
                                g.z * dsilu_f(acc[4 * j + 2] * ss), g.w * dsilu_f(acc[4 * j + 3] * ss));
        }
        if constexpr (MODE == 2) {  // the row's maximum over its four column blocks, through LDS
            float m = abs_max4(abs_max4(abs_max4(abs_max4(0.f, gz[0]), gz[1]), gz[2]), gz[3]);
            m = fmaxf(m, __shfl_xor(m, 32, 64));
            if (h == 0) pmax[ct][rt * 32 + l32] = m;
        }
        __syncthreads();  // every wave is done reading u (and the row maxima are complete)
        RowScale rs = {1.f, 1.f};
        if constexpr (MODE == 2) {
            const int r = rt * 32 + l32;
            rs = row_scale(fmaxf(fmaxf(pmax[0][r], pmax[1][r]), fmaxf(pmax[2][r], pmax[3][r])));
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if constexpr (MODE == 2) gz[j] = mul4(gz[j], rs.s);
            amax = frag_amax<MODE>(amax, gz[j], gz[j]);
            frag_put4<MODE>(Uf, rt * 8 + ct * 2 + (j >> 1), l32 + 32 * (j & 1), h, gz[j]);
        }
        __syncthreads();  // g_z complete
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = 0.f;
        gemm_res<MODE>(acc, wt, Uf, rt, lane);  // g_u columns 32 ct + 8 j + 4 h .. +3 of the row
        // g_b partial over this lane's 16 u columns, then over the lane halves
        float gb[TB_K];
#pragma unroll
        for (int k = 0; k < TB_K; ++k) gb[k] = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float gu = acc[i] * (sst * rs.inv);
            const float *wr = Wa + tb_wa_row(ct * 32 + 8 * (i >> 2) + 4 * h + (i & 3));
#pragma unroll
            for (int k = 0; k < TB_K; ++k) gb[k] = fmaf(wr[k], gu, gb[k]);
        }
#pragma unroll
        for (int k = 0; k < TB_K; ++k) {
            const float o = __shfl_xor(gb[k], 32, 64);
            gb[k] = h ? o + gb[k] : gb[k] + o;
        }
        if (h == 0) {
#pragma unroll
            for (int k = 0; k < TB_K; ++k) part[ct][rt * 32 + l32][k] = gb[k];
        }
        __syncthreads();  // partials complete; every wave is done reading g_z
        for (int e = tid; e < BM * TB_K; e += 512) {
            const int r = e >> 4, k = e & 15;
            if (m0 + r < M)
                g_basis[(m0 + r) * TB_K + k] = ((part[0][r][k] + part[1][r][k]) + part[2][r][k]) + part[3][r][k];
        }
        __syncthreads();  // part is read before the next tile overwrites it
    }
    report_range<MODE>(amax, range_flag);
}

// FFN backward: g_x = ((g W2) * SiLU'(p)) W1, with w1t = W1^T, w2t = W2^T row-major.
template <int MODE>
__global__ __launch_bounds__(256, 3) void ffn_bwd_kernel(int64_t M, const float *__restrict__ g,
                                                         const float *__restrict__ P, const uint4 *__restrict__ W1t,
                                                         const uint4 *__restrict__ W2t, float *__restrict__ g_x,
                                                         float *__restrict__ g_res, const float *__restrict__ res_w,
                                                         EnvTerm et, unsigned *range_flag) {
    __shared__ __align__(16) float T[BM * LDT];
    __shared__ float rinv[BM];  // MODE 2: 2^-k of each row's g / g_p scaling
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int h = lane >> 5, l32 = lane & 31;
    const int64_t m0 = (int64_t)blockIdx.x * BM;
    const float w1s = take_wscale<MODE>(W1t), w2s = take_wscale<MODE>(W2t);
    // two-plane modes: g, then g_p, pass through T pre-split into fragment units
    constexpr bool PS = Npl<MODE>::v == 2;
    uint4 *Tf = reinterpret_cast<uint4 *>(T);
    v16f acc[2][1];
    zero_acc(acc);
    float amax = 0.f;
    if constexpr (PS) {
        Rows128 gx;
        load_rows128(gx, g, m0, M, tid);
        if (g_res) store_res128(gx, g_res, res_w, m0, M, tid);
        const float sr = tile_row_scale<MODE>(MODE == 2 ? rows128_absmax(gx) : 0.f, rinv, tid);
        amax = stage_rows128<MODE>(Tf, gx, tid, amax, sr);
        __syncthreads();
        gemm_frag_packed<MODE, 2, 1, MATRIS_D / 16, true>(acc, Tf, MATRIS_D / 16, 0, W2t, wave, MATRIS_D / 16, 0,
                                                          lane);
    } else {
        stage_tile128(T, g, MATRIS_D, m0, M, tid);
        __syncthreads();
        if (g_res) store_tile128_scaled(T, g_res, res_w, m0, M, tid);
        amax = gemm_lds_packed<MODE, 2, 1, MATRIS_D / 16, true>(acc, T, LDT, W2t, wave, MATRIS_D / 16, 0, lane);
    }
    scale_acc<MODE>(acc, w2s);
    // g_p = g_h * SiLU'(p): lane = row, 4 consecutive columns per register group
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        const int64_t row = m0 + rt * 32 + l32;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = wave * 32 + 8 * j + 4 * h;
            const float4 p = row < M ? *reinterpret_cast<const float4 *>(P + row * MATRIS_D + col)
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
            acc[rt][0][4 * j] *= dsilu_f(p.x);
            acc[rt][0][4 * j + 1] *= dsilu_f(p.y);
            acc[rt][0][4 * j + 2] *= dsilu_f(p.z);
            acc[rt][0][4 * j + 3] *= dsilu_f(p.w);
        }
    }
    __syncthreads();  // every wave is done reading g
    if constexpr (PS) {
        // lane (row rt*32 + l32, half h) holds g_p columns 32 wave + 8 j + 4 h .. +3: half h
        // of unit (rt, k-block 2 wave + j/2), lane l32 + 32 (j%2)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 v = make_float4(acc[rt][0][4 * j], acc[rt][0][4 * j + 1], acc[rt][0][4 * j + 2],
                                             acc[rt][0][4 * j + 3]);
                amax = frag_amax<MODE>(amax, v, v);
                frag_put4<MODE>(Tf, rt * 8 + 2 * wave + (j >> 1), l32 + 32 * (j & 1), h, v);
            }
        __syncthreads();
        zero_acc(acc);
        gemm_frag_packed<MODE, 2, 1, MATRIS_D / 16, true>(acc, Tf, MATRIS_D / 16, 0, W1t, wave, MATRIS_D / 16, 0,
                                                          lane);
    } else {
        acc_t_to_lds<2, 1>(acc, T, LDT, wave * 32, lane);
        __syncthreads();
        zero_acc(acc);
        amax = fmaxf(amax,
                     gemm_lds_packed<MODE, 2, 1, MATRIS_D / 16, true>(acc, T, LDT, W1t, wave, MATRIS_D / 16, 0, lane));
    }
    scale_acc<MODE>(acc, w1s);
    unscale_rows_t<MODE, 1>(acc, rinv, l32);
    __syncthreads();
    acc_t_to_lds<2, 1>(acc, T, LDT, wave * 32, lane);
    __syncthreads();
    store_tile128_env(T, g_x, m0, M, tid, et);
    report_range<MODE>(amax, range_flag);
}

// ------------------------------------------------------------------------------------
// projection pair: out0 = x W[0:128]^T, out1 = x W[128:256]^T ; backward
// g_x = g0 W[0:128] + g1 W[128:256]
// The forward also serves W of 256 * gridDim.y rows: block y writes x W[256y : 256y+256]^T
// to columns 256y .. 256y+255 of out0 / out1 (row stride ldo).
// ------------------------------------------------------------------------------------
template <int MODE>
__global__ __launch_bounds__(256, MODE == 6 ? 2 : 3) void pair_fwd_kernel(int64_t M, const float *__restrict__ x,
                                                          const uint4 *__restrict__ W, float *__restrict__ out0,
                                                          float *__restrict__ out1, int64_t ldo,
                                                          unsigned *range_flag) {
    __shared__ __align__(16) float T0[BM * LDT];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int64_t m0 = (int64_t)blockIdx.x * BM;
    const float ws = take_wscale<MODE>(W);
    const int nt0 = 8 * blockIdx.y + 2 * wave;  // first 32-column tile of this wave
    out0 += 256 * blockIdx.y;
    out1 += 256 * blockIdx.y;
    // wave w -> output columns [64w, 64w+64) of the 256: waves 0,1 -> out0, 2,3 -> out1
    v16f acc[2][2];
    zero_acc(acc);
    float amax = 0.f;
    if constexpr (Npl<MODE>::v == 2) {  // x pre-split into fragment units in T0
        uint4 *Tf = reinterpret_cast<uint4 *>(T0);
        amax = stage_frag128<MODE>(Tf, x, m0, M, tid, amax);
        __syncthreads();
        gemm_frag_packed<MODE, 2, 2, MATRIS_D / 16, true>(acc, Tf, MATRIS_D / 16, 0, W, nt0, MATRIS_D / 16, 0, lane);
    } else {
        stage_tile128(T0, x, MATRIS_D, m0, M, tid);
        __syncthreads();
        amax = gemm_lds_packed<MODE, 2, 2, MATRIS_D / 16, true>(acc, T0, LDT, W, nt0, MATRIS_D / 16, 0, lane);
    }
    scale_acc<MODE>(acc, ws);
    // out0 (waves 0, 1), then out1 (waves 2, 3), pass through the one tile
    __syncthreads();  // T0 free
    if (wave < 2) acc_t_to_lds<2, 2>(acc, T0, LDT, (wave & 1) * 64, lane);
    __syncthreads();
    store_tile128(T0, out0, ldo, m0, M, tid);
    __syncthreads();
    if (wave >= 2) acc_t_to_lds<2, 2>(acc, T0, LDT, (wave & 1) * 64, lane);
    __syncthreads();
    store_tile128(T0, out1, ldo, m0, M, tid);
    report_range<MODE>(amax, range_flag);
}

template <int MODE>
__global__ __launch_bounds__(256, 3) void pair_bwd_kernel(int64_t M, const float *__restrict__ g0,
                                                          const float *__restrict__ g1, const uint4 *__restrict__ Wt,
                                                          float *__restrict__ g_x, const float *__restrict__ res,
                                                          const float *__restrict__ res_w, int accumulate,
                                                          unsigned *range_flag) {
    // Wt = W^T ([128, 256]) packed: g_x[m][k] = sum_n g[m][n] Wt[k][n], k-blocks 0..7
    // pair with g0, 8..15 with g1; g0 then g1 pass through the one LDS tile
    __shared__ __align__(16) float T[BM * LDT];
    __shared__ float rinv[BM];  // MODE 2: 2^-k of each row's common g0 / g1 scaling
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int64_t m0 = (int64_t)blockIdx.x * BM;
    const float ws = take_wscale<MODE>(Wt);
    v16f acc[2][1];
    zero_acc(acc);
    float amax = 0.f;
    if constexpr (Npl<MODE>::v == 2) {  // g0, then g1, pre-split into fragment units in T
        uint4 *Tf = reinterpret_cast<uint4 *>(T);
        Rows128 x0, x1;
        load_rows128(x0, g0, m0, M, tid);
        load_rows128(x1, g1, m0, M, tid);
        // one scale per row for both halves: they accumulate into the same sums
        const float sr = tile_row_scale<MODE>(MODE == 2 ? fmaxf(rows128_absmax(x0), rows128_absmax(x1)) : 0.f,
                                              rinv, tid);
        amax = stage_rows128<MODE>(Tf, x0, tid, amax, sr);
        __syncthreads();
        gemm_frag_packed<MODE, 2, 1, MATRIS_D / 16, true>(acc, Tf, MATRIS_D / 16, 0, Wt, wave, 256 / 16, 0, lane);
        __syncthreads();
        amax = stage_rows128<MODE>(Tf, x1, tid, amax, sr);
        __syncthreads();
        gemm_frag_packed<MODE, 2, 1, MATRIS_D / 16, true>(acc, Tf, MATRIS_D / 16, 0, Wt, wave, 256 / 16,
                                                          MATRIS_D / 16, lane);
    } else {
        stage_tile128(T, g0, MATRIS_D, m0, M, tid);
        __syncthreads();
        amax = gemm_lds_packed<MODE, 2, 1, MATRIS_D / 16, true>(acc, T, LDT, Wt, wave, 256 / 16, 0, lane);
        __syncthreads();
        stage_tile128(T, g1, MATRIS_D, m0, M, tid);
        __syncthreads();
        amax = fmaxf(amax, gemm_lds_packed<MODE, 2, 1, MATRIS_D / 16, true>(acc, T, LDT, Wt, wave, 256 / 16,
                                                                            MATRIS_D / 16, lane));
    }
    scale_acc<MODE>(acc, ws);  // both halves share the one weight scale
    unscale_rows_t<MODE, 1>(acc, rinv, lane & 31);
    __syncthreads();
    acc_t_to_lds<2, 1>(acc, T, LDT, wave * 32, lane);
    __syncthreads();
    store_tile128(T, g_x, MATRIS_D, m0, M, tid, res, res_w, accumulate);
    report_range<MODE>(amax, range_flag);
}

// ------------------------------------------------------------------------------------
// Line-graph attention backward with the logit projections' input gradient
// (interaction_block.py:104-134: the two softmaxes' backward, then that of
// source_weight_linear / target_weight_linear, which read the same angle rows): per row r,
// t = t_idx[r], s = s_idx[r],
//   p_t = exp(alpha_t[r] - lse_t[t]),  p_s = exp(alpha_s[r] - lse_s[s])
//   g_e[r]  = base[r] + p_t g_yt[t] + p_s g_ys[s]
//   g_at    = p_t g_yt[t] (e[r] - y_t[t]),  g_as = p_s g_ys[s] (e[r] - y_s[s])
//   g_tb[r] = g_as W_s + g_at W_t + res_w * base[r]
// with Wt the pack matris_pair_bwd takes (k-blocks 0..7 pair with g_as, 8..15 with g_at).
// The logit gradients never reach memory: a 64-row tile converts g_at into pre-split rows
// in LDS (rowfrag_put4) and holds g_as in registers until g_at's product is in, then
// converts g_as into the same rows -- one power-of-two scale per row for both in MODE 2.
// Rows: a half-wave per row, 4 columns per lane, the arithmetic of matris_attn_bwd (g_e is
// the same bits).  Two-plane modes.
// ------------------------------------------------------------------------------------
template <int MODE>
__global__ __launch_bounds__(256, 3) void attn_pair_bwd_kernel(
    int64_t M, const float *__restrict__ alpha_t, const float *__restrict__ alpha_s, int64_t lda,
    const float *__restrict__ e, const int32_t *__restrict__ t_idx, const int32_t *__restrict__ s_idx,
    const float *__restrict__ y_t, const float *__restrict__ y_s, const float *__restrict__ lse_t,
    const float *__restrict__ lse_s, const float *__restrict__ g_yt, const float *__restrict__ g_ys, int64_t ldgy,
    const float *__restrict__ base, const uint4 *__restrict__ Wt, const float *__restrict__ res_w,
    float *__restrict__ g_e, float *__restrict__ g_tb, unsigned *range_flag) {
    static_assert(Npl<MODE>::v == 2, "two-plane modes");
    __shared__ __align__(16) float T[BM * LDT];  // pre-split rows (128 floats of each), then the g_tb tile
    __shared__ float rinv[BM];                   // MODE 2: 2^-k of each row's g_at / g_as scaling
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, half = lane >> 5, l32 = lane & 31;
    const int c = 4 * l32;
    const int64_t m0 = (int64_t)blockIdx.x * BM;
    const float ws = take_wscale<MODE>(Wt);
    float amax = 0.f;
    float4 gs_keep[BM / 8];
#pragma unroll
    for (int i = 0; i < BM / 8; ++i) {
        const int row = wave * (BM / 4) + 2 * i + half;
        const int64_t r = m0 + row;
        const bool in = r < M;
        const int64_t rr = in ? r : M - 1;  // rows past M read row M-1 and count as zeros
        const int64_t t = t_idx[rr], s = s_idx[rr];
        const float4 at = *reinterpret_cast<const float4 *>(alpha_t + rr * lda + c);
        const float4 as = *reinterpret_cast<const float4 *>(alpha_s + rr * lda + c);
        const float4 ev = *reinterpret_cast<const float4 *>(e + rr * MATRIS_D + c);
        const float4 lt = *reinterpret_cast<const float4 *>(lse_t + t * MATRIS_D + c);
        const float4 ls = *reinterpret_cast<const float4 *>(lse_s + s * MATRIS_D + c);
        const float4 gt = *reinterpret_cast<const float4 *>(g_yt + t * ldgy + c);
        const float4 gs = *reinterpret_cast<const float4 *>(g_ys + s * ldgy + c);
        const float4 yt = *reinterpret_cast<const float4 *>(y_t + t * MATRIS_D + c);
        const float4 ys = *reinterpret_cast<const float4 *>(y_s + s * MATRIS_D + c);
        float4 ge = base ? *reinterpret_cast<const float4 *>(base + rr * MATRIS_D + c) : make_float4(0.f, 0.f, 0.f, 0.f);
        float4 gat, gas;
#define ATTN_PAIR_COL(k)                                                       \
    {                                                                          \
        const float pt = exp_neg_f(lt.k - at.k), ps = exp_neg_f(ls.k - as.k); \
        ge.k += pt * gt.k + ps * gs.k;                                         \
        gat.k = pt * gt.k * (ev.k - yt.k);                                     \
        gas.k = ps * gs.k * (ev.k - ys.k);                                     \
    }
        ATTN_PAIR_COL(x) ATTN_PAIR_COL(y) ATTN_PAIR_COL(z) ATTN_PAIR_COL(w)
#undef ATTN_PAIR_COL
        if (in) {
            *reinterpret_cast<float4 *>(g_e + r * MATRIS_D + c) = ge;
        } else {
            gat = gas = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if constexpr (MODE == 2) {  // one scale for the row's 256 values (both sums meet in g_tb)
            float mx = row16_max(abs_max4(abs_max4(0.f, gat), gas));
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            const RowScale rs = row_scale(mx);
            gat = mul4(gat, rs.s);
            gas = mul4(gas, rs.s);
            if (l32 == 0) rinv[row] = rs.inv;
        }
        amax = frag_amax<MODE>(amax, gat, gas);
        rowfrag_put4<MODE>(T + row * LDT, c, gat);
        gs_keep[i] = gas;
        // at most two row pairs of loads in flight: the registers of 16 would spill
        if (i & 1) __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();
    // wave w: g_tb columns [32w, 32w + 32), rows in lanes
    v16f acc[2][1];
    zero_acc(acc);
    gemm_frag_src<MODE, 2, 1, MATRIS_D / 16, true>(acc, AFragRows{T, LDT}, 0, Wt, wave, 256 / 16, MATRIS_D / 16,
                                                   lane);
    __syncthreads();  // every wave is done reading g_at
#pragma unroll
    for (int i = 0; i < BM / 8; ++i) rowfrag_put4<MODE>(T + (wave * (BM / 4) + 2 * i + half) * LDT, c, gs_keep[i]);
    __syncthreads();
    gemm_frag_src<MODE, 2, 1, MATRIS_D / 16, true>(acc, AFragRows{T, LDT}, 0, Wt, wave, 256 / 16, 0, lane);
    scale_acc<MODE>(acc, ws);
    unscale_rows_t<MODE, 1>(acc, rinv, l32);
    __syncthreads();  // every wave is done reading g_as
    acc_t_to_lds<2, 1>(acc, T, LDT, wave * 32, lane);
    __syncthreads();
    store_tile128(T, g_tb, MATRIS_D, m0, M, tid, base, res_w);
    report_range<MODE>(amax, range_flag);
}

// ------------------------------------------------------------------------------------
// C ABI
// ------------------------------------------------------------------------------------
// ------------------------------------------------------------------------------------
// Edge embedding (feature_embed.py:42-148, evaluated once per undirected bond as the
// reference's mean of two identical directed copies is): bond u, d = len[u2d[u]],
//   rbf6 = B_6(d), rbf4 = B_4(d)   (the enveloped Bessel bases of the two cutoffs, out)
//   h1 = rbf6 W1^T [7 -> 128],  h2 = h1 W2^T,  y = LayerNorm(h2) (gamma, beta, eps),
//   e = SiLU(y Ws^T)
// The forward saves h3 = y Ws^T, xhat = (h2 - mu) / sigma and 1 / sigma per bond; the
// backward returns the length gradient through every path (e, rbf6 and rbf4 are each
// read by later layers), written at row u2d[u] of g_len.
// ------------------------------------------------------------------------------------
#define EE_NR 7  // radial functions per cutoff (num_radial)

struct EdgeEmbedArgs {
    const float *len;
    const int32_t *u2d;
    const float *f6, *f4;  // frequencies of the two bases [EE_NR]
    BesselParams P6, P4;
    float rc6, rc4;
    const float *w1;  // [128, EE_NR] fp32 (Linear(7, 128).weight)
    const float *ln_g, *ln_b;
    float eps;
};

__device__ __forceinline__ float group4_sum(float v) {
    v += dpp_f<0xB1>(v);  // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);  // quad_perm [2,3,0,1]
    return v;
}

// W1 into LDS: W1s[j * EE_NR + k] = W1[j][k]
__device__ __forceinline__ void ee_stage_w1(float *W1s, const float *__restrict__ w1, int tid) {
    for (int i = tid; i < MATRIS_D * EE_NR; i += 256) W1s[i] = w1[i];
}

// A thread's 32 columns of row tid/4 in the Rows128 layout, from / to an LDS tile.
__device__ __forceinline__ void ee_tile_get(Rows128 &x, const float *T, int tid) {
    const int r = tid >> 2, q = tid & 3;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float *p = T + r * LDT + 8 * (q + 4 * i);
        x.u[i] = *reinterpret_cast<const float4 *>(p);
        x.v[i] = *reinterpret_cast<const float4 *>(p + 4);
    }
}
__device__ __forceinline__ void ee_tile_put(float *T, const Rows128 &x, int tid) {
    const int r = tid >> 2, q = tid & 3;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float *p = T + r * LDT + 8 * (q + 4 * i);
        *reinterpret_cast<float4 *>(p) = x.u[i];
        *reinterpret_cast<float4 *>(p + 4) = x.v[i];
    }
}

template <int MODE>
__global__ __launch_bounds__(256, 3) void edge_embed_fwd_kernel(int64_t M, EdgeEmbedArgs a,
                                                                const uint4 *__restrict__ W2,
                                                                const uint4 *__restrict__ Ws, float *__restrict__ e,
                                                                float *__restrict__ rbf6, float *__restrict__ rbf4,
                                                                float *__restrict__ save_h3,
                                                                float *__restrict__ save_xhat,
                                                                float *__restrict__ save_rstd, unsigned *range_flag) {
    __shared__ __align__(16) float T[BM * LDT];
    __shared__ float R[BM][EE_NR];
    __shared__ float W1s[MATRIS_D * EE_NR];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r = tid >> 2, q = tid & 3;
    const int64_t m0 = (int64_t)blockIdx.x * BM;
    const float w2s = take_wscale<MODE>(W2), wss = take_wscale<MODE>(Ws);
    ee_stage_w1(W1s, a.w1, tid);
    if (tid < BM) {
        const int64_t u = m0 + tid;
        float b6[EE_NR], b4[EE_NR];
        if (u < M) {
            const float d = a.len[a.u2d[u]];
            bessel_row(d, EE_NR, a.f6, a.P6, a.rc6, b6);
            bessel_row(d, EE_NR, a.f4, a.P4, a.rc4, b4);
#pragma unroll
            for (int k = 0; k < EE_NR; ++k) {
                rbf6[u * EE_NR + k] = b6[k];
                rbf4[u * EE_NR + k] = b4[k];
            }
        } else {
#pragma unroll
            for (int k = 0; k < EE_NR; ++k) b6[k] = 0.f;
        }
#pragma unroll
        for (int k = 0; k < EE_NR; ++k) R[tid][k] = b6[k];
    }
    __syncthreads();
    {  // h1 = rbf6 W1^T
        float b[EE_NR];
#pragma unroll
        for (int k = 0; k < EE_NR; ++k) b[k] = R[r][k];
        Rows128 h;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c0 = 8 * (q + 4 * i);
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float t = 0.f;
#pragma unroll
                for (int k = 0; k < EE_NR; ++k) t = fmaf(b[k], W1s[(c0 + j) * EE_NR + k], t);
                v[j] = t;
            }
            h.u[i] = make_float4(v[0], v[1], v[2], v[3]);
            h.v[i] = make_float4(v[4], v[5], v[6], v[7]);
        }
        ee_tile_put(T, h, tid);
    }
    __syncthreads();
    v16f acc[2][1];
    zero_acc(acc);
    float amax = gemm_lds_packed<MODE, 2, 1, MATRIS_D / 16, true>(acc, T, LDT, W2, wave, MATRIS_D / 16, 0, lane);
    scale_acc<MODE>(acc, w2s);
    __syncthreads();  // every wave is done reading h1
    acc_t_to_lds<2, 1>(acc, T, LDT, wave * 32, lane);
    __syncthreads();
    {  // LayerNorm over the row (4 threads per row), y back to the tile
        Rows128 x;
        ee_tile_get(x, T, tid);
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            s += (x.u[i].x + x.u[i].y + x.u[i].z + x.u[i].w) + (x.v[i].x + x.v[i].y + x.v[i].z + x.v[i].w);
        const float mu = group4_sum(s) * (1.0f / MATRIS_D);
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 du = make_float4(x.u[i].x - mu, x.u[i].y - mu, x.u[i].z - mu, x.u[i].w - mu);
            const float4 dv = make_float4(x.v[i].x - mu, x.v[i].y - mu, x.v[i].z - mu, x.v[i].w - mu);
            ss += (du.x * du.x + du.y * du.y + du.z * du.z + du.w * du.w) +
                  (dv.x * dv.x + dv.y * dv.y + dv.z * dv.z + dv.w * dv.w);
            x.u[i] = du;
            x.v[i] = dv;
        }
        const float rstd = rsqrtf(group4_sum(ss) * (1.0f / MATRIS_D) + a.eps);
        const bool in = m0 + r < M;
        if (in && q == 0) save_rstd[m0 + r] = rstd;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c0 = 8 * (q + 4 * i);
            const float4 xu = mul4(x.u[i], rstd), xv = mul4(x.v[i], rstd);
            if (in) {
                st_nt4(save_xhat + (m0 + r) * MATRIS_D + c0, xu);
                st_nt4(save_xhat + (m0 + r) * MATRIS_D + c0 + 4, xv);
            }
            const float4 gu = *reinterpret_cast<const float4 *>(a.ln_g + c0);
            const float4 gv = *reinterpret_cast<const float4 *>(a.ln_g + c0 + 4);
            const float4 bu = *reinterpret_cast<const float4 *>(a.ln_b + c0);
            const float4 bv = *reinterpret_cast<const float4 *>(a.ln_b + c0 + 4);
            x.u[i] = make_float4(xu.x * gu.x + bu.x, xu.y * gu.y + bu.y, xu.z * gu.z + bu.z, xu.w * gu.w + bu.w);
            x.v[i] = make_float4(xv.x * gv.x + bv.x, xv.y * gv.y + bv.y, xv.z * gv.z + bv.z, xv.w * gv.w + bv.w);
        }
        ee_tile_put(T, x, tid);  // the thread's own columns: no other thread reads them here
    }
    __syncthreads();
    zero_acc(acc);
    amax = fmaxf(amax, gemm_lds_packed<MODE, 2, 1, MATRIS_D / 16, true>(acc, T, LDT, Ws, wave, MATRIS_D / 16, 0, lane));
    scale_acc<MODE>(acc, wss);
    __syncthreads();  // every wave is done reading y
    acc_t_to_lds<2, 1>(acc, T, LDT, wave * 32, lane);
    __syncthreads();
#pragma unroll
    for (int it = 0; it < (BM * 32) / 256; ++it) {
        const int qq = it * 256 + tid;
        const int rr = qq >> 5, c4 = (qq & 31) * 4;
        if (m0 + rr < M) {
            const float4 v = *reinterpret_cast<const float4 *>(T + rr * LDT + c4);
            st_nt4(save_h3 + (m0 + rr) * MATRIS_D + c4, v);
            *reinterpret_cast<float4 *>(e + (m0 + rr) * MATRIS_D + c4) =
                make_float4(silu_f(v.x), silu_f(v.y), silu_f(v.z), silu_f(v.w));
        }
    }
    report_range<MODE>(amax, range_flag);
}

// One backward GEMM of the edge embedding: acc = rows W (W the pack of a transposed
// weight), the rows scaled per row in MODE 2 (rinv receives 2^-k), staged pre-split in
// the two-plane modes.  Leaves the result unscaled in the tile T (fp32, [64, 128]).
template <int MODE>
__device__ __forceinline__ float ee_bwd_gemm(float *T, float *rinv, const Rows128 &x, const uint4 *__restrict__ W,
                                             int tid, int wave, int lane, float amax) {
    constexpr bool PS = Npl<MODE>::v == 2;
    uint4 *Tf = reinterpret_cast<uint4 *>(T);
    const float ws = take_wscale<MODE>(W);
    const float sr = tile_row_scale<MODE>(MODE == 2 ? rows128_absmax(x) : 0.f, rinv, tid);
    v16f acc[2][1];
    zero_acc(acc);
    if constexpr (PS) {
        amax = stage_rows128<MODE>(Tf, x, tid, amax, sr);
        __syncthreads();
        gemm_frag_packed<MODE, 2, 1, MATRIS_D / 16, true>(acc, Tf, MATRIS_D / 16, 0, W, wave, MATRIS_D / 16, 0, lane);
    } else {
        ee_tile_put(T, x, tid);
        __syncthreads();
        amax = fmaxf(amax, gemm_lds_packed<MODE, 2, 1, MATRIS_D / 16, true>(acc, T, LDT, W, wave, MATRIS_D / 16, 0,
                                                                            lane));
    }
    scale_acc<MODE>(acc, ws);
    unscale_rows_t<MODE, 1>(acc, rinv, lane & 31);
    __syncthreads();  // every wave is done reading the operand (and rinv)
    acc_t_to_lds<2, 1>(acc, T, LDT, wave * 32, lane);
    __syncthreads();
    return amax;
}

template <int MODE>
__global__ __launch_bounds__(256, 3) void edge_embed_bwd_kernel(int64_t M, EdgeEmbedArgs a,
                                                                const uint4 *__restrict__ Wst,
                                                                const uint4 *__restrict__ W2t,
                                                                const float *__restrict__ g_e,
                                                                const float *__restrict__ g_rbf6,
                                                                const float *__restrict__ g_rbf4,
                                                                const float *__restrict__ save_h3,
                                                                const float *__restrict__ save_xhat,
                                                                const float *__restrict__ save_rstd,
                                                                float *__restrict__ g_len, unsigned *range_flag) {
    __shared__ __align__(16) float T[BM * LDT];
    __shared__ float rinv[BM];
    __shared__ float W1s[MATRIS_D * EE_NR];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r = tid >> 2, q = tid & 3;
    const int64_t m0 = (int64_t)blockIdx.x * BM;
    const bool in = m0 + r < M;
    ee_stage_w1(W1s, a.w1, tid);
    // g_h3 = g_e * SiLU'(h3)
    Rows128 g, h;
    load_rows128(g, g_e, m0, M, tid);
    load_rows128(h, save_h3, m0, M, tid);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        g.u[i] = make_float4(g.u[i].x * dsilu_f(h.u[i].x), g.u[i].y * dsilu_f(h.u[i].y), g.u[i].z * dsilu_f(h.u[i].z),
                             g.u[i].w * dsilu_f(h.u[i].w));
        g.v[i] = make_float4(g.v[i].x * dsilu_f(h.v[i].x), g.v[i].y * dsilu_f(h.v[i].y), g.v[i].z * dsilu_f(h.v[i].z),
                             g.v[i].w * dsilu_f(h.v[i].w));
    }
    load_rows128(h, save_xhat, m0, M, tid);  // xhat, for the LayerNorm backward
    const float rstd = in ? save_rstd[m0 + r] : 0.f;
    float amax = ee_bwd_gemm<MODE>(T, rinv, g, Wst, tid, wave, lane, 0.f);  // g_y = g_h3 Ws
    {  // LayerNorm backward: g_xhat = g_y gamma, g_h2 = rstd (g_xhat - mean(g_xhat) - xhat mean(g_xhat xhat))
        ee_tile_get(g, T, tid);
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c0 = 8 * (q + 4 * i);
            const float4 gu = *reinterpret_cast<const float4 *>(a.ln_g + c0);
            const float4 gv = *reinterpret_cast<const float4 *>(a.ln_g + c0 + 4);
            g.u[i] = make_float4(g.u[i].x * gu.x, g.u[i].y * gu.y, g.u[i].z * gu.z, g.u[i].w * gu.w);
            g.v[i] = make_float4(g.v[i].x * gv.x, g.v[i].y * gv.y, g.v[i].z * gv.z, g.v[i].w * gv.w);
            s1 += (g.u[i].x + g.u[i].y + g.u[i].z + g.u[i].w) + (g.v[i].x + g.v[i].y + g.v[i].z + g.v[i].w);
            s2 += (g.u[i].x * h.u[i].x + g.u[i].y * h.u[i].y + g.u[i].z * h.u[i].z + g.u[i].w * h.u[i].w) +
                  (g.v[i].x * h.v[i].x + g.v[i].y * h.v[i].y + g.v[i].z * h.v[i].z + g.v[i].w * h.v[i].w);
        }
        const float m1 = group4_sum(s1) * (1.0f / MATRIS_D), m2 = group4_sum(s2) * (1.0f / MATRIS_D);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            g.u[i] = make_float4(rstd * (g.u[i].x - m1 - h.u[i].x * m2), rstd * (g.u[i].y - m1 - h.u[i].y * m2),
                                 rstd * (g.u[i].z - m1 - h.u[i].z * m2), rstd * (g.u[i].w - m1 - h.u[i].w * m2));
            g.v[i] = make_float4(rstd * (g.v[i].x - m1 - h.v[i].x * m2), rstd * (g.v[i].y - m1 - h.v[i].y * m2),
                                 rstd * (g.v[i].z - m1 - h.v[i].z * m2), rstd * (g.v[i].w - m1 - h.v[i].w * m2));
        }
        __syncthreads();  // every thread has read g_y from the tile the next operand overwrites
    }
    amax = ee_bwd_gemm<MODE>(T, rinv, g, W2t, tid, wave, lane, amax);  // g_h1 = g_h2 W2
    // g_rbf6 = g_h1 W1 (+ its other readers' gradient); the length through both bases
    float p[EE_NR];
#pragma unroll
    for (int k = 0; k < EE_NR; ++k) p[k] = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c0 = 8 * (q + 4 * i);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float gv = T[r * LDT + c0 + j];
#pragma unroll
            for (int k = 0; k < EE_NR; ++k) p[k] = fmaf(gv, W1s[(c0 + j) * EE_NR + k], p[k]);
        }
    }
#pragma unroll
    for (int k = 0; k < EE_NR; ++k) p[k] = group4_sum(p[k]);
    if (in && q == 0) {
        const int64_t u = m0 + r;
        const int64_t ei = a.u2d[u];
        const float d = a.len[ei];
        if (g_rbf6) {
#pragma unroll
            for (int k = 0; k < EE_NR; ++k) p[k] += g_rbf6[u * EE_NR + k];
        }
        float gd = bessel_row_grad(d, EE_NR, a.f6, a.P6, a.rc6, p);
        if (g_rbf4) {
            float g4[EE_NR];
#pragma unroll
            for (int k = 0; k < EE_NR; ++k) g4[k] = g_rbf4[u * EE_NR + k];
            gd += bessel_row_grad(d, EE_NR, a.f4, a.P4, a.rc4, g4);
        }
        g_len[ei] = gd;
    }
    report_range<MODE>(amax, range_flag);
}

#define MLP_DISPATCH(KERNEL, ...)                                                         \
    do {                                                                                  \
        unsigned *flag_ = nullptr;                                                        \
        if (mode == 2 && !(flag_ = matris_range_flag())) return MATRIS_E_ARG;             \
        const dim3 grid_(matris_blocks(m, BM));                                           \
        hipStream_t st_ = (hipStream_t)stream;                                            \
        MATRIS_MODE_DISPATCH(KERNEL, grid_, st_, __VA_ARGS__, flag_);                     \
    } while (0)

static bool mlp_args_ok(int mode, std::initializer_list<const void *> ptrs) {
    if (!matris_mode_ok(mode)) return false;
    for (const void *p : ptrs)
        if (!p || ((uintptr_t)p & 15)) return false;
    return true;
}

// The weight-stationary FFN backward and projection pair pay their per-work-group weight
// load back only over many row tiles: below this many rows the tiled kernels are as fast
// or faster (C3's bond and edge layers, 34k-67k rows, measured on MI355X); the FFN
// forward is weight-stationary at every size.
static bool weight_stationary(int64_t m) { return m >= (int64_t(1) << 17); }

// Work-groups of a persistent launch: one 512-thread work-group per CU (the register
// budget of the weight-stationary kernels), never more than the tiles.
static dim3 persistent_grid(int64_t m) {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (!cus[dev] && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus[dev] = 256;
    const int64_t tiles = matris_blocks(m, BM);
    return dim3((unsigned)std::min<int64_t>(tiles, (int64_t)cus[dev]));
}

extern "C" int matris_ffn_fwd(int64_t m, const float *x, const void *w1p, const void *w2p, float *out,
                              float *save_p, const float *res, const float *res_w, int mode, void *stream) {
    if (m < 0 || !mlp_args_ok(mode, {x, w1p, w2p, out}) || ((uintptr_t)save_p & 15)) return MATRIS_E_ARG;
    if (res && (((uintptr_t)res & 15) || !res_w || ((uintptr_t)res_w & 15))) return MATRIS_E_ARG;
    if (m == 0) return 0;
    if (mode == 6) {
        MLP_DISPATCH(ffn_fwd_kernel, m, x, (const uint4 *)w1p, (const uint4 *)w2p, out, save_p, res, res_w);
    } else {
        unsigned *flag = nullptr;
        if (mode == 2 && !(flag = matris_range_flag())) return MATRIS_E_ARG;
        const dim3 grid = persistent_grid(m);
        hipStream_t st = (hipStream_t)stream;
        if (mode == 0)
            ffn_fwd_ws_kernel<0><<<grid, 512, 0, st>>>(m, x, (const uint4 *)w1p, (const uint4 *)w2p, out, save_p, res,
                                                       res_w, flag);
        else if (mode == 2)
            ffn_fwd_ws_kernel<2><<<grid, 512, 0, st>>>(m, x, (const uint4 *)w1p, (const uint4 *)w2p, out, save_p, res,
                                                       res_w, flag);
        else
            ffn_fwd_ws_kernel<3><<<grid, 512, 0, st>>>(m, x, (const uint4 *)w1p, (const uint4 *)w2p, out, save_p, res,
                                                       res_w, flag);
    }
    MATRIS_CHECK_LAUNCH();
    return 0;
}

static int ffn_bwd_launch(int64_t m, const float *g, const float *p, const void *w1tp, const void *w2tp, float *g_x,
                          float *g_res, const float *res_w, const EnvTerm &et, int mode, void *stream) {
    if (m < 0 || !mlp_args_ok(mode, {g, p, w1tp, w2tp, g_x})) return MATRIS_E_ARG;
    if (g_res && (((uintptr_t)g_res & 15) || !res_w || ((uintptr_t)res_w & 15))) return MATRIS_E_ARG;
    if (m == 0) return 0;
    if (mode == 6 || !weight_stationary(m)) {
        MLP_DISPATCH(ffn_bwd_kernel, m, g, p, (const uint4 *)w1tp, (const uint4 *)w2tp, g_x, g_res, res_w, et);
    } else {
        unsigned *flag = nullptr;
        if (mode == 2 && !(flag = matris_range_flag())) return MATRIS_E_ARG;
        const dim3 grid = persistent_grid(m);
        hipStream_t st = (hipStream_t)stream;
        const uint4 *w1t = (const uint4 *)w1tp, *w2t = (const uint4 *)w2tp;
        if (mode == 0)
            ffn_bwd_ws_kernel<0><<<grid, 512, 0, st>>>(m, g, p, w1t, w2t, g_x, g_res, res_w, et, flag);
        else if (mode == 2)
            ffn_bwd_ws_kernel<2><<<grid, 512, 0, st>>>(m, g, p, w1t, w2t, g_x, g_res, res_w, et, flag);
        else
            ffn_bwd_ws_kernel<3><<<grid, 512, 0, st>>>(m, g, p, w1t, w2t, g_x, g_res, res_w, et, flag);
    }
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_ffn_bwd(int64_t m, const float *g, const float *p, const void *w1tp, const void *w2tp,
                              float *g_x, float *g_res, const float *res_w, int mode, void *stream) {
    return ffn_bwd_launch(m, g, p, w1tp, w2tp, g_x, g_res, res_w, EnvTerm{nullptr, nullptr, nullptr, nullptr}, mode,
                          stream);
}

extern "C" int matris_ffn_bwd_env(int64_t m, const float *g, const float *p, const void *w1tp, const void *w2tp,
                                  float *g_x, const float *g_agg_env, const float *env, const int32_t *t_idx,
                                  const int32_t *s_idx, int mode, void *stream) {
    if (!g_agg_env || !env || !t_idx || !s_idx || ((uintptr_t)g_agg_env & 15) || ((uintptr_t)env & 15))
        return MATRIS_E_ARG;
    return ffn_bwd_launch(m, g, p, w1tp, w2tp, g_x, nullptr, nullptr, EnvTerm{g_agg_env, env, t_idx, s_idx}, mode,
                          stream);
}

extern "C" int matris_pair_fwd(int64_t m, const float *x, const void *wp, float *out0, float *out1, int mode,
                               void *stream) {
    if (m < 0 || !mlp_args_ok(mode, {x, wp, out0, out1})) return MATRIS_E_ARG;
    if (m == 0) return 0;
    if (mode == 6 || !weight_stationary(m)) {
        MLP_DISPATCH(pair_fwd_kernel, m, x, (const uint4 *)wp, out0, out1, (int64_t)MATRIS_D);
    } else {
        unsigned *flag = nullptr;
        if (mode == 2 && !(flag = matris_range_flag())) return MATRIS_E_ARG;
        const dim3 grid = persistent_grid(m);
        hipStream_t st = (hipStream_t)stream;
        const uint4 *w = (const uint4 *)wp;
        const int64_t ld = MATRIS_D;
        if (mode == 0)
            proj_ws_kernel<0><<<grid, 512, 0, st>>>(m, x, w, out0, out1, ld, flag);
        else if (mode == 2)
            proj_ws_kernel<2><<<grid, 512, 0, st>>>(m, x, w, out0, out1, ld, flag);
        else
            proj_ws_kernel<3><<<grid, 512, 0, st>>>(m, x, w, out0, out1, ld, flag);
    }
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_gmlp_project(int64_t m, const float *x, const void *wp, int n_blk, float *out, int mode,
                                   void *stream) {
    if (m < 0 || n_blk < 1 || n_blk > 4 || !mlp_args_ok(mode, {x, wp, out})) return MATRIS_E_ARG;
    if (m == 0) return 0;
    unsigned *flag = nullptr;
    if (mode == 2 && !(flag = matris_range_flag())) return MATRIS_E_ARG;
    hipStream_t st = (hipStream_t)stream;
    const int64_t ldo = 256 * (int64_t)n_blk;
    if (mode == 6) {
        const dim3 grid(matris_blocks(m, BM), n_blk);
        MATRIS_MODE_DISPATCH(pair_fwd_kernel, grid, st, m, x, (const uint4 *)wp, out, out + MATRIS_D, ldo, flag);
    } else {
        // one 512-thread work-group per CU in total, split over the column blocks
        const dim3 pg = persistent_grid(m);
        const dim3 grid(std::max(1u, pg.x / (unsigned)n_blk), n_blk);
        const uint4 *w = (const uint4 *)wp;
        if (mode == 0)
            proj_ws_kernel<0><<<grid, 512, 0, st>>>(m, x, w, out, out + MATRIS_D, ldo, flag);
        else if (mode == 2)
            proj_ws_kernel<2><<<grid, 512, 0, st>>>(m, x, w, out, out + MATRIS_D, ldo, flag);
        else
            proj_ws_kernel<3><<<grid, 512, 0, st>>>(m, x, w, out, out + MATRIS_D, ldo, flag);
    }
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_pair_bwd(int64_t m, const float *g0, const float *g1, const void *wtp, float *g_x,
                               const float *res, const float *res_w, int accumulate, int mode, void *stream) {
    if (m < 0 || !mlp_args_ok(mode, {g0, g1, wtp, g_x})) return MATRIS_E_ARG;
    if (res && (((uintptr_t)res & 15) || !res_w || ((uintptr_t)res_w & 15))) return MATRIS_E_ARG;
    if (m == 0) return 0;
    MLP_DISPATCH(pair_bwd_kernel, m, g0, g1, (const uint4 *)wtp, g_x, res, res_w, accumulate);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_attn_pair_bwd(int64_t n_rows, const float *alpha_t, const float *alpha_s, int64_t lda,
                                    const float *e, const int32_t *t_idx, const int32_t *s_idx, const float *y_t,
                                    const float *y_s, const float *lse_t, const float *lse_s, const float *g_yt,
                                    const float *g_ys, int64_t ldgy, const float *base, const void *wtp,
                                    const float *res_w, int mode, float *g_e, float *g_tb, void *stream) {
    if (n_rows < 0 || (mode != 0 && mode != 2 && mode != 3)) return MATRIS_E_ARG;
    if (lda < MATRIS_D || (lda % 4) || ldgy < MATRIS_D || (ldgy % 4)) return MATRIS_E_ARG;
    if (!mlp_args_ok(mode, {alpha_t, alpha_s, e, y_t, y_s, lse_t, lse_s, g_yt, g_ys, wtp, g_e, g_tb}) || !t_idx ||
        !s_idx)
        return MATRIS_E_ARG;
    if ((base && ((uintptr_t)base & 15)) || (res_w && (!base || ((uintptr_t)res_w & 15)))) return MATRIS_E_ARG;
    if (n_rows == 0) return 0;
    unsigned *flag = nullptr;
    if (mode == 2 && !(flag = matris_range_flag())) return MATRIS_E_ARG;
    const dim3 grid(matris_blocks(n_rows, BM));
    hipStream_t st = (hipStream_t)stream;
    const uint4 *w = (const uint4 *)wtp;
#define ATTN_PAIR_ARGS n_rows, alpha_t, alpha_s, lda, e, t_idx, s_idx, y_t, y_s, lse_t, lse_s, g_yt, g_ys, ldgy, base, w, \
                       res_w, g_e, g_tb, flag
    if (mode == 0)
        attn_pair_bwd_kernel<0><<<grid, 256, 0, st>>>(ATTN_PAIR_ARGS);
    else if (mode == 2)
        attn_pair_bwd_kernel<2><<<grid, 256, 0, st>>>(ATTN_PAIR_ARGS);
    else
        attn_pair_bwd_kernel<3><<<grid, 256, 0, st>>>(ATTN_PAIR_ARGS);
#undef ATTN_PAIR_ARGS
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_tb_embed_fwd(int64_t m, const float *basis, const float *wa, const void *wsp, float *out,
                                   int mode, void *stream) {
    if (m < 0 || (mode != 0 && mode != 2 && mode != 3) || !mlp_args_ok(mode, {basis, wa, wsp, out}))
        return MATRIS_E_ARG;
    if (m == 0) return 0;
    unsigned *flag = nullptr;
    if (mode == 2 && !(flag = matris_range_flag())) return MATRIS_E_ARG;
    const dim3 grid = persistent_grid(m);
    hipStream_t st = (hipStream_t)stream;
    const uint4 *ws = (const uint4 *)wsp;
    if (mode == 0)
        tb_embed_fwd_kernel<0><<<grid, 512, 0, st>>>(m, basis, wa, ws, out, flag);
    else if (mode == 2)
        tb_embed_fwd_kernel<2><<<grid, 512, 0, st>>>(m, basis, wa, ws, out, flag);
    else
        tb_embed_fwd_kernel<3><<<grid, 512, 0, st>>>(m, basis, wa, ws, out, flag);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_tb_embed_bwd(int64_t m, const float *basis, const float *g_tb, const float *wa,
                                   const void *wsp, const void *wstp, float *g_basis, int mode, void *stream) {
    if (m < 0 || (mode != 0 && mode != 2 && mode != 3) || !mlp_args_ok(mode, {basis, g_tb, wa, wsp, wstp, g_basis}))
        return MATRIS_E_ARG;
    if (m == 0) return 0;
    unsigned *flag = nullptr;
    if (mode == 2 && !(flag = matris_range_flag())) return MATRIS_E_ARG;
    const dim3 grid = persistent_grid(m);
    hipStream_t st = (hipStream_t)stream;
    const uint4 *ws = (const uint4 *)wsp, *wst = (const uint4 *)wstp;
    if (mode == 0)
        tb_embed_bwd_kernel<0><<<grid, 512, 0, st>>>(m, basis, g_tb, wa, ws, wst, g_basis, flag);
    else if (mode == 2)
        tb_embed_bwd_kernel<2><<<grid, 512, 0, st>>>(m, basis, g_tb, wa, ws, wst, g_basis, flag);
    else
        tb_embed_bwd_kernel<3><<<grid, 512, 0, st>>>(m, basis, g_tb, wa, ws, wst, g_basis, flag);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

static bool edge_embed_args(EdgeEmbedArgs &a, int64_t n_bonds, const float *edge_len, const int32_t *u2d,
                            const float *freq6, double cutoff6, const float *freq4, double cutoff4, int num_radial,
                            double envelope_exponent, const float *w1, const float *ln_g, const float *ln_b,
                            double ln_eps) {
    if (n_bonds < 0 || num_radial != EE_NR || !(cutoff6 > 0) || !(cutoff4 > 0) || !(envelope_exponent > 0) ||
        !edge_len || !u2d || !freq6 || !freq4 || !w1 || !ln_g || ((uintptr_t)ln_g & 15) ||
        (ln_b && ((uintptr_t)ln_b & 15)))
        return false;
    a = EdgeEmbedArgs{edge_len, u2d, freq6, freq4, bessel_params(cutoff6, envelope_exponent),
                      bessel_params(cutoff4, envelope_exponent), (float)cutoff6, (float)cutoff4, w1, ln_g, ln_b,
                      (float)ln_eps};
    return true;
}

extern "C" int matris_edge_embed_fwd(int64_t n_bonds, const float *edge_len, const int32_t *u2d, const float *freq6,
                                     double cutoff6, const float *freq4, double cutoff4, int num_radial,
                                     double envelope_exponent, const float *w1, const void *w2p, const float *ln_g,
                                     const float *ln_b, double ln_eps, const void *wsp, float *e, float *rbf6,
                                     float *rbf4, float *save_h3, float *save_xhat, float *save_rstd, int mode,
                                     void *stream) {
    EdgeEmbedArgs a;
    if (!edge_embed_args(a, n_bonds, edge_len, u2d, freq6, cutoff6, freq4, cutoff4, num_radial, envelope_exponent,
                         w1, ln_g, ln_b, ln_eps) ||
        !ln_b || !mlp_args_ok(mode, {w2p, wsp, e, save_h3, save_xhat}) || !rbf6 || !rbf4 || !save_rstd)
        return MATRIS_E_ARG;
    const int64_t m = n_bonds;
    if (m == 0) return 0;
    MLP_DISPATCH(edge_embed_fwd_kernel, m, a, (const uint4 *)w2p, (const uint4 *)wsp, e, rbf6, rbf4, save_h3, save_xhat,
                 save_rstd);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_edge_embed_bwd(int64_t n_bonds, const float *edge_len, const int32_t *u2d, const float *freq6,
                                     double cutoff6, const float *freq4, double cutoff4, int num_radial,
                                     double envelope_exponent, const float *w1, const void *w2tp, const float *ln_g,
                                     const void *wstp, const float *g_e, const float *g_rbf6, const float *g_rbf4,
                                     const float *save_h3, const float *save_xhat, const float *save_rstd,
                                     float *g_len, int mode, void *stream) {
    EdgeEmbedArgs a;
    if (!edge_embed_args(a, n_bonds, edge_len, u2d, freq6, cutoff6, freq4, cutoff4, num_radial, envelope_exponent,
                         w1, ln_g, nullptr, 0.0) ||
        !mlp_args_ok(mode, {w2tp, wstp, g_e, save_h3, save_xhat}) || !save_rstd || !g_len)
        return MATRIS_E_ARG;
    const int64_t m = n_bonds;
    if (m == 0) return 0;
    MLP_DISPATCH(edge_embed_bwd_kernel, m, a, (const uint4 *)wstp, (const uint4 *)w2tp, g_e, g_rbf6, g_rbf4, save_h3,
                 save_xhat, save_rstd, g_len);
    MATRIS_CHECK_LAUNCH();
    return 0;
}
