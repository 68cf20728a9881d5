// Segmented reductions, gathers and the fused segment attention (softmax by target and
// by source, alpha * e', both segment sums) for gfx950.
//
// All of these are HBM-bound.  Layout: one 64-lane wavefront per segment (or per pair of
// rows); each half-wave owns a 128-wide fp32 row at a time with 16-byte lanes, so every
// row access is one coalesced 512-byte transaction.  Reductions run in a fixed CSR
// order inside the wave: deterministic, no float atomics.
#include "common.h"

#define WAVES_PER_BLOCK 4

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ void st4(float *p, float4 v) { *reinterpret_cast<float4 *>(p) = v; }
__device__ __forceinline__ float4 max4(const float4 &a, const float4 &b) {
    return make_float4(fmaxf(a.x, b.x), fmaxf(a.y, b.y), fmaxf(a.z, b.z), fmaxf(a.w, b.w));
}
__device__ __forceinline__ float4 shfl_xor4(const float4 &v, int o) {
    return make_float4(__shfl_xor(v.x, o, 64), __shfl_xor(v.y, o, 64), __shfl_xor(v.z, o, 64), __shfl_xor(v.w, o, 64));
}


// ------------------------------------------------------------------------------------
// segment sum (CSR)
// ------------------------------------------------------------------------------------
// One wave per segment; each half-wave sums every other row with 16-byte lanes and the
// halves combine at the end (fixed order: deterministic).
__device__ __forceinline__ float4 mul4(const float4 &a, const float4 &b) {
    return make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
}

// Partial sum of the rows i = start, start + stride, ... < end of one CSR segment, eight
// (then four, then one) rows in flight (16-byte lanes, xc = row base + column offset of
// the lane); the adds run in row order whatever the chunking.  MUL: row r
// contributes x[r] * mc[midx ? midx[r] : r] (mc = a [*, 128] table + the lane's column;
// the product first, as the reference's h * w before its index_add_).
template <bool MUL>
__device__ __forceinline__ float4 seg_rows(const float *__restrict__ xc, int64_t ldx,
                                           const int32_t *__restrict__ perm, int i, int end, int stride,
                                           const float *__restrict__ mc = nullptr,
                                           const int32_t *__restrict__ midx = nullptr) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (; i + 7 * stride < end; i += 8 * stride) {  // eight rows in flight
        int64_t r[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) r[k] = perm ? perm[i + k * stride] : i + k * stride;
        float4 v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = ld4(xc + r[k] * ldx);
        if constexpr (MUL) {
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = mul4(v[k], ld4(mc + (midx ? (int64_t)midx[r[k]] : r[k]) * MATRIS_D));
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            acc.x += v[k].x; acc.y += v[k].y; acc.z += v[k].z; acc.w += v[k].w;
        }
    }
    for (; i + 3 * stride < end; i += 4 * stride) {
        const int64_t r0 = perm ? perm[i] : i, r1 = perm ? perm[i + stride] : i + stride;
        const int64_t r2 = perm ? perm[i + 2 * stride] : i + 2 * stride;
        const int64_t r3 = perm ? perm[i + 3 * stride] : i + 3 * stride;
        float4 v0 = ld4(xc + r0 * ldx), v1 = ld4(xc + r1 * ldx);
        float4 v2 = ld4(xc + r2 * ldx), v3 = ld4(xc + r3 * ldx);
        if constexpr (MUL) {
            v0 = mul4(v0, ld4(mc + (midx ? (int64_t)midx[r0] : r0) * MATRIS_D));
            v1 = mul4(v1, ld4(mc + (midx ? (int64_t)midx[r1] : r1) * MATRIS_D));
            v2 = mul4(v2, ld4(mc + (midx ? (int64_t)midx[r2] : r2) * MATRIS_D));
            v3 = mul4(v3, ld4(mc + (midx ? (int64_t)midx[r3] : r3) * MATRIS_D));
        }
        acc.x += v0.x; acc.y += v0.y; acc.z += v0.z; acc.w += v0.w;
        acc.x += v1.x; acc.y += v1.y; acc.z += v1.z; acc.w += v1.w;
        acc.x += v2.x; acc.y += v2.y; acc.z += v2.z; acc.w += v2.w;
        acc.x += v3.x; acc.y += v3.y; acc.z += v3.z; acc.w += v3.w;
    }
    for (; i < end; i += stride) {
        const int64_t r = perm ? perm[i] : i;
        float4 v = ld4(xc + r * ldx);
        if constexpr (MUL) v = mul4(v, ld4(mc + (midx ? (int64_t)midx[r] : r) * MATRIS_D));
        acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
    }
    return acc;
}

struct SegSrc {
    const float *x;  // nullptr: no second source
    int64_t ldx, col_off;
    const int32_t *rowptr, *perm;
    float scale;
    const float *mul;        // optional per-row multiplier rows mul[mul_idx[r]] ([*, 128])
    const int32_t *mul_idx;
    // tile > 0: rows ascend by segment (no perm) and x holds tile-run partial sums (the
    // GatedMLP backward's matris_gmlp_bwd_runs): a segment [rs, re) adds only its row rs
    // and each later multiple of `tile` below re -- one partial per tile it spans.
    int tile;
};

// The k-th summed row of a tile-run segment starting at row rs (see SegSrc::tile).
__device__ __forceinline__ int64_t tile_run_row(int64_t rs, int k, int tile) {
    return k == 0 ? rs : (rs / tile + k) * (int64_t)tile;
}

// Partial sum of the tile-run rows k = off, off + stride, ... of the segment [rs, re).
__device__ __forceinline__ float4 seg_tile_rows(const float *__restrict__ xc, int64_t ldx, int64_t rs, int64_t re,
                                                int tile, int off, int stride) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k = off;; k += stride) {
        const int64_t r = tile_run_row(rs, k, tile);
        if (r >= re) break;
        const float4 v = ld4(xc + r * ldx);
        acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
    }
    return acc;
}

__device__ __forceinline__ float4 add4(const float4 &a, const float4 &b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// Projection of a 128-wide row onto K (<= 8) basis columns, out[k] = sum_c row[c] wt[k][c]
// with wt [K, 128] row-major (a Linear(K, 128) weight, transposed), the row held as one
// float4 per lane of a 32-lane half-wave (lane l: columns 4l .. 4l+3).  Every lane of the
// half-wave must be active; lane 16 of it stores the K values.  This is the input gradient
// of a Linear(K, 128) without bias (the learnable envelope, interaction_block.py:240-246)
// formed in the epilogue of the kernel that produces the 128-wide gradient row, so that
// row never reaches memory.  Each term: one coalesced float4 of wt, a 16-lane DPP sum and
// one DPP broadcast between the half-wave's two rows.
#define MATRIS_PROJ_KMAX 8
// The two 16-lane DPP rows of a half-wave combined: lanes 16 .. 31 (and 48 .. 63) gain the
// value of lane 15 (47) of the row before them (DPP row_bcast:15 on rows 1 and 3).
__device__ __forceinline__ float rows_combine(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xa, 0xf, false));
}
// wt: global or LDS (a block's staged copy).  Lanes 16 .. 31 all end with the K sums;
// lane 16 + k stores sum k (added to dst[k] with accumulate, whose load is issued first so
// that the dot products cover its latency).
__device__ __forceinline__ void proj_row_store(const float4 &t, int l, const float *wt, int K, int accumulate,
                                               float *__restrict__ dst) {
    const int k_own = l - 16;
    const bool owner = k_own >= 0 && k_own < K;
    const float prev = (accumulate && owner) ? dst[k_own] : 0.f;
    float mine = 0.f;
#pragma unroll
    for (int k = 0; k < MATRIS_PROJ_KMAX; ++k) {
        if (k < K) {
            const float4 w = *reinterpret_cast<const float4 *>(wt + k * MATRIS_D + 4 * l);
            const float pk = rows_combine(row16_sum(t.x * w.x + t.y * w.y + t.z * w.z + t.w * w.w));
            if (k == k_own) mine = pk;
        }
    }
    if (owner) dst[k_own] = accumulate ? prev + mine : mine;
}

template <bool MUL>
__device__ __forceinline__ float4 seg_src_rows(const SegSrc &v, int64_t s, int c, int off, int stride) {
    if (v.tile > 0) return seg_tile_rows(v.x + v.col_off + c, v.ldx, v.rowptr[s], v.rowptr[s + 1], v.tile, off, stride);
    if (MUL && v.mul)
        return seg_rows<true>(v.x + v.col_off + c, v.ldx, v.perm, v.rowptr[s] + off, v.rowptr[s + 1], stride,
                              v.mul + c, v.mul_idx);
    return seg_rows<false>(v.x + v.col_off + c, v.ldx, v.perm, v.rowptr[s] + off, v.rowptr[s + 1], stride);
}

// out[s] (+)= a.scale * sum_{rows of a's segment s} a.x[row] + b.scale * (the same for b)
// [+ base_w * base[s]: a residual term, as the reference's `de + res_weight * feat`].
// WPS waves per segment: 1 (four segments per work-group), or 4 for long segments (the
// waves take interleaved row slices and combine through LDS).  In a wave the half-waves
// take alternating rows.  Every combination runs in a fixed order: deterministic.
template <int WPS, bool MUL>
__global__ __launch_bounds__(256) void seg_sum_kernel(SegSrc a, SegSrc b, int64_t n_seg, int accumulate,
                                                      const float *__restrict__ base,
                                                      const float *__restrict__ base_w, float *__restrict__ out) {
    const int w = threadIdx.x >> 6, half = (threadIdx.x >> 5) & 1, l = threadIdx.x & 31, c = 4 * l;
    const int64_t s = (int64_t)blockIdx.x * (WAVES_PER_BLOCK / WPS) + w / WPS;
    const int slice = w % WPS;
    const bool live = s < n_seg;
    float4 ta = make_float4(0.f, 0.f, 0.f, 0.f), tb = ta;
    if (live) {
        const int off = 2 * slice + half, stride = 2 * WPS;
        ta = seg_src_rows<MUL>(a, s, c, off, stride);
        if (b.x) tb = seg_src_rows<MUL>(b, s, c, off, stride);
        // half 0 + half 1, the same order in both halves
        const float4 oa = shfl_xor4(ta, 32), ob = shfl_xor4(tb, 32);
        ta = half ? add4(oa, ta) : add4(ta, oa);
        tb = half ? add4(ob, tb) : add4(tb, ob);
    }
    if constexpr (WPS > 1) {
        __shared__ float4 part[WAVES_PER_BLOCK][2][32];
        if (half == 0) {
            part[w][0][l] = ta;
            part[w][1][l] = tb;
        }
        __syncthreads();
        if (!live || slice != 0 || half) return;
#pragma unroll
        for (int k = 1; k < WPS; ++k) {
            ta = add4(ta, part[w + k][0][l]);
            tb = add4(tb, part[w + k][1][l]);
        }
    } else {
        if (!live || half) return;
    }
    float4 t = make_float4(ta.x * a.scale, ta.y * a.scale, ta.z * a.scale, ta.w * a.scale);
    if (b.x) t = add4(t, make_float4(tb.x * b.scale, tb.y * b.scale, tb.z * b.scale, tb.w * b.scale));
    float *op = out + s * MATRIS_D + c;
    if (base) t = add4(t, mul4(ld4(base_w + c), ld4(base + s * MATRIS_D + c)));
    if (accumulate) t = add4(t, ld4(op));
    st4(op, t);
}

// Short segments (at most 4 rows on average, e.g. the two directed copies of a bond): a
// wave takes 4 consecutive segments, and each half-wave loads the first row of its parity
// in all four before summing (4 rows in flight where one wave per segment had 1), then
// any further rows.  Rows are added in the order seg_rows adds them and the halves
// combine as in seg_sum_kernel: the results are identical.
template <bool MUL>
__device__ __forceinline__ void seg_rows4(const SegSrc &v, int64_t s0, int64_t n_seg, int half, int c,
                                          float4 (&acc)[4]) {
    const float *xc = v.x + v.col_off + c;
    int b[4], e[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const bool in = s0 + j < n_seg;
        b[j] = in ? v.rowptr[s0 + j] : 0;
        e[j] = in ? v.rowptr[s0 + j + 1] : 0;
    }
    if (v.tile > 0) {  // tile-run partials: the same rows and order as seg_sum_kernel's
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = seg_tile_rows(xc, v.ldx, b[j], e[j], v.tile, half, 2);
        return;
    }
    int64_t r[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = b[j] + half;
        r[j] = i < e[j] ? (v.perm ? (int64_t)v.perm[i] : (int64_t)i) : -1;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r[j] >= 0) {
            x = ld4(xc + r[j] * v.ldx);
            if constexpr (MUL) x = mul4(x, ld4(v.mul + c + (v.mul_idx ? (int64_t)v.mul_idx[r[j]] : r[j]) * MATRIS_D));
        }
        acc[j] = x;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        for (int i = b[j] + half + 2; i < e[j]; i += 2) {
            const int64_t rr = v.perm ? (int64_t)v.perm[i] : (int64_t)i;
            float4 x = ld4(xc + rr * v.ldx);
            if constexpr (MUL) x = mul4(x, ld4(v.mul + c + (v.mul_idx ? (int64_t)v.mul_idx[rr] : rr) * MATRIS_D));
            acc[j] = add4(acc[j], x);
        }
    }
}

// With proj_w (a [K, 128] transposed Linear weight), each segment's row is projected
// (proj_row_store) into proj_out [n_seg, K] (added to it with accumulate) instead of being
// written to out.
template <bool MUL, bool PROJ = false>
__global__ __launch_bounds__(256) void seg_sum_short_kernel(SegSrc a, SegSrc b, int64_t n_seg, int accumulate,
                                                            const float *__restrict__ base,
                                                            const float *__restrict__ base_w,
                                                            float *__restrict__ out,
                                                            const float *__restrict__ proj_w, int proj_k,
                                                            float *__restrict__ proj_out) {
    const int w = threadIdx.x >> 6, half = (threadIdx.x >> 5) & 1, l = threadIdx.x & 31, c = 4 * l;
    __shared__ __align__(16) float wts[PROJ ? MATRIS_PROJ_KMAX * MATRIS_D : 4];
    if constexpr (PROJ) {  // the block's copy of the projection weights (before any wave leaves)
        for (int q = threadIdx.x; q < proj_k * MATRIS_D / 4; q += blockDim.x)
            reinterpret_cast<float4 *>(wts)[q] = ld4(proj_w + 4 * q);
        lds_barrier();
    }
    const int64_t s0 = ((int64_t)blockIdx.x * WAVES_PER_BLOCK + w) * 4;
    if (s0 >= n_seg) return;  // whole wave
    float4 ta[4], tb[4];
    seg_rows4<MUL>(a, s0, n_seg, half, c, ta);
    if (b.x) seg_rows4<MUL>(b, s0, n_seg, half, c, tb);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float4 oa = shfl_xor4(ta[j], 32);
        ta[j] = half ? add4(oa, ta[j]) : add4(ta[j], oa);
        if (b.x) {
            const float4 ob = shfl_xor4(tb[j], 32);
            tb[j] = half ? add4(ob, tb[j]) : add4(tb[j], ob);
        }
    }
    if (half) return;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t s = s0 + j;
        if (s >= n_seg) break;
        float4 t = make_float4(ta[j].x * a.scale, ta[j].y * a.scale, ta[j].z * a.scale, ta[j].w * a.scale);
        if (b.x) t = add4(t, make_float4(tb[j].x * b.scale, tb[j].y * b.scale, tb[j].z * b.scale, tb[j].w * b.scale));
        if constexpr (PROJ) {  // uniform over the wave: s < n_seg is the same for all its lanes
            proj_row_store(t, l, wts, proj_k, accumulate, proj_out + s * proj_k);
            continue;
        }
        float *op = out + s * MATRIS_D + c;
        if (base) t = add4(t, mul4(ld4(base_w + c), ld4(base + s * MATRIS_D + c)));
        if (accumulate) t = add4(t, ld4(op));
        st4(op, t);
    }
}

static bool seg_src_ok(const SegSrc &v) {
    return v.rowptr && v.ldx >= MATRIS_D && v.col_off >= 0 && v.col_off + MATRIS_D <= v.ldx && !(v.ldx % 4) &&
           !(v.col_off % 4) && v.tile >= 0 && !(v.tile > 0 && (v.perm || v.mul));
}

// proj_w / proj_k / proj_out: project each segment's row onto the K rows of proj_w
// ([K, 128], K <= 8) into proj_out [n_seg, K] instead of writing out (short segments only:
// rows_hint <= 4 n_seg; no base; accumulate adds to proj_out).
static int seg_sum_launch(const SegSrc &a, const SegSrc &b, int64_t n_seg, int64_t rows_hint, int accumulate,
                          float *out, void *stream, const float *base = nullptr, const float *base_w = nullptr,
                          const float *proj_w = nullptr, int proj_k = 0, float *proj_out = nullptr) {
    if (n_seg < 0 || !seg_src_ok(a) || (b.x && !seg_src_ok(b)) || (base && !base_w)) return MATRIS_E_ARG;
    // rows_hint 0 means "not given", except for a projection, which passes the row count
    // itself (0: every segment is empty and projects to zeros)
    const bool short_segs = (rows_hint > 0 || proj_w) && rows_hint >= 0 && rows_hint <= 4 * n_seg;
    if (proj_w) {
        if (!proj_out || proj_k < 1 || proj_k > MATRIS_PROJ_KMAX || !short_segs || base)
            return MATRIS_E_ARG;
    } else if (!out) {
        return MATRIS_E_ARG;
    }
    if (n_seg == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    const bool mul = a.mul || (b.x && b.mul);
    const bool wide = rows_hint >= 32 * n_seg;  // long segments: a work-group each
    if (short_segs) {  // short segments: four per wave
        const unsigned g4 = (unsigned)matris_blocks(n_seg, 4 * WAVES_PER_BLOCK);
        if (mul && proj_w)
            seg_sum_short_kernel<true, true><<<g4, 256, 0, st>>>(a, b, n_seg, accumulate, base, base_w, out, proj_w,
                                                                 proj_k, proj_out);
        else if (mul)
            seg_sum_short_kernel<true><<<g4, 256, 0, st>>>(a, b, n_seg, accumulate, base, base_w, out, nullptr, 0,
                                                           nullptr);
        else if (proj_w)
            seg_sum_short_kernel<false, true><<<g4, 256, 0, st>>>(a, b, n_seg, accumulate, base, base_w, out, proj_w,
                                                                  proj_k, proj_out);
        else
            seg_sum_short_kernel<false><<<g4, 256, 0, st>>>(a, b, n_seg, accumulate, base, base_w, out, nullptr, 0,
                                                            nullptr);
        MATRIS_CHECK_LAUNCH();
        return 0;
    }
    const unsigned grid = wide ? (unsigned)n_seg : (unsigned)matris_blocks(n_seg, WAVES_PER_BLOCK);
    if (wide && mul)
        seg_sum_kernel<4, true><<<grid, 256, 0, st>>>(a, b, n_seg, accumulate, base, base_w, out);
    else if (wide)
        seg_sum_kernel<4, false><<<grid, 256, 0, st>>>(a, b, n_seg, accumulate, base, base_w, out);
    else if (mul)
        seg_sum_kernel<1, true><<<grid, 256, 0, st>>>(a, b, n_seg, accumulate, base, base_w, out);
    else
        seg_sum_kernel<1, false><<<grid, 256, 0, st>>>(a, b, n_seg, accumulate, base, base_w, out);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_seg_sum(const float *x, int64_t ldx, int64_t col_off, const int32_t *rowptr,
                              const int32_t *perm, int64_t n_seg, float scale, int accumulate, float *out,
                              void *stream) {
    const SegSrc a{x, ldx, col_off, rowptr, perm, scale, nullptr, nullptr};
    const SegSrc none{nullptr, MATRIS_D, 0, nullptr, nullptr, 0.f, nullptr, nullptr};
    return seg_sum_launch(a, none, n_seg, 0, accumulate, out, stream);
}

extern "C" int matris_seg_sum2(int64_t n_seg, int64_t rows_hint, const float *xa, int64_t lda, int64_t offa,
                               const int32_t *rowptr_a, const int32_t *perm_a, float scale_a, const float *xb,
                               int64_t ldb, int64_t offb, const int32_t *rowptr_b, const int32_t *perm_b,
                               float scale_b, int accumulate, const float *base, const float *base_w, float *out,
                               void *stream) {
    const SegSrc a{xa, lda, offa, rowptr_a, perm_a, scale_a, nullptr, nullptr};
    const SegSrc b{xb, ldb, offb, rowptr_b, perm_b, scale_b, nullptr, nullptr};
    return seg_sum_launch(a, b, n_seg, rows_hint, accumulate, out, stream, base, base_w);
}

extern "C" int matris_seg_sum2_runs(int64_t n_seg, int64_t rows_hint, const float *xa, int64_t lda, int64_t offa,
                                    const int32_t *rowptr_a, int tile_a, float scale_a, const float *xb, int64_t ldb,
                                    int64_t offb, const int32_t *rowptr_b, const int32_t *perm_b, float scale_b,
                                    int accumulate, float *out, void *stream) {
    if (tile_a <= 0) return MATRIS_E_ARG;
    const SegSrc a{xa, lda, offa, rowptr_a, nullptr, scale_a, nullptr, nullptr, tile_a};
    const SegSrc b{xb, ldb, offb, rowptr_b, perm_b, scale_b, nullptr, nullptr};
    return seg_sum_launch(a, b, n_seg, rows_hint, accumulate, out, stream);
}

extern "C" int matris_seg_sum_mul(int64_t n_seg, int64_t rows_hint, const float *x, int64_t ldx, int64_t col_off,
                                  const int32_t *rowptr, const int32_t *perm, const float *mul,
                                  const int32_t *mul_idx, float scale, int accumulate, float *out, void *stream) {
    if (!mul) return MATRIS_E_ARG;
    const SegSrc a{x, ldx, col_off, rowptr, perm, scale, mul, mul_idx};
    const SegSrc none{nullptr, MATRIS_D, 0, nullptr, nullptr, 0.f, nullptr, nullptr};
    return seg_sum_launch(a, none, n_seg, rows_hint, accumulate, out, stream);
}

extern "C" int matris_seg_sum_mul_proj(int64_t n_seg, int64_t rows_hint, const float *x, int64_t ldx,
                                       int64_t col_off, const int32_t *rowptr, const int32_t *perm, const float *mul,
                                       const int32_t *mul_idx, float scale, const float *proj_w, int proj_k,
                                       int accumulate, float *proj_out, void *stream) {
    if (!mul || !proj_w || ((uintptr_t)proj_w & 15)) return MATRIS_E_ARG;
    const SegSrc a{x, ldx, col_off, rowptr, perm, scale, mul, mul_idx};
    const SegSrc none{nullptr, MATRIS_D, 0, nullptr, nullptr, 0.f, nullptr, nullptr};
    return seg_sum_launch(a, none, n_seg, rows_hint, accumulate, nullptr, stream, nullptr, nullptr, proj_w, proj_k,
                          proj_out);
}

// ------------------------------------------------------------------------------------
// segment sums of narrow rows (width <= 32 floats: per-graph energies, per-graph strain
// and lattice gradients of a batch), in a fixed order: one wave per segment; lane l takes
// column l % width of rows b + l / width, b + l / width + slots, ... (slots = 64 / width),
// then lanes 0 .. width-1 add the slots' partial sums in slot order from LDS.  No atomics:
// the per-graph sums of a batch are bitwise reproducible.
// ------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void seg_sum_narrow_kernel(int64_t n_seg, const int32_t *__restrict__ rowptr,
                                                             const float *__restrict__ x, int width,
                                                             float *__restrict__ out) {
    __shared__ float part[WAVES_PER_BLOCK][64];
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int64_t seg = (int64_t)blockIdx.x * WAVES_PER_BLOCK + w;
    const int slots = 64 / width;
    float acc = 0.f;
    if (seg < n_seg && l < slots * width) {
        const int64_t b = rowptr[seg], e = rowptr[seg + 1];
        const int col = l % width;
        for (int64_t r = b + l / width; r < e; r += slots) acc += x[r * width + col];
    }
    part[w][l] = acc;
    __syncthreads();
    if (seg < n_seg && l < width) {
        float t = 0.f;
        for (int k = 0; k < slots; ++k) t += part[w][k * width + l];
        out[seg * width + l] = t;
    }
}

extern "C" int matris_seg_sum_narrow(int64_t n_seg, const int32_t *rowptr, const float *x, int width, float *out,
                                     void *stream) {
    if (n_seg < 0 || width < 1 || width > 32) return MATRIS_E_ARG;
    if (n_seg == 0) return 0;
    if (!rowptr || !out) return MATRIS_E_ARG;
    seg_sum_narrow_kernel<<<matris_blocks(n_seg, WAVES_PER_BLOCK), 256, 0, (hipStream_t)stream>>>(n_seg, rowptr, x,
                                                                                               width, out);
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

// out[r] (+)= a[ia[r]] * b[ib[r]] (index NULL: the identity), one float4 per thread.
__global__ __launch_bounds__(256) void gather_mul_kernel(int64_t n_rows, const float *__restrict__ a,
                                                         const int32_t *__restrict__ ia,
                                                         const float *__restrict__ b,
                                                         const int32_t *__restrict__ ib, int accumulate,
                                                         float *__restrict__ out) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t r = t >> 5;
    if (r >= n_rows) return;
    const int q = (int)(t & 31) * 4;
    const int64_t ra = ia ? ia[r] : r, rb = ib ? ib[r] : r;
    float4 v = mul4(ld4(a + ra * MATRIS_D + q), ld4(b + rb * MATRIS_D + q));
    float *o = out + r * MATRIS_D + q;
    if (accumulate) v = add4(ld4(o), v);
    st4(o, v);
}

extern "C" int matris_gather_mul(int64_t n_rows, const float *a, const int32_t *ia, const float *b,
                                 const int32_t *ib, int accumulate, float *out, void *stream) {
    if (n_rows < 0 || !a || !b || !out) return MATRIS_E_ARG;
    if (n_rows == 0) return 0;
    gather_mul_kernel<<<matris_blocks(n_rows * 32, 256), 256, 0, (hipStream_t)stream>>>(n_rows, a, ia, b, ib,
                                                                                     accumulate, out);
    MATRIS_CHECK_LAUNCH();
    return 0;
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
// edge-vector backward: vec[e] = cart[tgt[e]] - cart[src[e]] - shift[e]  =>
//   g_cart[i] = sum_{tgt[e]=i} g_vec[e] - sum_{src[e]=i} g_vec[e]
// One wave per atom walks its target and source CSR rows (lanes stride the rows) and
// reduces the three components across the wave: a fixed summation order.
// ------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void edge_vec_bwd_kernel(int64_t n, const float *__restrict__ g,
                                                           const int32_t *__restrict__ t_ptr,
                                                           const int32_t *__restrict__ t_perm,
                                                           const int32_t *__restrict__ s_ptr,
                                                           const int32_t *__restrict__ s_perm,
                                                           float *__restrict__ g_cart) {
    const int64_t a = (int64_t)blockIdx.x * WAVES_PER_BLOCK + (threadIdx.x >> 6);
    if (a >= n) return;
    const int lane = threadIdx.x & 63;
    float x = 0.f, y = 0.f, z = 0.f;
    for (int i = t_ptr[a] + lane; i < t_ptr[a + 1]; i += 64) {
        const int64_t r = t_perm ? t_perm[i] : i;
        x += g[3 * r];
        y += g[3 * r + 1];
        z += g[3 * r + 2];
    }
    for (int i = s_ptr[a] + lane; i < s_ptr[a + 1]; i += 64) {
        const int64_t r = s_perm ? s_perm[i] : i;
        x -= g[3 * r];
        y -= g[3 * r + 1];
        z -= g[3 * r + 2];
    }
    x = wave_sum(x);
    y = wave_sum(y);
    z = wave_sum(z);
    if (lane == 0) {
        g_cart[3 * a] = x;
        g_cart[3 * a + 1] = y;
        g_cart[3 * a + 2] = z;
    }
}

extern "C" int matris_edge_vec_bwd(int64_t n_atoms, const float *g_vec, const int32_t *t_ptr, const int32_t *t_perm,
                                   const int32_t *s_ptr, const int32_t *s_perm, float *g_cart, void *stream) {
    if (n_atoms < 0 || !t_ptr || !s_ptr || !g_cart) return MATRIS_E_ARG;
    if (n_atoms == 0) return 0;
    edge_vec_bwd_kernel<<<matris_blocks(n_atoms, WAVES_PER_BLOCK), 256, 0, (hipStream_t)stream>>>(
        n_atoms, g_vec, t_ptr, t_perm, s_ptr, s_perm, g_cart);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

// ------------------------------------------------------------------------------------
// Edge geometry of one graph with the strain trick, forward and backward in a few
// launches instead of a chain of small tensor operations:
//   sym = (S + S^T) / 2,  x' = x + x sym (atoms),  L' = L + L sym,
//   vec[e] = x'[tgt[e]] - (x'[src[e]] + image[e] L'),  len = |vec|,  unit = vec / len.
// Without a strain sym is zero and x' = x, L' = L exactly.
// ------------------------------------------------------------------------------------
__device__ __forceinline__ void geom_sym(const float *__restrict__ S, float sym[9]) {
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) sym[3 * i + j] = S ? 0.5f * (S[3 * i + j] + S[3 * j + i]) : 0.f;
}

// y = x + x sym for a row vector x
__device__ __forceinline__ void geom_strain_row(const float x[3], const float sym[9], float y[3]) {
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        float t = x[0] * sym[j];
        t = fmaf(x[1], sym[3 + j], t);
        t = fmaf(x[2], sym[6 + j], t);
        y[j] = x[j] + t;
    }
}

__global__ __launch_bounds__(256) void edge_geom_fwd_kernel(int64_t n, const float *__restrict__ cart,
                                                            const float *__restrict__ lat,
                                                            const float *__restrict__ S,
                                                            const float *__restrict__ image,
                                                            const int32_t *__restrict__ tgt,
                                                            const int32_t *__restrict__ src,
                                                            float *__restrict__ len_out,
                                                            float *__restrict__ unit_out,
                                                            float *__restrict__ lat_out,
                                                            float *__restrict__ vol_out) {
    float sym[9], Ls[9];
    geom_sym(S, sym);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const float row[3] = {lat[3 * i], lat[3 * i + 1], lat[3 * i + 2]};
        geom_strain_row(row, sym, Ls + 3 * i);
    }
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e == 0) {
#pragma unroll
        for (int k = 0; k < 9; ++k) lat_out[k] = Ls[k];
        // det of the unstrained lattice: L0 . (L1 x L2)
        const float c0 = lat[4] * lat[8] - lat[5] * lat[7];
        const float c1 = lat[5] * lat[6] - lat[3] * lat[8];
        const float c2 = lat[3] * lat[7] - lat[4] * lat[6];
        vol_out[0] = lat[0] * c0 + lat[1] * c1 + lat[2] * c2;
    }
    if (e >= n) return;
    const int64_t t = tgt[e], s = src[e];
    const float xt[3] = {cart[3 * t], cart[3 * t + 1], cart[3 * t + 2]};
    const float xs[3] = {cart[3 * s], cart[3 * s + 1], cart[3 * s + 2]};
    const float im[3] = {image[3 * e], image[3 * e + 1], image[3 * e + 2]};
    float yt[3], ys[3], v[3];
    geom_strain_row(xt, sym, yt);
    geom_strain_row(xs, sym, ys);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        float sh = im[0] * Ls[j];
        sh = fmaf(im[1], Ls[3 + j], sh);
        sh = fmaf(im[2], Ls[6 + j], sh);
        v[j] = yt[j] - (ys[j] + sh);
    }
    const float l = sqrtf(fmaf(v[2], v[2], fmaf(v[1], v[1], v[0] * v[0])));
    len_out[e] = l;
#pragma unroll
    for (int j = 0; j < 3; ++j) unit_out[3 * e + j] = v[j] / l;
}

// Per edge: g_vec = g_len unit + (g_unit - (g_unit . unit) unit) / len, written out, and
// this block's share of P = sum_e image[e]^T g_vec[e] (3 x 3), reduced in a fixed order.
__global__ __launch_bounds__(256) void edge_geom_bwd_edge_kernel(int64_t n, const float *__restrict__ g_len,
                                                                 const float *__restrict__ g_unit,
                                                                 const float *__restrict__ len,
                                                                 const float *__restrict__ unit,
                                                                 const float *__restrict__ image,
                                                                 float *__restrict__ g_vec,
                                                                 float *__restrict__ partial) {
    float P[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) P[k] = 0.f;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
        const float u[3] = {unit[3 * e], unit[3 * e + 1], unit[3 * e + 2]};
        float gv[3] = {0.f, 0.f, 0.f};
        if (g_len) {
            const float gl = g_len[e];
#pragma unroll
            for (int j = 0; j < 3; ++j) gv[j] = gl * u[j];
        }
        if (g_unit) {
            const float gu[3] = {g_unit[3 * e], g_unit[3 * e + 1], g_unit[3 * e + 2]};
            const float d = fmaf(gu[2], u[2], fmaf(gu[1], u[1], gu[0] * u[0]));
            const float l = len[e];
#pragma unroll
            for (int j = 0; j < 3; ++j) gv[j] += (gu[j] - d * u[j]) / l;
        }
#pragma unroll
        for (int j = 0; j < 3; ++j) g_vec[3 * e + j] = gv[j];
        const float im[3] = {image[3 * e], image[3 * e + 1], image[3 * e + 2]};
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = 0; j < 3; ++j) P[3 * i + j] = fmaf(im[i], gv[j], P[3 * i + j]);
    }
    __shared__ float part[4][9];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        const float v = wave_sum(P[k]);
        if (lane == 0) part[w][k] = v;
    }
    __syncthreads();
    if (threadIdx.x < 9)
        partial[9 * blockIdx.x + threadIdx.x] =
            ((part[0][threadIdx.x] + part[1][threadIdx.x]) + part[2][threadIdx.x]) + part[3][threadIdx.x];
}

// One work-group: P from the partials, C = sum_a x_a^T g'_a over the atoms (g' = the
// gradient of the strained positions, in g_cart), then
//   g_cart = g' + g' sym^T,  g_sym = C + L^T (-P),  g_S = (g_sym + g_sym^T) / 2.
__global__ __launch_bounds__(1024) void edge_geom_bwd_final_kernel(int64_t n_atoms, int n_part,
                                                                   const float *__restrict__ partial,
                                                                   const float *__restrict__ cart,
                                                                   const float *__restrict__ lat,
                                                                   const float *__restrict__ S,
                                                                   float *__restrict__ g_cart,
                                                                   float *__restrict__ g_strain) {
    float sym[9], acc[18];
    geom_sym(S, sym);
#pragma unroll
    for (int k = 0; k < 18; ++k) acc[k] = 0.f;
    for (int b = threadIdx.x; b < n_part; b += 1024)
#pragma unroll
        for (int k = 0; k < 9; ++k) acc[k] += partial[9 * b + k];
    for (int64_t a = threadIdx.x; a < n_atoms; a += 1024) {
        const float g[3] = {g_cart[3 * a], g_cart[3 * a + 1], g_cart[3 * a + 2]};
        const float x[3] = {cart[3 * a], cart[3 * a + 1], cart[3 * a + 2]};
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = 0; j < 3; ++j) acc[9 + 3 * i + j] = fmaf(x[i], g[j], acc[9 + 3 * i + j]);
#pragma unroll
        for (int j = 0; j < 3; ++j) {  // sym is symmetric: g sym^T = g sym
            float t = g[0] * sym[j];
            t = fmaf(g[1], sym[3 + j], t);
            t = fmaf(g[2], sym[6 + j], t);
            g_cart[3 * a + j] = g[j] + t;
        }
    }
    __shared__ float part[16][18];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < 18; ++k) {
        const float v = wave_sum(acc[k]);
        if (lane == 0) part[w][k] = v;
    }
    __syncthreads();
    __shared__ float tot[18];
    if (threadIdx.x < 18) {
        float s = 0.f;
        for (int q = 0; q < 16; ++q) s += part[q][threadIdx.x];
        tot[threadIdx.x] = s;
    }
    __syncthreads();
    if (threadIdx.x == 0 && g_strain) {
        float gs[9];
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = 0; j < 3; ++j) {  // (L^T (-P))[i][j] = -sum_k L[k][i] P[k][j]
                float t = lat[i] * tot[j];
                t = fmaf(lat[3 + i], tot[3 + j], t);
                t = fmaf(lat[6 + i], tot[6 + j], t);
                gs[3 * i + j] = tot[9 + 3 * i + j] - t;
            }
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = 0; j < 3; ++j) g_strain[3 * i + j] = 0.5f * (gs[3 * i + j] + gs[3 * j + i]);
    }
}

// Cartesian positions of one graph, cart[i] = frac[i] L (a row vector times the lattice,
// each column summed in index order with FMA), and the zero strain [3, 3] the stress is
// taken against (zero9, optional), in one launch.
__global__ __launch_bounds__(256) void frac_cart_kernel(int64_t n, const float *__restrict__ frac,
                                                        const float *__restrict__ lat, float *__restrict__ cart,
                                                        float *__restrict__ zero9) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (zero9 && i < 9) zero9[i] = 0.f;
    if (i >= n) return;
    const float f0 = frac[3 * i], f1 = frac[3 * i + 1], f2 = frac[3 * i + 2];
#pragma unroll
    for (int j = 0; j < 3; ++j) cart[3 * i + j] = fmaf(f2, lat[6 + j], fmaf(f1, lat[3 + j], f0 * lat[j]));
}

// The same for a batch of graphs: atom i uses the lattice of its graph gidx[i]; an index
// outside [0, n_graphs) sets MATRIS_STATUS_CSR_KEY in the status word and leaves the
// atom's row unwritten.  zero: nz floats set to zero (the batch's zero strains).
__global__ __launch_bounds__(256) void frac_cart_batch_kernel(int64_t n, int64_t n_graphs,
                                                              const float *__restrict__ frac,
                                                              const float *__restrict__ lat,
                                                              const int32_t *__restrict__ gidx,
                                                              float *__restrict__ cart, int64_t nz,
                                                              float *__restrict__ zero, unsigned *status) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (zero && i < nz) zero[i] = 0.f;
    if (i >= n) return;
    const int g = gidx[i];
    if (g < 0 || g >= n_graphs) {
        atomicOr(status, (unsigned)MATRIS_STATUS_CSR_KEY);
        return;
    }
    const float *L = lat + 9 * (int64_t)g;
    const float f0 = frac[3 * i], f1 = frac[3 * i + 1], f2 = frac[3 * i + 2];
#pragma unroll
    for (int j = 0; j < 3; ++j) cart[3 * i + j] = fmaf(f2, L[6 + j], fmaf(f1, L[3 + j], f0 * L[j]));
}

extern "C" int matris_frac_to_cart_batch(int64_t n, int64_t n_graphs, const float *frac, const float *lattice,
                                         const int32_t *graph_of_atom, float *cart, float *strain_zero,
                                         void *stream) {
    if (n < 0 || n_graphs < 1 || (n > 0 && (!frac || !lattice || !graph_of_atom || !cart))) return MATRIS_E_ARG;
    const int64_t nz = strain_zero ? 9 * n_graphs : 0;
    if (n == 0 && nz == 0) return 0;
    unsigned *status = matris_range_flag();
    if (!status) return MATRIS_E_ARG;
    frac_cart_batch_kernel<<<matris_blocks(n > nz ? n : nz, 256), 256, 0, (hipStream_t)stream>>>(
        n, n_graphs, frac, lattice, graph_of_atom, cart, nz, strain_zero, status);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_frac_to_cart(int64_t n, const float *frac, const float *lattice, float *cart,
                                   float *strain_zero, void *stream) {
    if (n < 0 || (n > 0 && (!frac || !lattice || !cart))) return MATRIS_E_ARG;
    if (n == 0 && !strain_zero) return 0;
    frac_cart_kernel<<<matris_blocks(n > 9 ? n : 9, 256), 256, 0, (hipStream_t)stream>>>(n, frac, lattice, cart,
                                                                                         strain_zero);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

static inline int geom_parts(int64_t n_edges) {
    const int b = matris_blocks(n_edges, 256);
    return b < MATRIS_GEOM_PARTS ? b : MATRIS_GEOM_PARTS;
}

extern "C" int matris_edge_geom_fwd(int64_t n_edges, const float *cart, const float *lattice, const float *strain,
                                    const float *image, const int32_t *tgt, const int32_t *src, float *length,
                                    float *unit, float *lattice_out, float *volume, void *stream) {
    if (n_edges < 0 || !lattice || !lattice_out || !volume) return MATRIS_E_ARG;
    if (n_edges > 0 && (!cart || !image || !tgt || !src || !length || !unit)) return MATRIS_E_ARG;
    edge_geom_fwd_kernel<<<matris_blocks(n_edges, 256), 256, 0, (hipStream_t)stream>>>(
        n_edges, cart, lattice, strain, image, tgt, src, length, unit, lattice_out, volume);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_edge_geom_bwd(int64_t n_atoms, int64_t n_edges, const float *g_length, const float *g_unit,
                                    const float *length, const float *unit, const float *cart, const float *lattice,
                                    const float *strain, const float *image, const int32_t *t_ptr,
                                    const int32_t *t_perm, const int32_t *s_ptr, const int32_t *s_perm,
                                    float *g_vec, float *partial, float *g_cart, float *g_strain, void *stream) {
    if (n_atoms < 0 || n_edges < 0 || !cart || !lattice || !t_ptr || !s_ptr || !partial || !g_cart)
        return MATRIS_E_ARG;
    if (n_edges > 0 && (!length || !unit || !image || !g_vec)) return MATRIS_E_ARG;
    if (g_strain && !strain) return MATRIS_E_ARG;
    const int parts = geom_parts(n_edges);
    hipStream_t st = (hipStream_t)stream;
    if (n_edges > 0) {
        edge_geom_bwd_edge_kernel<<<parts, 256, 0, st>>>(n_edges, g_length, g_unit, length, unit, image, g_vec,
                                                         partial);
        MATRIS_CHECK_LAUNCH();
    }
    if (n_atoms > 0) {
        edge_vec_bwd_kernel<<<matris_blocks(n_atoms, WAVES_PER_BLOCK), 256, 0, st>>>(n_atoms, g_vec, t_ptr, t_perm,
                                                                                     s_ptr, s_perm, g_cart);
        MATRIS_CHECK_LAUNCH();
    }
    if (strain) {  // g' -> g_cart through the strained positions, and the strain's gradient
        edge_geom_bwd_final_kernel<<<1, 1024, 0, st>>>(n_atoms, n_edges > 0 ? parts : 0, partial, cart, lattice,
                                                       strain, g_cart, g_strain);
        MATRIS_CHECK_LAUNCH();
    }
    return 0;
}

// ------------------------------------------------------------------------------------
// Edge geometry of a disjoint batch of graphs: the kernels above with each edge (and, in
// the backward, each graph's atoms and edges) using its own graph's lattice and strain.
// ------------------------------------------------------------------------------------
// Per edge e of graph gidx[e]: vec = x'[tgt] - (x'[src] + image L'_g) with the graph's
// strain; threads g < n_graphs also write that graph's L'_g and det(L_g).  A graph index
// outside [0, n_graphs) sets MATRIS_STATUS_CSR_KEY and leaves the edge's outputs unwritten.
__global__ __launch_bounds__(256) void edge_geom_fwd_batch_kernel(int64_t n, int64_t n_graphs,
                                                                  const float *__restrict__ cart,
                                                                  const float *__restrict__ lat,
                                                                  const float *__restrict__ S,
                                                                  const float *__restrict__ image,
                                                                  const int32_t *__restrict__ tgt,
                                                                  const int32_t *__restrict__ src,
                                                                  const int32_t *__restrict__ gidx,
                                                                  float *__restrict__ len_out,
                                                                  float *__restrict__ unit_out,
                                                                  float *__restrict__ lat_out,
                                                                  float *__restrict__ vol_out, unsigned *status) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    float sym[9], Ls[9];
    if (e < n_graphs) {  // graph e's strained lattice and volume
        const float *L = lat + 9 * e;
        geom_sym(S ? S + 9 * e : nullptr, sym);
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const float row[3] = {L[3 * i], L[3 * i + 1], L[3 * i + 2]};
            geom_strain_row(row, sym, Ls + 3 * i);
        }
#pragma unroll
        for (int k = 0; k < 9; ++k) lat_out[9 * e + k] = Ls[k];
        const float c0 = L[4] * L[8] - L[5] * L[7];
        const float c1 = L[5] * L[6] - L[3] * L[8];
        const float c2 = L[3] * L[7] - L[4] * L[6];
        vol_out[e] = L[0] * c0 + L[1] * c1 + L[2] * c2;
    }
    if (e >= n) return;
    const int g = gidx[e];
    if (g < 0 || g >= n_graphs) {
        atomicOr(status, (unsigned)MATRIS_STATUS_CSR_KEY);
        return;
    }
    const float *L = lat + 9 * (int64_t)g;
    geom_sym(S ? S + 9 * (int64_t)g : nullptr, sym);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const float row[3] = {L[3 * i], L[3 * i + 1], L[3 * i + 2]};
        geom_strain_row(row, sym, Ls + 3 * i);
    }
    const int64_t t = tgt[e], s = src[e];
    const float xt[3] = {cart[3 * t], cart[3 * t + 1], cart[3 * t + 2]};
    const float xs[3] = {cart[3 * s], cart[3 * s + 1], cart[3 * s + 2]};
    const float im[3] = {image[3 * e], image[3 * e + 1], image[3 * e + 2]};
    float yt[3], ys[3], v[3];
    geom_strain_row(xt, sym, yt);
    geom_strain_row(xs, sym, ys);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        float sh = im[0] * Ls[j];
        sh = fmaf(im[1], Ls[3 + j], sh);
        sh = fmaf(im[2], Ls[6 + j], sh);
        v[j] = yt[j] - (ys[j] + sh);
    }
    const float l = sqrtf(fmaf(v[2], v[2], fmaf(v[1], v[1], v[0] * v[0])));
    len_out[e] = l;
#pragma unroll
    for (int j = 0; j < 3; ++j) unit_out[3 * e + j] = v[j] / l;
}

// Per edge: g_vec = g_len unit + (g_unit - (g_unit . unit) unit) / len.
__global__ __launch_bounds__(256) void edge_gvec_kernel(int64_t n, const float *__restrict__ g_len,
                                                        const float *__restrict__ g_unit,
                                                        const float *__restrict__ len,
                                                        const float *__restrict__ unit, float *__restrict__ g_vec) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= n) return;
    const float u[3] = {unit[3 * e], unit[3 * e + 1], unit[3 * e + 2]};
    float gv[3] = {0.f, 0.f, 0.f};
    if (g_len) {
        const float gl = g_len[e];
#pragma unroll
        for (int j = 0; j < 3; ++j) gv[j] = gl * u[j];
    }
    if (g_unit) {
        const float gu[3] = {g_unit[3 * e], g_unit[3 * e + 1], g_unit[3 * e + 2]};
        const float d = fmaf(gu[2], u[2], fmaf(gu[1], u[1], gu[0] * u[0]));
        const float l = len[e];
#pragma unroll
        for (int j = 0; j < 3; ++j) gv[j] += (gu[j] - d * u[j]) / l;
    }
#pragma unroll
    for (int j = 0; j < 3; ++j) g_vec[3 * e + j] = gv[j];
}

// One work-group per graph g (its atoms [atom_ptr[g], atom_ptr[g+1]), its edges
// [edge_ptr[g], edge_ptr[g+1])): P = sum_e image[e]^T g_vec[e], C = sum_a x_a^T g'_a, then
//   g_cart = g' + g' sym^T,  g_sym = C + L^T (-P),  g_S = (g_sym + g_sym^T) / 2,
// every sum in a fixed order (thread-strided, then the waves in order).
__global__ __launch_bounds__(256) void edge_geom_bwd_graph_kernel(const int32_t *__restrict__ atom_ptr,
                                                                  const int32_t *__restrict__ edge_ptr,
                                                                  const float *__restrict__ g_vec,
                                                                  const float *__restrict__ image,
                                                                  const float *__restrict__ cart,
                                                                  const float *__restrict__ lat,
                                                                  const float *__restrict__ S,
                                                                  float *__restrict__ g_cart,
                                                                  float *__restrict__ g_strain) {
    const int64_t g = blockIdx.x;
    float sym[9], acc[18];
    geom_sym(S + 9 * g, sym);
#pragma unroll
    for (int k = 0; k < 18; ++k) acc[k] = 0.f;
    for (int64_t e = edge_ptr[g] + threadIdx.x; e < edge_ptr[g + 1]; e += 256) {
        const float im[3] = {image[3 * e], image[3 * e + 1], image[3 * e + 2]};
        const float gv[3] = {g_vec[3 * e], g_vec[3 * e + 1], g_vec[3 * e + 2]};
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = 0; j < 3; ++j) acc[3 * i + j] = fmaf(im[i], gv[j], acc[3 * i + j]);
    }
    for (int64_t a = atom_ptr[g] + threadIdx.x; a < atom_ptr[g + 1]; a += 256) {
        const float gp[3] = {g_cart[3 * a], g_cart[3 * a + 1], g_cart[3 * a + 2]};
        const float x[3] = {cart[3 * a], cart[3 * a + 1], cart[3 * a + 2]};
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = 0; j < 3; ++j) acc[9 + 3 * i + j] = fmaf(x[i], gp[j], acc[9 + 3 * i + j]);
#pragma unroll
        for (int j = 0; j < 3; ++j) {  // sym is symmetric: g sym^T = g sym
            float t = gp[0] * sym[j];
            t = fmaf(gp[1], sym[3 + j], t);
            t = fmaf(gp[2], sym[6 + j], t);
            g_cart[3 * a + j] = gp[j] + t;
        }
    }
    __shared__ float part[4][18];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < 18; ++k) {
        const float v = wave_sum(acc[k]);
        if (lane == 0) part[w][k] = v;
    }
    __syncthreads();
    if (threadIdx.x == 0 && g_strain) {
        float tot[18], gs[9];
#pragma unroll
        for (int k = 0; k < 18; ++k) tot[k] = ((part[0][k] + part[1][k]) + part[2][k]) + part[3][k];
        const float *L = lat + 9 * g;
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = 0; j < 3; ++j) {  // (L^T (-P))[i][j] = -sum_k L[k][i] P[k][j]
                float t = L[i] * tot[j];
                t = fmaf(L[3 + i], tot[3 + j], t);
                t = fmaf(L[6 + i], tot[6 + j], t);
                gs[3 * i + j] = tot[9 + 3 * i + j] - t;
            }
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
            for (int j = 0; j < 3; ++j) g_strain[9 * g + 3 * i + j] = 0.5f * (gs[3 * i + j] + gs[3 * j + i]);
    }
}

extern "C" int matris_edge_geom_fwd_batch(int64_t n_graphs, int64_t n_edges, const float *cart, const float *lattice,
                                          const float *strain, const float *image, const int32_t *tgt,
                                          const int32_t *src, const int32_t *graph_of_edge, float *length,
                                          float *unit, float *lattice_out, float *volume, void *stream) {
    if (n_graphs < 1 || n_edges < 0 || !lattice || !lattice_out || !volume) return MATRIS_E_ARG;
    if (n_edges > 0 && (!cart || !image || !tgt || !src || !graph_of_edge || !length || !unit)) return MATRIS_E_ARG;
    unsigned *status = matris_range_flag();
    if (!status) return MATRIS_E_ARG;
    const int64_t nt = n_edges > n_graphs ? n_edges : n_graphs;
    edge_geom_fwd_batch_kernel<<<matris_blocks(nt, 256), 256, 0, (hipStream_t)stream>>>(
        n_edges, n_graphs, cart, lattice, strain, image, tgt, src, graph_of_edge, length, unit, lattice_out, volume,
        status);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_edge_geom_bwd_batch(int64_t n_graphs, int64_t n_atoms, int64_t n_edges, const float *g_length,
                                          const float *g_unit, const float *length, const float *unit,
                                          const float *cart, const float *lattice, const float *strain,
                                          const float *image, const int32_t *t_ptr, const int32_t *t_perm,
                                          const int32_t *s_ptr, const int32_t *s_perm, const int32_t *atom_ptr,
                                          const int32_t *edge_ptr, float *g_vec, float *g_cart, float *g_strain,
                                          void *stream) {
    if (n_graphs < 1 || n_atoms < 0 || n_edges < 0 || !cart || !lattice || !t_ptr || !s_ptr || !g_cart)
        return MATRIS_E_ARG;
    if (n_edges > 0 && (!length || !unit || !image || !g_vec)) return MATRIS_E_ARG;
    if (g_strain && !strain) return MATRIS_E_ARG;
    if (strain && (!atom_ptr || !edge_ptr)) return MATRIS_E_ARG;
    hipStream_t st = (hipStream_t)stream;
    if (n_edges > 0) {
        edge_gvec_kernel<<<matris_blocks(n_edges, 256), 256, 0, st>>>(n_edges, g_length, g_unit, length, unit,
                                                                      g_vec);
        MATRIS_CHECK_LAUNCH();
    }
    if (n_atoms > 0) {
        edge_vec_bwd_kernel<<<matris_blocks(n_atoms, WAVES_PER_BLOCK), 256, 0, st>>>(n_atoms, g_vec, t_ptr, t_perm,
                                                                                     s_ptr, s_perm, g_cart);
        MATRIS_CHECK_LAUNCH();
    }
    if (strain) {  // per graph: g' -> g_cart through the strained positions, and the strain's gradient
        edge_geom_bwd_graph_kernel<<<(unsigned)n_graphs, 256, 0, st>>>(atom_ptr, edge_ptr, g_vec, image, cart,
                                                                       lattice, strain, g_cart, g_strain);
        MATRIS_CHECK_LAUNCH();
    }
    return 0;
}

// ------------------------------------------------------------------------------------
// segment attention forward: one wave per (segment, side).  Each half-wave owns every
// other row of the segment with 16-byte lanes (4 columns) and runs an online softmax
// taken eight of its rows at a time (sixteen rows of loads in flight per wave), then four,
// then one: the running maximum moves once per chunk (one rescale exponential), then
// one exponential per row, all on v_exp_f32 (exp_neg_f).  The two halves' (max, sum,
// weighted sum) states merge at the end.  An empty segment writes y = 0 and no log-sum-exp
// (the backward reads the statistics of non-empty segments only).
// ------------------------------------------------------------------------------------
struct OnlineSoftmax4 {
    float4 m, s, acc;
    __device__ void init() {
        m = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        s = acc = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    // raise the running maximum to mn, rescaling (s, acc) (nothing to rescale while m = -inf)
    __device__ void raise(const float4 &mn) {
#define OS_RAISE(k)                                                          \
    {                                                                        \
        const float c = m.k == -INFINITY ? 0.f : exp_neg_f(mn.k - m.k);     \
        s.k *= c;                                                            \
        acc.k *= c;                                                          \
        m.k = mn.k;                                                          \
    }
        OS_RAISE(x) OS_RAISE(y) OS_RAISE(z) OS_RAISE(w)
#undef OS_RAISE
    }
    // fold a row whose logits do not exceed m
    __device__ void add(const float4 &x, const float4 &ev) {
#define OS_ADD(k)                                    \
    {                                                \
        const float w = exp_neg_f(m.k - x.k);        \
        s.k += w;                                    \
        acc.k += w * ev.k;                           \
    }
        OS_ADD(x) OS_ADD(y) OS_ADD(z) OS_ADD(w)
#undef OS_ADD
    }
};


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
    // wave w -> segment w / 2, side w % 2: the two sides of nearby segments run together,
    // so the source side's second read of e' rows tends to find them still in cache
    // the atom-graph launch (N segments, rows gathered from the bonds' logits) reads less
    // from HBM with each XCD on one range of atoms; the line-graph launch is faster with
    // the hardware's round-robin spread
    int64_t w = (HAS_AIDX ? xcd_block() : (int64_t)blockIdx.x) * WAVES_PER_BLOCK + (threadIdx.x >> 6);
    if (w >= 2 * n_seg) return;
    const bool src_side = w & 1;
    const int64_t seg = w >> 1;
    const int32_t *ptr = src_side ? s_ptr : t_ptr;
    const int32_t *perm = src_side ? s_perm : t_perm;
    const int half = (threadIdx.x >> 5) & 1, c = 4 * (threadIdx.x & 31);
    const float *alpha = (src_side ? alpha_s : alpha_t) + c;
    const float *ec = e + c;
    const int b = ptr[seg], end = ptr[seg + 1];
    float *yo = (src_side ? y_s : y_t) + seg * MATRIS_D + c;
    if (end <= b) {
        if (half == 0) st4(yo, make_float4(0.f, 0.f, 0.f, 0.f));
        return;
    }
    auto row = [&](int i) -> int64_t { return perm ? perm[i] : i; };
    auto arow = [&](int64_t r) -> int64_t { return HAS_AIDX ? (int64_t)aidx[r] : r; };
    OnlineSoftmax4 st;
    st.init();
    int i = b + half;  // this half's rows: i, i + 2, i + 4, ...
    for (; i + 14 < end; i += 16) {
        int64_t r[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) r[k] = row(i + 2 * k);
        float4 x[8], ev[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            x[k] = ld4(alpha + arow(r[k]) * lda);
            ev[k] = ld4(ec + r[k] * MATRIS_D);
        }
        st.raise(max4(st.m, max4(max4(max4(x[0], x[1]), max4(x[2], x[3])), max4(max4(x[4], x[5]), max4(x[6], x[7])))));
#pragma unroll
        for (int k = 0; k < 8; ++k) st.add(x[k], ev[k]);
    }
    for (; i + 6 < end; i += 8) {
        const int64_t r0 = row(i), r1 = row(i + 2), r2 = row(i + 4), r3 = row(i + 6);
        const float4 x0 = ld4(alpha + arow(r0) * lda), x1 = ld4(alpha + arow(r1) * lda);
        const float4 x2 = ld4(alpha + arow(r2) * lda), x3 = ld4(alpha + arow(r3) * lda);
        const float4 e0 = ld4(ec + r0 * MATRIS_D), e1 = ld4(ec + r1 * MATRIS_D);
        const float4 e2 = ld4(ec + r2 * MATRIS_D), e3 = ld4(ec + r3 * MATRIS_D);
        st.raise(max4(st.m, max4(max4(x0, x1), max4(x2, x3))));
        st.add(x0, e0);
        st.add(x1, e1);
        st.add(x2, e2);
        st.add(x3, e3);
    }
    for (; i < end; i += 2) {
        const int64_t r0 = row(i);
        const float4 x0 = ld4(alpha + arow(r0) * lda), e0 = ld4(ec + r0 * MATRIS_D);
        st.raise(max4(st.m, x0));
        st.add(x0, e0);
    }
    // merge the other half's state (lane ^ 32 holds the same columns); a half with no rows
    // (a one-row segment) has m = -inf and contributes nothing
    const float4 om = shfl_xor4(st.m, 32), os = shfl_xor4(st.s, 32), oa = shfl_xor4(st.acc, 32);
    float4 y, l;
#define OS_MERGE(k)                                                                       \
    {                                                                                     \
        const float mm = fmaxf(st.m.k, om.k);                                             \
        const float c0 = st.m.k == -INFINITY ? 0.f : exp_neg_f(mm - st.m.k);              \
        const float c1 = om.k == -INFINITY ? 0.f : exp_neg_f(mm - om.k);                  \
        const float ss = st.s.k * c0 + os.k * c1;                                         \
        y.k = (st.acc.k * c0 + oa.k * c1) / ss;                                           \
        l.k = mm + logf(ss);                                                              \
    }
    OS_MERGE(x) OS_MERGE(y) OS_MERGE(z) OS_MERGE(w)
#undef OS_MERGE
    if (half == 0) {
        st4(yo, y);
        st4((src_side ? lse_s : lse_t) + seg * MATRIS_D + c, l);
    }
}

extern "C" int matris_attn_fwd(int64_t n_rows, int64_t n_seg, const float *alpha_t, const float *alpha_s,
                               int64_t lda, const int32_t *alpha_idx, const float *e, const int32_t *t_ptr,
                               const int32_t *t_perm, const int32_t *s_ptr, const int32_t *s_perm, float *y_t,
                               float *y_s, float *lse_t, float *lse_s, void *stream) {
    if (n_rows < 0 || n_seg < 0 || lda < MATRIS_D || (lda % 4) || !t_ptr || !s_ptr || !y_t || !y_s || !lse_t ||
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
// segment attention backward: two rows per wave (half-wave per row, 16-byte lanes)
//   p = exp(alpha - lse[seg]) (exp_neg_f);  g_e = p_t g_yt + p_s g_ys;
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
    const int64_t r = ((int64_t)blockIdx.x * WAVES_PER_BLOCK + (threadIdx.x >> 6)) * 2 + ((threadIdx.x >> 5) & 1);
    if (r >= n_rows) return;
    const int c = 4 * (threadIdx.x & 31);
    const int64_t a = HAS_AIDX ? aidx[r] : r;
    const int64_t t = t_idx[r], s = s_idx[r];
    const float4 at = ld4(alpha_t + a * lda + c), as = ld4(alpha_s + a * lda + c);
    const float4 ev = ld4(e + r * MATRIS_D + c);
    const float4 lt = ld4(lse_t + t * MATRIS_D + c), ls = ld4(lse_s + s * MATRIS_D + c);
    const float4 gt = ld4(g_yt + t * ldgy + c), gs = ld4(g_ys + s * ldgy + c);
    const float4 yt = ld4(y_t + t * MATRIS_D + c), ys = ld4(y_s + s * MATRIS_D + c);
    float4 ge = g_e_base ? ld4(g_e_base + r * MATRIS_D + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    float4 gat, gas;
#define ATTN_BWD_COL(k)                                                  \
    {                                                                    \
        const float pt = exp_neg_f(lt.k - at.k), ps = exp_neg_f(ls.k - as.k); \
        ge.k += pt * gt.k + ps * gs.k;                                   \
        gat.k = pt * gt.k * (ev.k - yt.k);                               \
        gas.k = ps * gs.k * (ev.k - ys.k);                               \
    }
    ATTN_BWD_COL(x) ATTN_BWD_COL(y) ATTN_BWD_COL(z) ATTN_BWD_COL(w)
#undef ATTN_BWD_COL
    st4(g_e + r * MATRIS_D + c, ge);
    st4(g_alpha_t + r * MATRIS_D + c, gat);
    st4(g_alpha_s + r * MATRIS_D + c, gas);
}

// The atom-graph backward by undirected bond: the logits are per bond (read by both
// directed copies through d2u), so one wave takes a bond's directed rows (its d2u segment,
// half-waves on alternate rows), reads the bond's logit rows and base gradient once, writes
// g_e per directed row and the bond's g_alpha_t / g_alpha_s (the sums over its rows, the
// halves combined) -- the d2u reductions of per-row logit gradients and the gather of the
// base gradient happen here instead of in three more launches.
__global__ __launch_bounds__(256) void attn_bwd_bond_kernel(
    int64_t n_bond, const float *__restrict__ alpha_t, const float *__restrict__ alpha_s, int64_t lda,
    const float *__restrict__ e, const int32_t *__restrict__ u_ptr, const int32_t *__restrict__ u_perm,
    const int32_t *__restrict__ t_idx, const int32_t *__restrict__ s_idx, const float *__restrict__ y_t,
    const float *__restrict__ y_s, const float *__restrict__ lse_t, const float *__restrict__ lse_s,
    const float *__restrict__ g_yt, const float *__restrict__ g_ys, int64_t ldgy, const float *__restrict__ g_base,
    float base_scale, float *__restrict__ g_alpha_t, float *__restrict__ g_alpha_s, float *__restrict__ g_e) {
    const int64_t u = (int64_t)blockIdx.x * WAVES_PER_BLOCK + (threadIdx.x >> 6);
    if (u >= n_bond) return;
    const int half = (threadIdx.x >> 5) & 1, c = 4 * (threadIdx.x & 31);
    const float4 at = ld4(alpha_t + u * lda + c), as = ld4(alpha_s + u * lda + c);
    float4 gb = make_float4(0.f, 0.f, 0.f, 0.f);
    if (g_base) {
        const float4 v = ld4(g_base + u * MATRIS_D + c);
        gb = make_float4(base_scale * v.x, base_scale * v.y, base_scale * v.z, base_scale * v.w);
    }
    float4 sat = make_float4(0.f, 0.f, 0.f, 0.f), sas = sat;
    const int b = u_ptr[u], end = u_ptr[u + 1];
    for (int i = b + half; i < end; i += 2) {
        const int64_t r = u_perm ? u_perm[i] : i;
        const int64_t t = t_idx[r], s = s_idx[r];
        const float4 ev = ld4(e + r * MATRIS_D + c);
        const float4 lt = ld4(lse_t + t * MATRIS_D + c), ls = ld4(lse_s + s * MATRIS_D + c);
        const float4 gt = ld4(g_yt + t * ldgy + c), gs = ld4(g_ys + s * ldgy + c);
        const float4 yt = ld4(y_t + t * MATRIS_D + c), ys = ld4(y_s + s * MATRIS_D + c);
        float4 ge = gb;
#define ATTN_BWD_COL(k)                                                       \
    {                                                                         \
        const float pt = exp_neg_f(lt.k - at.k), ps = exp_neg_f(ls.k - as.k); \
        ge.k += pt * gt.k + ps * gs.k;                                        \
        sat.k += pt * gt.k * (ev.k - yt.k);                                   \
        sas.k += ps * gs.k * (ev.k - ys.k);                                   \
    }
        ATTN_BWD_COL(x) ATTN_BWD_COL(y) ATTN_BWD_COL(z) ATTN_BWD_COL(w)
#undef ATTN_BWD_COL
        st4(g_e + r * MATRIS_D + c, ge);
    }
    const float4 ot = shfl_xor4(sat, 32), os = shfl_xor4(sas, 32);
    if (half == 0) {
        st4(g_alpha_t + u * MATRIS_D + c, make_float4(sat.x + ot.x, sat.y + ot.y, sat.z + ot.z, sat.w + ot.w));
        st4(g_alpha_s + u * MATRIS_D + c, make_float4(sas.x + os.x, sas.y + os.y, sas.z + os.z, sas.w + os.w));
    }
}

extern "C" int matris_attn_bwd_bond(int64_t n_bond, const float *alpha_t, const float *alpha_s, int64_t lda,
                                    const float *e, const int32_t *u_ptr, const int32_t *u_perm,
                                    const int32_t *t_idx, const int32_t *s_idx, const float *y_t, const float *y_s,
                                    const float *lse_t, const float *lse_s, const float *g_yt, const float *g_ys,
                                    int64_t ldgy, const float *g_base, float base_scale, float *g_alpha_t,
                                    float *g_alpha_s, float *g_e, void *stream) {
    if (n_bond < 0 || lda < MATRIS_D || (lda % 4) || ldgy < MATRIS_D || (ldgy % 4) || !alpha_t || !alpha_s || !e ||
        !u_ptr || !t_idx || !s_idx || !y_t || !y_s || !lse_t || !lse_s || !g_yt || !g_ys || !g_alpha_t ||
        !g_alpha_s || !g_e)
        return MATRIS_E_ARG;
    if (n_bond == 0) return 0;
    attn_bwd_bond_kernel<<<matris_blocks(n_bond, WAVES_PER_BLOCK), 256, 0, (hipStream_t)stream>>>(
        n_bond, alpha_t, alpha_s, lda, e, u_ptr, u_perm, t_idx, s_idx, y_t, y_s, lse_t, lse_s, g_yt, g_ys, ldgy,
        g_base, base_scale, g_alpha_t, g_alpha_s, g_e);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_attn_bwd(int64_t n_rows, int64_t n_seg, const float *alpha_t, const float *alpha_s,
                               int64_t lda, const int32_t *alpha_idx, const float *e, const int32_t *t_idx,
                               const int32_t *s_idx, const float *y_t, const float *y_s, const float *lse_t,
                               const float *lse_s, const float *g_yt, const float *g_ys, int64_t ldgy,
                               float *g_alpha_t, float *g_alpha_s, float *g_e, const float *g_e_base, void *stream) {
    if (n_rows < 0 || n_seg < 0 || lda < MATRIS_D || (lda % 4) || ldgy < MATRIS_D || (ldgy % 4) || !t_idx ||
        !s_idx || !g_alpha_t || !g_alpha_s || !g_e)
        return MATRIS_E_ARG;
    if (n_rows == 0) return 0;
    if (alpha_idx)
        attn_bwd_kernel<true><<<matris_blocks(n_rows, 2 * WAVES_PER_BLOCK), 256, 0, (hipStream_t)stream>>>(
            n_rows, alpha_t, alpha_s, lda, alpha_idx, e, t_idx, s_idx, y_t, y_s, lse_t, lse_s, g_yt, g_ys, ldgy,
            g_alpha_t, g_alpha_s, g_e, g_e_base);
    else
        attn_bwd_kernel<false><<<matris_blocks(n_rows, 2 * WAVES_PER_BLOCK), 256, 0, (hipStream_t)stream>>>(
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
// One wave per segment; the two half-waves take alternating rows (16-byte lanes, four
// rows each in flight) and combine in the same order in both halves.
__global__ __launch_bounds__(256) void env_agg_fwd_kernel(int64_t n_seg, const float *__restrict__ h,
                                                          const float *__restrict__ env,
                                                          const int32_t *__restrict__ t_ptr,
                                                          const int32_t *__restrict__ t_perm,
                                                          const int32_t *__restrict__ s_idx, float *__restrict__ S,
                                                          float *__restrict__ agg) {
    const int64_t seg = (int64_t)blockIdx.x * WAVES_PER_BLOCK + (threadIdx.x >> 6);
    if (seg >= n_seg) return;
    const int half = (threadIdx.x >> 5) & 1, c = 4 * (threadIdx.x & 31);
    const int b = t_ptr[seg], end = t_ptr[seg + 1];
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    int i = b + half;
    for (; i + 6 < end; i += 8) {
        const int64_t r0 = t_perm ? t_perm[i] : i, r1 = t_perm ? t_perm[i + 2] : i + 2;
        const int64_t r2 = t_perm ? t_perm[i + 4] : i + 4, r3 = t_perm ? t_perm[i + 6] : i + 6;
        const int64_t s0 = s_idx[r0], s1 = s_idx[r1], s2 = s_idx[r2], s3 = s_idx[r3];
        const float4 h0 = ld4(h + r0 * MATRIS_D + c), h1 = ld4(h + r1 * MATRIS_D + c);
        const float4 h2 = ld4(h + r2 * MATRIS_D + c), h3 = ld4(h + r3 * MATRIS_D + c);
        const float4 w0 = ld4(env + s0 * MATRIS_D + c), w1 = ld4(env + s1 * MATRIS_D + c);
        const float4 w2 = ld4(env + s2 * MATRIS_D + c), w3 = ld4(env + s3 * MATRIS_D + c);
        acc.x += h0.x * w0.x; acc.y += h0.y * w0.y; acc.z += h0.z * w0.z; acc.w += h0.w * w0.w;
        acc.x += h1.x * w1.x; acc.y += h1.y * w1.y; acc.z += h1.z * w1.z; acc.w += h1.w * w1.w;
        acc.x += h2.x * w2.x; acc.y += h2.y * w2.y; acc.z += h2.z * w2.z; acc.w += h2.w * w2.w;
        acc.x += h3.x * w3.x; acc.y += h3.y * w3.y; acc.z += h3.z * w3.z; acc.w += h3.w * w3.w;
    }
    for (; i < end; i += 2) {
        const int64_t r0 = t_perm ? t_perm[i] : i;
        const float4 h0 = ld4(h + r0 * MATRIS_D + c), w0 = ld4(env + (int64_t)s_idx[r0] * MATRIS_D + c);
        acc.x += h0.x * w0.x; acc.y += h0.y * w0.y; acc.z += h0.z * w0.z; acc.w += h0.w * w0.w;
    }
    const float4 o = shfl_xor4(acc, 32);
    const float4 t = half ? make_float4(o.x + acc.x, o.y + acc.y, o.z + acc.z, o.w + acc.w)
                          : make_float4(acc.x + o.x, acc.y + o.y, acc.z + o.z, acc.w + o.w);
    if (half) return;
    const float4 et = ld4(env + seg * MATRIS_D + c);
    st4(S + seg * MATRIS_D + c, t);
    st4(agg + seg * MATRIS_D + c, make_float4(et.x * t.x, et.y * t.y, et.z * t.z, et.w * t.w));
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

// g_env: one wave per source segment, half-waves on alternating rows as in the forward;
// with ge given, also ge[b] = g_agg[b] * env[b] (the per-bond factor of g_h's term).
template <bool PROJ>
__global__ __launch_bounds__(256) void env_agg_bwd_env_kernel(int64_t n_seg, const float *__restrict__ h,
                                                              const float *__restrict__ env,
                                                              const float *__restrict__ g_agg,
                                                              const float *__restrict__ S,
                                                              const int32_t *__restrict__ s_ptr,
                                                              const int32_t *__restrict__ s_perm,
                                                              const int32_t *__restrict__ t_idx,
                                                              float *__restrict__ g_env, float *__restrict__ ge,
                                                              const float *__restrict__ proj_w, int proj_k,
                                                              int accumulate) {
    __shared__ __align__(16) float wts[PROJ ? MATRIS_PROJ_KMAX * MATRIS_D : 4];
    if constexpr (PROJ) {  // the block's copy of wt (before any wave leaves)
        for (int q = threadIdx.x; q < proj_k * MATRIS_D / 4; q += blockDim.x)
            reinterpret_cast<float4 *>(wts)[q] = ld4(proj_w + 4 * q);
        lds_barrier();
    }
    const int64_t seg = (int64_t)blockIdx.x * WAVES_PER_BLOCK + (threadIdx.x >> 6);
    if (seg >= n_seg) return;
    const int half = (threadIdx.x >> 5) & 1, c = 4 * (threadIdx.x & 31);
    const int b = s_ptr[seg], end = s_ptr[seg + 1];
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    int i = b + half;
    for (; i + 6 < end; i += 8) {
        const int64_t r0 = s_perm ? s_perm[i] : i, r1 = s_perm ? s_perm[i + 2] : i + 2;
        const int64_t r2 = s_perm ? s_perm[i + 4] : i + 4, r3 = s_perm ? s_perm[i + 6] : i + 6;
        const int64_t t0 = t_idx[r0], t1 = t_idx[r1], t2 = t_idx[r2], t3 = t_idx[r3];
        const float4 h0 = ld4(h + r0 * MATRIS_D + c), h1 = ld4(h + r1 * MATRIS_D + c);
        const float4 h2 = ld4(h + r2 * MATRIS_D + c), h3 = ld4(h + r3 * MATRIS_D + c);
        const float4 g0 = ld4(g_agg + t0 * MATRIS_D + c), g1 = ld4(g_agg + t1 * MATRIS_D + c);
        const float4 g2 = ld4(g_agg + t2 * MATRIS_D + c), g3 = ld4(g_agg + t3 * MATRIS_D + c);
        const float4 e0 = ld4(env + t0 * MATRIS_D + c), e1 = ld4(env + t1 * MATRIS_D + c);
        const float4 e2 = ld4(env + t2 * MATRIS_D + c), e3 = ld4(env + t3 * MATRIS_D + c);
        acc.x += g0.x * e0.x * h0.x; acc.y += g0.y * e0.y * h0.y; acc.z += g0.z * e0.z * h0.z; acc.w += g0.w * e0.w * h0.w;
        acc.x += g1.x * e1.x * h1.x; acc.y += g1.y * e1.y * h1.y; acc.z += g1.z * e1.z * h1.z; acc.w += g1.w * e1.w * h1.w;
        acc.x += g2.x * e2.x * h2.x; acc.y += g2.y * e2.y * h2.y; acc.z += g2.z * e2.z * h2.z; acc.w += g2.w * e2.w * h2.w;
        acc.x += g3.x * e3.x * h3.x; acc.y += g3.y * e3.y * h3.y; acc.z += g3.z * e3.z * h3.z; acc.w += g3.w * e3.w * h3.w;
    }
    for (; i < end; i += 2) {
        const int64_t r0 = s_perm ? s_perm[i] : i;
        const int64_t t0 = t_idx[r0];
        const float4 h0 = ld4(h + r0 * MATRIS_D + c), g0 = ld4(g_agg + t0 * MATRIS_D + c);
        const float4 e0 = ld4(env + t0 * MATRIS_D + c);
        acc.x += g0.x * e0.x * h0.x; acc.y += g0.y * e0.y * h0.y; acc.z += g0.z * e0.z * h0.z; acc.w += g0.w * e0.w * h0.w;
    }
    const float4 o = shfl_xor4(acc, 32);
    const float4 t = half ? make_float4(o.x + acc.x, o.y + acc.y, o.z + acc.z, o.w + acc.w)
                          : make_float4(acc.x + o.x, acc.y + o.y, acc.z + o.z, acc.w + o.w);
    if (half) return;
    const float4 gs = ld4(g_agg + seg * MATRIS_D + c), sv = ld4(S + seg * MATRIS_D + c);
    if (ge) {
        const float4 es = ld4(env + seg * MATRIS_D + c);
        st4(ge + seg * MATRIS_D + c, make_float4(gs.x * es.x, gs.y * es.y, gs.z * es.z, gs.w * es.w));
    }
    const float4 gv = make_float4(gs.x * sv.x + t.x, gs.y * sv.y + t.y, gs.z * sv.z + t.z, gs.w * sv.w + t.w);
    if constexpr (PROJ)  // g_env projected onto the envelope's basis: [n_seg, K]
        proj_row_store(gv, threadIdx.x & 31, wts, proj_k, accumulate, g_env + seg * proj_k);
    else
        st4(g_env + seg * MATRIS_D + c, gv);
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
    // h, env, g_agg, S and g_h are read as float4 rows
    if (((uintptr_t)h | (uintptr_t)env | (uintptr_t)g_agg | (uintptr_t)S | (uintptr_t)g_h | (uintptr_t)g_env) & 15)
        return MATRIS_E_ARG;
    hipStream_t st = (hipStream_t)stream;
    if (n_rows > 0) {
        env_agg_bwd_rows_kernel<<<matris_blocks(n_rows * 32, 256), 256, 0, st>>>(n_rows, g_agg, env, t_idx, s_idx,
                                                                               accumulate, g_h);
        MATRIS_CHECK_LAUNCH();
    }
    if (n_seg > 0) {
        env_agg_bwd_env_kernel<false><<<matris_blocks(n_seg, WAVES_PER_BLOCK), 256, 0, st>>>(
            n_seg, h, env, g_agg, S, s_ptr, s_perm, t_idx, g_env, nullptr, nullptr, 0, 0);
        MATRIS_CHECK_LAUNCH();
    }
    return 0;
}

extern "C" int matris_env_agg_bwd_env(int64_t n_seg, const float *h, const float *env, const float *g_agg,
                                      const float *S, const int32_t *t_idx, const int32_t *s_ptr,
                                      const int32_t *s_perm, float *g_env, float *g_agg_env, void *stream) {
    if (n_seg < 0 || !h || !env || !g_agg || !S || !t_idx || !s_ptr || !g_env) return MATRIS_E_ARG;
    if (((uintptr_t)h | (uintptr_t)env | (uintptr_t)g_agg | (uintptr_t)S | (uintptr_t)g_env | (uintptr_t)g_agg_env) &
        15)
        return MATRIS_E_ARG;
    if (n_seg == 0) return 0;
    env_agg_bwd_env_kernel<false><<<matris_blocks(n_seg, WAVES_PER_BLOCK), 256, 0, (hipStream_t)stream>>>(
        n_seg, h, env, g_agg, S, s_ptr, s_perm, t_idx, g_env, g_agg_env, nullptr, 0, 0);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_env_agg_bwd_env_proj(int64_t n_seg, const float *h, const float *env, const float *g_agg,
                                           const float *S, const int32_t *t_idx, const int32_t *s_ptr,
                                           const int32_t *s_perm, const float *proj_w, int proj_k, int accumulate,
                                           float *g_basis, float *g_agg_env, void *stream) {
    if (n_seg < 0 || !h || !env || !g_agg || !S || !t_idx || !s_ptr || !g_basis || !proj_w || proj_k < 1 ||
        proj_k > MATRIS_PROJ_KMAX)
        return MATRIS_E_ARG;
    if (((uintptr_t)h | (uintptr_t)env | (uintptr_t)g_agg | (uintptr_t)S | (uintptr_t)g_agg_env | (uintptr_t)proj_w) &
        15)
        return MATRIS_E_ARG;
    if (n_seg == 0) return 0;
    env_agg_bwd_env_kernel<true><<<matris_blocks(n_seg, WAVES_PER_BLOCK), 256, 0, (hipStream_t)stream>>>(
        n_seg, h, env, g_agg, S, s_ptr, s_perm, t_idx, g_basis, g_agg_env, proj_w, proj_k, accumulate);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

// ------------------------------------------------------------------------------------
// the learnable envelope (interaction_block.py:240-246): env = basis W^T, a Linear(K, 128)
// without bias on each bond's K basis values (K <= 8).  A half-wave per row (lane l:
// columns 4l .. 4l+3) with the lane's K float4 of W^T held in registers over a
// grid-stride loop of 32-row passes.
// ------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void env_linear_kernel(int64_t n, int K, const float *__restrict__ basis,
                                                         const float *__restrict__ wt, float *__restrict__ env) {
    // per block pass: 32 rows, their K basis values staged in LDS by one coalesced load;
    // half-wave j takes rows j, j + 8, j + 16, j + 24 of the pass
    __shared__ float bs[32 * MATRIS_PROJ_KMAX];
    const int l = threadIdx.x & 31, hw = threadIdx.x >> 5;
    float4 w[MATRIS_PROJ_KMAX];
#pragma unroll
    for (int k = 0; k < MATRIS_PROJ_KMAX; ++k) w[k] = k < K ? ld4(wt + k * MATRIS_D + 4 * l) : make_float4(0.f, 0.f, 0.f, 0.f);
    for (int64_t r0 = (int64_t)blockIdx.x * 32; r0 < n; r0 += (int64_t)gridDim.x * 32) {  // uniform over the block
        const int64_t nr = n - r0 < 32 ? n - r0 : 32;
        const float bv = threadIdx.x < nr * K ? basis[r0 * K + threadIdx.x] : 0.f;
        lds_barrier();  // the previous pass is done reading bs (W's loads stay in flight)
        if (threadIdx.x < nr * K) bs[threadIdx.x] = bv;
        lds_barrier();
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int rr = hw + 8 * q;
            if (rr >= nr) break;
            const float *b = bs + rr * K;
            float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int k = 0; k < MATRIS_PROJ_KMAX; ++k)
                if (k < K) {
                    const float x = b[k];
                    o.x = fmaf(x, w[k].x, o.x);
                    o.y = fmaf(x, w[k].y, o.y);
                    o.z = fmaf(x, w[k].z, o.z);
                    o.w = fmaf(x, w[k].w, o.w);
                }
            st4(env + (r0 + rr) * MATRIS_D + 4 * l, o);
        }
    }
}

extern "C" int matris_env_linear(int64_t n, int k, const float *basis, const float *wt, float *env, void *stream) {
    if (n < 0 || k < 1 || k > MATRIS_PROJ_KMAX) return MATRIS_E_ARG;
    if (n == 0) return 0;
    if (!basis || !wt || !env || (((uintptr_t)env | (uintptr_t)wt) & 15)) return MATRIS_E_ARG;
    const int64_t nb = matris_blocks(n, 32), blocks = nb < 2048 ? nb : 2048;
    env_linear_kernel<<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>(n, k, basis, wt, env);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" const char *matris_version(void) { return "matris_hip 0.1 gfx950"; }
