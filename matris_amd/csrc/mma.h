// MFMA building blocks shared by the fused GEMM kernels (gmlp.hip, mlp.hip).
//
// Fragments.  Every GEMM here runs on 32x32 output tiles with K consumed in 16-wide
// blocks.  The operand fragment of one 32-row tile and one k-block is, for lane
// l = l32 + 32h, the 8 values (row l32, k = 8h .. 8h+7).  It is held as NPL 16-byte
// "planes":
//   MODE 0  fp32 operands: planes = the 8 floats (2 x float4); v_mfma_f32_32x32x2f32 step
//           s (0..7) consumes element s, i.e. k = 8h + s for lane half h.
//   MODE 3  x = hi + mid (+ residual), hi = x truncated to bf16, mid = bf16(x - hi)
//           rounded: planes hi, mid; 3 bf16 products (hi*hi + hi*mid + mid*hi) on
//           v_mfma_f32_32x32x16_bf16.
//   MODE 6  x = hi + mid + lo exactly (truncated hi, mid; exact lo): planes hi, mid, lo;
//           6 products (adds hi*lo + mid*mid + lo*hi): fp32-grade products.
//   MODE 2  fp16 split on v_mfma_f32_32x32x16_f16.  Activations: hi = fp16(x), lo =
//           fp16((x - hi) 2^11) (both round-to-nearest), so x = hi + 2^-11 lo to ~2^-22 |x|
//           (subnormal fp16 keeps the absolute error of tiny x near 2^-36).  Weights are
//           scaled by a power of two s per matrix (max |s w| in [2^14, 2^15)) and stored
//           as u0 = fp16(s w), u1 = fp16(s w - u0); a third register plane u0 2^-11 is made
//           at use (one v_pk_mul_f16 per register).  3 products into one accumulator:
//           u1 hi + (2^-11 u0) lo + u0 hi = s w x to ~2^-22 relative, and the result is
//           scaled back by 1/s (exact).  fp16 has a finite range: activations with
//           |x| >= 65504 are flagged (report_range) so the caller can redo the work in
//           MODE 6.
// A and B fragments use the same k assignment, so every mode sums over the same k.
// The bf16 / f16 instructions' layout (A lane l: row l%32, k = 8(l/32)..+7; B lane l:
// k = 8(l/32)..+7, column l%32) is exactly this fragment.
//
// Weights (B operands) are packed once per parameter version by matris_pack_b into
// fragment-major order: 16-byte unit ((nt * KB + kb) * NPL + plane) * 64 + lane for
// output-column tile nt, k-block kb (KB = K / 16).  A wave's fragment load is then one
// contiguous 1 KB read per plane and no weight is converted inside a GEMM loop.  A
// MODE 2 image starts with a 16-byte header {1/s, s, 0, 0} (take_wscale).
#pragma once
#include "common.h"

typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float f2v __attribute__((ext_vector_type(2)));

#define BM 64    // rows per work-group
#define LDH 260  // LDS row stride (floats) of a [64, 256] fp32 tile
#define LDT 132  // LDS row stride of a [64, 128] fp32 tile

template <int MODE>
struct Npl {
    static constexpr int v = MODE == 6 ? 3 : 2;
};

// Register planes: MODE 2 weight fragments carry the derived plane u0 2^-11 (prep_w) as
// p[2]; activation fragments leave it unused.
template <int MODE>
struct Frag {
    uint4 p[MODE == 2 ? 3 : Npl<MODE>::v];
};

// fp16 overflow threshold of the MODE 2 activation split.
#define MATRIS_F16_MAX 65504.0f

// Streaming (non-temporal) stores for rows that no kernel reads back soon: they do not
// displace the gathered tables and weights that later loads of the same kernel hit in L2.
typedef float matris_f4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void st_nt4(float *p, float4 v) {
    const matris_f4v w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<matris_f4v *>(p));
}
__device__ __forceinline__ void st_nt(float *p, float v) { __builtin_nontemporal_store(v, p); }

// Per-row power-of-two scaling of MODE 2 gradient operands.  fp16's exponent range keeps
// ~22 bits of an activation only inside [2^-14, 2^16); the backward GEMMs' operands are
// gradients whose rows can sit far below it (the RMSNorm Jacobian divides by the row's
// norm, so large features mean small gradients).  Their producers therefore scale each
// row by 2^k with max |row| 2^k in [2^10, 2^11) -- five bits of headroom for what the row
// becomes downstream -- and the consumers multiply that row's accumulators by 2^-k.  Both
// factors are powers of two, so a row already inside the range gives the same products.
// k is clamped to [-100, 100]; a zero or non-finite maximum leaves the row unscaled.
struct RowScale {
    float s, inv;
};
__device__ __forceinline__ RowScale row_scale(float m) {
    if (!(m > 0.f) || m == INFINITY) return {1.f, 1.f};
    const int e = (int)((__float_as_uint(m) >> 23) & 0xffu) - 127;  // floor(log2 m); -127 if subnormal
    const int k = max(-100, min(100, 10 - e));
    return {__uint_as_float((uint32_t)(127 + k) << 23), __uint_as_float((uint32_t)(127 - k) << 23)};
}

template <int CTRL>
__device__ __forceinline__ float dpp_max(float x) {
    return fmaxf(x, dpp_f<CTRL>(x));
}
// max over lanes 4q .. 4q+3, over lanes 8q .. 8q+7, over a DPP row of 16 lanes
__device__ __forceinline__ float group4_max(float v) { return dpp_max<0x4E>(dpp_max<0xB1>(v)); }
__device__ __forceinline__ float group8_max(float v) { return dpp_max<0x141>(group4_max(v)); }
__device__ __forceinline__ float row16_max(float v) { return dpp_max<0x140>(group8_max(v)); }

__device__ __forceinline__ float abs_max4(float m, const float4 &v) {
    return fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
}
__device__ __forceinline__ float4 mul4(const float4 &v, float s) { return make_float4(v.x * s, v.y * s, v.z * s, v.w * s); }

template <class To, class From>
__device__ __forceinline__ To bitcast(const From &x) {
    static_assert(sizeof(To) == sizeof(From), "size");
    return __builtin_bit_cast(To, x);
}

__device__ __forceinline__ v16f mfma32(float a, float b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v16f mfma_bf16(const v8bf &a, const v8bf &b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v16f mfma_f16(const v8h &a, const v8h &b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// sigmoid = 1 / (1 + e^-x) with v_rcp_f32 (1 ulp); SiLU = x sigmoid(x).
__device__ __forceinline__ float sigm_f(float x) { return __builtin_amdgcn_rcpf(1.0f + exp_neg_f(x)); }
__device__ __forceinline__ float silu_f(float x) { return x * sigm_f(x); }
__device__ __forceinline__ float dsilu_f(float x) {
    float s = sigm_f(x);
    return s * (1.0f + x * (1.0f - s));
}

// Row of accumulator register i of a 32x32 tile for lane half h (column = lane % 32).
__device__ __forceinline__ int acc_row(int i, int h) { return (i >> 2) * 8 + h * 4 + (i & 3); }

// 8 fp32 values (k order) -> fragment planes.  The split truncates instead of rounding:
// hi = x with the low 16 bits cleared (the top 8 significant bits, a bf16), r = x - hi
// (exact), mid = r with the low 16 bits cleared, lo = r - mid (exact, at most 8
// significant bits, so it is a bf16 as well): x = hi + mid + lo exactly, with integer
// masks and one v_perm per packed pair instead of round-to-nearest conversions.
// MODE 3 keeps round-to-nearest for mid (its last term).
template <int MODE>
__device__ __forceinline__ void make_frag(Frag<MODE> &f, const float4 &u, const float4 &v) {
    if constexpr (MODE == 0) {
        f.p[0] = bitcast<uint4>(u);
        f.p[1] = bitcast<uint4>(v);
    } else if constexpr (MODE == 2) {
        // hi = fp16(x) and lo = fp16((x - hi) 2^11), two values per v_cvt_pk_f16_f32
        const f2v x0 = {u.x, u.y}, x1 = {u.z, u.w}, x2 = {v.x, v.y}, x3 = {v.z, v.w};
        const h2v h0 = __builtin_convertvector(x0, h2v), h1 = __builtin_convertvector(x1, h2v);
        const h2v h2 = __builtin_convertvector(x2, h2v), h3 = __builtin_convertvector(x3, h2v);
        const h2v l0 = __builtin_convertvector((x0 - __builtin_convertvector(h0, f2v)) * 2048.0f, h2v);
        const h2v l1 = __builtin_convertvector((x1 - __builtin_convertvector(h1, f2v)) * 2048.0f, h2v);
        const h2v l2 = __builtin_convertvector((x2 - __builtin_convertvector(h2, f2v)) * 2048.0f, h2v);
        const h2v l3 = __builtin_convertvector((x3 - __builtin_convertvector(h3, f2v)) * 2048.0f, h2v);
        f.p[0] = make_uint4(bitcast<uint32_t>(h0), bitcast<uint32_t>(h1), bitcast<uint32_t>(h2), bitcast<uint32_t>(h3));
        f.p[1] = make_uint4(bitcast<uint32_t>(l0), bitcast<uint32_t>(l1), bitcast<uint32_t>(l2), bitcast<uint32_t>(l3));
    } else {
        const float x[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
        uint32_t hb[8], mb[8], lb[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            hb[j] = bitcast<uint32_t>(x[j]) & 0xffff0000u;
            const float r = x[j] - bitcast<float>(hb[j]);
            if constexpr (MODE == 6) {
                mb[j] = bitcast<uint32_t>(r) & 0xffff0000u;
                lb[j] = bitcast<uint32_t>(r - bitcast<float>(mb[j]));
            } else {
                mb[j] = (uint32_t)bitcast<uint16_t>((__bf16)r) << 16;
            }
        }
        // pack the upper halves of (even, odd) pairs: bytes 2,3 of the even word, 2,3 of the odd
        auto pk = [](uint32_t even, uint32_t odd) { return __builtin_amdgcn_perm(odd, even, 0x07060302u); };
        f.p[0] = make_uint4(pk(hb[0], hb[1]), pk(hb[2], hb[3]), pk(hb[4], hb[5]), pk(hb[6], hb[7]));
        f.p[1] = make_uint4(pk(mb[0], mb[1]), pk(mb[2], mb[3]), pk(mb[4], mb[5]), pk(mb[6], mb[7]));
        if constexpr (MODE == 6) f.p[2] = make_uint4(pk(lb[0], lb[1]), pk(lb[2], lb[3]), pk(lb[4], lb[5]), pk(lb[6], lb[7]));
    }
}

// Running max |x| of the values a MODE 2 conversion sees (0 in the other modes, which have
// no range limit).  NaN inputs are not counted: they give NaN in every mode.
template <int MODE>
__device__ __forceinline__ float frag_amax(float m, const float4 &u, const float4 &v) {
    if constexpr (MODE == 2) {
        m = fmaxf(m, fmaxf(fmaxf(fabsf(u.x), fabsf(u.y)), fmaxf(fabsf(u.z), fabsf(u.w))));
        return fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    } else {
        return m;
    }
}

// The derived plane of a MODE 2 weight fragment, made once its load has landed.
template <int MODE>
__device__ __forceinline__ void prep_w(Frag<MODE> &w) {
    if constexpr (MODE == 2) w.p[2] = bitcast<uint4>(bitcast<v8h>(w.p[0]) * (_Float16)0.00048828125f);
}

// MODE 2: the weight's 1/s from the header of its packed image, which the pointer then
// skips; 1 in the other modes.
template <int MODE>
__device__ __forceinline__ float take_wscale(const uint4 *__restrict__ &W) {
    if constexpr (MODE == 2) {
        const float s = reinterpret_cast<const float *>(W)[0];
        W += 1;
        return s;
    } else {
        return 1.0f;
    }
}

template <int MODE, int NRT, int NCT>
__device__ __forceinline__ void scale_acc(v16f (&acc)[NRT][NCT], float s) {
    if constexpr (MODE == 2) {
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) acc[rt][ct] *= s;
    }
}

// MODE 2: flag the device's range word if any lane converted a value fp16 cannot hold.
template <int MODE>
__device__ __forceinline__ void report_range(float amax, unsigned *flag) {
    if constexpr (MODE == 2) {
        if (__ballot(amax >= MATRIS_F16_MAX) != 0 && (threadIdx.x & 63) == 0 && flag)
            atomicOr(flag, (unsigned)MATRIS_STATUS_F16_RANGE);
    }
}

// acc += A-fragment * B-fragment over one 16-wide k block.  Smallest products first.
// (Modes 0, 3, 6; MODE 2 goes through mma_wx / mma_xw, which know the weight side.)
template <int MODE>
__device__ __forceinline__ void mma_frag(v16f &acc, const Frag<MODE> &a, const Frag<MODE> &b) {
    if constexpr (MODE == 0) {
        const float4 a0 = bitcast<float4>(a.p[0]), a1 = bitcast<float4>(a.p[1]);
        const float4 b0 = bitcast<float4>(b.p[0]), b1 = bitcast<float4>(b.p[1]);
        acc = mfma32(a0.x, b0.x, acc);
        acc = mfma32(a0.y, b0.y, acc);
        acc = mfma32(a0.z, b0.z, acc);
        acc = mfma32(a0.w, b0.w, acc);
        acc = mfma32(a1.x, b1.x, acc);
        acc = mfma32(a1.y, b1.y, acc);
        acc = mfma32(a1.z, b1.z, acc);
        acc = mfma32(a1.w, b1.w, acc);
    } else {
        const v8bf ah = bitcast<v8bf>(a.p[0]), am = bitcast<v8bf>(a.p[1]);
        const v8bf bh = bitcast<v8bf>(b.p[0]), bm = bitcast<v8bf>(b.p[1]);
        if constexpr (MODE == 6) {
            const v8bf al = bitcast<v8bf>(a.p[2]), bl = bitcast<v8bf>(b.p[2]);
            acc = mfma_bf16(al, bh, acc);
            acc = mfma_bf16(am, bm, acc);
            acc = mfma_bf16(ah, bl, acc);
        }
        acc = mfma_bf16(am, bh, acc);
        acc = mfma_bf16(ah, bm, acc);
        acc = mfma_bf16(ah, bh, acc);
    }
}

// acc += W-fragment (MFMA A operand) * X-fragment (B operand): the transposed products.
template <int MODE>
__device__ __forceinline__ void mma_wx(v16f &acc, const Frag<MODE> &w, const Frag<MODE> &x) {
    if constexpr (MODE == 2) {
        const v8h xh = bitcast<v8h>(x.p[0]), xl = bitcast<v8h>(x.p[1]);
        acc = mfma_f16(bitcast<v8h>(w.p[1]), xh, acc);
        acc = mfma_f16(bitcast<v8h>(w.p[2]), xl, acc);
        acc = mfma_f16(bitcast<v8h>(w.p[0]), xh, acc);
    } else {
        mma_frag<MODE>(acc, w, x);
    }
}

// acc += X-fragment (MFMA A operand) * W-fragment (B operand).
template <int MODE>
__device__ __forceinline__ void mma_xw(v16f &acc, const Frag<MODE> &x, const Frag<MODE> &w) {
    if constexpr (MODE == 2) {
        const v8h xh = bitcast<v8h>(x.p[0]), xl = bitcast<v8h>(x.p[1]);
        acc = mfma_f16(xh, bitcast<v8h>(w.p[1]), acc);
        acc = mfma_f16(xl, bitcast<v8h>(w.p[2]), acc);
        acc = mfma_f16(xh, bitcast<v8h>(w.p[0]), acc);
    } else {
        mma_frag<MODE>(acc, x, w);
    }
}

// B fragments of output tiles nt0 .. nt0+NCT-1, k-block kb, of a packed weight with KB
// k-blocks.
template <int MODE, int NCT>
__device__ __forceinline__ void load_bfrags(Frag<MODE> (&b)[NCT], const uint4 *__restrict__ W, int nt0, int KB, int kb,
                                            int lane) {
    constexpr int NPL = Npl<MODE>::v;
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
        for (int pl = 0; pl < NPL; ++pl)
            b[ct].p[pl] = W[((int64_t)((nt0 + ct) * KB + kb) * NPL + pl) * 64 + lane];
}

// A fragments of NRT 32-row tiles of an fp32 row-major LDS array, k-block kb.
template <int MODE, int NRT>
__device__ __forceinline__ void lds_afrags(Frag<MODE> (&a)[NRT], const float *base, int ld, int kb, int lane,
                                           float &amax) {
    const int h = lane >> 5, l32 = lane & 31;
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
        const float *r = base + (rt * 32 + l32) * ld + kb * 16 + h * 8;
        const float4 u = *reinterpret_cast<const float4 *>(r), v = *reinterpret_cast<const float4 *>(r + 4);
        amax = frag_amax<MODE>(amax, u, v);
        make_frag<MODE>(a[rt], u, v);
    }
}

// acc[rt][ct] += A[rt tile, k-blocks 0..KBA) * B[k-blocks kb0.., tile nt0 + ct] with A an
// fp32 row-major LDS array and B a packed weight (KBW k-blocks); the next k-block's B
// fragments are loaded while the current one is consumed.  The prefetch is
// unconditional (the last step reloads its own block) so the compiler's load counting
// stays exact.
// TRANS computes the transposed product instead, acc[rt][ct] = (B^T A^T) tile: the packed
// weight fragment is the MFMA A operand and the LDS rows the B operand, so lane l holds
// row rt*32 + l%32 of A and its 16 registers are output columns ct*32 + acc_row(i, l/32)
// (four runs of four consecutive columns) -- a layout with whole rows in lanes.
// Returns the running max |A| of a MODE 2 conversion (0 otherwise).  MODE 2 sums carry the
// weight's scale s: the caller applies scale_acc once its last product is in.
// One k-block of gemm_lds_packed: prefetch k-block `kpf` into BPF, then accumulate
// k-block `kb` (A from LDS, B = BCUR).
template <int MODE, int NRT, int NCT, bool TRANS>
__device__ __forceinline__ void gemm_lds_step(v16f (&acc)[NRT][NCT], const float *a_base, int lda,
                                              const uint4 *__restrict__ W, int nt0, int KBW, int kb, int kpf,
                                              Frag<MODE> (&BCUR)[NCT], Frag<MODE> (&BPF)[NCT], int lane,
                                              float &amax) {
    load_bfrags<MODE, NCT>(BPF, W, nt0, KBW, kpf, lane);
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of this step's MFMAs
    Frag<MODE> a[NRT];
    lds_afrags<MODE, NRT>(a, a_base, lda, kb, lane, amax);
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) prep_w<MODE>(BCUR[ct]);
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
            if constexpr (TRANS)
                mma_wx<MODE>(acc[rt][ct], BCUR[ct], a[rt]);
            else
                mma_xw<MODE>(acc[rt][ct], a[rt], BCUR[ct]);
        }
}

// acc[rt][ct] += A[rt tile, k-blocks 0..KBA) * B[k-blocks kb0.., tile nt0 + ct] with A an
// fp32 row-major LDS array and B a packed weight (KBW k-blocks).  With two output tiles
// per wave in a two-plane mode the B fragments are prefetched three k-blocks ahead in a
// ring of four register sets; otherwise one ahead (MODE 6's three planes, or one-tile
// kernels, whose occupancy the deeper ring would lower).  Prefetches past the end reload
// the last k-block, so the compiler's load counting stays exact.
// TRANS computes the transposed product instead, acc[rt][ct] = (B^T A^T) tile: the packed
// weight fragment is the MFMA A operand and the LDS rows the B operand, so lane l holds
// row rt*32 + l%32 of A and its 16 registers are output columns ct*32 + acc_row(i, l/32)
// (four runs of four consecutive columns) -- a layout with whole rows in lanes.
// Returns the running max |A| of a MODE 2 conversion (0 otherwise).  MODE 2 sums carry the
// weight's scale s: the caller applies scale_acc once its last product is in.
template <int MODE, int NRT, int NCT, int KBA, bool TRANS = false>
__device__ __forceinline__ float gemm_lds_packed(v16f (&acc)[NRT][NCT], const float *a_base, int lda,
                                                 const uint4 *__restrict__ W, int nt0, int KBW, int kb0, int lane) {
    float amax = 0.f;
    if constexpr (Npl<MODE>::v == 2 && NCT == 2) {
        static_assert(KBA % 4 == 0, "ring of four");
        Frag<MODE> b0[NCT], b1[NCT], b2[NCT], b3[NCT];
        load_bfrags<MODE, NCT>(b0, W, nt0, KBW, kb0, lane);
        load_bfrags<MODE, NCT>(b1, W, nt0, KBW, kb0 + 1, lane);
        load_bfrags<MODE, NCT>(b2, W, nt0, KBW, kb0 + 2, lane);
#pragma unroll 1
        for (int kb = 0; kb < KBA; kb += 4) {
            gemm_lds_step<MODE, NRT, NCT, TRANS>(acc, a_base, lda, W, nt0, KBW, kb, kb0 + min(kb + 3, KBA - 1), b0,
                                                 b3, lane, amax);
            gemm_lds_step<MODE, NRT, NCT, TRANS>(acc, a_base, lda, W, nt0, KBW, kb + 1, kb0 + min(kb + 4, KBA - 1),
                                                 b1, b0, lane, amax);
            gemm_lds_step<MODE, NRT, NCT, TRANS>(acc, a_base, lda, W, nt0, KBW, kb + 2, kb0 + min(kb + 5, KBA - 1),
                                                 b2, b1, lane, amax);
            gemm_lds_step<MODE, NRT, NCT, TRANS>(acc, a_base, lda, W, nt0, KBW, kb + 3, kb0 + min(kb + 6, KBA - 1),
                                                 b3, b2, lane, amax);
        }
    } else {
        constexpr int kUnroll = NCT >= 2 ? 1 : 2;  // 2-tile bodies are long enough; keeps pressure down
        Frag<MODE> cur[NCT], nxt[NCT];
        load_bfrags<MODE, NCT>(cur, W, nt0, KBW, kb0, lane);
#pragma unroll kUnroll
        for (int kb = 0; kb < KBA; ++kb) {
            gemm_lds_step<MODE, NRT, NCT, TRANS>(acc, a_base, lda, W, nt0, KBW, kb, kb0 + min(kb + 1, KBA - 1), cur,
                                                 nxt, lane, amax);
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) cur[ct] = nxt[ct];
        }
    }
    return amax;
}

// ------------------------------------------------------------------------------------
// Pre-split operand tiles in LDS (two-plane modes): a tile of rows x K stored as fragment
// units [rt][kb][plane][64 lanes] x 16 bytes, so a GEMM reads its A / B fragments with
// one 16-byte LDS read per plane and converts nothing.  The writer converts each value
// once.
// ------------------------------------------------------------------------------------

// Fragment planes of 4 consecutive k values (half of a unit): 8 bytes per plane (MODE 2:
// fp16 hi / lo; MODE 3: bf16 hi / mid).  MODE 0 keeps fp32 (frag_put4 writes plane h).
template <int MODE>
__device__ __forceinline__ void frag4(const float4 &v, uint2 &p0, uint2 &p1) {
    if constexpr (MODE == 2) {
        const f2v x0 = {v.x, v.y}, x1 = {v.z, v.w};
        const h2v h0 = __builtin_convertvector(x0, h2v), h1 = __builtin_convertvector(x1, h2v);
        const h2v l0 = __builtin_convertvector((x0 - __builtin_convertvector(h0, f2v)) * 2048.0f, h2v);
        const h2v l1 = __builtin_convertvector((x1 - __builtin_convertvector(h1, f2v)) * 2048.0f, h2v);
        p0 = make_uint2(bitcast<uint32_t>(h0), bitcast<uint32_t>(h1));
        p1 = make_uint2(bitcast<uint32_t>(l0), bitcast<uint32_t>(l1));
    } else {
        Frag<MODE> f;
        make_frag<MODE>(f, v, v);
        p0 = make_uint2(f.p[0].x, f.p[0].y);
        p1 = make_uint2(f.p[1].x, f.p[1].y);
    }
}

// Store 4 values (k = 4 hh .. 4 hh + 3 of unit `unit`, fragment lane `fl`) of a two-plane
// fragment buffer.
template <int MODE>
__device__ __forceinline__ void frag_put4(uint4 *buf, int unit, int fl, int hh, const float4 &v) {
    static_assert(Npl<MODE>::v == 2, "two-plane modes");
    if constexpr (MODE == 0) {
        buf[(unit * 2 + hh) * 64 + fl] = bitcast<uint4>(v);
    } else {
        uint2 p0, p1;
        frag4<MODE>(v, p0, p1);
        reinterpret_cast<uint2 *>(buf + (unit * 2 + 0) * 64 + fl)[hh] = p0;
        reinterpret_cast<uint2 *>(buf + (unit * 2 + 1) * 64 + fl)[hh] = p1;
    }
}

// Store 8 values (a whole unit) of a two-plane fragment buffer.
template <int MODE>
__device__ __forceinline__ void frag_put8(uint4 *buf, int unit, int fl, const float4 &u, const float4 &v) {
    static_assert(Npl<MODE>::v == 2, "two-plane modes");
    Frag<MODE> f;
    make_frag<MODE>(f, u, v);
    buf[(unit * 2 + 0) * 64 + fl] = f.p[0];
    buf[(unit * 2 + 1) * 64 + fl] = f.p[1];
}

// Pre-split rows (two-plane modes): the 32 fragment units of a 128-column row kept inside
// 128 floats of the row itself, unit (k-block kb, plane pl, half h) at float offset
// ((kb * 2 + pl) * 2 + h) * 4 (h: which 8 columns of the 16-column k-block), so a pass
// that owns a row can convert its values into a free half of that row with no barrier.
// Store 4 values, columns col .. col+3 (col % 4 == 0), of such a row.
template <int MODE>
__device__ __forceinline__ void rowfrag_put4(float *row, int col, const float4 &v) {
    static_assert(Npl<MODE>::v == 2, "two-plane modes");
    const int kb = col >> 4, h = (col >> 3) & 1, hh = (col >> 2) & 1;
    if constexpr (MODE == 0) {  // the planes are the unit's two fp32 halves
        *reinterpret_cast<float4 *>(row + ((kb * 2 + hh) * 2 + h) * 4) = v;
    } else {
        uint2 p0, p1;
        frag4<MODE>(v, p0, p1);
        reinterpret_cast<uint2 *>(row + ((kb * 2 + 0) * 2 + h) * 4)[hh] = p0;
        reinterpret_cast<uint2 *>(row + ((kb * 2 + 1) * 2 + h) * 4)[hh] = p1;
    }
}

// Where a GEMM reads its pre-split A fragments from: a fragment buffer
// [rt][kb][plane][64 lanes] x 16 bytes with aKB k-blocks per row tile ...
struct AFragBuf {
    const uint4 *buf;
    int aKB;
    template <int MODE, int NRT>
    __device__ __forceinline__ void get(Frag<MODE> (&a)[NRT], int kb, int lane) const {
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
            for (int pl = 0; pl < 2; ++pl) a[rt].p[pl] = buf[((rt * aKB + kb) * 2 + pl) * 64 + lane];
    }
};
// ... or pre-split rows (rowfrag_put4) of row stride ld: lane l reads row rt*32 + l%32.
struct AFragRows {
    const float *base;
    int ld;
    template <int MODE, int NRT>
    __device__ __forceinline__ void get(Frag<MODE> (&a)[NRT], int kb, int lane) const {
        const int h = lane >> 5, l32 = lane & 31;
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
            const float *r = base + (rt * 32 + l32) * ld;
#pragma unroll
            for (int pl = 0; pl < 2; ++pl) a[rt].p[pl] = *reinterpret_cast<const uint4 *>(r + ((kb * 2 + pl) * 2 + h) * 4);
        }
    }
};

// One k-block of gemm_frag_packed: prefetch k-block `kpf` of B into BPF, then accumulate
// k-block `kb` (A fragments from the pre-split buffer, B = BCUR).
template <int MODE, int NRT, int NCT, bool TRANS, class ASRC>
__device__ __forceinline__ void gemm_frag_step(v16f (&acc)[NRT][NCT], const ASRC &asrc, int akb,
                                               const uint4 *__restrict__ W, int nt0, int KBW, int kpf,
                                               Frag<MODE> (&BCUR)[NCT], Frag<MODE> (&BPF)[NCT], int lane) {
    load_bfrags<MODE, NCT>(BPF, W, nt0, KBW, kpf, lane);
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of this step's MFMAs
    Frag<MODE> a[NRT];
    asrc.template get<MODE, NRT>(a, akb, lane);
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) prep_w<MODE>(BCUR[ct]);
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
            if constexpr (TRANS)
                mma_wx<MODE>(acc[rt][ct], BCUR[ct], a[rt]);
            else
                mma_xw<MODE>(acc[rt][ct], a[rt], BCUR[ct]);
        }
}

// gemm_lds_packed with a pre-split A (two-plane modes): k-blocks akb0 .. akb0+KBA-1 of the
// fragments asrc holds (AFragBuf, AFragRows); same B prefetch rings (RING: the ring of four
// for one output tile as well, where the caller has the registers for it).
template <int MODE, int NRT, int NCT, int KBA, bool TRANS = false, bool RING = (NCT == 2), class ASRC>
__device__ __forceinline__ void gemm_frag_src(v16f (&acc)[NRT][NCT], const ASRC &asrc, int akb0,
                                              const uint4 *__restrict__ W, int nt0, int KBW, int kb0, int lane) {
    static_assert(Npl<MODE>::v == 2, "two-plane modes");
    if constexpr (RING) {
        static_assert(KBA % 4 == 0, "ring of four");
        Frag<MODE> b0[NCT], b1[NCT], b2[NCT], b3[NCT];
        load_bfrags<MODE, NCT>(b0, W, nt0, KBW, kb0, lane);
        load_bfrags<MODE, NCT>(b1, W, nt0, KBW, kb0 + 1, lane);
        load_bfrags<MODE, NCT>(b2, W, nt0, KBW, kb0 + 2, lane);
#pragma unroll 1
        for (int kb = 0; kb < KBA; kb += 4) {
            gemm_frag_step<MODE, NRT, NCT, TRANS>(acc, asrc, akb0 + kb, W, nt0, KBW, kb0 + min(kb + 3, KBA - 1),
                                                  b0, b3, lane);
            gemm_frag_step<MODE, NRT, NCT, TRANS>(acc, asrc, akb0 + kb + 1, W, nt0, KBW,
                                                  kb0 + min(kb + 4, KBA - 1), b1, b0, lane);
            gemm_frag_step<MODE, NRT, NCT, TRANS>(acc, asrc, akb0 + kb + 2, W, nt0, KBW,
                                                  kb0 + min(kb + 5, KBA - 1), b2, b1, lane);
            gemm_frag_step<MODE, NRT, NCT, TRANS>(acc, asrc, akb0 + kb + 3, W, nt0, KBW,
                                                  kb0 + min(kb + 6, KBA - 1), b3, b2, lane);
        }
    } else {
        Frag<MODE> cur[NCT], nxt[NCT];
        load_bfrags<MODE, NCT>(cur, W, nt0, KBW, kb0, lane);
#pragma unroll 2
        for (int kb = 0; kb < KBA; ++kb) {
            gemm_frag_step<MODE, NRT, NCT, TRANS>(acc, asrc, akb0 + kb, W, nt0, KBW, kb0 + min(kb + 1, KBA - 1),
                                                  cur, nxt, lane);
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) cur[ct] = nxt[ct];
        }
    }
}

// gemm_frag_src from a fragment buffer holding aKB k-blocks per row tile.
template <int MODE, int NRT, int NCT, int KBA, bool TRANS = false, bool RING = (NCT == 2)>
__device__ __forceinline__ void gemm_frag_packed(v16f (&acc)[NRT][NCT], const uint4 *abuf, int aKB, int akb0,
                                                 const uint4 *__restrict__ W, int nt0, int KBW, int kb0, int lane) {
    gemm_frag_src<MODE, NRT, NCT, KBA, TRANS, RING>(acc, AFragBuf{abuf, aKB}, akb0, W, nt0, KBW, kb0, lane);
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

// Write a wave's accumulators (rows row0 + rt*32 + .., columns col0 + ct*32 + lane%32),
// plus an optional per-column bias, into an fp32 LDS tile of row stride ld.
template <int NRT, int NCT>
__device__ __forceinline__ void acc_to_lds_rc(const v16f (&acc)[NRT][NCT], float *tile, int ld, int row0, int col0,
                                              int lane, const float *__restrict__ bias = nullptr) {
    const int h = lane >> 5, l32 = lane & 31;
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
        const int col = col0 + ct * 32 + l32;
        const float b = bias ? bias[col] : 0.f;
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
            for (int i = 0; i < 16; ++i) tile[(row0 + rt * 32 + acc_row(i, h)) * ld + col] = acc[rt][ct][i] + b;
    }
}

// Transposed accumulators (rows in lanes, see gemm_lds_packed<..., TRANS>) plus an optional
// per-column bias into a row-major fp32 LDS tile: row rt*32 + lane%32, columns col0 + ct*32 + 8j + 4h
// .. +3 as one 16-byte write each.
template <int NRT, int NCT>
__device__ __forceinline__ void acc_t_to_lds(const v16f (&acc)[NRT][NCT], float *tile, int ld, int col0, int lane,
                                             const float *__restrict__ bias = nullptr) {
    const int h = lane >> 5, l32 = lane & 31;
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = col0 + ct * 32 + 8 * j + 4 * h;
            const float4 b = bias ? *reinterpret_cast<const float4 *>(bias + col) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt)
                *reinterpret_cast<float4 *>(tile + (rt * 32 + l32) * ld + col) =
                    make_float4(acc[rt][ct][4 * j] + b.x, acc[rt][ct][4 * j + 1] + b.y, acc[rt][ct][4 * j + 2] + b.z,
                                acc[rt][ct][4 * j + 3] + b.w);
        }
}

// The 64-row form used by the 4-waves-by-columns kernels.
template <int NCT>
__device__ __forceinline__ void acc_to_lds(const v16f (&acc)[2][NCT], float *tile, int ld, int col0, int lane,
                                           const float *__restrict__ bias = nullptr) {
    acc_to_lds_rc<2, NCT>(acc, tile, ld, 0, col0, lane, bias);
}

// MFMA arithmetic modes the GEMM kernels are built for.
static inline bool matris_mode_ok(int mode) { return mode == 0 || mode == 2 || mode == 3 || mode == 6; }

// ------------------------------------------------------------------------------------
// 64-row tiles of [*, 128] rows staged by 512 threads (two-plane modes)
// ------------------------------------------------------------------------------------
// Rows of a [*, 128] array for tile rows m0 .. m0+63, 512 threads: thread (row tid/8,
// 8-column groups q and q+8 for q = tid%8); rows past M read row M-1.
__device__ __forceinline__ void load_rows4(float4 (&xr)[4], const float *__restrict__ x, int64_t m0, int64_t M,
                                           int tid) {
    const int64_t row = min(m0 + (tid >> 3), M - 1);
    const float4 *p = reinterpret_cast<const float4 *>(x + row * MATRIS_D) + (tid & 7) * 2;
    xr[0] = p[0];
    xr[1] = p[1];
    xr[2] = p[16];
    xr[3] = p[17];
}

// Stage those rows as fragment planes: group g of row r is fragment unit (r/32) * 8 + g/2,
// lane r%32 + 32 (g%2).
template <int MODE>
__device__ __forceinline__ float stage_rows4(uint4 *buf, const float4 (&xr)[4], int tid, float amax) {
    const int r = tid >> 3, q = tid & 7;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int g = q + 8 * i;
        const int unit = (r >> 5) * 8 + (g >> 1), fl = (r & 31) + 32 * (g & 1);
        amax = frag_amax<MODE>(amax, xr[2 * i], xr[2 * i + 1]);
        Frag<MODE> f;
        make_frag<MODE>(f, xr[2 * i], xr[2 * i + 1]);
        buf[(unit * 2 + 0) * 64 + fl] = f.p[0];
        buf[(unit * 2 + 1) * 64 + fl] = f.p[1];
    }
    return amax;
}

// MODE 2: scale the thread's share of its row (load_rows4 layout: 8 threads per row) by the
// row's 2^k (row_scale) and record 2^-k in rinv[row].
template <int MODE>
__device__ __forceinline__ void scale_rows4(float4 (&xr)[4], float *rinv, int tid) {
    if constexpr (MODE == 2) {
        const float m = abs_max4(abs_max4(abs_max4(abs_max4(0.f, xr[0]), xr[1]), xr[2]), xr[3]);
        const RowScale rs = row_scale(group8_max(m));
#pragma unroll
        for (int i = 0; i < 4; ++i) xr[i] = mul4(xr[i], rs.s);
        if ((tid & 7) == 0) rinv[tid >> 3] = rs.inv;
    }
}

// Launch KERNEL<mode> (mode already checked by matris_mode_ok).
#define MATRIS_MODE_DISPATCH(KERNEL, GRID, STREAM, ...)                                     \
    do {                                                                                    \
        if (mode == 0) KERNEL<0><<<(GRID), 256, 0, (STREAM)>>>(__VA_ARGS__);                \
        else if (mode == 2) KERNEL<2><<<(GRID), 256, 0, (STREAM)>>>(__VA_ARGS__);           \
        else if (mode == 3) KERNEL<3><<<(GRID), 256, 0, (STREAM)>>>(__VA_ARGS__);           \
        else KERNEL<6><<<(GRID), 256, 0, (STREAM)>>>(__VA_ARGS__);                          \
    } while (0)


// Bytes of a packed [n, k] weight in `mode` (n % 32 == 0, k % 16 == 0).
__host__ __device__ inline size_t packed_b_bytes(int64_t n, int64_t k, int mode) {
    return (size_t)n * (size_t)k * (mode == 6 ? 6 : 4) + (mode == 2 ? 16 : 0);
}
