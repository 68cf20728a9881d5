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
// chunk suffices and no wave converts X values itself; the pre-packed W1 fragments come
// straight from global (L2) one k-block ahead.  Each wave owns 64 output columns (2x2
// tiles of 32x32) and both GEMMs run transposed (P^T = W1 X^T, Z^T = W2 H^T: the weight
// fragment is the MFMA A operand), so every lane holds whole-row segments: lane
// (row l % 32 of a row tile, half l / 32) has columns 32 ct + 8 j + 4 (l / 32) .. +3.
// p and z go to an LDS tile with 16-byte writes.  One pass copies p out with 16-byte row
// stores and turns it into h = SiLU(p), GEMM2's operand; a row pass with 16 lanes per
// row saves z, applies the two RMSNorms (16-lane DPP sums), SiLU, sigmoid and their
// product, and writes out with 512-byte row stores.  p and z are written for the
// backward, with streaming stores.
//
// Backward (input gradients only) recomputes the norm/activation Jacobians row-wise
// from z, then runs g_h = g_z W2 and g_x = (g_h * SiLU'(p)) W1 through the same MFMA
// tiling, with packed transposed weights.  In the two-plane modes it runs with eight
// waves per 64-row tile (gmlp_bwd8_kernel: 32 columns per wave, 128 registers, so a CU
// holds 16 waves); MODE 6 keeps four (gmlp_bwd_kernel).  In the two-plane modes g_z and g_p are stored
// in LDS already split into fragment units by the pass that produces them, so neither
// GEMM converts anything (g_p is otherwise re-split by every wave of every column pass).
//
// This file also owns the device status word: MODE 2 (fp16 split) kernels of every GEMM
// file set bit 0 when an activation exceeds the fp16 range, deferred CSR builds set bit 1
// on a key outside its segment range; matris_status_take reads and clears it.
#include "mma.h"

// Bits set by kernels of this library (MATRIS_STATUS_*); one copy per device.
static __device__ unsigned matris_status_word;

unsigned *matris_range_flag() {
    static unsigned *ptr[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    if (!ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(matris_status_word)) != hipSuccess) return nullptr;
        ptr[dev] = (unsigned *)p;
    }
    return ptr[dev];
}

__global__ void range_reset_kernel(unsigned *flag) { flag[0] = 0u; }

struct GmlpSrc {
    const float *ptr[4];
    const int32_t *idx[4];
};

// Projected sources (gather after GEMM): row r of the GEMM1 output gains
// ptr[j][idx[j][r] * ld[j] + c] for c < 256, rows already multiplied by their block of W1.
struct GmlpProj {
    const float *ptr[3];
    const int32_t *idx[3];
    int64_t ld[3];
    int n;
};

// A tail on the output rows (a Refinement's edge_FFN, interaction_block.py:269-275):
//   t = W1 out (saved to save_p when given),  ffn_out = W2 SiLU(t) (+ res_w * res if res)
// with W1, W2 packs of the FFN's [128, 128] Linear weights.
struct FfnTail {
    const uint4 *W1, *W2;
    float *save_p, *out;
    const float *res, *res_w;
};

// A projection pair on the residual source's rows (the line graph attention's logits,
// interaction_block.py:104-112: W_s and W_t applied to the same angle rows as the edge
// update's residual): o0 = res W[0:128]^T, o1 = res W[128:256]^T, W the pack that
// matris_pair_fwd takes.  The residual rows are already in registers for res_out.
struct PairOut {
    const uint4 *W;
    float *o0, *o1;
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

template <int MODE, bool TAIL = false, bool PTAIL = false>
__global__ __launch_bounds__(256, 2) void gmlp_fwd_kernel(int64_t M, int nsrc, GmlpSrc src, GmlpProj proj,
                                                          const uint4 *__restrict__ W1, const float *__restrict__ b1,
                                                          const uint4 *__restrict__ W2, const float *__restrict__ b2,
                                                          const float *__restrict__ norm_c,
                                                          const float *__restrict__ norm_g, float eps,
                                                          float *__restrict__ out, float *__restrict__ save_p,
                                                          float *__restrict__ save_z,
                                                          const float *__restrict__ res_src,
                                                          const float *__restrict__ res_w,
                                                          float *__restrict__ res_out, FfnTail tail,
                                                          PairOut pout, unsigned *range_flag) {
    constexpr int NPL = Npl<MODE>::v;
    constexpr int CHUNK = 2 * 2 * NPL * 64;  // uint4 per LDS chunk: [rt 2][kb 2][plane][lane]
    constexpr bool PRE = NPL == 2;           // the tails' GEMM operands as pre-split rows
    __shared__ __align__(16) float smem[BM * LDH];
    uint4 *Xp = reinterpret_cast<uint4 *>(smem);  // two chunk buffers (<= 24 KB)
    float *Ts = smem;                             // [BM, 256] tile: p, then h, then z
    // Per-column vectors b1 [256], b2 [256], norm_c [128], norm_g [128], res_w [128] in LDS:
    // read there, they never wait behind this work-group's global stores (a load from
    // global memory waits for every earlier store of its wave).  Loaded into registers at
    // kernel start, written to LDS once the projected-row gather is in flight.
    __shared__ __align__(16) float cvec[896];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    float cv[4];  // cvec entries tid, tid + 256, tid + 512 and (tid < 128) tid + 768
    cv[0] = b1 ? b1[tid] : 0.f;
    cv[1] = b2 ? b2[tid] : 0.f;
    cv[2] = tid < 128 ? norm_c[tid] : norm_g[tid - 128];
    cv[3] = (tid < 128 && res_w) ? res_w[tid] : 0.f;
    const int64_t m0 = (int64_t)blockIdx.x * BM;
    const int KB = nsrc * (MATRIS_D / 16);  // k-blocks of W1 (none without gathered sources)
    // MODE 2: the accumulator holds s * (W1 x) until scale_acc multiplies by 1/s
    const float w1up = (MODE == 2 && nsrc > 0) ? reinterpret_cast<const float *>(W1)[1] : 1.0f;
    const float w1s = nsrc > 0 ? take_wscale<MODE>(W1) : 1.0f, w2s = take_wscale<MODE>(W2);
    float amax = 0.f;
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

    // Prefetch depth: two register sets of gathered X (A, B) -- chunk c+1 is converted
    // from one set while chunk c+3 loads into it -- and the weight fragments in a ring of
    // four, three k-blocks ahead; the loop body covers two chunks so that every ring slot
    // is a fixed register set.
    float4 xa0, xa1, xb0, xb1;
#define GMLP_LOADX(kc, r0, r1)                                                                           \
    do {                                                                                                 \
        const int j_ = (kc) >> 7, cc_ = (kc) & 127;                                                      \
        const float *sp_ = j_ == 0 ? src.ptr[0] + sr0 * MATRIS_D                                         \
                         : j_ == 1 ? src.ptr[1] + sr1 * MATRIS_D                                         \
                         : j_ == 2 ? src.ptr[2] + sr2 * MATRIS_D                                         \
                                   : src.ptr[3] + sr3 * MATRIS_D;                                        \
        const float4 *xp_ = reinterpret_cast<const float4 *>(sp_ + cc_ + xc);                            \
        r0 = xp_[0];                                                                                     \
        r1 = xp_[1];                                                                                     \
    } while (0)
#define GMLP_STOREX(buf, r0, r1)                                                                         \
    do {                                                                                                 \
        Frag<MODE> f_;                                                                                   \
        amax = frag_amax<MODE>(amax, r0, r1);                                                            \
        make_frag<MODE>(f_, r0, r1);                                                                     \
        _Pragma("unroll") for (int pl_ = 0; pl_ < NPL; ++pl_) Xp[(buf) * CHUNK + xslot + pl_ * 64] = f_.p[pl_]; \
    } while (0)
#define GMLP_SUB(kb, sub, xb, BCUR, BPF)                                                                 \
    do {                                                                                                 \
        load_bfrags<MODE, 2>(BPF, W1, 2 * wave, KB, min((kb) + BDIST, KB - 1), lane);                    \
        __builtin_amdgcn_sched_barrier(0);                                                               \
        Frag<MODE> a[2];                                                                                 \
        _Pragma("unroll") for (int rt = 0; rt < 2; ++rt)                                                 \
            _Pragma("unroll") for (int pl = 0; pl < NPL; ++pl)                                           \
                a[rt].p[pl] = xb[((rt * 2 + (sub)) * NPL + pl) * 64 + lane];                             \
        prep_w<MODE>(BCUR[0]);                                                                           \
        prep_w<MODE>(BCUR[1]);                                                                           \
        _Pragma("unroll") for (int rt = 0; rt < 2; ++rt)                                                 \
            _Pragma("unroll") for (int ct = 0; ct < 2; ++ct) mma_wx<MODE>(acc[rt][ct], BCUR[ct], a[rt]); \
    } while (0)
#define GMLP_CHUNK(c, r0, r1, BS0, BS1, BP0, BP1)                                                        \
    do {                                                                                                 \
        const uint4 *xb = Xp + ((c) & 1) * CHUNK;                                                        \
        GMLP_SUB(2 * (c), 0, xb, BS0, BP0);                                                              \
        GMLP_SUB(2 * (c) + 1, 1, xb, BS1, BP1);                                                          \
        GMLP_STOREX(((c) + 1) & 1, r0, r1); /* chunk c+1; unread after the last chunk */                 \
        GMLP_LOADX(min((c) + 3, nchunk - 1) * 32, r0, r1);                                               \
        __syncthreads();                                                                                 \
    } while (0)

    // GEMM1's first three chunks are requested before the projected-row gather below, so
    // their latency overlaps it
    float4 x00, x01;
    if (nsrc > 0) {
        GMLP_LOADX(0, x00, x01);
        GMLP_LOADX(min(1, nchunk - 1) * 32, xa0, xa1);
        GMLP_LOADX(min(2, nchunk - 1) * 32, xb0, xb1);
    }
    v16f acc[2][2];
    zero_acc(acc);
    // Projected rows go straight into the accumulator (layout of acc_t_to_lds: row
    // rt*32 + lane%32, columns 64 wave + 32 ct + 8 j + 4 (lane/32) .. +3).  Issued before
    // GEMM1's first loads, they arrive while the pipeline fills.
    if (proj.n > 0) {
        const int h = lane >> 5, l32 = lane & 31;
        // every table's row of a 32-row tile is loaded before any is added: one round
        // trip per row tile instead of one per table
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const int64_t r = min(m0 + rt * 32 + l32, M - 1);
            float4 v[3][2][4];
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                if (j < proj.n) {
                    const int64_t pr = proj.idx[j] ? (int64_t)proj.idx[j][r] : r;
                    const float *pp = proj.ptr[j] + pr * proj.ld[j] + wave * 64 + 4 * h;
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                        for (int jj = 0; jj < 4; ++jj) v[j][ct][jj] = *reinterpret_cast<const float4 *>(pp + ct * 32 + 8 * jj);
                }
            }
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                if (j < proj.n) {
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                        for (int jj = 0; jj < 4; ++jj) {
                            acc[rt][ct][4 * jj] += v[j][ct][jj].x;
                            acc[rt][ct][4 * jj + 1] += v[j][ct][jj].y;
                            acc[rt][ct][4 * jj + 2] += v[j][ct][jj].z;
                            acc[rt][ct][4 * jj + 3] += v[j][ct][jj].w;
                        }
                }
            }
        }
        if (MODE == 2 && nsrc > 0) scale_acc<MODE>(acc, w1up);  // power of two: exact
    }
    cvec[tid] = cv[0];
    cvec[256 + tid] = cv[1];
    cvec[512 + tid] = cv[2];
    if (tid < 128) cvec[768 + tid] = cv[3];
    if (nsrc > 0) {
        constexpr int BDIST = 3;
        Frag<MODE> bq0[2], bq1[2], bq2[2], bq3[2];
        load_bfrags<MODE, 2>(bq0, W1, 2 * wave, KB, 0, lane);
        load_bfrags<MODE, 2>(bq1, W1, 2 * wave, KB, min(1, KB - 1), lane);
        load_bfrags<MODE, 2>(bq2, W1, 2 * wave, KB, min(2, KB - 1), lane);
        GMLP_STOREX(0, x00, x01);
        __syncthreads();
#pragma unroll 1
        for (int c = 0; c < nchunk; c += 2) {  // nchunk = 4 nsrc is even
            GMLP_CHUNK(c, xa0, xa1, bq0, bq1, bq3, bq0);
            GMLP_CHUNK(c + 1, xb0, xb1, bq2, bq3, bq1, bq2);
        }
    }
#undef GMLP_CHUNK
#undef GMLP_SUB
#undef GMLP_LOADX
#undef GMLP_STOREX

    // p = acc + b1 -> LDS (rows in lanes: 16-byte writes); one pass copies p out with
    // 16-byte row stores and turns it into h = SiLU(p) in place.  (Pre-splitting h into
    // fragment units here, as the backward does for g_z / g_p, measured slower: it costs
    // a barrier and 24 more VGPRs for a conversion that two waves share.)
    scale_acc<MODE>(acc, w1s);
    if (nsrc == 0) __syncthreads();  // cvec written (GEMM1's barriers cover it otherwise)
    acc_t_to_lds<2, 2>(acc, Ts, LDH, wave * 64, lane, cvec);
    __syncthreads();
#pragma unroll
    for (int it = 0; it < (BM * 64) / 256; ++it) {
        const int q = it * 256 + tid;
        const int row = q >> 6, c4 = (q & 63) * 4;
        float4 *t = reinterpret_cast<float4 *>(Ts + row * LDH + c4);
        float4 v = *t;
        // p and z are read again only by the backward: streaming (non-temporal) stores
        if (save_p && m0 + row < M) st_nt4(save_p + (m0 + row) * 256 + c4, v);
        v.x = silu_f(v.x); v.y = silu_f(v.y); v.z = silu_f(v.z); v.w = silu_f(v.w);
        *t = v;
    }
    __syncthreads();

    // GEMM2, transposed: wave w -> z columns [64w, 64w+64) of both row tiles, rows in lanes;
    // block = w/2 (0 core, 1 gate)
    const int blk = wave >> 1;
    zero_acc(acc);
    amax = fmaxf(amax, gemm_lds_packed<MODE, 2, 2, MATRIS_D / 16, true>(acc, Ts + blk * MATRIS_D, LDH, W2, 2 * wave,
                                                                        MATRIS_D / 16, 0, lane));
    scale_acc<MODE>(acc, w2s);
    // the residual rows of the row pass below, loaded before its z and out stores so
    // that waiting for them does not wait for those stores too
    const int c4 = (lane & 15) * 4;
    float4 rx0[BM / 16], rx1[BM / 16];
    if (res_out) {
#pragma unroll
        for (int rr = 0; rr < BM / 16; ++rr) {
            const int64_t grow = min(m0 + wave * (BM / 4) + rr * 4 + (lane >> 4), M - 1);
            rx0[rr] = *reinterpret_cast<const float4 *>(res_src + grow * MATRIS_D + c4);
            rx1[rr] = *reinterpret_cast<const float4 *>(res_src + grow * MATRIS_D + 64 + c4);
        }
    }
    // the tail's residual rows (layout of its final row stores), loaded here for the same reason
    float4 tres[(BM * 32) / 256];
    if (TAIL && tail.res) {
#pragma unroll
        for (int it = 0; it < (BM * 32) / 256; ++it) {
            const int q = it * 256 + tid;
            const int64_t grow = min(m0 + (q >> 5), M - 1);
            tres[it] = *reinterpret_cast<const float4 *>(tail.res + grow * MATRIS_D + (q & 31) * 4);
        }
    }
    __syncthreads();  // every wave is done reading h

    // z = acc + b2 -> LDS (16-byte writes); then a row pass with 16 lanes per row: lane
    // c of a row holds core columns 4c .. 4c+3 and 64 + 4c .. +3 and the same gate
    // columns, so each store instruction writes 256 contiguous bytes of a row; each
    // RMSNorm sum is a 16-lane DPP sum
    acc_t_to_lds<2, 2>(acc, Ts, LDH, wave * 64, lane, cvec + 256);
    __syncthreads();
    const float4 wc0 = *reinterpret_cast<const float4 *>(cvec + 512 + c4);
    const float4 wc1 = *reinterpret_cast<const float4 *>(cvec + 512 + 64 + c4);
    const float4 wg0 = *reinterpret_cast<const float4 *>(cvec + 640 + c4);
    const float4 wg1 = *reinterpret_cast<const float4 *>(cvec + 640 + 64 + c4);
#pragma unroll
    for (int rr = 0; rr < BM / 16; ++rr) {
        const int row = wave * (BM / 4) + rr * 4 + (lane >> 4);
        const float *zr = Ts + row * LDH;
        const float4 zc0 = *reinterpret_cast<const float4 *>(zr + c4);
        const float4 zc1 = *reinterpret_cast<const float4 *>(zr + 64 + c4);
        const float4 zg0 = *reinterpret_cast<const float4 *>(zr + MATRIS_D + c4);
        const float4 zg1 = *reinterpret_cast<const float4 *>(zr + MATRIS_D + 64 + c4);
        const int64_t grow = m0 + row;
        if (save_z && grow < M) {
            float *zo = save_z + grow * 256 + c4;
            st_nt4(zo, zc0);
            st_nt4(zo + 64, zc1);
            st_nt4(zo + MATRIS_D, zg0);
            st_nt4(zo + MATRIS_D + 64, zg1);
        }
        const float rc = rsqrtf(row16_sum(zc0.x * zc0.x + zc0.y * zc0.y + zc0.z * zc0.z + zc0.w * zc0.w +
                                          zc1.x * zc1.x + zc1.y * zc1.y + zc1.z * zc1.z + zc1.w * zc1.w) *
                                    (1.0f / MATRIS_D) + eps);
        const float rg = rsqrtf(row16_sum(zg0.x * zg0.x + zg0.y * zg0.y + zg0.z * zg0.z + zg0.w * zg0.w +
                                          zg1.x * zg1.x + zg1.y * zg1.y + zg1.z * zg1.z + zg1.w * zg1.w) *
                                    (1.0f / MATRIS_D) + eps);
        float4 o0, o1;
        o0.x = silu_f(zc0.x * rc * wc0.x) * sigm_f(zg0.x * rg * wg0.x);
        o0.y = silu_f(zc0.y * rc * wc0.y) * sigm_f(zg0.y * rg * wg0.y);
        o0.z = silu_f(zc0.z * rc * wc0.z) * sigm_f(zg0.z * rg * wg0.z);
        o0.w = silu_f(zc0.w * rc * wc0.w) * sigm_f(zg0.w * rg * wg0.w);
        o1.x = silu_f(zc1.x * rc * wc1.x) * sigm_f(zg1.x * rg * wg1.x);
        o1.y = silu_f(zc1.y * rc * wc1.y) * sigm_f(zg1.y * rg * wg1.y);
        o1.z = silu_f(zc1.z * rc * wc1.z) * sigm_f(zg1.z * rg * wg1.z);
        o1.w = silu_f(zc1.w * rc * wc1.w) * sigm_f(zg1.w * rg * wg1.w);
        if (grow < M) {
            float *orow = out + grow * MATRIS_D + c4;
            *reinterpret_cast<float4 *>(orow) = o0;
            *reinterpret_cast<float4 *>(orow + 64) = o1;
            if (res_out) {
                const float4 w0 = *reinterpret_cast<const float4 *>(cvec + 768 + c4);
                const float4 w1 = *reinterpret_cast<const float4 *>(cvec + 768 + 64 + c4);
                const float4 x0 = rx0[rr], x1 = rx1[rr];
                float *ro = res_out + grow * MATRIS_D + c4;
                *reinterpret_cast<float4 *>(ro) = make_float4(o0.x + w0.x * x0.x, o0.y + w0.y * x0.y, o0.z + w0.z * x0.z,
                                                              o0.w + w0.w * x0.w);
                *reinterpret_cast<float4 *>(ro + 64) = make_float4(o1.x + w1.x * x1.x, o1.y + w1.y * x1.y,
                                                                   o1.z + w1.z * x1.z, o1.w + w1.w * x1.w);
            }
        }
        // The tail's GEMM operand (the out rows) or the pair's (the residual rows), written
        // over this row's z (already read).  Two-plane modes convert it once here, into the
        // row's gate half as pre-split units (rowfrag_put4): the tail GEMMs give each wave
        // one 32-column tile, so every wave would convert all 64 rows again.
        if constexpr (TAIL || PTAIL) {
            const float4 a0 = TAIL ? o0 : rx0[rr], a1 = TAIL ? o1 : rx1[rr];
            if constexpr (PRE) {
                amax = frag_amax<MODE>(amax, a0, a1);
                rowfrag_put4<MODE>(Ts + row * LDH + MATRIS_D, c4, a0);
                rowfrag_put4<MODE>(Ts + row * LDH + MATRIS_D, 64 + c4, a1);
            } else {
                *reinterpret_cast<float4 *>(Ts + row * LDH + c4) = a0;
                *reinterpret_cast<float4 *>(Ts + row * LDH + 64 + c4) = a1;
            }
        }
    }
    if constexpr (PTAIL) {
        // o0 = res W[0:128]^T, then o1 = res W[128:256]^T: each wave one 32-column tile of
        // the pass, through the half of the tile the GEMM does not read (it reads the
        // pre-split rows in columns 128..255, or fp32 rows in columns 0..127)
        const float ps = take_wscale<MODE>(pout.W);
        constexpr int OUTC = PRE ? 0 : MATRIS_D;
#pragma unroll 1
        for (int half = 0; half < 2; ++half) {
            v16f pa[2][1];
            zero_acc(pa);
            __syncthreads();  // residual rows complete; the previous pass's rows stored
            if constexpr (PRE)
                gemm_frag_src<MODE, 2, 1, MATRIS_D / 16, true>(pa, AFragRows{Ts + MATRIS_D, LDH}, 0, pout.W,
                                                               4 * half + wave, MATRIS_D / 16, 0, lane);
            else
                amax = fmaxf(amax, gemm_lds_packed<MODE, 2, 1, MATRIS_D / 16, true>(pa, Ts, LDH, pout.W,
                                                                                    4 * half + wave, MATRIS_D / 16, 0,
                                                                                    lane));
            scale_acc<MODE>(pa, ps);
            acc_t_to_lds<2, 1>(pa, Ts + OUTC, LDH, wave * 32, lane);
            __syncthreads();
            float *dst = half ? pout.o1 : pout.o0;
#pragma unroll
            for (int it = 0; it < (BM * 32) / 256; ++it) {
                const int q = it * 256 + tid;
                const int row = q >> 5, cc = (q & 31) * 4;
                if (m0 + row < M)
                    st_nt4(dst + (m0 + row) * MATRIS_D + cc,
                           *reinterpret_cast<const float4 *>(Ts + row * LDH + OUTC + cc));
            }
        }
    }
    if constexpr (TAIL) {
        // t = W1 out -> the half of the tile GEMM A does not read; one pass saves t and
        // applies SiLU (two-plane modes: writing SiLU(t) pre-split into columns 128..255,
        // which GEMM A has finished reading); W2 SiLU(t) -> columns 0..127; rows leave with
        // the residual.  Without pre-split rows: out in columns 0..127, t in 128..255.
        const uint4 *tw1 = tail.W1, *tw2 = tail.W2;
        const float t1s = take_wscale<MODE>(tw1), t2s = take_wscale<MODE>(tw2);
        constexpr int TC = PRE ? 0 : MATRIS_D;  // t's columns
        v16f ta[2][1];
        zero_acc(ta);
        __syncthreads();  // out rows complete
        if constexpr (PRE)
            gemm_frag_src<MODE, 2, 1, MATRIS_D / 16, true>(ta, AFragRows{Ts + MATRIS_D, LDH}, 0, tw1, wave,
                                                           MATRIS_D / 16, 0, lane);
        else
            amax = fmaxf(amax, gemm_lds_packed<MODE, 2, 1, MATRIS_D / 16, true>(ta, Ts, LDH, tw1, wave, MATRIS_D / 16,
                                                                                0, lane));
        scale_acc<MODE>(ta, t1s);
        acc_t_to_lds<2, 1>(ta, Ts + TC, LDH, wave * 32, lane);
        __syncthreads();
#pragma unroll
        for (int it = 0; it < (BM * 32) / 256; ++it) {
            const int q = it * 256 + tid;
            const int row = q >> 5, cc = (q & 31) * 4;
            float4 *t = reinterpret_cast<float4 *>(Ts + row * LDH + TC + cc);
            float4 v = *t;
            if (tail.save_p && m0 + row < M) st_nt4(tail.save_p + (m0 + row) * MATRIS_D + cc, v);
            v.x = silu_f(v.x); v.y = silu_f(v.y); v.z = silu_f(v.z); v.w = silu_f(v.w);
            if constexpr (PRE) {
                amax = frag_amax<MODE>(amax, v, v);
                rowfrag_put4<MODE>(Ts + row * LDH + MATRIS_D, cc, v);
            } else {
                *t = v;
            }
        }
        __syncthreads();
        zero_acc(ta);
        if constexpr (PRE)
            gemm_frag_src<MODE, 2, 1, MATRIS_D / 16, true>(ta, AFragRows{Ts + MATRIS_D, LDH}, 0, tw2, wave,
                                                           MATRIS_D / 16, 0, lane);
        else
            amax = fmaxf(amax, gemm_lds_packed<MODE, 2, 1, MATRIS_D / 16, true>(ta, Ts + MATRIS_D, LDH, tw2, wave,
                                                                                MATRIS_D / 16, 0, lane));
        scale_acc<MODE>(ta, t2s);
        // columns 0..127: GEMM B reads 128..255, and every wave is past the SiLU pass's
        // reads of t (barrier above)
        acc_t_to_lds<2, 1>(ta, Ts, LDH, wave * 32, lane);
        __syncthreads();
#pragma unroll
        for (int it = 0; it < (BM * 32) / 256; ++it) {
            const int q = it * 256 + tid;
            const int row = q >> 5, cc = (q & 31) * 4;
            if (m0 + row < M) {
                float4 v = *reinterpret_cast<const float4 *>(Ts + row * LDH + cc);
                if (tail.res) {
                    const float4 w = *reinterpret_cast<const float4 *>(tail.res_w + cc);
                    const float4 x = tres[it];
                    v.x += w.x * x.x; v.y += w.y * x.y; v.z += w.z * x.z; v.w += w.w * x.w;
                }
                st_nt4(tail.out + (m0 + row) * MATRIS_D + cc, v);  // read again only by the next block
            }
        }
    }
    report_range<MODE>(amax, range_flag);
}

// ------------------------------------------------------------------------------------
// backward
// ------------------------------------------------------------------------------------
// A head in front of the backward (the line refinement's edge_FFN backward, with the
// envelope term of the aggregate, interaction_block.py:243-275): the GatedMLP's output
// gradient is not read but computed per tile,
//   g_out = ((g W2) * SiLU'(p)) W1 + ge[t] * env[s]      (ge == NULL: no envelope term)
// with g, p [M,128] the FFN's output gradient and saved W1 x, W1t / W2t packs of W1^T /
// W2^T (as matris_ffn_bwd takes them), ge [*,128] = g_agg * env per bond.  With gidx, g is
// read through it and scaled: row r of the FFN's output gradient is gscale * g[gidx[r]]
// (the atom-graph Refinement: half the bond gradient of each directed copy).
struct FfnHead {
    const float *g, *p;
    const uint4 *W1t, *W2t;
    const float *ge, *env;
    const int32_t *t, *s;
    const int32_t *gidx;
    float gscale;
};

// A projection added to source 0's gradient before it leaves (the line graph attention's
// W_s / W_t backward, interaction_block.py:104-112: the attention logits are projections
// of the same angle rows as the edge update's source 0):
//   g_x0 += g0 W[0:128] + g1 W[128:256]
// with g0, g1 [M,128] and Wt the pack of W^T ([128, 256]) that matris_pair_bwd takes.
struct PairTail {
    const float *g0, *g1;
    const uint4 *Wt;
};
// Store a wave's [64, 32*NCT] accumulators to rows of dst (row stride ld) at column
// col + ct*32 + lane%32, rows below nrows only, with streaming stores (the gradient rows
// are read once, by the segment sums that follow).
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
                if (row < nrows) st_nt(dst + row * ld + col + ct * 32 + l32, acc[rt][ct][i]);
            }
}

// Tile-run sums instead of rows (rows ascending by key): for each run of equal keys among
// the tile's rows [s, e) -- `starts` has bit s set for every run start -- store the sum
// of the run's rows at row s (columns col + ct*32 + lane%32); other rows are not written.
// Each lane adds its rows in row order, then lane half 0 + half 1: deterministic.
template <int NCT>
__device__ __forceinline__ void store_acc_runs(const v16f (&acc)[2][NCT], float *__restrict__ dst, int ld, int col,
                                               uint64_t starts, int nrows, int lane) {
    const int h = lane >> 5, l32 = lane & 31;
    while (starts) {  // wave-uniform
        const int s = __builtin_ctzll(starts);
        starts &= starts - 1;
        const int e = starts ? __builtin_ctzll(starts) : nrows;
        // row of element (rt, i) = rt*32 + acc_row(i, 0) + 4h: compare the constant part
        // against the run's bounds shifted by 4h
        const int s4 = s - 4 * h, e4 = e - 4 * h;
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
            float t = 0.f;
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int r0 = rt * 32 + acc_row(i, 0);
                    t += (r0 >= s4 && r0 < e4) ? acc[rt][ct][i] : 0.f;
                }
            const float o = __shfl_xor(t, 32, 64);
            t = h ? o + t : t + o;
            if (h == 0) dst[(int64_t)s * ld + col + ct * 32 + l32] = t;
        }
    }
}

// MODE 2: multiply accumulator rows (layout of store_acc_rows: element i of lane half h is
// row rt*32 + 8 (i/4) + 4h + i%4) by their rows' factors, four rows per 16-byte LDS read.
template <int MODE, int NCT>
__device__ __forceinline__ void unscale_acc_rows(v16f (&a)[2][NCT], const float *rinv, int h) {
    if constexpr (MODE == 2) {
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 r = *reinterpret_cast<const float4 *>(rinv + rt * 32 + 8 * q + 4 * h);
#pragma unroll
                for (int ct = 0; ct < NCT; ++ct) {
                    a[rt][ct][4 * q] *= r.x;
                    a[rt][ct][4 * q + 1] *= r.y;
                    a[rt][ct][4 * q + 2] *= r.z;
                    a[rt][ct][4 * q + 3] *= r.w;
                }
            }
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
                                                          int acc0, const float *__restrict__ res_w,
                                                          const float *__restrict__ res_src,
                                                          const int32_t *__restrict__ run_key, int run_blk,
                                                          unsigned *range_flag) {
    __shared__ __align__(16) float G[BM * LDH];
    __shared__ __align__(16) float rinv[BM];  // MODE 2: 2^-k w1s for each row (g_z / g_p scaled by 2^k)
    // Two-plane modes keep g_z, then g_p, in G pre-split into fragment units
    // [rt 2][kb 16][plane 2][64 lanes] (64 KB, converted once by their writer); MODE 6
    // keeps fp32 rows and converts at each fragment read.
    constexpr bool PS = Npl<MODE>::v == 2;
    uint4 *Gf = reinterpret_cast<uint4 *>(G);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int h = lane >> 5, l32 = lane & 31;
    const int64_t m0 = (int64_t)blockIdx.x * BM;
    const float w1s = take_wscale<MODE>(W1t), w2s = take_wscale<MODE>(W2t);
    float amax = 0.f;
    // run_key: source block run_blk leaves as tile-run sums (store_acc_runs); each wave
    // reads the tile's 64 keys now, lane r holding row r's
    const int run_k = run_key ? run_key[min(m0 + lane, M - 1)] : 0;

    // phase 1: row-wise Jacobian of out = SiLU(RMS(z_c) w_c) * sigmoid(RMS(z_g) w_g).
    // 16 lanes per row (4 rows per wave per pass, wave w owns rows [16w, 16w+16)): lane c
    // of a row owns core and gate columns 4c .. 4c+3 and 64 + 4c .. +3, so each load
    // instruction reads 256 contiguous bytes of a row; the four row reductions are
    // 16-lane DPP sums.  Rows past M read zeros (g = 0).
    {
        const int c4 = (lane & 15) * 4;
        float wc[8], wg[8];
        {
            const float4 a0 = *reinterpret_cast<const float4 *>(norm_c + c4);
            const float4 a1 = *reinterpret_cast<const float4 *>(norm_c + 64 + c4);
            const float4 b0 = *reinterpret_cast<const float4 *>(norm_g + c4);
            const float4 b1 = *reinterpret_cast<const float4 *>(norm_g + 64 + c4);
            wc[0] = a0.x; wc[1] = a0.y; wc[2] = a0.z; wc[3] = a0.w; wc[4] = a1.x; wc[5] = a1.y; wc[6] = a1.z; wc[7] = a1.w;
            wg[0] = b0.x; wg[1] = b0.y; wg[2] = b0.z; wg[3] = b0.w; wg[4] = b1.x; wg[5] = b1.y; wg[6] = b1.z; wg[7] = b1.w;
        }
        // every row group's z / g_out loads are requested before any is used: unconditional
        // (rows past M read row M-1, then count as zeros) so that they all stay in flight
        float4 ld_z[BM / 16][4], ld_g[BM / 16][2];
#pragma unroll
        for (int rr = 0; rr < BM / 16; ++rr) {
            const int64_t m = min(m0 + wave * (BM / 4) + rr * 4 + (lane >> 4), M - 1);
            const float4 *zr = reinterpret_cast<const float4 *>(Z + m * 256 + c4);
            const float4 *gr = reinterpret_cast<const float4 *>(g_out + m * MATRIS_D + c4);
            ld_z[rr][0] = zr[0];
            ld_z[rr][1] = zr[16];
            ld_z[rr][2] = zr[MATRIS_D / 4];
            ld_z[rr][3] = zr[MATRIS_D / 4 + 16];
            ld_g[rr][0] = gr[0];
            ld_g[rr][1] = gr[16];
        }
#pragma unroll
        for (int rr = 0; rr < BM / 16; ++rr) {
            const int row = wave * (BM / 4) + rr * 4 + (lane >> 4);
            const int64_t m = m0 + row;
            float zc[8], zg[8], go[8];
            {
                const float4 z0 = ld_z[rr][0], z1 = ld_z[rr][1], y0 = ld_z[rr][2], y1 = ld_z[rr][3];
                const float4 g0 = ld_g[rr][0], g1 = ld_g[rr][1];
                zc[0] = z0.x; zc[1] = z0.y; zc[2] = z0.z; zc[3] = z0.w; zc[4] = z1.x; zc[5] = z1.y; zc[6] = z1.z; zc[7] = z1.w;
                zg[0] = y0.x; zg[1] = y0.y; zg[2] = y0.z; zg[3] = y0.w; zg[4] = y1.x; zg[5] = y1.y; zg[6] = y1.z; zg[7] = y1.w;
                go[0] = g0.x; go[1] = g0.y; go[2] = g0.z; go[3] = g0.w; go[4] = g1.x; go[5] = g1.y; go[6] = g1.z; go[7] = g1.w;
            }
            if (m >= M) {
#pragma unroll
                for (int e = 0; e < 8; ++e) zc[e] = zg[e] = go[e] = 0.f;
            }
            float sc2 = 0.f, sg2 = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                sc2 += zc[e] * zc[e];
                sg2 += zg[e] * zg[e];
            }
            const float rc = rsqrtf(row16_sum(sc2) * (1.0f / MATRIS_D) + eps);
            const float rg = rsqrtf(row16_sum(sg2) * (1.0f / MATRIS_D) + eps);
            float nc[8], ng[8], gnc[8], gng[8], dcs = 0.f, dgs = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                nc[e] = zc[e] * rc;
                ng[e] = zg[e] * rg;
                const float ac = nc[e] * wc[e], ag = ng[e] * wg[e];
                const float sc = sigm_f(ac), gate = sigm_f(ag);
                gnc[e] = go[e] * gate * (sc * (1.f + ac * (1.f - sc))) * wc[e];
                gng[e] = go[e] * (ac * sc) * (gate * (1.f - gate)) * wg[e];
                dcs += gnc[e] * nc[e];
                dgs += gng[e] * ng[e];
            }
            const float dc = row16_sum(dcs) * (1.0f / MATRIS_D), dg = row16_sum(dgs) * (1.0f / MATRIS_D);
            float4 vc[2], vg[2];
#pragma unroll
            for (int e4 = 0; e4 < 2; ++e4) {
                vc[e4] = make_float4((gnc[4 * e4] - nc[4 * e4] * dc) * rc, (gnc[4 * e4 + 1] - nc[4 * e4 + 1] * dc) * rc,
                                     (gnc[4 * e4 + 2] - nc[4 * e4 + 2] * dc) * rc,
                                     (gnc[4 * e4 + 3] - nc[4 * e4 + 3] * dc) * rc);
                vg[e4] = make_float4((gng[4 * e4] - ng[4 * e4] * dg) * rg, (gng[4 * e4 + 1] - ng[4 * e4 + 1] * dg) * rg,
                                     (gng[4 * e4 + 2] - ng[4 * e4 + 2] * dg) * rg,
                                     (gng[4 * e4 + 3] - ng[4 * e4 + 3] * dg) * rg);
            }
            if constexpr (MODE == 2) {  // the row's g_z (and later g_p) scaled by 2^k
                const float m = abs_max4(abs_max4(abs_max4(abs_max4(0.f, vc[0]), vc[1]), vg[0]), vg[1]);
                const RowScale rs = row_scale(row16_max(m));
#pragma unroll
                for (int e4 = 0; e4 < 2; ++e4) {
                    vc[e4] = mul4(vc[e4], rs.s);
                    vg[e4] = mul4(vg[e4], rs.s);
                }
                if ((lane & 15) == 0) rinv[row] = rs.inv * w1s;  // phase 3's weight scale folded in
            }
            if constexpr (PS) {
                // g_z columns c (= 4c' and 64 + 4c', core; + 128, gate) of this row: half
                // (c/4 % 2) of fragment unit (rt = row/32, kb = c/16), lane row%32 + 32 (c/8 % 2)
                amax = frag_amax<MODE>(frag_amax<MODE>(amax, vc[0], vc[1]), vg[0], vg[1]);
                const int rb = (row >> 5) * 16, fr = row & 31;
#pragma unroll
                for (int e4 = 0; e4 < 2; ++e4) {
                    const int c = c4 + 64 * e4;
                    const int fl = fr + 32 * ((c >> 3) & 1), hh = (c >> 2) & 1;
                    frag_put4<MODE>(Gf, rb + (c >> 4), fl, hh, vc[e4]);
                    frag_put4<MODE>(Gf, rb + 8 + (c >> 4), fl, hh, vg[e4]);
                }
            } else {
                float *gr = G + row * LDH + c4;
#pragma unroll
                for (int e4 = 0; e4 < 2; ++e4) {
                    *reinterpret_cast<float4 *>(gr + 64 * e4) = vc[e4];
                    *reinterpret_cast<float4 *>(gr + MATRIS_D + 64 * e4) = vg[e4];
                }
            }
        }
    }
    __syncthreads();

    // phase 2: g_h = g_z W2 (block diagonal); wave w -> columns [64w, 64w+64).  W2t is
    // packed from [W2c^T ; W2g^T] ([256, 128]), so output tile nt reads block nt / 4.
    // g_p = g_h * SiLU'(p); rows past M read row 0 of the tile (their results are unused).
    const int blk = wave >> 1;
    const int nrows = (int)min((int64_t)BM, M - m0);
    const float *__restrict__ Pt = P + m0 * 256;
    v16f acc[2][2];
    zero_acc(acc);
    if constexpr (PS) {
        // transposed (rows in lanes): lane (row rt*32 + l32, half h) holds columns
        // 64 wave + 32 ct + 8 j + 4 h .. +3, read from P as 16-byte runs and written back
        // as half fragment units of g_p
        gemm_frag_packed<MODE, 2, 2, MATRIS_D / 16, true>(acc, Gf, 16, blk * 8, W2t, 2 * wave, MATRIS_D / 16, 0,
                                                          lane);
        scale_acc<MODE>(acc, w2s);
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const int row = rt * 32 + l32;
            const float *pr = Pt + (row < nrows ? row : 0) * 256 + wave * 64 + 4 * h;
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float4 pv = *reinterpret_cast<const float4 *>(pr + ct * 32 + 8 * j);
                    acc[rt][ct][4 * j] *= dsilu_f(pv.x);
                    acc[rt][ct][4 * j + 1] *= dsilu_f(pv.y);
                    acc[rt][ct][4 * j + 2] *= dsilu_f(pv.z);
                    acc[rt][ct][4 * j + 3] *= dsilu_f(pv.w);
                }
        }
        __syncthreads();  // every wave is done reading g_z
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float4 v = make_float4(acc[rt][ct][4 * j], acc[rt][ct][4 * j + 1], acc[rt][ct][4 * j + 2],
                                                 acc[rt][ct][4 * j + 3]);
                    amax = frag_amax<MODE>(amax, v, v);
                    frag_put4<MODE>(Gf, rt * 16 + 4 * wave + 2 * ct + (j >> 1), l32 + 32 * (j & 1), h, v);
                }
    } else {
        amax = gemm_lds_packed<MODE, 2, 2, MATRIS_D / 16>(acc, G + blk * MATRIS_D, LDH, W2t, 2 * wave, MATRIS_D / 16,
                                                          0, lane);
        scale_acc<MODE>(acc, w2s);
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
    }
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
    // bit r: row r (< nrows) starts a run of equal keys within the tile (the shuffle runs
    // on every lane: a lane reading from one that skipped it would see no value)
    const int run_prev = __shfl(run_k, (lane + 63) & 63, 64);
    const uint64_t run_starts =
        run_key ? (uint64_t)__ballot(lane < nrows && (lane == 0 || run_k != run_prev)) : 0;
    const int run_c0 = run_blk * MATRIS_D;  // the reduced block's columns [run_c0, run_c0 + 128)
    float *__restrict__ gxr = g_x ? g_x + m0 * ldr : nullptr;
    const bool epi0 = g_x0 != nullptr || res_w != nullptr;
    if (K % 256) {
        const int cb = K - MATRIS_D;
        v16f a2[2][1];
        zero_acc(a2);
        const int col0 = cb + wave * 32;
        if constexpr (PS)
            gemm_frag_packed<MODE, 2, 1, 256 / 16>(a2, Gf, 16, 0, W1t, col0 / 32, 256 / 16, 0, lane);
        else
            amax = fmaxf(amax, gemm_lds_packed<MODE, 2, 1, 256 / 16>(a2, G, LDH, W1t, col0 / 32, 256 / 16, 0, lane));
        if constexpr (MODE == 2)
            unscale_acc_rows<MODE, 1>(a2, rinv, h);  // 2^-k w1s per row
        else
            scale_acc<MODE>(a2, w1s);
        if (run_key && col0 >= run_c0 && col0 < run_c0 + MATRIS_D)
            store_acc_runs<1>(a2, gxr, ldr, col0 - coff, run_starts, nrows, lane);
        else if (cb > 0 || !epi0)
            store_acc_rows<1>(a2, gxr, ldr, col0 - coff, nrows, lane);
        if (cb == 0 && epi0) {  // K == 128: every wave holds source-0 columns
            __syncthreads();
            acc_to_lds<1>(a2, G, LDH, col0, lane);
        }
    }
    for (int cb = (K / 256 - 1) * 256; cb >= 0; cb -= 256) {
        v16f a2[2][2];
        zero_acc(a2);
        const int col0 = cb + wave * 64;
        if constexpr (PS)
            gemm_frag_packed<MODE, 2, 2, 256 / 16>(a2, Gf, 16, 0, W1t, col0 / 32, 256 / 16, 0, lane);
        else
            amax = fmaxf(amax, gemm_lds_packed<MODE, 2, 2, 256 / 16>(a2, G, LDH, W1t, col0 / 32, 256 / 16, 0, lane));
        if constexpr (MODE == 2)
            unscale_acc_rows<MODE, 2>(a2, rinv, h);  // 2^-k w1s per row
        else
            scale_acc<MODE>(a2, w1s);
        if (run_key && col0 >= run_c0 && col0 < run_c0 + MATRIS_D)
            store_acc_runs<2>(a2, gxr, ldr, col0 - coff, run_starts, nrows, lane);
        else if (col0 >= MATRIS_D || !epi0)
            store_acc_rows<2>(a2, gxr, ldr, col0 - coff, nrows, lane);
        if (cb == 0 && epi0) {
            __syncthreads();  // all waves are done reading G
            if (col0 < MATRIS_D) acc_to_lds<2>(a2, G, LDH, col0, lane);
        }
    }
    if (epi0) {
        __syncthreads();
        float *__restrict__ gx0 = g_x0 ? g_x0 + m0 * MATRIS_D : gxr;
        const int ld0 = g_x0 ? MATRIS_D : ldr;
        const float *__restrict__ got = (res_src ? res_src : g_out) + m0 * MATRIS_D;
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
    report_range<MODE>(amax, range_flag);
}


// The backward with eight waves per 64-row tile (two-plane modes): the same three phases
// as gmlp_bwd_kernel with each wave owning 8 rows in phase 1 and one 32-column tile in
// phases 2 and 3 -- half the registers per wave, so a CU holds 16 waves instead of 8 at
// the same LDS per work-group.  Phase 3 runs 256-column passes from the top of K, source
// 0's block last (for K = 384 / 128 only waves 0-3 have columns in the last pass).
template <int MODE, bool HEAD = false, bool PAIR = false>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) void gmlp_bwd8_kernel(int64_t M, int K, const float *__restrict__ g_out,
                                                           const float *__restrict__ P, const float *__restrict__ Z,
                                                           const uint4 *__restrict__ W1t,
                                                           const uint4 *__restrict__ W2t,
                                                           const float *__restrict__ norm_c,
                                                           const float *__restrict__ norm_g, float eps,
                                                           float *__restrict__ g_x, float *__restrict__ g_x0,
                                                           int acc0, const float *__restrict__ res_w,
                                                           const float *__restrict__ res_src,
                                                           const int32_t *__restrict__ run_key, int run_blk,
                                                           FfnHead head, PairTail pair, unsigned *range_flag) {
    static_assert(Npl<MODE>::v == 2, "two-plane modes");
    __shared__ __align__(16) float G[BM * LDH];
    __shared__ __align__(16) float rinv[BM];
    uint4 *Gf = reinterpret_cast<uint4 *>(G);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int h = lane >> 5, l32 = lane & 31;
    const int64_t m0 = (int64_t)blockIdx.x * BM;
    const float w1s = take_wscale<MODE>(W1t), w2s = take_wscale<MODE>(W2t);
    float amax = 0.f;
    const int run_k = run_key ? run_key[min(m0 + lane, M - 1)] : 0;

    // phase 0 (head): the tile's g_out into G's first 32 KB as fp32 [64, 128].  g is staged
    // pre-split in G's first half, (g W2) * SiLU'(p) pre-split in its second half; wave w
    // computes the 32 x 32 tile (rows 32 (w / 4), columns 32 (w % 4)) of both products.
    float *gh = G;
    if constexpr (HEAD) {
        __shared__ float hinv[BM];  // MODE 2: 2^-k of each row's scaling of g
        const uint4 *hw1 = head.W1t, *hw2 = head.W2t;
        const float h1s = take_wscale<MODE>(hw1), h2s = take_wscale<MODE>(hw2);
        const int hrt = wave >> 2, hct = wave & 3;
        const int64_t hrow = min(m0 + hrt * 32 + l32, M - 1);
        float4 xr[4], pv[4];
        if (head.gidx) {  // load_rows4's layout, rows read through gidx and scaled
            const int64_t gr = head.gidx[min(m0 + (tid >> 3), M - 1)];
            const float4 *gp = reinterpret_cast<const float4 *>(head.g + gr * MATRIS_D) + (tid & 7) * 2;
            xr[0] = gp[0]; xr[1] = gp[1]; xr[2] = gp[16]; xr[3] = gp[17];
#pragma unroll
            for (int q = 0; q < 4; ++q) xr[q] = mul4(xr[q], head.gscale);
        } else {
            load_rows4(xr, head.g, m0, M, tid);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
            pv[j] = *reinterpret_cast<const float4 *>(head.p + hrow * MATRIS_D + hct * 32 + 8 * j + 4 * h);
        scale_rows4<MODE>(xr, hinv, tid);
        amax = stage_rows4<MODE>(Gf, xr, tid, amax);
        __syncthreads();
        v16f ha[1][1];
        zero_acc(ha);
        gemm_frag_packed<MODE, 1, 1, MATRIS_D / 16, true>(ha, Gf + hrt * (8 * 2 * 64), 8, 0, hw2, hct, 8, 0, lane);
        uint4 *Hf = Gf + 2 * 8 * 2 * 64;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 v = make_float4(ha[0][0][4 * j] * h2s * dsilu_f(pv[j].x), ha[0][0][4 * j + 1] * h2s * dsilu_f(pv[j].y),
                                         ha[0][0][4 * j + 2] * h2s * dsilu_f(pv[j].z),
                                         ha[0][0][4 * j + 3] * h2s * dsilu_f(pv[j].w));
            amax = frag_amax<MODE>(amax, v, v);
            frag_put4<MODE>(Hf, hrt * 8 + hct * 2 + (j >> 1), l32 + 32 * (j & 1), h, v);
        }
        __syncthreads();  // the second product's operand complete; every wave is past the first
        float4 ev[4];
        if (head.ge) {
            const int64_t tr = head.t[hrow], sr = head.s[hrow];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int col = hct * 32 + 8 * j + 4 * h;
                const float4 a = *reinterpret_cast<const float4 *>(head.ge + tr * MATRIS_D + col);
                const float4 b = *reinterpret_cast<const float4 *>(head.env + sr * MATRIS_D + col);
                ev[j] = make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
            }
        }
        zero_acc(ha);
        gemm_frag_packed<MODE, 1, 1, MATRIS_D / 16, true>(ha, Hf + hrt * (8 * 2 * 64), 8, 0, hw1, hct, 8, 0, lane);
        const float sc = MODE == 2 ? h1s * hinv[hrt * 32 + l32] : h1s;  // both powers of two
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float4 v = make_float4(ha[0][0][4 * j] * sc, ha[0][0][4 * j + 1] * sc, ha[0][0][4 * j + 2] * sc,
                                   ha[0][0][4 * j + 3] * sc);
            if (head.ge) {
                v.x += ev[j].x; v.y += ev[j].y; v.z += ev[j].z; v.w += ev[j].w;
            }
            *reinterpret_cast<float4 *>(gh + (hrt * 32 + l32) * MATRIS_D + hct * 32 + 8 * j + 4 * h) = v;
        }
        __syncthreads();
    }

    // phase 1: wave w owns rows [8w, 8w + 8), 16 lanes per row
    {
        const int c4 = (lane & 15) * 4;
        // HEAD: the wave's g_out rows, all read before any wave writes g_z over them
        float hg[2][8];
        if constexpr (HEAD) {
#pragma unroll
            for (int rr = 0; rr < 2; ++rr) {
                const float *gr = gh + (wave * (BM / 8) + rr * 4 + (lane >> 4)) * MATRIS_D + c4;
                const float4 g0 = *reinterpret_cast<const float4 *>(gr);
                const float4 g1 = *reinterpret_cast<const float4 *>(gr + 64);
                hg[rr][0] = g0.x; hg[rr][1] = g0.y; hg[rr][2] = g0.z; hg[rr][3] = g0.w;
                hg[rr][4] = g1.x; hg[rr][5] = g1.y; hg[rr][6] = g1.z; hg[rr][7] = g1.w;
            }
            __syncthreads();
        }
        float wc[8], wg[8];
        {
            const float4 a0 = *reinterpret_cast<const float4 *>(norm_c + c4);
            const float4 a1 = *reinterpret_cast<const float4 *>(norm_c + 64 + c4);
            const float4 b0 = *reinterpret_cast<const float4 *>(norm_g + c4);
            const float4 b1 = *reinterpret_cast<const float4 *>(norm_g + 64 + c4);
            wc[0] = a0.x; wc[1] = a0.y; wc[2] = a0.z; wc[3] = a0.w; wc[4] = a1.x; wc[5] = a1.y; wc[6] = a1.z; wc[7] = a1.w;
            wg[0] = b0.x; wg[1] = b0.y; wg[2] = b0.z; wg[3] = b0.w; wg[4] = b1.x; wg[5] = b1.y; wg[6] = b1.z; wg[7] = b1.w;
        }
#pragma unroll 1
        for (int rr = 0; rr < BM / 32; ++rr) {
            const int row = wave * (BM / 8) + rr * 4 + (lane >> 4);
            const int64_t m = m0 + row;
            float zc[8], zg[8], go[8];
            {
                const int64_t ml = min(m, M - 1);  // rows past M read row M-1, then count as zeros
                const float4 *zr = reinterpret_cast<const float4 *>(Z + ml * 256 + c4);
                const float4 z0 = zr[0], z1 = zr[16], y0 = zr[MATRIS_D / 4], y1 = zr[MATRIS_D / 4 + 16];
                zc[0] = z0.x; zc[1] = z0.y; zc[2] = z0.z; zc[3] = z0.w; zc[4] = z1.x; zc[5] = z1.y; zc[6] = z1.z; zc[7] = z1.w;
                zg[0] = y0.x; zg[1] = y0.y; zg[2] = y0.z; zg[3] = y0.w; zg[4] = y1.x; zg[5] = y1.y; zg[6] = y1.z; zg[7] = y1.w;
                if constexpr (HEAD) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) go[e] = rr ? hg[1][e] : hg[0][e];
                } else {
                    const float4 *gr = reinterpret_cast<const float4 *>(g_out + ml * MATRIS_D + c4);
                    const float4 g0 = gr[0], g1 = gr[16];
                    go[0] = g0.x; go[1] = g0.y; go[2] = g0.z; go[3] = g0.w; go[4] = g1.x; go[5] = g1.y; go[6] = g1.z; go[7] = g1.w;
                }
            }
            if (m >= M) {
#pragma unroll
                for (int e = 0; e < 8; ++e) zc[e] = zg[e] = go[e] = 0.f;
            }
            float sc2 = 0.f, sg2 = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                sc2 += zc[e] * zc[e];
                sg2 += zg[e] * zg[e];
            }
            const float rc = rsqrtf(row16_sum(sc2) * (1.0f / MATRIS_D) + eps);
            const float rg = rsqrtf(row16_sum(sg2) * (1.0f / MATRIS_D) + eps);
            float nc[8], ng[8], gnc[8], gng[8], dcs = 0.f, dgs = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                nc[e] = zc[e] * rc;
                ng[e] = zg[e] * rg;
                const float ac = nc[e] * wc[e], ag = ng[e] * wg[e];
                const float sc = sigm_f(ac), gate = sigm_f(ag);
                gnc[e] = go[e] * gate * (sc * (1.f + ac * (1.f - sc))) * wc[e];
                gng[e] = go[e] * (ac * sc) * (gate * (1.f - gate)) * wg[e];
                dcs += gnc[e] * nc[e];
                dgs += gng[e] * ng[e];
            }
            const float dc = row16_sum(dcs) * (1.0f / MATRIS_D), dg = row16_sum(dgs) * (1.0f / MATRIS_D);
            float4 vc[2], vg[2];
#pragma unroll
            for (int e4 = 0; e4 < 2; ++e4) {
                vc[e4] = make_float4((gnc[4 * e4] - nc[4 * e4] * dc) * rc, (gnc[4 * e4 + 1] - nc[4 * e4 + 1] * dc) * rc,
                                     (gnc[4 * e4 + 2] - nc[4 * e4 + 2] * dc) * rc,
                                     (gnc[4 * e4 + 3] - nc[4 * e4 + 3] * dc) * rc);
                vg[e4] = make_float4((gng[4 * e4] - ng[4 * e4] * dg) * rg, (gng[4 * e4 + 1] - ng[4 * e4 + 1] * dg) * rg,
                                     (gng[4 * e4 + 2] - ng[4 * e4 + 2] * dg) * rg,
                                     (gng[4 * e4 + 3] - ng[4 * e4 + 3] * dg) * rg);
            }
            if constexpr (MODE == 2) {
                const float mx = abs_max4(abs_max4(abs_max4(abs_max4(0.f, vc[0]), vc[1]), vg[0]), vg[1]);
                const RowScale rs = row_scale(row16_max(mx));
#pragma unroll
                for (int e4 = 0; e4 < 2; ++e4) {
                    vc[e4] = mul4(vc[e4], rs.s);
                    vg[e4] = mul4(vg[e4], rs.s);
                }
                if ((lane & 15) == 0) rinv[row] = rs.inv * w1s;
            }
            amax = frag_amax<MODE>(frag_amax<MODE>(amax, vc[0], vc[1]), vg[0], vg[1]);
            const int rb = (row >> 5) * 16, fr = row & 31;
#pragma unroll
            for (int e4 = 0; e4 < 2; ++e4) {
                const int c = c4 + 64 * e4;
                const int fl = fr + 32 * ((c >> 3) & 1), hh = (c >> 2) & 1;
                frag_put4<MODE>(Gf, rb + (c >> 4), fl, hh, vc[e4]);
                frag_put4<MODE>(Gf, rb + 8 + (c >> 4), fl, hh, vg[e4]);
            }
        }
    }
    __syncthreads();

    // phase 2: g_h = g_z W2, wave w -> columns [32w, 32w + 32) (block w / 4), then
    // g_p = g_h * SiLU'(p) written back pre-split.  (With the FFN head, phases 2 and 3
    // prefetch their weight fragments three k-blocks ahead instead of one: -4% for that
    // instance; the others lose or spill with the deeper ring.)
    const int blk = wave >> 2;
    const int nrows = (int)min((int64_t)BM, M - m0);
    const float *__restrict__ Pt = P + m0 * 256;
    {
        v16f acc[2][1];
        zero_acc(acc);
        gemm_frag_packed<MODE, 2, 1, MATRIS_D / 16, true, HEAD>(acc, Gf, 16, blk * 8, W2t, wave, MATRIS_D / 16, 0, lane);
        scale_acc<MODE>(acc, w2s);
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const int row = rt * 32 + l32;
            const float *pr = Pt + (row < nrows ? row : 0) * 256 + wave * 32 + 4 * h;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 pv = *reinterpret_cast<const float4 *>(pr + 8 * j);
                acc[rt][0][4 * j] *= dsilu_f(pv.x);
                acc[rt][0][4 * j + 1] *= dsilu_f(pv.y);
                acc[rt][0][4 * j + 2] *= dsilu_f(pv.z);
                acc[rt][0][4 * j + 3] *= dsilu_f(pv.w);
            }
        }
        __syncthreads();  // every wave is done reading g_z
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 v = make_float4(acc[rt][0][4 * j], acc[rt][0][4 * j + 1], acc[rt][0][4 * j + 2],
                                             acc[rt][0][4 * j + 3]);
                amax = frag_amax<MODE>(amax, v, v);
                frag_put4<MODE>(Gf, rt * 16 + 2 * wave + (j >> 1), l32 + 32 * (j & 1), h, v);
            }
    }
    __syncthreads();

    // phase 3: g_x = g_p W1 in 256-column passes from the top of K; the last pass holds
    // source 0 ([0, 128)), whose gradient goes through LDS when g_x0 or res_w is given
    const int coff = g_x0 ? MATRIS_D : 0;
    const int ldr = K - coff;
    float *__restrict__ gxr = g_x ? g_x + m0 * ldr : nullptr;
    const bool epi0 = g_x0 != nullptr || res_w != nullptr;
    const int run_prev = __shfl(run_k, (lane + 63) & 63, 64);
    const uint64_t run_starts =
        run_key ? (uint64_t)__ballot(lane < nrows && (lane == 0 || run_k != run_prev)) : 0;
    const int run_c0 = run_blk * MATRIS_D;
    int top = K;
    while (top > 0) {
        const bool last = top <= 256;
        const int base = last ? 0 : top - 256;
        const int col0 = base + 32 * wave;
        const bool active = col0 < top;
        // an opaque copy of the row stride: the store addresses below are computed in this
        // pass instead of being hoisted out of the loop (32 live 64-bit offsets would spill)
        int ldp = ldr;
        asm volatile("" : "+s"(ldp));
        v16f a2[2][1];
        zero_acc(a2);
        if (active) gemm_frag_packed<MODE, 2, 1, 256 / 16, false, HEAD>(a2, Gf, 16, 0, W1t, col0 / 32, 256 / 16, 0, lane);
        if constexpr (MODE == 2)
            unscale_acc_rows<MODE, 1>(a2, rinv, h);  // 2^-k w1s per row
        else
            scale_acc<MODE>(a2, w1s);
        if (active) {
            if (run_key && col0 >= run_c0 && col0 < run_c0 + MATRIS_D)
                store_acc_runs<1>(a2, gxr, ldp, col0 - coff, run_starts, nrows, lane);
            else if (col0 >= MATRIS_D || !epi0)
                store_acc_rows<1>(a2, gxr, ldp, col0 - coff, nrows, lane);
        }
        if (last && epi0) {
            __syncthreads();  // all waves are done reading G
            // with the pair tail, source 0's block goes to G's first 32 KB (row stride 128)
            // and the other 32 KB stage g0, then g1
            constexpr int LD0 = PAIR ? MATRIS_D : LDH;
            if (active && col0 < MATRIS_D) acc_to_lds<1>(a2, G, LD0, col0, lane);
            if constexpr (PAIR) {
                // wave w adds the 32 x 32 tile (rows 32 (w / 4), columns 32 (w % 4)) of
                // g0 W[0:128] + g1 W[128:256] to source 0's block (one power-of-two scale
                // per row for g0 and g1 in MODE 2)
                __shared__ float pinv[BM];
                uint4 *Pf = Gf + 2 * 8 * 2 * 64;
                const uint4 *pw = pair.Wt;
                const float pws = take_wscale<MODE>(pw);
                const int prt = wave >> 2, pct = wave & 3;
                float4 xa[4], xb[4];
                load_rows4(xa, pair.g0, m0, M, tid);
                load_rows4(xb, pair.g1, m0, M, tid);
                if constexpr (MODE == 2) {
                    float mx = 0.f;
#pragma unroll
                    for (int q = 0; q < 4; ++q) mx = abs_max4(abs_max4(mx, xa[q]), xb[q]);
                    const RowScale rs = row_scale(group8_max(mx));
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        xa[q] = mul4(xa[q], rs.s);
                        xb[q] = mul4(xb[q], rs.s);
                    }
                    if ((tid & 7) == 0) pinv[tid >> 3] = rs.inv * pws;
                }
                amax = stage_rows4<MODE>(Pf, xa, tid, amax);
                __syncthreads();
                v16f pa[1][1];
                zero_acc(pa);
                gemm_frag_packed<MODE, 1, 1, MATRIS_D / 16, true>(pa, Pf + prt * (8 * 2 * 64), 8, 0, pw, pct, 256 / 16,
                                                                  0, lane);
                __syncthreads();  // every wave is done reading g0
                amax = stage_rows4<MODE>(Pf, xb, tid, amax);
                __syncthreads();
                gemm_frag_packed<MODE, 1, 1, MATRIS_D / 16, true>(pa, Pf + prt * (8 * 2 * 64), 8, 0, pw, pct, 256 / 16,
                                                                  MATRIS_D / 16, lane);
                const float sc = MODE == 2 ? pinv[prt * 32 + l32] : pws;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    float4 *t = reinterpret_cast<float4 *>(G + (prt * 32 + l32) * MATRIS_D + pct * 32 + 8 * j + 4 * h);
                    float4 v = *t;
                    v.x += pa[0][0][4 * j] * sc; v.y += pa[0][0][4 * j + 1] * sc;
                    v.z += pa[0][0][4 * j + 2] * sc; v.w += pa[0][0][4 * j + 3] * sc;
                    *t = v;
                }
            }
        }
        top = base;
    }
    if (epi0) {
        __syncthreads();
        float *__restrict__ gx0 = g_x0 ? g_x0 + m0 * MATRIS_D : gxr;
        const int ld0 = g_x0 ? MATRIS_D : ldr;
        const float *__restrict__ got = (res_src ? res_src : g_out) + m0 * MATRIS_D;
#pragma unroll
        for (int it = 0; it < (BM * 32) / 512; ++it) {
            const int q = it * 512 + tid;
            const int r = q >> 5, c4 = (q & 31) * 4;
            if (r < nrows) {
                float4 v = *reinterpret_cast<const float4 *>(G + r * (PAIR ? MATRIS_D : LDH) + c4);
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
    report_range<MODE>(amax, range_flag);
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

static int gmlp_fwd_launch(int64_t m, int n_src, const float *const *src_host, const int32_t *const *src_idx_host,
                           int n_proj, const float *const *proj_host, const int32_t *const *proj_idx_host,
                           const int64_t *proj_ld_host, const void *w1p, const float *b1, const void *w2p, const float *b2,
                           const float *norm_c, const float *norm_g, float eps, float *out, float *save_p,
                           float *save_z, const float *res_src, const float *res_w, float *res_out,
                           const FfnTail &tail, const PairOut &pout, int mode, void *stream) {
    if (!matris_mode_ok(mode)) return MATRIS_E_ARG;
    if (m < 0 || n_src < 0 || n_src > 4 || n_proj < 0 || n_proj > 3 || n_src + n_proj < 1 ||
        (n_src && (!src_host || !w1p)) || !b1 || !w2p || !b2 || !norm_c || !norm_g || !out)
        return MATRIS_E_ARG;
    if (n_proj && (!proj_host || !proj_ld_host)) return MATRIS_E_ARG;
    if (m == 0) return 0;
    GmlpSrc s;
    for (int j = 0; j < 4; ++j) {
        s.ptr[j] = j < n_src ? src_host[j] : nullptr;
        s.idx[j] = (j < n_src && src_idx_host) ? src_idx_host[j] : nullptr;
        if (j < n_src && (!s.ptr[j] || !aligned16(s.ptr[j]))) return MATRIS_E_ARG;
    }
    GmlpProj pj;
    pj.n = n_proj;
    for (int j = 0; j < 3; ++j) {
        pj.ptr[j] = j < n_proj ? proj_host[j] : nullptr;
        pj.idx[j] = (j < n_proj && proj_idx_host) ? proj_idx_host[j] : nullptr;
        pj.ld[j] = j < n_proj ? proj_ld_host[j] : 0;
        if (j < n_proj && (!pj.ptr[j] || !aligned16(pj.ptr[j]) || pj.ld[j] < 256 || (pj.ld[j] & 3)))
            return MATRIS_E_ARG;
    }
    if ((n_src && !aligned16(w1p)) || !aligned16(w2p)) return MATRIS_E_ARG;
    if (res_out && (!res_src || !res_w)) return MATRIS_E_ARG;
    const bool has_tail = tail.W1 != nullptr;
    if (has_tail && (res_out || !aligned16(tail.W1) || !tail.W2 || !aligned16(tail.W2) || !tail.out ||
                     !aligned16(tail.out) || !aligned16(tail.res) || (tail.res && !tail.res_w) ||
                     !aligned16(tail.res_w) || !aligned16(tail.save_p)))
        return MATRIS_E_ARG;
    const bool has_pair = pout.W != nullptr;
    if (has_pair && (has_tail || !res_out || !aligned16(pout.W) || !pout.o0 || !aligned16(pout.o0) || !pout.o1 ||
                     !aligned16(pout.o1)))
        return MATRIS_E_ARG;
    const dim3 grid(matris_blocks(m, BM));
    hipStream_t st = (hipStream_t)stream;
    const uint4 *w1 = n_src ? (const uint4 *)w1p : nullptr, *w2 = (const uint4 *)w2p;
    unsigned *flag = nullptr;
    if (mode == 2 && !(flag = matris_range_flag())) return MATRIS_E_ARG;
#define GMLP_FWD(M_, T_, P_)                                                                                       \
    gmlp_fwd_kernel<M_, T_, P_><<<grid, 256, 0, st>>>(m, n_src, s, pj, w1, b1, w2, b2, norm_c, norm_g, eps, out,   \
                                                      save_p, save_z, res_src, res_w, res_out, tail, pout, flag)
    if (!has_tail && !has_pair) {
        MATRIS_MODE_DISPATCH(gmlp_fwd_kernel, grid, st, m, n_src, s, pj, w1, b1, w2, b2, norm_c, norm_g, eps, out,
                             save_p, save_z, res_src, res_w, res_out, tail, pout, flag);
    } else if (has_tail) {
        if (mode == 0) GMLP_FWD(0, true, false);
        else if (mode == 2) GMLP_FWD(2, true, false);
        else if (mode == 3) GMLP_FWD(3, true, false);
        else GMLP_FWD(6, true, false);
    } else {
        if (mode == 0) GMLP_FWD(0, false, true);
        else if (mode == 2) GMLP_FWD(2, false, true);
        else if (mode == 3) GMLP_FWD(3, false, true);
        else GMLP_FWD(6, false, true);
    }
#undef GMLP_FWD
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_gmlp_fwd(int64_t m, int n_src, const float *const *src_host,
                               const int32_t *const *src_idx_host, const void *w1p, const float *b1, const void *w2p,
                               const float *b2, const float *norm_c, const float *norm_g, float eps, float *out,
                               float *save_p, float *save_z, const float *res_src, const float *res_w,
                               float *res_out, int mode, void *stream) {
    if (n_src < 1) return MATRIS_E_ARG;
    return gmlp_fwd_launch(m, n_src, src_host, src_idx_host, 0, nullptr, nullptr, nullptr, w1p, b1, w2p, b2, norm_c, norm_g,
                           eps, out, save_p, save_z, res_src, res_w, res_out, FfnTail{}, PairOut{}, mode, stream);
}

extern "C" int matris_gmlp_fwd_proj(int64_t m, int n_src, const float *const *src_host,
                                    const int32_t *const *src_idx_host, int n_proj, const float *const *proj_host,
                                    const int32_t *const *proj_idx_host, const int64_t *proj_ld_host,
                                    const void *w1p,
                                    const float *b1, const void *w2p, const float *b2, const float *norm_c,
                                    const float *norm_g, float eps, float *out, float *save_p, float *save_z,
                                    const float *res_src, const float *res_w, float *res_out, int mode,
                                    void *stream) {
    return gmlp_fwd_launch(m, n_src, src_host, src_idx_host, n_proj, proj_host, proj_idx_host, proj_ld_host, w1p, b1, w2p,
                           b2, norm_c, norm_g, eps, out, save_p, save_z, res_src, res_w, res_out, FfnTail{},
                           PairOut{}, mode, stream);
}

extern "C" int matris_gmlp_fwd_pair(int64_t m, int n_src, const float *const *src_host,
                                    const int32_t *const *src_idx_host, int n_proj, const float *const *proj_host,
                                    const int32_t *const *proj_idx_host, const int64_t *proj_ld_host,
                                    const void *w1p, const float *b1, const void *w2p, const float *b2,
                                    const float *norm_c, const float *norm_g, float eps, float *out, float *save_p,
                                    float *save_z, const float *res_src, const float *res_w, float *res_out,
                                    const void *pair_wp, float *pair_out0, float *pair_out1, int mode,
                                    void *stream) {
    if (!pair_wp) return MATRIS_E_ARG;
    const PairOut pout{(const uint4 *)pair_wp, pair_out0, pair_out1};
    return gmlp_fwd_launch(m, n_src, src_host, src_idx_host, n_proj, proj_host, proj_idx_host, proj_ld_host, w1p, b1, w2p,
                           b2, norm_c, norm_g, eps, out, save_p, save_z, res_src, res_w, res_out, FfnTail{}, pout,
                           mode, stream);
}

extern "C" int matris_gmlp_fwd_ffn(int64_t m, int n_src, const float *const *src_host,
                                   const int32_t *const *src_idx_host, int n_proj, const float *const *proj_host,
                                   const int32_t *const *proj_idx_host, const int64_t *proj_ld_host, const void *w1p,
                                   const float *b1, const void *w2p, const float *b2, const float *norm_c,
                                   const float *norm_g, float eps, float *out, float *save_p, float *save_z,
                                   const void *ffn_w1p, const void *ffn_w2p, float *ffn_save_p, const float *ffn_res,
                                   const float *ffn_res_w, float *ffn_out, int mode, void *stream) {
    if (!ffn_w1p) return MATRIS_E_ARG;
    const FfnTail tail{(const uint4 *)ffn_w1p, (const uint4 *)ffn_w2p, ffn_save_p, ffn_out, ffn_res, ffn_res_w};
    return gmlp_fwd_launch(m, n_src, src_host, src_idx_host, n_proj, proj_host, proj_idx_host, proj_ld_host, w1p, b1, w2p,
                           b2, norm_c, norm_g, eps, out, save_p, save_z, nullptr, nullptr, nullptr, tail,
                           PairOut{}, mode, stream);
}

static int gmlp_bwd_launch(int64_t m, int k, const float *g_out, const float *p, const float *z, const void *w1tp,
                           const void *w2tp, const float *norm_c, const float *norm_g, float eps, float *g_x,
                           float *g_x0, int acc0, const float *res_w, const float *res_src, const int32_t *run_key,
                           int run_blk, const FfnHead &head, const PairTail &pair, int mode, void *stream) {
    if (!matris_mode_ok(mode)) return MATRIS_E_ARG;
    const bool has_head = head.W1t != nullptr, has_pair = pair.Wt != nullptr;
    if (has_pair && (has_head || mode == 6 || !g_x0 || k < 2 * MATRIS_D || !pair.g0 || !aligned16(pair.g0) ||
                     !pair.g1 || !aligned16(pair.g1) || !aligned16(pair.Wt)))
        return MATRIS_E_ARG;
    if (m < 0 || k < MATRIS_D || k > 4 * MATRIS_D || (k % MATRIS_D) || (!g_out && !has_head) || !p || !z || !w1tp ||
        !w2tp || !norm_c || !norm_g || (!g_x && !(g_x0 && k == MATRIS_D)))
        return MATRIS_E_ARG;
    if (has_head && (mode == 6 || !aligned16(head.W1t) || !head.W2t || !aligned16(head.W2t) || !head.g ||
                     !aligned16(head.g) || !head.p || !aligned16(head.p) || !aligned16(head.ge) ||
                     (head.ge && (!head.env || !aligned16(head.env) || !head.t || !head.s))))
        return MATRIS_E_ARG;
    // the reduced block goes to g_x: not source 0 when source 0 has its own output
    if (run_key && (!g_x || run_blk < (g_x0 ? 1 : 0) || run_blk >= k / MATRIS_D)) return MATRIS_E_ARG;
    if (m == 0) return 0;
    if (!aligned16(w1tp) || !aligned16(w2tp)) return MATRIS_E_ARG;
    if (acc0 && !g_x0) return MATRIS_E_ARG;
    if (res_src && !res_w) return MATRIS_E_ARG;
    const dim3 grid(matris_blocks(m, BM));
    hipStream_t st = (hipStream_t)stream;
    const uint4 *w1t = (const uint4 *)w1tp, *w2t = (const uint4 *)w2tp;
    unsigned *flag = nullptr;
    if (mode == 2 && !(flag = matris_range_flag())) return MATRIS_E_ARG;
    if (mode == 6) {
        gmlp_bwd_kernel<6><<<grid, 256, 0, st>>>(m, k, g_out, p, z, w1t, w2t, norm_c, norm_g, eps, g_x, g_x0, acc0,
                                                 res_w, res_src, run_key, run_blk, flag);
    } else {
#define GMLP_BWD8(M_, H_, P_)                                                                                      \
    gmlp_bwd8_kernel<M_, H_, P_><<<grid, 512, 0, st>>>(m, k, g_out, p, z, w1t, w2t, norm_c, norm_g, eps, g_x, g_x0, \
                                                       acc0, res_w, res_src, run_key, run_blk, head, pair, flag)
        if (has_head) {
            if (mode == 0) GMLP_BWD8(0, true, false);
            else if (mode == 2) GMLP_BWD8(2, true, false);
            else GMLP_BWD8(3, true, false);
        } else if (has_pair) {
            if (mode == 0) GMLP_BWD8(0, false, true);
            else if (mode == 2) GMLP_BWD8(2, false, true);
            else GMLP_BWD8(3, false, true);
        } else {
            if (mode == 0) GMLP_BWD8(0, false, false);
            else if (mode == 2) GMLP_BWD8(2, false, false);
            else GMLP_BWD8(3, false, false);
        }
#undef GMLP_BWD8
    }
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_gmlp_bwd(int64_t m, int k, const float *g_out, const float *p, const float *z, const void *w1tp,
                               const void *w2tp, const float *norm_c, const float *norm_g, float eps, float *g_x,
                               float *g_x0, int acc0, const float *res_w, int mode, void *stream) {
    return gmlp_bwd_launch(m, k, g_out, p, z, w1tp, w2tp, norm_c, norm_g, eps, g_x, g_x0, acc0, res_w, nullptr,
                           nullptr, -1, FfnHead{}, PairTail{}, mode, stream);
}

extern "C" int matris_gmlp_bwd_runs(int64_t m, int k, const float *g_out, const float *p, const float *z,
                                    const void *w1tp, const void *w2tp, const float *norm_c, const float *norm_g,
                                    float eps, float *g_x, float *g_x0, int acc0, const float *res_w,
                                    const float *res_src, const int32_t *run_key, int run_blk, int mode,
                                    void *stream) {
    return gmlp_bwd_launch(m, k, g_out, p, z, w1tp, w2tp, norm_c, norm_g, eps, g_x, g_x0, acc0, res_w, res_src,
                           run_key, run_key ? run_blk : -1, FfnHead{}, PairTail{}, mode, stream);
}

extern "C" int matris_gmlp_bwd_ffn(int64_t m, int k, const float *p, const float *z, const void *w1tp,
                                   const void *w2tp, const float *norm_c, const float *norm_g, float eps, float *g_x,
                                   float *g_x0, const float *res_w, const int32_t *run_key, int run_blk,
                                   const float *ffn_g, const int32_t *ffn_g_idx, float ffn_g_scale,
                                   const float *ffn_p, const void *ffn_w1tp, const void *ffn_w2tp,
                                   const float *g_agg_env, const float *env, const int32_t *t_idx,
                                   const int32_t *s_idx, int mode, void *stream) {
    if (!ffn_w1tp || (ffn_g_idx && res_w)) return MATRIS_E_ARG;
    const FfnHead head{ffn_g,  ffn_p, (const uint4 *)ffn_w1tp, (const uint4 *)ffn_w2tp, g_agg_env, env, t_idx, s_idx,
                       ffn_g_idx, ffn_g_idx ? ffn_g_scale : 1.0f};
    // the residual term of source 0's gradient is res_w * (the FFN's output gradient)
    return gmlp_bwd_launch(m, k, nullptr, p, z, w1tp, w2tp, norm_c, norm_g, eps, g_x, g_x0, 0, res_w,
                           res_w ? ffn_g : nullptr, run_key, run_key ? run_blk : -1, head, PairTail{}, mode, stream);
}

extern "C" int matris_gmlp_bwd_pair(int64_t m, int k, const float *g_out, const float *p, const float *z,
                                    const void *w1tp, const void *w2tp, const float *norm_c, const float *norm_g,
                                    float eps, float *g_x, float *g_x0, const float *res_w, const float *res_src,
                                    const int32_t *run_key, int run_blk, const float *pair_g0, const float *pair_g1,
                                    const void *pair_wtp, int mode, void *stream) {
    if (!pair_wtp) return MATRIS_E_ARG;
    const PairTail pair{pair_g0, pair_g1, (const uint4 *)pair_wtp};
    return gmlp_bwd_launch(m, k, g_out, p, z, w1tp, w2tp, norm_c, norm_g, eps, g_x, g_x0, 0, res_w, res_src, run_key,
                           run_key ? run_blk : -1, FfnHead{}, pair, mode, stream);
}

extern "C" int matris_gmlp_tile_rows(void) { return BM; }

// ------------------------------------------------------------------------------------
// weight packing: [n, k] row-major fp32 (rows = output columns of the GEMM) -> fragment
// planes, one thread per (tile, k-block, lane)
// ------------------------------------------------------------------------------------
// MODE 2 header {1/s, s, 0, 0}: s = 2^(14 - e) with 2^e <= max |w| < 2^(e+1), so the
// scaled weights reach [2^14, 2^15) at most (s = 1 for an all-zero or non-finite matrix).
// One work-group of 1024 threads (count is a multiple of 512, w 16-byte aligned).
__global__ __launch_bounds__(1024) void wscale_kernel(int64_t count, const float *__restrict__ w,
                                                      float *__restrict__ hdr) {
    __shared__ float part[16];
    float m = 0.f;
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    for (int64_t i = threadIdx.x; i < count / 4; i += blockDim.x) {
        const float4 v = w4[i];
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        m = 0.f;
        for (int i = 0; i < 16; ++i) m = fmaxf(m, part[i]);
        int e = 0;
        if (m > 0.f && m <= 3.0e38f) e = ilogbf(m) - 14;  // s = 2^-e
        e = max(-120, min(120, e));
        hdr[0] = ldexpf(1.0f, e);
        hdr[1] = ldexpf(1.0f, -e);
        hdr[2] = 0.f;
        hdr[3] = 0.f;
    }
}

template <int MODE>
__global__ void pack_b_kernel(int64_t n, int64_t k, const float *__restrict__ w, uint4 *__restrict__ out) {
    constexpr int NPL = Npl<MODE>::v;
    const int64_t KB = k / 16;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // (nt * KB + kb) * 64 + lane
    if (t >= n / 32 * KB * 64) return;
    const int lane = (int)(t & 63);
    const int64_t ntkb = t >> 6, nt = ntkb / KB, kb = ntkb % KB;
    const float *r = w + (nt * 32 + (lane & 31)) * k + kb * 16 + (lane >> 5) * 8;
    const float4 u = *reinterpret_cast<const float4 *>(r), v = *reinterpret_cast<const float4 *>(r + 4);
    if constexpr (MODE == 2) {
        // u0 = fp16(s w), u1 = fp16(s w - u0) after the header written by wscale_kernel
        const float sc = reinterpret_cast<const float *>(out)[1];
        const float x[8] = {u.x * sc, u.y * sc, u.z * sc, u.w * sc, v.x * sc, v.y * sc, v.z * sc, v.w * sc};
        uint32_t p0[4], p1[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const f2v xv = {x[2 * j], x[2 * j + 1]};
            const h2v hv = __builtin_convertvector(xv, h2v);
            p0[j] = bitcast<uint32_t>(hv);
            p1[j] = bitcast<uint32_t>(__builtin_convertvector(xv - __builtin_convertvector(hv, f2v), h2v));
        }
        out += 1;
        out[(ntkb * NPL + 0) * 64 + lane] = make_uint4(p0[0], p0[1], p0[2], p0[3]);
        out[(ntkb * NPL + 1) * 64 + lane] = make_uint4(p1[0], p1[1], p1[2], p1[3]);
    } else {
        Frag<MODE> f;
        make_frag<MODE>(f, u, v);
#pragma unroll
        for (int pl = 0; pl < NPL; ++pl) out[(ntkb * NPL + pl) * 64 + lane] = f.p[pl];
    }
}

extern "C" size_t matris_pack_b_bytes(int64_t n, int64_t k, int mode) { return packed_b_bytes(n, k, mode); }

extern "C" int matris_pack_b(int64_t n, int64_t k, const float *w, int mode, void *out, void *stream) {
    if (!matris_mode_ok(mode)) return MATRIS_E_ARG;
    if (n < 0 || k < 0 || (n % 32) || (k % 16) || !w || !out || !aligned16(w) || !aligned16(out)) return MATRIS_E_ARG;
    const int64_t threads = n / 32 * (k / 16) * 64;
    hipStream_t st = (hipStream_t)stream;
    if (mode == 2) {  // the header comes first, also for an empty matrix
        wscale_kernel<<<1, 1024, 0, st>>>(n * k, w, (float *)out);
        MATRIS_CHECK_LAUNCH();
    }
    if (threads == 0) return 0;
    const dim3 grid(matris_blocks(threads, 256));
    MATRIS_MODE_DISPATCH(pack_b_kernel, grid, st, n, k, w, (uint4 *)out);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_status_take(unsigned *bits, void *stream) {
    if (!bits) return MATRIS_E_ARG;
    unsigned *flag = matris_range_flag();
    if (!flag) return MATRIS_E_ARG;
    hipStream_t st = (hipStream_t)stream;
    // read, then clear with a kernel (no memset node), both ordered on the caller's stream
    unsigned v = 0u;
    hipError_t e = hipMemcpyAsync(&v, flag, sizeof(v), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) {
        range_reset_kernel<<<1, 1, 0, st>>>(flag);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    *bits = e == hipSuccess ? v : 0u;
    return (int)e;
}
