// Graph construction on gfx950: periodic radius graph (G1), directed->undirected pairing
// (G3/G4), bond->angle line graph (G5), stable CSR builder, exclusive scans.
//
// Integer / fp64 decision work: HBM- and latency-bound, no MFMA.  Every fp64 decision
// uses the evaluation order of the CPU oracle (oracle/graph_oracle.c) with FMA
// contraction disabled, so inclusion tests agree bit-for-bit with the oracle.
#pragma clang fp contract(off)

#include <math.h>
#include <string.h>

#include <mutex>

#include "common.h"

// ------------------------------------------------------------------------------------
// exclusive scans (three-pass: block sums, scan of sums, block rescan)
// ------------------------------------------------------------------------------------
#define SCAN_BLOCK 256
#define SCAN_ITEMS 4
#define SCAN_TILE (SCAN_BLOCK * SCAN_ITEMS)

template <typename TIN>
__global__ void scan_tile_sums(const TIN *__restrict__ in, int64_t n, int64_t *__restrict__ tile_sums) {
    __shared__ int64_t red[SCAN_BLOCK / 64];
    int64_t base = (int64_t)blockIdx.x * SCAN_TILE;
    int64_t s = 0;
    for (int k = 0; k < SCAN_ITEMS; ++k) {
        int64_t i = base + (int64_t)k * SCAN_BLOCK + threadIdx.x;
        if (i < n) s += (int64_t)in[i];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        int64_t t = 0;
        for (int w = 0; w < SCAN_BLOCK / 64; ++w) t += red[w];
        tile_sums[blockIdx.x] = t;
    }
}

// Single work-group exclusive scan of the tile sums (in place); writes the grand total.
__global__ void scan_tile_offsets(int64_t *__restrict__ sums, int64_t n_tiles, int64_t *__restrict__ total) {
    __shared__ int64_t buf[SCAN_BLOCK];
    int64_t carry = 0;
    for (int64_t b = 0; b < n_tiles; b += SCAN_BLOCK) {
        int64_t i = b + threadIdx.x;
        int64_t v = i < n_tiles ? sums[i] : 0;
        buf[threadIdx.x] = v;
        __syncthreads();
        for (int o = 1; o < SCAN_BLOCK; o <<= 1) {
            int64_t t = threadIdx.x >= o ? buf[threadIdx.x - o] : 0;
            __syncthreads();
            buf[threadIdx.x] += t;
            __syncthreads();
        }
        if (i < n_tiles) sums[i] = carry + buf[threadIdx.x] - v;
        carry += buf[SCAN_BLOCK - 1];
        __syncthreads();
    }
    if (threadIdx.x == 0) *total = carry;
}

template <typename TIN, typename TOUT>
__global__ void scan_tile_apply(const TIN *__restrict__ in, int64_t n, const int64_t *__restrict__ offsets,
                                const int64_t *__restrict__ total, TOUT *__restrict__ out) {
    __shared__ int64_t buf[SCAN_TILE];
    int64_t base = (int64_t)blockIdx.x * SCAN_TILE;
    for (int k = 0; k < SCAN_ITEMS; ++k) {
        int64_t i = base + (int64_t)k * SCAN_BLOCK + threadIdx.x;
        buf[k * SCAN_BLOCK + threadIdx.x] = i < n ? (int64_t)in[i] : 0;
    }
    __syncthreads();
    // serial per-thread chunk of SCAN_ITEMS, then block scan of chunk totals
    __shared__ int64_t part[SCAN_BLOCK];
    int64_t loc[SCAN_ITEMS];
    int64_t run = 0;
    for (int k = 0; k < SCAN_ITEMS; ++k) {
        loc[k] = run;
        run += buf[threadIdx.x * SCAN_ITEMS + k];
    }
    part[threadIdx.x] = run;
    __syncthreads();
    for (int o = 1; o < SCAN_BLOCK; o <<= 1) {
        int64_t t = threadIdx.x >= o ? part[threadIdx.x - o] : 0;
        __syncthreads();
        part[threadIdx.x] += t;
        __syncthreads();
    }
    int64_t excl = part[threadIdx.x] - run + offsets[blockIdx.x];
    for (int k = 0; k < SCAN_ITEMS; ++k) {
        int64_t i = base + threadIdx.x * SCAN_ITEMS + k;
        if (i < n) out[i] = (TOUT)(excl + loc[k]);
    }
    if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) out[n] = (TOUT)(*total);
}

static size_t scan_workspace_bytes(int64_t n) {
    int64_t tiles = (n + SCAN_TILE - 1) / SCAN_TILE;
    return (size_t)(tiles + 2) * sizeof(int64_t);
}

// out[0..n] = exclusive scan of in[0..n-1] with out[n] = total.
template <typename TIN, typename TOUT>
static int scan_exclusive(const TIN *in, int64_t n, TOUT *out, void *ws, hipStream_t st) {
    int64_t tiles = (n + SCAN_TILE - 1) / SCAN_TILE;
    if (tiles < 1) tiles = 1;
    int64_t *sums = (int64_t *)ws;
    int64_t *total = sums + tiles;
    scan_tile_sums<TIN><<<(unsigned)tiles, SCAN_BLOCK, 0, st>>>(in, n, sums);
    scan_tile_offsets<<<1, SCAN_BLOCK, 0, st>>>(sums, tiles, total);
    scan_tile_apply<TIN, TOUT><<<(unsigned)tiles, SCAN_BLOCK, 0, st>>>(in, n, sums, total, out);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

template <typename T>
__global__ void fill_kernel(T *p, int64_t n, T v) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

template <typename T>
static void fill(T *p, int64_t n, T v, hipStream_t st) {
    if (n > 0) fill_kernel<T><<<matris_blocks(n, 256), 256, 0, st>>>(p, n, v);
}

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// ------------------------------------------------------------------------------------
// G1: radius graph with a cell list in fractional space
// ------------------------------------------------------------------------------------
struct RGPlan {
    double L[9];
    int g[3], r[3];
};

__device__ __forceinline__ void frac_to_cart_d(const double *f, const double *L, double *c) {
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        double t = f[0] * L[0 * 3 + k];
        t = t + f[1] * L[1 * 3 + k];
        t = t + f[2] * L[2 * 3 + k];
        c[k] = t;
    }
}

// Same expression as pair_dist() in oracle/graph_oracle.c.
__device__ __forceinline__ double pair_dist_d(const double *ci, const double *cj, const double *L, int n0, int n1,
                                              int n2) {
    double d2 = 0.0;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        double s = (double)n0 * L[0 * 3 + k];
        s = s + (double)n1 * L[1 * 3 + k];
        s = s + (double)n2 * L[2 * 3 + k];
        double d = (cj[k] - ci[k]) + s;
        d2 = d2 + d * d;
    }
    return sqrt(d2);
}

struct RGWork {
    double *cart;     // [n,3]
    int *wrap;        // [n,3] floor(frac)
    int *cell;        // [n]   linear cell id
    int *cell_start;  // [ncell+1]
    int *cell_atoms;  // [n]
    int *cursor;      // [ncell]
    void *scan_ws;
};

static RGWork rg_carve(void *ws, int64_t n, int64_t ncell) {
    RGWork w;
    char *p = (char *)ws;
    w.cart = (double *)p; p += align256(sizeof(double) * 3 * n);
    w.wrap = (int *)p; p += align256(sizeof(int) * 3 * n);
    w.cell = (int *)p; p += align256(sizeof(int) * n);
    w.cell_start = (int *)p; p += align256(sizeof(int) * (ncell + 1));
    w.cell_atoms = (int *)p; p += align256(sizeof(int) * n);
    w.cursor = (int *)p; p += align256(sizeof(int) * ncell);
    w.scan_ws = p;
    return w;
}

__global__ void rg_bin_kernel(int64_t n, const double *__restrict__ frac, RGPlan plan, RGWork w) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    double f[3] = {frac[3 * i], frac[3 * i + 1], frac[3 * i + 2]};
    double c[3];
    frac_to_cart_d(f, plan.L, c);
    int cid = 0;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        w.cart[3 * i + k] = c[k];
        double fl = floor(f[k]);
        w.wrap[3 * i + k] = (int)fl;
        int ck = (int)floor((f[k] - fl) * plan.g[k]);
        ck = ck < 0 ? 0 : (ck >= plan.g[k] ? plan.g[k] - 1 : ck);
        cid = cid * plan.g[k] + ck;
    }
    w.cell[i] = cid;
    atomicAdd(&w.cursor[cid], 1);
}

__global__ void rg_scatter_kernel(int64_t n, RGWork w) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int cid = w.cell[i];
    int pos = w.cell_start[cid] + atomicAdd(&w.cursor[cid], 1);
    w.cell_atoms[pos] = (int)i;
}

__device__ __forceinline__ bool key_less(int ja, const int *na, int jb, const int *nb) {
    if (ja != jb) return ja < jb;
    if (na[0] != nb[0]) return na[0] < nb[0];
    if (na[1] != nb[1]) return na[1] < nb[1];
    return na[2] < nb[2];
}

// Count and fill passes, one wave per atom: the 64 lanes of a wave share the atom's
// candidates.  The (2r+1)^3 candidate cells are taken 64 at a time (one per lane:
// its cell id, image shift and atom range), a wave scan of the cell sizes gives each
// chunk's candidate offsets, and every lane takes candidates k = lane, lane + 64, ...
// (the cell found by binary search over the offsets); the candidate's image is the cell's
// periodic shift in the wrapped frame taken back to the original frame.  An edge is
// accepted when tol < |r_j + n L - r_i| <= cutoff (pair_dist_d, the oracle's expression).
// Edges emitted by a fill are ordered by (neighbor, image): the key is unique within a
// row, so every emission order gives the same row.
#define RG_ROW_CAP 1024  // edges a wave sorts in LDS; longer rows sort in place in global

struct RGChunk {
    int off[65];  // candidate offset of each cell of the chunk (exclusive), off[64] = total
    int start[64], q[64], s0[64], s1[64], s2[64];
};

// Load chunk `c0 .. c0+63` of the candidate cells of an atom in cell (c0_, c1_, c2_).
__device__ __forceinline__ void rg_chunk(RGChunk &ch, const RGPlan &plan, const RGWork &w, int cell0, int ncells,
                                         int a_c0, int a_c1, int a_c2, int lane) {
    const int c = cell0 + lane;
    int size = 0, st = 0, q = 0, s0 = 0, s1 = 0, s2 = 0;
    if (c < ncells) {
        const int n1 = 2 * plan.r[1] + 1, n2 = 2 * plan.r[2] + 1;
        const int d0 = c / (n1 * n2) - plan.r[0], d1 = (c / n2) % n1 - plan.r[1], d2 = c % n2 - plan.r[2];
        const int a0 = a_c0 + d0, a1 = a_c1 + d1, a2 = a_c2 + d2;
        s0 = (int)floor((double)a0 / plan.g[0]);
        s1 = (int)floor((double)a1 / plan.g[1]);
        s2 = (int)floor((double)a2 / plan.g[2]);
        const int q0 = a0 - s0 * plan.g[0], q1 = a1 - s1 * plan.g[1], q2 = a2 - s2 * plan.g[2];
        q = (q0 * plan.g[1] + q1) * plan.g[2] + q2;
        st = w.cell_start[q];
        size = w.cell_start[q + 1] - st;
    }
    // inclusive wave scan of the sizes
    int incl = size;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(incl, o, 64);
        if (lane >= o) incl += t;
    }
    ch.off[lane] = incl - size;
    if (lane == 63) ch.off[64] = incl;
    ch.start[lane] = st;
    ch.q[lane] = q;
    ch.s0[lane] = s0;
    ch.s1[lane] = s1;
    ch.s2[lane] = s2;
}

// Candidate k of the chunk: the cell cc with off[cc] <= k < off[cc + 1].
__device__ __forceinline__ int rg_cell_of(const RGChunk &ch, int k) {
    int lo = 0, hi = 63;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (ch.off[mid] <= k) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// Visit every candidate of atom i with the wave; f(accept, j, n0, n1, n2, d) is called by
// every lane on every round (accept false on idle lanes) so that it can use ballots.
template <typename F>
__device__ __forceinline__ void rg_visit_wave(int64_t i, const RGPlan &plan, const RGWork &w, double cutoff,
                                              double tol, RGChunk &ch, int lane, F &&f) {
    const double ci[3] = {w.cart[3 * i], w.cart[3 * i + 1], w.cart[3 * i + 2]};
    const int cid = w.cell[i];
    const int c2 = cid % plan.g[2], c1 = (cid / plan.g[2]) % plan.g[1], c0 = cid / (plan.g[2] * plan.g[1]);
    const int wi0 = w.wrap[3 * i], wi1 = w.wrap[3 * i + 1], wi2 = w.wrap[3 * i + 2];
    const int ncells = (2 * plan.r[0] + 1) * (2 * plan.r[1] + 1) * (2 * plan.r[2] + 1);
    for (int cell0 = 0; cell0 < ncells; cell0 += 64) {
        rg_chunk(ch, plan, w, cell0, ncells, c0, c1, c2, lane);
        __syncthreads();  // one wave per work-group: orders the chunk's LDS writes and reads
        const int total = ch.off[64];
        for (int k0 = 0; k0 < total; k0 += 64) {
            const int k = k0 + lane;
            bool acc = false;
            int j = 0, n0 = 0, n1 = 0, n2 = 0;
            double d = 0.0;
            if (k < total) {
                const int cc = rg_cell_of(ch, k);
                j = w.cell_atoms[ch.start[cc] + (k - ch.off[cc])];
                n0 = ch.s0[cc] - w.wrap[3 * j] + wi0;
                n1 = ch.s1[cc] - w.wrap[3 * j + 1] + wi1;
                n2 = ch.s2[cc] - w.wrap[3 * j + 2] + wi2;
                d = pair_dist_d(ci, w.cart + 3 * j, plan.L, n0, n1, n2);
                acc = d <= cutoff && d > tol;
            }
            f(acc, j, n0, n1, n2, d);
        }
        __syncthreads();  // the chunk is read before the next one overwrites it
    }
}

__global__ __launch_bounds__(64) void rg_count_wave_kernel(int64_t n, RGPlan plan, RGWork w, double cutoff,
                                                           double tol, int32_t *__restrict__ row_count) {
    __shared__ RGChunk ch;
    const int64_t i = blockIdx.x;
    const int lane = threadIdx.x;
    int cnt = 0;
    rg_visit_wave(i, plan, w, cutoff, tol, ch, lane, [&](bool acc, int, int, int, int, double) {
        cnt += __popcll(__ballot(acc));
    });
    if (lane == 0) row_count[i] = cnt;
}

__global__ __launch_bounds__(64) void rg_fill_wave_kernel(int64_t n, RGPlan plan, RGWork w, double cutoff,
                                                          double tol, const int64_t *__restrict__ row_ptr,
                                                          int32_t *__restrict__ center, int32_t *__restrict__ neighbor,
                                                          int32_t *__restrict__ image, double *__restrict__ dist) {
    __shared__ RGChunk ch;
    __shared__ int sj[RG_ROW_CAP], sn[RG_ROW_CAP][3];
    __shared__ double sd[RG_ROW_CAP];
    const int64_t i = blockIdx.x;
    const int lane = threadIdx.x;
    const int64_t b = row_ptr[i];
    const int64_t m = row_ptr[i + 1] - b;
    const bool in_lds = m <= RG_ROW_CAP;
    int64_t e = 0;  // edges emitted so far (wave-uniform)
    rg_visit_wave(i, plan, w, cutoff, tol, ch, lane, [&](bool acc, int j, int n0, int n1, int n2, double d) {
        const uint64_t bal = __ballot(acc);
        const int64_t o = e + lanes_below(bal);
        if (acc && o < m) {  // o < m always holds (count and fill accept the same edges)
            if (in_lds) {
                sj[o] = j;
                sn[o][0] = n0;
                sn[o][1] = n1;
                sn[o][2] = n2;
                sd[o] = d;
            } else {
                neighbor[b + o] = j;
                image[3 * (b + o)] = n0;
                image[3 * (b + o) + 1] = n1;
                image[3 * (b + o) + 2] = n2;
                dist[b + o] = d;
            }
        }
        e += __popcll(bal);
    });
    if (in_lds) {
        __syncthreads();
        // rank sort: the unique key's rank is its position in the row
        for (int a = lane; a < (int)m; a += 64) {
            const int ja = sj[a];
            const int na[3] = {sn[a][0], sn[a][1], sn[a][2]};
            int rank = 0;
            for (int c = 0; c < (int)m; ++c) rank += key_less(sj[c], sn[c], ja, na) ? 1 : 0;
            neighbor[b + rank] = ja;
            image[3 * (b + rank)] = na[0];
            image[3 * (b + rank) + 1] = na[1];
            image[3 * (b + rank) + 2] = na[2];
            dist[b + rank] = sd[a];
            center[b + rank] = (int32_t)i;
        }
    } else if (lane == 0) {
        // a row longer than the LDS buffer: insertion sort in place (rows this long are rare)
        for (int64_t a = 1; a < m; ++a) {
            const int ja = neighbor[b + a];
            const int na[3] = {image[3 * (b + a)], image[3 * (b + a) + 1], image[3 * (b + a) + 2]};
            const double da = dist[b + a];
            int64_t p = a - 1;
            while (p >= 0) {
                const int nb[3] = {image[3 * (b + p)], image[3 * (b + p) + 1], image[3 * (b + p) + 2]};
                if (!key_less(ja, na, neighbor[b + p], nb)) break;
                neighbor[b + p + 1] = neighbor[b + p];
                image[3 * (b + p + 1)] = nb[0];
                image[3 * (b + p + 1) + 1] = nb[1];
                image[3 * (b + p + 1) + 2] = nb[2];
                dist[b + p + 1] = dist[b + p];
                --p;
            }
            neighbor[b + p + 1] = ja;
            image[3 * (b + p + 1)] = na[0];
            image[3 * (b + p + 1) + 1] = na[1];
            image[3 * (b + p + 1) + 2] = na[2];
            dist[b + p + 1] = da;
        }
        for (int64_t a = 0; a < m; ++a) center[b + a] = (int32_t)i;
    }
}

static void rg_make_plan(const double *lattice_host, const int *grid_host, const int *search_host, RGPlan *plan) {
    memcpy(plan->L, lattice_host, sizeof(plan->L));
    for (int k = 0; k < 3; ++k) {
        plan->g[k] = grid_host[k];
        plan->r[k] = search_host[k];
    }
}

extern "C" int matris_radius_graph_plan(const double *L, double cutoff, int *grid_host, int *search_host) {
    if (!L || !grid_host || !search_host || !(cutoff > 0)) return MATRIS_E_ARG;
    double cr[3][3];
    for (int k = 0; k < 3; ++k) {
        const double *u = L + 3 * ((k + 1) % 3), *v = L + 3 * ((k + 2) % 3);
        cr[k][0] = u[1] * v[2] - u[2] * v[1];
        cr[k][1] = u[2] * v[0] - u[0] * v[2];
        cr[k][2] = u[0] * v[1] - u[1] * v[0];
    }
    double vol = fabs(L[0] * cr[0][0] + L[1] * cr[0][1] + L[2] * cr[0][2]);
    if (!(vol > 0)) return MATRIS_E_ARG;
    for (int k = 0; k < 3; ++k) {
        double h = vol / sqrt(cr[k][0] * cr[k][0] + cr[k][1] * cr[k][1] + cr[k][2] * cr[k][2]);
        int g = (int)floor(h / cutoff);
        if (g < 1) g = 1;
        if (g > 256) g = 256;
        int r = (int)floor(cutoff * g / h + 1e-9) + 2;
        if (r > 511) return MATRIS_E_IMAGES;
        grid_host[k] = g;
        search_host[k] = r;
    }
    return 0;
}

extern "C" size_t matris_radius_graph_workspace_bytes(int64_t n, const int *g) {
    int64_t ncell = (int64_t)g[0] * g[1] * g[2];
    return align256(sizeof(double) * 3 * n) + align256(sizeof(int) * 3 * n) + 2 * align256(sizeof(int) * n) +
           align256(sizeof(int) * (ncell + 1)) + align256(sizeof(int) * ncell) + align256(sizeof(int) * n) +
           scan_workspace_bytes(n > ncell ? n : ncell) + 256;
}

extern "C" int matris_radius_graph_count(int64_t n, const double *frac, const double *lattice_host, double cutoff,
                                         double tol, const int *grid_host, const int *search_host,
                                         int32_t *row_count, int64_t *row_ptr, void *workspace,
                                         size_t workspace_bytes, void *stream) {
    if (n <= 0 || !frac || !row_count || !row_ptr || !workspace) return MATRIS_E_ARG;
    if (workspace_bytes < matris_radius_graph_workspace_bytes(n, grid_host)) return MATRIS_E_ARG;
    hipStream_t st = (hipStream_t)stream;
    RGPlan plan;
    rg_make_plan(lattice_host, grid_host, search_host, &plan);
    int64_t ncell = (int64_t)plan.g[0] * plan.g[1] * plan.g[2];
    RGWork w = rg_carve(workspace, n, ncell);
    fill<int>(w.cursor, ncell, 0, st);
    rg_bin_kernel<<<matris_blocks(n, 256), 256, 0, st>>>(n, frac, plan, w);
    int rc = scan_exclusive<int, int>(w.cursor, ncell, w.cell_start, w.scan_ws, st);
    if (rc) return rc;
    fill<int>(w.cursor, ncell, 0, st);
    rg_scatter_kernel<<<matris_blocks(n, 256), 256, 0, st>>>(n, w);
    rg_count_wave_kernel<<<(unsigned)n, 64, 0, st>>>(n, plan, w, cutoff, tol, row_count);
    MATRIS_CHECK_LAUNCH();
    return scan_exclusive<int32_t, int64_t>(row_count, n, row_ptr, w.scan_ws, st);
}

extern "C" int matris_radius_graph_fill(int64_t n, const double *lattice_host, double cutoff, double tol,
                                        const int *grid_host, const int *search_host, const int64_t *row_ptr,
                                        int32_t *center, int32_t *neighbor, int32_t *image, double *dist,
                                        void *workspace, size_t workspace_bytes, void *stream) {
    if (n <= 0 || !row_ptr || !center || !neighbor || !image || !dist || !workspace) return MATRIS_E_ARG;
    if (workspace_bytes < matris_radius_graph_workspace_bytes(n, grid_host)) return MATRIS_E_ARG;
    RGPlan plan;
    rg_make_plan(lattice_host, grid_host, search_host, &plan);
    int64_t ncell = (int64_t)plan.g[0] * plan.g[1] * plan.g[2];
    RGWork w = rg_carve(workspace, n, ncell);
    rg_fill_wave_kernel<<<(unsigned)n, 64, 0, (hipStream_t)stream>>>(n, plan, w, cutoff, tol, row_ptr, center,
                                                                       neighbor, image, dist);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

// ------------------------------------------------------------------------------------
// G1 from a Verlet-skin candidate list.  The candidates are a radius graph built at
// cutoff + skin (canonical order, rows by center); dk[n,3] is each atom's integer frame
// jump since then (the wrap of its fractional coordinates).  The candidate (i, j, n) is
// the pair (i, j, n + dk_j - dk_i) in the current frame: the shift is one vector per
// (i, j) group, so the group's image order is kept.  The decision is the builder's own
// (frac_to_cart_d, pair_dist_d, tol < d <= cutoff), and a stable compaction keeps the
// canonical order: when every atom moved less than skin / 2 the result is the radius
// graph a fresh build at cutoff returns, edge for edge.
// ------------------------------------------------------------------------------------
__device__ __forceinline__ bool skin_accept(int64_t e, const double *__restrict__ frac, const double *L,
                                            const int32_t *__restrict__ cc, const int32_t *__restrict__ cn,
                                            const int32_t *__restrict__ ci, const int32_t *__restrict__ dk,
                                            double cutoff, double tol, int *img, double *dist) {
    const int i = cc[e], j = cn[e];
    double fi[3] = {frac[3 * i], frac[3 * i + 1], frac[3 * i + 2]};
    double fj[3] = {frac[3 * j], frac[3 * j + 1], frac[3 * j + 2]};
    double ri[3], rj[3];
    frac_to_cart_d(fi, L, ri);
    frac_to_cart_d(fj, L, rj);
#pragma unroll
    for (int k = 0; k < 3; ++k) img[k] = ci[3 * e + k] + dk[3 * j + k] - dk[3 * i + k];
    const double d = pair_dist_d(ri, rj, L, img[0], img[1], img[2]);
    *dist = d;
    return d <= cutoff && d > tol;
}

__global__ void skin_flag_kernel(int64_t n_cand, const double *__restrict__ frac, RGPlan plan,
                                 const int32_t *__restrict__ cc, const int32_t *__restrict__ cn,
                                 const int32_t *__restrict__ ci, const int32_t *__restrict__ dk, double cutoff,
                                 double tol, int32_t *__restrict__ flag) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_cand) return;
    int img[3];
    double d;
    flag[e] = skin_accept(e, frac, plan.L, cc, cn, ci, dk, cutoff, tol, img, &d) ? 1 : 0;
}

// row_ptr[i] = pos[cand_row_ptr[i]] (i = 0..n); row_count[i] = its difference
__global__ void skin_rows_kernel(int64_t n, const int64_t *__restrict__ cand_row_ptr,
                                 const int64_t *__restrict__ pos, int64_t *__restrict__ row_ptr,
                                 int32_t *__restrict__ row_count) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i > n) return;
    row_ptr[i] = pos[cand_row_ptr[i]];
    if (i < n) row_count[i] = (int32_t)(pos[cand_row_ptr[i + 1]] - pos[cand_row_ptr[i]]);
}

__global__ void skin_fill_kernel(int64_t n_cand, const double *__restrict__ frac, RGPlan plan,
                                 const int32_t *__restrict__ cc, const int32_t *__restrict__ cn,
                                 const int32_t *__restrict__ ci, const int32_t *__restrict__ dk, double cutoff,
                                 double tol, const int64_t *__restrict__ pos, int32_t *__restrict__ center,
                                 int32_t *__restrict__ neighbor, int32_t *__restrict__ image,
                                 double *__restrict__ dist) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_cand) return;
    const int64_t o = pos[e];
    if (pos[e + 1] == o) return;  // rejected by the count pass (same decision)
    int img[3];
    double d;
    skin_accept(e, frac, plan.L, cc, cn, ci, dk, cutoff, tol, img, &d);
    center[o] = cc[e];
    neighbor[o] = cn[e];
    image[3 * o] = img[0];
    image[3 * o + 1] = img[1];
    image[3 * o + 2] = img[2];
    dist[o] = d;
}

extern "C" size_t matris_skin_filter_workspace_bytes(int64_t n_cand) {
    if (n_cand < 0) return 0;
    return align256(sizeof(int32_t) * (size_t)(n_cand + 1)) + align256(sizeof(int64_t) * (size_t)(n_cand + 1)) +
           scan_workspace_bytes(n_cand) + 256;
}

static bool skin_args_ok(int64_t n, int64_t n_cand, const double *frac, const double *lattice_host,
                         const int32_t *cc, const int32_t *cn, const int32_t *ci, const int32_t *dk, void *ws,
                         size_t ws_bytes) {
    return n > 0 && n_cand >= 0 && frac && lattice_host && dk && ws &&
           (n_cand == 0 || (cc && cn && ci)) && ws_bytes >= matris_skin_filter_workspace_bytes(n_cand);
}

extern "C" int matris_skin_filter_count(int64_t n, int64_t n_cand, const double *frac, const double *lattice_host,
                                        double cutoff, double tol, const int32_t *cand_center,
                                        const int32_t *cand_neighbor, const int32_t *cand_image,
                                        const int64_t *cand_row_ptr, const int32_t *dk, int32_t *row_count,
                                        int64_t *row_ptr, void *workspace, size_t workspace_bytes, void *stream) {
    if (!skin_args_ok(n, n_cand, frac, lattice_host, cand_center, cand_neighbor, cand_image, dk, workspace,
                      workspace_bytes) ||
        !cand_row_ptr || !row_count || !row_ptr || !(cutoff > 0))
        return MATRIS_E_ARG;
    hipStream_t st = (hipStream_t)stream;
    RGPlan plan;
    memcpy(plan.L, lattice_host, sizeof(plan.L));
    char *p = (char *)workspace;
    int32_t *flag = (int32_t *)p;
    p += align256(sizeof(int32_t) * (size_t)(n_cand + 1));
    int64_t *pos = (int64_t *)p;
    p += align256(sizeof(int64_t) * (size_t)(n_cand + 1));
    if (n_cand > 0)
        skin_flag_kernel<<<matris_blocks(n_cand, 256), 256, 0, st>>>(n_cand, frac, plan, cand_center, cand_neighbor,
                                                                      cand_image, dk, cutoff, tol, flag);
    int rc = scan_exclusive<int32_t, int64_t>(flag, n_cand, pos, p, st);
    if (rc) return rc;
    skin_rows_kernel<<<matris_blocks(n + 1, 256), 256, 0, st>>>(n, cand_row_ptr, pos, row_ptr, row_count);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_skin_filter_fill(int64_t n, int64_t n_cand, const double *frac, const double *lattice_host,
                                       double cutoff, double tol, const int32_t *cand_center,
                                       const int32_t *cand_neighbor, const int32_t *cand_image, const int32_t *dk,
                                       int32_t *center, int32_t *neighbor, int32_t *image, double *dist,
                                       void *workspace, size_t workspace_bytes, void *stream) {
    if (!skin_args_ok(n, n_cand, frac, lattice_host, cand_center, cand_neighbor, cand_image, dk, workspace,
                      workspace_bytes) ||
        !center || !neighbor || !image || !dist || !(cutoff > 0))
        return MATRIS_E_ARG;
    if (n_cand == 0) return 0;
    RGPlan plan;
    memcpy(plan.L, lattice_host, sizeof(plan.L));
    const int64_t *pos = (const int64_t *)((char *)workspace + align256(sizeof(int32_t) * (size_t)(n_cand + 1)));
    skin_fill_kernel<<<matris_blocks(n_cand, 256), 256, 0, (hipStream_t)stream>>>(
        n_cand, frac, plan, cand_center, cand_neighbor, cand_image, dk, cutoff, tol, pos, center, neighbor, image,
        dist);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

// ------------------------------------------------------------------------------------
// G3/G4: pairing (canonical order makes the reverse edge a binary search in its row)
// ------------------------------------------------------------------------------------
__device__ __forceinline__ int cmp_key(int ja, const int32_t *ia, int jb, int n0, int n1, int n2) {
    if (ja != jb) return ja < jb ? -1 : 1;
    if (ia[0] != n0) return ia[0] < n0 ? -1 : 1;
    if (ia[1] != n1) return ia[1] < n1 ? -1 : 1;
    if (ia[2] != n2) return ia[2] < n2 ? -1 : 1;
    return 0;
}

__global__ void pair_rev_kernel(int64_t n_atoms, int64_t E, const int32_t *__restrict__ center,
                                const int32_t *__restrict__ neighbor, const int32_t *__restrict__ image,
                                const int64_t *__restrict__ row_ptr, int32_t *__restrict__ rev,
                                int32_t *__restrict__ creator, int *__restrict__ err) {
    int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= E) return;
    int c = center[k], nb = neighbor[k];
    const int32_t *im = image + 3 * k;
    // canonical order check against the previous edge
    if (k > 0) {
        int pc = center[k - 1];
        if (pc > c || (pc == c && cmp_key(neighbor[k - 1], image + 3 * (k - 1), nb, im[0], im[1], im[2]) >= 0))
            atomicOr(err, 2);
    }
    if (nb < 0 || nb >= n_atoms || c < 0 || c >= n_atoms) {
        atomicOr(err, 4);
        rev[k] = -1;
        creator[k] = 0;
        return;
    }
    int64_t lo = row_ptr[nb], hi = row_ptr[nb + 1] - 1, found = -1;
    while (lo <= hi) {
        int64_t mid = (lo + hi) >> 1;
        int r = cmp_key(neighbor[mid], image + 3 * mid, c, -im[0], -im[1], -im[2]);
        if (r == 0) { found = mid; break; }
        if (r < 0) lo = mid + 1; else hi = mid - 1;
    }
    rev[k] = (int32_t)found;
    if (found < 0) atomicOr(err, 1);
    creator[k] = (found < 0 || found > k) ? 1 : 0;
}

__global__ void pair_assign_kernel(int64_t E, const int32_t *__restrict__ rev, const int32_t *__restrict__ creator,
                                   const int32_t *__restrict__ uid, int32_t *__restrict__ d2u,
                                   int32_t *__restrict__ u2d, int32_t *__restrict__ u_second) {
    int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= E) return;
    int r = rev[k];
    int64_t owner = (creator[k] || r < 0) ? k : r;
    int u = uid[owner];
    d2u[k] = u;
    if (creator[k]) {
        u2d[u] = (int32_t)k;
        u_second[u] = r;
    }
}

extern "C" size_t matris_pair_edges_workspace_bytes(int64_t E) {
    return 2 * align256(sizeof(int32_t) * (E + 1)) + scan_workspace_bytes(E) + 512;
}

extern "C" int matris_pair_edges(int64_t n_atoms, int64_t E, const int32_t *center, const int32_t *neighbor,
                                 const int32_t *image, const int64_t *row_ptr, int32_t *rev, int32_t *d2u,
                                 int32_t *u2d, int32_t *u_second, int64_t *n_undirected_host, void *workspace,
                                 size_t workspace_bytes, void *stream) {
    if (E <= 0 || !center || !neighbor || !image || !row_ptr || !rev || !d2u || !u2d || !u_second || !workspace ||
        !n_undirected_host)
        return MATRIS_E_ARG;
    if (workspace_bytes < matris_pair_edges_workspace_bytes(E) || E >= INT32_MAX) return MATRIS_E_ARG;
    hipStream_t st = (hipStream_t)stream;
    char *p = (char *)workspace;
    int32_t *creator = (int32_t *)p; p += align256(sizeof(int32_t) * (E + 1));
    int32_t *uid = (int32_t *)p; p += align256(sizeof(int32_t) * (E + 1));
    int *err = (int *)p; p += 256;
    void *scan_ws = p;
    fill<int>(err, 1, 0, st);
    pair_rev_kernel<<<matris_blocks(E, 256), 256, 0, st>>>(n_atoms, E, center, neighbor, image, row_ptr, rev, creator,
                                                           err);
    int rc = scan_exclusive<int32_t, int32_t>(creator, E, uid, scan_ws, st);
    if (rc) return rc;
    pair_assign_kernel<<<matris_blocks(E, 256), 256, 0, st>>>(E, rev, creator, uid, d2u, u2d, u_second);
    MATRIS_CHECK_LAUNCH();
    int host[2] = {0, 0};
    hipError_t e = hipMemcpyAsync(&host[0], err, sizeof(int), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipMemcpyAsync(&host[1], uid + E, sizeof(int32_t), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return (int)e;
    *n_undirected_host = host[1];
    if (host[0] & 2) return MATRIS_E_ORDER;
    if (host[0] & 4) return MATRIS_E_ARG;
    if (host[0] & 1) return MATRIS_E_UNPAIRED;
    return 0;
}

// ------------------------------------------------------------------------------------
// G5: line graph
// ------------------------------------------------------------------------------------
__global__ void lg_short_count_kernel(int64_t n_atoms, const int64_t *__restrict__ row_ptr,
                                      const double *__restrict__ dist, double cutoff, int32_t *__restrict__ c_short) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_atoms) return;
    int c = 0;
    for (int64_t e = row_ptr[i]; e < row_ptr[i + 1]; ++e) c += dist[e] < cutoff ? 1 : 0;
    c_short[i] = c;
}

__global__ void lg_bond_count_kernel(int64_t n_u, const int32_t *__restrict__ center,
                                     const int32_t *__restrict__ neighbor, const double *__restrict__ dist,
                                     const int32_t *__restrict__ u2d, const int32_t *__restrict__ u_second,
                                     const int32_t *__restrict__ c_short, double cutoff, int32_t *__restrict__ cnt,
                                     int *__restrict__ err) {
    int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= n_u) return;
    int k = u2d[u], rk = u_second[u];
    int v = 0;
    if (!(dist[k] > cutoff)) {  // inclusive (radiusgraph.py:450)
        if (rk < 0) {
            atomicOr(err, 1);
        } else {
            v = (c_short[center[k]] - (dist[k] < cutoff ? 1 : 0)) + (c_short[neighbor[k]] - (dist[rk] < cutoff ? 1 : 0));
        }
    }
    cnt[u] = v;
}

__global__ void lg_fill_kernel(int64_t n_u, const int32_t *__restrict__ center, const int32_t *__restrict__ neighbor,
                               const double *__restrict__ dist, const int64_t *__restrict__ row_ptr,
                               const int32_t *__restrict__ d2u, const int32_t *__restrict__ u2d,
                               const int32_t *__restrict__ u_second, double cutoff,
                               const int32_t *__restrict__ angle_ptr, int32_t *__restrict__ lg) {
    int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= n_u) return;
    int64_t o = angle_ptr[u], end = angle_ptr[u + 1];
    if (o == end) return;
    int k = u2d[u], rk = u_second[u];
    int ends[2] = {center[k], neighbor[k]};
    int des[2] = {k, rk};
    for (int s = 0; s < 2; ++s) {
        int c = ends[s], de = des[s];
        for (int64_t e = row_ptr[c]; e < row_ptr[c + 1]; ++e) {
            if (e == de) continue;
            if (dist[e] < cutoff) {  // strict (radiusgraph.py:477)
                int32_t *row = lg + 5 * o;
                row[0] = c;
                row[1] = (int32_t)u;
                row[2] = de;
                row[3] = d2u[e];
                row[4] = (int32_t)e;
                ++o;
            }
        }
    }
}

extern "C" size_t matris_line_graph_workspace_bytes(int64_t n_atoms, int64_t n_u) {
    return align256(sizeof(int32_t) * (n_atoms + 1)) + align256(sizeof(int32_t) * (n_u + 1)) + 256 +
           scan_workspace_bytes(n_u) + 256;
}

extern "C" int matris_line_graph_count(int64_t n_atoms, int64_t E, int64_t n_u, const int32_t *center,
                                       const int32_t *neighbor, const double *dist, const int64_t *row_ptr,
                                       const int32_t *u2d, const int32_t *u_second, double cutoff,
                                       int32_t *angle_ptr, int64_t *n_angles_host, void *workspace,
                                       size_t workspace_bytes, void *stream) {
    if (n_atoms <= 0 || n_u <= 0 || !angle_ptr || !n_angles_host || !workspace) return MATRIS_E_ARG;
    if (workspace_bytes < matris_line_graph_workspace_bytes(n_atoms, n_u)) return MATRIS_E_ARG;
    hipStream_t st = (hipStream_t)stream;
    char *p = (char *)workspace;
    int32_t *c_short = (int32_t *)p; p += align256(sizeof(int32_t) * (n_atoms + 1));
    int32_t *cnt = (int32_t *)p; p += align256(sizeof(int32_t) * (n_u + 1));
    int *err = (int *)p; p += 256;
    void *scan_ws = p;
    fill<int>(err, 1, 0, st);
    lg_short_count_kernel<<<matris_blocks(n_atoms, 256), 256, 0, st>>>(n_atoms, row_ptr, dist, cutoff, c_short);
    lg_bond_count_kernel<<<matris_blocks(n_u, 256), 256, 0, st>>>(n_u, center, neighbor, dist, u2d, u_second, c_short,
                                                                  cutoff, cnt, err);
    int rc = scan_exclusive<int32_t, int32_t>(cnt, n_u, angle_ptr, scan_ws, st);
    if (rc) return rc;
    int64_t total = 0;
    int h_err = 0;
    int64_t *sums = (int64_t *)scan_ws;
    int64_t tiles = (n_u + SCAN_TILE - 1) / SCAN_TILE;
    if (tiles < 1) tiles = 1;
    hipError_t e = hipMemcpyAsync(&total, sums + tiles, sizeof(int64_t), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipMemcpyAsync(&h_err, err, sizeof(int), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return (int)e;
    if (h_err) return MATRIS_E_UNPAIRED;
    if (total >= INT32_MAX / 5) return MATRIS_E_CAPACITY;
    *n_angles_host = total;
    return 0;
}

extern "C" int matris_line_graph_fill(int64_t n_atoms, int64_t E, int64_t n_u, const int32_t *center,
                                      const int32_t *neighbor, const double *dist, const int64_t *row_ptr,
                                      const int32_t *d2u, const int32_t *u2d, const int32_t *u_second, double cutoff,
                                      const int32_t *angle_ptr, int32_t *line_graph, void *stream) {
    if (n_u <= 0 || !angle_ptr || !line_graph) return MATRIS_E_ARG;
    lg_fill_kernel<<<matris_blocks(n_u, 256), 256, 0, (hipStream_t)stream>>>(n_u, center, neighbor, dist, row_ptr,
                                                                             d2u, u2d, u_second, cutoff, angle_ptr,
                                                                             line_graph);
    MATRIS_CHECK_LAUNCH();
    return 0;
}

// ------------------------------------------------------------------------------------
// stable CSR builder
// ------------------------------------------------------------------------------------
__global__ void csr_hist_kernel(int64_t n, const int32_t *__restrict__ keys, int64_t ks, int64_t nseg,
                                int *__restrict__ cnt, unsigned *__restrict__ err, unsigned err_bit) {
    int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= n) return;
    int k = keys[r * ks];
    if (k < 0 || k >= nseg) {
        atomicOr(err, err_bit);
        return;
    }
    atomicAdd(&cnt[k], 1);
}

__global__ void csr_scatter_kernel(int64_t n, const int32_t *__restrict__ keys, int64_t ks, int64_t nseg,
                                   const int32_t *__restrict__ rowptr, int *__restrict__ cursor,
                                   int32_t *__restrict__ tmp) {
    int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= n) return;
    int k = keys[r * ks];
    if (k < 0 || k >= nseg) return;
    tmp[rowptr[k] + atomicAdd(&cursor[k], 1)] = (int32_t)r;
}

// One wave per segment: rank-by-count places rows ascending (keys are unique row ids).
__global__ void csr_sort_kernel(int64_t nseg, const int32_t *__restrict__ rowptr, const int32_t *__restrict__ tmp,
                                int32_t *__restrict__ perm) {
    int64_t s = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x / 64);
    if (s >= nseg) return;
    int lane = threadIdx.x & 63;
    int b = rowptr[s], e = rowptr[s + 1];
    for (int i = b + lane; i < e; i += 64) {
        int v = tmp[i];
        int rank = 0;
        for (int q = b; q < e; ++q) rank += tmp[q] < v ? 1 : 0;
        perm[b + rank] = v;
    }
}

// Row pointers of keys already in ascending order (no permutation): thread i in [0, n]
// writes rowptr[s] = i for the segments s in (key[i-1], key[i]] (key[-1] = -1, key[n] =
// nseg).  A key outside [0, nseg) or a descent sets err_bit; every value written is a row
// position in [0, n] and rowptr is zero-filled first, so even then no reader goes out of
// bounds.
__global__ void csr_sorted_kernel(int64_t n, const int32_t *__restrict__ keys, int64_t ks, int64_t nseg,
                                  int32_t *__restrict__ rowptr, unsigned *__restrict__ err, unsigned err_bit) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i > n) return;
    const int64_t kp = i > 0 ? (int64_t)keys[(i - 1) * ks] : -1;
    const int64_t k = i < n ? (int64_t)keys[i * ks] : nseg;
    if ((i < n && (k < 0 || k >= nseg)) || kp > k) atomicOr(err, err_bit);
    const int64_t s1 = min(k, nseg);
    for (int64_t s = max(kp + 1, (int64_t)0); s <= s1; ++s) rowptr[s] = (int32_t)i;
}

extern "C" size_t matris_csr_workspace_bytes(int64_t n_rows, int64_t nseg) {
    return align256(sizeof(int) * (nseg + 1)) + align256(sizeof(int32_t) * (n_rows + 1)) + 256 +
           scan_workspace_bytes(nseg) + 256;
}

// Histogram, scan, scatter and per-segment sort on `stream`; out-of-range keys are not
// placed and set err_bit in *err.  perm NULL: the keys are ascending, rowptr only.
static int csr_build_launch(int64_t n_rows, const int32_t *keys, int64_t key_stride, int64_t nseg, int32_t *rowptr,
                            int32_t *perm, void *workspace, size_t workspace_bytes, unsigned *err, unsigned err_bit,
                            hipStream_t st) {
    if (n_rows < 0 || nseg <= 0 || !rowptr || !workspace || (n_rows > 0 && !keys)) return MATRIS_E_ARG;
    if (workspace_bytes < matris_csr_workspace_bytes(n_rows, nseg) || n_rows >= INT32_MAX) return MATRIS_E_ARG;
    if (!perm) {
        fill<int32_t>(rowptr, nseg + 1, 0, st);
        csr_sorted_kernel<<<matris_blocks(n_rows + 1, 256), 256, 0, st>>>(n_rows, keys, key_stride, nseg, rowptr,
                                                                          err, err_bit);
        MATRIS_CHECK_LAUNCH();
        return 0;
    }
    char *p = (char *)workspace;
    int *cnt = (int *)p; p += align256(sizeof(int) * (nseg + 1));
    int32_t *tmp = (int32_t *)p; p += align256(sizeof(int32_t) * (n_rows + 1));
    p += 256;  // (the synchronous form's error word)
    void *scan_ws = p;
    fill<int>(cnt, nseg, 0, st);
    if (n_rows > 0)
        csr_hist_kernel<<<matris_blocks(n_rows, 256), 256, 0, st>>>(n_rows, keys, key_stride, nseg, cnt, err, err_bit);
    int rc = scan_exclusive<int, int32_t>(cnt, nseg, rowptr, scan_ws, st);
    if (rc) return rc;
    if (n_rows > 0) {
        fill<int>(cnt, nseg, 0, st);
        csr_scatter_kernel<<<matris_blocks(n_rows, 256), 256, 0, st>>>(n_rows, keys, key_stride, nseg, rowptr, cnt,
                                                                       tmp);
        csr_sort_kernel<<<matris_blocks(nseg, 4), 256, 0, st>>>(nseg, rowptr, tmp, perm);
    }
    MATRIS_CHECK_LAUNCH();
    return 0;
}

extern "C" int matris_csr_build(int64_t n_rows, const int32_t *keys, int64_t key_stride, int64_t nseg,
                                int32_t *rowptr, int32_t *perm, void *workspace, size_t workspace_bytes,
                                void *stream) {
    if (n_rows < 0 || nseg <= 0 || !workspace || workspace_bytes < matris_csr_workspace_bytes(n_rows, nseg))
        return MATRIS_E_ARG;
    hipStream_t st = (hipStream_t)stream;
    char *p = (char *)workspace;
    p += align256(sizeof(int) * (nseg + 1)) + align256(sizeof(int32_t) * (n_rows + 1));
    unsigned *err = (unsigned *)p;
    fill<unsigned>(err, 1, 0u, st);
    int rc = csr_build_launch(n_rows, keys, key_stride, nseg, rowptr, perm, workspace, workspace_bytes, err, 1u, st);
    if (rc) return rc;
    unsigned h_err = 0;
    hipError_t e = hipMemcpyAsync(&h_err, err, sizeof(h_err), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return (int)e;
    return h_err ? MATRIS_E_ARG : 0;
}

extern "C" int matris_csr_build_deferred(int64_t n_rows, const int32_t *keys, int64_t key_stride, int64_t nseg,
                                         int32_t *rowptr, int32_t *perm, void *workspace, size_t workspace_bytes,
                                         void *stream) {
    unsigned *status = matris_range_flag();
    if (!status) return MATRIS_E_ARG;
    return csr_build_launch(n_rows, keys, key_stride, nseg, rowptr, perm, workspace, workspace_bytes, status,
                            (unsigned)MATRIS_STATUS_CSR_KEY, (hipStream_t)stream);
}

// ------------------------------------------------------------------------------------
// matris_csr_build_noalloc: matris_csr_build_deferred with its workspace carved from a
// file-scope device array instead of a caller allocation.  Each device holds its own copy
// of the array (MATRIS_CSR_SCRATCH_BYTES) from the library's first use on it until the
// process ends; its address on a device is taken once, with that device current, and kept
// per device.  Host code never passes the array's name to a kernel or a copy: on the host
// it is a stand-in symbol, not a device address.
// ------------------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[MATRIS_CSR_SCRATCH_BYTES];

static void *csr_scratch_ptr() {
    static std::mutex mu;
    static void *ptr[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (!ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
        ptr[dev] = p;
    }
    return ptr[dev];
}

extern "C" int matris_csr_build_noalloc(int64_t n_rows, const int32_t *keys, int64_t key_stride, int64_t nseg,
                                        int32_t *rowptr, int32_t *perm, void *stream) {
    if (n_rows < 0 || nseg <= 0) return MATRIS_E_ARG;
    const size_t need = matris_csr_workspace_bytes(n_rows, nseg);
    if (need > (size_t)MATRIS_CSR_SCRATCH_BYTES) return MATRIS_E_SCRATCH;
    unsigned *status = matris_range_flag();
    void *ws = csr_scratch_ptr();
    if (!status || !ws) return MATRIS_E_ARG;
    // csr_build_launch zero-fills what must start at zero (the counts) with a kernel on
    // `stream`, so the previous call's contents never leak into this one.
    return csr_build_launch(n_rows, keys, key_stride, nseg, rowptr, perm, ws, need, status,
                            (unsigned)MATRIS_STATUS_CSR_KEY, (hipStream_t)stream);
}
