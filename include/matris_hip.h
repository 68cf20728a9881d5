/*
 * matris_hip.h -- C ABI of the MI355X (gfx950) MatRIS efsm hot path.
 *
 * Library: matris_amd/csrc/libmatris_hip.so (hipcc --offload-arch=gfx950).
 *
 * Conventions (every entry point):
 *   - returns 0 on success, a hipError_t value (> 0) on a HIP failure, or a negative
 *     MATRIS_E_* code when an argument is rejected before any launch;
 *   - all array pointers are DEVICE pointers unless the parameter name ends in `_host`;
 *   - nothing here allocates or frees device memory: callers pass outputs and, where
 *     stated, a workspace of the size the matching *_workspace_bytes() call returns;
 *   - kernels are enqueued on `stream` (a hipStream_t) and are not synchronised;
 *   - feature rows are fp32, 128 wide, row-major and contiguous unless a leading
 *     dimension is given; graph indices are int32.
 *
 * Each declaration names the reference interface it replaces (paths relative to the
 * HPC-AI-Team/MatRIS tree).
 */
#ifndef MATRIS_HIP_H
#define MATRIS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MATRIS_E_ARG (-1001)       /* invalid size / pointer argument            */
#define MATRIS_E_CAPACITY (-1002)  /* per-atom neighbour capacity exceeded        */
#define MATRIS_E_IMAGES (-1003)    /* periodic image range beyond +-511           */
#define MATRIS_E_UNPAIRED (-1004)  /* a directed edge has no reverse partner      */
#define MATRIS_E_ORDER (-1005)     /* edges not in canonical (center, neighbor, image) order */
#define MATRIS_E_SCRATCH (-1006)   /* the call needs more than the library's static scratch */

/* Library version / build identification (for tests: "is the HIP path loaded"). */
const char *matris_version(void);

/* ------------------------------------------------------------------------------------
 * Graph construction (rows G1-G5)
 * ------------------------------------------------------------------------------------ */

/* G1: periodic radius graph.  Replaces pymatgen Structure.get_neighbor_list(r, sites,
 * numerical_tol) as called at matris/graph/converter.py:85-87.  Edges (i, j, n) with
 * tol < |r_j + n.L - r_i| <= cutoff, emitted in canonical order (i, j, n0, n1, n2
 * ascending), all decisions in fp64 with a fixed evaluation order.
 * The structure is periodic along all three axes (a pymatgen Structure always is; the
 * calculator pads non-periodic axes, matris/applications/base.py:70-93).
 * Two phases: count (per-atom counts and their exclusive scan row_ptr[n+1]) then fill.
 *   frac [n,3] fp64 (device); lattice_host [3][3] fp64, rows are lattice vectors;
 *   grid_host[3] = cells per axis, search_host[3] = cell reach per axis (from
 *   matris_radius_graph_plan); workspace of matris_radius_graph_workspace_bytes(). */
int matris_radius_graph_plan(const double *lattice_host, double cutoff, int *grid_host, int *search_host);
size_t matris_radius_graph_workspace_bytes(int64_t n, const int *grid_host);
int matris_radius_graph_count(int64_t n, const double *frac, const double *lattice_host, double cutoff, double tol,
                              const int *grid_host, const int *search_host, int32_t *row_count, int64_t *row_ptr,
                              void *workspace, size_t workspace_bytes, void *stream);
int matris_radius_graph_fill(int64_t n, const double *lattice_host, double cutoff, double tol, const int *grid_host,
                             const int *search_host, const int64_t *row_ptr, int32_t *center, int32_t *neighbor,
                             int32_t *image, double *dist, void *workspace, size_t workspace_bytes, void *stream);

/* G1 by Verlet-skin reuse (no counterpart in the reference, whose MD driver rebuilds the
 * graph every step, matris/applications/base.py:96-97; it replaces that per-step
 * get_neighbor_list call when the atoms moved less than skin / 2).  The candidates are a
 * matris_radius_graph_count/fill result at cutoff + skin (cand_* [n_cand], rows by center,
 * cand_row_ptr [n+1]); dk [n,3] int32 is each atom's integer frame jump since that build
 * (floor of its fractional coordinates now minus then, i.e. the wrap).  Edges are
 * re-decided with the builder's fp64 expression on the current frac and compacted stably,
 * so the output equals matris_radius_graph_count/fill at cutoff on the same frac, edge for
 * edge, whenever every atom moved less than skin / 2 (the caller checks that).  Two phases,
 * as the builder: count (row_count, row_ptr; row_ptr[n] = E) then fill, with the same
 * workspace of matris_skin_filter_workspace_bytes(n_cand). */
size_t matris_skin_filter_workspace_bytes(int64_t n_cand);
int matris_skin_filter_count(int64_t n, int64_t n_cand, const double *frac, const double *lattice_host, double cutoff,
                             double tol, const int32_t *cand_center, const int32_t *cand_neighbor,
                             const int32_t *cand_image, const int64_t *cand_row_ptr, const int32_t *dk,
                             int32_t *row_count, int64_t *row_ptr, void *workspace, size_t workspace_bytes,
                             void *stream);
int matris_skin_filter_fill(int64_t n, int64_t n_cand, const double *frac, const double *lattice_host, double cutoff,
                            double tol, const int32_t *cand_center, const int32_t *cand_neighbor,
                            const int32_t *cand_image, const int32_t *dk, int32_t *center, int32_t *neighbor,
                            int32_t *image, double *dist, void *workspace, size_t workspace_bytes, void *stream);

/* G3/G4: directed -> undirected pairing.  Replaces create_graph()
 * (matris/graph/fast_converter_libraries/create_graph.c:100-219) and the Python
 * Graph.add_edge / adjacency_list / undirected2directed (matris/graph/radiusgraph.py:
 * 298-410, 489-496) for edge lists in canonical order (as emitted by G1; checked).
 * Outputs: rev[E] (index of the reverse edge), d2u[E], u2d[E_u] (first directed edge),
 * u_second[E_u] (second directed edge); *n_undirected_host receives E_u (one readback).
 * workspace: matris_pair_edges_workspace_bytes(E). */
size_t matris_pair_edges_workspace_bytes(int64_t n_edges);
int matris_pair_edges(int64_t n_atoms, int64_t n_edges, const int32_t *center, const int32_t *neighbor,
                      const int32_t *image, const int64_t *row_ptr, int32_t *rev, int32_t *d2u, int32_t *u2d,
                      int32_t *u_second, int64_t *n_undirected_host, void *workspace, size_t workspace_bytes,
                      void *stream);

/* G5: bond -> angle line graph.  Replaces Graph.line_graph_adjacency_list(cutoff)
 * (matris/graph/radiusgraph.py:412-487): bonds with length <= cutoff (inclusive) as
 * first bond, partners with length < cutoff (strict), rows [center, u1, DE1, u2, DE2].
 * angle_ptr[E_u+1] is the exclusive scan of per-bond angle counts, i.e. the CSR of the
 * angles grouped by u1 (rows are emitted sorted by u1).
 * count: fills angle_ptr and *n_angles_host (one readback).  fill: writes line_graph. */
size_t matris_line_graph_workspace_bytes(int64_t n_atoms, int64_t n_undirected);
int matris_line_graph_count(int64_t n_atoms, int64_t n_edges, int64_t n_undirected, const int32_t *center,
                            const int32_t *neighbor, const double *dist, const int64_t *row_ptr,
                            const int32_t *u2d, const int32_t *u_second, double cutoff, int32_t *angle_ptr,
                            int64_t *n_angles_host, void *workspace, size_t workspace_bytes, void *stream);
int matris_line_graph_fill(int64_t n_atoms, int64_t n_edges, int64_t n_undirected, const int32_t *center,
                           const int32_t *neighbor, const double *dist, const int64_t *row_ptr,
                           const int32_t *d2u, const int32_t *u2d, const int32_t *u_second, double cutoff,
                           const int32_t *angle_ptr, int32_t *line_graph, void *stream);

/* CSR of rows grouped by an int32 key (stable: rows ascending within each segment).
 * Used for every gather's backward (the deterministic replacement of index_add_,
 * matris/model/functions.py:156-157) and for the source side of the segment softmax
 * (functions.py:110-123).  keys may be strided (key of row r = keys[r * key_stride]).
 * workspace: matris_csr_workspace_bytes(n_rows, n_segments).  perm NULL: the caller
 * guarantees ascending keys, and only rowptr is built (one pass over the keys); a descent
 * is reported like an out-of-range key. */
size_t matris_csr_workspace_bytes(int64_t n_rows, int64_t n_segments);
int matris_csr_build(int64_t n_rows, const int32_t *keys, int64_t key_stride, int64_t n_segments,
                     int32_t *rowptr, int32_t *perm, void *workspace, size_t workspace_bytes, void *stream);
/* matris_csr_build without its host read: a key outside [0, nseg) is left out and sets
 * MATRIS_STATUS_CSR_KEY in the device status word (matris_status_take) instead of
 * returning MATRIS_E_ARG, so a model evaluation's groupings cost no stream syncs. */
int matris_csr_build_deferred(int64_t n_rows, const int32_t *keys, int64_t key_stride, int64_t nseg,
                              int32_t *rowptr, int32_t *perm, void *workspace, size_t workspace_bytes,
                              void *stream);
/* matris_csr_build_deferred that allocates nothing and takes no workspace: for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  It has no counterpart in the reference.  Its
 * workspace is a static device array of MATRIS_CSR_SCRATCH_BYTES per device, held from
 * the library's first use on that device until the process ends; a call whose
 * matris_csr_workspace_bytes(n_rows, nseg) exceeds it returns MATRIS_E_SCRATCH before any
 * launch (48 MiB covers n_rows + n_segments up to about 12.5 M, e.g. the 9.0 M angles
 * and 0.95 M bonds of a 32,000-atom cell).  Every call on one device shares that device's
 * array: calls that overlap on one device (two streams, or two host threads) race, so
 * callers order them on one stream.  Results, errors (MATRIS_STATUS_CSR_KEY) and launches
 * are those of matris_csr_build_deferred. */
#define MATRIS_CSR_SCRATCH_BYTES (48u << 20)
int matris_csr_build_noalloc(int64_t n_rows, const int32_t *keys, int64_t key_stride, int64_t nseg,
                             int32_t *rowptr, int32_t *perm, void *stream);

/* ------------------------------------------------------------------------------------
 * Segmented reductions and gathers (row M3)
 * ------------------------------------------------------------------------------------ */

/* out[s, :] = (accumulate ? out[s, :] : 0) + scale * sum_{i in [rowptr[s], rowptr[s+1])}
 *             x[(perm ? perm[i] : i) * ldx + col_off + :128]
 * Replaces aggregate() / GraphPooling (matris/model/functions.py:129-160, 340-365):
 * index_add_ with average=False (scale 1) or the d2u mean (scale 0.5), summed in a
 * fixed CSR order -- deterministic, no atomics.  ldx and col_off multiples of 4 (16-byte
 * aligned rows). */
int matris_seg_sum(const float *x, int64_t ldx, int64_t col_off, const int32_t *rowptr, const int32_t *perm,
                   int64_t n_seg, float scale, int accumulate, float *out, void *stream);

/* out[s, :] = (accumulate ? out[s, :] : 0) + scale_a * (segment sum of source a)
 *             + scale_b * (segment sum of source b) [+ base_w * base[s, :]],
 * source b optional (xb NULL): two index_add_ calls into one output (the target- and
 * source-side scatters of a gathered GatedMLP input, interaction_block.py:96-100 /
 * functions.py:129-160) in one pass.  Both groupings have n_seg segments.  rows_hint (the
 * rows of the larger grouping) selects one work-group per segment for long segments
 * (>= 32 rows on average) instead of one wave.  base (optional, [n_seg, 128], with
 * base_w [128]) adds a residual term, the `de + res_weight * edge_feat` of
 * interaction_block.py:274-275 (order: the sums, then + base_w * base, then + out).
 * Same order-fixed, atomic-free sums as matris_seg_sum. */
int matris_seg_sum2(int64_t n_seg, int64_t rows_hint, const float *xa, int64_t lda, int64_t offa,
                    const int32_t *rowptr_a, const int32_t *perm_a, float scale_a, const float *xb, int64_t ldb,
                    int64_t offb, const int32_t *rowptr_b, const int32_t *perm_b, float scale_b, int accumulate,
                    const float *base, const float *base_w, float *out, void *stream);

/* matris_seg_sum2 whose first source holds tile-run partial sums (the output of
 * matris_gmlp_bwd_runs): its rows ascend by segment (rowptr_a, no permutation) and
 * segment s = rows [rs, re) adds only row rs and each later multiple of tile_a below re
 * -- one partial per tile of tile_a rows that the segment spans -- instead of every row.
 * The second source (xb may be NULL) is summed as in matris_seg_sum2.  Completes the
 * reference's aggregate / index_add_ of a gathered source's gradient (functions.py:
 * 131-160) when its rows were pre-summed inside the GatedMLP backward's tiles. */
int matris_seg_sum2_runs(int64_t n_seg, int64_t rows_hint, const float *xa, int64_t lda, int64_t offa,
                         const int32_t *rowptr_a, int tile_a, float scale_a, const float *xb, int64_t ldb,
                         int64_t offb, const int32_t *rowptr_b, const int32_t *perm_b, float scale_b, int accumulate,
                         float *out, void *stream);

/* The readout (model.py:238-244 readout_norm; readout.py:18-75 EnergyHead with
 * mlp_hidden_dims (128, 128); readout.py:77-133 MagmomHead with hidden 256) on n node rows
 * x [n, 128] (16-byte aligned), fused per row:
 *   nrm = x rsqrt(mean(x^2) + eps) wn          (nn.RMSNorm(128); eps its own or fp32 epsilon)
 *   e   = w3 . SiLU(W2 SiLU(W1 nrm + b1) + b2) + b3          -> e [n]
 *   m   = | w5 . SiLU(W4 nrm + b4) + b5 |                     -> m [n]
 * with w1t = W1^T, w2t = W2^T ([128][128] row-major), w4t = W4^T ([128][256]), w3 [128],
 * w5 [256], b1, b2 [128], b4 [256], b3 and b5 device scalars.
 * matris_readout_bwd: g_x [n, 128] (+)= d(sum_r g_e[r] e[r]) / dx, the energy branch's
 * backward (the magmom head is not differentiated), recomputing the forward of its rows;
 * w1, w2 the untransposed [128][128] weights.  fp32 sums in a fixed order. */
int matris_readout_fwd(int64_t n, const float *x, const float *wn, const float *w1t, const float *b1,
                       const float *w2t, const float *b2, const float *w3, const float *b3, const float *w4t,
                       const float *b4, const float *w5, const float *b5, float eps, float *e, float *m,
                       void *stream);
int matris_readout_bwd(int64_t n, const float *x, const float *wn, const float *w1t, const float *b1,
                       const float *w1, const float *w2t, const float *b2, const float *w2, const float *w3,
                       float eps, const float *g_e, int accumulate, float *g_x, void *stream);

/* out[s, :] = sum over rows r in [rowptr[s], rowptr[s+1]) of x[r, :] for narrow rows
 * (x, out row-major with `width` floats per row, 1 <= width <= 32), summed in a fixed order
 * (no atomics): the per-graph pooling of a batch's atom energies (functions.py:340-365,
 * GraphPooling, readout.py:70-75) and the per-graph sums of its strain and lattice
 * gradients (processgraph.py:169-199, the backward of the per-graph broadcasts). */
int matris_seg_sum_narrow(int64_t n_seg, const int32_t *rowptr, const float *x, int width, float *out,
                          void *stream);

/* out[r, :] = (accumulate ? out[r, :] : 0) + scale * src[idx ? idx[r] : r, :]
 * torch.index_select(x, 0, idx) (interaction_block.py:96-100) and the backward of a
 * segment sum. */
int matris_gather_rows(const float *src, const int32_t *idx, int64_t n_rows, float scale, int accumulate,
                       float *out, void *stream);

/* Envelope weighting of the atom-graph Refinement (interaction_block.py:243-258 with
 * is_atom_graph: w = env[d2u]; aggregate(h * w, target)) without materialising h * w:
 *   matris_seg_sum_mul: out[s, :] = (accumulate ? out[s, :] : 0) + scale *
 *     sum_{rows r of segment s} x[r, col_off:col_off+128] * mul[mul_idx[r], :]
 *     (the product first, then the order-fixed segment sum of matris_seg_sum2; mul
 *     [*, 128] rows; mul_idx NULL: row r's own index; rows_hint as in matris_seg_sum2);
 *   matris_gather_mul: out[r, :] = (accumulate ? out[r, :] : 0) + a[ia[r], :] * b[ib[r], :]
 *     (an index may be NULL for the identity).
 * The refinement's backward is g_h = g_edge_ffn + g_agg[tgt] * env[d2u] (gather_mul) and
 * g_env = segment sums over d2u of h * g_agg[tgt] (seg_sum_mul). */
int matris_seg_sum_mul(int64_t n_seg, int64_t rows_hint, const float *x, int64_t ldx, int64_t col_off,
                       const int32_t *rowptr, const int32_t *perm, const float *mul, const int32_t *mul_idx,
                       float scale, int accumulate, float *out, void *stream);
int matris_gather_mul(int64_t n_rows, const float *a, const int32_t *ia, const float *b, const int32_t *ib,
                      int accumulate, float *out, void *stream);
/* matris_seg_sum_mul for short segments (rows_hint <= 4 n_seg, e.g. the two directed
 * copies of each bond) with each segment's sum projected onto the learnable envelope's
 * basis instead of written: proj_out[s, k] = sum_c sum_s[c] proj_wt[k, c] ([n_seg, proj_k],
 * proj_k <= 8, proj_wt the Linear(proj_k, 128) weight transposed, [proj_k, 128] row-major,
 * 16-byte aligned; accumulate: added to proj_out).  The atom-graph Refinement's g_env =
 * sum_{d2u} h * g_agg[tgt] goes straight to the input gradient of learnable_envelope
 * (interaction_block.py:240-241), accumulated over the blocks that share the basis. */
int matris_seg_sum_mul_proj(int64_t n_seg, int64_t rows_hint, const float *x, int64_t ldx, int64_t col_off,
                            const int32_t *rowptr, const int32_t *perm, const float *mul, const int32_t *mul_idx,
                            float scale, const float *proj_wt, int proj_k, int accumulate, float *proj_out,
                            void *stream);

/* Backward of the edge vectors vec[e] = cart[tgt[e]] - (cart[src[e]] + shift[e])
 * (row P1, matris/model/processgraph.py:192-199): g_cart [n_atoms, 3] fp32 =
 * sum over the atom's target rows of g_vec [E, 3] minus the sum over its source rows,
 * through the CSR groupings of tgt and src (perm NULL = identity).  Deterministic;
 * replaces the sort-based backward of the two index_select gathers. */
int matris_edge_vec_bwd(int64_t n_atoms, const float *g_vec, const int32_t *t_ptr, const int32_t *t_perm,
                        const int32_t *s_ptr, const int32_t *s_perm, float *g_cart, void *stream);

/* Cartesian positions of one graph (row P1, matris/model/processgraph.py:87,
 * atom_frac_coord @ lattice): cart[i, j] = sum_k frac[i, k] lattice[k, j] (frac, cart
 * [n, 3], lattice [3, 3], fp32), and, with strain_zero non-NULL, strain_zero[0 .. 8] = 0
 * (the zero strain of processgraph.py:173-177, which the stress differentiates against). */
int matris_frac_to_cart(int64_t n, const float *frac, const float *lattice, float *cart, float *strain_zero,
                        void *stream);

/* The same for a disjoint batch of graphs (row P1, matris/model/processgraph.py:87 per
 * graph, then the batch concatenation of :120-130): atom i of the batch uses the lattice of
 * its graph, cart[i] = frac[i] lattice[graph_of_atom[i]] (frac, cart [n, 3], lattice
 * [n_graphs, 3, 3], graph_of_atom [n] int32), in the same arithmetic as
 * matris_frac_to_cart; with strain_zero non-NULL, strain_zero[0 .. 9 n_graphs - 1] = 0.
 * An index outside [0, n_graphs) sets MATRIS_STATUS_CSR_KEY in the status word
 * (matris_status_take) and leaves that atom's row unwritten.  One launch in place of one
 * [n_g, 3] x [3, 3] product per graph. */
int matris_frac_to_cart_batch(int64_t n, int64_t n_graphs, const float *frac, const float *lattice,
                              const int32_t *graph_of_atom, float *cart, float *strain_zero, void *stream);

/* Edge geometry of one graph with the strain trick (row P1, matris/model/processgraph.py:
 * 169-199: symmetric_strains, the strained positions and lattice, neighbor_pos + image @
 * lattice, edge_vectors, edge_lengths, unit_edge_vectors), forward in one launch.  With
 * sym = (strain + strain^T) / 2 (strain [3,3] fp32, NULL = no strain: sym = 0),
 * x' = cart + cart sym, L' = lattice + lattice sym:
 *   vec[e] = x'[tgt[e]] - (x'[src[e]] + image[e] L')   (cart [N,3], image [E,3] fp32;
 *   tgt, src int32 [E] atom indices), length [E] = |vec|, unit [E,3] = vec / length,
 *   lattice_out [3,3] = L', volume [1] = det(lattice) (unstrained, for the stress). */
int matris_edge_geom_fwd(int64_t n_edges, const float *cart, const float *lattice, const float *strain,
                         const float *image, const int32_t *tgt, const int32_t *src, float *length, float *unit,
                         float *lattice_out, float *volume, void *stream);

/* Blocks of the backward's per-edge pass: its partial array holds 9 * MATRIS_GEOM_PARTS
 * floats at most. */
#define MATRIS_GEOM_PARTS 512

/* Backward of matris_edge_geom_fwd, the autograd chain of processgraph.py:169-199 for the
 * positions and the strain: g_length [E] and g_unit [E,3] (either NULL = zero) give
 * g_vec [E,3] (written out); g_cart [n_atoms,3] = g' + g' sym with g' the sum of g_vec
 * over the atom's target rows minus its source rows (the CSR groupings of tgt and src,
 * perm NULL = identity); g_strain [3,3] (NULL = not needed; needs strain) =
 * sym-part of (cart^T g' - lattice^T sum_e image[e]^T g_vec[e]).  partial: workspace of
 * 9 * MATRIS_GEOM_PARTS floats.  Every sum runs in a fixed order (reproducible). */
int matris_edge_geom_bwd(int64_t n_atoms, int64_t n_edges, const float *g_length, const float *g_unit,
                         const float *length, const float *unit, const float *cart, const float *lattice,
                         const float *strain, const float *image, const int32_t *t_ptr, const int32_t *t_perm,
                         const int32_t *s_ptr, const int32_t *s_perm, float *g_vec, float *partial, float *g_cart,
                         float *g_strain, void *stream);

/* Edge geometry of a disjoint batch of graphs (row P1, processgraph.py:169-199 per graph,
 * as the reference's batched tensors do it), forward in one launch: matris_edge_geom_fwd
 * with edge e using the lattice and strain of its graph graph_of_edge[e] (int32 [E]);
 * lattice [G,3,3], strain [G,3,3] or NULL, lattice_out [G,3,3] (the strained lattices),
 * volume [G] (det of each unstrained lattice); cart [N,3] and tgt / src are the batch's
 * (offset) atom rows.  A graph index outside [0, n_graphs) sets MATRIS_STATUS_CSR_KEY in the
 * status word and leaves that edge's outputs unwritten. */
int matris_edge_geom_fwd_batch(int64_t n_graphs, int64_t n_edges, const float *cart, const float *lattice,
                               const float *strain, const float *image, const int32_t *tgt, const int32_t *src,
                               const int32_t *graph_of_edge, float *length, float *unit, float *lattice_out,
                               float *volume, void *stream);

/* Backward of matris_edge_geom_fwd_batch (three launches): g_vec per edge, g_cart through
 * the CSR groupings of tgt / src as in matris_edge_geom_bwd, then, with a strain, one
 * work-group per graph over its atoms [atom_ptr[g], atom_ptr[g+1]) and edges
 * [edge_ptr[g], edge_ptr[g+1]) (int32 [G+1] each: the batch's graphs are contiguous row
 * ranges) for g_cart's strain term and g_strain [G,3,3] (when non-NULL).  Every sum runs in
 * a fixed order (reproducible). */
int matris_edge_geom_bwd_batch(int64_t n_graphs, int64_t n_atoms, int64_t n_edges, const float *g_length,
                               const float *g_unit, const float *length, const float *unit, const float *cart,
                               const float *lattice, const float *strain, const float *image, const int32_t *t_ptr,
                               const int32_t *t_perm, const int32_t *s_ptr, const int32_t *s_perm,
                               const int32_t *atom_ptr, const int32_t *edge_ptr, float *g_vec, float *g_cart,
                               float *g_strain, void *stream);

/* ------------------------------------------------------------------------------------
 * Segment attention (rows M2 + M4 / M5): Dimwise_softmax by target and by source,
 * alpha * e' and both segment sums, fused.  Replaces interaction_block.py:113-134 with
 * functions.py:97-160.
 *   alpha_t / alpha_s: logits, row r at (alpha_idx ? alpha_idx[r] : r) * lda;
 *   e [R,128]; target CSR (t_ptr, t_perm|NULL), source CSR (s_ptr, s_perm|NULL),
 *   both over n_seg segments.
 * fwd writes y_t, y_s [n_seg,128] (zero rows for empty segments) and the per-segment
 * log-sum-exp lse_t, lse_s [n_seg,128] needed by the backward (rows of empty segments,
 * which no row of the backward reads, are left unwritten).
 * lda (and ldgy) are multiples of 4 (16-byte aligned rows).
 * bwd (input gradients only): given g_yt, g_ys (rows of stride ldgy >= 128), writes
 * g_alpha_t, g_alpha_s [R,128] (per row r, before any alpha_idx reduction) and
 * g_e [R,128] (= g_e_base + the attention term when g_e_base is non-NULL; g_e_base may
 * alias g_e); t_idx[R], s_idx[R] are the target / source segment of each row. */
int matris_attn_fwd(int64_t n_rows, int64_t n_seg, const float *alpha_t, const float *alpha_s, int64_t lda,
                    const int32_t *alpha_idx, const float *e, const int32_t *t_ptr, const int32_t *t_perm,
                    const int32_t *s_ptr, const int32_t *s_perm, float *y_t, float *y_s, float *lse_t,
                    float *lse_s, void *stream);
int matris_attn_bwd(int64_t n_rows, int64_t n_seg, const float *alpha_t, const float *alpha_s, int64_t lda,
                    const int32_t *alpha_idx, const float *e, const int32_t *t_idx, const int32_t *s_idx,
                    const float *y_t, const float *y_s, const float *lse_t, const float *lse_s, const float *g_yt,
                    const float *g_ys, int64_t ldgy, float *g_alpha_t, float *g_alpha_s, float *g_e,
                    const float *g_e_base, void *stream);
/* The atom-graph matris_attn_bwd by undirected bond (interaction_block.py:104-134 with
 * is_atom_graph: the logits W bond are per bond, read by both directed copies through
 * d2u): alpha_t / alpha_s [n_bond, lda] per bond, the directed rows of bond u are the d2u
 * CSR segment u (u_ptr [n_bond+1], u_perm or NULL); t_idx / s_idx, e and g_e per directed
 * row.  g_alpha_t / g_alpha_s [n_bond,128] are the sums over each bond's rows (the d2u
 * reduction of matris_attn_bwd's per-row outputs) and g_e = base_scale * g_base[bond] +
 * the attention term (g_base [n_bond,128] or NULL). */
int matris_attn_bwd_bond(int64_t n_bond, const float *alpha_t, const float *alpha_s, int64_t lda, const float *e,
                         const int32_t *u_ptr, const int32_t *u_perm, const int32_t *t_idx, const int32_t *s_idx,
                         const float *y_t, const float *y_s, const float *lse_t, const float *lse_s,
                         const float *g_yt, const float *g_ys, int64_t ldgy, const float *g_base, float base_scale,
                         float *g_alpha_t, float *g_alpha_s, float *g_e, void *stream);

/* Envelope-weighted aggregation of the line-graph Refinement (interaction_block.py:243-258:
 * smooth_weight = env[source] * env[target]; aggregate(h * smooth_weight, target)):
 *   S[b] = sum_{a: tgt(a)=b} h[a] * env[src(a)],  agg[b] = env[b] * S[b]   (n_seg = rows of env)
 * with the target CSR (t_ptr, t_perm|NULL) and s_idx = source of each row.
 * bwd: g_h[a] = (accumulate ? g_h[a] : 0) + g_agg[tgt(a)] * env[tgt(a)] * env[src(a)];
 *      g_env[b] = g_agg[b] * S[b] + sum_{a: src(a)=b} g_agg[tgt(a)] * env[tgt(a)] * h[a]
 * (source CSR s_ptr, s_perm|NULL; t_idx = target of each row). */
int matris_env_agg_fwd(int64_t n_seg, const float *h, const float *env, const int32_t *t_ptr, const int32_t *t_perm,
                       const int32_t *s_idx, float *S, float *agg, void *stream);
int matris_env_agg_bwd(int64_t n_rows, int64_t n_seg, const float *h, const float *env, const float *g_agg,
                       const float *S, const int32_t *t_idx, const int32_t *s_idx, const int32_t *s_ptr,
                       const int32_t *s_perm, int accumulate, float *g_h, float *g_env, void *stream);
/* g_env of matris_env_agg_bwd alone, plus (g_agg_env non-NULL) the per-bond factor of the
 * g_h term, g_agg_env[b] = g_agg[b] * env[b] (n_seg rows); matris_ffn_bwd_env then adds
 * g_agg_env[tgt(a)] * env[src(a)] to the FFN input gradient it writes, so g_h makes one
 * trip through memory. */
int matris_env_agg_bwd_env(int64_t n_seg, const float *h, const float *env, const float *g_agg, const float *S,
                           const int32_t *t_idx, const int32_t *s_ptr, const int32_t *s_perm, float *g_env,
                           float *g_agg_env, void *stream);
/* matris_env_agg_bwd_env with g_env projected onto the learnable envelope's basis in the
 * same pass: g_basis[b, k] = sum_c g_env[b, c] wt[k, c] ([n_seg, proj_k], proj_k <= 8; wt
 * the Linear(proj_k, 128) weight transposed, row-major [proj_k, 128], 16-byte aligned) --
 * the input gradient of learnable_envelope (interaction_block.py:244), so g_env never
 * reaches memory; accumulate adds it to g_basis (the blocks sharing one basis). */
int matris_env_agg_bwd_env_proj(int64_t n_seg, const float *h, const float *env, const float *g_agg,
                                const float *S, const int32_t *t_idx, const int32_t *s_ptr, const int32_t *s_perm,
                                const float *proj_wt, int proj_k, int accumulate, float *g_basis, float *g_agg_env,
                                void *stream);
/* The learnable envelope itself (interaction_block.py:240-246, nn.Linear(num_basis, 128,
 * bias=False)): env[r, c] = sum_k basis[r, k] wt[k, c], basis [n, k] (k <= 8), wt the
 * weight transposed [k, 128] row-major, env [n, 128] (wt and env 16-byte aligned). */
int matris_env_linear(int64_t n, int k, const float *basis, const float *wt, float *env, void *stream);

/* ------------------------------------------------------------------------------------
 * Basis functions of the embeddings (rows E2, E3), thread per row, with input gradients.
 * ------------------------------------------------------------------------------------ */

/* E2: Bessel basis times the polynomial envelope (matris/model/basis_function.py:8-50,
 * 116-186), out [n, num_radial] with
 *   out[i,k] = env(d_i/cutoff) * (sqrt(2/cutoff) * sin(freq[k] * d_i/cutoff) / d_i),
 *   env(x) = 1 + a x^p + b x^(p+1) + c x^(p+2) (x < 1), 0 otherwise (p = envelope_exponent).
 * bwd: g_dist[i] (+)= sum_k g_out[i,k] d out[i,k] / d d_i (frequency gradients are not
 * produced). */
int matris_bessel_fwd(int64_t n, int num_radial, const float *dist, const float *freq, double cutoff,
                      double envelope_exponent, float *out, void *stream);
int matris_bessel_bwd(int64_t n, int num_radial, const float *dist, const float *freq, double cutoff,
                      double envelope_exponent, const float *g_out, int accumulate, float *g_dist, void *stream);

/* E2 with the edge embedding after it, one row per undirected bond (EdgeBasisEmbedding,
 * matris/model/feature_embed.py:42-148, which evaluates both directed copies and averages
 * them; the copies are equal, so once per bond gives the same values and gradient).
 * Bond u, d = edge_len[u2d[u]] (edge_len [E], u2d int32 [n_bonds]):
 *   rbf6 [n_bonds, 7] = the enveloped Bessel basis at cutoff6 (frequencies freq6),
 *   rbf4 [n_bonds, 7] = the same at cutoff4 (freq4), both written out (they also weight
 *     the atom- and line-graph aggregations),
 *   e = SiLU(LayerNorm(rbf6 W1^T W2^T; ln_g, ln_b, ln_eps) Ws^T)   [n_bonds, 128]
 * with W1 [128, 7] fp32 (edge_linear1), w2p / wsp the packs of edge_linear2 and the swish
 * layer's linear (as matris_ffn_fwd takes them).  num_radial must be 7.  Saves h3 (the
 * pre-activation), xhat (the normalised rows) [n_bonds, 128] and 1/sigma [n_bonds] for
 * the backward. */
int matris_edge_embed_fwd(int64_t n_bonds, const float *edge_len, const int32_t *u2d, const float *freq6,
                          double cutoff6, const float *freq4, double cutoff4, int num_radial,
                          double envelope_exponent, const float *w1, const void *w2p, const float *ln_g,
                          const float *ln_b, double ln_eps, const void *wsp, float *e, float *rbf6, float *rbf4,
                          float *save_h3, float *save_xhat, float *save_rstd, int mode, void *stream);
/* Backward of matris_edge_embed_fwd in the bond lengths: from g_e [n_bonds, 128] and the
 * other readers' g_rbf6, g_rbf4 [n_bonds, 7] (either NULL = zero), writes
 * g_len[u2d[u]] = dL/dd of bond u (the other rows of g_len are left as they are: the
 * caller zeroes them).  w2tp / wstp: the packs of W2^T and Ws^T (as matris_ffn_bwd takes
 * them). */
int matris_edge_embed_bwd(int64_t n_bonds, const float *edge_len, const int32_t *u2d, const float *freq6,
                          double cutoff6, const float *freq4, double cutoff4, int num_radial,
                          double envelope_exponent, const float *w1, const void *w2tp, const float *ln_g,
                          const void *wstp, const float *g_e, const float *g_rbf6, const float *g_rbf4,
                          const float *save_h3, const float *save_xhat, const float *save_rstd, float *g_len,
                          int mode, void *stream);

/* E3: spherical three-body basis (feature_embed.py:183-201, basis_function.py:53-77,
 * 222-338, max_n = max_l = 4): for angle row a with t = de_t[a] (the line graph's
 * target_DE_index) and s = de_s[a] (source_DE_index) into unit [E_d, 3]:
 *   c = (unit[t] . unit[s]) (1 - 1e-6), x = |unit[s]| / cutoff,
 *   out[a, 4n+j] = sqrt(2/cutoff^3) R_{n,j}(x) Y_n(cos(acos c)),  out [A, 16].
 * bwd: g_unit[d] (+)= the gradient of every row that reads unit[d] as t (CSR t_ptr/t_perm
 * of de_t over E_d) or as s (CSR s_ptr/s_perm of de_s), summed in CSR order
 * (deterministic): each row's two contributions are computed once into work
 * [n_angles, 6] (thread per row), then summed per directed edge (thread per edge). */
int matris_sbf_fwd(int64_t n_angles, const float *unit, const int32_t *de_t, const int32_t *de_s, double cutoff,
                   float *out, void *stream);
int matris_sbf_bwd(int64_t n_edges, int64_t n_angles, const float *unit, const int32_t *de_t, const int32_t *de_s,
                   const float *g_basis, const int32_t *t_ptr, const int32_t *t_perm, const int32_t *s_ptr,
                   const int32_t *s_perm, double cutoff, int accumulate, float *work, float *g_unit,
                   void *stream);

/* ------------------------------------------------------------------------------------
 * MFMA arithmetic and packed weights (shared by the gated MLP, FFN and projection pair).
 * `mode` selects the arithmetic (fp32 in, fp32 accumulate in every mode):
 *   MATRIS_MMA_FP32   v_mfma_f32_32x32x2f32 on the fp32 operands;
 *   MATRIS_MMA_BF16X6 operands split exactly into three bf16 parts, six partial
 *                     products on v_mfma_f32_32x32x16_bf16 (fp32-grade accuracy);
 *   MATRIS_MMA_BF16X3 two bf16 parts, three partial products (~2^-16 per product);
 *   MATRIS_MMA_F16X3  activations split into fp16 hi + 2^-11 lo, weights scaled by a
 *                     power of two and split into two fp16 parts, three partial products
 *                     on v_mfma_f32_32x32x16_f16 (~2^-22 per product, fp32-grade).  fp16
 *                     bounds the activations: a kernel that meets |x| >= 65504 in an
 *                     operand it splits sets MATRIS_STATUS_F16_RANGE in the device's
 *                     status word (its results are then unusable; matris_status_take).
 * Every weight operand ("...p" arguments) is passed pre-packed by matris_pack_b in the
 * SAME mode as the call that reads it: a [n, k] row-major fp32 matrix whose rows are the
 * GEMM's output columns (an nn.Linear weight, or the transpose of one for a backward)
 * becomes fragment-major planes of matris_pack_b_bytes(n, k, mode) bytes (n % 32 == 0,
 * k % 16 == 0; 4 bytes per element in modes 0, 2 and 3, 6 in mode 6, plus a 16-byte
 * scale header in mode 2).  No counterpart in the reference: it replaces the per-call
 * weight reads of the nn.Linear layers below.
 * ------------------------------------------------------------------------------------ */
#define MATRIS_MMA_FP32 0
#define MATRIS_MMA_F16X3 2
#define MATRIS_MMA_BF16X3 3
#define MATRIS_MMA_BF16X6 6
size_t matris_pack_b_bytes(int64_t n, int64_t k, int mode);
int matris_pack_b(int64_t n, int64_t k, const float *w, int mode, void *out, void *stream);
/* The device status word: bits set by kernels of this library since the last take.
 *   MATRIS_STATUS_F16_RANGE  a MATRIS_MMA_F16X3 kernel met an activation outside the fp16
 *                            range (its outputs are unusable: redo in MATRIS_MMA_BF16X6);
 *   MATRIS_STATUS_CSR_KEY    matris_csr_build_deferred met a key outside [0, nseg).
 * *bits = the word of the current device, which is then cleared.  Synchronizes `stream`
 * (the kernels to check must have been launched on it or before it).  No counterpart in
 * the reference: it lets one host read per model evaluation replace a read per check. */
#define MATRIS_STATUS_F16_RANGE 1u
#define MATRIS_STATUS_CSR_KEY 2u
int matris_status_take(unsigned *bits, void *stream);

/* ------------------------------------------------------------------------------------
 * Fused gated MLP on MFMA (row M1).  Replaces GatedMLP.forward
 * (matris/model/functions.py:297-311) with its MLP / RMSNorm / FusedSiLU / FusedSigmoid
 * parts (functions.py:163-242, 10-36; op/fused_silu_op.py; op/fuse_sigmoid_op.py) and
 * the torch.cat of gathered rows that feeds it (interaction_block.py:96-107, 232-254).
 *   input row m = concat_j src_j[(src_idx_j ? src_idx_j[m] : m), 0:128], j < n_src
 *   (n_src in {1..4}, K = 128 n_src); src_host / src_idx_host are host arrays of n_src
 *   device pointers (an index pointer may be NULL for the identity);
 *   w1p = pack of [mlp_core.layers.0.weight; mlp_gate.layers.0.weight] ([256, K]), b1 [256];
 *   w2p = pack of [mlp_core.layers.3.weight; mlp_gate.layers.3.weight] ([256, 128]), b2 [256];
 *   norm_c / norm_g [128] = core_norm.weight / gate_norm.weight, RMSNorm eps.
 * fwd writes out [M,128]; save_p / save_z [M,256] (layer-1 pre-activation and layer-2
 * output, both halves) when non-NULL -- the backward needs them; with res_out non-NULL
 * also res_out = out + res_w * res_src (the residual update `out + res_weight * feat`
 * of interaction_block.py:140-141, res_w [128], res_src [M,128]).
 * bwd (input gradients only) reads g_out [M,128], p, z and the packed transposes
 * w1tp = pack of w1^T ([K, 256]) and w2tp = pack of [W2core^T; W2gate^T] ([256, 128]);
 * writes g_x [M,K], or, when g_x0 is non-NULL, source 0's columns to g_x0 [M,128]
 * (added to its contents if acc0) and the rest to g_x [M,K-128] (NULL allowed if K=128).
 * res_w non-NULL adds res_w * g_out to source 0's gradient (backward of res_out when
 * res_src is source 0). */
int matris_gmlp_fwd(int64_t m, int n_src, const float *const *src_host, const int32_t *const *src_idx_host,
                    const void *w1p, const float *b1, const void *w2p, const float *b2, const float *norm_c,
                    const float *norm_g, float eps, float *out, float *save_p, float *save_z,
                    const float *res_src, const float *res_w, float *res_out, int mode, void *stream);
int matris_gmlp_bwd(int64_t m, int k, const float *g_out, const float *p, const float *z, const void *w1tp,
                    const void *w2tp, const float *norm_c, const float *norm_g, float eps, float *g_x, float *g_x0,
                    int acc0, const float *res_w, int mode, void *stream);

/* matris_gmlp_bwd with two options:
 * - run_key (may be NULL): for a gathered source whose index run_key [m] (int32) ascends
 *   with the row (the target bond of angle rows, the centre atom of edge rows), source
 *   block run_blk (its columns 128 run_blk .. +127 of the K; not source 0 when g_x0 is
 *   given) leaves as tile-run partial sums -- within each tile of matris_gmlp_tile_rows()
 *   rows, the sum of every run of equal keys, at the run's first row of g_x; the block's
 *   other rows are not written.  matris_seg_sum2_runs with the same tile size completes the
 *   segment sums (functions.py:131-160) from those partials, reading one row per run
 *   instead of every gathered row.
 * - res_src (may be NULL): the residual term source 0's gradient gains is res_w * res_src
 *   [m,128] instead of res_w * g_out (the residual branch of the layer's output when it
 *   does not pass through this GatedMLP, e.g. tb' = FFN(h) + r tb).
 * Other sources and outputs are those of matris_gmlp_bwd. */
int matris_gmlp_bwd_runs(int64_t m, int k, const float *g_out, const float *p, const float *z, const void *w1tp,
                         const void *w2tp, const float *norm_c, const float *norm_g, float eps, float *g_x,
                         float *g_x0, int acc0, const float *res_w, const float *res_src, const int32_t *run_key,
                         int run_blk, int mode, void *stream);
/* The GatedMLP backward of a Refinement with the edge_FFN backward in front of it, in
 * one kernel (two-plane modes 0, 2, 3; interaction_block.py:218-278): the output gradient
 * g_out of matris_gmlp_bwd is not read but computed per tile as
 *   g_out = ((G W2) * SiLU'(ffn_p)) W1 + g_agg_env[t_idx] * env[s_idx]
 * (matris_ffn_bwd_env's g_x; g_agg_env may be NULL for no envelope term), with G the
 * gradient of the FFN's output -- ffn_g [m,128], or with ffn_g_idx (may be NULL) row r of
 * G is ffn_g_scale * ffn_g[ffn_g_idx[r]] (the atom graph: half the bond gradient of each
 * directed copy) -- ffn_p the FFN's saved W1 h and ffn_w1tp / ffn_w2tp the packs
 * matris_ffn_bwd takes.  Source 0's gradient gains res_w * ffn_g (res_w may be NULL; not
 * with ffn_g_idx).  run_key / run_blk as in matris_gmlp_bwd_runs (run_key may be NULL). */
int matris_gmlp_bwd_ffn(int64_t m, int k, const float *p, const float *z, const void *w1tp, const void *w2tp,
                        const float *norm_c, const float *norm_g, float eps, float *g_x, float *g_x0,
                        const float *res_w, const int32_t *run_key, int run_blk, const float *ffn_g,
                        const int32_t *ffn_g_idx, float ffn_g_scale, const float *ffn_p, const void *ffn_w1tp,
                        const void *ffn_w2tp, const float *g_agg_env, const float *env, const int32_t *t_idx,
                        const int32_t *s_idx, int mode, void *stream);
/* matris_gmlp_bwd_runs (two-plane modes 0, 2, 3; g_x0 required, K >= 256) with a
 * projection added to source 0's gradient before it is stored: g_x0 = source 0's
 * gradient + pair_g0 W[0:128] + pair_g1 W[128:256] (+ res_w * res_src), pair_wtp the pack
 * of W^T that matris_pair_bwd takes.  The line graph attention (interaction_block.py:104-
 * 134): its logits are W_s tb and W_t tb of the same angle rows as the edge update's
 * source 0, so their backward lands in the same gradient rows (matris_pair_bwd with
 * accumulate, without the separate read-modify-write of g_x0). */
int matris_gmlp_bwd_pair(int64_t m, int k, const float *g_out, const float *p, const float *z, const void *w1tp,
                         const void *w2tp, const float *norm_c, const float *norm_g, float eps, float *g_x,
                         float *g_x0, const float *res_w, const float *res_src, const int32_t *run_key, int run_blk,
                         const float *pair_g0, const float *pair_g1, const void *pair_wtp, int mode, void *stream);
/* Rows per GatedMLP work-group tile (the tile of matris_gmlp_bwd_runs's partial sums). */
int matris_gmlp_tile_rows(void);

/* GatedMLP forward with the layer-1 product of gathered sources taken before the gather
 * (same layer as matris_gmlp_fwd, GatedMLP.forward in functions.py:297-311, for inputs
 * such as [angle, bond[tgt], bond[src]] whose gathered rows repeat): a source j read
 * through an index costs one product per table row instead of one per output row.
 *   matris_gmlp_project: out [m, 256 n_blk] = x W^T for x [m,128] and W [256 n_blk, 128]
 *     packed by matris_pack_b -- block b of W is W1's column block of one source
 *     ([256, 128]: the core rows, then the gate rows), written to columns 256b .. 256b+255.
 *   matris_gmlp_fwd_proj: matris_gmlp_fwd over the n_src (0..4) sources still multiplied
 *     in place (w1p = pack of W1's columns of those sources, unused when n_src = 0) plus
 *     n_proj (0..3) projected sources: row r of the layer-1 output gains
 *     proj_host[j][proj_idx_host[j][r] * proj_ld_host[j] + c], c < 256 (an index may be
 *     NULL for the identity; row strides >= 256 and multiples of 4; pointers 16-byte
 *     aligned; the three arrays are host arrays of n_proj entries).
 * Outputs and saved p / z are those of matris_gmlp_fwd, so matris_gmlp_bwd with the full
 * W1^T is its backward. */
int matris_gmlp_project(int64_t m, const float *x, const void *wp, int n_blk, float *out, int mode, void *stream);
int matris_gmlp_fwd_proj(int64_t m, int n_src, const float *const *src_host, const int32_t *const *src_idx_host,
                         int n_proj, const float *const *proj_host, const int32_t *const *proj_idx_host,
                         const int64_t *proj_ld_host, const void *w1p, const float *b1, const void *w2p, const float *b2,
                         const float *norm_c, const float *norm_g, float eps, float *out, float *save_p,
                         float *save_z, const float *res_src, const float *res_w, float *res_out, int mode,
                         void *stream);
/* matris_gmlp_fwd_proj (n_src may be 0 when every source is projected, n_proj 0 when none
 * is) with the line Refinement's edge_FFN on the output rows, in the same kernel
 * (interaction_block.py:263-275: tb' = edge_FFN(h) + r_e tb with h this GatedMLP's out):
 *   t = h W1^T (saved to ffn_save_p [m,128] when non-NULL),
 *   ffn_out [m,128] = SiLU(t) W2^T + ffn_res_w * ffn_res   (ffn_res may be NULL: no residual,
 *   as in the atom-graph Refinement, whose residual comes after the d2u mean)
 * with ffn_w1p, ffn_w2p the packs matris_ffn_fwd takes.  out (h) is still written; the
 * GatedMLP residual (res_src / res_w / res_out) is not available here.  Equal to
 * matris_gmlp_fwd_proj followed by matris_ffn_fwd up to the FFN's fp32 sum order. */
int matris_gmlp_fwd_ffn(int64_t m, int n_src, const float *const *src_host, const int32_t *const *src_idx_host,
                        int n_proj, const float *const *proj_host, const int32_t *const *proj_idx_host,
                        const int64_t *proj_ld_host, const void *w1p, const float *b1, const void *w2p,
                        const float *b2, const float *norm_c, const float *norm_g, float eps, float *out,
                        float *save_p, float *save_z, const void *ffn_w1p, const void *ffn_w2p, float *ffn_save_p,
                        const float *ffn_res, const float *ffn_res_w, float *ffn_out, int mode, void *stream);
/* matris_gmlp_fwd_proj with the line graph attention's logit projections of the residual
 * source's rows in the same kernel (interaction_block.py:104-112: source_weight_linear and
 * target_weight_linear applied to the angle rows tb, which are also the edge update's
 * residual, tb' = e + r_e tb):
 *   pair_out0 [m,128] = res_src W[0:128]^T,  pair_out1 [m,128] = res_src W[128:256]^T
 * with pair_wp the pack matris_pair_fwd takes (W = [W_s; W_t]).  Needs the residual
 * (res_src, res_w, res_out).  Equal to matris_gmlp_fwd_proj followed by matris_pair_fwd on
 * res_src. */
int matris_gmlp_fwd_pair(int64_t m, int n_src, const float *const *src_host, const int32_t *const *src_idx_host,
                         int n_proj, const float *const *proj_host, const int32_t *const *proj_idx_host,
                         const int64_t *proj_ld_host, const void *w1p, const float *b1, const void *w2p,
                         const float *b2, const float *norm_c, const float *norm_g, float eps, float *out,
                         float *save_p, float *save_z, const float *res_src, const float *res_w, float *res_out,
                         const void *pair_wp, float *pair_out0, float *pair_out1, int mode, void *stream);

/* ------------------------------------------------------------------------------------
 * Dense layers on MFMA, 128-wide rows, no bias.
 * ------------------------------------------------------------------------------------ */

/* FFN out = W2 SiLU(W1 x): Refinement.node_FFN / edge_FFN, MLP(hidden=int, bias=False)
 * (matris/model/functions.py:198-205, interaction_block.py:198-210, 269-270).
 * w1p, w2p = packs of the [128,128] Linear weights; save_p [M,128] = W1 x (for bwd);
 * res non-NULL: out += res_w * res (the residual update, interaction_block.py:274-275).
 * bwd: g_x = ((g W2) * SiLU'(p)) W1 with w1tp, w2tp = packs of w1^T, w2^T; g_res
 * non-NULL receives res_w * g (gradient of the residual input). */
int matris_ffn_fwd(int64_t m, const float *x, const void *w1p, const void *w2p, float *out, float *save_p,
                   const float *res, const float *res_w, int mode, void *stream);
int matris_ffn_bwd(int64_t m, const float *g, const float *p, const void *w1tp, const void *w2tp, float *g_x,
                   float *g_res, const float *res_w, int mode, void *stream);
/* matris_ffn_bwd plus the envelope term of the line Refinement's hidden-row gradient
 * (interaction_block.py:243-258, 269-270: h feeds both edge_FFN and the envelope-weighted
 * aggregate): g_x[a] = FFN input gradient + g_agg_env[t_idx[a]] * env[s_idx[a]], with
 * g_agg_env from matris_env_agg_bwd_env (the g_h of matris_env_agg_bwd with accumulate,
 * in one kernel and one write). */
int matris_ffn_bwd_env(int64_t m, const float *g, const float *p, const void *w1tp, const void *w2tp, float *g_x,
                       const float *g_agg_env, const float *env, const int32_t *t_idx, const int32_t *s_idx, int mode,
                       void *stream);

/* Attention projection pair (interaction_block.py:33-38, 110-111):
 * out0 = x W[0:128]^T (source_weight_linear), out1 = x W[128:256]^T (target);
 * wp = pack of W = [W_s; W_t] ([256,128]).
 * bwd: g_x = g0 W[0:128] + g1 W[128:256] (+ res_w * res when res is non-NULL), plus
 * g_x's previous contents (added last) when accumulate, with wtp = pack of W^T
 * ([128,256]). */
int matris_pair_fwd(int64_t m, const float *x, const void *wp, float *out0, float *out1, int mode, void *stream);
int matris_pair_bwd(int64_t m, const float *g0, const float *g1, const void *wtp, float *g_x, const float *res,
                    const float *res_w, int accumulate, int mode, void *stream);
/* The line graph attention's backward with its logit projections' backward in one launch
 * (interaction_block.py:104-134: Dimwise_softmax of W_s tb and W_t tb over the angle rows'
 * source and target bonds, then source_weight_linear / target_weight_linear), replacing
 * matris_attn_bwd + matris_pair_bwd on the line graph: per angle row r (t_idx, s_idx its
 * target / source bond, int32),
 *   p_t = exp(alpha_t[r] - lse_t[t]), p_s = exp(alpha_s[r] - lse_s[s]),
 *   g_e[r] = base[r] + p_t g_yt[t] + p_s g_ys[s]                 (as matris_attn_bwd)
 *   g_tb[r] = g_as W[0:128] + g_at W[128:256] + res_w * base[r]  (as matris_pair_bwd)
 * with g_at = p_t g_yt[t] (e[r] - y_t[t]), g_as likewise, which are never written; wtp the
 * pack of W^T ([128,256]) matris_pair_bwd takes.  alpha rows of stride lda, g_y rows of
 * stride ldgy (both >= 128, multiples of 4), other rows 128 floats; base and res_w optional
 * (res_w needs base).  Modes 0, 2, 3 (two fragment planes). */
int matris_attn_pair_bwd(int64_t n_rows, const float *alpha_t, const float *alpha_s, int64_t lda, const float *e,
                         const int32_t *t_idx, const int32_t *s_idx, const float *y_t, const float *y_s,
                         const float *lse_t, const float *lse_s, const float *g_yt, const float *g_ys, int64_t ldgy,
                         const float *base, const void *wtp, const float *res_w, int mode, float *g_e, float *g_tb,
                         void *stream);

/* Three-body embedding (row E3's consumer): tb = SiLU(Ws (Wa b)) for b [m, 16] the angle
 * basis, wa = Wa [128, 16] row-major fp32 (angle_embedding, no bias), wsp = Ws [128, 128]
 * packed by matris_pack_b (SwishLayer linear, no bias) -- ThreebodyEmbedding.forward's
 * angle_embedding + swish_layer (feature_embed.py:151-203, functions.py:70-95).  Backward:
 * g_b = Wa^T (Ws^T (g_tb * SiLU'(z))), z = Ws Wa b recomputed from b; wstp = Ws^T packed.
 * Modes 0, 2, 3 (two fragment planes). */
int matris_tb_embed_fwd(int64_t m, const float *basis, const float *wa, const void *wsp, float *out, int mode,
                        void *stream);
int matris_tb_embed_bwd(int64_t m, const float *basis, const float *g_tb, const float *wa, const void *wsp,
                        const void *wstp, float *g_basis, int mode, void *stream);

/* ------------------------------------------------------------------------------------
 * SiLU derivatives: the reference's torch op library matris_op (op/src/RegisterOp.cpp:
 * 9-13, Opdefine.h:7-10; arithmetic of op/fused_silu_op.py:5-28), element-wise over n
 * floats (any layout, 16-byte vectors when every pointer is aligned):
 *   matris_silu_bwd:      out = dgrad * s'(x)                (fuse_silu_bwd)
 *   matris_silu_grad_bwd: ggo = ggi * s'(x), gx = ggi * go * s''(x)  (fuse_silu_grad_bwd)
 * with s(x) = x sigmoid(x).  torch.ops.matris_op.fuse_silu_bwd / fuse_silu_grad_bwd
 * (matris_amd.torch_ops) wrap them with the reference's schemas. */
int matris_silu_bwd(int64_t n, const float *dgrad, const float *x, float *out, void *stream);
int matris_silu_grad_bwd(int64_t n, const float *ggi, const float *go, const float *x, float *ggo, float *gx,
                         void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MATRIS_HIP_H */
