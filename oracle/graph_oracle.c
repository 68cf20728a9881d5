/*
 * CPU oracle for MatRIS graph construction -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load the
 * library built from this file.  The product path never links it.
 *
 * Three pieces, each a plain restatement of the reference algorithm:
 *
 *  og_neighbor_list  -- the periodic radius graph (row G1).  The reference delegates this
 *      to pymatgen Structure.get_neighbor_list(r, numerical_tol=1e-8)
 *      (matris/graph/converter.py:85-87; pymatgen==2025.10.07, requirements.txt:3), which
 *      is not installed here.  Restated from its published semantics: every (i, j, n)
 *      with |r_j + n.L - r_i| <= r, minus pairs at distance <= tol (the atom itself).
 *      Emission order is canonical (center, neighbor, n0, n1, n2 ascending): pymatgen's
 *      own order is PARITY UNPINNED (no pymatgen, no reference tests).  The edge SET is
 *      pinned by closed-form shell counts and by the (i,j,n) <-> (j,i,-n) symmetry.
 *      All fp64 arithmetic is written out with a fixed evaluation order and no FMA
 *      contraction (build with -ffp-contract=off) so that the GPU kernel, which uses the
 *      same expressions, reproduces every inclusion decision bit-for-bit.
 *
 *  og_pair_edges     -- directed -> undirected pairing (row G3), restating
 *      create_graph.c:100-219 with is_reversed_directed_edge :254-270 and
 *      find_in_undirected :276-299.  Pinned against oracle/_ref (the reference C file
 *      compiled in place) on the same inputs.
 *
 *  og_line_graph     -- bond -> angle line graph (row G5), restating
 *      Graph.line_graph_adjacency_list (matris/graph/radiusgraph.py:412-487) with the
 *      neighbour-group order of create_graph.c:382-423 (uthash insertion order).
 *      Pinned by golden vectors from the reference's radiusgraph.Graph
 *      (tests/golden/) and by closed-form angle counts.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------
 * fp64 geometry with a fixed evaluation order (shared definition with the HIP kernel)
 * ------------------------------------------------------------------------------------ */
static void frac_to_cart(const double *f, const double *L, double *c) {
    for (int k = 0; k < 3; ++k) {
        double t = f[0] * L[0 * 3 + k];
        t = t + f[1] * L[1 * 3 + k];
        t = t + f[2] * L[2 * 3 + k];
        c[k] = t;
    }
}

static double pair_dist(const double *ci, const double *cj, const double *L, long n0, long n1, long n2) {
    double d2 = 0.0;
    for (int k = 0; k < 3; ++k) {
        double s = (double)n0 * L[0 * 3 + k];
        s = s + (double)n1 * L[1 * 3 + k];
        s = s + (double)n2 * L[2 * 3 + k];
        double d = (cj[k] - ci[k]) + s;
        d2 = d2 + d * d;
    }
    return sqrt(d2);
}

/* r / h_k per axis, h_k the interplanar spacing of the planes spanned by the other two
 * lattice vectors.  A displacement with fractional component x_k along axis k has length
 * at least |x_k| h_k, so only images with |df_k + n_k| <= r / h_k can be within r. */
static void reach(const double *L, double r, double *rk) {
    double cr[3][3];
    for (int k = 0; k < 3; ++k) {
        const double *u = L + 3 * ((k + 1) % 3), *v = L + 3 * ((k + 2) % 3);
        cr[k][0] = u[1] * v[2] - u[2] * v[1];
        cr[k][1] = u[2] * v[0] - u[0] * v[2];
        cr[k][2] = u[0] * v[1] - u[1] * v[0];
    }
    double vol = fabs(L[0] * cr[0][0] + L[1] * cr[0][1] + L[2] * cr[0][2]);
    for (int k = 0; k < 3; ++k)
        rk[k] = r / (vol / sqrt(cr[k][0] * cr[k][0] + cr[k][1] * cr[k][1] + cr[k][2] * cr[k][2]));
}

/* Radius graph in canonical order.  Writes at most `cap` edges; returns the total count
 * (call once with cap=0 to size the buffers). */
long og_neighbor_list(long n, const double *frac, const double *lattice, const int *pbc, double r,
                      double tol, long cap, long *center, long *neighbor, long *image, double *dist) {
    double *cart = (double *)malloc(sizeof(double) * 3 * (n > 0 ? n : 1));
    for (long i = 0; i < n; ++i) frac_to_cart(frac + 3 * i, lattice, cart + 3 * i);
    double rk[3];
    reach(lattice, r, rk);
    long count = 0;
    for (long i = 0; i < n; ++i)
        for (long j = 0; j < n; ++j) {
            long lo[3], hi[3];
            for (int k = 0; k < 3; ++k) {
                double df = frac[3 * j + k] - frac[3 * i + k];
                lo[k] = pbc[k] ? (long)ceil(-rk[k] - df - 1e-6) : 0;
                hi[k] = pbc[k] ? (long)floor(rk[k] - df + 1e-6) : 0;
            }
            for (long a = lo[0]; a <= hi[0]; ++a)
                for (long b = lo[1]; b <= hi[1]; ++b)
                    for (long c = lo[2]; c <= hi[2]; ++c) {
                        double d = pair_dist(cart + 3 * i, cart + 3 * j, lattice, a, b, c);
                        if (!(d <= r) || !(d > tol)) continue;
                        if (count < cap) {
                            center[count] = i;
                            neighbor[count] = j;
                            image[3 * count + 0] = a;
                            image[3 * count + 1] = b;
                            image[3 * count + 2] = c;
                            dist[count] = d;
                        }
                        ++count;
                    }
        }
    free(cart);
    return count;
}

/* Cartesian coordinates with the shared evaluation order (exposed for tests). */
void og_frac_to_cart(long n, const double *frac, const double *lattice, double *cart) {
    for (long i = 0; i < n; ++i) frac_to_cart(frac + 3 * i, lattice, cart + 3 * i);
}

/* ------------------------------------------------------------------------------------
 * pairing (create_graph.c:100-219)
 * ------------------------------------------------------------------------------------ */
typedef struct {
    long key_a, key_b;  /* unordered node pair as first inserted */
    long *bonds;        /* undirected ids in creation order */
    long nb, cap;
    int used;
} group_t;

static uint64_t mix64(uint64_t x) {
    x ^= x >> 33; x *= 0xff51afd7ed558ccdULL; x ^= x >> 33; x *= 0xc4ceb9fe1a85ec53ULL; x ^= x >> 33;
    return x;
}

/* Returns the number of undirected bonds E_u.  Outputs (all length E_d, caller-sized):
 *   d2u[k]         undirected id of directed edge k
 *   u_de[2*u+s]    s-th directed edge of bond u (-1 if absent)
 *   u_nde[u]       number of directed edges joined to u (the reference keeps all)  */
long og_pair_edges(long E, const long *center, const long *neighbor, const long *image,
                   long *d2u, long *u_de, long *u_nde) {
    long tsize = 16;
    while (tsize < 2 * E + 16) tsize <<= 1;
    group_t *tab = (group_t *)calloc((size_t)tsize, sizeof(group_t));
    long nu = 0;
    for (long k = 0; k < E; ++k) {
        long c = center[k], nb = neighbor[k];
        long lo = c < nb ? c : nb, hi = c < nb ? nb : c;
        uint64_t h = mix64(((uint64_t)lo << 32) ^ (uint64_t)hi) & (uint64_t)(tsize - 1);
        group_t *g = NULL;
        for (;;) {
            group_t *t = &tab[h];
            if (!t->used) break;
            long tlo = t->key_a < t->key_b ? t->key_a : t->key_b;
            long thi = t->key_a < t->key_b ? t->key_b : t->key_a;
            if (tlo == lo && thi == hi) { g = t; break; }
            h = (h + 1) & (uint64_t)(tsize - 1);
        }
        int joined = 0;
        if (g) {
            for (long q = 0; q < g->nb; ++q) {
                long u = g->bonds[q];
                long e0 = u_de[2 * u]; /* first directed edge of the bond */
                int rev = 1;
                for (int x = 0; x < 3; ++x)
                    if (image[3 * e0 + x] != -image[3 * k + x]) rev = 0;
                if (rev && center[e0] == nb && neighbor[e0] == c) {
                    d2u[k] = u;
                    if (u_nde[u] == 1) u_de[2 * u + 1] = k;
                    u_nde[u] += 1;
                    joined = 1;
                    break;
                }
            }
        }
        if (!joined) {
            long u = nu++;
            d2u[k] = u;
            u_de[2 * u] = k;
            u_de[2 * u + 1] = -1;
            u_nde[u] = 1;
            if (!g) {
                g = &tab[h];
                g->used = 1;
                g->key_a = c;
                g->key_b = nb;
                g->cap = 2;
                g->nb = 0;
                g->bonds = (long *)malloc(sizeof(long) * 2);
            }
            if (g->nb == g->cap) {
                g->cap *= 2;
                g->bonds = (long *)realloc(g->bonds, sizeof(long) * g->cap);
            }
            g->bonds[g->nb++] = u;
        }
    }
    for (long t = 0; t < tsize; ++t)
        if (tab[t].used) free(tab[t].bonds);
    free(tab);
    return nu;
}

/* Order in which Graph.line_graph_adjacency_list visits the directed edges of each node:
 * neighbour keys in order of first appearance (uthash insertion order,
 * create_graph.c:382-423), each key's edges in directed-index order.
 * Outputs node_ptr[n+1] and node_edges[E]. */
void og_node_edge_order(long n, long E, const long *center, const long *neighbor, long *node_ptr,
                        long *node_edges) {
    long *cnt = (long *)calloc((size_t)n + 1, sizeof(long));
    for (long k = 0; k < E; ++k) cnt[center[k] + 1]++;
    node_ptr[0] = 0;
    for (long i = 0; i < n; ++i) node_ptr[i + 1] = node_ptr[i] + cnt[i + 1];
    long *own = (long *)malloc(sizeof(long) * (E > 0 ? E : 1));
    long *fill = (long *)calloc((size_t)n, sizeof(long));
    for (long k = 0; k < E; ++k) {
        long c = center[k];
        own[node_ptr[c] + fill[c]++] = k;
    }
    /* stable grouping by neighbour key in order of first appearance */
    for (long i = 0; i < n; ++i) {
        long b = node_ptr[i], e = node_ptr[i + 1], w = b;
        char *done = (char *)calloc((size_t)(e - b) + 1, 1);
        for (long p = b; p < e; ++p) {
            if (done[p - b]) continue;
            long key = neighbor[own[p]];
            for (long q = p; q < e; ++q)
                if (!done[q - b] && neighbor[own[q]] == key) {
                    node_edges[w++] = own[q];
                    done[q - b] = 1;
                }
        }
        free(done);
    }
    free(own);
    free(fill);
    free(cnt);
}

/* Line graph rows [center, u1, DE1, u2, DE2] (radiusgraph.py:445-486).  Writes at most
 * `cap` rows into lg (5 longs each); returns the total row count, or -1 - u when bond u
 * within the cutoff does not have exactly two directed edges (the reference asserts,
 * radiusgraph.py:457-464, and the converter then keeps an empty line graph,
 * converter.py:99-106). */
long og_line_graph(long n, long E, long nu, const long *center, const long *neighbor, const double *dist,
                   const long *d2u, const long *u_de, const long *u_nde, double cutoff, long cap, long *lg) {
    long *node_ptr = (long *)malloc(sizeof(long) * (n + 1));
    long *node_edges = (long *)malloc(sizeof(long) * (E > 0 ? E : 1));
    og_node_edge_order(n, E, center, neighbor, node_ptr, node_edges);
    long count = 0;
    for (long u = 0; u < nu; ++u) {
        long k = u_de[2 * u];
        if (dist[k] > cutoff) continue; /* inclusive: d == cutoff is kept (:450) */
        if (u_nde[u] != 2) { count = -1 - u; break; }
        long ends[2] = {center[k], neighbor[k]};
        long des[2] = {u_de[2 * u], u_de[2 * u + 1]};
        for (int s = 0; s < 2; ++s) {
            long c = ends[s], de = des[s];
            for (long p = node_ptr[c]; p < node_ptr[c + 1]; ++p) {
                long e = node_edges[p];
                if (e == de) continue;
                if (dist[e] < cutoff) { /* strict (:477) */
                    if (count < cap) {
                        long *row = lg + 5 * count;
                        row[0] = c; row[1] = u; row[2] = de; row[3] = d2u[e]; row[4] = e;
                    }
                    ++count;
                }
            }
        }
    }
    free(node_ptr);
    free(node_edges);
    return count;
}
