/*
 * Harness around the reference's own C pairing routine -- TEST INFRASTRUCTURE ONLY.
 *
 * The reference source is compiled where it lies (the Makefile passes its directory with
 * -I; nothing is copied): matris/graph/fast_converter_libraries/create_graph.c together
 * with its vendored uthash.h.  This file only flattens the structures create_graph()
 * returns (create_graph.c:59-66) into plain arrays, the same way the reference's Cython
 * bridge walks them (matris/graph/cygraph.pyx:86-172), and frees them afterwards.
 */
#include "create_graph.c"

/* Returns E_u.  d2u[E], u_de[2*E_u] (second slot -1 if absent), u_nde[E_u],
 * node_ptr[n+1], node_edges[E] (per node: neighbour groups in get_neighbors() order,
 * each group's directed edges in stored order). */
long ref_pair_edges(long E, long *center, long *neighbor, long *image, double *dist, long n,
                    long *d2u, long *u_de, long *u_nde, long *node_ptr, long *node_edges) {
    ReturnElems2 *r = create_graph(center, E, neighbor, image, dist, n);
    for (long k = 0; k < r->num_directed_edges; ++k)
        d2u[r->directed_edges_list[k]->index] = r->directed_edges_list[k]->undirected_edge_index;
    for (long u = 0; u < r->num_undirected_edges; ++u) {
        UndirectedEdge *ue = r->undirected_edges_list[u];
        u_nde[u] = ue->num_directed_edges;
        u_de[2 * u] = ue->directed_edge_indices[0];
        u_de[2 * u + 1] = ue->num_directed_edges > 1 ? ue->directed_edge_indices[1] : -1;
    }
    long w = 0;
    node_ptr[0] = 0;
    for (long i = 0; i < r->num_nodes; ++i) {
        LongToDirectedEdgeList **nb = get_neighbors(&r->nodes[i]);
        for (long j = 0; j < r->nodes[i].num_neighbors; ++j)
            for (int q = 0; q < nb[j]->num_directed_edges_in_group; ++q)
                node_edges[w++] = nb[j]->directed_edges_list[q]->index;
        free(nb);
        node_ptr[i + 1] = w;
    }
    long nu = r->num_undirected_edges;
    for (long k = 0; k < r->num_directed_edges; ++k) free(r->directed_edges_list[k]);
    for (long u = 0; u < r->num_undirected_edges; ++u) {
        free(r->undirected_edges_list[u]->directed_edge_indices);
        free(r->undirected_edges_list[u]);
    }
    free_LongToDirectedEdgeList_in_nodes(r->nodes, r->num_nodes);
    free(r->directed_edges_list);
    free(r->undirected_edges_list);
    free(r->nodes);
    free(r);
    return nu;
}
