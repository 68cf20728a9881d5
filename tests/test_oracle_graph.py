"""Pins of the C graph oracle (oracle/graph_oracle.c) -- CPU only.

  * pairing vs the reference's own create_graph.c, compiled in place (oracle/_ref) and
    recorded in tests/golden/lg_cases.npz;
  * line graph vs the reference's Python Graph.line_graph_adjacency_list
    (radiusgraph.py:412-487) recorded in the golden fixtures;
  * neighbour list vs closed-form fcc shell counts, (i,j,n)<->(j,i,-n) symmetry and an
    independent numpy brute force on tiny cells.
"""
import numpy as np
import pytest

from matris_amd import workloads as W
from oracle import graph_ref


def test_c1_closed_forms():
    cr = W.c1_cu4()
    g = graph_ref.build_graph(cr.frac, cr.lattice, cr.z)
    # 12 neighbours at a/sqrt2 = 3.84 A and 6 self images at 5.43 A per atom
    assert len(g["center"]) == 72 and len(g["u2d"]) == 36
    assert np.bincount(g["center"]).tolist() == [18] * 4
    d = np.sort(np.unique(np.round(g["dist"], 6)))
    assert np.allclose(d, [5.43 / np.sqrt(2), 5.43])
    # each atom has 12 short (< 4 A) directed edges -> 12 x 11 ordered pairs per atom
    assert len(g["line_graph"]) == 528


def test_c3_noiseless_closed_forms():
    cr = W.fcc_supercell(3.61, 6)
    g = graph_ref.build_graph(cr.frac, cr.lattice, cr.z)
    # fcc shells within 6 A: 12 + 6 + 24 + 12 + 24 = 78 neighbours per atom
    assert len(g["center"]) == 864 * 78
    # 12 + 6 short (< 4 A) directed edges per atom -> 18 x 17 ordered pairs per atom
    assert len(g["line_graph"]) == 864 * 18 * 17


def _np_neighbors(frac, lat, r, tol=1e-8, span=3):
    """Independent brute force (numpy, fp64, minimum-free image loop)."""
    cart = frac @ lat
    out = []
    rng = range(-span, span + 1)
    for i in range(len(frac)):
        for j in range(len(frac)):
            for a in rng:
                for b in rng:
                    for c in rng:
                        d = cart[j] + np.array([a, b, c]) @ lat - cart[i]
                        dd = np.sqrt(d @ d)
                        if tol < dd <= r:
                            out.append((i, j, a, b, c))
    return out


@pytest.mark.parametrize("seed,n", [(5, 2), (6, 3)])
def test_neighbor_list_vs_numpy_bruteforce(seed, n):
    rng = np.random.default_rng(seed)
    cr = W.random_cell(rng, n)
    c, nb, im, d = graph_ref.neighbor_list(cr.frac, cr.lattice, 6.0)
    ref = _np_neighbors(cr.frac, cr.lattice, 6.0, span=6)
    got = list(zip(c.tolist(), nb.tolist(), *im.T.tolist()))
    assert sorted(ref) == got  # same set, and the oracle emits canonical (sorted) order


def test_neighbor_list_symmetry():
    rng = np.random.default_rng(7)
    cr = W.random_cell(rng, 9)
    c, nb, im, d = graph_ref.neighbor_list(cr.frac, cr.lattice, 6.0)
    key = {(a, b, *x): k for k, (a, b, x) in enumerate(zip(c.tolist(), nb.tolist(), im.tolist()))}
    for (a, b, x0, x1, x2), k in key.items():
        r = key[(b, a, -x0, -x1, -x2)]
        assert d[r] == d[k]  # bit-identical fp64 distances


def test_pairing_matches_reference_c(golden):
    z = golden("lg_cases.npz")
    for name in ("cscl4", "sc3"):
        d2u, u_de, _ = graph_ref.pair_edges(z[f"{name}_center"], z[f"{name}_neighbor"], z[f"{name}_image"])
        assert np.array_equal(d2u, z[f"{name}_cref_d2u"])
        assert np.array_equal(u_de, z[f"{name}_cref_u_de"])
    cells = golden("cells_small.npz")
    for i in range(int(cells["n_cells"])):
        d2u, u_de, _ = graph_ref.pair_edges(cells[f"g{i}_center"], cells[f"g{i}_neighbor"], cells[f"g{i}_image"])
        assert np.array_equal(d2u, z[f"cell{i}_cref_d2u"])
        assert np.array_equal(u_de, z[f"cell{i}_cref_u_de"])
        ptr, edges = graph_ref.node_edge_order(len(cells[f"g{i}_z"]), cells[f"g{i}_center"], cells[f"g{i}_neighbor"])
        assert np.array_equal(ptr, z[f"cell{i}_cref_node_ptr"])
        assert np.array_equal(edges, z[f"cell{i}_cref_node_edges"])


@pytest.mark.skipif(not graph_ref.ref_available(), reason="oracle/_ref not built (no /root/reference)")
def test_pairing_matches_reference_c_live():
    """Live comparison with the reference create_graph() on shuffled edge lists, where
    insertion order differs from the canonical one."""
    rng = np.random.default_rng(3)
    for n in (4, 7, 12):
        cr = W.random_cell(rng, n)
        c, nb, im, d = graph_ref.neighbor_list(cr.frac, cr.lattice, 6.0)
        p = rng.permutation(len(c))
        c, nb, im, d = c[p], nb[p], im[p], d[p]
        ours = graph_ref.pair_edges(c, nb, im)
        ref = graph_ref.ref_pair_edges(n, c, nb, im, d)
        assert np.array_equal(ours[0], ref[0]) and np.array_equal(ours[1], ref[1])
        assert np.array_equal(ours[2], ref[2])
        ptr, edges = graph_ref.node_edge_order(n, c, nb)
        assert np.array_equal(ptr, ref[3]) and np.array_equal(edges, ref[4])


def test_line_graph_matches_reference_python(golden):
    for fixture, prefixes in (("c1_cu4.npz", ["g_"]), ("cells_small.npz", ["g0_", "g1_", "g2_"]),
                              ("lg_cases.npz", ["cscl4_", "sc3_"])):
        z = golden(fixture)
        for p in prefixes:
            d2u, u_de, u_nde = graph_ref.pair_edges(z[p + "center"], z[p + "neighbor"], z[p + "image"])
            assert np.array_equal(d2u, z[p + "d2u"]) and np.array_equal(u_de[:, 0], z[p + "u2d"])
            lg = graph_ref.line_graph(len(z[p + "z"]), z[p + "center"], z[p + "neighbor"], z[p + "dist"], d2u, u_de,
                                      u_nde, 4.0)
            assert np.array_equal(lg, z[p + "line_graph"]), (fixture, p)


def test_line_graph_cutoff_semantics(golden):
    """Bonds of exactly 4.0 A are first bonds (inclusive, radiusgraph.py:450) but never
    partners (strict, :477): the cscl4 line graph is not closed under swapping."""
    z = golden("lg_cases.npz")
    lg, dist = z["cscl4_line_graph"], z["cscl4_dist"]
    assert (dist[lg[:, 2]] == 4.0).any() and not (dist[lg[:, 4]] == 4.0).any()
    swapped = {(r[0], r[3], r[4], r[1], r[2]) for r in lg.tolist()}
    assert swapped != {tuple(r) for r in lg.tolist()}


def test_unpaired_edge_raises_like_reference_assert():
    # an edge without its reverse keeps a one-edge bond; the reference asserts in the
    # line-graph builder (radiusgraph.py:457-464)
    c = np.array([0, 1, 0]); nb = np.array([1, 0, 1]); im = np.array([[0, 0, 0], [0, 0, 0], [1, 0, 0]])
    d2u, u_de, nde = graph_ref.pair_edges(c, nb, im)
    assert nde.tolist() == [2, 1]
    with pytest.raises(ValueError):
        graph_ref.line_graph(2, c, nb, np.array([1.0, 1.0, 2.0]), d2u, u_de, nde, 4.0)
