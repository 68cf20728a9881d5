"""ctypes front-end of the C graph oracle -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module.  It loads oracle/liboracle_graph.so (our restatement, graph_oracle.c) and, when
present, oracle/_ref/libref_create_graph.so (the reference's create_graph.c compiled in
place by oracle/Makefile).  Function-level citations live in graph_oracle.c.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

_P = ctypes.c_void_p
_L = ctypes.c_long
_D = ctypes.c_double


def build(ref: bool = True) -> None:
    """Compile the oracle (and the reference C file when /root/reference exists)."""
    subprocess.run(["make", "-s", "-C", _HERE, "all"], check=True)
    if ref and os.path.isdir("/root/reference/matris/graph/fast_converter_libraries"):
        subprocess.run(["make", "-s", "-C", _HERE, "ref"], check=True)


def _lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle_graph.so")
        if not os.path.exists(path):
            build(ref=False)
        lib = ctypes.CDLL(path)
        lib.og_neighbor_list.restype = _L
        lib.og_neighbor_list.argtypes = [_L, _P, _P, _P, _D, _D, _L, _P, _P, _P, _P]
        lib.og_pair_edges.restype = _L
        lib.og_pair_edges.argtypes = [_L, _P, _P, _P, _P, _P, _P]
        lib.og_node_edge_order.restype = None
        lib.og_node_edge_order.argtypes = [_L, _L, _P, _P, _P, _P]
        lib.og_line_graph.restype = _L
        lib.og_line_graph.argtypes = [_L, _L, _L, _P, _P, _P, _P, _P, _P, _D, _L, _P]
        lib.og_frac_to_cart.restype = None
        lib.og_frac_to_cart.argtypes = [_L, _P, _P, _P]
        _LIB = lib
    return _LIB


def ref_available() -> bool:
    return os.path.exists(os.path.join(_HERE, "_ref", "libref_create_graph.so"))


def _ref():
    global _REF
    if _REF is None:
        lib = ctypes.CDLL(os.path.join(_HERE, "_ref", "libref_create_graph.so"))
        lib.ref_pair_edges.restype = _L
        lib.ref_pair_edges.argtypes = [_L, _P, _P, _P, _P, _L, _P, _P, _P, _P, _P]
        _REF = lib
    return _REF


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_P)


def frac_to_cart(frac, lattice) -> np.ndarray:
    frac = np.ascontiguousarray(frac, dtype=np.float64)
    lattice = np.ascontiguousarray(lattice, dtype=np.float64)
    out = np.empty_like(frac)
    _lib().og_frac_to_cart(len(frac), _ptr(frac), _ptr(lattice), _ptr(out))
    return out


def neighbor_list(frac, lattice, cutoff: float, pbc=(True, True, True), tol: float = 1e-8):
    """Canonical-order periodic radius graph: (center, neighbor, image[E,3], dist)."""
    frac = np.ascontiguousarray(frac, dtype=np.float64)
    lattice = np.ascontiguousarray(lattice, dtype=np.float64)
    pbc = np.ascontiguousarray(pbc, dtype=np.int32)
    n = len(frac)
    lib = _lib()
    e = lib.og_neighbor_list(n, _ptr(frac), _ptr(lattice), _ptr(pbc), cutoff, tol, 0, None, None, None, None)
    c = np.empty(e, np.int64); nb = np.empty(e, np.int64)
    im = np.empty((e, 3), np.int64); d = np.empty(e, np.float64)
    e2 = lib.og_neighbor_list(n, _ptr(frac), _ptr(lattice), _ptr(pbc), cutoff, tol, e, _ptr(c), _ptr(nb),
                              _ptr(im), _ptr(d))
    assert e2 == e
    return c, nb, im, d


def pair_edges(center, neighbor, image):
    """(d2u[E], u_de[E_u,2], u_nde[E_u]) following create_graph.c:100-219."""
    center = np.ascontiguousarray(center, dtype=np.int64)
    neighbor = np.ascontiguousarray(neighbor, dtype=np.int64)
    image = np.ascontiguousarray(image, dtype=np.int64)
    E = len(center)
    d2u = np.empty(E, np.int64); u_de = np.empty(2 * max(E, 1), np.int64); nde = np.empty(max(E, 1), np.int64)
    nu = _lib().og_pair_edges(E, _ptr(center), _ptr(neighbor), _ptr(image), _ptr(d2u), _ptr(u_de), _ptr(nde))
    return d2u, u_de[: 2 * nu].reshape(nu, 2), nde[:nu]


def node_edge_order(n, center, neighbor):
    center = np.ascontiguousarray(center, dtype=np.int64)
    neighbor = np.ascontiguousarray(neighbor, dtype=np.int64)
    ptr = np.empty(n + 1, np.int64); edges = np.empty(max(len(center), 1), np.int64)
    _lib().og_node_edge_order(n, len(center), _ptr(center), _ptr(neighbor), _ptr(ptr), _ptr(edges))
    return ptr, edges[: len(center)]


def line_graph(n, center, neighbor, dist, d2u, u_de, u_nde, cutoff: float):
    """[A,5] rows (center, u1, DE1, u2, DE2); raises ValueError where the reference asserts."""
    center = np.ascontiguousarray(center, dtype=np.int64)
    neighbor = np.ascontiguousarray(neighbor, dtype=np.int64)
    dist = np.ascontiguousarray(dist, dtype=np.float64)
    d2u = np.ascontiguousarray(d2u, dtype=np.int64)
    u_de = np.ascontiguousarray(u_de, dtype=np.int64).reshape(-1)
    u_nde = np.ascontiguousarray(u_nde, dtype=np.int64)
    lib = _lib()
    args = (n, len(center), len(u_nde), _ptr(center), _ptr(neighbor), _ptr(dist), _ptr(d2u), _ptr(u_de), _ptr(u_nde),
            cutoff)
    a = lib.og_line_graph(*args, 0, None)
    if a < 0:
        raise ValueError(f"undirected bond {-1 - a} does not have two directed edges")
    out = np.empty((max(a, 1), 5), np.int64)
    lib.og_line_graph(*args, a, _ptr(out))
    return out[:a]


def ref_pair_edges(n, center, neighbor, image, dist):
    """The reference create_graph() (oracle/_ref), flattened: (d2u, u_de, u_nde, node_ptr, node_edges)."""
    center = np.ascontiguousarray(center, dtype=np.int64)
    neighbor = np.ascontiguousarray(neighbor, dtype=np.int64)
    image = np.ascontiguousarray(image, dtype=np.int64)
    dist = np.ascontiguousarray(dist, dtype=np.float64)
    E = len(center)
    d2u = np.empty(E, np.int64); u_de = np.empty(2 * max(E, 1), np.int64); nde = np.empty(max(E, 1), np.int64)
    ptr = np.empty(n + 1, np.int64); edges = np.empty(max(E, 1), np.int64)
    nu = _ref().ref_pair_edges(E, _ptr(center), _ptr(neighbor), _ptr(image), _ptr(dist), n, _ptr(d2u), _ptr(u_de),
                               _ptr(nde), _ptr(ptr), _ptr(edges))
    return d2u, u_de[: 2 * nu].reshape(nu, 2), nde[:nu], ptr, edges[:E]


def build_graph(frac, lattice, z, atom_cutoff=6.0, line_cutoff=4.0, pbc=(True, True, True)):
    """Full oracle graph: dict of int64/fp64 numpy arrays in RadiusGraph terms."""
    c, nb, im, d = neighbor_list(frac, lattice, atom_cutoff, pbc)
    d2u, u_de, u_nde = pair_edges(c, nb, im)
    lg = line_graph(len(frac), c, nb, d, d2u, u_de, u_nde, line_cutoff)
    return dict(center=c, neighbor=nb, image=im, dist=d, d2u=d2u, u2d=u_de[:, 0].copy(), u_de=u_de,
                u_nde=u_nde, line_graph=lg, atomic_number=np.asarray(z, np.int64),
                frac=np.asarray(frac, np.float64), lattice=np.asarray(lattice, np.float64))
