"""The per-graph index range check that runs before any kernel reads through a graph's
indices (CPU: process_graphs refuses a bad graph before its first device op)."""
import numpy as np
import pytest
import torch

from matris_amd.graph import RadiusGraph
from matris_amd.model.batch import process_graphs, validate_graph_indices
from oracle import graph_ref
from matris_amd import workloads as W


def _graph():
    cr = W.c1_cu4()
    og = graph_ref.build_graph(cr.frac, cr.lattice, cr.z)
    t = lambda a, dt=torch.int32: torch.as_tensor(np.asarray(a), dtype=dt)
    return RadiusGraph(graph_id=None, mp_id=None, composition=None, atomic_number=t(cr.z),
                       atom_frac_coord=t(cr.frac, torch.float32), lattice=t(cr.lattice, torch.float32),
                       neighbor_image=t(og["image"], torch.float32),
                       atom_graph=t(np.stack([og["center"], og["neighbor"]], 1)), atom_graph_cutoff=6.0,
                       line_graph=t(og["line_graph"]), line_graph_cutoff=4.0, directed2undirected=t(og["d2u"]),
                       undirected2directed=t(og["u2d"]))


def test_valid_graph_passes_and_is_marked():
    g = _graph()
    validate_graph_indices(g)
    assert g.meta["indices_checked"] == g.index_signature()


@pytest.mark.parametrize("field,row,col,delta", [
    ("line_graph", 3, 1, 5), ("line_graph", 0, 0, 4), ("line_graph", 7, 4, 1), ("atom_graph", 2, 1, 4),
    ("directed2undirected", 9, None, 1), ("undirected2directed", 1, None, 1), ("line_graph", 5, 2, -10**6)])
def test_out_of_range_index_refused_before_device_work(field, row, col, delta):
    g = _graph()
    t = getattr(g, field)
    N, E, U = len(g.atomic_number), len(g.atom_graph), len(g.undirected2directed)
    lim = {"line_graph": [N, U, E, U, E], "atom_graph": [N, N], "directed2undirected": U,
           "undirected2directed": E}[field]
    if col is None:
        t[row] = lim - 1 + delta if delta > 0 else delta
    else:
        t[row, col] = lim[col] - 1 + delta if delta > 0 else delta
    with pytest.raises(ValueError, match="outside its range"):
        process_graphs([g])  # raises before any op that needs a GPU
    assert "indices_checked" not in g.meta


@pytest.mark.parametrize("how", ["in_place", "replaced"])
def test_edit_after_a_passed_check_is_checked_again(how):
    """A graph whose indices passed the check and were then edited (in place, which bumps
    the tensor's version counter, or by assigning a new tensor) is checked again: the
    out-of-range index is refused before any device work."""
    g = _graph()
    validate_graph_indices(g)
    U = len(g.undirected2directed)
    if how == "in_place":
        g.line_graph[3, 1] = U + 7
    else:
        lg = g.line_graph.clone()
        lg[3, 1] = U + 7
        g.line_graph = lg
    with pytest.raises(ValueError, match="outside its range"):
        process_graphs([g])
    assert "indices_checked" not in g.meta


def test_storage_swap_changes_the_signature():
    """A storage swapped in through set_() bumps no version counter; the signature still
    changes (it holds the storage object's address), so the range check and the kept
    topology are redone."""
    g = _graph()
    validate_graph_indices(g)
    sig = g.index_signature()
    lg = g.line_graph.clone()
    lg[3, 1] = len(g.undirected2directed) + 7
    g.line_graph.set_(lg)
    assert g.index_signature() != sig
    with pytest.raises(ValueError, match="outside its range"):
        process_graphs([g])


def test_unchanged_graph_is_not_checked_twice(monkeypatch):
    """The remembered check holds while no index tensor changes (one host read per graph)."""
    g = _graph()
    validate_graph_indices(g)
    calls = []
    monkeypatch.setattr(torch, "stack", lambda *a, **k: calls.append(1) or torch.cat([x[None] for x in a[0]]))
    validate_graph_indices(g)
    assert not calls
