"""The error_graph.cif dump of a failed line-graph build (converter.py:99-106), on the CPU.

The CIF writer is checked by parsing its text back: the cell parameters against closed
forms (cubic, hexagonal, a general triclinic cell rebuilt from its parameters), the sites
against the input; the converter's failure branch runs with its device builders replaced
by CPU stand-ins and the line-graph builder raising."""
import math
import warnings

import numpy as np
import pytest
import torch

from matris_amd.graph import converter as conv
from matris_amd.graph.cif import SYMBOLS, cell_parameters, cif_text


def _parse(text):
    keys, sites, in_sites = {}, [], False
    for line in text.splitlines():
        t = line.split()
        if not t:
            continue
        if t[0].startswith("_cell_"):
            keys[t[0]] = float(t[1])
        if t[0] == "_atom_site_occupancy":
            in_sites = True
            continue
        if in_sites:
            sites.append((t[0], t[1], float(t[3]), float(t[4]), float(t[5])))
    return keys, sites


def _lattice_from_parameters(a, b, c, al, be, ga):
    """Rows a, b, c of a cell with the given lengths and angles (a along x, b in the xy plane)."""
    al, be, ga = (math.radians(v) for v in (al, be, ga))
    va = np.array([a, 0.0, 0.0])
    vb = np.array([b * math.cos(ga), b * math.sin(ga), 0.0])
    cx = c * math.cos(be)
    cy = c * (math.cos(al) - math.cos(be) * math.cos(ga)) / math.sin(ga)
    vc = np.array([cx, cy, math.sqrt(c * c - cx * cx - cy * cy)])
    return np.stack([va, vb, vc])


def test_symbol_table():
    assert SYMBOLS[1] == "H" and SYMBOLS[8] == "O" and SYMBOLS[14] == "Si" and SYMBOLS[29] == "Cu"
    assert SYMBOLS[79] == "Au" and SYMBOLS[92] == "U" and SYMBOLS[118] == "Og" and len(SYMBOLS) == 119


def test_cell_parameters_closed_forms():
    np.testing.assert_allclose(cell_parameters(3.61 * np.eye(3)), (3.61, 3.61, 3.61, 90, 90, 90), atol=1e-12)
    hexa = np.array([[2.5, 0, 0], [-1.25, 2.5 * math.sqrt(3) / 2, 0], [0, 0, 4.1]])
    np.testing.assert_allclose(cell_parameters(hexa), (2.5, 2.5, 4.1, 90, 90, 120), atol=1e-12)
    par = (4.2, 5.1, 6.3, 77.0, 84.0, 101.0)
    np.testing.assert_allclose(cell_parameters(_lattice_from_parameters(*par)), par, atol=1e-10)
    # a rotation of the cell changes no parameter
    th = 0.7
    rot = np.array([[math.cos(th), -math.sin(th), 0], [math.sin(th), math.cos(th), 0], [0, 0, 1]])
    np.testing.assert_allclose(cell_parameters(_lattice_from_parameters(*par) @ rot.T), par, atol=1e-10)


def test_cif_text_round_trip():
    rng = np.random.default_rng(3)
    lat = _lattice_from_parameters(4.2, 5.1, 6.3, 77.0, 84.0, 101.0)
    frac = rng.random((5, 3))
    z = np.array([14, 8, 8, 29, 8])
    keys, sites = _parse(cif_text(frac, lat, z))
    np.testing.assert_allclose([keys["_cell_length_a"], keys["_cell_length_b"], keys["_cell_length_c"],
                                keys["_cell_angle_alpha"], keys["_cell_angle_beta"], keys["_cell_angle_gamma"]],
                               (4.2, 5.1, 6.3, 77.0, 84.0, 101.0), atol=1e-7)
    np.testing.assert_allclose(keys["_cell_volume"], abs(np.linalg.det(lat)), rtol=1e-8)
    assert [s[0] for s in sites] == ["Si", "O", "O", "Cu", "O"]
    assert [s[1] for s in sites] == ["Si0", "O0", "O1", "Cu0", "O2"]
    np.testing.assert_allclose([s[2:] for s in sites], frac, atol=1e-8)
    with pytest.raises(ValueError):
        cif_text(frac, lat, z[:4])


def test_failed_line_graph_writes_error_cif(tmp_path, monkeypatch):
    """A RuntimeError from the line-graph builder: error_graph.cif in the working directory,
    a warning, and a RadiusGraph with an empty line graph."""
    monkeypatch.chdir(tmp_path)
    frac = np.array([[0.0, 0.0, 0.0], [0.5, 0.5, 0.5]])
    lat = 2.9 * np.eye(3)
    z = np.array([26, 26])
    # two atoms, each the other's only neighbour (one image): E = 2 directed edges
    center = torch.tensor([0, 1], dtype=torch.int32)
    neighbor = torch.tensor([1, 0], dtype=torch.int32)
    image = torch.zeros(2, 3, dtype=torch.int32)
    dist = torch.full((2,), 2.5, dtype=torch.float64)
    row_ptr = torch.tensor([0, 1, 2], dtype=torch.int32)
    row_count = torch.tensor([1, 1], dtype=torch.int32)

    def pair_edges(n, c, nb, im, rp):
        return (torch.tensor([1, 0], dtype=torch.int32), torch.tensor([0, 0], dtype=torch.int32),
                torch.tensor([0], dtype=torch.int32), torch.tensor([1], dtype=torch.int32))

    def line_graph(*args):
        raise RuntimeError("matris_line_graph_count: MATRIS_E_CAPACITY (capacity exceeded)")

    monkeypatch.setattr(conv, "pair_edges_device", pair_edges)
    monkeypatch.setattr(conv, "line_graph_device", line_graph)
    gc = conv.GraphConverter(device="cpu")
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        g = gc.from_arrays(frac, lat, z, neighbors=(center, neighbor, image, dist, row_ptr, row_count))
    assert any("error_graph.cif" in str(x.message) for x in w)
    assert g.line_graph.shape == (0, 5)
    keys, sites = _parse((tmp_path / "error_graph.cif").read_text())
    assert keys["_cell_length_a"] == pytest.approx(2.9) and keys["_cell_angle_gamma"] == pytest.approx(90.0)
    assert [s[0] for s in sites] == ["Fe", "Fe"]
    np.testing.assert_allclose([s[2:] for s in sites], frac, atol=1e-8)


def test_failed_line_graph_in_an_unwritable_directory_still_builds(tmp_path, monkeypatch):
    """The dump failing (here: error_graph.cif is a directory) is reported in the warning;
    the graph is still built with an empty line graph."""
    monkeypatch.chdir(tmp_path)
    (tmp_path / "error_graph.cif").mkdir()
    center = torch.tensor([0, 1], dtype=torch.int32)
    neighbor = torch.tensor([1, 0], dtype=torch.int32)
    nb = (center, neighbor, torch.zeros(2, 3, dtype=torch.int32), torch.full((2,), 2.5, dtype=torch.float64),
          torch.tensor([0, 1, 2], dtype=torch.int32), torch.tensor([1, 1], dtype=torch.int32))
    monkeypatch.setattr(conv, "pair_edges_device", lambda *a: (torch.tensor([1, 0], dtype=torch.int32),
                                                               torch.tensor([0, 0], dtype=torch.int32),
                                                               torch.tensor([0], dtype=torch.int32),
                                                               torch.tensor([1], dtype=torch.int32)))

    def line_graph(*args):
        raise RuntimeError("line graph failed")

    monkeypatch.setattr(conv, "line_graph_device", line_graph)
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        g = conv.GraphConverter(device="cpu").from_arrays(np.array([[0.0, 0, 0], [0.5, 0.5, 0.5]]), 2.9 * np.eye(3),
                                                          np.array([26, 26]), neighbors=nb)
    assert any("could not be written" in str(x.message) for x in w)
    assert g.line_graph.shape == (0, 5)
