"""Synthetic configuration generators: deterministic and with the advertised geometry."""
import numpy as np

from matris_amd import workloads as W
from oracle import graph_ref


def _min_periodic_dist(cr):
    cart = graph_ref.frac_to_cart(cr.frac, cr.lattice)
    L = cr.lattice[0, 0]
    d = cart[:, None, :] - cart[None, :, :]
    d -= L * np.round(d / L)
    r = np.sqrt((d * d).sum(-1))
    np.fill_diagonal(r, np.inf)
    return r.min()


def test_c3_shape_and_determinism():
    a, b = W.c3_cu864(), W.c3_cu864()
    assert len(a) == 864 and np.array_equal(a.frac, b.frac)
    assert np.allclose(a.lattice, np.eye(3) * 21.66)
    disp = (a.frac - W.fcc_supercell(3.61, 6).frac) @ a.lattice
    assert 0.04 < disp.std() < 0.06


def test_c2_density_and_min_distance():
    cr = W.c2_rsa4096()
    assert len(cr) == 4096
    assert abs(4096 / np.linalg.det(cr.lattice) - 0.085) < 1e-9
    assert _min_periodic_dist(cr) >= 1.8


def test_c4_batch():
    cells = W.c4_batch64()
    assert len(cells) == 64 and all(8 <= len(c) <= 64 for c in cells)
    for c in cells[:8]:
        v = abs(np.linalg.det(c.lattice)) / len(c)
        assert 10 - 1e-9 <= v <= 25 + 1e-9 and 1 <= c.z.min() and c.z.max() <= 94


def test_sio2_composition_density():
    cr = W.sio2(3000, seed=4)
    assert (cr.z == 14).sum() == 1000 and (cr.z == 8).sum() == 2000
    mass = (1000 * 28.0855 + 2000 * 15.999) * W.AMU_G
    assert abs(mass / (np.linalg.det(cr.lattice) * 1e-24) - 2.2) < 1e-9
    assert _min_periodic_dist(cr) >= 1.5
