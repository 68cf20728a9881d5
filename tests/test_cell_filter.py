"""The native cell filter (CellFilterDOF, used by StructOptimizer.relax(relax_cell=True)
without ASE), CPU: its generalised forces must be minus the gradient of the energy in its
coordinates.  Checked by central differences on an analytic periodic pair potential whose
forces and stress are exact (stress = (1/V) dE/d(strain), ASE's sign), so a wrong sign, a
transposed deformation gradient or a missing volume factor fails."""
import itertools

import numpy as np

from matris_amd.applications import SimpleAtoms
from matris_amd.applications.relax import CellFilterDOF, fire_relax

RC = 3.2


class PairCalc:
    """E = sum over pairs within RC (all periodic images) of (RC - r)^4 - 0.8 (RC - r)^3."""

    def _terms(self, atoms):
        pos, cell = atoms.get_positions(), atoms.get_cell()
        n = len(pos)
        e, f, w = 0.0, np.zeros_like(pos), np.zeros((3, 3))
        for i, j in itertools.product(range(n), range(n)):
            for img in itertools.product(range(-2, 3), repeat=3):
                if i == j and img == (0, 0, 0):
                    continue
                d = pos[j] + np.asarray(img, float) @ cell - pos[i]
                r = np.linalg.norm(d)
                if r >= RC:
                    continue
                x = RC - r
                e += 0.5 * (x ** 4 - 0.8 * x ** 3)
                dphi = -(4 * x ** 3 - 2.4 * x ** 2)  # dphi/dr
                f[i] += dphi * d / r  # each ordered pair carries half the energy: both halves act on i alike
                w += 0.5 * dphi * np.outer(d, d) / r
        return e, f, w / abs(np.linalg.det(cell))

    def get_potential_energy(self, atoms):
        return self._terms(atoms)[0]

    def get_forces(self, atoms):
        return self._terms(atoms)[1]

    def get_stress(self, atoms):
        return self._terms(atoms)[2]


def _atoms(seed=0):
    rng = np.random.default_rng(seed)
    cell = np.array([[3.6, 0.1, 0.0], [0.2, 3.4, 0.1], [0.0, 0.3, 3.8]])
    frac = np.array([[0, 0, 0], [0.5, 0.5, 0], [0.5, 0, 0.5], [0, 0.5, 0.5]]) + 0.03 * rng.normal(size=(4, 3))
    a = SimpleAtoms.from_fractional(frac, cell, [29] * 4)
    a.calc = PairCalc()
    return a


def test_pair_calc_is_consistent():
    """The test potential itself: forces and stress against central differences."""
    a = _atoms()
    e0, f, s = a.calc._terms(a)
    h = 1e-6
    pos = a.get_positions()
    p = pos.copy()
    p[1, 2] += h
    a.set_positions(p)
    ep = a.calc.get_potential_energy(a)
    p[1, 2] -= 2 * h
    a.set_positions(p)
    em = a.calc.get_potential_energy(a)
    assert abs(-(ep - em) / (2 * h) - f[1, 2]) < 1e-6
    a.set_positions(pos)
    cell, vol = a.get_cell(), abs(np.linalg.det(a.get_cell()))
    eps = np.zeros((3, 3)); eps[0, 1] = eps[1, 0] = h
    a.set_cell(cell @ (np.eye(3) + eps), scale_atoms=True)
    ep = a.calc.get_potential_energy(a)
    a.set_cell(cell @ (np.eye(3) - eps), scale_atoms=True)
    em = a.calc.get_potential_energy(a)
    assert abs((ep - em) / (2 * h) / vol - (s[0, 1] + s[1, 0])) < 1e-6


def test_generalised_forces_are_energy_gradients():
    a = _atoms(1)
    flt = CellFilterDOF(a, scalar_pressure=0.01)
    rng = np.random.default_rng(2)
    x0 = flt.get_positions()
    x0[-3:] += len(a) * 0.02 * rng.normal(size=(3, 3))  # a sheared, non-symmetric F
    flt.set_positions(x0)
    x, g = flt.get_positions(), flt.get_forces()
    np.testing.assert_allclose(x, x0, atol=1e-12)

    def enthalpy(y):
        flt.set_positions(y)
        return a.calc.get_potential_energy(a) + 0.01 * abs(np.linalg.det(a.get_cell()))
    for _ in range(3):
        d = rng.normal(size=x.shape)
        h = 1e-5
        fd = (enthalpy(x + h * d) - enthalpy(x - h * d)) / (2 * h)
        assert abs(fd + float((g * d).sum())) < 1e-6 * max(1.0, abs(fd)), fd


def test_fire_cell_relaxation_reaches_zero_stress():
    a = _atoms(3)
    a.set_cell(a.get_cell() * 1.05, scale_atoms=True)
    flt = CellFilterDOF(a)
    assert fire_relax(flt, fmax=1e-3, steps=2000)
    assert np.abs(a.calc.get_forces(a)).max() < 1e-3
    assert np.abs(a.calc.get_stress(a)).max() * abs(np.linalg.det(a.get_cell())) / len(a) < 1e-3
