"""Host logic of the application layer (no GPU): the reference's non-periodic cell
padding, the Atoms stand-in, and the native FIRE optimiser on an analytic potential."""
import numpy as np
import pytest

from matris_amd.applications.calculator import GPA, SimpleAtoms, padded_cell
from matris_amd.applications.relax import FIRE_DEFAULTS, fire_relax


def test_gpa_is_ase_unit():
    # ase.units (CODATA 2014, its default): 1 GPa = 1e9 J/m^3 = 1e9 / 1.6021766208e-19 eV / 1e30 A^3
    assert GPA == pytest.approx(1e9 / 1.6021766208e-19 / 1e30, rel=1e-12)


def test_padded_cell_matches_reference_rule():
    """base.py:70-93: non-periodic vectors -> axis * (max|pos| + 1) * max(5, L) * cutoff."""
    pos = np.array([[0.0, 1.0, -2.5], [3.0, -0.5, 0.2]])
    cell = np.diag([4.0, 5.0, 6.0])
    out = padded_cell(pos, cell, [True, False, False], cutoff=6.0, num_layers=10)
    span = 3.0 + 1.0
    np.testing.assert_array_equal(out[0], cell[0])
    np.testing.assert_allclose(out[1], [0.0, span * 10 * 6.0, 0.0])
    np.testing.assert_allclose(out[2], [0.0, 0.0, span * 10 * 6.0])
    # fewer layers than 5 still expands by 5
    out = padded_cell(pos, cell, [False, True, True], cutoff=4.0, num_layers=3)
    np.testing.assert_allclose(out[0], [span * 5 * 4.0, 0.0, 0.0])
    np.testing.assert_array_equal(padded_cell(pos, cell, [True] * 3, 6.0, 6), cell)


def test_simple_atoms_coordinates():
    lat = np.array([[4.0, 0.0, 0.0], [1.0, 5.0, 0.0], [0.5, 0.3, 6.0]])
    frac = np.array([[0.1, 0.2, 0.3], [0.9, 1.2, -0.1]])
    at = SimpleAtoms.from_fractional(frac, lat, [29, 8])
    np.testing.assert_allclose(at.get_scaled_positions(wrap=False), frac, atol=1e-12)
    np.testing.assert_allclose(at.get_scaled_positions(), frac % 1.0, atol=1e-12)
    at2 = at.copy()
    at2.set_cell(lat * 1.1, scale_atoms=True)
    np.testing.assert_allclose(at2.get_scaled_positions(wrap=False), frac, atol=1e-12)
    assert len(at) == 2 and at.get_pbc().all()


class _Harmonic:
    """E = sum_i k/2 |r_i - r0_i|^2 with an anisotropic k: a calculator stand-in."""

    def __init__(self, r0, k):
        self.r0, self.k, self.calls = r0, k, 0

    def get_forces(self, atoms):
        self.calls += 1
        return -self.k * (atoms.get_positions() - self.r0)


def test_fire_converges_on_harmonic_well():
    rng = np.random.default_rng(0)
    r0 = rng.normal(size=(6, 3))
    k = np.array([1.0, 4.0, 9.0])
    at = SimpleAtoms(r0 + rng.normal(scale=0.3, size=r0.shape), np.eye(3) * 10, [1] * 6)
    at.calc = _Harmonic(r0, k)
    assert fire_relax(at, fmax=1e-4, steps=2000)
    f = at.calc.get_forces(at)
    assert np.sqrt((f * f).sum(1)).max() < 1e-4
    np.testing.assert_allclose(at.get_positions(), r0, atol=2e-4)


def test_fire_step_is_capped():
    at = SimpleAtoms(np.zeros((1, 3)), np.eye(3) * 10, [1])
    at.calc = _Harmonic(np.array([[100.0, 0.0, 0.0]]), np.array([1.0, 1.0, 1.0]))
    fire_relax(at, fmax=1e-3, steps=1)
    assert np.linalg.norm(at.get_positions()) == pytest.approx(FIRE_DEFAULTS["maxstep"])


def test_fire_reports_failure_within_budget():
    at = SimpleAtoms(np.zeros((1, 3)), np.eye(3) * 10, [1])
    at.calc = _Harmonic(np.array([[50.0, 0.0, 0.0]]), np.array([1.0, 1.0, 1.0]))
    assert not fire_relax(at, fmax=1e-6, steps=3)
    assert at.calc.calls == 4  # initial evaluation + one per step


def test_native_relax_validates_the_cell_filter_name():
    """relax.py:88-98 refuses unknown filter names; without ASE the native cell DOF runs
    for the UnitCellFilter-type names and warns for the other two (same stationary point)."""
    import pytest

    from matris_amd.applications import relax as R

    class _Calc:
        pass

    opt = R.StructOptimizer.__new__(R.StructOptimizer)
    opt.optimizer, opt.calculator = "FIRE", _Calc()
    a = SimpleAtoms.from_fractional([[0, 0, 0]], [[3.0, 0, 0], [0, 3.0, 0], [0, 0, 3.0]], [29])
    with pytest.raises(ValueError, match="Invalid ase_filter"):
        opt.relax(a, ase_filter="StrainFilter", verbose=False)
    with pytest.raises(ValueError, match="Invalid ase_filter"):
        opt.relax(a, ase_filter="NoSuchFilter", verbose=False)


def test_crystal_feature_logging_is_refused_with_the_reason():
    """The reference's CrystalFeasObserver records a crystal_fea the model never produces
    (its first step raises KeyError): asking for it is refused up front, before a model is
    touched."""
    from matris_amd.applications.md import MolecularDynamics
    from matris_amd.applications.relax import StructOptimizer
    with pytest.raises(NotImplementedError, match="crystal_fea"):
        MolecularDynamics(atoms=None, model=None, crystal_feas_logfile="feas.pkl")
    with pytest.raises(NotImplementedError, match="crystal_fea"):
        StructOptimizer.relax(object.__new__(StructOptimizer), atoms=None, crystal_feas_save_path="feas.pkl")
