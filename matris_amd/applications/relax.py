"""Structure relaxation with MatRIS forces.

Reference: matris/applications/relax.py:20-147 (StructOptimizer) and the observer of
base.py:125-175 (TrajectoryObserver).  With ASE installed, relax() runs the reference's
flow: the chosen ASE optimizer on the atoms, wrapped in the chosen ASE cell filter when
relax_cell, with MatRISCalculator attached and the trajectory observer called every
loginterval steps.  ASE is not part of this image; without it, relax() runs the FIRE
optimizer natively on the atomic positions (relax_cell=False) -- the published method
(Bitzek, Koskinen, Gaehler, Moseler & Gumbsch, Phys. Rev. Lett. 97, 170201 (2006)) with
ASE's default FIRE parameters and its cap on the step length -- over the atomic
positions, or with relax_cell over positions and cell together (CellFilterDOF, the
deformation-gradient filter), and raises for another optimizer.
"""
from __future__ import annotations

import contextlib
import io
import sys
import warnings

import numpy as np

from .calculator import MatRISCalculator, SimpleAtoms

OPTIMIZER_NAMES = ("BFGS", "BFGSLineSearch", "FIRE", "LBFGS", "LBFGSLineSearch", "MDMin")
FIRE_DEFAULTS = dict(dt=0.1, maxstep=0.2, dtmax=1.0, Nmin=5, finc=1.1, fdec=0.5, astart=0.1, fa=0.99)


class TrajectoryObserver:
    """Energies, forces, stresses, magmoms, positions and cells along a relaxation
    (the fields of the reference observer, base.py:125-175)."""

    def __init__(self, atoms):
        self.atoms = atoms
        self.energies: list = []
        self.forces: list = []
        self.stresses: list = []
        self.magmoms: list = []
        self.atom_positions: list = []
        self.cells: list = []

    def __call__(self) -> None:
        a = self.atoms
        self.energies.append(float(a.get_potential_energy()))
        self.forces.append(np.asarray(a.get_forces()))
        self.stresses.append(np.asarray(a.get_stress()))
        m = a.get_magnetic_moments() if hasattr(a, "get_magnetic_moments") else None
        self.magmoms.append(None if m is None else np.asarray(m))
        self.atom_positions.append(np.asarray(a.get_positions()).copy())
        cell = a.get_cell()
        self.cells.append(np.asarray(getattr(cell, "array", cell)).copy())

    def __len__(self) -> int:
        return len(self.energies)

    def save(self, filename: str) -> None:
        """Write the trajectory as a compressed npz (arrays only)."""
        np.savez_compressed(filename, energy=np.asarray(self.energies), forces=np.asarray(self.forces),
                            stresses=np.asarray(self.stresses), atom_positions=np.asarray(self.atom_positions),
                            cell=np.asarray(self.cells))


def fire_relax(atoms, fmax: float = 0.05, steps: int = 500, observer=None, loginterval: int = 1, **params) -> bool:
    """FIRE on the positions of `atoms` (which carries the calculator).  Returns True
    when max_i |f_i| < fmax was reached within `steps` force evaluations."""
    p = dict(FIRE_DEFAULTS, **params)
    dt, a, n_pos = p["dt"], p["astart"], 0
    v = None
    r = np.asarray(atoms.get_positions(), dtype=np.float64)
    for step in range(int(steps) + 1):
        f = np.asarray(atoms.get_forces(), dtype=np.float64)
        if observer is not None and step % loginterval == 0:
            observer()
        if np.sqrt((f * f).sum(axis=1)).max() < fmax:
            return True
        if step == steps:
            return False
        if v is None:
            v = np.zeros_like(r)
        else:
            vf = float((f * v).sum())
            if vf > 0.0:  # keep going downhill; mix the velocity toward the force
                v = (1.0 - a) * v + a * f / np.sqrt((f * f).sum()) * np.sqrt((v * v).sum())
                if n_pos > p["Nmin"]:
                    dt = min(dt * p["finc"], p["dtmax"])
                    a *= p["fa"]
                n_pos += 1
            else:  # uphill: stop, restart the mixing, shrink the step
                v[:] = 0.0
                a = p["astart"]
                dt *= p["fdec"]
                n_pos = 0
        v += dt * f
        dr = dt * v
        norm = np.sqrt((dr * dr).sum())
        if norm > p["maxstep"]:
            dr *= p["maxstep"] / norm
        r = r + dr
        atoms.set_positions(r)
    return False


def _stress33(s) -> np.ndarray:
    s = np.asarray(s, dtype=np.float64)
    if s.shape == (6,):  # Voigt order xx, yy, zz, yz, xz, xy
        xx, yy, zz, yz, xz, xy = s
        return np.array([[xx, xy, xz], [xy, yy, yz], [xz, yz, zz]])
    return s.reshape(3, 3)


class CellFilterDOF:
    """Positions and cell as one set of generalised coordinates, restated from the
    deformation-gradient cell filter that ASE's UnitCellFilter implements (Tadmor, Smith,
    Bernstein & Kaxiras, Phys. Rev. B 59, 235 (1999)): with F the deformation gradient of
    the current cell against the starting one (cell = cell0 F^T, r = r0 F^T), the
    coordinates are (r0 [n,3], c F [3,3]) with c = n_atoms, and their forces are
    (f F, W F^-T / c) with the virial W = -V (stress + p I).  A converged state has zero
    atomic forces and zero stress (or the hydrostatic pressure p, eV/A^3)."""

    def __init__(self, atoms, scalar_pressure: float = 0.0):
        self.atoms = atoms
        self.cell0 = np.asarray(atoms.get_cell(), dtype=np.float64).reshape(3, 3).copy()
        self.c = float(len(atoms))
        self.p = float(scalar_pressure)
        self.F = np.eye(3)

    def get_positions(self) -> np.ndarray:
        r0 = np.linalg.solve(self.F, np.asarray(self.atoms.get_positions(), np.float64).T).T
        return np.vstack([r0, self.c * self.F])

    def set_positions(self, x) -> None:
        x = np.asarray(x, dtype=np.float64)
        n = len(self.atoms)
        self.F = x[n:] / self.c
        self.atoms.set_cell(self.cell0 @ self.F.T, scale_atoms=False)
        self.atoms.set_positions(x[:n] @ self.F.T)

    def get_forces(self) -> np.ndarray:
        f = np.asarray(self.atoms.get_forces(), dtype=np.float64) @ self.F
        vol = abs(np.linalg.det(np.asarray(self.atoms.get_cell(), np.float64).reshape(3, 3)))
        virial = -vol * (_stress33(self.atoms.get_stress()) + self.p * np.eye(3))
        return np.vstack([f, np.linalg.solve(self.F, virial.T).T / self.c])


# Cell filters whose stationary point (zero forces, stress equal to -scalar_pressure) the
# native deformation-gradient coordinates reach; ASE's StrainFilter keeps the atoms fixed.
NATIVE_CELL_FILTERS = ("UnitCellFilter", "FrechetCellFilter", "ExpCellFilter")


def _ase_filter_class(ase_filter, filter_classes):
    """relax.py:88-98: a Filter subclass of ase.filters by name (ValueError for other
    names), or a class passed as is."""
    if not isinstance(ase_filter, str):
        return ase_filter
    import inspect
    valid = [n for n, c in inspect.getmembers(filter_classes, inspect.isclass) if issubclass(c, filter_classes.Filter)]
    if ase_filter not in valid:
        raise ValueError(f"Invalid ase_filter={ase_filter!r}, must be one of {valid}. ")
    return getattr(filter_classes, ase_filter)


class StructOptimizer:
    """Structure optimiser with the reference's constructor (relax.py:23-52)."""

    def __init__(self, model="matris_10m_oam", task: str = "efs", optimizer: str = "FIRE", device: str | None = None):
        if isinstance(optimizer, str) and optimizer not in OPTIMIZER_NAMES:
            raise ValueError(f"Optimizer {optimizer} not found. Select from {list(OPTIMIZER_NAMES)}")
        self.optimizer = optimizer
        self.calculator = MatRISCalculator(model=model, task=task, device=device)

    def relax(self, atoms, fmax: float = 0.05, steps: int = 500, relax_cell: bool = True,
              ase_filter: str = "FrechetCellFilter", save_path: str | None = None, loginterval: int = 1,
              crystal_feas_save_path: str | None = None, verbose: bool = True, assign_magmoms: bool = True,
              **kwargs) -> dict:
        """Relax `atoms` (ASE Atoms, SimpleAtoms, or a pymatgen Structure when pymatgen is
        installed) until max |f| < fmax or `steps` optimiser steps (relax.py:54-147).
        Returns {"final_structure": relaxed structure, "trajectory": TrajectoryObserver}."""
        if crystal_feas_save_path:
            from .md import CRYSTAL_FEAS_UNSUPPORTED
            raise NotImplementedError(CRYSTAL_FEAS_UNSUPPORTED)
        try:
            import ase.filters as filters  # noqa: F401
            import ase.optimize as ase_optimize
            have_ase = True
        except ImportError:
            have_ase = False
        if hasattr(atoms, "frac_coords") and hasattr(atoms, "lattice"):  # pymatgen Structure
            if have_ase:
                from pymatgen.io.ase import AseAtomsAdaptor
                atoms = AseAtomsAdaptor().get_atoms(atoms)
            else:
                atoms = SimpleAtoms.from_fractional(atoms.frac_coords, atoms.lattice.matrix,
                                                    [s.specie.Z for s in atoms])
        atoms.calc = self.calculator
        obs = TrajectoryObserver(atoms)
        stream = sys.stdout if verbose else io.StringIO()
        if have_ase and not isinstance(atoms, SimpleAtoms):
            import ase.filters as filter_classes
            filter_cls = _ase_filter_class(ase_filter, filter_classes)
            opt_cls = getattr(ase_optimize, self.optimizer) if isinstance(self.optimizer, str) else self.optimizer
            with contextlib.redirect_stdout(stream):
                target = filter_cls(atoms) if relax_cell else atoms
                opt = opt_cls(target, **kwargs)
                opt.attach(obs, interval=loginterval)
                opt.run(fmax=fmax, steps=steps)
                obs()
        else:
            if self.optimizer != "FIRE":
                raise NotImplementedError("without ASE this build relaxes with FIRE only (optimizer='FIRE')")
            name = ase_filter if isinstance(ase_filter, str) else getattr(ase_filter, "__name__", str(ase_filter))
            if relax_cell and name not in NATIVE_CELL_FILTERS:
                raise ValueError(f"Invalid ase_filter={name!r}, must be one of {list(NATIVE_CELL_FILTERS)} "
                                 "(without ASE the cell relaxes through the native deformation-gradient filter)")
            if relax_cell and name != "UnitCellFilter":
                warnings.warn(f"without ASE, ase_filter={name!r} relaxes the cell through UnitCellFilter's "
                              "deformation-gradient coordinates (same stationary point, different path)",
                              RuntimeWarning, stacklevel=2)
            with contextlib.redirect_stdout(stream):
                target = CellFilterDOF(atoms, kwargs.pop("scalar_pressure", 0.0)) if relax_cell else atoms
                fire_relax(target, fmax=fmax, steps=steps, observer=obs, loginterval=loginterval, **kwargs)
                obs()
        if save_path is not None:
            obs.save(save_path)
        final = atoms  # without pymatgen and ASE: the relaxed atoms object itself
        if have_ase and not isinstance(atoms, SimpleAtoms):
            try:  # relax.py:137-146: always a pymatgen Structure when pymatgen is there
                from pymatgen.io.ase import AseAtomsAdaptor
            except ImportError:
                AseAtomsAdaptor = None
            if AseAtomsAdaptor is not None:
                final = AseAtomsAdaptor.get_structure(atoms)
                if assign_magmoms and atoms.get_magnetic_moments() is not None:
                    for key in list(final.site_properties):
                        final.remove_site_property(property_name=key)
                    final.add_site_property("magmom", [float(m) for m in atoms.get_magnetic_moments()])
        return {"final_structure": final, "trajectory": obs}
