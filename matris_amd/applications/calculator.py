"""ASE calculator on the MI355X MatRIS path.

Reference: matris/applications/base.py:24-122 (MatRISCalculator).  One calculate() call
is one efsm evaluation: the structure goes through the GPU radius-graph / line-graph
builder (GraphConverter) and the model, and the results follow the reference's
conventions (base.py:107-122):
  energy  = e * n_atoms for an intensive model (total energy, eV)
  forces  = f [n, 3] (eV/A)
  stress  = s * GPa, the model's 3x3 stress in GPa converted to eV/A^3
  magmoms = m [n]
Non-periodic directions get the reference's padded cell (base.py:70-93) before the graph
is built.

ASE is optional here: with ASE installed the class is an ase Calculator (attach it to
Atoms as usual); without it, a minimal base class with the same calculate / results /
get_* interface is used, and any object with get_positions / get_cell /
get_atomic_numbers / get_pbc (or get_scaled_positions and a cell) can be evaluated.
"""
from __future__ import annotations

import numpy as np

from ..config import EV_A3_TO_GPA

GPA = 1.0 / EV_A3_TO_GPA  # 1 GPa in eV/A^3 (ase.units.GPa)
PROPERTIES = ("energy", "forces", "stress", "magmoms")


class _CalculatorBase:
    """The part of ase.calculators.calculator.Calculator that MatRISCalculator relies on:
    results cached per structure, get_property and the get_* accessors."""

    implemented_properties: tuple = ()

    def __init__(self, **kwargs):
        self.atoms = None
        self.results: dict = {}
        self.parameters = dict(kwargs)

    @staticmethod
    def _state(atoms):
        pos = np.asarray(atoms.get_positions(), dtype=np.float64)
        cell = np.asarray(_cell_array(atoms), dtype=np.float64)
        return pos, cell, np.asarray(atoms.get_atomic_numbers()), np.asarray(atoms.get_pbc(), dtype=bool)

    def check_state(self, atoms) -> list:
        if self.atoms is None:
            return ["positions"]
        old, new = self._state(self.atoms), self._state(atoms)
        return [] if all(a.shape == b.shape and np.array_equal(a, b) for a, b in zip(old, new)) else ["positions"]

    def calculate(self, atoms=None, properties=None, system_changes=None):
        if atoms is not None:
            self.atoms = atoms.copy() if hasattr(atoms, "copy") else atoms
        self.results = {}

    def get_property(self, name, atoms=None, allow_calculation=True):
        if atoms is None:
            atoms = self.atoms
        if self.check_state(atoms) or name not in self.results:
            if not allow_calculation:
                return None
            self.calculate(atoms, [name], ["positions"])
        return self.results[name]

    def get_potential_energy(self, atoms=None, force_consistent=False):
        return self.get_property("energy", atoms)

    def get_forces(self, atoms=None):
        return self.get_property("forces", atoms)

    def get_stress(self, atoms=None):
        return self.get_property("stress", atoms)

    def get_magnetic_moments(self, atoms=None):
        return self.get_property("magmoms", atoms)


try:  # the reference's base class when ASE is present
    from ase.calculators.calculator import Calculator as _Base
except ImportError:  # pragma: no cover - ASE is not part of this image
    _Base = _CalculatorBase


def _cell_array(atoms) -> np.ndarray:
    cell = atoms.get_cell() if hasattr(atoms, "get_cell") else atoms.cell
    return np.asarray(getattr(cell, "array", cell), dtype=np.float64)


def padded_cell(positions, cell, pbc, cutoff: float, num_layers: int) -> np.ndarray:
    """The cell the reference gives a structure with non-periodic directions
    (base.py:70-93): each non-periodic lattice vector becomes the Cartesian axis times
    (max |position| + 1) * max(5, num_layers) * cutoff."""
    cell = np.array(cell, dtype=np.float64, copy=True)
    pbc = np.asarray(pbc, dtype=bool)
    if pbc.all():
        return cell
    span = np.max(np.abs(np.asarray(positions, dtype=np.float64))) + 1
    expand = max(5, int(num_layers))
    eye = np.identity(3)
    for k in range(3):
        if not pbc[k]:
            cell[k, :] = span * expand * cutoff * eye[k, :]
    return cell


class MatRISCalculator(_Base):
    """MatRIS calculator with the reference's constructor (base.py:27-53).

    model: a MatRIS instance, a reference model name ("matris_10m_oam", ...; needs the
    local checkpoint, see MatRIS.load) or a checkpoint path.  task: "e", "ef", "efs",
    "efsm" (forces and stress are autograd derivatives of the energy).  device: the ROCm
    device ("cuda", the default); "cpu" is rejected because this build has no CPU
    path.
    """

    implemented_properties = PROPERTIES

    def __init__(self, model="matris_10m_oam", task: str = "efs", device: str | None = None, **kwargs):
        super().__init__(**kwargs)
        import torch

        from ..model.model import MatRIS
        if device is not None and torch.device(device).type != "cuda":
            raise ValueError(f"device={device!r}: MatRISCalculator runs on the ROCm device only")
        if isinstance(model, MatRIS):
            self.model = model if device is None else model.to(device)
        elif isinstance(model, str) and (model.endswith(".tar") or model.endswith(".pth") or "/" in model):
            self.model = MatRIS.load(path=model, device=device)
        else:
            self.model = MatRIS.load(model_name=model, device=device)
        self.device = next(self.model.parameters()).device
        self.task = task
        self.stress_unit = GPA
        self.key = set(["atoms_per_graph", "ref_energy"] + list(task))

    def calculate(self, atoms=None, properties=None, system_changes=None) -> None:
        """One efsm evaluation of `atoms` (base.py:55-122)."""
        super().calculate(atoms, properties or list(PROPERTIES), system_changes or ["positions"])
        if atoms is None:
            atoms = self.atoms
        # as in the reference, the padded cell is set on the caller's atoms (base.py:92-93)
        pbc = np.asarray(atoms.get_pbc(), dtype=bool)
        if not pbc.all():
            cell = padded_cell(atoms.get_positions(), _cell_array(atoms), pbc, self.model.config["pairwise_cutoff"],
                               self.model.config["num_layers"])
            atoms.set_cell(cell, scale_atoms=False)
        frac, lat, z = _fractional(atoms)
        graph = self.model.graph_converter.from_arrays(frac, lat, z)
        pred = self.model([graph], task=self.task, is_training=False)
        n_atoms = len(z) if self.model.is_intensive else 1

        def last(key):  # the reference keeps the last graph's entry of each key
            v = pred.get(key)
            if v is None:
                return None
            if isinstance(v, (int, float)):
                return np.asarray(v, dtype=np.float64)
            seq = list(v) if isinstance(v, (list, tuple)) else [v[i] for i in range(v.shape[0])]
            return seq[-1].detach().cpu().numpy() if seq else None

        e = last("e")
        s = last("s") if "s" in self.task else None
        self.results.update(
            ref_energy=float(np.asarray(last("ref_energy"))) * n_atoms,
            energy=float(e) * n_atoms,
            forces=last("f") if "f" in self.task else None,
            stress=s * self.stress_unit if s is not None else None,
            magmoms=last("m") if "m" in self.task else None,
        )


class SimpleAtoms:
    """The subset of ase.Atoms the calculator, optimizer and MD driver use, for running
    without ASE: positions (A, Cartesian), cell rows (A), atomic numbers, pbc."""

    def __init__(self, positions, cell, numbers, pbc=(True, True, True)):
        self.positions = np.array(positions, dtype=np.float64, copy=True).reshape(-1, 3)
        self.cell = np.array(cell, dtype=np.float64, copy=True).reshape(3, 3)
        self.numbers = np.array(numbers, dtype=np.int64, copy=True).reshape(-1)
        self.pbc = np.array(pbc, dtype=bool).reshape(3) if np.ndim(pbc) else np.array([bool(pbc)] * 3)
        self.calc = None

    @classmethod
    def from_fractional(cls, frac, lattice, numbers, pbc=(True, True, True)):
        lat = np.asarray(lattice, dtype=np.float64)
        return cls(np.asarray(frac, dtype=np.float64) @ lat, lat, numbers, pbc)

    def __len__(self):
        return len(self.numbers)

    def copy(self):
        return SimpleAtoms(self.positions, self.cell, self.numbers, self.pbc)

    def get_positions(self):
        return self.positions.copy()

    def set_positions(self, positions):
        self.positions = np.array(positions, dtype=np.float64, copy=True).reshape(-1, 3)

    def get_cell(self):
        return self.cell.copy()

    def set_cell(self, cell, scale_atoms: bool = False):
        new = np.array(cell, dtype=np.float64, copy=True).reshape(3, 3)
        if scale_atoms:
            self.positions = self.positions @ np.linalg.solve(self.cell, new)
        self.cell = new

    def get_atomic_numbers(self):
        return self.numbers.copy()

    def get_pbc(self):
        return self.pbc.copy()

    def get_scaled_positions(self, wrap: bool = True):
        frac = np.linalg.solve(self.cell.T, self.positions.T).T
        return frac % 1.0 if wrap else frac

    def get_potential_energy(self):
        return self.calc.get_potential_energy(self)

    def get_forces(self):
        return self.calc.get_forces(self)

    def get_stress(self):
        return self.calc.get_stress(self)

    def get_magnetic_moments(self):
        return self.calc.get_magnetic_moments(self)


def _fractional(atoms):
    """(frac fp64 [n,3], lattice fp64 [3,3], Z int64 [n]) of an Atoms-like object."""
    lat = _cell_array(atoms)
    if hasattr(atoms, "get_scaled_positions"):
        try:
            frac = np.asarray(atoms.get_scaled_positions(wrap=False), dtype=np.float64)
        except TypeError:
            frac = np.asarray(atoms.get_scaled_positions(), dtype=np.float64)
    else:
        frac = np.linalg.solve(lat.T, np.asarray(atoms.get_positions(), dtype=np.float64).T).T
    return frac, lat, np.asarray(atoms.get_atomic_numbers(), dtype=np.int64)
