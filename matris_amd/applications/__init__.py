"""Callers of the efsm path with the reference's interfaces (matris/applications)."""
from .calculator import MatRISCalculator, SimpleAtoms  # noqa: F401
from .md import MolecularDynamics  # noqa: F401
from .relax import StructOptimizer, TrajectoryObserver  # noqa: F401
