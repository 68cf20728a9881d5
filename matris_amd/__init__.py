"""matris_amd: MI355X-native (gfx950) MatRIS efsm hot path.

Public API mirrors the reference package layout:
  matris_amd.model.MatRIS                       (matris.model.MatRIS)
  matris_amd.graph.RadiusGraph, GraphConverter  (matris.graph)
  matris_amd.applications.MatRISCalculator, StructOptimizer, MolecularDynamics
"""
__version__ = "0.1.0"
