"""Load the reference's own model modules from /root/reference for golden-vector writing.

Runs in the build container only (the reference tree does not exist on the GPU box and
nothing here is imported by tests or by the product).  The reference package __init__
files pull in pymatgen (matris/graph/converter.py:13, matris/model/reference_energy.py:7),
which is not installed; rather than standing in for pymatgen, this loader registers the
`matris`, `matris.graph` and `matris.model` package namespaces without executing those
__init__ files and then imports the pymatgen-free submodules the efsm path uses:
radiusgraph, processgraph, basis_function, functions (+ op/), feature_embed,
interaction_block and readout.  `MatRIS` itself (model.py) imports GraphConverter and
AtomRef, so its constructor/forward glue (model.py:100-178, 183-250) is composed in
make_golden.py from those reference modules.
"""
from __future__ import annotations

import importlib
import sys
import types

REF_ROOT = "/root/reference"


def load():
    if "matris.model.readout" in sys.modules:
        return sys.modules["matris"]
    pkg = types.ModuleType("matris")
    pkg.__path__ = [f"{REF_ROOT}/matris"]
    sys.modules["matris"] = pkg
    for sub in ("graph", "model"):
        m = types.ModuleType(f"matris.{sub}")
        m.__path__ = [f"{REF_ROOT}/matris/{sub}"]
        sys.modules[f"matris.{sub}"] = m
        setattr(pkg, sub, m)
    rg = importlib.import_module("matris.graph.radiusgraph")
    sys.modules["matris.graph"].RadiusGraph = rg.RadiusGraph
    sys.modules["matris.graph"].datatype = rg.datatype
    for name in ("basis_function", "functions", "feature_embed", "interaction_block", "readout", "processgraph"):
        importlib.import_module(f"matris.model.{name}")
    return pkg
