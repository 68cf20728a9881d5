"""RadiusGraph: the per-structure graph container of the reference
(matris/graph/radiusgraph.py:17-175), same field names, dtypes and methods.

Graphs built by this package's GraphConverter additionally carry `meta`, a dict of
device-side extras (canonical-order flag, reverse-edge index, fp64 distances) that
process_graphs uses to skip work; reference-built graphs simply lack it.
"""
from __future__ import annotations

import os
from typing import Any

import torch
from torch import Tensor

datatype = torch.float32


class RadiusGraph:
    def __init__(self, graph_id: str | None, mp_id: str | None, composition: str | None, atomic_number: Tensor,
                 atom_frac_coord: Tensor, lattice: Tensor, neighbor_image: Tensor, atom_graph: Tensor,
                 atom_graph_cutoff: float, line_graph: Tensor, line_graph_cutoff: float,
                 directed2undirected: Tensor, undirected2directed: Tensor, meta: dict | None = None):
        self.graph_id = graph_id
        self.mp_id = mp_id
        self.composition = composition
        self.atomic_number = atomic_number
        self.atom_frac_coord = atom_frac_coord
        self.lattice = lattice
        self.neighbor_image = neighbor_image
        self.line_graph = line_graph
        self.line_graph_cutoff = line_graph_cutoff
        self.atom_graph = atom_graph
        self.atom_graph_cutoff = atom_graph_cutoff
        self.directed2undirected = directed2undirected
        self.undirected2directed = undirected2directed
        self.meta = meta or {}
        # radiusgraph.py:92-95
        assert len(directed2undirected) == 2 * len(undirected2directed), (
            f"Number of directed indices ({len(directed2undirected)}) != "
            f"2 * number of undirected indices ({2 * len(undirected2directed)})!")

    _FIELDS = ("atomic_number", "atom_frac_coord", "lattice", "neighbor_image", "atom_graph", "line_graph",
               "directed2undirected", "undirected2directed")
    _INDEX_FIELDS = ("atomic_number", "atom_graph", "line_graph", "directed2undirected", "undirected2directed")

    def index_signature(self) -> tuple:
        """Identity and version of every index tensor (and the atom count).  Any in-place
        edit bumps a tensor's version counter and assigning a new tensor changes its
        identity, so a range check remembered under this signature -- and the topology
        (CSR groupings) that process_graphs keeps per graph under it -- is redone after
        either.  A storage swapped in through `.data = ...` or `set_()` bumps no version
        counter; the signature also holds the address of the storage object, which such a
        swap changes, but an allocator that hands the old addresses back cannot be told
        apart.  Edit index tensors in place or assign new tensors; do not swap their storage
        through `.data` or `set_()`."""
        return tuple((f, id(t), t.data_ptr(), t.untyped_storage()._cdata, t._version, tuple(t.shape))
                     for f in self._INDEX_FIELDS for t in (getattr(self, f),))

    def to(self, device: str = "cpu") -> "RadiusGraph":
        """radiusgraph.py:97-113."""
        kw = {f: getattr(self, f).to(device) for f in self._FIELDS}
        meta = {k: (v.to(device) if isinstance(v, Tensor) else v) for k, v in self.meta.items()}
        return RadiusGraph(graph_id=self.graph_id, mp_id=self.mp_id, composition=self.composition,
                           atom_graph_cutoff=self.atom_graph_cutoff, line_graph_cutoff=self.line_graph_cutoff,
                           meta=meta, **kw)

    def to_dict(self) -> dict[str, Any]:
        """radiusgraph.py:115-130 (the reference keys only)."""
        d = {"graph_id": self.graph_id, "mp_id": self.mp_id, "composition": self.composition}
        d.update({f: getattr(self, f) for f in self._FIELDS})
        d["atom_graph_cutoff"] = self.atom_graph_cutoff
        d["line_graph_cutoff"] = self.line_graph_cutoff
        return d

    def save(self, fname: str | None = None, save_dir: str = ".") -> str:
        """radiusgraph.py:132-146 (a torch.save of to_dict())."""
        if fname is not None:
            name = os.path.join(save_dir, fname)
        elif self.graph_id is not None:
            name = os.path.join(save_dir, f"{self.graph_id}.pt")
        else:
            name = os.path.join(save_dir, f"{self.composition}.pt")
        torch.save({k: (v.cpu() if isinstance(v, Tensor) else v) for k, v in self.to_dict().items()}, f=name)
        return name

    @classmethod
    def from_file(cls, file_name: str) -> "RadiusGraph":
        """Load a file written by save() (tensors only: weights_only loading)."""
        obj = torch.load(file_name, weights_only=True)
        return cls.from_dict(obj) if isinstance(obj, dict) else obj

    @classmethod
    def from_dict(cls, dic: dict[str, Any]) -> "RadiusGraph":
        return cls(**dic)

    def __repr__(self) -> str:
        return (f"RadiusGraph(composition={self.composition!r}, atom_graph_cutoff={self.atom_graph_cutoff}, "
                f"line_graph_cutoff={self.line_graph_cutoff}, n_atoms={len(self.atomic_number)}, "
                f"atom_graph_len={len(self.atom_graph)}, line_graph_len={len(self.line_graph)})")
