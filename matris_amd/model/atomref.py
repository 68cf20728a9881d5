"""Elemental reference energy (reference_energy.py:14-201): a bias-free linear model on the
composition.  For graph g with atomic numbers Z, feature c_z = (number of atoms with
Z = z) [/ n_atoms when intensive], z = 1 .. 94, and E_ref(g) = w . c.  The weights come
pre-fitted from one of three datasets (atomref_tables) or from a least-squares fit.
Same module layout (`fc`, a Linear(94, 1) without bias) and state_dict keys as the
reference, so checkpoints that carry `reference_energy.fc.weight` load unchanged."""
from __future__ import annotations

from collections.abc import Sequence

import numpy as np
import torch
from torch import nn

from .atomref_tables import TABLES


class AtomRef(nn.Module):
    def __init__(self, reference_energy: str | None = None, is_intensive: bool = True,
                 max_num_elements: int = 94) -> None:
        super().__init__()
        self.is_intensive = is_intensive
        self.max_num_elements = max_num_elements
        # created like the reference's, so it consumes the same random numbers at construction
        self.fc = nn.Linear(max_num_elements, 1, bias=False)
        self.fitted = False
        if reference_energy is not None:
            self.initialize_from(reference_energy)
        for p in self.parameters():
            p.requires_grad = False

    def initialize_from_MPtrj(self) -> None:
        """reference_energy.py:116-145: the MPtrj table."""
        self.initialize_from("mptrj")

    def initialize_from_OMat(self) -> None:
        """reference_energy.py:147-176: the OMat24 table."""
        self.initialize_from("omat")

    def initialize_from_MPA(self) -> None:
        """reference_energy.py:178-207: the sAlex + MPtrj table."""
        self.initialize_from("mpa")

    def initialize_from(self, dataset: str) -> None:
        """Load a pre-fitted table: "mptrj" (or "demo"), "omat" or "mpa" (all intensive)."""
        key = dataset.lower()
        if key not in TABLES:
            raise NotImplementedError(f"{dataset=} not supported yet")
        with torch.no_grad():
            self.fc.weight.copy_(torch.tensor(TABLES[key], dtype=torch.float32).view(1, -1))
        self.is_intensive = True
        self.fitted = True

    def _composition(self, atomic_number: torch.Tensor) -> torch.Tensor:
        c = torch.bincount(atomic_number.long() - 1, minlength=self.max_num_elements)
        if self.is_intensive:
            c = c / atomic_number.shape[0]
        return c

    def forward(self, graphs) -> torch.Tensor:
        """E_ref of each graph, [G] (float32, on the graphs' device)."""
        feats = torch.stack([self._composition(g.atomic_number) for g in graphs], 0).float()
        return self.fc(feats.to(self.fc.weight.device)).view(-1)

    def fit(self, structures_or_graphs: Sequence, energies: Sequence[float]) -> None:
        """Least-squares weights w = pinv(C^T C) C^T e over the given structures or graphs
        (reference_energy.py:57-101: RadiusGraph objects with an `atomic_number` tensor, or
        structures with `atomic_numbers`, as pymatgen's Structure) and their energies."""
        def numbers(x):
            z = x.atomic_number if hasattr(x, "atomic_number") else x.atomic_numbers
            return torch.as_tensor(np.asarray(z.cpu() if torch.is_tensor(z) else z, dtype=np.int64))

        feats = np.stack([self._composition(numbers(x)).float().cpu().numpy() for x in structures_or_graphs], 0)
        e = np.asarray(energies, dtype=np.float32)
        w = np.linalg.pinv(feats.T @ feats) @ feats.T @ e
        with torch.no_grad():
            self.fc.weight.copy_(torch.as_tensor(w, dtype=torch.float32).view(1, -1))
        self.fitted = True
