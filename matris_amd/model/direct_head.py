"""The direct (non-conservative) force and stress head of MatRIS, `is_conservation=False`
(readout.py:136-252, 255-334; functions.py:368-463), as torch layers on the device.

Forces: each directed edge's final bond features through an MLP to three weights, times
the edge's unit vector, summed over the edges of each centre atom.  Stress: a gated
equivariant network on the readout-normalised atom features and the l <= 2 harmonics of
each atom's position direction gives nine irrep components per atom; their per-structure
mean, read as an l = 0 and an l = 2 irrep (the l = 1 part dropped), is turned into a
symmetric 3 x 3 tensor and scaled by 160.21766208 / volume (eV/A^3 -> GPa).

The conservative head (forces and stress as gradients of the energy) is MatRIS's default
and the path the gfx950 kernels serve; this head is evaluated in the forward only.
"""
from __future__ import annotations

import math

import torch
from torch import Tensor, nn

from ..config import EV_A3_TO_GPA


def sphere_harmonics_l2(v: Tensor) -> Tensor:
    """[n, 9]: the real harmonics of l = 0, 1, 2 of the rows of v (x, y, z), in the order
    1; x, y, z; sqrt3 xz, sqrt3 xy, y^2 - (x^2 + z^2)/2, sqrt3 yz, sqrt3/2 (z^2 - x^2)
    (functions.py:436-463)."""
    x, y, z = v[..., 0], v[..., 1], v[..., 2]
    r3 = math.sqrt(3.0)
    return torch.stack([torch.ones_like(x), x, y, z, r3 * x * z, r3 * x * y, y * y - 0.5 * (x * x + z * z),
                        r3 * y * z, 0.5 * r3 * (z * z - x * x)], dim=-1)


def _irrep_to_cartesian() -> Tensor:
    """[9, 9]: row k maps irrep component k of a rank-2 tensor to its Cartesian entries
    (xx, xy, xz, yx, yy, yz, zx, zy, zz).  Row 0 is the trace part I / sqrt3; rows 1-3 the
    antisymmetric parts (yz - zy, zx - xz, xy - yx) / sqrt2; rows 4-8 the orthonormal
    symmetric traceless matrices T with r^T T r proportional to the l = 2 harmonics above,
    in their order (xz, xy, the y-axial one, yz, z^2 - x^2)."""
    def sym(a, b):
        m = torch.zeros(3, 3, dtype=torch.float64)
        m[a, b] = m[b, a] = 2 ** -0.5
        return m

    def anti(a, b):
        m = torch.zeros(3, 3, dtype=torch.float64)
        m[a, b], m[b, a] = 2 ** -0.5, -(2 ** -0.5)
        return m

    rows = [torch.eye(3, dtype=torch.float64) / math.sqrt(3.0), anti(1, 2), anti(2, 0), anti(0, 1),
            sym(0, 2), sym(0, 1), torch.diag(torch.tensor([-1.0, 2.0, -1.0], dtype=torch.float64)) / math.sqrt(6.0),
            sym(1, 2), torch.diag(torch.tensor([-1.0, 0.0, 1.0], dtype=torch.float64)) / math.sqrt(2.0)]
    return torch.stack([r.reshape(9) for r in rows]).float()


IRREP_TO_CARTESIAN = _irrep_to_cartesian()
_IRREP_ON = {}  # device -> its copy (made by the first eager evaluation, not inside a capture)


def stress_from_irreps(l0: Tensor, l2: Tensor) -> Tensor:
    """[G, 3, 3] from the l = 0 component l0 [G] and the l = 2 components l2 [G, 5]
    (reshape_stress, functions.py:414-433)."""
    m = _IRREP_ON.get(l0.device)
    if m is None:
        m = _IRREP_ON[l0.device] = IRREP_TO_CARTESIAN.to(l0.device)
    return (l0[:, None] * m[0] + l2 @ m[4:]).view(-1, 3, 3)


class GatedEquivariantBlock(nn.Module):
    """readout.py:255-292 (Schuett et al. 2021): scalar features s [N, h] and vector
    features V [N, 9, h]; s' , g = split(MLP([s, |W1 V|])), V' = g * (W2 V)."""

    def __init__(self, hidden_channels: int, out_channels: int, activation=None):
        super().__init__()
        self.out_channels = out_channels
        self.vec1_proj = nn.Linear(hidden_channels, hidden_channels, bias=False)
        self.vec2_proj = nn.Linear(hidden_channels, out_channels, bias=False)
        self.act = activation
        self.update_net = nn.Sequential(nn.Linear(hidden_channels * 2, hidden_channels), self.act,
                                        nn.Linear(hidden_channels, out_channels * 2))

    def forward(self, feas: Tensor, vec_feas: Tensor):
        vec1 = torch.norm(self.vec1_proj(vec_feas), dim=-2)
        vec2 = self.vec2_proj(vec_feas)
        feas, gate = torch.split(self.update_net(torch.cat([feas, vec1], dim=-1)), self.out_channels, dim=-1)
        vec_feas = gate.unsqueeze(1) * vec2
        if self.act is not None:
            feas = self.act(feas)
        return feas, vec_feas


class EquivariantHead(nn.Module):
    """readout.py:295-334 with lmax = 2: [N, 9] irrep components per atom."""

    def __init__(self, feas_dim: int = 64, lmax: int = 2, use_bias: bool = False, make_activation=None):
        """make_activation() gives each block its own activation module (or None)."""
        super().__init__()
        if lmax != 2:
            raise NotImplementedError("the stress head reads the l = 0 and l = 2 components (lmax = 2)")
        act = make_activation or (lambda: None)
        self.feas_wise_linear = nn.Linear(feas_dim, feas_dim, bias=False)
        self.basis_wise_linear = nn.Linear(1, feas_dim, bias=False)
        self.equivariant_block = nn.ModuleList([
            GatedEquivariantBlock(feas_dim, feas_dim // 2, activation=act()),
            GatedEquivariantBlock(feas_dim // 2, 1, activation=act())])

    def forward(self, feas: Tensor, vec: Tensor) -> Tensor:
        vec_feas = self.basis_wise_linear(sphere_harmonics_l2(vec).unsqueeze(2))  # [N, 9, dim]
        feas = self.feas_wise_linear(feas)
        for layer in self.equivariant_block:
            feas, vec_feas = layer(feas, vec_feas)
        return vec_feas.squeeze(-1)  # [N, 9]


def direct_forces(force_head: nn.Module, edge_feat: Tensor, bg: dict) -> Tensor:
    """[N, 3]: sum over each centre atom's directed edges of force_head(bond features of
    the edge) * unit edge vector (readout.py:240-251)."""
    w = force_head(torch.index_select(edge_feat, 0, bg["directed2undirected"]))  # [E_d, 3]
    contrib = w * bg["unit_edge_vectors"]
    n = bg["atomic_numbers"].shape[0]
    out = torch.zeros(n, 3, dtype=contrib.dtype, device=contrib.device)
    return out.index_add_(0, bg["atom_graph_dict"]["target_index"], contrib)


def direct_stress(stress_head: EquivariantHead, node_feat: Tensor, bg: dict) -> Tensor:
    """[G, 3, 3] in GPa (readout.py:225-239): the head on the atom features and position
    directions, averaged per structure, converted from irreps, over the cell volume."""
    from . import ops
    coord = bg["batch_cart_coords"]
    direction = coord / (torch.norm(coord, dim=1) * (1 - 1e-6) + 1e-6).unsqueeze(1)
    comp = stress_head(node_feat, direction)  # [N, 9]
    n_graphs = len(bg["atoms_per_graph"])
    rowptr = bg.get("atom_rowptr")  # atoms of a structure are contiguous
    if rowptr is None:  # one structure: [0, N] made on the device (no host copy, capturable)
        apg = bg["atoms_per_graph32"]
        rowptr = torch.cat([apg.new_zeros(1), apg])
    sums = ops.seg_sum_narrow_raw(comp, rowptr, n_graphs)
    mean = sums / bg["atoms_per_graph32"].to(sums.dtype)[:, None]
    stress = stress_from_irreps(mean[:, 0], mean[:, 4:9])
    return stress * (EV_A3_TO_GPA / bg["volumes"]).view(-1, 1, 1)
