"""GraphConverter on the GPU (rows G1-G6).

Mirrors the reference GraphConverter (matris/graph/converter.py:22-129): the same
constructor arguments, `forward(structure, graph_id, mp_id) -> RadiusGraph`, the same
RadiusGraph field dtypes and the same error behaviour (isolated atom -> ValueError;
line-graph failure -> the structure written to error_graph.cif and an empty line graph).  The host work of the reference (pymatgen
neighbour search, C/Cython pairing, the Python line-graph loop) is replaced by the
gfx950 kernels of libmatris_hip.so, driven through the C ABI:

  matris_radius_graph_count/fill   periodic radius graph, canonical order, fp64
  matris_pair_edges                directed -> undirected pairing (d2u, u2d)
  matris_line_graph_count/fill     bond -> angle line graph, rows sorted by u1

The only host readbacks are the three sizes (E_d, E_u, A) plus the isolated-atom check.
"""
from __future__ import annotations

import ctypes
import warnings

import numpy as np
import torch
from torch import nn

from .. import _lib
from .cif import write_cif
from .radiusgraph import RadiusGraph, datatype


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _structure_arrays(structure):
    """(frac fp64 [n,3], lattice fp64 [3,3], Z int [n], formula) from a pymatgen Structure,
    an ASE Atoms, an object with frac/lattice/z attributes, or a (frac, lattice, z) tuple."""
    if hasattr(structure, "frac_coords") and hasattr(structure, "lattice"):  # pymatgen Structure
        frac = np.asarray(structure.frac_coords, dtype=np.float64)
        lat = np.asarray(structure.lattice.matrix, dtype=np.float64)
        z = np.array([site.specie.Z for site in structure], dtype=np.int64)
        return frac, lat, z, structure.composition.formula
    if hasattr(structure, "get_scaled_positions") and hasattr(structure, "cell"):  # ASE Atoms
        frac = np.asarray(structure.get_scaled_positions(wrap=False), dtype=np.float64)
        lat = np.asarray(structure.cell.array, dtype=np.float64)
        z = np.asarray(structure.numbers, dtype=np.int64)
        return frac, lat, z, structure.get_chemical_formula()
    if hasattr(structure, "frac") and hasattr(structure, "lattice"):
        return (np.asarray(structure.frac, np.float64), np.asarray(structure.lattice, np.float64),
                np.asarray(structure.z, np.int64), None)
    frac, lat, z = structure
    return np.asarray(frac, np.float64), np.asarray(lat, np.float64), np.asarray(z, np.int64), None


def radius_graph_device(frac: torch.Tensor, lattice: np.ndarray, cutoff: float, tol: float = 1e-8):
    """G1 on the device.  frac: fp64 [n,3] device tensor.  Returns
    (center, neighbor, image int32 [E,3], dist fp64, row_ptr int64 [n+1], row_count int32)."""
    lib = _lib.load()
    dev = frac.device
    if frac.dtype != torch.float64 or frac.dim() != 2 or frac.shape[1] != 3:
        raise ValueError(f"frac must be fp64 [n, 3], got {frac.dtype} {tuple(frac.shape)}")
    frac = frac.contiguous()
    n = frac.shape[0]
    lat = np.ascontiguousarray(lattice, dtype=np.float64)
    grid = (ctypes.c_int * 3)()
    search = (ctypes.c_int * 3)()
    _lib.check(lib.matris_radius_graph_plan(lat.ctypes.data_as(ctypes.c_void_p), float(cutoff), grid, search),
               "matris_radius_graph_plan")
    ws_bytes = lib.matris_radius_graph_workspace_bytes(n, grid)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    row_count = torch.empty(n, dtype=torch.int32, device=dev)
    row_ptr = torch.empty(n + 1, dtype=torch.int64, device=dev)
    latp = lat.ctypes.data_as(ctypes.c_void_p)
    _lib.check(lib.matris_radius_graph_count(n, _p(frac), latp, float(cutoff), float(tol), grid, search,
                                             _p(row_count), _p(row_ptr), _p(ws), ws_bytes, _stream()),
               "matris_radius_graph_count")
    E = int(row_ptr[n].item())
    center = torch.empty(max(E, 1), dtype=torch.int32, device=dev)
    neighbor = torch.empty(max(E, 1), dtype=torch.int32, device=dev)
    image = torch.empty(max(E, 1), 3, dtype=torch.int32, device=dev)
    dist = torch.empty(max(E, 1), dtype=torch.float64, device=dev)
    _lib.check(lib.matris_radius_graph_fill(n, latp, float(cutoff), float(tol), grid, search, _p(row_ptr),
                                            _p(center), _p(neighbor), _p(image), _p(dist), _p(ws), ws_bytes,
                                            _stream()), "matris_radius_graph_fill")
    return center[:E], neighbor[:E], image[:E], dist[:E], row_ptr, row_count


class SkinNeighborList:
    """G1 with Verlet-skin reuse for MD (no counterpart in the reference, which rebuilds the
    neighbour list every step, base.py:96-97).  Candidates come from one radius graph at
    cutoff + skin; each later call re-decides them on the current coordinates on the GPU
    (matris_skin_filter_count/fill) until some atom has moved skin / 2 or more since the
    candidate build, which triggers a fresh candidate build.  Every call returns exactly
    what radius_graph_device(frac, lattice, cutoff) returns for the same frac.

    update(frac, x, pos): frac = the wrapped fractional coordinates the graph is built
    from (fp64 [n,3] device), x = the same coordinates unwrapped (frac = x - integer),
    pos = unwrapped Cartesian positions (fp64 [n,3]), used for the displacement test.
    The lattice is fixed for the list's lifetime."""

    def __init__(self, lattice: np.ndarray, cutoff: float, skin: float, tol: float = 1e-8):
        if not skin > 0:
            raise ValueError(f"skin must be positive, got {skin}")
        self.lattice = np.ascontiguousarray(lattice, dtype=np.float64)
        self.cutoff, self.skin, self.tol = float(cutoff), float(skin), float(tol)
        self.n_builds = 0
        self._cand = None

    def _rebuild(self, frac, x, pos):
        c, nb, im, _, rp, _ = radius_graph_device(frac, self.lattice, self.cutoff + self.skin, self.tol)
        self._cand = (c.contiguous(), nb.contiguous(), im.contiguous(), rp)
        self._frame0 = (x - frac).clone()  # the integer wrap of every atom at the candidate build
        self._pos0 = pos.clone()
        self.n_builds += 1

    def update(self, frac: torch.Tensor, x: torch.Tensor, pos: torch.Tensor):
        """(center, neighbor, image int32 [E,3], dist fp64, row_ptr int64 [n+1], row_count int32)."""
        frac = frac.contiguous()
        n = frac.shape[0]
        if self._cand is None or self._cand[3].shape[0] != n + 1:
            self._rebuild(frac, x, pos)
        else:
            # strict margin below skin / 2: the rounding of the candidate decisions cannot matter
            moved = float(torch.linalg.vector_norm(pos - self._pos0, dim=1).max().item())
            if moved >= 0.5 * self.skin * (1.0 - 1e-9):
                self._rebuild(frac, x, pos)
        cc, cn, ci, crp = self._cand
        dk = torch.round((x - frac) - self._frame0).to(torch.int32).contiguous()
        lib = _lib.load()
        dev = frac.device
        n_cand = cc.shape[0]
        ws_bytes = lib.matris_skin_filter_workspace_bytes(n_cand)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        row_count = torch.empty(n, dtype=torch.int32, device=dev)
        row_ptr = torch.empty(n + 1, dtype=torch.int64, device=dev)
        latp = self.lattice.ctypes.data_as(ctypes.c_void_p)
        _lib.check(lib.matris_skin_filter_count(n, n_cand, _p(frac), latp, self.cutoff, self.tol, _p(cc), _p(cn),
                                                _p(ci), _p(crp), _p(dk), _p(row_count), _p(row_ptr), _p(ws),
                                                ws_bytes, _stream()), "matris_skin_filter_count")
        E = int(row_ptr[n].item())
        center = torch.empty(max(E, 1), dtype=torch.int32, device=dev)
        neighbor = torch.empty(max(E, 1), dtype=torch.int32, device=dev)
        image = torch.empty(max(E, 1), 3, dtype=torch.int32, device=dev)
        dist = torch.empty(max(E, 1), dtype=torch.float64, device=dev)
        _lib.check(lib.matris_skin_filter_fill(n, n_cand, _p(frac), latp, self.cutoff, self.tol, _p(cc), _p(cn),
                                               _p(ci), _p(dk), _p(center), _p(neighbor), _p(image), _p(dist),
                                               _p(ws), ws_bytes, _stream()), "matris_skin_filter_fill")
        return center[:E], neighbor[:E], image[:E], dist[:E], row_ptr, row_count


def pair_edges_device(n: int, center, neighbor, image, row_ptr):
    """G3/G4 on the device: (rev, d2u, u2d, u_second)."""
    lib = _lib.load()
    dev = center.device
    E = center.shape[0]
    rev = torch.empty(E, dtype=torch.int32, device=dev)
    d2u = torch.empty(E, dtype=torch.int32, device=dev)
    u2d = torch.empty(E, dtype=torch.int32, device=dev)
    u_second = torch.empty(E, dtype=torch.int32, device=dev)
    ws_bytes = lib.matris_pair_edges_workspace_bytes(E)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    nu = ctypes.c_int64(0)
    _lib.check(lib.matris_pair_edges(n, E, _p(center), _p(neighbor), _p(image), _p(row_ptr), _p(rev), _p(d2u),
                                     _p(u2d), _p(u_second), ctypes.byref(nu), _p(ws), ws_bytes, _stream()),
               "matris_pair_edges")
    U = nu.value
    return rev, d2u, u2d[:U], u_second[:U]


def line_graph_device(n: int, center, neighbor, dist, row_ptr, d2u, u2d, u_second, cutoff: float):
    """G5 on the device: (line_graph int32 [A,5], angle_ptr int32 [E_u+1])."""
    lib = _lib.load()
    dev = center.device
    E, U = center.shape[0], u2d.shape[0]
    angle_ptr = torch.empty(U + 1, dtype=torch.int32, device=dev)
    ws_bytes = lib.matris_line_graph_workspace_bytes(n, U)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    na = ctypes.c_int64(0)
    _lib.check(lib.matris_line_graph_count(n, E, U, _p(center), _p(neighbor), _p(dist), _p(row_ptr), _p(u2d),
                                           _p(u_second), float(cutoff), _p(angle_ptr), ctypes.byref(na), _p(ws),
                                           ws_bytes, _stream()), "matris_line_graph_count")
    A = na.value
    lg = torch.empty(max(A, 1), 5, dtype=torch.int32, device=dev)
    if A > 0:
        _lib.check(lib.matris_line_graph_fill(n, E, U, _p(center), _p(neighbor), _p(dist), _p(row_ptr), _p(d2u),
                                              _p(u2d), _p(u_second), float(cutoff), _p(angle_ptr), _p(lg),
                                              _stream()), "matris_line_graph_fill")
    return lg[:A], angle_ptr


class GraphConverter(nn.Module):
    """Convert a structure to a RadiusGraph on the GPU (converter.py:22-129)."""

    def __init__(self, atom_graph_cutoff: float = 6, line_graph_cutoff: float = 4, verbose: bool = False,
                 device: str | torch.device | None = None) -> None:
        super().__init__()
        self.atom_graph_cutoff = atom_graph_cutoff
        self.line_graph_cutoff = atom_graph_cutoff if line_graph_cutoff is None else line_graph_cutoff
        self.algorithm = "gfx950"
        self.device = device
        if verbose:
            print(self)

    def __repr__(self) -> str:
        return (f"GraphConverter(algorithm={self.algorithm!r}, atom_graph_cutoff={self.atom_graph_cutoff}, "
                f"line_graph_cutoff={self.line_graph_cutoff})")

    def _device(self):
        if self.device is not None:
            return torch.device(self.device)
        return torch.device("cuda", torch.cuda.current_device())

    def forward(self, structure, graph_id=None, mp_id=None) -> RadiusGraph:
        frac, lat, z, formula = _structure_arrays(structure)
        return self.from_arrays(frac, lat, z, graph_id=graph_id, mp_id=mp_id, composition=formula)

    def from_arrays(self, frac, lattice, z, graph_id=None, mp_id=None, composition=None,
                    frac_device: torch.Tensor | None = None, neighbors=None) -> RadiusGraph:
        """Build from fractional coordinates (fp64), lattice rows (fp64) and atomic numbers.
        frac_device: an fp64 device copy of frac, when the caller already holds one.
        neighbors: the atom-graph edges when the caller already holds them for this frac and
        the atom-graph cutoff (SkinNeighborList.update's result)."""
        dev = self._device()
        n = len(z)
        lat = np.asarray(lattice, dtype=np.float64)
        # the kernels read [n, 3] row-major: make any strided input (a transposed or
        # Fortran-ordered array, a column slice) contiguous first
        f64 = (frac_device if frac_device is not None else
               torch.as_tensor(np.ascontiguousarray(frac, dtype=np.float64), device=dev)).contiguous()
        center, neighbor, image, dist, row_ptr, row_count = (
            neighbors if neighbors is not None else radius_graph_device(f64, lat, self.atom_graph_cutoff))
        # converter.py:108-113: isolated atoms stop the calculation
        n_isolated = int((row_count == 0).sum().item())
        if n_isolated:
            raise ValueError(f"Error: Detected {n_isolated} isolated atom. Calculation stopped")
        rev, d2u, u2d, u_second = pair_edges_device(n, center, neighbor, image, row_ptr)
        try:
            lg, angle_ptr = line_graph_device(n, center, neighbor, dist, row_ptr, d2u, u2d, u_second,
                                              self.line_graph_cutoff)
        except RuntimeError as exc:
            # converter.py:99-106: the structure is dumped to error_graph.cif in the working
            # directory and the graph keeps an empty line graph
            try:
                write_cif("error_graph.cif", frac if frac is not None else f64.cpu().numpy(), lat, z)
                where = "the structure was written to error_graph.cif"
            except OSError as err:  # an unwritable working directory must not hide the failure
                where = f"error_graph.cif could not be written ({err})"
            warnings.warn(f"line graph construction failed ({exc}); {where} and the line graph is empty")
            lg = torch.zeros(0, 5, dtype=torch.int32, device=dev)
            angle_ptr = None
        atom_graph = torch.stack([center, neighbor], dim=1)
        # the indices come from this builder's own kernels: valid by construction
        meta = dict(canonical=True, dist=dist, rev=rev, u_second=u_second, row_ptr=row_ptr, angle_ptr=angle_ptr,
                    frac64=f64)
        g = RadiusGraph(
            graph_id=graph_id, mp_id=mp_id, composition=composition,
            atomic_number=torch.as_tensor(np.asarray(z), dtype=torch.int32, device=dev),
            atom_frac_coord=f64.to(datatype),
            lattice=torch.as_tensor(lat, dtype=datatype, device=dev),
            neighbor_image=image.to(datatype),
            atom_graph=atom_graph,
            atom_graph_cutoff=self.atom_graph_cutoff,
            line_graph=lg,
            line_graph_cutoff=self.line_graph_cutoff,
            directed2undirected=d2u,
            undirected2directed=u2d,
            meta=meta)
        g.meta["indices_checked"] = g.index_signature()
        return g

    def as_dict(self) -> dict:
        return {"atom_graph_cutoff": self.atom_graph_cutoff, "line_graph_cutoff": self.line_graph_cutoff,
                "algorithm": self.algorithm}

    @classmethod
    def from_dict(cls, dict) -> "GraphConverter":  # noqa: A002 (the reference's parameter name)
        kwargs = {k: v for k, v in dict.items() if k != "algorithm"}
        return cls(**kwargs)
