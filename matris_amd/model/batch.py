"""process_graphs on the device (row P1): batching, strain, edge geometry and the CSR
groupings every gather / segment kernel needs.

Mirrors matris/model/processgraph.py:6-245 (same keys and meaning).  Differences by
design: no host-side per-graph offset tensors, no [E, 3G] block-diagonal image matrix
(each edge reads its own graph's lattice), no bincount syncs; the groupings are stable
CSR structures built by matris_csr_build.
"""
from __future__ import annotations

import collections
import weakref

import torch

from . import ops
from .ops import Grouping


def _sorted(x: torch.Tensor) -> bool:
    return x.numel() < 2 or bool((x[1:] >= x[:-1]).all().item())


def validate_graph_indices(g) -> tuple:
    """Raise ValueError unless every index array of graph g is inside its range: atom_graph
    [E, 2] in [0, N), directed2undirected [E] in [0, U), undirected2directed [U] in [0, E)
    and the line graph's columns (center atom, bond, directed edge, bond, directed edge).
    The gather and segment kernels read rows through these indices, so they are checked
    before any of them runs: one host read per graph.  The result is remembered in g.meta
    under the index tensors' identities and version counters (RadiusGraph.index_signature),
    so an index tensor edited in place or replaced after a check is checked again.  Graphs
    built by GraphConverter are valid by construction and carry the mark already.
    Returns the signature."""
    sig = g.index_signature()
    if g.meta.get("indices_checked") == sig:
        return sig
    g.meta.pop("indices_checked", None)
    N = int(g.atomic_number.shape[0])
    E = int(g.atom_graph.shape[0])
    U = int(g.undirected2directed.shape[0])
    lg = g.line_graph
    if g.atom_graph.dim() != 2 or g.atom_graph.shape[1] != 2 or g.directed2undirected.shape[0] != E or \
            (len(lg) and (lg.dim() != 2 or lg.shape[1] != 5)):
        raise ValueError("graph index arrays have the wrong shape")
    checks = [(g.atom_graph, N), (g.directed2undirected, U), (g.undirected2directed, E)]
    if len(lg):
        checks += [(lg[:, 0], N), (lg[:, 1], U), (lg[:, 2], E), (lg[:, 3], U), (lg[:, 4], E)]
    flags = [((x < 0) | (x >= n)).any() for x, n in checks if x.numel()]
    if flags and bool(torch.stack(flags).any()):
        raise ValueError("graph index outside its range (atom, bond, directed-edge or angle index)")
    g.meta["indices_checked"] = sig
    return sig


def _topology(graphs, n_atoms, n_dir, n_und, n_ang) -> dict:
    """Everything of a batch that depends on its graphs' index arrays only: the int32 index
    columns (offset per graph) and their CSR groupings.  Deferred builds: a key outside
    its range surfaces in the status word that MatRIS.forward reads once per evaluation."""
    device = graphs[0].lattice.device
    N, E, U, A = sum(n_atoms), sum(n_dir), sum(n_und), sum(n_ang)
    canonical = all(g.meta.get("canonical", False) for g in graphs)
    a_off = u_off = d_off = 0
    ag, d2u, u2d, lgs = [], [], [], []
    for g, na, nd, nu, nl in zip(graphs, n_atoms, n_dir, n_und, n_ang):
        ag.append(g.atom_graph.to(torch.int32) + a_off)
        d2u.append(g.directed2undirected.to(torch.int32) + u_off)
        u2d.append(g.undirected2directed.to(torch.int32) + d_off)
        if nl:
            if a_off or u_off or d_off:
                off = torch.tensor([a_off, u_off, d_off, u_off, d_off], dtype=torch.int32, device=device)
                lgs.append(g.line_graph.to(torch.int32) + off)
            else:  # the first graph: no offsets, and no host-to-device copy
                lgs.append(g.line_graph.to(torch.int32))
        a_off += na
        u_off += nu
        d_off += nd
    atom_graph = torch.cat(ag, 0)
    tgt32 = atom_graph[:, 0].contiguous()
    src32 = atom_graph[:, 1].contiguous()
    d2u32 = torch.cat(d2u, 0).contiguous()
    u2d32 = torch.cat(u2d, 0).contiguous()
    # per-graph counts on the device, made once here: the evaluation itself then copies
    # nothing from the host (which also keeps it capturable in a HIP graph)
    atoms_len = torch.tensor(n_atoms, device=device)
    dir_len = torch.tensor(n_dir, device=device)
    zero = torch.zeros(1, dtype=torch.int32, device=device)
    atom_rowptr = torch.cat([zero, torch.cumsum(atoms_len, 0).to(torch.int32)])
    dir_rowptr = torch.cat([zero, torch.cumsum(dir_len, 0).to(torch.int32)])
    if len(graphs) == 1:
        atom_segment = torch.zeros(N, dtype=torch.long, device=device)
    else:
        atom_segment = torch.repeat_interleave(torch.arange(len(graphs), device=device), atoms_len, output_size=N)
    t = dict(atom_graph=atom_graph, tgt=tgt32.long(), src=src32.long(), d2u32=d2u32, u2d32=u2d32,
             d2u64=d2u32.long(), u2d64=u2d32.long(), atom_segment=atom_segment, atoms_len=atoms_len,
             dir_len=dir_len, atoms_per_graph32=atoms_len.to(torch.int32), atom_rowptr=atom_rowptr,
             dir_rowptr=dir_rowptr, atom_graph32=atom_segment.to(torch.int32),
             dir_graph32=(torch.zeros(E, dtype=torch.int32, device=device) if len(graphs) == 1 else
                          torch.repeat_interleave(torch.arange(len(graphs), device=device, dtype=torch.int32),
                                                  dir_len, output_size=E)),
             grp_tgt=Grouping.build(tgt32, N, sorted_rows=canonical or _sorted(tgt32), deferred=True),
             grp_src=Grouping.build(src32, N, deferred=True),
             grp_d2u=Grouping.build(d2u32, U, sorted_rows=False, deferred=True))
    if A:
        lg = torch.cat(lgs, 0)
        cols = [lg[:, k].contiguous() for k in range(5)]
        t["line_graph_dict"] = dict(
            line_graph=torch.stack((cols[0], cols[1], cols[3]), 1), atom_list=cols[0].long(),
            target_index=cols[1].long(), source_index=cols[3].long(), target_DE_index=cols[2].long(),
            source_DE_index=cols[4].long(),
            grp_tgt=Grouping.build(cols[1], U, sorted_rows=True, deferred=True),
            grp_src=Grouping.build(cols[3], U, deferred=True),
            grp_atom=Grouping.build(cols[0], N, deferred=True),
            # directed edges read by each angle (three-body basis and its backward)
            grp_de_t=Grouping.build(cols[2], E, deferred=True),
            grp_de_s=Grouping.build(cols[4], E, deferred=True))
    else:
        t["line_graph_dict"] = dict(line_graph=torch.zeros(0, 3, dtype=torch.int64, device=device))
    return t


# Topology of single graphs, remembered per graph object under its index signature (the
# identity, data pointer, storage, version and shape of every index tensor): an edited,
# replaced or moved index tensor misses.  Batches are remembered the same way, the last
# few of them, under their graphs' identities and signatures.  Positions, lattice and
# everything derived from them are recomputed on every call.
_TOPOLOGY: "weakref.WeakKeyDictionary" = weakref.WeakKeyDictionary()
_BATCH_TOPOLOGY: "collections.OrderedDict" = collections.OrderedDict()
_BATCH_TOPOLOGY_MAX = 4


def _batch_topology(graphs, sigs, n_atoms, n_dir, n_und, n_ang) -> dict:
    key = tuple(id(g) for g in graphs)
    hit = _BATCH_TOPOLOGY.get(key)
    if hit is not None:
        refs, hsigs, topo = hit
        if all(r() is g for r, g in zip(refs, graphs)) and hsigs == tuple(sigs):
            _BATCH_TOPOLOGY.move_to_end(key)
            return topo
    topo = _topology(graphs, n_atoms, n_dir, n_und, n_ang)
    _BATCH_TOPOLOGY[key] = ([weakref.ref(g) for g in graphs], tuple(sigs), topo)
    while len(_BATCH_TOPOLOGY) > _BATCH_TOPOLOGY_MAX:
        _BATCH_TOPOLOGY.popitem(last=False)
    return topo


def process_graphs(graphs, compute_stress: bool = True) -> dict:
    sigs = [validate_graph_indices(g) for g in graphs]
    device = graphs[0].lattice.device
    dtype = graphs[0].lattice.dtype
    G = len(graphs)
    n_atoms = [int(g.atomic_number.shape[0]) for g in graphs]
    n_dir = [int(g.atom_graph.shape[0]) for g in graphs]
    n_und = [int(g.undirected2directed.shape[0]) for g in graphs]
    n_ang = [int(g.line_graph.shape[0]) if len(g.line_graph) else 0 for g in graphs]
    N, E, U, A = sum(n_atoms), sum(n_dir), sum(n_und), sum(n_ang)
    if G == 1:
        sig = sigs[0]
        hit = _TOPOLOGY.get(graphs[0])
        if hit is None or hit[0] != sig:
            hit = (sig, _topology(graphs, n_atoms, n_dir, n_und, n_ang))
            _TOPOLOGY[graphs[0]] = hit
        topo = hit[1]
    else:
        topo = _batch_topology(graphs, sigs, n_atoms, n_dir, n_und, n_ang)

    if G == 1 and dtype == torch.float32 and graphs[0].atom_frac_coord.dtype == torch.float32 and \
            graphs[0].neighbor_image.dtype == torch.float32:
        return _one_graph(graphs[0], topo, compute_stress, n_atoms, N, E, U, A)

    atom_graph, tgt, src = topo["atom_graph"], topo["tgt"], topo["src"]
    d2u32, u2d32 = topo["d2u32"], topo["u2d32"]
    grp_tgt, grp_src = topo["grp_tgt"], topo["grp_src"]
    # fp32 throughout, the dtype of the reference's graphs (radiusgraph.py, `datatype`): a
    # graph built with integer images or fp64 coordinates is converted here
    f32 = torch.float32
    lattice = torch.cat([g.lattice.detach().to(f32) for g in graphs], 0)  # [3G, 3]
    image = torch.cat([g.neighbor_image.to(f32) for g in graphs], 0)
    atom_segment = topo["atom_segment"]
    lat3 = lattice.reshape(G, 3, 3)
    # processgraph.py:87 for every graph and the zero strains in one launch (each atom reads
    # its own graph's lattice) instead of one small product per graph
    frac = torch.cat([g.atom_frac_coord.detach().to(f32) for g in graphs], 0)
    cart, strains = ops.frac_to_cart_batch(frac, lat3, topo["atom_graph32"], compute_stress)
    cart.requires_grad_(True)
    if strains is not None:
        strains.requires_grad_(True)
    # the strain trick and the edge geometry (processgraph.py:169-199) of every graph in one
    # launch each way, each edge with its own graph's lattice and strain
    length, unit, lat_s, volumes = ops.edge_geometry_batch(cart, strains, lat3, image, grp_tgt, grp_src,
                                                           topo["dir_graph32"], topo["atom_rowptr"],
                                                           topo["dir_rowptr"])
    lattice = lat_s.reshape(-1, 3)

    out = dict(atomic_numbers=torch.cat([g.atomic_number for g in graphs], 0), edge_lengths=length,
               unit_edge_vectors=unit, atom_segment=atom_segment, atoms_per_graph=n_atoms,
               atoms_len=topo["atoms_len"], atoms_per_graph32=topo["atoms_per_graph32"],
               atom_rowptr=topo["atom_rowptr"],
               directed2undirected=topo["d2u64"], undirected2directed=topo["u2d64"], u2d32=topo["u2d32"],
               volumes=volumes,
               lattice=lattice, batch_cart_coords=cart, batch_strains=strains,
               n_atoms=N, n_directed=E, n_undirected=U, n_angles=A)
    out["grp_d2u"] = topo["grp_d2u"]
    out["atom_graph_dict"] = dict(
        atom_graph=atom_graph, target_index=tgt, source_index=src,
        grp_tgt=grp_tgt, grp_src=grp_src)
    out["line_graph_dict"] = dict(topo["line_graph_dict"])
    return out


def _one_graph(g, topo, compute_stress, n_atoms, N, E, U, A) -> dict:
    """process_graphs for one fp32 graph: the same fields, with the strain trick and the
    edge geometry (processgraph.py:169-199) in one launch (ops.edge_geometry) and the
    topology's columns used as they are (no per-call concatenations or casts).  Only the
    position leaf (frac @ lattice, processgraph.py:87) and the zero strain are made
    besides it, both in one more launch (ops.frac_to_cart), so the host issues few
    operations before the first layer."""
    lat = g.lattice.detach()
    cart, strains = ops.frac_to_cart(g.atom_frac_coord.detach(), lat, compute_stress)
    cart.requires_grad_(True)
    if strains is not None:
        strains.requires_grad_(True)
    grp_tgt, grp_src = topo["grp_tgt"], topo["grp_src"]
    length, unit, lattice, volumes = ops.edge_geometry(cart, strains, lat, g.neighbor_image, grp_tgt, grp_src)
    out = dict(atomic_numbers=g.atomic_number, edge_lengths=length, unit_edge_vectors=unit,
               atom_segment=topo["atom_segment"], atoms_per_graph=n_atoms, atoms_len=topo["atoms_len"],
               atoms_per_graph32=topo["atoms_per_graph32"],
               directed2undirected=topo["d2u64"], undirected2directed=topo["u2d64"], u2d32=topo["u2d32"],
               volumes=volumes,
               lattice=lattice, batch_cart_coords=cart, batch_strains=strains,
               n_atoms=N, n_directed=E, n_undirected=U, n_angles=A)
    out["grp_d2u"] = topo["grp_d2u"]
    out["atom_graph_dict"] = dict(atom_graph=topo["atom_graph"], target_index=topo["tgt"],
                                  source_index=topo["src"], grp_tgt=grp_tgt, grp_src=grp_src)
    out["line_graph_dict"] = dict(topo["line_graph_dict"])
    return out
