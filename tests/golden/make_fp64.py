"""Write tests/golden/fp64_oracle.npz: the CPU oracle (oracle/model_ref.py) evaluated in
fp64 on the same graphs and seed-0 weights as the reference golden fixtures.

Purpose: it measures the fp32 noise floor of the reference computation itself
(|e_ref_fp32 - e_fp64|).  The random-init model's energies are small sums with strong
cancellation (e.g. C1 e = -1.4e-3 eV/atom, and the three-body basis evaluates spherical
Bessel functions at x = 1/6 where j_3 ~ x^3/105 cancels between O(1) terms).

The fp64 model computes the same function as the fp32 one: nn.RMSNorm(eps=None) takes
eps = finfo(input dtype).eps, 1.19e-7 for the fp32 reference but 2.2e-16 in float64, and
rows whose mean square is small (the symmetric C1 cell, bias-free MLP-then-norm updates)
feel the difference (6e-4 of the C1 energy), so every RMSNorm here gets the fp32 constant.

    python tests/golden/make_fp64.py [--big]
    python tests/golden/make_fp64.py --only variants    (the non-default forms and options)
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from matris_amd.config import DEFAULT_CONFIG, MATRIS_10M  # noqa: E402
from oracle.model_ref import MatRISRef  # noqa: E402


def graph(z, prefix):
    dt = torch.float64
    return dict(atomic_number=torch.tensor(z[prefix + "z"], dtype=torch.int32),
                atom_frac_coord=torch.tensor(z[prefix + "frac"], dtype=dt),
                lattice=torch.tensor(z[prefix + "lattice"], dtype=dt),
                neighbor_image=torch.tensor(z[prefix + "image"], dtype=dt),
                atom_graph=torch.tensor(z[prefix + "atom_graph"], dtype=torch.int32),
                directed2undirected=torch.tensor(z[prefix + "d2u"], dtype=torch.int32),
                undirected2directed=torch.tensor(z[prefix + "u2d"], dtype=torch.int32),
                line_graph=torch.tensor(z[prefix + "line_graph"], dtype=torch.int32))


EPS32 = float(torch.finfo(torch.float32).eps)

# the non-default update forms of tests/golden/configs.npz and the other constructor
# options of tests/golden/options.npz (two blocks, seed 0)
VARIANTS = {"ln": dict(norm_type="layer"), "bn": dict(norm_type="batch"),
            "mlp": dict(graph_conv_mlp="MLP"), "mlp_ln": dict(graph_conv_mlp="MLP", norm_type="layer"),
            "gauss": dict(distance_expansion="Gaussian"), "fourier": dict(three_body_expansion="fourier"),
            "sh33": dict(max_n=3, max_l=3), "sh24": dict(max_n=2, max_l=4),
            "noenv": dict(envelope_exponent=None), "nr9": dict(num_radial=9, num_angular=9),
            "fixed": dict(learnable_basis=False), "extensive": dict(is_intensive=False),
            "direct": dict(is_conservation=False), "gelu": dict(activation_type="gelu"),
            "relu": dict(activation_type="relu"),
            "dim64": dict(node_feat_dim=64, edge_feat_dim=64, three_body_feat_dim=64, mlp_hidden_dims=(64, 64)),
            "mixed": dict(node_feat_dim=128, edge_feat_dim=96, three_body_feat_dim=64)}


def model64(cfg):
    torch.manual_seed(0)
    m = MatRISRef(**cfg).eval().double()
    for mod in m.modules():
        if hasattr(mod, "coef"):
            mod.coef = mod.coef.double()
        if isinstance(mod, torch.nn.RMSNorm) and mod.eps is None:
            mod.eps = EPS32
    return m


def run(m, graphs, energy_only=False):
    if energy_only:  # forward only: the fp64 autograd tape of C3 does not fit in host memory
        with torch.no_grad():
            o = m(graphs, task="em")
        return dict(e=o["e"].detach().numpy(), m=torch.cat(o["m"]).detach().numpy())
    o = m(graphs, task="efsm")
    return dict(e=o["e"].detach().numpy(), f=torch.cat(o["f"]).detach().numpy(),
                s=torch.stack(o["s"]).detach().numpy(), m=torch.cat(o["m"]).detach().numpy())


def _oracle_graph(cr):
    from oracle import graph_ref
    og = graph_ref.build_graph(cr.frac, cr.lattice, cr.z)
    return graph(dict(g_z=cr.z, g_frac=cr.frac, g_lattice=cr.lattice, g_image=og["image"],
                      g_atom_graph=np.stack([og["center"], og["neighbor"]], 1), g_d2u=og["d2u"], g_u2d=og["u2d"],
                      g_line_graph=og["line_graph"]), "g_")


def main():
    """python tests/golden/make_fp64.py [--big] [--only degenerate c4 variants]: --only adds
    or replaces just those entries of the existing fp64_oracle.npz."""
    torch.set_num_threads(8)
    path = os.path.join(HERE, "fp64_oracle.npz")
    only = sys.argv[sys.argv.index("--only") + 1:] if "--only" in sys.argv else None
    out = dict(np.load(path)) if only else {}
    m10 = model64(MATRIS_10M)
    if only is None:
        z = np.load(os.path.join(HERE, "c1_cu4.npz"))
        for k, v in run(m10, [graph(z, "g_")]).items():
            out[f"c1_{k}"] = v
        for k, v in run(model64(DEFAULT_CONFIG), [graph(z, "g_")]).items():
            out[f"c1l6_{k}"] = v
        z = np.load(os.path.join(HERE, "cells_small.npz"))
        for k, v in run(m10, [graph(z, f"g{i}_") for i in range(int(z["n_cells"]))]).items():
            out[f"cells_{k}"] = v
    if only is None and "--big" in sys.argv:
        from matris_amd import workloads as W
        for k, v in run(m10, [_oracle_graph(W.c3_cu864())], energy_only=True).items():
            out[f"c3_{k}"] = v
    if only is None or "degenerate" in only:
        z = np.load(os.path.join(HERE, "degenerate.npz"))
        for k, v in run(m10, [graph(z, "dil_")]).items():
            out[f"dil_{k}"] = v
        for k, v in run(m10, [graph(z, p) for p in ("cu_", "dil_", "tri_")]).items():
            out[f"mixed_{k}"] = v
    if only is None or "variants" in only:
        zc, zs = np.load(os.path.join(HERE, "c1_cu4.npz")), np.load(os.path.join(HERE, "cells_small.npz"))
        for name, over in VARIANTS.items():
            m = model64(dict(DEFAULT_CONFIG, num_layers=2, **over))
            for k, v in run(m, [graph(zc, "g_")]).items():
                out[f"{name}_c1_{k}"] = v
            for k, v in run(m, [graph(zs, f"g{i}_") for i in range(3)]).items():
                out[f"{name}_cells_{k}"] = v
    if (only is None and "--big" in sys.argv) or (only and "c4" in only):
        from matris_amd import workloads as W
        for k, v in run(m10, [_oracle_graph(cr) for cr in W.c4_batch64()], energy_only=True).items():
            out[f"c4_{k}"] = v
    np.savez_compressed(path, **out)
    print({k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
