"""Host-side structure of the model (no kernel launches): every layer of the MatRIS-10M
configuration takes the fused MI355X path, and the large-cell memory policy switches on
at the sizes it should."""
import math

import pytest
import torch

from matris_amd.config import DEFAULT_CONFIG, MATRIS_10M
from matris_amd.model import fused
from matris_amd.model.model import MatRIS


def test_every_line_layer_and_gated_mlp_is_fusable():
    model = MatRIS(**MATRIS_10M)
    assert len(model.interaction_block) == 10
    for blk in model.interaction_block:
        assert fused.line_attention_fusable(blk.attn_block_line_graph)
        assert fused.line_refinement_fusable(blk.refine_block_line_graph)
        assert not fused.line_refinement_fusable(blk.refine_block_atom_graph)  # atom graph: generic path
        for g in (blk.attn_block_atom_graph.edge_nonlinear_update, blk.attn_block_atom_graph.node_nonlinear_update,
                  blk.refine_block_atom_graph.edge_nonlinear_update):
            assert g._fusable()


def test_block_checkpoint_policy():
    gib = 2 ** 30
    hbm = 288 * gib
    # C3 (A = 264,384, E_d = 67,396): no checkpointing; C5 (A ~ 9.03 M, E_d ~ 1.89 M): on
    assert not fused.checkpoint_needed(264_384, 67_396, 10, total_bytes=hbm)
    assert fused.checkpoint_needed(9_027_734, 1_892_918, 10, total_bytes=hbm)
    assert not fused.checkpoint_needed(0, 100, 10, total_bytes=hbm)
    # C5: two blocks' saved activations (~80 GB each by the upper-bound estimate) fit the
    # 55% budget, so the last two blocks keep them and the first eight are checkpointed
    assert fused.blocks_to_checkpoint(9_027_734, 1_892_918, 10, total_bytes=hbm) == 8
    assert fused.blocks_to_checkpoint(264_384, 67_396, 10, total_bytes=hbm) == 0
    assert fused.blocks_to_checkpoint(10 ** 9, 0, 10, total_bytes=hbm) == 10


@pytest.mark.parametrize("over", [dict(norm_type="layer"), dict(norm_type="batch"), dict(graph_conv_mlp="MLP"),
                                  dict(graph_conv_mlp="MLP", norm_type="layer")])
def test_non_default_update_forms_take_the_generic_layer_path(over):
    """LayerNorm / BatchNorm GatedMLPs and the MLP-then-norm updates of graph_conv_mlp="MLP"
    are not the form the fused kernels implement: every layer runs its generic path."""
    from matris_amd.model.model import GatedMLP
    model = MatRIS(**dict(DEFAULT_CONFIG, num_layers=1, **over))
    blk = model.interaction_block[0]
    assert not fused.line_attention_fusable(blk.attn_block_line_graph)
    assert not fused.atom_attention_fusable(blk.attn_block_atom_graph)
    assert not fused.line_refinement_fusable(blk.refine_block_line_graph)
    assert not fused.atom_refinement_fusable(blk.refine_block_atom_graph)
    upd = blk.attn_block_atom_graph.edge_nonlinear_update
    if over.get("graph_conv_mlp") == "MLP":
        assert isinstance(upd, torch.nn.Sequential) and not isinstance(upd, GatedMLP)
        norm = {"layer": torch.nn.LayerNorm}.get(over.get("norm_type"), torch.nn.RMSNorm)
        assert isinstance(upd[1], norm) and upd[0].layers[0].bias is None  # MLP(bias=use_bias)
    else:
        assert isinstance(upd, GatedMLP) and upd.mlp_core.layers[0].bias is not None


def test_fp16_mlps_are_not_fused():
    from matris_amd.model.model import GatedMLP, Refinement
    assert GatedMLP(384, 128, 128, norm_type="rms")._fusable()
    assert not GatedMLP(384, 128, 128, norm_type="rms", use_fp16=True)._fusable()
    r = Refinement(128, 128, 128, 7, norm_type="rms", graph_type="atom graph", use_fp16=True)
    assert not fused.atom_refinement_fusable(r)
    assert fused.atom_refinement_fusable(Refinement(128, 128, 128, 7, norm_type="rms", graph_type="atom graph"))


def test_unknown_update_form_raises():
    with pytest.raises(NotImplementedError, match="mlp_type"):
        MatRIS(**dict(DEFAULT_CONFIG, num_layers=1, graph_conv_mlp="KAN"))


def test_direct_head_change_of_basis():
    """The direct stress head's irrep -> Cartesian matrix, built from its definition, equals
    the reference's table as the oracle restates it (functions.py:368-398), is orthonormal,
    and its l = 2 rows reproduce the l = 2 harmonics as r^T T r (sqrt(2/3) |r|^2 scale)."""
    import numpy as np
    from matris_amd.model.direct_head import IRREP_TO_CARTESIAN, sphere_harmonics_l2
    from oracle.model_ref import CG_CHANGE_MAT
    m = IRREP_TO_CARTESIAN.double()
    assert torch.allclose(IRREP_TO_CARTESIAN, torch.tensor(CG_CHANGE_MAT, dtype=torch.float32), atol=0, rtol=0)
    assert torch.allclose(m @ m.T, torch.eye(9, dtype=torch.float64), atol=1e-7)
    r = torch.tensor(np.random.default_rng(0).normal(size=(5, 3)))
    y2 = sphere_harmonics_l2(r)[:, 4:]
    quad = torch.einsum("ni,kij,nj->nk", r, m[4:].view(5, 3, 3), r)
    assert torch.allclose(quad * math.sqrt(3.0 / 2.0), y2, atol=1e-6)


def test_generic_bases_match_the_oracle_on_the_cpu():
    """The torch forms of the non-default bases (basis_generic) against the oracle's
    restatements of the reference, on the same inputs: SH bases of every size up to 4 x 4,
    the Gaussian and Fourier expansions and the Bessel basis without envelope."""
    from matris_amd.model import basis_generic as B
    from oracle import model_ref as R
    gen = torch.Generator().manual_seed(0)
    d = 0.9 + 0.2 * torch.rand(200, generator=gen)
    ang = 3.1 * torch.rand(200, generator=gen)
    r = 0.7 + 5.0 * torch.rand(200, generator=gen)
    for mn in range(1, 5):
        for ml in range(1, 5):
            o = R.SphericalExpansion(mn, ml, 6)
            ref = o(d, ang)
            assert torch.allclose(B.spherical_basis(d, ang, mn, ml, 6, o.factor), ref, rtol=1e-6,
                                  atol=1e-6 * float(ref.abs().max())), (mn, ml)
    assert torch.allclose(B.GaussianExpansion(0.0, 6.0, 7, 2.0)(r), R.GaussianExpansion(0.0, 6.0, 7, 2.0)(r),
                          rtol=1e-6, atol=1e-7)
    assert torch.allclose(B.FourierExpansion(3)(ang), R.FourierExpansion(3)(ang), rtol=1e-6, atol=1e-7)
    ob = R.BesselExpansion(7, 6.0, None)
    assert torch.allclose(B.bessel_plain(r, ob.frequencies, ob.inv_cutoff, ob.norm_const), ob(r), rtol=1e-6,
                          atol=1e-7)


@pytest.mark.parametrize("act", ["relu", "gelu", "tanh", "sigmoid", "softplus"])
def test_other_activations_take_the_generic_gated_mlp_path(act):
    """The fused GatedMLP kernels compute SiLU: a GatedMLP built with another
    activation_type runs its module forward, the readout likewise; the Refinement FFNs
    keep SiLU whatever activation_type is (interaction_block.py:198-210 passes none), so
    they stay fused."""
    model = MatRIS(**dict(DEFAULT_CONFIG, num_layers=1, activation_type=act))
    blk = model.interaction_block[0]
    assert not blk.attn_block_atom_graph.edge_nonlinear_update._fusable()
    assert not fused.line_attention_fusable(blk.attn_block_line_graph)
    assert not fused.line_refinement_fusable(blk.refine_block_line_graph)
    assert not model._readout_fusable()
    assert fused._ffn_fusable(blk.refine_block_line_graph.node_FFN)


def test_active_dropout_leaves_the_fused_kernels():
    """A GatedMLP or FFN with dropout > 0 in training mode runs its module forward (the
    fused kernels apply no dropout); in eval mode it is fused again.  MatRIS's dropout
    keyword reaches only the refinement layers' edge updates, as in the reference
    (interaction_block.py:321-365 passes it to the Refinement layers alone)."""
    from matris_amd.model.model import MLP, GatedMLP
    g = GatedMLP(384, 128, 128, dropout=0.1, norm_type="rms").train()
    f = MLP(128, 128, 128, dropout=0.1, bias=False).train()
    assert not g._fusable() and not fused._ffn_fusable(f)
    g.eval(); f.eval()
    assert g._fusable() and fused._ffn_fusable(f)
    model = MatRIS(**dict(DEFAULT_CONFIG, num_layers=1, dropout=0.1)).train()
    active = sorted({n.rsplit(".", 2)[0] for n, l in model.named_modules()
                     if isinstance(l, torch.nn.Dropout) and l.p > 0})
    assert active == [f"interaction_block.0.refine_block_{k}_graph.edge_nonlinear_update.{m}"
                      for k in ("atom", "line") for m in ("mlp_core", "mlp_gate")]
    blk = model.interaction_block[0]
    assert not fused.line_refinement_fusable(blk.refine_block_line_graph)
    assert fused.line_attention_fusable(blk.attn_block_line_graph)
    model.eval()
    assert fused.line_refinement_fusable(blk.refine_block_line_graph)
