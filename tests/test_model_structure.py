"""Host-side structure of the model (no kernel launches): every layer of the MatRIS-10M
configuration takes the fused MI355X path, and the large-cell memory policy switches on
at the sizes it should."""
from matris_amd.config import MATRIS_10M
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
