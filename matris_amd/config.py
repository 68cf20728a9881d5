"""Model configuration pins shared by the product path, the oracle and the benchmarks.

`MatRIS.__init__` keyword defaults are those of the reference constructor
(matris/model/model.py:33-59).  The reference repository never defines the
"MatRIS-10M" architecture in code (its checkpoints carry the config and are
download-only, model.py:281-304).  The defaults give 6,286,736 parameters; the only
single-knob change that lands at ~10M with every tensor shape unchanged is
`num_layers=10` (10,379,664 parameters), which is the pin used here.
"""
from __future__ import annotations

DEFAULT_CONFIG = dict(
    num_layers=6,
    node_feat_dim=128,
    edge_feat_dim=128,
    three_body_feat_dim=128,
    mlp_hidden_dims=(128, 128),
    dropout=0.0,
    use_bias=False,
    distance_expansion="Bessel",
    three_body_expansion="SH",
    num_radial=7,
    num_angular=7,
    max_l=4,
    max_n=4,
    envelope_exponent=8,
    graph_conv_mlp="GateMLP",
    activation_type="silu",
    norm_type="rms",
    pairwise_cutoff=6,
    three_body_cutoff=4,
    use_smoothed_for_delta_edge=False,
    learnable_basis=True,
    is_intensive=True,
    is_conservation=True,
    reference_energy=None,
)

MATRIS_10M = dict(DEFAULT_CONFIG, num_layers=10)
MATRIS_10M_PARAMS = 10_379_664
MATRIS_6M_PARAMS = 6_286_736

# Unit conversion used by the conservative stress head (matris/model/readout.py:214):
# eV/A^3 -> GPa.
EV_A3_TO_GPA = 160.21766208


def matris_10m_config() -> dict:
    """Return a fresh copy of the pinned MatRIS-10M constructor kwargs."""
    return dict(MATRIS_10M)
