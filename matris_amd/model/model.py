"""MatRIS on MI355X: the reference module tree (same class names, attribute names,
construction order and state_dict keys, so `torch.manual_seed(s)` gives the reference's
weights and a reference checkpoint loads unchanged) whose forward runs the gfx950
kernels of libmatris_hip.so:

  gated MLPs (every GatedMLP, with its input concatenation)  -> matris_gmlp_fwd / _bwd
  node_FFN / edge_FFN, W_s / W_t projection pairs              -> matris_ffn_* / matris_pair_*
  Dimwise_softmax x2 + alpha * e' + both aggregations         -> matris_attn_fwd / _bwd
  envelope-weighted line-graph aggregation                    -> matris_env_agg_fwd / _bwd
  aggregate(), index_select and their backward scatters      -> matris_seg_sum / _gather_rows
  graph construction                                          -> GraphConverter (G1-G5 kernels)

The two line-graph layers of each block (attention, refinement) run as single autograd
nodes with an explicit backward (fused.py) so their residual updates and gradient sums
stay inside the kernels; the edge and three-body embeddings, the learnable envelopes
and the readout heads have kernels of their own as well (matris_edge_embed_*,
matris_tb_embed_*, matris_env_*, matris_readout_*).  Forces and stress come from
torch.autograd.grad exactly as in the reference (readout.py:202-217); every custom op
supplies its own input-gradient kernel.

Constructor options outside the MatRIS-10M form (LayerNorm / BatchNorm GatedMLPs,
graph_conv_mlp="MLP", fp16 MLPs, Gaussian / Fourier / smaller SH bases, no envelope,
more than 8 radial functions, the direct force/stress head) build the same module tree
and run each layer's generic path: the library's gathers and segment kernels with the
option's own pieces as torch layers on the device (basis_generic.py, direct_head.py).

Reference: matris/model/model.py, interaction_block.py, feature_embed.py, functions.py,
readout.py, basis_function.py.
"""
from __future__ import annotations

import contextlib
import math
import weakref
from collections.abc import Sequence

import torch
import torch.nn.functional as F
import torch.utils.checkpoint
from torch import Tensor, nn

from ..config import EV_A3_TO_GPA
from ..graph.converter import GraphConverter
from . import basis_generic, direct_head, fused, ops
from .atomref import AtomRef
from .basis_generic import FourierExpansion, GaussianExpansion
from .batch import process_graphs


# ------------------------------------------------------------------------------------
# primitives (functions.py)
# ------------------------------------------------------------------------------------
class FusedSiLU(nn.Module):
    """functions.py:10-22 (the activation inside the fused kernels; F.silu elsewhere)."""

    def forward(self, x):
        return F.silu(x)


class FusedSigmoid(nn.Module):
    """functions.py:24-36."""

    def forward(self, x):
        return torch.sigmoid(x)


def get_activation(name: str) -> nn.Module:
    """functions.py:38-55."""
    table = {"relu": nn.ReLU, "silu": FusedSiLU, "gelu": nn.GELU, "softplus": nn.Softplus, "sigmoid": FusedSigmoid,
             "tanh": nn.Tanh}
    if name.lower() not in table:
        raise NotImplementedError(f"Activation '{name}' is not implemented. Supported activations: {list(table)}")
    return table[name.lower()]()


def get_normalization(name: str, dim: int | None = None) -> nn.Module | None:
    """functions.py:57-68 (LayerNorm / RMSNorm / BatchNorm1d construction consumes no RNG)."""
    if name is None:
        return None
    name = name.lower()
    if name == "layer":
        return nn.LayerNorm(dim)
    if name == "rms":
        return nn.RMSNorm(dim)
    if name == "batch":
        return nn.BatchNorm1d(dim)
    raise KeyError(name)


class SwishLayer(nn.Module):
    """functions.py:70-95."""

    def __init__(self, input_dim: int = 128, output_dim: int = 128, bias: bool = True):
        super().__init__()
        self.linear = nn.Linear(input_dim, output_dim, bias=bias)
        self.act = get_activation("silu")

    def forward(self, x):
        return self.act(self.linear(x))


class MLP(nn.Module):
    """functions.py:163-242."""

    def __init__(self, input_dim=128, hidden_dim=(128, 128), output_dim=128, dropout=0.0, activation="silu",
                 bias=True, use_fp16=False):
        super().__init__()
        if not 0.0 <= dropout < 1.0:
            raise ValueError(f"Dropout rate must be in [0.0, 1.0), got {dropout}")
        self.use_fp16 = use_fp16
        act = get_activation(activation)
        layers: list[nn.Module] = []
        if hidden_dim in (None, 0):
            layers += [nn.Dropout(dropout), nn.Linear(input_dim, output_dim, bias=bias)]
        elif isinstance(hidden_dim, int):
            layers += [nn.Linear(input_dim, hidden_dim, bias=bias), act, nn.Dropout(dropout),
                       nn.Linear(hidden_dim, output_dim, bias=bias)]
        elif isinstance(hidden_dim, Sequence):
            layers += [nn.Linear(input_dim, hidden_dim[0], bias=bias), act]
            for i in range(len(hidden_dim) - 1):
                layers += [nn.Dropout(dropout), nn.Linear(hidden_dim[i], hidden_dim[i + 1], bias=bias), act]
            layers += [nn.Dropout(dropout), nn.Linear(hidden_dim[-1], output_dim, bias=bias)]
        else:
            raise TypeError(f"hidden_dim must be an integer, sequence of integers, or None, got "
                            f"{type(hidden_dim).__name__}")
        self.layers = nn.Sequential(*layers)

    def forward(self, x):
        if self.use_fp16 and x.is_cuda:  # functions.py:231-236: fp16 autocast, fp32 result
            with torch.autocast(device_type="cuda", dtype=torch.float16):
                out = self.layers(x)
            return out.to(torch.float32)
        return self.layers(x)


def dropout_off(mlp) -> bool:
    """Every Dropout of the MLP is the identity (p = 0, or eval mode): the fused kernels
    apply none."""
    return all(l.p == 0.0 or not l.training for l in mlp.layers if isinstance(l, nn.Dropout))


class GatedMLP(nn.Module):
    """functions.py:245-311.  `fused(sources)` runs the whole block -- gathers, concat,
    two MLPs, RMSNorm, SiLU, sigmoid, product -- in matris_gmlp_fwd."""

    def __init__(self, input_dim=128, hidden_dim=(128, 128), output_dim=128, dropout=0.0, activation="silu",
                 norm_type="layer", bias=True, use_fp16=False):
        super().__init__()
        self.use_fp16 = use_fp16
        self.activation_func = get_activation(activation)
        self.activation_gate = get_activation("sigmoid")
        self.gate_norm = get_normalization(name=norm_type, dim=output_dim)
        self.core_norm = get_normalization(name=norm_type, dim=output_dim)
        self.mlp_core = MLP(input_dim, hidden_dim, output_dim, dropout, activation, bias, use_fp16)
        self.mlp_gate = MLP(input_dim, hidden_dim, output_dim, dropout, activation, bias, use_fp16)
        self._pack = ops.GmlpPack()

    def _fusable(self) -> bool:
        """The form matris_gmlp_fwd / _bwd compute: RMSNorm, one 128-wide hidden layer with
        biases, SiLU as the hidden and the core activation (activation_type="silu"), fp32."""
        return (isinstance(self.core_norm, nn.RMSNorm) and len(self.mlp_core.layers) == 4
                and self.mlp_core.layers[0].bias is not None and self.mlp_core.layers[0].out_features == 128
                and self.mlp_core.layers[3].out_features == 128 and not self.use_fp16
                and not self.mlp_core.use_fp16 and not self.mlp_gate.use_fp16
                and isinstance(self.activation_func, FusedSiLU) and isinstance(self.mlp_core.layers[1], FusedSiLU)
                and isinstance(self.mlp_gate.layers[1], FusedSiLU) and dropout_off(self.mlp_core)
                and dropout_off(self.mlp_gate))

    def forward(self, x):
        core = self.activation_func(self.core_norm(self.mlp_core(x)))
        gate = self.activation_gate(self.gate_norm(self.mlp_gate(x)))
        return core * gate

    def fused(self, sources):
        """The block on the concatenation of `sources` ((rows, grouping or None) pairs, the
        grouping's keys selecting rows): matris_gmlp_fwd for the MatRIS-10M form (RMSNorm,
        one 128-wide hidden layer, biases); any other form (LayerNorm or BatchNorm, other
        widths, the fp16 autocast MLPs) runs this module's own forward on the gathered
        concatenation, on the device."""
        if (self._fusable() and all(t.dim() == 2 and t.shape[1] == 128 for t, _ in sources)
                and self.mlp_core.layers[0].in_features == 128 * len(sources)):
            return ops.gated_mlp(self, self._pack, sources)
        return self(gathered_concat(sources))


def gathered_concat(sources):
    """torch.cat of the sources' rows ((tensor, grouping or None) pairs; a grouping's keys
    select the rows, ops.gather) along the feature axis: the reference's index_select +
    cat (interaction_block.py:96-106, 230-237)."""
    return torch.cat([t if g is None else ops.gather(t, g) for t, g in sources], dim=1)


def nonlinear_update(module, sources):
    """A layer's edge or node update on its concatenated sources: GatedMLP.fused, or, for
    graph_conv_mlp="MLP" (an MLP followed by a norm, interaction_block.py:39-62, 172-184),
    the module on the gathered concatenation."""
    if isinstance(module, GatedMLP):
        return module.fused(sources)
    return module(gathered_concat(sources))


def _mlp_update(in_dim, hidden_dim, out_dim, dropout, use_bias, activation, norm_type, use_fp16=False):
    """interaction_block.py:39-62 / 172-184 (mlp_type "MLP"): MLP then a norm."""
    return nn.Sequential(MLP(in_dim, hidden_dim, out_dim, dropout, activation, use_bias, use_fp16),
                         get_normalization(name=norm_type, dim=out_dim))


class GraphPooling(nn.Module):
    """functions.py:340-365 (graph sums of a [N, 1] quantity)."""

    def __init__(self, average: bool = False):
        super().__init__()
        self.average = average

    def forward(self, node_feat, segment, n_graphs: int, rowptr=None):
        """Per-graph sums in a fixed order (no float atomics, so the energies are bitwise
        reproducible): one reduction for one graph, otherwise a segmented reduction over
        the atoms, which are contiguous per graph (ops.SegSumNarrow with the graphs' int32
        row pointers; made from segment when not given)."""
        if n_graphs == 1:
            out = node_feat.sum(0, keepdim=True)
        else:
            if rowptr is None:
                cnt = torch.bincount(segment, minlength=n_graphs)
                rowptr = torch.cat([cnt.new_zeros(1), torch.cumsum(cnt, 0)]).to(torch.int32)
            out = ops.SegSumNarrow.apply(node_feat, rowptr, segment, n_graphs)
        if self.average:
            out = out / torch.bincount(segment, minlength=n_graphs).clamp_min(1)[:, None]
        return out


# ------------------------------------------------------------------------------------
# basis functions (basis_function.py)
# ------------------------------------------------------------------------------------
class PolynomialEnvelope(nn.Module):
    """basis_function.py:8-50."""

    def __init__(self, cutoff: float = 6, envelope_exponent: float = 8):
        super().__init__()
        assert envelope_exponent > 0
        self.cutoff = cutoff
        self.p = float(envelope_exponent)
        self.a = -(self.p + 1) * (self.p + 2) / 2
        self.b = self.p * (self.p + 2)
        self.c = -self.p * (self.p + 1) / 2

    def forward(self, dist):
        x = dist / self.cutoff
        env = 1 + self.a * x ** self.p + self.b * x ** (self.p + 1) + self.c * x ** (self.p + 2)
        return torch.where(x < 1, env, torch.zeros_like(x))


class BesselExpansion(nn.Module):
    """basis_function.py:116-186."""

    def __init__(self, num_radial=9, cutoff=6, envelope_exponent=8, learnable=False):
        super().__init__()
        self.num_radial = num_radial
        self.inv_cutoff = 1 / cutoff
        self.norm_const = (2 * self.inv_cutoff) ** 0.5
        freq = math.pi * torch.arange(1, num_radial + 1, dtype=torch.float)
        if learnable:
            self.frequencies = nn.Parameter(freq, requires_grad=True)
        else:
            self.register_buffer("frequencies", freq)
        self.envelope_func = PolynomialEnvelope(cutoff, envelope_exponent) if envelope_exponent is not None else None

    def forward(self, dist, return_smooth_factor=False):
        """B_n(r) env(r) on the device (matris_bessel_fwd / _bwd); without an envelope
        (envelope_exponent=None) the plain basis as torch on the device.  With
        return_smooth_factor, (basis, env(r) [n, 1]) when there is an envelope."""
        if not dist.is_cuda:
            raise RuntimeError("matris_amd ops run on the ROCm device only (no CPU fallback)")
        if self.envelope_func is None:
            return basis_generic.bessel_plain(dist, self.frequencies, self.inv_cutoff, self.norm_const)
        out = ops.bessel(dist, self.frequencies, self.envelope_func.cutoff, self.envelope_func.p)
        if return_smooth_factor:
            return out, self.envelope_func(dist[:, None])
        return out


class SphericalExpansion(nn.Module):
    """basis_function.py:222-338: the spherical-Bessel radial table times Legendre Y_l.
    The 4 x 4 basis is computed on the device by matris_sbf_fwd / _bwd (which hold the
    root table); smaller ones (max_n, max_l <= 4) by basis_generic.spherical_basis."""

    def __init__(self, max_n=4, max_l=4, cutoff=6):
        super().__init__()
        if not (1 <= max_n <= 4 and 1 <= max_l <= 4):
            raise ValueError("SphericalExpansion: max_n and max_l must be 1..4")
        self.max_n, self.max_l, self.cutoff = max_n, max_l, cutoff
        self.register_buffer("factor", torch.sqrt(torch.tensor(2.0 / (cutoff ** 3))))

    def forward(self, dist, three_body):
        return basis_generic.spherical_basis(dist, three_body, self.max_n, self.max_l, self.cutoff, self.factor)


# ------------------------------------------------------------------------------------
# embeddings (feature_embed.py)
# ------------------------------------------------------------------------------------
class AtomTypeEmbedding(nn.Module):
    """feature_embed.py:16-39."""

    def __init__(self, atom_feat_dim: int, max_num_elements: int = 94):
        super().__init__()
        self.embedding = nn.Embedding(max_num_elements, atom_feat_dim)
        self.atom_swish_layer = SwishLayer(atom_feat_dim, atom_feat_dim, bias=False)
        self._memo = None  # (weakref to the atomic numbers, key, features)

    def forward(self, atom_type):
        return self.atom_swish_layer(self.embedding(atom_type))

    def embed(self, atomic_numbers: Tensor) -> Tensor:
        """forward(atomic_numbers - 1) without a gradient (the efsm path differentiates in
        positions and strain only), remembered while the same atomic-number tensor (held
        by a weak reference, so a freed tensor never matches) and the weights keep their
        storage and version counters: repeated evaluations of one structure (MD,
        relaxation) issue no operations for it."""
        prm = [p for p in self.parameters()]
        key = (atomic_numbers.data_ptr(), atomic_numbers._version, tuple(atomic_numbers.shape),
               tuple((p.data_ptr(), p._version) for p in prm))
        m = self._memo
        if m is not None and m[0]() is atomic_numbers and m[1] == key:
            return m[2]
        with torch.no_grad():
            out = self.forward(atomic_numbers.long() - 1)
        self._memo = (weakref.ref(atomic_numbers), key, out)
        return out


class EdgeBasisEmbedding(nn.Module):
    """feature_embed.py:42-148.  The reference expands W1 rbf to both directed copies,
    applies W2 and LayerNorm, then averages the two identical copies; evaluating once
    per undirected bond gives the same values and the same gradient (g/2 + g/2)."""

    def __init__(self, pairwise_cutoff=6, three_body_cutoff=4, num_radial=7, edge_feat_dim=128,
                 envelope_exponent=8, distance_expansion="Bessel", learnable=False):
        super().__init__()
        self.distance_expansion = distance_expansion
        if distance_expansion.lower() == "bessel":
            self.pairwise_rbf_expansion = BesselExpansion(num_radial, pairwise_cutoff, envelope_exponent, learnable)
            self.threebody_rbf_expansion = BesselExpansion(num_radial, three_body_cutoff, envelope_exponent, learnable)
        elif distance_expansion.lower() == "gaussian":  # torch on the device (basis_generic)
            self.pairwise_rbf_expansion = GaussianExpansion(0.0, pairwise_cutoff, num_radial, 2.0)
            self.threebody_rbf_expansion = GaussianExpansion(0.0, three_body_cutoff, num_radial, 2.0)
        else:
            raise NotImplementedError(f"Unknown distance_expansion: {distance_expansion}")
        self.edge_linear1 = nn.Linear(num_radial, edge_feat_dim, bias=False)
        self.edge_linear2 = nn.Linear(edge_feat_dim, edge_feat_dim, bias=False)
        self.swish_layer = SwishLayer(edge_feat_dim, edge_feat_dim, bias=False)
        self.edge_init_norm = get_normalization(name="layer", dim=edge_feat_dim)
        self._pack = ops._WeightPack()

    def _fusable(self) -> bool:
        """The configuration matris_edge_embed_fwd implements (MatRIS-10M's)."""
        b6, b4, ln = self.pairwise_rbf_expansion, self.threebody_rbf_expansion, self.edge_init_norm
        return (isinstance(b6, BesselExpansion) and isinstance(b4, BesselExpansion) and b6.envelope_func is not None and b4.envelope_func is not None and b6.num_radial == 7
                and b4.num_radial == 7 and b6.envelope_func.p == b4.envelope_func.p
                and self.edge_linear1.bias is None and tuple(self.edge_linear1.weight.shape) == (128, 7)
                and self.edge_linear2.bias is None and tuple(self.edge_linear2.weight.shape) == (128, 128)
                and self.swish_layer.linear.bias is None and tuple(self.swish_layer.linear.weight.shape) == (128, 128)
                and isinstance(ln, nn.LayerNorm) and ln.elementwise_affine and ln.bias is not None
                and tuple(ln.normalized_shape) == (128,))

    def forward(self, graphs):
        if "u2d32" in graphs and self._fusable():
            # one launch per direction: the basis of both cutoffs, the two linears, the
            # LayerNorm and the swish layer (matris_edge_embed_fwd / _bwd)
            e, rbf6, rbf4 = ops.edge_embed(graphs["edge_lengths"], graphs["u2d32"], self)
            return e, {"atom graph": rbf6, "line graph": rbf4}
        lengths = torch.index_select(graphs["edge_lengths"], 0, graphs["undirected2directed"])
        rbf6 = self.pairwise_rbf_expansion(lengths)
        rbf4 = self.threebody_rbf_expansion(lengths)
        e = self.edge_init_norm(self.edge_linear2(self.edge_linear1(rbf6)))
        e = self.swish_layer(e)
        return e, {"atom graph": rbf6, "line graph": rbf4}


class ThreebodyEmbedding(nn.Module):
    """feature_embed.py:151-203.  The 4 x 4 SH expansion runs on the device kernels
    (matris_sbf_*, matris_tb_embed_*); a smaller SH basis and the Fourier expansion
    (three_body_expansion="fourier", num_angular features) as torch on the device."""

    def __init__(self, num_angular=7, max_n=4, max_l=4, cutoff=6, three_body_feat_dim=128,
                 three_body_expansion="fourier", learnable=True):
        super().__init__()
        self.three_body_expansion = three_body_expansion.lower()
        if self.three_body_expansion == "fourier":
            self.expansion = FourierExpansion(max_f=(num_angular - 1) // 2, learnable=learnable)
            self.angle_embedding = nn.Linear(num_angular, three_body_feat_dim, bias=False)
        elif self.three_body_expansion == "sh":
            self.expansion = SphericalExpansion(max_n=max_n, max_l=max_l, cutoff=cutoff)
            self.angle_embedding = nn.Linear(max_n * max_l, three_body_feat_dim, bias=False)
        else:
            raise NotImplementedError(f"Unknown three_body_expansion: {three_body_expansion}")
        self.swish_layer = SwishLayer(three_body_feat_dim, three_body_feat_dim, bias=False)
        self._pack = ops._WeightPack()

    def _generic(self, graphs):
        """The basis from the angle between each angle's two unit edge vectors (the
        reference's acos of their dot product times 1 - 1e-6), torch on the device."""
        lg = graphs["line_graph_dict"]
        u = graphs["unit_edge_vectors"]
        v_ij = torch.index_select(u, 0, lg["target_DE_index"])
        v_jk = torch.index_select(u, 0, lg["source_DE_index"])
        angle = torch.acos(torch.sum(v_ij * v_jk, dim=1) * (1 - 1e-6))
        if self.three_body_expansion == "sh":
            return self.expansion(torch.norm(v_jk, dim=1), angle)
        return self.expansion(angle)

    def forward(self, graphs):
        lg = graphs["line_graph_dict"]
        if not graphs["unit_edge_vectors"].is_cuda:
            raise RuntimeError("matris_amd ops run on the ROCm device only (no CPU fallback)")
        if self.three_body_expansion != "sh" or self.expansion.max_n != 4 or self.expansion.max_l != 4:
            return self.swish_layer(self.angle_embedding(self._generic(graphs)))
        basis = ops.spherical_basis(graphs["unit_edge_vectors"], lg["grp_de_t"], lg["grp_de_s"], self.expansion.cutoff)
        lin = self.swish_layer.linear
        if (ops.tb_embed_supported() and self.angle_embedding.bias is None and lin.bias is None
                and tuple(self.angle_embedding.weight.shape) == (128, 16) and tuple(lin.weight.shape) == (128, 128)):
            return ops.tb_embed(basis, self.angle_embedding.weight, lin.weight, self._pack)
        return self.swish_layer(self.angle_embedding(basis))  # bf16x6 mode: library GEMMs on the device


# ------------------------------------------------------------------------------------
# interaction block (interaction_block.py)
# ------------------------------------------------------------------------------------
class Graph_Attention_Layer(nn.Module):
    """interaction_block.py:17-143.  The fused kernels take the MatRIS-10M form (RMSNorm
    GatedMLPs, 128-wide); LayerNorm / BatchNorm GatedMLPs and graph_conv_mlp "MLP" run the
    generic path below (device gathers, segment attention and sums; the update module
    itself as torch layers on the device)."""

    def __init__(self, node_feat_dim=128, edge_feat_dim=128, hidden_dim=128, use_bias=False, dropout=0.0,
                 mlp_type="GateMLP", activation_type="silu", norm_type="layer", use_fp16=False):
        super().__init__()
        self.source_weight_linear = nn.Linear(edge_feat_dim, edge_feat_dim, bias=False)
        self.target_weight_linear = nn.Linear(edge_feat_dim, edge_feat_dim, bias=False)
        if mlp_type.lower() == "mlp":
            self.node_nonlinear_update = _mlp_update(edge_feat_dim * 2 + node_feat_dim, hidden_dim, node_feat_dim,
                                                     dropout, use_bias, activation_type, norm_type)
            self.edge_nonlinear_update = _mlp_update(node_feat_dim * 2 + edge_feat_dim, hidden_dim, edge_feat_dim,
                                                     dropout, use_bias, activation_type, norm_type, use_fp16)
        elif mlp_type.lower() == "gatemlp":
            self.node_nonlinear_update = GatedMLP(edge_feat_dim * 2 + node_feat_dim, hidden_dim, node_feat_dim,
                                                  norm_type=norm_type, dropout=dropout, activation=activation_type)
            self.edge_nonlinear_update = GatedMLP(node_feat_dim * 2 + edge_feat_dim, hidden_dim, edge_feat_dim,
                                                  norm_type=norm_type, dropout=dropout, activation=activation_type,
                                                  use_fp16=use_fp16)
        else:
            raise NotImplementedError(f"Unknown mlp_type: {mlp_type}")
        self.node_res_weight = nn.Parameter(torch.ones(1, node_feat_dim), requires_grad=True)
        self.edge_res_weight = nn.Parameter(torch.ones(1, edge_feat_dim), requires_grad=True)
        self._proj = ops._WeightPack()

    def _projections(self, edge_feat):
        """(source, target) attention logits (:110-111) in one MFMA pass."""
        lin_s, lin_t = self.source_weight_linear, self.target_weight_linear
        if lin_s.weight.shape == (128, 128) and lin_s.bias is None and lin_t.bias is None:
            return ops.proj_pair(self._proj.get(lin_s.weight, lin_t.weight), edge_feat)
        return lin_s(edge_feat), lin_t(edge_feat)

    def forward(self, node_feat, edge_feat, graph, d2u: ops.Grouping | None = None, recompute: bool = False):
        tgt, src = graph["grp_tgt"], graph["grp_src"]
        if d2u is None and fused.line_attention_fusable(self):  # one node, explicit backward
            return fused.line_attention(self, node_feat, edge_feat, graph, recompute)
        if d2u is not None and fused.atom_attention_fusable(self):
            return fused.atom_attention(self, node_feat, edge_feat, graph, d2u)
        if d2u is None:  # line graph: edges are the angles themselves
            e = nonlinear_update(self.edge_nonlinear_update, [(edge_feat, None), (node_feat, tgt), (node_feat, src)])
            a_s, a_t = self._projections(edge_feat)
            y_t, y_s = ops.seg_attention(a_t, a_s, e, tgt, src)
        else:  # atom graph: undirected bond rows expanded through d2u inside the kernels
            e = nonlinear_update(self.edge_nonlinear_update, [(edge_feat, d2u), (node_feat, tgt), (node_feat, src)])
            a_s, a_t = self._projections(edge_feat)
            y_t, y_s = ops.seg_attention(a_t, a_s, e, tgt, src, alpha_grp=d2u)
            e = ops.seg_sum(e, d2u, 0.5)  # mean of the two directed copies (:121-122)
        n = nonlinear_update(self.node_nonlinear_update, [(node_feat, None), (y_t, None), (y_s, None)])
        return n + self.node_res_weight * node_feat, e + self.edge_res_weight * edge_feat


class Refinement(nn.Module):
    """interaction_block.py:146-278; update forms as in Graph_Attention_Layer."""

    def __init__(self, node_feat_dim=128, edge_feat_dim=128, hidden_dim=128, num_basis=7, dropout=0.0,
                 mlp_type="GateMLP", activation_type="silu", norm_type="layer", use_bias=False,
                 graph_type="atom graph", atom_feat_dim=128, use_smoothed_for_delta_edge=False, use_fp16=False):
        super().__init__()
        self.graph_type = graph_type
        self.use_smoothed_for_delta_edge = use_smoothed_for_delta_edge
        input_dim = 2 * node_feat_dim + edge_feat_dim if graph_type == "atom graph" else \
            atom_feat_dim + 2 * node_feat_dim + edge_feat_dim
        if mlp_type.lower() == "mlp":
            self.edge_nonlinear_update = _mlp_update(input_dim, hidden_dim, edge_feat_dim, dropout, use_bias,
                                                     activation_type, norm_type, use_fp16)
        elif mlp_type.lower() == "gatemlp":
            self.edge_nonlinear_update = GatedMLP(input_dim, hidden_dim, edge_feat_dim, dropout=dropout,
                                                  norm_type=norm_type, activation=activation_type, use_fp16=use_fp16)
        else:
            raise NotImplementedError(f"Unknown mlp_type: {mlp_type}")
        self.node_FFN = MLP(edge_feat_dim, node_feat_dim, node_feat_dim, bias=use_bias)
        self.edge_FFN = MLP(edge_feat_dim, edge_feat_dim, edge_feat_dim, bias=use_bias, use_fp16=use_fp16)
        self.learnable_envelope = nn.Linear(num_basis, edge_feat_dim, bias=False)
        self.node_res_weight = nn.Parameter(torch.ones(1, node_feat_dim), requires_grad=True)
        self.edge_res_weight = nn.Parameter(torch.ones(1, edge_feat_dim), requires_grad=True)
        self._node_ffn = ops._WeightPack()
        self._edge_ffn = ops._WeightPack()
        self._env = ops._WeightPack()  # learnable_envelope.weight^T for the fused kernels

    @staticmethod
    def _ffn(mlp, pack, x):
        """MLP(hidden=int, bias=False) as one fused MFMA kernel (functions.py:198-205)."""
        L = mlp.layers
        if (len(L) == 4 and L[0].bias is None and L[3].bias is None and L[0].weight.shape == (128, 128)
                and L[3].weight.shape == (128, 128) and isinstance(L[1], FusedSiLU) and not mlp.use_fp16
                and dropout_off(mlp)):
            return ops.ffn(pack.get(L[0].weight, L[3].weight), x)
        return mlp(x)

    def forward(self, node_feat, edge_feat, smooth_weight, graph, d2u: ops.Grouping | None = None, atom_feat=None,
                recompute: bool = False):
        tgt, src = graph["grp_tgt"], graph["grp_src"]
        if self.graph_type == "atom graph" and fused.atom_refinement_fusable(self):  # one node, explicit backward
            return fused.atom_refinement(self, node_feat, edge_feat, smooth_weight, graph, d2u)
        if self.graph_type == "atom graph":
            w = ops.gather(self.learnable_envelope(smooth_weight), d2u)
            h = nonlinear_update(self.edge_nonlinear_update, [(edge_feat, d2u), (node_feat, tgt), (node_feat, src)])
        elif fused.line_refinement_fusable(self):  # one node, explicit backward
            return fused.line_refinement(self, edge_feat, atom_feat, node_feat, smooth_weight, graph, recompute)
        else:
            env = self.learnable_envelope(smooth_weight)
            w = ops.gather(env, src) * ops.gather(env, tgt)
            h = nonlinear_update(self.edge_nonlinear_update, [(edge_feat, None), (atom_feat, graph["grp_atom"]),
                                                              (node_feat, tgt), (node_feat, src)])
        hw = h * w
        agg = ops.seg_sum(hw, tgt)
        to_edge = hw if (self.graph_type == "atom graph" and self.use_smoothed_for_delta_edge) else h
        dn = self._ffn(self.node_FFN, self._node_ffn, agg)
        de = self._ffn(self.edge_FFN, self._edge_ffn, to_edge)
        if self.graph_type == "atom graph":
            de = ops.seg_sum(de, d2u, 0.5)
        return dn + self.node_res_weight * node_feat, de + self.edge_res_weight * edge_feat


def _ckpt_contexts():
    """torch.utils.checkpoint context_fn: the original pass of a checkpointed block writes no
    saved-for-backward activations (ops.discard_saves); the recomputation writes them."""
    return ops.discard_saves(), contextlib.nullcontext()


class Interaction_Block(nn.Module):
    """interaction_block.py:281-446.  The reference checkpoints the two line-graph layers
    when A > 60000 (:400-413); here the fused line layers recompute their forward inside
    their own backward when batch_graph["line_recompute"] is set (MatRIS.forward sets it
    from the activation footprint, or from MatRIS.line_recompute), and the [A, 384/512]
    concatenations are never materialised either way."""

    def __init__(self, node_feat_dim=128, edge_feat_dim=128, three_body_feat_dim=128, num_radial=7, num_angular=7,
                 dropout=0.0, use_bias=False, use_smoothed_for_delta_edge=False, mlp_type="GateMLP",
                 norm_type="layer", activation_type="silu"):
        super().__init__()
        self.attn_block_atom_graph = Graph_Attention_Layer(node_feat_dim, edge_feat_dim, node_feat_dim, use_bias,
                                                           mlp_type=mlp_type, norm_type=norm_type,
                                                           activation_type=activation_type)
        self.attn_block_line_graph = Graph_Attention_Layer(edge_feat_dim, three_body_feat_dim, edge_feat_dim,
                                                           use_bias, mlp_type=mlp_type, norm_type=norm_type,
                                                           activation_type=activation_type)
        self.refine_block_atom_graph = Refinement(node_feat_dim, edge_feat_dim, node_feat_dim, num_radial, dropout,
                                                  mlp_type, activation_type, norm_type, use_bias, "atom graph",
                                                  use_smoothed_for_delta_edge=use_smoothed_for_delta_edge)
        self.refine_block_line_graph = Refinement(edge_feat_dim, three_body_feat_dim, edge_feat_dim, num_angular,
                                                  dropout, mlp_type, activation_type, norm_type, use_bias,
                                                  "line graph", atom_feat_dim=node_feat_dim)

    def forward(self, batch_graph, node_feat, edge_feat, threebody_feat, smooth_weight):
        attn_edge, attn_tb = edge_feat, threebody_feat
        upd_edge, upd_tb = edge_feat, threebody_feat
        lg, ag, d2u = batch_graph["line_graph_dict"], batch_graph["atom_graph_dict"], batch_graph["grp_d2u"]
        rc = batch_graph.get("line_recompute", False)
        if threebody_feat is not None:
            attn_edge, attn_tb = self.attn_block_line_graph(edge_feat, threebody_feat, lg, recompute=rc)
        attn_node, attn_edge = self.attn_block_atom_graph(node_feat, attn_edge, ag, d2u)
        # read by both Refinements: their fused backwards build its gradient in one buffer
        attn_node = fused.shared_grad(attn_node)
        if threebody_feat is not None:
            upd_edge, upd_tb = self.refine_block_line_graph(attn_edge, attn_tb, smooth_weight["line graph"], lg,
                                                            atom_feat=attn_node, recompute=rc)
        upd_node, upd_edge = self.refine_block_atom_graph(attn_node, upd_edge, smooth_weight["atom graph"], ag,
                                                          d2u=d2u)
        return upd_node, upd_edge, upd_tb


# ------------------------------------------------------------------------------------
# readout (readout.py)
# ------------------------------------------------------------------------------------
class EnergyHead(nn.Module):
    """readout.py:18-75 (mlp_type='mlp')."""

    def __init__(self, feat_dim=128, hidden_dim=128, output_dim=1, mlp_type="mlp", activation_type="silu"):
        super().__init__()
        hd = [hidden_dim] if isinstance(hidden_dim, int) else list(hidden_dim)
        if mlp_type.lower() != "mlp":
            raise NotImplementedError(f"Unknown mlp_type: {mlp_type}")
        self.energy_head = MLP(feat_dim, hd, output_dim, activation=activation_type)
        self.pooling = GraphPooling(average=False)

    def forward(self, batch_graph, node_feat):
        e = self.energy_head(node_feat)
        return self.pooling(e, batch_graph["atom_segment"], len(batch_graph["atoms_per_graph"]),
                            batch_graph.get("atom_rowptr")).view(-1)


class MagmomHead(nn.Module):
    """readout.py:77-133 (mlp_type='mlp')."""

    def __init__(self, feat_dim=128, hidden_dim=128, output_dim=1, mlp_type="mlp", activation_type="silu"):
        super().__init__()
        hd = [hidden_dim] if isinstance(hidden_dim, int) else list(hidden_dim)
        if mlp_type.lower() != "mlp":
            raise NotImplementedError(f"Unknown mlp_type: {mlp_type}")
        self.magmom_head = MLP(feat_dim, hd, output_dim, activation=activation_type)

    def forward(self, batch_graph, node_feat):
        m = torch.abs(self.magmom_head(node_feat))
        return list(torch.split(m.view(-1), batch_graph["atoms_per_graph"]))


class ForceStressHead(nn.Module):
    """readout.py:136-252.  Conservative (the default): forces and stress by autograd.
    Direct (is_conservation=False): an equivariant stress head and an MLP force head
    (direct_head.py), evaluated in the forward."""

    def __init__(self, is_conservation=True, feat_dim=128, hidden_dim=128, output_dim=3, mlp_type="mlp",
                 activation_type="silu"):
        super().__init__()
        self.is_conservation = is_conservation
        if not is_conservation:
            hd = [hidden_dim] if isinstance(hidden_dim, int) else list(hidden_dim)
            self.stress_head = direct_head.EquivariantHead(feat_dim, lmax=2, use_bias=False,
                                                           make_activation=lambda: get_activation(activation_type))
            if mlp_type.lower() == "mlp":
                self.force_head = MLP(feat_dim, hd, output_dim, activation=activation_type)
            elif mlp_type.lower() == "gatemlp":  # readout.py:175-184
                self.force_head = nn.Sequential(GatedMLP(feat_dim, hd, hd[-1], norm_type="layer",
                                                         activation=activation_type),
                                                nn.Linear(hd[-1], output_dim))
            else:
                raise NotImplementedError(f"Unknown mlp_type: {mlp_type}")

    def forward(self, batch_graph, compute_force=True, compute_stress=True, total_energy=None, is_training=False,
                node_feat=None, edge_feat=None):
        pred = {}
        if not self.is_conservation:
            if compute_stress:
                pred["s"] = list(torch.unbind(direct_head.direct_stress(self.stress_head, node_feat, batch_graph), 0))
            if compute_force:
                f = direct_head.direct_forces(self.force_head, edge_feat, batch_graph)
                pred["f"] = torch.split(f, batch_graph["atoms_per_graph"])
            return pred
        if compute_force and compute_stress:
            gc, gs = torch.autograd.grad(total_energy.sum(),
                                         [batch_graph["batch_cart_coords"], batch_graph["batch_strains"]],
                                         create_graph=is_training, retain_graph=is_training)
            pred["f"] = torch.split(-1 * gc, batch_graph["atoms_per_graph"])
            pred["s"] = list(torch.unbind(gs * (1 / batch_graph["volumes"] * EV_A3_TO_GPA), dim=0))
        elif compute_force:
            (gc,) = torch.autograd.grad(total_energy.sum(), [batch_graph["batch_cart_coords"]],
                                        create_graph=is_training, retain_graph=is_training)
            pred["f"] = torch.split(-1 * gc, batch_graph["atoms_per_graph"])
        return pred


# ------------------------------------------------------------------------------------
# MatRIS (model.py)
# ------------------------------------------------------------------------------------
class MatRIS(nn.Module):
    """model.py:30-317 with the same constructor keywords and forward signature."""

    def __init__(self, num_layers: int = 6, node_feat_dim: int = 128, edge_feat_dim: int = 128,
                 three_body_feat_dim: int = 128, mlp_hidden_dims=(128, 128), dropout: float = 0.0,
                 use_bias: bool = False, distance_expansion: str = "Bessel", three_body_expansion: str = "SH",
                 num_radial: int = 7, num_angular: int = 7, max_l: int = 4, max_n: int = 4,
                 envelope_exponent: int = 8, graph_conv_mlp: str = "GateMLP", activation_type: str = "silu",
                 norm_type: str = "rms", pairwise_cutoff: float = 6, three_body_cutoff: float = 4,
                 use_smoothed_for_delta_edge: bool = False, learnable_basis: bool = True, is_intensive: bool = True,
                 is_conservation: bool = True, reference_energy: str | None = None, verbose: bool = False):
        super().__init__()
        self.config = {k: v for k, v in locals().items() if k not in ("self", "__class__", "verbose")}
        self.is_intensive = is_intensive
        # Memory modes for large cells.  block_checkpoint: None = decided per call from the
        # activation footprint (fused.blocks_to_checkpoint: the leading blocks that do not
        # fit), True / False = all / none, an int k = the first k blocks; a checkpointed block
        # keeps only its inputs and reruns its forward in the backward.
        # line_recompute: the two line-graph layers alone keep only their inputs.
        self.block_checkpoint: bool | int | None = None
        self.line_recompute: bool = False
        # created before the other modules, as in the reference (model.py:104-109): its Linear
        # consumes random numbers, so the seed-0 weights of the rest match with it too
        self.reference_energy = (AtomRef(reference_energy=reference_energy, is_intensive=is_intensive)
                                 if reference_energy is not None else None)
        self.graph_converter = GraphConverter(atom_graph_cutoff=pairwise_cutoff, line_graph_cutoff=three_body_cutoff)
        self.atom_embedding = AtomTypeEmbedding(atom_feat_dim=node_feat_dim)
        self.edge_embedding = EdgeBasisEmbedding(pairwise_cutoff, three_body_cutoff, num_radial, edge_feat_dim,
                                                 envelope_exponent, distance_expansion, learnable_basis)
        self.three_body_embedding = ThreebodyEmbedding(num_angular, max_n, max_l, pairwise_cutoff,
                                                       three_body_feat_dim, three_body_expansion, learnable_basis)
        self.interaction_block = nn.ModuleList([
            Interaction_Block(node_feat_dim, edge_feat_dim, three_body_feat_dim, num_radial, num_angular, dropout,
                              use_bias, use_smoothed_for_delta_edge, graph_conv_mlp, norm_type, activation_type)
            for _ in range(num_layers)])
        self.readout_norm = get_normalization(norm_type, dim=node_feat_dim)
        self.energy_head = EnergyHead(node_feat_dim, mlp_hidden_dims, 1, "mlp", activation_type)
        self.magmom_head = MagmomHead(node_feat_dim, 2 * node_feat_dim, 1, "mlp", activation_type)
        self.force_stress_head = ForceStressHead(is_conservation, edge_feat_dim, mlp_hidden_dims, 3, "mlp",
                                                 activation_type)
        self._readout_pack = ops.ReadoutPack()  # the fused readout's weight layouts (no RNG)
        if verbose:
            print(f"MatRIS initialized with {self.get_params()} parameters")

    def forward(self, graphs, task: str = "ef", is_training: bool = False) -> dict:
        """model.py:183-250.

        The evaluation ends with one read of the device status word (the only stream
        sync of an evaluation): a graph index outside its range (found by the groupings'
        deferred checks) raises; in the "f16x3" MFMA arithmetic, a GEMM operand beyond the
        fp16 range makes the whole evaluation run again in "bf16x6" (a warning says so),
        so results never carry an overflow."""
        if is_training:
            raise NotImplementedError("training (double backward) is outside the efsm inference path")
        dev = next(self.parameters()).device
        try:
            pred = self._evaluate(graphs, task)
        except BaseException:
            ops.status_take(dev)  # leave no bits of a failed evaluation behind
            raise
        bits = ops.status_take(dev)
        if bits & ops.STATUS_CSR_KEY:
            raise RuntimeError("MatRIS: a graph index is outside its range (atom, bond or angle index)")
        if bits & ops.STATUS_F16_RANGE and ops.get_mma_precision() == "f16x3":
            import warnings
            warnings.warn("MatRIS: an activation exceeded the fp16 range of the f16x3 GEMMs; "
                          "the evaluation was redone in bf16x6", RuntimeWarning, stacklevel=2)
            with ops.mma_precision("bf16x6"):
                pred = self._evaluate(graphs, task)
            ops.status_take(dev)
        return pred

    def _readout_fusable(self) -> bool:
        """The configuration matris_readout_fwd implements: an affine RMSNorm(128), the energy
        MLP 128-128-128-1 and the magmom MLP 128-256-1 with biases and SiLU, no active dropout."""
        def lin(l, i, o):
            return isinstance(l, nn.Linear) and tuple(l.weight.shape) == (o, i) and l.bias is not None

        def drop_off(l):
            return isinstance(l, nn.Dropout) and (l.p == 0.0 or not l.training)

        n = self.readout_norm
        if not (isinstance(n, nn.RMSNorm) and n.weight is not None and tuple(n.normalized_shape) == (128,)):
            return False
        E, M = self.energy_head.energy_head, self.magmom_head.magmom_head
        if E.use_fp16 or M.use_fp16:
            return False
        L, K = list(E.layers), list(M.layers)
        return (len(L) == 7 and lin(L[0], 128, 128) and isinstance(L[1], FusedSiLU) and drop_off(L[2])
                and lin(L[3], 128, 128) and isinstance(L[4], FusedSiLU) and drop_off(L[5]) and lin(L[6], 128, 1)
                and len(K) == 4 and lin(K[0], 128, 256) and isinstance(K[1], FusedSiLU) and drop_off(K[2])
                and lin(K[3], 256, 1))

    def capture(self, graphs, task: str = "efsm", warmup: int = 2):
        """Opt-in: this evaluation of `graphs` recorded as a HIP graph (capture.py).  The
        returned object's replay() gives forward(graphs, task)'s outputs for the graphs'
        current positions and lattices, with their index arrays held fixed, the weights and
        MFMA arithmetic of capture time, and the same one status read per evaluation."""
        from .capture import CapturedEvaluation
        return CapturedEvaluation(self, graphs, task, warmup)

    def _evaluate(self, graphs, task: str) -> dict:
        is_training = False
        pred = {}
        bg = process_graphs(graphs, compute_stress="s" in task)
        bg["line_recompute"] = bool(self.line_recompute)
        n_blocks = len(self.interaction_block)
        if self.block_checkpoint is None:
            n_ckpt = fused.blocks_to_checkpoint(bg["n_angles"], bg["n_directed"], n_blocks,
                                                bg["atomic_numbers"].device)
        elif isinstance(self.block_checkpoint, bool):
            n_ckpt = n_blocks if self.block_checkpoint else 0
        else:
            n_ckpt = max(0, min(int(self.block_checkpoint), n_blocks))
        node = self.atom_embedding.embed(bg["atomic_numbers"])
        edge, smooth = self.edge_embedding(graphs=bg)
        # each basis is read by the Refinement of every block: one gradient buffer each
        smooth = {k: fused.shared_grad(v) for k, v in smooth.items()}
        tb = None
        if bg["n_angles"] != 0:
            tb = self.three_body_embedding(graphs=bg)
        for i, layer in enumerate(self.interaction_block):
            if i < n_ckpt:  # keep only the block inputs; the block's forward reruns in the backward
                node, edge, tb = torch.utils.checkpoint.checkpoint(layer, bg, node, edge, tb, smooth,
                                                                   use_reentrant=False, context_fn=_ckpt_contexts)
            else:
                node, edge, tb = layer(bg, node, edge, tb, smooth)
        if self._readout_fusable() and self.force_stress_head.is_conservation:
            # readout_norm, the energy MLP and the magmom MLP in one launch (matris_readout_fwd);
            # the energy's backward in one more (matris_readout_bwd)
            pack = self._readout_pack.get(self.readout_norm, self.energy_head.energy_head,
                                          self.magmom_head.magmom_head)
            e_atom, m_atom = ops.Readout.apply(node, pack)
            total = self.energy_head.pooling(e_atom.view(-1, 1), bg["atom_segment"], len(bg["atoms_per_graph"]),
                                             bg.get("atom_rowptr")).view(-1)
            pred.update(self.force_stress_head(bg, compute_force="f" in task, compute_stress="s" in task,
                                               total_energy=total, is_training=is_training))
            if "m" in task:
                pred["m"] = list(torch.split(m_atom, bg["atoms_per_graph"]))
        else:
            node = self.readout_norm(node)
            total = self.energy_head(bg, node)
            pred.update(self.force_stress_head(bg, compute_force="f" in task, compute_stress="s" in task,
                                               total_energy=total, is_training=is_training, node_feat=node,
                                               edge_feat=edge))
            if "m" in task:
                pred["m"] = self.magmom_head(bg, node)
        apg = bg["atoms_per_graph32"]  # made with the graph's topology: no host-to-device copy here
        pred["e"] = total / apg if self.is_intensive else total
        pred["atoms_per_graph"] = apg.clone()  # the caller's own copy, not the kept topology's
        # model.py:245-249: the composition energy of AtomRef (no position dependence)
        ref = 0 if self.reference_energy is None else self.reference_energy(graphs)
        pred["e"] = pred["e"] + ref
        pred["ref_energy"] = ref
        return pred

    def get_params(self) -> int:
        return sum(p.numel() for p in self.parameters())

    @classmethod
    def from_dict(cls, dct: dict):
        """model.py:256-260: {"config": kwargs, "state_dict": ...}."""
        m = cls(**dct["config"])
        m.load_state_dict(dct["state_dict"])
        return m

    @classmethod
    def load(cls, model_name: str = "matris_10m_oam", device: str | None = None, path: str | None = None):
        """model.py:262-317 without the network download: loads a local checkpoint
        ({"config", "state_dict"}, read with weights_only=True)."""
        import os
        if path is None:
            files = {"matris_10m_omat": "MatRIS_10M_OMAT.pth.tar", "matris_10m_oam": "MatRIS_10M_OAM.pth.tar",
                     "matris_10m_mp": "MatRIS_10M_MP.pth.tar", "matris_6m_mp": "MatRIS_6M_MP.pth.tar"}
            path = os.path.join(os.path.expanduser("~/.cache/matris"), files[model_name.lower()])
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not found (no network download on this path)")
        ckpt = torch.load(path, map_location="cpu", weights_only=True)
        model = cls.from_dict(ckpt)
        return model.to(device or ("cuda" if torch.cuda.is_available() else "cpu"))
