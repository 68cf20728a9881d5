"""CPU oracle for the MatRIS efsm path -- TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may
import this module, and only as the checker / the timed CPU baseline.  The product path
(`matris_amd`) never imports it.

This is a plain fp32 PyTorch (CPU) restatement of the reference forward pass plus
autograd forces / stress, written to mirror the reference module tree and construction
order so that `torch.manual_seed(s)` yields the same weights (and the same
`state_dict` keys) as the reference `MatRIS(**cfg)`.

Pins (see tests/test_oracle_model.py):
  * seed-0 state_dict fingerprint and C1 e/f/s/m golden vectors written by
    tests/golden/make_golden.py from the reference's own modules;
  * the non-default update forms (LayerNorm / BatchNorm GatedMLPs, graph_conv_mlp "MLP"
    with RMSNorm and with LayerNorm): per-tensor state_dict sums and the e/f/s/m of C1 and
    of three batched triclinic cells, from the reference modules (tests/golden/configs.npz);
  * the other constructor options (Gaussian and Fourier bases, smaller SH bases, no
    envelope, 9 radial functions, fixed bases, extensive energy, the direct force/stress
    head, GELU and ReLU activations, feature widths of 64 and of 128 / 96 / 64) in the
    same form (tests/golden/options.npz);
  * parameter counts 6,286,736 (defaults) / 10,379,664 (num_layers=10);
  * sum of forces = 0, stress symmetry, rotation equivariance, finite-difference
    forces and stress in fp64.

Each class / function cites the reference file:line it restates.
"""
from __future__ import annotations

import math
from collections.abc import Sequence

import torch
import torch.nn.functional as F
import torch.utils.checkpoint
from torch import Tensor, nn


# --------------------------------------------------------------------------------------
# primitives (matris/model/functions.py)
# --------------------------------------------------------------------------------------
class _SiLU(nn.Module):
    """functions.py:10-22 (CPU branch is F.silu)."""

    def forward(self, x):
        return F.silu(x)


class _Sigmoid(nn.Module):
    """functions.py:24-36 (CPU branch is torch.sigmoid)."""

    def forward(self, x):
        return torch.sigmoid(x)


def _act(name: str) -> nn.Module:
    """functions.py:38-55."""
    table = {"relu": nn.ReLU, "silu": _SiLU, "gelu": nn.GELU, "softplus": nn.Softplus, "sigmoid": _Sigmoid,
             "tanh": nn.Tanh}
    return table[name.lower()]()


def _norm(name: str, dim: int) -> nn.Module:
    """functions.py:57-68.  The reference builds all three norms and returns one;
    none of them consumes RNG, so building only the requested one is equivalent."""
    name = name.lower()
    if name == "layer":
        return nn.LayerNorm(dim)
    if name == "rms":
        return nn.RMSNorm(dim)
    if name == "batch":
        return nn.BatchNorm1d(dim)
    raise KeyError(name)


class SwishLayer(nn.Module):
    """functions.py:70-95: SiLU(Linear(x))."""

    def __init__(self, input_dim=128, output_dim=128, bias=True):
        super().__init__()
        self.linear = nn.Linear(input_dim, output_dim, bias=bias)
        self.act = _SiLU()

    def forward(self, x):
        return self.act(self.linear(x))


def dimwise_softmax(feas: Tensor, segment: Tensor, num_segment=None) -> Tensor:
    """functions.py:97-127: per-column softmax within segments."""
    num, dim = feas.shape
    if num_segment is None:
        num_segment = int(segment.max()) + 1
    seg = segment.unsqueeze(1).expand(-1, dim)
    fmax = torch.full((num_segment, dim), float("-inf"), dtype=feas.dtype)
    fmax = fmax.scatter_reduce(0, seg, feas, reduce="amax", include_self=False)
    out = (feas - fmax[segment]).exp()
    ssum = torch.zeros(num_segment, dim, dtype=feas.dtype)
    ssum = ssum.scatter_reduce(0, seg, out, reduce="sum", include_self=False)
    return out / ssum[segment]


def aggregate(data: Tensor, segment: Tensor, bin_count=None, average=True,
              num_segment=None) -> Tensor:
    """functions.py:129-160: index_add_ segment sum (optionally mean)."""
    if bin_count is None:
        bin_count = torch.bincount(segment)
        bin_count = bin_count.where(bin_count != 0, bin_count.new_ones(1))
    if num_segment is not None and bin_count.shape[0] != num_segment:
        bin_count = torch.cat([bin_count, bin_count.new_ones(num_segment - bin_count.shape[0])])
    out = data.new_zeros([bin_count.shape[0], data.shape[1]])
    out = out.index_add_(0, segment, data)
    if average:
        out = (out.T / bin_count).T
    return out


class MLP(nn.Module):
    """functions.py:163-242 (dropout is 0 in every config used here)."""

    def __init__(self, input_dim=128, hidden_dim=(128, 128), output_dim=128,
                 dropout=0.0, activation="silu", bias=True):
        super().__init__()
        act = _act(activation)
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
            raise TypeError(type(hidden_dim))
        self.layers = nn.Sequential(*layers)

    def forward(self, x):
        return self.layers(x)


class GatedMLP(nn.Module):
    """functions.py:245-311: SiLU(norm(MLP_core(x))) * sigmoid(norm(MLP_gate(x)))."""

    def __init__(self, input_dim=128, hidden_dim=(128, 128), output_dim=128, dropout=0.0,
                 activation="silu", norm_type="layer", bias=True):
        super().__init__()
        self.activation_func = _act(activation)
        self.activation_gate = _Sigmoid()
        self.gate_norm = _norm(norm_type, output_dim)
        self.core_norm = _norm(norm_type, output_dim)
        self.mlp_core = MLP(input_dim, hidden_dim, output_dim, dropout, activation, bias)
        self.mlp_gate = MLP(input_dim, hidden_dim, output_dim, dropout, activation, bias)

    def forward(self, x):
        core = self.activation_func(self.core_norm(self.mlp_core(x)))
        gate = self.activation_gate(self.gate_norm(self.mlp_gate(x)))
        return core * gate


class GraphPooling(nn.Module):
    """functions.py:340-365."""

    def __init__(self, average=False):
        super().__init__()
        self.average = average

    def forward(self, x, segment):
        return aggregate(x, segment, None, self.average, None)


# --------------------------------------------------------------------------------------
# basis functions (matris/model/basis_function.py)
# --------------------------------------------------------------------------------------
class PolynomialEnvelope(nn.Module):
    """basis_function.py:8-50."""

    def __init__(self, cutoff=6, envelope_exponent=8):
        super().__init__()
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
    """basis_function.py:116-186 (learnable frequencies n*pi)."""

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

    def forward(self, dist):
        dist = dist[:, None]
        out = self.norm_const * torch.sin(self.frequencies * (dist * self.inv_cutoff)) / dist
        return out if self.envelope_func is None else self.envelope_func(dist) * out


class GaussianExpansion(nn.Module):
    """basis_function.py:189-219."""

    def __init__(self, start=0.0, stop=6.0, num_gaussians=7, basis_width_scalar=2.0):
        super().__init__()
        offset = torch.linspace(start, stop, num_gaussians)
        self.coeff = -0.5 / (basis_width_scalar * (offset[1] - offset[0])).item() ** 2
        self.register_buffer("offset", offset)

    def forward(self, dist):
        return torch.exp(self.coeff * (dist.view(-1, 1) - self.offset.view(1, -1)) ** 2)


class FourierExpansion(nn.Module):
    """basis_function.py:79-113."""

    def __init__(self, max_f=5, scale=math.pi, learnable=False):
        super().__init__()
        self.max_f, self.scale = max_f, math.sqrt(scale)
        freq = torch.arange(1, max_f + 1, dtype=torch.float)
        if learnable:
            self.frequencies = nn.Parameter(freq, requires_grad=True)
        else:
            self.register_buffer("frequencies", freq)

    def forward(self, angle):
        out = angle.new_zeros(angle.shape[0], 1 + 2 * self.max_f)
        out[:, 0] = 1.0 / math.sqrt(2.0)
        t = torch.outer(angle, self.frequencies)
        out[:, 1:self.max_f + 1] = torch.sin(t)
        out[:, self.max_f + 1:] = torch.cos(t)
        return out / self.scale


def spherical_harmonics_l3(x: Tensor, lmax: int = 3) -> Tensor:
    """basis_function.py:53-77 (Y_l(cos theta), m=0, l = 0..lmax)."""
    y0 = torch.ones_like(x) * 0.5 * math.sqrt(1.0 / math.pi)
    y1 = math.sqrt(3.0 / (4.0 * math.pi)) * x
    y2 = math.sqrt(5.0 / (16.0 * math.pi)) * (3.0 * x ** 2 - 1.0)
    y3 = math.sqrt(7.0 / (16.0 * math.pi)) * x * (5.0 * x ** 2 - 3.0)
    return torch.stack([y0, y1, y2, y3][:lmax + 1], dim=-1)


# Coefficient table of the spherical Bessel radial functions, basis_function.py:241-274
# (float32 values as stored by the reference in a float32 tensor).
SBF_COEF = {
    "z1": [3.14159274101257, 6.28318548202515, 9.42477798461914, 12.5663709640503],
    "c1": [[-1.02446483277785, -1.00834335996107, -1.00419641763893, -1.00252381898662],
           [4.49340963363647, 7.7252516746521, 10.9041213989258, 14.0661935806274],
           [0.22799275301076, 0.130525632358311, 0.092093290316619, 0.0712718627992818],
           [4.49340963363647, 7.7252516746521, 10.9041213989258, 14.0661935806274]],
    "c2": [[-1.04807944170731, -1.01861796359391, -1.01002272174988, -1.00628955560036],
           [5.76345920562744, 9.09501171112061, 12.322940826416, 15.5146026611328],
           [0.545547077361439, 0.335992298618515, 0.245888396928293, 0.194582402961821],
           [5.76345920562744, 9.09501171112061, 12.322940826416, 15.5146026611328],
           [0.0946561878721665, 0.0369424811413594, 0.0199537107571916, 0.0125418876146463],
           [5.76345920562744, 9.09501171112061, 12.322940826416, 15.5146026611328]],
    "c3": [[1.06942831392075, 1.0292173312802, 1.01650804843248, 1.01069656069999],
           [6.9879322052002, 10.4171180725098, 13.6980228424072, 16.9236221313477],
           [0.918235852195231, 0.592803493701152, 0.445250264272671, 0.358326327374518],
           [6.9879322052002, 10.4171180725098, 13.6980228424072, 16.9236221313477],
           [0.328507713452024, 0.142266673367543, 0.0812617757677838, 0.0529328657590962],
           [6.9879322052002, 10.4171180725098, 13.6980228424072, 16.9236221313477],
           [0.0470107184508114, 0.0136570088173405, 0.0059323726279831, 0.00312775039221944],
           [6.9879322052002, 10.4171180725098, 13.6980228424072, 16.9236221313477]],
}


class SphericalExpansion(nn.Module):
    """basis_function.py:222-338 (max_n, max_l <= 4)."""

    def __init__(self, max_n=4, max_l=4, cutoff=6):
        super().__init__()
        assert 1 <= max_n <= 4 and 1 <= max_l <= 4
        self.max_n, self.max_l, self.cutoff = max_n, max_l, cutoff
        self.register_buffer("factor", torch.sqrt(torch.tensor(2.0 / (cutoff ** 3))))
        coef = torch.zeros(4, 9, 4)
        coef[0, 0, :] = torch.tensor(SBF_COEF["z1"])
        coef[1, :4, :] = torch.tensor(SBF_COEF["c1"])
        coef[2, :6, :] = torch.tensor(SBF_COEF["c2"])
        coef[3, :8, :] = torch.tensor(SBF_COEF["c3"])
        self.coef = coef

    def forward(self, dist, three_body):
        c = self.coef
        x = dist / self.cutoff
        rbfs = []
        L = range(self.max_l)
        for j in L:
            rbfs.append(torch.sin(c[0, 0, j] * x) / x)
        if self.max_n > 1:
            for j in L:
                rbfs.append((c[1, 0, j] * x * torch.cos(c[1, 1, j] * x) + c[1, 2, j] * torch.sin(c[1, 3, j] * x))
                            / x ** 2)
        if self.max_n > 2:
            for j in L:
                rbfs.append((c[2, 0, j] * x ** 2 * torch.sin(c[2, 1, j] * x) - c[2, 2, j] * x * torch.cos(c[2, 3, j] * x)
                             + c[2, 4, j] * torch.sin(c[2, 5, j] * x)) / x ** 3)
        if self.max_n > 3:
            for j in L:
                rbfs.append((c[3, 0, j] * x ** 3 * torch.cos(c[3, 1, j] * x)
                             - c[3, 2, j] * x ** 2 * torch.sin(c[3, 3, j] * x)
                             - c[3, 4, j] * x * torch.cos(c[3, 5, j] * x) + c[3, 6, j] * torch.sin(c[3, 7, j] * x))
                            / x ** 4)
        rbfs = torch.stack(rbfs, dim=-1) * self.factor
        cbfs = spherical_harmonics_l3(torch.cos(three_body), self.max_l - 1).repeat_interleave(self.max_n, dim=1)
        return rbfs * cbfs


# --------------------------------------------------------------------------------------
# embeddings (matris/model/feature_embed.py)
# --------------------------------------------------------------------------------------
class AtomTypeEmbedding(nn.Module):
    """feature_embed.py:16-39."""

    def __init__(self, atom_feat_dim, max_num_elements=94):
        super().__init__()
        self.embedding = nn.Embedding(max_num_elements, atom_feat_dim)
        self.atom_swish_layer = SwishLayer(atom_feat_dim, atom_feat_dim, bias=False)

    def forward(self, atom_type):
        return self.atom_swish_layer(self.embedding(atom_type))


class EdgeBasisEmbedding(nn.Module):
    """feature_embed.py:42-148."""

    def __init__(self, pairwise_cutoff=6, three_body_cutoff=4, num_radial=7, edge_feat_dim=128,
                 envelope_exponent=8, distance_expansion="Bessel", learnable=False):
        super().__init__()
        if distance_expansion.lower() == "bessel":
            self.pairwise_rbf_expansion = BesselExpansion(num_radial, pairwise_cutoff, envelope_exponent, learnable)
            self.threebody_rbf_expansion = BesselExpansion(num_radial, three_body_cutoff, envelope_exponent, learnable)
        else:
            assert distance_expansion.lower() == "gaussian"
            self.pairwise_rbf_expansion = GaussianExpansion(0.0, pairwise_cutoff, num_radial, 2.0)
            self.threebody_rbf_expansion = GaussianExpansion(0.0, three_body_cutoff, num_radial, 2.0)
        self.edge_linear1 = nn.Linear(num_radial, edge_feat_dim, bias=False)
        self.edge_linear2 = nn.Linear(edge_feat_dim, edge_feat_dim, bias=False)
        self.swish_layer = SwishLayer(edge_feat_dim, edge_feat_dim, bias=False)
        self.edge_init_norm = _norm("layer", edge_feat_dim)

    def forward(self, g):
        lengths = torch.index_select(g["edge_lengths"], 0, g["undirected2directed"])
        rbf6 = self.pairwise_rbf_expansion(lengths)
        rbf4 = self.threebody_rbf_expansion(lengths)
        e = self.edge_linear1(rbf6)
        e = torch.index_select(e, 0, g["directed2undirected"])
        e = self.edge_init_norm(self.edge_linear2(e))
        e = aggregate(e, g["directed2undirected"], None, True, None)
        e = self.swish_layer(e)
        return e, {"atom graph": rbf6, "line graph": rbf4}


class ThreebodyEmbedding(nn.Module):
    """feature_embed.py:151-203."""

    def __init__(self, num_angular=7, max_n=4, max_l=4, cutoff=6, three_body_feat_dim=128,
                 three_body_expansion="sh", learnable=True):
        super().__init__()
        self.sh = three_body_expansion.lower() == "sh"
        if self.sh:
            self.expansion = SphericalExpansion(max_n, max_l, cutoff)
            self.angle_embedding = nn.Linear(max_n * max_l, three_body_feat_dim, bias=False)
        else:
            assert three_body_expansion.lower() == "fourier"
            self.expansion = FourierExpansion((num_angular - 1) // 2, learnable=learnable)
            self.angle_embedding = nn.Linear(num_angular, three_body_feat_dim, bias=False)
        self.swish_layer = SwishLayer(three_body_feat_dim, three_body_feat_dim, bias=False)

    def forward(self, g):
        lg = g["line_graph_dict"]
        vij = torch.index_select(g["unit_edge_vectors"], 0, lg["target_DE_index"])
        vjk = torch.index_select(g["unit_edge_vectors"], 0, lg["source_DE_index"])
        cos_t = torch.sum(vij * vjk, dim=1) * (1 - 1e-6)
        angle = torch.acos(cos_t)
        basis = self.expansion(torch.norm(vjk, dim=1), angle) if self.sh else self.expansion(angle)
        return self.swish_layer(self.angle_embedding(basis))


# --------------------------------------------------------------------------------------
# interaction block (matris/model/interaction_block.py)
# --------------------------------------------------------------------------------------
def _update(mlp_type, input_dim, hidden_dim, output_dim, norm_type, bias, activation="silu"):
    """The nonlinear update of an attention / refinement layer: a GatedMLP (its MLPs keep
    their biases), or, for mlp_type "MLP", MLP(bias=use_bias) followed by the norm
    (interaction_block.py:39-74, 172-197)."""
    if mlp_type.lower() == "gatemlp":
        return GatedMLP(input_dim, hidden_dim, output_dim, activation=activation, norm_type=norm_type)
    if mlp_type.lower() == "mlp":
        return nn.Sequential(MLP(input_dim, hidden_dim, output_dim, activation=activation, bias=bias),
                             _norm(norm_type, output_dim))
    raise NotImplementedError(mlp_type)


class GraphAttentionLayer(nn.Module):
    """interaction_block.py:17-143."""

    def __init__(self, node_feat_dim=128, edge_feat_dim=128, hidden_dim=128, norm_type="layer",
                 mlp_type="GateMLP", use_bias=False, activation="silu"):
        super().__init__()
        self.source_weight_linear = nn.Linear(edge_feat_dim, edge_feat_dim, bias=False)
        self.target_weight_linear = nn.Linear(edge_feat_dim, edge_feat_dim, bias=False)
        self.node_nonlinear_update = _update(mlp_type, edge_feat_dim * 2 + node_feat_dim, hidden_dim, node_feat_dim,
                                             norm_type, use_bias, activation)
        self.edge_nonlinear_update = _update(mlp_type, node_feat_dim * 2 + edge_feat_dim, hidden_dim, edge_feat_dim,
                                             norm_type, use_bias, activation)
        self.node_res_weight = nn.Parameter(torch.ones(1, node_feat_dim))
        self.edge_res_weight = nn.Parameter(torch.ones(1, edge_feat_dim))

    def forward(self, node_feat, edge_feat, graph, d2u=None):
        src, tgt = graph["source_index"], graph["target_index"]
        src_f = torch.index_select(node_feat, 0, src)
        tgt_f = torch.index_select(node_feat, 0, tgt)
        e0 = torch.index_select(edge_feat, 0, d2u) if d2u is not None else edge_feat
        e = self.edge_nonlinear_update(torch.cat([e0, tgt_f, src_f], dim=1))
        a_s = dimwise_softmax(self.source_weight_linear(e0), src)
        a_t = dimwise_softmax(self.target_weight_linear(e0), tgt)
        sw, tw = a_s * e, a_t * e
        if d2u is not None:
            e = aggregate(e, d2u, None, True, None)
        ys = aggregate(sw, src, graph["source_bincount"], False, len(node_feat))
        yt = aggregate(tw, tgt, graph["target_bincount"], False, len(node_feat))
        n = self.node_nonlinear_update(torch.cat([node_feat, yt, ys], dim=1))
        return n + self.node_res_weight * node_feat, e + self.edge_res_weight * edge_feat


class Refinement(nn.Module):
    """interaction_block.py:146-278."""

    def __init__(self, node_feat_dim=128, edge_feat_dim=128, hidden_dim=128, num_basis=7,
                 norm_type="layer", graph_type="atom graph", atom_feat_dim=128,
                 use_smoothed_for_delta_edge=False, use_bias=False, mlp_type="GateMLP", activation="silu"):
        super().__init__()
        self.graph_type = graph_type
        self.use_smoothed_for_delta_edge = use_smoothed_for_delta_edge
        if graph_type == "atom graph":
            input_dim = 2 * node_feat_dim + edge_feat_dim
        else:
            input_dim = atom_feat_dim + 2 * node_feat_dim + edge_feat_dim
        self.edge_nonlinear_update = _update(mlp_type, input_dim, hidden_dim, edge_feat_dim, norm_type, use_bias,
                                             activation)
        self.node_FFN = MLP(edge_feat_dim, node_feat_dim, node_feat_dim, bias=use_bias)
        self.edge_FFN = MLP(edge_feat_dim, edge_feat_dim, edge_feat_dim, bias=use_bias)
        self.learnable_envelope = nn.Linear(num_basis, edge_feat_dim, bias=False)
        self.node_res_weight = nn.Parameter(torch.ones(1, node_feat_dim))
        self.edge_res_weight = nn.Parameter(torch.ones(1, edge_feat_dim))

    def forward(self, node_feat, edge_feat, smooth_weight, graph, d2u=None, atom_feat=None):
        atom_graph = self.graph_type == "atom graph"
        e0 = torch.index_select(edge_feat, 0, d2u) if atom_graph else edge_feat
        src_f = torch.index_select(node_feat, 0, graph["source_index"])
        tgt_f = torch.index_select(node_feat, 0, graph["target_index"])
        if atom_graph:
            w = self.learnable_envelope(torch.index_select(smooth_weight, 0, d2u))
            x = torch.cat([e0, tgt_f, src_f], dim=1)
        else:
            env = self.learnable_envelope(smooth_weight)
            w = torch.index_select(env, 0, graph["source_index"]) * torch.index_select(env, 0, graph["target_index"])
            x = torch.cat([e0, torch.index_select(atom_feat, 0, graph["atom_list"]), tgt_f, src_f], dim=1)
        h = self.edge_nonlinear_update(x)
        hw = h * w
        agg = aggregate(hw, graph["target_index"], graph["target_bincount"], False, len(node_feat))
        to_edge = hw if (atom_graph and self.use_smoothed_for_delta_edge) else h
        dn = self.node_FFN(agg)
        de = self.edge_FFN(to_edge)
        if atom_graph:
            de = aggregate(de, d2u, None, True, None)
        return dn + self.node_res_weight * node_feat, de + self.edge_res_weight * edge_feat


class InteractionBlock(nn.Module):
    """interaction_block.py:281-446 (checkpointing changes memory, not values)."""

    def __init__(self, node_feat_dim=128, edge_feat_dim=128, three_body_feat_dim=128, num_radial=7,
                 num_angular=7, use_bias=False, use_smoothed_for_delta_edge=False, norm_type="layer",
                 mlp_type="GateMLP", activation="silu"):
        super().__init__()
        self.attn_block_atom_graph = GraphAttentionLayer(node_feat_dim, edge_feat_dim, node_feat_dim, norm_type,
                                                         mlp_type, use_bias, activation)
        self.attn_block_line_graph = GraphAttentionLayer(edge_feat_dim, three_body_feat_dim, edge_feat_dim, norm_type,
                                                         mlp_type, use_bias, activation)
        self.refine_block_atom_graph = Refinement(node_feat_dim, edge_feat_dim, node_feat_dim, num_radial, norm_type,
                                                  "atom graph", use_smoothed_for_delta_edge=use_smoothed_for_delta_edge,
                                                  use_bias=use_bias, mlp_type=mlp_type, activation=activation)
        self.refine_block_line_graph = Refinement(edge_feat_dim, three_body_feat_dim, edge_feat_dim, num_angular,
                                                  norm_type, "line graph", atom_feat_dim=node_feat_dim,
                                                  use_bias=use_bias, mlp_type=mlp_type, activation=activation)

    def forward(self, g, node_feat, edge_feat, tb_feat, smooth_weight):
        attn_edge, attn_tb = edge_feat, tb_feat
        upd_edge, upd_tb = edge_feat, tb_feat
        # interaction_block.py:15,400-413: the two line-graph layers are checkpointed above
        # 60,000 angles (same values, less memory, their forward rerun in the backward)
        ckpt = tb_feat is not None and tb_feat.shape[0] > 60000 and torch.is_grad_enabled()

        def run(layer, *args, **kw):
            if ckpt:
                return torch.utils.checkpoint.checkpoint(layer, *args, use_reentrant=False, **kw)
            return layer(*args, **kw)

        if tb_feat is not None:
            attn_edge, attn_tb = run(self.attn_block_line_graph, edge_feat, tb_feat, g["line_graph_dict"])
        attn_node, attn_edge = self.attn_block_atom_graph(node_feat, attn_edge, g["atom_graph_dict"],
                                                          g["directed2undirected"])
        if tb_feat is not None:
            upd_edge, upd_tb = run(self.refine_block_line_graph, attn_edge, attn_tb, smooth_weight["line graph"],
                                   g["line_graph_dict"], atom_feat=attn_node)
        upd_node, upd_edge = self.refine_block_atom_graph(attn_node, upd_edge, smooth_weight["atom graph"],
                                                          g["atom_graph_dict"], d2u=g["directed2undirected"])
        return upd_node, upd_edge, upd_tb


# --------------------------------------------------------------------------------------
# batching (matris/model/processgraph.py)
# --------------------------------------------------------------------------------------
def process_graphs(graphs, compute_stress=True):
    """processgraph.py:6-245, for CPU tensors.  Each graph is a dict/object with the
    RadiusGraph fields (radiusgraph.py:17-95)."""
    get = (lambda gr, k: gr[k]) if isinstance(graphs[0], dict) else (lambda gr, k: getattr(gr, k))
    out = {}
    zs, ags, lgs, segs, napg = [], [], [], [], []
    lats, imgs, carts, d2us, u2ds = [], [], [], [], []
    a_off = u_off = d_off = 0
    for gi, gr in enumerate(graphs):
        z = get(gr, "atomic_number")
        n = z.shape[0]
        zs.append(z)
        napg.append(n)
        frac = get(gr, "atom_frac_coord").detach()
        lat = get(gr, "lattice").detach()
        carts.append(frac @ lat)
        lats.append(lat)
        imgs.append(get(gr, "neighbor_image"))
        ag = get(gr, "atom_graph")
        ags.append(ag.to(torch.int64) + a_off)
        d2us.append(get(gr, "directed2undirected").to(torch.int64) + u_off)
        u2ds.append(get(gr, "undirected2directed").to(torch.int64) + d_off)
        lg = get(gr, "line_graph")
        if len(lg) != 0:
            lg = lg.to(torch.int64).clone()
            lg[:, 0] += a_off
            lg[:, 1] += u_off
            lg[:, 3] += u_off
            lg[:, 2] += d_off
            lg[:, 4] += d_off
            lgs.append(lg)
        segs.append(torch.full((n,), gi, dtype=torch.int64))
        a_off += n
        u_off += len(get(gr, "undirected2directed"))
        d_off += len(get(gr, "directed2undirected"))
    G = len(graphs)
    ag = torch.cat(ags, 0)
    seg = torch.cat(segs, 0)
    lat = torch.cat(lats, 0)
    cart = torch.cat(carts, 0)
    image = torch.block_diag(*imgs)
    lat3 = lat.reshape(G, 3, 3)
    vol = torch.einsum("ni,ni->n", lat3[:, 0], torch.linalg.cross(lat3[:, 1], lat3[:, 2]))[:, None, None]
    cart.requires_grad_(True)
    strains = None
    if compute_stress:
        strains = torch.zeros((G, 3, 3), dtype=lat.dtype, requires_grad=True)
        sym = 0.5 * (strains + strains.transpose(-1, -2))
        cart = cart + torch.einsum("be,bec->bc", cart, sym[seg])
        lat = (lat.view(-1, 3, 3) + torch.matmul(lat.view(-1, 3, 3), sym)).view(-1, 3)
    tgt, src = ag[:, 0], ag[:, 1]
    vec = cart[tgt] - (cart[src] + image @ lat)
    length = torch.norm(vec, dim=1)
    out.update(atomic_numbers=torch.cat(zs, 0), edge_lengths=length, unit_edge_vectors=vec / length[:, None],
               atom_segment=seg, atoms_per_graph=napg, directed2undirected=torch.cat(d2us, 0),
               undirected2directed=torch.cat(u2ds, 0), volumes=vol, lattice=lat,
               batch_cart_coords=cart, batch_strains=strains)
    bc = lambda i: (lambda b: b.where(b != 0, b.new_ones(1)))(torch.bincount(i))
    out["atom_graph_dict"] = dict(atom_graph=ag, target_index=tgt, source_index=src,
                                  source_bincount=bc(src), target_bincount=bc(tgt))
    lgd = {}
    if lgs:
        lg = torch.cat(lgs, 0)
        lgd = dict(line_graph=lg[:, [0, 1, 3]], atom_list=lg[:, 0], target_index=lg[:, 1], source_index=lg[:, 3],
                   target_DE_index=lg[:, 2], source_DE_index=lg[:, 4], source_bincount=bc(lg[:, 3]),
                   target_bincount=bc(lg[:, 1]))
    else:
        lgd = dict(line_graph=torch.tensor([]))
    out["line_graph_dict"] = lgd
    # 'batch_cart_coords' holds the strained coordinates (processgraph.py:179-185,
    # :213); readout.py:205-208 differentiates w.r.t. that tensor and the strain leaf.
    return out


# --------------------------------------------------------------------------------------
# direct force / stress head (matris/model/readout.py:136-334, functions.py:368-463)
# --------------------------------------------------------------------------------------
# functions.py:368-398: rows map the 9 irrep components (l = 0; l = 1 x3; l = 2 x5) of a
# rank-2 tensor to its Cartesian entries (xx, xy, xz, yx, yy, yz, zx, zy, zz)
_S2, _S3, _S6 = 2 ** -0.5, 3 ** -0.5, 6 ** -0.5
CG_CHANGE_MAT = [[_S3, 0, 0, 0, _S3, 0, 0, 0, _S3],
                 [0, 0, 0, 0, 0, _S2, 0, -_S2, 0],
                 [0, 0, -_S2, 0, 0, 0, _S2, 0, 0],
                 [0, _S2, 0, -_S2, 0, 0, 0, 0, 0],
                 [0, 0, _S2, 0, 0, 0, _S2, 0, 0],
                 [0, _S2, 0, _S2, 0, 0, 0, 0, 0],
                 [-_S6, 0, 0, 0, 2 * _S6, 0, 0, 0, -_S6],
                 [0, 0, 0, 0, 0, _S2, 0, _S2, 0],
                 [-_S2, 0, 0, 0, 0, 0, 0, 0, _S2]]


def sphere_l2(v):
    """functions.py:436-463, lmax = 2."""
    x, y, z = v[:, 0], v[:, 1], v[:, 2]
    return torch.stack([torch.ones_like(x), x, y, z, math.sqrt(3.0) * x * z, math.sqrt(3.0) * x * y,
                        y.pow(2) - 0.5 * (x.pow(2) + z.pow(2)), math.sqrt(3.0) * y * z,
                        math.sqrt(3.0) / 2.0 * (z.pow(2) - x.pow(2))], dim=-1)


class GatedEquivariantBlock(nn.Module):
    """readout.py:255-292."""

    def __init__(self, hidden_channels, out_channels, activation="silu"):
        super().__init__()
        self.out_channels = out_channels
        self.vec1_proj = nn.Linear(hidden_channels, hidden_channels, bias=False)
        self.vec2_proj = nn.Linear(hidden_channels, out_channels, bias=False)
        self.act = _act(activation)
        self.update_net = nn.Sequential(nn.Linear(hidden_channels * 2, hidden_channels), self.act,
                                        nn.Linear(hidden_channels, out_channels * 2))

    def forward(self, feas, vec_feas):
        vec1 = torch.norm(self.vec1_proj(vec_feas), dim=-2)
        vec2 = self.vec2_proj(vec_feas)
        feas, vec_feas = torch.split(self.update_net(torch.cat([feas, vec1], dim=-1)), self.out_channels, dim=-1)
        return self.act(feas), vec_feas.unsqueeze(1) * vec2


class EquivariantHead(nn.Module):
    """readout.py:295-334 (lmax = 2)."""

    def __init__(self, feas_dim=64, activation="silu"):
        super().__init__()
        self.feas_wise_linear = nn.Linear(feas_dim, feas_dim, bias=False)
        self.basis_wise_linear = nn.Linear(1, feas_dim, bias=False)
        self.equivariant_block = nn.ModuleList([GatedEquivariantBlock(feas_dim, feas_dim // 2, activation),
                                                GatedEquivariantBlock(feas_dim // 2, 1, activation)])

    def forward(self, feas, vec):
        vec_feas = self.basis_wise_linear(sphere_l2(vec).unsqueeze(2))
        feas = self.feas_wise_linear(feas)
        for layer in self.equivariant_block:
            feas, vec_feas = layer(feas, vec_feas)
        return vec_feas.squeeze(-1)


class DirectHead(nn.Module):
    """readout.py:136-252, is_conservation=False (mlp_type "mlp", as model.py:171-178)."""

    def __init__(self, feat_dim, hidden_dims, activation="silu"):
        super().__init__()
        self.stress_head = EquivariantHead(feat_dim, activation)
        self.force_head = MLP(feat_dim, hidden_dims, 3, activation=activation)

    def forward(self, g, node_feat, edge_feat, compute_force, compute_stress):
        pred = {}
        if compute_stress:
            c = g["batch_cart_coords"]
            vec = c / ((torch.norm(c, dim=1) * (1 - 1e-6) + 1e-6).unsqueeze(1))
            st = aggregate(self.stress_head(node_feat, vec), g["atom_segment"], None, True, None)
            irreps = st.new_zeros(st.shape[0], 9)
            irreps[:, 0] = st[:, 0]
            irreps[:, 4:9] = st[:, 4:9]
            cart = (irreps @ torch.tensor(CG_CHANGE_MAT, dtype=st.dtype)).view(-1, 3, 3)
            pred["s"] = list(torch.unbind(cart * (1 / g["volumes"] * 160.21766208), dim=0))
        if compute_force:
            w = self.force_head(torch.index_select(edge_feat, 0, g["directed2undirected"])) * g["unit_edge_vectors"]
            f = aggregate(w, g["atom_graph_dict"]["target_index"], None, False, len(node_feat))
            pred["f"] = torch.split(f, g["atoms_per_graph"])
        return pred


# --------------------------------------------------------------------------------------
# model (matris/model/model.py, readout.py)
# --------------------------------------------------------------------------------------
class MatRISRef(nn.Module):
    """model.py:30-250 with the conservative readout (readout.py:18-133,193-224), or the
    direct one (is_conservation=False)."""

    def __init__(self, num_layers=6, node_feat_dim=128, edge_feat_dim=128, three_body_feat_dim=128,
                 mlp_hidden_dims=(128, 128), dropout=0.0, use_bias=False, distance_expansion="Bessel",
                 three_body_expansion="SH", num_radial=7, num_angular=7, max_l=4, max_n=4,
                 envelope_exponent=8, graph_conv_mlp="GateMLP", activation_type="silu", norm_type="rms",
                 pairwise_cutoff=6, three_body_cutoff=4, use_smoothed_for_delta_edge=False,
                 learnable_basis=True, is_intensive=True, is_conservation=True, reference_energy=None):
        super().__init__()
        assert reference_energy is None
        self.is_intensive = is_intensive
        self.is_conservation = is_conservation
        self.atom_embedding = AtomTypeEmbedding(node_feat_dim)
        self.edge_embedding = EdgeBasisEmbedding(pairwise_cutoff, three_body_cutoff, num_radial, edge_feat_dim,
                                                 envelope_exponent, distance_expansion, learnable_basis)
        self.three_body_embedding = ThreebodyEmbedding(num_angular, max_n, max_l, pairwise_cutoff,
                                                       three_body_feat_dim, three_body_expansion, learnable_basis)
        self.interaction_block = nn.ModuleList([
            InteractionBlock(node_feat_dim, edge_feat_dim, three_body_feat_dim, num_radial, num_angular,
                             use_bias, use_smoothed_for_delta_edge, norm_type, graph_conv_mlp, activation_type)
            for _ in range(num_layers)])
        self.readout_norm = _norm(norm_type, node_feat_dim)
        hd = [mlp_hidden_dims] if isinstance(mlp_hidden_dims, int) else list(mlp_hidden_dims)
        self.energy_head = nn.Module()
        self.energy_head.energy_head = MLP(node_feat_dim, hd, 1, activation=activation_type)
        self.energy_head.pooling = GraphPooling(False)
        self.magmom_head = nn.Module()
        self.magmom_head.magmom_head = MLP(node_feat_dim, [2 * node_feat_dim], 1, activation=activation_type)
        if not is_conservation:
            self.force_stress_head = DirectHead(edge_feat_dim, hd, activation_type)

    def forward(self, graphs, task="ef", is_training=False):
        g = process_graphs(graphs, compute_stress="s" in task)
        node = self.atom_embedding(g["atomic_numbers"] - 1)
        edge, smooth = self.edge_embedding(g)
        tb = self.three_body_embedding(g) if len(g["line_graph_dict"]["line_graph"]) != 0 else None
        for blk in self.interaction_block:
            node, edge, tb = blk(g, node, edge, tb, smooth)
        node = self.readout_norm(node)
        e_atoms = self.energy_head.energy_head(node)
        total = self.energy_head.pooling(e_atoms, g["atom_segment"]).view(-1)
        pred = {}
        if not self.is_conservation:
            pred.update(self.force_stress_head(g, node, edge, "f" in task, "s" in task))
        elif "f" in task and "s" in task:
            gc, gs = torch.autograd.grad(total.sum(), [g["batch_cart_coords"], g["batch_strains"]],
                                         create_graph=is_training, retain_graph=is_training)
            pred["f"] = torch.split(-gc, g["atoms_per_graph"])
            pred["s"] = list(torch.unbind(gs * (1 / g["volumes"] * 160.21766208), dim=0))
        elif "f" in task:
            (gc,) = torch.autograd.grad(total.sum(), [g["batch_cart_coords"]], create_graph=is_training,
                                        retain_graph=is_training)
            pred["f"] = torch.split(-gc, g["atoms_per_graph"])
        if "m" in task:
            m = torch.abs(self.magmom_head.magmom_head(node))
            pred["m"] = list(torch.split(m.view(-1), g["atoms_per_graph"]))
        apg = torch.tensor(g["atoms_per_graph"], dtype=torch.int32)
        pred["e"] = (total / apg if self.is_intensive else total) + 0
        pred["atoms_per_graph"] = apg
        pred["ref_energy"] = 0
        return pred
