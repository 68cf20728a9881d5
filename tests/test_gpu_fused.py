"""The explicit-backward line-graph layers (matris_amd/model/fused.py) against an fp64
torch restatement of the reference layers, forward values and every input gradient.

Reference: matris/model/interaction_block.py:17-143 (Graph_Attention_Layer) and
:146-278 (Refinement, line graph), functions.py:97-160 (Dimwise_softmax, aggregate),
functions.py:245-311 (GatedMLP with RMSNorm).
"""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

DEV = "cuda"
EPS32 = torch.finfo(torch.float32).eps  # RMSNorm(eps=None) in the fp32 reference


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


def _gmlp64(mod, x):
    """GatedMLP forward in fp64 from the module's parameters (RMSNorm with fp32 eps)."""
    def mlp(m):
        L = m.layers
        return F.linear(F.silu(F.linear(x, L[0].weight.double(), L[0].bias.double())), L[3].weight.double(),
                        L[3].bias.double())

    def rms(v, w):
        return v * torch.rsqrt((v * v).mean(-1, keepdim=True) + EPS32) * w.double()

    core = F.silu(rms(mlp(mod.mlp_core), mod.core_norm.weight))
    gate = torch.sigmoid(rms(mlp(mod.mlp_gate), mod.gate_norm.weight))
    return core * gate


def _ffn64(mlp, x):
    L = mlp.layers
    return F.linear(F.silu(F.linear(x, L[0].weight.double())), L[3].weight.double())


def _softmax_sum(a, e, key, S):
    key = key.long()
    mx = torch.full((S, a.shape[1]), float("-inf"), dtype=a.dtype).scatter_reduce(
        0, key[:, None].expand_as(a), a, "amax", include_self=False)
    ex = (a - mx[key]).exp()
    den = torch.zeros(S, a.shape[1], dtype=a.dtype).index_add(0, key, ex)
    return torch.zeros(S, a.shape[1], dtype=a.dtype).index_add(0, key, ex / den[key] * e)


def _graph(A, E, N, seed):
    from matris_amd.model import ops
    g = torch.Generator().manual_seed(seed)
    tgt = torch.sort(torch.randint(0, E, (A,), generator=g))[0].to(torch.int32)
    src = torch.randint(0, E, (A,), generator=g).to(torch.int32)
    atom = torch.randint(0, N, (A,), generator=g).to(torch.int32)
    lg = {"grp_tgt": ops.Grouping.build(tgt.to(DEV), E, sorted_rows=True),
          "grp_src": ops.Grouping.build(src.to(DEV), E),
          "grp_atom": ops.Grouping.build(atom.to(DEV), N)}
    return lg, tgt.long(), src.long(), atom.long()


def _randomize(mod, seed):
    torch.manual_seed(seed)
    with torch.no_grad():
        for name, p in mod.named_parameters():
            if "res_weight" in name or "norm" in name:
                p.uniform_(0.5, 1.5)


@pytest.mark.parametrize("recompute", [False, True])
@pytest.mark.parametrize("A,E", [(3000, 400), (257, 64), (1, 1)])
def test_line_attention_vs_fp64(A, E, recompute):
    from matris_amd.model import fused
    from matris_amd.model.model import Graph_Attention_Layer
    torch.manual_seed(A)
    layer = Graph_Attention_Layer(128, 128, 128, norm_type="rms")
    _randomize(layer, A + 1)
    lg, tgt, src, _ = _graph(A, E, 5, A + 2)
    bond, tb = torch.randn(E, 128), torch.randn(A, 128)
    g_b, g_t = torch.randn(E, 128), torch.randn(A, 128)
    # fp64 reference
    b64, t64 = bond.double().requires_grad_(True), tb.double().requires_grad_(True)
    e = _gmlp64(layer.edge_nonlinear_update, torch.cat([t64, b64[tgt], b64[src]], 1))
    a_s = t64 @ layer.source_weight_linear.weight.double().t()
    a_t = t64 @ layer.target_weight_linear.weight.double().t()
    y_t, y_s = _softmax_sum(a_t, e, tgt, E), _softmax_sum(a_s, e, src, E)
    n = _gmlp64(layer.node_nonlinear_update, torch.cat([b64, y_t, y_s], 1))
    bn_r = n + layer.node_res_weight.double() * b64
    tn_r = e + layer.edge_res_weight.double() * t64
    ((bn_r * g_b.double()).sum() + (tn_r * g_t.double()).sum()).backward()
    # device
    layer = layer.to(DEV)
    assert fused.line_attention_fusable(layer)
    bd, td = bond.to(DEV).requires_grad_(True), tb.to(DEV).requires_grad_(True)
    bn, tn = fused.line_attention(layer, bd, td, lg, recompute)
    assert _rel(bn, bn_r) < 1e-5 and _rel(tn, tn_r) < 1e-5
    torch.autograd.backward([bn, tn], [g_b.to(DEV), g_t.to(DEV)])
    assert _rel(bd.grad, b64.grad) < 1e-5
    assert _rel(td.grad, t64.grad) < 1e-5


@pytest.mark.parametrize("recompute", [False, True])
@pytest.mark.parametrize("A,E,N", [(3000, 400, 60), (300, 64, 7)])
def test_line_refinement_vs_fp64(A, E, N, recompute):
    from matris_amd.model import fused
    from matris_amd.model.model import Refinement
    torch.manual_seed(A + N)
    layer = Refinement(128, 128, 128, 7, norm_type="rms", graph_type="line graph", atom_feat_dim=128)
    _randomize(layer, A + 3)
    lg, tgt, src, atom_l = _graph(A, E, N, A + 4)
    tb, atom, bond = torch.randn(A, 128), torch.randn(N, 128), torch.randn(E, 128)
    basis = torch.rand(E, 7) + 0.1  # the smooth weights the learnable envelope maps to env
    g_b, g_t = torch.randn(E, 128), torch.randn(A, 128)
    leaves = [x.double().requires_grad_(True) for x in (tb, atom, bond, basis)]
    t64, a64, b64, basis64 = leaves
    env64 = basis64 @ layer.learnable_envelope.weight.double().t()
    h = _gmlp64(layer.edge_nonlinear_update, torch.cat([t64, a64[atom_l], b64[tgt], b64[src]], 1))
    hw = h * (env64[src] * env64[tgt])
    agg = torch.zeros(E, 128, dtype=torch.float64).index_add(0, tgt, hw)
    bn_r = _ffn64(layer.node_FFN, agg) + layer.node_res_weight.double() * b64
    tn_r = _ffn64(layer.edge_FFN, h) + layer.edge_res_weight.double() * t64
    ((bn_r * g_b.double()).sum() + (tn_r * g_t.double()).sum()).backward()
    layer = layer.to(DEV)
    assert fused.line_refinement_fusable(layer)
    dev_leaves = [x.to(DEV).requires_grad_(True) for x in (tb, atom, bond, basis)]
    bn, tn = fused.line_refinement(layer, *dev_leaves, lg, recompute)
    assert _rel(bn, bn_r) < 1e-5 and _rel(tn, tn_r) < 1e-5
    torch.autograd.backward([bn, tn], [g_b.to(DEV), g_t.to(DEV)])
    for d, r in zip(dev_leaves, leaves):
        assert _rel(d.grad, r.grad) < 1e-5


def test_line_layers_unused_output_gradient():
    """An output whose gradient is None (e.g. the last block's three-body features)."""
    from matris_amd.model import fused
    from matris_amd.model.model import Refinement
    torch.manual_seed(0)
    layer = Refinement(128, 128, 128, 7, norm_type="rms", graph_type="line graph").to(DEV)
    lg, _, _, _ = _graph(500, 80, 9, 9)
    xs = [torch.randn(n, 128, device=DEV).requires_grad_(True) for n in (500, 9, 80)]
    basis = (torch.rand(80, 7, device=DEV) + 0.1).requires_grad_(True)
    bn, _ = fused.line_refinement(layer, *xs, basis, lg)
    bn.sum().backward()
    assert all(torch.isfinite(x.grad).all() for x in xs) and torch.isfinite(basis.grad).all()


def _atom_graph(N, E_u, seed):
    """A random directed atom graph: every bond u appears twice (d2u), with sorted targets."""
    from matris_amd.model import ops
    g = torch.Generator().manual_seed(seed)
    a = torch.randint(0, N, (E_u,), generator=g)
    b = (a + torch.randint(1, N, (E_u,), generator=g)) % N
    tgt = torch.cat([a, b])
    src = torch.cat([b, a])
    d2u = torch.cat([torch.arange(E_u), torch.arange(E_u)])
    order = torch.sort(tgt, stable=True)[1]
    tgt, src, d2u = tgt[order], src[order], d2u[order]
    ag = {"grp_tgt": ops.Grouping.build(tgt.to(torch.int32).to(DEV), N, sorted_rows=True),
          "grp_src": ops.Grouping.build(src.to(torch.int32).to(DEV), N)}
    gd2u = ops.Grouping.build(d2u.to(torch.int32).to(DEV), E_u)
    return ag, gd2u, tgt, src, d2u


@pytest.mark.parametrize("N,E_u", [(60, 700), (7, 9)])
def test_atom_attention_vs_fp64(N, E_u):
    from matris_amd.model import fused
    from matris_amd.model.model import Graph_Attention_Layer
    torch.manual_seed(N)
    layer = Graph_Attention_Layer(128, 128, 128, norm_type="rms")
    _randomize(layer, N + 5)
    ag, gd2u, tgt, src, d2u = _atom_graph(N, E_u, N + 6)
    atom, bond = torch.randn(N, 128), torch.randn(E_u, 128)
    g_a, g_b = torch.randn(N, 128), torch.randn(E_u, 128)
    a64, b64 = atom.double().requires_grad_(True), bond.double().requires_grad_(True)
    e = _gmlp64(layer.edge_nonlinear_update, torch.cat([b64[d2u], a64[tgt], a64[src]], 1))
    a_s = b64 @ layer.source_weight_linear.weight.double().t()
    a_t = b64 @ layer.target_weight_linear.weight.double().t()
    y_t, y_s = _softmax_sum(a_t[d2u], e, tgt, N), _softmax_sum(a_s[d2u], e, src, N)
    n = _gmlp64(layer.node_nonlinear_update, torch.cat([a64, y_t, y_s], 1))
    an_r = n + layer.node_res_weight.double() * a64
    bn_r = 0.5 * torch.zeros(E_u, 128, dtype=torch.float64).index_add(0, d2u, e) + layer.edge_res_weight.double() * b64
    ((an_r * g_a.double()).sum() + (bn_r * g_b.double()).sum()).backward()
    layer = layer.to(DEV)
    assert fused.atom_attention_fusable(layer)
    ad, bd = atom.to(DEV).requires_grad_(True), bond.to(DEV).requires_grad_(True)
    an, bn = fused.atom_attention(layer, ad, bd, ag, gd2u)
    assert _rel(an, an_r) < 1e-5 and _rel(bn, bn_r) < 1e-5
    torch.autograd.backward([an, bn], [g_a.to(DEV), g_b.to(DEV)])
    assert _rel(ad.grad, a64.grad) < 1e-5
    assert _rel(bd.grad, b64.grad) < 1e-5


@pytest.mark.parametrize("smoothed", [False, True])
def test_atom_refinement_vs_fp64(smoothed):
    from matris_amd.model import fused
    from matris_amd.model.model import Refinement
    N, E_u = 50, 600
    torch.manual_seed(E_u)
    layer = Refinement(128, 128, 128, 7, norm_type="rms", graph_type="atom graph",
                       use_smoothed_for_delta_edge=smoothed)
    _randomize(layer, 3)
    ag, gd2u, tgt, src, d2u = _atom_graph(N, E_u, 4)
    atom, bond, basis = torch.randn(N, 128), torch.randn(E_u, 128), torch.rand(E_u, 7) + 0.1
    g_a, g_b = torch.randn(N, 128), torch.randn(E_u, 128)
    leaves = [x.double().requires_grad_(True) for x in (atom, bond, basis)]
    a64, b64, basis64 = leaves
    env64 = basis64 @ layer.learnable_envelope.weight.double().t()
    h = _gmlp64(layer.edge_nonlinear_update, torch.cat([b64[d2u], a64[tgt], a64[src]], 1))
    hw = h * env64[d2u]
    agg = torch.zeros(N, 128, dtype=torch.float64).index_add(0, tgt, hw)
    an_r = _ffn64(layer.node_FFN, agg) + layer.node_res_weight.double() * a64
    de = _ffn64(layer.edge_FFN, hw if smoothed else h)
    bn_r = 0.5 * torch.zeros(E_u, 128, dtype=torch.float64).index_add(0, d2u, de) + layer.edge_res_weight.double() * b64
    ((an_r * g_a.double()).sum() + (bn_r * g_b.double()).sum()).backward()
    layer = layer.to(DEV)
    assert fused.atom_refinement_fusable(layer)
    dev_leaves = [x.to(DEV).requires_grad_(True) for x in (atom, bond, basis)]
    an, bn = fused.atom_refinement(layer, *dev_leaves, ag, gd2u)
    assert _rel(an, an_r) < 1e-5 and _rel(bn, bn_r) < 1e-5
    torch.autograd.backward([an, bn], [g_a.to(DEV), g_b.to(DEV)])
    for d, r in zip(dev_leaves, leaves):
        assert _rel(d.grad, r.grad) < 1e-5
