"""The torch op library (matris_amd.torch_ops) on the GPU.

* matris_op::fuse_silu_bwd / fuse_silu_grad_bwd against an fp64 restatement of the
  reference's arithmetic (op/fused_silu_op.py:5-28) -- odd sizes and misaligned views
  included -- and fused_silu's first and second derivatives against torch's SiLU in fp64;
* torch.library.opcheck (schema, fake tensors, autograd registration) on the ops;
* every matris_hip op bit-identical with the internal path it wraps (ops.*_raw with the
  same packed weights), the segment sums against fp64 index_add_, the radius graph
  against the CPU oracle;
* the ops inside a HIP graph: captured once, replayed with new inputs copied in and
  eager work in between, every replay equal to the eager result.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def T():
    import matris_amd.torch_ops as mod
    return mod


def _silu_d(x):
    s = torch.sigmoid(x)
    return s * (1 + x * (1 - s)), s * (1 - s) * (2 + x * (1 - 2 * s))


def _within(got, ref, scale, ref32):
    """|got - ref| <= 4 ulp-scale bound of the fp32 formula: 2e-6 * (the size of its
    largest intermediate, `scale`), elementwise, and no larger than 4x the error of the
    reference's formula evaluated in fp32 by torch (ref32) plus that bound's floor."""
    err = (got.double() - ref).abs()
    assert bool((err <= 2e-6 * scale + 1e-30).all()), float((err / (scale + 1e-30)).max())
    assert float(err.max()) <= 4 * float((ref32.double() - ref).abs().max()) + 1e-7


@pytest.mark.parametrize("n,offset", [(1, 0), (7, 0), (4096, 0), (1000003, 0), (4099, 1), (64, 3)])
def test_silu_ops_vs_fp64(T, n, offset):
    """Against fp64 (the reference's arithmetic, fused_silu_op.py:5-28): the first
    derivative to fp32 rounding of its result; the second one, whose factor
    2 + x (1 - 2 sigmoid(x)) cancels near |x| = 2.4, to fp32 rounding of its largest
    intermediate, as the reference's own fp32 formula."""
    g = torch.Generator(device=DEV).manual_seed(n)
    base = [torch.randn(n + offset, device=DEV, generator=g) * s for s in (1.0, 4.0, 1.0)]
    dgrad, x, go = (b[offset:] for b in base)  # offset > 0: pointers not 16-byte aligned
    x64 = x.double()
    d1, d2 = _silu_d(x64)
    s32 = 1 / (1 + torch.exp(-x))
    d1_32 = s32 * (1 + x * (1 - s32))
    d2_32 = s32 * (1 - s32) * (2 + x * (1 - 2 * s32))
    out = torch.ops.matris_op.fuse_silu_bwd(dgrad, x)
    scale1 = dgrad.double().abs() * (1 + x64.abs())
    _within(out, dgrad.double() * d1, scale1, dgrad * d1_32)
    ggo, gx = torch.ops.matris_op.fuse_silu_grad_bwd(dgrad, go, x)
    _within(ggo, dgrad.double() * d1, scale1, dgrad * d1_32)
    scale2 = (dgrad.double() * go.double()).abs() * (2 + x64.abs())
    _within(gx, dgrad.double() * go.double() * d2, scale2, dgrad * go * d2_32)


def test_fused_silu_first_and_second_derivatives(T):
    torch.manual_seed(0)
    x = (torch.randn(1000, 128, device=DEV) * 3).requires_grad_(True)
    g, h = torch.randn(1000, 128, device=DEV), torch.randn(1000, 128, device=DEV)
    y = T.fused_silu(x)
    (gx,) = torch.autograd.grad(y, x, g, create_graph=True)
    (gxx,) = torch.autograd.grad((gx * h).sum(), x)
    x64 = x.detach().double().requires_grad_(True)
    y64 = torch.nn.functional.silu(x64)
    (gx64,) = torch.autograd.grad(y64, x64, g.double(), create_graph=True)
    (gxx64,) = torch.autograd.grad((gx64 * h.double()).sum(), x64)
    assert torch.equal(y, torch.nn.functional.silu(x.detach()))
    # fp32 rounding of the formulas' largest intermediates (see test_silu_ops_vs_fp64)
    xa = x.detach().double().abs()
    err1 = (gx.double() - gx64).abs()
    assert bool((err1 <= 2e-6 * g.double().abs() * (1 + xa) + 1e-30).all())
    err2 = (gxx.double() - gxx64).abs()
    assert bool((err2 <= 2e-6 * (g.double() * h.double()).abs() * (2 + xa) + 1e-30).all())


def _csr(key, n_seg):
    return torch.ops.matris_hip.csr_build(key, n_seg)


def test_opcheck(T):
    from torch.library import opcheck
    torch.manual_seed(1)
    R, S = 300, 40
    x = torch.randn(R, 128, device=DEV)
    key = torch.randint(0, S, (R,), device=DEV, dtype=torch.int32)
    rowptr, perm = _csr(key, S)
    utils = ("test_schema", "test_autograd_registration", "test_faketensor")
    opcheck(torch.ops.matris_op.fuse_silu_bwd, (x, x), test_utils=utils)
    opcheck(torch.ops.matris_op.fuse_silu_grad_bwd, (x, x, x), test_utils=utils)
    opcheck(torch.ops.matris_hip.seg_sum, (x.clone().requires_grad_(True), key, rowptr, perm), test_utils=utils)
    src = torch.randn(S, 128, device=DEV, requires_grad=True)
    opcheck(torch.ops.matris_hip.gather, (src, key, rowptr, perm), test_utils=utils)
    w0, w1 = torch.randn(128, 128, device=DEV) / 11, torch.randn(128, 128, device=DEV) / 11
    opcheck(torch.ops.matris_hip.pair_fwd, (x, w0, w1), test_utils=("test_schema", "test_faketensor"))
    opcheck(torch.ops.matris_hip.ffn_fwd, (x, w0, w1), test_utils=("test_schema", "test_faketensor"))


def test_segment_ops_and_autograd(T):
    torch.manual_seed(2)
    R, S = 5000, 700
    x = torch.randn(R, 128, device=DEV, requires_grad=True)
    key = torch.randint(0, S, (R,), device=DEV, dtype=torch.int32)
    rowptr, perm = _csr(key, S)
    y = torch.ops.matris_hip.seg_sum(x, key, rowptr, perm)
    ref = torch.zeros(S, 128, dtype=torch.float64, device=DEV).index_add_(0, key.long(), x.detach().double())
    torch.testing.assert_close(y.double(), ref, rtol=0, atol=1e-5 * ref.abs().max().item())
    g = torch.randn(S, 128, device=DEV)
    (gx,) = torch.autograd.grad(y, x, g)
    assert torch.equal(gx, g[key.long()])
    src = torch.randn(S, 128, device=DEV, requires_grad=True)
    z = torch.ops.matris_hip.gather(src, key, rowptr, perm)
    assert torch.equal(z, src.detach()[key.long()])
    gz = torch.randn(R, 128, device=DEV)
    (gsrc,) = torch.autograd.grad(z, src, gz)
    ref = torch.zeros(S, 128, dtype=torch.float64, device=DEV).index_add_(0, key.long(), gz.double())
    torch.testing.assert_close(gsrc.double(), ref, rtol=0, atol=1e-5 * ref.abs().max().item())


def _gmlp_weights(K, seed):
    from matris_amd.model.model import GatedMLP
    torch.manual_seed(seed)
    mod = GatedMLP(K, 128, 128, norm_type="rms").to(DEV)
    c, gt = mod.mlp_core.layers, mod.mlp_gate.layers
    w = dict(w1=torch.cat([c[0].weight, gt[0].weight]).detach().contiguous(),
             b1=torch.cat([c[0].bias, gt[0].bias]).detach().contiguous(),
             w2=torch.cat([c[3].weight, gt[3].weight]).detach().contiguous(),
             b2=torch.cat([c[3].bias, gt[3].bias]).detach().contiguous(),
             norm_c=mod.core_norm.weight.detach().contiguous(), norm_g=mod.gate_norm.weight.detach().contiguous(),
             eps=float(mod.core_norm.eps if mod.core_norm.eps is not None else torch.finfo(torch.float32).eps))
    return mod, w


@pytest.mark.parametrize("M", [1000, 70001])
def test_gated_mlp_ffn_pair_ops_match_internal_paths(T, M):
    from matris_amd.model import ops
    mod, w = _gmlp_weights(384, M)
    args = (w["w1"], w["b1"], w["w2"], w["b2"], w["norm_c"], w["norm_g"], w["eps"])
    bond = torch.randn(M // 8 + 1, 128, device=DEV)
    tb = torch.randn(M, 128, device=DEV)
    it = torch.randint(0, bond.shape[0], (M,), device=DEV, dtype=torch.int32)
    out, p, z = torch.ops.matris_hip.gated_mlp_fwd([tb, bond, bond], [None, it, it.flip(0).contiguous()], M, *args)
    mode = ops._MMA["mode"]
    pack = ops.GmlpPack().get(mod)
    ro, rp, rz, _ = ops.gmlp_fwd_raw(pack, [tb, bond, bond], [None, it, it.flip(0).contiguous()], M, mode)
    assert torch.equal(out, ro) and torch.equal(p, rp) and torch.equal(z, rz)
    g = torch.randn(M, 128, device=DEV)
    assert torch.equal(torch.ops.matris_hip.gated_mlp_bwd(g, p, z, *args), ops.gmlp_bwd_raw(pack, g, p, z, 384, mode))
    w0, w1 = torch.randn(128, 128, device=DEV) / 11, torch.randn(128, 128, device=DEV) / 11
    wp = ops._WeightPack().get(w0, w1)
    o, q = torch.ops.matris_hip.ffn_fwd(tb, w0, w1)
    ro, rq = ops.ffn_fwd_raw(wp, tb, mode)
    assert torch.equal(o, ro) and torch.equal(q, rq)
    assert torch.equal(torch.ops.matris_hip.ffn_bwd(g, q, w0, w1), ops.ffn_bwd_raw(wp, g, q, mode))
    a, b = torch.ops.matris_hip.pair_fwd(tb, w0, w1)
    ra, rb = ops.pair_fwd_raw(wp, tb, mode)
    assert torch.equal(a, ra) and torch.equal(b, rb)
    assert torch.equal(torch.ops.matris_hip.pair_bwd(g, a, w0, w1), ops.pair_bwd_raw(wp, g, a, mode))


def test_attention_and_graph_ops(T):
    from matris_amd import workloads as W
    from matris_amd.graph import GraphConverter
    from matris_amd.model import ops
    from oracle import graph_ref
    cr = W.c3_cu864()
    frac = torch.tensor(cr.frac, device=DEV)
    c, nb, im, d, rp = torch.ops.matris_hip.radius_graph(frac, torch.tensor(cr.lattice), 6.0)
    oc, onb, oim, od = graph_ref.neighbor_list(cr.frac, cr.lattice, 6.0)
    assert np.array_equal(c.cpu().numpy(), oc) and np.array_equal(nb.cpu().numpy(), onb)
    assert np.array_equal(im.cpu().numpy().astype(np.int64), oim) and np.array_equal(d.cpu().numpy(), od)
    assert int(rp[-1]) == len(oc)
    g = GraphConverter(device=DEV)(cr)
    lg = g.line_graph.view(-1, 5)
    A, U = lg.shape[0], g.undirected2directed.shape[0]
    tk, sk = lg[:, 1].contiguous(), lg[:, 3].contiguous()
    trp, _ = _csr(tk, U)
    srp, sperm = _csr(sk, U)
    torch.manual_seed(3)
    at, as_, e = (torch.randn(A, 128, device=DEV) for _ in range(3))
    yt, ys, lt, ls = torch.ops.matris_hip.line_attn_fwd(at, as_, e, tk, trp, None, sk, srp, sperm)
    tgt, src = ops.Grouping(tk, trp, None, U), ops.Grouping(sk, srp, sperm, U)
    r = ops.attn_fwd_raw(at, as_, e, tgt, src, None)
    assert torch.equal(yt, r[0]) and torch.equal(ys, r[1])
    gyt, gys = torch.randn(U, 128, device=DEV), torch.randn(U, 128, device=DEV)
    got = torch.ops.matris_hip.line_attn_bwd(at, as_, e, yt, ys, lt, ls, gyt, gys, tk, sk, U)
    ref = ops.attn_bwd_raw(at, as_, e, r[0], r[1], r[2], r[3], gyt, gys, tgt, src, None)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)


def test_ops_in_a_hip_graph(T):
    """Capture gather -> segment sum -> line attention -> gated MLP -> projection pair once;
    replay with two input sets copied in turn into the static inputs, with eager work and a
    synchronisation between replays: every replay equals the eager run of its inputs."""
    torch.manual_seed(4)
    R, S = 6000, 800
    key = torch.sort(torch.randint(0, S, (R,), device=DEV, dtype=torch.int32)).values
    skey = torch.randint(0, S, (R,), device=DEV, dtype=torch.int32)
    trp, tperm = _csr(key, S)
    srp, sperm = _csr(skey, S)
    _, w = _gmlp_weights(384, 5)
    args = (w["w1"], w["b1"], w["w2"], w["b2"], w["norm_c"], w["norm_g"], w["eps"])
    w0, w1 = torch.randn(128, 128, device=DEV) / 11, torch.randn(128, 128, device=DEV) / 11
    sets = [(torch.randn(S, 128, device=DEV), torch.randn(R, 128, device=DEV)) for _ in range(2)]
    bond, tb = (t.clone() for t in sets[0])  # the static inputs

    def run():
        e = torch.ops.matris_hip.gather(bond, key, trp, tperm)
        agg = torch.ops.matris_hip.seg_sum(e, skey, srp, sperm)
        a_s, a_t = torch.ops.matris_hip.pair_fwd(tb, w0, w1)
        yt, ys, _, _ = torch.ops.matris_hip.line_attn_fwd(a_t, a_s, e, key, trp, None, skey, srp, sperm)
        out, _, _ = torch.ops.matris_hip.gated_mlp_fwd([tb, agg, yt], [None, skey, key], R, *args)
        return agg, ys, out

    eager = []
    for b, t in sets:
        bond.copy_(b)
        tb.copy_(t)
        eager.append([x.clone() for x in run()])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = run()
    for rep in range(4):
        b, t = sets[rep % 2]
        bond.copy_(b)
        tb.copy_(t)
        graph.replay()
        torch.cuda.synchronize()
        for got, ref in zip(static_out, eager[rep % 2]):
            assert torch.equal(got, ref), rep
        torch.ops.matris_hip.seg_sum(tb, skey, srp, sperm)  # eager work between replays
        torch.cuda.synchronize()
