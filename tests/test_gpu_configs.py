"""The C2 and C5 configurations at their full sizes on the GPU.

C2 (4096-atom random packing, seed 1; A = 1,881,708 angles): the line-attention core
(Dimwise_softmax by target and by source, alpha * e', both segment sums; functions.py:97-160,
interaction_block.py:113-134) forward and input gradients, and the angle -> bond segment
sums, against an fp64 torch restatement of the reference ops run on the device
(scatter_reduce amax, exp, index_add_ in float64), on the bench's inputs (N(0,1), seed 1,
in the order alpha_s, alpha_t, e').  Bar: 1e-5 of the largest magnitude (the fp32
kernels' rounding; the fp64 reference is exact to ~1e-15).  The whole C2 efsm evaluation
too, by invariants (forces summing to zero, symmetric stress, rotation equivariance with
the index arrays held) and the default arithmetic against plain fp32 MFMA products.

C5 (32,000-atom a-SiO2, seed 4; A ~ 9.0 M): one efs evaluation with the default memory
mode (the leading blocks checkpointed, the trailing ones keeping their activations),
checked by what holds at any size:
  * every output finite; sum of forces 0 (translation invariance) to fp32 rounding;
    stress symmetric;
  * the auto split is bitwise equal to every block checkpointed (the kernels are
    deterministic, so a recomputed block reproduces its forward exactly);
  * the default f16x3 arithmetic agrees with plain fp32 MFMA products (MODE 0) within
    the north-star tolerances (energy 1e-5 relative, forces 1e-4 eV/A, stress 1e-4
    relative to the largest component).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
D = 128


def _rel(a, b):
    return ((a.double() - b.double()).abs().max() / b.double().abs().max().clamp_min(1e-30)).item()


@pytest.fixture(scope="module")
def c2_graph():
    from matris_amd import workloads as W
    from matris_amd.graph.converter import GraphConverter
    cr = W.c2_rsa4096()
    g = GraphConverter(device=DEV).from_arrays(cr.frac, cr.lattice, cr.z)
    print(f"C2: A={len(g.line_graph)} U={len(g.undirected2directed)}", flush=True)
    return g


def _softmax_sum64(a, e, key, S):
    """Dimwise_softmax by `key` then the segment sum of alpha * e, in fp64 on the device."""
    k = key.long()[:, None].expand_as(a)
    mx = torch.full((S, D), float("-inf"), dtype=a.dtype, device=a.device).scatter_reduce(
        0, k, a, "amax", include_self=False)
    ex = (a - mx[key.long()]).exp()
    den = torch.zeros(S, D, dtype=a.dtype, device=a.device).index_add(0, key.long(), ex)
    return torch.zeros(S, D, dtype=a.dtype, device=a.device).index_add(0, key.long(), ex / den[key.long()] * e)


def test_c2_line_attention_full_size_vs_fp64(c2_graph):
    from matris_amd.model import ops
    lg = c2_graph.line_graph
    A, U = int(lg.shape[0]), int(c2_graph.undirected2directed.shape[0])
    assert A > 1_800_000
    tkey, skey = lg[:, 1].contiguous(), lg[:, 3].contiguous()
    tgt = ops.Grouping.build(tkey, U, sorted_rows=True)
    src = ops.Grouping.build(skey, U)
    gen = torch.Generator().manual_seed(1)
    a_s, a_t, e = (torch.randn(A, D, generator=gen).to(DEV) for _ in range(3))
    g_yt, g_ys = (torch.randn(U, D, generator=gen).to(DEV) for _ in range(2))
    at, as_, ed = (t.clone().requires_grad_(True) for t in (a_t, a_s, e))
    y_t, y_s = ops.seg_attention(at, as_, ed, tgt, src, None)
    torch.autograd.backward([y_t, y_s], [g_yt, g_ys])
    at64, as64, e64 = (t.double().requires_grad_(True) for t in (a_t, a_s, e))
    yt64 = _softmax_sum64(at64, e64, tkey, U)
    ys64 = _softmax_sum64(as64, e64, skey, U)
    torch.autograd.backward([yt64, ys64], [g_yt.double(), g_ys.double()])
    errs = dict(yt=_rel(y_t, yt64), ys=_rel(y_s, ys64), g_at=_rel(at.grad, at64.grad),
                g_as=_rel(as_.grad, as64.grad), g_e=_rel(ed.grad, e64.grad))
    print("C2 attention rel errors:", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    assert all(v < 1e-5 for v in errs.values()), errs


def test_c2_segment_sums_full_size_vs_fp64(c2_graph):
    """Angle -> bond sums by target (rows ascending, no permutation) and by source (through
    the stable CSR permutation), the reference's aggregate / index_add_."""
    from matris_amd.model import ops
    lg = c2_graph.line_graph
    A, U = int(lg.shape[0]), int(c2_graph.undirected2directed.shape[0])
    gen = torch.Generator().manual_seed(2)
    x = torch.randn(A, D, generator=gen).to(DEV)
    for col, sorted_rows in ((1, True), (3, False)):
        key = lg[:, col].contiguous()
        grp = ops.Grouping.build(key, U, sorted_rows=sorted_rows)
        out = torch.empty(U, D, device=DEV)
        ops.seg_sum_raw(x, grp, out=out)
        ref = torch.zeros(U, D, dtype=torch.float64, device=DEV).index_add(0, key.long(), x.double())
        err = _rel(out, ref)
        print(f"C2 seg_sum col {col}: rel {err:.2e}", flush=True)
        assert err < 1e-5


def _efs(model, g):
    out = model([g], task="efs")
    return dict(e=out["e"].detach().double().cpu().numpy(), f=out["f"][0].detach().double().cpu().numpy(),
                s=out["s"][0].detach().double().cpu().numpy())


def test_c5_efs_32k_auto_split_invariants_and_arithmetic():
    from matris_amd import workloads as W
    from matris_amd.config import MATRIS_10M
    from matris_amd.model import MatRIS, fused, ops
    torch.manual_seed(0)
    model = MatRIS(**MATRIS_10M).to(DEV).eval()
    g = model.graph_converter(W.c5_sio2_32k())
    A, E = int(g.line_graph.shape[0]), int(g.atom_graph.shape[0])
    n_ckpt = fused.blocks_to_checkpoint(A, E, len(model.interaction_block), torch.device(DEV))
    print(f"C5: N=32000 E={E} A={A} auto checkpoint {n_ckpt} of 10", flush=True)
    assert A > 8_500_000 and 0 < n_ckpt < 10  # a mixed split
    auto = _efs(model, g)
    for k, v in auto.items():
        assert np.all(np.isfinite(v)), k
    f = auto["f"]
    assert np.abs(f.sum(0)).max() <= 1e-5 * np.abs(f).sum(0).max()
    s = auto["s"]
    assert np.abs(s - s.T).max() <= 1e-6 * np.abs(s).max()
    print(f"C5: e={auto['e'][0]:.6e} |f|max={np.abs(f).max():.3e} s={np.diag(s)}", flush=True)

    model.block_checkpoint = True
    full = _efs(model, g)
    for k in auto:
        assert np.array_equal(auto[k], full[k]), k
    model.block_checkpoint = None

    with ops.mma_precision("fp32"):
        ref = _efs(model, g)
    e_rel = abs(auto["e"][0] - ref["e"][0]) / abs(ref["e"][0])
    f_abs = np.abs(auto["f"] - ref["f"]).max()
    s_rel = np.abs(auto["s"] - ref["s"]).max() / np.abs(ref["s"]).max()
    print(f"C5 f16x3 vs fp32 MFMA: e_rel={e_rel:.2e} f_abs={f_abs:.2e} s_rel={s_rel:.2e}", flush=True)
    assert e_rel <= 1e-5 and f_abs <= 1e-4 and s_rel <= 1e-4


def test_c2_efsm_full_size_invariants_and_arithmetic(c2_graph):
    """The whole efsm evaluation at C2's full size (4,096 atoms, 1.88 M angles), checked by
    what holds at any size: forces summing to zero, symmetric stress, the default f16x3
    arithmetic against plain fp32 MFMA products within the north-star tolerances, and
    rotation equivariance (the lattice rotated with the fractional coordinates and every
    index array unchanged: e the same, forces and stress rotated)."""
    from matris_amd.config import MATRIS_10M
    from matris_amd.graph import RadiusGraph
    from matris_amd.model import MatRIS, ops
    torch.manual_seed(0)
    model = MatRIS(**MATRIS_10M).to(DEV).eval()
    g = c2_graph
    out = model([g], task="efsm")
    e = out["e"].detach().double().cpu().numpy()
    f = out["f"][0].detach().double().cpu().numpy()
    s = out["s"][0].detach().double().cpu().numpy()
    m = out["m"][0].detach().double().cpu().numpy()
    for k, v in (("e", e), ("f", f), ("s", s), ("m", m)):
        assert np.all(np.isfinite(v)), k
    assert np.abs(f.sum(0)).max() <= 1e-5 * np.abs(f).sum(0).max()
    assert np.abs(s - s.T).max() <= 1e-6 * np.abs(s).max()

    with ops.mma_precision("fp32"):
        ref = _efs(model, g)
    e_rel = abs(e[0] - ref["e"][0]) / abs(ref["e"][0])
    f_abs = np.abs(f - ref["f"]).max()
    s_rel = np.abs(s - ref["s"]).max() / np.abs(ref["s"]).max()
    print(f"C2 f16x3 vs fp32 MFMA: e_rel={e_rel:.2e} f_abs={f_abs:.2e} s_rel={s_rel:.2e}", flush=True)
    assert e_rel <= 1e-5 and f_abs <= 1e-4 and s_rel <= 1e-4

    th, ph = 0.6, 0.35
    rz = np.array([[np.cos(th), -np.sin(th), 0], [np.sin(th), np.cos(th), 0], [0, 0, 1]])
    rx = np.array([[1, 0, 0], [0, np.cos(ph), -np.sin(ph)], [0, np.sin(ph), np.cos(ph)]])
    R = rz @ rx
    lat = g.lattice.detach().double().cpu().numpy()
    g_rot = RadiusGraph(graph_id=None, mp_id=None, composition=None, atomic_number=g.atomic_number,
                        atom_frac_coord=g.atom_frac_coord,
                        lattice=torch.tensor(lat @ R.T, dtype=torch.float32, device=DEV),
                        neighbor_image=g.neighbor_image, atom_graph=g.atom_graph,
                        atom_graph_cutoff=g.atom_graph_cutoff, line_graph=g.line_graph,
                        line_graph_cutoff=g.line_graph_cutoff, directed2undirected=g.directed2undirected,
                        undirected2directed=g.undirected2directed)
    rot = _efs(model, g_rot)
    e_rot = abs(rot["e"][0] - e[0]) / abs(e[0])
    f_rot = np.abs(rot["f"] - f @ R.T).max()
    s_rot = np.abs(rot["s"] - R @ s @ R.T).max() / np.abs(s).max()
    print(f"C2 rotated: e_rel={e_rot:.2e} f_abs={f_rot:.2e} s_rel={s_rot:.2e}", flush=True)
    assert e_rot <= 1e-5 and f_rot <= 1e-4 and s_rot <= 1e-4
