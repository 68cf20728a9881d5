"""Kernel-level parity on the GPU: every floating-point kernel against a plain torch
fp64 restatement of the reference op on identical inputs; integer kernels bit-exact.

Reference ops restated here: aggregate / index_add_ (functions.py:129-160),
index_select, Dimwise_softmax + attention sums (functions.py:97-127,
interaction_block.py:113-134), GatedMLP with RMSNorm (functions.py:245-311), the
bias-free FFN MLP (functions.py:198-205) and the W_s / W_t projections
(interaction_block.py:33-38, 110-111).
"""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _ops():
    from matris_amd.model import ops
    return ops


def _keys(R, S, seed, empty_every=7):
    g = torch.Generator().manual_seed(seed)
    k = torch.randint(0, S, (R,), generator=g)
    k = torch.where(k % empty_every == 3, (k + 1) % S, k)  # leave some segments empty
    return k.to(torch.int32)


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


@pytest.mark.parametrize("R,S", [(1, 1), (37, 5), (5000, 800), (20000, 3)])
def test_csr_build_is_stable_argsort(R, S):
    ops = _ops()
    key = _keys(R, S, R + S).to(DEV)
    grp = ops.Grouping.build(key, S)
    ref_perm = torch.argsort(key.cpu().long(), stable=True).to(torch.int32)
    ref_ptr = torch.zeros(S + 1, dtype=torch.int64)
    ref_ptr[1:] = torch.cumsum(torch.bincount(key.cpu().long(), minlength=S), 0)
    assert torch.equal(grp.perm.cpu(), ref_perm)
    assert torch.equal(grp.rowptr.cpu().long(), ref_ptr)


@pytest.mark.parametrize("R,S", [(0, 5), (1, 1), (264384, 33698), (5000, 800), (7, 40)])
def test_csr_sorted_keys_rowptr_only(R, S):
    """Sorted keys (perm NULL): the one-pass row pointers equal the full build's, with
    empty leading, trailing and interior segments; a descent is flagged like an
    out-of-range key (status bit when deferred, an error when synchronous)."""
    ops = _ops()
    ops.status_take()
    key = torch.sort(_keys(R, S, R + 3))[0].to(DEV) if R else torch.zeros(0, dtype=torch.int32, device=DEV)
    a = ops.Grouping.build(key, S, sorted_rows=True, deferred=True)
    b = ops.Grouping.build(key, S)
    assert a.perm is None and torch.equal(a.rowptr, b.rowptr)
    assert ops.status_take() == 0
    if R > 1:
        bad = key.clone()
        bad[0] = S - 1  # a descent after the first row (keys stay in range)
        if bool((bad[1:] < bad[:-1]).any()):
            ops.Grouping.build(bad, S, sorted_rows=True, deferred=True)
            assert ops.status_take() == ops.STATUS_CSR_KEY
            with pytest.raises(RuntimeError):
                ops.Grouping.build(bad, S, sorted_rows=True)
    assert ops.status_take() == 0


@pytest.mark.parametrize("R,S,scale,acc", [(3000, 500, 1.0, False), (3000, 500, 0.5, True), (10, 40, 1.0, False)])
def test_seg_sum_matches_index_add(R, S, scale, acc):
    ops = _ops()
    torch.manual_seed(0)
    key = _keys(R, S, 1).to(DEV)
    grp = ops.Grouping.build(key, S)
    x = torch.randn(R, 384, device=DEV)
    base = torch.randn(S, 128, device=DEV)
    out = base.clone()
    ops.seg_sum_raw(x, grp, scale, ldx=384, col_off=128, out=out, accumulate=acc)
    ref = torch.zeros(S, 128, dtype=torch.float64).index_add_(0, key.cpu().long(), x[:, 128:256].double().cpu())
    ref = ref * scale + (base.double().cpu() if acc else 0)
    assert _rel(out, ref) < 2e-6


@pytest.mark.parametrize("R,S", [(37, 5), (5000, 800), (20000, 3), (3000, 100), (0, 4), (67396, 33698), (61, 59),
                                 (6400, 90)])
@pytest.mark.parametrize("acc", [False, True])
def test_seg_sum_two_groupings_one_pass(R, S, acc):
    """matris_seg_sum2: two groupings of different row sets into one output (the target-
    and source-side scatters): segments of at most 4 rows on average (four per wave, as
    the two directed copies of a bond), of more (a wave each) and long ones (a work-group
    each, R/S >= 32), against two fp64 index_add_ calls."""
    ops = _ops()
    torch.manual_seed(R + S)
    ka, kb = _keys(R, S, 2).to(DEV), _keys(R + 7, S, 3).to(DEV)
    ga, gb = ops.Grouping.build(ka, S), ops.Grouping.build(kb, S)
    x = torch.randn(max(R, 1), 384, device=DEV)[:R]
    xb = torch.randn(R + 7, 256, device=DEV)
    base = torch.randn(S, 128, device=DEV)
    out = base.clone()
    ops.seg_sum_raw(x, ga, 0.5, ldx=384, col_off=256, out=out, accumulate=acc, second=(xb, gb, 1.0, 256, 128))
    ref = torch.zeros(S, 128, dtype=torch.float64).index_add_(0, ka.cpu().long(), x[:, 256:].double().cpu()) * 0.5
    ref = ref.index_add_(0, kb.cpu().long(), xb[:, 128:].double().cpu())
    ref = ref + (base.double().cpu() if acc else 0)
    assert _rel(out, ref) < 2e-6
    with pytest.raises(ValueError):
        ops.seg_sum_raw(x, ga, second=(xb, ops.Grouping.build(kb, S + 1), 1.0, 256, 128))


@pytest.mark.parametrize("lengths,width", [([54, 0, 18, 1, 63, 200], 1), ([3000, 1, 0, 64, 65], 9),
                                           ([7, 129], 32), ([0, 0], 4), ([5000], 1)])
def test_seg_sum_narrow(lengths, width):
    """matris_seg_sum_narrow: per-segment sums of narrow rows (batched energies, per-graph
    strain / lattice gradients) against fp64 sums, empty segments included; two calls are
    bitwise equal (fixed order, no atomics)."""
    ops = _ops()
    torch.manual_seed(sum(lengths) + width)
    R = sum(lengths)
    x = torch.randn(max(R, 1), width, device=DEV)[:R]
    ptr = torch.tensor([0] + list(torch.cumsum(torch.tensor(lengths), 0)), dtype=torch.int32, device=DEV)
    out = ops.seg_sum_narrow_raw(x, ptr, len(lengths))
    x64 = x.double().cpu()
    ref = torch.stack([x64[int(a):int(b)].sum(0) for a, b in zip(ptr[:-1].cpu(), ptr[1:].cpu())])
    assert tuple(out.shape) == (len(lengths), width)
    assert (out.double().cpu() - ref).abs().max().item() <= 1e-5 * max(1.0, ref.abs().max().item())
    assert torch.equal(out, ops.seg_sum_narrow_raw(x, ptr, len(lengths)))


@pytest.mark.parametrize("N", [864, 1, 0, 300])
def test_frac_to_cart(N):
    """matris_frac_to_cart: positions frac @ lattice (processgraph.py:87) against the fp64
    product, and the zero strain written in the same launch."""
    ops = _ops()
    torch.manual_seed(N + 3)
    frac = torch.rand(N, 3, device=DEV)
    lat = (torch.eye(3) * 9.0 + torch.randn(3, 3)).to(DEV)
    cart, strain = ops.frac_to_cart(frac, lat, True)
    ref = frac.double().cpu() @ lat.double().cpu()
    assert tuple(cart.shape) == (N, 3) and tuple(strain.shape) == (1, 3, 3)
    if N:
        assert float((cart.double().cpu() - ref).abs().max()) < 4e-6
    assert torch.equal(strain.cpu(), torch.zeros(1, 3, 3))
    cart2, none = ops.frac_to_cart(frac, lat, False)
    assert none is None and torch.equal(cart2, cart)
    with pytest.raises(ValueError):
        ops.frac_to_cart(frac, lat[:2], True)


@pytest.mark.parametrize("sizes", [[24, 1, 64, 0, 8], [2162], [0, 0], [5] * 64])
def test_frac_to_cart_batch(sizes):
    """matris_frac_to_cart_batch: every atom's frac @ its own graph's lattice against the
    fp64 products, bitwise equal to matris_frac_to_cart graph by graph (the one-graph path),
    the zero strains of all graphs, and a graph index outside [0, G) reported in the status
    word with the atom's row left as it was."""
    ops = _ops()
    G, N = len(sizes), sum(sizes)
    torch.manual_seed(G * 7 + N)
    frac = torch.rand(N, 3, device=DEV)
    lat = (torch.eye(3) * 9.0 + torch.randn(G, 3, 3)).to(DEV)
    gidx = torch.repeat_interleave(torch.arange(G), torch.tensor(sizes)).to(torch.int32).to(DEV)
    ops.status_take()
    cart, strain = ops.frac_to_cart_batch(frac, lat, gidx, True)
    assert ops.status_take() == 0
    assert tuple(cart.shape) == (N, 3) and tuple(strain.shape) == (G, 3, 3)
    assert torch.equal(strain.cpu(), torch.zeros(G, 3, 3))
    ref = torch.bmm(frac.double().cpu().unsqueeze(1), lat.double().cpu()[gidx.long().cpu()]).squeeze(1)
    if N:
        assert float((cart.double().cpu() - ref).abs().max()) < 4e-6
    o = 0
    for g, n in enumerate(sizes):
        one, _ = ops.frac_to_cart(frac[o:o + n], lat[g], False)
        assert torch.equal(one, cart[o:o + n])
        o += n
    cart2, none = ops.frac_to_cart_batch(frac, lat, gidx, False)
    assert none is None and torch.equal(cart2, cart)
    if N:
        bad = gidx.clone()
        bad[N - 1] = G  # one past the last graph: no read, a status bit
        out = ops.frac_to_cart_batch(frac, lat, bad, False)[0]
        assert ops.status_take() == ops.STATUS_CSR_KEY
        assert torch.equal(out[:N - 1], cart[:N - 1])
    with pytest.raises(ValueError):
        ops.frac_to_cart_batch(frac, lat, gidx.long(), True)
    with pytest.raises(ValueError):
        ops.frac_to_cart_batch(frac, lat[:, :2], gidx, True)


@pytest.mark.parametrize("E,K", [(33698, 7), (1, 7), (0, 7), (513, 1), (777, 8), (100, 3)])
def test_env_linear(E, K):
    """matris_env_linear: the learnable envelope env = basis W^T (interaction_block.py:
    240-246, Linear(K, 128) without bias) against the fp64 product."""
    ops = _ops()
    torch.manual_seed(E + K)
    basis = torch.randn(E, K, device=DEV)
    w = torch.randn(128, K, device=DEV) / 3
    env = ops.env_linear_raw(basis, w.t().contiguous())
    assert tuple(env.shape) == (E, 128)
    if E:
        ref = basis.double().cpu() @ w.double().cpu().t()
        assert _rel(env, ref) < 1e-6
    with pytest.raises(ValueError):
        ops.env_linear_raw(basis, torch.randn(K, 64, device=DEV))


@pytest.mark.parametrize("R,E_u,K", [(67396, 33698, 7), (2, 1, 7), (0, 5, 7), (1000, 500, 8), (10, 5, 1)])
def test_seg_sum_mul_proj(R, E_u, K):
    """matris_seg_sum_mul_proj: the atom-graph envelope gradient sum_{d2u} h * g_agg[tgt]
    (two directed copies per bond) projected onto the envelope's basis, g_env W ([E_u, K]),
    against fp64 index_add_ followed by the fp64 product; the unprojected sums as a second
    check of the same rows."""
    ops = _ops()
    torch.manual_seed(R + K)
    d2u = torch.arange(R, dtype=torch.int32) // 2 if R else torch.zeros(0, dtype=torch.int32)
    d2u = torch.minimum(d2u, torch.tensor(E_u - 1, dtype=torch.int32))
    grp = ops.Grouping.build(d2u.to(DEV), E_u)
    h = torch.randn(max(R, 1), 128, device=DEV)[:R]
    T = 400
    g_agg = torch.randn(T, 128, device=DEV)
    tk = torch.randint(0, T, (R,), dtype=torch.int32, device=DEV)
    w = torch.randn(128, K, device=DEV) / 5
    g_basis = ops.seg_sum_mul_proj_raw(h, grp, g_agg, tk, w.t().contiguous())
    g_env = torch.zeros(E_u, 128, dtype=torch.float64).index_add_(
        0, d2u.long(), h.double().cpu() * g_agg.double().cpu()[tk.cpu().long()])
    ref = g_env @ w.double().cpu()
    assert tuple(g_basis.shape) == (E_u, K)
    assert _rel(g_basis, ref) < 2e-6
    plain = ops.seg_sum_mul_raw(h, grp, g_agg, tk)
    assert _rel(plain.double().cpu() @ w.double().cpu(), ref) < 2e-6
    # accumulate: added to an existing buffer (the blocks sharing one basis)
    base = torch.randn(E_u, K, device=DEV)
    acc = base.clone()
    assert ops.seg_sum_mul_proj_raw(h, grp, g_agg, tk, w.t().contiguous(), out=acc) is acc
    assert _rel(acc, base.double().cpu() + ref) < 2e-6


@pytest.mark.parametrize("A,E,K", [(264384, 33698, 7), (3000, 400, 7), (50, 9, 8)])
def test_env_agg_bwd_env_proj(A, E, K):
    """matris_env_agg_bwd_env_proj: the line Refinement's g_env (interaction_block.py:243-258)
    projected onto the envelope's basis in the same pass.  g_agg_env is bit-identical to the
    unprojected entry point's; g_basis equals its g_env times W to fp32 rounding (fp64
    product of the fp32 g_env)."""
    ops = _ops()
    torch.manual_seed(A + K)
    tkey = torch.sort(_keys(A, E, A + 1))[0].to(DEV)
    skey = _keys(A, E, A + 2).to(DEV)
    tgt = ops.Grouping.build(tkey, E, sorted_rows=True)
    src = ops.Grouping.build(skey, E)
    h = torch.randn(A, 128, device=DEV)
    env, g_agg, S = torch.rand(E, 128, device=DEV), torch.randn(E, 128, device=DEV), torch.randn(E, 128, device=DEV)
    w = torch.randn(128, K, device=DEV) / 5
    g_env, ge = ops.env_agg_bwd_env_raw(h, env, g_agg, S, tgt, src)
    g_basis, ge2 = ops.env_agg_bwd_env_raw(h, env, g_agg, S, tgt, src, proj_wt=w.t().contiguous())
    assert torch.equal(ge, ge2)
    assert tuple(g_basis.shape) == (E, K)
    assert _rel(g_basis, g_env.double().cpu() @ w.double().cpu()) < 2e-6
    # accumulate into an existing g_basis: that buffer plus the same projection, bitwise
    base = torch.randn(E, K, device=DEV)
    acc = base.clone()
    out, ge3 = ops.env_agg_bwd_env_raw(h, env, g_agg, S, tgt, src, proj_wt=w.t().contiguous(), g_basis=acc)
    assert out is acc and torch.equal(ge, ge3)
    assert torch.equal(acc, base + g_basis)


@pytest.mark.parametrize("R,S,T", [(67396, 864, 33698), (5000, 800, 300), (37, 5, 11), (0, 4, 3), (67396, 33698, 864),
                                   (9, 7, 5)])
@pytest.mark.parametrize("acc", [False, True])
def test_seg_sum_mul_and_gather_mul(R, S, T, acc):
    """matris_seg_sum_mul: segment sums of x[r] * mul[mul_idx[r]] (the atom-graph envelope
    weighting h * env[d2u] summed by target; 78 rows per segment in the first case, one
    work-group per segment) and matris_gather_mul: out (+)= a[ia] * b[ib], against fp64
    products followed by index_add_."""
    ops = _ops()
    torch.manual_seed(R + S)
    key = _keys(R, S, 4).to(DEV)
    grp = ops.Grouping.build(key, S)
    x = torch.randn(max(R, 1), 128, device=DEV)[:R]
    mul = torch.randn(T, 128, device=DEV)
    midx = torch.randint(0, T, (R,), dtype=torch.int32, device=DEV)
    base = torch.randn(S, 128, device=DEV)
    out = base.clone()
    ops.seg_sum_mul_raw(x, grp, mul, midx, out=out, accumulate=acc)
    prod = x.double().cpu() * mul.double().cpu()[midx.cpu().long()]
    ref = torch.zeros(S, 128, dtype=torch.float64).index_add_(0, key.cpu().long(), prod)
    ref = ref + (base.double().cpu() if acc else 0)
    assert _rel(out, ref) < 2e-6
    a = torch.randn(S, 128, device=DEV)
    o2 = torch.randn(R, 128, device=DEV)
    ref2 = a.double().cpu()[key.cpu().long()] * mul.double().cpu()[midx.cpu().long()]
    ref2 = ref2 + (o2.double().cpu() if acc else 0)
    ops.gather_mul_raw(a, key, mul, midx, out=o2, accumulate=acc)
    if R:
        assert _rel(o2, ref2) < 1e-6
    ident = ops.gather_mul_raw(x, None, x, None, out=torch.empty_like(x))
    assert torch.equal(ident, x * x)


@pytest.mark.parametrize("R,S", [(67396, 33698), (5000, 80)])
@pytest.mark.parametrize("acc", [False, True])
def test_seg_sum_residual_base(R, S, acc):
    """matris_seg_sum2 with base: out = 0.5 * (segment sums) + w * feat (the atom-graph
    layers' mean of the two directed copies plus the residual), against fp64."""
    ops = _ops()
    torch.manual_seed(R)
    key = _keys(R, S, 5).to(DEV)
    grp = ops.Grouping.build(key, S)
    x = torch.randn(R, 384, device=DEV)
    feat = torch.randn(S, 128, device=DEV)
    w = torch.rand(128, device=DEV)
    prior = torch.randn(S, 128, device=DEV)
    out = ops.seg_sum_raw(x, grp, 0.5, ldx=384, col_off=128, base=(feat, w), out=prior.clone(), accumulate=acc)
    ref = torch.zeros(S, 128, dtype=torch.float64).index_add_(0, key.cpu().long(), x[:, 128:256].double().cpu())
    ref = 0.5 * ref + w.double().cpu() * feat.double().cpu() + (prior.double().cpu() if acc else 0)
    assert _rel(out, ref) < 2e-6


def test_deferred_csr_build_flags_bad_keys():
    """matris_csr_build_deferred: valid keys give the same grouping as the synchronous
    build; a key outside [0, n_seg) is left out and sets STATUS_CSR_KEY (the synchronous
    build raises instead)."""
    ops = _ops()
    ops.status_take()
    key = _keys(5000, 300, 9).to(DEV)
    a, b = ops.Grouping.build(key, 300), ops.Grouping.build(key, 300, deferred=True)
    assert torch.equal(a.rowptr, b.rowptr) and torch.equal(a.perm, b.perm)
    assert ops.status_take() == 0
    bad = key.clone()
    bad[17] = 300
    g = ops.Grouping.build(bad, 300, deferred=True)
    assert ops.status_take() == ops.STATUS_CSR_KEY
    assert int(g.rowptr[-1]) == 4999  # the bad row is not placed
    with pytest.raises(RuntimeError):
        ops.Grouping.build(bad, 300)
    assert ops.status_take() == 0


def test_gather_exact():
    ops = _ops()
    src = torch.randn(100, 128, device=DEV)
    idx = torch.randint(0, 100, (1000,), device=DEV, dtype=torch.int32)
    assert torch.equal(ops.gather_raw(src, idx), src[idx.long()])


def _attn_ref(at, as_, e, tkey, skey, S):
    """Dimwise_softmax (functions.py:97-127) by target and by source, alpha * e, index_add."""
    def side(a, key):
        key = key.long()
        mx = torch.full((S, a.shape[1]), float("-inf"), dtype=a.dtype).scatter_reduce(
            0, key[:, None].expand_as(a), a, "amax", include_self=False)
        ex = (a - mx[key]).exp()
        den = torch.zeros(S, a.shape[1], dtype=a.dtype).index_add(0, key, ex)
        p = ex / den[key]
        return torch.zeros(S, a.shape[1], dtype=a.dtype).index_add(0, key, p * e)
    return side(at, tkey), side(as_, skey)


@pytest.mark.parametrize("with_alpha_idx", [False, True])
def test_seg_attention_fwd_bwd(with_alpha_idx):
    ops = _ops()
    torch.manual_seed(1)
    R, S = 4000, 600
    tkey = torch.sort(_keys(R, S, 2))[0].to(torch.int32)
    skey = _keys(R, S, 3)
    ra = 1500 if with_alpha_idx else R
    aidx = torch.randint(0, ra, (R,), dtype=torch.int32) if with_alpha_idx else None
    at = (2 * torch.randn(ra, 128)).requires_grad_(True)
    as_ = (2 * torch.randn(ra, 128)).requires_grad_(True)
    e = torch.randn(R, 128).requires_grad_(True)
    gyt, gys = torch.randn(S, 128), torch.randn(S, 128)
    # reference in fp64 on the CPU
    at64, as64, e64 = (t.detach().double().requires_grad_(True) for t in (at, as_, e))
    ai = aidx.long() if with_alpha_idx else torch.arange(R)
    yt_r, ys_r = _attn_ref(at64[ai], as64[ai], e64, tkey, skey, S)
    (yt_r * gyt.double()).sum().add((ys_r * gys.double()).sum()).backward()
    # device
    tg = ops.Grouping.build(tkey.to(DEV), S, sorted_rows=True)
    sg = ops.Grouping.build(skey.to(DEV), S)
    ag = ops.Grouping.build(aidx.to(DEV), ra) if with_alpha_idx else None
    atd, asd, ed = (t.detach().to(DEV).requires_grad_(True) for t in (at, as_, e))
    yt, ys = ops.seg_attention(atd, asd, ed, tg, sg, ag)
    assert _rel(yt, yt_r) < 1e-5 and _rel(ys, ys_r) < 1e-5
    torch.autograd.backward([yt, ys], [gyt.to(DEV), gys.to(DEV)])
    assert _rel(atd.grad, at64.grad) < 1e-5
    assert _rel(asd.grad, as64.grad) < 1e-5
    assert _rel(ed.grad, e64.grad) < 1e-5


class _TorchGMLP(torch.nn.Module):
    """functions.py:245-311 with RMSNorm, in fp64."""

    def __init__(self, K):
        super().__init__()
        self.c1, self.c2 = torch.nn.Linear(K, 128), torch.nn.Linear(128, 128)
        self.g1, self.g2 = torch.nn.Linear(K, 128), torch.nn.Linear(128, 128)
        # fp32's eps, the constant RMSNorm(eps=None) uses in the fp32 reference
        eps = torch.finfo(torch.float32).eps
        self.nc, self.ng = torch.nn.RMSNorm(128, eps=eps), torch.nn.RMSNorm(128, eps=eps)
        with torch.no_grad():
            self.nc.weight.uniform_(0.5, 1.5)
            self.ng.weight.uniform_(0.5, 1.5)

    def forward(self, x):
        core = F.silu(self.nc(self.c2(F.silu(self.c1(x)))))
        gate = torch.sigmoid(self.ng(self.g2(F.silu(self.g1(x)))))
        return core * gate


class _ShimGated(torch.nn.Module):
    """Exposes the attribute layout ops.GmlpPack reads (mlp_core.layers[0/3], norms)."""

    def __init__(self, t):
        super().__init__()
        self.mlp_core = torch.nn.Module()
        self.mlp_core.layers = torch.nn.ModuleList([t.c1, torch.nn.Identity(), torch.nn.Identity(), t.c2])
        self.mlp_gate = torch.nn.Module()
        self.mlp_gate.layers = torch.nn.ModuleList([t.g1, torch.nn.Identity(), torch.nn.Identity(), t.g2])
        self.core_norm, self.gate_norm = t.nc, t.ng


@pytest.mark.parametrize("gtg", [True, False])
@pytest.mark.parametrize("mode,tol", [("fp32", 1e-5), ("bf16x6", 1e-5), ("f16x3", 1e-5), ("bf16x3", 1e-4)])
@pytest.mark.parametrize("nsrc,M", [(3, 1000), (4, 777), (3, 64), (4, 5)])
def test_gated_mlp_fwd_bwd(nsrc, M, mode, tol, gtg):
    """GatedMLP over [x0, x1[i1], ...] against fp64; with gtg the gathered tables of at
    most M/2 rows (M = 1000, 777 here) are multiplied before their gather."""
    ops = _ops()
    with ops.gather_after_gemm(gtg, min_rows=0, ratio=2):
        _gated_mlp_case(ops, nsrc, M, mode, tol)


@pytest.mark.parametrize("gtg", [True, False])
@pytest.mark.parametrize("mode,tol", [("fp32", 1e-5), ("bf16x6", 1e-5), ("f16x3", 1e-5), ("bf16x3", 1e-4)])
@pytest.mark.parametrize("M", [1, 64, 4097, 70001])
def test_gated_mlp_fwd_ffn_tail(M, mode, tol, gtg):
    """matris_gmlp_fwd_ffn (the line refinement's [tb, atom[i], bond[t], bond[s]] GatedMLP
    with edge_FFN(h) + r tb on its output rows): out, p and z bit-identical to the plain
    forward; the tail's t and output against fp64 of the kernel's own h (and against
    matris_ffn_fwd on it to the same bar); nothing saved when saves are discarded."""
    ops = _ops()
    ops.set_mma_precision(mode)
    try:
        torch.manual_seed(M + 3)
        mod = _ShimGated(_TorchGMLP(512)).to(DEV)
        pack = ops.GmlpPack().get(mod)
        mm = ops._MMA["mode"]
        n_atom, n_bond = max(1, M // 300), max(1, M // 8)
        tb = torch.randn(M, 128, device=DEV)
        atom, bond = torch.randn(n_atom, 128, device=DEV), torch.randn(n_bond, 128, device=DEV)
        idx = [None, torch.randint(0, n_atom, (M,), dtype=torch.int32, device=DEV),
               torch.randint(0, n_bond, (M,), dtype=torch.int32, device=DEV),
               torch.randint(0, n_bond, (M,), dtype=torch.int32, device=DEV)]
        srcs = [tb, atom, bond, bond]
        w1, w2 = torch.randn(128, 128, device=DEV) / 11, torch.randn(128, 128, device=DEV) / 11
        fp = ops._WeightPack().get(w1, w2)
        r = torch.rand(128, device=DEV)
        with ops.gather_after_gemm(gtg, min_rows=1 << 12, ratio=4):
            h0, p0, z0, _ = ops.gmlp_fwd_raw(pack, srcs, idx, M, mm)
            h, p, z, t_out, t_p = ops.gmlp_fwd_ffn_raw(pack, srcs, idx, M, mm, fp, tb, r)
            assert torch.equal(h, h0) and torch.equal(p, p0) and torch.equal(z, z0)
            h64 = h.double()
            t64 = h64 @ w1.double().t()
            o64 = F.silu(t64) @ w2.double().t() + r.double() * tb.double()
            assert _rel(t_p, t64) < tol and _rel(t_out, o64) < tol
            o_sep, p_sep = ops.ffn_fwd_raw(fp, h, mm, res=(tb, r))
            assert _rel(t_out, o_sep.double()) < tol and _rel(t_p, p_sep.double()) < tol
            with ops.discard_saves():
                _, _, _, t_out2, _ = ops.gmlp_fwd_ffn_raw(pack, srcs, idx, M, mm, fp, tb, r)
            assert torch.equal(t_out2, t_out)
            # no residual (the atom-graph Refinement's edge FFN)
            _, _, _, t_out4, t_p4 = ops.gmlp_fwd_ffn_raw(pack, srcs, idx, M, mm, fp)
            assert torch.equal(t_p4, t_p)
            assert _rel(t_out4, F.silu(t64) @ w2.double().t()) < tol
            _, p3, z3, t_out3, t_p3 = ops.gmlp_fwd_ffn_raw(pack, srcs, idx, M, mm, fp, tb, r, save=False)
            assert p3 is None and z3 is None and t_p3 is None and torch.equal(t_out3, t_out)
    finally:
        ops.set_mma_precision(ops.DEFAULT_MMA)


@pytest.mark.parametrize("gtg", [True, False])
@pytest.mark.parametrize("mode,tol", [("fp32", 1e-5), ("bf16x6", 1e-5), ("f16x3", 1e-5), ("bf16x3", 1e-4)])
@pytest.mark.parametrize("M", [1, 64, 4097, 70001])
def test_gated_mlp_fwd_pair_tail(M, mode, tol, gtg):
    """matris_gmlp_fwd_pair (the line attention's [tb, bond[t], bond[s]] GatedMLP with the
    logit projections W_s tb, W_t tb in the same launch): out, p, z and res_out
    bit-identical to the plain forward with the residual; the projections against fp64
    and against matris_pair_fwd on tb to the same bar; unchanged when saves are skipped
    or discarded."""
    ops = _ops()
    ops.set_mma_precision(mode)
    try:
        torch.manual_seed(M + 5)
        mod = _ShimGated(_TorchGMLP(384)).to(DEV)
        pack = ops.GmlpPack().get(mod)
        mm = ops._MMA["mode"]
        n_bond = max(1, M // 8)
        tb, bond = torch.randn(M, 128, device=DEV), torch.randn(n_bond, 128, device=DEV)
        idx = [None, torch.randint(0, n_bond, (M,), dtype=torch.int32, device=DEV),
               torch.randint(0, n_bond, (M,), dtype=torch.int32, device=DEV)]
        srcs = [tb, bond, bond]
        ws, wt = torch.randn(128, 128, device=DEV) / 11, torch.randn(128, 128, device=DEV) / 11
        pp = ops._WeightPack().get(ws, wt)
        r = torch.rand(128, device=DEV)
        with ops.gather_after_gemm(gtg, min_rows=1 << 12, ratio=4):
            e0, p0, z0, tbn0 = ops.gmlp_fwd_raw(pack, srcs, idx, M, mm, res=(tb, r))
            e, p, z, tbn, a_s, a_t = ops.gmlp_fwd_pair_raw(pack, srcs, idx, M, mm, (tb, r), pp)
            assert torch.equal(e, e0) and torch.equal(p, p0) and torch.equal(z, z0) and torch.equal(tbn, tbn0)
            t64 = tb.double()
            assert _rel(a_s, t64 @ ws.double().t()) < tol and _rel(a_t, t64 @ wt.double().t()) < tol
            s_sep, t_sep = ops.pair_fwd_raw(pp, tb, mm)
            assert _rel(a_s, s_sep.double()) < tol and _rel(a_t, t_sep.double()) < tol
            with ops.discard_saves():
                _, _, _, tbn2, a_s2, a_t2 = ops.gmlp_fwd_pair_raw(pack, srcs, idx, M, mm, (tb, r), pp)
            assert torch.equal(tbn2, tbn) and torch.equal(a_s2, a_s) and torch.equal(a_t2, a_t)
            _, p3, z3, _, a_s3, a_t3 = ops.gmlp_fwd_pair_raw(pack, srcs, idx, M, mm, (tb, r), pp, save=False)
            assert p3 is None and z3 is None and torch.equal(a_s3, a_s) and torch.equal(a_t3, a_t)
    finally:
        ops.set_mma_precision(ops.DEFAULT_MMA)


@pytest.mark.parametrize("mode,tol", [("fp32", 1e-5), ("bf16x6", 1e-5), ("f16x3", 1e-5), ("bf16x3", 1e-4)])
@pytest.mark.parametrize("layout", ["atom_graph", "one_table", "big"])
def test_gated_mlp_all_sources_projected(layout, mode, tol):
    """matris_gmlp_project + matris_gmlp_fwd_proj with no source multiplied in place
    (layer 1 is only gathered products): the atom-graph layout [bond[d2u], atom[tgt],
    atom[src]] (two tables), three gathers of one table (one projection of three blocks),
    and a 40,000-row table (several row tiles per projection work-group). Values and
    input gradients against fp64, and against the plain forward."""
    ops = _ops()
    ops.set_mma_precision(mode)
    torch.manual_seed({"atom_graph": 5, "one_table": 6, "big": 7}[layout])
    M = 90001 if layout == "big" else 4099
    sizes = {"atom_graph": [2011, 300, 300], "one_table": [1500] * 3, "big": [40000, 300, 300]}[layout]
    two = layout != "one_table"
    base = [torch.randn(sizes[0], 128), torch.randn(sizes[1], 128)][:2 if two else 1]
    idxs = [torch.randint(0, n, (M,), dtype=torch.int32) for n in sizes]
    ref = _TorchGMLP(384)
    b64 = [b.double().requires_grad_(True) for b in base]
    t64 = [b64[0], b64[1], b64[1]] if two else [b64[0]] * 3
    x = torch.cat([t64[j][idxs[j].long()] for j in range(3)], 1)
    ref64 = _TorchGMLP(384).double()
    ref64.load_state_dict({k: v.double() for k, v in ref.state_dict().items()})
    out_r = ref64(x)
    g = torch.randn(M, 128)
    (out_r * g.double()).sum().backward()
    mod = _ShimGated(ref).to(DEV)
    pack = ops.GmlpPack()
    bd = [b.to(DEV).requires_grad_(True) for b in base]
    td = [bd[0], bd[1], bd[1]] if two else [bd[0]] * 3
    try:
        spec = [(td[j], ops.Grouping.build(idxs[j].to(DEV), sizes[j])) for j in range(3)]
        with ops.gather_after_gemm(True, min_rows=0, ratio=2):
            out = ops.gated_mlp(mod, pack, spec)
        assert _rel(out, out_r) < tol
        out.backward(g.to(DEV))
        for j in range(len(base)):
            assert _rel(bd[j].grad, b64[j].grad) < tol, j
        with torch.no_grad(), ops.gather_after_gemm(False):
            plain = ops.gated_mlp(mod, pack, spec)
        assert _rel(out.detach(), plain.double()) < tol
    finally:
        ops.set_mma_precision(ops.DEFAULT_MMA)


def _gated_mlp_case(ops, nsrc, M, mode, tol):
    ops.set_mma_precision(mode)
    torch.manual_seed(nsrc * 100 + M)
    K = 128 * nsrc
    ref = _TorchGMLP(K)
    sizes = [M] + [300 + 17 * j for j in range(1, nsrc)]
    srcs = [torch.randn(n, 128) for n in sizes]
    idxs = [None] + [torch.randint(0, n, (M,), dtype=torch.int32) for n in sizes[1:]]
    # fp64 reference
    s64 = [s.double().requires_grad_(True) for s in srcs]
    x = torch.cat([s64[0]] + [s64[j][idxs[j].long()] for j in range(1, nsrc)], 1)
    ref64 = _TorchGMLP(K).double()
    ref64.load_state_dict({k: v.double() for k, v in ref.state_dict().items()})
    out_r = ref64(x)
    g = torch.randn(M, 128)
    (out_r * g.double()).sum().backward()
    # device
    mod = _ShimGated(ref).to(DEV)
    pack = ops.GmlpPack()
    sd = [s.to(DEV).requires_grad_(True) for s in srcs]
    srcs_spec = [(sd[0], None)] + [(sd[j], ops.Grouping.build(idxs[j].to(DEV), sizes[j])) for j in range(1, nsrc)]
    try:
        out = ops.gated_mlp(mod, pack, srcs_spec)
        assert _rel(out, out_r) < tol
        out.backward(g.to(DEV))
        for j in range(nsrc):
            assert _rel(sd[j].grad, s64[j].grad) < tol, j
    finally:
        ops.set_mma_precision(ops.DEFAULT_MMA)


_MODES = [("fp32", 1e-5), ("bf16x6", 1e-5), ("f16x3", 1e-5), ("bf16x3", 1e-4)]


@pytest.mark.parametrize("mode,tol", [("fp32", 1e-5), ("f16x3", 1e-5), ("bf16x3", 1e-4)])
@pytest.mark.parametrize("M", [1, 63, 64, 1000, 40961])
def test_three_body_embedding_fwd_bwd(M, mode, tol):
    """matris_tb_embed_fwd / _bwd: SiLU(Ws (Wa b)) over the [M, 16] angle basis and its input
    gradient (ThreebodyEmbedding's angle_embedding + swish_layer, no biases) against fp64."""
    ops = _ops()
    ops.set_mma_precision(mode)
    torch.manual_seed(M)
    wa = torch.nn.Linear(16, 128, bias=False).weight.detach()
    ws = torch.nn.Linear(128, 128, bias=False).weight.detach()
    b = torch.randn(M, 16)
    g = torch.randn(M, 128)
    b64 = b.double().requires_grad_(True)
    ref = F.silu(F.linear(F.linear(b64, wa.double()), ws.double()))
    (ref * g.double()).sum().backward()
    bd = b.to(DEV).requires_grad_(True)
    try:
        out = ops.tb_embed(bd, wa.to(DEV), ws.to(DEV), ops._WeightPack())
        assert _rel(out, ref) < tol
        out.backward(g.to(DEV))
        assert _rel(bd.grad, b64.grad) < tol
    finally:
        ops.set_mma_precision(ops.DEFAULT_MMA)


def test_pack_b_fragment_layout():
    """Packed weight = fragment planes: unit ((nt*KB + kb)*NPL + plane)*64 + lane holds
    row n = 32 nt + lane%32, k = 16 kb + 8 (lane//32) + j, j = 0..7."""
    ops = _ops()
    torch.manual_seed(3)
    n, k = 64, 48
    w = torch.randn(n, k) * torch.logspace(-3, 3, k)[None, :]
    nn_, kk = torch.meshgrid(torch.arange(n), torch.arange(k), indexing="ij")
    nt, kb, lane, j = nn_ // 32, kk // 16, nn_ % 32 + 32 * ((kk % 16) // 8), kk % 8
    # mode 0: the fp32 values themselves, 8 per lane as two 16-byte planes
    p0 = ops.pack_b(w.to(DEV), 0).cpu().view(torch.float32).view(n // 32, k // 16, 2, 64, 4)
    assert torch.equal(p0[nt, kb, j // 4, lane, j % 4], w)
    # mode 6: hi = w truncated to bf16 (low 16 bits cleared), mid likewise for w - hi,
    # and hi + mid + lo == w exactly
    p6 = ops.pack_b(w.to(DEV), 6).cpu().view(torch.bfloat16).view(n // 32, k // 16, 3, 64, 8)
    hi, mid, lo = (p6[nt, kb, q, lane, j].double() for q in range(3))
    trunc = (w.view(torch.int32) & -65536).view(torch.float32)
    assert torch.equal(p6[nt, kb, 0, lane, j].float(), trunc)
    assert torch.equal(hi + mid + lo, w.double())
    assert (mid.abs() < hi.abs() * 2.0 ** -7).all() and (lo.abs() < mid.abs() * 2.0 ** -7).all()
    # mode 3: the same hi plane; mid = round-to-nearest bf16 of w - hi
    p3 = ops.pack_b(w.to(DEV), 3).cpu().view(torch.bfloat16).view(n // 32, k // 16, 2, 64, 8)
    assert torch.equal(p3[:, :, 0], p6[:, :, 0])
    assert torch.equal(p3[nt, kb, 1, lane, j], (w - trunc).to(torch.bfloat16))
    # mode 2: header {1/s, s, 0, 0} with s = 2^(14 - floor(log2 max|w|)); then u0 =
    # round-to-nearest fp16 of s w and u1 = fp16 of s w - u0
    raw = ops.pack_b(w.to(DEV), 2).cpu()
    hdr = raw[:16].view(torch.float32)
    e = int(torch.floor(torch.log2(w.abs().max())).item())
    assert hdr.tolist() == [2.0 ** (e - 14), 2.0 ** (14 - e), 0.0, 0.0]
    p2 = raw[16:].view(torch.float16).view(n // 32, k // 16, 2, 64, 8)
    sw = w * 2.0 ** (14 - e)
    assert sw.abs().max().item() < 2.0 ** 15
    u0 = sw.to(torch.float16)
    assert torch.equal(p2[nt, kb, 0, lane, j], u0)
    assert torch.equal(p2[nt, kb, 1, lane, j], (sw - u0.float()).to(torch.float16))
    big = sw.abs() >= 2.0 ** -3  # where the residual plane is a normal fp16
    err = (u0.double() + p2[nt, kb, 1, lane, j].double() - sw.double()).abs()
    assert (err[big] <= sw.double().abs()[big] * 2.0 ** -21).all()


@pytest.mark.parametrize("kind", ["gmlp", "ffn", "pair"])
def test_f16x3_range_flag(kind):
    """A forward activation beyond the fp16 range sets the device's range flag in every
    f16x3 kernel family; values inside the range leave it clear.  The backward kernels scale
    each gradient row by a power of two first (mma.h row_scale), so a gradient row with an
    element of 2e5 or one of 1e-9 is carried at full precision without the flag: its input
    gradient matches the plain fp32 MFMA mode's."""
    ops = _ops()
    torch.manual_seed(11)
    M = 200
    w1, w2 = torch.randn(128, 128, device=DEV) / 11, torch.randn(128, 128, device=DEV) / 11
    ref = _TorchGMLP(128)
    shim = _ShimGated(ref).to(DEV)

    def run(x, g=None):
        xd = x.clone().requires_grad_(True)
        if kind == "gmlp":
            out = ops.gated_mlp(shim, ops.GmlpPack(), [(xd, None)])
        elif kind == "ffn":
            out = ops.ffn(ops._WeightPack().get(w1, w2), xd)
        else:
            out = ops.proj_pair(ops._WeightPack().get(w1, w2), xd)[0]
        if g is not None:
            out.backward(g)
        return out, xd.grad

    ops.set_mma_precision("f16x3")
    try:
        assert not ops.f16_range_take()
        for big in (False, True):
            x = torch.randn(M, 128, device=DEV)
            if big:
                x[77, 5] = 1.0e5
            run(x)
            assert ops.f16_range_take() == big, ("forward", big)
        x = torch.randn(M, 128, device=DEV)
        g = torch.randn(M, 128, device=DEV)
        g[3, 9] = -2.0e5   # a row far above the fp16 range
        g[40] *= 1e-9      # a row far below its normal range
        _, gx = run(x, g)
        assert not ops.f16_range_take(), "backward"
        with ops.mma_precision("fp32"):
            _, gx32 = run(x, g)
        for r in (3, 40, 100):
            err = ((gx[r] - gx32[r]).abs().max() / gx32[r].abs().max()).item()
            assert err < 1e-5, (r, err)
    finally:
        ops.set_mma_precision(ops.DEFAULT_MMA)


def test_discarded_saves_leave_outputs_unchanged():
    """ops.discard_saves (the original pass of a checkpointed block): the GatedMLP and FFN
    forwards return the same outputs bit for bit, and placeholders of the saved tensors'
    shapes instead of written p / z."""
    ops = _ops()
    torch.manual_seed(3)
    ref = _TorchGMLP(384)
    mod = _ShimGated(ref).to(DEV)
    pack = ops.GmlpPack()
    M = 140001
    tb, bond = torch.randn(M, 128, device=DEV), torch.randn(5000, 128, device=DEV)
    it = torch.randint(0, 5000, (M,), device=DEV, dtype=torch.int32)
    isrc = torch.randint(0, 5000, (M,), device=DEV, dtype=torch.int32)
    args = (pack.get(mod), [tb, bond, bond], [None, it, isrc], M, ops._MMA["mode"])
    out, p, z, _ = ops.gmlp_fwd_raw(*args)
    with ops.discard_saves():
        out2, p2, z2, _ = ops.gmlp_fwd_raw(*args)
    assert torch.equal(out, out2) and p2.shape == p.shape and z2.shape == z.shape
    l1, l2 = torch.randn(128, 128, device=DEV) / 11, torch.randn(128, 128, device=DEV) / 11
    wp = ops._WeightPack().get(l1, l2)
    o, q = ops.ffn_fwd_raw(wp, tb, ops._MMA["mode"])
    with ops.discard_saves():
        o2, q2 = ops.ffn_fwd_raw(wp, tb, ops._MMA["mode"])
    assert torch.equal(o, o2) and q2.shape == q.shape


def _sorted_keys(M, S, seed):
    """Ascending int32 keys in [0, S): random segment lengths with empty segments, one-row
    segments and one segment of 200 rows (spanning four 64-row tiles when M allows)."""
    g = torch.Generator().manual_seed(seed)
    k = torch.sort(torch.randint(0, S, (M,), generator=g)).values
    if M > 400 and S > 10:
        k[100:300] = k[100]
        k = torch.sort(k).values
    return k.to(torch.int32)


@pytest.mark.parametrize("mode", ["f16x3", "fp32", "bf16x6"])
@pytest.mark.parametrize("K,blk,with_x0", [(384, 1, True), (512, 2, True), (384, 1, False), (384, 0, False)])
@pytest.mark.parametrize("M,S", [(5000, 300), (4097, 20), (64, 3), (1, 1), (70001, 9000)])
def test_gmlp_bwd_tile_run_sums(M, S, K, blk, with_x0, mode):
    """matris_gmlp_bwd_runs + matris_seg_sum2_runs: the segment sums of the run-summed
    block (rows ascending by key) equal the fp64 sums of the plain backward's rows
    (matris_gmlp_bwd) to fp32 rounding (1e-5 of the largest), also paired with a second,
    permuted source in one pass; every other output is bit-identical."""
    ops = _ops()
    ops.set_mma_precision(mode)
    try:
        torch.manual_seed(M + K)
        mod = _ShimGated(_TorchGMLP(K)).to(DEV)
        pack = ops.GmlpPack().get(mod)
        mm = ops._MMA["mode"]
        srcs = [torch.randn(M, 128, device=DEV) for _ in range(K // 128)]
        _, p, z, _ = ops.gmlp_fwd_raw(pack, srcs, [None] * (K // 128), M, mm)
        g = torch.randn(M, 128, device=DEV)
        key = _sorted_keys(M, S, M).to(DEV)
        base = torch.randn(M, 128, device=DEV)
        x0a, x0b = (base.clone(), base.clone()) if with_x0 else (None, None)
        gxa = ops.gmlp_bwd_raw(pack, g, p, z, K, mm, g_x0=x0a, acc0=with_x0)
        gxb = ops.gmlp_bwd_raw(pack, g, p, z, K, mm, g_x0=x0b, acc0=with_x0, runs=(key, blk))
        c = (blk - (1 if with_x0 else 0)) * 128
        ld = gxa.shape[1]
        keep = torch.ones(ld, dtype=torch.bool)
        keep[c:c + 128] = False
        assert torch.equal(gxa[:, keep.to(DEV)], gxb[:, keep.to(DEV)])
        if with_x0:
            assert torch.equal(x0a, x0b)
        grp = ops.Grouping.build(key, S, sorted_rows=True)
        T = ops.gmlp_tile_rows()
        got = ops.seg_sum_raw(gxb, grp, ldx=ld, col_off=c, tile_rows=T)
        ref = torch.zeros(S, 128, dtype=torch.float64).index_add_(0, key.long().cpu(), gxa[:, c:c + 128].double().cpu())
        assert _rel(got, ref) < 1e-5
        # paired with a second, permuted source (the source-bond block of the line graph)
        other = 0 if c else 128
        skey = _keys(M, S, M + 1).to(DEV)
        sgrp = ops.Grouping.build(skey, S)
        acc = torch.randn(S, 128, device=DEV)
        got2 = ops.seg_sum_raw(gxb, grp, ldx=ld, col_off=c, tile_rows=T, out=acc.clone(), accumulate=True,
                               second=(gxa, sgrp, 1.0, ld, other))
        ref2 = (acc.double().cpu() + ref).index_add_(0, skey.long().cpu(), gxa[:, other:other + 128].double().cpu())
        assert _rel(got2, ref2) < 1e-5
    finally:
        ops.set_mma_precision(ops.DEFAULT_MMA)


@pytest.mark.parametrize("mode,tol", [("f16x3", 1e-5), ("fp32", 1e-5), ("bf16x3", 1e-4)])
@pytest.mark.parametrize("M,E", [(1, 1), (64, 9), (4097, 600), (140001, 18000)])
@pytest.mark.parametrize("env,runs", [(True, True), (False, False)])
def test_gmlp_bwd_ffn_head(M, E, env, runs, mode, tol):
    """matris_gmlp_bwd_ffn (the edge_FFN backward computed per tile in front of the
    GatedMLP backward) against matris_ffn_bwd(_env) followed by matris_gmlp_bwd_runs with
    the same residual source: every gradient equal to fp32 rounding of the largest."""
    ops = _ops()
    ops.set_mma_precision(mode)
    try:
        torch.manual_seed(M + 17)
        mod = _ShimGated(_TorchGMLP(512)).to(DEV)
        pack = ops.GmlpPack().get(mod)
        mm = ops._MMA["mode"]
        srcs = [torch.randn(M, 128, device=DEV) for _ in range(4)]
        _, p, z, _ = ops.gmlp_fwd_raw(pack, srcs, [None] * 4, M, mm)
        fp = ops._WeightPack().get(torch.randn(128, 128, device=DEV) / 11, torch.randn(128, 128, device=DEV) / 11)
        g_new, p_de = torch.randn(M, 128, device=DEV), torch.randn(M, 128, device=DEV)
        r = torch.rand(128, device=DEV)
        tkey = _sorted_keys(M, E, M).to(DEV)
        tgt = ops.Grouping.build(tkey, E, sorted_rows=True)
        src = ops.Grouping.build(_keys(M, E, M + 9).to(DEV), E)
        et = (torch.randn(E, 128, device=DEV), torch.rand(E, 128, device=DEV), tgt, src) if env else None
        rn = (tkey, 2) if runs else None
        g_h = ops.ffn_bwd_raw(fp, g_new, p_de, mm, env_term=et)
        x0a, x0b = torch.empty(M, 128, device=DEV), torch.empty(M, 128, device=DEV)
        gxa = ops.gmlp_bwd_raw(pack, g_h, p, z, 512, mm, g_x0=x0a, res_w=r, res_src=g_new, runs=rn)
        gxb = ops.gmlp_bwd_ffn_raw(pack, p, z, 512, mm, fp, g_new, p_de, env_term=et, g_x0=x0b, res_w=r, runs=rn)
        assert _rel(x0b, x0a) < tol
        if runs:  # the run-summed block holds partials at run starts only: compare the rest
            assert _rel(torch.cat([gxb[:, :128], gxb[:, 256:]], 1), torch.cat([gxa[:, :128], gxa[:, 256:]], 1)) < tol
            grp = ops.Grouping.build(tkey, E, sorted_rows=True)
            T = ops.gmlp_tile_rows()
            sa = ops.seg_sum_raw(gxa, grp, ldx=384, col_off=128, tile_rows=T)
            sb = ops.seg_sum_raw(gxb, grp, ldx=384, col_off=128, tile_rows=T)
            assert _rel(sb, sa) < tol
        else:
            assert _rel(gxb, gxa) < tol
        with pytest.raises(ValueError):
            ops.gmlp_bwd_ffn_raw(pack, p, z, 512, 6, fp, g_new, p_de)
    finally:
        ops.set_mma_precision(ops.DEFAULT_MMA)


@pytest.mark.parametrize("mode,tol", [("f16x3", 1e-5), ("fp32", 1e-5), ("bf16x3", 1e-4)])
@pytest.mark.parametrize("M,U,N", [(1, 1, 1), (300, 150, 20), (67396, 33698, 864)])
def test_gmlp_bwd_ffn_head_gathered(M, U, N, mode, tol):
    """matris_gmlp_bwd_ffn as the atom-graph Refinement uses it: the FFN's output gradient
    read through the directed-to-undirected index at half scale, the term g_agg[tgt] *
    env[d2u], no residual, the centre-atom block run-summed -- against matris_gather,
    matris_ffn_bwd, matris_gather_mul and matris_gmlp_bwd_runs, to fp32 rounding."""
    ops = _ops()
    ops.set_mma_precision(mode)
    try:
        torch.manual_seed(M + 23)
        mod = _ShimGated(_TorchGMLP(384)).to(DEV)
        pack = ops.GmlpPack().get(mod)
        mm = ops._MMA["mode"]
        srcs = [torch.randn(M, 128, device=DEV) for _ in range(3)]
        _, p, z, _ = ops.gmlp_fwd_raw(pack, srcs, [None] * 3, M, mm)
        fp = ops._WeightPack().get(torch.randn(128, 128, device=DEV) / 11, torch.randn(128, 128, device=DEV) / 11)
        g_b, p_de = torch.randn(U, 128, device=DEV), torch.randn(M, 128, device=DEV)
        env, g_agg = torch.rand(U, 128, device=DEV), torch.randn(N, 128, device=DEV)
        d2u = ops.Grouping.build(_keys(M, U, M + 2, empty_every=10 ** 9).to(DEV), U)
        tkey = _sorted_keys(M, N, M + 4).to(DEV)
        tgt = ops.Grouping.build(tkey, N, sorted_rows=True)
        g_te = ops.ffn_bwd_raw(fp, ops.gather_raw(g_b, d2u.key, 0.5), p_de, mm)
        g_h = ops.gather_mul_raw(g_agg, tkey, env, d2u.key, out=g_te, accumulate=True)
        gxa = ops.gmlp_bwd_raw(pack, g_h, p, z, 384, mm, runs=(tkey, 1))
        gxb = ops.gmlp_bwd_ffn_raw(pack, p, z, 384, mm, fp, g_b, p_de, env_term=(g_agg, env, tgt, d2u),
                                   runs=(tkey, 1), ffn_g_idx=d2u.key, ffn_g_scale=0.5)
        assert _rel(torch.cat([gxb[:, :128], gxb[:, 256:]], 1), torch.cat([gxa[:, :128], gxa[:, 256:]], 1)) < tol
        T = ops.gmlp_tile_rows()
        sa = ops.seg_sum_raw(gxa, tgt, ldx=384, col_off=128, tile_rows=T)
        sb = ops.seg_sum_raw(gxb, tgt, ldx=384, col_off=128, tile_rows=T)
        assert _rel(sb, sa) < tol
        with pytest.raises(ValueError):  # a gathered G has no residual term
            ops.gmlp_bwd_ffn_raw(pack, p, z, 384, mm, fp, g_b, p_de, g_x0=torch.empty(M, 128, device=DEV),
                                 res_w=env[0], ffn_g_idx=d2u.key, ffn_g_scale=0.5)
    finally:
        ops.set_mma_precision(ops.DEFAULT_MMA)


@pytest.mark.parametrize("mode,tol", [("f16x3", 1e-6), ("fp32", 1e-6), ("bf16x3", 1e-5)])
@pytest.mark.parametrize("M", [1, 64, 4097, 70001])
@pytest.mark.parametrize("runs", [True, False])
def test_gmlp_bwd_pair_tail(M, runs, mode, tol):
    """matris_gmlp_bwd_pair (the line attention's projection backward added to source 0's
    gradient inside the GatedMLP backward) against matris_gmlp_bwd_runs followed by
    matris_pair_bwd with accumulate: source 0's gradient equal to a few fp32 roundings of
    its largest value (the sum order differs), every other output bit-identical."""
    ops = _ops()
    ops.set_mma_precision(mode)
    try:
        torch.manual_seed(M + 31)
        mod = _ShimGated(_TorchGMLP(384)).to(DEV)
        pack = ops.GmlpPack().get(mod)
        mm = ops._MMA["mode"]
        srcs = [torch.randn(M, 128, device=DEV) for _ in range(3)]
        _, p, z, _ = ops.gmlp_fwd_raw(pack, srcs, [None] * 3, M, mm)
        pp = ops._WeightPack().get(torch.randn(128, 128, device=DEV) / 11, torch.randn(128, 128, device=DEV) / 11)
        g, g_as, g_at, g_new = (torch.randn(M, 128, device=DEV) for _ in range(4))
        r = torch.rand(128, device=DEV)
        rn = (_sorted_keys(M, max(1, M // 8), M).to(DEV), 1) if runs else None
        x0a, x0b = torch.empty(M, 128, device=DEV), torch.empty(M, 128, device=DEV)
        gxa = ops.gmlp_bwd_raw(pack, g, p, z, 384, mm, g_x0=x0a, runs=rn)
        ops.pair_bwd_raw(pp, g_as, g_at, mm, res=g_new, res_w=r, out=x0a, accumulate=True)
        gxb = ops.gmlp_bwd_raw(pack, g, p, z, 384, mm, g_x0=x0b, res_w=r, res_src=g_new, runs=rn, pair=(pp, g_as, g_at))
        assert _rel(x0b, x0a) < tol
        if runs:
            assert torch.equal(gxb[:, 128:], gxa[:, 128:])
        else:
            assert torch.equal(gxb, gxa)
        with pytest.raises(ValueError):
            ops.gmlp_bwd_raw(pack, g, p, z, 384, mm, pair=(pp, g_as, g_at))
    finally:
        ops.set_mma_precision(ops.DEFAULT_MMA)


@pytest.mark.parametrize("mode,tol", [("f16x3", 1e-6), ("fp32", 1e-6), ("bf16x3", 1e-5)])
@pytest.mark.parametrize("M,S", [(1, 1), (63, 9), (4097, 700), (70001, 9000)])
def test_attn_pair_bwd(M, S, mode, tol):
    """matris_attn_pair_bwd (the line attention's backward and its logit projections' in
    one launch) against matris_attn_bwd followed by matris_pair_bwd of its logit gradients
    with the residual term: g_e bit-identical, g_tb equal to a few fp32 roundings of its
    largest value (the two k-halves are summed in the other order).  Statistics from
    matris_attn_fwd on the same rows; targets ascending with empty segments, sources
    random.  Rows past the last full tile and one-row segments included."""
    ops = _ops()
    ops.set_mma_precision(mode)
    try:
        torch.manual_seed(M + S)
        mm = ops._MMA["mode"]
        tkey = _sorted_keys(M, S, M + 5).to(DEV)
        skey = _keys(M, S, M + 6).to(DEV)
        tgt = ops.Grouping.build(tkey, S, sorted_rows=True)
        src = ops.Grouping.build(skey, S)
        a_t, a_s = 2 * torch.randn(M, 128, device=DEV), 2 * torch.randn(M, 128, device=DEV)
        e = torch.randn(M, 128, device=DEV)
        y_t, y_s, lse_t, lse_s = ops.attn_fwd_raw(a_t, a_s, e, tgt, src, None)
        g_y = torch.randn(S, 256, device=DEV) * 1e-2
        base = torch.randn(M, 128, device=DEV) * 1e-2
        r = torch.rand(128, device=DEV)
        pp = ops._WeightPack().get(torch.randn(128, 128, device=DEV) / 11, torch.randn(128, 128, device=DEV) / 11)
        g_at, g_as, ge_ref = ops.attn_bwd_raw(a_t, a_s, e, y_t, y_s, lse_t, lse_s, g_y, g_y[:, 128:], tgt, src, None,
                                              ldgy=256, g_e_base=base)
        gtb_ref = ops.pair_bwd_raw(pp, g_as, g_at, mm, res=base, res_w=r)
        g_e, g_tb = ops.attn_pair_bwd_raw(a_t, a_s, e, y_t, y_s, lse_t, lse_s, g_y, tgt, src, base, pp, r, mm)
        assert torch.equal(g_e, ge_ref)
        assert _rel(g_tb, gtb_ref) < tol
        assert ops.status_take() == 0
    finally:
        ops.set_mma_precision(ops.DEFAULT_MMA)


@pytest.mark.parametrize("mode", ["f16x3", "fp32", "bf16x6"])
@pytest.mark.parametrize("M", [1, 64, 4097, 70001])
def test_gmlp_bwd_res_src(M, mode):
    """matris_gmlp_bwd_runs with res_src: source 0's gradient gains res_w * res_src in the
    epilogue, equal (to one fp32 rounding) to the plain backward accumulating onto
    res_w * res_src written beforehand; the other sources' gradients are bit-identical."""
    ops = _ops()
    ops.set_mma_precision(mode)
    try:
        torch.manual_seed(M + 11)
        mod = _ShimGated(_TorchGMLP(512)).to(DEV)
        pack = ops.GmlpPack().get(mod)
        mm = ops._MMA["mode"]
        srcs = [torch.randn(M, 128, device=DEV) for _ in range(4)]
        _, p, z, _ = ops.gmlp_fwd_raw(pack, srcs, [None] * 4, M, mm)
        g, r_src = torch.randn(M, 128, device=DEV), torch.randn(M, 128, device=DEV)
        r_w = torch.rand(128, device=DEV)
        x0a = r_w * r_src
        gxa = ops.gmlp_bwd_raw(pack, g, p, z, 512, mm, g_x0=x0a, acc0=True)
        x0b = torch.full((M, 128), float("nan"), device=DEV)
        gxb = ops.gmlp_bwd_raw(pack, g, p, z, 512, mm, g_x0=x0b, acc0=False, res_w=r_w, res_src=r_src)
        assert torch.equal(gxa, gxb)
        assert (x0b - x0a).abs().max().item() <= 2e-6 * x0a.abs().max().item()
        key = _sorted_keys(M, max(1, M // 7), M).to(DEV)
        x0c = torch.full((M, 128), float("nan"), device=DEV)
        ops.gmlp_bwd_raw(pack, g, p, z, 512, mm, g_x0=x0c, acc0=False, res_w=r_w, res_src=r_src, runs=(key, 2))
        assert torch.equal(x0b, x0c)
        with pytest.raises(ValueError):
            ops.gmlp_bwd_raw(pack, g, p, z, 512, mm, g_x0=x0c, res_src=r_src)
    finally:
        ops.set_mma_precision(ops.DEFAULT_MMA)


@pytest.mark.parametrize("mode", ["f16x3", "fp32", "bf16x6", "bf16x3"])
@pytest.mark.parametrize("M,E", [(1, 1), (1000, 130), (140001, 18000), (264384, 33698)])
def test_ffn_bwd_env_term(M, E, mode):
    """matris_env_agg_bwd_env + matris_ffn_bwd_env (the refinement's hidden-row gradient in
    one write) against matris_ffn_bwd followed by matris_env_agg_bwd with accumulate:
    g_env bit-identical, g_agg_env = g_agg * env exactly, g_h equal to one fp32 rounding
    (the term's product and sum may fuse into one FMA), and the added term equal to its
    fp64 value to fp32 rounding."""
    ops = _ops()
    ops.set_mma_precision(mode)
    try:
        torch.manual_seed(M)
        mm = ops._MMA["mode"]
        wp = ops._WeightPack().get(torch.randn(128, 128, device=DEV) / 11, torch.randn(128, 128, device=DEV) / 11)
        tkey = _sorted_keys(M, E, M).to(DEV)
        skey = _keys(M, E, M + 5).to(DEV)
        tgt = ops.Grouping.build(tkey, E, sorted_rows=True)
        src = ops.Grouping.build(skey, E)
        h, g, p = (torch.randn(M, 128, device=DEV) for _ in range(3))
        env, g_agg, S = torch.rand(E, 128, device=DEV), torch.randn(E, 128, device=DEV), torch.randn(E, 128, device=DEV)
        g_h_ref = ops.ffn_bwd_raw(wp, g, p, mm)
        g_ffn = g_h_ref.clone()
        g_env_ref = ops.env_agg_bwd_raw(h, env, g_agg, S, tgt, src, g_h_ref, accumulate=True)
        g_env, ge = ops.env_agg_bwd_env_raw(h, env, g_agg, S, tgt, src)
        assert torch.equal(ge, g_agg * env)
        assert torch.equal(g_env, g_env_ref)
        g_h = ops.ffn_bwd_raw(wp, g, p, mm, env_term=(ge, env, tgt, src))
        ulp = 2.0 ** -23 * (g_ffn.abs() + (ge[tkey.long()] * env[skey.long()]).abs())
        assert bool(((g_h - g_h_ref).abs() <= ulp).all())
        term = (g_agg.double() * env.double())[tkey.long()] * env.double()[skey.long()]
        assert _rel(g_h.double() - g_ffn.double(), term) < 1e-6
        with pytest.raises(ValueError):
            ops.ffn_bwd_raw(wp, g, p, mm, g_res=torch.empty_like(g), res_w=env[0], env_term=(ge, env, tgt, src))
    finally:
        ops.set_mma_precision(ops.DEFAULT_MMA)


@pytest.mark.parametrize("case", ["c3", "small", "uneven"])
def test_attn_bwd_by_bond(case):
    """matris_attn_bwd_bond (the atom-graph attention backward by undirected bond) against
    matris_attn_bwd through d2u followed by the d2u segment sums of its logit gradients
    and the gathered base gradient: bit-identical when every bond has its two directed
    copies (C3 atom graph, a small random graph), to fp32 rounding when segments are
    uneven (d2u segments of 0-5 rows)."""
    ops = _ops()
    torch.manual_seed(3)
    if case == "c3":
        from matris_amd import workloads as W
        from matris_amd.model.batch import process_graphs
        from matris_amd.model.model import MatRIS
        g = MatRIS().to(DEV).graph_converter(W.c3_cu864())
        bg = process_graphs([g])
        tgt, src = bg["atom_graph_dict"]["grp_tgt"], bg["atom_graph_dict"]["grp_src"]
        d2u_key = bg["directed2undirected"].to(torch.int32).contiguous()
        N, U = tgt.n_seg, bg["n_undirected"]
    else:
        N, U = 50, 400
        if case == "small":
            d2u_key = torch.arange(U, dtype=torch.int32).repeat_interleave(2)[torch.randperm(2 * U)]
        else:
            d2u_key = torch.randint(0, U, (2 * U,), dtype=torch.int32)
        d2u_key = d2u_key.to(DEV)
        R = d2u_key.numel()
        tgt = ops.Grouping.build(torch.sort(torch.randint(0, N, (R,), device=DEV)).values.to(torch.int32), N,
                                 sorted_rows=True)
        src = ops.Grouping.build(torch.randint(0, N, (R,), dtype=torch.int32, device=DEV), N)
    R = d2u_key.numel()
    d2u = ops.Grouping.build(d2u_key, U)
    a_t, a_s = torch.randn(U, 128, device=DEV), torch.randn(U, 128, device=DEV)
    e = torch.randn(R, 128, device=DEV)
    y_t, y_s, lse_t, lse_s = ops.attn_fwd_raw(a_t, a_s, e, tgt, src, d2u)
    g_y = torch.randn(N, 256, device=DEV)
    g_b = torch.randn(U, 128, device=DEV)
    base = ops.gather_raw(g_b, d2u.key, 0.5)
    at_r, as_r, ge_r = ops.attn_bwd_raw(a_t, a_s, e, y_t, y_s, lse_t, lse_s, g_y, g_y[:, 128:], tgt, src, d2u,
                                        ldgy=256, g_e_base=base)
    at_r, as_r = ops.seg_sum_raw(at_r, d2u), ops.seg_sum_raw(as_r, d2u)
    at_b, as_b, ge_b = ops.attn_bwd_bond_raw(a_t, a_s, e, y_t, y_s, lse_t, lse_s, g_y, g_y[:, 128:], tgt, src, d2u,
                                             ldgy=256, g_base=g_b, base_scale=0.5)
    assert torch.equal(ge_b, ge_r)
    if case == "uneven":
        assert _rel(at_b, at_r) < 1e-6 and _rel(as_b, as_r) < 1e-6
    else:
        assert torch.equal(at_b, at_r) and torch.equal(as_b, as_r)


@pytest.mark.parametrize("mode,tol", _MODES)
@pytest.mark.parametrize("M", [1, 63, 64, 1000, 4097, 140001])
def test_ffn_fwd_bwd(M, mode, tol):
    """FFN (Linear -> SiLU -> Linear, no bias) against fp64; 140,001 rows take the
    weight-stationary kernels (modes 0, 2, 3), the others the tiled ones."""
    ops = _ops()
    ops.set_mma_precision(mode)
    torch.manual_seed(M)
    l1 = torch.nn.Linear(128, 128, bias=False)
    l2 = torch.nn.Linear(128, 128, bias=False)
    x = torch.randn(M, 128)
    g = torch.randn(M, 128)
    x64 = x.double().requires_grad_(True)
    out_r = F.linear(F.silu(F.linear(x64, l1.weight.double())), l2.weight.double())
    (out_r * g.double()).sum().backward()
    w1, w2 = l1.weight.to(DEV), l2.weight.to(DEV)
    xd = x.to(DEV).requires_grad_(True)
    try:
        out = ops.ffn(ops._WeightPack().get(w1, w2), xd)
        assert _rel(out, out_r) < tol
        out.backward(g.to(DEV))
        assert _rel(xd.grad, x64.grad) < tol
    finally:
        ops.set_mma_precision(ops.DEFAULT_MMA)


@pytest.mark.parametrize("mode,tol", _MODES)
@pytest.mark.parametrize("M", [1, 65, 3000, 140001])
def test_proj_pair_fwd_bwd(M, mode, tol):
    """W_s x, W_t x and the input gradient against fp64 (140,001 rows: the weight-stationary
    forward in modes 0, 2, 3)."""
    ops = _ops()
    ops.set_mma_precision(mode)
    torch.manual_seed(7 + M)
    ws, wt = torch.randn(128, 128) / 11, torch.randn(128, 128) / 11
    x = torch.randn(M, 128)
    g0, g1 = torch.randn(M, 128), torch.randn(M, 128)
    x64 = x.double().requires_grad_(True)
    o0r, o1r = x64 @ ws.double().t(), x64 @ wt.double().t()
    ((o0r * g0.double()).sum() + (o1r * g1.double()).sum()).backward()
    xd = x.to(DEV).requires_grad_(True)
    try:
        o0, o1 = ops.proj_pair(ops._WeightPack().get(ws.to(DEV), wt.to(DEV)), xd)
        assert _rel(o0, o0r) < tol and _rel(o1, o1r) < tol
        torch.autograd.backward([o0, o1], [g0.to(DEV), g1.to(DEV)])
        assert _rel(xd.grad, x64.grad) < tol
        # one output unused: its gradient arrives as None
        xd.grad = None
        o0, _ = ops.proj_pair(ops._WeightPack().get(ws.to(DEV), wt.to(DEV)), xd)
        o0.backward(g0.to(DEV))
        assert _rel(xd.grad, (g0.double() @ ws.double())) < tol
    finally:
        ops.set_mma_precision(ops.DEFAULT_MMA)


@pytest.mark.parametrize("N,E", [(864, 67396), (5, 7), (1, 0)])
def test_edge_vectors_backward_vs_fp64(N, E):
    """matris_edge_vec_bwd: g_cart = sum over target rows - sum over source rows (the
    backward of cart[tgt] - (cart[src] + shift)), against fp64 autograd."""
    from matris_amd.model import ops
    g = torch.Generator().manual_seed(N + E)
    tgt = torch.sort(torch.randint(0, N, (E,), generator=g))[0]
    src = torch.randint(0, N, (E,), generator=g)
    cart, shift, gv = torch.randn(N, 3, generator=g), torch.randn(E, 3, generator=g), torch.randn(E, 3, generator=g)
    c64, s64 = cart.double().requires_grad_(True), shift.double().requires_grad_(True)
    ref = c64[tgt] - (c64[src] + s64)
    (ref * gv.double()).sum().backward()
    gt = ops.Grouping.build(tgt.to(torch.int32).to("cuda"), N, sorted_rows=True)
    gs = ops.Grouping.build(src.to(torch.int32).to("cuda"), N)
    cd, sd = cart.to("cuda").requires_grad_(True), shift.to("cuda").requires_grad_(True)
    out = ops.edge_vectors(cd, sd, gt, gs)
    assert torch.allclose(out.double().cpu(), ref.detach(), atol=1e-6)
    out.backward(gv.to("cuda"))
    assert torch.allclose(cd.grad.double().cpu(), c64.grad, atol=1e-4, rtol=1e-5)
    assert torch.equal(sd.grad.cpu(), -gv)


@pytest.mark.parametrize("N,E,strain,use", [(864, 67396, True, "both"), (5, 7, True, "both"), (64, 900, False, "both"),
                                            (40, 500, True, "length"), (1, 0, True, "both")])
def test_edge_geometry_vs_fp64(N, E, strain, use):
    """matris_edge_geom_fwd / _bwd against an fp64 autograd restatement of
    processgraph.py:169-199 with a non-zero, non-symmetric strain: sym = (S + S^T)/2,
    x' = x + x sym, L' = L + L sym, vec = x'[tgt] - (x'[src] + image L'), length, unit;
    the gradients of the positions and of the strain."""
    from matris_amd.model import ops
    g = torch.Generator().manual_seed(N + E + int(strain))
    tgt = torch.sort(torch.randint(0, N, (E,), generator=g))[0]
    src = torch.randint(0, N, (E,), generator=g)
    cart = 10 * torch.rand(N, 3, generator=g)
    lat = 8 * torch.eye(3) + torch.randn(3, 3, generator=g)
    img = torch.randint(-2, 3, (E, 3), generator=g).float()
    img[(tgt == src) & (img.abs().sum(1) == 0), 0] = 1.0  # no zero-length edge
    S = 0.01 * torch.randn(1, 3, 3, generator=g)
    # no edge shorter than 1 Angstrom (as in a real graph): fp32 rounding of vec would dominate
    pre = cart.double()[tgt] - (cart.double()[src] + img.double() @ lat.double())
    keep = pre.norm(dim=1) >= 1.0
    tgt, src, img = tgt[keep], src[keep], img[keep]
    E = int(keep.sum())
    gl, gu = torch.randn(E, generator=g), torch.randn(E, 3, generator=g)

    x64 = cart.double().requires_grad_(True)
    S64 = S.double().requires_grad_(True)
    sym = 0.5 * (S64 + S64.transpose(-1, -2))[0] if strain else torch.zeros(3, 3, dtype=torch.float64)
    xs = x64 + x64 @ sym
    Ls = lat.double() + lat.double() @ sym
    vec = xs[tgt] - (xs[src] + img.double() @ Ls)
    l64 = torch.norm(vec, dim=1)
    u64 = vec / l64[:, None]
    loss = (l64 * gl.double()).sum() + ((u64 * gu.double()).sum() if use == "both" else 0)
    ref_g = torch.autograd.grad(loss, [x64, S64] if strain else [x64], allow_unused=True) if E else None

    gt = ops.Grouping.build(tgt.to(torch.int32).to(DEV), N, sorted_rows=True)
    gs = ops.Grouping.build(src.to(torch.int32).to(DEV), N)
    cd = cart.to(DEV).requires_grad_(True)
    Sd = S.to(DEV).requires_grad_(True) if strain else None
    length, unit, lat_out, vol = ops.edge_geometry(cd, Sd, lat.to(DEV), img.to(DEV), gt, gs)
    assert _rel(lat_out, Ls.detach()) < 1e-6
    assert abs(vol.item() - torch.linalg.det(lat.double()).item()) < 1e-5 * abs(torch.linalg.det(lat.double()).item())
    if E == 0:
        return
    assert _rel(length, l64.detach()) < 1e-6
    # fp32 rounding of the operands of vec (|x'| and |image L'|, tens of Angstrom) over the
    # edge length bounds each unit vector's error
    mag = xs.detach()[tgt].norm(dim=1) + xs.detach()[src].norm(dim=1) + (img.double() @ Ls.detach()).norm(dim=1)
    bound = 4 * 2.0 ** -24 * mag / l64.detach() + 2.0 ** -23
    assert ((unit.double().cpu() - u64.detach()).abs().max(dim=1).values <= bound).all()
    loss_d = (length * gl.to(DEV)).sum() + ((unit * gu.to(DEV)).sum() if use == "both" else 0)
    got = torch.autograd.grad(loss_d, [cd, Sd] if strain else [cd])
    assert _rel(got[0], ref_g[0]) < 1e-5
    if strain:
        # the strain gradient sums over every edge and atom: bound by the sums of magnitudes
        err = (got[1].double().cpu() - ref_g[1]).abs().max().item()
        scale = (x64.detach().abs().T @ ref_g[0].abs()).max().item() + \
            (lat.double().abs().T @ (img.double().abs().T @ (gl.double().abs()[:, None] + gu.double().abs()))).max().item()
        assert err < 1e-5 * scale, (err, scale)


def _edge_basis64(d, mod):
    """fp64 enveloped Bessel bases of both cutoffs (basis_function.py:8-50, 116-186)."""
    def basis(b):
        rc, p = b.envelope_func.cutoff, b.envelope_func.p
        a_, b_, c_ = -(p + 1) * (p + 2) / 2, p * (p + 2), -p * (p + 1) / 2
        x = d / rc
        env = torch.where(x < 1, 1 + a_ * x ** p + b_ * x ** (p + 1) + c_ * x ** (p + 2), torch.zeros_like(x))
        f = b.frequencies.detach().double().cpu()
        return env[:, None] * ((2 / rc) ** 0.5 * torch.sin(f[None, :] * d[:, None] / rc) / d[:, None])
    return basis(mod.pairwise_rbf_expansion), basis(mod.threebody_rbf_expansion)


def _edge_mlp64(r6, mod):
    """fp64 rest of EdgeBasisEmbedding (feature_embed.py:42-148) on the radial basis r6:
    two bias-free linears, LayerNorm, the swish layer."""
    w = lambda lin: lin.weight.detach().double().cpu()
    ln = mod.edge_init_norm
    h2 = r6 @ w(mod.edge_linear1).t() @ w(mod.edge_linear2).t()
    y = F.layer_norm(h2, (128,), ln.weight.detach().double().cpu(), ln.bias.detach().double().cpu(), ln.eps)
    return F.silu(y @ w(mod.swish_layer.linear).t())


@pytest.mark.parametrize("mode,tol", [("fp32", 1e-5), ("bf16x6", 1e-5), ("f16x3", 1e-5), ("bf16x3", 1e-4)])
@pytest.mark.parametrize("U", [1, 64, 65, 5000])
def test_edge_embedding_vs_fp64(U, mode, tol):
    """matris_edge_embed_fwd / _bwd (EdgeBasisEmbedding once per bond) against an fp64
    restatement: both bases (also bitwise against matris_bessel_fwd, the reference's fp32
    evaluation), e from the kernel's own fp32 basis (the basis's fp32 rounding, ~1e-6
    absolute, is amplified by the LayerNorm's 1/sigma like any fp32 evaluation's), and the
    edge-length gradient through e and both bases (fp64 derivatives of the bases), written
    at the bonds' first directed edges only."""
    from matris_amd.model.model import EdgeBasisEmbedding
    ops = _ops()
    ops.set_mma_precision(mode)
    try:
        torch.manual_seed(U + 11)
        mod = EdgeBasisEmbedding(6, 4, 7, 128, 8, "Bessel", learnable=True).to(DEV)
        with torch.no_grad():  # trained-looking parameters: off the initial values
            for prm in (mod.pairwise_rbf_expansion.frequencies, mod.threebody_rbf_expansion.frequencies):
                prm.mul_(1 + 0.05 * torch.randn_like(prm))
            mod.edge_init_norm.weight.copy_(1 + 0.1 * torch.randn(128))
            mod.edge_init_norm.bias.copy_(0.1 * torch.randn(128))
        assert mod._fusable()
        E = 2 * U
        length = 0.8 + 5.6 * torch.rand(E, device=DEV)  # across both cutoffs
        u2d = torch.randperm(E, device=DEV)[:U].to(torch.int32)
        ld = length.clone().requires_grad_(True)
        e, r6, r4 = ops.edge_embed(ld, u2d, mod)
        d64 = length.double().cpu()[u2d.long().cpu()].requires_grad_(True)
        r664, r464 = _edge_basis64(d64, mod)
        assert _rel(r6, r664.detach()) < 1e-5 and _rel(r4, r464.detach()) < 1e-5
        r6_own = r6.detach().double().cpu().requires_grad_(True)
        e64 = _edge_mlp64(r6_own, mod)
        assert _rel(e, e64.detach()) < tol
        b = mod.pairwise_rbf_expansion
        assert torch.equal(r6, ops.bessel(length[u2d.long()], b.frequencies, b.envelope_func.cutoff, b.envelope_func.p))
        ge, g6, g4 = torch.randn(U, 128, device=DEV), torch.randn(U, 7, device=DEV), torch.randn(U, 7, device=DEV)
        (g_len,) = torch.autograd.grad((e * ge).sum() + (r6 * g6).sum() + (r4 * g4).sum(), [ld])
        (g_r6,) = torch.autograd.grad((e64 * ge.double().cpu()).sum(), [r6_own])
        (g64,) = torch.autograd.grad((r664 * (g_r6 + g6.double().cpu())).sum() + (r464 * g4.double().cpu()).sum(),
                                     [d64])
        mask = torch.zeros(E, dtype=torch.bool)
        mask[u2d.long().cpu()] = True
        assert torch.all(g_len.cpu()[~mask] == 0)
        assert _rel(g_len[u2d.long()], g64) < 10 * tol
    finally:
        ops.set_mma_precision(ops.DEFAULT_MMA)


@pytest.mark.parametrize("N", [864, 1, 17, 5000])
def test_readout_fused_vs_fp64(N):
    """matris_readout_fwd / _bwd: readout_norm (RMSNorm), the energy MLP 128-128-128-1 and the
    magmom MLP 128-256-1 (model.py readout, readout.py:18-133) against the same torch modules
    evaluated in fp64: per-row energies, |magmom| and the energy branch's input gradient."""
    from matris_amd.model.model import EnergyHead, MagmomHead, get_normalization
    ops = _ops()
    torch.manual_seed(N)
    norm = get_normalization("rms", 128)
    norm.eps = torch.finfo(torch.float32).eps  # eps=None's fp32 value, also in the fp64 evaluation
    eh, mh = EnergyHead(128, (128, 128), 1, "mlp", "silu"), MagmomHead(128, 256, 1, "mlp", "silu")
    with torch.no_grad():
        norm.weight.uniform_(0.5, 1.5)
        for p in list(eh.parameters()) + list(mh.parameters()):
            p.add_(0.05 * torch.randn_like(p))
    x = torch.randn(N, 128) * 2
    g_e = torch.randn(N)
    x64 = x.double().requires_grad_(True)
    n64 = norm.double()(x64)
    e64 = eh.energy_head.double()(n64).view(-1)
    m64 = torch.abs(mh.magmom_head.double()(n64)).view(-1)
    (e64 * g_e.double()).sum().backward()
    pack = ops.ReadoutPack().get(norm.float().to(DEV), eh.energy_head.float().to(DEV), mh.magmom_head.float().to(DEV))
    xd = x.to(DEV)
    e, m = ops.readout_fwd_raw(pack, xd)
    g_x = ops.readout_bwd_raw(pack, xd, g_e.to(DEV))
    assert _rel(e, e64.detach()) < 1e-5 and _rel(m, m64.detach()) < 1e-5
    assert _rel(g_x, x64.grad) < 1e-5
    e2, _ = ops.readout_fwd_raw(pack, xd)
    assert torch.equal(e, e2)  # fixed summation order
