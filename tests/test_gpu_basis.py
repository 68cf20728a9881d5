"""Basis-function kernels (E2 Bessel x envelope, E3 spherical three-body basis) against
the fp64 torch restatement of the reference (oracle/model_ref.py's modules on the CPU,
which restate basis_function.py / feature_embed.py), values and input gradients.
"""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


@pytest.mark.parametrize("cutoff", [6.0, 4.0])
def test_bessel_envelope_vs_fp64(cutoff):
    from matris_amd.model import ops
    from oracle.model_ref import BesselExpansion
    torch.manual_seed(int(cutoff))
    mod = BesselExpansion(7, cutoff, 8, learnable=True)
    # distances across the envelope cutoff (zero basis beyond it) and near 0.5 A
    d = torch.cat([torch.rand(5000) * 7.5 + 0.5, torch.tensor([cutoff, cutoff - 1e-3, 0.5])])
    g = torch.randn(d.shape[0], 7)
    d64 = d.double().requires_grad_(True)
    mod64 = BesselExpansion(7, cutoff, 8, learnable=True).double()
    mod64.load_state_dict({k: v.double() for k, v in mod.state_dict().items()})
    ref = mod64(d64)  # the oracle's restatement of the reference formula, in fp64
    (ref * g.double()).sum().backward()
    dd = d.to(DEV).requires_grad_(True)
    out = ops.bessel(dd, mod.frequencies.to(DEV), cutoff, 8.0)
    assert _rel(out, ref) < 1e-5
    out.backward(g.to(DEV))
    assert _rel(dd.grad, d64.grad) < 1e-4


def _unit_vectors(E, seed):
    g = torch.Generator().manual_seed(seed)
    v = torch.randn(E, 3, generator=g)
    return v / v.norm(dim=1, keepdim=True)


@pytest.mark.parametrize("E,A", [(500, 4000), (7, 9)])
def test_spherical_basis_vs_fp64(E, A):
    from matris_amd.model import ops
    from oracle.model_ref import SphericalExpansion
    torch.manual_seed(E)
    unit = _unit_vectors(E, E + 1)
    g = torch.Generator().manual_seed(A)
    de_t = torch.randint(0, E, (A,), generator=g)
    de_s = (de_t + torch.randint(1, E, (A,), generator=g)) % E  # a different edge
    gb = torch.randn(A, 16, generator=g)
    # fp64 reference: feature_embed.py:183-201 with SphericalExpansion (cutoff 6)
    u64 = unit.double().requires_grad_(True)
    vij, vjk = u64[de_t], u64[de_s]
    ang = torch.acos((vij * vjk).sum(1) * (1 - 1e-6))
    ref = SphericalExpansion(4, 4, 6).double()(vjk.norm(dim=1), ang)
    (ref * gb.double()).sum().backward()
    # device
    ud = unit.to(DEV).requires_grad_(True)
    gt = ops.Grouping.build(de_t.to(torch.int32).to(DEV), E)
    gs = ops.Grouping.build(de_s.to(torch.int32).to(DEV), E)
    out = ops.spherical_basis(ud, gt, gs, 6.0)
    assert out.shape == (A, 16)
    assert _rel(out, ref) < 2e-5
    out.backward(gb.to(DEV))
    assert _rel(ud.grad, u64.grad) < 2e-4


def test_spherical_basis_l0_is_constant_times_radial():
    """Y_0 = 1/(2 sqrt(pi)): basis[:, 0] = sqrt(2/6^3) sin(pi x)/x at x = 1/6 for unit vectors."""
    from matris_amd.model import ops
    unit = _unit_vectors(20, 3).to(DEV)
    de_t = torch.arange(20, dtype=torch.int32, device=DEV)
    de_s = torch.roll(de_t, 1)
    out = ops.spherical_basis(unit, ops.Grouping.build(de_t, 20), ops.Grouping.build(de_s, 20), 6.0)
    x = 1.0 / 6.0
    expect = math.sqrt(2.0 / 216.0) * math.sin(math.pi * x) / x * 0.5 / math.sqrt(math.pi)
    assert torch.allclose(out[:, 0].cpu(), torch.full((20,), expect), rtol=1e-5)
