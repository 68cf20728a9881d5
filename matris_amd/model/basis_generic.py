"""The embedding bases of MatRIS's non-default constructor options, as torch on the device.

The MatRIS-10M configuration (enveloped Bessel pairwise basis with 7 radial functions, the
4 x 4 spherical three-body basis) runs on the gfx950 kernels (matris_bessel_*,
matris_edge_embed_*, matris_sbf_*, matris_tb_embed_*).  The other options of the
reference build the same module tree and evaluate through the forms here:

  distance_expansion="Gaussian"    GaussianExpansion   (basis_function.py:189-219)
  three_body_expansion="fourier"   FourierExpansion    (basis_function.py:79-113)
  max_n, max_l < 4 (SH)            spherical_basis     (basis_function.py:54-77, 222-338)
  envelope_exponent=None           bessel_plain        (basis_function.py:162-186)

Each is a few elementwise operations per row, differentiated by autograd.
"""
from __future__ import annotations

import math

import torch
from torch import Tensor, nn

# Roots and coefficients of the spherical Bessel radial functions j_n(z x) for orders
# n = 0..3 and the first four roots z of each order (basis_function.py:241-274; the
# float32 values the reference stores).  Order 0: sin(z x) / x with z = j * pi.  Orders
# 1..3 (pairs (coefficient, frequency) per term, x^(n-1), ..., x^0 in turn):
#   n = 1: (a x cos(z x) + b sin(z x)) / x^2
#   n = 2: (a x^2 sin(z x) - b x cos(z x) + c sin(z x)) / x^3
#   n = 3: (a x^3 cos(z x) - b x^2 sin(z x) - c x cos(z x) + d sin(z x)) / x^4
SBF_ROOTS = (
    (3.14159274101257, 6.28318548202515, 9.42477798461914, 12.5663709640503),
    (4.49340963363647, 7.7252516746521, 10.9041213989258, 14.0661935806274),
    (5.76345920562744, 9.09501171112061, 12.322940826416, 15.5146026611328),
    (6.9879322052002, 10.4171180725098, 13.6980228424072, 16.9236221313477),
)
SBF_COEFS = (
    (),
    ((-1.02446483277785, -1.00834335996107, -1.00419641763893, -1.00252381898662),
     (0.22799275301076, 0.130525632358311, 0.092093290316619, 0.0712718627992818)),
    ((-1.04807944170731, -1.01861796359391, -1.01002272174988, -1.00628955560036),
     (0.545547077361439, 0.335992298618515, 0.245888396928293, 0.194582402961821),
     (0.0946561878721665, 0.0369424811413594, 0.0199537107571916, 0.0125418876146463)),
    ((1.06942831392075, 1.0292173312802, 1.01650804843248, 1.01069656069999),
     (0.918235852195231, 0.592803493701152, 0.445250264272671, 0.358326327374518),
     (0.328507713452024, 0.142266673367543, 0.0812617757677838, 0.0529328657590962),
     (0.0470107184508114, 0.0136570088173405, 0.0059323726279831, 0.00312775039221944)),
)


def _f32(v: float) -> float:
    """v rounded to float32, as the reference's float32 coefficient tensor holds it."""
    return float(torch.tensor(v, dtype=torch.float32))


# the tables as the float32 values the products use
_ROOTS32 = tuple(tuple(_f32(v) for v in r) for r in SBF_ROOTS)
_COEFS32 = tuple(tuple(tuple(_f32(v) for v in t) for t in c) for c in SBF_COEFS)


def radial_sbf(n: int, j: int, x: Tensor) -> Tensor:
    """The order-n spherical Bessel radial function at its j-th root, at x = d / cutoff."""
    z = _ROOTS32[n][j]
    c = [t[j] for t in _COEFS32[n]]
    s, co = torch.sin(z * x), torch.cos(z * x)
    if n == 0:
        return s / x
    if n == 1:
        return (c[0] * x * co + c[1] * s) / x ** 2
    if n == 2:
        return (c[0] * x ** 2 * s - c[1] * x * co + c[2] * s) / x ** 3
    return (c[0] * x ** 3 * co - c[1] * x ** 2 * s - c[2] * x * co + c[3] * s) / x ** 4


def legendre_y(l_max: int, x: Tensor) -> Tensor:
    """[n, l_max + 1]: the m = 0 spherical harmonics Y_l(cos theta) = sqrt((2l+1)/4pi)
    P_l(x) for l = 0..l_max (l_max <= 3)."""
    if not 0 <= l_max <= 3:
        raise ValueError("legendre_y: l_max must be 0..3")
    p = [torch.ones_like(x), x, 0.5 * (3.0 * x ** 2 - 1.0), 0.5 * x * (5.0 * x ** 2 - 3.0)]
    return torch.stack([math.sqrt((2 * l + 1) / (4.0 * math.pi)) * p[l] for l in range(l_max + 1)], dim=-1)


def spherical_basis(dist: Tensor, angle: Tensor, max_n: int, max_l: int, cutoff: float, factor: Tensor) -> Tensor:
    """[n, max_n * max_l]: column n * max_l + j holds the order-n radial function at root
    j times Y_l(cos angle) with l = (n * max_l + j) // max_n (the harmonics repeated
    max_n times each), scaled by sqrt(2 / cutoff^3)."""
    x = dist / cutoff
    rbf = torch.stack([radial_sbf(n, j, x) for n in range(max_n) for j in range(max_l)], dim=-1) * factor
    cbf = legendre_y(max_l - 1, torch.cos(angle)).repeat_interleave(max_n, dim=1)
    return rbf * cbf


def bessel_plain(dist: Tensor, frequencies: Tensor, inv_cutoff: float, norm_const: float) -> Tensor:
    """[n, num_radial]: sqrt(2 / cutoff) sin(f_k d / cutoff) / d, without an envelope."""
    d = dist[:, None]
    return norm_const * torch.sin(frequencies * (d * inv_cutoff)) / d


class GaussianExpansion(nn.Module):
    """basis_function.py:189-219: exp(coeff (d - mu_k)^2) with centres mu_k evenly spaced
    over [start, stop] and coeff = -1 / (2 (w (mu_1 - mu_0))^2)."""

    def __init__(self, start: float = 0.0, stop: float = 6.0, num_gaussians: int = 7,
                 basis_width_scalar: float = 2.0):
        super().__init__()
        self.num_output = num_gaussians
        offset = torch.linspace(start, stop, num_gaussians)
        self.coeff = -0.5 / (basis_width_scalar * (offset[1] - offset[0])).item() ** 2
        self.register_buffer("offset", offset)

    def forward(self, dist: Tensor) -> Tensor:
        return torch.exp(self.coeff * (dist.view(-1, 1) - self.offset.view(1, -1)) ** 2)


class FourierExpansion(nn.Module):
    """basis_function.py:79-113: [1 / sqrt 2, sin(k theta), cos(k theta)] / sqrt(pi) for
    k = 1..max_f (frequencies learnable or fixed)."""

    def __init__(self, max_f: int = 5, scale: float = math.pi, learnable: bool = False):
        super().__init__()
        self.max_f = max_f
        self.scale = math.sqrt(scale)
        freq = torch.arange(1, max_f + 1, dtype=torch.float)
        if learnable:
            self.frequencies = nn.Parameter(freq, requires_grad=True)
        else:
            self.register_buffer("frequencies", freq)

    def forward(self, angle: Tensor) -> Tensor:
        t = torch.outer(angle, self.frequencies)
        const = torch.full((angle.shape[0], 1), 1.0 / math.sqrt(2.0), dtype=angle.dtype, device=angle.device)
        return torch.cat([const, torch.sin(t), torch.cos(t)], dim=1) / self.scale
