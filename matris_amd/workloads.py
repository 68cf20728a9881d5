"""Deterministic synthetic structures for the benchmark / parity configurations.

Every generator returns plain numpy data (fp64 fractional coordinates, fp64 lattice with
lattice vectors as rows, int atomic numbers), i.e. what a pymatgen ``Structure`` or ASE
``Atoms`` would hand to ``GraphConverter`` (matris/graph/converter.py:79-87).

  C1  4-atom cubic fcc Cu, a = 5.43 A (the reference README example)
  C2  4096-atom random sequential addition, 0.085 atoms/A^3, d_min 1.8 A, seed 1
  C3  fcc Cu 6x6x6 conventional supercell (864 atoms), a = 3.61 A, sigma 0.05 A, seed 2
  C4  64 random triclinic cells of 8-64 atoms, Z in 1..94, seed 3
  C5  32,000-atom amorphous SiO2 (Si:O = 1:2, 2.2 g/cm^3), d_min 1.5 A, seed 4
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

AMU_G = 1.66053906660e-24


@dataclass
class Crystal:
    frac: np.ndarray      # [n, 3] fp64
    lattice: np.ndarray   # [3, 3] fp64, rows are lattice vectors
    z: np.ndarray         # [n] int64 atomic numbers

    @property
    def cart(self) -> np.ndarray:
        return self.frac @ self.lattice

    def __len__(self) -> int:
        return len(self.z)


FCC_BASIS = np.array([[0.0, 0.0, 0.0], [0.0, 0.5, 0.5], [0.5, 0.0, 0.5], [0.5, 0.5, 0.0]])


def c1_cu4() -> Crystal:
    return Crystal(FCC_BASIS.copy(), np.eye(3) * 5.43, np.full(4, 29, np.int64))


def fcc_supercell(a: float, reps: int, sigma: float = 0.0, seed: int | None = None, z: int = 29) -> Crystal:
    """ASE ``Atoms.repeat`` order: cell (m0, m1, m2) with m2 fastest, then the basis."""
    cells = np.array([(m0, m1, m2) for m0 in range(reps) for m1 in range(reps) for m2 in range(reps)], float)
    frac = ((cells[:, None, :] + FCC_BASIS[None, :, :]) / reps).reshape(-1, 3)
    lattice = np.eye(3) * (a * reps)
    if sigma > 0:
        rng = np.random.default_rng(seed)
        cart = frac @ lattice + rng.normal(0.0, sigma, size=frac.shape)
        frac = cart @ np.linalg.inv(lattice)
    return Crystal(frac, lattice, np.full(len(frac), z, np.int64))


def c3_cu864() -> Crystal:
    return fcc_supercell(3.61, 6, sigma=0.05, seed=2)


def _rsa_cubic(n: int, box: float, dmin: float, rng: np.random.Generator, max_tries: int = 200_000_000):
    """Periodic random sequential addition in a cubic box using a cell grid."""
    ncell = max(1, int(box // dmin))
    cs = box / ncell
    grid: dict[tuple, list[int]] = {}
    pos = np.empty((n, 3))
    placed = 0
    tries = 0
    d2min = dmin * dmin
    while placed < n:
        tries += 1
        if tries > max_tries:
            raise RuntimeError("random sequential addition did not converge")
        p = rng.random(3) * box
        ci = (p // cs).astype(int) % ncell
        ok = True
        for dx in (-1, 0, 1):
            for dy in (-1, 0, 1):
                for dz in (-1, 0, 1):
                    key = ((ci[0] + dx) % ncell, (ci[1] + dy) % ncell, (ci[2] + dz) % ncell)
                    for j in grid.get(key, ()):
                        d = pos[j] - p
                        d -= box * np.round(d / box)
                        if d @ d < d2min:
                            ok = False
                            break
                    if not ok:
                        break
                if not ok:
                    break
            if not ok:
                break
        if ok:
            pos[placed] = p
            grid.setdefault((int(ci[0]), int(ci[1]), int(ci[2])), []).append(placed)
            placed += 1
    return pos


def c2_rsa4096() -> Crystal:
    n = 4096
    box = (n / 0.085) ** (1.0 / 3.0)
    pos = _rsa_cubic(n, box, 1.8, np.random.default_rng(1))
    lattice = np.eye(3) * box
    return Crystal(pos / box, lattice, np.full(n, 14, np.int64))


def sio2(n_total: int = 32_000, density: float = 2.2, dmin: float = 1.5, seed: int = 4) -> Crystal:
    n_si = int(round(n_total / 3))
    n_o = n_total - n_si
    mass_g = (n_si * 28.0855 + n_o * 15.999) * AMU_G
    box = (mass_g / density * 1e24) ** (1.0 / 3.0)
    rng = np.random.default_rng(seed)
    pos = _rsa_cubic(n_total, box, dmin, rng)
    z = np.array([14] * n_si + [8] * n_o, np.int64)
    z = z[rng.permutation(n_total)]
    return Crystal(pos / box, np.eye(3) * box, z)


def c5_sio2_32k() -> Crystal:
    return sio2(32_000, seed=4)


def _random_lattice(rng: np.random.Generator, volume: float) -> np.ndarray:
    while True:
        al, be, ga = np.radians(rng.uniform(60.0, 120.0, size=3))
        ratios = rng.uniform(0.8, 1.25, size=3)
        ca, cb, cg = np.cos(al), np.cos(be), np.cos(ga)
        metric = 1 - ca * ca - cb * cb - cg * cg + 2 * ca * cb * cg
        if metric <= 0.05:
            continue
        a, b, c = ratios
        # standard triclinic construction (a along x, b in xy plane)
        lat = np.zeros((3, 3))
        lat[0] = [a, 0, 0]
        lat[1] = [b * cg, b * np.sin(ga), 0]
        cx = c * cb
        cy = c * (ca - cb * cg) / np.sin(ga)
        cz = np.sqrt(max(c * c - cx * cx - cy * cy, 1e-12))
        lat[2] = [cx, cy, cz]
        vol = abs(np.linalg.det(lat))
        return lat * (volume / vol) ** (1.0 / 3.0)


def random_cell(rng: np.random.Generator, n: int, dmin: float = 1.5) -> Crystal:
    lat = _random_lattice(rng, n * rng.uniform(10.0, 25.0))
    shifts = np.array([(i, j, k) for i in range(-2, 3) for j in range(-2, 3) for k in range(-2, 3)], float) @ lat
    frac = np.empty((n, 3))
    placed = 0
    tries = 0
    while placed < n:
        tries += 1
        if tries > 100_000:
            raise RuntimeError("random cell packing did not converge")
        f = rng.random(3)
        p = f @ lat
        ok = True
        for j in range(placed + 1):
            q = (frac[j] @ lat) if j < placed else p
            d = (q - p)[None, :] + shifts
            dd = np.einsum("ij,ij->i", d, d)
            if j == placed:
                dd = dd[np.any(shifts != 0, axis=1)]
            if dd.min() < dmin * dmin:
                ok = False
                break
        if ok:
            frac[placed] = f
            placed += 1
    z = rng.integers(1, 95, size=n).astype(np.int64)
    return Crystal(frac, lat, z)


def c4_batch64() -> list[Crystal]:
    rng = np.random.default_rng(3)
    sizes = rng.integers(8, 65, size=64)
    return [random_cell(rng, int(n)) for n in sizes]


CONFIGS = {
    "C1": c1_cu4,
    "C2": c2_rsa4096,
    "C3": c3_cu864,
    "C4": c4_batch64,
    "C5": c5_sio2_32k,
}
