"""A minimal CIF writer: one periodic structure as a P1 cell.

The reference GraphConverter dumps the structure it failed on to `error_graph.cif`
(matris/graph/converter.py:99-106, through pymatgen's `Structure.to`).  pymatgen is not a
dependency here, so the same dump is written from the arrays the converter holds: the cell
as lengths and angles, every site with its element symbol and fractional coordinates, in
the site order of the input.
"""
from __future__ import annotations

import math

import numpy as np

# element symbols by atomic number (index 0 unused)
SYMBOLS = (
    "X H He Li Be B C N O F Ne Na Mg Al Si P S Cl Ar K Ca Sc Ti V Cr Mn Fe Co Ni Cu Zn Ga Ge As Se Br Kr "
    "Rb Sr Y Zr Nb Mo Tc Ru Rh Pd Ag Cd In Sn Sb Te I Xe Cs Ba La Ce Pr Nd Pm Sm Eu Gd Tb Dy Ho Er Tm Yb "
    "Lu Hf Ta W Re Os Ir Pt Au Hg Tl Pb Bi Po At Rn Fr Ra Ac Th Pa U Np Pu Am Cm Bk Cf Es Fm Md No Lr "
    "Rf Db Sg Bh Hs Mt Ds Rg Cn Nh Fl Mc Lv Ts Og").split()


def cell_parameters(lattice) -> tuple[float, float, float, float, float, float]:
    """(a, b, c, alpha, beta, gamma) of a lattice given as rows a, b, c (angles in degrees:
    alpha between b and c, beta between a and c, gamma between a and b)."""
    m = np.asarray(lattice, dtype=np.float64).reshape(3, 3)
    a, b, c = (float(np.linalg.norm(v)) for v in m)

    def angle(u, v):
        cosv = float(np.dot(u, v)) / (float(np.linalg.norm(u)) * float(np.linalg.norm(v)))
        return math.degrees(math.acos(max(-1.0, min(1.0, cosv))))

    return a, b, c, angle(m[1], m[2]), angle(m[0], m[2]), angle(m[0], m[1])


def cif_text(frac, lattice, z, name: str = "error_graph") -> str:
    """The CIF text of one structure: P1 cell, sites in input order."""
    frac = np.asarray(frac, dtype=np.float64).reshape(-1, 3)
    z = np.asarray(z, dtype=np.int64).reshape(-1)
    if frac.shape[0] != z.shape[0]:
        raise ValueError(f"cif_text: {frac.shape[0]} sites but {z.shape[0]} atomic numbers")
    a, b, c, al, be, ga = cell_parameters(lattice)
    m = np.asarray(lattice, dtype=np.float64).reshape(3, 3)
    vol = abs(float(np.linalg.det(m)))
    lines = [f"data_{name}",
             "_symmetry_space_group_name_H-M   'P 1'",
             f"_cell_length_a   {a:.8f}",
             f"_cell_length_b   {b:.8f}",
             f"_cell_length_c   {c:.8f}",
             f"_cell_angle_alpha   {al:.8f}",
             f"_cell_angle_beta   {be:.8f}",
             f"_cell_angle_gamma   {ga:.8f}",
             "_symmetry_Int_Tables_number   1",
             f"_cell_volume   {vol:.8f}",
             f"_cell_formula_units_Z   1",
             "loop_",
             " _symmetry_equiv_pos_site_id",
             " _symmetry_equiv_pos_as_xyz",
             "  1  'x, y, z'",
             "loop_",
             " _atom_site_type_symbol",
             " _atom_site_label",
             " _atom_site_symmetry_multiplicity",
             " _atom_site_fract_x",
             " _atom_site_fract_y",
             " _atom_site_fract_z",
             " _atom_site_occupancy"]
    count: dict[str, int] = {}
    for (x, y, w), zi in zip(frac, z):
        sym = SYMBOLS[int(zi)] if 0 < int(zi) < len(SYMBOLS) else f"Z{int(zi)}"
        count[sym] = count.get(sym, 0) + 1
        lines.append(f"  {sym}  {sym}{count[sym] - 1}  1  {x:.8f}  {y:.8f}  {w:.8f}  1")
    return "\n".join(lines) + "\n"


def write_cif(path: str, frac, lattice, z, name: str = "error_graph") -> None:
    """Write one structure to `path` as a P1 CIF (cif_text)."""
    with open(path, "w") as f:
        f.write(cif_text(frac, lattice, z, name=name))
