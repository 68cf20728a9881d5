"""Molecular dynamics on the GPU with MatRIS forces.

Reference: matris/applications/md.py:31-330 (MolecularDynamics), which wraps ASE's
VelocityVerlet (NVE) and NVTBerendsen (NVT, thermostat "Berendsen*") integrators around
MatRISCalculator.  ASE is not part of this build, so the two integrators are restated
from their published methods and run with every per-atom array resident on the device:

  velocity Verlet (Swope, Andersen, Berendsen & Wilson, J. Chem. Phys. 76, 637 (1982)):
      v += dt/2 a(x);  x += dt v;  a = F(x)/m;  v += dt/2 a
  Berendsen weak coupling (Berendsen et al., J. Chem. Phys. 81, 3684 (1984)), applied to
  the velocities before each Verlet step:
      lambda = sqrt(1 + dt/tau (T0/T - 1)), clamped to [0.9, 1.1]
  with the kinetic temperature T = 2 KE / (3 N k_B).

Each step rebuilds the radius graph and line graph on the GPU (GraphConverter) from the
current positions and evaluates MatRIS (task "ef" plus whatever `task` asks for).
Units: positions in Angstrom, time in fs, velocities in Angstrom/fs, masses in amu,
energies in eV.
"""
from __future__ import annotations

import math
import time

import numpy as np
import torch

# Standard atomic weights (amu) for Z = 1..94 (IUPAC conventional / abridged values;
# the mass number of the longest-lived isotope for elements without a standard weight).
ATOMIC_MASSES = np.array([
    1.008, 4.0026, 6.94, 9.0122, 10.81, 12.011, 14.007, 15.999, 18.998, 20.180,
    22.990, 24.305, 26.982, 28.085, 30.974, 32.06, 35.45, 39.948, 39.098, 40.078,
    44.956, 47.867, 50.942, 51.996, 54.938, 55.845, 58.933, 58.693, 63.546, 65.38,
    69.723, 72.630, 74.922, 78.971, 79.904, 83.798, 85.468, 87.62, 88.906, 91.224,
    92.906, 95.95, 97.0, 101.07, 102.91, 106.42, 107.87, 112.41, 114.82, 118.71,
    121.76, 127.60, 126.90, 131.29, 132.91, 137.33, 138.91, 140.12, 140.91, 144.24,
    145.0, 150.36, 151.96, 157.25, 158.93, 162.50, 164.93, 167.26, 168.93, 173.05,
    174.97, 178.49, 180.95, 183.84, 186.21, 190.23, 192.22, 195.08, 196.97, 200.59,
    204.38, 207.2, 208.98, 209.0, 210.0, 222.0, 223.0, 226.0, 227.0, 232.04,
    231.04, 238.03, 237.0, 244.0])

KB_EV = 8.617333262e-5            # Boltzmann constant, eV/K
AMU_A2_FS2_EV = 103.642691        # 1 amu * (Angstrom/fs)^2 in eV
FORCE_TO_ACC = 1.0 / AMU_A2_FS2_EV  # (eV/Angstrom)/amu -> Angstrom/fs^2


def _detached(v):
    """Results without the autograd graph of the forward (tensors or lists of tensors)."""
    if isinstance(v, torch.Tensor):
        return v.detach()
    if isinstance(v, (list, tuple)):
        return type(v)(t.detach() if isinstance(t, torch.Tensor) else t for t in v)
    return v


class MolecularDynamics:
    """GPU molecular dynamics with the reference's constructor keywords (md.py:34-54).

    atoms: (frac [n,3], lattice [3,3] rows, Z [n]) arrays, an object with frac / lattice /
    z attributes (matris_amd.workloads.Crystal), or an ASE Atoms when ASE is installed.
    model: a MatRIS instance (reference names such as "matris_10m_oam" need a local
    checkpoint, see MatRIS.load).  Supported: ensemble "nve", or "nvt" with a
    "Berendsen*" thermostat; the other reference choices (Nose-Hoover, NPT) rely on ASE
    and raise NotImplementedError.
    """

    def __init__(self, atoms, model="matris_10m_oam", ensemble: str = "nvt",
                 thermostat: str = "Berendsen_inhomogeneous", temperature: float = 300,
                 starting_temperature: float | None = None, timestep: float = 2.0, pressure: float = 1.01325e-4,
                 taut: float | None = None, taup: float | None = None, bulk_modulus: float | None = None,
                 trajectory=None, logfile: str | None = None, loginterval: int = 1,
                 crystal_feas_logfile: str | None = None, append_trajectory: bool = False, task: str = "efs",
                 device: str | None = None, seed: int | None = None, skin: float = 0.0):
        from ..graph.converter import _structure_arrays
        from ..model.model import MatRIS
        self.ensemble, self.thermostat = ensemble.lower(), thermostat
        if self.ensemble not in ("nve", "nvt") or (self.ensemble == "nvt"
                                                    and not thermostat.lower().startswith("berendsen")):
            raise NotImplementedError(f"ensemble={ensemble!r} thermostat={thermostat!r} needs ASE; "
                                      "this build runs 'nve' and 'nvt' with a Berendsen thermostat")
        if isinstance(model, str):
            model = MatRIS.load(model, device=device)
        self.model = model
        self.device = torch.device(device) if device is not None else next(model.parameters()).device
        if self.device.type != "cuda":
            raise RuntimeError("MolecularDynamics runs on the ROCm device only")
        frac, lat, z, _ = _structure_arrays(atoms)
        self.z = np.asarray(z, np.int64)
        self.n = len(self.z)
        self.lattice = np.asarray(lat, np.float64)
        self._lat_t = torch.as_tensor(self.lattice, device=self.device)
        self._inv_lat_t = torch.linalg.inv(self._lat_t)
        self.pos = torch.as_tensor(np.asarray(frac, np.float64) @ self.lattice, device=self.device)
        self.masses = torch.as_tensor(ATOMIC_MASSES[self.z - 1], device=self.device)
        self.vel = torch.zeros_like(self.pos)
        momenta = getattr(atoms, "get_momenta", None)
        if momenta is not None:  # ASE Atoms: momenta in sqrt(amu eV) -> v in Angstrom/fs
            p = torch.as_tensor(np.asarray(momenta(), np.float64), device=self.device)
            self.vel = p / self.masses[:, None] * math.sqrt(1.0 / AMU_A2_FS2_EV)
        if starting_temperature is not None:
            self.maxwell_boltzmann(starting_temperature, seed)
        self.temperature = float(temperature)
        self.timestep = float(timestep)
        self.taut = float(taut) if taut is not None else 100.0 * timestep
        self.task = task if "f" in task else task + "f"
        self.logfile, self.loginterval = logfile, loginterval
        self.trajectory = trajectory
        self.nsteps = 0
        self.timings = {"graph": 0.0, "model": 0.0}
        self.results = None
        self._forces = None
        # skin > 0: Verlet-skin reuse of the neighbour list (graphs identical to a rebuild
        # every step, which is what the reference does and what skin = 0 keeps)
        self.skin = float(skin)
        self._neighbors = None
        if self.skin > 0:
            from ..graph.converter import SkinNeighborList
            self._neighbors = SkinNeighborList(self.lattice, self.model.graph_converter.atom_graph_cutoff, self.skin)

    # --------------------------------------------------------------------------------
    def maxwell_boltzmann(self, temperature: float, seed: int | None = None) -> None:
        """Velocities from the Maxwell-Boltzmann distribution at `temperature`, zero total
        momentum, then rescaled to exactly `temperature` (ASE's MaxwellBoltzmannDistribution
        with force_temp=True followed by Stationary, restated)."""
        rng = np.random.default_rng(seed)
        m = self.masses.cpu().numpy()
        sigma = np.sqrt(KB_EV * temperature / (m * AMU_A2_FS2_EV))
        v = rng.standard_normal((self.n, 3)) * sigma[:, None]
        v -= (m[:, None] * v).sum(0) / m.sum()  # zero total momentum
        self.vel = torch.as_tensor(v, device=self.device)
        t = self.kinetic_temperature()
        if t > 0:
            self.vel *= math.sqrt(temperature / t)

    def kinetic_energy(self) -> float:
        return float(0.5 * (self.masses[:, None] * self.vel * self.vel).sum() * AMU_A2_FS2_EV)

    def kinetic_temperature(self) -> float:
        return 2.0 * self.kinetic_energy() / (3.0 * self.n * KB_EV)

    # --------------------------------------------------------------------------------
    def _evaluate(self):
        """Rebuild the graph on the GPU from the current positions and evaluate the model."""
        t0 = time.perf_counter()
        x = self.pos @ self._inv_lat_t
        frac = x.remainder(1.0).contiguous()  # wrap: the graph is periodic
        nbrs = self._neighbors.update(frac, x, self.pos) if self._neighbors is not None else None
        graph = self.model.graph_converter.from_arrays(None, self.lattice, self.z, frac_device=frac, neighbors=nbrs)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        pred = self.model([graph], task=self.task)
        forces = pred["f"][0].to(torch.float64)
        torch.cuda.synchronize()
        self.timings["graph"] += t1 - t0
        self.timings["model"] += time.perf_counter() - t1
        self.results = {k: _detached(v) for k, v in pred.items()}
        return forces

    def step(self) -> None:
        dt = self.timestep
        if self._forces is None:
            self._forces = self._evaluate()
        if self.ensemble == "nvt":
            t = self.kinetic_temperature()
            lam = math.sqrt(1.0 + dt / self.taut * (self.temperature / t - 1.0)) if t > 0 else 1.0
            self.vel *= min(max(lam, 0.9), 1.1)
        inv_m = (FORCE_TO_ACC / self.masses)[:, None]
        self.vel += 0.5 * dt * self._forces * inv_m
        self.pos += dt * self.vel
        self._forces = self._evaluate()
        self.vel += 0.5 * dt * self._forces * inv_m
        self.nsteps += 1
        if self.logfile and self.nsteps % self.loginterval == 0:
            with open(self.logfile, "a") as fh:
                e = float(self.results["e"][0]) * self.n
                fh.write(f"{self.nsteps * dt:10.3f} fs  Epot {e:14.6f} eV  Ekin {self.kinetic_energy():12.6f} eV  "
                         f"T {self.kinetic_temperature():9.2f} K\n")

    def run(self, steps: int) -> None:
        """Advance `steps` MD steps (md.py:297-310)."""
        for _ in range(int(steps)):
            self.step()

    def get_positions(self) -> np.ndarray:
        return self.pos.cpu().numpy()
