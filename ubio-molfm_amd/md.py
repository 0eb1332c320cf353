"""Device-resident velocity-Verlet (NVE) for configuration 4.

Mirrors TorchLangevin.step with friction 0 (src/molfm/interface/ase/torch_ext/
torch_langevin.py:192-283): fp64 state (positions, velocities), fp32 model
positions, one energy + force evaluation per step with the neighbour list
rebuilt every step, centre-of-mass momentum removed at start (FixCom,
src/molfm/interface/ase/torch_ext/ase_runner.py:403-404).  Units are ASE's
(eV, Angstrom, amu); 1 fs = 0.09822694788464063 ASE time units.
"""
from __future__ import annotations

import math

import numpy as np
import torch

FS = 0.09822694788464063          # ase.units.fs
KB = 8.617330337217213e-05        # ase.units.kB  (eV / K)
MASS = {1: 1.008, 6: 12.011, 7: 14.007, 8: 15.999, 16: 32.06}


def masses_for(Z: np.ndarray) -> np.ndarray:
    return np.array([MASS.get(int(z), 12.0) for z in Z], np.float64)


def maxwell_boltzmann(Z, T=300.0, seed=0):
    m = masses_for(Z)
    rng = np.random.default_rng(seed)
    v = rng.normal(size=(len(Z), 3)) * np.sqrt(KB * T / m)[:, None]
    v -= (m[:, None] * v).sum(0) / m.sum()          # zero total momentum
    return v


class VelocityVerlet:
    def __init__(self, model, sysd, device, dt_fs=1.0, T=300.0, seed=0, wrap=True):
        self.model = model
        self.sys = sysd
        self.dev = device
        self.dt = dt_fs * FS
        Z = np.asarray(sysd["Z"])
        self.Z = torch.as_tensor(Z, device=device)
        self.m = torch.as_tensor(masses_for(Z), device=device, dtype=torch.float64)[:, None]
        self.x = torch.as_tensor(np.asarray(sysd["pos"], np.float64), device=device)
        self.v = torch.as_tensor(maxwell_boltzmann(Z, T, seed), device=device)
        self.cell = np.asarray(sysd["cell"], np.float32)
        self.wrap = wrap and bool(np.all(sysd["pbc"]))
        self.L = torch.as_tensor(np.diag(self.cell[0]).astype(np.float64), device=device)
        # wrapped positions lie in [0, L): the neighbour grid is the cell (no bounding-box readback)
        ortho = np.count_nonzero(self.cell[0] - np.diag(np.diag(self.cell[0]))) == 0
        self.grid_box = (np.stack([np.zeros(3), np.diag(self.cell[0])])[:, None, :].astype(np.float32)
                         if self.wrap and ortho else None)
        self.f = None
        self.e = None
        self.n_edges = 0

    def _wrap(self):
        if self.wrap:
            self.x = torch.remainder(self.x, self.L)

    def forces(self):
        e, f, nl = self.model.energy_forces_flat(self.x.float(), self.Z, self.sys["graph_ptr"], self.cell,
                                                 self.sys["pbc"], grid_box=self.grid_box)
        self.n_edges = nl.n_edges
        return e, f.double()

    def kinetic(self):
        return 0.5 * float((self.m * self.v * self.v).sum())

    def step(self):
        if self.f is None:
            self.e, self.f = self.forces()
        a = self.f / self.m
        self.x = self.x + self.v * self.dt + 0.5 * a * self.dt * self.dt
        self._wrap()
        e_new, f_new = self.forces()
        self.v = self.v + 0.5 * (a + f_new / self.m) * self.dt
        self.e, self.f = e_new, f_new
        return self.e
