"""Device-resident velocity-Verlet (NVE) for configuration 4.

Mirrors ``TorchLangevin.step`` with friction 0 (src/molfm/interface/ase/
torch_ext/torch_langevin.py:192-283; c1 = dt/2, c2 = 0, no noise) driven by
``ASERunner`` with ``fixcm`` on (ase_runner.py:101,403-404), i.e. with the
``TorchFixCom`` constraint applied on every step to the forces
(torch_constraints.py:78-88), the new positions (:58-67) and the new momenta
(:69-76).  State is float64 positions and momenta (TorchAtoms dtype,
torch_atoms.py:34); the model sees float32 positions
(e2former_calculator.py:165).  Units are ASE's (eV, Angstrom, amu);
1 fs = 0.09822694788464063 ASE time units.

The integrator state is never wrapped, as in the reference.  For a fully
periodic cell the positions handed to the model are wrapped into the cell
through fractional coordinates (a lattice translation per atom, so energy and
forces are unchanged); the neighbour grid is then the cell's bounding box and
the builder needs no bounding-box readback.
"""
from __future__ import annotations

import numpy as np
import torch

FS = 0.09822694788464063          # ase.units.fs
KB = 8.617330337217213e-05        # ase.units.kB  (eV / K)
MASS = {1: 1.008, 6: 12.011, 7: 14.007, 8: 15.999, 16: 32.06}


def masses_for(Z: np.ndarray) -> np.ndarray:
    return np.array([MASS.get(int(z), 12.0) for z in Z], np.float64)


def maxwell_boltzmann(Z, T=300.0, seed=0):
    """Maxwell-Boltzmann velocities with the centre-of-mass momentum removed
    (ASE's distribution followed by the FixCom momentum projection that
    ``TorchAtoms.set_momenta`` applies)."""
    m = masses_for(Z)
    rng = np.random.default_rng(seed)
    v = rng.normal(size=(len(Z), 3)) * np.sqrt(KB * T / m)[:, None]
    v -= (m[:, None] * v).sum(0) / m.sum()
    return v


def fixcom_forces(f: torch.Tensor, m: torch.Tensor) -> torch.Tensor:
    """F - m (sum m F) / (sum m^2); m is [N, 1]."""
    return f - m * ((m * f).sum(0) / (m * m).sum())


def fixcom_positions(x_old: torch.Tensor, x_new: torch.Tensor, m: torch.Tensor) -> torch.Tensor:
    """Shift x_new so that its mass-weighted centre equals that of x_old."""
    ms = m.sum()
    return x_new + ((m * x_old).sum(0) / ms - (m * x_new).sum(0) / ms)


def fixcom_momenta(p: torch.Tensor, m: torch.Tensor) -> torch.Tensor:
    """p - m (sum p) / (sum m)."""
    return p - m * (p.sum(0) / m.sum())


def wrappable(cell: np.ndarray, pbc) -> bool:
    cell = np.asarray(cell, np.float64).reshape(3, 3)
    return bool(np.all(np.asarray(pbc).reshape(3))) and abs(np.linalg.det(cell)) > 1e-9


def wrap_positions(x: torch.Tensor, cell) -> torch.Tensor:
    """Positions mapped into the cell spanned by the rows of ``cell`` through
    fractional coordinates (frac - floor(frac)): each atom moves by a lattice
    vector, so every periodic pair distance is unchanged (triclinic cells
    included)."""
    A = torch.as_tensor(np.asarray(cell, np.float64).reshape(3, 3), device=x.device, dtype=torch.float64)
    frac = x.to(torch.float64) @ torch.linalg.inv(A)
    return (frac - torch.floor(frac)) @ A


def cell_bounding_box(cell) -> np.ndarray:
    """(lo, hi) [2, 3] of the parallelepiped spanned by the rows of ``cell``."""
    A = np.asarray(cell, np.float64).reshape(3, 3)
    corners = np.array([[a, b, c] for a in (0, 1) for b in (0, 1) for c in (0, 1)], np.float64) @ A
    return np.stack([corners.min(0), corners.max(0)])


class VelocityVerlet:
    """NVE velocity-Verlet over one or more graphs (graphs contiguous in
    ``sysd``); ``fixcm`` applies the FixCom projections to the whole system, as
    the reference does for its one ``TorchAtoms`` object."""

    def __init__(self, model, sysd, device, dt_fs=1.0, T=300.0, seed=0, fixcm=True, wrap=True):
        self.model = model
        self.sys = sysd
        self.dev = device
        self.dt = dt_fs * FS
        self.fixcm = fixcm
        Z = np.asarray(sysd["Z"])
        self.Z = torch.as_tensor(Z, device=device)
        self.m = torch.as_tensor(masses_for(Z), device=device, dtype=torch.float64)[:, None]
        self.x = torch.as_tensor(np.asarray(sysd["pos"], np.float64), device=device)
        self.p = torch.as_tensor(maxwell_boltzmann(Z, T, seed), device=device) * self.m
        self.cells = np.asarray(sysd["cell"], np.float32).reshape(-1, 3, 3)
        self.pbcs = np.asarray(sysd["pbc"], bool).reshape(-1, 3)
        self.ptr = np.asarray(sysd["graph_ptr"], np.int64)
        self.wrap = wrap and all(wrappable(c, p) for c, p in zip(self.cells, self.pbcs))
        self.grid_box = None
        if self.wrap:
            bb = np.stack([cell_bounding_box(c) for c in self.cells], axis=1)     # [2, B, 3]
            self.grid_box = bb.astype(np.float32)
        self.f = None
        self.e = None
        self.n_edges = 0
        self.last_nl = None

    @property
    def v(self) -> torch.Tensor:
        return self.p / self.m

    def model_positions(self, x: torch.Tensor) -> torch.Tensor:
        """float32 positions given to the model (wrapped copy for periodic cells)."""
        if not self.wrap:
            return x.float()
        parts = [wrap_positions(x[self.ptr[g]:self.ptr[g + 1]], self.cells[g]) for g in range(len(self.ptr) - 1)]
        return (parts[0] if len(parts) == 1 else torch.cat(parts)).float()

    def forces_at(self, x: torch.Tensor):
        """(energy per graph, raw model forces float64) at positions x."""
        e, f, nl = self.model.energy_forces_flat(self.model_positions(x), self.Z, self.ptr, self.cells, self.pbcs,
                                                 grid_box=self.grid_box)
        self.n_edges = nl.n_edges
        self.last_nl = nl
        return e, f.double()

    def forces(self):
        return self.forces_at(self.x)

    def kinetic(self):
        return 0.5 * float((self.p * self.p / self.m).sum())

    def step(self):
        if self.f is None:
            self.e, self.f = self.forces()
        m, dt, c1 = self.m, self.dt, 0.5 * self.dt
        f = fixcom_forces(self.f, m) if self.fixcm else self.f
        x_new = self.x + dt * (self.p / m + c1 * f / m)
        if self.fixcm:
            x_new = fixcom_positions(self.x, x_new, m)
        e_new, f_new = self.forces_at(x_new)
        fn = fixcom_forces(f_new, m) if self.fixcm else f_new
        p_new = ((x_new - self.x) / dt + c1 * fn / m) * m
        if self.fixcm:
            p_new = fixcom_momenta(p_new, m)
        self.x, self.p, self.e, self.f = x_new, p_new, e_new, f_new
        return self.e
