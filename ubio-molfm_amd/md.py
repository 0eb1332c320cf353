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

No host readback per step: after the first (exact) neighbour build, each step
builds its list into arrays sized from the previous count plus a margin (the
capacity build of ``neighbors.build_neighbors``).  The build's counters (edge
count, longest row, atom outside the grid box, overflow) are copied to pinned
host memory without waiting, and checked when the next step starts, by which
time the device has long finished that build; a step whose list overflowed is
recomputed from its saved starting state with an exact build (bitwise the same
result, since the capacity only pads the edge arrays).  ``sync()`` resolves the
last step; until then the state after ``step()`` is provisional.

With ``graph=True`` the step (capacity neighbour build, energy, autograd forces,
FixCom and the Verlet updates: about 300 kernels) is captured once, after one
eager step, as a HIP graph that advances a static state in place, after copying it to a backup
inside the same graph; each step is then one graph launch.  The build's counters
land in a static pinned buffer and are checked before the next launch (waiting
for the previous step only); an overflowing step is redone from the backup with
an exact build and the graph is captured again for the new capacity.  The
replayed kernels are those of the eager step, so the trajectory is bitwise the
same.  ``evaluate_only=True`` makes a step an energy + force evaluation at fixed
positions (the benchmark's eval mode), graphed the same way.
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


# The projections below are written as few fused elementwise operations, with
# the constant mass sums passed in as numbers when known, so that a step
# launches about 25 small kernels instead of about 45.  (Mass-weighted sums as
# [1, N] x [N, 3] float64 GEMMs were measured far slower: the library runs such
# a shape's whole K loop in one tile.)

def fixcom_forces(f: torch.Tensor, m: torch.Tensor, mm: float = None) -> torch.Tensor:
    """F - m (sum m F) / (sum m^2); m is [N, 1], mm = sum m^2 when known."""
    mm = float((m * m).sum()) if mm is None else mm
    return torch.addcmul(f, m, (m * f).sum(0), value=-1.0 / mm)


def fixcom_positions(x_old: torch.Tensor, x_new: torch.Tensor, m: torch.Tensor, ms: float = None) -> torch.Tensor:
    """Shift x_new so that its mass-weighted centre equals that of x_old
    (ms = sum m when known)."""
    ms = float(m.sum()) if ms is None else ms
    return torch.add(x_new, (m * (x_old - x_new)).sum(0), alpha=1.0 / ms)


def fixcom_momenta(p: torch.Tensor, m: torch.Tensor, ms: float = None) -> torch.Tensor:
    """p - m (sum p) / (sum m)."""
    ms = float(m.sum()) if ms is None else ms
    return torch.addcmul(p, m, p.sum(0), value=-1.0 / ms)


def wrappable(cell: np.ndarray, pbc) -> bool:
    cell = np.asarray(cell, np.float64).reshape(3, 3)
    return bool(np.all(np.asarray(pbc).reshape(3))) and abs(np.linalg.det(cell)) > 1e-9


def cell_matrices(cell, device):
    """(A, A^-1) float64 on the device for the cell spanned by the rows of ``cell``
    (the inverse taken on the host: no device solver and no host sync)."""
    A = np.asarray(cell, np.float64).reshape(3, 3)
    return (torch.as_tensor(A, device=device), torch.as_tensor(np.linalg.inv(A), device=device))


def wrap_positions(x: torch.Tensor, cell=None, mats=None) -> torch.Tensor:
    """Positions mapped into the cell spanned by the rows of ``cell`` through
    fractional coordinates (frac - floor(frac)): each atom moves by a lattice
    vector, so every periodic pair distance is unchanged (triclinic cells
    included).  mats: the cell's ``cell_matrices``, if already on the device."""
    A, Ainv = cell_matrices(cell, x.device) if mats is None else mats
    frac = x.to(torch.float64) @ Ainv
    return torch.remainder(frac, 1.0) @ A          # frac - floor(frac), one kernel


def cell_bounding_box(cell) -> np.ndarray:
    """(lo, hi) [2, 3] of the parallelepiped spanned by the rows of ``cell``."""
    A = np.asarray(cell, np.float64).reshape(3, 3)
    corners = np.array([[a, b, c] for a in (0, 1) for b in (0, 1) for c in (0, 1)], np.float64) @ A
    return np.stack([corners.min(0), corners.max(0)])


class VelocityVerlet:
    """NVE velocity-Verlet over one or more graphs (graphs contiguous in
    ``sysd``); ``fixcm`` applies the FixCom projections to the whole system, as
    the reference does for its one ``TorchAtoms`` object."""

    # capacity of the next build: the last count plus this fraction and a fixed margin
    CAP_FRAC, CAP_EDGES, CAP_ROW = 0.04, 4096, 64

    def __init__(self, model, sysd, device, dt_fs=1.0, T=300.0, seed=0, fixcm=True, wrap=True, lagged=True,
                 graph=False, evaluate_only=False):
        self.model = model
        self.sys = sysd
        self.dev = device
        self.dt = dt_fs * FS
        self.fixcm = fixcm
        Z = np.asarray(sysd["Z"])
        self.Z = torch.as_tensor(Z, device=device)
        mnp = masses_for(Z)
        self.m = torch.as_tensor(mnp, device=device, dtype=torch.float64)[:, None]
        self.inv_m = 1.0 / self.m
        self.msum, self.mmsum = float(mnp.sum()), float((mnp * mnp).sum())
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
            self.cell_mats = [cell_matrices(c, device) for c in self.cells]
        self.f = None
        self.e = None
        self.n_edges = 0
        self.last_nl = None
        # the capacity build needs the cell's grid box (wrapped positions)
        self.lagged = lagged and self.wrap and device.type == "cuda"
        self.capacity = None          # (edges, longest row) of the next capacity build
        self.pending = None           # (pinned counters, event, state before the step) of the last one
        self.edge_counts = []         # edges of every step's build, in order (complete after sync())
        self.redone = 0               # steps recomputed after an overflowing capacity build
        self.evaluate_only = evaluate_only
        # HIP-graph mode: capacity builds only; the first WARM_STEPS steps run eagerly
        self.use_graph = graph and self.lagged
        self.graph = None             # (CUDAGraph, capacity) of the captured step
        self._gstate = self._gbackup = self._gstats = self._gevent = None
        self.graph_launches = 0
        self.captures = 0
        self._eager_steps = 0

    @property
    def v(self) -> torch.Tensor:
        return self.p / self.m

    def model_positions(self, x: torch.Tensor) -> torch.Tensor:
        """float32 positions given to the model (wrapped copy for periodic cells)."""
        if not self.wrap:
            return x.float()
        parts = [wrap_positions(x[self.ptr[g]:self.ptr[g + 1]], mats=self.cell_mats[g]) for g in range(len(self.ptr) - 1)]
        return (parts[0] if len(parts) == 1 else torch.cat(parts)).float()

    def forces_at(self, x: torch.Tensor, capacity=None):
        """(energy per graph, raw model forces float64) at positions x; with
        ``capacity`` the neighbour list is a capacity build whose counters the
        caller checks (``self.last_nl.stats``)."""
        kw = {} if capacity is None else {"nbr_capacity": capacity}
        e, f, nl = self.model.energy_forces_flat(self.model_positions(x), self.Z, self.ptr, self.cells, self.pbcs,
                                                 grid_box=self.grid_box, **kw)
        if capacity is None:
            self.n_edges = nl.n_edges
            self._size_from(nl.n_edges, getattr(nl, "max_row", 0))
        self.last_nl = nl
        return e, f.double()

    def _size_from(self, n_edges: int, longest: int):
        self.capacity = (int(n_edges * (1 + self.CAP_FRAC)) + self.CAP_EDGES, min(longest + self.CAP_ROW, 4096))

    def _resolve(self):
        """Check the last capacity build (waits for that build only, not the step)."""
        if self.pending is None:
            return
        host, ev, state = self.pending
        self.pending = None
        ev.synchronize()
        E, longest, outside, overflow = (int(v) for v in host.tolist())
        if outside or overflow:
            # recompute the step from its starting state with an exact build
            self.x, self.p, self.e, self.f = state
            self.redone += 1
            self._advance(None)
            return
        self.n_edges = E
        self.edge_counts.append(E)
        if E > self.capacity[0] - self.CAP_EDGES // 2 or longest > self.capacity[1] - self.CAP_ROW // 2:
            self._size_from(E, longest)

    def sync(self):
        """Resolve the last step (after it the state is final)."""
        self._resolve()
        self._resolve_graph()

    def forces(self):
        return self.forces_at(self.x)

    def kinetic(self):
        return 0.5 * float((self.p * self.p / self.m).sum())

    WARM_STEPS = 1                    # eager steps before the graph is captured

    def step(self):
        if self.use_graph and self._eager_steps >= self.WARM_STEPS:
            return self._graph_step()
        self._resolve()
        if self.f is None:
            self.e, self.f = self.forces()
        self._advance(self.capacity if self.lagged else None)
        self._eager_steps += 1
        return self.e

    def _verlet(self, x, p, f, capacity):
        """(x', p', e', f') of one step from (x, p, f), fresh tensors: the NVE
        velocity-Verlet update with FixCom, or with ``evaluate_only`` the energy and
        forces at x (x, p returned as they are)."""
        if self.evaluate_only:
            e_new, f_new = self.forces_at(x, capacity)
            return x, p, e_new, f_new
        m, dt, c1 = self.m, self.dt, 0.5 * self.dt
        fc = fixcom_forces(f, m, self.mmsum) if self.fixcm else f
        # x + dt (p / m + c1 f / m)
        x_new = torch.addcmul(x, self.inv_m, p, value=dt).addcmul_(self.inv_m, fc, value=dt * c1)
        if self.fixcm:
            x_new = fixcom_positions(x, x_new, m, self.msum)
        e_new, f_new = self.forces_at(x_new, capacity)
        fn = fixcom_forces(f_new, m, self.mmsum) if self.fixcm else f_new
        # ((x_new - x) / dt + c1 fn / m) m
        p_new = torch.addcmul(fn * c1, x_new - x, m, value=1.0 / dt)
        if self.fixcm:
            p_new = fixcom_momenta(p_new, m, self.msum)
        return x_new, p_new, e_new, f_new

    def _advance(self, capacity):
        state = (self.x, self.p, self.e, self.f)
        x_new, p_new, e_new, f_new = self._verlet(self.x, self.p, self.f, capacity)
        if capacity is not None:
            self.pending = (self.last_nl.stats_host, self.last_nl.stats_event, state)
        else:
            self.edge_counts.append(self.n_edges)
        self.x, self.p, self.e, self.f = x_new, p_new, e_new, f_new

    # -- HIP graph of one step ------------------------------------------------------
    def _capture(self):
        """Capture one step at the current capacity: the graph copies the static
        state to the backup, runs the step (capacity build, counters copied to the
        static pinned buffer) and writes the new state over the static one.  Capture
        records the kernels without running them."""
        self.graph = None
        state = tuple(t.clone() for t in (self.x, self.p, self.e, self.f))
        backup = tuple(torch.empty_like(t) for t in state)
        stats = torch.zeros(4, dtype=torch.int32, pin_memory=True)
        cap = (self.capacity[0], self.capacity[1], stats)
        torch.cuda.synchronize(self.dev)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for b, t in zip(backup, state):
                b.copy_(t)
            x, p, e, f = state
            new = self._verlet(x, p, f, cap)
            for t, n in zip(state, new):
                if n is not t:
                    t.copy_(n)
        self.graph = (g, self.capacity)
        self._gstate, self._gbackup, self._gstats = state, backup, stats
        self.x, self.p, self.e, self.f = state
        self.captures += 1

    def _graph_step(self):
        self._resolve()
        self._resolve_graph()
        if self.graph is None or self.graph[1] != self.capacity:
            self._capture()
        self.graph[0].replay()
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.dev))
        self._gevent = ev
        self.graph_launches += 1
        return self.e

    def _resolve_graph(self):
        """Check the last graph launch's neighbour counters (waits for that launch);
        redo an overflowing step from the backup with an exact build."""
        ev = self._gevent
        if ev is None:
            return
        self._gevent = None
        ev.synchronize()
        E, longest, outside, overflow = (int(v) for v in self._gstats.tolist())
        if outside or overflow:
            state = self._gstate
            for t, b in zip(state, self._gbackup):
                t.copy_(b)
            self.redone += 1
            x, p, e, f = state
            new = self._verlet(x, p, f, None)            # exact build: sets n_edges and the capacity
            for t, n in zip(state, new):
                if n is not t:
                    t.copy_(n)
            self.edge_counts.append(self.n_edges)
            return
        self.n_edges = E
        self.edge_counts.append(E)
        if E > self.capacity[0] - self.CAP_EDGES // 2 or longest > self.capacity[1] - self.CAP_ROW // 2:
            self._size_from(E, longest)                    # captured again at the next step
