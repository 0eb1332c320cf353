"""NVE integrator: the oracle step (restated TorchLangevin.step, fr = 0, FixCom)
pinned by closed forms and invariants, and the product integrator
(md.VelocityVerlet) against it with a stand-in force model on the CPU."""
import math

import numpy as np
import pytest
import torch

from oracle import md as omd

FS = 0.09822694788464063
M_HHO = torch.tensor([1.008, 1.008, 15.999], dtype=torch.float64)


def _harmonic(x0, k):
    return lambda x: -k * (x - x0)


def test_harmonic_spring_closed_form():
    """The reference's own integrator check drives 3 atoms (H, H, O) with
    harmonic springs F = -k (x - x0) (torch_langevin.py:294-369, k = 10,
    dt = 0.5 fs).  Without FixCom each coordinate follows velocity-Verlet's
    exact discrete solution x_n - x0 = A cos(n t) + B sin(n t) with
    cos t = 1 - w^2 dt^2 / 2, w^2 = k / m, and v_n = (x_{n+1} - x_n)/dt +
    w^2 dt/2 (x_n - x0).  A full instead of a half kick (c1 = dt), forces
    from the new instead of the old positions in the drift, or a missing
    second kick each break the closed form within the first two steps (each
    mutation was run against this test on the CPU)."""
    k, dt = 10.0, 0.5 * FS
    x0 = torch.tensor([[0.0, 0.0, 0.0], [0.96, 0.0, 0.0], [0.24, 0.93, 0.0]], dtype=torch.float64)
    rng = np.random.default_rng(0)
    x = x0 + torch.as_tensor(rng.normal(scale=0.05, size=(3, 3)))
    v0 = torch.as_tensor(rng.normal(scale=0.02, size=(3, 3)))
    p = v0 * M_HHO[:, None]
    fn = _harmonic(x0, k)
    f = fn(x)
    xs, vs = [x], [v0]
    for _ in range(60):
        x, p, f = omd.nve_step(x, p, M_HHO, f, fn, dt, fixcom=False)
        xs.append(x); vs.append(p / M_HHO[:, None])
    w2 = (k / M_HHO)[:, None]
    th = torch.arccos(1 - w2 * dt * dt / 2)
    a0 = xs[0] - x0
    x1 = xs[0] + v0 * dt - w2 * a0 * dt * dt / 2
    B = (x1 - x0 - a0 * torch.cos(th)) / torch.sin(th)
    for n in range(len(xs)):
        xn = x0 + a0 * torch.cos(n * th) + B * torch.sin(n * th)
        assert float((xs[n] - xn).abs().max()) < 1e-12, n
    for n in range(len(xs) - 1):
        vn = (xs[n + 1] - xs[n]) / dt + w2 * dt / 2 * (xs[n] - x0)
        assert float((vs[n] - vn).abs().max()) < 1e-9, n


def test_fixcom_projections():
    """FixCom (torch_constraints.py:55-88): projected forces have zero
    mass-weighted sum (this fixes the denominator sum m^2: sum m would leave a
    residual for unequal masses), projected momenta sum to zero, the position
    projection keeps the mass-weighted centre, and each projection is
    idempotent."""
    rng = np.random.default_rng(1)
    m = torch.as_tensor(rng.uniform(1.0, 32.0, 7))
    f = torch.as_tensor(rng.normal(size=(7, 3)))
    fp = omd.fixcom_forces(f, m)
    assert float((m[:, None] * fp).sum(0).abs().max()) < 1e-12
    assert torch.allclose(omd.fixcom_forces(fp, m), fp, atol=1e-14)
    p = torch.as_tensor(rng.normal(size=(7, 3)))
    pp = omd.fixcom_momenta(p, m)
    assert float(pp.sum(0).abs().max()) < 1e-12
    x = torch.as_tensor(rng.normal(size=(7, 3)))
    xn = x + torch.as_tensor(rng.normal(size=(7, 3)))
    xa = omd.fixcom_positions(x, xn, m)
    cm = lambda y: (m[:, None] * y).sum(0) / m.sum()
    assert torch.allclose(cm(xa), cm(x), atol=1e-13)
    assert torch.allclose(xa - xn, (cm(x) - cm(xn)).expand_as(xn))


def test_fixcom_trajectory_invariants():
    """With FixCom on and unequal masses under an external (non-momentum-
    conserving) force, the mass-weighted centre stays where it started and the
    total momentum stays zero at every step; for pair forces (Newton's third
    law) with equal masses the projections are no-ops and the trajectory equals
    the unconstrained one."""
    rng = np.random.default_rng(2)
    m = torch.as_tensor(rng.uniform(1.0, 16.0, 5))
    x = torch.as_tensor(rng.normal(size=(5, 3)))
    p = omd.fixcom_momenta(torch.as_tensor(rng.normal(scale=0.3, size=(5, 3))), m)
    ext = torch.as_tensor(rng.normal(size=(5, 3)))
    fn = lambda y: -2.0 * y + ext
    f = fn(x)
    cm0 = (m[:, None] * x).sum(0) / m.sum()
    for _ in range(20):
        x, p, f = omd.nve_step(x, p, m, f, fn, 0.5, fixcom=True)
        assert torch.allclose((m[:, None] * x).sum(0) / m.sum(), cm0, atol=1e-12)
        assert float(p.sum(0).abs().max()) < 1e-12

    me = torch.full((5,), 4.0, dtype=torch.float64)

    def pair(y):
        d = y[:, None, :] - y[None, :, :]
        return -(d * 1.5).sum(1)

    xa = xb = torch.as_tensor(rng.normal(size=(5, 3)))
    pa = pb = omd.fixcom_momenta(torch.as_tensor(rng.normal(size=(5, 3))), me)
    fa = fb = pair(xa)
    for _ in range(20):
        xa, pa, fa = omd.nve_step(xa, pa, me, fa, pair, 0.3, fixcom=True)
        xb, pb, fb = omd.nve_step(xb, pb, me, fb, pair, 0.3, fixcom=False)
    assert torch.allclose(xa, xb, atol=1e-12) and torch.allclose(pa, pb, atol=1e-12)


class _SpringModel:
    """Stand-in for MolfmAtomic.energy_forces_flat: harmonic springs to x0
    (float32 positions in, like the model)."""

    def __init__(self, x0, k=3.0):
        self.x0, self.k = x0, k

    def energy_forces_flat(self, pos, Z, graph_ptr, cell, pbc, grid_box=None):
        d = pos.double() - self.x0
        e = 0.5 * self.k * (d * d).sum().reshape(1)
        return e.float(), (-self.k * d).float(), type("NL", (), {"n_edges": 0})()


@pytest.mark.parametrize("fixcm", [True, False])
def test_product_integrator_matches_oracle_step(pkg, fixcm):
    """md.VelocityVerlet against oracle.md.nve_step for 10 steps with the same
    force function (non-periodic: the model sees the unwrapped positions)."""
    from ubio_molfm_amd import md
    rng = np.random.default_rng(3)
    Z = np.array([8, 1, 1, 6, 7, 16])
    pos = rng.normal(scale=2.0, size=(6, 3))
    sysd = dict(pos=pos.astype(np.float32), Z=Z, graph_ptr=np.array([0, 6]), cell=np.zeros((1, 3, 3), np.float32),
                pbc=np.zeros((1, 3), bool))
    x0 = torch.as_tensor(pos + 0.1)
    integ = md.VelocityVerlet(_SpringModel(x0), sysd, torch.device("cpu"), dt_fs=1.0, T=300.0, seed=0, fixcm=fixcm)
    m = integ.m[:, 0]
    x, p = integ.x.clone(), integ.p.clone()
    assert float(p.sum(0).abs().max()) < 1e-12          # MB velocities with the COM momentum removed
    fn = lambda y: integ.forces_at(y)[1]
    f = fn(x)
    for _ in range(10):
        integ.step()
        x, p, f = omd.nve_step(x, p, m, f, fn, integ.dt, fixcom=fixcm)
        assert torch.allclose(integ.x, x, rtol=0, atol=1e-12)
        assert torch.allclose(integ.p, p, rtol=0, atol=1e-12)


def test_wrap_keeps_minimum_image_distances(pkg):
    """Wrapping into a triclinic cell moves every atom by a lattice vector:
    all periodic pair distances (minimum over images) are unchanged."""
    from ubio_molfm_amd import md
    cell = np.array([[9.0, 0.0, 0.0], [3.1, 8.2, 0.0], [-2.0, 1.7, 7.5]])
    rng = np.random.default_rng(4)
    x = torch.as_tensor(rng.uniform(-15, 25, size=(12, 3)))
    xw = md.wrap_positions(x, cell)
    A = torch.as_tensor(cell)
    frac = xw @ torch.linalg.inv(A)
    assert float(frac.min()) >= 0.0 and float(frac.max()) < 1.0
    shifts = torch.as_tensor([[a, b, c] for a in range(-8, 9) for b in range(-8, 9) for c in range(-8, 9)],
                             dtype=torch.float64) @ A

    def min_image(y):
        d = y[:, None, None, :] - y[None, :, None, :] + shifts[None, None]
        return d.norm(dim=-1).min(-1).values
    assert torch.allclose(min_image(x), min_image(xw), atol=1e-9)
    lo, hi = md.cell_bounding_box(cell)
    assert np.all(xw.numpy() >= lo - 1e-9) and np.all(xw.numpy() <= hi + 1e-9)
