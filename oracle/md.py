"""CPU restatement of the reference NVE integrator (test infrastructure only).

``nve_step`` follows ``TorchLangevin.step`` with friction 0
(src/molfm/interface/ase/torch_ext/torch_langevin.py:192-283): with fr = 0 the
coefficients are c1 = dt/2, c2 = 0, sigma = 0 (:158-175), so the two cores
(:21-56) reduce to velocity-Verlet with the velocity reconstructed from the
actual (constrained) displacement.  ``ASERunner`` attaches a ``FixCom``
constraint when ``fixcm`` is on (its default; ase_runner.py:101,403-404), and
``TorchAtoms`` then applies ``TorchFixCom`` (torch_constraints.py:55-97) in
three places of every step:

* ``get_forces(md=True)`` -> ``redistribute_forces_md`` = ``adjust_forces``:
  F - m * (sum m F) / (sum m^2)  (torch_atoms.py:475-508);
* ``set_positions(x_new)`` -> ``adjust_positions``: x_new + (cm(x) - cm(x_new))
  with cm the mass-weighted centre (torch_atoms.py:431-438);
* ``set_momenta(p)`` -> ``adjust_momenta``: p - m * (sum p) / (sum m)
  (torch_atoms.py:460-472).

State is float64 (TorchAtoms dtype, torch_atoms.py:34).  Units are ASE's.
"""
from __future__ import annotations

from typing import Callable, Tuple

import torch


def fixcom_forces(f: torch.Tensor, m: torch.Tensor) -> torch.Tensor:
    """torch_constraints.py:78-88 (m is [N])."""
    lmd = (m[:, None] * f).sum(0) / m.square().sum()
    return f - m[:, None] * lmd


def fixcom_positions(x_old: torch.Tensor, x_new: torch.Tensor, m: torch.Tensor) -> torch.Tensor:
    """torch_constraints.py:58-67."""
    ms = m.sum()
    old_cm = (m[:, None] * x_old).sum(0) / ms
    new_cm = (m[:, None] * x_new).sum(0) / ms
    return x_new + (old_cm - new_cm)


def fixcom_momenta(p: torch.Tensor, m: torch.Tensor) -> torch.Tensor:
    """torch_constraints.py:69-76."""
    return p - m[:, None] * (p.sum(0) / m.sum())


def nve_step(x: torch.Tensor, p: torch.Tensor, m: torch.Tensor, f: torch.Tensor,
             forces_fn: Callable[[torch.Tensor], torch.Tensor], dt: float,
             fixcom: bool = True) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """One step from (x, p) with the raw forces ``f`` at x; returns (x', p', f')
    where f' are the raw forces at x' (the caller keeps them for the next step,
    as the reference's calculator cache does)."""
    c1 = dt / 2.0                                          # torch_langevin.py:171 with fr = 0
    minv = 1.0 / m[:, None]
    fx = fixcom_forces(f, m) if fixcom else f
    v = p * minv                                           # torch_atoms.py:443-448
    v_half = v + c1 * fx * minv                            # :33 (c2 = 0, no noise)
    x_new = x + dt * v_half                                # :34
    if fixcom:
        x_new = fixcom_positions(x, x_new, m)
    f_new = forces_fn(x_new)
    fnx = fixcom_forces(f_new, m) if fixcom else f_new
    v = (x_new - x) / dt                                   # :52 (rnd_pos = 0)
    v = v + c1 * fnx * minv                                # :53
    p_new = v * m[:, None]                                 # :54
    if fixcom:
        p_new = fixcom_momenta(p_new, m)
    return x_new, p_new, f_new
