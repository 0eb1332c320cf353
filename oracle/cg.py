"""e3nn conventions restated in float64 numpy (oracle; test infrastructure only).

Follows the published algorithm of e3nn (the reference imports it privately:
``src/molfm/models/e2former/wigner6j/so2_tensor_product.py:27``):

* ``su2_clebsch_gordan``      -- Racah formula, e3nn ``_su2_clebsch_gordan``
* ``real_to_complex``         -- e3nn ``change_basis_real_to_complex`` (incl. the
                                 ``(-1j)**l`` phase)
* ``wigner_3j_wonorm``        -- ``so2_tensor_product.py:29-45`` (norm=False)
* ``so2_tables``              -- ``SO2_TP_givenl2.__init__`` ``so2_tensor_product.py:182-262``
* ``wigner_D`` / ``z_rot_mat``-- ``module_utils.py:266-306``
* ``edge_rot_euler_angles``   -- ``module_utils.py:181-221`` (eval mode: gamma=0)

Pins (tests/test_oracle_cg.py):
* sympy's independent CG implementation for the SU(2) coefficients;
* SO(3) equivariance of every real-basis CG against Wigner-D built from the
  reference's own J matrices (``Jd.pt`` l=0..2, committed as a fixture);
* CG column orthonormality (a closed form of the SU(2) coefficients);
* D^1 of the frame angles maps r/|r| onto +y (the SO(2) frame definition);
* J_l generated here by the CG recursion equals ``Jd.pt`` for l = 0..11.
"""
from __future__ import annotations

import math
from fractions import Fraction
from math import factorial
from functools import lru_cache

import numpy as np


def _cg_coeff(j1, m1, j2, m2, j3, m3) -> float:
    """<j1 m1 j2 m2 | j3 m3>, Racah's closed form (integer spins only here)."""
    if m3 != m1 + m2:
        return 0.0
    vmin = int(max(-j1 + j2 + m3, -j1 + m1, 0))
    vmax = int(min(j2 + j3 + m1, j3 - j1 + j2, j3 + m3))
    f = lambda n: factorial(round(n))
    pre = (2 * j3 + 1) * Fraction(
        f(j3 + j1 - j2) * f(j3 - j1 + j2) * f(j1 + j2 - j3) * f(j3 + m3) * f(j3 - m3),
        f(j1 + j2 + j3 + 1) * f(j1 - m1) * f(j1 + m1) * f(j2 - m2) * f(j2 + m2),
    )
    s = Fraction(0)
    for v in range(vmin, vmax + 1):
        s += (-1) ** int(v + j2 + m2) * Fraction(
            f(j2 + j3 + m1 - v) * f(j1 - m1 + v),
            f(v) * f(j3 - j1 + j2 - v) * f(j3 + m3 - v) * f(v + j1 - j2 - m3),
        )
    return float(pre) ** 0.5 * float(s)


@lru_cache(maxsize=None)
def su2_clebsch_gordan(j1: int, j2: int, j3: int) -> np.ndarray:
    mat = np.zeros((2 * j1 + 1, 2 * j2 + 1, 2 * j3 + 1))
    if abs(j1 - j2) <= j3 <= j1 + j2:
        for m1 in range(-j1, j1 + 1):
            for m2 in range(-j2, j2 + 1):
                if abs(m1 + m2) <= j3:
                    mat[j1 + m1, j2 + m2, j3 + m1 + m2] = _cg_coeff(j1, m1, j2, m2, j3, m1 + m2)
    return mat


def real_to_complex(l: int) -> np.ndarray:
    q = np.zeros((2 * l + 1, 2 * l + 1), dtype=np.complex128)
    for m in range(-l, 0):
        q[l + m, l + abs(m)] = 1 / 2 ** 0.5
        q[l + m, l - abs(m)] = -1j / 2 ** 0.5
    q[l, l] = 1
    for m in range(1, l + 1):
        q[l + m, l + abs(m)] = (-1) ** m / 2 ** 0.5
        q[l + m, l - abs(m)] = 1j * (-1) ** m / 2 ** 0.5
    return (-1j) ** l * q


@lru_cache(maxsize=None)
def wigner_3j_wonorm(l1: int, l2: int, l3: int) -> np.ndarray:
    """Real-basis coupling tensor C[m1, m2, m3] (un-normalised SU(2) CG)."""
    assert abs(l2 - l3) <= l1 <= l2 + l3
    Q1, Q2, Q3 = real_to_complex(l1), real_to_complex(l2), real_to_complex(l3)
    C = su2_clebsch_gordan(l1, l2, l3).astype(np.complex128)
    C = np.einsum("ij,kl,mn,ikn->jlm", Q1, Q2, np.conj(Q3.T), C)
    assert np.abs(C.imag).max() < 1e-5
    return np.ascontiguousarray(C.real)


def so2_tables(lmax: int = 2, l2: int = 1):
    """(legal paths, l3_sequential, selected_idx, CG_weight, path_norm) of
    ``SO2_TP_givenl2(l1_list=range(lmax+1), l2=1, l3_legal=range(lmax+1))``."""
    legal = []
    start = 0
    for l1 in range(lmax + 1):
        for l3 in range(abs(l1 - l2), l1 + l2 + 1):
            if l3 <= lmax:
                legal.append((l1, l2, l3, start))
        start += 2 * l1 + 1
    legal = sorted(legal, key=lambda x: x[2])  # stable, like sorted(key=l3)
    l3_seq = []
    for ins in legal:
        if l3_seq and l3_seq[-1][0] == ins[2]:
            l3_seq[-1][1] += 1
        else:
            l3_seq.append([ins[2], 1])
    path_norm = np.concatenate([np.ones(2 * l3 + 1) * cnt for l3, cnt in l3_seq])
    path_norm = np.float32(1.0) / np.sqrt(path_norm.astype(np.float32))
    sel, w = [], []
    for (l1, l2_, l3, s) in legal:
        C = wigner_3j_wonorm(l1, l2_, l3)[:, l2_]
        for m3 in range(2 * l3 + 1):
            nz = np.nonzero(C[:, m3])[0]
            if len(nz) == 0:
                sel.append(0)
                w.append(0.0)
            elif len(nz) == 1:
                sel.append(int(nz[0]) + s)
                w.append(C[nz[0], m3])
            else:
                raise ValueError("CG coeff is wrong")
    return legal, l3_seq, np.array(sel, np.int64), np.array(w, np.float32), path_norm


def z_rot_mat(angle: np.ndarray, l: int) -> np.ndarray:
    angle = np.asarray(angle, dtype=np.float64)
    M = np.zeros(angle.shape + (2 * l + 1, 2 * l + 1))
    for i in range(2 * l + 1):
        f = l - i
        M[..., i, 2 * l - i] = np.sin(f * angle)
        M[..., i, i] = np.cos(f * angle)
    return M


def wigner_D(l: int, a, b, c, J) -> np.ndarray:
    return z_rot_mat(a, l) @ J[l] @ z_rot_mat(b, l) @ J[l] @ z_rot_mat(c, l)


def edge_rot_euler_angles(v: np.ndarray):
    """Eval-mode angles of ``init_edge_rot_euler_angles`` (gamma = 0)."""
    v = np.asarray(v, np.float64)
    r = np.linalg.norm(v, axis=-1)
    r = np.where(r < 1e-5, 1.0, r)
    x = v / r[..., None]
    beta = np.arccos(np.clip(x[..., 1], -1.0, 1.0))
    alpha = np.arctan2(x[..., 0], x[..., 2])
    gamma = np.zeros_like(alpha)
    return -gamma, -beta, -alpha


def j_from_cg(lmax: int) -> list:
    """J_l for l = 0..lmax generated from the real CG alone.

    D^1 is the Cartesian matrix in the (x, y, z) basis; D^l is built by the
    CG recursion D^l = C^T (D^{l-1} (x) D^1) C with C = wigner_3j_wonorm(l-1, 1, l)
    (orthonormal columns).  J_l = (-1)^l D^l(Q) with Q the rotation by pi about
    (x+y)/sqrt(2); for l = 1 this is the matrix (x, y, z) -> (-y, -x, z).
    """
    Q = np.array([[0.0, 1.0, 0.0], [1.0, 0.0, 0.0], [0.0, 0.0, -1.0]])
    out = [np.ones((1, 1))]
    D = Q.copy()
    Ds = [np.ones((1, 1)), Q]
    for l in range(2, lmax + 1):
        C = wigner_3j_wonorm(l - 1, 1, l).reshape((2 * l - 1) * 3, 2 * l + 1)
        Dl = C.T @ np.kron(Ds[l - 1], Q) @ C
        Ds.append(Dl)
    for l in range(1, lmax + 1):
        out.append(((-1) ** l) * Ds[l])
    return out


def cartesian_tp_table(lmax: int = 2):
    """T[t, r, k] with out[t] = sum_{r,k} T[t,r,k] v[r] u[k]: the l2=1 coupling of
    node irreps v (rows r over l1 = 0..lmax, 9 rows) with a Cartesian vector u in
    the (x, y, z) basis, output rows t in l3-sequential order (20 rows)."""
    legal, l3_seq, _, _, _ = so2_tables(lmax)
    n_in = (lmax + 1) ** 2
    n_out = sum((2 * l3 + 1) * c for l3, c in l3_seq)
    T = np.zeros((n_out, n_in, 3))
    t0 = 0
    for (l1, l2, l3, s) in legal:
        C = wigner_3j_wonorm(l1, l2, l3)
        T[t0:t0 + 2 * l3 + 1, s:s + 2 * l1 + 1, :] = np.transpose(C, (2, 0, 1))
        t0 += 2 * l3 + 1
    return T
