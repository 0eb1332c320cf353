"""SO(3) tables for the E2Former-V2 path (product side).

* ``real_cg(l1, l2, l3)``: real-basis coupling tensor C[m1, m2, m3] in e3nn's
  y-polar real basis, un-normalised (``wigner_3j_wonorm``,
  src/molfm/models/e2former/wigner6j/so2_tensor_product.py:29-45).  The SU(2)
  coefficients come from sympy's ``CG``; the real/complex basis change is
  e3nn's ``change_basis_real_to_complex`` including its ``(-1j)**l`` phase.
* ``so2_gather_tables``: ``selected_idx`` / ``CG_weight`` / ``path_norm`` /
  ``l3_sequential`` of ``SO2_TP_givenl2`` (so2_tensor_product.py:182-262).  These
  are state_dict parameters in the reference and are initialised from here.
* ``cartesian_tp_table``: T[t, r, k] such that the reference's node-frame
  first-order product, summed over edges, equals
  sum_e w_e sum_{r,k} T[t, r, k] v_j[r] dvec_e[k]   (t: 20 l3-sequential rows,
  r: 9 irreps rows, k: x, y, z).
* ``wigner_J``: e3nn's J_l (l = 0..11, ``E2former.Jd_list``) from the CG
  recursion D^l = C^T (D^{l-1} (x) D^1) C and J_l = (-1)^l D^l(pi about (x+y)/sqrt2).
"""
from __future__ import annotations

import math
from functools import lru_cache

import numpy as np


@lru_cache(maxsize=None)
def _su2(j1: int, j2: int, j3: int) -> np.ndarray:
    from sympy.physics.quantum.cg import CG
    out = np.zeros((2 * j1 + 1, 2 * j2 + 1, 2 * j3 + 1))
    if not (abs(j1 - j2) <= j3 <= j1 + j2):
        return out
    for m1 in range(-j1, j1 + 1):
        for m2 in range(-j2, j2 + 1):
            m3 = m1 + m2
            if abs(m3) <= j3:
                out[j1 + m1, j2 + m2, j3 + m3] = float(CG(j1, m1, j2, m2, j3, m3).doit())
    return out


def _basis(l: int) -> np.ndarray:
    q = np.zeros((2 * l + 1, 2 * l + 1), dtype=np.complex128)
    r2 = 1.0 / math.sqrt(2.0)
    for m in range(1, l + 1):
        q[l - m, l + m] = r2
        q[l - m, l - m] = -1j * r2
        q[l + m, l + m] = (-1) ** m * r2
        q[l + m, l - m] = 1j * (-1) ** m * r2
    q[l, l] = 1.0
    return ((-1j) ** l) * q


@lru_cache(maxsize=None)
def real_cg(l1: int, l2: int, l3: int) -> np.ndarray:
    C = _su2(l1, l2, l3).astype(np.complex128)
    A, B, Cc = _basis(l1), _basis(l2), np.conj(_basis(l3))
    R = np.einsum("ij,kl,nm,ikn->jlm", A, B, Cc, C)
    if np.abs(R.imag).max() > 1e-9:
        raise ValueError(f"coupling ({l1},{l2},{l3}) is not real")
    return np.ascontiguousarray(R.real)


def so2_gather_tables(lmax: int = 2):
    """(paths, l3_sequential, selected_idx int64[20], CG_weight float32[20],
    path_norm float32[9])."""
    paths = []
    off = 0
    for l1 in range(lmax + 1):
        for l3 in range(abs(l1 - 1), l1 + 2):
            if l3 <= lmax:
                paths.append((l1, l3, off))
        off += 2 * l1 + 1
    paths.sort(key=lambda p: p[1])
    seq = []
    for (_, l3, _) in paths:
        if seq and seq[-1][0] == l3:
            seq[-1][1] += 1
        else:
            seq.append([l3, 1])
    sel, w = [], []
    for (l1, l3, o) in paths:
        sl = real_cg(l1, 1, l3)[:, 1, :]
        for m3 in range(2 * l3 + 1):
            nz = np.flatnonzero(np.abs(sl[:, m3]) > 1e-12)
            if nz.size == 0:
                sel.append(0); w.append(0.0)
            elif nz.size == 1:
                sel.append(o + int(nz[0])); w.append(sl[nz[0], m3])
            else:
                raise ValueError("SO(2) gather needs one m1 per m3")
    cnt = np.concatenate([np.full(2 * l3 + 1, c, np.float32) for l3, c in seq])
    pn = np.float32(1.0) / np.sqrt(cnt)
    return paths, seq, np.array(sel, np.int64), np.array(w, np.float32), pn.astype(np.float32)


def cartesian_tp_table(lmax: int = 2) -> np.ndarray:
    paths, seq, _, _, _ = so2_gather_tables(lmax)
    n_out = sum((2 * l3 + 1) * c for l3, c in seq)
    T = np.zeros((n_out, (lmax + 1) ** 2, 3))
    t0 = 0
    for (l1, l3, o) in paths:
        C = real_cg(l1, 1, l3)
        T[t0:t0 + 2 * l3 + 1, o:o + 2 * l1 + 1, :] = np.transpose(C, (2, 0, 1))
        t0 += 2 * l3 + 1
    return T


def path_rows(lmax: int = 2):
    """Row ranges [t0, t1) of each coupling path in the 20-row layout."""
    paths, _, _, _, _ = so2_gather_tables(lmax)
    out, t0 = [], 0
    for (l1, l3, o) in paths:
        out.append((t0, t0 + 2 * l3 + 1))
        t0 += 2 * l3 + 1
    return out


def wigner_J(lmax: int = 11) -> list:
    Q = np.array([[0.0, 1.0, 0.0], [1.0, 0.0, 0.0], [0.0, 0.0, -1.0]])
    D = [np.ones((1, 1)), Q]
    for l in range(2, lmax + 1):
        C = real_cg(l - 1, 1, l).reshape((2 * l - 1) * 3, 2 * l + 1)
        D.append(C.T @ np.kron(D[l - 1], Q) @ C)
    return [np.ones((1, 1))] + [((-1) ** l) * D[l] for l in range(1, lmax + 1)]


def so2_row_layout(lmax: int = 2, C: int = 256):
    """Placement of the SO(2) product's l3-sequential output rows in the
    l3-grouped layout of the attention kernels' output: the rows of output degree
    l3 hold their cnt coupling paths side by side, a [2 l3 + 1][N][cnt C] block
    (the input of the per-l3 Linear(cnt C -> C) of so2_tensor_product.py:276-290
    as one GEMM operand); the blocks follow in l3 order.  Row t = (l3, path p,
    order m) of channel c of atom i sits at N a[t] + i ld[t] + col[t] + c.
    Returns (a, ld, col, groups) with groups = [(l3, cnt, start / N)]."""
    _, seq, _, _, _ = so2_gather_tables(lmax)
    a, ld, col, groups = [], [], [], []
    start = 0
    for l3, cnt in seq:
        groups.append((l3, cnt, start))
        for p in range(cnt):
            for m in range(2 * l3 + 1):
                a.append(start + m * cnt * C)
                ld.append(cnt * C)
                col.append(p * C)
        start += (2 * l3 + 1) * cnt * C
    return a, ld, col, groups


def render_tp_header(lmax: int = 2) -> str:
    """C++ header with the nonzeros of the Cartesian table (generated)."""
    T = cartesian_tp_table(lmax)
    lines = ["// Generated by ubio-molfm_amd/so3.py:render_tp_header -- do not edit.",
             "// Nonzeros of T[t][r][k]: out[t] = sum T[t][r][k] * v[r] * u[k] (l2 = 1 coupling,",
             "// 9 irreps rows -> 20 l3-sequential rows, u in the (x, y, z) basis).",
             "#pragma once", "namespace e2v2 {",
             f"constexpr int kTpRows = {T.shape[0]};", f"constexpr int kTpIn = {T.shape[1]};"]
    nz = [(t, r, k, T[t, r, k]) for t in range(T.shape[0]) for r in range(T.shape[1]) for k in range(3)
          if abs(T[t, r, k]) > 1e-12]
    lines.append(f"constexpr int kTpNnz = {len(nz)};")
    lines.append("struct TpEntry { int t, r, k; float c; };")
    lines.append("constexpr TpEntry kTp[kTpNnz] = {")
    for (t, r, k, c) in nz:
        lines.append(f"    {{{t}, {r}, {k}, {float(np.float32(c))!r}f}},")
    lines.append("};")
    a, ld, col, _ = so2_row_layout(lmax)
    lines.append("// l3-grouped output rows: row t of channel c of atom i at N kRowA[t] + i kRowLd[t] + kRowCol[t] + c")
    lines.append("constexpr int kRowA[kTpRows] = {" + ", ".join(str(x) for x in a) + "};")
    lines.append("constexpr int kRowLd[kTpRows] = {" + ", ".join(str(x) for x in ld) + "};")
    lines.append("constexpr int kRowCol[kTpRows] = {" + ", ".join(str(x) for x in col) + "};")
    lines.append("}  // namespace e2v2")
    return "\n".join(lines) + "\n"


if __name__ == "__main__":
    import sys
    sys.stdout.write(render_tp_header())
