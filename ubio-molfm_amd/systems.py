"""Seeded synthetic workloads for the five benchmark configurations.

All generators use ``numpy.random.default_rng(seed)`` and return a dict with
flattened real atoms: ``pos`` [N,3] float32, ``Z`` [N] int64, ``graph_ptr``
[B+1], ``cell`` [B,3,3] float32, ``pbc`` [B,3] bool, ``name``.
``to_padded`` turns that into the reference's padded batch
(``src/molfm/data/collator.py:25-52``: pos [B,L,3], atomic_numbers [B,L],
atom_masks [B,L], cell, pbc).
"""
from __future__ import annotations

import math
import numpy as np

AMU_G = 1.66053906660e-24          # g per amu
MASS = {1: 1.008, 6: 12.011, 7: 14.007, 8: 15.999, 16: 32.06}
OH = 0.9572
HOH = math.radians(104.52)


def _rand_rot(rng, n):
    q = rng.normal(size=(n, 4))
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    w, x, y, z = q.T
    R = np.empty((n, 3, 3))
    R[:, 0, 0] = 1 - 2 * (y * y + z * z); R[:, 0, 1] = 2 * (x * y - z * w); R[:, 0, 2] = 2 * (x * z + y * w)
    R[:, 1, 0] = 2 * (x * y + z * w); R[:, 1, 1] = 1 - 2 * (x * x + z * z); R[:, 1, 2] = 2 * (y * z - x * w)
    R[:, 2, 0] = 2 * (x * z - y * w); R[:, 2, 1] = 2 * (y * z + x * w); R[:, 2, 2] = 1 - 2 * (x * x + y * y)
    return R


def _water_frame():
    s, c = math.sin(HOH / 2), math.cos(HOH / 2)
    return np.array([[0.0, 0.0, 0.0], [OH * s, OH * c, 0.0], [-OH * s, OH * c, 0.0]])


def _waters(rng, centers):
    R = _rand_rot(rng, len(centers))
    mol = np.einsum("nij,aj->nai", R, _water_frame()) + centers[:, None, :]
    return mol.reshape(-1, 3), np.tile(np.array([8, 1, 1]), len(centers))


def _pack(pos, Z, L, name):
    pos = np.mod(pos, L).astype(np.float32)
    pos = np.where(pos >= np.float32(L), pos - np.float32(L), pos).astype(np.float32)
    return dict(pos=pos, Z=np.asarray(Z, np.int64), graph_ptr=np.array([0, len(pos)], np.int64),
                cell=(np.eye(3, dtype=np.float32) * np.float32(L))[None], pbc=np.ones((1, 3), bool), name=name)


def water_box(n_mol=216, L=18.64, seed=0):
    """Config 1: 216 H2O, cubic periodic box of side 18.64 A (1.0 g/cm^3)."""
    rng = np.random.default_rng(seed)
    centers = rng.uniform(0.0, L, size=(n_mol, 3))
    pos, Z = _waters(rng, centers)
    return _pack(pos, Z, L, f"water{n_mol}")


def organics_batch(n_mol=64, nmin=20, nmax=80, seed=0):
    """Config 2: ragged batch of random covalent trees, no PBC."""
    rng = np.random.default_rng(seed)
    elems = np.array([1, 6, 7, 8, 16]); probs = np.array([0.50, 0.30, 0.08, 0.10, 0.02])
    P, Z, ptr = [], [], [0]
    for _ in range(n_mol):
        n = int(rng.integers(nmin, nmax + 1))
        z = rng.choice(elems, size=n, p=probs)
        p = np.zeros((n, 3))
        for a in range(1, n):
            parent = int(rng.integers(0, a))
            d = rng.normal(size=3); d /= np.linalg.norm(d)
            p[a] = p[parent] + rng.uniform(1.0, 1.5) * d
        p += rng.normal(scale=0.05, size=p.shape)
        P.append(p); Z.append(z); ptr.append(ptr[-1] + n)
    B = n_mol
    return dict(pos=np.concatenate(P).astype(np.float32), Z=np.concatenate(Z).astype(np.int64),
                graph_ptr=np.array(ptr, np.int64), cell=np.zeros((B, 3, 3), np.float32),
                pbc=np.zeros((B, 3), bool), name=f"organics{n_mol}")


def solvated_chains(n_atoms=1500, density=1.0, seed=0, residues_per_chain=150):
    """Configs 3-5: random-walk heavy-atom chains (C/N/O cycling, 1.45 A steps,
    self-avoidance >= 2.5 A within a chain, one H at 1.0 A per heavy atom)
    solvated by rigid TIP3P-geometry waters on a jittered grid, periodic cubic
    box whose side is set by the total mass at ``density`` g/cm^3."""
    rng = np.random.default_rng(seed)
    n_heavy = n_atoms // 10
    n_wat = (n_atoms - 2 * n_heavy) // 3
    extra_h = n_atoms - 2 * n_heavy - 3 * n_wat
    heavy_z = np.array([6, 7, 8])[np.arange(n_heavy) % 3]
    mass = sum(MASS[int(z)] for z in heavy_z) + (n_heavy + extra_h) * MASS[1] + n_wat * (MASS[8] + 2 * MASS[1])
    L = (mass * AMU_G / density / 1e-24) ** (1.0 / 3.0)
    chains, hs = [], []
    n_chains = max(1, math.ceil(n_heavy / residues_per_chain))
    sizes = [n_heavy // n_chains + (1 if c < n_heavy % n_chains else 0) for c in range(n_chains)]
    for c, m in enumerate(sizes):
        p = np.zeros((m, 3))
        p[0] = rng.uniform(0, L, 3) if c else np.full(3, L / 2)
        for a in range(1, m):
            for _try in range(100):
                d = rng.normal(size=3); d /= np.linalg.norm(d)
                cand = p[a - 1] + 1.45 * d
                if a < 2 or np.min(np.linalg.norm(p[:a - 1] - cand, axis=1)) >= 2.5:
                    break
            p[a] = cand
        h = np.zeros((m, 3))
        for a in range(m):
            for _try in range(50):
                d = rng.normal(size=3); d /= np.linalg.norm(d)
                cand = p[a] + 1.0 * d
                others = np.delete(p, a, axis=0)
                if len(others) == 0 or np.min(np.linalg.norm(others - cand, axis=1)) >= 1.2:
                    break
            h[a] = cand
        chains.append(p); hs.append(h)
    heavy = np.concatenate(chains)
    hyd = np.concatenate(hs)
    if extra_h:
        d = rng.normal(size=(extra_h, 3)); d /= np.linalg.norm(d, axis=1, keepdims=True)
        hyd = np.concatenate([hyd, heavy[:extra_h] + d])
    chain_pos = np.concatenate([heavy, hyd])
    chain_z = np.concatenate([heavy_z, np.ones(len(hyd), np.int64)])
    # water sites on a jittered grid, away from the chains (minimum image)
    from scipy.spatial import cKDTree
    g = int(math.ceil((n_wat * 1.6) ** (1.0 / 3.0)))
    ax = (np.arange(g) + 0.5) * (L / g)
    sites = np.stack(np.meshgrid(ax, ax, ax, indexing="ij"), -1).reshape(-1, 3)
    sites = sites + rng.uniform(-0.3, 0.3, size=sites.shape)
    tree = cKDTree(np.mod(chain_pos, L), boxsize=L)
    dmin, _ = tree.query(np.mod(sites, L))
    ok = np.nonzero(dmin >= 2.5)[0]
    if len(ok) < n_wat:
        ok = np.argsort(-dmin)[:n_wat]
    pick = rng.permutation(ok)[:n_wat]
    wpos, wz = _waters(rng, sites[pick])
    pos = np.concatenate([chain_pos, wpos])
    Z = np.concatenate([chain_z, wz])
    return _pack(pos, Z, L, f"solvated{n_atoms}")


CONFIGS = {
    1: lambda seed=0: water_box(seed=seed),
    2: lambda seed=0: organics_batch(seed=seed),
    3: lambda seed=0: solvated_chains(1500, seed=seed),
    4: lambda seed=0: solvated_chains(10000, seed=seed),
    5: lambda seed=0: solvated_chains(100000, seed=seed),
}


def small_water(n_mol=8, L=6.2, seed=0):
    """Small periodic water cell for fast oracle tests (box may be < rc)."""
    return water_box(n_mol, L, seed)


def to_padded(sys):
    """Reference padded batch from a flattened system."""
    import torch
    ptr = sys["graph_ptr"]
    B = len(ptr) - 1
    n = np.diff(ptr)
    Lmax = int(n.max())
    pos = np.zeros((B, Lmax, 3), np.float32)
    Z = np.zeros((B, Lmax), np.int64)
    mask = np.zeros((B, Lmax), bool)
    for b in range(B):
        pos[b, :n[b]] = sys["pos"][ptr[b]:ptr[b + 1]]
        Z[b, :n[b]] = sys["Z"][ptr[b]:ptr[b + 1]]
        mask[b, :n[b]] = True
    return dict(pos=torch.from_numpy(pos), atomic_numbers=torch.from_numpy(Z), atom_masks=torch.from_numpy(mask),
                cell=torch.from_numpy(np.asarray(sys["cell"], np.float32)), pbc=torch.from_numpy(np.asarray(sys["pbc"])))
