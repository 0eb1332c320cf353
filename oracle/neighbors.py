"""Radius-graph oracles (test infrastructure only).

Two restatements of the reference's neighbour construction:

``exact_neighbors`` (numpy, fp32 arithmetic, no FMA)
    The edge set of ``CellExpander.expand_includeself`` + ``construct_radius_neighbor``
    (``src/molfm/models/e2former/module_utils.py:953-988,1065-1274,3119-3242``):

    * shifts s with |s_d| <= min(pbc_cells, ceil(rc / h_d)) on periodic dims,
      s_d = 0 on the others (``module_utils.py:956-988,1145-1151``);
    * an image (j, s) exists iff some real atom of the graph lies strictly
      within rc of it (``module_utils.py:1118-1130``);
    * edge i <- (j, s) iff rmin <= d <= rc, both inclusive (``:3166,3181``).

    All arithmetic uses the one fp32 expression shared with the HIP kernel:
    off = ((s0*a0 + s1*b0) + s2*c0) per component, img = pos_j + off,
    dv = pos_i - img, d = sqrt((dx*dx + dy*dy) + dz*dz), each op rounded to fp32.
    Candidate pairs come from a scipy cKDTree query with radius rc + 1e-3 and are
    then filtered with that expression, so the result does not depend on the tree.
    Pinned by: brute force over all pairs and shifts on small cells, the dense
    torch restatement below, i<-j(s) <=> j<-i(-s) up to fp32 ties, lattice
    translation invariance, and the expected count 4/3 pi rc^3 rho.

``dense_reference_neighbors`` (torch CPU)
    Line-by-line semantics of the reference's dense path (B x T x (cells*T)
    distance tensor, ``torch.linalg.norm``), usable for a few thousand atoms.
    Returns the reference's own output format (expanded nodes, query/neighbor
    index, f_edge_vec, f_dist, f_poly_dist).
"""
from __future__ import annotations

import math
import numpy as np
import torch

F32 = np.float32


def max_offsets(cell: np.ndarray, rc: float, cap: int) -> list:
    """``CellExpander._get_cell_tensors._get_max_offset_for_dim`` in fp32 torch."""
    c = torch.as_tensor(np.asarray(cell, np.float32)).reshape(1, 3, 3)
    out = []
    for dim in range(3):
        v0 = c[:, dim, :]
        others = c[:, torch.arange(3) != dim, :]
        nrm = torch.cross(others[:, 0, :], others[:, 1, :], dim=-1)
        nrm = nrm / nrm.norm(dim=-1, keepdim=True)
        try:
            mo = int(torch.max(torch.ceil(rc / torch.abs(torch.sum(nrm * v0, dim=-1)))))
        except Exception:
            mo = cap
        out.append(mo)
    return out


def shift_list(cell: np.ndarray, pbc, rc: float, cap: int = 4) -> np.ndarray:
    """Integer shifts in the reference's order: [0,0,0] first, then the
    (i, j, k) lexicographic cells within the offsets, periodic dims only."""
    if not np.any(pbc):
        return np.zeros((1, 3), np.int32)
    mo = max_offsets(cell, rc, cap)
    sh = [(0, 0, 0)]
    rng = range(-cap, cap + 1)
    for i in rng:
        for j in rng:
            for k in rng:
                if i == 0 and j == 0 and k == 0:
                    continue
                s = (i, j, k)
                if any(abs(s[d]) > mo[d] for d in range(3)):
                    continue
                if any((s[d] != 0) and not pbc[d] for d in range(3)):
                    continue
                sh.append(s)
    return np.array(sh, np.int32)


def shift_offsets_f32(shifts: np.ndarray, cell: np.ndarray) -> np.ndarray:
    """off[c] = fl(fl(fl(s0*A0c) + fl(s1*A1c)) + fl(s2*A2c)) in fp32."""
    A = np.asarray(cell, F32).reshape(3, 3)
    s = shifts.astype(F32)
    t0 = s[:, 0:1] * A[0][None, :]
    t1 = s[:, 1:2] * A[1][None, :]
    t2 = s[:, 2:3] * A[2][None, :]
    return ((t0 + t1) + t2).astype(F32)


def fp32_dist(pi: np.ndarray, pj: np.ndarray, off: np.ndarray):
    img = (pj.astype(F32) + off.astype(F32)).astype(F32)
    dv = (pi.astype(F32) - img).astype(F32)
    sq = ((dv[:, 0] * dv[:, 0] + dv[:, 1] * dv[:, 1]) + dv[:, 2] * dv[:, 2]).astype(F32)
    return dv, np.sqrt(sq).astype(F32)


def exact_neighbors(pos, graph_ptr, cells, pbcs, rc=6.0, rmin=1e-4, cap=4, include=None):
    """Canonical exact edge list.  pos [N,3] fp32 (real atoms, graphs contiguous),
    graph_ptr [B+1], cells [B,3,3], pbcs [B,3].  Returns dict with
    i, j (int64), s (int32 [E,3]), dv (fp32 [E,3]), d (fp32 [E]) sorted
    lexicographically by (i, j, s).  include [N] bool (or None): only atoms j
    with include[j] are sources, the include_mask of module_utils.py:3165-3166
    applied to the expanded nodes (which image exists does not depend on it)."""
    from scipy.spatial import cKDTree
    pos = np.asarray(pos, F32)
    rc32, rmin32 = F32(rc), F32(rmin)
    I, Jn, S, DV, D = [], [], [], [], []
    for b in range(len(graph_ptr) - 1):
        p0, p1 = int(graph_ptr[b]), int(graph_ptr[b + 1])
        if p1 <= p0:
            continue
        P = pos[p0:p1]
        n = len(P)
        shifts = shift_list(cells[b], pbcs[b], rc, cap)
        offs = shift_offsets_f32(shifts, cells[b])
        periodic = bool(np.any(pbcs[b]))
        tree = cKDTree(P.astype(np.float64))
        for si in range(len(shifts)):
            img = (P + offs[si][None, :]).astype(F32)
            cand = tree.query_ball_point(img.astype(np.float64), r=float(rc) + 1e-3)
            jj = np.repeat(np.arange(n), [len(c) for c in cand])
            ii = np.concatenate([np.asarray(c, np.int64) for c in cand]) if n else np.zeros(0, np.int64)
            if len(ii) == 0:
                continue
            dv, d = fp32_dist(P[ii], P[jj], np.broadcast_to(offs[si], (len(ii), 3)))
            ok = (d >= rmin32) & (d <= rc32)
            if periodic:
                # image (jj, s) must have some atom strictly inside rc
                strict = d < rc32
                has = np.zeros(n, bool)
                np.logical_or.at(has, jj[strict], True)
                ok &= has[jj]
            if include is not None:
                ok &= np.asarray(include, bool)[p0:p1][jj]
            I.append(ii[ok] + p0); Jn.append(jj[ok] + p0)
            S.append(np.repeat(shifts[si][None], ok.sum(), 0)); DV.append(dv[ok]); D.append(d[ok])
    if not I:
        return dict(i=np.zeros(0, np.int64), j=np.zeros(0, np.int64), s=np.zeros((0, 3), np.int32),
                    dv=np.zeros((0, 3), F32), d=np.zeros(0, F32))
    i = np.concatenate(I); j = np.concatenate(Jn); s = np.concatenate(S); dv = np.concatenate(DV); d = np.concatenate(D)
    order = np.lexsort((s[:, 2], s[:, 1], s[:, 0], j, i))
    return dict(i=i[order], j=j[order], s=s[order], dv=dv[order], d=d[order])


def brute_force_neighbors(pos, graph_ptr, cells, pbcs, rc=6.0, rmin=1e-4, cap=4):
    """O(N^2 * shifts) version of ``exact_neighbors`` (same fp32 expression, no
    tree) for small systems; used to pin the tree-based candidate search."""
    pos = np.asarray(pos, F32)
    rc32, rmin32 = F32(rc), F32(rmin)
    out = []
    for b in range(len(graph_ptr) - 1):
        p0, p1 = int(graph_ptr[b]), int(graph_ptr[b + 1])
        P = pos[p0:p1]
        n = len(P)
        shifts = shift_list(cells[b], pbcs[b], rc, cap)
        offs = shift_offsets_f32(shifts, cells[b])
        periodic = bool(np.any(pbcs[b]))
        for si in range(len(shifts)):
            ii, jj = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
            ii = ii.ravel(); jj = jj.ravel()
            dv, d = fp32_dist(P[ii], P[jj], np.broadcast_to(offs[si], (len(ii), 3)))
            kept = np.ones(n, bool)
            if periodic:
                kept = np.zeros(n, bool)
                np.logical_or.at(kept, jj[d < rc32], True)
            ok = (d >= rmin32) & (d <= rc32) & kept[jj]
            for a, bb, v, dd in zip(ii[ok], jj[ok], dv[ok], d[ok]):
                out.append((a + p0, bb + p0, *shifts[si], *v, dd))
    out.sort(key=lambda t: t[:5])
    if not out:
        return dict(i=np.zeros(0, np.int64), j=np.zeros(0, np.int64), s=np.zeros((0, 3), np.int32),
                    dv=np.zeros((0, 3), F32), d=np.zeros(0, F32))
    a = np.array(out, dtype=object)
    return dict(i=a[:, 0].astype(np.int64), j=a[:, 1].astype(np.int64), s=a[:, 2:5].astype(np.int32),
                dv=a[:, 5:8].astype(F32), d=a[:, 8].astype(F32))


# --------------------------------------------------------------------------
# Dense restatement of the reference (torch CPU), reference output format.
# --------------------------------------------------------------------------
def polynomial(dist, cutoff, exponent=5):
    """``module_utils.py:1946-1954``."""
    a = -(exponent + 1) * (exponent + 2) / 2
    b = exponent * (exponent + 2)
    c = -exponent * (exponent + 1) / 2
    ratio = dist / cutoff
    env_val = 1 + ratio ** exponent * (a + ratio * (b + c * ratio))
    return torch.where(ratio < 1, env_val, 0)


def expand_includeself(pos, pbc, atomic_numbers, cell, rc, cap=4, padding_mask=None, dtype=torch.float32):
    """``CellExpander.expand_includeself`` (``module_utils.py:1065-1274``) with
    ``neighbors_radius=(None, rc)``.  pos [B,T,3] (may require grad)."""
    B, T = pos.shape[:2]
    if padding_mask is None:
        padding_mask = torch.zeros((B, T), dtype=torch.bool)
    pos = torch.where(padding_mask.unsqueeze(-1).repeat(1, 1, 3), 999.0, pos.to(dtype))
    cell = cell.to(dtype)
    # candidate cells (the reference's self.cells, [0,0,0] excluded), then mask by offsets
    cells = torch.tensor([[i, j, k] for i in range(-cap, cap + 1) for j in range(-cap, cap + 1)
                          for k in range(-cap, cap + 1) if not (i == 0 and j == 0 and k == 0)])
    cmask_pbc = cells != 0
    mo = []
    for dim in range(3):
        v0 = cell[:, dim, :]
        others = cell[:, torch.arange(3) != dim, :]
        nrm = torch.cross(others[:, 0, :], others[:, 1, :], dim=-1)
        nrm = nrm / nrm.norm(dim=-1, keepdim=True)
        try:
            mo.append(int(torch.max(torch.ceil(rc / torch.abs(torch.sum(nrm * v0, dim=-1))))))
        except Exception:
            mo.append(cap)
    sel = (cells.abs() <= torch.tensor(mo)).all(dim=-1)
    cell_tensor = torch.cat([torch.zeros((1, 3)), cells[sel].float()], 0)
    cell_mask = torch.cat([torch.zeros((1, 3), dtype=torch.bool), cmask_pbc[sel]], 0)
    cell_tensor = cell_tensor.unsqueeze(0).repeat(B, 1, 1).to(cell.dtype)
    n_cell = cell_tensor.size(1)
    offset = torch.bmm(cell_tensor, cell)
    expand_pos = (pos.unsqueeze(1) + offset.unsqueeze(2)).view(B, -1, 3)
    expand_dist = torch.norm(pos.unsqueeze(2) - expand_pos.unsqueeze(1), p=2, dim=-1)
    expand_mask = expand_dist < rc
    expand_mask = (expand_mask & (~padding_mask.repeat(1, n_cell).unsqueeze(1))
                   & (~(atomic_numbers.eq(0).unsqueeze(-1))))
    expand_mask = torch.sum(expand_mask, dim=1) > 0
    expand_mask = expand_mask & (~(atomic_numbers.eq(0).repeat(1, n_cell)))
    cmask = (torch.all(pbc.unsqueeze(1) >= cell_mask.unsqueeze(0), dim=-1)
             .unsqueeze(-1).repeat(1, 1, T).reshape(expand_mask.size()))
    expand_mask &= cmask
    expand_len = torch.sum(expand_mask, dim=-1)
    L2 = int(torch.max(expand_len))
    outcell = torch.zeros([B, L2], dtype=torch.long)
    exp_pos = torch.zeros([B, L2, 3], dtype=pos.dtype)
    all_idx = torch.arange(T).repeat(n_cell)
    shift_of = cell_tensor[0].long().repeat_interleave(T, 0)  # [n_cell*T, 3]
    exp_shift = torch.zeros([B, L2, 3], dtype=torch.long)
    exp_pos_list = []
    for b in range(B):
        n = int(expand_len[b])
        outcell[b, :n] = all_idx[expand_mask[b]]
        exp_shift[b, :n] = shift_of[expand_mask[b]]
        exp_pos_list.append(expand_pos[b, expand_mask[b], :])
    exp_pos = torch.stack([torch.cat([e, torch.zeros(L2 - e.shape[0], 3, dtype=pos.dtype)], 0)
                           for e in exp_pos_list], 0)
    ar = torch.arange(L2).unsqueeze(0)
    emask = ar < expand_len.unsqueeze(1)
    return dict(expand_node_pos=exp_pos.to(dtype), outcell_index=outcell, expand_node_mask=emask,
                expand_shift=exp_shift)


def smooth_polynomial_bell(dist, cutoff_min, cutoff_max, exponent=2):
    """``module_utils.py:1956-1985``: (1 - t^2)^exponent with t the distance
    mapped linearly from [cutoff_min, cutoff_max] onto [-1, 1] and clamped."""
    cmin = torch.tensor(cutoff_min, dtype=dist.dtype)
    cmax = torch.maximum(torch.tensor(cutoff_max, dtype=dist.dtype), cmin + 1e-8)
    t = (2 * dist - (cmin + cmax)) / (cmax - cmin)
    t = torch.clamp(t, -1.0, 1.0)
    return (1.0 - t ** 2) ** exponent


def _fixed_norm(v):
    """The fp32 expression sqrt((dx*dx + dy*dy) + dz*dz), each op rounded (the
    build's fixed form of torch.linalg.norm for fp32 vectors).  The square root
    is taken in float64 and rounded once to fp32, which is the correctly rounded
    fp32 root (torch's CPU fp32 sqrt is not correctly rounded in every case)."""
    a = v.to(torch.float32)
    s = (a[..., 0] * a[..., 0] + a[..., 1] * a[..., 1]) + a[..., 2] * a[..., 2]
    return torch.sqrt(s.double()).float()


def construct_radius_neighbor(node_pos, node_mask, expand_node_pos, expand_node_mask,
                              max_dist, min_dist=1e-4, max_neighbors=None, include_mask=None,
                              poly="poly", fixed_norm=False):
    """``module_utils.py:3119-3242`` (metadata omitted: the CSR is rebuilt where
    needed).  ``fixed_norm`` replaces torch.linalg.norm by the fixed fp32
    expression (the two agree to about one ulp); ties in the per-row sort keep
    the expanded-slot order (a stable sort)."""
    B, L = node_pos.shape[:2]
    expand_ptr = torch.cat([torch.zeros(1, dtype=torch.int64),
                            torch.cumsum(torch.sum(expand_node_mask, dim=-1), dim=-1)])
    edge_vec = node_pos.unsqueeze(2) - expand_node_pos.unsqueeze(1)
    dist = _fixed_norm(edge_vec) if fixed_norm else torch.linalg.norm(edge_vec, dim=-1, keepdim=False)
    dist = torch.where(dist >= min_dist, dist, max_dist + 1000)
    if include_mask is not None:
        dist = torch.where(include_mask.unsqueeze(1), dist, max_dist + 1000)
    within = torch.max(torch.sum(dist <= max_dist, dim=-1)[node_mask])
    _, nidx = dist.sort(dim=-1, descending=False, stable=True)
    if max_neighbors is not None:
        topK = max(min(expand_node_pos.shape[1], max_neighbors, int(within)), 1)
    else:
        topK = max(min(expand_node_pos.shape[1], int(within)), 1)
    nidx = nidx[:, :, :topK]
    dist = torch.gather(dist, dim=-1, index=nidx)
    f_dist = dist[node_mask]
    f_attn_mask = (f_dist > max_dist).unsqueeze(-1)
    if poly == "poly":
        f_poly = polynomial(f_dist, max_dist)
    elif poly == "poly_bell":
        f_poly = smooth_polynomial_bell(f_dist, min_dist, max_dist, exponent=2)
    else:
        raise ValueError("sorry, you must set poly or poly_bell")
    f_poly = torch.where(f_attn_mask.squeeze(-1), 0, f_poly)
    f_sparse = (nidx + expand_ptr[:B, None, None])[node_mask]
    f_sparse = torch.clamp(f_sparse, max=int(expand_ptr[B]) - 1)
    f_edge_vec = node_pos[node_mask].unsqueeze(1) - expand_node_pos[expand_node_mask][f_sparse]
    valid = ~f_attn_mask.squeeze(-1)
    N, K = f_sparse.shape
    query_idx = torch.arange(N).unsqueeze(1).expand(N, K)[valid].contiguous()
    neighbor_idx = f_sparse[valid].contiguous()
    return dict(query_idx=query_idx, neighbor_idx=neighbor_idx,
                f_edge_vec=f_edge_vec[valid].contiguous(), f_dist=f_dist[valid].contiguous(),
                f_poly_dist=f_poly[valid].contiguous())
