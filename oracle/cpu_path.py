"""Oracle evaluation with the exact cell-list neighbour list (test
infrastructure / CPU baseline only).

For systems where the reference's dense B x T x (cells*T) expansion does not
fit, the expanded nodes are built from the exact edge list instead: one
expanded node per distinct (j, s) image, positions pos_j + s.cell with
autograd, then the reference's own decoder and head run unchanged.  The edge
set equals the dense path's (pinned by test_oracle.py).
"""
from __future__ import annotations

import numpy as np
import torch

from .neighbors import exact_neighbors, polynomial


def reference_batch(om, sysd, pos: torch.Tensor):
    """Build the reference's batched_data + neighbour info for one periodic or
    non-periodic system from the exact edge list."""
    nb = exact_neighbors(sysd["pos"], sysd["graph_ptr"], sysd["cell"], sysd["pbc"],
                         om.decoder.max_radius)
    ptr = np.asarray(sysd["graph_ptr"])
    assert len(ptr) == 2, "cpu_path handles one graph"
    key = nb["j"] * 1000003 + ((nb["s"][:, 0] + 8) * 17 + (nb["s"][:, 1] + 8)) * 17 + (nb["s"][:, 2] + 8)
    uniq, inv = np.unique(key, return_inverse=True)
    first = np.zeros(len(uniq), np.int64)
    first[inv[::-1]] = np.arange(len(inv))[::-1]
    exp_j = torch.as_tensor(nb["j"][first])
    exp_s = torch.as_tensor(nb["s"][first].astype(np.float32))
    cell = torch.as_tensor(np.asarray(sysd["cell"][0], np.float32))
    exp_pos = pos[exp_j] + exp_s @ cell
    qi = torch.as_tensor(nb["i"])
    ni = torch.as_tensor(inv)
    vec = pos[qi] - exp_pos[ni]
    dist = torch.linalg.norm(vec, dim=-1)
    poly = polynomial(dist, om.decoder.max_radius)
    return dict(query_idx=qi, neighbor_idx=ni, f_edge_vec=vec, f_dist=dist, f_poly_dist=poly,
                f_exp_node_pos=exp_pos, f_outcell_index=exp_j), len(nb["i"])


def energy_forces_with_neighbors(om, sysd, progress=None):
    """(energy, forces, edge count) of one graph; ``progress(msg)`` is called after
    the neighbour list, the forward and the backward when given."""
    pos = torch.as_tensor(np.asarray(sysd["pos"], np.float32)).clone().requires_grad_(True)
    Z = torch.as_tensor(np.asarray(sysd["Z"]))
    nbinfo, n_edges = reference_batch(om, sysd, pos)
    if progress:
        progress(f"neighbour list: {n_edges} edges")
    bd = dict(pos=pos.unsqueeze(0), atomic_numbers=Z.unsqueeze(0),
              atom_masks=torch.ones(1, len(Z), dtype=torch.bool),
              pbc=torch.as_tensor(np.asarray(sysd["pbc"])), cell=torch.as_tensor(np.asarray(sysd["cell"])))
    bd.update(nbinfo)
    dec = om.decoder
    tok = dec.embedding(bd["atomic_numbers"])
    a, v, irr = dec.decoder(bd, tok, None)
    e = om.head(dict(node_featuresBxN=a), bd, next(iter(om.head.energy_heads.keys())))[0]
    if progress:
        progress("forward done")
    f = -torch.autograd.grad(e, pos, torch.ones_like(e))[0]
    if progress:
        progress("backward done")
    return e.detach(), f, n_edges
