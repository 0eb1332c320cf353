"""Drop-in model classes: E2FormerBackbone, MolfmAtomic, MDEnergyForceMultiHead.

* ``E2FormerBackbone(**backbone_config).forward(batched_data)`` mirrors
  src/molfm/models/e2former/e2former_wrapper.py:140-339 (same constructor
  kwargs, same output keys ``node_featuresBxN``, ``node_vec_featuresBxN``,
  ``node_irrepsBxN``, ``data``, ``neighbor_info``).  The neighbour list comes
  from the HIP cell-list builder instead of CellExpander / FAISS.
* ``MolfmAtomic`` mirrors src/molfm/tasks/pretrain_smallmol.py:170-251 with
  the MLP energy head and the autograd force head
  (src/molfm/pipeline/head.py:305-341,483-580).
* ``Potential.energy_forces`` is the flat entry point used by the MD loop and
  the benchmark: flattened atoms, graphs contiguous.
"""
from __future__ import annotations

import weakref
from types import SimpleNamespace
from typing import Dict, Optional

import numpy as np
import torch
from torch import nn

from . import _lib
from . import second_order
from .modules import E2former, EdgeContext, atom_type_slots, parse_irreps
from .neighbors import build_neighbors
from .ops import EdgeGeometryFn


def graph_bounds(pos: torch.Tensor, counts: torch.Tensor):
    """Per-graph coordinate minimum and maximum [B, 3] (graphs contiguous)."""
    if counts.shape[0] == 1:
        return pos.amin(0, keepdim=True), pos.amax(0, keepdim=True)
    lo = torch.segment_reduce(pos, "min", lengths=counts, axis=0, unsafe=True)
    hi = torch.segment_reduce(pos, "max", lengths=counts, axis=0, unsafe=True)
    return lo, hi


def spatial_order(pos: torch.Tensor, graph_ptr) -> torch.Tensor:
    """Permutation that sorts the atoms of every graph along a 30-bit Morton
    (Z-order) curve of their positions; graphs stay contiguous and in order.
    Neighbouring rows of the CSR then gather neighbouring source rows, which the
    XCD-contiguous row mapping of the kernels keeps in one L2."""
    N = pos.shape[0]
    if N == 0:
        return torch.zeros(0, dtype=torch.long, device=pos.device)
    counts_np = np.diff(np.asarray(graph_ptr))
    B = len(counts_np)
    pos = pos.detach().float().contiguous()
    gid = None
    if B == 1:   # no host copies or syncs for a single graph
        lo, hi = pos.amin(0, keepdim=True), pos.amax(0, keepdim=True)
    else:
        counts = torch.as_tensor(counts_np, device=pos.device)
        gid = torch.repeat_interleave(torch.arange(B, device=pos.device, dtype=torch.int32), counts,
                                      output_size=N)
        lo, hi = graph_bounds(pos, counts)
    lo = lo.contiguous()
    span = (hi - lo).clamp_min(1e-6).contiguous()
    key = torch.empty(N, dtype=torch.int64, device=pos.device)
    _lib.call("e2v2_morton_keys", _lib.vp(pos.data_ptr()), None if gid is None else _lib.vp(gid.data_ptr()),
              _lib.vp(lo.data_ptr()), _lib.vp(span.data_ptr()), _lib.i32(N), _lib.vp(key.data_ptr()),
              _lib.vp(torch.cuda.current_stream(pos.device).cuda_stream))
    return torch.sort(key, stable=True).indices


def _as_int_or_none(v):
    if v is None or (isinstance(v, str) and v.lower() == "none"):
        return None
    return int(v)


class E2FormerBackbone(nn.Module):
    def __init__(self, use_faiss: bool = False, **kwargs):
        super().__init__()
        self.kwargs = kwargs
        self.use_faiss = use_faiss  # accepted for signature compatibility; the HIP builder replaces FAISS
        C, lmax = parse_irreps(kwargs["irreps_node_embedding"])
        self.scalar_dim = C
        if kwargs.get("encoder", "default") != "default":
            raise NotImplementedError("encoder != 'default' is outside the MI355X path")
        self.embedding = nn.Embedding(256, C)
        self.embedding_charge = nn.Embedding(30, C)
        self.embedding_multiplicity = nn.Embedding(30, C)
        self.mix_cm = nn.Sequential(nn.Linear(2 * C, C), nn.SiLU())
        self.unifiedtokentoembedding = nn.Linear(C, C)
        kw = dict(kwargs)
        kw["max_neighbors"] = _as_int_or_none(kw.get("max_neighbors", None))
        self.decoder = E2former(**kw)
        self.max_neighbors = self.decoder.max_neighbors
        self.max_radius = float(self.decoder.max_radius)
        self.cells_per_direction = int(kwargs.get("pbc_expanded_num_cell_per_direction", 4))
        self._types = []
        self.set_compute_dtype(kwargs.get("compute_dtype", "fp32"))

    def set_compute_dtype(self, dtype) -> None:
        """'fp32' (default) or 'bf16': in bf16 mode every GEMM of the stack (per-node
        irreps linears, Q/K projections and heads, SO(2) output linears, gate) takes
        bf16 operands with fp32 accumulation and the attention's gathered
        activations are stored in bf16; parameters stay fp32 (bf16 copies are
        cached), the radial-profile tables, softmax statistics, normalisations
        and all reductions are fp32."""
        name = {torch.float32: "fp32", torch.bfloat16: "bf16"}.get(dtype, dtype)
        if name not in ("fp32", "float32", "bf16", "bfloat16"):
            raise ValueError(f"compute_dtype must be 'fp32' or 'bf16', got {dtype!r}")
        self.compute_bf16 = name in ("bf16", "bfloat16")

    def type_slots(self, Z: torch.Tensor, graph_ptr=None):
        """``modules.atom_type_slots`` of Z and its graphs: (type_z, type_key, slot).
        One host readback per new Z tensor; repeated calls with the same live tensor
        and graphs (an MD loop) reuse the result."""
        gkey = None if graph_ptr is None else np.asarray(graph_ptr, np.int64).tobytes()
        # the last few live Z tensors (several integrators may share one model)
        self._types = [c for c in self._types if c[0]() is not None]
        for c in self._types:
            if c[0]() is Z and c[1] == Z._version and c[2] == gkey:
                return c[3]
        out = atom_type_slots(Z, graph_ptr)
        self._types = (self._types + [(weakref.ref(Z), Z._version, gkey, out)])[-4:]
        return out

    # -- flat interface -------------------------------------------------------
    def forward_flat(self, pos: torch.Tensor, Z: torch.Tensor, graph_ptr, cell, pbc, charge=None,
                     multiplicity=None, nl=None, reorder: bool = True, grid_box=None, nbr_capacity=None):
        """pos [N,3] (may require grad), Z [N] on the GPU; graph_ptr/cell/pbc on the host.
        Returns (node_irreps [N,9,C], neighbour list, perm): rows of node_irreps and
        the neighbour list refer to atoms ``perm`` (Morton order within each graph;
        identity when ``reorder`` is False).  grid_box, nbr_capacity = (edges,
        longest row[, pinned int32 [4] counter buffer]) (the capacity build, no host
        readback): see ``build_neighbors``.  In training mode the decoder runs the
        twice-differentiable training path (``second_order``): gradients reach
        every parameter, and forces taken with create_graph=True can be
        differentiated again."""
        perm = None
        type_z, type_key, slot = self.type_slots(Z, graph_ptr)
        if reorder and nl is None:
            perm = spatial_order(pos.detach(), graph_ptr)
            pos = pos[perm]
            slot = slot[perm]
        if nl is None:
            nl = build_neighbors(pos.detach(), graph_ptr, cell, pbc, self.max_radius, 1e-4, self.max_neighbors,
                                 self.cells_per_direction, grid_box=grid_box,
                                 capacity=None if nbr_capacity is None else tuple(nbr_capacity[:2]),
                                 stats_host=None if nbr_capacity is None or len(nbr_capacity) < 3 else nbr_capacity[2])
        train = self.training
        dvec, dist = (nl.dvec, nl.dist) if train else EdgeGeometryFn.apply(pos, nl)
        ctx = EdgeContext(nl, dvec, dist, slot.contiguous(), type_z, type_key, self.decoder.rbf, self.max_radius,
                          self.compute_bf16)
        long_ctx = None
        if self.decoder.cluster:
            long_ctx = self.long_range_context(pos, Z if perm is None else Z[perm], graph_ptr, cell, pbc, slot,
                                               type_z, type_key)
        sys_node = None
        if charge is not None:
            B = len(graph_ptr) - 1
            sys_emb = self.mix_cm(torch.cat([self.embedding_charge(torch.clip(charge, -10, 10) + 10),
                                             self.embedding_multiplicity(torch.clip(multiplicity, 0, 20))],
                                            dim=-1)).reshape(B, -1)
            counts = torch.as_tensor(np.diff(np.asarray(graph_ptr)), device=pos.device)
            sys_node = torch.repeat_interleave(sys_emb, counts, dim=0)
        if train:
            return second_order.decoder_forward(self.decoder, ctx, pos, sys_node, long_ctx), nl, perm
        return self.decoder.forward_flat(ctx, sys_node, long_ctx), nl, perm

    def long_range_context(self, pos, Z, graph_ptr, cell, pbc, slot, type_z, type_key) -> EdgeContext:
        """Edge context of the long-range cluster blocks (e2former_wrapper.py:223-243):
        neighbours j with long_cutoff_lower <= d <= long_cutoff_upper whose atomic
        number is neither 0 nor 1, at most 2.5 max_neighbors per atom (all when
        max_neighbors is None), rbf_long as the distance basis and the bell or
        polynomial envelope of with_cluster."""
        dec = self.decoder
        lo, hi = float(dec.long_cutoff_lower), float(dec.long_cutoff_upper)
        include = (Z != 0) & (Z != 1)
        mx = None if self.max_neighbors is None else int(2.5 * self.max_neighbors)
        nl = build_neighbors(pos.detach(), graph_ptr, cell, pbc, hi, lo, mx, self.cells_per_direction,
                             src_include=include.contiguous())
        dvec, dist = (nl.dvec, nl.dist) if self.training else EdgeGeometryFn.apply(pos, nl)
        kind, env_lo = dec.long_envelope()
        return EdgeContext(nl, dvec, dist, slot.contiguous(), type_z, type_key, dec.rbf_long, hi, self.compute_bf16,
                           kind, env_lo)

    # -- reference interface -------------------------------------------------
    def forward(self, batched_data, **kwargs) -> Dict:
        pos = batched_data["pos"]
        mask = batched_data["atom_masks"].bool()
        B, L = pos.shape[:2]
        Z = batched_data["atomic_numbers"].reshape(B, L)
        counts = mask.sum(-1).cpu().numpy()
        graph_ptr = np.concatenate([[0], np.cumsum(counts)])
        cell = batched_data.get("cell", None)
        pbc = batched_data.get("pbc", None)
        cell = np.zeros((B, 3, 3), np.float32) if cell is None else cell.detach().float().cpu().numpy()
        pbc = np.zeros((B, 3), bool) if pbc is None else pbc.detach().cpu().numpy().astype(bool)
        fpos = pos.float()[mask]
        fZ = Z[mask]
        charge = batched_data.get("charge", None)
        mult = batched_data.get("multiplicity", None)
        x, nl, perm = self.forward_flat(fpos, fZ, graph_ptr, cell, pbc, charge, mult)
        x = x.permute(1, 0, 2)                       # m-major -> [N, 9, C]
        if perm is not None:
            x = x.index_select(0, torch.argsort(perm))
        node_irreps = x.new_zeros((B, L, x.shape[1], x.shape[2]))
        node_irreps = node_irreps.masked_scatter(mask[:, :, None, None], x)
        info = neighbor_info(nl, perm, fpos.detach(), graph_ptr, cell, self.max_radius)
        batched_data.update(f_exp_node_pos=info.pop("f_exp_node_pos"), f_outcell_index=info.pop("f_outcell_index"))
        return {"node_featuresBxN": node_irreps[:, :, 0], "node_vec_featuresBxN": node_irreps[:, :, 1:4],
                "node_irrepsBxN": node_irreps, "data": batched_data, "neighbor_info": info}


def _segment_metadata(row_index: torch.Tensor, col_index: torch.Tensor, num_rows: int):
    """(row_ptr, sorted col_index, edge_perm) int32 of a stable sort by row
    (triton_sparse_qk_autograd.py:617-633)."""
    perm = torch.argsort(row_index, stable=True)
    counts = torch.bincount(row_index.long(), minlength=num_rows)
    row_ptr = torch.zeros(num_rows + 1, dtype=torch.int32, device=row_index.device)
    row_ptr[1:] = counts.cumsum(0).to(torch.int32)
    return row_ptr, col_index[perm].to(torch.int32).contiguous(), perm.to(torch.int32).contiguous()


def neighbor_info(nl, perm: Optional[torch.Tensor], pos: torch.Tensor, graph_ptr, cells, rc: float) -> Dict:
    """The neighbour list as the reference's ``construct_neighbor`` dict
    (module_utils.py:3233-3242) in the caller's atom order: ``query_idx``
    ascending with each row ordered by distance, ``neighbor_idx`` into the
    flattened expanded nodes, the 6-tuple CSR ``metadata``
    (triton_sparse_qk_autograd.py:635-652), ``f_edge_vec``, ``f_dist``,
    ``f_poly_dist``; plus the expanded nodes themselves (``f_exp_node_pos``,
    ``f_outcell_index``, e2former_wrapper.py:213-216).  Expanded nodes are, per
    graph, every real atom (the [0,0,0] cell, atom order) followed by the images
    that carry edges, in (cell, atom) order; images of the reference's expansion
    that carry no edge (within 1e-4 of an atom but no other atom in range) are
    not listed.  ``shift`` [E,3] gives each edge's integer cell offset."""
    from .ops import ENV_A, ENV_B, ENV_C
    dev = pos.device
    N, E = nl.n_atoms, nl.n_edges
    graph_ptr = np.asarray(graph_ptr, np.int64)
    cells = torch.as_tensor(np.asarray(cells, np.float32).reshape(-1, 3, 3), device=dev)
    to_in = perm if perm is not None else torch.arange(N, device=dev)
    qi = to_in[nl.edge_row.long()]
    order = torch.argsort(qi, stable=True)            # rows keep their distance order
    qi = qi[order]
    j = to_in[nl.col.long()][order]
    sidx = nl.shift_idx.long()[order]
    shifts = nl.shifts.to(dev)
    # per-graph [0,0,0] row of the shift table, and the graph of every atom
    counts = torch.as_tensor(np.diff(graph_ptr), device=dev)
    gid = torch.repeat_interleave(torch.arange(len(counts), device=dev), counts, output_size=N)
    sptr0 = torch.as_tensor(np.asarray(nl.shift_ptr, np.int64)[:-1], device=dev)
    key_real = sptr0[gid] * N + torch.arange(N, device=dev)
    key_edge = sidx * N + j
    exp_keys, inv = torch.unique(torch.cat([key_real, key_edge]), sorted=True, return_inverse=True)
    nbr = inv[N:]
    out_j = exp_keys % N
    out_s = exp_keys // N
    off = shifts[out_s].float()
    cg = cells[gid[out_j]]
    img_off = (off[:, 0:1] * cg[:, 0] + off[:, 1:2] * cg[:, 1]) + off[:, 2:3] * cg[:, 2]
    exp_pos = pos[out_j] + img_off
    vec = nl.dvec[order]
    dist = nl.dist[order]
    ratio = dist / rc                                   # module_utils.py:1946-1954
    poly = torch.where(ratio < 1, 1 + ratio ** 5 * (ENV_A + ratio * (ENV_B + ENV_C * ratio)), 0)
    q_ptr, q_col, q_perm = _segment_metadata(qi, nbr, N)
    k_ptr, k_col, k_perm = _segment_metadata(nbr, qi, exp_keys.shape[0])
    return {"query_idx": qi, "neighbor_idx": nbr, "metadata": (q_ptr, q_col, q_perm, k_ptr, k_col, k_perm),
            "f_edge_vec": vec, "f_dist": dist, "f_poly_dist": poly, "shift": shifts[sidx],
            "f_exp_node_pos": exp_pos, "f_outcell_index": out_j}


class MLP_energy_head(nn.Module):
    """head.py:330-341."""

    def __init__(self, embedding_dim, lmax=2):
        super().__init__()
        self.mlp = nn.Sequential(nn.Linear(embedding_dim, embedding_dim), nn.SiLU(),
                                 nn.Linear(embedding_dim, embedding_dim), nn.SiLU(), nn.Linear(embedding_dim, 1))

    def forward(self, embedding, irreps=None):
        return self.mlp(embedding)


class GradientHead(nn.Module):
    """head.py:305-328: forces = -dE/dpos, with create_graph in training mode
    (the backbone then runs its twice-differentiable training path)."""

    def forward(self, pos, pred_energy):
        return -torch.autograd.grad(pred_energy, pos, torch.ones_like(pred_energy), create_graph=self.training)[0]


class MDEnergyForceMultiHead(nn.Module):
    """head.py:483-580 (MLP energy head + gradient force head)."""

    def __init__(self, args):
        super().__init__()
        C, lmax = parse_irreps(args.backbone_config["irreps_node_embedding"])
        self.energy_heads = nn.ModuleDict()
        self.force_heads = nn.ModuleDict()
        rename = {"svp-enhance": "tzvpd", "tzvpd-small": "tzvpd", "tzvpd-forceatomfilter": "tzvpd"}
        if "share" in getattr(args, "head_cfg_str", ""):
            rename.update({k: "omol25" for k in ("svp-enhance", "tzvpd-small", "tzvpd", "tzvpd-forceatomfilter")})
        self.dataset_rename = rename
        for name in str(args.dataset_name_list).split(","):
            head = rename.get(name, name)
            if head not in self.energy_heads:
                self.energy_heads[head] = MLP_energy_head(C, lmax)
                self.force_heads[head] = GradientHead()

    def head_name(self, name: Optional[str]):
        if name is None:
            return next(iter(self.energy_heads.keys()))
        return self.dataset_rename.get(name, name)


class MolfmAtomic(nn.Module):
    """pretrain_smallmol.py:170-251 restricted to energy + autograd forces."""

    def __init__(self, args, loss_fn=None, not_init=False):
        super().__init__()
        if not_init:
            return
        self.args = args
        name = args.backbone_config["name"]
        if name not in {"e2former", "e2formerv2"}:
            raise ValueError(f"Unsupported backbone: {name}")
        cfg = dict(args.backbone_config)
        cfg.pop("name", None)
        self.decoder = E2FormerBackbone(**cfg)
        self.head = MDEnergyForceMultiHead(args)

    def energy_flat(self, pos, Z, graph_ptr, cell, pbc, head=None, charge=None, multiplicity=None, nl=None,
                    grid_box=None, nbr_capacity=None):
        x, nl, _ = self.decoder.forward_flat(pos, Z, graph_ptr, cell, pbc, charge, multiplicity, nl,
                                             grid_box=grid_box, nbr_capacity=nbr_capacity)
        h = self.head.head_name(head)
        e_atom = self.head.energy_heads[h](x[0]).squeeze(-1)     # x is m-major [9, N, C]
        B = len(graph_ptr) - 1
        if B == 1:
            energy = e_atom.sum().reshape(1)
        else:   # deterministic per-graph sums (no atomics)
            counts = torch.as_tensor(np.diff(np.asarray(graph_ptr)), device=pos.device)
            energy = torch.segment_reduce(e_atom, "sum", lengths=counts, axis=0, unsafe=True)
        return energy, nl

    def energy_forces_flat(self, pos, Z, graph_ptr, cell, pbc, head=None, charge=None, multiplicity=None,
                           grid_box=None, nbr_capacity=None):
        pos = pos.detach().float().requires_grad_(True)
        energy, nl = self.energy_flat(pos, Z, graph_ptr, cell, pbc, head, charge, multiplicity, grid_box=grid_box,
                                      nbr_capacity=nbr_capacity)
        if self.training:   # forces that can be differentiated again (the training path)
            forces = -torch.autograd.grad(energy, pos, torch.ones_like(energy), create_graph=True)[0]
            return energy, forces, nl
        forces = -torch.autograd.grad(energy, pos, torch.ones_like(energy))[0]
        return energy.detach(), forces, nl

    def forward(self, batched_data, need_force=True, **unused):
        pos = batched_data["pos"]
        if need_force:
            pos.requires_grad_(True)
        out = self.decoder(dict(batched_data))
        data_name = batched_data.get("data_name", [None])
        h = self.head.head_name(data_name[0] if data_name else None)
        mask = batched_data["atom_masks"].bool()
        e_atom = self.head.energy_heads[h](out["node_featuresBxN"]).squeeze(-1).masked_fill(~mask, 0.0)
        energy = e_atom.sum(dim=-1)
        res = {"pred_energy": energy, "pred_energy_per_atom": energy / mask.sum(-1).reshape(-1)}
        if need_force:
            res["pred_forces"] = self.head.force_heads[h](pos, energy)
        return res


def default_args(max_radius=6.0, max_neighbors=None, num_layers=4, heads=("omol25",)):
    """Backbone configuration of the benchmark, with the
    reference's config keys (config_file/backbone_config/e2former.yaml)."""
    bb = dict(name="e2former", irreps_node_embedding="256x0e+256x1e+256x2e", irreps_head="2x0e+2x1e+2x2e",
              attn_scalar_head=8, num_attn_heads=128, number_of_basis=256, max_radius=max_radius,
              max_neighbors=max_neighbors, num_layers=num_layers, alpha_drop=0.0, basis_type="gaussiansmear",
              norm_layer="rms_norm_sh", attn_type="so2-first-order", tp_type="QK_alpha", edge_embedtype="default",
              ffn_type="s3", encoder="default", with_cluster=False, pbc_expanded_num_cell_per_direction=4)
    return SimpleNamespace(backbone_config=bb, dataset_name_list=",".join(heads), head_cfg_str="",
                           AutoGradForce=True)
