"""Autograd operators over libe2v2.so (HIP, gfx950).

Each Function computes on the current stream of the input tensors' device and
calls the C ABI of include/e2v2.h; there is no CPU or PyTorch fallback.
Weights of the radial MLPs are constants of these Functions (inference and
force evaluation need input gradients only); ``create_graph=True`` (double
backward) raises NotImplementedError instead of returning wrong gradients.
"""
from __future__ import annotations

import math
from typing import List, Optional

import numpy as np
import torch
from torch import nn

from . import _lib, gemm, so3
from .neighbors import NeighborList

ENV_EXPONENT = 5
ENV_A = -(ENV_EXPONENT + 1) * (ENV_EXPONENT + 2) / 2
ENV_B = ENV_EXPONENT * (ENV_EXPONENT + 2)
ENV_C = -ENV_EXPONENT * (ENV_EXPONENT + 1) / 2


# Placement of the 20 SO(2) output rows in the attention kernels' l3-grouped layout (so3.so2_row_layout):
# row t of channel c of atom i at N SO2_A[t] + i SO2_LD[t] + SO2_COL[t] + c; per output degree l3 a block
# [2 l3 + 1][N][cnt 256] starting at N start (SO2_GROUPS = [(l3, cnt, start)]).
SO2_A, SO2_LD, SO2_COL, SO2_GROUPS = so3.so2_row_layout()


def so2_rows(flat: torch.Tensor, n_atoms: int) -> torch.Tensor:
    """[20, N, 256] l3-sequential rows (a copy) of an l3-grouped attention output."""
    N = int(n_atoms)
    out = flat.new_empty(len(SO2_A), N, 256)
    for t in range(len(SO2_A)):
        out[t] = torch.as_strided(flat, (N, 256), (SO2_LD[t], 1), N * SO2_A[t] + SO2_COL[t])
    return out


def so2_grouped(rows: torch.Tensor) -> torch.Tensor:
    """The l3-grouped layout (flat) of [20, N, 256] l3-sequential rows."""
    N = rows.shape[1]
    flat = rows.new_empty(rows.numel())
    for t in range(len(SO2_A)):
        torch.as_strided(flat, (N, 256), (SO2_LD[t], 1), N * SO2_A[t] + SO2_COL[t]).copy_(rows[t])
    return flat


def _stream(t: torch.Tensor):
    return _lib.vp(torch.cuda.current_stream(t.device).cuda_stream)


def _p(t: Optional[torch.Tensor]):
    return None if t is None else _lib.vp(t.data_ptr())


def _need_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("the e2v2 HIP path needs GPU tensors (no CPU fallback)")


def _no_double_backward():
    if torch.is_grad_enabled():
        raise NotImplementedError("the HIP E2Former path implements first-order input gradients only "
                                  "(create_graph=True / double backward is not supported)")


class RadialTable:
    """Distance table of radial profiles RadialProfile [256 + 2E -> 128 -> 128 -> 256]
    (src/molfm/models/e2former/module_utils.py:2151-2178) over
    x_edge = [rbf(d), tgt[z_i], src[z_j]] for the atom types ``type_z``: one
    profile (an attention layer's fc_easy, 256 channels gate | inputhead) or the
    degree embedding's three (768 channels).  Built in float64 on the device
    (e2v2_radial_table), then checked at every interval midpoint against the
    float64 profile (e2v2_radial_table_check); starting from the spacing of
    ``min_refine`` (-1: 2^(floor(log2(0.2 sigma)) + 1), 0.0156 A for the 256-basis
    RBF at 6 A) the node spacing is halved until the interpolation error is at
    most ``tol_value`` of the largest |f| and ``tol_deriv`` of the largest |f'|
    (one host readback per build).  The coarsest passing table keeps the edge
    kernels' table reads in L2.

    ``pairs`` (host sequence of (a, b) type-slot pairs, a the query atom's) chooses
    the type pairs the table holds, one slot each in the order given; None: all
    T^2 pairs (slot a T + b).  Every pair an edge can join must have a slot (the
    products of each graph's own type set, ``atom_type_slots``); the kernels map a
    pair to its slot through ``pair_slot`` [T^2] (slot or -1).

    ``layout`` places the channels: "plain" (rows [pairs][nodes][4][nc], profile
    m at 256 m + c), "attn" (one fc_easy profile in the attention kernels' slice
    order, gate and inputhead of head h at 32 (h // 16) + h % 16 and 16 positions
    on, stored slice-major [pairs][8][nodes][4][32]), "deg" (three profiles,
    channel c of profile l at 96 (c // 32) + 32 l + c % 32, stored slice-major
    [pairs][8][nodes][4][96]) or "degh": the three profiles' 128 hidden channels
    (the last Linear's input; e2v2_radial_hidden_table), hidden channel k of
    profile l at 96 (k // 32) + 32 l + k % 32, stored slice-major
    [pairs][4][nodes][4][96].  The hidden table is checked on the profile's output
    W3 h~ + b3, with the same tolerances, and keeps the packed last Linears for the
    degree embedding's per-node GEMMs (``w3_pack``: [W3_l | b3_l | 0] as a
    144 -> 256 weight, ``w3t_pack``: W3_l^T, ``b3``: [3, 256])."""

    LAYOUTS = {
        "plain": lambda m: (256 * m, 256, 256, 0, 0, 0),
        "attn": lambda m: (0, 128, 16, 32, 16, 32),
        "deg": lambda m: (32 * m, 256, 32, 96, 0, 96),
        "degh": lambda m: (32 * m, 128, 32, 96, 0, 96),
    }
    HIDDEN = ("degh",)

    def __init__(self, nets, tgt: nn.Embedding, src: nn.Embedding, rbf_offset: torch.Tensor, rbf_coeff: float,
                 rc: float, type_z: torch.Tensor, tol_value: float = 1e-6, tol_deriv: float = 1e-5,
                 max_refine: int = 3, layout: str = "plain", min_refine: int = -1, pairs=None):
        dev = type_z.device
        if (layout not in self.LAYOUTS or (layout == "attn" and len(nets) != 1)
                or (layout in ("deg", "degh") and len(nets) != 3)):
            raise ValueError(f"radial table layout {layout!r} does not fit {len(nets)} profiles")
        self.layout = layout
        hidden = layout in self.HIDDEN
        self._layouts = [_lib.RadialLayout(*self.LAYOUTS[layout](m)) for m in range(len(nets))]
        self.nc = (128 if hidden else 256) * len(nets)
        build, check = (("e2v2_radial_hidden_table", "e2v2_radial_hidden_table_check") if hidden
                        else ("e2v2_radial_table", "e2v2_radial_table_check"))
        self.n_types = T = int(type_z.numel())
        if T < 1 or T > MAX_TYPES:
            raise NotImplementedError(f"{T} atom types: atomic numbers index embeddings of {MAX_TYPES} entries")
        if pairs is None:
            self.pairs = None
            self.n_pairs = T * T
            self.pair_slot = self.pair_ab = None
        else:
            pairs = [(int(a), int(b)) for a, b in pairs]
            if not pairs or len(set(pairs)) != len(pairs) or any(not (0 <= a < T and 0 <= b < T) for a, b in pairs):
                raise ValueError(f"radial table pairs must be distinct type-slot pairs of {T} types")
            if len(pairs) > MAX_PAIRS:
                raise NotImplementedError(f"{len(pairs)} type pairs: a table holds at most {MAX_PAIRS}")
            self.pairs = tuple(pairs)
            self.n_pairs = len(pairs)
            slot = np.full(T * T, -1, np.int32)
            ab = np.array([a * T + b for a, b in pairs], np.int32)
            slot[ab] = np.arange(len(pairs), dtype=np.int32)
            self.pair_slot = torch.as_tensor(slot, device=dev)
            self.pair_ab = torch.as_tensor(ab, device=dev)
        with torch.no_grad():
            self._keep = [t.detach().float().contiguous() for t in (tgt.weight, src.weight, rbf_offset)]
            tgt_w, src_w, mu = self._keep
            self._structs = [self._net(n, tgt_w, src_w) for n in nets]
        self.type_z = type_z.to(torch.int32).contiguous()
        st = _stream(type_z)
        for refine in range(min_refine, max_refine + 1):
            n = _lib.C.c_int32(); h = _lib.C.c_float()
            _lib.call("e2v2_radial_table_size", _lib.f32(rc), _lib.f32(rbf_coeff), _lib.i32(refine), _lib.C.byref(n),
                      _lib.C.byref(h))
            self.n_nodes, self.h = n.value, h.value
            self.tab = torch.empty(self.n_pairs, self.n_nodes, 4, self.nc, dtype=torch.float32, device=dev)
            err = torch.zeros(len(nets), 4, dtype=torch.int32, device=dev)
            for m, W in enumerate(self._structs):
                args = (_lib.C.byref(W), _p(mu), _lib.f32(rbf_coeff), _p(self.type_z), _lib.i32(self.n_types),
                        _lib.vp(self.pair_slot_ptr(self.pair_ab)), _lib.i32(self.n_pairs), _lib.i32(self.n_nodes),
                        _lib.f32(self.h))
                lo = _lib.C.byref(self._layouts[m])
                _lib.call(build, *args, _p(self.tab), _lib.i32(self.nc), lo, st)
                _lib.call(check, *args, _p(self.tab), _lib.i32(self.nc), lo, _lib.vp(err[m].data_ptr()), st)
            e = err.cpu().view(torch.float32).double()
            self.value_err = float((e[:, 0] / e[:, 1].clamp_min(1e-30)).max())
            self.deriv_err = float((e[:, 2] / e[:, 3].clamp_min(1e-30)).max())
            if self.value_err <= tol_value and self.deriv_err <= tol_deriv:
                break
        else:
            raise RuntimeError(f"radial table: interpolation error {self.value_err:.2e} (value) / "
                               f"{self.deriv_err:.2e} (derivative) above tolerance after {max_refine} refinements")
        if hidden:
            with torch.no_grad():
                w3 = torch.stack([n[6].weight.detach().float() for n in nets])          # [3, 256, 128]
                b3 = torch.stack([n[6].bias.detach().float() for n in nets])            # [3, 256]
                wb = torch.zeros(len(nets), 256, 144, dtype=torch.float32, device=dev)
                wb[:, :, :128] = w3
                wb[:, :, 128] = b3
                self.w3_pack = gemm.pack(wb)                    # hs [.., 144] -> x0 [.., 256]
                self.w3t_pack = gemm.pack(w3, transpose=True)   # grad_x0 [.., 256] -> grad_h [.., 128]
                self.b3 = b3.contiguous()

    def pair_slot_ptr(self, t="slot"):
        """Device address of the pair -> slot map (or of ``t``), None for all pairs."""
        t = self.pair_slot if isinstance(t, str) else t
        return None if t is None else t.data_ptr()

    def _net(self, net: nn.Sequential, tgt_w: torch.Tensor, src_w: torch.Tensor) -> _lib.RadialNet:
        lin1, ln1, lin2, ln2, lin3 = net[0], net[1], net[3], net[4], net[6]
        if not (isinstance(net[2], nn.SiLU) and isinstance(net[5], nn.SiLU)):
            raise NotImplementedError("RadialProfile activations must be SiLU")
        if not (abs(ln1.eps - 1e-5) < 1e-12 and abs(ln2.eps - 1e-5) < 1e-12):
            raise NotImplementedError("RadialProfile LayerNorm eps must be 1e-5")
        E = tgt_w.shape[1]
        if (lin1.weight.shape != (128, 256 + 2 * E) or lin2.weight.shape != (128, 128)
                or lin3.weight.shape != (256, 128) or src_w.shape[1] != E):
            raise NotImplementedError(f"RadialProfile {tuple(lin1.weight.shape)} -> {tuple(lin3.weight.shape)} is "
                                      "not the [256 + 2E, 128, 128, 256] profile the radial tables are built for")
        ts = [t.detach().float().contiguous() for t in (lin1.weight, lin1.bias, ln1.weight, ln1.bias, lin2.weight,
                                                         lin2.bias, ln2.weight, ln2.bias, lin3.weight, lin3.bias)]
        self._keep += ts
        w1, b1, g1, be1, w2, b2, g2, be2, w3, b3 = [t.data_ptr() for t in ts]
        return _lib.RadialNet(w1, 256 + 2 * E, E, b1, g1, be1, w2, b2, g2, be2, w3, b3, tgt_w.data_ptr(),
                              src_w.data_ptr())


MAX_TYPES = 256
MAX_PAIRS = 65535


def _version_key(params):
    return tuple((p.data_ptr(), p._version, p.dtype, str(p.device)) for p in params)


class RadialCache:
    """Rebuild a RadialTable only when a parameter, the basis or the type set changed
    (an MD loop builds each table once)."""

    def __init__(self):
        self.key = None
        self.table: Optional[RadialTable] = None

    def get(self, nets, tgt_emb: nn.Embedding, src_emb: nn.Embedding, rbf_offset: torch.Tensor, rbf_coeff: float,
            rc: float, type_z: torch.Tensor, type_key: tuple, layout: str = "plain", pairs=None):
        """type_key: the host key of the type set (and of ``pairs``, the table's type pairs)."""
        params = [p for n in nets for p in n.parameters()] + [tgt_emb.weight, src_emb.weight, rbf_offset]
        key = (_version_key(params), float(rbf_coeff), float(rc), type_key, pairs, layout)
        if key != self.key:
            self.table = None
            self.table = RadialTable(nets, tgt_emb, src_emb, rbf_offset, rbf_coeff, rc, type_z, layout=layout,
                                     pairs=pairs)
            self.key = key
        return self.table


class EdgeGeometryFn(torch.autograd.Function):
    """(dvec, dist) of every edge as a function of the positions; backward is the
    deterministic row-minus-column reduction of e2v2_edge_to_pos."""

    @staticmethod
    def forward(ctx, pos, nl: NeighborList):
        _need_cuda(pos)
        ctx.nl = nl
        return nl.dvec.clone(), nl.dist.clone()

    @staticmethod
    def backward(ctx, g_dvec, g_dist):
        _no_double_backward()
        nl = ctx.nl
        dev = nl.dvec.device
        if g_dvec is None:
            g_dvec = torch.zeros_like(nl.dvec)
        if g_dist is None:
            g_dist = torch.zeros_like(nl.dist)
        g_dvec = g_dvec.float().contiguous(); g_dist = g_dist.float().contiguous()
        dpos = torch.empty(nl.n_atoms, 3, dtype=torch.float32, device=dev)
        _lib.call("e2v2_edge_to_pos", _lib.i32(nl.n_atoms), _p(nl.row_ptr), _p(nl.key_ptr), _p(nl.key_eid),
                  _p(nl.dvec), _p(nl.dist), _p(g_dvec), _p(g_dist), _p(dpos), _stream(dpos))
        return dpos, None


class DegreeEmbedFn(torch.autograd.Function):
    """EdgeDegreeEmbeddingNetwork_higherorder.forward (e2former.py:689-753) with its
    three gbf_projs profiles (module_utils.py:2151-2178) split at their last Linear:
    the kernels sum the interpolated hidden channels times Y_m p over each row's
    edges (hs [9, N, 144]: 128 hidden sums, the sum of Y_m p, zeros), and one
    per-node split GEMM applies [W3_l | b3_l] (x0 = hs W^T, 144 -> 256 per degree l).
    The backward runs the transposed GEMM (grad_h = grad_x0 W3_l) and the bias
    column's grad_s = grad_x0 . b3_l before the edge kernel.  A "deg" table (the
    profiles' outputs) runs e2v2_deg_fwd / e2v2_deg_bwd directly.  Nothing per edge
    is saved."""

    WIDX = (0, 1, 1, 1, 2, 2, 2, 2, 2)   # profile of each m-row

    @staticmethod
    def forward(ctx, dvec, dist, nl: NeighborList, atom_type, table: RadialTable, avg: float, rc: float):
        _need_cuda(dvec, dist)
        dev = dvec.device
        dargs = deg_args(nl, atom_type, table, avg, rc)
        N = nl.n_atoms
        x0 = torch.empty(9, N, 256, dtype=torch.float32, device=dev)   # m-major
        if table.layout == "degh":
            hs = torch.empty(9, N, 144, dtype=torch.float32, device=dev)
            _lib.call("e2v2_deg_hidden_fwd", _lib.C.byref(dargs), _p(hs), _stream(hs))
            if N:
                gemm.gemm(hs, table.w3_pack, x0, DegreeEmbedFn.WIDX)
            del hs
        else:
            _lib.call("e2v2_deg_fwd", _lib.C.byref(dargs), _p(x0), _stream(x0))
        ctx.nl, ctx.atom_type, ctx.table, ctx.avg, ctx.rc = nl, atom_type, table, avg, rc
        return x0

    @staticmethod
    def backward(ctx, gx0):
        _no_double_backward()
        nl, table = ctx.nl, ctx.table
        dev = nl.dvec.device
        E, N = nl.n_edges, nl.n_atoms
        gx0 = gx0.float().contiguous()
        dargs = deg_args(nl, ctx.atom_type, table, ctx.avg, ctx.rc)
        ddv = torch.empty(max(E, 1), 3, dtype=torch.float32, device=dev)
        dd = torch.empty(max(E, 1), dtype=torch.float32, device=dev)
        nb = int(_lib.load().e2v2_deg_bwd_workspace(E))     # per-slice partials of this call
        ws = torch.empty(max(nb, 16), dtype=torch.uint8, device=dev)
        if table.layout == "degh":
            gh = torch.empty(9, N, 128, dtype=torch.float32, device=dev)
            gs = torch.empty(9, max(N, 1), dtype=torch.float32, device=dev)
            if N:
                gemm.gemm(gx0, table.w3t_pack, gh, DegreeEmbedFn.WIDX)
            _lib.call("e2v2_deg_bias_grad", _p(gx0), _p(table.b3), _lib.i32(N), _p(gs), _stream(gx0))
            _lib.call("e2v2_deg_hidden_bwd", _lib.C.byref(dargs), _p(gh), _p(gs), _p(ddv), _p(dd), _p(ws),
                      _lib.C.c_size_t(ws.numel()), _stream(gx0))
            del gh, gs
        else:
            _lib.call("e2v2_deg_bwd", _lib.C.byref(dargs), _p(gx0), _p(ddv), _p(dd), _p(ws),
                      _lib.C.c_size_t(ws.numel()), _stream(gx0))
        del ws
        return ddv[:E], dd[:E], None, None, None, None, None


def deg_args(nl: NeighborList, atom_type: torch.Tensor, table: RadialTable, avg: float, rc: float):
    if not ((table.layout == "deg" and table.nc == 768) or (table.layout == "degh" and table.nc == 384)):
        raise ValueError("the degree embedding needs the table of its three profiles in slices (layout 'deg', "
                         "or 'degh' for their hidden channels)")
    return _lib.DegArgs(nl.n_atoms, nl.n_edges, 128 if table.layout == "degh" else 256, nl.row_ptr.data_ptr(),
                        nl.dvec.data_ptr(), nl.dist.data_ptr(), nl.col.data_ptr(), table.tab.data_ptr(),
                        atom_type.data_ptr(), table.n_types, table.n_nodes, table.h, float(avg), float(rc), ENV_A,
                        ENV_B, ENV_C, table.pair_slot_ptr())


WEIGHT_ACTS = {"softmax": 0, "softplus": 1, "sigmoid": 2}


def attn_args(nl: NeighborList, q, k, v, atom_type, table: RadialTable, q_div: float, rc: float, bf: int,
              zero_order: bool = False, env=(0, 0.0), ext_gate=None, ext_dgate=None, weight_act: str = "softmax"):
    """e2v2_attn_args over the neighbour list (with its column clusters when built).
    zero_order selects the zero-order aggregation; env = (kind, lower end): kind 0
    the polynomial envelope on [0, rc], 1 the smooth bell on [lower end, rc];
    ext_gate [E, 128] fp32 (or None) replaces the table's gate rows, ext_dgate
    [E, 128] receives its gradient in the backward; weight_act the weight form
    ("softmax", or "softplus" / "sigmoid" of tp_type's "+softplus" / "+sigmoid",
    e2former.py:329-332)."""
    if weight_act not in WEIGHT_ACTS:
        raise ValueError(f"weight form {weight_act!r} is not one of {sorted(WEIGHT_ACTS)}")
    if table.nc != 256 or table.layout != "attn":
        raise ValueError("the attention needs the table of its fc_easy profile in slice order (layout 'attn')")
    a = _lib.AttnArgs(nl.n_atoms, nl.n_edges, 128, 8, 256, nl.row_ptr.data_ptr(), nl.col.data_ptr(),
                      nl.edge_row.data_ptr(), nl.key_ptr.data_ptr(), nl.key_eid.data_ptr(), nl.dvec.data_ptr(),
                      nl.dist.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), table.tab.data_ptr(),
                      atom_type.data_ptr(), table.n_types, table.n_nodes, table.h, float(q_div), float(rc), ENV_A,
                      ENV_B, ENV_C, int(bf))
    a.zero_order = int(bool(zero_order))
    a.env_kind, a.env_lo = int(env[0]), float(env[1])
    a.pair_slot = table.pair_slot_ptr()
    a.weight_act = WEIGHT_ACTS[weight_act]
    if ext_gate is not None:
        if ext_gate.shape != (nl.n_edges, 128) or ext_gate.dtype != torch.float32 or not ext_gate.is_contiguous():
            raise ValueError(f"ext_gate must be a contiguous float32 [{nl.n_edges}, 128] tensor")
        a.ext_gate = ext_gate.data_ptr() if nl.n_edges else None
        a.ext_dgate = None if ext_dgate is None or nl.n_edges == 0 else ext_dgate.data_ptr()
    if nl.col_slot_member is not None:
        a.col_span = nl.col_span
        a.col_slot_member = nl.col_slot_member.data_ptr()
        a.col_slot_edge = nl.col_slot_edge.data_ptr()
        a.col_n_slots = nl.col_n_slots.data_ptr()
    return a


def attention_forward(q, k, v, nl: NeighborList, atom_type, table: RadialTable, rc: float, q_div: float,
                      act_dtype=torch.float32, zero_order: bool = False, env=(0, 0.0), ext_gate=None,
                      weight_act: str = "softmax"):
    """e2v2_attn_fwd: (out, mrow, srow, cnt, q, k, v, ext_gate), the last four in the
    storage the kernels read (what ``attention_backward`` takes back)."""
    if act_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"attention activations must be float32 or bfloat16, got {act_dtype}")
    dev = q.device
    N = nl.n_atoms
    q = q.to(act_dtype).contiguous(); k = k.to(act_dtype).contiguous(); v = v.to(act_dtype).contiguous()
    bf = int(act_dtype == torch.bfloat16)
    if ext_gate is not None:
        ext_gate = ext_gate.float().contiguous()
    args = attn_args(nl, q, k, v, atom_type, table, q_div, rc, bf, zero_order, env, ext_gate,
                     weight_act=weight_act)
    if zero_order:
        out = torch.empty(9, N, 256, dtype=act_dtype, device=dev)
    else:
        out = torch.empty(20 * N * 256, dtype=act_dtype, device=dev)   # l3-grouped rows
    mrow = torch.empty(N, 128, dtype=torch.float32, device=dev)
    srow = torch.empty(N, 128, dtype=torch.float32, device=dev)
    cnt = torch.empty(N, 128, dtype=torch.int32, device=dev)
    _lib.call("e2v2_attn_fwd", _lib.C.byref(args), _p(out), _p(mrow), _p(srow), _p(cnt), _stream(q))
    return out, mrow, srow, cnt, q, k, v, ext_gate


def attention_backward(gout, q, k, v, out, mrow, srow, cnt, ext_gate, nl: NeighborList, atom_type,
                       table: RadialTable, rc: float, q_div: float, zero_order: bool = False, env=(0, 0.0),
                       weight_act: str = "softmax"):
    """e2v2_attn_bwd on the state of ``attention_forward``: (dq, dk, dv, ddvec [E, 3],
    ddist [E], dL/dgate or None), all fp32."""
    dev = q.device
    E = nl.n_edges
    bf = int(q.dtype == torch.bfloat16)
    gout = gout.to(out.dtype).contiguous()
    dgate = None if ext_gate is None else torch.empty(E, 128, dtype=torch.float32, device=dev)
    args = attn_args(nl, q, k, v, atom_type, table, q_div, rc, bf, zero_order, env, ext_gate, dgate, weight_act)
    f = dict(dtype=torch.float32, device=dev)
    ddv = torch.empty(max(E, 1), 3, **f)
    dd = torch.empty(max(E, 1), **f)
    dq = torch.empty(q.shape, **f); dk = torch.empty(k.shape, **f); dv = torch.empty(v.shape, **f)
    # workspace of this call (per-edge weights handed from the row pass to the column pass, per-slice
    # partial edge gradients), freed when the call returns
    nb = int(_lib.load().e2v2_attn_bwd_workspace(E))
    ws = torch.empty(max(nb, 16), dtype=torch.uint8, device=dev)
    _lib.call("e2v2_attn_bwd", _lib.C.byref(args), _p(gout), _p(out), _p(mrow), _p(srow), _p(cnt), _p(ddv),
              _p(dd), _p(dq), _p(dk), _p(dv), _p(ws), _lib.C.c_size_t(ws.numel()), _stream(gout))
    del ws
    return dq, dk, dv, ddv[:E], dd[:E], dgate


class AttentionFn(torch.autograd.Function):
    """Edge part of E2AttentionArbOrder_sparse.forward (e2former.py:238-433) up to
    the SO(2) product's forward_linear: returns the 20 l3-sequential rows of
    h_a - h_b of so2_tensor_product.py:385 for every query atom in the
    l3-grouped layout (flat, 20 N 256 values; ``so2_rows`` gives [20, N, 256]);
    q, k [N, 128, 8], v [9, N, 256], the channels of v and of the output in the
    kernels' slice order (modules.slice_perm).  gate and inputhead
    (fc_easy, e2former.py:258-306) are interpolated from the layer's radial table
    inside the kernels: only node-level tensors are saved.

    With ``zero_order`` the edge part of the zero-order attention
    (e2former.py:411-416) instead: the 9 rows sum_j alpha_ij,h(c) v_j (no 1/r, no
    SO(2) product), [9, N, 256] m-major in the same slice order of channels."""

    @staticmethod
    def forward(ctx, q, k, v, dvec, dist, nl: NeighborList, atom_type, table: RadialTable, rc: float,
                q_div: float, act_dtype=torch.float32, zero_order: bool = False, env=(0, 0.0), ext_gate=None,
                weight_act: str = "softmax"):
        """act_dtype: storage of q, k, v and of the output rows (torch.float32, or
        torch.bfloat16 in the bf16 mode: half the gather traffic, fp32 math).
        env: the distance envelope (kind, lower end), see attn_args.  ext_gate
        [E, 128]: the gate of every (edge, head) (the QKdot variants' gates, in the
        edge order of nl); the table then only supplies the inputhead.  weight_act:
        the weight form, see attn_args."""
        _need_cuda(q, k, v, dvec, dist)
        out, mrow, srow, cnt, q, k, v, ext_gate = attention_forward(q, k, v, nl, atom_type, table, rc, q_div,
                                                                    act_dtype, zero_order, env, ext_gate,
                                                                    weight_act)
        ctx.save_for_backward(q, k, v, out, mrow, srow, cnt, ext_gate)
        ctx.nl, ctx.atom_type, ctx.table, ctx.rc, ctx.q_div = nl, atom_type, table, rc, q_div
        ctx.zero_order, ctx.env, ctx.weight_act = zero_order, env, weight_act
        return out

    @staticmethod
    def backward(ctx, gout):
        _no_double_backward()
        q, k, v, out, mrow, srow, cnt, ext_gate = ctx.saved_tensors
        dq, dk, dv, ddv, dd, dgate = attention_backward(gout, q, k, v, out, mrow, srow, cnt, ext_gate, ctx.nl,
                                                        ctx.atom_type, ctx.table, ctx.rc, ctx.q_div, ctx.zero_order,
                                                        ctx.env, ctx.weight_act)
        return dq, dk, dv, ddv, dd, None, None, None, None, None, None, None, None, dgate, None


class RadialEvalFn(torch.autograd.Function):
    """Per-edge values [E, nc] of a "plain"-layout RadialTable (e2v2_radial_eval):
    the radial profiles of the QKdot gates (rad_func_m0, e2former.py:278; the
    second half of fc_easy, e2former.py:293-294) at every edge of nl, for the
    type pair (atom_type[row], atom_type[col]).  Gradient: dist only (the table
    is a constant of the weights)."""

    @staticmethod
    def forward(ctx, dist, nl: NeighborList, atom_type, table: RadialTable):
        _need_cuda(dist)
        if table.layout != "plain":
            raise ValueError("RadialEvalFn needs a table in the 'plain' layout")
        E = nl.n_edges
        dist = dist.float().contiguous()
        out = torch.empty(E, table.nc, dtype=torch.float32, device=dist.device)
        _lib.call("e2v2_radial_eval", *_radial_eval_args(nl, atom_type, table, dist), _p(out), _stream(dist))
        ctx.save_for_backward(dist)
        ctx.nl, ctx.atom_type, ctx.table = nl, atom_type, table
        return out

    @staticmethod
    def backward(ctx, g):
        _no_double_backward()
        (dist,) = ctx.saved_tensors
        g = g.float().contiguous()
        dd = torch.empty_like(dist)
        _lib.call("e2v2_radial_eval_bwd", *_radial_eval_args(ctx.nl, ctx.atom_type, ctx.table, dist), _p(g), _p(dd),
                  _stream(dist))
        return dd, None, None, None


def _radial_eval_args(nl: NeighborList, atom_type, table: RadialTable, dist):
    # e_end = row_ptr[N] on the device: a capacity build's slots past the real edges are not read
    e_end = _lib.vp(nl.row_ptr.data_ptr() + 4 * nl.n_atoms) if nl.n_edges else None
    return (_p(table.tab), _lib.i32(table.n_types), _lib.vp(table.pair_slot_ptr()), _lib.i32(table.n_nodes),
            _lib.f32(table.h), _lib.i32(table.nc), _p(atom_type), _p(nl.edge_row), _p(nl.col), _p(dist),
            _lib.i64(nl.n_edges), e_end)


class QKdotGateFn(torch.autograd.Function):
    """The gate [E, 128] of tp_type QKdot_alpha (e2former.py:270-283):
    fc_m0(cat_l(sum_{m in l} Y[e, m] xd[m, row(e)]) * rad_func_m0(x_edge)) with
    the profile read from its 768-channel "plain" table and the 768-wide edge
    operand formed inside the GEMM (e2v2_qkdot_gate_fwd / _bwd): no per-edge
    tensor wider than the gate exists in either direction.  Y [E, 9] (the edge's
    normalised spherical harmonics), xd [9, N, 256] (dot_linear of the layer
    input), packs = (fc_m0.weight packed, its transpose packed) of one piece
    count, bias [128].  Gradients to dist, Y and xd."""

    @staticmethod
    def forward(ctx, dist, Y, xd, nl: NeighborList, atom_type, table: RadialTable, packs, bias):
        _need_cuda(dist, Y, xd)
        if table.layout != "plain" or table.nc != 768:
            raise ValueError("QKdotGateFn needs the 768-channel rad_func_m0 table in the 'plain' layout")
        if packs[0].n != 128 or packs[0].k != 768 or packs[1].n != 768 or packs[1].k != 128 or \
                packs[0].pieces != packs[1].pieces:
            raise ValueError("QKdotGateFn: fc_m0 must be Linear(768, 128), packed both ways with one piece count")
        E, N = nl.n_edges, nl.n_atoms
        Y = Y.float().contiguous()
        xd = xd.float().contiguous()
        if Y.shape != (E, 9) or xd.shape != (9, N, 256):
            raise ValueError(f"QKdotGateFn: Y {tuple(Y.shape)}, xd {tuple(xd.shape)} for {E} edges and {N} atoms")
        dist = dist.float().contiguous()
        bias = bias.float().contiguous()
        if dist.shape != (E,) or bias.shape != (128,) or atom_type.dtype != torch.int32 or atom_type.numel() < N:
            raise ValueError(f"QKdotGateFn: dist {tuple(dist.shape)} (needs [{E}]), bias {tuple(bias.shape)} "
                             f"(needs [128]), atom_type {atom_type.dtype} [{atom_type.numel()}] (int32, {N} atoms)")
        args = _qkdot_args(nl, atom_type, table, dist, Y, xd, packs[0].pieces)
        gate = torch.empty(E, 128, dtype=torch.float32, device=dist.device)
        _lib.call("e2v2_qkdot_gate_fwd", _lib.C.byref(args), _p(packs[0].buf), _p(bias), _p(gate), _stream(dist))
        ctx.save_for_backward(dist, Y, xd)
        ctx.nl, ctx.atom_type, ctx.table, ctx.packs = nl, atom_type, table, packs
        return gate

    @staticmethod
    def backward(ctx, dgate):
        _no_double_backward()
        dist, Y, xd = ctx.saved_tensors
        nl = ctx.nl
        dgate = dgate.float().contiguous()
        args = _qkdot_args(nl, ctx.atom_type, ctx.table, dist, Y, xd, ctx.packs[0].pieces)
        dY = torch.empty_like(Y)
        ddist = torch.empty_like(dist)
        dxd = torch.empty_like(xd)
        nb = int(_lib.load().e2v2_qkdot_gate_bwd_workspace(nl.n_edges))
        ws = torch.empty(max(nb, 16), dtype=torch.uint8, device=dist.device)
        _lib.call("e2v2_qkdot_gate_bwd", _lib.C.byref(args), _p(ctx.packs[1].buf), _p(dgate), _p(dY), _p(ddist),
                  _p(dxd), _p(ws), _lib.C.c_size_t(ws.numel()), _stream(dgate))
        del ws
        return ddist, dY, dxd, None, None, None, None, None


def _qkdot_args(nl: NeighborList, atom_type, table: RadialTable, dist, Y, xd, pieces: int):
    # e_end = row_ptr[N] on the device: a capacity build's slots past the real edges are not read
    e_end = _lib.vp(nl.row_ptr.data_ptr() + 4 * nl.n_atoms) if nl.n_edges else None
    return _lib.QkdotArgs(nl.n_atoms, nl.n_edges, nl.row_ptr.data_ptr(), nl.edge_row.data_ptr(), nl.col.data_ptr(),
                          dist.data_ptr(), e_end, Y.data_ptr(), xd.data_ptr(), table.tab.data_ptr(),
                          atom_type.data_ptr(), table.n_types, table.n_nodes, table.h, table.pair_slot_ptr(),
                          int(pieces))


class ShContractFn(torch.autograd.Function):
    """x0 [E, 3, C] with x0[e, l] = sum_{m in l} Y[e, m] xn[m, row(e)] (e2v2_sh_contract):
    the per-edge x_0_extra of the QKdot gates (e2former.py:271-276, 288-296).  Y
    [E, 9] in the edge order of nl (rows contiguous), xn [9, N, C] m-major,
    C <= 256.  Gradients to Y and xn (per-row sums, deterministic)."""

    @staticmethod
    def forward(ctx, Y, xn, nl: NeighborList):
        _need_cuda(Y, xn)
        Y = Y.float().contiguous()
        xn = xn.float().contiguous()
        C = xn.shape[-1]
        if Y.shape != (nl.n_edges, 9) or xn.shape[:2] != (9, nl.n_atoms):
            raise ValueError(f"ShContractFn: Y {tuple(Y.shape)}, xn {tuple(xn.shape)} for {nl.n_edges} edges and "
                             f"{nl.n_atoms} rows")
        x0 = torch.empty(nl.n_edges, 3, C, dtype=torch.float32, device=Y.device)
        _lib.call("e2v2_sh_contract", _p(Y), _p(xn), _p(nl.row_ptr), _lib.i32(nl.n_atoms), _lib.i32(C), _p(x0),
                  _stream(Y))
        ctx.save_for_backward(Y, xn)
        ctx.nl = nl
        return x0

    @staticmethod
    def backward(ctx, g):
        _no_double_backward()
        Y, xn = ctx.saved_tensors
        nl = ctx.nl
        g = g.float().contiguous()
        dY = torch.empty_like(Y)
        dxn = torch.empty_like(xn)
        _lib.call("e2v2_sh_contract_bwd", _p(Y), _p(xn), _p(nl.row_ptr), _lib.i32(nl.n_atoms), _lib.i32(xn.shape[-1]),
                  _p(g), _p(dY), _p(dxn), _stream(Y))
        return dY, dxn, None
