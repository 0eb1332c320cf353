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

import torch
from torch import nn

from . import _lib
from .neighbors import NeighborList

ENV_EXPONENT = 5
ENV_A = -(ENV_EXPONENT + 1) * (ENV_EXPONENT + 2) / 2
ENV_B = ENV_EXPONENT * (ENV_EXPONENT + 2)
ENV_C = -ENV_EXPONENT * (ENV_EXPONENT + 1) / 2


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


def rbf_table_size(rc: float, rbf_coeff: float):
    """(nodes, spacing) of the rbf-block table for this basis and cutoff."""
    n = _lib.C.c_int32(); h = _lib.C.c_float()
    _lib.call("e2v2_mlp_rbf_table_size", _lib.f32(rc), _lib.f32(rbf_coeff), _lib.C.byref(n), _lib.C.byref(h))
    return n.value, h.value


class PackedMLP:
    """Device-ready weights of one RadialProfile [K0 + 2 E -> 128 -> 128 -> 256]
    (src/molfm/models/e2former/module_utils.py:2151-2178) whose input is
    [rbf(256), target_table[z_i], source_table[z_j]]: the rbf block of Linear1
    as an interpolation table over [0, rc] (e2v2_mlp_rbf_table), the type blocks
    as per-type tables, Linear2/3 as GEMM operands."""

    def __init__(self, net: nn.Sequential, tgt: torch.Tensor, src: torch.Tensor, rbf_offset: torch.Tensor,
                 rbf_coeff: float, rc: float, n_rbf: int = 256, bf16: bool = False):
        lin1, ln1, lin2, ln2, lin3 = net[0], net[1], net[3], net[4], net[6]
        self.bf16 = bf16
        if n_rbf != 256 or rbf_offset.numel() != 256:
            raise NotImplementedError("the HIP radial MLP is built for 256 Gaussian basis functions")
        with torch.no_grad():
            W1 = lin1.weight.detach().float().contiguous()
            e = tgt.shape[1]
            self.w1 = W1
            self.ttgt = (tgt.detach().float() @ W1[:, n_rbf:n_rbf + e].t() + lin1.bias.detach().float()).contiguous()
            self.tsrc = (src.detach().float() @ W1[:, n_rbf + e:n_rbf + 2 * e].t()).contiguous()
            self.g1 = ln1.weight.detach().float().contiguous(); self.be1 = ln1.bias.detach().float().contiguous()
            self.w2 = lin2.weight.detach().float().contiguous(); self.w2t = _lane_pack(self.w2.t())
            self.b2 = lin2.bias.detach().float().contiguous()
            self.g2 = ln2.weight.detach().float().contiguous(); self.be2 = ln2.bias.detach().float().contiguous()
            self.w3 = lin3.weight.detach().float().contiguous(); self.w3t = _lane_pack(self.w3.t())
            # fp32 GEMM B operands, lane-packed: forward W2^T, W3^T; backward W3, W2
            self.w2p = _lane_pack(self.w2); self.w3p = _lane_pack(self.w3)
            self.b3 = lin3.bias.detach().float().contiguous()
            # bf16 GEMM operands as B^T row-major: forward W2, W3; backward W3^T, W2^T
            self.bf = None
            if bf16:
                b = torch.bfloat16
                self.bf = [self.w2.to(b).contiguous(), self.w3.to(b).contiguous(),
                           self.w3.t().to(b).contiguous(), self.w2.t().to(b).contiguous()]
        if not (abs(ln1.eps - 1e-5) < 1e-12 and abs(ln2.eps - 1e-5) < 1e-12):
            raise NotImplementedError("RadialProfile LayerNorm eps must be 1e-5")
        if W1.shape[0] != 128 or self.w2.shape != (128, 128) or self.w3.shape != (256, 128):
            raise NotImplementedError(f"RadialProfile shape {tuple(W1.shape)} -> {tuple(self.w3.shape)} "
                                      "is not the [256+2E, 128, 128, 256] profile of the HIP kernels")
        self.rtab_n, self.rtab_h = rbf_table_size(rc, rbf_coeff)
        self.rtab = torch.empty(self.rtab_n, 4, 128, dtype=torch.float32, device=W1.device)
        self.rbf_offset = rbf_offset.detach().float().contiguous()
        _lib.call("e2v2_mlp_rbf_table", _p(W1), _lib.i32(W1.shape[1]), _p(self.rbf_offset), _lib.f32(rbf_coeff),
                  _lib.i32(self.rtab_n), _lib.f32(self.rtab_h), _p(self.rtab), _stream(W1))

    def struct(self) -> _lib.MlpWeights:
        bf = [t.data_ptr() for t in self.bf] if self.bf is not None else [None] * 4
        return _lib.MlpWeights(self.rtab.data_ptr(), self.rtab_n, self.rtab_h, self.ttgt.data_ptr(),
                               self.tsrc.data_ptr(), self.g1.data_ptr(), self.be1.data_ptr(), self.w2t.data_ptr(),
                               self.b2.data_ptr(), self.g2.data_ptr(), self.be2.data_ptr(), self.w3t.data_ptr(),
                               self.b3.data_ptr(), self.w2p.data_ptr(), self.w3p.data_ptr(), *bf)


def _lane_pack(B: torch.Tensor) -> torch.Tensor:
    """B [K][N] (fp32) in the lane-packed order of the HIP MLP's fp32 GEMMs: one
    float4 per (wave w, 16-column group ct, 16-k block b, lane l), holding
    B[16 b + 4 (l // 16) + s][w N/4 + 16 ct + l % 16] for s = 0..3."""
    K, N = B.shape
    return B.contiguous().view(K // 16, 4, 4, 4, N // 64, 16).permute(3, 4, 0, 1, 5, 2).contiguous()


def _version_key(params):
    return tuple((p.data_ptr(), p._version, p.dtype, str(p.device)) for p in params)


class MLPCache:
    """Repack weights only when a parameter (or the basis) changed (MD loops reuse them)."""

    def __init__(self):
        self.key = None
        self.packed: List[PackedMLP] = []

    def get(self, nets, tgt_emb: nn.Embedding, src_emb: nn.Embedding, rbf_offset: torch.Tensor, rbf_coeff: float,
            rc: float, bf16: bool = False):
        params = [p for n in nets for p in n.parameters()] + [tgt_emb.weight, src_emb.weight, rbf_offset]
        key = (_version_key(params), float(rbf_coeff), float(rc), bf16)
        if key != self.key:
            self.packed = [PackedMLP(n, tgt_emb.weight, src_emb.weight, rbf_offset, rbf_coeff, rc, bf16=bf16)
                           for n in nets]
            self.key = key
        return self.packed


def mlp_args(nl: NeighborList, node_type: torch.Tensor, packed: List[PackedMLP],
             save_n: Optional[torch.Tensor] = None, save_r: Optional[torch.Tensor] = None) -> _lib.MlpArgs:
    ws = (_lib.MlpWeights * 3)()
    for m, pk in enumerate(packed):
        ws[m] = pk.struct()
    bf16 = packed[0].bf16
    if any(pk.bf16 != bf16 for pk in packed):
        raise ValueError("mixed fp32/bf16 RadialProfile packs in one launch")
    return _lib.MlpArgs(nl.n_edges, len(packed), int(bf16), nl.dist.data_ptr(), nl.edge_row.data_ptr(),
                        nl.col.data_ptr(), node_type.data_ptr(),
                        None if save_n is None else save_n.data_ptr(), None if save_r is None else save_r.data_ptr(),
                        ws)


def mlp_save_buffers(n_mlp: int, E: int, dev):
    """Normalised LayerNorm inputs kept from the forward for the backward."""
    return (torch.empty(n_mlp, max(E, 1), 256, dtype=torch.float32, device=dev),
            torch.empty(n_mlp, max(E, 1), 2, dtype=torch.float32, device=dev))


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
    """EdgeDegreeEmbeddingNetwork_higherorder.forward (e2former.py:689-753)."""

    @staticmethod
    def forward(ctx, dvec, dist, nl: NeighborList, node_type, rbf_offset, rbf_coeff: float, packed, avg: float,
                rc: float):
        _need_cuda(dvec, dist)
        dev = dvec.device
        E, N = nl.n_edges, nl.n_atoms
        fea = torch.empty(max(E, 1), 3 * 256, dtype=torch.float32, device=dev)
        sn, sr = mlp_save_buffers(len(packed), E, dev)
        margs = mlp_args(nl, node_type, packed, sn, sr)
        _lib.call("e2v2_mlp_fwd", _lib.C.byref(margs), _p(fea), _lib.i32(768), _stream(fea))
        dargs = _lib.DegArgs(N, E, 256, nl.row_ptr.data_ptr(), nl.dvec.data_ptr(), nl.dist.data_ptr(),
                             fea.data_ptr(), float(avg), float(rc), ENV_A, ENV_B, ENV_C)
        x0 = torch.empty(9, N, 256, dtype=torch.float32, device=dev)   # m-major
        _lib.call("e2v2_deg_fwd", _lib.C.byref(dargs), _p(x0), _stream(x0))
        ctx.save_for_backward(fea, sn, sr)
        ctx.nl, ctx.margs_src = nl, (node_type, rbf_offset, rbf_coeff, packed)
        ctx.avg, ctx.rc = avg, rc
        return x0

    @staticmethod
    def backward(ctx, gx0):
        _no_double_backward()
        fea, sn, sr = ctx.saved_tensors
        nl = ctx.nl
        node_type, rbf_offset, rbf_coeff, packed = ctx.margs_src
        dev = fea.device
        E, N = nl.n_edges, nl.n_atoms
        gx0 = gx0.float().contiguous()
        dargs = _lib.DegArgs(N, E, 256, nl.row_ptr.data_ptr(), nl.dvec.data_ptr(), nl.dist.data_ptr(),
                             fea.data_ptr(), float(ctx.avg), float(ctx.rc), ENV_A, ENV_B, ENV_C)
        ddv = torch.empty(max(E, 1), 3, dtype=torch.float32, device=dev)
        dd = torch.empty(max(E, 1), dtype=torch.float32, device=dev)
        _lib.call("e2v2_deg_bwd", _lib.C.byref(dargs), _p(gx0), None, _p(ddv), _p(dd), _stream(gx0))
        margs = mlp_args(nl, node_type, packed, sn, sr)
        # the MLP backward forms the [E, 3, 256] feature gradient per edge tile from gx0
        _lib.call("e2v2_mlp_bwd_deg", _lib.C.byref(margs), _lib.C.byref(dargs), _p(gx0), _p(dd), _lib.i32(1),
                  _stream(gx0))
        return ddv[:E], dd[:E], None, None, None, None, None, None, None


def attn_args(nl: NeighborList, q, k, v, gi, q_div: float, rc: float, bf: int):
    """e2v2_attn_args over the neighbour list (with its column clusters when built)."""
    a = _lib.AttnArgs(nl.n_atoms, nl.n_edges, 128, 8, 256, nl.row_ptr.data_ptr(), nl.col.data_ptr(),
                      nl.edge_row.data_ptr(), nl.key_ptr.data_ptr(), nl.key_eid.data_ptr(), nl.dvec.data_ptr(),
                      nl.dist.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), gi.data_ptr(), float(q_div),
                      float(rc), ENV_A, ENV_B, ENV_C, int(bf))
    if nl.col_slot_member is not None:
        a.col_span = nl.col_span
        a.col_slot_member = nl.col_slot_member.data_ptr()
        a.col_slot_edge = nl.col_slot_edge.data_ptr()
        a.col_n_slots = nl.col_n_slots.data_ptr()
    return a


class AttentionFn(torch.autograd.Function):
    """Edge part of E2AttentionArbOrder_sparse.forward (e2former.py:238-433) up to
    the SO(2) product's forward_linear: returns the 20-row l3-sequential tensor
    h_a - h_b of so2_tensor_product.py:385 for every query atom, m-major
    [20, N, 256]; q, k [N, 128, 8], v [9, N, 256]."""

    @staticmethod
    def forward(ctx, q, k, v, dvec, dist, nl: NeighborList, node_type, rbf_offset, rbf_coeff: float, packed,
                rc: float, q_div: float, act_dtype=torch.float32):
        """act_dtype: storage of q, k, v and of the output rows (torch.float32, or
        torch.bfloat16 in the bf16 mode: half the gather traffic, fp32 math)."""
        _need_cuda(q, k, v, dvec, dist)
        if act_dtype not in (torch.float32, torch.bfloat16):
            raise ValueError(f"attention activations must be float32 or bfloat16, got {act_dtype}")
        dev = q.device
        E, N = nl.n_edges, nl.n_atoms
        q = q.to(act_dtype).contiguous(); k = k.to(act_dtype).contiguous(); v = v.to(act_dtype).contiguous()
        bf = int(act_dtype == torch.bfloat16)
        gi = torch.empty(max(E, 1), 256, dtype=torch.float32, device=dev)
        sn, sr = mlp_save_buffers(1, E, dev)
        margs = mlp_args(nl, node_type, packed, sn, sr)
        _lib.call("e2v2_mlp_fwd", _lib.C.byref(margs), _p(gi), _lib.i32(256), _stream(q))
        args = attn_args(nl, q, k, v, gi, q_div, rc, bf)
        out = torch.empty(20, N, 256, dtype=act_dtype, device=dev)   # m-major
        mrow = torch.empty(N, 128, dtype=torch.float32, device=dev)
        srow = torch.empty(N, 128, dtype=torch.float32, device=dev)
        cnt = torch.empty(N, 128, dtype=torch.int32, device=dev)
        _lib.call("e2v2_attn_fwd", _lib.C.byref(args), _p(out), _p(mrow), _p(srow), _p(cnt), _stream(q))
        ctx.save_for_backward(q, k, v, gi, out, mrow, srow, cnt, sn, sr)
        ctx.nl, ctx.margs_src, ctx.rc, ctx.q_div = nl, (node_type, rbf_offset, rbf_coeff, packed), rc, q_div
        ctx.bf = bf
        return out

    @staticmethod
    def backward(ctx, gout):
        _no_double_backward()
        q, k, v, gi, out, mrow, srow, cnt, sn, sr = ctx.saved_tensors
        nl = ctx.nl
        node_type, rbf_offset, rbf_coeff, packed = ctx.margs_src
        dev = q.device
        E, N = nl.n_edges, nl.n_atoms
        gout = gout.to(out.dtype).contiguous()
        args = attn_args(nl, q, k, v, gi, ctx.q_div, ctx.rc, ctx.bf)
        f = dict(dtype=torch.float32, device=dev)
        dgi = torch.empty(max(E, 1), 256, **f)
        ddv = torch.empty(max(E, 1), 3, **f)
        dd = torch.empty(max(E, 1), **f)
        dq = torch.empty(q.shape, **f); dk = torch.empty(k.shape, **f); dv = torch.empty(v.shape, **f)
        w_e = torch.empty(max(E, 1), 128, **f)
        dqk = torch.empty(max(E, 1), 128, **f)
        _lib.call("e2v2_attn_bwd", _lib.C.byref(args), _p(gout), _p(out), _p(mrow), _p(srow), _p(cnt), _p(dgi),
                  _p(ddv), _p(dd), _p(dq), _p(dk), _p(dv), _p(w_e), _p(dqk), _stream(gout))
        del w_e, dqk
        margs = mlp_args(nl, node_type, packed, sn, sr)
        _lib.call("e2v2_mlp_bwd", _lib.C.byref(margs), _p(dgi), _lib.i32(256), _p(dd), _lib.i32(1), _stream(gout))
        return dq, dk, dv, ddv[:E], dd[:E], None, None, None, None, None, None, None, None
