"""The training path: a twice-differentiable forward of the E2former decoder
for force training (``create_graph=True``: the reference's training step with
``AutoGradForce``, src/molfm/pipeline/head.py:305-328, differentiates the forces
once more through its second-order Triton classes,
triton_dr/triton_sparse_qk_autograd.py:754-836,
sparse_v_agg_edge_index_cblocked_bench.py:361-425,
edge_degree_outer_autograd.py:259-296).

The fused attention and degree kernels give first-order input gradients only.
In training mode (``module.train()``) the backbone instead composes each layer
from the op-level HIP functions of ``sparse_ops`` -- the segment QK dot, the
alpha sum, the value aggregation and the degree outer product, each with
second- and higher-order gradients -- and PyTorch ops for the per-node and
per-edge dense parts, as the reference composes them
(e2former.py:223-436, 623-753, 958-1145 with ``use_triton``), so gradients of
the forces reach every parameter and the positions.  The first-order SO(2)
product runs in its Cartesian form (the sum over the 9 value rows and the three
components of the edge vector with the coupling table of ``so3``; the identity
with the node-frame product is pinned in the tests), as three value
aggregations with weights w * dvec[:, k].  The radial profiles are evaluated per
edge (no distance tables: their parameters receive gradients).  fp32 only.

Every edge operation still runs on the GPU through libe2v2.so; nothing here
falls back to the CPU."""
from __future__ import annotations

import math
from typing import Optional

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from . import so3
from . import sparse_ops
from .ops import ENV_A, ENV_B, ENV_C

_EXPAND = {}
_CART = {}
_ROW0 = {}


def _expand(lmax: int, device) -> torch.Tensor:
    """Degree l of each of the (lmax + 1)^2 m-rows."""
    key = (lmax, str(device))
    if key not in _EXPAND:
        _EXPAND[key] = torch.tensor([l for l in range(lmax + 1) for _ in range(2 * l + 1)], device=device)
    return _EXPAND[key]


def _row0(n: int, ref: torch.Tensor) -> torch.Tensor:
    """[n, 1, 1] indicator of the degree-0 row in ref's dtype and device.  A bias
    on row 0 is added as row0 * bias over all rows (rows 1.. gain an exact
    zero), so neither pass of the double backward slices or concatenates the
    [n, N, C] tensor."""
    key = (n, ref.dtype, str(ref.device))
    if key not in _ROW0:
        m = torch.zeros(n, 1, 1, dtype=ref.dtype)
        m[0] = 1
        _ROW0[key] = m.to(ref.device)
    return _ROW0[key]


_LN_WIDTHS = (64, 128, 192, 256, 384, 512)


def _p(t: Optional[torch.Tensor]):
    return None if t is None else _lib.vp(t.data_ptr())


def _ln_parts(n: int) -> int:
    """Blocks (rows of the parameter partial sums) of the LayerNorm + SiLU gradient passes."""
    return max(1, min((n + 3) // 4, 2048))


class _LNSiLUFn(torch.autograd.Function):
    """silu(LayerNorm(x) * g + b) on rows x [n, w] (a RadialProfile's nn.LayerNorm +
    nn.SiLU, module_utils.py:2151-2178) through e2v2_ln_silu_fwd; its backward is
    _LNSiLUGradFn, itself differentiable once more, so the forces' parameter and
    position gradients come from two fused kernels instead of torch's composed
    double backward of layer_norm and silu."""

    @staticmethod
    def forward(ctx, x, g, b, eps: float):
        n, w = x.shape
        y = torch.empty_like(x)
        st = x.new_empty(n, 2)
        _lib.call("e2v2_ln_silu_fwd", _p(x), _p(g), _p(b), _p(y), _p(st), _lib.i32(n), _lib.i32(w), _lib.f32(eps),
                  sparse_ops._stream(x.device))
        ctx.save_for_backward(x, g, b, st)
        return y

    @staticmethod
    def backward(ctx, gy):
        x, g, b, st = ctx.saved_tensors
        gx, gg, gb = _LNSiLUGradFn.apply(gy, x, g, b, st)
        return gx, gg, gb, None


class _LNSiLUGradFn(torch.autograd.Function):
    """(gx, dg, db) of _LNSiLUFn given gy (e2v2_ln_silu_bwd_param); its backward is
    the second-order pass e2v2_ln_silu_bwd2 (mean and rstd enter as constants: the
    kernel differentiates through them analytically)."""

    @staticmethod
    def forward(ctx, gy, x, g, b, st):
        gy = gy.contiguous()
        n, w = x.shape
        npart = _ln_parts(n)
        gx = torch.empty_like(x)
        pg, pb = x.new_empty(npart, w), x.new_empty(npart, w)
        _lib.call("e2v2_ln_silu_bwd_param", _p(x), _p(g), _p(b), _p(st), _p(gy), _p(gx), _p(pg), _p(pb),
                  _lib.i32(n), _lib.i32(w), _lib.i32(npart), sparse_ops._stream(x.device))
        ctx.save_for_backward(gy, x, g, b, st)
        ctx.set_materialize_grads(False)
        return gx, pg.sum(0), pb.sum(0)

    @staticmethod
    def backward(ctx, qx, qg, qb):
        gy, x, g, b, st = ctx.saved_tensors
        n, w = x.shape
        npart = _ln_parts(n)
        qx = None if qx is None else qx.contiguous()
        qg = None if qg is None else qg.contiguous()
        qb = None if qb is None else qb.contiguous()
        dgy, dx = torch.empty_like(x), torch.empty_like(x)
        pg, pb = x.new_empty(npart, w), x.new_empty(npart, w)
        _lib.call("e2v2_ln_silu_bwd2", _p(x), _p(g), _p(b), _p(st), _p(gy), _p(qx), _p(qg), _p(qb), _p(dgy),
                  _p(dx), _p(pg), _p(pb), _lib.i32(n), _lib.i32(w), _lib.i32(npart), sparse_ops._stream(x.device))
        return dgy, dx, pg.sum(0), pb.sum(0), None


_EDGE_ROWS = 16384   # rows from which a Linear takes the split-K weight gradient


def _will_run(node) -> bool:
    """Whether the running backward needs the gradient flowing into node (False
    only when the engine reports that it will not execute it: autograd.grad of
    other inputs, as the forces' first differentiation)."""
    if node is None:
        return False
    try:
        return bool(torch._C._will_engine_execute_node(node))
    except (AttributeError, RuntimeError):
        return True


def _splitk_tn(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a^T b for a [E, m], b [E, n] with E >> m, n: s batched partial products
    over row blocks, summed (one GEMM with K = E leaves most of the chip idle)."""
    a, b = a.contiguous(), b.contiguous()
    E = a.shape[0]
    s = max(1, min(32, E // 2048))
    if s == 1:
        return a.t() @ b
    E0 = E // s * s
    out = torch.bmm(a[:E0].view(s, E0 // s, -1).transpose(1, 2), b[:E0].view(s, E0 // s, -1)).sum(0)
    if E0 < E:
        out = out + a[E0:].t() @ b[E0:]
    return out


class _EdgeLinearFn(torch.autograd.Function):
    """y = x W^T (+ b) on per-edge rows x [E, k] (the nn.Linear layers of the
    RadialProfile nets, module_utils.py:2151-2178) with gradients of any order:
    the input gradient is this function again (gy W), the weight gradient the
    split-K _EdgeWGradFn, skipped when the running backward does not need it."""

    @staticmethod
    def forward(ctx, x, W, b):
        ctx.save_for_backward(x, W)
        ctx.has_b = b is not None
        return torch.addmm(b, x, W.t()) if b is not None else x @ W.t()

    @staticmethod
    def backward(ctx, gy):
        x, W = ctx.saved_tensors
        nxt = ctx.next_functions
        gx = _EdgeLinearFn.apply(gy, W.t(), None) if ctx.needs_input_grad[0] else None
        gW = _EdgeWGradFn.apply(gy, x) if ctx.needs_input_grad[1] and _will_run(nxt[1][0]) else None
        gb = gy.sum(0) if ctx.has_b and ctx.needs_input_grad[2] and _will_run(nxt[2][0]) else None
        return gx, gW, gb


class _EdgeWGradFn(torch.autograd.Function):
    """a^T b over the edge rows (split-K); gradients b Q^T and a Q."""

    @staticmethod
    def forward(ctx, a, b):
        ctx.save_for_backward(a, b)
        return _splitk_tn(a, b)

    @staticmethod
    def backward(ctx, Q):
        a, b = ctx.saved_tensors
        ga = _EdgeLinearFn.apply(b, Q, None) if ctx.needs_input_grad[0] else None
        gb = _EdgeLinearFn.apply(a, Q.t(), None) if ctx.needs_input_grad[1] else None
        return ga, gb


def edge_linear(lin: nn.Linear, x: torch.Tensor) -> torch.Tensor:
    """lin(x) on per-edge rows through _EdgeLinearFn."""
    return _EdgeLinearFn.apply(x, lin.weight, lin.bias)


def ln_silu_fusable(ln: nn.LayerNorm, x: torch.Tensor) -> bool:
    """Whether _LNSiLUFn takes silu(ln(x)): fp32 GPU rows of a width the kernels
    are built for and an affine LayerNorm over that width with fp32 parameters."""
    w = x.shape[-1]
    return (x.is_cuda and x.dtype == torch.float32 and tuple(ln.normalized_shape) == (w,) and w in _LN_WIDTHS
            and ln.weight is not None and ln.bias is not None and ln.weight.dtype == torch.float32
            and ln.bias.dtype == torch.float32 and ln.weight.is_contiguous() and ln.bias.is_contiguous())


def ln_silu(ln: nn.LayerNorm, x: torch.Tensor) -> torch.Tensor:
    """silu(ln(x)) over the last dimension through _LNSiLUFn."""
    sparse_ops._need_gpu(x)
    if not ln_silu_fusable(ln, x):
        raise ValueError(f"ln_silu: fp32 rows of width {_LN_WIDTHS} with an fp32 affine LayerNorm, got "
                         f"{tuple(x.shape)} {x.dtype}")
    w = x.shape[-1]
    y = _LNSiLUFn.apply(x.reshape(-1, w).contiguous(), ln.weight, ln.bias, float(ln.eps))
    return y.view(x.shape)


def run_seq(mods, h: torch.Tensor) -> torch.Tensor:
    """nn.Sequential over mods with each nn.LayerNorm + nn.SiLU pair as ln_silu (where
    ln_silu_fusable; other widths run the two modules) and each nn.Linear on at
    least _EDGE_ROWS rows as edge_linear."""
    mods = list(mods) if isinstance(mods, (nn.Sequential, list, tuple)) else [mods]
    i = 0
    while i < len(mods):
        if (isinstance(mods[i], nn.LayerNorm) and i + 1 < len(mods) and isinstance(mods[i + 1], nn.SiLU)
                and ln_silu_fusable(mods[i], h)):
            h = ln_silu(mods[i], h)
            i += 2
        elif isinstance(mods[i], nn.Linear) and h.dim() == 2 and h.shape[0] >= _EDGE_ROWS:
            h = edge_linear(mods[i], h)
            i += 1
        else:
            h = mods[i](h)
            i += 1
    return h


def _cartesian(device) -> torch.Tensor:
    """The Cartesian coupling table T [20, 9, 3] of the first-order product."""
    key = str(device)
    if key not in _CART:
        _CART[key] = torch.as_tensor(np.asarray(so3.cartesian_tp_table(), np.float32), device=device)
    return _CART[key]


# --------------------------------------------------------------------------- per-node layers (m-major [9, N, C])

def so3_linear(mod, x: torch.Tensor) -> torch.Tensor:
    """SO3_Linear_e2former (module_utils.py:2010-2052): row m times W_l(m)^T, the
    bias on row 0."""
    w = mod.weight.index_select(0, _expand(mod.lmax, x.device))          # [9, Cout, Cin]
    out = torch.matmul(x, w.transpose(1, 2))
    return out + _row0(out.shape[0], out) * mod.bias.reshape(-1)


def so3_linear2scalar(mod, x: torch.Tensor) -> torch.Tensor:
    """SO3_Linear2Scalar_e2former (module_utils.py:2198-2272): two SO(3) linears
    (the bias on the first one's row 0), their m-contraction per degree, then
    final_linear."""
    e = _expand(mod.lmax, x.device)
    a = torch.matmul(x, mod.weight.index_select(0, e).transpose(1, 2))
    a = a + _row0(a.shape[0], a) * mod.bias.reshape(-1)
    b = torch.matmul(x, mod.weight2.index_select(0, e).transpose(1, 2))
    ab = (a * b).split([2 * l + 1 for l in range(mod.lmax + 1)], dim=0)
    return run_seq(mod.final_linear, torch.cat([p.sum(0) for p in ab], dim=-1))


class _RMSNormFn(torch.autograd.Function):
    """rms_norm_sh on x [9, N, 256] (e2v2_rmsnorm_fwd; the module's balance weights
    are the kernels' 1 / ((2l + 1)(lmax + 1))); its backward is _RMSNormGradFn,
    differentiable once more, in place of the composed norm's double backward."""

    @staticmethod
    def forward(ctx, x, w, b, eps: float):
        n = x.shape[1]
        y = torch.empty_like(x)
        _lib.call("e2v2_rmsnorm_fwd", _p(x), _p(w), _p(b), _p(y), _lib.i32(n), _lib.f32(eps),
                  sparse_ops._stream(x.device))
        ctx.save_for_backward(x, w)
        ctx.eps = eps
        return y

    @staticmethod
    def backward(ctx, gy):
        x, w = ctx.saved_tensors
        gx, gw, gb = _RMSNormGradFn.apply(gy, x, w, ctx.eps)
        return gx, gw, gb, None


def _rms_parts(n: int) -> int:
    return max(1, min(n, 1024))


class _RMSNormGradFn(torch.autograd.Function):
    """(gx, dw, db) of _RMSNormFn given gy (e2v2_rmsnorm_bwd_param); its backward
    is e2v2_rmsnorm_bwd2."""

    @staticmethod
    def forward(ctx, gy, x, w, eps: float):
        gy = gy.contiguous()
        n = x.shape[1]
        npart = _rms_parts(n)
        gx = torch.empty_like(x)
        part = x.new_empty(npart, 4, x.shape[2])
        _lib.call("e2v2_rmsnorm_bwd_param", _p(x), _p(w), _p(gy), _p(gx), _p(part), _lib.i32(n), _lib.i32(npart),
                  _lib.f32(eps), sparse_ops._stream(x.device))
        ctx.save_for_backward(gy, x, w)
        ctx.eps = eps
        ctx.set_materialize_grads(False)
        p = part.sum(0)
        return gx, p[:3].contiguous(), p[3].contiguous()

    @staticmethod
    def backward(ctx, qx, qw, qb):
        gy, x, w = ctx.saved_tensors
        n = x.shape[1]
        npart = _rms_parts(n)
        qx = None if qx is None else qx.contiguous()
        qw = None if qw is None else qw.contiguous()
        qb = None if qb is None else qb.contiguous()
        dgy, dx = torch.empty_like(x), torch.empty_like(x)
        part = x.new_empty(npart, 3, x.shape[2])
        _lib.call("e2v2_rmsnorm_bwd2", _p(x), _p(w), _p(gy), _p(qx), _p(qw), _p(qb), _p(dgy), _p(dx), _p(part),
                  _lib.i32(n), _lib.i32(npart), _lib.f32(ctx.eps), sparse_ops._stream(x.device))
        return dgy, dx, part.sum(0), None


def rms_norm(mod, x: torch.Tensor) -> torch.Tensor:
    """EquivariantRMSNormArraySphericalHarmonicsV2_BL (module_utils.py:1663-1772):
    row 0 centred over the channels, the degree-balanced mean square over rows
    and channels, the affine weight of each row's degree, the bias on row 0.
    fp32 GPU rows [9, N, 256] run _RMSNormFn; other inputs the composition below."""
    if (x.is_cuda and x.dtype == torch.float32 and x.dim() == 3 and tuple(x.shape[::2]) == (9, 256)
            and mod.lmax == 2 and mod.affine_weight.dtype == torch.float32 and mod.affine_weight.is_contiguous()):
        return _RMSNormFn.apply(x.contiguous(), mod.affine_weight, mod.affine_bias, float(mod.eps))
    r0 = _row0(x.shape[0], x)
    f = x - x.mean(dim=2, keepdim=True) * r0
    bw = mod.balance_degree_weight.view(-1, 1, 1).to(x.dtype)
    fn = (f.pow(2) * bw).sum(0, keepdim=True).mean(dim=2, keepdim=True)
    fn = (fn + mod.eps).pow(-0.5)
    w = mod.affine_weight.index_select(0, _expand(mod.lmax, x.device)).unsqueeze(1)
    return f * (fn * w) + r0 * mod.affine_bias.reshape(-1)


class _GateActFn(torch.autograd.Function):
    """Gate_s3's activations on x [9, N, 256] from the logits sc [N, 768]
    (e2v2_gate_fwd); backward _GateActGradFn, differentiable once more."""

    @staticmethod
    def forward(ctx, sc, x, k1: float, k2: float):
        y = torch.empty_like(x)
        _lib.call("e2v2_gate_fwd", _p(sc), _p(x), _p(y), _lib.i32(x.shape[1]), _lib.f32(k1), _lib.f32(k2),
                  sparse_ops._stream(x.device))
        ctx.save_for_backward(sc, x)
        ctx.k = (k1, k2)
        return y

    @staticmethod
    def backward(ctx, gy):
        sc, x = ctx.saved_tensors
        gsc, gx = _GateActGradFn.apply(gy, sc, x, *ctx.k)
        return gsc, gx, None, None


class _GateActGradFn(torch.autograd.Function):
    """(gsc, gx) of _GateActFn given gy (e2v2_gate_bwd); backward e2v2_gate_bwd2."""

    @staticmethod
    def forward(ctx, gy, sc, x, k1: float, k2: float):
        gy = gy.contiguous()
        gsc, gx = torch.empty_like(sc), torch.empty_like(x)
        _lib.call("e2v2_gate_bwd", _p(sc), _p(x), _p(gy), _p(gsc), _p(gx), _lib.i32(x.shape[1]), _lib.f32(k1),
                  _lib.f32(k2), sparse_ops._stream(x.device))
        ctx.save_for_backward(gy, sc, x)
        ctx.k = (k1, k2)
        ctx.set_materialize_grads(False)
        return gsc, gx

    @staticmethod
    def backward(ctx, qsc, qx):
        gy, sc, x = ctx.saved_tensors
        qsc = None if qsc is None else qsc.contiguous()
        qx = None if qx is None else qx.contiguous()
        dgy, dsc, dx = torch.empty_like(x), torch.empty_like(sc), torch.empty_like(x)
        _lib.call("e2v2_gate_bwd2", _p(sc), _p(x), _p(gy), _p(qsc), _p(qx), _p(dgy), _p(dsc), _p(dx),
                  _lib.i32(x.shape[1]), _lib.f32(ctx.k[0]), _lib.f32(ctx.k[1]), sparse_ops._stream(x.device))
        return dgy, dsc, dx, None, None


def gate_s3(mod, x: torch.Tensor, silu_norm: float, sigmoid_norm: float) -> torch.Tensor:
    """Gate_s3 (module_utils.py:2694-2746): logits from row 0, SiLU on row 0,
    the sigmoid of each degree's logits on its rows.  fp32 GPU rows [9, N, 256]
    take the activations through _GateActFn; other inputs the composition."""
    C, n, N = mod.sphere_channels, x.shape[0], x.shape[1]
    lmax = math.isqrt(n) - 1
    x0, xr = x.split([1, n - 1], dim=0)
    if x.is_cuda and x.dtype == torch.float32 and n == 9 and C == 256 and x.shape[2] == 256:
        sc = mod.gates(x0.squeeze(0)).contiguous()
        return _GateActFn.apply(sc, x.contiguous(), float(silu_norm), float(sigmoid_norm))
    s0, sr = mod.gates(x0.squeeze(0)).split([C, lmax * C], dim=1)
    g = torch.sigmoid(sr).view(N, lmax, C).transpose(0, 1)                # [lmax, N, C]
    g = g.index_select(0, _expand(lmax, x.device)[1:] - 1)                # row m <- its degree
    return torch.cat([(F.silu(s0) * silu_norm).unsqueeze(0), g * sigmoid_norm * xr], dim=0)


def ffn(mod, x: torch.Tensor, silu_norm: float, sigmoid_norm: float) -> torch.Tensor:
    """FeedForwardNetwork_s3 (module_utils.py:2755-2797)."""
    return so3_linear(mod.slinear_2, gate_s3(mod.gate, so3_linear(mod.slinear_1, x), silu_norm, sigmoid_norm))


# --------------------------------------------------------------------------- edges

class TrainEdges:
    """The edge inputs of one neighbour list for the training path: query row
    and source atom of every edge (query-row order), the edge vector and distance
    as differentiable functions of the positions, each atom's atomic number, the
    Gaussian basis and cutoff, the envelope, and the segment metadata of the
    sparse ops built from the neighbour list's own CSRs (no sort)."""

    def __init__(self, ctx, pos: torch.Tensor):
        nl = ctx.nl
        N, E = nl.n_atoms, nl.n_edges
        self.nl, self.rc, self.N, self.E = nl, float(ctx.rc), N, E
        self.row32, self.col32 = nl.edge_row[:E].contiguous(), nl.col[:E].contiguous()
        self.qi, self.nj = self.row32.long(), self.col32.long()
        # the cell shift of each edge, a constant: dvec = pos_i - pos_j + off
        base = pos[self.qi] - pos[self.nj]
        off = (nl.dvec[:E] - base.detach()).detach()
        self.dvec = base + off
        self.dist = self.dvec.norm(dim=-1)
        self.Z = ctx.type_z.long()[ctx.atom_type.long()]
        self.offset, self.coeff = ctx.rbf_offset, float(ctx.rbf_coeff)
        self.env_kind, self.env_lo = ctx.env_kind, ctx.env_lo
        eid = torch.arange(E, dtype=torch.int32, device=pos.device)
        key_eid = nl.key_eid[:E].contiguous()
        # (query row_ptr, partner rows, edge ids) then the same by key: the 6-tuple of
        # prepare_sparse_qk_edge_index_metadata for an edge list in row order
        self.md = (nl.row_ptr, self.col32, eid, nl.key_ptr, self.row32.index_select(0, key_eid.long()), key_eid)

    def rbf(self) -> torch.Tensor:
        """GaussianSmearing (module_utils.py:1853-1869) of the distances."""
        return torch.exp(self.coeff * (self.dist.view(-1, 1) - self.offset.view(1, -1)).pow(2))

    def envelope(self) -> torch.Tensor:
        """polynomial(d, rc) (module_utils.py:1946-1954) or, for the long-range
        list of with_cluster "node_bell", smooth_polynomial_bell(d, lo, rc)
        (module_utils.py:1956-1985)."""
        d = self.dist
        if self.env_kind == 0:
            r = d / self.rc
            return torch.where(r < 1, 1 + r ** 5 * (ENV_A + r * (ENV_B + ENV_C * r)), torch.zeros_like(r))
        lo, hi = self.env_lo, max(self.rc, self.env_lo + 1e-8)
        t = torch.clamp((2 * d - (lo + hi)) / (hi - lo), -1.0, 1.0)
        return (1.0 - t * t) ** 2

    def edge_input(self, tgt_emb, src_emb, rbf: torch.Tensor) -> "EdgeInput":
        """x_edge = [rbf(d), tgt[z_i], src[z_j]] (e2former.py:258-266, 709-733), applied to
        radial profiles without being formed (EdgeInput)."""
        return EdgeInput(self, tgt_emb, src_emb, rbf)


    def gather_q(self, x: torch.Tensor) -> torch.Tensor:
        """x [N, F] -> x[qi] [E, F] (gradient: the sum over each query row's edges)."""
        return sparse_ops.sparse_gather_edge_index(x, self.row32, self.N, (self.md[0], self.md[2]))

    def gather_k(self, x: torch.Tensor) -> torch.Tensor:
        """x [N, F] -> x[nj] [E, F] (gradient: the sum over each source atom's edges)."""
        return sparse_ops.sparse_gather_edge_index(x, self.col32, self.N, (self.md[3], self.md[5]))

    def qk(self, q: torch.Tensor, k: torch.Tensor) -> torch.Tensor:
        return sparse_ops.sparse_qk_edge_index_triton(q, k, self.row32, self.col32, metadata=self.md)

    def v_agg(self, value: torch.Tensor, alpha: torch.Tensor) -> torch.Tensor:
        """value [N, Cv, H], alpha [E, H] -> [N, Cv, H]."""
        return sparse_ops.sparse_v_agg_edge_index_triton_cblocked(value, alpha, self.row32, self.col32, self.N,
                                                                 metadata=self.md)

    def row_sum(self, alpha: torch.Tensor) -> torch.Tensor:
        return sparse_ops.sparse_alpha_sum_edge_index_triton(alpha, self.row32, self.N,
                                                            metadata=(self.nl.row_ptr, self.md[2]))

    def outer(self, sh: torch.Tensor, fea: torch.Tensor) -> torch.Tensor:
        return sparse_ops.edge_degree_outer_triton(sh, fea, self.row32, self.N,
                                                  metadata=(self.nl.row_ptr, None, self.md[2], None, None, None))


class EdgeInput:
    """x_edge = [rbf(d), tgt[z_i], src[z_j]] as the input of RadialProfile nets
    (module_utils.py:2151-2178) without the [E, 256 + 2 n_emb] tensor: the first
    Linear's type blocks act on the embedding rows per atom and are gathered per edge,
    W x_edge + b = W_rbf rbf + (tgt[Z] W_t^T)[i] + (src[Z] W_s^T)[j] + b (the same sum,
    fp32 rounding of another association); the rest of the net follows unchanged, so
    every parameter (the embeddings included) keeps its gradients to any order."""

    def __init__(self, edges, tgt_emb, src_emb, rbf: torch.Tensor):
        self.edges, self.tgt, self.src, self.rbf = edges, tgt_emb, src_emb, rbf

    def __call__(self, prof) -> torch.Tensor:
        net = prof.net
        lin1 = net[0]
        K, ne = self.rbf.shape[1], self.tgt.weight.shape[1]
        W = lin1.weight
        e = self.edges
        ht = self.tgt(e.Z) @ W[:, K:K + ne].t()                  # [N, hidden] per atom
        hs = self.src(e.Z) @ W[:, K + ne:K + 2 * ne].t()
        h = _EdgeLinearFn.apply(self.rbf, W[:, :K], lin1.bias) + e.gather_q(ht) + e.gather_k(hs)
        return run_seq(net[1:], h)


class _RowMaxFn(torch.autograd.Function):
    """m[i, h] = max over the edges of row i of logit[e, h] (scatter_reduce amax from
    -inf, e2former.py:335-347), with scatter_reduce's gradient -- g[i, h] split evenly
    over the edges that attain the maximum -- composed from the segment gather and
    row sum, so its own derivative comes from those ops (the tie mask is piecewise
    constant in the logits)."""

    @staticmethod
    def forward(ctx, logit, edges):
        H = logit.shape[1]
        m = torch.full((edges.N, H), -torch.inf, dtype=logit.dtype, device=logit.device)
        m = m.scatter_reduce(0, edges.qi.view(-1, 1).expand(-1, H), logit, reduce="amax", include_self=True)
        ctx.save_for_backward(logit, m)
        ctx.edges = edges
        return m

    @staticmethod
    def backward(ctx, g):
        logit, m = ctx.saved_tensors
        edges = ctx.edges
        tie = (logit == edges.gather_q(m)).to(logit.dtype)
        cnt = edges.row_sum(tie).clamp_min(1.0)
        return edges.gather_q(g / cnt) * tie, None


def attention_weights(logit, p, ih, edges: TrainEdges, form: str) -> torch.Tensor:
    """alpha [E, H] (e2former.py:327-364): the segmented softmax with the row
    maximum by scatter_reduce(amax) (its gradient split over ties) and the
    +1e-3 in the denominator, or the softplus / sigmoid forms."""
    if form == "softplus":
        return F.softplus(logit) * ih * p.unsqueeze(-1)
    if form == "sigmoid":
        return torch.sigmoid(logit) * ih * p.unsqueeze(-1)
    amax = _RowMaxFn.apply(logit, edges)
    e = torch.exp(logit - edges.gather_q(amax)) * p.unsqueeze(-1)
    s = edges.row_sum(e)
    return e * ih * edges.gather_q(1.0 / (s + 1e-3))       # the reciprocal per row, not per edge


def _sh_integral(v: torch.Tensor) -> torch.Tensor:
    from .modules import _sh_integral as f
    return f(v)


def _raw_sh(v: torch.Tensor) -> torch.Tensor:
    from .modules import _raw_sh as f
    return f(v)


def qkdot_gate(ga, x: torch.Tensor, edges: TrainEdges, x_edge: EdgeInput):
    """(gate, inputhead) of the QKdot variants (e2former.py:270-300)."""
    H = ga.num_attn_heads
    xd = so3_linear(ga.dot_linear, x)                                        # [9, N, Cd]
    L9, N, Cd = xd.shape
    xq = edges.gather_q(xd.permute(1, 0, 2).reshape(N, L9 * Cd)).view(-1, L9, Cd).permute(1, 0, 2)  # [9, E, Cd]
    if ga.tp_type == "QKdot_alpha":
        Y = _sh_integral(edges.dvec)                                         # [E, 9]
        x0 = torch.cat([(Y[:, l * l:(l + 1) ** 2].t().unsqueeze(-1) * xq[l * l:(l + 1) ** 2]).sum(0)
                        for l in range(ga.lmax + 1)], dim=-1)                # [E, 3 Cd]
        gate = ga.fc_m0(x0 * x_edge(ga.rad_func_m0))
        return gate, x_edge(ga.fc_easy).reshape(-1, H)
    lxs = _raw_sh(edges.dvec)                                                # [E, 9]
    x0 = torch.einsum("lec,el,ls->esc", xq, lxs, ga.sum_vec.to(xq.dtype)).reshape(xq.shape[1], -1)[:, :H]
    ih, eg = x_edge(ga.fc_easy).split([H, x0.shape[1]], dim=1)
    return run_seq(ga.direction_linear, x0 * eg), ih


def so2_forward_linear(tp, so2: torch.Tensor) -> torch.Tensor:
    """SO2_TP_givenl2.forward_linear (so2_tensor_product.py:276-290) on the 20
    l3-sequential rows [20, N, C]: per output degree its cnt paths side by side
    through out_linear, times path_norm; rows scaled by any loaded CG_weight
    path scale first."""
    sc = tp.path_scales()
    if sc is not None:
        so2 = so2 * sc.view(-1, 1, 1).to(so2.dtype)
    N = so2.shape[1]
    outs = []
    parts = so2.split([cnt * (2 * l3 + 1) for l3, cnt in tp.l3_sequential], dim=0)
    for idx, ((l3, cnt), part) in enumerate(zip(tp.l3_sequential, parts)):
        nr = 2 * l3 + 1
        blk = part.reshape(cnt, nr, N, -1).permute(1, 2, 0, 3).reshape(nr, N, -1)
        outs.append(tp.out_linear[idx](blk))
    return torch.cat(outs, dim=0) * tp.path_norm.view(-1, 1, 1).to(so2.dtype)


def attention(ga, x: torch.Tensor, edges: TrainEdges, rbf: torch.Tensor) -> torch.Tensor:
    """E2AttentionArbOrder_sparse.forward (e2former.py:223-436) on x [9, N, C]."""
    N, H = x.shape[1], ga.num_attn_heads
    q = so3_linear2scalar(ga.query_linear, x).reshape(N, H, -1)
    k = so3_linear2scalar(ga.key_linear, x).reshape(N, H, -1)
    x_edge = edges.edge_input(ga.target_embedding, ga.source_embedding, rbf)
    if ga.tp_type == "QK_alpha":
        eg = x_edge(ga.fc_easy)
        gate, ih = eg.split([H, eg.shape[1] - H], dim=1)
    else:
        gate, ih = qkdot_gate(ga, x, edges, x_edge)
    qk = edges.qk(q / math.sqrt(q.shape[-1]), k)
    alpha = attention_weights(gate * qk, edges.envelope(), ih, edges, ga.weight_act)
    alpha = ga.alpha_dropout(alpha)
    v = so3_linear(ga.proj_value, x)                                         # [9, N, C]
    C = v.shape[-1]
    vh = v.permute(1, 0, 2).reshape(N, -1, H)                                # channel c -> head c mod H
    if ga.attn_type == "zero-order":
        agg = edges.v_agg(vh, alpha).reshape(N, -1, C).permute(1, 0, 2)      # [9, N, C]
        return so3_linear(ga.proj_zero, agg)
    T = _cartesian(x.device)
    so2, u = 0, (edges.dvec / edges.dist.clamp_min(1e-6).unsqueeze(-1)).unbind(1)   # alpha / d * dvec_k
    for kk in range(3):
        a = edges.v_agg(vh, alpha * u[kk].unsqueeze(-1)).reshape(N, -1, C)    # [N, 9, C]
        so2 = so2 + torch.einsum("tr,nrc->tnc", T[:, :, kk], a)
    return so3_linear(ga.proj_first, so2_forward_linear(ga.first_order_tp.so2_tp, so2))


def degree_embedding(mod, edges: TrainEdges, rbf: torch.Tensor) -> torch.Tensor:
    """EdgeDegreeEmbeddingNetwork_higherorder.forward (e2former.py:689-753):
    per degree the profile times the envelope, its outer product with the
    unit-vector spherical harmonics reduced over each row, / avg."""
    emb = edges.edge_input(mod.target_embedding, mod.source_embedding, rbf)
    u = F.normalize(edges.dvec, dim=-1)
    lxs = _raw_sh(u)
    p = edges.envelope().view(-1, 1)
    rows = []
    for l in range(mod.lmax + 1):
        fea = emb(mod.gbf_projs[l]) * p
        rows.append(edges.outer(lxs[:, l * l:(l + 1) ** 2].contiguous(), fea))   # [N, 2l+1, C]
    return torch.cat(rows, dim=1).permute(1, 0, 2) / mod.avg_aggregate_num


def block(blk, x: torch.Tensor, edges: TrainEdges, rbf: torch.Tensor, sys_node, norms) -> torch.Tensor:
    """TransBlock.forward (e2former.py:600-620): pre-norm residual attention and FFN."""
    h = rms_norm(blk.norm_1, x)
    if sys_node is not None:
        h = h + _row0(h.shape[0], h) * sys_node
    x = x + attention(blk.ga, h, edges, rbf)
    return x + ffn(blk.ffn, rms_norm(blk.norm_ffn, x), *norms)


def decoder_forward(dec, ctx, pos: torch.Tensor, sys_node: Optional[torch.Tensor] = None, long_ctx=None):
    """E2former's decoder (e2former.py:958-1145) on the training path: node
    irreps [9, N, C] as twice-differentiable functions of pos and the parameters."""
    from .modules import SILU_NORM, SIGMOID_NORM
    if ctx.bf16:
        raise NotImplementedError("the training path runs in fp32 (set_compute_dtype('fp32'))")
    norms = (SILU_NORM, SIGMOID_NORM)
    edges = TrainEdges(ctx, pos)
    rbf = edges.rbf()
    x = degree_embedding(dec.edge_deg_embed_dense, edges, rbf)
    for blk in dec.blocks:
        x = block(blk, x, edges, rbf, sys_node, norms)
    if not dec.cluster:
        return rms_norm(dec.norm_final, x)
    if long_ctx is None:
        raise ValueError("cluster_neighbor_info is required when with_cluster contains 'node'.")
    short = x
    x = rms_norm(dec.pre_norm_node, x)
    long_edges = TrainEdges(long_ctx, pos)
    rbf_l = long_edges.rbf()
    for blk in dec.long_blocks:
        x = block(blk, x, long_edges, rbf_l, sys_node, norms)
    x = rms_norm(dec.norm_cluster, x)
    return so3_linear(dec.final_linear, torch.cat([short, x], dim=-1))
