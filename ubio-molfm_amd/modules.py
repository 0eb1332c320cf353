"""E2Former-V2 module tree on the HIP edge path.

Class names, constructor arguments, parameter/buffer names and shapes follow the
reference (src/molfm/models/e2former/e2former.py, module_utils.py,
wigner6j/so2_tensor_product.py), so a reference state_dict loads with
``strict=True``.  Every edge-level operation runs in libe2v2.so through ``ops``;
the per-node dense layers run as fp32 GEMMs on bf16 MFMA by the exact
three-piece operand split of ``gemm`` (e2v2_gemm_s3) in fp32 mode, and as bf16
hipBLASLt GEMMs in bf16 mode.  ``E2V2_FP32_GEMM=native`` in the environment
selects hipBLASLt's fp32 GEMMs instead of the split ones (a measurement switch).
"""
from __future__ import annotations

import math
import os
from typing import Optional

import numpy as np
import torch
from torch import nn
from torch.profiler import record_function

from . import so3
from . import _lib
from . import gemm as s3gemm
from .ops import AttentionFn, DegreeEmbedFn, QKdotGateFn, RadialCache, RadialEvalFn, ShContractFn, \
    attention_backward, attention_forward


def _e3nn_normalize2mom(f) -> float:
    """Second-moment normaliser of e3nn.math.normalize2mom: (E[f(z)^2])^-1/2 from
    1e6 float64 N(0,1) samples of torch.Generator().manual_seed(0)."""
    gen = torch.Generator(device="cpu").manual_seed(0)
    z = torch.randn(1_000_000, generator=gen, dtype=torch.float64)
    return f(z).pow(2).mean().pow(-0.5).item()


SILU_NORM = _e3nn_normalize2mom(torch.nn.functional.silu)
SIGMOID_NORM = _e3nn_normalize2mom(torch.sigmoid)


def _expand_index(lmax: int) -> torch.Tensor:
    return torch.tensor([l for l in range(lmax + 1) for _ in range(2 * l + 1)], dtype=torch.long)


FP32_GEMM = os.environ.get("E2V2_FP32_GEMM", "split")


def split_gemm_on() -> bool:
    """fp32 per-node GEMMs on the split-bf16 kernel (else hipBLASLt fp32)."""
    return FP32_GEMM != "native"


def _stream():
    return _lib.vp(torch.cuda.current_stream().cuda_stream)


def _dp(t):
    return _lib.vp(t.data_ptr())


BF16 = torch.bfloat16


def _bf(a):
    return a if a.dtype == BF16 else a.to(BF16)


def _mm_into(a, b, out):
    """out = a @ b for an fp32 activation a and a weight operand b.  With a bf16
    weight the activation is rounded to bf16 and the product is accumulated in
    fp32 and stored in out's dtype (bf16 MFMA operands; fp32, or a bf16
    activation consumed only by a bf16 kernel)."""
    if b.dtype == BF16:
        if out.dtype == BF16:
            return torch.mm(_bf(a), b, out=out)
        return torch.mm(_bf(a), b, out_dtype=torch.float32, out=out)
    return torch.mm(a, b, out=out)


def _mm_bias_into(a, b, bias, out):
    """out = a @ b + bias (bias broadcast over rows; fused into the GEMM for fp32
    operands) with the operand rule of ``_mm_into``."""
    if b.dtype == BF16:
        _mm_into(a, b, out)
        return out.add_(bias)
    return torch.addmm(bias, a, b, out=out)


def _addmm_into(c, a, b, out):
    """out = c + a @ b with the operand rule of ``_mm_into``."""
    if b.dtype == BF16:
        return torch.addmm(c, _bf(a), b, out_dtype=torch.float32, out=out)
    return torch.addmm(c, a, b, out=out)


def cached(owner, name: str, params, build):
    """Per-object cache of a tensor derived from ``params`` (rebuilt when any of
    them is replaced or modified in place)."""
    key = tuple((p.data_ptr(), p._version) for p in params)
    ent = owner.__dict__.get("_c_" + name)
    if ent is None or ent[0] != key:
        ent = (key, build())
        owner.__dict__["_c_" + name] = ent
    return ent[1]


_SLICE_PERM = {}


def slice_perm(device) -> torch.Tensor:
    """Channel order of the attention kernels (the header's slice order): the
    model channel held at each position p of a v / output row, P[p].  Position p
    belongs to head h = 16 (p // 32) + p % 16 and holds its first channel (h)
    for p % 32 < 16, its second (128 + h) otherwise, so the 16 heads of slice
    s = p // 32 occupy one contiguous 32-channel run."""
    key = str(device)
    if key not in _SLICE_PERM:
        p = np.arange(256)
        h = 16 * (p // 32) + p % 16
        _SLICE_PERM[key] = torch.as_tensor(np.where(p % 32 < 16, h, 128 + h), device=device)
    return _SLICE_PERM[key]


def gemm_weight(mod, name: str, bf16: bool):
    """A module's weight as a GEMM operand: the parameter itself in fp32 mode,
    a cached bf16 copy in bf16 mode."""
    p = getattr(mod, name)
    if not bf16:
        return p.detach()
    return cached(mod, name + "_bf16", (p,), lambda: p.detach().to(BF16).contiguous())


class MRowWeight:
    """Per-l weight W [lmax+1, O, Cin] of an SO(3) linear as GEMM operands: ``w``
    for per-l GEMMs (fp32, or a bf16 copy), and in fp32 its per-m-row expansions
    for one batched GEMM over the (lmax+1)^2 m-rows (one launch instead of lmax+1,
    fewer partial tiles): ``fwd`` [M, Cin, O] and ``bwd`` [M, O, Cin]; in bf16 the
    per-l transpose ``wt`` [lmax+1, Cin, O] (B operand of the fused projection's backward).
    ``s3f()`` / ``s3b()``: the per-l weights packed for the split GEMM (W_l for
    y = x W_l^T, W_l^T for the input gradient), packed on first use: the exact
    three-piece split of an fp32 weight, the bf16 weight itself as one piece (the
    bf16 mode's GEMMs, bf16 operands with fp32 accumulation)."""
    __slots__ = ("w", "fwd", "bwd", "wt", "_s3f", "_s3b")

    def __init__(self, w, fwd=None, bwd=None, wt=None):
        self.w, self.fwd, self.bwd, self.wt = w, fwd, bwd, wt
        self._s3f = self._s3b = None

    @property
    def pieces(self) -> int:
        return 1 if self.w.dtype == BF16 else 3

    def split_ok(self) -> bool:
        w = self.w
        return ((w.dtype == BF16 or (split_gemm_on() and w.dtype == torch.float32)) and w.is_cuda
                and s3gemm.supported(w.shape[1], w.shape[2]) and s3gemm.supported(w.shape[2], w.shape[1]))

    def s3f(self):
        if self._s3f is None:
            self._s3f = s3gemm.pack(self.w, pieces=self.pieces)
        return self._s3f

    def s3b(self):
        if self._s3b is None:
            self._s3b = s3gemm.pack(self.w, transpose=True, pieces=self.pieces)
        return self._s3b


def _m_index(lmax: int, device):
    return torch.tensor([l for l in range(lmax + 1) for _ in range(2 * l + 1)], device=device)


def _m_degrees(lmax: int):
    return [l for l in range(lmax + 1) for _ in range(2 * l + 1)]


def mrow_weight(owner, name: str, w, bf16: bool, lmax: int):
    """MRowWeight of the weight tensor w (a parameter of ``owner`` or a tensor built
    from its parameters; cached under ``name`` until w changes)."""
    if bf16:
        def build_bf16():
            wb = w.detach().to(BF16).contiguous()
            return MRowWeight(wb, wt=wb.transpose(1, 2).contiguous())
        return cached(owner, name + "_mrow_bf16", (w,), build_bf16)

    def build():
        wd = w.detach()
        e = wd[_m_index(lmax, wd.device)]
        return MRowWeight(wd, e.transpose(1, 2).contiguous(), e.contiguous())
    return cached(owner, name + "_mrow", (w,), build)


def _mrow_gemm(x, Wop: MRowWeight, bias):
    """y[m] = x[m] W_l(m)^T (+ bias on row 0) for x [M, N, Cin] (fp32, batched)."""
    if Wop.split_ok():
        y = x.new_empty(x.shape[0], x.shape[1], Wop.w.shape[1])
        return s3gemm.gemm(x, Wop.s3f(), y, _m_degrees(Wop.w.shape[0] - 1), bias=bias, bias_batches=1)
    y = torch.bmm(x, Wop.fwd)
    if bias is not None:
        y[0].add_(bias)
    return y


class SO3LinearFn(torch.autograd.Function):
    """y[rows(l)] = res[rows(l)] + x[rows(l)] W_l^T (+ bias on row 0) on the
    m-major layout x[(lmax+1)^2, N, Cin]: each l block is one 2-D GEMM written in
    place (addmm when a residual is fused).  W and bias are constants (input
    gradients only)."""

    @staticmethod
    def forward(ctx, x, Wop, bias, lmax: int, res=None):
        x = x.contiguous()
        ctx.Wop, ctx.lmax, ctx.has_res = Wop, lmax, res is not None
        if Wop.split_ok():
            y = x.new_empty(x.shape[0], x.shape[1], Wop.w.shape[1])
            return s3gemm.gemm(x, Wop.s3f(), y, _m_degrees(lmax), bias=bias, bias_batches=1,
                               res=None if res is None else res.contiguous())
        if Wop.fwd is not None and res is None:
            return _mrow_gemm(x, Wop, bias)
        W = Wop.w
        L2, N, Cin = x.shape
        O = W.shape[1]
        y = x.new_empty(L2, N, O)
        if res is not None:
            res = res.contiguous()
        xa = _bf(x) if W.dtype == BF16 else x
        for l in range(lmax + 1):
            a, b = l * l, (l + 1) ** 2
            if res is not None:
                _addmm_into(res[a:b].view(-1, O), xa[a:b].view(-1, Cin), W[l].t(), out=y[a:b].view(-1, O))
            elif l == 0 and bias is not None:
                _mm_bias_into(xa[0], W[0].t(), bias, out=y[0])
            else:
                _mm_into(xa[a:b].view(-1, Cin), W[l].t(), out=y[a:b].view(-1, O))
        if bias is not None and res is not None:
            y[0].add_(bias)
        return y

    @staticmethod
    def backward(ctx, gy):
        Wop = ctx.Wop
        gy = gy.contiguous()
        if Wop.split_ok():
            gx = gy.new_empty(gy.shape[0], gy.shape[1], Wop.w.shape[2])
            return (s3gemm.gemm(gy, Wop.s3b(), gx, _m_degrees(ctx.lmax)), None, None, None,
                    (gy if ctx.has_res else None))
        if Wop.bwd is not None:
            return torch.bmm(gy, Wop.bwd), None, None, None, (gy if ctx.has_res else None)
        W = Wop.w
        L2, N, O = gy.shape
        Cin = W.shape[2]
        gx = gy.new_empty(L2, N, Cin)
        ga = _bf(gy) if W.dtype == BF16 else gy
        for l in range(ctx.lmax + 1):
            a, b = l * l, (l + 1) ** 2
            _mm_into(ga[a:b].view(-1, O), W[l], out=gx[a:b].view(-1, Cin))
        return gx, None, None, None, (gy if ctx.has_res else None)


def _qk_fused(x, Wop: MRowWeight, Wvop, C: int, hid: int, lmax: int):
    """Which fused HIP projection covers this call: "fp32" (``e2v2_qk_proj_fwd/bwd``:
    fp32 weights with per-m expansions) or "bf16" (``e2v2_qk_proj_*_bf16``: bf16
    weights with per-l transposes), for an fp32 input, lmax 2, C a multiple of 128,
    hid of 64 and a value width of 64; else None (per-l GEMMs + pair-dot kernels)."""
    if not (x.dtype == torch.float32 and lmax == 2 and C % 128 == 0 and hid % 64 == 0):
        return None
    if Wop.fwd is not None and Wop.w.dtype == torch.float32:
        if Wvop is None or (Wvop.fwd is not None and Wvop.fwd.shape[2] % 64 == 0):
            return "fp32"
    if Wop.wt is not None and Wop.w.dtype == BF16:
        if Wvop is None or (Wvop.wt is not None and Wvop.wt.shape[2] % 64 == 0):
            return "bf16"
    return None


class QKProjFn(torch.autograd.Function):
    """Fused per-l GEMM of the query and key SO3_Linear2Scalar products and their
    m-contraction: x[9][N][C] -> hq, hk [N][3 hid] (before final_linear)."""

    @staticmethod
    def forward(ctx, x, Wop, bias, lmax: int, hid: int, Wvop=None, bv=None, s3=None):
        """Wop, Wvop: MRowWeight.  With the value projection's weight Wvop
        ([lmax+1, Cv, C]) and bias bv it also returns v = SO3_Linear(x) [9, N, Cv]
        (else None), so that the backward sums the two input gradients inside the
        GEMMs.  s3: the split-GEMM packs of the same weights (gemm.QKPacks), which
        take the fp32 projection when given."""
        x = x.contiguous()
        L2, N, C = x.shape
        W = Wop.w
        fused = "s3" if s3 is not None and x.dtype == torch.float32 and lmax == 2 else _qk_fused(x, Wop, Wvop, C,
                                                                                                   hid, lmax)
        ctx.fused, ctx.s3 = fused, s3
        if fused == "s3":
            # split-GEMM projection, the m-contraction in its epilogue; y kept in the paired column order
            hq, hk, y = s3gemm.qk_forward(x, s3)
        elif fused:
            # projection GEMM with the m-contraction on its accumulators (HIP, MFMA);
            # the bf16 form rounds x while staging it and keeps y in bf16
            y = x.new_empty(L2, N, 4 * hid, dtype=BF16 if fused == "bf16" else torch.float32)
            hq = x.new_empty(N, 3 * hid); hk = x.new_empty(N, 3 * hid)
            _lib.call("e2v2_qk_proj_fwd" if fused == "fp32" else "e2v2_qk_proj_fwd_bf16", _dp(x), _dp(W),
                      _lib.vp(bias.data_ptr() if bias is not None else 0), _dp(y), _dp(hq), _dp(hk),
                      _lib.i32(N), _lib.i32(hid), _lib.i32(C), _stream())
        elif Wop.fwd is not None:
            y = _mrow_gemm(x, Wop, bias)
        else:
            y = x.new_empty(L2, N, 4 * hid)
            xa = _bf(x) if W.dtype == BF16 else x
            for l in range(lmax + 1):
                a, b = l * l, (l + 1) ** 2
                if l == 0:
                    _mm_bias_into(xa[0], W[0].t(), bias, out=y[0])
                else:
                    _mm_into(xa[a:b].view(-1, C), W[l].t(), out=y[a:b].view(-1, 4 * hid))
        if not fused:
            hq = x.new_empty(N, 3 * hid); hk = x.new_empty(N, 3 * hid)
            _lib.call("e2v2_pairdot_fwd", _dp(y), _dp(hq), _dp(hk), _lib.i32(N), _lib.i32(hid), _stream())
        v = None
        if Wvop is not None:
            Wv = Wvop.w
            Cv = Wv.shape[1]
            if Wvop.fwd is not None:
                v = _mrow_gemm(x, Wvop, bv)
            else:
                v = x.new_empty(L2, N, Cv)
                xv = _bf(x) if Wv.dtype == BF16 else x
                for l in range(lmax + 1):
                    a, b = l * l, (l + 1) ** 2
                    if l == 0:
                        _mm_bias_into(xv[0], Wv[0].t(), bv, out=v[0])
                    else:
                        _mm_into(xv[a:b].view(-1, C), Wv[l].t(), out=v[a:b].view(-1, Cv))
        ctx.save_for_backward(y)
        ctx.Wop, ctx.Wvop = Wop, Wvop
        ctx.lmax, ctx.hid = lmax, hid
        return hq, hk, v

    @staticmethod
    def backward(ctx, ghq, ghk, gv):
        (y,) = ctx.saved_tensors
        Wop, Wvop = ctx.Wop, ctx.Wvop
        L2, N, F = y.shape
        hid = ctx.hid
        ghq = torch.zeros(N, 3 * hid, device=y.device) if ghq is None else ghq.contiguous()
        ghk = torch.zeros(N, 3 * hid, device=y.device) if ghk is None else ghk.contiguous()
        if ctx.fused == "s3":
            return s3gemm.qk_backward(y, ghq, ghk, gv, ctx.s3), None, None, None, None, None, None, None
        if ctx.fused:
            # gy = the m-contraction's gradient, formed while the GEMM stages it; the
            # value projection's gradient gv W_v enters as further K stages
            C = Wop.w.shape[2]
            gx = y.new_empty(L2, N, C, dtype=torch.float32)
            with_v = Wvop is not None and gv is not None
            gvc = gv.float().contiguous() if with_v else None
            bt = Wop.fwd if ctx.fused == "fp32" else Wop.wt            # [M or lmax+1, C, 4 hid]
            bvt = (Wvop.fwd if ctx.fused == "fp32" else Wvop.wt) if with_v else None
            _lib.call("e2v2_qk_proj_bwd" if ctx.fused == "fp32" else "e2v2_qk_proj_bwd_bf16", _dp(y), _dp(ghq),
                      _dp(ghk), _dp(bt), _lib.vp(gvc.data_ptr() if with_v else 0),
                      _lib.vp(bvt.data_ptr() if with_v else 0), _dp(gx), _lib.i32(N), _lib.i32(hid), _lib.i32(C),
                      _lib.i32(bvt.shape[2] if with_v else 0), _stream())
            return gx, None, None, None, None, None, None, None
        gy = torch.empty_like(y)
        _lib.call("e2v2_pairdot_bwd", _dp(y), _dp(ghq), _dp(ghk), _dp(gy), _lib.i32(N), _lib.i32(hid), _stream())
        W = Wop.w
        C = W.shape[2]
        if Wop.bwd is not None:
            gx = torch.bmm(gy, Wop.bwd)
        else:
            gx = y.new_empty(L2, N, C)
            ga = _bf(gy) if W.dtype == BF16 else gy
            for l in range(ctx.lmax + 1):
                a, b = l * l, (l + 1) ** 2
                _mm_into(ga[a:b].view(-1, F), W[l], out=gx[a:b].view(-1, C))
        if Wvop is not None and gv is not None:
            gv = gv.contiguous()
            if Wvop.bwd is not None:
                gx.baddbmm_(gv, Wvop.bwd)
            else:
                Wv = Wvop.w
                Cv = Wv.shape[1]
                for l in range(ctx.lmax + 1):
                    a, b = l * l, (l + 1) ** 2
                    _addmm_into(gx[a:b].view(-1, C), gv[a:b].view(-1, Cv), Wv[l], out=gx[a:b].view(-1, C))
        return gx, None, None, None, None, None, None, None


class SO2OutFn(torch.autograd.Function):
    """y = res + proj_first(forward_linear(so2)) as one GEMM per output degree l3
    (so2_tensor_product.py:276-290, e2former.py:215-219,433).  so2 is the
    attention output in its l3-grouped layout: the 2 l3 + 1 rows of degree l3
    hold their cnt coupling paths side by side, [2 l3 + 1][N][cnt C], the
    operand of forward_linear's Linear(cnt C -> C); its weight (path_norm and the
    path scales folded, input rows in the kernels' slice order) times
    proj_first's W_l3^T is one [cnt C, O] weight (``so2_out_weights``).  The
    zero-order rows [9][N][C] are the case cnt = 1 with proj_zero's W_l^T
    (``zero_out_weights``, e2former.py:411-416)."""

    @staticmethod
    def forward(ctx, so2, res, Wc, bias, N: int):
        so2 = so2.contiguous()
        res = None if res is None else res.contiguous()
        O = Wc[0][3].shape[1]
        y = so2.new_empty(9, N, O, dtype=torch.float32)
        # fp32 rows on three-piece packs, or the bf16 mode's one-piece packs (bf16 or fp32 rows)
        split = all(e[5] is not None for e in Wc) and (so2.dtype == torch.float32 or
                                                       all(e[5].pieces == 1 for e in Wc))
        problems = []
        for (l3, cnt, start, W, _, PF, _) in Wc:
            K = W.shape[0]
            A = so2[start * N:(start + (2 * l3 + 1) * K) * N].view(-1, K)
            a, b = l3 * l3, (l3 + 1) ** 2
            if split:
                problems.append({"a": A, "pw": PF, "out": y[a:b].view(-1, O), "bias": bias if l3 == 0 else None,
                                 "res": None if res is None else res[a:b].view(-1, O)})
            elif res is not None:
                _addmm_into(res[a:b].view(-1, O), A, W, out=y[a:b].view(-1, O))
            else:
                _mm_into(A, W, out=y[a:b].view(-1, O))
        if split:                                # one launch, the longest k first
            s3gemm.gemm_grouped(sorted(problems, key=lambda p: -p["pw"].k))
        else:
            y[0].add_(bias)
        ctx.has_res = res is not None
        ctx.Wc, ctx.N = Wc, N
        ctx.shape, ctx.so2_dtype = so2.shape, so2.dtype
        return y

    @staticmethod
    def backward(ctx, gy):
        gy = gy.contiguous()
        N = ctx.N
        O = gy.shape[2]
        gso2 = gy.new_empty(ctx.shape, dtype=ctx.so2_dtype)
        split = all(e[6] is not None for e in ctx.Wc) and (ctx.so2_dtype == torch.float32 or
                                                           all(e[6].pieces == 1 for e in ctx.Wc))
        problems = []
        for (l3, cnt, start, _, WT, _, PB) in ctx.Wc:
            K = WT.shape[1]
            a, b = l3 * l3, (l3 + 1) ** 2
            dst = gso2[start * N:(start + (2 * l3 + 1) * K) * N].view(-1, K)
            if split:
                problems.append({"a": gy[a:b].view(-1, O), "pw": PB, "out": dst})
            else:
                _mm_into(gy[a:b].view(-1, O), WT, out=dst)
        if split:                                # one launch, the most tiles first
            s3gemm.gemm_grouped(sorted(problems, key=lambda p: -p["out"].numel()))
        return gso2, (gy if ctx.has_res else None), None, None, None


class RMSNormFn(torch.autograd.Function):
    """rms_norm_sh on x[9][N][256] through e2v2_rmsnorm_fwd/bwd."""

    @staticmethod
    def forward(ctx, x, w, b, eps: float):
        x = x.contiguous()
        y = torch.empty_like(x)
        _lib.call("e2v2_rmsnorm_fwd", _dp(x), _dp(w), _dp(b), _dp(y), _lib.i32(x.shape[1]), _lib.f32(eps),
                  _stream())
        ctx.save_for_backward(x, w)
        ctx.eps = eps
        return y

    @staticmethod
    def backward(ctx, gy):
        x, w = ctx.saved_tensors
        gy = gy.contiguous()
        gx = torch.empty_like(x)
        _lib.call("e2v2_rmsnorm_bwd", _dp(x), _dp(w), _dp(gy), None, _dp(gx), _lib.i32(x.shape[1]),
                  _lib.f32(ctx.eps), _stream())
        return gx, None, None, None


class AddRMSNormFn(torch.autograd.Function):
    """(rms_norm_sh(xs), xs) with xs = x + delta (delta None: xs = x): the
    residual add of the producing block fused into the norm that follows it,
    and xs returned for the next residual branch, so that the backward adds the
    two gradients of xs inside the norm's kernel (no accumulation pass, no
    residual operand in the GEMMs)."""

    @staticmethod
    def forward(ctx, x, delta, w, b, eps: float):
        x = x.contiguous()
        y = torch.empty_like(x)
        if delta is None:
            xs = x
            _lib.call("e2v2_rmsnorm_fwd", _dp(x), _dp(w), _dp(b), _dp(y), _lib.i32(x.shape[1]), _lib.f32(eps),
                      _stream())
        else:
            delta = delta.contiguous()
            xs = torch.empty_like(x)
            _lib.call("e2v2_add_rmsnorm_fwd", _dp(x), _dp(delta), _dp(w), _dp(b), _dp(xs), _dp(y),
                      _lib.i32(x.shape[1]), _lib.f32(eps), _stream())
        ctx.save_for_backward(xs, w)
        ctx.eps, ctx.has_delta = eps, delta is not None
        ctx.set_materialize_grads(False)
        return y, xs

    @staticmethod
    def backward(ctx, gy, gres):
        xs, w = ctx.saved_tensors
        if gy is None:
            gx = gres
        else:
            gy = gy.contiguous()
            gres = None if gres is None else gres.contiguous()
            gx = torch.empty_like(xs)
            _lib.call("e2v2_rmsnorm_bwd", _dp(xs), _dp(w), _dp(gy), None if gres is None else _dp(gres), _dp(gx),
                      _lib.i32(xs.shape[1]), _lib.f32(ctx.eps), _stream())
        return gx, (gx if ctx.has_delta else None), None, None, None


class LNSiLUFn(torch.autograd.Function):
    """silu(LayerNorm(x)) on rows x [N, w] (the LayerNorm + SiLU of the Q/K head,
    module_utils.py:2230-2233) through e2v2_ln_silu_fwd/bwd; the LayerNorm
    affine parameters are constants (input gradient only)."""

    @staticmethod
    def forward(ctx, x, g, b, eps: float):
        x = x.contiguous()
        n, w = x.shape
        y = torch.empty_like(x)
        st = x.new_empty(n, 2)
        _lib.call("e2v2_ln_silu_fwd", _dp(x), _dp(g), _dp(b), _dp(y), _dp(st), _lib.i32(n), _lib.i32(w),
                  _lib.f32(eps), _stream())
        ctx.save_for_backward(x, g, b, st)
        return y

    @staticmethod
    def backward(ctx, gy):
        x, g, b, st = ctx.saved_tensors
        gy = gy.contiguous()
        gx = torch.empty_like(x)
        _lib.call("e2v2_ln_silu_bwd", _dp(x), _dp(g), _dp(b), _dp(st), _dp(gy), _dp(gx), _lib.i32(x.shape[0]),
                  _lib.i32(x.shape[1]), _stream())
        return gx, None, None, None


def _heads_tail(h1, P, out_dtype=torch.float32):
    """LayerNorm + SiLU of each head's first Linear output h1 [2, N, hid] and the
    second Linear (one two-batch launch): (out [2, N, n_out] in out_dtype, LayerNorm
    stats)."""
    N = h1.shape[1]
    a = torch.empty_like(h1)
    st = h1.new_empty(2, N, 2)
    for b in range(2):
        g, be, eps = P["ln"][b]
        _lib.call("e2v2_ln_silu_fwd", _dp(h1[b]), _dp(g), _dp(be), _dp(a[b]), _dp(st[b]), _lib.i32(N),
                  _lib.i32(h1.shape[2]), _lib.f32(eps), _stream())
    out = h1.new_empty(2, N, P["p2f"].n, dtype=out_dtype)
    s3gemm.gemm(a, P["p2f"], out, [0, 1], bias=P["b2"], bias_batches=2)
    return out, st


def _heads_backward(h1, st, gq, gk, P):
    """Input gradients [2, N, 3 hid] of the two final_linear stacks given the
    output gradients gq, gk [N, n_out] (None: zero)."""
    N = h1.shape[1]
    gq = torch.zeros(N, P["p2f"].n, device=h1.device) if gq is None else gq.float().contiguous()
    gk = torch.zeros(N, P["p2f"].n, device=h1.device) if gk is None else gk.float().contiguous()
    ga = torch.empty_like(h1)
    s3gemm.gemm([gq, gk], P["p2b"], ga, [0, 1])
    gh1 = torch.empty_like(h1)
    for b in range(2):
        g, be, _ = P["ln"][b]
        _lib.call("e2v2_ln_silu_bwd", _dp(h1[b]), _dp(g), _dp(be), _dp(st[b]), _dp(ga[b]), _dp(gh1[b]),
                  _lib.i32(N), _lib.i32(h1.shape[2]), _stream())
    gh = h1.new_empty(2, N, P["p1f"].k)
    s3gemm.gemm(gh1, P["p1b"], gh, [0, 1])
    return gh


class QKHeadsS3Fn(torch.autograd.Function):
    """final_linear of the query and of the key SO3_Linear2Scalar_e2former
    (module_utils.py:2230-2233: Linear(3 hid -> hid) -> LayerNorm -> SiLU ->
    Linear(hid -> out)) for both at once on the split GEMM: each Linear is one
    launch with the two heads as batches (per-head weights and biases), which fills
    twice the tiles of two separate launches.  Input gradients only."""

    @staticmethod
    def forward(ctx, hq, hk, P):
        hq, hk = hq.contiguous(), hk.contiguous()
        h1 = hq.new_empty(2, hq.shape[0], P["p1f"].n)
        s3gemm.gemm([hq, hk], P["p1f"], h1, [0, 1], bias=P["b1"], bias_batches=2)
        out, st = _heads_tail(h1, P)
        ctx.save_for_backward(h1, st)
        ctx.P = P
        return out[0], out[1]

    @staticmethod
    def backward(ctx, gq, gk):
        h1, st = ctx.saved_tensors
        gh = _heads_backward(h1, st, gq, gk, ctx.P)
        return gh[0], gh[1], None


class AttnProjS3Fn(torch.autograd.Function):
    """The attention's node projections on the split GEMMs, fp32: the query / key
    SO3_Linear2Scalar_e2former (module_utils.py:2198-2266) with its final_linear
    for both (QKHeadsS3Fn) and the value SO3_Linear (e2former.py:300-303).  The
    value GEMM shares a launch with the heads' first Linear, which alone fills
    too few tiles to occupy the GPU; the backward folds the value gradient into
    the projection's backward GEMM.  Returns q, k [N, H D] and v [9, N, Cv]."""

    @staticmethod
    def forward(ctx, x, s3, P, Wvop, bv):
        x = x.contiguous()
        N = x.shape[1]
        hq, hk, y = s3gemm.qk_forward(x, s3)
        h1 = x.new_empty(2, N, P["p1f"].n)
        v = x.new_empty(x.shape[0], N, Wvop.w.shape[1])
        s3gemm.gemm_grouped([
            {"a": [hq, hk], "pw": P["p1f"], "out": h1, "widx": [0, 1], "bias": P["b1"], "bias_batches": 2},
            {"a": x, "pw": Wvop.s3f(), "out": v, "widx": _m_degrees(Wvop.w.shape[0] - 1), "bias": bv}])
        out, st = _heads_tail(h1, P)
        ctx.save_for_backward(y, h1, st)
        ctx.s3, ctx.P = s3, P
        return out[0], out[1], v

    @staticmethod
    def backward(ctx, gq, gk, gv):
        y, h1, st = ctx.saved_tensors
        gh = _heads_backward(h1, st, gq, gk, ctx.P)
        gx = s3gemm.qk_backward(y, gh[0], gh[1], None if gv is None else gv.contiguous(), ctx.s3)
        return gx, None, None, None, None


class AttnBlockBF16Fn(torch.autograd.Function):
    """The bf16 mode's attention from the layer input to the SO(2) rows in one
    autograd node: the node projections of AttnProjS3Fn on one-piece packs, whose
    GEMMs write q, k and v as bf16 (the storage the attention kernels gather), then
    the attention kernels (AttentionFn).  q, k, v never cross an autograd edge, so
    their fp32 gradients from the attention backward reach the projections'
    backward GEMMs unrounded and no cast kernel runs either way.  Inputs with
    gradients: x, dvec, dist and the external gate."""

    @staticmethod
    def forward(ctx, x, dvec, dist, ext_gate, s3, P, Wvop, bv, nl, atom_type, table, rc: float, q_div: float,
                zero_order: bool, env, weight_act: str = "softmax"):
        if not (x.is_cuda and dvec.is_cuda):
            raise RuntimeError("the e2v2 HIP path needs GPU tensors (no CPU fallback)")
        x = x.contiguous()
        N = x.shape[1]
        hq, hk, y = s3gemm.qk_forward(x, s3)
        h1 = x.new_empty(2, N, P["p1f"].n)
        v = x.new_empty(x.shape[0], N, Wvop.w.shape[1], dtype=BF16)
        s3gemm.gemm_grouped([
            {"a": [hq, hk], "pw": P["p1f"], "out": h1, "widx": [0, 1], "bias": P["b1"], "bias_batches": 2},
            {"a": x, "pw": Wvop.s3f(), "out": v, "widx": _m_degrees(Wvop.w.shape[0] - 1), "bias": bv}])
        qk, st = _heads_tail(h1, P, BF16)
        H = 128
        q, k = qk[0].reshape(N, H, -1), qk[1].reshape(N, H, -1)
        out, mrow, srow, cnt, q, k, v, ext_gate = attention_forward(q, k, v, nl, atom_type, table, rc, q_div, BF16,
                                                                    zero_order, env, ext_gate, weight_act)
        ctx.save_for_backward(y, h1, st, q, k, v, out, mrow, srow, cnt, ext_gate)
        ctx.s3, ctx.P, ctx.nl, ctx.atom_type, ctx.table = s3, P, nl, atom_type, table
        ctx.rc, ctx.q_div, ctx.zero_order, ctx.env, ctx.weight_act = rc, q_div, zero_order, env, weight_act
        return out

    @staticmethod
    def backward(ctx, gout):
        if torch.is_grad_enabled():
            raise NotImplementedError("the HIP E2Former path implements first-order input gradients only "
                                      "(create_graph=True / double backward is not supported)")
        y, h1, st, q, k, v, out, mrow, srow, cnt, ext_gate = ctx.saved_tensors
        dq, dk, dv, ddv, dd, dgate = attention_backward(gout, q, k, v, out, mrow, srow, cnt, ext_gate, ctx.nl,
                                                        ctx.atom_type, ctx.table, ctx.rc, ctx.q_div, ctx.zero_order,
                                                        ctx.env, ctx.weight_act)
        N = h1.shape[1]
        gh = _heads_backward(h1, st, dq.reshape(N, -1), dk.reshape(N, -1), ctx.P)
        gx = s3gemm.qk_backward(y, gh[0], gh[1], dv, ctx.s3)
        return (gx, ddv, dd, dgate) + (None,) * 12


def head_pair_packs(fq: nn.Sequential, fk: nn.Sequential, owner, bf16: bool = False):
    """Operands of QKHeadsS3Fn for two final_linear stacks (Linear, LayerNorm,
    SiLU, Linear) of the same shapes: each Linear's two weights stacked and packed
    for the forward and (transposed) for the input gradient (one bf16 piece in
    the bf16 mode), the biases as [2, n], the LayerNorm parameters per head.
    Cached on ``owner`` per weight version; None when the split GEMM does not
    apply."""
    w1, w2 = fq[0].weight, fq[3].weight
    if not ((bf16 or split_gemm_on()) and w1.is_cuda and w1.dtype == torch.float32
            and all(s3gemm.supported(*w.shape) and s3gemm.supported(*w.shape[::-1]) for w in (w1, w2))):
        return None
    pc = 1 if bf16 else 3
    params = [p for f in (fq, fk) for i in (0, 1, 3) for p in (f[i].weight, f[i].bias)]

    def build():
        W1 = torch.stack([fq[0].weight.detach(), fk[0].weight.detach()]).float().contiguous()
        W2 = torch.stack([fq[3].weight.detach(), fk[3].weight.detach()]).float().contiguous()
        ln = [(f[1].weight.detach().float().contiguous(), f[1].bias.detach().float().contiguous(),
               float(f[1].eps)) for f in (fq, fk)]
        return {"p1f": s3gemm.pack(W1, pieces=pc), "p1b": s3gemm.pack(W1, transpose=True, pieces=pc),
                "b1": torch.stack([fq[0].bias.detach(), fk[0].bias.detach()]).float().contiguous(),
                "p2f": s3gemm.pack(W2, pieces=pc), "p2b": s3gemm.pack(W2, transpose=True, pieces=pc),
                "b2": torch.stack([fq[3].bias.detach(), fk[3].bias.detach()]).float().contiguous(), "ln": ln}
    return cached(owner, "head_pair_bf16" if bf16 else "head_pair_s3", params, build)


def _ln_silu(x, ln: nn.LayerNorm):
    return LNSiLUFn.apply(x, ln.weight.detach().float().contiguous(), ln.bias.detach().float().contiguous(),
                          float(ln.eps))


class GateFn(torch.autograd.Function):
    """Gate_s3: sc = x[0] Wg^T + bg, then the activation kernel on x[9][N][C]."""

    @staticmethod
    def forward(ctx, x, Wg, bg, k1: float, k2: float, packs=None):
        x = x.contiguous()
        ctx.packs = packs
        if packs is not None:
            sc = x.new_empty(x.shape[1], packs[0].n)
            s3gemm.gemm(x[0], packs[0], sc, bias=bg)
        elif Wg.dtype == BF16:
            sc = torch.mm(_bf(x[0]), Wg.t(), out_dtype=torch.float32).add_(bg)
        else:
            sc = torch.addmm(bg, x[0], Wg.t())
        y = torch.empty_like(x)
        _lib.call("e2v2_gate_fwd", _dp(sc), _dp(x), _dp(y), _lib.i32(x.shape[1]), _lib.f32(k1), _lib.f32(k2),
                  _stream())
        ctx.save_for_backward(sc, x, Wg)
        ctx.k = (k1, k2)
        return y

    @staticmethod
    def backward(ctx, gy):
        sc, x, Wg = ctx.saved_tensors
        gy = gy.contiguous()
        gsc = torch.empty_like(sc); gx = torch.empty_like(x)
        _lib.call("e2v2_gate_bwd", _dp(sc), _dp(x), _dp(gy), _dp(gsc), _dp(gx), _lib.i32(x.shape[1]),
                  _lib.f32(ctx.k[0]), _lib.f32(ctx.k[1]), _stream())
        if ctx.packs is not None:                # the kernel leaves gx[0] = 0
            s3gemm.gemm(gsc, ctx.packs[1], gx[0])
        else:
            _mm_into(gsc, Wg, out=gx[0])
        return gx, None, None, None, None, None


class DenseFn(torch.autograd.Function):
    """y = x W^T + b for a constant weight W [O, K] (fp32, or bf16 operands with
    fp32 accumulation); input gradient only."""

    @staticmethod
    def forward(ctx, x, W, b):
        x = x.contiguous()
        y = x.new_empty(x.shape[0], W.shape[0])
        _mm_into(x, W.t(), out=y)
        if b is not None:
            y.add_(b)
        ctx.save_for_backward(W)
        return y

    @staticmethod
    def backward(ctx, gy):
        (W,) = ctx.saved_tensors
        gy = gy.contiguous()
        gx = gy.new_empty(gy.shape[0], W.shape[1])
        _mm_into(gy, W, out=gx)
        return gx, None, None


class DenseS3Fn(torch.autograd.Function):
    """y = x W^T + b for a constant fp32 weight on the split GEMM (packs of W for
    the forward and of W^T for the input gradient); input gradient only."""

    @staticmethod
    def forward(ctx, x, packs, b):
        x = x.contiguous()
        pf, pb = packs
        y = x.new_empty(x.shape[0], pf.n)
        s3gemm.gemm(x, pf, y, bias=b)
        ctx.pb = pb
        return y

    @staticmethod
    def backward(ctx, gy):
        gy = gy.contiguous()
        gx = gy.new_empty(gy.shape[0], ctx.pb.n)
        s3gemm.gemm(gy, ctx.pb, gx)
        return gx, None, None


def dense_packs(lin: nn.Linear, bf16: bool = False):
    """Split-GEMM packs (W, W^T) of an nn.Linear's weight (cached per version; one
    bf16 piece in the bf16 mode), or None when the split GEMM does not apply."""
    w = lin.weight
    if not ((bf16 or split_gemm_on()) and w.is_cuda and w.dtype == torch.float32
            and s3gemm.supported(w.shape[0], w.shape[1]) and s3gemm.supported(w.shape[1], w.shape[0])):
        return None
    pc = 1 if bf16 else 3
    return cached(lin, "s3_packs_bf16" if bf16 else "s3_packs", (w,),
                  lambda: (s3gemm.pack(w.detach(), pieces=pc), s3gemm.pack(w.detach(), transpose=True, pieces=pc)))


def _linear(x, lin: nn.Linear):
    if x.dim() == 2 and x.dtype == torch.float32:
        packs = dense_packs(lin)
        if packs is not None:
            b = None if lin.bias is None else lin.bias.detach().float().contiguous()
            return DenseS3Fn.apply(x, packs, b)
    return torch.nn.functional.linear(x, lin.weight.detach(), None if lin.bias is None else lin.bias.detach())


def _layer_norm(x, ln: nn.LayerNorm):
    return torch.nn.functional.layer_norm(x, ln.normalized_shape, ln.weight.detach(), ln.bias.detach(), ln.eps)


class GaussianSmearing(nn.Module):
    """module_utils.py:1853-1869 (evaluated inside the HIP edge kernels)."""

    def __init__(self, num_basis, cutoff: float = 5.0, basis_width_scalar: float = 2.0):
        super().__init__()
        offset = torch.linspace(0, cutoff, num_basis)
        self.coeff = -0.5 / (basis_width_scalar * (offset[1] - offset[0])).item() ** 2
        self.register_buffer("offset", offset)

    def forward(self, dist):
        d = dist.view(-1, 1) - self.offset.view(1, -1)
        return torch.exp(self.coeff * torch.pow(d, 2)).reshape(*dist.shape, -1)


class RadialProfile(nn.Module):
    """module_utils.py:2151-2178 (parameters only; evaluated through its distance table, ops.RadialTable)."""

    def __init__(self, ch_list, use_layer_norm=True, use_offset=True):
        super().__init__()
        mods = []
        cin = ch_list[0]
        for i in range(1, len(ch_list)):
            mods.append(nn.Linear(cin, ch_list[i], bias=use_offset))
            cin = ch_list[i]
            if i == len(ch_list) - 1:
                break
            if use_layer_norm:
                mods.append(nn.LayerNorm(ch_list[i]))
            mods.append(nn.SiLU())
        self.net = nn.Sequential(*mods)

    def forward(self, x):
        return self.net(x)


class SO3_Linear_e2former(nn.Module):
    """module_utils.py:2010-2052; input/output in the m-major layout [9, N, C]."""

    def __init__(self, in_features, out_features, lmax, bias=True):
        super().__init__()
        self.in_features, self.out_features, self.lmax = in_features, out_features, lmax
        self.weight = nn.Parameter(torch.randn(lmax + 1, out_features, in_features))
        bound = 1 / math.sqrt(in_features)
        nn.init.uniform_(self.weight, -bound, bound)
        self.bias = nn.Parameter(torch.zeros(out_features))
        self.register_buffer("expand_index", _expand_index(lmax), persistent=False)

    def forward(self, x, bf16: bool = False):
        return SO3LinearFn.apply(x, mrow_weight(self, "weight", self.weight, bf16, self.lmax), self.bias.detach(),
                                 self.lmax)


class SO3_Linear2Scalar_e2former(nn.Module):
    """module_utils.py:2198-2272 (bias on the first product's l = 0 row only)."""

    def __init__(self, in_features, out_features, lmax, hidden_features=None, bias=True):
        super().__init__()
        self.in_features, self.out_features, self.lmax = in_features, out_features, lmax
        hid = out_features // 2 if hidden_features is None else hidden_features
        self.weight = nn.Parameter(torch.randn(lmax + 1, hid, in_features))
        bound = 1 / math.sqrt(in_features)
        nn.init.uniform_(self.weight, -bound, bound)
        self.bias = nn.Parameter(torch.zeros(hid))
        self.weight2 = nn.Parameter(torch.randn(lmax + 1, hid, in_features))
        nn.init.uniform_(self.weight2, -bound, bound)
        self.bias = nn.Parameter(torch.zeros(1, 1, hid))
        self.register_buffer("expand_index", _expand_index(lmax))
        self.final_linear = nn.Sequential(nn.Linear(hid * (lmax + 1), hid), nn.LayerNorm(hid), nn.SiLU(),
                                          nn.Linear(hid, out_features))

    def stacked(self):
        """[W | W2] and [bias | 0] for one fused GEMM."""
        w = torch.cat([self.weight.detach(), self.weight2.detach()], dim=1)
        b = torch.cat([self.bias.detach().view(-1), torch.zeros_like(self.bias.detach().view(-1))])
        return w, b

    def head(self, h, bf16: bool = False):
        """final_linear on the m-contracted products h [N, (lmax+1) hid]."""
        fl = self.final_linear
        if not bf16:
            return _linear(_ln_silu(_linear(h, fl[0]), fl[1]), fl[3])
        h = DenseFn.apply(h, gemm_weight(fl[0], "weight", True), fl[0].bias.detach())
        h = _ln_silu(h, fl[1])
        return DenseFn.apply(h, gemm_weight(fl[3], "weight", True), fl[3].bias.detach())

    def forward(self, x):
        w, b = self.stacked()
        hid = self.weight.shape[1]
        # the pair kernel contracts (q_a, q_b) and (k_a, k_b); feed this product twice
        hq, _, _ = QKProjFn.apply(x, MRowWeight(torch.cat([w, w], dim=1)), torch.cat([b, b]), self.lmax, hid)
        return self.head(hq)


class EquivariantRMSNormArraySphericalHarmonicsV2_BL(nn.Module):
    """module_utils.py:1663-1772 (rms_norm_sh: centering, balanced degrees);
    HIP kernel on the m-major layout."""

    def __init__(self, lmax, num_channels, eps=1e-5, affine=True, normalization="component", centering=True,
                 std_balance_degrees=True):
        super().__init__()
        if not (affine and centering and std_balance_degrees and normalization == "component"):
            raise NotImplementedError("only the rms_norm_sh configuration of the reference is implemented")
        if lmax != 2 or num_channels != 256:
            raise NotImplementedError("the HIP RMS norm is built for lmax 2 and 256 channels")
        self.lmax, self.num_channels, self.eps = lmax, num_channels, eps
        self.affine_weight = nn.Parameter(torch.ones(lmax + 1, num_channels))
        self.affine_bias = nn.Parameter(torch.zeros(num_channels))
        self.register_buffer("expand_index", _expand_index(lmax))
        bw = torch.zeros((lmax + 1) ** 2, 1)
        for l in range(lmax + 1):
            bw[l * l:(l + 1) ** 2] = 1.0 / (2 * l + 1)
        self.register_buffer("balance_degree_weight", bw / (lmax + 1))

    def forward(self, x, batch=None):
        return RMSNormFn.apply(x, self.affine_weight.detach().float().contiguous(),
                               self.affine_bias.detach().float().contiguous(), float(self.eps))

    def add_forward(self, x, delta=None):
        """(norm(x + delta), x + delta); the gradient of the returned sum is added
        in the norm's backward."""
        return AddRMSNormFn.apply(x, delta, self.affine_weight.detach().float().contiguous(),
                                  self.affine_bias.detach().float().contiguous(), float(self.eps))


class Gate_s3(nn.Module):
    """module_utils.py:2694-2746 (HIP activation kernel)."""

    def __init__(self, sphere_channels, lmax, act_scalars="silu", act_vector="sigmoid"):
        super().__init__()
        self.sphere_channels, self.lmax = sphere_channels, lmax
        self.gates = nn.Linear(sphere_channels, sphere_channels * (lmax + 1))
        bound = 1 / math.sqrt(sphere_channels)
        nn.init.uniform_(self.gates.weight, -bound, bound)

    def forward(self, x, bf16: bool = False):
        packs = dense_packs(self.gates, bf16)
        return GateFn.apply(x, gemm_weight(self.gates, "weight", bf16), self.gates.bias.detach(), SILU_NORM,
                            SIGMOID_NORM, packs)


class GateFold:
    """Gate_s3's logit Linear folded into the FFN's first SO3 linear: the logits are
    sc = h[0] Wg^T + bg with h[0] = x[0] W1_0^T + b1 (the l = 0 row carries the bias),
    so sc = x[0] F^T + bs with F = Wg W1_0 [768, 256] and bs = Wg b1 + bg, formed in
    float64 once per weight version.  ``f``: F packed for sc = x[0] F^T; ``bk``: F^T
    packed for the logits' input gradient gsc F (``pieces`` as the FFN's other packs: 3 in
    fp32, 1 — the bf16 rounding of F — in the bf16 mode); ``b``: bs in fp32."""
    __slots__ = ("f", "bk", "b")

    def __init__(self, Wg, bg, W1_0, b1, pieces: int = 3):
        F = (Wg.detach().double() @ W1_0.detach().double()).float().contiguous()
        self.b = (Wg.detach().double() @ b1.detach().double() + bg.detach().double()).float().contiguous()
        self.f = s3gemm.pack(F, pieces=pieces)
        self.bk = s3gemm.pack(F, transpose=True, pieces=pieces)


class FFNS3Fn(torch.autograd.Function):
    """FeedForwardNetwork_s3 (module_utils.py:2755-2797) with Gate_s3 (:2694-2746) on the
    split GEMMs, fp32: one grouped launch forms h = x W1^T (+ b1 on row 0) and the gate
    logits sc = x[0] F^T + bs (GateFold), then y = res + gate(sc, h) W2^T (+ b2 on row 0)
    with the gate applied while the GEMM reads its operand (``e2v2_gemm_s3_gated``: the
    gated activation is never written).  Backward: gy = gout W2, the gate kernel
    (gsc and gh[1:]; h[0] enters only through the logits), and one grouped launch for
    gx[0] = gsc F and gx[1:] = gh[1:] W1.  Input gradients only."""

    @staticmethod
    def forward(ctx, x, W1op, b1, fold: GateFold, k1: float, k2: float, W2op, b2, lmax: int, res=None):
        x = x.contiguous()
        N = x.shape[1]
        f32 = dict(dtype=torch.float32, device=x.device)
        h = torch.empty(x.shape[0], N, W1op.w.shape[1], **f32)
        sc = torch.empty(N, fold.f.n, **f32)
        s3gemm.gemm_grouped([dict(a=x, pw=W1op.s3f(), out=h, widx=_m_degrees(lmax), bias=b1, bias_batches=1),
                             dict(a=x[0], pw=fold.f, out=sc, bias=fold.b)])
        y = torch.empty(x.shape[0], N, W2op.w.shape[1], **f32)
        s3gemm.gemm(h, W2op.s3f(), y, _m_degrees(lmax), bias=b2, bias_batches=1,
                    res=None if res is None else res.contiguous(), gate=(sc, k1, k2))
        ctx.save_for_backward(sc, h)
        ctx.W1op, ctx.fold, ctx.k, ctx.W2op, ctx.lmax, ctx.has_res = W1op, fold, (k1, k2), W2op, lmax, res is not None
        return y

    @staticmethod
    def backward(ctx, gout):
        sc, h = ctx.saved_tensors
        gout = gout.contiguous()
        gy = torch.empty_like(h)
        s3gemm.gemm(gout, ctx.W2op.s3b(), gy, _m_degrees(ctx.lmax))
        gsc = torch.empty_like(sc); gh = torch.empty_like(h)
        _lib.call("e2v2_gate_bwd", _dp(sc), _dp(h), _dp(gy), _dp(gsc), _dp(gh), _lib.i32(h.shape[1]),
                  _lib.f32(ctx.k[0]), _lib.f32(ctx.k[1]), _stream())
        gx = gh.new_empty(gh.shape[0], gh.shape[1], ctx.W1op.w.shape[2])
        s3gemm.gemm_grouped([dict(a=gsc, pw=ctx.fold.bk, out=gx[0]),            # K = 768 first
                             dict(a=gh[1:], pw=ctx.W1op.s3b(), out=gx[1:], widx=_m_degrees(ctx.lmax)[1:])])
        return gx, None, None, None, None, None, None, None, None, (gout if ctx.has_res else None)


class FeedForwardNetwork_s3(nn.Module):
    """module_utils.py:2755-2797."""

    def __init__(self, sphere_channels, hidden_channels, output_channels, lmax):
        super().__init__()
        self.slinear_1 = SO3_Linear_e2former(sphere_channels, hidden_channels, lmax=lmax, bias=True)
        self.gate = Gate_s3(hidden_channels, lmax=lmax)
        self.slinear_2 = SO3_Linear_e2former(hidden_channels, output_channels, lmax=lmax, bias=True)

    def forward(self, x, res=None, bf16: bool = False, **kw):
        with record_function("FeedForwardFunction"):
            s1, s2, g = self.slinear_1, self.slinear_2, self.gate.gates
            W1op = mrow_weight(s1, "weight", s1.weight, bf16, s1.lmax)
            W2op = mrow_weight(s2, "weight", s2.weight, bf16, s2.lmax)
            if (x.dtype == torch.float32 and W1op.split_ok() and W2op.split_ok()
                    and dense_packs(g, bf16) is not None and s1.lmax == s2.lmax == self.gate.lmax
                    and g.weight.shape == (s1.out_features * (s1.lmax + 1), s1.out_features)
                    and s1.out_features == s2.in_features):
                pc = W1op.pieces
                fold = cached(self, "gate_fold_bf16" if bf16 else "gate_fold", (g.weight, g.bias, s1.weight, s1.bias),
                              lambda: GateFold(g.weight, g.bias, s1.weight[0], s1.bias, pc))
                return FFNS3Fn.apply(x, W1op, s1.bias.detach(), fold, SILU_NORM, SIGMOID_NORM, W2op,
                                     s2.bias.detach(), s2.lmax, res)
            h = s1(x, bf16)
            h = self.gate(h, bf16)
            return SO3LinearFn.apply(h, W2op, s2.bias.detach(), s2.lmax, res)


class sph_fromxyz(nn.Module):
    """module_utils.py:136-176 (state_dict parameter W; not used on the path)."""

    def __init__(self, lmax=2):
        super().__init__()
        self.lmax = lmax
        rt5, rt15 = math.sqrt(5.0), math.sqrt(15.0)
        W = torch.zeros(5, 9)
        W[0, 2] = rt15; W[1, 1] = rt15; W[2, 4] = rt5; W[2, 0] = -0.5 * rt5; W[2, 8] = -0.5 * rt5
        W[3, 5] = rt15; W[4, 8] = 0.5 * rt15; W[4, 0] = -0.5 * rt15
        self.W = nn.Parameter(W.t(), requires_grad=False)


class SO2_TP_givenl2(nn.Module):
    """so2_tensor_product.py:182-290 for l1 = 0..lmax, l2 = 1 (table parameters +
    the per-l3 output linears).  The gather itself is folded into the edge kernel
    through the Cartesian coupling table of ``so3``; loaded ``CG_weight`` values
    scale each coupling path."""

    def __init__(self, lmax, in_c, out_c):
        super().__init__()
        paths, seq, sel, w, pn = so3.so2_gather_tables(lmax)
        self.l3_sequential = seq
        self.in_c, self.out_c = in_c, out_c
        self.out_linear = nn.ModuleList([nn.Linear(cnt * in_c, out_c, bias=False) for l3, cnt in seq])
        self.path_norm = nn.Parameter(torch.from_numpy(pn).reshape(1, -1, 1), requires_grad=False)
        self.selected_idx = nn.Parameter(torch.from_numpy(sel).long(), requires_grad=False)
        self.CG_weight = nn.Parameter(torch.from_numpy(w).float(), requires_grad=False)
        self._canon_sel = sel
        self._canon_w = w
        self._rows = so3.path_rows(lmax)
        self._scale_key = None
        self._scale = None

    def path_scales(self) -> Optional[torch.Tensor]:
        """Per-row scale of the 20 output rows implied by the loaded CG_weight
        relative to the canonical table, or None when they coincide (cached on
        the parameters' version counters: no host sync per call)."""
        key = (self.selected_idx._version, self.CG_weight._version, self.CG_weight.data_ptr(),
               self.selected_idx.data_ptr())
        if key != self._scale_key:
            self._scale = self._compute_scales()
            if self._scale is not None:
                self._scale = self._scale.to(self.CG_weight.device)
            self._scale_key = key
        return self._scale

    def _compute_scales(self) -> Optional[torch.Tensor]:
        sel = self.selected_idx.detach().cpu().numpy()
        w = self.CG_weight.detach().float().cpu().numpy()
        if not np.array_equal(sel, self._canon_sel):
            raise NotImplementedError("SO2_TP_givenl2.selected_idx differs from the canonical coupling table")
        if np.array_equal(w, self._canon_w):
            return None
        scale = np.ones(len(w), np.float32)
        for (t0, t1) in self._rows:
            c, l = self._canon_w[t0:t1], w[t0:t1]
            nz = np.abs(c) > 0
            r = l[nz] / c[nz]
            if not np.allclose(r, r[0], rtol=1e-6, atol=0) or np.any(l[~nz] != 0):
                raise NotImplementedError("CG_weight is not a per-path rescaling of the coupling table")
            scale[t0:t1] = r[0]
        return torch.from_numpy(scale)

    def folded_blocks(self, bf16: bool = False, sliced: bool = False):
        """Per output l3: list of (input row start, rows, W_p^T) with path_norm and
        loaded CG_weight path scales folded into W_p (cached on versions); bf16
        copies of the folded blocks in bf16 mode.  ``sliced``: the rows of W_p^T
        permuted to the attention kernels' slice order of the input channels."""
        if sliced:
            def build_sliced():
                P = slice_perm(self.path_norm.device)
                return [[(t0, nr, Wt[P].contiguous()) for (t0, nr, Wt) in lst] for lst in self.folded_blocks(bf16)]
            return cached(self, "fold_sl_bf16" if bf16 else "fold_sl", list(self.parameters()), build_sliced)
        if bf16:
            return cached(self, "fold_bf16", list(self.parameters()),
                          lambda: [[(t0, nr, Wt.to(BF16).contiguous()) for (t0, nr, Wt) in lst]
                                   for lst in self.folded_blocks()])
        key = tuple((p.data_ptr(), p._version) for p in self.parameters())
        if getattr(self, "_fold_key", None) == key:
            return self._fold
        sc = self._compute_scales()
        pn = self.path_norm.detach().view(-1)
        blocks, t0, o0 = [], 0, 0
        for idx, (l3, cnt) in enumerate(self.l3_sequential):
            W = self.out_linear[idx].weight.detach()
            lst = []
            for p in range(cnt):
                Wp = W[:, p * self.in_c:(p + 1) * self.in_c] * pn[o0]
                if sc is not None:
                    Wp = Wp * float(sc[t0])
                lst.append((t0, 2 * l3 + 1, Wp.t().contiguous()))
                t0 += 2 * l3 + 1
            blocks.append(lst)
            o0 += 2 * l3 + 1
        self._fold, self._fold_key = blocks, key
        return blocks

    def forward_linear(self, so2):
        """so2 [20, N, C] (m-major, l3-sequential rows) -> [9, N, C_out]."""
        N = so2.shape[1]
        outs = []
        for lst in self.folded_blocks():
            acc = None
            for (t0, nr, Wt) in lst:
                xin = so2[t0:t0 + nr].reshape(nr * N, -1)
                acc = torch.mm(xin, Wt) if acc is None else torch.addmm(acc, xin, Wt)
            outs.append(acc.view(-1, N, acc.shape[-1]))
        return torch.cat(outs, dim=0)


class E2TensorProductSO2_FirstOrder(nn.Module):
    """so2_tensor_product.py:297-389 (parameters; the product itself runs in the edge kernel)."""

    def __init__(self, irreps_in, irreps_out, head, order=1, lmax=2, in_c=256, out_c=256, **kw):
        super().__init__()
        self.head, self.in_c, self.out_c, self.lmax, self.order = head, in_c, out_c, lmax, order
        self.so2_tp = SO2_TP_givenl2(lmax, in_c, out_c)


class SmoothLeakyReLU(nn.Module):
    def __init__(self, negative_slope=0.2):
        super().__init__()
        self.alpha = negative_slope

    def forward(self, x):
        return (1 - self.alpha) * x * torch.sigmoid(x) + self.alpha * x


class EdgeContext:
    """Per-evaluation edge data shared by every layer: the neighbour list, the edge
    geometry, each atom's type slot (atom_type [N], into type_z [T], the atomic
    numbers present; type_key = (host tuple of type_z, the type-slot pairs the
    radial tables hold or None for all T^2), see ``atom_type_slots``) for the
    radial tables, and
    the distance envelope of the attention weights (poly_dist): env_kind 0 the
    polynomial on [0, rc] (module_utils.py:1946-1954), 1 the smooth bell on
    [env_lo, rc] (module_utils.py:1956-1985), the long-range list's "poly_bell"."""

    def __init__(self, nl, dvec, dist, atom_type, type_z, type_key, rbf: GaussianSmearing, rc: float,
                 bf16: bool = False, env_kind: int = 0, env_lo: float = 0.0):
        self.nl, self.dvec, self.dist = nl, dvec, dist
        self.atom_type, self.type_z, self.type_key = atom_type, type_z, type_key
        self.pairs = type_key[1]
        self.rbf_offset = rbf.offset.float().contiguous()
        self.rbf_coeff = float(rbf.coeff)
        self.rc = rc
        self.bf16 = bf16          # bf16 GEMM operands, fp32 accumulation and storage
        if env_kind not in (0, 1) or (env_kind == 1 and not 0.0 <= env_lo < rc):
            raise ValueError(f"envelope kind {env_kind} on [{env_lo}, {rc}] is not supported")
        self.env_kind, self.env_lo = int(env_kind), float(env_lo)


def atom_type_slots(Z: torch.Tensor, graph_ptr=None):
    """(type_z [T] int32: the atomic numbers present, ascending; type_key =
    (the same as a host tuple, pairs); slot [N] int32: each atom's index into
    type_z).  pairs: the ordered type-slot pairs (a, b) an edge can join, the
    union over the graphs (graph_ptr [B+1], host) of the products of each graph's
    own type set, since edges never leave their graph; None when that is every
    pair (one graph, or no graph_ptr): the radial tables then hold all T^2.  One
    host read."""
    Zl = Z.long()
    ptr = None if graph_ptr is None else np.asarray(graph_ptr, np.int64)
    if ptr is None or len(ptr) <= 2:
        codes = torch.unique(Zl).cpu().numpy()
        gz = None
    else:
        B = len(ptr) - 1
        gid = torch.repeat_interleave(torch.arange(B, device=Z.device), torch.as_tensor(np.diff(ptr), device=Z.device))
        codes = torch.unique(gid * 1024 + Zl).cpu().numpy()
        gz = (codes // 1024, codes % 1024)
        codes = np.unique(gz[1])
    key = tuple(int(z) for z in codes)
    if key and (key[0] < 0 or key[-1] > 255):
        raise ValueError(f"atomic numbers must lie in [0, 255], got {key[0]}..{key[-1]}")
    T = len(key)
    pairs = None
    if gz is not None:
        idx = {z: a for a, z in enumerate(key)}
        per = {}
        for g, z in zip(gz[0].tolist(), gz[1].tolist()):
            per.setdefault(g, []).append(idx[z])
        ps = sorted({(a, b) for sl in per.values() for a in sl for b in sl})
        pairs = None if len(ps) == T * T else tuple(ps)
    zs = torch.as_tensor(np.asarray(key, np.int64), device=Z.device)
    lut = torch.zeros(256, dtype=torch.int32, device=Z.device)
    lut[zs] = torch.arange(T, dtype=torch.int32, device=Z.device)
    return zs.to(torch.int32).contiguous(), (key, pairs), lut[Zl].contiguous()


_REF_CTX_KEY = "_e2v2_edge_context"


def reference_edge_context(batched_data, edge_vec, edge_dis, atomic_numbers, rbf, rc: float,
                           bf16: bool = False, env=(0, 0.0)) -> EdgeContext:
    """EdgeContext from the per-forward edge inputs of the reference's layers:
    batched_data's construct_radius_neighbor dict (query_idx, neighbor_idx,
    metadata) and f_outcell_index (expanded node -> atom), the edge vectors and
    distances (f_edge_vec, f_dist; gradients flow back to them), the flattened
    atomic numbers, the E2former's GaussianSmearing and cutoff.  Edges are taken
    in query-row order (the metadata's q_alpha_index, the identity for the
    reference's sorted lists).  env: the envelope (kind, lower end) of
    EdgeContext.  Built once per batched_data and reused by every layer (kept in
    batched_data under "_e2v2_edge_context")."""
    ent = batched_data.get(_REF_CTX_KEY)
    if ent is not None and ent[0] is batched_data["query_idx"] and ent[1] is edge_vec and ent[2] is edge_dis \
            and ent[3] is atomic_numbers and ent[5] == (float(rc), int(env[0]), float(env[1]), bool(bf16)):
        return ent[4]
    from .neighbors import neighbor_list_from_edges
    md = batched_data["metadata"]
    if len(md) != 6:
        raise ValueError("metadata must be a 6-tuple from prepare_sparse_qk_edge_index_metadata")
    order = md[2].long()
    src = batched_data["f_outcell_index"].long()[batched_data["neighbor_idx"].long().index_select(0, order)]
    dvec = edge_vec.index_select(0, order).float()
    dist = edge_dis.reshape(-1).index_select(0, order).float()
    N = int(atomic_numbers.shape[0])
    nl = neighbor_list_from_edges(md[0], src, dvec, dist, N)
    type_z, type_key, slot = atom_type_slots(atomic_numbers)
    ctx = EdgeContext(nl, dvec, dist, slot, type_z, type_key, rbf, float(rc), bf16, env[0], env[1])
    batched_data[_REF_CTX_KEY] = (batched_data["query_idx"], edge_vec, edge_dis, atomic_numbers, ctx,
                                  (float(rc), int(env[0]), float(env[1]), bool(bf16)))
    return ctx


def _raw_sh(v: torch.Tensor) -> torch.Tensor:
    """The raw real spherical-harmonic polynomials l <= 2 of e3nn's
    ``_spherical_harmonics`` (y the polar axis) of the vector v [E, 3] itself,
    [E, 9]: 1 | x, y, z | sqrt3 x z, sqrt3 x y, y^2 - (x^2 + z^2) / 2, sqrt3 y z,
    sqrt3 / 2 (z^2 - x^2)."""
    x, y, z = v[:, 0], v[:, 1], v[:, 2]
    s3 = math.sqrt(3.0)
    return torch.stack([torch.ones_like(x), x, y, z, s3 * x * z, s3 * x * y, y * y - 0.5 * (x * x + z * z),
                        s3 * y * z, s3 / 2 * (z * z - x * x)], dim=-1)


_SH_INTEGRAL = [math.sqrt(2 * l + 1) / math.sqrt(4 * math.pi) for l in (0, 1, 1, 1, 2, 2, 2, 2, 2)]


def _sh_integral(v: torch.Tensor) -> torch.Tensor:
    """e3nn.o3.spherical_harmonics(l, v, normalize=True) for l = 0, 1, 2
    concatenated, [E, 9]: the raw polynomials of v / |v| times
    sqrt(2 l + 1) / sqrt(4 pi) (e3nn's default "integral" normalisation)."""
    u = v / v.norm(dim=-1, keepdim=True)
    return _raw_sh(u) * torch.tensor(_SH_INTEGRAL, dtype=v.dtype, device=v.device)


def _profile_with_rows(net: nn.Sequential, w3: torch.Tensor, b3: torch.Tensor) -> nn.Sequential:
    """A RadialProfile net with the first five layers of ``net`` and a last Linear
    of the given rows (w3 [256, 128], b3 [256]): the 256-channel profiles the
    radial tables are built from, for profiles of another width (rows taken out
    of them, or zero rows for channels a table must hold but nothing reads)."""
    lin = nn.Linear(w3.shape[1], w3.shape[0]).to(w3.device)
    with torch.no_grad():
        lin.weight.copy_(w3)
        lin.bias.copy_(b3)
    return nn.Sequential(net[0], net[1], net[2], net[3], net[4], net[5], lin)


class E2AttentionArbOrder_sparse(nn.Module):
    """e2former.py:80-436 for attn_type so2-first-order or zero-order
    (proj_zero on the alpha-weighted sum of the neighbours' values,
    e2former.py:199-204,411-416) and tp_type QK_alpha, QKdot_alpha (gate from
    the spherical harmonics of the edge against dot_linear of the query node,
    e2former.py:143-154,270-283) or QKdotS_alpha (e2former.py:155-167,284-300),
    each with the segmented softmax or, with "+softplus" / "+sigmoid" in
    tp_type, alpha = act(gate q.k) inputhead p (e2former.py:123-124,329-332).
    The QKdot gates are formed per edge (e2v2_sh_contract, e2v2_radial_eval,
    the gate's small dense layers) and handed to the attention kernels as their
    gate; the inputhead stays a table inside the kernels."""

    def __init__(self, irreps_node_input="256x0e+256x1e+256x2e", attn_weight_input_dim=256, num_attn_heads=128,
                 attn_scalar_head=8, irreps_head="2x0e+2x1e+2x2e", alpha_drop=0.0, tp_type="QK_alpha",
                 attn_type="so2-first-order", atom_type_cnt=256, norm_layer="rms_norm_sh", C=256, lmax=2, **kw):
        super().__init__()
        self.num_attn_heads, self.attn_scalar_head, self.lmax = num_attn_heads, attn_scalar_head, lmax
        self.node_embed_dim = 128
        self.attn_type, self.tp_type = attn_type, tp_type.split("+")[0]
        # the weight form: substring tests on the whole tp_type, softplus first (e2former.py:123-124, 329-332)
        self.weight_act = "softplus" if "softplus" in tp_type else "sigmoid" if "sigmoid" in tp_type else "softmax"
        self.source_embedding = nn.Embedding(atom_type_cnt, 128)
        self.target_embedding = nn.Embedding(atom_type_cnt, 128)
        nn.init.uniform_(self.source_embedding.weight.data, -0.001, 0.001)
        nn.init.uniform_(self.target_embedding.weight.data, -0.001, 0.001)
        self.alpha_act = SmoothLeakyReLU(0.2)
        ecl = [attn_weight_input_dim + 256, min(128, attn_weight_input_dim // 2),
               min(128, attn_weight_input_dim // 2)]
        self.alpha_dropout = nn.Dropout(alpha_drop)
        H = num_attn_heads
        if self.tp_type == "QKdot_alpha":
            self.dot_linear = SO3_Linear_e2former(C, attn_weight_input_dim, lmax=lmax)
            self.rad_func_m0 = RadialProfile(ecl + [attn_weight_input_dim * (lmax + 1)])
            self.fc_m0 = nn.Linear(attn_weight_input_dim * (lmax + 1), H)
            self.fc_easy = RadialProfile(ecl + [H])
        elif self.tp_type == "QKdotS_alpha":
            sv = torch.zeros((lmax + 1) ** 2, lmax + 1)
            for l in range(lmax + 1):
                sv[l * l:(l + 1) ** 2, l] = 1
            self.sum_vec = nn.Parameter(sv, requires_grad=False)
            self.dot_linear = SO3_Linear_e2former(C, H // (lmax + 1) + 1, lmax=lmax)
            self.direction_linear = nn.Sequential(nn.Linear(H, H), nn.LayerNorm(H), nn.SiLU(), nn.Linear(H, H))
            self.fc_easy = RadialProfile(ecl + [2 * H])
        elif self.tp_type == "QK_alpha":
            self.fc_easy = RadialProfile(ecl + [2 * H])
        else:
            raise NotImplementedError(f"tp_type {tp_type!r}: the HIP path implements QK_alpha, QKdot_alpha and "
                                      "QKdotS_alpha")
        self._radial_m0 = RadialCache()
        self.query_linear = SO3_Linear2Scalar_e2former(C, num_attn_heads * attn_scalar_head, lmax=lmax)
        self.key_linear = SO3_Linear2Scalar_e2former(C, num_attn_heads * attn_scalar_head, lmax=lmax)
        self.proj_value = SO3_Linear_e2former(C, C, lmax=lmax)
        if attn_type == "zero-order":
            self.proj_zero = SO3_Linear_e2former(C, C, lmax=lmax)
        elif attn_type == "so2-first-order":
            self.first_order_tp = E2TensorProductSO2_FirstOrder(None, None, head=num_attn_heads, order=1,
                                                                lmax=lmax, in_c=C, out_c=C)
            self.proj_first = SO3_Linear_e2former(num_attn_heads * 2, C, lmax=lmax)
        else:
            raise NotImplementedError(f"attn_type {attn_type!r}: the HIP path implements so2-first-order and "
                                      "zero-order")
        self._radial = RadialCache()

    def qk_weights(self, bf16: bool = False):
        params = (self.query_linear.weight, self.query_linear.weight2, self.query_linear.bias,
                  self.key_linear.weight, self.key_linear.weight2, self.key_linear.bias)

        def build():
            wq, bq = self.query_linear.stacked()
            wk, bk = self.key_linear.stacked()
            w = torch.cat([wq, wk], dim=1).contiguous()
            return w, torch.cat([bq, bk]).float().contiguous()
        w, b = cached(self, "qk", params, build)
        return mrow_weight(self, "qk", w, bf16, self.lmax), b

    def qk_s3_packs(self, bf16: bool = False):
        """The split-GEMM packs of the Q/K projection (query and key weights, their
        bias, and the sliced value projection whose input gradient the backward
        adds; one bf16 piece in the bf16 mode), or None when the split GEMM does
        not apply (cached per version)."""
        Wop, b = self.qk_weights(False)
        wv, _ = self.value_weights_sliced()
        W = Wop.w
        if not ((bf16 or split_gemm_on()) and W.is_cuda and W.dtype == torch.float32
                and s3gemm.qk_supported(W.shape[1] // 4, W.shape[2], wv.shape[1])):
            return None
        pv = self.proj_value
        params = (self.query_linear.weight, self.query_linear.weight2, self.query_linear.bias,
                  self.key_linear.weight, self.key_linear.weight2, self.key_linear.bias, pv.weight, pv.bias)
        return cached(self, "qk_bf16" if bf16 else "qk_s3", params,
                      lambda: s3gemm.pack_qk(W, b, wv, pieces=1 if bf16 else 3))

    def qk_head_packs(self, bf16: bool = False):
        """Split-GEMM packs of the query and key final_linear (cached per version;
        one bf16 piece in the bf16 mode), or None when the split GEMM does not
        apply."""
        return head_pair_packs(self.query_linear.final_linear, self.key_linear.final_linear, self, bf16)

    def value_weights_sliced(self):
        """proj_value's weight and bias with the output channels in the attention
        kernels' slice order (cached per weight version)."""
        pv = self.proj_value

        def build():
            P = slice_perm(pv.weight.device)
            return pv.weight.detach()[:, P, :].contiguous(), pv.bias.detach()[P].contiguous()
        return cached(self, "v_sliced", (pv.weight, pv.bias), build)

    def bind_edge_basis(self, rbf, max_radius: float, poly: str = "poly", min_dist: float = 0.0):
        """The E2former's GaussianSmearing and cutoff, for calls with the
        reference's signature (attn_weight = rbf(edge_dis) is evaluated inside
        the kernels from the distance, as is poly_dist: poly "poly" for
        polynomial(d, max_radius), "poly_bell" for the bell on [min_dist,
        max_radius] of the long-range list)."""
        self._edge_basis = (rbf, float(max_radius), _env_of(poly, min_dist))
        return self

    def forward(self, *args, **kwargs):
        """forward(x [9, N, C], ctx: EdgeContext, res=None) -> [9, N, C] (the fused
        path of this package), or the reference's signature (e2former.py:223-236)
        -> (node_output [N, 9, C], attn_weight)."""
        if len(args) >= 2 and isinstance(args[1], EdgeContext):
            return self.forward_fused(*args, **kwargs)
        return self.forward_reference(*args, **kwargs)

    def forward_reference(self, node_pos, node_irreps_input, edge_dis, edge_vec, attn_weight, atomic_numbers,
                          poly_dist=None, attn_mask=None, batch=None, batched_data=None, rbf=None, max_radius=None,
                          poly=None, min_dist=None, **kwargs):
        """E2AttentionArbOrder_sparse.forward (e2former.py:223-436) with its
        arguments: node_irreps_input [N, 9, C]; batched_data holds query_idx,
        neighbor_idx, metadata and f_outcell_index; edge_vec / edge_dis are
        f_edge_vec / f_dist.  attn_weight must be rbf(edge_dis) and poly_dist
        polynomial(edge_dis, max_radius) (poly="poly", the default) or
        smooth_polynomial_bell(edge_dis, min_dist, max_radius) (poly="poly_bell"),
        both re-evaluated inside the kernels from the distance; rbf, max_radius,
        poly and min_dist come from the keywords or bind_edge_basis.  Returns
        (node_output [N, 9, C], attn_weight)."""
        if batched_data is None:
            raise ValueError("batched_data with the neighbour dict is required")
        basis = getattr(self, "_edge_basis", None)
        if rbf is None or max_radius is None:
            if basis is None:
                raise ValueError("pass rbf= and max_radius= (the E2former's GaussianSmearing and cutoff) or call "
                                 "bind_edge_basis(rbf, max_radius) once")
            rbf, max_radius = basis[:2]
        if poly is None and min_dist is None and basis is not None:
            env = basis[2]
        else:
            env = _env_of(poly or "poly", 0.0 if min_dist is None else min_dist)
        ctx = reference_edge_context(batched_data, edge_vec, edge_dis, atomic_numbers, rbf, max_radius, env=env)
        x = node_irreps_input.float().transpose(0, 1).contiguous()
        out = self.forward_fused(x, ctx)
        return out.transpose(0, 1).contiguous(), attn_weight

    def _attn_profile(self):
        """The net of the attention kernels' table (256 channels: gate | inputhead):
        fc_easy itself for QK_alpha; for the QKdot variants, whose gate comes from
        outside, zero gate rows and the inputhead rows of fc_easy (all of its 128
        for QKdot_alpha, its first 128 for QKdotS_alpha)."""
        net = self.fc_easy.net
        if self.tp_type == "QK_alpha":
            return net

        def build():
            w3, b3 = net[6].weight.detach(), net[6].bias.detach()
            H = self.num_attn_heads
            w = torch.cat([torch.zeros(H, w3.shape[1], device=w3.device), w3[:H]])
            b = torch.cat([torch.zeros(H, device=b3.device), b3[:H]])
            return _profile_with_rows(net, w, b)
        return cached(self, "attn_profile", list(self.fc_easy.parameters()), build)

    def _m0_profiles(self):
        """Nets of the per-edge radial profile of the QKdot gate, 256 channels each:
        rad_func_m0's 768 outputs in three (QKdot_alpha), or the second half of
        fc_easy then zero rows (QKdotS_alpha)."""
        if self.tp_type == "QKdot_alpha":
            net = self.rad_func_m0.net

            def build():
                w3, b3 = net[6].weight.detach(), net[6].bias.detach()
                return [_profile_with_rows(net, w3[256 * m:256 * (m + 1)], b3[256 * m:256 * (m + 1)])
                        for m in range(w3.shape[0] // 256)]
            return cached(self, "m0_profiles", list(self.rad_func_m0.parameters()), build)
        net = self.fc_easy.net

        def build_s():
            w3, b3 = net[6].weight.detach(), net[6].bias.detach()
            H = self.num_attn_heads
            w = torch.cat([w3[H:], torch.zeros(256 - H, w3.shape[1], device=w3.device)])
            b = torch.cat([b3[H:], torch.zeros(256 - H, device=b3.device)])
            return [_profile_with_rows(net, w, b)]
        return cached(self, "m0_profiles", list(self.fc_easy.parameters()), build_s)

    def qkdot_gate(self, x: torch.Tensor, ctx: EdgeContext) -> torch.Tensor:
        """The gate [E, H] of the QKdot variants in the edge order of ctx.nl, from
        the layer input x [9, N, C] (e2former.py:270-300)."""
        nl = ctx.nl
        E, H = nl.n_edges, self.num_attn_heads
        xd = self.dot_linear(x, ctx.bf16)                                     # [9, N, Cd]
        tab = self._radial_m0.get(self._m0_profiles(), self.target_embedding, self.source_embedding,
                                  ctx.rbf_offset, ctx.rbf_coeff, ctx.rc, ctx.type_z, ctx.type_key, layout="plain",
                                  pairs=ctx.pairs)
        if self.tp_type == "QKdot_alpha":
            packs = dense_packs(self.fc_m0, ctx.bf16)
            if packs is not None and xd.shape[2] == 256 and H == 128 and tab.nc == 768:
                # the 768-wide edge operand is formed inside the gate GEMM (no per-edge channel tensor)
                return QKdotGateFn.apply(ctx.dist, _sh_integral(ctx.dvec), xd, nl, ctx.atom_type, tab, packs,
                                         self.fc_m0.bias.detach())
            rad = RadialEvalFn.apply(ctx.dist, nl, ctx.atom_type, tab)
            x0 = ShContractFn.apply(_sh_integral(ctx.dvec), xd, nl).reshape(E, -1)    # [E, 3 Cd]
            return _linear(x0 * rad, self.fc_m0)
        rad = RadialEvalFn.apply(ctx.dist, nl, ctx.atom_type, tab)
        # checked once per version of sum_vec (a host readback), not on every evaluation
        if not cached(self, "sum_vec_ok", (self.sum_vec,),
                      lambda: torch.equal(self.sum_vec.detach().cpu(), self._sum_vec_blocks())):
            raise NotImplementedError("QKdotS_alpha: sum_vec must keep its l-block indicator values")
        x0 = ShContractFn.apply(_raw_sh(ctx.dvec), xd, nl).reshape(E, -1)[:, :H]     # [E, H]
        dl = self.direction_linear
        return _linear(_ln_silu(_linear(x0 * rad[:, :H], dl[0]), dl[1]), dl[3])

    def _sum_vec_blocks(self):
        L = self.lmax + 1
        sv = torch.zeros(L * L, L)
        for l in range(L):
            sv[l * l:(l + 1) ** 2, l] = 1
        return sv

    def zero_out_weights(self, bf16: bool = False):
        """proj_zero as the operand list of SO2OutFn for the zero-order rows
        [9, N, C]: per degree l, (l, 1, C l^2, W, W^T) with W = W_l^T [C, O], input
        rows in the kernels' slice order (bf16 copies in bf16 mode)."""
        pz = self.proj_zero

        def build():
            P = slice_perm(pz.weight.device)
            C = pz.weight.shape[2]
            dt = BF16 if bf16 else torch.float32
            out = []
            for l in range(self.lmax + 1):
                W = pz.weight.detach()[l][:, P].t()
                out.append((l, 1, C * l * l, W.to(dt).contiguous(), W.t().to(dt).contiguous()) + _so2_packs(W, bf16))
            return out
        key = "zero_out_bf16" if bf16 else ("zero_out_s3" if split_gemm_on() else "zero_out")
        return cached(self, key, (pz.weight,), build)

    def so2_out_weights(self, bf16: bool = False):
        """Per output degree l3 (l3 order): (l3, cnt, start, W, W^T) with W [cnt 256, O]
        = forward_linear's folded blocks of that degree stacked along K (input rows
        in the kernels' slice order, path_norm and path scales folded) times
        proj_first's W_l3^T, formed in float64 and rounded once (bf16 copies in bf16
        mode); start = the block's offset / N in the l3-grouped attention output.
        Cached on the parameters' versions."""
        tp = self.first_order_tp.so2_tp
        pf = self.proj_first
        params = list(tp.parameters()) + [pf.weight]

        def build():
            out = []
            for (l3, cnt, start), lst in zip(so3.so2_row_layout()[3], tp.folded_blocks(False, sliced=True)):
                Wcat = torch.cat([Wt.double() for (_, _, Wt) in lst], dim=0)
                W = Wcat @ pf.weight.detach()[l3].double().t()
                dt = BF16 if bf16 else torch.float32
                Wf = W.float()
                out.append((l3, cnt, start, W.to(dt).contiguous(), W.t().to(dt).contiguous()) + _so2_packs(Wf, bf16))
            return out
        key = "so2_out_bf16" if bf16 else ("so2_out_s3" if split_gemm_on() else "so2_out")
        return cached(self, key, params, build)

    def forward_fused(self, x: torch.Tensor, ctx: EdgeContext, res: Optional[torch.Tensor] = None):
        """x [9, N, C] (m-major) -> attention(x) (+ res when given), [9, N, C].
        v, the attention rows and their gradients run in the kernels' slice order
        of channels: the permutation is folded into proj_value (output rows) and
        forward_linear (input rows), so the layer's output is in model order."""
        N = x.shape[1]
        H = self.num_attn_heads
        if self.training and self.alpha_dropout.p > 0:
            raise NotImplementedError("attention dropout in training mode is not supported by the HIP path")
        bf16 = ctx.bf16
        W, b = self.qk_weights(bf16)
        hid = self.query_linear.weight.shape[1]
        pv = self.proj_value  # its GEMMs run inside QKProjFn (one input gradient)
        wv, bv = self.value_weights_sliced()
        with record_function("query key linear function"):
            s3 = self.qk_s3_packs(bf16)
            Wvop = mrow_weight(pv, "weight_sl", wv, bf16, pv.lmax)
            heads = self.qk_head_packs(bf16)
            # bf16 mode: projections and attention as one autograd node (AttnBlockBF16Fn, below)
            block_bf16 = bf16 and s3 is not None and heads is not None and Wvop.split_ok()
            if block_bf16:
                pass
            elif s3 is not None and heads is not None and Wvop.split_ok():
                q, k, v = AttnProjS3Fn.apply(x, s3, heads, Wvop, bv)
                q, k = q.reshape(N, H, -1), k.reshape(N, H, -1)
            elif heads is not None:
                hq, hk, v = QKProjFn.apply(x, W, b, self.lmax, hid, Wvop, bv, s3)
                q, k = QKHeadsS3Fn.apply(hq, hk, heads)
                q, k = q.reshape(N, H, -1), k.reshape(N, H, -1)
            else:
                hq, hk, v = QKProjFn.apply(x, W, b, self.lmax, hid, Wvop, bv, s3)
                q = self.query_linear.head(hq, bf16).reshape(N, H, -1)
                k = self.key_linear.head(hk, bf16).reshape(N, H, -1)
        with record_function("rbf function-a"):   # fc_easy as a distance table, built once per weight version
            table = self._radial.get([self._attn_profile()], self.target_embedding, self.source_embedding,
                                     ctx.rbf_offset, ctx.rbf_coeff, ctx.rc, ctx.type_z, ctx.type_key, layout="attn",
                                     pairs=ctx.pairs)
        zero = self.attn_type == "zero-order"
        with record_function("qk attention"):
            gate = None if self.tp_type == "QK_alpha" else self.qkdot_gate(x, ctx)
            if block_bf16:
                so2 = AttnBlockBF16Fn.apply(x, ctx.dvec, ctx.dist, gate, s3, heads, Wvop, bv, ctx.nl, ctx.atom_type,
                                            table, ctx.rc, math.sqrt(self.attn_scalar_head), zero,
                                            (ctx.env_kind, ctx.env_lo), self.weight_act)
            else:
                so2 = AttentionFn.apply(q, k, v, ctx.dvec, ctx.dist, ctx.nl, ctx.atom_type, table, ctx.rc,
                                        math.sqrt(q.shape[-1]), BF16 if bf16 else torch.float32, zero,
                                        (ctx.env_kind, ctx.env_lo), gate, self.weight_act)
        if zero:
            with record_function("zero-order"):
                return SO2OutFn.apply(so2.view(-1), res, self.zero_out_weights(bf16), self.proj_zero.bias.detach(),
                                      N)
        pf = self.proj_first
        with record_function("first-order"):
            return SO2OutFn.apply(so2, res, self.so2_out_weights(bf16), pf.bias.detach(), N)


def _so2_packs(W: torch.Tensor, bf16: bool):
    """(forward, backward) split-GEMM packs of an SO2OutFn operand W [K, O] (y = A W,
    gA = gy W^T; one bf16 piece in the bf16 mode), or (None, None) with the fp32
    split GEMM off or for an unsupported shape."""
    K, O = W.shape
    if (not bf16 and not split_gemm_on()) or not W.is_cuda or not (s3gemm.supported(O, K) and s3gemm.supported(K, O)):
        return (None, None)
    W = W.float().contiguous()
    pc = 1 if bf16 else 3
    return (s3gemm.pack(W, transpose=True, pieces=pc), s3gemm.pack(W, pieces=pc))


def _env_of(poly: str, min_dist: float):
    """EdgeContext's envelope (kind, lower end) of construct_radius_neighbor's
    ``poly`` argument (module_utils.py:3184-3191)."""
    if poly == "poly":
        return (0, 0.0)
    if poly == "poly_bell":
        return (1, float(min_dist))
    raise ValueError("sorry, you must set poly or poly_bell")


class TransBlock(nn.Module):
    """e2former.py:440-620."""

    def __init__(self, irreps_node_input="256x0e+256x1e+256x2e", irreps_node_output="256x0e+256x1e+256x2e",
                 attn_weight_input_dim=256, num_attn_heads=128, attn_scalar_head=8, irreps_head="2x0e+2x1e+2x2e",
                 alpha_drop=0.0, tp_type="QK_alpha", attn_type="so2-first-order", atom_type_cnt=256,
                 norm_layer="rms_norm_sh", ffn_type="s3", layer_id=0, C=256, lmax=2):
        super().__init__()
        self.lmax = lmax
        self.norm_1 = EquivariantRMSNormArraySphericalHarmonicsV2_BL(lmax, C)
        self.ga = E2AttentionArbOrder_sparse(irreps_node_input, attn_weight_input_dim, num_attn_heads,
                                             attn_scalar_head, irreps_head, alpha_drop, tp_type, attn_type,
                                             atom_type_cnt, norm_layer, C=C, lmax=lmax)
        self.norm_ffn = EquivariantRMSNormArraySphericalHarmonicsV2_BL(lmax, C)
        self.ffn = FeedForwardNetwork_s3(C, C, C, lmax)

    def forward(self, x, ctx: EdgeContext, sys_node_embedding=None):
        """x [9, N, C] m-major -> the block output."""
        x, d = self.forward_deferred(x, None, ctx, sys_node_embedding)
        return x + d

    def forward_deferred(self, x, delta, ctx: EdgeContext, sys_node_embedding=None):
        """(x', d) with block output x' + d for the input x + delta: each residual
        add is left to the RMS norm that reads its result next."""
        h, x = self.norm_1.add_forward(x, delta)
        if sys_node_embedding is not None:
            h = torch.cat([(h[0] + sys_node_embedding).unsqueeze(0), h[1:]], dim=0)
        d = self.ga(h, ctx)
        h, x = self.norm_ffn.add_forward(x, d)
        return x, self.ffn(h, bf16=ctx.bf16)


class EdgeDegreeEmbeddingNetwork_higherorder(nn.Module):
    """e2former.py:623-753 (use_atom_edge=True, layer norm on)."""

    def __init__(self, irreps_node_embedding="256x0e+256x1e+256x2e", avg_aggregate_num=23.01, number_of_basis=256,
                 cutoff=6.0, use_layer_norm=True, use_atom_edge=True, C=256, lmax=2, **kw):
        super().__init__()
        if not (use_atom_edge and use_layer_norm):
            raise NotImplementedError("the HIP degree embedding implements use_atom_edge=True with layer norm")
        self.cutoff, self.lmax, self.avg_aggregate_num = cutoff, lmax, avg_aggregate_num
        self.number_of_basis = number_of_basis
        self.gbf_projs = nn.ModuleList([RadialProfile([number_of_basis * 3, min(number_of_basis // 2, 128),
                                                       min(number_of_basis // 2, 128), C]) for _ in range(lmax + 1)])
        self.max_num_elements = 300
        self.weight_list = nn.ParameterList()
        self.source_embedding = nn.Embedding(300, number_of_basis)
        self.target_embedding = nn.Embedding(300, number_of_basis)
        self.sph = sph_fromxyz(lmax)
        self.proj = SO3_Linear_e2former(2 * C, C, lmax=lmax)
        self._radial = RadialCache()

    def forward(self, *args, **kwargs):
        """forward(ctx: EdgeContext) -> [9, N, C] (the fused path of this package), or
        the reference's signature (e2former.py:689-753) -> node_features [N, 9, C]."""
        if len(args) == 1 and isinstance(args[0], EdgeContext) and not kwargs:
            return self.forward_fused(args[0])
        if not args and isinstance(kwargs.get("ctx"), EdgeContext):
            return self.forward_fused(kwargs["ctx"])
        return self.forward_reference(*args, **kwargs)

    def forward_reference(self, node_input, node_pos, edge_dis, atomic_numbers, edge_vec, batched_data,
                          attn_mask=None, poly_dist=None, edge_scalars=None, rbf=None, max_radius=None, **kwargs):
        """EdgeDegreeEmbeddingNetwork_higherorder.forward (e2former.py:689-753) with
        its arguments; edge_scalars must be rbf(edge_dis) and poly_dist
        polynomial(edge_dis, cutoff), both evaluated inside the kernels.  rbf
        defaults to GaussianSmearing(number_of_basis, cutoff, 2), the E2former's
        own (e2former.py:831-834), max_radius to this module's cutoff."""
        if rbf is None:
            rbf = getattr(self, "_default_rbf", None)
            if rbf is None or rbf.offset.device != edge_dis.device:
                rbf = GaussianSmearing(self.number_of_basis, cutoff=self.cutoff, basis_width_scalar=2.0)
                rbf = rbf.to(edge_dis.device)
                self._default_rbf = rbf
        rc = self.cutoff if max_radius is None else float(max_radius)
        ctx = reference_edge_context(batched_data, edge_vec, edge_dis, atomic_numbers, rbf, rc)
        if int(node_input.shape[0]) != ctx.nl.n_atoms:
            raise ValueError(f"node_input has {node_input.shape[0]} rows for {ctx.nl.n_atoms} atoms")
        return self.forward_fused(ctx).transpose(0, 1).contiguous()

    def forward_fused(self, ctx: EdgeContext):
        table = self._radial.get([p.net for p in self.gbf_projs], self.target_embedding, self.source_embedding,
                                 ctx.rbf_offset, ctx.rbf_coeff, ctx.rc, ctx.type_z, ctx.type_key, layout="degh",
                                 pairs=ctx.pairs)
        # the edge spherical harmonics ("e3nn sph") are formed inside the degree kernels
        with record_function("e3nn sph"):
            return DegreeEmbedFn.apply(ctx.dvec, ctx.dist, ctx.nl, ctx.atom_type, table,
                                       float(self.avg_aggregate_num), ctx.rc)


class E2former(nn.Module):
    """e2former.py:758-1145 on flattened atoms, with the long-range cluster
    blocks of with_cluster="node*" (e2former.py:887-929,1088-1117)."""

    def __init__(self, irreps_node_embedding="256x0e+256x1e+256x2e", num_layers=4, max_neighbors=None,
                 max_radius=6.0, basis_type="gaussiansmear", number_of_basis=256, num_attn_heads=128,
                 attn_scalar_head=8, irreps_head="2x0e+2x1e+2x2e", norm_layer="rms_norm_sh", alpha_drop=0.0,
                 tp_type="QK_alpha", attn_type="so2-first-order", atom_type_cnt=256, edge_embedtype="default",
                 ffn_type="s3", avg_degree=23.01, with_cluster=False, long_range_layers=2, long_cutoff_lower=0.1,
                 long_cutoff_upper=12, **kwargs):
        super().__init__()
        C, lmax = parse_irreps(irreps_node_embedding)
        check_supported(C, lmax, num_attn_heads, attn_scalar_head, number_of_basis, irreps_head, norm_layer,
                        tp_type, attn_type, ffn_type, basis_type, with_cluster, edge_embedtype)
        self.max_neighbors, self.max_radius, self.number_of_basis = max_neighbors, max_radius, number_of_basis
        self.num_layers, self.num_attn_heads, self.lmax = num_layers, num_attn_heads, lmax
        # "a+b": type a for the first num_layers // 2 blocks, b for the rest (e2former.py:792-795,863)
        self.attn_type = attn_type.split("+") if "+" in attn_type else [attn_type, attn_type]
        self._node_scalar_dim = C
        self.default_node_embedding = nn.Embedding(atom_type_cnt, C)
        self.heads2basis = nn.Linear(num_attn_heads, number_of_basis, bias=True)
        self.rbf = GaussianSmearing(number_of_basis, cutoff=max_radius, basis_width_scalar=2)
        self.Jd_list = nn.ParameterList([nn.Parameter(torch.from_numpy(j).float(), requires_grad=False)
                                         for j in so3.wigner_J(11)])
        self.edge_deg_embed_dense = EdgeDegreeEmbeddingNetwork_higherorder(
            irreps_node_embedding, avg_degree, number_of_basis, max_radius, C=C, lmax=lmax)
        self.blocks = nn.ModuleList([
            TransBlock(irreps_node_embedding, irreps_node_embedding, number_of_basis, num_attn_heads,
                       attn_scalar_head, irreps_head, alpha_drop, tp_type,
                       self.attn_type[0] if i < num_layers // 2 else self.attn_type[1], 256, norm_layer,
                       ffn_type, i, C=C, lmax=lmax) for i in range(num_layers)])
        ga0 = self.blocks[0].ga
        self.l3_sequential = (ga0.first_order_tp.so2_tp.l3_sequential if hasattr(ga0, "first_order_tp")
                              else [(l, 1) for l in range(lmax + 1)])
        if self.attn_type[0] == "zero-order" and "so2-first-order" in self.attn_type and num_layers > 1:
            # the node frames are sized from block 0's product (e2former.py:877-881,991-1002): with a zero-order
            # block 0 the reference's first-order blocks get the 9-row frames and fail in their forward
            raise ValueError("attn_type 'zero-order+so2-first-order' is not runnable in the reference (its "
                             "first-order blocks take the frames sized for a zero-order block 0); use "
                             "'so2-first-order+zero-order'")
        self.norm_final = EquivariantRMSNormArraySphericalHarmonicsV2_BL(lmax, C)
        self.long_cutoff_lower, self.long_cutoff_upper = long_cutoff_lower, long_cutoff_upper
        self.with_cluster = str(with_cluster)
        if "node" in self.with_cluster:
            self.pre_norm_node = EquivariantRMSNormArraySphericalHarmonicsV2_BL(lmax, C)
            self.norm_cluster = EquivariantRMSNormArraySphericalHarmonicsV2_BL(lmax, C)
            self.final_linear = SO3_Linear_e2former(2 * C, C, lmax=lmax, bias=True)
            self.rbf_long = GaussianSmearing(number_of_basis, cutoff=long_cutoff_upper, basis_width_scalar=2)
            self.long_blocks = nn.ModuleList([
                TransBlock(irreps_node_embedding, irreps_node_embedding, number_of_basis, num_attn_heads,
                           attn_scalar_head, irreps_head, alpha_drop, tp_type, "zero-order", 256, norm_layer,
                           ffn_type, i, C=C, lmax=lmax) for i in range(long_range_layers)])
            self.norm_final = EquivariantRMSNormArraySphericalHarmonicsV2_BL(lmax, C)

    @property
    def cluster(self) -> bool:
        return "node" in self.with_cluster

    def long_envelope(self):
        """(kind, lower end) of the long-range list's envelope: the bell on
        [long_cutoff_lower, long_cutoff_upper] when with_cluster names "bell",
        else the polynomial on [0, long_cutoff_upper] (e2former_wrapper.py:240)."""
        return (1, float(self.long_cutoff_lower)) if "bell" in self.with_cluster else (0, 0.0)

    def forward_flat(self, ctx: EdgeContext, sys_node_embedding: Optional[torch.Tensor] = None,
                     long_ctx: Optional[EdgeContext] = None):
        """Returns the node irreps in the m-major layout [9, N, C].  long_ctx: the
        long-range neighbour list's edge context (with_cluster only)."""
        with record_function("node_initiliation"):
            x = self.edge_deg_embed_dense(ctx)
        d = None
        for i, blk in enumerate(self.blocks):
            with record_function(f"tranblock {i}"):
                x, d = blk.forward_deferred(x, d, ctx, sys_node_embedding)
        if not self.cluster:
            return self.norm_final.add_forward(x, d)[0]
        if long_ctx is None:
            raise ValueError("cluster_neighbor_info is required when with_cluster contains 'node'.")
        x, short = self.pre_norm_node.add_forward(x, d)
        d = None
        for i, blk in enumerate(self.long_blocks):
            with record_function(f"long-tranblock {i}"):
                x, d = blk.forward_deferred(x, d, long_ctx, sys_node_embedding)
        x = self.norm_cluster.add_forward(x, d)[0]
        return self.final_linear(torch.cat([short, x], dim=-1), bf16=ctx.bf16)


def parse_irreps(s: str):
    parts = [p.strip() for p in str(s).split("+")]
    muls, ls = [], []
    for p in parts:
        mul, ir = p.split("x")
        muls.append(int(mul)); ls.append(int(ir[:-1]))
    if ls != list(range(len(ls))) or len(set(muls)) != 1:
        raise NotImplementedError(f"irreps {s!r}: expected Cx0e+Cx1e+...+Cx(l)e")
    return muls[0], ls[-1]


def check_supported(C, lmax, heads, head_dim, n_basis, irreps_head, norm_layer, tp_type, attn_type, ffn_type,
                    basis_type, with_cluster, edge_embedtype):
    hc, hl = parse_irreps(irreps_head)
    ok = (C == 256 and lmax == 2 and heads == 128 and head_dim == 8 and n_basis == 256 and hc * heads == C
          and hl == lmax and norm_layer in ("rms_norm_sh", "rms_norm_sh_BL")
          and tp_type.split("+")[0] in ("QK_alpha", "QKdot_alpha", "QKdotS_alpha")
          and all(a in ("so2-first-order", "zero-order") for a in attn_type.split("+"))
          and len(attn_type.split("+")) <= 2 and ("s3" in ffn_type or "default" in ffn_type)
          and basis_type == "gaussiansmear" and "wolayernorm" not in edge_embedtype)
    if not ok:
        raise NotImplementedError(
            "the MI355X path implements the E2Former-V2 production configuration: irreps 256x0e+256x1e+256x2e, "
            "irreps_head 2x0e+2x1e+2x2e, 128 heads, attn_scalar_head 8, 256 basis, rms_norm_sh, tp_type QK_alpha / "
            "QKdot_alpha / QKdotS_alpha (softmax, +softplus or +sigmoid weights), attn_type so2-first-order / zero-order (or 'a+b' of the "
            "two), ffn s3")
    if "node" not in str(with_cluster) and str(with_cluster) not in ("False", "false", "0", "None", "none"):
        raise ValueError("Only with_cluster='node*' is restored in this release tree. "
                         "Other cluster modes require removed modules.")
