"""fp32 GEMMs of the per-node dense layers on bf16 MFMA (``e2v2_gemm_s3``).

Each fp32 operand is split exactly into three bf16 pieces (x0 = bf16(x), x1 =
bf16(x - x0), x2 = bf16(x - x0 - x1)) and a product is the sum of the six piece
products of order <= 2, accumulated in fp32 with a0 b0 kept apart from the
smaller terms: an fp32 GEMM to within a few units of fp32 rounding, at the bf16
MFMA rate.  Weights are split and packed once per weight version
(``e2v2_gemm_pack``, into the kernel's LDS image per 128-column tile and 16-k
stage); activations are split inside the kernel.

The bf16 mode runs the same kernels on one-piece packs (``pack(..., pieces=1)``:
the bf16 rounding of the weight alone): bf16 operands (the A operand rounded as it
is read, or read as bf16), one MFMA product, fp32 accumulation; the output can be
written as bf16 for the attention kernels that gather it.

Layers that use it (reference paths): SO3_Linear_e2former
(src/molfm/models/e2former/module_utils.py:2010-2052), FeedForwardNetwork_s3
(module_utils.py:2755-2797), forward_linear + proj_first
(wigner6j/so2_tensor_product.py:276-290, e2former.py:433), the final_linear of
SO3_Linear2Scalar_e2former (module_utils.py:2230-2233) and the gate logits of
Gate_s3 (module_utils.py:2694-2746), forward and input gradient.
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch

from . import _lib

TILE_N, TILE_K, MAX_BATCH = 128, 16, 16


class PackedWeight:
    """n_w fp32 weights W_w [n, k] split into ``pieces`` bf16 pieces (3: the exact
    split, 1: the bf16 rounding alone) and packed for ``e2v2_gemm_s3``."""
    __slots__ = ("buf", "n_w", "n", "k", "pieces")

    def __init__(self, buf, n_w, n, k, pieces=3):
        self.buf, self.n_w, self.n, self.k, self.pieces = buf, n_w, n, k, pieces


def supported(n: int, k: int) -> bool:
    return n > 0 and k > 0 and n % TILE_N == 0 and k % TILE_K == 0


def pack(w: torch.Tensor, transpose: bool = False, pieces: int = 3) -> PackedWeight:
    """Pack w [n_w, n, k] (W_w = w[w]) or, with ``transpose``, w [n_w, k, n]
    (W_w = w[w]^T, read without a copy); a 2-D w is one weight.  fp32 on the GPU
    (a bf16 weight is widened exactly).  pieces = 1 packs bf16(W) alone."""
    w = w.detach()
    if w.dim() == 2:
        w = w.unsqueeze(0)
    if w.dtype == torch.bfloat16:
        w = w.float()
    if w.dtype != torch.float32 or not w.is_cuda or pieces not in (1, 3):
        raise ValueError("gemm.pack: fp32 weights on the GPU, 1 or 3 pieces")
    w = w.contiguous()
    n_w = w.shape[0]
    if transpose:
        k, n = w.shape[1], w.shape[2]
        ld_n, ld_k = 1, n
    else:
        n, k = w.shape[1], w.shape[2]
        ld_n, ld_k = k, 1
    if not supported(n, k) or not 0 < n_w <= MAX_BATCH:
        raise ValueError(f"gemm.pack: unsupported shape n_w={n_w} n={n} k={k}")
    nbytes = int(_lib.load().e2v2_gemm_packed_bytes(n_w, n, k, pieces))
    buf = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=w.device)
    _lib.call("e2v2_gemm_pack", _lib.vp(w.data_ptr()), _lib.i64(ld_n), _lib.i64(ld_k), _lib.i64(w.stride(0)),
              _lib.i32(n_w), _lib.i32(n), _lib.i32(k), _lib.i32(pieces), _lib.vp(buf.data_ptr()),
              _lib.vp(torch.cuda.current_stream(w.device).cuda_stream))
    return PackedWeight(buf, n_w, n, k, pieces)


def _as3(t: torch.Tensor) -> torch.Tensor:
    return t.unsqueeze(0) if t.dim() == 2 else t


def _batch_view(a):
    """(base pointer, row stride, batch stride, batch, m, k, holder) of an A operand given as a
    tensor [batch, m, k] / [m, k] or as a list of same-layout 2-D tensors (batch b at base + b * bs,
    bs of either sign); holder is what must stay referenced until the launch is enqueued."""
    if isinstance(a, (list, tuple)):
        t0 = a[0]
        el = t0.element_size()
        for t in a:
            if (t.dim() != 2 or t.shape != t0.shape or t.stride() != t0.stride() or t.dtype != t0.dtype
                    or t0.dtype not in (torch.float32, torch.bfloat16)
                    or t.stride(1) != 1 or (t.stride(0) * el) % 16 or t.data_ptr() % 16):
                raise ValueError("gemm: batch matrices must share shape, dtype and a 16-byte aligned row layout")
        steps = {(a[b + 1].data_ptr() - a[b].data_ptr()) for b in range(len(a) - 1)}
        if len(steps) > 1 or any(d % el for d in steps):
            raise ValueError("gemm: batch matrices must be evenly spaced in memory")
        bs = steps.pop() // el if steps else 0
        return t0.data_ptr(), t0.stride(0), bs, len(a), t0.shape[0], t0.shape[1], a
    a3 = _as3(a)
    if a3.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("gemm: A must be fp32 or bf16")
    if a3.stride(2) != 1 or (a3.stride(1) * a3.element_size()) % 16 or a3.data_ptr() % 16:
        a3 = a3.contiguous()
    return a3.data_ptr(), a3.stride(1), a3.stride(0), a3.shape[0], a3.shape[1], a3.shape[2], a3


def _args(a, pw: PackedWeight, out: torch.Tensor, widx=None, bias=None, bias_batches: int = 1, res=None):
    """(e2v2_gemm_args, fp32 work, operand holder) of one GEMM (None for an empty one); checks
    the operands."""
    o3 = _as3(out)
    r3 = None if res is None else _as3(res)
    a_ptr, lda, a_bs, batch, m, k, holder = _batch_view(a)
    a_bf16 = (a[0] if isinstance(a, (list, tuple)) else a).dtype == torch.bfloat16
    if k != pw.k or o3.shape != (batch, m, pw.n) or o3.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"gemm: a [{batch}, {m}, {k}] / out {tuple(o3.shape)} do not fit W [{pw.n}, {pw.k}]")
    if a_bf16 and pw.pieces != 1:
        raise ValueError("gemm: a bf16 A operand needs a one-piece (bf16) packed weight")
    if r3 is not None and r3.dtype != torch.float32:
        raise ValueError("gemm: the residual is fp32")
    if o3.stride(2) != 1 or (r3 is not None and (r3.shape != o3.shape or r3.stride(2) != 1)):
        raise ValueError("gemm: operands need a contiguous last dimension")
    widx = list(range(batch)) if widx is None else list(widx)
    if len(widx) != batch or batch > MAX_BATCH or any(not 0 <= i < pw.n_w for i in widx):
        raise ValueError(f"gemm: weight index {widx} for {pw.n_w} weights")
    if m == 0:
        return None, 0.0, holder
    g = _lib.GemmArgs()
    g.pieces, g.a_bf16, g.c_bf16 = pw.pieces, int(a_bf16), int(o3.dtype == torch.bfloat16)
    g.a, g.lda, g.a_bs = a_ptr, lda, a_bs
    g.b, g.n_w = pw.buf.data_ptr(), pw.n_w
    g.c, g.ldc, g.c_bs = o3.data_ptr(), o3.stride(1), o3.stride(0)
    if r3 is not None:
        g.r, g.ldr, g.r_bs = r3.data_ptr(), r3.stride(1), r3.stride(0)
    if bias is not None:
        bias = bias.detach()
        per_batch = bias.dim() == 2
        if (bias.shape[-1] != pw.n or bias.dtype != torch.float32 or not bias.is_contiguous()
                or (per_batch and bias.shape[0] < min(bias_batches, batch))):
            raise ValueError("gemm: bias must be a contiguous fp32 [n] or [batch, n]")
        g.bias, g.bias_bs, g.bias_batches = bias.data_ptr(), (pw.n if per_batch else 0), int(bias_batches)
    g.m, g.n, g.k, g.batch = m, pw.n, pw.k, batch
    for b, i in enumerate(widx):
        g.widx[b] = int(i)
    return g, 2.0 * batch * m * pw.n * pw.k, holder


def gemm(a, pw: PackedWeight, out: torch.Tensor, widx: Optional[Sequence[int]] = None,
         bias: Optional[torch.Tensor] = None, bias_batches: int = 1, res: Optional[torch.Tensor] = None,
         gate=None):
    """out[b] = a[b] W_{widx[b]}^T (+ bias for b < bias_batches) (+ res[b]).
    a [batch, m, k] or [m, k] fp32 (rows may be strided, k contiguous), or a list of
    same-layout [m, k] matrices; out and res [batch, m, n] (res may be out); bias [n]
    (shared) or [batch, n] (one per batch).  gate = (s, k1, k2): Gate_s3's activation
    applied to A as it is read (``e2v2_gemm_s3_gated``): batch 0 takes silu(s[:, :k]) k1,
    batch b >= 1 takes a[b] * sigmoid(s[:, k widx[b]:k (widx[b] + 1)]) k2."""
    g, work, keep = _args(a, pw, out, widx, bias, bias_batches, res)   # keep: referenced until the launch
    if g is None:
        return out
    st = _lib.vp(torch.cuda.current_stream(out.device).cuda_stream)
    entry = "e2v2_gemm_s3" if gate is None else "e2v2_gemm_s3_gated"
    if gate is not None:
        sg, k1, k2 = gate
        if sg.dtype != torch.float32 or sg.dim() != 2 or sg.stride(1) != 1 or sg.shape[0] != _as3(out).shape[1]:
            raise ValueError("gemm: gate logits must be fp32 [m, ld] with contiguous rows")
        # the logit columns read (k of them per weight index) must lie inside the view, not merely inside
        # its row stride: a narrowed view s[:, :w] of a wider tensor would read past its own columns
        nb = _as3(out).shape[0]
        top = max(int(g.widx[b]) for b in range(1, nb)) + 1 if nb > 1 else 0
        if pw.k * max(top, 1) > sg.shape[1]:
            raise ValueError(f"gemm: gate logits of {sg.shape[1]} columns, the batches read {pw.k * max(top, 1)}")
        _lib.call("e2v2_gemm_s3_gated", _lib.C.byref(g), _lib.vp(sg.data_ptr()), _lib.i64(sg.stride(0)),
                  _lib.f32(k1), _lib.f32(k2), st)
    else:
        _lib.call("e2v2_gemm_s3", _lib.C.byref(g), st)
    del keep
    if _lib._timer is not None:
        _lib._timer.add_work(entry, work)
    return out


MAX_GROUPS = 4


def gemm_grouped(problems):
    """Up to four independent GEMMs in one launch (``e2v2_gemm_s3_grouped``):
    ``problems`` is a sequence of dicts with the arguments of :func:`gemm`
    (a, pw, out and optionally widx, bias, bias_batches, res).  Put the problems
    with the longest k first: their tiles are dispatched first."""
    if not 0 < len(problems) <= MAX_GROUPS:
        raise ValueError(f"gemm_grouped: {len(problems)} problems (1 .. {MAX_GROUPS})")
    keep = []   # operands (and any contiguous copies) referenced until the launch is enqueued
    arr = (_lib.GemmArgs * MAX_GROUPS)()
    n, work, dev = 0, 0.0, problems[0]["out"].device
    for p in problems:
        g, w, holder = _args(p["a"], p["pw"], p["out"], p.get("widx"), p.get("bias"), p.get("bias_batches", 1),
                             p.get("res"))
        keep.append(holder)
        if g is not None:
            arr[n] = g
            n += 1
            work += w
    if n:
        _lib.call("e2v2_gemm_s3_grouped", arr, _lib.i32(n), _lib.vp(torch.cuda.current_stream(dev).cuda_stream))
        if _lib._timer is not None:
            _lib._timer.add_work("e2v2_gemm_s3_grouped", work)
    del keep


# ---------------------------------------------------------------------------------------------
# Q/K projection of SO3_Linear2Scalar_e2former with its m-contraction (e2v2_qk_proj_fwd_s3 /
# e2v2_qk_proj_bwd_s3).  The stacked weight W [3, 4 hid, C] has the columns
# [q_a | q_b | k_a | k_b] (hid each); pair p < 2 hid is (q_a, q_b) column p for p < hid, else
# (k_a, k_b) column p - hid.

def pair_col(p: int, ab: int, hid: int) -> int:
    """Column of W holding the a- (ab = 0) or b-side (ab = 1) of pair p."""
    if p < hid:
        return hid + p if ab else p
    return 2 * hid + p if ab else hid + p


def qk_orders(hid: int):
    """(forward, backward) column orders: the forward's packed column i is W column
    fwd[i] (128-column tile t = a-sides of pairs 64 t .. +63, then their b-sides);
    the kept y and the backward's K index s hold W column bwd[s]
    (s = 16 (p // 8) + 8 ab + p % 8)."""
    fwd = [pair_col(64 * (i // 128) + (i % 128) % 64, (i % 128) // 64, hid) for i in range(4 * hid)]
    bwd = [0] * (4 * hid)
    for p in range(2 * hid):
        for ab in (0, 1):
            bwd[16 * (p // 8) + 8 * ab + p % 8] = pair_col(p, ab, hid)
    return fwd, bwd


class QKPacks:
    """Packed operands of the split Q/K projection: ``fwd`` (W in the forward order),
    ``bias`` (in the same order), ``bwd`` ([W rows in the backward order ; Wv]^T per
    l), hid, C and Cv."""
    __slots__ = ("fwd", "bias", "bwd", "hid", "c", "cv")


def qk_supported(hid: int, c: int, cv: int) -> bool:
    return hid > 0 and hid % 64 == 0 and c > 0 and c % TILE_N == 0 and cv > 0 and cv % TILE_K == 0


def pack_qk(W: torch.Tensor, bias: Optional[torch.Tensor], Wv: torch.Tensor, pieces: int = 3) -> QKPacks:
    """W [3, 4 hid, C] (stacked query and key weights), bias [4 hid] or None, Wv
    [3, Cv, C] (the value projection, whose input gradient the backward adds)."""
    W = W.detach().float()
    Wv = Wv.detach().float()
    hid, c, cv = W.shape[1] // 4, W.shape[2], Wv.shape[1]
    if not qk_supported(hid, c, cv) or W.shape[0] != 3 or Wv.shape[0] != 3 or Wv.shape[2] != c:
        raise ValueError(f"pack_qk: unsupported shapes W {tuple(W.shape)} Wv {tuple(Wv.shape)}")
    fwd, bwd = qk_orders(hid)
    fi = torch.as_tensor(fwd, device=W.device)
    bi = torch.as_tensor(bwd, device=W.device)
    P = QKPacks()
    P.fwd = pack(W[:, fi, :].contiguous(), pieces=pieces)
    P.bias = None if bias is None else bias.detach().float()[fi].contiguous()
    P.bwd = pack(torch.cat([W[:, bi, :], Wv], dim=1).contiguous(), transpose=True, pieces=pieces)
    P.hid, P.c, P.cv = hid, c, cv
    return P


def qk_forward(x: torch.Tensor, P: QKPacks, y_bf16: Optional[bool] = None):
    """(hq, hk [N, 3 hid], y [9, N, 4 hid] in the backward order) from x [9, N, C];
    y_bf16: y kept as bf16 for the backward (default: with one-piece packs, the
    bf16 mode)."""
    x = x.contiguous()
    _, n, c = x.shape
    if y_bf16 is None:
        y_bf16 = P.fwd.pieces == 1
    if y_bf16 and P.fwd.pieces != 1:
        raise ValueError("qk_forward: a bf16 y needs one-piece packs")
    y = x.new_empty(9, n, 4 * P.hid, dtype=torch.bfloat16 if y_bf16 else torch.float32)
    hq = x.new_empty(n, 3 * P.hid)
    hk = x.new_empty(n, 3 * P.hid)
    st = _lib.vp(torch.cuda.current_stream(x.device).cuda_stream)
    _lib.call("e2v2_qk_proj_fwd_s3", _lib.vp(x.data_ptr()), _lib.vp(P.fwd.buf.data_ptr()),
              _lib.vp(0 if P.bias is None else P.bias.data_ptr()), _lib.vp(y.data_ptr()), _lib.vp(hq.data_ptr()),
              _lib.vp(hk.data_ptr()), _lib.i32(n), _lib.i32(P.hid), _lib.i32(c), _lib.i32(P.fwd.pieces),
              _lib.i32(int(y_bf16)), st)
    return hq, hk, y


def qk_backward(y: torch.Tensor, ghq: torch.Tensor, ghk: torch.Tensor, gv: Optional[torch.Tensor], P: QKPacks):
    """gx [9, N, C] (with gv [9, N, Cv] W_v added when gv is given); y fp32, or bf16
    from qk_forward(y_bf16=True)."""
    n = y.shape[1]
    gx = y.new_empty(9, n, P.c, dtype=torch.float32)
    y_bf16 = y.dtype == torch.bfloat16
    ghq, ghk = ghq.contiguous(), ghk.contiguous()
    gv = None if gv is None else gv.float().contiguous()
    st = _lib.vp(torch.cuda.current_stream(y.device).cuda_stream)
    _lib.call("e2v2_qk_proj_bwd_s3", _lib.vp(y.data_ptr()), _lib.vp(ghq.data_ptr()), _lib.vp(ghk.data_ptr()),
              _lib.vp(P.bwd.buf.data_ptr()), _lib.vp(0 if gv is None else gv.data_ptr()), _lib.vp(gx.data_ptr()),
              _lib.i32(n), _lib.i32(P.hid), _lib.i32(P.c), _lib.i32(P.cv), _lib.i32(P.bwd.pieces),
              _lib.i32(int(y_bf16)), st)
    return gx
