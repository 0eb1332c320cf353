"""fp32 GEMMs of the per-node dense layers on bf16 MFMA (``e2v2_gemm_s3``).

Each fp32 operand is split exactly into three bf16 pieces (x0 = bf16(x), x1 =
bf16(x - x0), x2 = bf16(x - x0 - x1)) and a product is the sum of the six piece
products of order <= 2, accumulated in fp32 with a0 b0 kept apart from the
smaller terms: an fp32 GEMM to within a few units of fp32 rounding, at the bf16
MFMA rate.  Weights are split and packed once per weight version
(``e2v2_gemm_pack``, into the kernel's LDS image per 128-column tile and 16-k
stage); activations are split inside the kernel.

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
    """n_w fp32 weights W_w [n, k] split and packed for ``e2v2_gemm_s3``."""
    __slots__ = ("buf", "n_w", "n", "k")

    def __init__(self, buf, n_w, n, k):
        self.buf, self.n_w, self.n, self.k = buf, n_w, n, k


def supported(n: int, k: int) -> bool:
    return n > 0 and k > 0 and n % TILE_N == 0 and k % TILE_K == 0


def pack(w: torch.Tensor, transpose: bool = False) -> PackedWeight:
    """Pack w [n_w, n, k] (W_w = w[w]) or, with ``transpose``, w [n_w, k, n]
    (W_w = w[w]^T, read without a copy); a 2-D w is one weight.  fp32 on the GPU."""
    w = w.detach()
    if w.dim() == 2:
        w = w.unsqueeze(0)
    if w.dtype != torch.float32 or not w.is_cuda:
        raise ValueError("gemm.pack: fp32 weights on the GPU")
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
    nbytes = int(_lib.load().e2v2_gemm_packed_bytes(n_w, n, k))
    buf = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=w.device)
    _lib.call("e2v2_gemm_pack", _lib.vp(w.data_ptr()), _lib.i64(ld_n), _lib.i64(ld_k), _lib.i64(w.stride(0)),
              _lib.i32(n_w), _lib.i32(n), _lib.i32(k), _lib.vp(buf.data_ptr()),
              _lib.vp(torch.cuda.current_stream(w.device).cuda_stream))
    return PackedWeight(buf, n_w, n, k)


def _as3(t: torch.Tensor) -> torch.Tensor:
    return t.unsqueeze(0) if t.dim() == 2 else t


def gemm(a: torch.Tensor, pw: PackedWeight, out: torch.Tensor, widx: Optional[Sequence[int]] = None,
         bias: Optional[torch.Tensor] = None, bias_batches: int = 1, res: Optional[torch.Tensor] = None):
    """out[b] = a[b] W_{widx[b]}^T (+ bias for b < bias_batches) (+ res[b]).
    a [batch, m, k] or [m, k] fp32 (rows may be strided, k contiguous), out and
    res [batch, m, n] (res may be out)."""
    a3, o3 = _as3(a), _as3(out)
    r3 = None if res is None else _as3(res)
    batch, m, k = a3.shape
    if k != pw.k or o3.shape != (batch, m, pw.n) or a3.dtype != torch.float32 or o3.dtype != torch.float32:
        raise ValueError(f"gemm: a {tuple(a3.shape)} / out {tuple(o3.shape)} do not fit W [{pw.n}, {pw.k}]")
    if a3.stride(2) != 1 or o3.stride(2) != 1 or (r3 is not None and (r3.shape != o3.shape or r3.stride(2) != 1)):
        raise ValueError("gemm: operands need a contiguous last dimension")
    if a3.stride(1) % 4 or a3.data_ptr() % 16:
        a3 = a3.contiguous()
    widx = list(range(batch)) if widx is None else list(widx)
    if len(widx) != batch or batch > MAX_BATCH or any(not 0 <= i < pw.n_w for i in widx):
        raise ValueError(f"gemm: weight index {widx} for {pw.n_w} weights")
    if m == 0:
        return out
    g = _lib.GemmArgs()
    g.a, g.lda, g.a_bs = a3.data_ptr(), a3.stride(1), a3.stride(0)
    g.b, g.n_w = pw.buf.data_ptr(), pw.n_w
    g.c, g.ldc, g.c_bs = o3.data_ptr(), o3.stride(1), o3.stride(0)
    if r3 is not None:
        g.r, g.ldr, g.r_bs = r3.data_ptr(), r3.stride(1), r3.stride(0)
    if bias is not None:
        bias = bias.detach().reshape(-1)
        if bias.numel() != pw.n or bias.dtype != torch.float32 or not bias.is_contiguous():
            raise ValueError("gemm: bias must be a contiguous fp32 [n]")
        g.bias, g.bias_batches = bias.data_ptr(), int(bias_batches)
    g.m, g.n, g.k, g.batch = m, pw.n, pw.k, batch
    for b, i in enumerate(widx):
        g.widx[b] = int(i)
    _lib.call("e2v2_gemm_s3", _lib.C.byref(g), _lib.vp(torch.cuda.current_stream(a.device).cuda_stream))
    return out
