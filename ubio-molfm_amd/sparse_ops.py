"""Op-level drop-ins for the reference's sparse edge operators
(src/molfm/models/e2former/triton_dr/), with the reference's names,
arguments, metadata tuples, output dtypes and errors:

* ``prepare_sparse_qk_edge_index_metadata`` / ``sparse_qk_edge_index_triton``
  (triton_sparse_qk_autograd.py:601-652, 839-871);
* ``prepare_sparse_alpha_sum_edge_index_metadata`` /
  ``sparse_alpha_sum_edge_index_triton`` (sparse_alpha_sum_edge_index_autograd.py:102-213);
* ``prepare_sparse_v_agg_edge_index_metadata`` /
  ``sparse_v_agg_edge_index_triton_cblocked`` (sparse_v_agg_lastdim_autograd.py:235-241;
  sparse_v_agg_edge_index_cblocked_bench.py:243-449);
* ``prepare_edge_degree_outer_metadata`` / ``edge_degree_outer_triton``
  (edge_degree_outer_autograd.py:299-375).

Every kernel is a HIP segment kernel of libe2v2.so (csrc/sparse.hip, the
metadata builder in csrc/nbr.hip); there is no CPU path.  Arithmetic is fp32;
outputs take the dtype the reference gives them.  Each backward is written with
the same autograd Functions as the forwards (the gradient of a segment dot is a
segment reduce over the same or the transposed layout and vice versa; the alpha
sum and the row gather are each other's gradients; the degree outer product and
its gradient close the same way), so second- and higher-order gradients follow
the reference's ``*_Backward_Fn`` classes without separate kernels.

The model's own attention and degree-embedding paths run fused
(ops.AttentionFn / ops.DegreeEmbedFn) in evaluation mode; in training mode they
are composed from these functions (``second_order``) so that forces can be
differentiated again."""
from __future__ import annotations

import ctypes as C
from typing import Optional, Sequence

import torch

from . import _lib

_I32 = torch.int32


def _vp(t: Optional[torch.Tensor]):
    return None if t is None or t.numel() == 0 else _lib.vp(t.data_ptr())


def _stream(dev):
    return _lib.vp(torch.cuda.current_stream(dev).cuda_stream)


def _strides(t: torch.Tensor):
    return (C.c_int64 * 3)(*(list(t.stride()) + [0, 0, 0])[:3])


def _need_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("the sparse edge ops run on the GPU only (HIP library, no CPU path): "
                               f"got a tensor on {t.device}")


def _i32(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous().to(_I32)


# ---------------------------------------------------------------------------
# segment metadata (triton_sparse_qk_autograd.py:601-652)
# ---------------------------------------------------------------------------
def _prepare_segment_metadata(row_index, col_index, num_rows):
    """(row_ptr [num_rows+1], col_index sorted by row, alpha_index = the stable
    order of the edges by row) -- triton_sparse_qk_autograd.py:615-632."""
    _need_gpu(row_index, col_index)
    num_rows = int(num_rows)
    dev = row_index.device
    row, other = _i32(row_index), _i32(col_index)
    E = row.numel()
    if other.numel() != E:
        raise ValueError(f"row and column index lengths differ ({E} vs {other.numel()})")
    row_ptr = torch.empty(num_rows + 1, dtype=_I32, device=dev)
    cnt = torch.empty(max(num_rows, 1), dtype=_I32, device=dev)
    stats = torch.empty(3, dtype=_I32, device=dev)
    st = _stream(dev)
    _lib.call("e2v2_segment_metadata", _vp(row), _vp(other), _lib.i64(E), _lib.i32(num_rows), _vp(row_ptr), None,
              None, _vp(cnt), None, _vp(stats), _lib.i32(0), st)
    if E == 0:
        empty = torch.empty(0, dtype=_I32, device=dev)
        return row_ptr, empty, empty
    bad = int(stats[2].item())  # one host read, like the reference's sortedness check
    if bad:
        raise RuntimeError(f"segment metadata: {bad} row indices outside [0, {num_rows})")
    col = torch.empty(E, dtype=_I32, device=dev)
    perm = torch.empty(E, dtype=_I32, device=dev)
    tkey = torch.empty(E, dtype=torch.int64, device=dev)
    _lib.call("e2v2_segment_metadata", _vp(row), _vp(other), _lib.i64(E), _lib.i32(num_rows), _vp(row_ptr),
              _vp(col), _vp(perm), _vp(cnt), _vp(tkey), _vp(stats), _lib.i32(1), st)
    return row_ptr, col, perm


def prepare_sparse_qk_edge_index_metadata(query_index, neighbor_index, num_queries, num_keys):
    """triton_sparse_qk_autograd.py:635-652: (q_row_ptr, q_col_index,
    q_alpha_index, key_row_ptr, key_col_index, key_alpha_index), int32."""
    q = _prepare_segment_metadata(query_index, neighbor_index, num_queries)
    k = _prepare_segment_metadata(neighbor_index, query_index, num_keys)
    return (*q, *k)


def prepare_sparse_alpha_sum_edge_index_metadata(query_index, num_queries):
    """sparse_alpha_sum_edge_index_autograd.py:102-109: (row_ptr, alpha_index)."""
    row_ptr, _, alpha_index = _prepare_segment_metadata(query_index, query_index, num_queries)
    return row_ptr, alpha_index


def prepare_sparse_v_agg_edge_index_metadata(query_index, value_index, num_queries, num_values):
    """sparse_v_agg_lastdim_autograd.py:235-241 (the QK metadata of the pair)."""
    return prepare_sparse_qk_edge_index_metadata(query_index, value_index, num_queries, num_values)


def prepare_edge_degree_outer_metadata(query_index, num_queries):
    """edge_degree_outer_autograd.py:336-345: the QK metadata of (query, edge id)."""
    q = _i32(query_index)
    eid = torch.arange(q.numel(), dtype=_I32, device=q.device)
    return prepare_sparse_qk_edge_index_metadata(q, eid, num_queries, eid.numel())


# ---------------------------------------------------------------------------
# segment layouts
# ---------------------------------------------------------------------------
class _Layouts:
    """The two segment layouts of one edge list: side 0 = rows by query (partner
    rows index the key operand), side 1 = rows by key.  Holds the metadata
    tensors for the lifetime of the autograd graph."""

    def __init__(self, metadata: Sequence[torch.Tensor], n_q: int, n_k: int, n_e: int):
        md = [_i32(t) for t in metadata]
        _need_gpu(*md)
        self.md = md
        self.n = (int(n_q), int(n_k))
        self.n_e = int(n_e)
        self.segs = []
        for side in (0, 1):
            ptr, col, alpha = md[3 * side: 3 * side + 3]
            if ptr.numel() != self.n[side] + 1:
                raise ValueError(f"metadata row_ptr of length {ptr.numel()} for {self.n[side]} rows")
            if col.numel() != alpha.numel():
                raise ValueError("metadata col_index and alpha_index lengths differ")
            self.segs.append(_lib.Segments(_vp(ptr), _vp(col), _vp(alpha), self.n[side], self.n[1 - side],
                                           col.numel(), self.n_e))

    def rows(self, side: int) -> int:
        return self.n[side]


class _AlphaLayout:
    """Rows by query with no partner operand (the alpha sum and the degree outer product)."""

    def __init__(self, row_ptr, alpha_index, query_index, n_rows: int, n_e: int):
        self.row_ptr, self.alpha_index, self.query_index = _i32(row_ptr), _i32(alpha_index), _i32(query_index)
        _need_gpu(self.row_ptr, self.alpha_index, self.query_index)
        self.n_rows, self.n_e = int(n_rows), int(n_e)
        if self.row_ptr.numel() != self.n_rows + 1:
            raise ValueError(f"metadata row_ptr of length {self.row_ptr.numel()} for {self.n_rows} rows")
        if self.query_index.numel() != self.n_e:
            raise ValueError(f"query_index has {self.query_index.numel()} entries for {self.n_e} edges")
        self.seg = _lib.Segments(_vp(self.row_ptr), None, _vp(self.alpha_index), self.n_rows, 0,
                                 self.alpha_index.numel(), self.n_e)


def _logical(t: torch.Tensor, cblocked: bool) -> torch.Tensor:
    """[rows, H, D] view: the [M, C, H] operands of the value aggregation are viewed [M, H, C]."""
    return t.permute(0, 2, 1) if cblocked else t


def _seg_dot(L: _Layouts, side: int, A, B, cblocked: bool):
    A, B = A.float(), B.float()
    a, b = _logical(A, cblocked), _logical(B, cblocked)
    H, D = a.shape[1], a.shape[2]
    if a.shape[0] != L.rows(side) or b.shape[0] != L.rows(1 - side) or tuple(b.shape[1:]) != (H, D):
        raise AssertionError(f"segment dot operands {tuple(A.shape)} x {tuple(B.shape)} do not match the layout "
                             f"({L.rows(side)} x {L.rows(1 - side)} rows)")
    out = torch.zeros(L.n_e, H, dtype=torch.float32, device=A.device)
    if L.n_e == 0 or a.shape[0] == 0:
        return out
    os_ = (C.c_int64 * 3)(*out.stride(), 0)
    _lib.call("e2v2_seg_dot", C.byref(L.segs[side]), _vp(a), _strides(a), _vp(b), _strides(b), _lib.i32(H),
              _lib.i32(D), _vp(out), os_, _stream(A.device))
    return out


def _seg_reduce(L: _Layouts, side: int, W, X, cblocked: bool):
    W, X = W.float(), X.float()
    x = _logical(X, cblocked)
    H, D = x.shape[1], x.shape[2]
    if x.shape[0] != L.rows(1 - side) or tuple(W.shape) != (L.n_e, H):
        raise AssertionError(f"segment reduce operands {tuple(W.shape)}, {tuple(X.shape)} do not match the layout")
    shape = (L.rows(side), D, H) if cblocked else (L.rows(side), H, D)
    out = torch.empty(shape, dtype=torch.float32, device=X.device)
    if out.numel() == 0:
        return out
    o = _logical(out, cblocked)
    _lib.call("e2v2_seg_reduce", C.byref(L.segs[side]), _vp(W), _strides(W), _vp(x), _strides(x), _lib.i32(H),
              _lib.i32(D), _vp(out), _strides(o), _stream(X.device))
    return out


class _SegDotFn(torch.autograd.Function):
    """out[e, h] = <A[row_e, h, :], B[col_e, h, :]> over the layout's side."""

    @staticmethod
    def forward(ctx, A, B, L, side, cblocked):
        ctx.save_for_backward(A, B)
        ctx.L, ctx.side, ctx.cblocked = L, side, cblocked
        return _seg_dot(L, side, A, B, cblocked)

    @staticmethod
    def backward(ctx, g):
        A, B = ctx.saved_tensors
        L, side, cb = ctx.L, ctx.side, ctx.cblocked
        dA = _SegReduceFn.apply(g, B, L, side, cb) if ctx.needs_input_grad[0] else None
        dB = _SegReduceFn.apply(g, A, L, 1 - side, cb) if ctx.needs_input_grad[1] else None
        return dA, dB, None, None, None


class _SegReduceFn(torch.autograd.Function):
    """out[r, h, d] = sum over the slots of row r of W[e, h] X[col, h, d]."""

    @staticmethod
    def forward(ctx, W, X, L, side, cblocked):
        ctx.save_for_backward(W, X)
        ctx.L, ctx.side, ctx.cblocked = L, side, cblocked
        return _seg_reduce(L, side, W, X, cblocked)

    @staticmethod
    def backward(ctx, g):
        W, X = ctx.saved_tensors
        L, side, cb = ctx.L, ctx.side, ctx.cblocked
        dW = _SegDotFn.apply(g, X, L, side, cb) if ctx.needs_input_grad[0] else None
        dX = _SegReduceFn.apply(W, g, L, 1 - side, cb) if ctx.needs_input_grad[1] else None
        return dW, dX, None, None, None


def _check_metadata6(metadata, name):
    if len(metadata) != 6:
        raise ValueError(f"metadata must be a 6-tuple from {name}")


# ---------------------------------------------------------------------------
# sparse_qk_edge_index_triton (triton_sparse_qk_autograd.py:839-871)
# ---------------------------------------------------------------------------
def sparse_qk_edge_index_triton(query, key, query_index, neighbor_index, metadata=None):
    """query [N, H, D], key [M, H, D] -> out [E, H] fp32,
    out[e, h] = dot(query[query_index[e], h], key[neighbor_index[e], h])."""
    if query.ndim != 3 or key.ndim != 3 or tuple(query.shape[1:]) != tuple(key.shape[1:]):
        raise AssertionError(f"query {tuple(query.shape)} and key {tuple(key.shape)} must be [N, H, D] and [M, H, D]")
    _need_gpu(query, key, query_index, neighbor_index)
    if metadata is None:
        metadata = prepare_sparse_qk_edge_index_metadata(query_index, neighbor_index, query.shape[0], key.shape[0])
    else:
        _check_metadata6(metadata, "prepare_sparse_qk_edge_index_metadata")
    E = query_index.numel()
    if E == 0:
        return torch.empty((0, query.shape[1]), device=query.device, dtype=torch.float32)
    L = _Layouts(metadata, query.shape[0], key.shape[0], E)
    if torch.is_grad_enabled() and (query.requires_grad or key.requires_grad):
        return _SegDotFn.apply(query.float(), key.float(), L, 0, False)
    return _seg_dot(L, 0, query, key, False)


sparse_qk_edge_index = sparse_qk_edge_index_triton


# ---------------------------------------------------------------------------
# sparse_v_agg_edge_index_triton_cblocked (sparse_v_agg_edge_index_cblocked_bench.py:243-449)
# ---------------------------------------------------------------------------
def sparse_v_agg_edge_index_triton_cblocked(value, alpha, query_index, value_index, num_queries, metadata=None):
    """value [M, C, H], alpha [E, H] -> out [N, C, H] in value's dtype,
    out[query_index[e], c, h] += alpha[e, h] * value[value_index[e], c, h]."""
    if value.ndim != 3:
        raise ValueError("value must be [M, C, H]")
    if alpha.ndim != 2:
        raise ValueError("alpha must be [E, H]")
    _need_gpu(value, alpha, query_index, value_index)
    if metadata is None:
        metadata = prepare_sparse_v_agg_edge_index_metadata(query_index, value_index, num_queries, value.shape[0])
    elif len(metadata) != 6:
        raise ValueError("metadata must be a 6-tuple from prepare_sparse_v_agg_edge_index_metadata")
    n_rows = metadata[0].numel() - 1
    L = _Layouts(metadata, n_rows, value.shape[0], alpha.shape[0])
    return _SegReduceFn.apply(alpha.float(), value.float(), L, 0, True).to(value.dtype)


sparse_v_agg_edge_index_cblocked = sparse_v_agg_edge_index_triton_cblocked


# ---------------------------------------------------------------------------
# sparse_alpha_sum_edge_index_triton (sparse_alpha_sum_edge_index_autograd.py:102-213)
# ---------------------------------------------------------------------------
def _alpha_sum(A: _AlphaLayout, alpha):
    alpha = alpha.float()
    H = alpha.shape[1]
    out = torch.empty(A.n_rows, H, dtype=torch.float32, device=alpha.device)
    if out.numel() == 0:
        return out
    ws = (C.c_int64 * 2)(*alpha.stride())
    os_ = (C.c_int64 * 3)(out.stride(0), out.stride(1), 0)
    _lib.call("e2v2_seg_reduce", C.byref(A.seg), _vp(alpha), ws, None, None, _lib.i32(H), _lib.i32(1), _vp(out),
              os_, _stream(alpha.device))
    return out


def _gather_rows(A: _AlphaLayout, x):
    x = x.float().contiguous()
    out = torch.empty(A.n_e, x.shape[1], dtype=torch.float32, device=x.device)
    if out.numel() == 0:
        return out
    _lib.call("e2v2_gather_rows", _vp(x), _lib.i64(x.shape[0]), _vp(A.query_index), _lib.i64(A.n_e),
              _lib.i32(x.shape[1]), _vp(out), _stream(x.device))
    return out


class _AlphaSumFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, alpha, A):
        ctx.A = A
        return _alpha_sum(A, alpha)

    @staticmethod
    def backward(ctx, g):
        return _GatherRowsFn.apply(g, ctx.A), None


class _GatherRowsFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, A):
        ctx.A = A
        return _gather_rows(A, x)

    @staticmethod
    def backward(ctx, g):
        return _AlphaSumFn.apply(g, ctx.A), None


def sparse_alpha_sum_edge_index_triton(alpha, query_index, num_queries, metadata=None):
    """alpha [E, H] -> out [num_queries, H] in alpha's dtype, out[q] = sum of alpha over the edges of q."""
    _need_gpu(alpha, query_index)
    if alpha.ndim != 2:
        raise ValueError(f"alpha {tuple(alpha.shape)} must be [E, H]")
    if metadata is None:
        metadata = prepare_sparse_alpha_sum_edge_index_metadata(query_index, num_queries)
    row_ptr, alpha_index = metadata
    A = _AlphaLayout(row_ptr, alpha_index, query_index, num_queries, alpha.shape[0])
    if torch.is_grad_enabled() and alpha.requires_grad:
        return _AlphaSumFn.apply(alpha.float(), A).to(alpha.dtype)
    return _alpha_sum(A, alpha).to(alpha.dtype)


sparse_alpha_sum_edge_index = sparse_alpha_sum_edge_index_triton


def sparse_gather_edge_index(x, index, num_rows, metadata):
    """x [num_rows, F] -> out [E, F], out[e] = x[index[e]], whose gradient sums
    the edges of each row by the segments metadata = (row_ptr, edge ids in
    segment order) of index (e2v2_gather_rows forward, e2v2_seg_reduce backward,
    each the other's gradient to any order): the per-edge gathers of the
    RadialProfile input (e2former.py:258-266, the tgt[z_i] and src[z_j] blocks)
    without torch's sort-based index backward."""
    _need_gpu(x, index)
    if x.ndim != 2 or x.shape[0] != num_rows:
        raise ValueError(f"x {tuple(x.shape)} must be [{num_rows}, F]")
    row_ptr, alpha_index = metadata
    A = _AlphaLayout(row_ptr, alpha_index, index, num_rows, index.numel())
    if torch.is_grad_enabled() and x.requires_grad:
        return _GatherRowsFn.apply(x.float(), A).to(x.dtype)
    return _gather_rows(A, x).to(x.dtype)


# ---------------------------------------------------------------------------
# edge_degree_outer_triton (edge_degree_outer_autograd.py:299-375)
# ---------------------------------------------------------------------------
def _outer(A: _AlphaLayout, sh, fea):
    sh, fea = sh.float().contiguous(), fea.float().contiguous()
    Lh, H = sh.shape[1], fea.shape[1]
    out = torch.empty(A.n_rows, Lh, H, dtype=torch.float32, device=sh.device)
    if out.numel() == 0:
        return out
    _lib.call("e2v2_outer_reduce", C.byref(A.seg), _vp(sh), _vp(fea), _lib.i32(Lh), _lib.i32(H), _vp(out),
              _stream(sh.device))
    return out


def _outer_bwd(A: _AlphaLayout, g, sh, fea):
    """(dsh[e, l] = sum_h g[q_e, l, h] fea[e, h], dfea[e, h] = sum_l g[q_e, l, h] sh[e, l])."""
    g, sh, fea = g.float().contiguous(), sh.float().contiguous(), fea.float().contiguous()
    E, Lh, H = A.n_e, sh.shape[1], fea.shape[1]
    dsh = torch.empty(E, Lh, dtype=torch.float32, device=g.device)
    dfea = torch.empty(E, H, dtype=torch.float32, device=g.device)
    if E > 0:
        _lib.call("e2v2_outer_bwd", _vp(g), _lib.i32(A.n_rows), _vp(sh), _vp(fea), _vp(A.query_index),
                  _lib.i64(E), _lib.i32(Lh), _lib.i32(H), _vp(dsh), _vp(dfea), _stream(g.device))
    return dsh, dfea


class _OuterFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, sh, fea, A):
        ctx.save_for_backward(sh, fea)
        ctx.A = A
        return _outer(A, sh, fea)

    @staticmethod
    def backward(ctx, g):
        sh, fea = ctx.saved_tensors
        d_sh, d_fea = _OuterBwdFn.apply(g, sh, fea, ctx.A)
        return d_sh, d_fea, None


class _OuterBwdFn(torch.autograd.Function):
    """(dsh, dfea) of the outer product for the output gradient g."""

    @staticmethod
    def forward(ctx, g, sh, fea, A):
        ctx.save_for_backward(g, sh, fea)
        ctx.A = A
        return _outer_bwd(A, g, sh, fea)

    @staticmethod
    def backward(ctx, gg_dsh, gg_dfea):
        g, sh, fea = ctx.saved_tensors
        A = ctx.A
        if gg_dsh is None:
            gg_dsh = torch.zeros_like(sh)
        if gg_dfea is None:
            gg_dfea = torch.zeros_like(fea)
        d_g = None
        if ctx.needs_input_grad[0]:
            d_g = _OuterFn.apply(gg_dsh, fea, A) + _OuterFn.apply(sh, gg_dfea, A)
        d_sh = d_fea = None
        if ctx.needs_input_grad[1] or ctx.needs_input_grad[2]:
            # d sh[e, l] = sum_h gg_dfea[e, h] g[q_e, l, h]; d fea[e, h] = sum_l gg_dsh[e, l] g[q_e, l, h]
            d_sh, d_fea = _OuterBwdFn.apply(g, gg_dsh, gg_dfea, A)
        return d_g, d_sh, d_fea, None


def edge_degree_outer_triton(edge_sh, edge_fea, query_index, num_queries, metadata=None):
    """edge_sh [E, L], edge_fea [E, H] -> out [num_queries, L, H] in edge_fea's dtype,
    out[n, l, h] = sum over the edges e of n of edge_sh[e, l] edge_fea[e, h]."""
    _need_gpu(edge_sh, edge_fea, query_index)
    if edge_sh.ndim != 2 or edge_fea.ndim != 2 or edge_sh.shape[0] != edge_fea.shape[0]:
        raise ValueError(f"edge_sh {tuple(edge_sh.shape)} and edge_fea {tuple(edge_fea.shape)} must be [E, L], [E, H]")
    q = _i32(query_index)
    if metadata is None:
        q_row_ptr, _, q_alpha_index, _, _, _ = prepare_edge_degree_outer_metadata(q, num_queries)
    elif isinstance(metadata, (tuple, list)):
        if len(metadata) == 6:
            q_row_ptr, _, q_alpha_index, _, _, _ = metadata
        else:
            raise ValueError("metadata must be a 6-tuple")
    else:
        raise ValueError("metadata must be a tuple/list")
    A = _AlphaLayout(q_row_ptr, q_alpha_index, q, num_queries, edge_sh.shape[0])
    return _OuterFn.apply(edge_sh.float(), edge_fea.float(), A).to(edge_fea.dtype)


edge_degree_outer = edge_degree_outer_triton
