"""Edge-chunked CPU restatements of the reference's sparse edge ops (test
infrastructure / CPU baseline only).

Same results as the reference's torch fallbacks, without materialising the
per-edge gathers for all edges at once (at 10k atoms the value gather alone is
E x 58 x 128 floats = 25 GB):

* ``sparse_qk``: out[e, h] = sum_d q[i_e, h, d] k[j_e, h, d]
  (semantics of ``sparse_qk_edge_index_triton``,
  triton_dr/triton_sparse_qk_autograd.py:839-871; fallback e2former.py:320-325);
* ``sparse_v_agg``: out[i, c, h] = sum_{e: i_e = i} a[e, h] v[j_e, c, h]
  (semantics of ``sparse_v_agg_edge_index_triton_cblocked``,
  triton_dr/sparse_v_agg_edge_index_cblocked_bench.py:428-449; fallback
  e2former.py:393-407).

Backward passes recompute the gathers chunk by chunk (first order only).

``segment_metadata`` / ``qk_metadata``: the CSR metadata of
``_prepare_segment_metadata`` / ``prepare_sparse_qk_edge_index_metadata``
(triton_dr/triton_sparse_qk_autograd.py:607-652) in numpy: row_ptr from a
bincount and cumulative sum, alpha_index the stable argsort of the row index,
col_index permuted by it.  Pinned by a per-row brute-force listing.
"""
from __future__ import annotations

import numpy as np
import torch

CHUNK = 1 << 15


class _SparseQK(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, qi, nj):
        out = torch.empty(qi.shape[0], q.shape[1], dtype=q.dtype)
        for s in range(0, qi.shape[0], CHUNK):
            sl = slice(s, s + CHUNK)
            out[sl] = (q[qi[sl]] * k[nj[sl]]).sum(-1)
        ctx.save_for_backward(q, k, qi, nj)
        return out

    @staticmethod
    def backward(ctx, g):
        q, k, qi, nj = ctx.saved_tensors
        dq, dk = torch.zeros_like(q), torch.zeros_like(k)
        for s in range(0, qi.shape[0], CHUNK):
            sl = slice(s, s + CHUNK)
            gs = g[sl].unsqueeze(-1)
            dq.index_add_(0, qi[sl], gs * k[nj[sl]])
            dk.index_add_(0, nj[sl], gs * q[qi[sl]])
        return dq, dk, None, None


class _SparseVAgg(torch.autograd.Function):
    @staticmethod
    def forward(ctx, v, a, qi, nj, n_rows):
        out = torch.zeros(n_rows, v.shape[1], v.shape[2], dtype=v.dtype)
        for s in range(0, qi.shape[0], CHUNK):
            sl = slice(s, s + CHUNK)
            out.index_add_(0, qi[sl], v[nj[sl]] * a[sl].unsqueeze(1))
        ctx.save_for_backward(v, a, qi, nj)
        return out

    @staticmethod
    def backward(ctx, g):
        v, a, qi, nj = ctx.saved_tensors
        dv, da = torch.zeros_like(v), torch.empty_like(a)
        for s in range(0, qi.shape[0], CHUNK):
            sl = slice(s, s + CHUNK)
            gs = g[qi[sl]]
            da[sl] = (gs * v[nj[sl]]).sum(1)
            dv.index_add_(0, nj[sl], gs * a[sl].unsqueeze(1))
        return dv, da, None, None, None


def sparse_qk(q, k, qi, nj):
    return _SparseQK.apply(q, k, qi, nj)


def sparse_v_agg(v, a, qi, nj, n_rows: int):
    return _SparseVAgg.apply(v, a, qi, nj, n_rows)


def segment_metadata(row_index, col_index, num_rows: int):
    """(row_ptr, col_index, alpha_index), int32 numpy (triton_sparse_qk_autograd.py:607-632)."""
    row = np.asarray(row_index, np.int64).reshape(-1)
    col = np.asarray(col_index, np.int64).reshape(-1)
    if row.size and (row.min() < 0 or row.max() >= num_rows):
        raise ValueError("row index outside [0, num_rows)")
    perm = np.argsort(row, kind="stable")
    row_ptr = np.zeros(num_rows + 1, np.int64)
    row_ptr[1:] = np.cumsum(np.bincount(row, minlength=num_rows))
    return row_ptr.astype(np.int32), col[perm].astype(np.int32), perm.astype(np.int32)


def qk_metadata(query_index, neighbor_index, num_queries: int, num_keys: int):
    """The 6-tuple of prepare_sparse_qk_edge_index_metadata (triton_sparse_qk_autograd.py:635-652)."""
    return (*segment_metadata(query_index, neighbor_index, num_queries),
            *segment_metadata(neighbor_index, query_index, num_keys))
