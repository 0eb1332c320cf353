"""Plain-PyTorch references of the HIP operators (float64, CPU, autograd-able).

Each one restates the reference's own torch formulation of the op:
* ``mlp_ref``   RadialProfile(cat[rbf, tgt[z_i], src[z_j]])      e2former.py:258-266,302 (and 709-733)
* ``attn_ref``  logits/softmax/aggregation of e2former.py:327-433 with the
                first-order product written as the per-edge Cartesian coupling
* ``deg_ref``   EdgeDegreeEmbeddingNetwork_higherorder fallback   e2former.py:689-753
* ``attn0_ref`` zero-order aggregation of e2former.py:393-416 (value reshaped to
                [M, 9 C / H, H]: channel c weighted by head c mod H), with the
                polynomial or the bell envelope (module_utils.py:1946-1985)
Both take the weight form ``act``: None for the segmented softmax, "softplus" /
"sigmoid" for alpha = act(a) ih p (e2former.py:329-332).
"""
import math

import numpy as np
import torch

ENV = (-21.0, 35.0, -15.0)


def envelope(d, rc):
    r = d / rc
    return torch.where(r < 1, 1 + r ** 5 * (ENV[0] + r * (ENV[1] + ENV[2] * r)), torch.zeros_like(r))


def rbf(d, offset, coeff):
    return torch.exp(coeff * (d.view(-1, 1) - offset.view(1, -1)) ** 2)


def mlp_ref(d, zi, zj, net, tgt_w, src_w, offset, coeff):
    x = torch.cat([rbf(d, offset, coeff), tgt_w[zi], src_w[zj]], dim=-1)
    return net(x)


def weights(a, p, ih, row, N, act=None):
    """alpha [E, H] of the logits a, envelope p [E] and inputhead ih."""
    if act == "softplus":
        return torch.nn.functional.softplus(a) * ih * p.unsqueeze(-1)
    if act == "sigmoid":
        return torch.sigmoid(a) * ih * p.unsqueeze(-1)
    H = a.shape[1]
    rh = row.view(-1, 1).expand(-1, H)
    amax = torch.full((N, H), -torch.inf, dtype=a.dtype).scatter_reduce(0, rh, a, "amax", include_self=True)
    e = torch.exp(a - amax[row]) * p.unsqueeze(-1)
    s = torch.zeros((N, H), dtype=a.dtype).scatter_add(0, rh, e)
    return e * ih / (s[row] + 1e-3)


def attn_ref(q, k, v, dvec, dist, row, col, gi, T, rc, N, act=None):
    H = q.shape[1]
    qs = q / math.sqrt(q.shape[-1])
    qk = (qs[row] * k[col]).sum(-1)
    gate, ih = gi[:, :H], gi[:, H:]
    alpha = weights(gate * qk, envelope(dist, rc), ih, row, N, act)
    w = alpha / dist.clamp_min(1e-6).unsqueeze(-1)
    C = v.shape[-1]
    wc = w[:, torch.arange(C) % H]                       # [E, C]
    vj = v[col]                                          # [E, 9, C]
    M = torch.einsum("trk,ek->etr", T, dvec)             # [E, 20, 9]
    contrib = torch.einsum("etr,erc->etc", M, vj) * wc.unsqueeze(1)
    out = torch.zeros((N, T.shape[0], C), dtype=contrib.dtype).index_add(0, row, contrib)
    return out


def raw_sh(u):
    x, y, z = u[:, 0], u[:, 1], u[:, 2]
    s3 = math.sqrt(3.0)
    return torch.stack([torch.ones_like(x), x, y, z, s3 * x * z, s3 * x * y, y ** 2 - 0.5 * (x ** 2 + z ** 2),
                        s3 * y * z, s3 / 2 * (z ** 2 - x ** 2)], dim=-1)


def deg_ref(dvec, dist, row, fea, avg, rc, N):
    u = torch.nn.functional.normalize(dvec, dim=-1)
    Y = raw_sh(u)
    p = envelope(dist, rc).unsqueeze(-1)
    C = fea.shape[-1] // 3
    f = fea.view(-1, 3, C) * p.unsqueeze(-1)
    lidx = torch.tensor([0, 1, 1, 1, 2, 2, 2, 2, 2])
    contrib = Y.unsqueeze(-1) * f[:, lidx, :]
    return torch.zeros((N, 9, C), dtype=contrib.dtype).index_add(0, row, contrib) / avg


def bell(d, lo, hi):
    """(1 - t^2)^2, t = (2 d - (lo + hi)) / (hi - lo) clamped to [-1, 1]."""
    hi = max(hi, lo + 1e-8)
    t = torch.clamp((2 * d - (lo + hi)) / (hi - lo), -1.0, 1.0)
    return (1 - t * t) ** 2


def attn0_ref(q, k, v, dist, row, col, gi, env, N, act=None):
    """Zero-order aggregation: out[i, r, c] = sum over edges (i, j) of
    alpha_e,(c mod H) v[j, r, c], alpha the row softmax (or the act form) with
    the envelope env(d)."""
    H = q.shape[1]
    qs = q / math.sqrt(q.shape[-1])
    qk = (qs[row] * k[col]).sum(-1)
    gate, ih = gi[:, :H], gi[:, H:]
    alpha = weights(gate * qk, env(dist), ih, row, N, act)
    C = v.shape[-1]
    contrib = v[col] * alpha[:, torch.arange(C) % H].unsqueeze(1)     # [E, 9, C]
    return torch.zeros((N, v.shape[1], C), dtype=contrib.dtype).index_add(0, row, contrib)
