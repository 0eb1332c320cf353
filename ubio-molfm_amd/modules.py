"""E2Former-V2 module tree on the HIP edge path.

Class names, constructor arguments, parameter/buffer names and shapes follow the
reference (src/molfm/models/e2former/e2former.py, module_utils.py,
wigner6j/so2_tensor_product.py), so a reference state_dict loads with
``strict=True``.  Dense per-node algebra stays in PyTorch (hipBLASLt GEMMs);
every edge-level operation runs in libe2v2.so through ``ops``.
"""
from __future__ import annotations

import math
from typing import Optional

import numpy as np
import torch
from torch import nn

from . import so3
from .ops import AttentionFn, DegreeEmbedFn, MLPCache


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


def _per_l_matmul(x: torch.Tensor, weight: torch.Tensor, lmax: int) -> torch.Tensor:
    """out[:, rows(l), :] = x[:, rows(l), :] @ weight[l].T (SO3 linear, no bias)."""
    outs = []
    for l in range(lmax + 1):
        outs.append(torch.matmul(x[:, l * l:(l + 1) ** 2, :], weight[l].t()))
    return torch.cat(outs, dim=1)


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
    """module_utils.py:2151-2178 (parameters only; evaluated by e2v2_mlp_*)."""

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
    """module_utils.py:2010-2052."""

    def __init__(self, in_features, out_features, lmax, bias=True):
        super().__init__()
        self.in_features, self.out_features, self.lmax = in_features, out_features, lmax
        self.weight = nn.Parameter(torch.randn(lmax + 1, out_features, in_features))
        bound = 1 / math.sqrt(in_features)
        nn.init.uniform_(self.weight, -bound, bound)
        self.bias = nn.Parameter(torch.zeros(out_features))
        self.register_buffer("expand_index", _expand_index(lmax), persistent=False)

    def forward(self, x):
        shp = x.shape[:-2]
        ls = x.shape[-2]
        x = x.reshape(-1, ls, x.shape[-1])
        out = _per_l_matmul(x, self.weight, self.lmax)
        out[:, 0, :] = out[:, 0, :] + self.bias
        return out.reshape(shp + (ls, self.out_features))


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

    def forward(self, x):
        shp = x.shape[:-2]
        ls = x.shape[-2]
        x = x.reshape(-1, ls, x.shape[-1])
        hid = self.weight.shape[1]
        # both products in one GEMM per l: [rows, C] @ [C, 2 hid]
        wcat = torch.cat([self.weight, self.weight2], dim=1)
        o = _per_l_matmul(x, wcat, self.lmax)
        a, b = o[..., :hid], o[..., hid:]
        a = torch.cat([a[:, :1] + self.bias.view(1, 1, hid), a[:, 1:]], dim=1)
        parts = [torch.sum(a[:, l * l:(l + 1) ** 2] * b[:, l * l:(l + 1) ** 2], dim=1) for l in range(self.lmax + 1)]
        return self.final_linear(torch.cat(parts, dim=-1)).reshape(shp + (self.out_features,))


class EquivariantRMSNormArraySphericalHarmonicsV2_BL(nn.Module):
    """module_utils.py:1663-1772 (rms_norm_sh: centering, balanced degrees)."""

    def __init__(self, lmax, num_channels, eps=1e-5, affine=True, normalization="component", centering=True,
                 std_balance_degrees=True):
        super().__init__()
        if not (affine and centering and std_balance_degrees and normalization == "component"):
            raise NotImplementedError("only the rms_norm_sh configuration of the reference is implemented")
        self.lmax, self.num_channels, self.eps = lmax, num_channels, eps
        self.affine_weight = nn.Parameter(torch.ones(lmax + 1, num_channels))
        self.affine_bias = nn.Parameter(torch.zeros(num_channels))
        self.register_buffer("expand_index", _expand_index(lmax))
        bw = torch.zeros((lmax + 1) ** 2, 1)
        for l in range(lmax + 1):
            bw[l * l:(l + 1) ** 2] = 1.0 / (2 * l + 1)
        self.register_buffer("balance_degree_weight", bw / (lmax + 1))

    def forward(self, x, batch=None):
        shp = x.shape[:-2]
        f = x.reshape(-1, (self.lmax + 1) ** 2, self.num_channels)
        f0 = f[:, :1] - f[:, :1].mean(dim=2, keepdim=True)
        f = torch.cat([f0, f[:, 1:]], dim=1)
        fn = (f.pow(2) * self.balance_degree_weight.view(1, -1, 1)).sum(dim=1, keepdim=True)
        fn = (fn.mean(dim=2, keepdim=True) + self.eps).pow(-0.5)
        w = self.affine_weight.index_select(0, self.expand_index).unsqueeze(0)
        out = f * (fn * w)
        out = torch.cat([out[:, :1] + self.affine_bias.view(1, 1, -1), out[:, 1:]], dim=1)
        return out.reshape(shp + ((self.lmax + 1) ** 2, self.num_channels))


class Gate_s3(nn.Module):
    """module_utils.py:2694-2746."""

    def __init__(self, sphere_channels, lmax, act_scalars="silu", act_vector="sigmoid"):
        super().__init__()
        self.sphere_channels, self.lmax = sphere_channels, lmax
        self.gates = nn.Linear(sphere_channels, sphere_channels * (lmax + 1))
        bound = 1 / math.sqrt(sphere_channels)
        nn.init.uniform_(self.gates.weight, -bound, bound)

    def forward(self, x):
        shp = x.shape
        x = x.reshape(-1, shp[-2], shp[-1])
        C = self.sphere_channels
        sc = self.gates(x[:, 0:1])
        out = [torch.nn.functional.silu(sc[:, :, :C]) * SILU_NORM]
        st = 1
        for l in range(1, self.lmax + 1):
            out.append(torch.sigmoid(sc[:, :, l * C:(l + 1) * C]) * SIGMOID_NORM * x[:, st:st + 2 * l + 1])
            st += 2 * l + 1
        return torch.cat(out, dim=1).reshape(shp)


class FeedForwardNetwork_s3(nn.Module):
    """module_utils.py:2755-2797."""

    def __init__(self, sphere_channels, hidden_channels, output_channels, lmax):
        super().__init__()
        self.slinear_1 = SO3_Linear_e2former(sphere_channels, hidden_channels, lmax=lmax, bias=True)
        self.gate = Gate_s3(hidden_channels, lmax=lmax)
        self.slinear_2 = SO3_Linear_e2former(hidden_channels, output_channels, lmax=lmax, bias=True)

    def forward(self, x, **kw):
        return self.slinear_2(self.gate(self.slinear_1(x)))


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

    def path_scales(self) -> Optional[torch.Tensor]:
        """Per-row scale of the 20 output rows implied by the loaded CG_weight
        relative to the canonical table, or None when they coincide."""
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

    def forward_linear(self, so2):
        bs = so2.shape[0]
        st = 0
        outs = []
        for idx, (l3, cnt) in enumerate(self.l3_sequential):
            en = st + (2 * l3 + 1) * cnt
            blk = so2[:, st:en].reshape(bs, cnt, 2 * l3 + 1, -1).permute(0, 2, 1, 3).reshape(bs, 2 * l3 + 1, -1)
            outs.append(self.out_linear[idx](blk))
            st = en
        return torch.cat(outs, dim=1) * self.path_norm


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
    """Per-evaluation edge data shared by every layer."""

    def __init__(self, nl, dvec, dist, node_type, rbf: GaussianSmearing, rc: float):
        self.nl, self.dvec, self.dist = nl, dvec, dist
        self.node_type = node_type
        self.rbf_offset = rbf.offset.float().contiguous()
        self.rbf_coeff = float(rbf.coeff)
        self.rc = rc


class E2AttentionArbOrder_sparse(nn.Module):
    """e2former.py:80-436 for tp_type=QK_alpha, attn_type=so2-first-order."""

    def __init__(self, irreps_node_input="256x0e+256x1e+256x2e", attn_weight_input_dim=256, num_attn_heads=128,
                 attn_scalar_head=8, irreps_head="2x0e+2x1e+2x2e", alpha_drop=0.0, tp_type="QK_alpha",
                 attn_type="so2-first-order", atom_type_cnt=256, norm_layer="rms_norm_sh", C=256, lmax=2, **kw):
        super().__init__()
        self.num_attn_heads, self.attn_scalar_head, self.lmax = num_attn_heads, attn_scalar_head, lmax
        self.node_embed_dim = 128
        self.attn_type, self.tp_type = attn_type, tp_type.split("+")[0]
        self.source_embedding = nn.Embedding(atom_type_cnt, 128)
        self.target_embedding = nn.Embedding(atom_type_cnt, 128)
        nn.init.uniform_(self.source_embedding.weight.data, -0.001, 0.001)
        nn.init.uniform_(self.target_embedding.weight.data, -0.001, 0.001)
        self.alpha_act = SmoothLeakyReLU(0.2)
        ecl = [attn_weight_input_dim + 256, min(128, attn_weight_input_dim // 2),
               min(128, attn_weight_input_dim // 2)]
        self.alpha_dropout = nn.Dropout(alpha_drop)
        self.fc_easy = RadialProfile(ecl + [2 * num_attn_heads])
        self.query_linear = SO3_Linear2Scalar_e2former(C, num_attn_heads * attn_scalar_head, lmax=lmax)
        self.key_linear = SO3_Linear2Scalar_e2former(C, num_attn_heads * attn_scalar_head, lmax=lmax)
        self.proj_value = SO3_Linear_e2former(C, C, lmax=lmax)
        self.first_order_tp = E2TensorProductSO2_FirstOrder(None, None, head=num_attn_heads, order=1, lmax=lmax,
                                                            in_c=C, out_c=C)
        self.proj_first = SO3_Linear_e2former(num_attn_heads * 2, C, lmax=lmax)
        self._mlp = MLPCache()

    def forward(self, x: torch.Tensor, ctx: EdgeContext):
        N = x.shape[0]
        H = self.num_attn_heads
        if self.training and self.alpha_dropout.p > 0:
            raise NotImplementedError("attention dropout in training mode is not supported by the HIP path")
        q = self.query_linear(x).reshape(N, H, -1)
        k = self.key_linear(x).reshape(N, H, -1)
        v = self.proj_value(x)
        packed = self._mlp.get([self.fc_easy.net], self.target_embedding, self.source_embedding)
        so2 = AttentionFn.apply(q, k, v, ctx.dvec, ctx.dist, ctx.nl, ctx.node_type, ctx.rbf_offset, ctx.rbf_coeff,
                                packed, ctx.rc, math.sqrt(q.shape[-1]))
        tp = self.first_order_tp.so2_tp
        sc = tp.path_scales()
        if sc is not None:
            so2 = so2 * sc.to(so2.device).view(1, -1, 1)
        return self.proj_first(tp.forward_linear(so2))


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
        x = x[:, :(self.lmax + 1) ** 2]
        res = x
        h = self.norm_1(x)
        if sys_node_embedding is not None:
            h = torch.cat([h[:, :1] + sys_node_embedding.unsqueeze(1), h[:, 1:]], dim=1)
        x = self.ga(h, ctx) + res
        return x + self.ffn(self.norm_ffn(x))


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
        self._mlp = MLPCache()

    def forward(self, ctx: EdgeContext):
        packed = self._mlp.get([p.net for p in self.gbf_projs], self.target_embedding, self.source_embedding)
        return DegreeEmbedFn.apply(ctx.dvec, ctx.dist, ctx.nl, ctx.node_type, ctx.rbf_offset, ctx.rbf_coeff, packed,
                                   float(self.avg_aggregate_num), ctx.rc)


class E2former(nn.Module):
    """e2former.py:758-1145 (with_cluster off) on flattened atoms."""

    def __init__(self, irreps_node_embedding="256x0e+256x1e+256x2e", num_layers=4, max_neighbors=None,
                 max_radius=6.0, basis_type="gaussiansmear", number_of_basis=256, num_attn_heads=128,
                 attn_scalar_head=8, irreps_head="2x0e+2x1e+2x2e", norm_layer="rms_norm_sh", alpha_drop=0.0,
                 tp_type="QK_alpha", attn_type="so2-first-order", atom_type_cnt=256, edge_embedtype="default",
                 ffn_type="s3", avg_degree=23.01, with_cluster=False, **kwargs):
        super().__init__()
        C, lmax = parse_irreps(irreps_node_embedding)
        check_supported(C, lmax, num_attn_heads, attn_scalar_head, number_of_basis, irreps_head, norm_layer,
                        tp_type, attn_type, ffn_type, basis_type, with_cluster, edge_embedtype)
        self.max_neighbors, self.max_radius, self.number_of_basis = max_neighbors, max_radius, number_of_basis
        self.num_layers, self.num_attn_heads, self.lmax = num_layers, num_attn_heads, lmax
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
                       attn_scalar_head, irreps_head, alpha_drop, tp_type, attn_type, atom_type_cnt, norm_layer,
                       ffn_type, i, C=C, lmax=lmax) for i in range(num_layers)])
        self.l3_sequential = self.blocks[0].ga.first_order_tp.so2_tp.l3_sequential
        self.norm_final = EquivariantRMSNormArraySphericalHarmonicsV2_BL(lmax, C)

    def forward_flat(self, ctx: EdgeContext, sys_node_embedding: Optional[torch.Tensor] = None):
        x = self.edge_deg_embed_dense(ctx)
        for blk in self.blocks:
            x = blk(x, ctx, sys_node_embedding)
        return self.norm_final(x)


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
          and hl == lmax and norm_layer in ("rms_norm_sh", "rms_norm_sh_BL") and tp_type.split("+")[0] == "QK_alpha"
          and attn_type == "so2-first-order" and ("s3" in ffn_type or "default" in ffn_type)
          and basis_type == "gaussiansmear" and str(with_cluster) in ("False", "false", "0", "None", "none")
          and "wolayernorm" not in edge_embedtype)
    if not ok:
        raise NotImplementedError(
            "the MI355X path implements the E2Former-V2 production configuration: irreps 256x0e+256x1e+256x2e, "
            "irreps_head 2x0e+2x1e+2x2e, 128 heads, attn_scalar_head 8, 256 basis, rms_norm_sh, tp_type QK_alpha, "
            "attn_type so2-first-order, ffn s3, no cluster blocks")
