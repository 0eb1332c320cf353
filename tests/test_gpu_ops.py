"""GPU parity of each HIP operator against its plain-PyTorch float64 reference.

Tolerances: fp32 kernels vs float64 references, relative to the output scale:
forward 2e-5, input gradients 1e-4 (fp32 accumulation over ~100-edge rows).
"""
import copy
import math

import numpy as np
import pytest
import torch

from op_reference import attn0_ref, attn_ref, bell, deg_ref, envelope, mlp_ref

pytestmark = pytest.mark.gpu


def relerr(a, b):
    a = a.detach().double().cpu(); b = b.detach().double().cpu()
    return float((a - b).norm() / (b.norm() + 1e-30))


def _graph(pkg, cuda, n_mol=8, L=6.2, seed=0):
    from ubio_molfm_amd import systems, neighbors
    s = systems.small_water(n_mol, L, seed=seed)
    pos = torch.as_tensor(s["pos"], device=cuda)
    nl = neighbors.build_neighbors(pos, s["graph_ptr"], s["cell"], s["pbc"], 6.0)
    return s, pos, nl


def _profile(seed, n_in):
    """A RadialProfile [n_in, 128, 128, 256] with non-trivial LayerNorm affines."""
    from ubio_molfm_amd import modules
    torch.manual_seed(seed)
    prof = modules.RadialProfile([n_in, 128, 128, 256])
    for m in prof.modules():
        if isinstance(m, torch.nn.LayerNorm):
            m.weight.data.uniform_(0.5, 1.5); m.bias.data.uniform_(-0.2, 0.2)
    return prof


def _embeddings(seed, rows, width):
    g = torch.Generator().manual_seed(seed)
    tgt = torch.nn.Embedding(rows, width); src = torch.nn.Embedding(rows, width)
    with torch.no_grad():
        tgt.weight.copy_(torch.randn(rows, width, generator=g)); src.weight.copy_(torch.randn(rows, width, generator=g))
    return tgt, src


def _profile_fn(net, tgt_row, src_row, offset, coeff):
    """f(d) [256] of one profile for fixed type rows, in float64 with explicit ops
    (forward-mode differentiable to any order)."""
    lin1, ln1, lin2, ln2, lin3 = [net[i] for i in (0, 1, 3, 4, 6)]
    W = [t.detach().double() for t in (lin1.weight, lin1.bias, ln1.weight, ln1.bias, lin2.weight, lin2.bias,
                                        ln2.weight, ln2.bias, lin3.weight, lin3.bias)]
    mu = offset.double()

    def ln(x, g, b):
        m = x.mean(-1, keepdim=True)
        v = ((x - m) ** 2).mean(-1, keepdim=True)
        return (x - m) / torch.sqrt(v + 1e-5) * g + b

    def silu(x):
        return x * torch.sigmoid(x)

    def f(d):
        x = torch.cat([torch.exp(coeff * (d - mu) ** 2), tgt_row, src_row])
        h = silu(ln(W[0] @ x + W[1], W[2], W[3]))
        h = silu(ln(W[4] @ h + W[5], W[6], W[7]))
        return W[8] @ h + W[9]
    return f


def test_radial_table_jets_and_interpolation(pkg, cuda):
    """The float64 jet propagation of e2v2_radial_table against nested
    forward-mode autodiff of the same profile (torch.func, float64): rows
    h^k d^k f/dd^k, k = 0..3, at sampled nodes of every type pair, to fp32
    rounding; then the quintic Hermite interpolant of the fp32 table (rows 0..2
    for the value, 1..3 for the derivative, the kernels' interval arithmetic) at
    2000 random distances against the float64 profile: value within 1e-6 and
    derivative within 1e-5 of the profile's scale, as the table's own midpoint
    check reports."""
    from torch.func import jacfwd, vmap
    from ubio_molfm_amd import modules, ops
    rc = 6.0
    rb = modules.GaussianSmearing(256, rc, 2.0)
    prof = _profile(3, 512)
    tgt, src = _embeddings(4, 256, 128)
    net = copy.deepcopy(prof).net
    tw, sw = tgt.weight.detach().clone(), src.weight.detach().clone()
    type_z = torch.tensor([1, 6, 8], dtype=torch.int32, device=cuda)
    tab = ops.RadialTable([prof.to(cuda).net], tgt.to(cuda), src.to(cuda), rb.offset.to(cuda), rb.coeff, rc, type_z)
    T = tab.tab.cpu().double()                               # [9, n, 4, 256]
    h, n = tab.h, tab.n_nodes
    print(f"[radial table] n={n} h={h} check: value {tab.value_err:.2e} derivative {tab.deriv_err:.2e}", flush=True)
    assert tab.value_err <= 1e-6 and tab.deriv_err <= 1e-5
    coeff = float(np.float32(rb.coeff))
    rng = np.random.default_rng(0)
    zs = [1, 6, 8]
    for p in range(9):
        f = _profile_fn(net, tw[zs[p // 3]].double(), sw[zs[p % 3]].double(), rb.offset, coeff)
        f1 = jacfwd(f); f2 = jacfwd(f1); f3 = jacfwd(f2)
        nodes = torch.tensor([0, 1, 100, n // 2, n - 1] + list(rng.integers(0, n, 3)))
        d = nodes.double() * h
        with torch.no_grad():
            rows = [vmap(g)(d) for g in (f, f1, f2, f3)]
        for k in range(4):
            ref = rows[k] * h ** k
            err = float((T[p, nodes, k] - ref).abs().max() / ref.abs().max())
            assert err < 2e-6, (p, k, err)
        dq = torch.as_tensor(np.concatenate([rng.uniform(0.5, rc, 250), [rc]])).float()
        u = torch.clamp(dq * (1.0 / h), max=float(n - 2))
        k0 = torch.floor(u).long()
        t = (u - k0).double()[:, None]
        H = [w for w in (1 - 10 * t ** 3 + 15 * t ** 4 - 6 * t ** 5, t - 6 * t ** 3 + 8 * t ** 4 - 3 * t ** 5,
                         0.5 * (t ** 2 - 3 * t ** 3 + 3 * t ** 4 - t ** 5), 10 * t ** 3 - 15 * t ** 4 + 6 * t ** 5,
                         -4 * t ** 3 + 7 * t ** 4 - 3 * t ** 5, 0.5 * (t ** 3 - 2 * t ** 4 + t ** 5))]
        A, B = T[p, k0], T[p, k0 + 1]
        val = H[0] * A[:, 0] + H[1] * A[:, 1] + H[2] * A[:, 2] + H[3] * B[:, 0] + H[4] * B[:, 1] + H[5] * B[:, 2]
        der = (H[0] * A[:, 1] + H[1] * A[:, 2] + H[2] * A[:, 3] + H[3] * B[:, 1] + H[4] * B[:, 2]
               + H[5] * B[:, 3]) / h
        with torch.no_grad():
            fv, fd = vmap(f)(dq.double()), vmap(f1)(dq.double())
        ev = float((val - fv).abs().max() / fv.abs().max())
        ed = float((der - fd).abs().max() / fd.abs().max())
        assert ev < 1e-6 and ed < 1e-5, (p, ev, ed)


def _attn_inputs(nl, cuda, seed=2):
    g = torch.Generator().manual_seed(seed)
    N = nl.n_atoms
    q = torch.randn(N, 128, 8, generator=g); k = torch.randn(N, 128, 8, generator=g)
    v = torch.randn(N, 9, 256, generator=g)
    return q, k, v


def _types(pkg, cuda, Z):
    """(type_z device, slot per atom device) as the model forms them."""
    zs = sorted(set(int(z) for z in np.asarray(Z)))
    lut = {z: i for i, z in enumerate(zs)}
    return (torch.tensor(zs, dtype=torch.int32, device=cuda),
            torch.tensor([lut[int(z)] for z in np.asarray(Z)], dtype=torch.int32, device=cuda))


def _attention_case(pkg, cuda, act_dtype, clusters=True, graph=None):
    """Attention fwd + bwd through the C ABI against the float64 reference, whose
    gate | inputhead come from the float64 fc_easy profile of each edge (so the
    distance gradient includes the profile's derivative).  With bf16 storage the
    inputs (q, k, v, grad) are rounded to bf16 for both sides, so the remaining
    differences are the bf16 output rows (also used by the backward's D_h) and
    fp32 arithmetic."""
    from ubio_molfm_amd import _lib, modules, ops, so3
    s, pos, nl = graph if graph is not None else _graph(pkg, cuda, seed=4)
    N, E = nl.n_atoms, nl.n_edges
    bf = act_dtype == torch.bfloat16
    print(f"[attn {act_dtype}] N={N} E={E}", flush=True)
    q, k, v = _attn_inputs(nl, cuda)
    G = torch.randn(N, 20, 256, generator=torch.Generator().manual_seed(7))
    if bf:
        q, k, v, G = (t.to(torch.bfloat16).float() for t in (q, k, v, G))
    rb = modules.GaussianSmearing(256, 6.0, 2.0)
    prof = _profile(9, 512)
    tgt, src = _embeddings(10, 256, 128)
    net64 = copy.deepcopy(prof).double().net
    tw, sw = tgt.weight.detach().double().clone(), src.weight.detach().double().clone()
    type_z, slot = _types(pkg, cuda, s["Z"])
    tab = ops.RadialTable([prof.to(cuda).net], tgt.to(cuda), src.to(cuda), rb.offset.to(cuda), rb.coeff, 6.0, type_z,
                          layout="attn")
    st = _lib.vp(torch.cuda.current_stream().cuda_stream)
    # the kernels hold v, out and their gradients in slice order: position p holds model channel P[p]
    P = modules.slice_perm(cuda)
    Pinv = torch.argsort(P)
    qd, kd = (t.to(cuda).to(act_dtype).contiguous() for t in (q, k))
    vd = v.permute(1, 0, 2).to(cuda)[:, :, P].contiguous().to(act_dtype)          # m-major [9, N, C]
    args = ops.attn_args(nl, qd, kd, vd, slot, tab, math.sqrt(8.0), 6.0, int(bf))
    if not clusters:
        args.col_slot_member = args.col_slot_edge = args.col_n_slots = None
    out = torch.empty(20 * N * 256, device=cuda, dtype=act_dtype)   # l3-grouped rows
    m = torch.empty(N, 128, device=cuda)
    sr = torch.empty(N, 128, device=cuda); cnt = torch.empty(N, 128, dtype=torch.int32, device=cuda)
    _lib.call("e2v2_attn_fwd", _lib.C.byref(args), _lib.vp(out.data_ptr()), _lib.vp(m.data_ptr()),
              _lib.vp(sr.data_ptr()), _lib.vp(cnt.data_ptr()), st)
    T = torch.as_tensor(so3.cartesian_tp_table())
    row = nl.edge_row.long().cpu(); col = nl.col.long().cpu()
    Z = torch.as_tensor(np.asarray(s["Z"]))
    leaves = [t.double().requires_grad_(True) for t in (q, k, v, nl.dvec.cpu(), nl.dist.cpu())]
    gi = mlp_ref(leaves[4], Z[row], Z[col], net64, tw, sw, rb.offset.double(), float(np.float32(rb.coeff)))
    ref = attn_ref(*leaves[:5], row, col, gi, T, 6.0, N)
    e_f = relerr(ops.so2_rows(out, N).float()[:, :, Pinv].permute(1, 0, 2), ref)
    grads = torch.autograd.grad((ref * G.double()).sum(), leaves)
    Gd = ops.so2_grouped(G.permute(1, 0, 2).to(cuda)[:, :, P].contiguous()).to(act_dtype)
    f = dict(device=cuda)
    ddv = torch.empty(E, 3, **f); dd = torch.empty(E, **f)
    dq = torch.empty(qd.shape, **f); dk = torch.empty(kd.shape, **f); dv = torch.empty(vd.shape, **f)
    nb = int(_lib.load().e2v2_attn_bwd_workspace(E))
    ws = torch.empty(nb, dtype=torch.uint8, device=cuda)
    _lib.call("e2v2_attn_bwd", _lib.C.byref(args), _lib.vp(Gd.data_ptr()), _lib.vp(out.data_ptr()),
              _lib.vp(m.data_ptr()), _lib.vp(sr.data_ptr()), _lib.vp(cnt.data_ptr()),
              _lib.vp(ddv.data_ptr()), _lib.vp(dd.data_ptr()), _lib.vp(dq.data_ptr()), _lib.vp(dk.data_ptr()),
              _lib.vp(dv.data_ptr()), _lib.vp(ws.data_ptr()), _lib.C.c_size_t(nb), st)
    errs = dict(q=relerr(dq, grads[0]), k=relerr(dk, grads[1]), v=relerr(dv[:, :, Pinv].permute(1, 0, 2), grads[2]),
                dvec=relerr(ddv, grads[3]), dist=relerr(dd, grads[4]))
    print(f"[attn {act_dtype}] fwd rel {e_f:.2e} bwd {errs}", flush=True)
    return e_f, errs


@pytest.mark.parametrize("clusters", [True, False], ids=["clusters", "per_column"])
def test_attention_forward_backward(pkg, cuda, clusters):
    e_f, errs = _attention_case(pkg, cuda, torch.float32, clusters)
    assert e_f < 2e-5
    for name, e in errs.items():
        assert e < 1e-4, (name, e)


def test_attention_ragged_clusters_isolated_atoms(pkg, cuda):
    """Column clusters that end part-way (N = 23, not a multiple of 4) and atoms
    with no edges at all (two atoms 100 A away, non-periodic): every row and
    column still matches the float64 reference, isolated rows give zero output."""
    from ubio_molfm_amd import neighbors
    rng = np.random.default_rng(21)
    p = rng.normal(size=(23, 3)) * 1.8
    p[21] = [100.0, 0.0, 0.0]
    p[22] = [0.0, -100.0, 0.0]
    s = dict(pos=p.astype(np.float32), Z=np.full(23, 6), graph_ptr=np.array([0, 23]),
             cell=np.zeros((1, 3, 3), np.float32), pbc=np.zeros((1, 3), bool))
    pos = torch.as_tensor(s["pos"], device=cuda)
    nl = neighbors.build_neighbors(pos, s["graph_ptr"], s["cell"], s["pbc"], 6.0)
    deg = np.diff(nl.row_ptr.cpu().numpy())
    assert deg[21] == 0 and deg[22] == 0 and nl.n_atoms % 4 != 0
    e_f, errs = _attention_case(pkg, cuda, torch.float32, True, (s, pos, nl))
    assert e_f < 2e-5
    for name, e in errs.items():
        assert e < 1e-4, (name, e)


@pytest.mark.parametrize("clusters", [True, False], ids=["col_clusters", "col_rows"])
def test_attention_bf16_storage(pkg, cuda, clusters):
    """bf16 storage of q, k, v, out and grad (fp32 math): forward within 4e-3
    (one bf16 rounding of the output rows), gradients within 1e-2; the column
    pass over key-column clusters and the one-column-per-workgroup form."""
    e_f, errs = _attention_case(pkg, cuda, torch.bfloat16, clusters=clusters)
    assert e_f < 4e-3
    for name, e in errs.items():
        assert e < 1e-2, (name, e)


@pytest.mark.parametrize("env, act, form", [("poly", "fp32", None), ("bell", "fp32", None), ("poly", "bf16", None),
                                            ("bell", "bf16", None), ("bell", "fp32", "softplus"),
                                            ("poly", "fp32", "sigmoid"), ("bell", "bf16", "sigmoid")])
def test_zero_order_attention(pkg, cuda, env, act, form):
    """The zero-order attention of the long-range blocks through AttentionFn
    (e2v2_attn_fwd / e2v2_attn_bwd with zero_order set) on the long-range list
    (12 A, lower cutoff 0.1 A, sources O only), against the float64 reference
    with the profile evaluated per edge: the polynomial envelope on [0, 12] or
    the bell on [0.1, 12]; the segmented softmax or the softplus / sigmoid
    weights.  The output does not depend on dvec: its gradient is exactly zero;
    the distance gradient carries the envelope, the profile and the weights.
    fp32: forward 2e-5, gradients 1e-4; bf16 storage (inputs and output
    gradient rounded to bf16 on both sides): 4e-3 and 1e-2."""
    from ubio_molfm_amd import modules, neighbors, ops, systems
    rc, lo = 12.0, 0.1
    bf = act == "bf16"
    adt = torch.bfloat16 if bf else torch.float32
    s = systems.small_water(8, 6.2, seed=6)
    pos = torch.as_tensor(s["pos"], device=cuda)
    inc = torch.as_tensor(np.asarray(s["Z"]) != 1, device=cuda)
    nl = neighbors.build_neighbors(pos, s["graph_ptr"], s["cell"], s["pbc"], rc, lo, src_include=inc)
    N, E = nl.n_atoms, nl.n_edges
    print(f"[attn zero-order {env} {act} {form}] N={N} E={E}", flush=True)
    q, k, v = _attn_inputs(nl, cuda, seed=12)
    G = torch.randn(N, 9, 256, generator=torch.Generator().manual_seed(13))
    if bf:
        q, k, v, G = (t.to(torch.bfloat16).float() for t in (q, k, v, G))
    rb = modules.GaussianSmearing(256, rc, 2.0)
    prof = _profile(14, 512)
    tgt, src = _embeddings(15, 256, 128)
    net64 = copy.deepcopy(prof).double().net
    tw, sw = tgt.weight.detach().double().clone(), src.weight.detach().double().clone()
    type_z, slot = _types(pkg, cuda, s["Z"])
    tab = ops.RadialTable([prof.to(cuda).net], tgt.to(cuda), src.to(cuda), rb.offset.to(cuda), rb.coeff, rc, type_z,
                          layout="attn")
    P = modules.slice_perm(cuda)
    Pinv = torch.argsort(P)
    env_t = (1, lo) if env == "bell" else (0, 0.0)
    dvec = nl.dvec.clone().requires_grad_(True)
    dist = nl.dist.clone().requires_grad_(True)
    qd = q.to(cuda).requires_grad_(True); kd = k.to(cuda).requires_grad_(True)
    vd = v.permute(1, 0, 2).to(cuda)[:, :, P].contiguous().requires_grad_(True)
    out = ops.AttentionFn.apply(qd, kd, vd, dvec, dist, nl, slot, tab, rc, math.sqrt(8.0), adt, True, env_t, None,
                                form or "softmax")
    assert out.shape == (9, N, 256)
    Gd = G.permute(1, 0, 2).to(cuda)[:, :, P].contiguous()
    out.backward(Gd.to(out.dtype))
    row = nl.edge_row.long().cpu(); col = nl.col.long().cpu()
    Z = torch.as_tensor(np.asarray(s["Z"]))
    leaves = [t.double().requires_grad_(True) for t in (q, k, v, nl.dist.cpu())]
    gi = mlp_ref(leaves[3], Z[row], Z[col], net64, tw, sw, rb.offset.double(), float(np.float32(rb.coeff)))
    env_fn = (lambda d: bell(d, lo, rc)) if env == "bell" else (lambda d: envelope(d, rc))
    ref = attn0_ref(*leaves[:3], leaves[3], row, col, gi, env_fn, N, form)
    e_f = relerr(out.float()[:, :, Pinv].permute(1, 0, 2), ref)
    grads = torch.autograd.grad((ref * G.double()).sum(), leaves)
    errs = dict(q=relerr(qd.grad, grads[0]), k=relerr(kd.grad, grads[1]),
                v=relerr(vd.grad[:, :, Pinv].permute(1, 0, 2), grads[2]), dist=relerr(dist.grad, grads[3]))
    print(f"[attn zero-order {env} {act} {form}] fwd rel {e_f:.2e} bwd {errs}", flush=True)
    assert torch.count_nonzero(dvec.grad) == 0
    assert e_f < (4e-3 if bf else 2e-5)
    for name, e in errs.items():
        assert e < (1e-2 if bf else 1e-4), (name, e)


def test_attention_external_gate(pkg, cuda):
    """The attention kernels with the caller's gate per (edge, head) (the QKdot
    variants): forward and gradients against the float64 reference fed the same
    gate and the table's inputhead; the gate's gradient comes back as dL/dgate
    [E, H] and the distance gradient carries only the inputhead, envelope and 1/d
    terms.  fp32: forward 2e-5, gradients 1e-4."""
    from ubio_molfm_amd import modules, ops, so3
    s, pos, nl = _graph(pkg, cuda, seed=5)
    N, E = nl.n_atoms, nl.n_edges
    print(f"[attn ext gate] N={N} E={E}", flush=True)
    q, k, v = _attn_inputs(nl, cuda, seed=16)
    gate = torch.randn(E, 128, generator=torch.Generator().manual_seed(17), dtype=torch.float64)
    G = torch.randn(N, 20, 256, generator=torch.Generator().manual_seed(18))
    rb = modules.GaussianSmearing(256, 6.0, 2.0)
    prof = _profile(19, 512)
    tgt, src = _embeddings(20, 256, 128)
    net64 = copy.deepcopy(prof).double().net
    tw, sw = tgt.weight.detach().double().clone(), src.weight.detach().double().clone()
    type_z, slot = _types(pkg, cuda, s["Z"])
    tab = ops.RadialTable([prof.to(cuda).net], tgt.to(cuda), src.to(cuda), rb.offset.to(cuda), rb.coeff, 6.0, type_z,
                          layout="attn")
    P = modules.slice_perm(cuda)
    Pinv = torch.argsort(P)
    dvec = nl.dvec.clone().requires_grad_(True)
    dist = nl.dist.clone().requires_grad_(True)
    qd = q.to(cuda).requires_grad_(True); kd = k.to(cuda).requires_grad_(True)
    vd = v.permute(1, 0, 2).to(cuda)[:, :, P].contiguous().requires_grad_(True)
    gd = gate.float().to(cuda).requires_grad_(True)
    out = ops.AttentionFn.apply(qd, kd, vd, dvec, dist, nl, slot, tab, 6.0, math.sqrt(8.0), torch.float32, False,
                                (0, 0.0), gd)
    out.backward(ops.so2_grouped(G.permute(1, 0, 2).to(cuda)[:, :, P].contiguous()))
    T = torch.as_tensor(so3.cartesian_tp_table())
    row = nl.edge_row.long().cpu(); col = nl.col.long().cpu()
    Z = torch.as_tensor(np.asarray(s["Z"]))
    leaves = [t.double().requires_grad_(True) for t in (q, k, v, nl.dvec.cpu(), nl.dist.cpu())] + \
        [gate.clone().requires_grad_(True)]
    gi = mlp_ref(leaves[4], Z[row], Z[col], net64, tw, sw, rb.offset.double(), float(np.float32(rb.coeff)))
    gi = torch.cat([leaves[5], gi[:, 128:]], dim=1)
    ref = attn_ref(*leaves[:5], row, col, gi, T, 6.0, N)
    e_f = relerr(ops.so2_rows(out.detach(), N)[:, :, Pinv].permute(1, 0, 2), ref)
    grads = torch.autograd.grad((ref * G.double()).sum(), leaves)
    errs = dict(q=relerr(qd.grad, grads[0]), k=relerr(kd.grad, grads[1]),
                v=relerr(vd.grad[:, :, Pinv].permute(1, 0, 2), grads[2]), dvec=relerr(dvec.grad, grads[3]),
                dist=relerr(dist.grad, grads[4]), gate=relerr(gd.grad, grads[5]))
    print(f"[attn ext gate] fwd rel {e_f:.2e} bwd {errs}", flush=True)
    assert e_f < 2e-5
    for name, e in errs.items():
        assert e < 1e-4, (name, e)


@pytest.mark.parametrize("form, ext", [("softplus", False), ("sigmoid", False), ("sigmoid", True)])
def test_attention_act_weights(pkg, cuda, form, ext):
    """The first-order attention with tp_type's "+softplus" / "+sigmoid" weights
    alpha = act(gate q.k) ih p (e2former.py:329-332: no row maximum or sum),
    the gate from the table or from the caller: forward and gradients through
    AttentionFn against the float64 reference.  fp32: forward 2e-5, gradients
    1e-4."""
    from ubio_molfm_amd import modules, ops, so3
    s, pos, nl = _graph(pkg, cuda, seed=6)
    N, E = nl.n_atoms, nl.n_edges
    print(f"[attn {form} ext={ext}] N={N} E={E}", flush=True)
    q, k, v = _attn_inputs(nl, cuda, seed=21)
    gate = torch.randn(E, 128, generator=torch.Generator().manual_seed(22), dtype=torch.float64)
    G = torch.randn(N, 20, 256, generator=torch.Generator().manual_seed(23))
    rb = modules.GaussianSmearing(256, 6.0, 2.0)
    prof = _profile(24, 512)
    tgt, src = _embeddings(25, 256, 128)
    net64 = copy.deepcopy(prof).double().net
    tw, sw = tgt.weight.detach().double().clone(), src.weight.detach().double().clone()
    type_z, slot = _types(pkg, cuda, s["Z"])
    tab = ops.RadialTable([prof.to(cuda).net], tgt.to(cuda), src.to(cuda), rb.offset.to(cuda), rb.coeff, 6.0, type_z,
                          layout="attn")
    P = modules.slice_perm(cuda)
    Pinv = torch.argsort(P)
    dvec = nl.dvec.clone().requires_grad_(True)
    dist = nl.dist.clone().requires_grad_(True)
    qd = q.to(cuda).requires_grad_(True); kd = k.to(cuda).requires_grad_(True)
    vd = v.permute(1, 0, 2).to(cuda)[:, :, P].contiguous().requires_grad_(True)
    gd = gate.float().to(cuda).requires_grad_(True) if ext else None
    out = ops.AttentionFn.apply(qd, kd, vd, dvec, dist, nl, slot, tab, 6.0, math.sqrt(8.0), torch.float32, False,
                                (0, 0.0), gd, form)
    out.backward(ops.so2_grouped(G.permute(1, 0, 2).to(cuda)[:, :, P].contiguous()))
    T = torch.as_tensor(so3.cartesian_tp_table())
    row = nl.edge_row.long().cpu(); col = nl.col.long().cpu()
    Z = torch.as_tensor(np.asarray(s["Z"]))
    leaves = [t.double().requires_grad_(True) for t in (q, k, v, nl.dvec.cpu(), nl.dist.cpu())]
    gi = mlp_ref(leaves[4], Z[row], Z[col], net64, tw, sw, rb.offset.double(), float(np.float32(rb.coeff)))
    if ext:
        leaves.append(gate.clone().requires_grad_(True))
        gi = torch.cat([leaves[5], gi[:, 128:]], dim=1)
    ref = attn_ref(*leaves[:5], row, col, gi, T, 6.0, N, form)
    e_f = relerr(ops.so2_rows(out.detach(), N)[:, :, Pinv].permute(1, 0, 2), ref)
    grads = torch.autograd.grad((ref * G.double()).sum(), leaves)
    errs = dict(q=relerr(qd.grad, grads[0]), k=relerr(kd.grad, grads[1]),
                v=relerr(vd.grad[:, :, Pinv].permute(1, 0, 2), grads[2]), dvec=relerr(dvec.grad, grads[3]),
                dist=relerr(dist.grad, grads[4]))
    if ext:
        errs["gate"] = relerr(gd.grad, grads[5])
    print(f"[attn {form} ext={ext}] fwd rel {e_f:.2e} bwd {errs}", flush=True)
    assert e_f < 2e-5
    for name, e in errs.items():
        assert e < 1e-4, (name, e)


def test_radial_eval_per_edge(pkg, cuda):
    """e2v2_radial_eval / _bwd: three profiles in the plain layout (768 channels)
    at every edge against the float64 profiles, value within 2e-6 of the scale,
    and dL/dd for a random weighting against float64 autograd (1e-5)."""
    from ubio_molfm_amd import modules, ops
    s, pos, nl = _graph(pkg, cuda, seed=6)
    E = nl.n_edges
    rb = modules.GaussianSmearing(256, 6.0, 2.0)
    profs = [_profile(30 + m, 512) for m in range(3)]
    tgt, src = _embeddings(33, 256, 128)
    tw, sw = tgt.weight.detach().double().clone(), src.weight.detach().double().clone()
    type_z, slot = _types(pkg, cuda, s["Z"])
    tab = ops.RadialTable([copy.deepcopy(p).to(cuda).net for p in profs], tgt.to(cuda), src.to(cuda),
                          rb.offset.to(cuda), rb.coeff, 6.0, type_z, layout="plain")
    dist = nl.dist.clone().requires_grad_(True)
    out = ops.RadialEvalFn.apply(dist, nl, slot, tab)
    g = torch.randn(E, 768, generator=torch.Generator().manual_seed(34))
    out.backward(g.to(cuda))
    row = nl.edge_row.long().cpu(); col = nl.col.long().cpu()
    Z = torch.as_tensor(np.asarray(s["Z"]))
    d64 = nl.dist.cpu().double().requires_grad_(True)
    ref = torch.cat([mlp_ref(d64, Z[row], Z[col], copy.deepcopy(p).double().net, tw, sw, rb.offset.double(),
                             float(np.float32(rb.coeff))) for p in profs], dim=1)
    (dref,) = torch.autograd.grad((ref * g.double()).sum(), [d64])
    ev = float((out.detach().cpu().double() - ref).abs().max() / ref.abs().max())
    ed = relerr(dist.grad, dref)
    print(f"[radial eval] E={E} value {ev:.2e} ddist relL2 {ed:.2e}", flush=True)
    assert ev < 2e-6 and ed < 1e-5


@pytest.mark.parametrize("pieces, ragged", [(3, False), (3, True), (1, False)])
def test_qkdot_gate_fused(pkg, cuda, pieces, ragged):
    """e2v2_qkdot_gate_fwd / _bwd (QKdotGateFn): gate = fc_m0(x0 * rad) with
    x0[e, l] = sum_{m in l} Y[e, m] xd[m, row(e)] and rad the three 256-channel
    profiles at every edge, against float64 (profiles evaluated per edge); the
    gradients to Y, xd (per-row sums over rows that cross the 128-edge tiles, and
    zero for atoms without edges) and dist (through rad).  pieces 3 (fp32): gate
    2e-6 of the scale, gradients 1e-5; pieces 1 (the bf16 mode: W and the edge
    operand rounded to bf16): 1e-2.  "ragged": 150 atoms in a ball of radius
    2.9 A (rows of 149 edges, so rows span up to three 128-edge tiles) plus two
    isolated atoms, an edge count that is not a multiple of 128."""
    from ubio_molfm_amd import gemm as s3gemm, modules, neighbors, ops
    if ragged:
        rng = np.random.default_rng(61)
        u = rng.normal(size=(152, 3))
        p = u / np.linalg.norm(u, axis=1, keepdims=True) * 2.9 * rng.uniform(0, 1, size=(152, 1)) ** (1 / 3)
        p[150] = [100.0, 0.0, 0.0]
        p[151] = [0.0, -100.0, 0.0]
        s = dict(pos=p.astype(np.float32), Z=rng.choice([1, 6, 8], size=152), graph_ptr=np.array([0, 152]),
                 cell=np.zeros((1, 3, 3), np.float32), pbc=np.zeros((1, 3), bool))
        nl = neighbors.build_neighbors(torch.as_tensor(s["pos"], device=cuda), s["graph_ptr"], s["cell"], s["pbc"],
                                       6.0)
        deg = np.diff(nl.row_ptr.cpu().numpy())
        assert deg[150] == 0 and deg[151] == 0 and nl.n_edges % 128 != 0 and deg.max() > 128
    else:
        s, pos, nl = _graph(pkg, cuda, seed=8)
    N, E = nl.n_atoms, nl.n_edges
    print(f"[qkdot gate pieces={pieces} ragged={ragged}] N={N} E={E}", flush=True)
    gen = torch.Generator().manual_seed(70 + pieces)
    rb = modules.GaussianSmearing(256, 6.0, 2.0)
    profs = [_profile(71 + m, 512) for m in range(3)]
    tgt, src = _embeddings(74, 256, 128)
    tw, sw = tgt.weight.detach().double().clone(), src.weight.detach().double().clone()
    type_z, slot = _types(pkg, cuda, s["Z"])
    tab = ops.RadialTable([copy.deepcopy(p).to(cuda).net for p in profs], tgt.to(cuda), src.to(cuda),
                          rb.offset.to(cuda), rb.coeff, 6.0, type_z, layout="plain")
    fc = torch.nn.Linear(768, 128)
    with torch.no_grad():
        fc.weight.normal_(0.0, 0.05, generator=gen); fc.bias.normal_(0.0, 0.1, generator=gen)
    W = fc.weight.detach().to(cuda)
    packs = (s3gemm.pack(W, pieces=pieces), s3gemm.pack(W, transpose=True, pieces=pieces))
    Y = torch.randn(E, 9, generator=gen); xd = torch.randn(9, N, 256, generator=gen)
    G = torch.randn(E, 128, generator=gen)
    if pieces == 1:
        W = W.to(torch.bfloat16).float()
    dist = nl.dist.clone().requires_grad_(True)
    Yd = Y.to(cuda).requires_grad_(True); xdd = xd.to(cuda).requires_grad_(True)
    gate = ops.QKdotGateFn.apply(dist, Yd, xdd, nl, slot, tab, packs, fc.bias.detach().to(cuda))
    gate.backward(G.to(cuda))
    row = nl.edge_row.long().cpu(); col = nl.col.long().cpu()
    Z = torch.as_tensor(np.asarray(s["Z"]))
    d64 = nl.dist.cpu().double().requires_grad_(True)
    Y64, x64 = Y.double().requires_grad_(True), xd.double().requires_grad_(True)
    rad = torch.cat([mlp_ref(d64, Z[row], Z[col], copy.deepcopy(p).double().net, tw, sw, rb.offset.double(),
                             float(np.float32(rb.coeff))) for p in profs], dim=1)
    blocks = [(0, 1), (1, 4), (4, 9)]
    x0 = torch.cat([torch.einsum("em,mec->ec", Y64[:, a:b], x64[a:b][:, row]) for a, b in blocks], dim=1)
    ref = (x0 * rad) @ W.cpu().double().t() + fc.bias.detach().double()
    gY, gx, gd = torch.autograd.grad((ref * G.double()).sum(), [Y64, x64, d64])
    ev = float((gate.detach().cpu().double() - ref).abs().max() / ref.abs().max())
    errs = dict(dY=relerr(Yd.grad, gY), dxd=relerr(xdd.grad, gx), ddist=relerr(dist.grad, gd))
    print(f"[qkdot gate pieces={pieces} ragged={ragged}] gate {ev:.2e} {errs}", flush=True)
    tol_v, tol_g = (2e-6, 1e-5) if pieces == 3 else (1e-2, 1e-2)
    assert ev < tol_v
    for name, e in errs.items():
        assert e < tol_g, (name, e)
    if ragged:
        assert torch.count_nonzero(xdd.grad[:, 150:]) == 0


@pytest.mark.parametrize("C", [256, 43])
def test_sh_contract(pkg, cuda, C):
    """e2v2_sh_contract / _bwd: x0[e, l] = sum_{m in l} Y[e, m] xn[m, row(e)] and
    its gradients (dY per edge, dxn summed over each row's edges) against
    float64; C = 256 (QKdot_alpha) and 43 (QKdotS_alpha's H // 3 + 1)."""
    from ubio_molfm_amd import ops
    s, pos, nl = _graph(pkg, cuda, seed=7)
    N, E = nl.n_atoms, nl.n_edges
    gen = torch.Generator().manual_seed(40 + C)
    Y = torch.randn(E, 9, generator=gen); xn = torch.randn(9, N, C, generator=gen)
    g = torch.randn(E, 3, C, generator=gen)
    Yd = Y.to(cuda).requires_grad_(True); xd = xn.to(cuda).requires_grad_(True)
    x0 = ops.ShContractFn.apply(Yd, xd, nl)
    x0.backward(g.to(cuda))
    row = nl.edge_row.long().cpu()
    Y64, x64 = Y.double().requires_grad_(True), xn.double().requires_grad_(True)
    blocks = [(0, 1), (1, 4), (4, 9)]
    ref = torch.stack([torch.einsum("em,mec->ec", Y64[:, a:b], x64[a:b][:, row]) for a, b in blocks], dim=1)
    gY, gx = torch.autograd.grad((ref * g.double()).sum(), [Y64, x64])
    errs = dict(x0=relerr(x0, ref), dY=relerr(Yd.grad, gY), dxn=relerr(xd.grad, gx))
    print(f"[sh contract C={C}] E={E} {errs}", flush=True)
    for name, e in errs.items():
        assert e < 1e-6, (name, e)


def test_degree_forward_backward(pkg, cuda):
    """Degree embedding fwd + bwd through the C ABI against the float64 restated
    fallback, with the three gbf_projs profiles evaluated in float64 per edge
    (the distance gradient includes their derivative)."""
    from ubio_molfm_amd import _lib, modules, ops
    s, pos, nl = _graph(pkg, cuda, seed=5)
    N, E = nl.n_atoms, nl.n_edges
    rb = modules.GaussianSmearing(256, 6.0, 2.0)
    profs = [_profile(20 + l, 768) for l in range(3)]
    tgt, src = _embeddings(23, 300, 256)
    nets64 = [copy.deepcopy(p_).double().net for p_ in profs]
    tw, sw = tgt.weight.detach().double().clone(), src.weight.detach().double().clone()
    type_z, slot = _types(pkg, cuda, s["Z"])
    tab = ops.RadialTable([p_.to(cuda).net for p_ in profs], tgt.to(cuda), src.to(cuda), rb.offset.to(cuda),
                          rb.coeff, 6.0, type_z, layout="deg")
    st = _lib.vp(torch.cuda.current_stream().cuda_stream)
    a = ops.deg_args(nl, slot, tab, 23.01, 6.0)
    x0 = torch.empty(9, N, 256, device=cuda)
    _lib.call("e2v2_deg_fwd", _lib.C.byref(a), _lib.vp(x0.data_ptr()), st)
    row = nl.edge_row.long().cpu(); col = nl.col.long().cpu()
    Z = torch.as_tensor(np.asarray(s["Z"]))
    leaves = [nl.dvec.cpu().double().requires_grad_(True), nl.dist.cpu().double().requires_grad_(True)]
    coeff = float(np.float32(rb.coeff))
    fea = torch.cat([mlp_ref(leaves[1], Z[row], Z[col], n64, tw, sw, rb.offset.double(), coeff) for n64 in nets64],
                    dim=-1)
    ref = deg_ref(leaves[0], leaves[1], row, fea, 23.01, 6.0, N)
    G = torch.randn(N, 9, 256, generator=torch.Generator().manual_seed(9))
    grads = torch.autograd.grad((ref * G.double()).sum(), leaves)
    Gd = G.permute(1, 0, 2).contiguous().to(cuda)
    ddv = torch.empty(E, 3, device=cuda); dd = torch.empty(E, device=cuda)
    nb = int(_lib.load().e2v2_deg_bwd_workspace(E))
    ws = torch.empty(nb, dtype=torch.uint8, device=cuda)
    _lib.call("e2v2_deg_bwd", _lib.C.byref(a), _lib.vp(Gd.data_ptr()), _lib.vp(ddv.data_ptr()),
              _lib.vp(dd.data_ptr()), _lib.vp(ws.data_ptr()), _lib.C.c_size_t(nb), st)
    errs = dict(fwd=relerr(x0.permute(1, 0, 2), ref), dvec=relerr(ddv, grads[0]), dist=relerr(dd, grads[1]))
    print(f"[deg] {errs}", flush=True)
    assert errs["fwd"] < 2e-5
    for k_, e in errs.items():
        assert e < 1e-4, (k_, e)


def test_degree_hidden_table_forward_backward(pkg, cuda):
    """Degree embedding through the profiles' hidden channels (layout "degh":
    kernel sums of the interpolated hidden channels, then the per-node split GEMM
    with [W3 | b3], and in the backward the transposed GEMM and the bias column's
    gradient) via ops.DegreeEmbedFn, against the float64 per-edge profiles; and
    against the output-table kernels ("deg") on the same graph.  The hidden table
    meets the output tolerances (1e-6 value, 1e-5 derivative) through its check."""
    from ubio_molfm_amd import _lib, modules, ops
    s, pos, nl = _graph(pkg, cuda, seed=5)
    N, E = nl.n_atoms, nl.n_edges
    rb = modules.GaussianSmearing(256, 6.0, 2.0)
    profs = [_profile(20 + l, 768) for l in range(3)]
    tgt, src = _embeddings(23, 300, 256)
    nets64 = [copy.deepcopy(p_).double().net for p_ in profs]
    assert all(float(n[6].bias.abs().max()) > 1e-3 for n in nets64)   # the bias column carries a term
    tw, sw = tgt.weight.detach().double().clone(), src.weight.detach().double().clone()
    type_z, slot = _types(pkg, cuda, s["Z"])
    nets = [p_.to(cuda).net for p_ in profs]
    tabh = ops.RadialTable(nets, tgt.to(cuda), src.to(cuda), rb.offset.to(cuda), rb.coeff, 6.0, type_z,
                           layout="degh")
    assert tabh.nc == 384 and tabh.value_err <= 1e-6 and tabh.deriv_err <= 1e-5, (tabh.value_err, tabh.deriv_err)
    row = nl.edge_row.long().cpu(); col = nl.col.long().cpu()
    Z = torch.as_tensor(np.asarray(s["Z"]))
    leaves = [nl.dvec.cpu().double().requires_grad_(True), nl.dist.cpu().double().requires_grad_(True)]
    coeff = float(np.float32(rb.coeff))
    fea = torch.cat([mlp_ref(leaves[1], Z[row], Z[col], n64, tw, sw, rb.offset.double(), coeff) for n64 in nets64],
                    dim=-1)
    ref = deg_ref(leaves[0], leaves[1], row, fea, 23.01, 6.0, N)
    G = torch.randn(N, 9, 256, generator=torch.Generator().manual_seed(9))
    grads = torch.autograd.grad((ref * G.double()).sum(), leaves)
    outs = {}
    for lay, tab in (("degh", tabh), ("deg", ops.RadialTable(nets, tgt.to(cuda), src.to(cuda), rb.offset.to(cuda),
                                                              rb.coeff, 6.0, type_z, layout="deg"))):
        dvec = nl.dvec.clone().requires_grad_(True); dist = nl.dist.clone().requires_grad_(True)
        x0 = ops.DegreeEmbedFn.apply(dvec, dist, nl, slot, tab, 23.01, 6.0)
        x0.backward(G.permute(1, 0, 2).contiguous().to(cuda))
        outs[lay] = (x0.detach().permute(1, 0, 2), dvec.grad, dist.grad)
        errs = dict(fwd=relerr(outs[lay][0], ref), dvec=relerr(dvec.grad, grads[0]), dist=relerr(dist.grad, grads[1]))
        print(f"[deg {lay}] E={E} {errs}", flush=True)
        assert errs["fwd"] < 2e-5, (lay, errs)
        for k_, e in errs.items():
            assert e < 1e-4, (lay, k_, e)
    cross = [relerr(a_, b_.double().cpu()) for a_, b_ in zip(outs["degh"], outs["deg"])]
    print(f"[deg degh vs deg] {cross}", flush=True)
    assert max(cross) < 1e-4, cross


def test_morton_keys(pkg, cuda):
    """e2v2_morton_keys against a numpy restatement (fp32 quantisation, 10-bit
    interleave), one graph and a ragged batch of three graphs."""
    from ubio_molfm_amd import _lib

    def spread(v):
        v = v.astype(np.uint64) & np.uint64(0x3FF)
        for sh, mask in ((16, 0x030000FF), (8, 0x0300F00F), (4, 0x030C30C3), (2, 0x09249249)):
            v = (v | (v << np.uint64(sh))) & np.uint64(mask)
        return v

    rng = np.random.default_rng(3)
    for counts in ([500], [7, 300, 41]):
        n = sum(counts)
        pos = (rng.normal(size=(n, 3)) * 5).astype(np.float32)
        gid = np.repeat(np.arange(len(counts)), counts).astype(np.int32)
        lo = np.stack([pos[gid == g].min(0) for g in range(len(counts))]).astype(np.float32)
        hi = np.stack([pos[gid == g].max(0) for g in range(len(counts))]).astype(np.float32)
        span = np.maximum(hi - lo, np.float32(1e-6)).astype(np.float32)
        u = (pos - lo[gid]) / span[gid] * np.float32(1023.0)
        q = np.clip(u, 0, 1023).astype(np.int64)
        ref = (gid.astype(np.uint64) << np.uint64(32)) | spread(q[:, 0]) | (spread(q[:, 1]) << np.uint64(1)) \
            | (spread(q[:, 2]) << np.uint64(2))
        t = lambda a: torch.as_tensor(np.ascontiguousarray(a), device=cuda)
        pd, gd, ld, sd = t(pos), t(gid), t(lo), t(span)
        key = torch.empty(n, dtype=torch.int64, device=cuda)
        _lib.call("e2v2_morton_keys", _lib.vp(pd.data_ptr()), None if len(counts) == 1 else _lib.vp(gd.data_ptr()),
                  _lib.vp(ld.data_ptr()), _lib.vp(sd.data_ptr()), _lib.i32(n), _lib.vp(key.data_ptr()),
                  _lib.vp(torch.cuda.current_stream().cuda_stream))
        got = key.cpu().numpy().view(np.uint64)
        assert np.array_equal(got, ref), (counts, int((got != ref).sum()))


def test_edge_to_pos(pkg, cuda):
    from ubio_molfm_amd import _lib
    s, pos, nl = _graph(pkg, cuda, seed=6)
    N, E = nl.n_atoms, nl.n_edges
    g = torch.Generator().manual_seed(1)
    gdv = torch.randn(E, 3, generator=g); gd = torch.randn(E, generator=g)
    out = torch.empty(N, 3, device=cuda)
    gdv_d, gd_d = gdv.to(cuda), gd.to(cuda)   # held until the kernel has run
    _lib.call("e2v2_edge_to_pos", _lib.i32(N), _lib.vp(nl.row_ptr.data_ptr()), _lib.vp(nl.key_ptr.data_ptr()),
              _lib.vp(nl.key_eid.data_ptr()), _lib.vp(nl.dvec.data_ptr()), _lib.vp(nl.dist.data_ptr()),
              _lib.vp(gdv_d.data_ptr()), _lib.vp(gd_d.data_ptr()), _lib.vp(out.data_ptr()),
              _lib.vp(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    p64 = torch.as_tensor(s["pos"], dtype=torch.float64).requires_grad_(True)
    off = torch.as_tensor((nl.shifts.numpy()[nl.shift_idx.cpu().numpy()] @ s["cell"][0].astype(np.float64)))
    row = nl.edge_row.long().cpu(); col = nl.col.long().cpu()
    dv = p64[row] - (p64[col] + off)
    d = dv.norm(dim=-1)
    ref = torch.autograd.grad((dv * gdv.double()).sum() + (d * gd.double()).sum(), p64)[0]
    e = relerr(out, ref)
    print(f"[pos] rel {e:.2e}", flush=True)
    assert e < 1e-5


@pytest.mark.parametrize("n,w", [(37, 512), (8, 128), (1, 1024)])
def test_ln_silu(pkg, cuda, n, w):
    """LayerNorm + SiLU of the Q/K head (LNSiLUFn) against float64 torch: forward
    and input gradient within 2e-6 relative; rows not a multiple of the four
    rows per workgroup."""
    from ubio_molfm_amd import modules
    torch.manual_seed(3)
    x = torch.randn(n, w, dtype=torch.float64) * 2.0 + 0.5
    ln = torch.nn.LayerNorm(w).double()
    ln.weight.data.uniform_(0.5, 1.5); ln.bias.data.uniform_(-0.3, 0.3)
    xl = x.clone().requires_grad_(True)
    yr = torch.nn.functional.silu(ln(xl))
    G = torch.randn_like(yr)
    gr = torch.autograd.grad((yr * G).sum(), xl)[0]
    lnd = torch.nn.LayerNorm(w).to(cuda)
    lnd.load_state_dict({k: v.float() for k, v in ln.state_dict().items()})
    xd = x.float().to(cuda).requires_grad_(True)
    yd = modules._ln_silu(xd, lnd)
    gd = torch.autograd.grad((yd * G.float().to(cuda)).sum(), xd)[0]
    ef, eb = relerr(yd, yr), relerr(gd, gr)
    print(f"[ln-silu {n}x{w}] fwd {ef:.2e} bwd {eb:.2e}", flush=True)
    assert ef < 2e-6 and eb < 2e-6


def test_node_kernels_rmsnorm_gate(pkg, cuda):
    """HIP rms_norm_sh and Gate_s3 (m-major) vs the oracle's torch modules."""
    from ubio_molfm_amd import modules
    from oracle.model import EquivariantRMSNormArraySphericalHarmonicsV2_BL as RefNorm, Gate_s3 as RefGate
    torch.manual_seed(4)
    N = 37
    x = torch.randn(N, 9, 256, dtype=torch.float64)
    ref_norm = RefNorm(2, 256).double()
    ref_norm.affine_weight.data.uniform_(0.5, 1.5); ref_norm.affine_bias.data.uniform_(-0.3, 0.3)
    xl = x.clone().requires_grad_(True)
    yr = ref_norm(xl)
    G = torch.randn_like(yr)
    gr = torch.autograd.grad((yr * G).sum(), xl)[0]
    norm = modules.EquivariantRMSNormArraySphericalHarmonicsV2_BL(2, 256).to(cuda)
    norm.load_state_dict({k: v.float() for k, v in ref_norm.state_dict().items()})
    xd = x.permute(1, 0, 2).float().contiguous().to(cuda).requires_grad_(True)
    yd = norm(xd)
    gd = torch.autograd.grad((yd * G.permute(1, 0, 2).float().to(cuda)).sum(), xd)[0]
    e1, e2 = relerr(yd.permute(1, 0, 2), yr), relerr(gd.permute(1, 0, 2), gr)
    ref_gate = RefGate(256, 2).double()
    gate = modules.Gate_s3(256, 2).to(cuda)
    gate.load_state_dict({k: v.float() for k, v in ref_gate.state_dict().items()})
    xl = x.clone().requires_grad_(True)
    yr = ref_gate(xl)
    gr = torch.autograd.grad((yr * G).sum(), xl)[0]
    xd = x.permute(1, 0, 2).float().contiguous().to(cuda).requires_grad_(True)
    yd = gate(xd)
    gd = torch.autograd.grad((yd * G.permute(1, 0, 2).float().to(cuda)).sum(), xd)[0]
    e3, e4 = relerr(yd.permute(1, 0, 2), yr), relerr(gd.permute(1, 0, 2), gr)
    print(f"[node] rms fwd {e1:.2e} bwd {e2:.2e} gate fwd {e3:.2e} bwd {e4:.2e}", flush=True)
    assert max(e1, e3) < 2e-6 and max(e2, e4) < 1e-5


@pytest.mark.parametrize("n,with_v,with_bias", [(1, True, True), (200, False, True), (1000, True, False)])
def test_qk_proj_fused(pkg, cuda, n, with_v, with_bias):
    """Fused Q/K projection + m-contraction (forward) and its input gradient with the
    value projection's gradient folded in (backward) against float64 GEMMs."""
    from ubio_molfm_amd import _lib
    torch.manual_seed(7)
    hid, C, Cv = 512, 256, 256
    print(f"[qk_proj] n={n} with_v={with_v} bias={with_bias}", flush=True)
    idx = torch.tensor([0, 1, 1, 1, 2, 2, 2, 2, 2], device=cuda)
    x = torch.randn(9, n, C, device=cuda)
    W = torch.randn(3, 4 * hid, C, device=cuda) / 16
    bias = torch.randn(4 * hid, device=cuda) if with_bias else None
    Wv = torch.randn(3, Cv, C, device=cuda) / 16
    Wt = W[idx].transpose(1, 2).contiguous()
    Wvt = Wv[idx].transpose(1, 2).contiguous()
    y = torch.empty(9, n, 4 * hid, device=cuda)
    hq = torch.empty(n, 3 * hid, device=cuda); hk = torch.empty_like(hq)
    st = _lib.vp(torch.cuda.current_stream().cuda_stream)
    p = lambda t: _lib.vp(t.data_ptr() if t is not None else 0)
    _lib.call("e2v2_qk_proj_fwd", p(x), p(W), p(bias), p(y), p(hq), p(hk), _lib.i32(n), _lib.i32(hid),
              _lib.i32(C), st)
    # float64 reference: per-m GEMM with the degree's weight, bias on m = 0, then the per-l pair sums
    yd = torch.bmm(x.double(), Wt.double())
    if with_bias:
        yd[0] += bias.double()
    a_q, b_q, a_k, b_k = yd.split(hid, dim=2)
    L = [slice(0, 1), slice(1, 4), slice(4, 9)]
    hqd = torch.cat([(a_q[s] * b_q[s]).sum(0) for s in L], dim=1)
    hkd = torch.cat([(a_k[s] * b_k[s]).sum(0) for s in L], dim=1)
    e_y, e_q, e_k = relerr(y, yd), relerr(hq, hqd), relerr(hk, hkd)
    ghq = torch.randn(n, 3 * hid, device=cuda); ghk = torch.randn(n, 3 * hid, device=cuda)
    gv = torch.randn(9, n, Cv, device=cuda) if with_v else None
    gx = torch.empty(9, n, C, device=cuda)
    _lib.call("e2v2_qk_proj_bwd", p(y), p(ghq), p(ghk), p(Wt), p(gv), p(Wvt if with_v else None), p(gx),
              _lib.i32(n), _lib.i32(hid), _lib.i32(C), _lib.i32(Cv if with_v else 0), st)
    # reference gradient: autograd through the float64 forward
    xd = x.double().requires_grad_(True)
    yr = torch.bmm(xd, Wt.double())
    if with_bias:
        shift = torch.zeros(9, 1, 4 * hid, device=cuda, dtype=torch.float64)
        shift[0, 0] = bias.double()
        yr = yr + shift
    aq, bq, ak, bk = yr.split(hid, dim=2)
    hq_r = torch.cat([(aq[s] * bq[s]).sum(0) for s in L], dim=1)
    hk_r = torch.cat([(ak[s] * bk[s]).sum(0) for s in L], dim=1)
    obj = (hq_r * ghq.double()).sum() + (hk_r * ghk.double()).sum()
    if with_v:
        obj = obj + (torch.bmm(xd, Wvt.double()) * gv.double()).sum()
    gxd, = torch.autograd.grad(obj, xd)
    e_g = relerr(gx, gxd)
    print(f"[qk_proj] n={n} y {e_y:.2e} hq {e_q:.2e} hk {e_k:.2e} gx {e_g:.2e}", flush=True)
    assert e_y < 2e-5 and e_q < 2e-5 and e_k < 2e-5
    assert e_g < 1e-4


@pytest.mark.parametrize("n,with_v", [(1, True), (300, False), (1000, True)])
def test_qk_proj_fused_bf16(pkg, cuda, n, with_v):
    """bf16-operand form of the fused projection against float64 GEMMs of the
    bf16-rounded operands.  Tolerances: y is stored in bf16 (2^-9 relative, test
    4e-3); hq / hk come from the fp32 accumulators (1e-4); the backward rounds its
    formed gradient operand to bf16 (1e-2)."""
    from ubio_molfm_amd import _lib
    torch.manual_seed(11)
    hid, C, Cv = 512, 256, 256
    print(f"[qk_proj bf16] n={n} with_v={with_v}", flush=True)
    bf = torch.bfloat16
    x = torch.randn(9, n, C, device=cuda)
    W = (torch.randn(3, 4 * hid, C, device=cuda) / 16).to(bf)
    Wv = (torch.randn(3, Cv, C, device=cuda) / 16).to(bf)
    bias = torch.randn(4 * hid, device=cuda)
    Wt = W.transpose(1, 2).contiguous(); Wvt = Wv.transpose(1, 2).contiguous()
    y = torch.empty(9, n, 4 * hid, device=cuda, dtype=bf)
    hq = torch.empty(n, 3 * hid, device=cuda); hk = torch.empty_like(hq)
    st = _lib.vp(torch.cuda.current_stream().cuda_stream)
    p = lambda t: _lib.vp(t.data_ptr() if t is not None else 0)
    _lib.call("e2v2_qk_proj_fwd_bf16", p(x), p(W), p(bias), p(y), p(hq), p(hk), _lib.i32(n), _lib.i32(hid),
              _lib.i32(C), st)
    idx = torch.tensor([0, 1, 1, 1, 2, 2, 2, 2, 2], device=cuda)
    xr = x.to(bf).double()
    yd = torch.bmm(xr, Wt.double()[idx])
    yd[0] += bias.double()
    L = [slice(0, 1), slice(1, 4), slice(4, 9)]
    a_q, b_q, a_k, b_k = yd.split(hid, dim=2)
    hqd = torch.cat([(a_q[s] * b_q[s]).sum(0) for s in L], dim=1)
    hkd = torch.cat([(a_k[s] * b_k[s]).sum(0) for s in L], dim=1)
    e_y, e_q, e_k = relerr(y.float(), yd), relerr(hq, hqd), relerr(hk, hkd)
    ghq = torch.randn(n, 3 * hid, device=cuda); ghk = torch.randn(n, 3 * hid, device=cuda)
    gv = torch.randn(9, n, Cv, device=cuda) if with_v else None
    gx = torch.empty(9, n, C, device=cuda)
    _lib.call("e2v2_qk_proj_bwd_bf16", p(y), p(ghq), p(ghk), p(Wt), p(gv), p(Wvt if with_v else None), p(gx),
              _lib.i32(n), _lib.i32(hid), _lib.i32(C), _lib.i32(Cv if with_v else 0), st)
    yy = y.double()
    gyd = torch.empty_like(yy)
    gq3 = ghq.double().view(n, 3, hid); gk3 = ghk.double().view(n, 3, hid)
    for m in range(9):
        l = 0 if m == 0 else (1 if m < 4 else 2)
        gyd[m, :, :hid] = gq3[:, l] * yy[m, :, hid:2 * hid]
        gyd[m, :, hid:2 * hid] = gq3[:, l] * yy[m, :, :hid]
        gyd[m, :, 2 * hid:3 * hid] = gk3[:, l] * yy[m, :, 3 * hid:]
        gyd[m, :, 3 * hid:] = gk3[:, l] * yy[m, :, 2 * hid:3 * hid]
    gxd = torch.bmm(gyd, W.double()[idx])
    if with_v:
        gxd = gxd + torch.bmm(gv.to(bf).double(), Wv.double()[idx])
    e_g = relerr(gx, gxd)
    print(f"[qk_proj bf16] n={n} y {e_y:.2e} hq {e_q:.2e} hk {e_k:.2e} gx {e_g:.2e}", flush=True)
    assert e_y < 4e-3 and e_q < 1e-4 and e_k < 1e-4
    assert e_g < 1e-2
