"""GPU parity of each HIP operator against its plain-PyTorch float64 reference.

Tolerances: fp32 kernels vs float64 references, relative to the output scale:
forward 2e-5, input gradients 1e-4 (fp32 accumulation over ~100-edge rows).
"""
import math

import numpy as np
import pytest
import torch

from op_reference import attn_ref, deg_ref, mlp_ref, mlp_ref_bf16

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


def test_mlp_forward_backward(pkg, cuda):
    from ubio_molfm_amd import modules, ops
    torch.manual_seed(1)
    s, pos, nl = _graph(pkg, cuda)
    E, N = nl.n_edges, nl.n_atoms
    print(f"[mlp] N={N} E={E}", flush=True)
    prof = modules.RadialProfile([768, 128, 128, 256])
    for m in prof.modules():
        if isinstance(m, torch.nn.LayerNorm):
            m.weight.data.uniform_(0.5, 1.5); m.bias.data.uniform_(-0.2, 0.2)
    tgt = torch.nn.Embedding(300, 256); src = torch.nn.Embedding(300, 256)
    rb = modules.GaussianSmearing(256, 6.0, 2.0)
    Z = torch.as_tensor(s["Z"], device=cuda).to(torch.int32)
    packed = [ops.PackedMLP(prof.to(cuda).net, tgt.weight.to(cuda), src.weight.to(cuda), rb.offset.to(cuda),
                            rb.coeff, 6.0)]
    sn, sr = ops.mlp_save_buffers(1, E, cuda)
    args = ops.mlp_args(nl, Z, packed, sn, sr)
    out = torch.empty(E, 256, device=cuda)
    from ubio_molfm_amd import _lib
    _lib.call("e2v2_mlp_fwd", _lib.C.byref(args), _lib.vp(out.data_ptr()), _lib.i32(256),
              _lib.vp(torch.cuda.current_stream().cuda_stream))
    d64 = nl.dist.double().cpu().requires_grad_(True)
    zi = torch.as_tensor(s["Z"])[nl.edge_row.long().cpu()]
    zj = torch.as_tensor(s["Z"])[nl.col.long().cpu()]
    net64 = prof.cpu().double().net
    ref = mlp_ref(d64, zi, zj, net64, tgt.weight.double(), src.weight.double(), rb.offset.double(), rb.coeff)
    e_f = relerr(out, ref)
    dout = torch.randn(E, 256, device=cuda)
    dd = torch.empty(E, device=cuda)
    _lib.call("e2v2_mlp_bwd", _lib.C.byref(args), _lib.vp(dout.data_ptr()), _lib.i32(256), _lib.vp(dd.data_ptr()),
              _lib.i32(0), _lib.vp(torch.cuda.current_stream().cuda_stream))
    g = torch.autograd.grad((ref * dout.double().cpu()).sum(), d64)[0]
    e_b = relerr(dd, g)
    print(f"[mlp] fwd rel {e_f:.2e} bwd rel {e_b:.2e}", flush=True)
    assert e_f < 2e-5 and e_b < 1e-4


def test_mlp_bf16_forward_backward(pkg, cuda):
    """bf16-operand edge MLP.  Against a float64 restatement that rounds at the
    kernel's rounding points: forward 3e-4, backward 1e-3 relative (fp32 and
    float64 values on either side of a bf16 rounding boundary round apart).  Against the
    plain float64 MLP (the whole bf16 error): forward and backward within 2e-2."""
    from ubio_molfm_amd import _lib, modules, ops
    torch.manual_seed(11)
    s, pos, nl = _graph(pkg, cuda, seed=5)
    E, N = nl.n_edges, nl.n_atoms
    print(f"[mlp-bf16] N={N} E={E}", flush=True)
    prof = modules.RadialProfile([768, 128, 128, 256])
    for m in prof.modules():
        if isinstance(m, torch.nn.LayerNorm):
            m.weight.data.uniform_(0.5, 1.5); m.bias.data.uniform_(-0.2, 0.2)
    tgt = torch.nn.Embedding(300, 256); src = torch.nn.Embedding(300, 256)
    rb = modules.GaussianSmearing(256, 6.0, 2.0)
    Z = torch.as_tensor(s["Z"], device=cuda).to(torch.int32)
    packed = [ops.PackedMLP(prof.to(cuda).net, tgt.weight.to(cuda), src.weight.to(cuda), rb.offset.to(cuda),
                            rb.coeff, 6.0, bf16=True)]
    sn, sr = ops.mlp_save_buffers(1, E, cuda)
    args = ops.mlp_args(nl, Z, packed, sn, sr)
    assert args.compute_bf16 == 1
    st = _lib.vp(torch.cuda.current_stream().cuda_stream)
    out = torch.empty(E, 256, device=cuda)
    _lib.call("e2v2_mlp_fwd", _lib.C.byref(args), _lib.vp(out.data_ptr()), _lib.i32(256), st)
    dout = torch.randn(E, 256, device=cuda)
    dd = torch.empty(E, device=cuda)
    _lib.call("e2v2_mlp_bwd", _lib.C.byref(args), _lib.vp(dout.data_ptr()), _lib.i32(256), _lib.vp(dd.data_ptr()),
              _lib.i32(0), st)
    zi = torch.as_tensor(s["Z"])[nl.edge_row.long().cpu()]
    zj = torch.as_tensor(s["Z"])[nl.col.long().cpu()]
    net64 = prof.cpu().double().net
    errs = {}
    for name, fn in (("emulated", mlp_ref_bf16), ("fp64", mlp_ref)):
        d64 = nl.dist.double().cpu().requires_grad_(True)
        ref = fn(d64, zi, zj, net64, tgt.weight.double(), src.weight.double(), rb.offset.double(), rb.coeff)
        g = torch.autograd.grad((ref * dout.double().cpu()).sum(), d64)[0]
        errs[name] = (relerr(out, ref), relerr(dd, g))
    print(f"[mlp-bf16] vs emulated fwd {errs['emulated'][0]:.2e} bwd {errs['emulated'][1]:.2e}; "
          f"vs fp64 fwd {errs['fp64'][0]:.2e} bwd {errs['fp64'][1]:.2e}", flush=True)
    assert errs["emulated"][0] < 3e-4 and errs["emulated"][1] < 1e-3
    assert errs["fp64"][0] < 2e-2 and errs["fp64"][1] < 2e-2


def _attn_inputs(nl, cuda, seed=2):
    g = torch.Generator().manual_seed(seed)
    N, E = nl.n_atoms, nl.n_edges
    q = torch.randn(N, 128, 8, generator=g); k = torch.randn(N, 128, 8, generator=g)
    v = torch.randn(N, 9, 256, generator=g)
    gi = torch.randn(E, 256, generator=g)
    return q, k, v, gi


def _hermite5(t):
    t2, t3, t4, t5 = t * t, t ** 3, t ** 4, t ** 5
    return (1 - 10 * t3 + 15 * t4 - 6 * t5, t - 6 * t3 + 8 * t4 - 3 * t5, 0.5 * (t2 - 3 * t3 + 3 * t4 - t5),
            10 * t3 - 15 * t4 + 6 * t5, -4 * t3 + 7 * t4 - 3 * t5, 0.5 * (t3 - 2 * t4 + t5))


def test_rbf_block_table(pkg, cuda):
    """The tabulated rbf block of Linear1 against its float64 closed form: node
    values and scaled derivatives (to fp32 rounding), and the quintic Hermite
    interpolant of the value and of the first derivative at 4000 random
    distances in [0, rc] (evaluated here in float64 from the fp32 table, with
    the kernel's interval arithmetic) -- relative to the function's scale."""
    from ubio_molfm_amd import _lib, modules, ops
    rc = 6.0
    rb = modules.GaussianSmearing(256, rc, 2.0)
    torch.manual_seed(5)
    W1 = (torch.rand(128, 512) - 0.5) * 0.1
    n, h = ops.rbf_table_size(rc, rb.coeff)
    assert h == 2.0 ** round(math.log2(h)) and n == math.floor(rc / h) + 2
    tab = torch.empty(n, 4, 128, device=cuda)
    W1d, mu = W1.to(cuda).contiguous(), rb.offset.to(cuda).contiguous()
    _lib.call("e2v2_mlp_rbf_table", _lib.vp(W1d.data_ptr()), _lib.i32(512), _lib.vp(mu.data_ptr()),
              _lib.f32(rb.coeff), _lib.i32(n), _lib.f32(h), _lib.vp(tab.data_ptr()),
              _lib.vp(torch.cuda.current_stream().cuda_stream))
    T = tab.cpu().double().numpy()
    c = float(np.float32(rb.coeff))
    Wr = W1[:, :256].double().numpy()
    m = rb.offset.double().numpy()

    def exact(d):
        x = d[:, None] - m[None, :]
        r = np.exp(c * x * x)
        return r @ Wr.T, (2 * c * x * r) @ Wr.T, ((2 * c + 4 * c * c * x * x) * r) @ Wr.T, \
            ((12 * c * c * x + 8 * c ** 3 * x ** 3) * r) @ Wr.T
    dn = np.arange(n) * h
    f0, f1, f2, f3 = exact(dn)
    scale = np.abs(f0).max()
    for k, (fk, hk) in enumerate([(f0, 1), (f1, h), (f2, h * h), (f3, h ** 3)]):
        err = np.abs(T[:, k, :] - fk * hk).max() / np.abs(fk * hk).max()
        assert err < 1e-6, (k, err)
    rng = np.random.default_rng(0)
    d = np.concatenate([rng.uniform(0, rc, 3998), [0.0, rc]]).astype(np.float32)
    u = np.minimum(d.astype(np.float32) * np.float32(1.0 / h), np.float32(n - 2))
    nn_ = np.floor(u).astype(np.int64)
    t = (u - nn_).astype(np.float64)
    H = _hermite5(t[:, None])
    val = (H[0] * T[nn_, 0] + H[1] * T[nn_, 1] + H[2] * T[nn_, 2] + H[3] * T[nn_ + 1, 0] + H[4] * T[nn_ + 1, 1]
           + H[5] * T[nn_ + 1, 2])
    der = (H[0] * T[nn_, 1] + H[1] * T[nn_, 2] + H[2] * T[nn_, 3] + H[3] * T[nn_ + 1, 1] + H[4] * T[nn_ + 1, 2]
           + H[5] * T[nn_ + 1, 3]) / h
    e0, e1, _, _ = exact(d.astype(np.float64))
    ev = np.abs(val - e0).max() / scale
    ed = np.abs(der - e1).max() / np.abs(e1).max()
    print(f"[rbf table] n={n} h={h} value {ev:.2e} derivative {ed:.2e}", flush=True)
    assert ev < 1e-6 and ed < 1e-6


def _attention_case(pkg, cuda, act_dtype, clusters=True, graph=None):
    """Attention fwd + bwd through the C ABI against the float64 reference.  With
    bf16 storage the inputs (q, k, v, grad) are rounded to bf16 for both sides,
    so the remaining differences are the bf16 output rows (also used by the
    backward's D_h) and fp32 arithmetic."""
    from ubio_molfm_amd import _lib, ops, so3
    s, pos, nl = graph if graph is not None else _graph(pkg, cuda, seed=4)
    N, E = nl.n_atoms, nl.n_edges
    bf = act_dtype == torch.bfloat16
    print(f"[attn {act_dtype}] N={N} E={E}", flush=True)
    q, k, v, gi = _attn_inputs(nl, cuda)
    G = torch.randn(N, 20, 256, generator=torch.Generator().manual_seed(7))
    if bf:
        q, k, v, G = (t.to(torch.bfloat16).float() for t in (q, k, v, G))
    st = _lib.vp(torch.cuda.current_stream().cuda_stream)
    qd, kd = (t.to(cuda).to(act_dtype).contiguous() for t in (q, k))
    gid = gi.to(cuda).contiguous()
    vd = v.permute(1, 0, 2).contiguous().to(cuda).to(act_dtype)        # m-major [9, N, C]
    args = ops.attn_args(nl, qd, kd, vd, gid, math.sqrt(8.0), 6.0, int(bf))
    if not clusters:
        args.col_slot_member = args.col_slot_edge = args.col_n_slots = None
    out = torch.empty(20, N, 256, device=cuda, dtype=act_dtype); m = torch.empty(N, 128, device=cuda)
    sr = torch.empty(N, 128, device=cuda); cnt = torch.empty(N, 128, dtype=torch.int32, device=cuda)
    _lib.call("e2v2_attn_fwd", _lib.C.byref(args), _lib.vp(out.data_ptr()), _lib.vp(m.data_ptr()),
              _lib.vp(sr.data_ptr()), _lib.vp(cnt.data_ptr()), st)
    T = torch.as_tensor(so3.cartesian_tp_table())
    row = nl.edge_row.long().cpu(); col = nl.col.long().cpu()
    leaves = [t.double().requires_grad_(True) for t in (q, k, v, nl.dvec.cpu(), nl.dist.cpu(), gi)]
    ref = attn_ref(*leaves[:5], row, col, leaves[5], T, 6.0, N)
    e_f = relerr(out.float().permute(1, 0, 2), ref)
    grads = torch.autograd.grad((ref * G.double()).sum(), leaves)
    Gd = G.permute(1, 0, 2).contiguous().to(cuda).to(act_dtype)
    f = dict(device=cuda)
    dgi = torch.empty(E, 256, **f); ddv = torch.empty(E, 3, **f); dd = torch.empty(E, **f)
    dq = torch.empty(qd.shape, **f); dk = torch.empty(kd.shape, **f); dv = torch.empty(vd.shape, **f)
    we = torch.empty(E, 128, **f); dqk = torch.empty(E, 128, **f)
    _lib.call("e2v2_attn_bwd", _lib.C.byref(args), _lib.vp(Gd.data_ptr()), _lib.vp(out.data_ptr()),
              _lib.vp(m.data_ptr()), _lib.vp(sr.data_ptr()), _lib.vp(cnt.data_ptr()), _lib.vp(dgi.data_ptr()),
              _lib.vp(ddv.data_ptr()), _lib.vp(dd.data_ptr()), _lib.vp(dq.data_ptr()), _lib.vp(dk.data_ptr()),
              _lib.vp(dv.data_ptr()), _lib.vp(we.data_ptr()), _lib.vp(dqk.data_ptr()), st)
    errs = dict(q=relerr(dq, grads[0]), k=relerr(dk, grads[1]), v=relerr(dv.permute(1, 0, 2), grads[2]),
                dvec=relerr(ddv, grads[3]),
                dist=relerr(dd, grads[4]), gi=relerr(dgi, grads[5]))
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


def test_degree_forward_backward(pkg, cuda):
    from ubio_molfm_amd import _lib, ops
    s, pos, nl = _graph(pkg, cuda, seed=5)
    N, E = nl.n_atoms, nl.n_edges
    fea = torch.randn(E, 768, generator=torch.Generator().manual_seed(3))
    feaD = fea.to(cuda)
    st = _lib.vp(torch.cuda.current_stream().cuda_stream)
    a = _lib.DegArgs(N, E, 256, nl.row_ptr.data_ptr(), nl.dvec.data_ptr(), nl.dist.data_ptr(), feaD.data_ptr(),
                     23.01, 6.0, ops.ENV_A, ops.ENV_B, ops.ENV_C)
    x0 = torch.empty(9, N, 256, device=cuda)
    _lib.call("e2v2_deg_fwd", _lib.C.byref(a), _lib.vp(x0.data_ptr()), st)
    row = nl.edge_row.long().cpu()
    leaves = [nl.dvec.cpu().double().requires_grad_(True), nl.dist.cpu().double().requires_grad_(True),
              fea.double().requires_grad_(True)]
    ref = deg_ref(leaves[0], leaves[1], row, leaves[2], 23.01, 6.0, N)
    G = torch.randn(N, 9, 256, generator=torch.Generator().manual_seed(9))
    grads = torch.autograd.grad((ref * G.double()).sum(), leaves)
    Gd = G.permute(1, 0, 2).contiguous().to(cuda)
    dfea = torch.empty_like(feaD); ddv = torch.empty(E, 3, device=cuda); dd = torch.empty(E, device=cuda)
    _lib.call("e2v2_deg_bwd", _lib.C.byref(a), _lib.vp(Gd.data_ptr()), _lib.vp(dfea.data_ptr()),
              _lib.vp(ddv.data_ptr()), _lib.vp(dd.data_ptr()), st)
    errs = dict(fwd=relerr(x0.permute(1, 0, 2), ref), dvec=relerr(ddv, grads[0]), dist=relerr(dd, grads[1]), fea=relerr(dfea, grads[2]))
    print(f"[deg] {errs}", flush=True)
    assert errs["fwd"] < 2e-5
    for k_, e in errs.items():
        assert e < 1e-4, (k_, e)


@pytest.mark.parametrize("bf16", [False, True], ids=["fp32", "bf16"])
def test_degree_mlp_backward_fused(pkg, cuda, bf16):
    """e2v2_mlp_bwd_deg (dOut formed per edge tile from the node gradient) against
    the stored-gradient path e2v2_deg_bwd(dfea) + e2v2_mlp_bwd(dfea) on the three
    l-profiles of the degree embedding; e2v2_deg_bwd without dfea leaves ddvec and
    ddist unchanged.  The two paths round p/avg at different points: fp32 within
    1e-5, bf16 (dOut rounded to bf16 in the tile) within 2e-3."""
    from ubio_molfm_amd import _lib, modules, ops
    torch.manual_seed(5)
    s, pos, nl = _graph(pkg, cuda, seed=8)
    E, N = nl.n_edges, nl.n_atoms
    profs = [modules.RadialProfile([768, 128, 128, 256]) for _ in range(3)]
    for prof in profs:
        for m in prof.modules():
            if isinstance(m, torch.nn.LayerNorm):
                m.weight.data.uniform_(0.5, 1.5); m.bias.data.uniform_(-0.2, 0.2)
    tgt = torch.nn.Embedding(300, 256); src = torch.nn.Embedding(300, 256)
    rb = modules.GaussianSmearing(256, 6.0, 2.0)
    Z = torch.as_tensor(s["Z"], device=cuda).to(torch.int32)
    packed = [ops.PackedMLP(p_.to(cuda).net, tgt.weight.to(cuda), src.weight.to(cuda), rb.offset.to(cuda),
                            rb.coeff, 6.0, bf16=bf16) for p_ in profs]
    sn, sr = ops.mlp_save_buffers(3, E, cuda)
    margs = ops.mlp_args(nl, Z, packed, sn, sr)
    st = _lib.vp(torch.cuda.current_stream().cuda_stream)
    fea = torch.empty(E, 768, device=cuda)
    _lib.call("e2v2_mlp_fwd", _lib.C.byref(margs), _lib.vp(fea.data_ptr()), _lib.i32(768), st)
    dargs = _lib.DegArgs(N, E, 256, nl.row_ptr.data_ptr(), nl.dvec.data_ptr(), nl.dist.data_ptr(), fea.data_ptr(),
                         23.01, 6.0, ops.ENV_A, ops.ENV_B, ops.ENV_C)
    G = torch.randn(9, N, 256, generator=torch.Generator().manual_seed(12)).to(cuda)
    f = dict(device=cuda)
    dfea = torch.empty(E, 768, **f); ddv0 = torch.empty(E, 3, **f); dd0 = torch.empty(E, **f)
    _lib.call("e2v2_deg_bwd", _lib.C.byref(dargs), _lib.vp(G.data_ptr()), _lib.vp(dfea.data_ptr()),
              _lib.vp(ddv0.data_ptr()), _lib.vp(dd0.data_ptr()), st)
    _lib.call("e2v2_mlp_bwd", _lib.C.byref(margs), _lib.vp(dfea.data_ptr()), _lib.i32(768),
              _lib.vp(dd0.data_ptr()), _lib.i32(1), st)
    ddv1 = torch.empty(E, 3, **f); dd1 = torch.empty(E, **f)
    _lib.call("e2v2_deg_bwd", _lib.C.byref(dargs), _lib.vp(G.data_ptr()), None, _lib.vp(ddv1.data_ptr()),
              _lib.vp(dd1.data_ptr()), st)
    _lib.call("e2v2_mlp_bwd_deg", _lib.C.byref(margs), _lib.C.byref(dargs), _lib.vp(G.data_ptr()),
              _lib.vp(dd1.data_ptr()), _lib.i32(1), st)
    e_dd = relerr(dd1, dd0)
    print(f"[deg-mlp {'bf16' if bf16 else 'fp32'}] E={E} ddvec equal {torch.equal(ddv1, ddv0)} dd rel {e_dd:.2e}",
          flush=True)
    assert torch.equal(ddv1, ddv0)
    assert e_dd < (2e-3 if bf16 else 1e-5)


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
