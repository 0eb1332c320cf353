"""The training path (``second_order``): in training mode the backbone's forces
are taken with create_graph=True and differentiated again, as the reference's
force training does (head.py:305-328 with AutoGradForce).  The loss
L = sum F . G + sum e g (random G, g) is differentiated with respect to
parameters of every kind (radial profiles, embeddings, SO(3) linears, the Q/K
projections, the SO(2) output linears, norms, the energy head), compared with
the float64 oracle's double backward on the same state dict, and to the
positions (a Hessian-vector product), compared with central differences of the
oracle's L in float64 along random directions (the oracle's own second
derivative in the positions passes through its Wigner frames, whose double
backward is not finite at every atom).  Gates: energies 1e-5 eV/atom, forces
1e-4 relative L2 (as the eval path), parameter gradients 5e-4 relative L2 per
tensor (fp32 against float64 through two differentiations), directional
position derivatives 1e-3 relative."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

PARAMS = [
    "decoder.decoder.edge_deg_embed_dense.gbf_projs.1.net.0.weight",
    "decoder.decoder.edge_deg_embed_dense.source_embedding.weight",
    "decoder.decoder.blocks.0.ga.fc_easy.net.6.weight",
    "decoder.decoder.blocks.0.ga.query_linear.weight",
    "decoder.decoder.blocks.0.ga.key_linear.final_linear.3.weight",
    "decoder.decoder.blocks.1.ga.proj_value.weight",
    "decoder.decoder.blocks.1.ga.target_embedding.weight",
    "decoder.decoder.blocks.2.ffn.gate.gates.weight",
    "decoder.decoder.blocks.3.norm_1.affine_weight",
    "decoder.decoder.blocks.3.ffn.slinear_2.bias",
    "decoder.decoder.norm_final.affine_bias",
    "head.energy_heads.omol25.mlp.0.weight",
    "decoder.decoder.blocks.0.ga.fc_easy.net.1.weight",
    "decoder.decoder.blocks.2.ga.fc_easy.net.4.bias",
    "decoder.decoder.edge_deg_embed_dense.gbf_projs.0.net.1.bias",
    "decoder.decoder.blocks.1.ga.query_linear.final_linear.1.weight",
]


def _pair(cuda, seed, **cfg):
    from ubio_molfm_amd import model
    from oracle.model import MolfmAtomic as OracleModel
    torch.manual_seed(seed)
    args = model.default_args()
    args.backbone_config.update(cfg)
    m = model.MolfmAtomic(args).to(cuda)
    om = OracleModel(**cfg)
    om.load_state_dict({k: v.cpu() for k, v in m.state_dict().items()}, strict=True)
    # the zero-initialised biases and unit norms would leave some second-order terms at zero
    g = torch.Generator().manual_seed(seed + 100)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if p.requires_grad and ("bias" in name or "affine" in name):
                p.add_(0.05 * torch.randn(p.shape, generator=g).to(cuda))
    om.load_state_dict({k: v.cpu() for k, v in m.state_dict().items()}, strict=True)
    return m.train(), om.double().train()


def _to(bd, dev, dtype):
    return {k: (v.to(dev, dtype) if torch.is_tensor(v) and v.is_floating_point() else
                (v.to(dev) if torch.is_tensor(v) else v)) for k, v in bd.items()}


def _oracle_ef(om, bd, create_graph):
    pos = bd["pos"]
    out = om.decoder(dict(bd))
    e, _ = om.head(out, bd, "omol25")
    f = -torch.autograd.grad(e, pos, torch.ones_like(e), create_graph=create_graph)[0]
    return e, f


def _second_order(m, bd, names, G, ge, dev, dtype, oracle=False):
    """(energy, forces of the real atoms, {name: dL/dparam}, dL/dpos or None) with
    L = sum F . G + sum e ge, forces taken with create_graph=True."""
    bd = _to(bd, dev, dtype)
    pos = bd["pos"].clone().requires_grad_(True)
    bd["pos"] = pos
    mask = bd["atom_masks"]
    if oracle:
        e, f = _oracle_ef(m, bd, True)
    else:
        res = m(bd)
        e, f = res["pred_energy"], res["pred_forces"]
    fr = f[mask]
    loss = (fr * G.to(dev, dtype)).sum() + (e * ge.to(dev, dtype)).sum()
    params = dict(m.named_parameters())
    wrt = [params[n] for n in names] + ([] if oracle else [pos])
    gs = torch.autograd.grad(loss, wrt)
    return e.detach(), fr.detach(), dict(zip(names, gs[:len(names)])), None if oracle else gs[-1][mask]


def _oracle_loss(om, bd, G, ge):
    """L of the oracle at the positions of bd (float64, first order only)."""
    bd = dict(bd)
    bd["pos"] = bd["pos"].clone().requires_grad_(True)
    e, f = _oracle_ef(om, bd, False)
    return float((f[bd["atom_masks"]] * G).sum() + (e.detach() * ge).sum())


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _case(cuda, sysd, seed, label, names=PARAMS, charge=None, **cfg):
    from ubio_molfm_amd import systems
    m, om = _pair(cuda, seed, **cfg)
    bd = systems.to_padded(sysd)
    if charge is not None:
        B = len(sysd["graph_ptr"]) - 1
        bd["charge"] = torch.full((B,), charge[0], dtype=torch.long)
        bd["multiplicity"] = torch.full((B,), charge[1], dtype=torch.long)
    n = int(bd["atom_masks"].sum())
    g = torch.Generator().manual_seed(seed + 7)
    G = torch.randn(n, 3, generator=g, dtype=torch.float64)
    ge = torch.randn(len(sysd["graph_ptr"]) - 1, generator=g, dtype=torch.float64)
    names = [k for k in names if k in dict(m.named_parameters())]
    e, f, gp, gx = _second_order(m, bd, names, G, ge, cuda, torch.float32)
    e0, f0, gp0, _ = _second_order(om, bd, names, G, ge, "cpu", torch.float64, oracle=True)
    natoms = torch.as_tensor(np.diff(sysd["graph_ptr"]), dtype=torch.float64)
    de = float(((e.cpu().double() - e0) / natoms).abs().max())
    errs = {k: _rel(gp[k], gp0[k]) for k in names}
    # dL/dpos along random directions against central differences of the oracle's L
    bd64 = _to(bd, "cpu", torch.float64)
    mask = bd64["atom_masks"]
    h, fd, ad = 1e-4, [], []
    for _ in range(3):
        u = torch.zeros_like(bd64["pos"])
        u[mask] = torch.randn(n, 3, generator=g, dtype=torch.float64)
        lp = _oracle_loss(om, dict(bd64, pos=bd64["pos"] + h * u), G, ge)
        lm = _oracle_loss(om, dict(bd64, pos=bd64["pos"] - h * u), G, ge)
        fd.append((lp - lm) / (2 * h))
        ad.append(float((gx.cpu().double() * u[mask]).sum()))
    errs["pos"] = _rel(torch.tensor(ad), torch.tensor(fd))
    worst = max(errs, key=errs.get)
    print(f"[train {label}] N={n} |dE|/atom={de:.2e} force relL2={_rel(f, f0):.2e} second order: worst "
          f"{worst} {errs[worst]:.2e}, pos {errs['pos']:.2e} (directional {ad} vs {fd})", flush=True)
    assert de < 1e-5 and _rel(f, f0) < 1e-4
    for k in names:
        assert gp0[k].abs().max() > 0, k
        assert errs[k] < 5e-4, (k, errs[k])
    assert errs["pos"] < 1e-3


def test_training_second_order_water(pkg, cuda):
    """Base model (QK_alpha, first-order SO(2) product) on a periodic water cell
    with charge / multiplicity: the shift of each periodic edge is a constant of
    the positions."""
    from ubio_molfm_amd import systems
    _case(cuda, systems.small_water(8, 6.2, seed=21), 31, "water", charge=(1, 2))


def test_training_second_order_variants(pkg, cuda):
    """QKdot_alpha with sigmoid weights and one bell cluster block (zero-order
    aggregation, the long-range list) on a ragged organic batch, plus the
    QKdot gate's own parameters (norm_final is not used with the cluster
    blocks, e2former.py:1088-1117)."""
    from ubio_molfm_amd import systems
    names = [k for k in PARAMS if "norm_final" not in k] + ["decoder.decoder.blocks.0.ga.rad_func_m0.net.3.weight",
                      "decoder.decoder.blocks.0.ga.fc_m0.weight",
                      "decoder.decoder.blocks.0.ga.dot_linear.weight",
                      "decoder.decoder.long_blocks.0.ga.proj_zero.weight",
                      "decoder.decoder.final_linear.weight",
                      "decoder.decoder.norm_cluster.affine_weight"]
    _case(cuda, systems.organics_batch(n_mol=2, nmin=8, nmax=14, seed=22), 32, "qkdot-sigmoid-cluster", names,
          tp_type="QKdot_alpha+sigmoid", with_cluster="node_bell", long_range_layers=1)


def test_training_second_order_qkdots_softplus(pkg, cuda):
    """QKdotS_alpha with softplus weights and zero-order short blocks
    ("so2-first-order+zero-order")."""
    from ubio_molfm_amd import systems
    names = PARAMS + ["decoder.decoder.blocks.1.ga.direction_linear.0.weight",
                      "decoder.decoder.blocks.3.ga.proj_zero.weight"]
    _case(cuda, systems.small_water(6, 5.6, seed=23), 33, "qkdots-softplus", names,
          tp_type="QKdotS_alpha+softplus", attn_type="so2-first-order+zero-order")


@pytest.mark.parametrize("w", [64, 128, 192, 512])
def test_ln_silu_second_order(pkg, cuda, w):
    """ln_silu (the fused LayerNorm + SiLU of the radial nets on the training
    path) against float64 layer_norm + silu: values and the first-order
    gradients of x, g, b (1e-5 relative L2), then the gradients of
    L = <gx, R0> + <dg, R1> + <db, R2> in x, g, b and the upstream gy (every
    term of the second-order pass; 1e-4 relative L2, fp32 against float64
    through two differentiations).  Rows not a multiple of the 4 rows per
    block, more rows than wavefronts (each strides over several)."""
    from ubio_molfm_amd import second_order as so
    torch.manual_seed(w)
    n = 4 * 2048 * 2 + 3 if w == 128 else 997
    ln = torch.nn.LayerNorm(w).to(cuda)
    with torch.no_grad():
        ln.weight.normal_(1.0, 0.3)
        ln.bias.normal_(0.0, 0.5)
    x = torch.randn(n, w, device=cuda) * 1.5 + 0.3
    gy = torch.randn(n, w, device=cuda)
    R = [torch.randn(n, w, device=cuda), torch.randn(w, device=cuda), torch.randn(w, device=cuda)]

    def run(f, g, b, dtype):
        xx = x.to(dtype).requires_grad_(True)
        gg = gy.to(dtype).requires_grad_(True)
        y = f(xx)
        gx, dg, db = torch.autograd.grad(y, (xx, g, b), gg, create_graph=True)
        L = (gx * R[0].to(dtype)).sum() + (dg * R[1].to(dtype)).sum() + (db * R[2].to(dtype)).sum()
        return [y, gx, dg, db] + list(torch.autograd.grad(L, (xx, g, b, gg)))

    got = run(lambda t: so.ln_silu(ln, t), ln.weight, ln.bias, torch.float32)
    g64 = ln.weight.detach().double().requires_grad_(True)
    b64 = ln.bias.detach().double().requires_grad_(True)
    ref = run(lambda t: torch.nn.functional.silu(torch.nn.functional.layer_norm(t, (w,), g64, b64, ln.eps)),
              g64, b64, torch.float64)
    names = ["y", "gx", "dg", "db", "d2x", "d2g", "d2b", "d2gy"]
    for k, (a, r) in enumerate(zip(got, ref)):
        err = _rel(a.double(), r)
        assert err < (1e-5 if k < 4 else 1e-4), (names[k], err)


def test_rms_norm_second_order(pkg, cuda):
    """The fused rms_norm_sh of the training path (e2v2_rmsnorm_fwd / _bwd_param /
    _bwd2) against the float64 composition on the CPU: values and the first-order
    gradients of x, the affine weight and bias (1e-5 relative L2), then the
    gradients of L = <gx, R0> + <dw, R1> + <db, R2> in x, the weight and the
    upstream gy (1e-4).  More nodes than workgroups (1,024): some workgroups
    stride over two nodes."""
    import copy
    from ubio_molfm_amd import modules
    from ubio_molfm_amd import second_order as so
    torch.manual_seed(5)
    mod = modules.EquivariantRMSNormArraySphericalHarmonicsV2_BL(2, 256).to(cuda)
    with torch.no_grad():
        mod.affine_weight.normal_(1.0, 0.3)
        mod.affine_bias.normal_(0.0, 0.5)
    N = 1500 + 37
    x = torch.randn(9, N, 256, device=cuda) * 1.3
    x[0] += 0.7
    gy = torch.randn_like(x)
    R = [torch.randn_like(x), torch.randn(3, 256, device=cuda), torch.randn(256, device=cuda)]

    def run(m, dtype, dev):
        xx = x.to(dev, dtype).requires_grad_(True)
        gg = gy.to(dev, dtype).requires_grad_(True)
        y = so.rms_norm(m, xx)
        gx, dw, db = torch.autograd.grad(y, (xx, m.affine_weight, m.affine_bias), gg, create_graph=True)
        L = sum((t * r.to(dev, dtype)).sum() for t, r in zip((gx, dw, db), R))
        return [y, gx, dw, db] + list(torch.autograd.grad(L, (xx, m.affine_weight, gg)))

    got = run(mod, torch.float32, cuda)
    ref = run(copy.deepcopy(mod).double().cpu(), torch.float64, "cpu")
    names = ["y", "gx", "dw", "db", "d2x", "d2w", "d2gy"]
    for k, (a, r) in enumerate(zip(got, ref)):
        err = _rel(a, r)
        assert err < (1e-5 if k < 4 else 1e-4), (names[k], err)


def test_gate_second_order(pkg, cuda):
    """The fused Gate_s3 activations of the training path (e2v2_gate_fwd / _bwd /
    _bwd2) against the float64 composition on the CPU: values, first-order
    gradients of x and the gate Linear's weight (1e-5 relative L2), and the
    gradients of L = <gx, R0> + <dWg, R1> in x, the weight and the upstream gy
    (1e-4)."""
    import copy
    from ubio_molfm_amd import modules
    from ubio_molfm_amd import second_order as so
    torch.manual_seed(6)
    mod = modules.Gate_s3(256, 2).to(cuda)
    N = 700
    x = torch.randn(9, N, 256, device=cuda)
    gy = torch.randn_like(x)
    R = [torch.randn_like(x), torch.randn_like(mod.gates.weight)]

    def run(m, dtype, dev):
        xx = x.to(dev, dtype).requires_grad_(True)
        gg = gy.to(dev, dtype).requires_grad_(True)
        y = so.gate_s3(m, xx, 1.679, 1.842)
        gx, dW = torch.autograd.grad(y, (xx, m.gates.weight), gg, create_graph=True)
        L = (gx * R[0].to(dev, dtype)).sum() + (dW * R[1].to(dev, dtype)).sum()
        return [y, gx, dW] + list(torch.autograd.grad(L, (xx, m.gates.weight, gg)))

    got = run(mod, torch.float32, cuda)
    ref = run(copy.deepcopy(mod).double().cpu(), torch.float64, "cpu")
    names = ["y", "gx", "dW", "d2x", "d2W", "d2gy"]
    for k, (a, r) in enumerate(zip(got, ref)):
        err = _rel(a, r)
        assert err < (1e-5 if k < 3 else 1e-4), (names[k], err)


def test_row_max_ties_match_scatter_reduce(pkg, cuda):
    """The softmax row maximum of the training path (_RowMaxFn: scatter_reduce amax
    forward, its tie-split gradient composed from the segment gather and row sum)
    against torch's scatter_reduce on logits with many exact ties, rows of 0-7
    edges: the maximum, the first-order gradient and the gradient of
    <d logit, R> in the upstream g."""
    from ubio_molfm_amd import sparse_ops
    from ubio_molfm_amd import second_order as so
    g = torch.Generator().manual_seed(8)
    N, H = 300, 16
    deg = torch.randint(0, 8, (N,), generator=g)
    qi = torch.repeat_interleave(torch.arange(N), deg).to(cuda)
    E = qi.numel()
    logit = torch.randint(-3, 3, (E, H), generator=g).float().to(cuda)

    class Edges:
        def __init__(self):
            self.qi, self.N, self.row32 = qi, N, qi.int()
            self.row_ptr = torch.cat([torch.zeros(1, dtype=torch.long), deg.cumsum(0)]).int().to(cuda)
            self.eid = torch.arange(E, dtype=torch.int32, device=cuda)

        def gather_q(self, x):
            return sparse_ops.sparse_gather_edge_index(x, self.row32, self.N, (self.row_ptr, self.eid))

        def row_sum(self, a):
            return sparse_ops.sparse_alpha_sum_edge_index_triton(a, self.row32, self.N,
                                                                metadata=(self.row_ptr, self.eid))

    up = torch.randn(N, H, device=cuda)
    R = torch.randn(E, H, device=cuda)

    def run(f):
        x = logit.clone().requires_grad_(True)
        gg = up.clone().requires_grad_(True)
        m = f(x)
        gx, = torch.autograd.grad(m, x, gg, create_graph=True)
        d2, = torch.autograd.grad((gx * R).sum(), gg)
        return m.detach(), gx.detach(), d2

    def ref(x):
        m = torch.full((N, H), -torch.inf, device=cuda)
        return m.scatter_reduce(0, qi.view(-1, 1).expand(-1, H), x, reduce="amax", include_self=True)

    got, want = run(lambda x: so._RowMaxFn.apply(x, Edges())), run(ref)
    rows = deg.to(cuda) > 0
    assert torch.equal(got[0][rows], want[0][rows])
    for a, b in zip(got[1:], want[1:]):
        assert torch.allclose(a, b, rtol=1e-6, atol=1e-7)


def test_eval_mode_keeps_the_fused_path(pkg, cuda):
    """eval(): the fused kernels run (their backward is first order, so a
    create_graph=True differentiation raises instead of silently dropping the
    second-order terms); train() on the same model gives the same energy and
    forces through the training path."""
    from ubio_molfm_amd import systems
    m, _ = _pair(cuda, 34)
    s = systems.small_water(4, 5.5, seed=24)
    pos = torch.as_tensor(s["pos"], device=cuda)
    Z = torch.as_tensor(s["Z"], device=cuda)
    m.eval()
    e_eval, f_eval, _ = m.energy_forces_flat(pos, Z, s["graph_ptr"], s["cell"], s["pbc"])
    m.train()
    e_tr, f_tr, _ = m.energy_forces_flat(pos, Z, s["graph_ptr"], s["cell"], s["pbc"])
    assert f_tr.requires_grad and not f_eval.requires_grad
    assert _rel(e_tr, e_eval) < 1e-5 and _rel(f_tr, f_eval) < 1e-4
    m.eval()
    p = pos.clone().requires_grad_(True)
    e, _ = m.energy_flat(p, Z, s["graph_ptr"], s["cell"], s["pbc"])
    with pytest.raises(NotImplementedError):
        torch.autograd.grad(e.sum(), p, create_graph=True)
