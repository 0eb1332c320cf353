"""Op-level drop-ins with the reference's signatures (ubio_molfm_amd.sparse_ops,
neighbors.construct_radius_neighbor) on the GPU: values, first- and
second-order gradients against float64 CPU evaluations of each op's defining
formula (the docstrings of triton_sparse_qk_autograd.py:839-852,
sparse_v_agg_edge_index_cblocked_bench.py:246-254 and :432-436,
sparse_alpha_sum_edge_index_autograd.py:207-213, edge_degree_outer_autograd.py:348-355),
the CSR metadata against the oracle's numpy restatement, and the padded-batch
neighbour search against the oracle's dense restatement."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = dict(rtol=2e-5, atol=2e-5)


def _edges(n_q, n_k, E, seed, isolated=()):
    g = torch.Generator().manual_seed(seed)
    qi = torch.randint(0, n_q, (E,), generator=g)
    for r in isolated:
        qi[qi == r] = (r + 1) % n_q
    nj = torch.randint(0, n_k, (E,), generator=g)
    return qi, nj


def _rand(shape, seed, dtype=torch.float64):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed), dtype=dtype)


def _close(a, b, tol=TOL):
    assert a.shape == b.shape, (a.shape, b.shape)
    torch.testing.assert_close(a.detach().double().cpu(), b.detach().double().cpu(), **tol)


def _second_order(fn, inputs, out_grad, weights):
    """d/d(inputs, out_grad) of sum_i <grad_i, w_i> with grad = d<fn(inputs), out_grad>/d inputs."""
    out = fn(*inputs)
    grads = torch.autograd.grad(out, inputs, out_grad, create_graph=True)
    s = sum((gr.double() * w).sum() for gr, w in zip(grads, weights))
    return grads, torch.autograd.grad(s, (*inputs, out_grad), allow_unused=True)


def _cpu_and_gpu(ts, cuda):
    cpu = [t.clone().requires_grad_(True) for t in ts]
    gpu = [t.to(cuda, torch.float32).requires_grad_(True) for t in ts]
    return cpu, gpu


# ---------------------------------------------------------------------------
def test_metadata_matches_restatement(pkg, cuda):
    from ubio_molfm_amd import sparse_ops as so
    from oracle.sparse_ops import qk_metadata
    for seed, (n_q, n_k, E) in enumerate(((13, 17, 200), (1, 3, 9), (40, 5, 3000), (6, 6, 0))):
        qi, nj = _edges(n_q, n_k, E, seed)
        got = so.prepare_sparse_qk_edge_index_metadata(qi.to(cuda), nj.to(cuda), n_q, n_k)
        want = qk_metadata(qi.numpy(), nj.numpy(), n_q, n_k)
        assert len(got) == 6
        for a, b in zip(got, want):
            assert a.dtype == torch.int32 and np.array_equal(a.cpu().numpy(), b)
    # a column longer than the in-LDS sort (256): sorted in global memory
    qi = torch.arange(600) % 3
    nj = torch.zeros(600, dtype=torch.int64)
    got = so.prepare_sparse_qk_edge_index_metadata(qi.to(cuda), nj.to(cuda), 3, 1)
    for a, b in zip(got, qk_metadata(qi.numpy(), nj.numpy(), 3, 1)):
        assert np.array_equal(a.cpu().numpy(), b)
    rp, ai = so.prepare_sparse_alpha_sum_edge_index_metadata(qi.to(cuda), 3)
    assert np.array_equal(ai.cpu().numpy(), np.argsort(qi.numpy(), kind="stable"))
    with pytest.raises(RuntimeError, match="outside"):
        so.prepare_sparse_qk_edge_index_metadata(torch.tensor([0, 5], device=cuda), torch.tensor([0, 0], device=cuda),
                                                 3, 1)


def test_sparse_qk_edge_index(pkg, cuda):
    from ubio_molfm_amd import sparse_ops as so
    n_q, n_k, E, H, D = 37, 29, 900, 16, 8
    qi, nj = _edges(n_q, n_k, E, 1, isolated=(4,))

    def ref(q, k):
        return (q[qi] * k[nj]).sum(-1)

    (qc, kc), (qg, kg) = _cpu_and_gpu([_rand((n_q, H, D), 2), _rand((n_k, H, D), 3)], cuda)
    qi_d, nj_d = qi.to(cuda), nj.to(cuda)
    md = so.prepare_sparse_qk_edge_index_metadata(qi_d, nj_d, n_q, n_k)
    out = so.sparse_qk_edge_index_triton(qg, kg, qi_d, nj_d, md)
    assert out.dtype == torch.float32 and out.shape == (E, H)
    _close(out, ref(qc, kc))
    with torch.no_grad():
        _close(so.sparse_qk_edge_index_triton(qg, kg, qi_d, nj_d), ref(qc, kc))
    g = _rand((E, H), 4)
    u, w = _rand((n_q, H, D), 5), _rand((n_k, H, D), 6)
    gc, gg = g.clone().requires_grad_(True), g.to(cuda, torch.float32).requires_grad_(True)
    g1c, g2c = _second_order(ref, (qc, kc), gc, (u, w))
    g1g, g2g = _second_order(lambda q, k: so.sparse_qk_edge_index_triton(q, k, qi_d, nj_d, md), (qg, kg), gg,
                             (u.to(cuda), w.to(cuda)))
    for a, b in zip(g1g + g2g, g1c + g2c):
        _close(a, b)
    with pytest.raises(ValueError, match="6-tuple"):
        so.sparse_qk_edge_index_triton(qg, kg, qi_d, nj_d, md[:3])


def test_sparse_v_agg_cblocked(pkg, cuda):
    from ubio_molfm_amd import sparse_ops as so
    n_q, n_v, E, C, H = 31, 23, 700, 58, 32
    qi, nj = _edges(n_q, n_v, E, 7, isolated=(0, 9))

    def ref(v, a):
        return torch.zeros(n_q, C, H, dtype=v.dtype).index_add(0, qi, a.unsqueeze(1) * v[nj])

    (vc, ac), (vg, ag) = _cpu_and_gpu([_rand((n_v, C, H), 8), _rand((E, H), 9)], cuda)
    qi_d, nj_d = qi.to(cuda), nj.to(cuda)
    out = so.sparse_v_agg_edge_index_triton_cblocked(vg, ag, qi_d, nj_d, n_q)
    assert out.dtype == torch.float32 and out.shape == (n_q, C, H)
    _close(out, ref(vc, ac))
    g = _rand((n_q, C, H), 10)
    u, w = _rand((n_v, C, H), 11), _rand((E, H), 12)
    gc, gg = g.clone().requires_grad_(True), g.to(cuda, torch.float32).requires_grad_(True)
    md = so.prepare_sparse_v_agg_edge_index_metadata(qi_d, nj_d, n_q, n_v)
    g1c, g2c = _second_order(ref, (vc, ac), gc, (u, w))
    g1g, g2g = _second_order(lambda v, a: so.sparse_v_agg_edge_index_triton_cblocked(v, a, qi_d, nj_d, n_q, md),
                             (vg, ag), gg, (u.to(cuda), w.to(cuda)))
    for a, b in zip(g1g + g2g, g1c + g2c):
        _close(a, b)
    with pytest.raises(ValueError, match=r"\[M, C, H\]"):
        so.sparse_v_agg_edge_index_triton_cblocked(vg[0], ag, qi_d, nj_d, n_q)


def test_sparse_alpha_sum(pkg, cuda):
    from ubio_molfm_amd import sparse_ops as so
    n_q, E, H = 45, 800, 24
    qi, _ = _edges(n_q, 1, E, 13, isolated=(3,))

    def ref(a):
        return torch.zeros(n_q, H, dtype=a.dtype).index_add(0, qi, a)

    (ac,), (ag,) = _cpu_and_gpu([_rand((E, H), 14)], cuda)
    qi_d = qi.to(cuda)
    out = so.sparse_alpha_sum_edge_index_triton(ag, qi_d, n_q)
    _close(out, ref(ac))
    g = _rand((n_q, H), 15)
    gc, gg = g.clone().requires_grad_(True), g.to(cuda, torch.float32).requires_grad_(True)
    g1c, g2c = _second_order(ref, (ac,), gc, (_rand((E, H), 16),))
    g1g, g2g = _second_order(lambda a: so.sparse_alpha_sum_edge_index_triton(a, qi_d, n_q), (ag,), gg,
                             (_rand((E, H), 16).to(cuda),))
    # the op is linear: its gradient does not depend on alpha
    for a, b in zip(g1g + (g2g[1],), g1c + (g2c[1],)):
        _close(a, b)
    assert g2c[0] is None and (g2g[0] is None or float(g2g[0].abs().max()) == 0.0)
    bf = so.sparse_alpha_sum_edge_index_triton(ag.detach().bfloat16(), qi_d, n_q)
    assert bf.dtype == torch.bfloat16


def test_edge_degree_outer(pkg, cuda):
    from ubio_molfm_amd import sparse_ops as so
    n_q, E, L, H = 27, 600, 5, 48
    qi, _ = _edges(n_q, 1, E, 17, isolated=(2, 11))

    def ref(sh, fea):
        return torch.zeros(n_q, L, H, dtype=sh.dtype).index_add(0, qi, sh.unsqueeze(2) * fea.unsqueeze(1))

    (sc, fc), (sg, fg) = _cpu_and_gpu([_rand((E, L), 18), _rand((E, H), 19)], cuda)
    qi_d = qi.to(cuda)
    out = so.edge_degree_outer_triton(sg, fg, qi_d, n_q)
    _close(out, ref(sc, fc))
    g = _rand((n_q, L, H), 20)
    u, w = _rand((E, L), 21), _rand((E, H), 22)
    gc, gg = g.clone().requires_grad_(True), g.to(cuda, torch.float32).requires_grad_(True)
    md = so.prepare_edge_degree_outer_metadata(qi_d, n_q)
    g1c, g2c = _second_order(ref, (sc, fc), gc, (u, w))
    g1g, g2g = _second_order(lambda s, f: so.edge_degree_outer_triton(s, f, qi_d, n_q, md), (sg, fg), gg,
                             (u.to(cuda), w.to(cuda)))
    for a, b in zip(g1g + g2g, g1c + g2c):
        _close(a, b)
    with pytest.raises(ValueError, match="6-tuple"):
        so.edge_degree_outer_triton(sg, fg, qi_d, n_q, md[:2])
    with pytest.raises(ValueError, match="tuple/list"):
        so.edge_degree_outer_triton(sg, fg, qi_d, n_q, md[0])


def test_malformed_metadata_slots_are_skipped(pkg, cuda):
    """Slots whose partner row or edge id lies outside its operand are skipped by
    the kernels' own bounds checks: the result equals the formula without them."""
    from ubio_molfm_amd import sparse_ops as so
    n_q, n_k, E, H, D = 9, 7, 60, 4, 8
    qi, nj = _edges(n_q, n_k, E, 23)
    md = list(so.prepare_sparse_qk_edge_index_metadata(qi.to(cuda), nj.to(cuda), n_q, n_k))
    col = md[1].clone()
    col[5] = n_k + 3           # partner row out of range
    alpha = md[2].clone()
    bad_e = int(alpha[7])
    alpha[7] = E + 11          # edge id out of range
    md[1], md[2] = col, alpha
    q, k = _rand((n_q, H, D), 24), _rand((n_k, H, D), 25)
    out = so.sparse_qk_edge_index_triton(q.to(cuda, torch.float32), k.to(cuda, torch.float32), qi.to(cuda),
                                         nj.to(cuda), tuple(md))
    want = (q[qi] * k[nj]).sum(-1)
    skipped_e = int(md[2][5]) if int(md[2][5]) < E else None
    keep = torch.ones(E, dtype=torch.bool)
    keep[bad_e] = False
    if skipped_e is not None:
        keep[skipped_e] = False
    _close(out.cpu()[keep], want[keep])
    assert float(out.cpu()[~keep].abs().max()) == 0.0


# ---------------------------------------------------------------------------
def _padded_batch(seed, B=3, L=40, cell=9.0):
    g = torch.Generator().manual_seed(seed)
    counts = [L, L - 7, L - 15][:B]
    pos = torch.full((B, L, 3), 999.0)
    mask = torch.zeros(B, L, dtype=torch.bool)
    for b, n in enumerate(counts):
        pos[b, :n] = torch.rand(n, 3, generator=g) * cell
        mask[b, :n] = True
    # expanded nodes: the atoms and one shifted copy of the first half (valid first, padding at 999)
    L2 = L + L // 2
    epos = torch.full((B, L2, 3), 999.0)
    emask = torch.zeros(B, L2, dtype=torch.bool)
    for b, n in enumerate(counts):
        m = n // 2
        epos[b, :n] = pos[b, :n]
        epos[b, n:n + m] = pos[b, :m] + torch.tensor([cell, 0.0, 0.0])
        emask[b, :n + m] = True
    inc = torch.rand(B, L2, generator=g) > 0.25
    return pos, mask, epos, emask, inc


@pytest.mark.parametrize("kw", [dict(), dict(max_neighbors=6), dict(include_mask=True, poly="poly_bell"),
                                dict(include_mask=True, max_neighbors=3)])
def test_construct_radius_neighbor_matches_dense_restatement(pkg, cuda, kw):
    from ubio_molfm_amd import neighbors, sparse_ops as so
    from oracle.neighbors import construct_radius_neighbor as oracle_crn
    from oracle.sparse_ops import qk_metadata
    pos, mask, epos, emask, inc = _padded_batch(31)
    kw = dict(kw)
    use_inc = kw.pop("include_mask", False)
    rc, rmin = 4.0, 1e-4
    got = neighbors.construct_radius_neighbor(pos.to(cuda), mask.to(cuda), epos.to(cuda), emask.to(cuda), rc,
                                              include_mask=inc.to(cuda) if use_inc else None, min_dist=rmin, **kw)
    want = oracle_crn(pos, mask, epos, emask, rc, rmin, kw.get("max_neighbors"),
                      include_mask=inc if use_inc else None, poly=kw.get("poly", "poly"), fixed_norm=True)
    assert list(got) == ["query_idx", "neighbor_idx", "metadata", "f_edge_vec", "f_dist", "f_poly_dist"]
    assert got["query_idx"].dtype == torch.int64 and got["neighbor_idx"].dtype == torch.int64
    assert torch.equal(got["query_idx"].cpu(), want["query_idx"])
    assert torch.equal(got["neighbor_idx"].cpu(), want["neighbor_idx"])
    assert torch.equal(got["f_dist"].cpu(), want["f_dist"])
    assert torch.equal(got["f_edge_vec"].cpu(), want["f_edge_vec"])
    torch.testing.assert_close(got["f_poly_dist"].cpu(), want["f_poly_dist"], rtol=1e-6, atol=1e-6)
    md = qk_metadata(want["query_idx"].numpy(), want["neighbor_idx"].numpy(), int(mask.sum()), int(emask.sum()))
    for a, b in zip(got["metadata"], md):
        assert np.array_equal(a.cpu().numpy(), b)
    # the same edges through the op-level QK product
    H, D = 4, 8
    q = torch.randn(int(mask.sum()), H, D, device=cuda)
    k = torch.randn(int(emask.sum()), H, D, device=cuda)
    out = so.sparse_qk_edge_index_triton(q, k, got["query_idx"], got["neighbor_idx"], got["metadata"])
    _close(out, (q[got["query_idx"]] * k[got["neighbor_idx"]]).sum(-1))


def test_construct_radius_neighbor_edge_cases(pkg, cuda):
    from ubio_molfm_amd import neighbors
    pos, mask, epos, emask, _ = _padded_batch(37, B=1, L=6)
    # cutoff below every distance: no edge, every output empty
    nb = neighbors.construct_radius_neighbor(pos.to(cuda), mask.to(cuda), epos.to(cuda), emask.to(cuda), 1e-6,
                                             min_dist=1e-4)
    assert nb["query_idx"].numel() == 0 and nb["f_edge_vec"].shape == (0, 3)
    # default min_dist -1 keeps the self pair at d = 0
    nb = neighbors.construct_radius_neighbor(pos.to(cuda), mask.to(cuda), epos.to(cuda), emask.to(cuda), 1e-6)
    assert nb["query_idx"].tolist() == list(range(6)) and nb["neighbor_idx"].tolist() == list(range(6))
    assert float(nb["f_dist"].abs().max()) == 0.0 and float((nb["f_poly_dist"] - 1).abs().max()) == 0.0
    with pytest.raises(ValueError, match="poly"):
        neighbors.construct_radius_neighbor(pos.to(cuda), mask.to(cuda), epos.to(cuda), emask.to(cuda), 3.0,
                                            poly="gauss")
    with pytest.raises(RuntimeError, match="no atom"):
        neighbors.construct_radius_neighbor(pos.to(cuda), torch.zeros_like(mask).to(cuda), epos.to(cuda),
                                            emask.to(cuda), 3.0)
