"""Radius graph from the HIP cell-list builder vs the exact fp32 oracle.

Bar: the canonical (i, j, shift) list is identical and dvec / d agree bitwise
(both sides evaluate the same fp32 expression).  Edges within 2 ulp of the
cutoff are counted and reported separately (their membership can differ from
torch.linalg.norm rounding in the reference).
"""
import numpy as np
import pytest
import torch

from oracle.neighbors import exact_neighbors

pytestmark = pytest.mark.gpu


def _check(pkg, cuda, sysd, rc=6.0, label="", rmin=1e-4, include=None):
    from ubio_molfm_amd import neighbors
    pos = torch.as_tensor(sysd["pos"], device=cuda)
    inc = None if include is None else torch.as_tensor(include, device=cuda)
    nl = neighbors.build_neighbors(pos, sysd["graph_ptr"], sysd["cell"], sysd["pbc"], rc, rmin, src_include=inc)
    got = nl.canonical()
    ref = exact_neighbors(sysd["pos"], sysd["graph_ptr"], sysd["cell"], sysd["pbc"], rc, rmin, include=include)
    shell = int(np.sum(np.abs(ref["d"] - np.float32(rc)) <= 2 * np.spacing(np.float32(rc))))
    print(f"[nbr {label}] N={len(sysd['pos'])} E={nl.n_edges} oracle E={len(ref['i'])} "
          f"max_row={nl.max_row} near-cutoff(2ulp)={shell}", flush=True)
    assert nl.n_edges == len(ref["i"])
    for k in ("i", "j", "s"):
        assert np.array_equal(got[k], ref[k]), k
    assert np.array_equal(got["dv"].view(np.uint32), ref["dv"].view(np.uint32))
    assert np.array_equal(got["d"].view(np.uint32), ref["d"].view(np.uint32))
    # rows sorted by distance
    rp = nl.row_ptr.cpu().numpy(); d = nl.dist.cpu().numpy()
    for r in range(min(len(rp) - 1, 200)):
        seg = d[rp[r]:rp[r + 1]]
        assert np.all(seg[1:] >= seg[:-1])
    # key CSR is the exact transpose, sorted by edge id
    kp = nl.key_ptr.cpu().numpy(); ke = nl.key_eid.cpu().numpy(); col = nl.col.cpu().numpy()
    assert kp[-1] == nl.n_edges
    for j in range(len(kp) - 1):
        seg = ke[kp[j]:kp[j + 1]]
        assert np.all(col[seg] == j) and np.all(np.diff(seg) > 0)
    if nl.n_edges:
        er = nl.edge_row.cpu().numpy()
        check_slots(kp, col, er, ke, nl.col_span, nl.col_slot_member, nl.col_slot_edge, nl.col_n_slots)
    return nl


def check_slots(seg_ptr, seg_of_edge, member_of_edge, item_eid, span, sm, se, ns):
    """Cluster slots (e2v2_cluster_slots) against their definition: every edge of
    a cluster in exactly one slot, in the column of its segment, under its member
    atom; slots sorted by atom with one slot per (atom, occurrence) unless the
    cluster overflowed (then one slot per item)."""
    sm, se, ns = sm.cpu().numpy(), se.cpu().numpy().reshape(-1, span), ns.cpu().numpy()
    n_seg = len(seg_ptr) - 1
    n_cl = (n_seg + span - 1) // span
    assert len(ns) >= n_cl
    E = len(seg_of_edge)
    seen = np.zeros(E, np.int64)
    for c in range(n_cl):
        s0, s1 = c * span, min(c * span + span, n_seg)
        b, n = seg_ptr[s0], seg_ptr[s1] - seg_ptr[s0]
        k = ns[c]
        assert 0 <= k <= n, (c, k, n)
        m = sm[b:b + k]; ed = se[b:b + k]
        rr, cc = np.nonzero(ed >= 0)
        e = ed[rr, cc]
        assert np.all(seg_of_edge[e] == s0 + cc)
        assert np.all(member_of_edge[e] == m[rr])
        seen[e] += 1
        items = np.arange(b, b + n)
        eids = items if item_eid is None else item_eid[items]
        assert np.array_equal(np.sort(e), np.sort(eids))
        if n <= 4096 and k:
            assert np.all(np.diff(m) >= 0)
            # one slot per (atom, occurrence): slots of an atom = its largest multiplicity in one segment
            atoms, per_atom = np.unique(m, return_counts=True)
            segm = seg_of_edge[eids] * (member_of_edge.max() + 1) + member_of_edge[eids]
            mult_of = {}
            for key, cnt in zip(*np.unique(segm, return_counts=True)):
                a = key % (member_of_edge.max() + 1)
                mult_of[a] = max(mult_of.get(a, 0), cnt)
            assert all(mult_of[a] == pa for a, pa in zip(atoms, per_atom))
    assert np.all(seen == 1)


def test_small_cell_below_cutoff(pkg, cuda):
    from ubio_molfm_amd import systems
    _check(pkg, cuda, systems.small_water(8, 6.2, seed=0), label="small")


def test_water_cfg1(pkg, cuda):
    from ubio_molfm_amd import systems
    _check(pkg, cuda, systems.CONFIGS[1](), label="cfg1")


def test_peptide_cfg3(pkg, cuda):
    from ubio_molfm_amd import systems
    _check(pkg, cuda, systems.CONFIGS[3](), label="cfg3")


def test_ragged_organics_cfg2(pkg, cuda):
    from ubio_molfm_amd import systems
    _check(pkg, cuda, systems.CONFIGS[2](), label="cfg2")


def test_triclinic_partial_pbc(pkg, cuda):
    rng = np.random.default_rng(5)
    cell = np.array([[9.0, 0.0, 0.0], [2.5, 8.0, 0.0], [1.0, -1.5, 10.0]], np.float32)
    frac = rng.uniform(0, 1, size=(60, 3))
    pos = (frac @ cell).astype(np.float32)
    sysd = dict(pos=pos, Z=np.full(60, 6), graph_ptr=np.array([0, 60]), cell=cell[None],
                pbc=np.array([[True, False, True]]))
    _check(pkg, cuda, sysd, label="triclinic")


def test_max_neighbors_keeps_nearest(pkg, cuda):
    from ubio_molfm_amd import neighbors, systems
    s = systems.CONFIGS[1]()
    pos = torch.as_tensor(s["pos"], device=cuda)
    full = neighbors.build_neighbors(pos, s["graph_ptr"], s["cell"], s["pbc"], 6.0)
    top = neighbors.build_neighbors(pos, s["graph_ptr"], s["cell"], s["pbc"], 6.0, max_neighbors=32)
    rp, rpt = full.row_ptr.cpu().numpy(), top.row_ptr.cpu().numpy()
    d, dt = full.dist.cpu().numpy(), top.dist.cpu().numpy()
    c, ct = full.col.cpu().numpy(), top.col.cpu().numpy()
    for r in range(len(rp) - 1):
        n = min(32, rp[r + 1] - rp[r])
        assert rpt[r + 1] - rpt[r] == n
        assert np.array_equal(d[rp[r]:rp[r] + n], dt[rpt[r]:rpt[r + 1]])
        assert np.array_equal(c[rp[r]:rp[r] + n], ct[rpt[r]:rpt[r + 1]])


def test_empty_and_isolated(pkg, cuda):
    # two far-apart atoms in a non-periodic graph: no edges at all
    sysd = dict(pos=np.array([[0, 0, 0], [50, 0, 0]], np.float32), Z=np.array([1, 1]), graph_ptr=np.array([0, 2]),
                cell=np.zeros((1, 3, 3), np.float32), pbc=np.zeros((1, 3), bool))
    nl = _check(pkg, cuda, sysd, label="isolated")
    assert nl.n_edges == 0


def test_coincident_atoms_below_min_dist(pkg, cuda):
    rng = np.random.default_rng(3)
    pos = rng.uniform(0, 8, size=(30, 3)).astype(np.float32)
    pos[7] = pos[3] + np.float32(5e-5)
    sysd = dict(pos=pos, Z=np.full(30, 6), graph_ptr=np.array([0, 30]),
                cell=(np.eye(3, dtype=np.float32) * 8.0)[None], pbc=np.ones((1, 3), bool))
    nl = _check(pkg, cuda, sysd, label="coincident")
    c = nl.canonical()
    assert not np.any((c["i"] == 3) & (c["j"] == 7) & np.all(c["s"] == 0, axis=1))


def test_cluster_slots_rows_and_overflow(pkg, cuda):
    """Row clusters (span 4 and 8) of a small periodic cell with many images, and
    a dense cell whose 8-column clusters exceed the per-cluster sort capacity
    (one slot per item)."""
    from ubio_molfm_amd import neighbors, systems
    s = systems.small_water(8, 6.2, seed=0)
    rng = np.random.default_rng(5)
    dense = dict(pos=rng.uniform(0, 10, size=(700, 3)).astype(np.float32), Z=np.full(700, 1),
                 graph_ptr=np.array([0, 700]), cell=(np.eye(3, dtype=np.float32) * 10.0)[None],
                 pbc=np.ones((1, 3), bool))
    for sysd, label in ((s, "images"), (dense, "dense")):
        pos = torch.as_tensor(sysd["pos"], device=cuda)
        nl = neighbors.build_neighbors(pos, sysd["graph_ptr"], sysd["cell"], sysd["pbc"], 6.0)
        rp = nl.row_ptr.cpu().numpy(); col = nl.col.cpu().numpy(); er = nl.edge_row.cpu().numpy()
        kp = nl.key_ptr.cpu().numpy(); ke = nl.key_eid.cpu().numpy()
        over = 0
        for span in (4, 8):
            sm, se, ns = neighbors.cluster_slots(nl.row_ptr, nl.n_atoms, nl.col, None, span)
            check_slots(rp, er, col, None, span, sm, se, ns)
            sm, se, ns = neighbors.cluster_slots(nl.key_ptr, nl.n_atoms, nl.edge_row, nl.key_eid, span)
            check_slots(kp, col, er, ke, span, sm, se, ns)
            over += int(np.sum(kp[np.minimum(np.arange(0, nl.n_atoms, span) + span, nl.n_atoms)]
                               - kp[np.arange(0, nl.n_atoms, span)] > 4096))
        print(f"[slots {label}] N={nl.n_atoms} E={nl.n_edges} overflowing clusters={over}", flush=True)
        if label == "dense":
            assert over > 0


def test_key_csr_long_column(pkg, cuda):
    """A column with more edges than the LDS sort holds (5000 rows point at atom
    0) is sorted in place in global memory: the key CSR equals a stable numpy
    sort of the edges by column."""
    from ubio_molfm_amd import _lib
    N = 6000
    rng = np.random.default_rng(4)
    rows, cols = [], []
    for i in range(N):
        if i < 5000:
            rows.append(i); cols.append(0)
        for j in rng.choice(N, size=3, replace=False):
            rows.append(i); cols.append(int(j))
    rows = np.asarray(rows, np.int32); cols = np.asarray(cols, np.int32)
    o = np.lexsort((cols, rows)); rows, cols = rows[o], cols[o]
    E = len(rows)
    row_ptr = np.zeros(N + 1, np.int32); np.add.at(row_ptr, rows + 1, 1); row_ptr = np.cumsum(row_ptr).astype(np.int32)
    i32 = dict(dtype=torch.int32, device=cuda)
    d_rp = torch.as_tensor(row_ptr, device=cuda); d_col = torch.as_tensor(cols, device=cuda)
    edge_row = torch.empty(E, **i32); kc = torch.empty(N, **i32); kp = torch.empty(N + 1, **i32)
    stats = torch.zeros(2, **i32); tkey = torch.empty(E, dtype=torch.int64, device=cuda); ke = torch.empty(E, **i32)
    st = _lib.vp(torch.cuda.current_stream().cuda_stream)
    for phase in (0, 1):
        _lib.call("e2v2_csr_transpose", _lib.vp(d_rp.data_ptr()), _lib.vp(d_col.data_ptr()), _lib.i32(N),
                  _lib.i32(N), _lib.i64(E), _lib.vp(edge_row.data_ptr()), _lib.vp(kc.data_ptr()),
                  _lib.vp(kp.data_ptr()), _lib.vp(stats.data_ptr()),
                  _lib.vp(tkey.data_ptr()) if phase else None, _lib.vp(ke.data_ptr()) if phase else None,
                  _lib.i32(phase), st)
    torch.cuda.synchronize()
    order = np.argsort(cols, kind="stable").astype(np.int32)
    ref_ptr = np.zeros(N + 1, np.int64); np.add.at(ref_ptr, cols + 1, 1); ref_ptr = np.cumsum(ref_ptr)
    print(f"[key csr] E={E} longest column={int(np.diff(ref_ptr).max())}", flush=True)
    assert int(np.diff(ref_ptr).max()) > 4096
    assert np.array_equal(kp.cpu().numpy(), ref_ptr.astype(np.int32))
    assert np.array_equal(ke.cpu().numpy(), order)
    assert np.array_equal(edge_row.cpu().numpy(), rows)


@pytest.mark.parametrize("box", ["cell", "padded", "shrunk", "shifted"])
def test_caller_grid_box_gives_same_edges(pkg, cuda, box):
    """A caller-supplied bin grid (the MD loop passes the cell of its wrapped
    positions) yields the same neighbour list as the read-back bounding box; a box
    that misses atoms ("shrunk", "shifted") is detected and the list rebuilt."""
    from ubio_molfm_amd import neighbors, systems
    s = systems.CONFIGS[1]()
    pos = torch.as_tensor(s["pos"], device=cuda)
    L = np.diag(s["cell"][0]).astype(np.float32)
    lo, hi = {"cell": (np.zeros(3, np.float32), L),
              "padded": (-0.2 * L, 1.3 * L),
              "shrunk": (0.3 * L, 0.6 * L),
              "shifted": (-0.5 * L, 0.7 * L)}[box]
    ref = neighbors.build_neighbors(pos, s["graph_ptr"], s["cell"], s["pbc"], 6.0)
    got = neighbors.build_neighbors(pos, s["graph_ptr"], s["cell"], s["pbc"], 6.0,
                                    grid_box=np.stack([lo, hi])[:, None, :])
    print(f"[grid_box {box}] E={ref.n_edges}/{got.n_edges}", flush=True)
    assert ref.n_edges == got.n_edges
    for name in ("row_ptr", "col", "shift_idx", "dist", "dvec", "key_ptr", "key_eid"):
        assert torch.equal(getattr(ref, name), getattr(got, name)), name


@pytest.mark.parametrize("case", ["water_pbc", "organics"])
def test_long_range_source_mask(pkg, cuda, case):
    """The long-range cluster list (e2former_wrapper.py:223-243): cutoff 12 A,
    lower cutoff 0.1 A, sources restricted to atoms whose atomic number is
    neither 0 nor 1 -- the same exact edge set, shifts and fp32 geometry as the
    oracle with the include mask."""
    from ubio_molfm_amd import systems
    s = systems.small_water(8, 6.2, seed=3) if case == "water_pbc" else \
        systems.organics_batch(n_mol=3, nmin=10, nmax=24, seed=8)
    include = ~np.isin(np.asarray(s["Z"]), [0, 1])
    nl = _check(pkg, cuda, s, rc=12.0, rmin=0.1, include=include, label=f"long-{case}")
    col = nl.col.cpu().numpy()
    assert nl.n_edges > 0 and np.all(include[col])
