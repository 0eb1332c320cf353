"""Product boundary on the GPU: E2FormerCalculator (device and host paths, with
the charge / multiplicity system embedding active and reference energies) and
the backbone's neighbor_info dict, against the CPU oracle; the MD integrator
against the restated reference NVE step with the same HIP forces."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _pair(cuda, seed=0):
    from ubio_molfm_amd import model
    from oracle.model import MolfmAtomic as OracleModel
    torch.manual_seed(seed)
    m = model.MolfmAtomic(model.default_args()).eval().to(cuda)
    om = OracleModel().eval()
    om.load_state_dict({k: v.cpu() for k, v in m.state_dict().items()}, strict=True)
    return m, om


def _oracle(om, sysd, charge, mult):
    from ubio_molfm_amd import systems
    bd = systems.to_padded(sysd)
    B = len(sysd["graph_ptr"]) - 1
    bd["charge"] = torch.as_tensor(charge, dtype=torch.int32).reshape(B)
    bd["multiplicity"] = torch.as_tensor(mult, dtype=torch.int32).reshape(B)
    r = om(bd)
    return r["pred_energy"].detach().double(), r["pred_forces"].detach()[bd["atom_masks"]].double()


class _AseLike:
    """Minimal ase.Atoms surface (ase is not installed here)."""

    def __init__(self, pos, Z, cell, pbc, charges):
        self.p, self.Z, self.c, self.b, self.q = pos, Z, cell, pbc, charges

    def get_positions(self):
        return self.p

    def get_atomic_numbers(self):
        return self.Z

    def get_cell(self):
        return self.c

    def get_pbc(self):
        return self.b

    def get_initial_charges(self):
        return self.q


def test_calculator_torch_path_charge_multiplicity(pkg, cuda):
    """Device path (TorchAtoms-style input): the calculator's charge and
    multiplicity feed the system embedding added to the l = 0 row of every
    layer (e2former_wrapper.py:249-259, e2former.py:582-583), and the reference
    energies sum[ref_energy[Z]] are added; energy and forces against the oracle
    MolfmAtomic on the same batch (gates 1e-5 eV/atom, 1e-4 force rel-L2).  The
    same weights with charge 0 give a different energy (the path is live: the
    random-init system embedding moves it by ~3e-5 eV, far above the 1e-8 eV
    float32 rounding of this 24-atom energy)."""
    from ubio_molfm_amd import calculator, systems
    m, om = _pair(cuda, seed=11)
    s = systems.small_water(8, 6.2, seed=5)
    ref_table = np.linspace(-3.0, -1.0, 120)
    calc = calculator.E2FormerCalculator(model=m, head_name="omol25", charge=1, multiplicity=2, ref_energy=ref_table,
                                         device=str(cuda))
    sysin = dict(positions=torch.as_tensor(s["pos"], device=cuda), numbers=torch.as_tensor(s["Z"], device=cuda),
                 cell=torch.as_tensor(s["cell"][0], device=cuda), pbc=torch.as_tensor(s["pbc"][0], device=cuda))
    res = calc.calculate_batch([sysin])[0]
    assert res["energy"].is_cuda and res["forces"].is_cuda and res["energy"].dtype == torch.float64
    e_ref, f_ref = _oracle(om, s, [1], [2])
    n = len(s["pos"])
    ref_sum = float(ref_table[np.asarray(s["Z"])].sum())
    de = abs(float(res["energy"]) - (float(e_ref[0]) + ref_sum)) / n
    rel = float((res["forces"].cpu().double() - f_ref).norm() / f_ref.norm())
    e0, _ = _oracle(om, s, [0], [1])
    print(f"[calculator torch] |dE|/atom={de:.3e} force relL2={rel:.3e} "
          f"charge effect={abs(float(e_ref[0] - e0[0])):.3e} eV", flush=True)
    assert de < 1e-5 and rel < 1e-4
    assert abs(float(e_ref[0] - e0[0])) > 1e-6
    calc.calculate(sysin, ["energy", "forces"])
    assert torch.equal(calc.results["energy"], res["energy"]) and torch.equal(calc.results["forces"], res["forces"])


def test_calculator_host_path_wraps_and_batches(pkg, cuda):
    """Host path (ase.Atoms-style input): periodic systems are wrapped into the
    primary cell, charge = sum of initial charges, multiplicity 1
    (interface/data_utils.py:20-33); a ragged batch of two systems, one periodic
    and shifted out of its cell, one molecule; numpy results against the oracle
    on the wrapped positions."""
    from ubio_molfm_amd import calculator, systems
    m, om = _pair(cuda, seed=12)
    w = systems.small_water(8, 6.2, seed=6)
    mol = systems.organics_batch(n_mol=1, nmin=12, nmax=16, seed=7)
    pw = np.asarray(w["pos"], np.float64) + np.array([7.0, -3.5, 13.0])
    a1 = _AseLike(pw, np.asarray(w["Z"]), np.asarray(w["cell"][0], np.float64), np.array([True] * 3),
                  np.r_[np.ones(2), np.zeros(len(pw) - 2)])
    a2 = _AseLike(np.asarray(mol["pos"], np.float64), np.asarray(mol["Z"]), np.zeros((3, 3)), np.zeros(3, bool),
                  np.zeros(len(mol["pos"])))
    calc = calculator.E2FormerCalculator(model=m, head_name="omol25", charge=5, multiplicity=3, device=str(cuda))
    out = calc.calculate_batch([a1, a2])
    table = calculator.head_ref_energy("omol25")          # added by default (add_ref_energy=True)
    assert isinstance(out[0]["energy"], float) and isinstance(out[0]["forces"], np.ndarray)
    wrapped = calculator.hard_wrap(pw, w["cell"][0], [True] * 3).astype(np.float32)
    frac = wrapped.astype(np.float64) @ np.linalg.inv(np.asarray(w["cell"][0], np.float64))
    assert frac.min() > -1e-6 and frac.max() < 1.0
    for a, sysd, q in ((a1, dict(w, pos=wrapped), 2), (a2, mol, 0)):
        e_ref, f_ref = _oracle(om, sysd, [q], [1])
        r = out[0] if a is a1 else out[1]
        n = len(sysd["pos"])
        de = abs(r["energy"] - (float(e_ref[0]) + float(table[np.asarray(sysd["Z"])].sum()))) / n
        rel = float(np.linalg.norm(r["forces"] - f_ref.numpy()) / f_ref.norm())
        print(f"[calculator host] N={n} |dE|/atom={de:.3e} force relL2={rel:.3e}", flush=True)
        assert de < 1e-5 and rel < 1e-4


@pytest.mark.parametrize("head", ["omol25", "svp"])
def test_calculator_from_yaml_and_checkpoint(pkg, cuda, tmp_path, head):
    """The model lifecycle of model_interface.py:172-245: the calculator built
    from a flattened yaml (config_path = its directory, which holds exactly one
    yaml) and a {"model": state_dict} checkpoint (loaded with weights_only) on a
    two-head model; the head's energy plus the head's reference energies
    (atom_reference * unit, molfm/data/utils.py, added by default) against the
    oracle with the same weights plus the table sum, 1e-5 eV/atom and 1e-4
    force rel-L2.  svp exercises the kcal/mol -> eV unit and its own head."""
    import yaml
    from ubio_molfm_amd import calculator, model, systems
    from oracle.model import MolfmAtomic as OracleModel
    args = model.default_args(heads=("omol25", "svp"))
    raw = dict(backbone="e2former", backbone_config=dict(args.backbone_config), dataset_name_list="omol25,svp",
               head_cfg_str="", AutoGradForce=True)
    raw["backbone_config"].pop("name")
    cfg_dir = tmp_path / "run"
    cfg_dir.mkdir()
    (cfg_dir / "config.yaml").write_text(yaml.safe_dump(raw))
    torch.manual_seed(21)
    src = model.MolfmAtomic(calculator.model_args_from_config(raw))
    torch.save({"model": src.state_dict()}, cfg_dir / "ckpt.pt")
    calc = calculator.E2FormerCalculator(config_path=str(cfg_dir), checkpoint_path=str(cfg_dir / "ckpt.pt"),
                                         head_name=head, device=str(cuda))
    assert calc.config_file == str(cfg_dir / "config.yaml") and calc.add_ref_energy
    om = OracleModel(head_names=("omol25", "svp")).eval()
    om.load_state_dict(src.state_dict(), strict=True)
    s = systems.organics_batch(n_mol=1, nmin=14, nmax=18, seed=22)
    sysin = dict(positions=np.asarray(s["pos"], np.float64), numbers=np.asarray(s["Z"]), cell=np.zeros((3, 3)),
                 pbc=np.zeros(3, bool), charge=np.zeros(len(s["pos"])))
    r = calc.calculate_batch([sysin])[0]
    bd = systems.to_padded(s)
    bd["charge"] = torch.zeros(1, dtype=torch.int32)
    bd["multiplicity"] = torch.ones(1, dtype=torch.int32)
    o = om(bd, head=head)
    table = calculator.head_ref_energy(head)
    ref_sum = float(table[np.asarray(s["Z"])].sum())
    n = len(s["pos"])
    de = abs(r["energy"] - (float(o["pred_energy"][0]) + ref_sum)) / n
    fr = o["pred_forces"].detach()[bd["atom_masks"]].double()
    rel = float(np.linalg.norm(r["forces"] - fr.numpy()) / fr.norm())
    print(f"[calculator yaml+ckpt {head}] ref sum {ref_sum:.3f} eV |dE|/atom={de:.3e} force relL2={rel:.3e}",
          flush=True)
    assert abs(ref_sum) > 100.0
    assert de < 1e-5 and rel < 1e-4
    # config_name picks one of several yamls; without it the directory must hold exactly one
    (cfg_dir / "other.yaml").write_text(yaml.safe_dump(raw))
    with pytest.raises(ValueError, match="exactly one yaml"):
        calculator.E2FormerCalculator(config_path=str(cfg_dir), checkpoint_path=str(cfg_dir / "ckpt.pt"),
                                      head_name=head, device=str(cuda))
    calc2 = calculator.E2FormerCalculator(config_path=str(cfg_dir), config_name="config.yaml",
                                          checkpoint_path=str(cfg_dir / "ckpt.pt"), head_name=head,
                                          device=str(cuda), add_ref_energy=False)
    r2 = calc2.calculate_batch([sysin])[0]
    assert abs(r2["energy"] - (r["energy"] - ref_sum)) / n < 1e-5


def test_neighbor_info_reference_dict(pkg, cuda):
    """E2FormerBackbone.forward returns neighbor_info with the reference's keys
    (module_utils.py:3233-3242) in the caller's atom order, its expanded nodes
    in batched_data: the edge set (query atom, source atom, image position)
    and f_edge_vec / f_dist equal the oracle's construct_radius_neighbor output
    on the same padded periodic batch; query_idx is ascending, each row ordered
    by distance, and the metadata is the query / key CSR of the edge list."""
    from ubio_molfm_amd import systems
    from oracle.model import MolfmAtomic as OracleModel
    m, om = _pair(cuda, seed=13)
    s = systems.small_water(8, 6.2, seed=8)
    perm = np.random.default_rng(0).permutation(len(s["pos"]))
    s = dict(s, pos=s["pos"][perm], Z=s["Z"][perm])
    bd = {k: v.to(cuda) for k, v in systems.to_padded(s).items()}
    with torch.no_grad():
        out = m.decoder(bd)
    info = out["neighbor_info"]
    for k in ("query_idx", "neighbor_idx", "metadata", "f_edge_vec", "f_dist", "f_poly_dist"):
        assert k in info, k
    qi = info["query_idx"].cpu().numpy(); ni = info["neighbor_idx"].cpu().numpy()
    d = info["f_dist"].cpu().numpy()
    assert np.all(np.diff(qi) >= 0)
    for r in np.unique(qi):
        seg = d[qi == r]
        assert np.all(np.diff(seg) >= 0)
    outc = out["data"]["f_outcell_index"].cpu().numpy()
    expp = out["data"]["f_exp_node_pos"].cpu().numpy()
    assert np.array_equal(outc[:len(s["pos"])], np.arange(len(s["pos"])))
    ref_bd = systems.to_padded(s)
    om.decoder(ref_bd)                       # fills the reference neighbour info into ref_bd
    rq = ref_bd["query_idx"].long().numpy(); rn = ref_bd["neighbor_idx"].long().numpy()
    r_out = ref_bd["f_outcell_index"].long().numpy(); r_exp = ref_bd["f_exp_node_pos"].detach().numpy()

    def canon(q, j, img, vec, dist):
        o = np.lexsort((img[:, 2], img[:, 1], img[:, 0], j, q))
        return q[o], j[o], img[o], vec[o], dist[o]
    got = canon(qi, outc[ni], expp[ni], info["f_edge_vec"].cpu().numpy(), d)
    ref = canon(rq, r_out[rn], r_exp[rn], ref_bd["f_edge_vec"].detach().numpy(), ref_bd["f_dist"].detach().numpy())
    print(f"[neighbor_info] E={len(qi)} oracle E={len(rq)} M={len(outc)} oracle M={len(r_out)}", flush=True)
    assert len(qi) == len(rq)
    assert np.array_equal(got[0], ref[0]) and np.array_equal(got[1], ref[1])
    assert np.allclose(got[2], ref[2], atol=1e-5)
    assert np.allclose(got[3], ref[3], atol=1e-5) and np.allclose(got[4], ref[4], atol=1e-5)
    q_ptr, q_col, q_perm, k_ptr, k_col, k_perm = [t.cpu().numpy() for t in info["metadata"]]
    assert np.array_equal(np.diff(q_ptr), np.bincount(qi, minlength=len(s["pos"])))
    assert np.array_equal(q_col, ni) and np.array_equal(q_perm, np.arange(len(qi)))
    assert np.array_equal(k_perm, np.argsort(ni, kind="stable")) and np.array_equal(k_col, qi[k_perm])
    assert np.array_equal(np.diff(k_ptr), np.bincount(ni, minlength=len(outc)))


def test_md_matches_oracle_nve_step(pkg, cuda):
    """md.VelocityVerlet (FixCom every step) against the restated reference
    step (oracle.md.nve_step, torch_langevin.py:192-283 with fr = 0 and the
    FixCom constraint) for 5 steps on a periodic water cell, with the same HIP
    force evaluation in both; positions and momenta agree to 1e-10."""
    from ubio_molfm_amd import md, systems
    from oracle import md as omd
    m, _ = _pair(cuda, seed=14)
    s = systems.small_water(8, 6.2, seed=9)
    integ = md.VelocityVerlet(m, s, cuda, dt_fs=1.0, T=300.0, seed=2)
    mass = integ.m[:, 0]
    x, p = integ.x.clone(), integ.p.clone()
    fn = lambda y: integ.forces_at(y)[1]
    f = fn(x)
    for step in range(5):
        integ.step()
        integ.sync()
        x, p, f = omd.nve_step(x, p, mass, f, fn, integ.dt, fixcom=True)
        dx = float((integ.x - x).abs().max()); dp = float((integ.p - p).abs().max())
        print(f"[md vs oracle step {step}] |dx|={dx:.2e} |dp|={dp:.2e}", flush=True)
        assert dx < 1e-10 and dp < 1e-10
    cm = (integ.m * integ.x).sum(0) / integ.m.sum()
    cm0 = (integ.m * torch.as_tensor(np.asarray(s["pos"], np.float64), device=cuda)).sum(0) / integ.m.sum()
    assert float((cm - cm0).abs().max()) < 1e-10 and float(integ.p.sum(0).abs().max()) < 1e-10


def test_md_capacity_builds_match_exact_and_recover_from_overflow(pkg, cuda):
    """The MD loop's capacity builds (edge arrays sized from the previous count,
    counters checked one step later: no host readback per step) give bitwise the
    trajectory of exact builds; a capacity too small for the list is detected at
    the next step and that step recomputed with an exact build."""
    from ubio_molfm_amd import md, systems
    m, _ = _pair(cuda, seed=14)
    s = systems.small_water(8, 6.2, seed=9)
    ref = md.VelocityVerlet(m, s, cuda, dt_fs=1.0, T=300.0, seed=2, lagged=False)
    lag = md.VelocityVerlet(m, s, cuda, dt_fs=1.0, T=300.0, seed=2)
    small = md.VelocityVerlet(m, s, cuda, dt_fs=1.0, T=300.0, seed=2)
    for k in range(6):
        ref.step(); lag.step(); small.step()
        if k == 1:
            small.sync()
            small.capacity = (small.n_edges - 10, small.capacity[1])      # the next build overflows
        if k == 3:
            small.sync()
            small.capacity = (small.capacity[0], 8)                        # rows longer than 8 overflow
    lag.sync(); small.sync()
    print(f"[md capacity] edges {lag.edge_counts} redone {lag.redone} / {small.redone}", flush=True)
    assert lag.last_nl.stats is not None and ref.last_nl.stats is None
    assert torch.equal(ref.x, lag.x) and torch.equal(ref.p, lag.p) and torch.equal(ref.f, lag.f)
    assert torch.equal(ref.x, small.x) and torch.equal(ref.p, small.p) and torch.equal(ref.f, small.f)
    assert ref.edge_counts == lag.edge_counts == small.edge_counts
    assert lag.redone == 0 and small.redone == 2


@pytest.mark.parametrize("tp", ["QKdot_alpha", "QKdotS_alpha"])
def test_md_capacity_builds_qkdot_gates(pkg, cuda, tp):
    """Capacity builds with the QKdot gates, whose per-edge kernels
    (e2v2_radial_eval and its backward) run over every edge slot: slots past the
    real edges (never written by the build) are bounded on the device by
    row_ptr[N] and not read, and the trajectory equals that of exact builds
    bitwise over 4 steps."""
    from ubio_molfm_amd import md, model, systems
    torch.manual_seed(16)
    args = model.default_args()
    args.backbone_config.update(tp_type=tp)
    m = model.MolfmAtomic(args).eval().to(cuda)
    s = systems.small_water(8, 6.2, seed=9)
    ref = md.VelocityVerlet(m, s, cuda, dt_fs=1.0, T=300.0, seed=2, lagged=False)
    lag = md.VelocityVerlet(m, s, cuda, dt_fs=1.0, T=300.0, seed=2)
    for _ in range(4):
        ref.step(); lag.step()
    lag.sync()
    nl = lag.last_nl
    real = int(nl.row_ptr[-1])
    print(f"[md capacity {tp}] slots {nl.n_edges} edges {real} redone {lag.redone}", flush=True)
    assert nl.stats is not None and nl.n_edges > real
    assert torch.equal(ref.x, lag.x) and torch.equal(ref.p, lag.p) and torch.equal(ref.f, lag.f)


def test_md_hip_graph_matches_eager_bitwise(pkg, cuda):
    """graph=True: after one eager step each step is one launch of the captured
    step graph.  Every replay (with the eager run's work and synchronisations
    between them) equals the eager capacity-build trajectory bitwise in positions,
    momenta, forces and energies over 6 steps; a capacity too small for the list,
    set after step 3, overflows inside the graph, is detected before the next
    launch, redone from the graph's backup with an exact build and captured again.
    evaluate_only: graphed evaluations at fixed positions equal eager ones."""
    from ubio_molfm_amd import md, systems
    m, _ = _pair(cuda, seed=14)
    s = systems.small_water(8, 6.2, seed=9)
    ref = md.VelocityVerlet(m, s, cuda, dt_fs=1.0, T=300.0, seed=2)
    gr = md.VelocityVerlet(m, s, cuda, dt_fs=1.0, T=300.0, seed=2, graph=True)
    for k in range(6):
        ref.step(); gr.step()
        ref.sync(); gr.sync()
        same = [torch.equal(a, b) for a, b in ((ref.x, gr.x), (ref.p, gr.p), (ref.f, gr.f), (ref.e, gr.e))]
        print(f"[md graph step {k}] launches {gr.graph_launches} captures {gr.captures} redone {gr.redone} "
              f"bitwise {same}", flush=True)
        assert all(same)
        if k == 3:
            gr.capacity = (gr.n_edges - 10, gr.capacity[1])             # the next (graphed) build overflows
    assert gr.graph_launches == 5 and gr.redone == 1 and gr.captures == 3
    assert ref.edge_counts == gr.edge_counts
    ev = md.VelocityVerlet(m, s, cuda, seed=2, evaluate_only=True)
    eg = md.VelocityVerlet(m, s, cuda, seed=2, evaluate_only=True, graph=True)
    for k in range(4):
        ev.step(); eg.step()
    ev.sync(); eg.sync()
    assert eg.graph_launches == 3 and torch.equal(ev.f, eg.f) and torch.equal(ev.e, eg.e)
    assert torch.equal(ev.x, eg.x) and torch.equal(eg.x, torch.as_tensor(np.asarray(s["pos"], np.float64), device=cuda))
