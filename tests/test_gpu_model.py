"""End-to-end parity of the MI355X model (HIP edge path) with the CPU oracle,
which restates the reference's own formulation (Wigner node frames, SO(2)
product, torch fallbacks).  Gates from the north star: fp32 per-atom energy
within 1e-5 eV/atom, forces within 1e-4 relative L2."""
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


def _compare(m, om, sysd, cuda, label):
    from ubio_molfm_amd import systems
    pos = torch.as_tensor(sysd["pos"], device=cuda)
    Z = torch.as_tensor(sysd["Z"], device=cuda)
    e, f, nl = m.energy_forces_flat(pos, Z, sysd["graph_ptr"], sysd["cell"], sysd["pbc"])
    r = om(systems.to_padded(sysd))
    ptr = np.asarray(sysd["graph_ptr"])
    n = np.diff(ptr)
    e_ref = r["pred_energy"].detach().double()
    de = float(((e.cpu().double() - e_ref).abs() / torch.as_tensor(n, dtype=torch.float64)).max())
    mask = systems.to_padded(sysd)["atom_masks"]
    f_ref = r["pred_forces"].detach()[mask]
    rel = float((f.cpu().double() - f_ref.double()).norm() / f_ref.double().norm())
    print(f"[model {label}] N={len(sysd['pos'])} E={nl.n_edges} |dE|/atom={de:.3e} force relL2={rel:.3e} "
          f"E={e.cpu().numpy()[:3]}", flush=True)
    assert de < 1e-5 and rel < 1e-4


def test_model_small_water(pkg, cuda):
    from ubio_molfm_amd import systems
    m, om = _pair(cuda)
    _compare(m, om, systems.small_water(8, 6.2, seed=2), cuda, "small-water")


def test_model_ragged_batch(pkg, cuda):
    from ubio_molfm_amd import systems
    m, om = _pair(cuda, seed=1)
    _compare(m, om, systems.organics_batch(n_mol=4, nmin=10, nmax=30, seed=3), cuda, "organics4")


def test_model_water_cfg1(pkg, cuda):
    from ubio_molfm_amd import systems
    m, om = _pair(cuda, seed=2)
    _compare(m, om, systems.CONFIGS[1](), cuda, "cfg1")


def test_reference_interface_padded(pkg, cuda):
    """The padded batched_data interface returns the same energies/forces."""
    from ubio_molfm_amd import systems
    m, om = _pair(cuda, seed=3)
    sysd = systems.organics_batch(n_mol=3, nmin=8, nmax=20, seed=4)
    bd = {k: v.to(cuda) for k, v in systems.to_padded(sysd).items()}
    res = m(bd)
    pos = torch.as_tensor(sysd["pos"], device=cuda)
    e, f, _ = m.energy_forces_flat(pos, torch.as_tensor(sysd["Z"], device=cuda), sysd["graph_ptr"], sysd["cell"],
                                   sysd["pbc"])
    mask = bd["atom_masks"]
    assert torch.allclose(res["pred_energy"].detach(), e, rtol=1e-6, atol=1e-6)
    assert torch.allclose(res["pred_forces"][mask], f, rtol=1e-5, atol=1e-7)
