"""E2FormerCalculator: ASE-calculator-shaped energy + forces entry point.

Mirrors src/molfm/interface/ase/calculator/e2former_calculator.py:32-269 and
the model lifecycle of src/molfm/interface/model_interface.py:64-281:

* constructor keywords of the reference (``config_path``, ``config_name``,
  ``checkpoint_path``, ``head_name``, ``device``, ``force_use_aperiodic``,
  ``add_ref_energy``, ``charge``, ``multiplicity``, ...); the compile / TF32 /
  FAISS / recompute keywords are accepted and have nothing to switch here;
* config resolution: ``config_path`` may be the yaml itself or its directory,
  ``config_name`` picks a file in it, otherwise the directory must hold exactly
  one yaml (model_interface.py:172-213); the flattened yaml is read with
  ``yaml.safe_load`` into the model arguments (model_interface.py:203-207);
* checkpoints: ``torch.load(..., weights_only=True)["model"]`` loaded with
  ``strict=False`` (model_interface.py:233-235);
* ``calculate(atoms, properties)`` sets ``results`` from ``calculate_batch``
  (:96-107); ``calculate_batch`` dispatches on the input flavour (:109-132):
  - torch inputs (dicts of device tensors, or objects exposing
    ``_torch_positions`` / ``_torch_numbers`` like TorchAtoms) take the
    device path: positions as given, the calculator's ``charge`` and
    ``multiplicity`` in the batch (:144-178), device tensors back (:180-198);
  - ASE ``Atoms`` (``get_positions``) or numpy dicts take the host path:
    periodic systems wrapped into the primary cell first (:239-246, ASE's
    ``wrap`` with eps = 1e-7), charge = sum of the initial charges and
    multiplicity 1 (interface/data_utils.py:20-33), numpy / float back;
* per-atom reference energies: with ``add_ref_energy`` (the default) the sum
  of ``ref_energy[Z]`` is added per system (:187-192, :255-260), where
  ``ref_energy = atom_reference * unit`` of the head (model_interface.py:208-223):
  the per-head tables of molfm/data/utils.py ``get_data_defult_config``,
  shipped as data in ``atom_reference.json`` and matched on ``head_name``
  as that function does (``startswith("svp")``, ``startswith("tzvpd")``,
  ``== "oc20"``, ``== "omol25"``, ``== "oc22"`` on the lower-cased name, in that
  order; any other name: zeros, unit 1).  An explicit ``ref_energy`` (eV per
  atomic number) replaces the head's table.  The sum is formed on the host in
  float64 (deterministic; the energy is then float64, as the reference's
  float32 + float64 sum is).
"""
from __future__ import annotations

import json
import os
from pathlib import Path
from types import SimpleNamespace
from typing import Any, Dict, List, Optional

import numpy as np
import torch
import yaml

from .model import MolfmAtomic, default_args

ALL_CHANGES = ["positions", "numbers", "cell", "pbc", "initial_charges", "initial_magmoms"]

_ATOM_REF = None


def atom_reference(head_name: str):
    """(atom_reference [n] float64, unit) of a head: the first table of
    ``atom_reference.json`` whose test matches ``head_name.lower()``
    (molfm/data/utils.py:17-289), else the default (zeros, unit 1)."""
    global _ATOM_REF
    if _ATOM_REF is None:
        _ATOM_REF = json.loads((Path(__file__).resolve().parent / "atom_reference.json").read_text())
    name = str(head_name).lower()
    for h in _ATOM_REF["heads"]:
        if (h["match"] == "startswith" and name.startswith(h["key"])) or (h["match"] == "eq" and name == h["key"]):
            return np.asarray(h["atom_reference"], np.float64), float(h["unit"])
    d = _ATOM_REF["default"]
    return np.asarray(d["atom_reference"], np.float64), float(d["unit"])


def head_ref_energy(head_name: str) -> np.ndarray:
    """ref_energy = atom_reference * unit of the head (model_interface.py:222), eV per Z."""
    ref, unit = atom_reference(head_name)
    return ref * unit


def resolve_config_file(config_path: Optional[str], config_name: Optional[str],
                        checkpoint_path: Optional[str]) -> str:
    """model_interface.py:172-213."""
    config_dir = config_path
    if config_dir is None:
        if checkpoint_path in (None, "none"):
            raise ValueError("Cannot resolve the config yaml: no config_path and no checkpoint directory "
                             "to fall back on.")
        config_dir = os.path.dirname(os.path.abspath(checkpoint_path))
    else:
        config_dir = os.path.abspath(config_dir)
        if os.path.isfile(config_dir):
            if config_name is None:
                return config_dir
            config_dir = os.path.dirname(config_dir)
        if not os.path.isdir(config_dir):
            raise FileNotFoundError(f"Config path {config_dir} does not exist.")
    if config_name is not None:
        cand = Path(config_name)
        if not cand.is_absolute():
            cand = Path(config_dir) / cand
        if cand.is_file():
            return str(cand)
        raise FileNotFoundError(f"Config file {cand} does not exist in {config_dir}.")
    ymls = sorted(os.path.join(config_dir, n) for n in os.listdir(config_dir) if n.endswith((".yaml", ".yml")))
    if len(ymls) != 1:
        raise ValueError(f"Expected exactly one yaml file in {config_dir}, found {len(ymls)}: {ymls}")
    return ymls[0]


def model_args_from_config(raw: Dict[str, Any]) -> SimpleNamespace:
    """The flattened training yaml (``SmallMolConfig`` fields,
    tasks/pretrain_smallmol.py:95-167) as model arguments: ``backbone_config``,
    ``dataset_name_list``, ``head_cfg_str``, ``AutoGradForce``."""
    args = default_args()
    bb = raw.get("backbone_config")
    if bb is None:
        raise ValueError("config yaml has no backbone_config")
    args.backbone_config = dict(bb)
    args.backbone_config.setdefault("name", raw.get("backbone", "e2former"))
    for k in ("dataset_name_list", "head_cfg_str", "AutoGradForce"):
        if k in raw:
            setattr(args, k, raw[k])
    return args


def _complete_cell(cell: np.ndarray) -> np.ndarray:
    """Cell with zero lattice vectors replaced by unit vectors orthogonal to the
    others (ASE's ``complete_cell``), so fractional coordinates exist."""
    A = np.array(cell, np.float64).reshape(3, 3)
    missing = [i for i in range(3) if np.linalg.norm(A[i]) < 1e-12]
    if len(missing) == 3:
        return np.eye(3)
    if len(missing) == 2:
        i = [k for k in range(3) if k not in missing][0]
        u = A[i] / np.linalg.norm(A[i])
        t = np.eye(3)[int(np.argmin(np.abs(u)))]
        a = np.cross(u, t); a /= np.linalg.norm(a)
        b = np.cross(u, a)
        A[missing[0]], A[missing[1]] = a, b
        if np.linalg.det(A) < 0:
            A[missing[1]] = -b
    elif len(missing) == 1:
        i, j = [k for k in range(3) if k not in missing]
        c = np.cross(A[i], A[j]); c /= np.linalg.norm(c)
        A[missing[0]] = c if np.linalg.det(np.stack([A[i], A[j], c])) > 0 else -c
    return A


def hard_wrap(pos: np.ndarray, cell: np.ndarray, pbc, eps: float = 1e-7) -> np.ndarray:
    """ASE ``Atoms.wrap()`` (``wrap_positions`` with eps 1e-7): fractional
    coordinates of the periodic directions mapped to [-eps, 1 - eps)."""
    pbc = np.asarray(pbc, bool).reshape(3)
    A = _complete_cell(cell)
    frac = np.linalg.solve(A.T, np.asarray(pos, np.float64).T).T
    shift = -eps
    for d in range(3):
        if pbc[d]:
            frac[:, d] = np.mod(frac[:, d] - shift, 1.0) + shift
    return frac @ A


def _torch_flavour(a) -> bool:
    if hasattr(a, "_torch_positions"):
        return True
    return isinstance(a, dict) and isinstance(a.get("positions"), torch.Tensor)


def _system(a) -> Dict[str, Any]:
    """positions / numbers / cell / pbc / charge of one input system."""
    if hasattr(a, "_torch_positions"):                     # TorchAtoms
        cell = a.get_cell() if hasattr(a, "get_cell") else getattr(a, "_torch_cell", None)
        pbc = a.get_pbc() if hasattr(a, "get_pbc") else getattr(a, "pbc", None)
        return dict(positions=a._torch_positions, numbers=a._torch_numbers, cell=cell, pbc=pbc, charge=None)
    if hasattr(a, "get_positions"):                        # ase.Atoms
        ch = a.get_initial_charges() if hasattr(a, "get_initial_charges") else np.zeros(len(a.get_positions()))
        return dict(positions=a.get_positions(), numbers=a.get_atomic_numbers(), cell=np.asarray(a.get_cell()),
                    pbc=np.asarray(a.get_pbc()), charge=float(np.sum(ch)))
    return dict(a)


def _np(x, dtype):
    if x is None:
        return None
    if isinstance(x, torch.Tensor):
        return x.detach().cpu().numpy().astype(dtype)
    return np.asarray(x, dtype)


class E2FormerCalculator:
    implemented_properties = ["energy", "forces"]
    discard_results_on_any_change = True
    default_parameters: Dict[str, Any] = {}

    def __init__(self, restart=None, ignore_bad_restart=False, label="e2former-calc", atoms=None, command=None,
                 config_path: Optional[str] = None, config_name: Optional[str] = None,
                 checkpoint_path: Optional[str] = None, head_name: Optional[str] = None, device: str = "cuda:0",
                 use_compile: bool = False, use_tf32: bool = False, use_faiss: bool = True,
                 recompute_budget: float = -1.0, force_use_aperiodic: bool = False, add_ref_energy: bool = True,
                 auto_setup: bool = True, charge: int = 0, multiplicity: int = 1,
                 model: Optional[MolfmAtomic] = None, ref_energy=None, compute_dtype: str = "fp32", **kwargs):
        self.label = label
        self.atoms = atoms
        self.results: Dict[str, Any] = {}
        self.force_use_aperiodic = force_use_aperiodic
        self.add_ref_energy = add_ref_energy
        self.charge, self.multiplicity = int(charge), int(multiplicity)
        self.config_path, self.config_name, self.checkpoint_path = config_path, config_name, checkpoint_path
        self.head_name = head_name
        self.device = torch.device(device)
        self.use_compile, self.use_tf32, self.use_faiss = use_compile, use_tf32, use_faiss
        self.recompute_budget = recompute_budget
        self.config_file = None
        self.model = None
        if ref_energy is not None:
            self.ref_energy = np.asarray(_np(ref_energy, np.float64), np.float64)
        elif head_name is not None:
            self.ref_energy = head_ref_energy(head_name)
        else:
            self.ref_energy = None
        if model is not None:
            self.model = model.eval().to(self.device).requires_grad_(False)
        elif auto_setup:
            self.setup_model_interface()
        if self.model is not None:
            self.model.decoder.set_compute_dtype(compute_dtype)

    # -- model lifecycle (model_interface.py:120-245) ---------------------------
    def setup_model_interface(self):
        if self.head_name is None:
            raise ValueError("Missing model interface init args: head_name")
        if self.checkpoint_path in (None, "none"):
            if self.config_path is None and self.config_name is None:
                raise ValueError("checkpoint_path is None/'none' (random weights). Pass config_path or "
                                 "config_name explicitly.")
        elif not os.path.exists(self.checkpoint_path):
            raise FileNotFoundError(f"Checkpoint path {self.checkpoint_path} does not exist.")
        self.config_file = resolve_config_file(self.config_path, self.config_name, self.checkpoint_path)
        with open(self.config_file, "r", encoding="utf-8") as f:
            raw = yaml.safe_load(f)
        model = MolfmAtomic(model_args_from_config(raw))
        if self.checkpoint_path not in (None, "none"):
            sd = torch.load(self.checkpoint_path, map_location="cpu", weights_only=True)
            model.load_state_dict(sd["model"] if "model" in sd else sd, strict=False)
        self.model = model.eval().to(self.device).requires_grad_(False)

    # -- ASE calculator surface --------------------------------------------------
    def calculate(self, atoms=None, properties=None, system_changes=ALL_CHANGES, symmetry="c1"):
        if properties is None:
            properties = ["energy"]
        for prop in properties:
            if prop not in self.implemented_properties:
                raise ValueError(f"Property {prop} is not implemented")
        if atoms is not None:
            self.atoms = atoms
        if self.atoms is None:
            raise RuntimeError("An Atoms object must be provided")
        self.results = self.calculate_batch([self.atoms], properties=properties)[0]

    def get_property(self, name: str, atoms=None):
        self.calculate(atoms, [name])
        return self.results[name]

    def get_potential_energy(self, atoms=None, force_consistent=False):
        return self.get_property("energy", atoms)

    def get_forces(self, atoms=None):
        return self.get_property("forces", atoms)

    # -- batched evaluation -------------------------------------------------------
    def calculate_batch(self, atoms_list: Optional[List[Any]] = None,
                        properties: Optional[List[str]] = None) -> List[Dict[str, Any]]:
        if not atoms_list:
            return []
        if properties is None:
            properties = ["energy", "forces"]
        torch_path = _torch_flavour(atoms_list[0])
        systems = [_system(a) for a in atoms_list]
        pos, Z, cells, pbcs, ptr, charges = [], [], [], [], [0], []
        for s in systems:
            n = len(s["positions"])
            cell = _np(s.get("cell"), np.float32)
            cell = np.zeros((3, 3), np.float32) if cell is None else cell.reshape(3, 3)
            pbc = _np(s.get("pbc"), bool)
            pbc = np.zeros(3, bool) if pbc is None else pbc.reshape(3)
            if self.force_use_aperiodic:
                cell, pbc = np.zeros((3, 3), np.float32), np.zeros(3, bool)
            if torch_path:
                p = torch.as_tensor(s["positions"], device=self.device).to(torch.float32).reshape(-1, 3)
                charges.append(self.charge)
            else:
                p = _np(s["positions"], np.float64)
                if pbc.any():
                    p = hard_wrap(p, cell, pbc)
                p = torch.as_tensor(p.astype(np.float32), device=self.device)
                ch = s.get("charge", None)
                charges.append(int(float(_np(ch, np.float64).sum())) if ch is not None else 0)   # int32 cast truncates
            pos.append(p)
            Z.append(torch.as_tensor(s["numbers"], device=self.device).to(torch.int64).reshape(-1))
            cells.append(cell); pbcs.append(pbc)
            ptr.append(ptr[-1] + n)
        B = len(systems)
        charge = torch.as_tensor(charges, dtype=torch.int64, device=self.device)
        mult = torch.full((B,), self.multiplicity if torch_path else 1, dtype=torch.int64, device=self.device)
        P = torch.cat(pos)
        Zt = torch.cat(Z)
        ptr = np.asarray(ptr)
        # forces are always evaluated, as in the reference (MolfmAtomic.forward ignores need_force and the
        # output processing returns pred_forces whenever present, :180-198)
        e, f, _ = self.model.energy_forces_flat(P, Zt, ptr, np.stack(cells), np.stack(pbcs), head=self.head_name,
                                                charge=charge, multiplicity=mult)
        ref = None
        if self.add_ref_energy and self.ref_energy is not None:
            zs = Zt.cpu().numpy()
            if zs.size and (zs.min() < 0 or zs.max() >= len(self.ref_energy)):
                raise IndexError(f"reference energies of head {self.head_name!r} cover Z < {len(self.ref_energy)}, "
                                 f"got Z = {int(zs.max())}")
            ref = np.array([self.ref_energy[zs[ptr[g]:ptr[g + 1]]].sum() for g in range(B)], np.float64)
        out = []
        for g in range(B):
            eg = e[g]
            if ref is not None:
                eg = eg.double() + float(ref[g])
            r: Dict[str, Any] = {}
            if torch_path:
                r["energy"] = eg.detach()
                if f is not None:
                    r["forces"] = f[ptr[g]:ptr[g + 1]].detach()
            else:
                r["energy"] = float(eg)
                if f is not None:
                    r["forces"] = f[ptr[g]:ptr[g + 1]].detach().cpu().numpy()
            out.append(r)
        return out
