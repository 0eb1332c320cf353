"""E2FormerCalculator-style batched energy + forces.

Mirrors ``E2FormerCalculator.calculate_batch`` of the reference
(src/molfm/interface/ase/calculator/e2former_calculator.py:109-198): a list of
systems in, a list of {"energy", "forces"} out.  Systems are dicts with
``positions`` [n,3], ``numbers`` [n], optional ``cell`` [3,3] and ``pbc`` [3]
(torch tensors or numpy arrays), or ASE ``Atoms`` when ase is importable.
Torch inputs get device tensors back (the TorchAtoms path); numpy / ASE inputs
get numpy arrays (the ASE path).  Periodic systems are wrapped into the primary
cell first, as the reference's ASE path does.
"""
from __future__ import annotations

from typing import Any, Dict, List, Optional

import numpy as np
import torch
import yaml

from .model import MolfmAtomic, default_args


def _to_system(a: Any):
    if hasattr(a, "get_positions"):  # ase.Atoms
        return dict(positions=a.get_positions(), numbers=a.get_atomic_numbers(), cell=np.asarray(a.get_cell()),
                    pbc=np.asarray(a.get_pbc())), False
    is_torch = isinstance(a["positions"], torch.Tensor)
    return a, is_torch


def _as_np(x, dtype):
    if isinstance(x, torch.Tensor):
        return x.detach().cpu().numpy().astype(dtype)
    return np.asarray(x, dtype)


class E2FormerCalculator:
    implemented_properties = ["energy", "forces"]

    def __init__(self, config_path: Optional[str] = None, checkpoint_path: Optional[str] = None,
                 head_name: Optional[str] = None, device: str = "cuda:0", model: Optional[MolfmAtomic] = None,
                 ref_energy: Optional[np.ndarray] = None, **unused):
        self.device = torch.device(device)
        if model is None:
            args = default_args()
            if config_path is not None:
                with open(config_path, "r", encoding="utf-8") as f:
                    raw = yaml.safe_load(f)
                bb = raw.get("backbone_config", raw)
                args.backbone_config.update(bb)
                if "dataset_name_list" in raw:
                    args.dataset_name_list = raw["dataset_name_list"]
            model = MolfmAtomic(args)
            if checkpoint_path not in (None, "none"):
                sd = torch.load(checkpoint_path, map_location="cpu", weights_only=True)
                model.load_state_dict(sd.get("model", sd), strict=False)
        self.model = model.eval().to(self.device).requires_grad_(False)  # force evaluation only
        self.head_name = head_name
        self.ref_energy = None if ref_energy is None else torch.as_tensor(ref_energy, device=self.device)

    def calculate_batch(self, atoms_list: List[Any], properties: Optional[List[str]] = None) -> List[Dict[str, Any]]:
        if not atoms_list:
            return []
        systems = [_to_system(a) for a in atoms_list]
        torch_path = systems[0][1]
        pos, Z, cells, pbcs, ptr = [], [], [], [], [0]
        for s, _ in systems:
            p = _as_np(s["positions"], np.float32)
            cell = _as_np(s.get("cell", np.zeros((3, 3))), np.float32).reshape(3, 3)
            pbc = _as_np(s.get("pbc", np.zeros(3, bool)), bool).reshape(3)
            if pbc.all() and abs(np.linalg.det(cell)) > 1e-9:  # hard wrap into the primary cell
                frac = p @ np.linalg.inv(cell)
                p = ((frac - np.floor(frac)) @ cell).astype(np.float32)
            pos.append(p); Z.append(_as_np(s["numbers"], np.int64)); cells.append(cell); pbcs.append(pbc)
            ptr.append(ptr[-1] + len(p))
        P = torch.as_tensor(np.concatenate(pos), device=self.device)
        Zt = torch.as_tensor(np.concatenate(Z), device=self.device)
        e, f, _ = self.model.energy_forces_flat(P, Zt, np.array(ptr), np.stack(cells), np.stack(pbcs),
                                                head=self.head_name)
        if self.ref_energy is not None:
            e = e + torch.zeros_like(e).index_add(
                0, torch.repeat_interleave(torch.arange(len(ptr) - 1, device=self.device),
                                           torch.as_tensor(np.diff(ptr), device=self.device)),
                self.ref_energy[Zt].to(e.dtype))
        out = []
        for g in range(len(ptr) - 1):
            eg, fg = e[g], f[ptr[g]:ptr[g + 1]]
            out.append({"energy": eg, "forces": fg} if torch_path else
                       {"energy": float(eg), "forces": fg.detach().cpu().numpy()})
        return out
