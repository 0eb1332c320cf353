"""Build libe2v2.so in-tree with hipcc for gfx950.

The shared library lands next to this file (``ubio-molfm_amd/libe2v2.so``)
so that it travels with the repository snapshot to the GPU box.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libe2v2.so"
SOURCES = ["api.hip", "nbr.hip", "radial.hip", "attn.hip", "deg.hip", "node.hip", "proj.hip", "sparse.hip", "gemm.hip", "qkdot.hip"]
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def regenerate_tables() -> None:
    sys.path.insert(0, str(HERE))
    try:
        import so3  # noqa: WPS433 (local module)
    finally:
        sys.path.pop(0)
    text = so3.render_tp_header()
    path = CSRC / "tp_table.h"
    if not path.exists() or path.read_text() != text:
        path.write_text(text)


def build(verbose: bool = False) -> Path:
    regenerate_tables()
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, *FLAGS, "-o", str(tmp), *[str(CSRC / s) for s in SOURCES]]
    res = subprocess.run(cmd, cwd=str(CSRC), capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-6000:]}")
    if verbose:
        noise = "is not a recognized feature for this target"
        print("\n".join(l for l in res.stderr.splitlines() if noise not in l and l.strip()))
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
