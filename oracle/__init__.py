"""CPU oracle for the E2Former-V2 sparse equivariant attention path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package may import, link or
execute anything under ``oracle/``; only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker.

Contents
--------
cg.py         e3nn Clebsch-Gordan / real-basis / Wigner-D restatement (float64)
neighbors.py  exact fp32 radius-graph oracle (numpy) + dense restatement of the
              reference CellExpander / construct_radius_neighbor (torch)
model.py      torch CPU restatement of E2former (reference module tree and
              parameter names, Wigner/SO(2) node-frame route) + energy head and
              autograd forces

Parity status of each function is listed in the module docstrings; a function
with no independent pin says "parity unpinned".
"""
