"""The no-allocation neighbour count (e2v2_nbr_count_noalloc, bin workspace in the
library's static device scratch) against the workspace entry points
e2v2_nbr_bin + e2v2_nbr_count on the same plan: identical row counts, row
pointers and stats, bit for bit, on two calls in a row with the second one
smaller (the scratch keeps the first call's contents; everything the count
reads is rebuilt or cleared by the call)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _with_workspace(pkg, pos, s):
    from ubio_molfm_amd import _lib, neighbors
    plan, keep, _, _ = neighbors.make_plan(pos, s["graph_ptr"], s["cell"], s["pbc"], 6.0)
    N = pos.shape[0]
    st = _lib.vp(torch.cuda.current_stream().cuda_stream)
    row_count = torch.empty(max(N, 1), dtype=torch.int32, device=pos.device)
    row_ptr = torch.empty(N + 1, dtype=torch.int32, device=pos.device)
    _lib.call("e2v2_nbr_bin", _lib.C.byref(plan), st)
    _lib.call("e2v2_nbr_count", _lib.C.byref(plan), _lib.vp(row_count.data_ptr()), _lib.vp(row_ptr.data_ptr()), st)
    return row_count[:N], row_ptr, keep["stats"]


def test_noalloc_count_matches_workspace_entry_points(pkg, cuda):
    from ubio_molfm_amd import neighbors, systems
    cases = [("cfg3", systems.CONFIGS[3]()), ("small-water", systems.small_water(8, 6.2, seed=1))]
    for label, s in cases:
        pos = torch.as_tensor(s["pos"], device=cuda)
        rc0, rp0, st0 = _with_workspace(pkg, pos, s)
        rc1, rp1, st1 = neighbors.count_neighbors_noalloc(pos, s["graph_ptr"], s["cell"], s["pbc"], 6.0)
        nl = neighbors.build_neighbors(pos, s["graph_ptr"], s["cell"], s["pbc"], 6.0)
        print(f"[noalloc {label}] N={pos.shape[0]} E={int(st1[0])} (workspace {int(st0[0])}, list {nl.n_edges}) "
              f"max_row={int(st1[1])} outside={int(st1[2])}", flush=True)
        # (the workspace plan's stats hold a fourth counter, the capacity build's overflow flag)
        assert torch.equal(rc0, rc1) and torch.equal(rp0, rp1) and torch.equal(st0[:3], st1)
        assert int(st1[0]) == nl.n_edges and int(st1[2]) == 0
        assert torch.equal(rp1, nl.row_ptr)
