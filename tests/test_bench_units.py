"""CPU checks of bench.py's accounting: the compulsory (reference-formulation)
bytes the roofline uses, the implementation byte counts per activation
storage type, the profile-traffic lookup's coverage, and the one-GPU guard."""
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


def test_attention_bytes_split_by_activation_type():
    N, E = 7, 53
    # fp32: every node / edge-list term at 4 bytes (the edge list once per 16-head slice, 8 slices), plus
    # the radial-table rows (6 per channel forward, 8 backward, 256 channels)
    fwd32 = 4 * (N * 128 * 8 * 2 + N * 9 * 256 + N * 20 * 256 + N * 3 * 128 + 8 * E * 6 + N + 1)
    assert bench.attn_fwd_bytes(N, E) == fwd32 + 4 * E * 256 * 6
    row32 = 4 * (N * 20 * 256 * 2 + N * 1024 * 3 + N * 9 * 256 + N * 3 * 128 + E * (8 * 6 + 256 + 8 * 4))
    col32 = 4 * (N * 20 * 256 + N * 1024 * 2 + N * 9 * 256 + 2 * N + E * (256 + 5))
    part32 = 4 * E * (8 * 4 + 4)
    assert bench.attn_bwd_bytes(N, E) == row32 + col32 + part32 + 4 * E * 256 * 8
    # bf16 storage halves exactly the activation terms: q, k, v, out, grad
    act_fwd = N * (128 * 8 * 2 + 9 * 256 + 20 * 256)
    assert bench.attn_fwd_bytes(N, E) - bench.attn_fwd_bytes(N, E, 2) == 2 * act_fwd
    act_bwd = N * (2 * 20 * 256 + 2 * 1024 + 9 * 256) + N * (20 * 256 + 1024)
    assert bench.attn_bwd_bytes(N, E) - bench.attn_bwd_bytes(N, E, 2) == 2 * act_bwd
    # the degree kernels read and write fp32 in both modes
    assert bench.deg_fwd_bytes(N, E, 2) == bench.deg_fwd_bytes(N, E)
    assert bench.deg_fwd_table_bytes(E) == 4 * E * 768 * 6 and bench.deg_bwd_table_bytes(E) == 4 * E * 768 * 8
    # the hidden-channel form reads half the table channels (3 x 128), over 4 slices, and writes hs [9][N][144]
    assert bench.deg_hidden_fwd_table_bytes(E) == 4 * E * 384 * 6
    assert bench.deg_hidden_bwd_table_bytes(E) == 4 * E * 384 * 8
    assert bench.deg_hidden_fwd_bytes(N, E) == 4 * (4 * E * 6 + N * 9 * 144) + 4 * E * 384 * 6


def _trace_calls():
    """{kernel: dispatches} of the committed kernel trace of the same workload."""
    calls = {}
    for line in (ROOT / "profiles" / "kernel_trace_cfg4_md10k.txt").read_text().splitlines():
        parts = line.split()
        if len(parts) >= 5 and not line.startswith("#") and parts[0].isdigit():
            calls[parts[4]] = int(parts[0])
    return calls


def test_profile_traffic_counts_every_dispatch_of_a_call():
    """The traffic of e2v2_attn_bwd per call, rebuilt from the two committed
    profiles on their own: dispatches per call from the kernel trace (one degree
    embedding and four attention layers per evaluation; k_edge_part_sum also runs
    once per degree backward) times the traffic per dispatch of the PMC summary.
    bench.py must agree within 1%; counting each kernel once (the old error)
    would report under half of it."""
    calls = _trace_calls()
    per = bench.profile_traffic_per_dispatch()
    # the degree embedding's kernels: the hidden-channel form (the model's path) or the output-table form
    deg_f, deg_b = ("k_degh_fwd_sl", "k_degh_bwd_sl") if "k_degh_fwd_sl" in calls else ("k_deg_fwd_sl", "k_deg_bwd_sl")
    n_eval = calls[deg_f]
    n_attn = 4 * n_eval
    assert calls["k_attn_fwd_sl"] == n_attn
    disp = {k: calls[k] / n_attn for k in ("k_attn_bwd_row_sl", "k_attn_bwd_col_grp")}
    disp["k_edge_part_sum"] = (calls["k_edge_part_sum"] - calls[deg_b]) / n_attn
    rebuilt = sum(per[k] * n for k, n in disp.items())
    got = bench.traffic_from_profile("e2v2_attn_bwd")
    assert abs(got - rebuilt) <= 0.01 * rebuilt, (got, rebuilt, disp)
    assert got > 1.5 * sum(per[k] for k in disp)
    fwd = bench.traffic_from_profile("e2v2_attn_fwd")
    assert abs(fwd - per["k_attn_fwd_sl"] * calls["k_attn_fwd_sl"] / n_attn) <= 0.01 * fwd


def test_profile_traffic_only_for_the_profiled_workload():
    t = bench.traffic_from_profile("e2v2_attn_bwd")
    assert t is not None and t > 1e9
    assert bench.traffic_from_profile("e2v2_attn_bwd", bf16=True) is None
    assert bench.traffic_from_profile("e2v2_attn_bwd", False, 5) is None
    assert bench.traffic_from_profile("e2v2_not_an_entry") is None


def test_cpu_sample_choice_follows_host_memory():
    """configs[3]'s CPU baseline times the full system when MemAvailable covers
    it and says why it falls back to the 2,000-atom sample otherwise."""
    big, small = 200 * 2**30, 64 * 2**30
    assert bench.cpu_sample_choice(4, "auto", big)[0] is True
    full, why = bench.cpu_sample_choice(4, "auto", small)
    assert full is False and "64 GiB" in why and "2,000-atom" in why
    assert bench.cpu_sample_choice(4, "full", small)[0] is True
    assert bench.cpu_sample_choice(4, "default", big)[0] is False
    assert bench.cpu_sample_choice(3, "auto", small)[0] is True


def test_more_than_one_gpu_exits_with_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert msg["n_gpus"] == 2 and "one GPU" in msg["error"]


def test_compulsory_bytes_reference_formulation():
    """One attention layer's forward at configs[3] (N = 10,000, M = 19,400
    expanded nodes, E = 0.86 M edges) moves about 0.96 GB: Q and K (2 N 1024),
    the merged value rows (M 29 256) and the output (N 29 256) in fp32, plus
    8 bytes per edge; the backward about twice that."""
    N, M, E = 10_000, 19_400, 860_000
    b = bench.attn_fwd_compulsory(N, M, E)
    assert abs(b - (4 * (2 * N * 1024 + M * 7424 + N * 7424) + 8 * E + 4 * (N + 1))) < 1
    assert 0.94e9 < b < 0.98e9
    assert bench.attn_bwd_compulsory(N, M, E) == 2 * b
    # bf16 activations halve exactly the activation terms
    assert b - bench.attn_fwd_compulsory(N, M, E, 2) == 2 * (2 * N * 1024 + M * 7424 + N * 7424)
    assert bench.deg_compulsory(N, M, E) == 4 * N * 9 * 256 + 8 * E


def test_expanded_nodes_counts_distinct_images():
    """M = real atoms + distinct (atom, nonzero shift) images carrying edges."""
    import numpy as np
    import torch
    from types import SimpleNamespace
    col = torch.tensor([1, 1, 2, 0, 1, 2, 2], dtype=torch.int32)
    sidx = torch.tensor([0, 3, 3, 0, 3, 5, 5], dtype=torch.int32)
    nl = SimpleNamespace(n_atoms=3, n_edges=7, col=col, shift_idx=sidx, shift_ptr=np.array([0, 27]),
                         row_ptr=torch.tensor([0, 2, 5, 7], dtype=torch.int32))
    assert bench.expanded_nodes(nl) == 3 + 3          # (3,1), (3,2), (5,2)


def test_expanded_nodes_counts_real_edges_only():
    """M = N + distinct (atom, nonzero shift) images over the real edges; the slots of
    a capacity build past row_ptr[N] hold stale values and must not count."""
    import types

    import numpy as np
    import torch
    N = 4
    # two graphs' shift tables: rows 0..2 for graph 0 (row 0 the zero shift), 3..4 for graph 1
    shift_ptr = np.array([0, 3, 5])
    row_ptr = torch.tensor([0, 2, 3, 5, 6], dtype=torch.int32)
    col = torch.tensor([1, 1, 0, 3, 3, 2] + [0, 1, 2, 3], dtype=torch.int32)
    sidx = torch.tensor([0, 1, 2, 4, 4, 3] + [1, 2, 1, 4], dtype=torch.int32)
    nl = types.SimpleNamespace(n_atoms=N, n_edges=10, row_ptr=row_ptr, col=col, shift_idx=sidx,
                               shift_ptr=shift_ptr)
    # real images: (1, shift 1), (0, shift 2), (3, shift 4); shifts 0 and 3 are zero shifts
    assert bench.expanded_nodes(nl) == N + 3
    nl.n_edges = 0
    assert bench.expanded_nodes(nl) == N
