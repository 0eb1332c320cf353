"""Benchmark: fp32 energy + autograd forces of the E2Former-V2 stack on the
10,000-atom periodic water/protein mix as a
velocity-Verlet NVE loop at 1 fs with the neighbour list rebuilt every step.

One step = neighbour rebuild + degree embedding + 4 attention layers, forward
and force backward, + integrator update.  Prints ONE JSON line.
"""
import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3
BF16_PEAK_TFLOPS = 2500.0


def load_package():
    import importlib.util
    if "ubio_molfm_amd" in sys.modules:
        return sys.modules["ubio_molfm_amd"]
    d = ROOT / "ubio-molfm_amd"
    spec = importlib.util.spec_from_file_location("ubio_molfm_amd", d / "__init__.py",
                                                  submodule_search_locations=[str(d)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["ubio_molfm_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


# ---------------------------------------------------------------------------------------------
# Algorithmic work per launch, the figure roofline.achieved uses.  Reference formulation of the
# compulsory HBM traffic: N real atoms, M expanded (periodic image) nodes of the reference's
# CellExpander, E directed edges, H = 128 heads x D = 8, S = 256 channels, 29 merged value rows.
# a = bytes per activation element (4 in fp32, 2 in the bf16 mode).

def compulsory_layer_bytes(N, M, E, act=4):
    """One attention layer's forward: read Q, K (N x H x D each), the merged
    value tensor (M x 29 x S), write the output (N x 29 x S), read the edge
    list (column index + shift id, 8 B per edge) and the row pointers."""
    return act * (2 * N * 128 * 8 + M * 29 * 256 + N * 29 * 256) + 8.0 * E + 4.0 * (N + 1)


def attn_fwd_compulsory(N, M, E, act=4):
    return compulsory_layer_bytes(N, M, E, act)


def attn_bwd_compulsory(N, M, E, act=4):
    """First-order backward of the gather/scatter part: about twice the forward."""
    return 2.0 * compulsory_layer_bytes(N, M, E, act)


def deg_compulsory(N, M, E, act=4):
    """Degree embedding node I/O (N x 9 x S fp32) plus the edge list, each direction."""
    return 4.0 * N * 9 * 256 + 8.0 * E


COMPULSORY = {"e2v2_attn_fwd": attn_fwd_compulsory, "e2v2_attn_bwd": attn_bwd_compulsory,
              "e2v2_deg_fwd": deg_compulsory, "e2v2_deg_bwd": deg_compulsory,
              "e2v2_deg_hidden_fwd": deg_compulsory, "e2v2_deg_hidden_bwd": deg_compulsory}


# Bytes the implementation's kernels read and write per launch, split into node / edge-list traffic
# and the radial-table reads (rows of the per-type-pair distance tables, mostly served by the L2 and
# the Infinity Cache: an attention layer's table is 16 pairs x 770 nodes x 4 KB = 50 MB at configs[3],
# spacing 2^-7 A, the first spacing at which the bench model's tables pass their check).
# The forward and the backward row pass run one wavefront per (row, 16-head slice): every slice reads
# the edge list (col, dvec, dist, source type: 6 words per edge) once, 8 times in all.
SLICES = 8


def attn_fwd_bytes(N, E, act=4):
    # read q, k, v, edge list per slice, row_ptr; write out, m, s, cnt
    node_edge = (act * N * (128 * 8 * 2 + 9 * 256 + 20 * 256) + 4.0 * (N * 3 * 128 + SLICES * E * 6 + N + 1))
    return node_edge + attn_fwd_table_bytes(E)


def attn_fwd_table_bytes(E):
    return 4.0 * E * 256 * 6          # gate | inputhead, rows 0..2 at two nodes


def attn_bwd_bytes(N, E, act=4):
    # row pass: read grad, out, q, k, v, m/s/cnt, edge list per slice; write dq, w, dqk, slice partials
    # column pass: read w, dqk, key CSR, grad rows, q; write dv, dk
    # partial sum: read the 8 slice partials, write ddvec, ddist
    row = (act * N * (2 * 20 * 256 + 2 * 1024 + 9 * 256)
           + 4.0 * (N * (1024 + 3 * 128) + E * (SLICES * 6 + 2 * 128 + SLICES * 4)))
    col = act * N * (20 * 256 + 1024) + 4.0 * (N * (9 * 256 + 1024 + 2) + E * (2 * 128 + 2 + 3))
    part = 4.0 * E * (SLICES * 4 + 4)
    return row + col + part + attn_bwd_table_bytes(E)


def attn_bwd_table_bytes(E):
    return 4.0 * E * 256 * 8          # rows 0..3 at two nodes (value and distance derivative)


def deg_fwd_bytes(N, E, act=4):
    # the edge list (dvec, dist, col, source type) once per slice; write x0
    return 4.0 * (SLICES * E * 6 + N * 9 * 256) + deg_fwd_table_bytes(E)


def deg_fwd_table_bytes(E):
    return 4.0 * E * 768 * 6


def deg_bwd_bytes(N, E, act=4):
    # read the edge list per slice and the node gradient; write the slice partials; sum them into ddvec, ddist
    return 4.0 * (SLICES * E * 6 + N * 9 * 256 + SLICES * E * 4 + SLICES * E * 4 + E * 4) + deg_bwd_table_bytes(E)


def deg_bwd_table_bytes(E):
    return 4.0 * E * 768 * 8


# The degree embedding through the profiles' hidden channels (the model's path): 384 table channels instead of
# 768, hs [9][N][144] written; the backward reads grad_h [9][N][128] and grad_s [9][N].  Its per-node GEMMs
# (144 -> 256 and 256 -> 128 per m-row) are e2v2_gemm_s3 calls, its bias-column gradient e2v2_deg_bias_grad.
DEG_HIDDEN_SLICES = 4   # 32 hidden channels of each profile per slice


def deg_hidden_fwd_bytes(N, E, act=4):
    return 4.0 * (DEG_HIDDEN_SLICES * E * 6 + N * 9 * 144) + deg_hidden_fwd_table_bytes(E)


def deg_hidden_fwd_table_bytes(E):
    return 4.0 * E * 384 * 6


def deg_hidden_bwd_bytes(N, E, act=4):
    S = DEG_HIDDEN_SLICES
    return 4.0 * (S * E * 6 + N * 9 * 129 + S * E * 4 + S * E * 4 + E * 4) + deg_hidden_bwd_table_bytes(E)


def deg_hidden_bwd_table_bytes(E):
    return 4.0 * E * 384 * 8


IMPL_BYTES = {"e2v2_attn_fwd": attn_fwd_bytes, "e2v2_attn_bwd": attn_bwd_bytes, "e2v2_deg_fwd": deg_fwd_bytes,
              "e2v2_deg_bwd": deg_bwd_bytes, "e2v2_deg_hidden_fwd": deg_hidden_fwd_bytes,
              "e2v2_deg_hidden_bwd": deg_hidden_bwd_bytes}
TABLE_BYTES = {"e2v2_attn_fwd": attn_fwd_table_bytes, "e2v2_attn_bwd": attn_bwd_table_bytes,
               "e2v2_deg_fwd": deg_fwd_table_bytes, "e2v2_deg_bwd": deg_bwd_table_bytes,
               "e2v2_deg_hidden_fwd": deg_hidden_fwd_table_bytes, "e2v2_deg_hidden_bwd": deg_hidden_bwd_table_bytes}
BYTES_OF = IMPL_BYTES


def stack_flops(N, E):
    """Algorithmic FLOPs of one energy + force evaluation, reference formulation:
    2 x (1.88 MFLOP per edge + 4 layers x 22.7 MFLOP per node) (forward plus
    first-order input-gradient backward)."""
    return 2.0 * (E * 1.88e6 + N * 4 * 22.7e6)


# fused Q/K projection (fp32), FLOPs per call: 9 m-rows x N nodes x C=256 inputs x 4 hid=2048 outputs,
# the backward also folds in the value projection's input gradient (256 more K columns)
PROJ_FLOPS = {"e2v2_qk_proj_fwd": lambda N: 2.0 * 9 * N * 256 * 2048,
              "e2v2_qk_proj_bwd": lambda N: 2.0 * 9 * N * 256 * (2048 + 256)}
PROJ_FLOPS["e2v2_qk_proj_fwd_bf16"] = PROJ_FLOPS["e2v2_qk_proj_fwd"]
PROJ_FLOPS["e2v2_qk_proj_bwd_bf16"] = PROJ_FLOPS["e2v2_qk_proj_bwd"]
PROJ_FLOPS["e2v2_qk_proj_fwd_s3"] = PROJ_FLOPS["e2v2_qk_proj_fwd"]
PROJ_FLOPS["e2v2_qk_proj_bwd_s3"] = PROJ_FLOPS["e2v2_qk_proj_bwd"]
# the QKdot_alpha gate GEMM (768 -> 128 per edge), forward and input gradient: per launch 2 E 768 128
EDGE_GEMM_FLOPS = {"e2v2_qkdot_gate_fwd": lambda E: 2.0 * E * 768 * 128,
                   "e2v2_qkdot_gate_bwd": lambda E: 2.0 * E * 768 * 128}
# fp32 GEMMs on the split kernels execute six bf16 MFMA products per fp32 multiply-add; the bf16 mode runs
# the same kernels on one-piece packs (bf16 operands): one product
SPLIT_PRODUCTS = 6
SPLIT_PRODUCTS_BF16 = 1
SPLIT_ENTRIES = ("e2v2_qk_proj_fwd_s3", "e2v2_qk_proj_bwd_s3", "e2v2_gemm_s3", "e2v2_gemm_s3_grouped", "e2v2_gemm_s3_gated")

# Kernels of each library entry point with their dispatches per call: e2v2_attn_bwd runs the row pass and
# the column pass once per head group (4 groups) and one partial sum.  k_edge_part_sum serves both the
# attention and the degree backward with the same [8][E][4] -> [E][4] shape, so its mean per dispatch is
# that of either.
KERNELS_OF = {"e2v2_attn_fwd": [("k_attn_fwd_sl", 1)],
              "e2v2_attn_bwd": [("k_attn_bwd_row_sl", 4), ("k_attn_bwd_col_grp", 4), ("k_edge_part_sum", 1)],
              "e2v2_deg_fwd": [("k_deg_fwd_sl", 1)], "e2v2_deg_bwd": [("k_deg_bwd_sl", 1), ("k_edge_part_sum", 1)],
              "e2v2_deg_hidden_fwd": [("k_degh_fwd_sl", 1)],
              "e2v2_deg_hidden_bwd": [("k_degh_bwd_sl", 1), ("k_edge_part_sum", 1)],
              "e2v2_deg_bias_grad": [("k_deg_bias_grad", 1)],
              "e2v2_nbr_count": [("k_nbr_count", 1)],
              "e2v2_qk_proj_fwd": [("k_qk_proj_fwd", 1)], "e2v2_qk_proj_bwd": [("k_qk_proj_bwd", 1)],
              "e2v2_qk_proj_fwd_s3": [("k_qk_s3_fwd", 1)], "e2v2_qk_proj_bwd_s3": [("k_qk_s3_bwd", 1)],
              "e2v2_gemm_s3": [("k_gemm_s3", 1)], "e2v2_gemm_s3_grouped": [("k_gemm_s3_grp", 1)],
              "e2v2_gemm_s3_gated": [("k_gemm_s3_gate", 1)]}


def expanded_nodes(nl) -> int:
    """M of the reference formulation: the real atoms plus the distinct periodic
    images (atom, nonzero cell shift) that carry edges.  Only the real edges
    (row_ptr[N] of them) are read: a capacity build's slots past them hold no edge."""
    import numpy as np
    import torch
    N = nl.n_atoms
    e_real = int(nl.row_ptr[N]) if nl.n_edges else 0
    if e_real == 0:
        return N
    zero = torch.as_tensor(np.asarray(nl.shift_ptr[:-1], np.int64), device=nl.col.device)
    sidx = nl.shift_idx[:e_real].long()
    img = ~torch.isin(sidx, zero)
    keys = sidx[img] * N + nl.col[:e_real].long()[img]
    return N + int(torch.unique(keys).numel())


TRAFFIC_PROFILE = ROOT / "profiles" / "hbm_traffic_cfg4_md10k.txt"


def profile_traffic_per_dispatch(path=TRAFFIC_PROFILE):
    """{kernel: HBM-side bytes per dispatch} of a committed FETCH_SIZE/WRITE_SIZE
    summary (its traffic_GB column, already scaled by the copy calibration)."""
    out = {}
    for line in path.read_text().splitlines():
        parts = line.split()
        if len(parts) == 4 and not line.startswith("#") and parts[0] != "kernel":
            out[parts[0]] = float(parts[3]) * 1e9
    return out


def traffic_from_profile(entry, bf16=False, config=4):
    """HBM-side bytes per call of a library entry point: the sum over its kernels
    of bytes per dispatch times dispatches per call, from the committed rocprofv3
    FETCH_SIZE/WRITE_SIZE summary of the fp32 configs[3] workload (--config 4),
    calibrated against a plain copy; None when the entry point, its precision or
    the workload is not covered by the summary."""
    ks = KERNELS_OF.get(entry)
    if ks is None or not TRAFFIC_PROFILE.exists() or bf16 or config != 4:
        return None
    per = profile_traffic_per_dispatch()
    if any(k not in per for k, _ in ks):
        return None
    return sum(per[k] * n for k, n in ks)


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# host memory the restated path needs for one evaluation of configs[3]'s own 10,000-atom system
# (~100 GB measured, with margin), and what that evaluation takes on 16 host threads (~60 s)
FULL_CFG4_HOST_BYTES = 128 * 2**30


def mem_available() -> int:
    """MemAvailable of /proc/meminfo in bytes (0 when unreadable)."""
    try:
        for line in open("/proc/meminfo"):
            if line.startswith("MemAvailable:"):
                return int(line.split()[1]) * 1024
    except (OSError, ValueError, IndexError):
        pass
    return 0


def cpu_sample_choice(config: int, sample: str, avail: int):
    """(full system?, reason) of the CPU baseline's sample: "auto" times
    configs[3]'s own system when the host has the memory for it, else the
    2,000-atom sample of its recipe."""
    if config != 4:
        return config in (1, 2, 3), "the configuration's own system"
    if sample == "full":
        return True, "requested with --cpu-sample full"
    if sample == "default":
        return False, "requested with --cpu-sample default"
    if avail >= FULL_CFG4_HOST_BYTES:
        return True, f"MemAvailable {avail / 2**30:.0f} GiB covers the ~100 GB the full system needs"
    return False, (f"MemAvailable {avail / 2**30:.0f} GiB is below the {FULL_CFG4_HOST_BYTES / 2**30:.0f} GiB "
                   "the full 10,000-atom system needs, so a 2,000-atom sample of its recipe is timed")


def cpu_baseline(pkg, config: int = 4, sample: str = "auto"):
    """The restated reference path (oracle/, torch CPU fp32; the attention's QK
    and value aggregation edge-chunked above 2^18 edges) timed on all host cores
    in this process's affinity, after a warm-up on a 12-atom cell, with the exact
    cell-list neighbour list.  Samples of each workload:
    config 1: the full 648-atom water box, one evaluation;
    config 2: the full 64-molecule batch, graph by graph;
    config 3: the full 1,500-atom system, one evaluation;
    config 4: configs[3]'s own 10,000-atom system, one evaluation (~60 s on 16
    threads, ~100 GB of RAM) when MemAvailable covers it ("auto", the default, or
    "full"); otherwise ("default", or too little memory) a 2,000-atom periodic
    water/protein mix built by its recipe (same density and element ratios), one
    evaluation;
    config 5: not run (hours per evaluation on the host), None."""
    import numpy as np
    import torch
    from ubio_molfm_amd import systems
    from oracle.model import MolfmAtomic as OracleModel
    from oracle.cpu_path import energy_forces_with_neighbors
    if config == 5:
        return None
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    torch.manual_seed(0)
    om = OracleModel().eval()
    energy_forces_with_neighbors(om, systems.small_water(4, 5.5, seed=1))
    full, why = cpu_sample_choice(config, sample, mem_available())
    print(f"[cpu baseline] configs[{config - 1}]: {'full system' if full else 'sample'} ({why})",
          file=sys.stderr, flush=True)
    if config == 3 or (config == 4 and full):
        graphs = [systems.CONFIGS[config]()]
        what = f"the full configs[{config - 1}] system ({len(graphs[0]['pos'])} atoms, {{e}} edges; {why})"
    elif config == 4:
        graphs = [systems.solvated_chains(2000, seed=0)]
        what = f"2,000-atom periodic water/protein mix (configs[{config - 1}] recipe, {{e}} edges; {why})"
    elif config == 1:
        graphs = [systems.CONFIGS[1]()]
        what = "the full configs[0] water box (648 atoms, {e} edges)"
    else:
        full = systems.CONFIGS[config]()
        ptr = np.asarray(full["graph_ptr"])
        graphs = [dict(pos=full["pos"][ptr[g]:ptr[g + 1]], Z=full["Z"][ptr[g]:ptr[g + 1]],
                       graph_ptr=np.array([0, ptr[g + 1] - ptr[g]]), cell=full["cell"][g:g + 1],
                       pbc=full["pbc"][g:g + 1], name=full["name"]) for g in range(len(ptr) - 1)]
        what = (f"the full configs[{config - 1}] system ({len(full['pos'])} atoms in {len(graphs)} graph(s), "
                "{e} edges, fp32)")
    n_atoms = sum(len(g["pos"]) for g in graphs)
    t0 = time.perf_counter()

    def progress(msg):
        print(f"[cpu baseline] {msg} ({time.perf_counter() - t0:.1f} s)", file=sys.stderr, flush=True)
    n_edges = sum(energy_forces_with_neighbors(om, g, progress if len(graphs) == 1 else None)[2] for g in graphs)
    t = time.perf_counter() - t0
    out = {"value": n_edges / t, "unit": "edges/s", "cores": cores, "kind": "port",
           "cpu": _cpu_model(), "atoms": n_atoms, "edges": int(n_edges), "seconds": round(t, 2),
           "sample": what.format(e=n_edges) + ": one energy+force evaluation (neighbour build included) of the "
                     f"restated reference path (oracle/, torch CPU fp32, {cores} threads) after a warm-up"}
    if config == 4:
        out["atom_steps_per_s"] = n_atoms / t
        out["atom_steps_note"] = "one MD step = one energy+force evaluation; N / t of that evaluation"
    return out


def train_line(args, dev):
    """One JSON line for force-training steps: the model in training mode (the backbone composed from the
    second-order op-level kernels, forces taken with create_graph=True), loss = mean e^2 / atom + mean |F|^2
    (zero targets: the work, not the fit, is measured), backward to every parameter through the forces,
    one Adam step; positions fixed, the neighbour list rebuilt inside every forward as in training."""
    import numpy as np
    import torch
    from ubio_molfm_amd import model, neighbors, systems
    torch.manual_seed(0)
    margs = model.default_args()
    margs.backbone_config.update(tp_type=args.tp_type, with_cluster=args.with_cluster)
    m = model.MolfmAtomic(margs).to(dev).train()
    sysd = systems.CONFIGS[args.config]()
    N = len(sysd["pos"])
    bd = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in systems.to_padded(sysd).items()}
    mask = bd["atom_masks"]
    nl = neighbors.build_neighbors(torch.as_tensor(sysd["pos"], device=dev), sysd["graph_ptr"], sysd["cell"],
                                   sysd["pbc"], 6.0)
    E = nl.n_edges
    opt = torch.optim.Adam(m.parameters(), lr=1e-5)

    def step():
        b = dict(bd)
        b["pos"] = bd["pos"].clone().requires_grad_(True)
        res = m(b)
        e, f = res["pred_energy"], res["pred_forces"]
        loss = (e / mask.sum(-1)).pow(2).mean() + f[mask].pow(2).sum(-1).mean()
        opt.zero_grad(set_to_none=True)
        loss.backward()
        opt.step()
        return loss

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        loss = step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = dt / args.steps * 1e3
    print(json.dumps({
        "metric": "force-training steps: edges/s (energy + forces with create_graph + parameter backward + Adam)",
        "value": E * args.steps / dt, "unit": "edges/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded generator, random-init weights, zero targets)",
        "config": {"workload": f"configs[{args.config - 1}] {sysd['name']}: {N} atoms, rc 6 A, force training "
                               f"(model.train(): second-order composition), fixed positions",
                   "atoms": N, "edges_per_step": E, "layers": 4, "parallelism": "single GPU",
                   "tp_type": args.tp_type, "with_cluster": args.with_cluster},
        "mode": "train", "atom_steps_per_s": N * args.steps / dt, "final_loss": float(loss),
        "peak_memory_gb": torch.cuda.max_memory_allocated(dev) / 1e9,
        "roofline": None, "cpu_baseline": None}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", type=int, default=4)
    ap.add_argument("--mode", choices=["md", "eval", "train"], default=None,
                    help="md: NVE velocity-Verlet steps (default for configs 1-4); eval: repeated energy+force "
                         "evaluations at fixed positions (default for config 5); train: force-training steps "
                         "(energy, forces with create_graph, loss on both, backward to every parameter, one Adam "
                         "step) of the model in training mode at fixed positions (a separate line, not the "
                         "headline metric)")
    ap.add_argument("--dtype", choices=["fp32", "bf16"], default=None,
                    help="GEMM operand precision (default: bf16 for configs 2 and 5, as they are specified, "
                         "else fp32); accumulation, activations and reductions are fp32 in both")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--exact-nbr", action="store_true",
                    help="MD: exact neighbour builds with one count readback per step instead of capacity builds "
                         "checked one step later")
    ap.add_argument("--cpu-sample", choices=["auto", "default", "full"], default="auto",
                    help="CPU baseline sample of configs[3]: its own 10,000-atom system when the host's "
                         "MemAvailable covers it, else a 2,000-atom sample (auto); always the sample (default); "
                         "always the full system (full)")
    ap.add_argument("--graph", action="store_true",
                    help="replay each step as one HIP graph (captured after one eager step) instead of launching "
                         "its kernels from Python; measured equal in time at configs 1, 3 and 4")
    ap.add_argument("--kernel-steps", type=int, default=5,
                    help="eager steps after the timed region whose library calls are timed with HIP events")
    ap.add_argument("--tp-type", default="QK_alpha",
                    help="tp_type of the model (variant lines: QKdot_alpha, QKdotS_alpha, +softplus / +sigmoid)")
    ap.add_argument("--with-cluster", default="False",
                    help="with_cluster of the model (variant lines: node, node_bell: two long-range blocks)")
    ap.add_argument("--pmc-calibration", action="store_true",
                    help="run one plain 256 MiB device copy first (scale reference for FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: the spatial sharding over several GPUs is "
                                   "designed but not launched", "n_gpus": args.gpus}))
        sys.exit(2)
    import numpy as np
    import torch
    pkg = load_package()
    from ubio_molfm_amd import _lib, md, model, systems
    dev = torch.device("cuda:0")
    if args.pmc_calibration:
        src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.mode == "train":
        train_line(args, dev)
        return
    torch.manual_seed(0)
    margs = model.default_args()
    margs.backbone_config.update(tp_type=args.tp_type, with_cluster=args.with_cluster)
    m = model.MolfmAtomic(margs).eval().to(dev).requires_grad_(False)
    dtype = args.dtype or ("bf16" if args.config in (2, 5) else "fp32")
    m.decoder.set_compute_dtype(dtype)
    bf16 = dtype == "bf16"
    sysd = systems.CONFIGS[args.config]()
    N = len(sysd["pos"])
    mode = args.mode or ("eval" if args.config == 5 else "md")
    graph = args.graph and not args.exact_nbr
    integ = md.VelocityVerlet(m, sysd, dev, dt_fs=1.0, T=300.0, seed=0, lagged=not args.exact_nbr, graph=graph,
                              evaluate_only=mode == "eval")
    integ.e, integ.f = integ.forces()          # setup: forces at t = 0
    # warm-up (with a graph: at least the eager steps and the step that captures it, so that the timed
    # region only launches the graph)
    warmup = max(args.warmup, integ.WARM_STEPS + 1) if graph else args.warmup
    for _ in range(warmup):
        integ.step()
    integ.sync()
    torch.cuda.synchronize()
    kinetic = (lambda: 0.0) if mode == "eval" else integ.kinetic
    e_start = integ.e.sum().item() + kinetic()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        integ.step()
    integ.sync()                             # the last step's neighbour counters (lagged check)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    edges = integ.edge_counts[-args.steps:]
    e_end = integ.e.sum().item() + kinetic()
    captures = integ.captures
    # per-kernel durations: HIP events around each library call of a few more steps run eagerly (the
    # kernels a graph replays are the same launches; replays do not pass through the Python wrappers)
    timer = _lib.KernelTimer(["e2v2_attn_fwd", "e2v2_attn_bwd",
                              "e2v2_deg_fwd", "e2v2_deg_bwd", "e2v2_deg_hidden_fwd", "e2v2_deg_hidden_bwd",
                              "e2v2_deg_bias_grad", "e2v2_nbr_count", "e2v2_nbr_fill",
                              "e2v2_qk_proj_fwd", "e2v2_qk_proj_bwd", "e2v2_qk_proj_fwd_bf16",
                              "e2v2_qk_proj_bwd_bf16", "e2v2_qk_proj_fwd_s3", "e2v2_qk_proj_bwd_s3",
                              "e2v2_gemm_s3", "e2v2_gemm_s3_grouped", "e2v2_gemm_s3_gated",
                              "e2v2_qkdot_gate_fwd", "e2v2_qkdot_gate_bwd"])
    integ.use_graph = False
    _lib.set_timer(timer)
    for _ in range(min(args.steps, args.kernel_steps)):
        integ.step()
    integ.sync()
    torch.cuda.synchronize()
    _lib.set_timer(None)
    if mode == "md":
        integ.forces()                       # untimed exact build: the list expanded_nodes reads
    dt = t1 - t0
    ms = dt / args.steps * 1e3
    E_mean = float(np.mean(edges))
    stats = timer.summary()
    peak_gb = torch.cuda.max_memory_allocated(dev) / 1e9
    act = 2 if bf16 else 4   # bytes per attention activation element
    M = expanded_nodes(integ.last_nl)     # reference formulation's expanded nodes (last step's list)
    peak_tf = BF16_PEAK_TFLOPS if bf16 else FP32_PEAK_TFLOPS
    per_kernel = {}
    for k, v in stats.items():
        ent = {"avg_ms": round(v["avg_ms"], 4), "count": v["count"], "total_ms": round(v["total_ms"], 3)}
        sec = v["avg_ms"] * 1e-3
        if k in COMPULSORY:
            b_alg = COMPULSORY[k](N, M, E_mean, act)
            b_imp = IMPL_BYTES[k](N, E_mean, act)
            b_tab = TABLE_BYTES[k](E_mean)
            ent.update(bound="hbm", bytes_per_launch=b_alg, achieved_gbs=round(b_alg / sec / 1e9, 1),
                       frac=round(b_alg / sec / 1e9 / HBM_PEAK_GBS, 4), impl_bytes_per_launch=b_imp,
                       impl_gbs=round(b_imp / sec / 1e9, 1), impl_frac=round(b_imp / sec / 1e9 / HBM_PEAK_GBS, 4),
                       impl_table_bytes_per_launch=b_tab)
        elif k in SPLIT_ENTRIES:
            # fp32 GEMMs executed as six bf16 MFMA products each (one in the bf16 mode): the executed bf16
            # rate against the bf16 peak (frac, comparable with SQ_VALU_MFMA_BUSY), and in fp32 the fp32 work
            # rate beside the fp32 peak
            fl = PROJ_FLOPS[k](N) if k in PROJ_FLOPS else v["work"] / v["count"]
            tf = fl / sec / 1e12
            prod = SPLIT_PRODUCTS_BF16 if bf16 else SPLIT_PRODUCTS
            ent.update(bound="mfma", flops_per_launch=fl, executed_flops_per_launch=prod * fl,
                       achieved_tflops=round(prod * tf, 2), peak_tflops=BF16_PEAK_TFLOPS,
                       frac=round(prod * tf / BF16_PEAK_TFLOPS, 4))
            if not bf16:
                ent.update(fp32_equivalent_tflops=round(tf, 2),
                           fp32_equivalent_over_fp32_peak=round(tf / FP32_PEAK_TFLOPS, 4))
        elif k in EDGE_GEMM_FLOPS:
            fl = EDGE_GEMM_FLOPS[k](E_mean)
            tf = fl / sec / 1e12
            prod = SPLIT_PRODUCTS_BF16 if bf16 else SPLIT_PRODUCTS
            ent.update(bound="mfma", flops_per_launch=fl, executed_flops_per_launch=prod * fl,
                       achieved_tflops=round(prod * tf, 2), peak_tflops=BF16_PEAK_TFLOPS,
                       frac=round(prod * tf / BF16_PEAK_TFLOPS, 4))
        elif k in PROJ_FLOPS:
            tf = PROJ_FLOPS[k](N) / sec / 1e12
            pk = BF16_PEAK_TFLOPS if k.endswith("_bf16") else FP32_PEAK_TFLOPS
            ent.update(bound="mfma", flops_per_launch=PROJ_FLOPS[k](N), achieved_tflops=round(tf, 2),
                       peak_tflops=pk, frac=round(tf / pk, 4))
        per_kernel[k] = ent
    # headline: the library entry point with the largest total time, at its algorithmic work per launch
    name = max(stats.items(), key=lambda kv: kv[1]["total_ms"])[0]
    ent = per_kernel[name]
    # the traffic profile and the CPU baseline cover the default model (QK_alpha, no cluster blocks)
    default_model = args.tp_type == "QK_alpha" and args.with_cluster in ("False", "false", "0", "None", "none")
    cfg_traffic = args.config if default_model else -1
    if ent.get("bound") == "hbm":
        roof = {"bound": "hbm", "achieved": ent["achieved_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": ent["frac"], "traffic": traffic_from_profile(name, bf16, cfg_traffic), "kernel": name,
                "algorithmic_bytes_per_launch": ent["bytes_per_launch"], "expanded_nodes": M}
    else:
        pk = ent.get("peak_tflops", FP32_PEAK_TFLOPS)
        roof = {"bound": "mfma", "achieved": ent.get("achieved_tflops"), "peak": pk, "unit": "TFLOP/s",
                "frac": ent.get("frac"), "traffic": traffic_from_profile(name, bf16, cfg_traffic), "kernel": name}
    # stack: whole evaluation against the MFMA roofline; HBM-bound kernels time-weighted
    stack_tf = stack_flops(N, E_mean) / (ms * 1e-3) / 1e12
    hb = [k for k in COMPULSORY if k in stats]
    hb_time = sum(stats[k]["total_ms"] for k in hb) * 1e-3
    hb_alg = sum(COMPULSORY[k](N, M, E_mean, act) * stats[k]["count"] for k in hb)
    hb_imp = sum(IMPL_BYTES[k](N, E_mean, act) * stats[k]["count"] for k in hb)
    roof["stack"] = {"bound": "mfma", "achieved": round(stack_tf, 2), "peak": peak_tf, "unit": "TFLOP/s",
                     "frac": round(stack_tf / peak_tf, 4), "flops_per_step": stack_flops(N, E_mean),
                     "note": "reference-formulation FLOPs; the per-edge radial MLPs (about 70% of them) run here "
                             "as distance-table interpolation, so this is an equivalent rate, not MFMA utilisation"}
    roof["hbm_kernels_time_weighted"] = {"kernels": hb, "achieved": round(hb_alg / hb_time / 1e9, 1),
                                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                         "frac": round(hb_alg / hb_time / 1e9 / HBM_PEAK_GBS, 4),
                                         "impl_frac": round(hb_imp / hb_time / 1e9 / HBM_PEAK_GBS, 4)}
    cpu = None
    if not args.no_cpu_baseline and default_model:
        cpu = cpu_baseline(pkg, args.config, args.cpu_sample)
    out = {
        "metric": "attn edges/s fwd+force-bwd & MD atom-steps/s at 10k atoms; % HBM roofline",
        "value": E_mean * args.steps / dt,
        "unit": "edges/s",
        "n_gpus": 1, "steps": args.steps, "warmup": warmup, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "hip_graph": {"used": graph, "captures": captures, "warmup_steps": warmup,
                      "kernel_timing": f"HIP events around each library call of {min(args.steps, args.kernel_steps)} "
                                       "eager steps after the timed region"},
        "dtype": "bf16 GEMM operands, f32 accumulate" if bf16 else "f32",
        "data": "synthetic (seeded generator, random-init weights)",
        "config": {"workload": f"configs[{args.config - 1}] {sysd['name']}: {N} atoms, rc 6 A, "
                               + ("NVE velocity-Verlet 1 fs, neighbour rebuild every step, energy+forces"
                                  if mode == "md" else "repeated energy+force evaluations (neighbour build "
                                                       "included)") + f", {dtype}",
                   "atoms": N, "edges_per_step": E_mean, "layers": 4, "parallelism": "single GPU",
                   "tp_type": args.tp_type, "with_cluster": args.with_cluster},
        "atom_steps_per_s": N * args.steps / dt,
        "mode": mode,
        "peak_memory_gb": peak_gb,
        "nve_energy_drift_ev_per_atom": (e_end - e_start) / N,
        "kernels": per_kernel,
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
