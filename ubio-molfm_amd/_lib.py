"""ctypes binding of libe2v2.so (the C ABI declared in include/e2v2.h).

There is no fallback: if the library is missing or a call fails, a
RuntimeError names the entry point and the library's own message.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libe2v2.so"

i32, i64, f32, vp = C.c_int32, C.c_int64, C.c_float, C.c_void_p

EXPORTS = [
    "e2v2_last_error", "e2v2_version", "e2v2_fill_i32", "e2v2_fill_f32", "e2v2_scan_i32",
    "e2v2_nbr_bin", "e2v2_nbr_count", "e2v2_nbr_count_noalloc", "e2v2_nbr_fill", "e2v2_nbr_cap", "e2v2_nbr_topk", "e2v2_csr_transpose", "e2v2_cluster_slots",
    "e2v2_morton_keys", "e2v2_radial_table_size", "e2v2_radial_table", "e2v2_radial_table_check",
    "e2v2_radial_hidden_table", "e2v2_radial_hidden_table_check",
    "e2v2_attn_fwd", "e2v2_attn_bwd", "e2v2_attn_bwd_workspace", "e2v2_deg_fwd", "e2v2_deg_bwd",
    "e2v2_deg_bwd_workspace", "e2v2_deg_hidden_fwd", "e2v2_deg_hidden_bwd", "e2v2_deg_bias_grad",
    "e2v2_edge_to_pos", "e2v2_rmsnorm_fwd", "e2v2_add_rmsnorm_fwd", "e2v2_rmsnorm_bwd", "e2v2_rmsnorm_bwd_param", "e2v2_rmsnorm_bwd2", "e2v2_gate_fwd",
    "e2v2_gate_bwd", "e2v2_gate_bwd2", "e2v2_ln_silu_fwd", "e2v2_ln_silu_bwd", "e2v2_ln_silu_bwd_param", "e2v2_ln_silu_bwd2",
    "e2v2_pairdot_fwd", "e2v2_pairdot_bwd", "e2v2_qk_proj_fwd", "e2v2_qk_proj_bwd",
    "e2v2_qk_proj_fwd_bf16", "e2v2_qk_proj_bwd_bf16",
    "e2v2_segment_metadata", "e2v2_pair_count", "e2v2_pair_emit", "e2v2_seg_dot", "e2v2_seg_reduce",
    "e2v2_gather_rows", "e2v2_outer_reduce", "e2v2_outer_bwd",
    "e2v2_radial_eval", "e2v2_radial_eval_bwd", "e2v2_sh_contract", "e2v2_sh_contract_bwd",
    "e2v2_gemm_s3", "e2v2_gemm_s3_grouped", "e2v2_gemm_s3_gated", "e2v2_gemm_pack", "e2v2_gemm_packed_bytes", "e2v2_qk_proj_fwd_s3", "e2v2_qk_proj_bwd_s3",
    "e2v2_qkdot_gate_fwd", "e2v2_qkdot_gate_bwd", "e2v2_qkdot_gate_bwd_workspace",
]


class NbrPlan(C.Structure):
    _fields_ = [("n_atoms", i32), ("n_graphs", i32), ("n_bins", i32), ("n_shifts", i32),
                ("rc", f32), ("rmin", f32),
                ("pos", vp), ("atom_graph", vp), ("graph_atom_ptr", vp), ("graph_shift_ptr", vp),
                ("graph_periodic", vp), ("shift_off", vp), ("grid_lo", vp), ("grid_h", vp), ("grid_dim", vp),
                ("bin_base", vp), ("atom_bin", vp), ("bin_count", vp), ("bin_start", vp), ("bin_atoms", vp),
                ("stats", vp), ("src_include", vp)]


class PairPlan(C.Structure):
    _fields_ = [("n_query", i32), ("n_graphs", i32), ("l2", i32), ("n_flat", i32), ("max_dist", f32),
                ("min_dist", f32), ("poly", i32), ("qpos", vp), ("qgraph", vp), ("spos", vp), ("include", vp),
                ("sbase", vp), ("sflat", vp)]


class Segments(C.Structure):
    _fields_ = [("row_ptr", vp), ("col_index", vp), ("alpha_index", vp), ("n_rows", i32), ("n_cols", i32),
                ("n_slots", i64), ("n_edges", i64)]


class RadialNet(C.Structure):
    _fields_ = [("w1", vp), ("ld_w1", i32), ("n_emb", i32), ("b1", vp), ("g1", vp), ("be1", vp), ("w2", vp),
                ("b2", vp), ("g2", vp), ("be2", vp), ("w3", vp), ("b3", vp), ("tgt", vp), ("src", vp)]


class RadialLayout(C.Structure):
    """Position of output channel o of a profile in a table row:
    col0 + ((o % split) // block) * block_stride + (o // split) * split_stride + o % block;
    slice_width w > 0 stores the table slice-major, [pairs][nc / w][nodes][4][w]."""
    _fields_ = [("col0", i32), ("split", i32), ("block", i32), ("block_stride", i32), ("split_stride", i32),
                ("slice_width", i32)]


class AttnArgs(C.Structure):
    _fields_ = [("n_rows", i32), ("n_edges", i64), ("n_heads", i32), ("head_dim", i32), ("channels", i32),
                ("row_ptr", vp), ("col", vp), ("edge_row", vp), ("key_ptr", vp), ("key_eid", vp),
                ("dvec", vp), ("dist", vp), ("q", vp), ("k", vp), ("v", vp), ("rtab", vp), ("atom_type", vp),
                ("n_types", i32), ("rtab_n", i32), ("rtab_h", f32), ("q_div", f32), ("rc", f32), ("env_a", f32), ("env_b", f32), ("env_c", f32), ("act_bf16", i32),
                ("col_span", i32), ("col_slot_member", vp), ("col_slot_edge", vp), ("col_n_slots", vp),
                ("zero_order", i32), ("env_kind", i32), ("env_lo", f32), ("ext_gate", vp), ("ext_dgate", vp),
                ("pair_slot", vp), ("weight_act", i32)]


class QkdotArgs(C.Structure):
    _fields_ = [("n_rows", i32), ("n_edges", i64), ("row_ptr", vp), ("edge_row", vp), ("col", vp), ("dist", vp),
                ("e_end", vp), ("Y", vp), ("xd", vp), ("rtab", vp), ("atom_type", vp), ("n_types", i32),
                ("rtab_n", i32), ("rtab_h", f32), ("pair_slot", vp), ("pieces", i32)]


class DegArgs(C.Structure):
    _fields_ = [("n_rows", i32), ("n_edges", i64), ("channels", i32), ("row_ptr", vp), ("dvec", vp),
                ("dist", vp), ("col", vp), ("rtab", vp), ("atom_type", vp), ("n_types", i32), ("rtab_n", i32),
                ("rtab_h", f32), ("avg", f32), ("rc", f32), ("env_a", f32), ("env_b", f32), ("env_c", f32),
                ("pair_slot", vp)]


class GemmArgs(C.Structure):
    _fields_ = [("a", vp), ("lda", i64), ("a_bs", i64), ("b", vp), ("n_w", i32), ("c", vp), ("ldc", i64), ("c_bs", i64),
                ("r", vp), ("ldr", i64), ("r_bs", i64), ("bias", vp), ("bias_bs", i64), ("bias_batches", i32),
                ("m", i32), ("n", i32), ("k", i32), ("batch", i32), ("widx", i32 * 16), ("pieces", i32),
                ("a_bf16", i32), ("c_bf16", i32)]


_lib = None


def load():
    """Load libe2v2.so once; raise if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python ubio-molfm_amd/build.py` "
                           "or __graft_entry__.build() (there is no CPU fallback)")
    lib = C.CDLL(str(LIB_PATH))
    for name in EXPORTS:
        getattr(lib, name)  # raises AttributeError if a symbol is absent
    lib.e2v2_last_error.restype = C.c_char_p
    lib.e2v2_attn_bwd_workspace.restype = C.c_size_t
    lib.e2v2_attn_bwd_workspace.argtypes = [C.c_int64]
    lib.e2v2_deg_bwd_workspace.restype = C.c_size_t
    lib.e2v2_deg_bwd_workspace.argtypes = [C.c_int64]
    lib.e2v2_qkdot_gate_bwd_workspace.restype = C.c_size_t
    lib.e2v2_qkdot_gate_bwd_workspace.argtypes = [C.c_int64]
    lib.e2v2_gemm_packed_bytes.restype = C.c_int64
    lib.e2v2_gemm_packed_bytes.argtypes = [C.c_int32, C.c_int32, C.c_int32, C.c_int32]
    _lib = lib
    return lib


class KernelTimer:
    """HIP-event timing of selected entry points on the stream they run on
    (torch's current stream, which every call in this package uses)."""

    def __init__(self, names):
        self.names = set(names)
        self.events = {n: [] for n in names}
        self.work = {n: 0.0 for n in names}

    def add_work(self, name, amount):
        """Algorithmic work (e.g. FLOPs) of one timed call whose size varies per call."""
        if name in self.work:
            self.work[name] += amount

    def wrap(self, name, fn):
        import torch
        if name not in self.names:
            return fn()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        out = fn()
        e.record()
        self.events[name].append((s, e))
        return out

    def summary(self):
        import torch
        torch.cuda.synchronize()
        out = {}
        for n, evs in self.events.items():
            if not evs:
                continue
            ts = [a.elapsed_time(b) for a, b in evs]
            out[n] = {"count": len(ts), "avg_ms": sum(ts) / len(ts), "total_ms": sum(ts), "work": self.work[n]}
        return out


_timer = None


def set_timer(t):
    global _timer
    _timer = t


def _call_raw(name, *args):
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.e2v2_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (code {rc}): {msg}")


def call(name: str, *args) -> None:  # noqa: F811  (timed variant)
    if _timer is not None:
        return _timer.wrap(name, lambda: _call_raw(name, *args))
    return _call_raw(name, *args)
