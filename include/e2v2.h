/*
 * e2v2 -- MI355X (gfx950) HIP library for the E2Former-V2 sparse equivariant
 * attention path.  C ABI: plain pointers and sizes, no torch types.
 *
 * Conventions
 *   - Every pointer is a device pointer owned by the caller (the PyTorch caching
 *     allocator in this repository).  The library never allocates or frees.
 *   - Every call enqueues work on the given stream and returns 0 on success or
 *     a nonzero code; e2v2_last_error() returns the message of the last failure
 *     on the calling thread.
 *   - Atoms of a batch are flattened; graph g owns atoms [graph_atom_ptr[g],
 *     graph_atom_ptr[g+1]).  Edge e = (i <- j, shift s) lives in row i of the
 *     query CSR; its source position is pos[j] + s . cell.
 *   - Results are deterministic: no floating-point atomics; column sums use
 *     the key CSR (edges of each source atom sorted by edge id).
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   e2v2_nbr_*          CellExpander.expand_includeself + construct_radius_neighbor
 *                       src/molfm/models/e2former/module_utils.py:1065-1274, 3119-3242
 *                       (FAISS twin: src/molfm/models/e2former/sp/dist_ner.py:27-86, 240-333)
 *   e2v2_csr_transpose  prepare_sparse_qk_edge_index_metadata
 *                       src/molfm/models/e2former/triton_dr/triton_sparse_qk_autograd.py:601-652
 *   e2v2_mlp_fwd/bwd    GaussianSmearing + RadialProfile over x_edge = [rbf, tgt, src]
 *                       src/molfm/models/e2former/e2former.py:258-266, 302 (fc_easy) and
 *                       e2former.py:709-733 (gbf_projs); module_utils.py:1853-1869, 2151-2178
 *   e2v2_attn_fwd       sparse_qk_edge_index_triton (triton_sparse_qk_autograd.py:839-871),
 *                       segmented softmax e2former.py:327-367 with
 *                       sparse_alpha_sum_edge_index_triton (sparse_alpha_sum_edge_index_autograd.py:207-213),
 *                       sparse_v_agg_edge_index_triton_cblocked (sparse_v_agg_edge_index_cblocked_bench.py:428-449)
 *                       and E2TensorProductSO2_FirstOrder.forward up to forward_linear
 *                       (src/molfm/models/e2former/wigner6j/so2_tensor_product.py:341-385)
 *   e2v2_attn_bwd       the first-order backward of the above autograd Functions
 *                       (triton_sparse_qk_autograd.py:740-749, sparse_alpha_sum_edge_index_autograd.py:155-169,
 *                        sparse_v_agg_edge_index_cblocked_bench.py:348-357)
 *   e2v2_deg_fwd/bwd    edge_degree_outer_triton (triton_dr/edge_degree_outer_autograd.py:299-375) with the
 *                       spherical harmonics and envelope of EdgeDegreeEmbeddingNetwork_higherorder.forward
 *                       (e2former.py:689-753)
 *   e2v2_rmsnorm_*      EquivariantRMSNormArraySphericalHarmonicsV2_BL (module_utils.py:1663-1772)
 *   e2v2_gate_*         Gate_s3 activation (module_utils.py:2694-2746)
 *   e2v2_pairdot_*      per-l m-contraction of SO3_Linear2Scalar_e2former (module_utils.py:2241-2266)
 *   e2v2_qk_proj_*      its projection GEMMs with the contraction fused (module_utils.py:2198-2266)
 *   e2v2_edge_to_pos    autograd of f_edge_vec / f_dist w.r.t. positions (module_utils.py:3161-3206),
 *                       consumed by GradientHead (src/molfm/pipeline/head.py:305-328)
 */
#ifndef E2V2_H
#define E2V2_H

#include <stdint.h>
#include <stddef.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define E2V2_MAX_MLP 3

const char* e2v2_last_error(void);
int e2v2_version(void);

/* ---- utilities -------------------------------------------------------- */
int e2v2_fill_i32(int32_t* p, int32_t v, int64_t n, hipStream_t s);
int e2v2_fill_f32(float* p, float v, int64_t n, hipStream_t s);
/* exclusive scan: out[0..n], out[n] = total; stats[0] = total, stats[1] = max(in) */
int e2v2_scan_i32(const int32_t* in, int n, int32_t* out, int32_t* stats, hipStream_t s);

/* ---- radius graph ------------------------------------------------------ */
typedef struct e2v2_nbr_plan {
  int32_t n_atoms, n_graphs, n_bins, n_shifts;
  float rc, rmin;                   /* keep rmin <= d <= rc (both inclusive)                */
  const float* pos;                 /* [n_atoms, 3]                                         */
  const int32_t* atom_graph;        /* [n_atoms]                                            */
  const int32_t* graph_atom_ptr;    /* [n_graphs + 1]                                       */
  const int32_t* graph_shift_ptr;   /* [n_graphs + 1] rows of shift_off per graph            */
  const int32_t* graph_periodic;    /* [n_graphs] 1 if any periodic direction               */
  const float* shift_off;           /* [n_shifts, 3] fp32 offsets s . cell                  */
  const float* grid_lo;             /* [n_graphs, 3] bin grid origin                        */
  const float* grid_h;              /* [n_graphs, 3] bin edge (>= rc)                       */
  const int32_t* grid_dim;          /* [n_graphs, 3]                                        */
  const int32_t* bin_base;          /* [n_graphs] first bin of each graph                   */
  int32_t* atom_bin;                /* workspace [n_atoms]                                  */
  int32_t* bin_count;               /* workspace [n_bins]                                   */
  int32_t* bin_start;               /* workspace [n_bins + 1]                               */
  int32_t* bin_atoms;               /* workspace [n_atoms]                                  */
  int32_t* stats;                   /* workspace [3], zeroed by the caller: scan total / max;
                                       [2] != 0 if an atom lies outside its graph's grid box */
} e2v2_nbr_plan;

int e2v2_nbr_bin(const e2v2_nbr_plan* plan, hipStream_t s);
/* row_count [n_atoms]; row_ptr [n_atoms+1]; plan->stats = {E, max row} */
int e2v2_nbr_count(const e2v2_nbr_plan* plan, int32_t* row_count, int32_t* row_ptr, hipStream_t s);
/* rows sorted by (distance, j, shift); tmp_* are [E] (tmp_dvec [E,3]) scratch */
int e2v2_nbr_fill(const e2v2_nbr_plan* plan, const int32_t* row_ptr, int64_t n_edges, int max_row,
                  int32_t* tmp_col, int32_t* tmp_shift, float* tmp_dvec, float* tmp_dist, uint64_t* tmp_key,
                  int32_t* col, int32_t* shift, float* dvec, float* dist, hipStream_t s);
/* keep the k nearest of each sorted row: phase 0 counts + scans (stats = {E', max}), phase 1 compacts */
int e2v2_nbr_topk(const int32_t* row_ptr, int n_rows, int k, int32_t* cnt, int32_t* new_ptr, int32_t* stats,
                  const int32_t* col, const int32_t* shift, const float* dvec, const float* dist,
                  int32_t* ocol, int32_t* oshift, float* odv, float* od, int phase, hipStream_t s);
/* 30-bit Morton (Z-order) keys of atoms within their graph's bounding box, for the spatial
   ordering of the rows: key[i] = g << 32 | interleave(q) with q = clamp((pos - lo[g]) / span[g]
   * 1023, 0, 1023) truncated; gid [n] the graph of each atom (NULL: one graph), lo/span [B][3].
   No reference counterpart: the row order that keeps a workgroup's neighbours in one L2. */
int e2v2_morton_keys(const float* pos, const int32_t* gid, const float* lo, const float* span, int n, int64_t* key,
                     hipStream_t s);
/* Clusters of `span` (1..8) consecutive segments of a CSR: seg_ptr = row_ptr with member = col and
   item_eid = NULL (query rows), or seg_ptr = key_ptr with member = edge_row and item_eid = key_eid (key
   columns).  Every distinct (member atom, occurrence) of a cluster becomes one slot, sorted by atom:
   slot_member[slot] = the atom, slot_edge[slot * span + r] = the edge joining it to segment r of the
   cluster or -1.  Slots of cluster c are stored from index seg_ptr[c * span] on; n_slots[c] counts them.
   Sizes: slot_member [n_items], slot_edge [n_items * span], n_slots [ceil(n_seg / span)].
   No reference counterpart: the layout the clustered edge kernels read. */
int e2v2_cluster_slots(const int32_t* seg_ptr, int32_t n_seg, const int32_t* member, const int32_t* item_eid,
                       int32_t span, int32_t* slot_member, int32_t* slot_edge, int32_t* n_slots, hipStream_t s);
/* key CSR: phase 0 -> edge_row, key_ptr, stats = {E, max column}; phase 1 -> key_eid (sorted by edge id;
   columns of any length, no host check needed between the phases) */
int e2v2_csr_transpose(const int32_t* row_ptr, const int32_t* col, int n_rows, int n_cols, int64_t n_edges,
                       int32_t* edge_row, int32_t* key_cnt, int32_t* key_ptr, int32_t* stats,
                       uint64_t* tmp_key, int32_t* key_eid, int phase, hipStream_t s);

/* ---- edge radial MLP --------------------------------------------------- */
typedef struct e2v2_mlp_weights {
  /* Linear1's rbf block as a function of the distance: rtab[n][k][c] =
     h^k d^k/dd^k (W1[c, 0:256] . rbf(d)) at d = n h, k = 0..3 (float64-built by
     e2v2_mlp_rbf_table); evaluated by quintic Hermite interpolation.            */
  const float* rtab;  /* [rtab_n][4][128]                                          */
  int32_t rtab_n;     /* nodes covering [0, rc]                                     */
  float rtab_h;       /* node spacing, a power of two                               */
  const float* ttgt;  /* [types][128] target-type block of Linear1 + bias         */
  const float* tsrc;  /* [types][128] source-type block of Linear1                */
  const float* g1; const float* be1;   /* LayerNorm(128)                            */
  /* fp32 GEMM operands B[K][N], lane-packed: one float4 per (wave w < 4, column group
     ct < N/64, k block b < K/16, lane l < 64) in that order, holding
     B[16 b + 4 (l / 16) + s][w N/4 + 16 ct + l % 16], s = 0..3.                  */
  const float* w2t;   /* B = Linear2^T [128][128] (forward)                       */
  const float* b2;
  const float* g2; const float* be2;
  const float* w3t;   /* B = Linear3^T [128][256] (forward)                       */
  const float* b3;
  const float* w2;    /* B = Linear2 [128][128] (backward)                        */
  const float* w3;    /* B = Linear3 [256][128] (backward)                        */
  /* bf16 operands (compute_bf16 = 1), each as B^T row-major [N][K]:              */
  const void* w2b;    /* [128][128] Linear2 (forward)                             */
  const void* w3b;    /* [256][128] Linear3 (forward)                             */
  const void* w3tb;   /* [128][256] Linear3^T (backward)                          */
  const void* w2tb;   /* [128][128] Linear2^T (backward)                          */
} e2v2_mlp_weights;

typedef struct e2v2_mlp_args {
  int64_t n_edges;
  int32_t n_mlp;                 /* 1..E2V2_MAX_MLP profiles sharing the edge input */
  int32_t compute_bf16;          /* 1: bf16 GEMM operands, fp32 accumulation       */
  const float* dist;             /* [E]                                            */
  const int32_t* edge_row;       /* [E] query atom                                 */
  const int32_t* col;            /* [E] source atom                                */
  const int32_t* node_type;      /* [N] atomic numbers                             */
  float* save_n;                 /* [n_mlp][E][256] normalised LN1 | LN2 inputs (written by fwd, read by bwd) */
  float* save_r;                 /* [n_mlp][E][2]   their rstd                                                */
  e2v2_mlp_weights w[E2V2_MAX_MLP];
} e2v2_mlp_args;

/* Node count and spacing (a power of two, about 0.17 of the Gaussian width) of the
   rbf-block table of a GaussianSmearing basis exp(rbf_coeff (d - mu)^2) over [0, rc]
   (module_utils.py:1853-1869). */
int e2v2_mlp_rbf_table_size(float rc, float rbf_coeff, int32_t* n_nodes, float* h);
/* rtab [n_nodes][4][128] of Linear1's rbf block w1 [128][ldw1] (columns 0..255) with
   centres rbf_offset [256]; float64 accumulation. */
int e2v2_mlp_rbf_table(const float* w1, int ldw1, const float* rbf_offset, float rbf_coeff, int32_t n_nodes,
                       float h, float* rtab, hipStream_t s);

/* out[e, 256 m + c] for profile m; fills save_n / save_r when they are non-null */
int e2v2_mlp_fwd(const e2v2_mlp_args* args, float* out, int ld_out, hipStream_t s);
/* dd[e] (+)= sum_m dL/dout_m . dout_m/dd  (input gradient w.r.t. the edge distance only);
   requires save_n / save_r from the forward of the same edges and weights */
int e2v2_mlp_bwd(const e2v2_mlp_args* args, const float* dout, int ld_dout, float* dd, int accumulate,
                 hipStream_t s);

/* ---- attention --------------------------------------------------------- */
typedef struct e2v2_attn_args {
  int32_t n_rows;                /* N query atoms (= source atoms)                  */
  int64_t n_edges;
  int32_t n_heads, head_dim, channels;   /* must be 128, 8, 256                     */
  const int32_t* row_ptr;        /* [N+1] query CSR                                 */
  const int32_t* col;            /* [E]                                             */
  const int32_t* edge_row;       /* [E]                                             */
  const int32_t* key_ptr;        /* [N+1] key CSR                                   */
  const int32_t* key_eid;        /* [E]                                             */
  const float* dvec;             /* [E,3] pos_i - (pos_j + s.cell)                   */
  const float* dist;             /* [E]                                             */
  const void* q;                 /* [N,H,D]            float, or bf16 if act_bf16   */
  const void* k;                 /* [N,H,D]            float, or bf16 if act_bf16   */
  const void* v;                 /* [9][N][C] m-major  float, or bf16 if act_bf16   */
  const float* gi;               /* [E,2H] gate | inputhead                         */
  float q_div;                   /* sqrt(D)                                         */
  float rc, env_a, env_b, env_c; /* polynomial envelope                             */
  int32_t act_bf16;              /* 1: q, k, v, out, grad_out stored as bf16 (fp32 math) */
  /* Optional key-CSR column clusters from e2v2_cluster_slots with span col_span = 4 (NULL: one
     workgroup per column); used by the fp32 column pass of e2v2_attn_bwd. */
  int32_t col_span;
  const int32_t* col_slot_member; const int32_t* col_slot_edge; const int32_t* col_n_slots;
} e2v2_attn_args;

/* v [9][N][C] and out [20][N][C] are m-major (row r of every atom contiguous);
   out (float, or bf16 if act_bf16): h_a - h_b rows of the SO(2) product; mrow/srow [N,H] softmax max / sum;
   cnt [N,H] number of maxima */
int e2v2_attn_fwd(const e2v2_attn_args* args, void* out, float* mrow, float* srow, int32_t* cnt, hipStream_t s);
/* grad_out, out [20][N][C] (float, or bf16 if act_bf16) -> dgi [E,2H], ddvec [E,3], ddist [E], dq, dk [N,H,D],
   dv [9][N][C] (all float); w_edge, dqk_edge [E,H] are outputs consumed by the column pass */
int e2v2_attn_bwd(const e2v2_attn_args* args, const void* grad_out, const void* out, const float* mrow,
                  const float* srow, const int32_t* cnt, float* dgi, float* ddvec, float* ddist, float* dq,
                  float* dk, float* dv, float* w_edge, float* dqk_edge, hipStream_t s);

/* ---- edge-degree embedding -------------------------------------------- */
typedef struct e2v2_deg_args {
  int32_t n_rows;
  int64_t n_edges;
  int32_t channels;              /* 256                                             */
  const int32_t* row_ptr;
  const float* dvec;             /* [E,3]                                           */
  const float* dist;             /* [E]                                             */
  const float* fea;              /* [E,3,C] radial-MLP outputs for l = 0, 1, 2      */
  float avg;                     /* avg_aggregate_num                               */
  float rc, env_a, env_b, env_c;
} e2v2_deg_args;

/* x0 [9][N][C] m-major */
int e2v2_deg_fwd(const e2v2_deg_args* args, float* x0, hipStream_t s);
/* dfea may be NULL (then only ddvec, ddist; e2v2_mlp_bwd_deg forms dfea itself) */
int e2v2_deg_bwd(const e2v2_deg_args* args, const float* grad_x0, float* dfea, float* ddvec, float* ddist,
                 hipStream_t s);
/* e2v2_mlp_bwd for the degree embedding's three l-profiles with dOut formed per edge tile from the
   node gradient grad_x0 [9][N][256] (m-major) instead of a stored [E][3][256] tensor:
   dOut[e, l, c] = p(d_e)/avg sum_{m in l} Y_m(u_e) grad_x0[m][i_e][c] (the transpose of the degree
   embedding's CSR reduce, e2former.py:719-741); deg supplies dvec, dist, avg and the envelope. */
int e2v2_mlp_bwd_deg(const e2v2_mlp_args* args, const e2v2_deg_args* deg, const float* grad_x0, float* dd,
                     int accumulate, hipStream_t s);

/* ---- per-node kernels (node layout m-major: x[9][N][256]) --------------- */
/* rms_norm_sh: EquivariantRMSNormArraySphericalHarmonicsV2_BL
 * (src/molfm/models/e2former/module_utils.py:1663-1772); w [3][256], b [256] */
int e2v2_rmsnorm_fwd(const float* x, const float* w, const float* b, float* y, int n, float eps, hipStream_t s);
/* The residual add of the producing block fused in: xs = x + delta (written) and y = rms_norm_sh(xs);
   delta = NULL is e2v2_rmsnorm_fwd (xs unused). */
int e2v2_add_rmsnorm_fwd(const float* x, const float* delta, const float* w, const float* b, float* xs, float* y,
                         int n, float eps, hipStream_t s);
/* gx = d(rms_norm_sh)/dx^T gy (+ gres when gres is not NULL: the gradient of a residual branch that reads x) */
int e2v2_rmsnorm_bwd(const float* x, const float* w, const float* gy, const float* gres, float* gx, int n, float eps,
                     hipStream_t s);
/* Gate_s3 activation (module_utils.py:2694-2746) from gate logits sc [N][768];
 * k1, k2 = normalize2mom constants of SiLU and sigmoid */
int e2v2_gate_fwd(const float* sc, const float* x, float* y, int n, float k1, float k2, hipStream_t s);
int e2v2_gate_bwd(const float* sc, const float* x, const float* gy, float* gsc, float* gx, int n, float k1,
                  float k2, hipStream_t s);

/* Q/K scalarisation of SO3_Linear2Scalar_e2former (module_utils.py:2241-2266):
 * y [9][N][4 hid] = (q_a | q_b | k_a | k_b) -> hq, hk [N][3 hid], h[l hid + c] = sum_{m in l} a b */
int e2v2_pairdot_fwd(const float* y, float* hq, float* hk, int n, int hid, hipStream_t s);
int e2v2_pairdot_bwd(const float* y, const float* ghq, const float* ghk, float* gy, int n, int hid, hipStream_t s);
/* The Q/K projection of SO3_Linear2Scalar_e2former with the above contraction fused (module_utils.py:2198-2266,
 * called for query and key at e2former.py:300-303), fp32 MFMA:
 *   fwd: y[m][n][o] = sum_k x[m][n][k] w[l(m)][o][k] (+ bias[o] on m = 0; bias may be NULL), x [9][N][C],
 *        w [3][4 hid][C]; writes y (kept for the backward) and hq, hk [N][3 hid].
 *   bwd: gx [9][N][C] = gy W with gy the contraction's gradient (formed from y, ghq, ghk; never stored),
 *        wt [9][C][4 hid] = w[l(m)]^T per m-row; with gv (NULL for none) also + gv Wv, gv [9][N][cv],
 *        wvt [9][C][cv] = Wv[l(m)]^T (the value projection, which reads the same x).
 * Requires hid % 64 == 0, C % 128 == 0 (bwd; C % 32 fwd), cv % 32 == 0. */
int e2v2_qk_proj_fwd(const float* x, const float* w, const float* bias, float* y, float* hq, float* hk, int n, int hid,
                     int c, hipStream_t s);
int e2v2_qk_proj_bwd(const float* y, const float* ghq, const float* ghk, const float* wt, const float* gv,
                     const float* wvt, float* gx, int n, int hid, int c, int cv, hipStream_t s);
/* The same with bf16 MFMA operands (bf16 compute mode): x, bias, hq, hk, ghq, ghk, gv and gx stay fp32 (x and gv
 * are rounded to bf16 as they are staged); w [3][4 hid][C], wt [3][C][4 hid] (per degree l, not per m-row),
 * wvt [3][C][cv] and the kept product y [9][N][4 hid] are bf16.  Requires hid % 64 == 0, C % 64 == 0 (fwd) /
 * C % 128 == 0 (bwd), cv % 64 == 0. */
int e2v2_qk_proj_fwd_bf16(const float* x, const void* w, const float* bias, void* y, float* hq, float* hk, int n,
                          int hid, int c, hipStream_t s);
int e2v2_qk_proj_bwd_bf16(const void* y, const float* ghq, const float* ghk, const void* wt, const float* gv,
                          const void* wvt, float* gx, int n, int hid, int c, int cv, hipStream_t s);
/* y = silu(LayerNorm(x) * g + b) on rows x [n][w] (w % 64 == 0, w <= 1024), the LayerNorm + SiLU of the
   Q/K head (final_linear of SO3_Linear2Scalar_e2former, module_utils.py:2230-2233,2268); stats [n][2] =
   (mean, rstd) kept for the backward, which returns the input gradient only. */
int e2v2_ln_silu_fwd(const float* x, const float* g, const float* b, float* y, float* stats, int n, int w, float eps,
                     hipStream_t s);
int e2v2_ln_silu_bwd(const float* x, const float* g, const float* b, const float* stats, const float* gy, float* gx,
                     int n, int w, hipStream_t s);

/* ---- positions --------------------------------------------------------- */
int e2v2_edge_to_pos(int n_atoms, const int32_t* row_ptr, const int32_t* key_ptr, const int32_t* key_eid,
                     const float* dvec, const float* dist, const float* ddvec, const float* ddist, float* dpos,
                     hipStream_t s);

#ifdef __cplusplus
}
#endif
#endif /* E2V2_H */
