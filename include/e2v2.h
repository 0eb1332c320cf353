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
 *   e2v2_segment_metadata src/molfm/models/e2former/triton_dr/triton_sparse_qk_autograd.py:601-652
 *   e2v2_pair_*         construct_radius_neighbor in its padded-batch form (module_utils.py:3119-3242)
 *   e2v2_seg_*, e2v2_gather_rows, e2v2_outer_*
 *                       the op-level Triton kernels of src/molfm/models/e2former/triton_dr/ behind
 *                       sparse_qk_edge_index_triton, sparse_alpha_sum_edge_index_triton,
 *                       sparse_v_agg_edge_index_triton_cblocked and edge_degree_outer_triton, first and
 *                       second order
 *   e2v2_radial_table*  GaussianSmearing + RadialProfile over x_edge = [rbf, tgt, src]
 *                       src/molfm/models/e2former/e2former.py:258-266, 302 (fc_easy) and
 *                       e2former.py:709-733 (gbf_projs); module_utils.py:1853-1869, 2151-2178,
 *                       as per-type-pair tables of the distance (the edge kernels interpolate them)
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
  const uint8_t* src_include;       /* [n_atoms] or NULL: only atoms j with src_include[j] != 0 are
                                       edge sources (the long-range list's include_mask,
                                       e2former_wrapper.py:225-231); images exist as before */
} e2v2_nbr_plan;

int e2v2_nbr_bin(const e2v2_nbr_plan* plan, hipStream_t s);
/* row_count [n_atoms]; row_ptr [n_atoms+1]; plan->stats = {E, max row} */
int e2v2_nbr_count(const e2v2_nbr_plan* plan, int32_t* row_count, int32_t* row_ptr, hipStream_t s);
/* rows sorted by (distance, j, shift); tmp_* are [E] (tmp_dvec [E,3]) scratch */
int e2v2_nbr_fill(const e2v2_nbr_plan* plan, const int32_t* row_ptr, int64_t n_edges, int max_row,
                  int32_t* tmp_col, int32_t* tmp_shift, float* tmp_dvec, float* tmp_dist, uint64_t* tmp_key,
                  int32_t* col, int32_t* shift, float* dvec, float* dist, hipStream_t s);
/* Capacity build, for callers that size the edge arrays without reading the count back (the MD loop):
 * after e2v2_nbr_count, clamp row_ptr to the first cap_edges edge slots and set stats[3] = 1 when the list
 * needs more than cap_edges edges or a row longer than cap_row (then it is truncated and must be rebuilt);
 * e2v2_nbr_fill is then called with n_edges = cap_edges, max_row = cap_row.  stats holds 4 ints. */
int e2v2_nbr_cap(int32_t* row_ptr, int n_rows, int64_t cap_edges, int cap_row, int32_t* stats, hipStream_t s);
/* keep the k nearest of each sorted row: phase 0 counts + scans (stats = {E', max}), phase 1 compacts */
int e2v2_nbr_topk(const int32_t* row_ptr, int n_rows, int k, int32_t* cnt, int32_t* new_ptr, int32_t* stats,
                  const int32_t* col, const int32_t* shift, const float* dvec, const float* dist,
                  int32_t* ocol, int32_t* oshift, float* odv, float* od, int phase, hipStream_t s);
/* No counterpart in the reference: for callers that cannot allocate device memory (code under HIP graph
   capture, tight serving loops).  e2v2_nbr_bin + e2v2_nbr_count in one call with the plan's workspace
   (atom_bin, bin_count, bin_start, bin_atoms, stats; those pointers are ignored) replaced by a static device
   array of the library (16 MB per GPU, held until the process ends): at most E2V2_NOALLOC_MAX_ATOMS atoms
   and E2V2_NOALLOC_MAX_BINS bins, larger plans are rejected before any launch.  Outputs as e2v2_nbr_count:
   row_count [n_atoms], row_ptr [n_atoms + 1]; stats_out [3] = {E, max row, 1 if an atom lies outside its
   graph's grid box} (cleared by the call).  Calls no allocator.  The array keeps the last call's contents
   and every call on a GPU shares it: calls that overlap on one device (other streams or threads) race. */
#define E2V2_NOALLOC_MAX_ATOMS (1 << 20)
#define E2V2_NOALLOC_MAX_BINS (1 << 20)
int e2v2_nbr_count_noalloc(const e2v2_nbr_plan* plan, int32_t* row_count, int32_t* row_ptr, int32_t* stats_out,
                           hipStream_t s);
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
   columns of any length, no host check needed between the phases).  The edges are those below
   min(n_edges, row_ptr[n_rows]) (the arrays may be sized for more, as in a capacity build). */
int e2v2_csr_transpose(const int32_t* row_ptr, const int32_t* col, int n_rows, int n_cols, int64_t n_edges,
                       int32_t* edge_row, int32_t* key_cnt, int32_t* key_ptr, int32_t* stats,
                       uint64_t* tmp_key, int32_t* key_eid, int phase, hipStream_t s);
/* Segment metadata of an edge list in any order, the (row_ptr, col_index, alpha_index) triple of
   _prepare_segment_metadata (src/molfm/models/e2former/triton_dr/triton_sparse_qk_autograd.py:615-632):
   the edges of row r in ascending edge order (a stable sort by row_index), col_index[p] =
   other_index[alpha_index[p]].  Phase 0: row_ptr [n_rows + 1] and stats [3] = {edges counted, longest
   row, entries of row_index outside [0, n_rows)}; the caller reads stats[2] and runs phase 1 (col_index,
   alpha_index [n_edges]) only when it is 0.  cnt [n_rows] and tmp_key [n_edges] are scratch. */
int e2v2_segment_metadata(const int32_t* row_index, const int32_t* other_index, int64_t n_edges, int n_rows,
                          int32_t* row_ptr, int32_t* col_index, int32_t* alpha_index, int32_t* cnt,
                          uint64_t* tmp_key, int32_t* stats, int phase, hipStream_t s);

/* Padded-batch radius search by direct distance evaluation: construct_radius_neighbor
   (src/molfm/models/e2former/module_utils.py:3119-3242).  Query q (a real atom, node_pos[node_mask]
   flattened) of batch row qgraph[q] meets all l2 padded expanded positions of that row (padding
   included, as in the reference); the pair (q, k) is kept when min_dist <= d <= max_dist and
   include[row][k] (NULL: all), d = sqrt((dx dx + dy dy) + dz dz) in fp32 of dv = node_pos - expand_pos.
   Rows are sorted by (d, k) and cut to their k_keep nearest; neighbor_idx = min(sbase[row] + k,
   n_flat - 1) indexes the flattened expanded nodes sflat (expand_node_pos[expand_node_mask]),
   f_edge_vec = qpos[q] - sflat[neighbor_idx], f_poly_dist = polynomial(d, max_dist) (poly 0,
   module_utils.py:1946-1954) or smooth_polynomial_bell(d, min_dist, max_dist, 2) (poly 1, :1956-1985). */
typedef struct e2v2_pair_plan {
  int32_t n_query, n_graphs, l2, n_flat;
  float max_dist, min_dist;
  int32_t poly;                     /* 0 polynomial envelope (exponent 5), 1 smooth bell (exponent 2)   */
  const float* qpos;                /* [n_query, 3]                                                     */
  const int32_t* qgraph;            /* [n_query] batch row of each query                                */
  const float* spos;                /* [n_graphs, l2, 3] padded expanded positions                      */
  const uint8_t* include;           /* [n_graphs, l2] or NULL                                           */
  const int32_t* sbase;             /* [n_graphs] flattened index of each row's first expanded node     */
  const float* sflat;               /* [n_flat, 3]                                                      */
} e2v2_pair_plan;
/* row_count [n_query], row_ptr [n_query + 1]; stats [2] = {pairs, longest row} */
int e2v2_pair_count(const e2v2_pair_plan* plan, int32_t* row_count, int32_t* row_ptr, int32_t* stats,
                    hipStream_t s);
/* new_ptr [n_query + 1]: the kept pairs per row, from e2v2_nbr_topk phase 0 over row_ptr with
   k_keep (rows are cut to their first new_ptr[q+1] - new_ptr[q] pairs); tmp_key [n_pairs] scratch;
   outputs of new_ptr[n_query] entries: query_idx, neighbor_idx (int64), edge_vec [., 3], dist, poly. */
int e2v2_pair_emit(const e2v2_pair_plan* plan, const int32_t* row_ptr, int64_t n_pairs, int max_row,
                   const int32_t* new_ptr, uint64_t* tmp_key, int64_t* query_idx, int64_t* neighbor_idx,
                   float* edge_vec, float* dist, float* poly, hipStream_t s);

/* ---- op-level sparse edge kernels -------------------------------------- */
/* The segment layout of the reference's Triton kernels: slot p of row r (row_ptr[r] <= p <
   row_ptr[r+1]) carries edge alpha_index[p] and partner row col_index[p].  Slots whose partner row is
   outside [0, n_cols) or whose edge is outside [0, n_edges) are skipped; row bounds are clamped to
   [0, n_slots].  Rows are summed in slot order by one workgroup each (deterministic).  Operands are
   fp32 with element strides: a logical [rows, H, D] operand A has A[r, h, d] at r s[0] + h s[1] + d s[2]. */
typedef struct e2v2_segments {
  const int32_t* row_ptr;           /* [n_rows + 1]                                                     */
  const int32_t* col_index;         /* [n_slots] (may be NULL where no partner operand is read)          */
  const int32_t* alpha_index;       /* [n_slots]                                                        */
  int32_t n_rows, n_cols;
  int64_t n_slots, n_edges;
} e2v2_segments;
/* out[alpha_index[p], h] = sum_d A[r, h, d] B[col_index[p], h, d] over the slots of every row r:
   _edge_qk_fwd_csr_kernel (triton_sparse_qk_autograd.py:52-130) and, with A, B viewed [M, H, C] from
   [M, C, H], _edge_dot_cblocked (sparse_v_agg_edge_index_cblocked_bench.py:133-161).  Slots not written
   keep their value. */
int e2v2_seg_dot(const e2v2_segments* seg, const float* A, const int64_t* a_strides, const float* B,
                 const int64_t* b_strides, int H, int D, float* out, const int64_t* out_strides, hipStream_t s);
/* out[r, h, d] = sum_p W[alpha_index[p], h] X[col_index[p], h, d] (every row written):
   _edge_grouped_reduce_triton / _bwdk_n_tiled_spmv (triton_sparse_qk_autograd.py:388-435, 655-673),
   _edge_index_cblocked_kernel and _edge_grouped_reduce_cblocked (sparse_v_agg_edge_index_cblocked_bench.py:
   164-294).  X NULL (D = 1): out[r, h] = sum_p W[alpha_index[p], h], _fwd_alpha_sum_edge_index
   (sparse_alpha_sum_edge_index_autograd.py:28-67, 112-126). */
int e2v2_seg_reduce(const e2v2_segments* seg, const float* W, const int64_t* w_strides, const float* X,
                    const int64_t* x_strides, int H, int D, float* out, const int64_t* out_strides, hipStream_t s);
/* out[e, :K] = in[index[e], :K] (zero rows for an index outside [0, n_in)): _bwd_alpha_sum_edge_index
   (sparse_alpha_sum_edge_index_autograd.py:70-99). */
int e2v2_gather_rows(const float* in, int64_t n_in, const int32_t* index, int64_t n, int K, float* out,
                     hipStream_t s);
/* out[r, l, h] = sum_p sh[alpha_index[p], l] fea[alpha_index[p], h], contiguous [E, L], [E, H], [R, L, H]:
   _edge_outer_reduce_kernel (triton_dr/edge_degree_outer_autograd.py:25-70, 181-204). */
int e2v2_outer_reduce(const e2v2_segments* seg, const float* sh, const float* fea, int L, int H, float* out,
                      hipStream_t s);
/* dsh[e, l] = sum_h grad[q_e, l, h] fea[e, h] and dfea[e, h] = sum_l grad[q_e, l, h] sh[e, l] (either
   output may be NULL; q_e outside [0, n_rows) gives 0): _edge_dsh_kernel / _edge_dfea_kernel
   (edge_degree_outer_autograd.py:81-178, 207-256). */
int e2v2_outer_bwd(const float* grad, int n_rows, const float* sh, const float* fea, const int32_t* query_index,
                   int64_t n_edges, int L, int H, float* dsh, float* dfea, hipStream_t s);

/* ---- radial profiles as distance tables ------------------------------- */
/* A RadialProfile [256 + 2 n_emb -> 128 -> LayerNorm -> SiLU -> 128 -> LayerNorm -> SiLU -> 256] over
   x_edge = [rbf(d), tgt[z_i], src[z_j]] is, for one pair of atom types, a function of the edge distance d
   alone.  Its table, for a set of n_types atom types (type slot a has atomic number type_z[a]), holds per
   table slot p of a type pair (a, b) (a: the query atom's type, b: the source atom's; the slots the caller
   chose, see e2v2_radial_table) and node n (d = n h, h a power of two) four rows of nc channels: row
   k = h^k d^k f / dd^k (k = 0..3), float64-built by exact Taylor-series propagation through every op.
   Layout tab[p][n][k][nc]; a profile's 256 output
   channels are placed in each row by an e2v2_radial_layout.  The edge kernels interpolate rows 0..2
   (value) and rows 1..3 (derivative) with quintic Hermite polynomials, and read the tables in these
   layouts:
     attention (nc = 256, fc_easy = gate | inputhead): the slice order below, i.e. the gate and the
       inputhead of head h at positions E2V2_POS0(h) and E2V2_POS1(h), stored slice-major;
       layout {col0 0, split 128, block 16, block_stride 32, split_stride 16, slice_width 32};
     degree embedding (nc = 768, profiles l = 0, 1, 2): channel c of profile l at
       96 (c / 32) + 32 l + c % 32, stored slice-major (each 32-channel slice of the three profiles
       contiguous); layout {col0 32 l, split 256, block 32, block_stride 96, split_stride 0,
       slice_width 96};
     contiguous (any other caller): channel c of profile m at 256 m + c;
       layout {col0 256 m, split 256, block 256, block_stride 0, split_stride 0, slice_width 0}. */
#define E2V2_MAX_TYPES 256
/* table slots per launch (one per type pair an edge can join) */
#define E2V2_MAX_PAIRS 65535
typedef struct e2v2_radial_net {
  const float* w1;  int32_t ld_w1;    /* Linear1 weight [128][ld_w1], ld_w1 = 256 + 2 n_emb     */
  int32_t n_emb;                      /* width of the type embeddings                           */
  const float* b1;                    /* [128]                                                  */
  const float* g1; const float* be1;  /* LayerNorm(128), eps 1e-5                               */
  const float* w2; const float* b2;   /* [128][128], [128]                                      */
  const float* g2; const float* be2;  /* LayerNorm(128)                                         */
  const float* w3; const float* b3;   /* [256][128], [256]                                      */
  const float* tgt;                   /* [n_types_max][n_emb] target (query atom) embedding     */
  const float* src;                   /* [n_types_max][n_emb] source atom embedding             */
} e2v2_radial_net;

/* Node spacing h = 2^(floor(log2(0.2 sigma)) - refine) (-3 <= refine <= 6) of a GaussianSmearing basis
   exp(coeff (d - mu)^2) (sigma = sqrt(-0.5 / coeff)) and the node count covering [0, rc]. */
int e2v2_radial_table_size(float rc, float rbf_coeff, int32_t refine, int32_t* n_nodes, float* h);
/* Position of output channel o (0..255) of a profile in a table row:
   pos = col0 + ((o % split) / block) * block_stride + (o / split) * split_stride + o % block
   (checked on the host: every channel inside the row, no two at one position).  slice_width = 0: the
   table is tab[p][n][k][nc], rows contiguous; slice_width = w > 0: it is tab[p][nc / w][n][k][w], channel
   position pos in slice pos / w at column pos % w (each slice of a pair contiguous, its four rows at a node
   4 w floats apart). */
typedef struct e2v2_radial_layout {
  int32_t col0, split, block, block_stride, split_stride, slice_width;
} e2v2_radial_layout;
/* Build one profile's channels of tab (device type_z [n_types], rbf_offset [256] = mu) for n_pairs table
   slots: slot p holds the type pair pair_ab[p] = a n_types + b (device int32), or, with pair_ab NULL,
   n_pairs = n_types^2 slots in the order p = a n_types + b.  Callers give a slot to every pair that an edge
   can join (e.g. the products of each graph's own type set) and map pairs to slots with pair_slot
   [n_types^2] (slot, or -1) in the edge kernels' arguments. */
int e2v2_radial_table(const e2v2_radial_net* net, const float* rbf_offset, float rbf_coeff, const int32_t* type_z,
                      int32_t n_types, const int32_t* pair_ab, int32_t n_pairs, int32_t n_nodes, float h, float* tab,
                      int32_t nc, const e2v2_radial_layout* layout, hipStream_t s);
/* Interpolation error of one profile's table at every interval midpoint against the float64 profile:
   err (uint32 [4], zeroed by the caller) receives the float bits of max |f - f~|, max |f|,
   max h |f' - f~'|, max h |f'|. */
int e2v2_radial_table_check(const e2v2_radial_net* net, const float* rbf_offset, float rbf_coeff,
                            const int32_t* type_z, int32_t n_types, const int32_t* pair_ab, int32_t n_pairs,
                            int32_t n_nodes, float h, const float* tab, int32_t nc, const e2v2_radial_layout* layout,
                            uint32_t* err, hipStream_t s);

/* The same table of a profile's 128 hidden channels (the output of its second SiLU, the input of its last
   Linear, module_utils.py:2159-2172), placed by the layout as channels o = 0..127: a profile's output is
   W3 h + b3 of the hidden channels h, so a sum over edges of outputs times edge factors equals W3 times the
   sum of hidden channels times the same factors plus b3 times the sum of the factors (the degree
   embedding, e2v2_deg_hidden_fwd).  The check's errors (err as for e2v2_radial_table_check) are those of the
   output W3 h~ + b3 formed in float64 from the interpolated h~ and h~', against the float64 output: the
   same tolerances as a table of the outputs.  Degree-embedding layout (nc = 384, profiles l = 0, 1, 2):
   hidden channel o of profile l at 96 (o / 32) + 32 l + o % 32, stored slice-major (four slices);
   layout {col0 32 l, split 128, block 32, block_stride 96, split_stride 0, slice_width 96}. */
int e2v2_radial_hidden_table(const e2v2_radial_net* net, const float* rbf_offset, float rbf_coeff,
                             const int32_t* type_z, int32_t n_types, const int32_t* pair_ab, int32_t n_pairs,
                             int32_t n_nodes, float h, float* tab, int32_t nc, const e2v2_radial_layout* layout,
                             hipStream_t s);
int e2v2_radial_hidden_table_check(const e2v2_radial_net* net, const float* rbf_offset, float rbf_coeff,
                                   const int32_t* type_z, int32_t n_types, const int32_t* pair_ab, int32_t n_pairs,
                                   int32_t n_nodes, float h, const float* tab, int32_t nc,
                                   const e2v2_radial_layout* layout, uint32_t* err, hipStream_t s);

/* Per-edge values of a "plain"-layout table ([pairs][n_nodes][4][nc], nc channels): out [E][nc] =
   f_c(dist[e]) for the pair (atom_type[edge_row[e]], atom_type[col[e]]), the quintic Hermite interpolant.
   Replaces the per-edge RadialProfile calls of the QKdot gates, rad_func_m0(x_edge) (e2former.py:278)
   and fc_easy(x_edge)[:, H:] (e2former.py:293-294).  e_end (device int32, or NULL for n_edges): the
   number of real edges, read on the device (the query CSR's row_ptr[n_rows]); slots e >= *e_end of a
   capacity build are not read and get out[e][:] = 0. */
int e2v2_radial_eval(const float* tab, int32_t n_types, const int32_t* pair_slot, int32_t n_nodes, float h,
                     int32_t nc, const int32_t* atom_type, const int32_t* edge_row, const int32_t* col,
                     const float* dist, int64_t n_edges, const int32_t* e_end, float* out, hipStream_t s);
/* ddist [E] = sum_c grad[e][c] f_c'(dist[e]) (fixed summation order); ddist[e] = 0 for e >= *e_end. */
int e2v2_radial_eval_bwd(const float* tab, int32_t n_types, const int32_t* pair_slot, int32_t n_nodes, float h,
                         int32_t nc, const int32_t* atom_type, const int32_t* edge_row, const int32_t* col,
                         const float* dist, int64_t n_edges, const int32_t* e_end, const float* grad, float* ddist,
                         hipStream_t s);
/* x0 [E][3][C] = sum_{m in l} Y[e][m] xn[m][row(e)][C] for l = 0, 1, 2 (Y [E][9], xn [9][n_rows][C]
   m-major, edges of a row contiguous by row_ptr [n_rows + 1], C <= 256): the x_0_extra of QKdot_alpha
   (e2former.py:271-276, Y the normalised spherical harmonics) and of QKdotS_alpha (e2former.py:288-296,
   the raw polynomials of edge_vec with sum_vec's l blocks). */
int e2v2_sh_contract(const float* Y, const float* xn, const int32_t* row_ptr, int32_t n_rows, int32_t C,
                     float* x0, hipStream_t s);
/* Its backward for the gradient g [E][3][C]: dY [E][9], dxn [9][n_rows][C] (per-row sums, no atomics). */
int e2v2_sh_contract_bwd(const float* Y, const float* xn, const int32_t* row_ptr, int32_t n_rows, int32_t C,
                         const float* g, float* dY, float* dxn, hipStream_t s);

/* ---- attention --------------------------------------------------------- */
/* Channel order of v, out, grad_out, dv and of the fc_easy table rows ("slice order"): position p of a
   row holds the first (model channel h, the gate in the table) or second (model channel 128 + h, the
   inputhead) channel of head h, at E2V2_POS0(h) and E2V2_POS1(h); slice s = p / 32 holds heads
   16 s .. 16 s + 15.  Callers fold the permutation into the producing and consuming weights. */
#define E2V2_POS0(h) (32 * ((h) / 16) + (h) % 16)
#define E2V2_POS1(h) (E2V2_POS0(h) + 16)
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
  const float* rtab;             /* fc_easy table [T*T][8][rtab_n][4][32]: slice order, slice-major */
  const int32_t* atom_type;      /* [N] type slot of each atom, 0 .. n_types - 1     */
  int32_t n_types, rtab_n;       /* T, table nodes                                  */
  float rtab_h;                  /* node spacing (a power of two)                   */
  float q_div;                   /* sqrt(D)                                         */
  float rc, env_a, env_b, env_c; /* polynomial envelope                             */
  int32_t act_bf16;              /* 1: q, k, v, out, grad_out stored as bf16 (fp32 math) */
  /* Optional key-CSR column clusters from e2v2_cluster_slots with span col_span = 4 (NULL: one
     workgroup per column); used by the fp32 column pass of e2v2_attn_bwd. */
  int32_t col_span;
  const int32_t* col_slot_member; const int32_t* col_slot_edge; const int32_t* col_n_slots;
  /* zero_order 0: the SO(2) first-order product ("so2-first-order", weights alpha / r, 20 output rows);
     1: the zero-order aggregation ("zero-order", e2former.py:411-416: out[r][i][c] = sum_e
     alpha_e,h(c) v_j[r][c], weights alpha, 9 output rows [9][N][C] m-major) */
  int32_t zero_order;
  /* envelope of the weights: env_kind 0 the polynomial (rc, env_a/b/c), 1 the smooth bell on
     [env_lo, rc] (module_utils.py:1956-1985, exponent 2) */
  int32_t env_kind;
  float env_lo;
  /* ext_gate [E][H] fp32 or NULL: the gate of every (edge, head) given by the caller (the QKdot_alpha /
     QKdotS_alpha logits gates, e2former.py:270-300) instead of the table's gate rows, which are then not
     read; with it e2v2_attn_bwd writes dL/dgate of every (edge, head) to ext_dgate [E][H] and leaves the
     gate's distance derivative out of ddist */
  const float* ext_gate;
  float* ext_dgate;
  /* type pair -> table slot [n_types^2] (device int32; NULL: slot a n_types + b, all pairs in the table) */
  const int32_t* pair_slot;
  /* weight form (e2former.py:329-360): 0 the segmented softmax alpha = exp(a - max) p ih / (sum + 1e-3);
     1 alpha = softplus(a) ih p (tp_type "+softplus"); 2 alpha = sigmoid(a) ih p ("+sigmoid"), with
     a = gate q.k / sqrt(D).  Forms 1 and 2 have no row statistics: mrow holds 0 and srow 0. */
  int32_t weight_act;
} e2v2_attn_args;

/* v [9][N][C] is m-major (row r of every atom contiguous), channels in slice order.  out holds the 20
   l3-sequential rows h_a - h_b of the SO(2) product (float, or bf16 if act_bf16; 20 N C values, channels in
   slice order) in the l3-grouped layout: the 2 l3 + 1 rows of output degree l3 keep their cnt coupling
   paths side by side, a block [2 l3 + 1][N][cnt C] (blocks in l3 order: l3 = 0 with 1 path, 1 with 3,
   2 with 2), so that each block is the [(2 l3 + 1) N, cnt C] operand of the per-l3 output Linear
   (so2_tensor_product.py:276-290).  Row t (path p, order m of degree l3) of channel c of atom i sits at
   N E2V2_SO2_A(t) + i E2V2_SO2_LD(t) + E2V2_SO2_COL(t) + c.  mrow/srow [N,H] softmax max / sum; cnt [N,H]
   number of maxima.  gate and inputhead of every edge are interpolated from rtab in the kernel (nothing
   per edge is stored). */
#define E2V2_SO2_A(t) ((t) == 0 ? 0 : (t) < 10 ? 256 + 768 * (((t) - 1) % 3) : 2560 + 512 * (((t) - 10) % 5))
#define E2V2_SO2_LD(t) ((t) == 0 ? 256 : (t) < 10 ? 768 : 512)
#define E2V2_SO2_COL(t) ((t) == 0 ? 0 : (t) < 10 ? 256 * (((t) - 1) / 3) : 256 * (((t) - 10) / 5))
int e2v2_attn_fwd(const e2v2_attn_args* args, void* out, float* mrow, float* srow, int32_t* cnt, hipStream_t s);
/* Bytes of device workspace e2v2_attn_bwd needs for n_edges edges (per-edge weights handed from the row
   pass to the column pass and per-slice partial edge gradients, alive during the call only). */
size_t e2v2_attn_bwd_workspace(int64_t n_edges);
/* grad_out, out (l3-grouped as above; float, or bf16 if act_bf16) -> ddvec [E,3], ddist [E] (including the radial
   profile's distance derivative, from the table), dq, dk [N,H,D], dv [9][N][C] (all float, dv in slice
   order); workspace: e2v2_attn_bwd_workspace(E) bytes, 16-byte aligned */
int e2v2_attn_bwd(const e2v2_attn_args* args, const void* grad_out, const void* out, const float* mrow,
                  const float* srow, const int32_t* cnt, float* ddvec, float* ddist, float* dq, float* dk, float* dv,
                  void* workspace, size_t workspace_bytes, hipStream_t s);

/* ---- edge-degree embedding -------------------------------------------- */
typedef struct e2v2_deg_args {
  int32_t n_rows;
  int64_t n_edges;
  int32_t channels;              /* 256                                             */
  const int32_t* row_ptr;
  const float* dvec;             /* [E,3]                                           */
  const float* dist;             /* [E]                                             */
  const int32_t* col;            /* [E] source atom                                 */
  const float* rtab;             /* gbf_projs table [T*T][8][rtab_n][4][96] (slice-major, profiles l = 0, 1, 2) */
  const int32_t* atom_type;      /* [N] type slot of each atom                      */
  int32_t n_types, rtab_n;
  float rtab_h;
  float avg;                     /* avg_aggregate_num                               */
  float rc, env_a, env_b, env_c;
  const int32_t* pair_slot;      /* type pair -> table slot [n_types^2], or NULL (all pairs) */
} e2v2_deg_args;

/* x0 [9][N][C] m-major */
int e2v2_deg_fwd(const e2v2_deg_args* args, float* x0, hipStream_t s);
/* Bytes of device workspace e2v2_deg_bwd needs for n_edges edges (per-slice partial edge gradients). */
size_t e2v2_deg_bwd_workspace(int64_t n_edges);
/* grad_x0 [9][N][C] -> ddvec [E,3], ddist [E] (spherical harmonics, envelope and the profiles' distance
   derivative from the table); workspace: e2v2_deg_bwd_workspace(E) bytes, 16-byte aligned */
int e2v2_deg_bwd(const e2v2_deg_args* args, const float* grad_x0, float* ddvec, float* ddist, void* workspace,
                 size_t workspace_bytes, hipStream_t s);

/* The degree embedding through the gbf_projs hidden channels (e2former.py:728-748 with the last Linear of
   each profile, module_utils.py:2159-2172, moved past the sum over edges):
     hs[m][i][k] = (1/avg) sum_e Y_m(e) p(e) h_l(m),k(e)   (k < 128),
     hs[m][i][128] = (1/avg) sum_e Y_m(e) p(e),   hs[m][i][129..143] = 0,
   hs [9][N][144] m-major (16-byte aligned); then x0[m] = hs[m] [W3_l | b3_l | 0]^T (a per-node GEMM, 144 -> 256) is the
   output of e2v2_deg_fwd.  args.rtab is the hidden table (e2v2_radial_hidden_table, degree layout, nc 384)
   and args.channels = 128. */
int e2v2_deg_hidden_fwd(const e2v2_deg_args* args, float* hs, hipStream_t s);
/* grad_h [9][N][128] (16-byte aligned) = grad_x0[m] W3_l and grad_s [9][N] = grad_x0[m] . b3_l (unscaled: the kernel applies
   1/avg) -> ddvec [E,3], ddist [E]; workspace: e2v2_deg_bwd_workspace(E) bytes, 16-byte aligned. */
int e2v2_deg_hidden_bwd(const e2v2_deg_args* args, const float* grad_h, const float* grad_s, float* ddvec,
                        float* ddist, void* workspace, size_t workspace_bytes, hipStream_t s);
/* grad_s [9][n] = sum_c grad_x0[m][i][c] b3[l(m)][c] (grad_x0 [9][n][256] m-major, b3 [3][256]; fixed order). */
int e2v2_deg_bias_grad(const float* grad_x0, const float* b3, int32_t n, float* grad_s, hipStream_t s);

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
/* rms_norm_sh on the training path (the reference's norm under torch's double backward, e2former.py:600-620
   with AutoGradForce's create_graph=True).  _bwd_param: gx as e2v2_rmsnorm_bwd plus the affine gradients as
   per-workgroup partial sums part [n_part][4][256] (rows dw_0, dw_1, dw_2, db; the caller sums the n_part
   blocks).  _bwd2: the derivative of that first-order pass given the upstream gradients qx [9][n][256],
   qw [3][256], qb [256] of (gx, dw, db) (each may be NULL: zero): dgy, dx [9][n][256] and the partial sums of
   the weight gradient part [n_part][3][256] (the bias does not enter the first-order pass).
   0 < n_part <= 65535 workgroups, nodes strided over them. */
int e2v2_rmsnorm_bwd_param(const float* x, const float* w, const float* gy, float* gx, float* part, int n, int n_part,
                           float eps, hipStream_t s);
int e2v2_rmsnorm_bwd2(const float* x, const float* w, const float* gy, const float* qx, const float* qw,
                      const float* qb, float* dgy, float* dx, float* part, int n, int n_part, float eps,
                      hipStream_t s);
/* Gate_s3 activation (module_utils.py:2694-2746) from gate logits sc [N][768];
 * k1, k2 = normalize2mom constants of SiLU and sigmoid */
int e2v2_gate_fwd(const float* sc, const float* x, float* y, int n, float k1, float k2, hipStream_t s);
int e2v2_gate_bwd(const float* sc, const float* x, const float* gy, float* gsc, float* gx, int n, float k1,
                  float k2, hipStream_t s);
/* Derivative of e2v2_gate_bwd for the training path's second differentiation (torch's double backward of
   Gate_s3's silu / sigmoid products): given the upstream gradients qsc [N][768] on gsc and qx [9][N][256] on gx
   (each may be NULL: zero), dgy, dx [9][N][256] and dsc [N][768]. */
int e2v2_gate_bwd2(const float* sc, const float* x, const float* gy, const float* qsc, const float* qx, float* dgy,
                   float* dsc, float* dx, int n, float k1, float k2, hipStream_t s);

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
/* Training-path LayerNorm + SiLU of the RadialProfile nets (module_utils.py:2151-2178: the nn.LayerNorm +
   nn.SiLU pairs, whose gradients torch composes for each autograd order).  With stats from e2v2_ln_silu_fwd:
   _bwd_param returns the input gradient gx and the affine gradients as per-block partial sums
   part_g / part_b [n_part][w] (the caller sums the n_part rows); _bwd2 differentiates that first-order
   pass once more: given the upstream gradients qx [n][w], qg [w], qb [w] of (gx, dg, db) (each may be NULL:
   zero) it returns dgy, dx [n][w] and the partial sums of the affine gradients.  w in {64, 128, 192, 256,
   384, 512}; 0 < n_part <= 65535 blocks of 4 wavefronts (one row per wavefront). */
int e2v2_ln_silu_bwd_param(const float* x, const float* g, const float* b, const float* stats, const float* gy,
                           float* gx, float* part_g, float* part_b, int n, int w, int n_part, hipStream_t s);
int e2v2_ln_silu_bwd2(const float* x, const float* g, const float* b, const float* stats, const float* gy,
                      const float* qx, const float* qg, const float* qb, float* dgy, float* dx, float* part_g,
                      float* part_b, int n, int w, int n_part, hipStream_t s);

/* ---- per-node dense layers: fp32 GEMMs on bf16 MFMA by the exact three-piece split ----
 * Replaces the GEMMs (forward and input gradient) of SO3_Linear_e2former (module_utils.py:2010-2052) and so of
 * FeedForwardNetwork_s3 (module_utils.py:2755-2797), the value projection and proj_first (e2former.py:215-219,
 * 300-303, 433), forward_linear (wigner6j/so2_tensor_product.py:276-290), the final_linear of
 * SO3_Linear2Scalar_e2former (module_utils.py:2230-2233) and the gate logits of Gate_s3 (module_utils.py:2694-2746).
 * Each fp32 operand x is split as x0 + x1 + x2 (bf16, round to nearest even, exact remainders) and a product is
 * the sum of the six piece products of order <= 2, accumulated in fp32: an fp32 GEMM to within a few units of
 * fp32 rounding (measured against float64: below the error of the fp32 MFMA GEMM of the same operands).
 *   c[b][i][j] = sum_k a[b][i][k] W_{widx[b]}[j][k] (+ bias[b bias_bs + j] for b < bias_batches) (+ r[b][i][j])
 * a: fp32, row stride lda (lda >= k, lda % 4 == 0, 16-byte aligned), batch b at a + b a_bs (elements; any
 * distance, so two separate matrices of the same layout form a batch);
 * b: n_w weights packed by e2v2_gemm_pack; c (and r, which may equal c): fp32 with row / batch strides.
 * Requires n % 128 == 0, k % 16 == 0, 1 <= batch <= 16, 0 <= widx[b] < n_w <= 16. */
typedef struct {
  const void* a;        /* fp32, or bf16 when a_bf16 */
  int64_t lda, a_bs;
  const void* b;
  int n_w;
  void* c;              /* fp32, or bf16 when c_bf16 */
  int64_t ldc, c_bs;
  const float* r;
  int64_t ldr, r_bs;
  const float* bias;
  int64_t bias_bs;      /* elements between the bias vectors of consecutive batches (0: one shared vector) */
  int bias_batches;
  int m, n, k, batch;
  int widx[16];
  int pieces;           /* operand pieces of b's packing: 3 (fp32 GEMM) or 1 (bf16 operands, fp32 accumulation) */
  int a_bf16;           /* 1: a is bf16 in memory (with pieces = 1; lda % 8 == 0) */
  int c_bf16;           /* 1: c is written as bf16 (rounded once from the fp32 result) */
} e2v2_gemm_args;
int e2v2_gemm_s3(const e2v2_gemm_args* args, hipStream_t s);
/* Up to four independent GEMMs (each as e2v2_gemm_s3, with its own shapes, operands and packed weight) in one
 * launch: the groups' tiles share the GPU instead of running one small launch after another; groups are
 * dispatched in the order given (put the longest k first).  Used for the per-degree GEMMs of forward_linear +
 * proj_first (so2_tensor_product.py:276-290, e2former.py:433) and their input gradients, which replace three
 * launches of 160-800 tiles. */
int e2v2_gemm_s3_grouped(const e2v2_gemm_args* groups, int n_groups, hipStream_t s);
/* e2v2_gemm_s3 with the activation of Gate_s3 (module_utils.py:2694-2746) applied to A as it is read, so that
 * the second Linear of FeedForwardNetwork_s3 (module_utils.py:2755-2797) takes the gate's inputs instead of its
 * output: batch 0's operand is silu(s[i][kk]) k1 (kk < k; args->a is not read for it), batch b >= 1's is
 * a[b][i][kk] sigmoid(s[i][k widx[b] + kk]) k2, with s the gate logits [m][ld_s] (16-byte aligned, ld_s % 4 == 0,
 * k (widx[b] + 1) <= ld_s).  The products are those of the gate kernel (e2v2_gate_fwd), so the result equals that
 * kernel followed by e2v2_gemm_s3. */
int e2v2_gemm_s3_gated(const e2v2_gemm_args* args, const float* s, int64_t ld_s, float k1, float k2, hipStream_t st);
/* Pack n_w weights W_w[j][k] = w[w w_stride + j ld_n + k ld_k] (j < n, k < k; so W or W^T of a row-major matrix
 * without a copy) into e2v2_gemm_packed_bytes(n_w, n, k, pieces) bytes at packed (16-byte aligned); the bytes
 * needed, or -1 for an unsupported shape.  pieces 3: the exact three-piece split; pieces 1: the bf16 rounding
 * alone, for the bf16 mode's GEMMs (bf16 operands, fp32 accumulation: one MFMA product, the A operand rounded
 * to bf16 as it is read, or read as bf16 with a_bf16). */
int64_t e2v2_gemm_packed_bytes(int n_w, int n, int k, int pieces);
/* The Q/K projection with its m-contraction (as e2v2_qk_proj_fwd / _bwd above) on the split GEMM.  Pairs
 * p < 2 hid: (q_a, q_b) columns p of the stacked w for p < hid, else (k_a, k_b) columns p - hid.
 *   fwd: wp = the three per-l [4 hid][C] weights packed with their columns in the tile-paired order (128-column
 *        tile t: the a-columns of pairs 64 t .. +63, then their b-columns), bias [4 hid] in that order (m = 0
 *        only; may be NULL); writes hq, hk [N][3 hid] and y [9][N][4 hid] with column 16 (p / 8) + 8 ab + p % 8
 *        holding side ab of pair p (kept for the backward).
 *   bwd: gx [9][N][C] = gy W (+ gv Wv when gv != NULL, gv [9][N][cv]), gy the contraction's gradient formed
 *        from y, ghq, ghk as the operand is read; wp = per l the packed [W rows in y's order ; Wv_l]^T
 *        ([C][4 hid + cv]).
 * y_bf16 = 1 (one piece only, the bf16 mode): y is stored as bf16 (rounded once; the forward's contraction uses
 * the fp32 sums) and read as bf16 by the backward: half the memory the backward keeps per layer.
 * Requires hid % 64 == 0, C % 16 (fwd) / % 128 (bwd), cv % 16 == 0; operands 16-byte aligned. */
int e2v2_qk_proj_fwd_s3(const float* x, const void* wp, const float* bias, void* y, float* hq, float* hk, int n,
                        int hid, int c, int pieces, int y_bf16, hipStream_t s);
int e2v2_qk_proj_bwd_s3(const void* y, const float* ghq, const float* ghk, const void* wp, const float* gv,
                        float* gx, int n, int hid, int c, int cv, int pieces, int y_bf16, hipStream_t s);
int e2v2_gemm_pack(const float* w, int64_t ld_n, int64_t ld_k, int64_t w_stride, int n_w, int n, int k, int pieces,
                   void* packed, hipStream_t s);

/* ---- QKdot_alpha gate ------------------------------------------------- */
/* The gate of tp_type QKdot_alpha (e2former.py:270-283) without per-edge channel tensors:
 *   gate[e][h] = bias[h] + sum_k A[e][k] W[h][k],   k < 768 = 3 x 256,
 *   A[e][256 l + c] = x0[e][l][c] rad[e][256 l + c],  x0[e][l][c] = sum_{m in l} Y[e][m] xd[m][i(e)][c],
 * with W the fc_m0 weight [128][768], Y [E][9] the edge's normalised spherical harmonics l <= 2, xd [9][N][256]
 * the query atoms' dot_linear output (m-major) and rad the rad_func_m0 profile (768 channels, "plain" table
 * layout [pairs][rtab_n][4][768], type pairs as in e2v2_attn_args).  A is formed as the GEMM reads it.  The
 * backward takes dL/dgate [E][128] and writes dL/dY [E][9], dL/ddist [E] (through rad) and dL/dxd
 * [9][N][256] (per-row sums in a fixed order, no atomics; atoms without edges get zeros); dL/dA is formed per
 * 128-edge tile in LDS and never stored.  Edges past *e_end (a device count, or NULL) give a zero gate and
 * zero gradients.  Operands fp32 and 16-byte aligned; W packed by e2v2_gemm_pack (forward: W as [128][768],
 * backward: W^T as [768][128]) with `pieces` 3 (fp32 accuracy) or 1 (bf16 mode). */
typedef struct e2v2_qkdot_args {
  int32_t n_rows;
  int64_t n_edges;
  const int32_t* row_ptr;        /* [N+1] query CSR                                 */
  const int32_t* edge_row;       /* [E]                                             */
  const int32_t* col;            /* [E] source atom                                 */
  const float* dist;             /* [E]                                             */
  const int32_t* e_end;          /* device count of valid edges, or NULL            */
  const float* Y;                /* [E][9]                                          */
  const float* xd;               /* [9][N][256]                                     */
  const float* rtab;             /* rad_func_m0 table, plain layout, 768 channels   */
  const int32_t* atom_type;
  int32_t n_types, rtab_n;
  float rtab_h;
  const int32_t* pair_slot;
  int32_t pieces;
} e2v2_qkdot_args;
int e2v2_qkdot_gate_fwd(const e2v2_qkdot_args* args, const void* w_packed, const float* bias, float* gate,
                        hipStream_t s);
/* Bytes of device workspace e2v2_qkdot_gate_bwd needs (per-tile partial sums, alive during the call). */
size_t e2v2_qkdot_gate_bwd_workspace(int64_t n_edges);
int e2v2_qkdot_gate_bwd(const e2v2_qkdot_args* args, const void* wt_packed, const float* dgate, float* dY,
                        float* ddist, float* dxd, void* workspace, size_t workspace_bytes, hipStream_t s);

/* ---- positions --------------------------------------------------------- */
int e2v2_edge_to_pos(int n_atoms, const int32_t* row_ptr, const int32_t* key_ptr, const int32_t* key_eid,
                     const float* dvec, const float* dist, const float* ddvec, const float* ddist, float* dpos,
                     hipStream_t s);

#ifdef __cplusplus
}
#endif
#endif /* E2V2_H */
