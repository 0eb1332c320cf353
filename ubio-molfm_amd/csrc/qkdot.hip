// The gate of tp_type QKdot_alpha (src/molfm/models/e2former/e2former.py:270-283):
//   x0_l = sum_{m in l} Y_m(edge) dot_linear(x)[query, m]        (e3nn spherical harmonics, normalize=True)
//   gate = fc_m0(cat_l(x0_l) * rad_func_m0(x_edge))               (768 -> 128)
// as one GEMM per direction whose edge-side operand is never stored.
//
// Forward (k_qkdot_fwd): gate = A W^T + b on the split GEMM of gemm_core.h (128 edges x 128 heads per
// workgroup, K = 768 in 48 stages of 16).  A lane forms its own A fragment (one edge, eight channels of
// the stage) in registers: rad from the six table rows of its distance interval (quintic Hermite, the
// Hermite weights and the table node formed once per edge) and x0 from the 2l + 1 rows of xd of the
// query atom, then splits it into the bf16 pieces; only W goes through LDS.
//
// Backward (k_qkdot_bwd): per (128-edge tile, 128-channel column tile) the GEMM dA = dgate W (K = 128)
// lands in LDS; thread pairs then walk the tile edge by edge (rad, its distance derivative and x0
// recomputed as in the forward) and form dx0 = dA rad (written back in place of dA), the edge's
// dL/ddist = sum dA x0 rad' and dL/dY_m = sum dx0 xd_m over the tile's channels (one partial per column
// tile and edge); threads per channel then sum Y_m dx0 over the edges of each query row in edge order
// (dL/dxd).  A row that lies inside the tile is written directly; a row that crosses a tile boundary
// leaves the tile's partial sum (as the tile's first or last row), and k_qkdot_rows adds the partials of
// such rows in tile order.  k_qkdot_edges adds the column tiles' partials of each edge.  Every sum runs in
// a fixed order: the results are deterministic.
#include "gemm_core.h"
#include "radial.h"

namespace e2v2 {
namespace {

constexpr int kQC = 256;            // channels per degree (attn_weight_input_dim)
constexpr int kQK = 3 * kQC;        // 768: the forward's K, the backward's N
constexpr int kQH = 128;            // heads: the forward's N, the backward's K
constexpr int kQSide = 9 * kQC;     // partial dL/dxd of one boundary row: [9][256]
constexpr int kQCt = kQK / kGN;     // column tiles of the backward: 6 (two per degree)
constexpr int kQPart = 6;           // per (column tile, edge): dL/ddist, then dL/dY of the tile's degree
constexpr int kQDl = kGN + 4;       // row stride (floats) of the dA tile in LDS

__device__ __forceinline__ int64_t qk_e_lim(const e2v2_qkdot_args& A) {
  return A.e_end ? min(A.n_edges, (int64_t)*A.e_end) : A.n_edges;
}

__device__ __forceinline__ floatx4 ld4(const float* p) { return *reinterpret_cast<const floatx4*>(p); }

// The per-edge state of the table lookup: offset of node n of the edge's interval and the Hermite weights.
struct QkEdge {
  int64_t toff;
  Hermite5 H;
};

__device__ __forceinline__ QkEdge qk_edge(const e2v2_qkdot_args& A, const RadialTab& R, int64_t e) {
  QkEdge q;
  float t;
  q.toff = radial_node(R, tab_pair(R, A.atom_type[A.edge_row[e]], A.atom_type[A.col[e]]), A.dist[e], t);
  q.H = hermite5(t);
  return q;
}

// x0 of the eight channels at p (channel offset within the degree) for degree L: sum over its 2L + 1 rows.
template <int L>
__device__ __forceinline__ void qk_x0(const float* xr, size_t xm, const float (&Y)[9], floatx4& x0, floatx4& x1) {
  x0 = floatx4{0.f, 0.f, 0.f, 0.f};
  x1 = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 2 * L + 1; ++j) {
    const float* p = xr + (size_t)(L * L + j) * xm;
    const floatx4 a = ld4(p), b = ld4(p + 4);
    const float y = Y[L * L + j];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      x0[q] = fmaf(y, a[q], x0[q]);
      x1[q] = fmaf(y, b[q], x1[q]);
    }
  }
}

template <int kP>
__global__ __launch_bounds__(kGT, 2) void k_qkdot_fwd(e2v2_qkdot_args A, const void* __restrict__ wp,
                                                        const float* __restrict__ bias, float* __restrict__ gate) {
  constexpr int SB = g_stage_bytes(kP, false);
  constexpr int nks = kQK / kGK;
  __shared__ __attribute__((aligned(16))) char lds[2 * SB];
  const int64_t E = A.n_edges;
  const int n_tiles = (int)((E + kGM - 1) / kGM);
  const int tile = xcd_row(blockIdx.x, n_tiles);
  if (tile >= n_tiles) return;
  const int t = threadIdx.x, lane = t & 63, wv = __builtin_amdgcn_readfirstlane(t >> 6), h = lane >> 5;
  const int64_t e0 = (int64_t)tile * kGM;
  const int ra = wv * 32 + (lane & 31);
  const int64_t e = e0 + ra;
  const bool ok = e < qk_e_lim(A);
  const RadialTab R{A.rtab, A.n_types, A.rtab_n, kQK, 1.0f / A.rtab_h, A.pair_slot};
  QkEdge q{};
  float Y[9];
  const float* xr = A.xd;
  if (ok) {
    q = qk_edge(A, R, e);
#pragma unroll
    for (int m = 0; m < 9; ++m) Y[m] = A.Y[e * 9 + m];
    xr = A.xd + (size_t)A.edge_row[e] * kQC;
  } else {
#pragma unroll
    for (int m = 0; m < 9; ++m) Y[m] = 0.f;
  }
  const size_t xm = (size_t)A.n_rows * kQC;
  const float* tb = R.tab + q.toff + 8 * h;
  const __amdgpu_buffer_rsrc_t br = b_rsrc<kP>(wp, 0, 1, 0, nks);
  floatx16 acc[4];
  kloop<kP, false>(lds, SB, nks, lane,
        [&](int ks, int buf) { load_b<kP>(br, ks, lds + buf * SB + a_stage_bytes(false), wv, lane); },
        [&](int ks, int buf, AFrag& f) {
          f.x0 = floatx4{0.f, 0.f, 0.f, 0.f};
          f.x1 = floatx4{0.f, 0.f, 0.f, 0.f};
          if (!ok || ks >= nks) return;
          const int l = ks >> 4;                           // 16 stages per degree
          const int c = ((ks & 15) << 4) + 8 * h;          // this lane's eight channels within the degree
          // rad: rows 0..2 at node n (ta) and n + 1 (ta + 4 rows)
          const float* ta = tb + l * kQC + ((ks & 15) << 4);
          floatx4 r0, r1;
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const float* p = ta + 4 * half;
            const floatx4 f0 = ld4(p), f1 = ld4(p + kQK), f2 = ld4(p + 2 * kQK);
            const floatx4 g0 = ld4(p + 4 * kQK), g1 = ld4(p + 5 * kQK), g2 = ld4(p + 6 * kQK);
            floatx4 v;
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = herm_value(q.H, f0[u], f1[u], f2[u], g0[u], g1[u], g2[u]);
            if (half == 0) r0 = v; else r1 = v;
          }
          floatx4 x0, x1;
          const float* xp = xr + c;
          if (l == 0) qk_x0<0>(xp, xm, Y, x0, x1);
          else if (l == 1) qk_x0<1>(xp, xm, Y, x0, x1);
          else qk_x0<2>(xp, xm, Y, x0, x1);
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            f.x0[u] = x0[u] * r0[u];
            f.x1[u] = x1[u] * r1[u];
          }
        },
        acc);
  const int64_t e_lim = qk_e_lim(A);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int col = 32 * j + (lane & 31);
    const float bv = bias ? bias[col] : 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = e0 + wv * 32 + acc_row(r, lane);
      if (row < E) gate[row * kQH + col] = row < e_lim ? acc[j][r] + bv : 0.f;
    }
  }
}

// Phase 1 of the backward for one edge and degree L: this thread's 64 channels (8 groups of 8) of column tile
// ct.  D holds dA of the edge row; dx0 replaces it.  Returns dL/ddist and dL/dY of the degree's rows.
template <int L>
__device__ __forceinline__ void qk_bwd_edge(const e2v2_qkdot_args& A, const RadialTab& R, const QkEdge& q,
                                            const float (&Y)[9], const float* xr, size_t xm, int cb, int c0,
                                            float* D, float& dd, float (&dY)[5]) {
#pragma unroll 1
  for (int g = 0; g < 8; ++g) {
    const int cc = c0 + 8 * g;                                  // channel within the column tile
    const float* ta = R.tab + q.toff + L * kQC + cb + cc;       // node n row 0
    floatx4* dp = reinterpret_cast<floatx4*>(D + cc);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const float* p = ta + 4 * half;
      const floatx4 f0 = ld4(p), f1 = ld4(p + kQK), f2 = ld4(p + 2 * kQK), f3 = ld4(p + 3 * kQK);
      const floatx4 g0 = ld4(p + 4 * kQK), g1 = ld4(p + 5 * kQK), g2 = ld4(p + 6 * kQK), g3 = ld4(p + 7 * kQK);
      floatx4 xv[2 * L + 1];
#pragma unroll
      for (int j = 0; j < 2 * L + 1; ++j) xv[j] = ld4(xr + (size_t)(L * L + j) * xm + cb + cc + 4 * half);
      const floatx4 da = dp[half];
      floatx4 dx;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float rad = herm_value(q.H, f0[u], f1[u], f2[u], g0[u], g1[u], g2[u]);
        const float rd = herm_value(q.H, f1[u], f2[u], f3[u], g1[u], g2[u], g3[u]) * R.inv_h;
        float x0 = 0.f;
#pragma unroll
        for (int j = 0; j < 2 * L + 1; ++j) x0 = fmaf(Y[L * L + j], xv[j][u], x0);
        dx[u] = da[u] * rad;
        dd = fmaf(da[u] * x0, rd, dd);
#pragma unroll
        for (int j = 0; j < 2 * L + 1; ++j) dY[j] = fmaf(dx[u], xv[j][u], dY[j]);
      }
      dp[half] = dx;
    }
  }
}

// Phase 2 for degree L: sums over the edges of each row of Y_m dx0 for channel cc, m-rows [m0, m1) of L.
template <int L>
__device__ __forceinline__ void qk_bwd_rows(const e2v2_qkdot_args& A, const float* D, const float (*Ys)[9],
                                            const int* rows, int n_valid, int64_t e0, int et, int cb, int cc, int m0,
                                            int m1, float* __restrict__ side, float* __restrict__ dxd) {
  float acc[3] = {0.f, 0.f, 0.f};
  const size_t xm = (size_t)A.n_rows * kQC;
  for (int er = 0; er < n_valid; ++er) {
    const int r = rows[er];
    const float d = D[er * kQDl + cc];
#pragma unroll
    for (int k = 0; k < 3; ++k)
      if (m0 + k < m1) acc[k] = fmaf(Ys[er][L * L + m0 + k], d, acc[k]);
    if (er + 1 == n_valid || rows[er + 1] != r) {
      const bool whole = A.row_ptr[r] >= e0 && A.row_ptr[r + 1] <= e0 + n_valid;
      float* out = whole ? dxd + xm * (size_t)(L * L) + (size_t)r * kQC + cb + cc
                         : side + ((size_t)et * 2 + (r == rows[0] ? 0 : 1)) * kQSide + (size_t)(L * L) * kQC + cb +
                               cc;
      const size_t ms = whole ? xm : (size_t)kQC;
#pragma unroll
      for (int k = 0; k < 3; ++k)
        if (m0 + k < m1) {
          out[(size_t)(m0 + k) * ms] = acc[k];
          acc[k] = 0.f;
        }
    }
  }
}

template <int kP>
__global__ __launch_bounds__(kGT, 2) void k_qkdot_bwd(e2v2_qkdot_args A, const void* __restrict__ wtp,
                                                        const float* __restrict__ dgate, float* __restrict__ part,
                                                        float* __restrict__ side, float* __restrict__ dxd) {
  constexpr int SB = g_stage_bytes(kP, false);
  constexpr int nks = kQH / kGK;
  constexpr int kLds = 2 * SB > kGM * kQDl * 4 ? 2 * SB : kGM * kQDl * 4;
  __shared__ __attribute__((aligned(16))) char lds[kLds];
  __shared__ float Ys[kGM][9];
  __shared__ int rows[kGM];
  const int64_t E = A.n_edges;
  const int n_et = (int)((E + kGM - 1) / kGM);
  const int tile = xcd_row(blockIdx.x, n_et * kQCt);
  if (tile >= n_et * kQCt) return;
  const int et = tile / kQCt, ct = tile % kQCt;
  const int t = threadIdx.x, lane = t & 63, wv = __builtin_amdgcn_readfirstlane(t >> 6), h = lane >> 5;
  const int64_t e0 = (int64_t)et * kGM;
  // dA = dgate W for 128 edges x 128 channels (rows past E read as zero through the buffer bound)
  const int64_t tile_rows = E - e0 < kGM ? E - e0 : kGM;
  const __amdgpu_buffer_rsrc_t arr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(dgate + e0 * kQH), (short)0, (int)((uint32_t)tile_rows * kQH * 4u), 0x00020000);
  uint32_t a_voff[kGAi / 4];
  a_offsets(wv, lane, kQH, a_voff);
  const __amdgpu_buffer_rsrc_t br = b_rsrc<kP>(wtp, 0, kQCt, ct, nks);
  const int ra = wv * 32 + (lane & 31);
  floatx16 acc[4];
  kloop<kP, false>(lds, SB, nks, lane,
        [&](int ks, int buf) {
          load_a(arr, a_voff, (uint32_t)(ks * kGK) * 4u, lds + buf * SB, wv);
          load_b<kP>(br, ks, lds + buf * SB + a_stage_bytes(false), wv, lane);
        },
        [&](int ks, int buf, AFrag& f) {
          const floatx4* As = reinterpret_cast<const floatx4*>(lds + buf * SB);
          f.x0 = As[a_slot(ra, 2 * h)];
          f.x1 = As[a_slot(ra, 2 * h + 1)];
        },
        acc);
  __syncthreads();   // every wavefront is past its last read of the stage buffers
  float* D = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) D[(wv * 32 + acc_row(r, lane)) * kQDl + 32 * j + (lane & 31)] = acc[j][r];
  __syncthreads();

  // phase 1: thread pair (2 er, 2 er + 1) on edge e0 + er, 64 channels each
  const int64_t e_lim = qk_e_lim(A);
  const int l = ct >> 1, cb = (ct & 1) * kGN;
  const RadialTab R{A.rtab, A.n_types, A.rtab_n, kQK, 1.0f / A.rtab_h, A.pair_slot};
  const size_t xm = (size_t)A.n_rows * kQC;
  {
    const int er = t >> 1, hf = t & 1;
    const int64_t e = e0 + er;
    float dd = 0.f, dY[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
    if (e < e_lim) {
      const QkEdge q = qk_edge(A, R, e);
      float Y[9];
#pragma unroll
      for (int m = 0; m < 9; ++m) Y[m] = A.Y[e * 9 + m];
      const int i = A.edge_row[e];
      if (hf == 0) {
        rows[er] = i;
#pragma unroll
        for (int m = 0; m < 9; ++m) Ys[er][m] = Y[m];
      }
      const float* xr = A.xd + (size_t)i * kQC;
      float* Dr = D + er * kQDl;
      if (l == 0) qk_bwd_edge<0>(A, R, q, Y, xr, xm, cb, 64 * hf, Dr, dd, dY);
      else if (l == 1) qk_bwd_edge<1>(A, R, q, Y, xr, xm, cb, 64 * hf, Dr, dd, dY);
      else qk_bwd_edge<2>(A, R, q, Y, xr, xm, cb, 64 * hf, Dr, dd, dY);
    } else if (hf == 0) {
      rows[er] = -1;
    }
    dd += __shfl_xor(dd, 1, 64);
#pragma unroll
    for (int j = 0; j < 5; ++j) dY[j] += __shfl_xor(dY[j], 1, 64);
    if (hf == 0 && e < E) {
      float* pp = part + ((size_t)ct * E + e) * kQPart;
      pp[0] = dd;
#pragma unroll
      for (int j = 0; j < 5; ++j) pp[1 + j] = dY[j];
    }
  }
  __syncthreads();

  // phase 2: channel cc of the column tile, m-rows of the degree split between the two thread halves
  const int64_t nv = e_lim - e0;
  const int n_valid = nv <= 0 ? 0 : (nv < kGM ? (int)nv : kGM);
  const int cc = t & (kGN - 1), grp = t >> 7;
  const int M = 2 * l + 1, mh = (M + 1) / 2;
  const int m0 = grp ? mh : 0, m1 = grp ? M : mh;
  if (m0 < m1 && n_valid > 0) {
    if (l == 0) qk_bwd_rows<0>(A, D, Ys, rows, n_valid, e0, et, cb, cc, m0, m1, side, dxd);
    else if (l == 1) qk_bwd_rows<1>(A, D, Ys, rows, n_valid, e0, et, cb, cc, m0, m1, side, dxd);
    else qk_bwd_rows<2>(A, D, Ys, rows, n_valid, e0, et, cb, cc, m0, m1, side, dxd);
  }
}

// Rows of dL/dxd that the tiles did not write: atoms without edges get zeros, rows that cross a tile boundary
// the sum of their tiles' partials in tile order.  One workgroup per row.
__global__ __launch_bounds__(256) void k_qkdot_rows(e2v2_qkdot_args A, const float* __restrict__ side,
                                                      float* __restrict__ dxd) {
  const int r = blockIdx.x;
  if (r >= A.n_rows) return;
  const int64_t b = A.row_ptr[r], en = A.row_ptr[r + 1];
  const size_t xm = (size_t)A.n_rows * kQC;
  if (en <= b) {
    for (int k = threadIdx.x; k < kQSide; k += 256) dxd[(size_t)(k / kQC) * xm + (size_t)r * kQC + k % kQC] = 0.f;
    return;
  }
  const int64_t ta = b / kGM, tb = (en - 1) / kGM;
  if (ta == tb) return;
  for (int k = threadIdx.x; k < kQSide; k += 256) {
    float s = 0.f;
    for (int64_t tt = ta; tt <= tb; ++tt) {
      const int sd = A.edge_row[tt * kGM] == r ? 0 : 1;
      s += side[((size_t)tt * 2 + sd) * kQSide + k];
    }
    dxd[(size_t)(k / kQC) * xm + (size_t)r * kQC + k % kQC] = s;
  }
}

// dL/ddist and dL/dY of every edge from the column tiles' partials (tiles 2l, 2l + 1 hold degree l).
__global__ __launch_bounds__(256) void k_qkdot_edges(e2v2_qkdot_args A, const float* __restrict__ part,
                                                       float* __restrict__ dY, float* __restrict__ ddist) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t E = A.n_edges;
  if (e >= E) return;
  const size_t cs = (size_t)E * kQPart;
  const float* p = part + (size_t)e * kQPart;
  float dd = 0.f;
#pragma unroll
  for (int c = 0; c < kQCt; ++c) dd += p[c * cs];
  ddist[e] = dd;
#pragma unroll
  for (int l = 0; l < 3; ++l)
#pragma unroll
    for (int j = 0; j < 2 * l + 1; ++j) dY[e * 9 + l * l + j] = p[(2 * l) * cs + 1 + j] + p[(2 * l + 1) * cs + 1 + j];
}

int check_qkdot(const e2v2_qkdot_args& A, const char* who) {
  E2V2_REQUIRE(A.n_rows >= 0 && A.n_edges >= 0, "%s: negative sizes", who);
  E2V2_REQUIRE(A.pieces == 1 || A.pieces == 3, "%s: %d pieces (1 or 3)", who, A.pieces);
  E2V2_REQUIRE(A.rtab && A.atom_type && A.n_types >= 1 && A.n_types <= E2V2_MAX_TYPES && A.rtab_n >= 2 &&
                   A.rtab_h > 0.f,
               "%s: needs the rad_func_m0 table and atom types (n_types %d, rtab_n %d)", who, A.n_types, A.rtab_n);
  E2V2_REQUIRE(A.row_ptr && A.edge_row && A.col && A.dist && A.Y && A.xd, "%s: null edge or node operand", who);
  E2V2_REQUIRE((((uintptr_t)A.xd | (uintptr_t)A.rtab) & 15) == 0, "%s: xd and the table must be 16-byte aligned",
               who);
  E2V2_REQUIRE(A.n_edges < (int64_t)1 << 31 && (uint64_t)kGM * kQH * 4u < (1ull << 31),
               "%s: %lld edges exceed the tile indexing", who, (long long)A.n_edges);
  return 0;
}
}  // namespace
}  // namespace e2v2

using namespace e2v2;

E2V2_API int e2v2_qkdot_gate_fwd(const e2v2_qkdot_args* args, const void* w_packed, const float* bias, float* gate,
                                 hipStream_t s) {
  E2V2_REQUIRE(args && w_packed && gate, "qkdot_gate_fwd: null argument");
  const e2v2_qkdot_args& A = *args;
  if (int rc = check_qkdot(A, "qkdot_gate_fwd")) return rc;
  if (A.n_edges == 0) return 0;
  const int n_tiles = (int)((A.n_edges + kGM - 1) / kGM);
  const dim3 grid(xcd_grid(n_tiles));
  if (A.pieces == 3)
    hipLaunchKernelGGL((k_qkdot_fwd<3>), grid, dim3(kGT), 0, s, A, w_packed, bias, gate);
  else
    hipLaunchKernelGGL((k_qkdot_fwd<1>), grid, dim3(kGT), 0, s, A, w_packed, bias, gate);
  E2V2_LAUNCHED("k_qkdot_fwd");
  return 0;
}

static size_t qkdot_part_floats(int64_t E) { return (size_t)kQCt * E * kQPart; }
static size_t qkdot_side_floats(int64_t E) { return (size_t)((E + kGM - 1) / kGM) * 2 * kQSide; }

E2V2_API size_t e2v2_qkdot_gate_bwd_workspace(int64_t n_edges) {
  return n_edges > 0 ? (qkdot_part_floats(n_edges) + qkdot_side_floats(n_edges)) * sizeof(float) : 0;
}

E2V2_API int e2v2_qkdot_gate_bwd(const e2v2_qkdot_args* args, const void* wt_packed, const float* dgate, float* dY,
                                 float* ddist, float* dxd, void* workspace, size_t workspace_bytes, hipStream_t s) {
  E2V2_REQUIRE(args && wt_packed && dgate && dY && ddist && dxd, "qkdot_gate_bwd: null argument");
  const e2v2_qkdot_args& A = *args;
  if (int rc = check_qkdot(A, "qkdot_gate_bwd")) return rc;
  E2V2_REQUIRE(((uintptr_t)dgate & 15) == 0, "qkdot_gate_bwd: dgate must be 16-byte aligned");
  const size_t need = e2v2_qkdot_gate_bwd_workspace(A.n_edges);
  E2V2_REQUIRE(workspace_bytes >= need && (need == 0 || workspace) && ((uintptr_t)workspace & 15) == 0,
               "qkdot_gate_bwd: workspace of %zu bytes (16-byte aligned) needed, got %zu", need, workspace_bytes);
  if (A.n_rows == 0) return 0;
  float* part = static_cast<float*>(workspace);
  float* side = part + qkdot_part_floats(A.n_edges);
  if (A.n_edges > 0) {
    const int n_et = (int)((A.n_edges + kGM - 1) / kGM);
    const dim3 grid(xcd_grid(n_et * kQCt));
    if (A.pieces == 3)
      hipLaunchKernelGGL((k_qkdot_bwd<3>), grid, dim3(kGT), 0, s, A, wt_packed, dgate, part, side, dxd);
    else
      hipLaunchKernelGGL((k_qkdot_bwd<1>), grid, dim3(kGT), 0, s, A, wt_packed, dgate, part, side, dxd);
    E2V2_LAUNCHED("k_qkdot_bwd");
  }
  hipLaunchKernelGGL(k_qkdot_rows, dim3((unsigned)A.n_rows), dim3(256), 0, s, A, side, dxd);
  E2V2_LAUNCHED("k_qkdot_rows");
  if (A.n_edges > 0) {
    hipLaunchKernelGGL(k_qkdot_edges, dim3((unsigned)((A.n_edges + 255) / 256)), dim3(256), 0, s, A, part, dY, ddist);
    E2V2_LAUNCHED("k_qkdot_edges");
  }
  return 0;
}
