// The gate of tp_type QKdot_alpha (src/molfm/models/e2former/e2former.py:270-283):
//   x0_l = sum_{m in l} Y_m(edge) dot_linear(x)[query, m]        (e3nn spherical harmonics, normalize=True)
//   gate = fc_m0(cat_l(x0_l) * rad_func_m0(x_edge))               (768 -> 128)
// as one GEMM per direction whose edge-side operand is never stored.
//
// Forward (k_qkdot_fwd): gate = A W^T + b on the split GEMM of gemm_core.h (128 edges x 128 heads per
// workgroup, K = 768 in 48 stages of 16).  A is built in LDS 32 channels at a time (double-buffered, one
// chunk ahead of the MFMAs): rad from the six table rows of each edge's distance interval (quintic
// Hermite; the table node and Hermite weights formed once per edge) and x0 from the 2l + 1 rows of xd of
// the query atom, eight lanes per edge so that every load reads whole 128-byte runs; the K loop then
// splits each lane's fragment into the bf16 pieces as in gemm_core.h.
//
// Backward (k_qkdot_bwd): per (128-edge tile, 128-channel column tile) the GEMM dA = dgate W (K = 128)
// lands in registers and, one 64-channel half at a time, in LDS; groups of 16 lanes then walk the tile edge
// by edge (rad, its distance derivative and x0 recomputed as in the forward) and form dx0 = dA rad (written
// back in place of dA), the edge's
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

// Edge setup of a 128-edge tile in LDS (thread t < 128 for edge e0 + t): table node offset, Hermite
// weights, Y and the query row (-1 past the valid edges).
struct QkTileEdges {
  int64_t toff[kGM];
  float H[kGM][6];
  float Y[kGM][9];
  int row[kGM];
};

__device__ __forceinline__ void qk_tile_setup(const e2v2_qkdot_args& A, const RadialTab& R, int64_t e0,
                                              int64_t e_lim, int t, QkTileEdges& S) {
  if (t >= kGM) return;
  const int64_t e = e0 + t;
  if (e < e_lim) {
    const QkEdge q = qk_edge(A, R, e);
    S.toff[t] = q.toff;
    S.H[t][0] = q.H.a0; S.H[t][1] = q.H.a1; S.H[t][2] = q.H.a2;
    S.H[t][3] = q.H.b0; S.H[t][4] = q.H.b1; S.H[t][5] = q.H.b2;
#pragma unroll
    for (int m = 0; m < 9; ++m) S.Y[t][m] = A.Y[e * 9 + m];
    S.row[t] = A.edge_row[e];
  } else {
    S.row[t] = -1;
  }
}

__device__ __forceinline__ Hermite5 qk_h(const QkTileEdges& S, int er) {
  Hermite5 H;
  H.a0 = S.H[er][0]; H.a1 = S.H[er][1]; H.a2 = S.H[er][2];
  H.b0 = S.H[er][3]; H.b1 = S.H[er][4]; H.b2 = S.H[er][5];
  return H;
}

// Forward A values of edge er, channels k .. k + 3 (k = 256 L + c within the 768): x0 of degree L times rad.
template <int L>
__device__ __forceinline__ floatx4 qk_a4(const RadialTab& R, const QkTileEdges& S, const float* xd, size_t xm,
                                         int er, int k) {
  const int c = k - L * kQC;
  const float* p = R.tab + S.toff[er] + k;
  const floatx4 f0 = ld4(p), f1 = ld4(p + kQK), f2 = ld4(p + 2 * kQK);
  const floatx4 g0 = ld4(p + 4 * kQK), g1 = ld4(p + 5 * kQK), g2 = ld4(p + 6 * kQK);
  const float* xr = xd + (size_t)S.row[er] * kQC + c;
  floatx4 xv[2 * L + 1];
#pragma unroll
  for (int j = 0; j < 2 * L + 1; ++j) xv[j] = ld4(xr + (size_t)(L * L + j) * xm);
  const Hermite5 H = qk_h(S, er);
  floatx4 a;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    float x0 = 0.f;
#pragma unroll
    for (int j = 0; j < 2 * L + 1; ++j) x0 = fmaf(S.Y[er][L * L + j], xv[j][u], x0);
    a[u] = x0 * herm_value(H, f0[u], f1[u], f2[u], g0[u], g1[u], g2[u]);
  }
  return a;
}

// The forward's A operand is built in LDS 32 channels (two stages) at a time, double-buffered: eight lanes per
// edge row (lane j: channels 4 j .. 4 j + 3), so that every load instruction reads whole 128-byte runs of the
// table and xd rows; granules are stored in the A slot order of the K loop (a_slot).
constexpr int kQCh = 32;                                    // channels per A chunk
constexpr int kQChG = kGM * kQCh / 4;                       // granules per chunk: 1024 (16 KB)

template <int kP>
__global__ __launch_bounds__(kGT, 2) void k_qkdot_fwd(e2v2_qkdot_args A, const void* __restrict__ wp,
                                                        const float* __restrict__ bias, float* __restrict__ gate) {
  constexpr int BS = 16 * kP * kGBg;                        // one B stage: kP pieces of 4 KB
  constexpr int nks = kQK / kGK;                            // 48
  __shared__ __attribute__((aligned(16))) char bl[2 * BS];
  __shared__ floatx4 Ac[2][kQChG];
  __shared__ QkTileEdges S;
  const int64_t E = A.n_edges;
  const int n_tiles = (int)((E + kGM - 1) / kGM);
  const int tile = xcd_row(blockIdx.x, n_tiles);
  if (tile >= n_tiles) return;
  const int t = threadIdx.x, lane = t & 63, wv = __builtin_amdgcn_readfirstlane(t >> 6), h = lane >> 5;
  const int64_t e0 = (int64_t)tile * kGM;
  const int64_t e_lim = qk_e_lim(A);
  const RadialTab R{A.rtab, A.n_types, A.rtab_n, kQK, 1.0f / A.rtab_h, A.pair_slot};
  const size_t xm = (size_t)A.n_rows * kQC;
  const __amdgpu_buffer_rsrc_t br = b_rsrc<kP>(wp, 0, 1, 0, nks);
  qk_tile_setup(A, R, e0, e_lim, t, S);
  // chunk c (stages 2c, 2c + 1) into buffer b
  auto build = [&](int c, int b) {
    const int j = t & 7, k = c * kQCh + 4 * j, L = k / kQC;
#pragma unroll 2
    for (int pass = 0; pass < kGM / 32; ++pass) {
      const int er = (t >> 3) + 32 * pass;
      floatx4 a = {0.f, 0.f, 0.f, 0.f};
      if (S.row[er] >= 0) {
        if (L == 0) a = qk_a4<0>(R, S, A.xd, xm, er, k);
        else if (L == 1) a = qk_a4<1>(R, S, A.xd, xm, er, k);
        else a = qk_a4<2>(R, S, A.xd, xm, er, k);
      }
      Ac[b][(j >> 2) * kGAg + a_slot(er, j & 3)] = a;     // stage j / 4 of the chunk, granule j % 4 of the row
    }
  };
  const int ra = wv * 32 + (lane & 31);
  auto read_a = [&](int ks, AFrag& f) {
    const floatx4* As = Ac[(ks >> 1) & 1] + (ks & 1) * kGAg;
    f.x0 = As[a_slot(ra, 2 * h)];
    f.x1 = As[a_slot(ra, 2 * h + 1)];
  };
  floatx16 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
  __syncthreads();                                          // the tile setup
  load_b<kP>(br, 0, bl, wv, lane);
  load_b<kP>(br, 1, bl + BS, wv, lane);
  build(0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  bf16x8 a_cur[kP];
  {
    AFrag f;
    read_a(0, f);
    split_pieces<kP>(f.x0, f.x1, a_cur);
  }
  for (int ks = 0; ks < nks; ++ks) {
    const bf16x8* Bs = reinterpret_cast<const bf16x8*>(bl + (ks & 1) * BS);
    bf16x8 b[kP][4];
#pragma unroll
    for (int p = 0; p < kP; ++p)
#pragma unroll
      for (int j = 0; j < 4; ++j) b[p][j] = Bs[p * kGBg + b_slot(32 * j + (lane & 31), h)];
    if (ks + 1 < nks) {
      __builtin_amdgcn_s_waitcnt(0);    // stage ks + 1 landed; this wavefront's reads of B buffer ks & 1 are done
      __syncthreads();
      if (ks + 2 < nks) load_b<kP>(br, ks + 2, bl + (ks & 1) * BS, wv, lane);
      // chunk (ks + 2) / 2 into the buffer of chunk ks / 2 - 1, whose last reader ran before this barrier; the
      // next iteration's barrier orders these writes before the first read (stage ks + 2)
      if ((ks & 1) == 0 && ks + 2 < nks) build((ks + 2) >> 1, ((ks + 2) >> 1) & 1);
    }
    AFrag f;
    if (ks + 1 < nks) read_a(ks + 1, f);
    if constexpr (kP == 3) {
      constexpr int kPa[6] = {0, 1, 2, 0, 1, 0}, kPb[6] = {0, 0, 0, 1, 1, 2};
#pragma unroll
      for (int q = 0; q < 6; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_cur[kPa[q]], b[kPb[q]][j], acc[j], 0, 0, 0);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_cur[0], b[0][j], acc[j], 0, 0, 0);
    }
    if (ks + 1 < nks) split_pieces<kP>(f.x0, f.x1, a_cur);
  }
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

// Phase 1 of the backward for one edge and degree L, one lane of the edge's 16: channels c .. c + 3 of the
// degree (each load instruction reads 256 contiguous bytes of a row per 16 lanes).  D points at the edge's
// dA values of those channels; dx0 replaces them.  Adds this lane's share of dL/ddist and dL/dY.
template <int L>
__device__ __forceinline__ void qk_bwd_edge(const RadialTab& R, int64_t toff, const Hermite5& H,
                                            const float (&Y)[9], const float* xr, size_t xm, int c, float* D,
                                            float& dd, float (&dY)[5]) {
  const float* p = R.tab + toff + L * kQC + c;                  // node n row 0
  const floatx4 f0 = ld4(p), f1 = ld4(p + kQK), f2 = ld4(p + 2 * kQK), f3 = ld4(p + 3 * kQK);
  const floatx4 g0 = ld4(p + 4 * kQK), g1 = ld4(p + 5 * kQK), g2 = ld4(p + 6 * kQK), g3 = ld4(p + 7 * kQK);
  floatx4 xv[2 * L + 1];
#pragma unroll
  for (int k = 0; k < 2 * L + 1; ++k) xv[k] = ld4(xr + (size_t)(L * L + k) * xm + c);
  floatx4* dp = reinterpret_cast<floatx4*>(D);
  const floatx4 da = *dp;
  floatx4 dx;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const float rad = herm_value(H, f0[u], f1[u], f2[u], g0[u], g1[u], g2[u]);
    const float rd = herm_value(H, f1[u], f2[u], f3[u], g1[u], g2[u], g3[u]) * R.inv_h;
    float x0 = 0.f;
#pragma unroll
    for (int k = 0; k < 2 * L + 1; ++k) x0 = fmaf(Y[L * L + k], xv[k][u], x0);
    dx[u] = da[u] * rad;
    dd = fmaf(da[u] * x0, rd, dd);
#pragma unroll
    for (int k = 0; k < 2 * L + 1; ++k) dY[k] = fmaf(dx[u], xv[k][u], dY[k]);
  }
  *dp = dx;
}

constexpr int kQDh = 64 + 4;        // row stride (floats) of a 64-channel half of the dA tile in LDS

// Phase 2 for degree L: sums over the edges of each row of Y_m dx0 for channel cd of the LDS half tile
// (degree channel c), m-rows mg and mg + 4 of L's 2 L + 1.
template <int L>
__device__ __forceinline__ void qk_bwd_rows(const e2v2_qkdot_args& A, const float* D, const float (*Ys)[9],
                                            const int* rows, int n_valid, int64_t e0, int et, int cd, int c, int mg,
                                            float* __restrict__ side, float* __restrict__ dxd) {
  constexpr int M = 2 * L + 1;
  float acc[2] = {0.f, 0.f};
  const size_t xm = (size_t)A.n_rows * kQC;
  for (int er = 0; er < n_valid; ++er) {
    const int r = rows[er];
    const float d = D[er * kQDh + cd];
#pragma unroll
    for (int k = 0; k < 2; ++k)
      if (mg + 4 * k < M) acc[k] = fmaf(Ys[er][L * L + mg + 4 * k], d, acc[k]);
    if (er + 1 == n_valid || rows[er + 1] != r) {
      const bool whole = A.row_ptr[r] >= e0 && A.row_ptr[r + 1] <= e0 + n_valid;
      float* out = whole ? dxd + xm * (size_t)(L * L) + (size_t)r * kQC + c
                         : side + ((size_t)et * 2 + (r == rows[0] ? 0 : 1)) * kQSide + (size_t)(L * L) * kQC + c;
      const size_t ms = whole ? xm : (size_t)kQC;
#pragma unroll
      for (int k = 0; k < 2; ++k)
        if (mg + 4 * k < M) {
          out[(size_t)(mg + 4 * k) * ms] = acc[k];
          acc[k] = 0.f;
        }
    }
  }
}

template <int kP>
__global__ __launch_bounds__(kGT, 3) void k_qkdot_bwd(e2v2_qkdot_args A, const void* __restrict__ wtp,
                                                        const float* __restrict__ dgate, float* __restrict__ part,
                                                        float* __restrict__ side, float* __restrict__ dxd) {
  constexpr int SB = g_stage_bytes(kP, false);
  constexpr int nks = kQH / kGK;
  // the stage buffers of the GEMM, then (reused) one 64-channel half of the dA tile
  constexpr int kLds = 2 * SB > kGM * kQDh * 4 ? 2 * SB : kGM * kQDh * 4;
  __shared__ __attribute__((aligned(16))) char lds[kLds];
  __shared__ float Ys[kGM][9];
  __shared__ float Hs[kGM][6];
  __shared__ int64_t Ts[kGM];
  __shared__ int rows[kGM];
  __shared__ float Pl[kGM][kQPart];   // the first half's per-edge partials
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

  // edge setup, once per edge in LDS
  const int64_t e_lim = qk_e_lim(A);
  const int l = ct >> 1, cb = (ct & 1) * kGN;
  const RadialTab R{A.rtab, A.n_types, A.rtab_n, kQK, 1.0f / A.rtab_h, A.pair_slot};
  const size_t xm = (size_t)A.n_rows * kQC;
  if (t < kGM) {
    const int64_t e = e0 + t;
    if (e < e_lim) {
      const QkEdge q = qk_edge(A, R, e);
      Ts[t] = q.toff;
      Hs[t][0] = q.H.a0; Hs[t][1] = q.H.a1; Hs[t][2] = q.H.a2;
      Hs[t][3] = q.H.b0; Hs[t][4] = q.H.b1; Hs[t][5] = q.H.b2;
#pragma unroll
      for (int m = 0; m < 9; ++m) Ys[t][m] = A.Y[e * 9 + m];
      rows[t] = A.edge_row[e];
    } else {
      rows[t] = -1;
    }
  }
  const int64_t nv = e_lim - e0;
  const int n_valid = nv <= 0 ? 0 : (nv < kGM ? (int)nv : kGM);
  float* D = reinterpret_cast<float*>(lds);
  // the tile's two 64-channel halves in turn (accumulator tiles j = 2 hf, 2 hf + 1)
  auto run_half = [&](auto hfc) {
    constexpr int hf = decltype(hfc)::value;
    __syncthreads();   // the stage buffers (hf 0) or the previous half (hf 1) are no longer read
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        D[(wv * 32 + acc_row(r, lane)) * kQDh + 32 * jj + (lane & 31)] = acc[2 * hf + jj][r];
    __syncthreads();
    const int ch = cb + 64 * hf;                 // first channel of the half within the degree
    // phase 1: the tile's edges in turn, 16 lanes per edge, four channels per lane
    const int j = t & 15;
#pragma unroll 1
    for (int er = t >> 4; er < kGM; er += kGT / 16) {
      const int64_t e = e0 + er;
      float dd = 0.f, dY[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
      if (e < e_lim) {
        Hermite5 H;
        H.a0 = Hs[er][0]; H.a1 = Hs[er][1]; H.a2 = Hs[er][2];
        H.b0 = Hs[er][3]; H.b1 = Hs[er][4]; H.b2 = Hs[er][5];
        float Y[9];
#pragma unroll
        for (int m = 0; m < 9; ++m) Y[m] = Ys[er][m];
        const float* xr = A.xd + (size_t)rows[er] * kQC;
        float* Dr = D + er * kQDh + 4 * j;
        if (l == 0) qk_bwd_edge<0>(R, Ts[er], H, Y, xr, xm, ch + 4 * j, Dr, dd, dY);
        else if (l == 1) qk_bwd_edge<1>(R, Ts[er], H, Y, xr, xm, ch + 4 * j, Dr, dd, dY);
        else qk_bwd_edge<2>(R, Ts[er], H, Y, xr, xm, ch + 4 * j, Dr, dd, dY);
      }
      // sums over the edge's 16 lanes (a fixed butterfly order)
#pragma unroll
      for (int o = 8; o >= 1; o >>= 1) {
        dd += __shfl_xor(dd, o, 64);
#pragma unroll
        for (int k = 0; k < 5; ++k) dY[k] += __shfl_xor(dY[k], o, 64);
      }
      if (j == 0) {
        if constexpr (hf == 0) {
          Pl[er][0] = dd;
#pragma unroll
          for (int k = 0; k < 5; ++k) Pl[er][1 + k] = dY[k];
        } else if (e < E) {
          float* pp = part + ((size_t)ct * E + e) * kQPart;
          pp[0] = Pl[er][0] + dd;
#pragma unroll
          for (int k = 0; k < 5; ++k) pp[1 + k] = Pl[er][1 + k] + dY[k];
        }
      }
    }
    __syncthreads();
    // phase 2: channel cd of the half, m-rows mg and mg + 4 of the degree
    const int cd = t & 63, mg = t >> 6;
    if (mg < 2 * l + 1 && n_valid > 0) {
      if (l == 0) qk_bwd_rows<0>(A, D, Ys, rows, n_valid, e0, et, cd, ch + cd, mg, side, dxd);
      else if (l == 1) qk_bwd_rows<1>(A, D, Ys, rows, n_valid, e0, et, cd, ch + cd, mg, side, dxd);
      else qk_bwd_rows<2>(A, D, Ys, rows, n_valid, e0, et, cd, ch + cd, mg, side, dxd);
    }
  };
  run_half(std::integral_constant<int, 0>{});
  run_half(std::integral_constant<int, 1>{});
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
