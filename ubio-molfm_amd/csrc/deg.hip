// Edge-degree embedding (src/molfm/models/e2former/e2former.py:689-753) and
// the edge -> position gradient assembly.
//
// Forward:
//   x0[i, m, c] = (1/avg) sum_e Y_m(dvec_e / |dvec_e|) * fea_l(m)(d_e)[c] * p(d_e)
// with Y the e3nn raw real spherical harmonics of degree <= 2 (unit norm per
// l block) and fea_l the three radial profiles (gbf_projs, l = 0, 1, 2) of
// (d_e, z_i, z_j), interpolated from their distance table (radial.h).
// Backward: dL/ddvec and dL/dd per edge, dL/dd including the profiles'
// distance derivative from the same table; nothing per edge is stored.
#include <algorithm>
#include <type_traits>
#include "common.h"
#include "radial.h"
#include "../../include/e2v2.h"

namespace e2v2 {

constexpr int kDC = 256;
constexpr int kDegC = 3 * kDC;   // channels per table row: profiles l = 0, 1, 2
constexpr int kDH = 128, kDHs = kDH + 16;   // hidden channels; row of hs: the hidden sums, the bias column, zeros

// dY/du for u = (x, y, z) given dL/dY -> dL/du
__device__ __forceinline__ void raw_sh2_bwd(float x, float y, float z, const float (&g)[9], float& gx, float& gy,
                                            float& gz) {
  const float s3 = 1.7320508075688772f;
  gx = g[1] + s3 * z * g[4] + s3 * y * g[5] - x * g[6] - s3 * x * g[8];
  gy = g[2] + s3 * x * g[5] + 2.f * y * g[6] + s3 * z * g[7];
  gz = g[3] + s3 * x * g[4] - z * g[6] + s3 * y * g[7] + s3 * z * g[8];
}

__device__ __forceinline__ int l_of(int m) { return m == 0 ? 0 : (m < 4 ? 1 : 2); }

template <bool kHid = false>
__device__ __forceinline__ RadialTab make_deg_tab(const e2v2_deg_args& A) {
  RadialTab R;
  R.tab = A.rtab; R.n_types = A.n_types; R.n_nodes = A.rtab_n; R.nc = kHid ? 3 * kDH : kDegC;
  R.inv_h = 1.0f / A.rtab_h;
  R.pair_slot = A.pair_slot;
  return R;
}

// Channel slices: slice s = 32 channels 32 s .. 32 s + 31 of every profile.  The
// kernels run one wavefront per (query row, slice), slice = blockIdx % 8, so
// XCD s (workgroups are dispatched round-robin over the 8 XCDs) keeps slice s of
// the table (96 channels per row: profiles l = 0, 1, 2) in its L2.  The table is
// stored slice-major, [pairs][8][nodes][4][96], column 32 l + u holding channel
// 32 s + u of profile l.  Lane (sub, q) = (lane / 8, lane % 8) owns channels
// 32 s + 4 q .. + 3 (16-byte table loads) and the row's edges sub, sub + 8, ...
// The hidden-channel table (kHid: the profiles' 128 hidden channels) has four
// slices of 32 channels per profile ([pairs][4][nodes][4][96]), slice s on the
// XCDs s and s + 4, the same lane mapping.
constexpr int kDSl = 8, kDSlC = kDC / kDSl;
template <bool kHid>
struct DegSl {
  static constexpr int NS = kHid ? 4 : kDSl;             // slices
  static constexpr int W = kDSlC;                         // channels of one profile per slice
  static constexpr int Row = 3 * W, Node = 4 * Row;      // floats per table row / node of a slice
  static constexpr int Q = W / 4, Sub = kWave / Q;       // lanes per edge, edges in flight per wavefront
};

// Four consecutive channels of one profile from rows r0 .. r0 + 2 at both nodes
// (p: the profile's columns of the lower node): the quintic Hermite interpolant.
template <int kRow>
__device__ __forceinline__ floatx4 deg_interp(const float* p, const Hermite5& H, int r0) {
  constexpr int kNode = 4 * kRow;
  const floatx4 f0 = *reinterpret_cast<const floatx4*>(p + r0 * kRow);
  const floatx4 f1 = *reinterpret_cast<const floatx4*>(p + (r0 + 1) * kRow);
  const floatx4 f2 = *reinterpret_cast<const floatx4*>(p + (r0 + 2) * kRow);
  const floatx4 g0 = *reinterpret_cast<const floatx4*>(p + kNode + r0 * kRow);
  const floatx4 g1 = *reinterpret_cast<const floatx4*>(p + kNode + (r0 + 1) * kRow);
  const floatx4 g2 = *reinterpret_cast<const floatx4*>(p + kNode + (r0 + 2) * kRow);
  floatx4 v;
#pragma unroll
  for (int u = 0; u < 4; ++u) v[u] = herm_value(H, f0[u], f1[u], f2[u], g0[u], g1[u], g2[u]);
  return v;
}

// Per-edge terms of a chunk of up to 64 edges, formed by thread-per-edge into LDS.
struct DegChunk {
  float Y[9][64];        // raw SH of the unit vector
  float u[3][64];        // unit vector
  float nrm[64];         // max(d, 1e-12)
  float p[64], dp[64];   // envelope and its derivative
  int64_t toff[64];      // slice-s table offset of the lower node
  float hw[6][64];       // quintic Hermite weights of the fraction in the node interval
};

template <int kRow, int kNS = kDSl>
__device__ __forceinline__ void deg_chunk(const e2v2_deg_args& A, const Envelope& env, const RadialTab& R, int ti,
                                          int s, int64_t e0, int nc, DegChunk& C) {
  const int t = threadIdx.x;
  if (t < nc) {
    const int64_t e = e0 + t;
    const float d = A.dist[e];
    const float nrm = fmaxf(d, 1e-12f);
    const float ux = A.dvec[3 * e] / nrm, uy = A.dvec[3 * e + 1] / nrm, uz = A.dvec[3 * e + 2] / nrm;
    float Y[9];
    raw_sh2(ux, uy, uz, Y);
#pragma unroll
    for (int m = 0; m < 9; ++m) C.Y[m][t] = Y[m];
    C.u[0][t] = ux; C.u[1][t] = uy; C.u[2][t] = uz;
    C.nrm[t] = nrm;
    float p, dp;
    env.eval(d, p, dp);
    C.p[t] = p; C.dp[t] = dp;
    float tt;
    C.toff[t] = radial_node_sliced(R, tab_pair(R, ti, A.atom_type[A.col[e]]), s, kNS, kRow, d, tt);
    const Hermite5 H = hermite5(tt);
    C.hw[0][t] = H.a0; C.hw[1][t] = H.a1; C.hw[2][t] = H.a2;
    C.hw[3][t] = H.b0; C.hw[4][t] = H.b1; C.hw[5][t] = H.b2;
  }
}

__device__ __forceinline__ Hermite5 chunk_hermite(const DegChunk& C, int el) {
  Hermite5 H;
  H.a0 = C.hw[0][el]; H.a1 = C.hw[1][el]; H.a2 = C.hw[2][el];
  H.b0 = C.hw[3][el]; H.b1 = C.hw[4][el]; H.b2 = C.hw[5][el];
  return H;
}

__device__ __forceinline__ Envelope deg_env(const e2v2_deg_args& A) {
  Envelope env;
  env.rc = A.rc; env.a = A.env_a; env.b = A.env_b; env.c = A.env_c;
  return env;
}

// Forward: x0[m][i][c] = (1/avg) sum_e Y_m(e) p(e) fea_l(m)(e)[c]; the edge
// subsets of the lanes are added by lane swaps (lane ^ Q, ^ 2 Q, ..., ^ 32: a
// fixed order).  kHid: the same sums of the hidden channels into hs [9][N][144]
// (row: 128 hidden sums, then (1/avg) sum_e Y_m p and 15 zeros, written by slice 0:
// lanes q = 0..3 of sub 0).
template <bool kHid>
__device__ __forceinline__ void deg_fwd_body(const e2v2_deg_args& A, float* __restrict__ out) {
  using S = DegSl<kHid>;
  constexpr int CH = 64;
  __shared__ DegChunk C;
  const int s = blockIdx.x % S::NS, i = blockIdx.x / S::NS;
  if (i >= A.n_rows) return;
  const int lane = threadIdx.x, sub = lane / S::Q, q = lane % S::Q;
  const int b = A.row_ptr[i], n = A.row_ptr[i + 1] - b;
  const Envelope env = deg_env(A);
  const RadialTab R = make_deg_tab<kHid>(A);
  const int ti = A.atom_type[i];
  floatx4 acc[9];
  float sacc[9];   // kHid: sum of Y_m p (the bias column)
#pragma unroll
  for (int m = 0; m < 9; ++m) {
    acc[m] = floatx4{0.f, 0.f, 0.f, 0.f};
    sacc[m] = 0.f;
  }
  for (int c0 = 0; c0 < n; c0 += CH) {
    const int nc = min(CH, n - c0);
    deg_chunk<S::Row, S::NS>(A, env, R, ti, s, (int64_t)b + c0, nc, C);
    __syncthreads();
    for (int el = sub; el < nc; el += S::Sub) {
      const float* tb = R.tab + C.toff[el] + 4 * q;
      const Hermite5 H = chunk_hermite(C, el);
      const float p = C.p[el];
      float Y[9];
#pragma unroll
      for (int m = 0; m < 9; ++m) Y[m] = C.Y[m][el];
      const floatx4 fa = deg_interp<S::Row>(tb, H, 0);
      const floatx4 fb = deg_interp<S::Row>(tb + S::W, H, 0);
      const floatx4 fc = deg_interp<S::Row>(tb + 2 * S::W, H, 0);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float f0 = fa[u] * p, f1 = fb[u] * p, f2 = fc[u] * p;
        acc[0][u] = fmaf(Y[0], f0, acc[0][u]);
#pragma unroll
        for (int m = 1; m < 4; ++m) acc[m][u] = fmaf(Y[m], f1, acc[m][u]);
#pragma unroll
        for (int m = 4; m < 9; ++m) acc[m][u] = fmaf(Y[m], f2, acc[m][u]);
      }
      if constexpr (kHid) {
#pragma unroll
        for (int m = 0; m < 9; ++m) sacc[m] = fmaf(Y[m], p, sacc[m]);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int m = 0; m < 9; ++m) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float v = acc[m][u];
#pragma unroll
      for (int o = S::Q; o < kWave; o <<= 1) v += __shfl_xor(v, o, kWave);
      acc[m][u] = v;
    }
    if constexpr (kHid) {
#pragma unroll
      for (int o = S::Q; o < kWave; o <<= 1) sacc[m] += __shfl_xor(sacc[m], o, kWave);
    }
  }
  if (sub == 0) {
    constexpr int ld = kHid ? kDHs : kDC;
#pragma unroll
    for (int m = 0; m < 9; ++m) {
      floatx4 o;
#pragma unroll
      for (int u = 0; u < 4; ++u) o[u] = acc[m][u] / A.avg;
      float* row = out + ((size_t)m * A.n_rows + i) * ld;
      *reinterpret_cast<floatx4*>(row + S::W * s + 4 * q) = o;
      if (kHid && s == 0 && q < 4)   // columns 128 + 4 q .. + 3: the bias column (q = 0) and zeros
        *reinterpret_cast<floatx4*>(row + kDH + 4 * q) = floatx4{q == 0 ? sacc[m] / A.avg : 0.f, 0.f, 0.f, 0.f};
    }
  }
}

__global__ __launch_bounds__(64) void k_deg_fwd_sl(e2v2_deg_args A, float* __restrict__ x0) {
  deg_fwd_body<false>(A, x0);
}
__global__ __launch_bounds__(64) void k_degh_fwd_sl(e2v2_deg_args A, float* __restrict__ hs) {
  deg_fwd_body<true>(A, hs);
}

// Sum over each group of 8 lanes (lanes 8 k .. 8 k + 7), left in every lane of the
// group: two quad permutes and the half-row mirror (fixed order).
__device__ __forceinline__ float sum8(float v) {
  v += dpp_mov<0xB1>(v);    // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);    // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);   // row_half_mirror
  return v;
}

// Sum over each quad of lanes (lanes 4 k .. 4 k + 3), left in every lane of the quad (fixed order).
__device__ __forceinline__ float sum4(float v) {
  v += dpp_mov<0xB1>(v);    // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);    // quad_perm [2,3,0,1]
  return v;
}

// Backward: per edge and slice, dfea_l[c] = p/avg sum_{m in l} Y_m G0[m][i][c];
// dL/dd = sum_{l,c} dfea_l[c] (p' fea_l[c] / p + fea_l'[c]) (envelope and profile
// derivative) and dL/dY -> dL/ddvec.  The Q lanes of an edge add their channel
// quads' sums and lane q = 0 writes the slice's partial part[s][e] =
// (dL/ddvec, dL/dd); e2v2_deg_bwd adds the 8 partials of every edge in slice order.
// kHid: G0 is grad_h [9][N][128] over the hidden channels, and slice 0 adds the
// bias column's terms from grad_s [9][N] (a channel of value 1 and derivative 0).
template <bool kHid>
__device__ __forceinline__ void deg_bwd_body(const e2v2_deg_args& A, const float* __restrict__ G0,
                                             const float* __restrict__ GS, float4* __restrict__ part) {
  using S = DegSl<kHid>;
  constexpr int CH = 64, ld = kHid ? kDH : kDC;
  __shared__ DegChunk C;
  const int s = blockIdx.x % S::NS, i = blockIdx.x / S::NS;
  if (i >= A.n_rows) return;
  const int lane = threadIdx.x, sub = lane / S::Q, q = lane % S::Q;
  const int b = A.row_ptr[i], n = A.row_ptr[i + 1] - b;
  const Envelope env = deg_env(A);
  const RadialTab R = make_deg_tab<kHid>(A);
  const int ti = A.atom_type[i];
  const int c = S::W * s + 4 * q;
  floatx4 g[9];
  float gs[9];
#pragma unroll
  for (int m = 0; m < 9; ++m) {
    const floatx4 v = *reinterpret_cast<const floatx4*>(G0 + ((size_t)m * A.n_rows + i) * ld + c);
#pragma unroll
    for (int u = 0; u < 4; ++u) g[m][u] = v[u] / A.avg;
    gs[m] = (kHid && s == 0) ? GS[(size_t)m * A.n_rows + i] / A.avg : 0.f;
  }
  for (int c0 = 0; c0 < n; c0 += CH) {
    const int nc = min(CH, n - c0);
    deg_chunk<S::Row, S::NS>(A, env, R, ti, s, (int64_t)b + c0, nc, C);
    __syncthreads();
    for (int el = sub; el < nc; el += S::Sub) {
      const float* tb = R.tab + C.toff[el] + 4 * q;
      const Hermite5 H = chunk_hermite(C, el);
      const float p = C.p[el];
      float Y[9];
#pragma unroll
      for (int m = 0; m < 9; ++m) Y[m] = C.Y[m][el];
      float dsh[9];
#pragma unroll
      for (int m = 0; m < 9; ++m) dsh[m] = 0.f;
      float s_val = 0.f, s_der = 0.f;   // sum dfea_l fea_l / p and sum dfea_l fea_l' / p
      // one degree block l (rows m0 .. m0 + 2l) at compile-time indices (the arrays stay in registers)
      auto block = [&](auto lc) {
        constexpr int l = decltype(lc)::value, m0 = l * l, m1 = (l + 1) * (l + 1);
        const floatx4 f = deg_interp<S::Row>(tb + l * S::W, H, 0);
        const floatx4 fd = deg_interp<S::Row>(tb + l * S::W, H, 1);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          float dl = 0.f;
#pragma unroll
          for (int m = m0; m < m1; ++m) {
            dl = fmaf(Y[m], g[m][u], dl);
            dsh[m] = fmaf(g[m][u], f[u] * p, dsh[m]);
          }
          s_val = fmaf(dl, f[u], s_val);
          s_der = fmaf(dl, fd[u], s_der);
        }
      };
      block(std::integral_constant<int, 0>{});
      block(std::integral_constant<int, 1>{});
      block(std::integral_constant<int, 2>{});
      auto sumq = [](float v) { return S::Q == 8 ? sum8(v) : sum4(v); };
      s_val = sumq(s_val);
      s_der = sumq(s_der);
#pragma unroll
      for (int m = 1; m < 9; ++m) dsh[m] = sumq(dsh[m]);
      if (q == 0) {
        if (kHid && s == 0) {   // the bias column: value 1, no distance derivative
#pragma unroll
          for (int m = 0; m < 9; ++m) {
            s_val = fmaf(Y[m], gs[m], s_val);
            dsh[m] = fmaf(gs[m], p, dsh[m]);
          }
        }
        const float ux = C.u[0][el], uy = C.u[1][el], uz = C.u[2][el], nrm = C.nrm[el];
        float gx, gy, gz;
        raw_sh2_bwd(ux, uy, uz, dsh, gx, gy, gz);
        // u = v / |v|:  dv = (du - u (u . du)) / |v|
        const float ud = ux * gx + uy * gy + uz * gz;
        part[(size_t)s * A.n_edges + b + c0 + el] =
            make_float4((gx - ux * ud) / nrm, (gy - uy * ud) / nrm, (gz - uz * ud) / nrm,
                        s_val * C.dp[el] + p * s_der * R.inv_h);
      }
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(64) void k_deg_bwd_sl(e2v2_deg_args A, const float* __restrict__ G0,
                                                   float4* __restrict__ part) {
  deg_bwd_body<false>(A, G0, nullptr, part);
}
__global__ __launch_bounds__(64) void k_degh_bwd_sl(e2v2_deg_args A, const float* __restrict__ GH,
                                                    const float* __restrict__ GS, float4* __restrict__ part) {
  deg_bwd_body<true>(A, GH, GS, part);
}

// grad_s[m][i] = sum_c grad_x0[m][i][c] b3[l(m)][c]: one wavefront per (m, i), four channels per lane, then a
// fixed-order wave sum.
__global__ __launch_bounds__(256) void k_deg_bias_grad(const float* __restrict__ gx0, const float* __restrict__ b3,
                                                       int n, float* __restrict__ gs) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);   // row m n + i of [9 n]
  if (r >= 9 * (int64_t)n) return;
  const int lane = threadIdx.x & 63, m = (int)(r / n);
  const floatx4 x = *reinterpret_cast<const floatx4*>(gx0 + r * kDC + 4 * lane);
  const floatx4 w = *reinterpret_cast<const floatx4*>(b3 + l_of(m) * kDC + 4 * lane);
  float v = x[0] * w[0];
  v = fmaf(x[1], w[1], v);
  v = fmaf(x[2], w[2], v);
  v = fmaf(x[3], w[3], v);
  v = wave_sum(v);
  if (lane == 0) gs[r] = v;
}

// dL/d dvec and dL/dd of every edge: the slices' partials part[s][e] (n_sl = 8 or 4) added in slice order.
__global__ __launch_bounds__(256) void k_edge_part_sum(const float4* __restrict__ part, int64_t n_edges,
                                                       float* __restrict__ ddv, float* __restrict__ dd, int n_sl) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= n_edges) return;
  float4 a = part[e];
#pragma unroll
  for (int s = 1; s < kDSl; ++s) {
    if (s >= n_sl) break;
    const float4 v = part[(int64_t)s * n_edges + e];
    a.x += v.x; a.y += v.y; a.z += v.z; a.w += v.w;
  }
  ddv[3 * e] = a.x;
  ddv[3 * e + 1] = a.y;
  ddv[3 * e + 2] = a.z;
  dd[e] = a.w;
}

int launch_edge_part_sum(const float* part, int64_t n_edges, float* ddv, float* dd, hipStream_t st, int n_sl) {
  if (n_edges <= 0) return 0;
  hipLaunchKernelGGL(k_edge_part_sum, dim3((unsigned)((n_edges + 255) / 256)), dim3(256), 0, st,
                     reinterpret_cast<const float4*>(part), n_edges, ddv, dd, n_sl);
  E2V2_LAUNCHED("k_edge_part_sum");
  return 0;
}

// dpos[a] = sum_{e in row a} g_e - sum_{e in column a} g_e,  g_e = ddv_e + dd_e dvec_e / d_e.
// One wavefront per atom: lanes stride over the row's and the column's edges,
// then a fixed-order wave reduction (deterministic).
constexpr int kPosWaves = 4;

__device__ __forceinline__ void edge_grad(int64_t e, const float* __restrict__ dvec, const float* __restrict__ dist,
                                          const float* __restrict__ ddv, const float* __restrict__ dd, float sign,
                                          float& gx, float& gy, float& gz) {
  const float s = dd[e] / dist[e];
  gx += sign * (ddv[3 * e] + s * dvec[3 * e]);
  gy += sign * (ddv[3 * e + 1] + s * dvec[3 * e + 1]);
  gz += sign * (ddv[3 * e + 2] + s * dvec[3 * e + 2]);
}

__global__ __launch_bounds__(64 * kPosWaves) void k_edge_to_pos(int n_atoms, const int32_t* __restrict__ row_ptr,
                                                                const int32_t* __restrict__ key_ptr,
                                                                const int32_t* __restrict__ key_eid,
                                                                const float* __restrict__ dvec,
                                                                const float* __restrict__ dist,
                                                                const float* __restrict__ ddv,
                                                                const float* __restrict__ dd, float* __restrict__ dpos) {
  const int lane = threadIdx.x & 63;
  for (int a = blockIdx.x * kPosWaves + (int)(threadIdx.x >> 6); a < n_atoms; a += gridDim.x * kPosWaves) {
    float gx = 0.f, gy = 0.f, gz = 0.f;
    for (int e = row_ptr[a] + lane; e < row_ptr[a + 1]; e += 64) edge_grad(e, dvec, dist, ddv, dd, 1.f, gx, gy, gz);
    for (int p = key_ptr[a] + lane; p < key_ptr[a + 1]; p += 64)
      edge_grad(key_eid[p], dvec, dist, ddv, dd, -1.f, gx, gy, gz);
    gx = wave_sum(gx); gy = wave_sum(gy); gz = wave_sum(gz);
    if (lane == 0) {
      dpos[3 * a] = gx;
      dpos[3 * a + 1] = gy;
      dpos[3 * a + 2] = gz;
    }
  }
}

}  // namespace e2v2

using namespace e2v2;

static int check_deg_table(const e2v2_deg_args& A, const char* who, int channels = kDC) {
  E2V2_REQUIRE(A.channels == channels, "%s: built for %d channels, got %d", who, channels, A.channels);
  E2V2_REQUIRE(A.rtab && A.atom_type && A.col && A.n_types >= 1 && A.n_types <= E2V2_MAX_TYPES && A.rtab_n >= 2 &&
                   A.rtab_h > 0.f && (double)A.rc * (1.0 / A.rtab_h) <= (double)(A.rtab_n - 1),
               "%s: needs the gbf_projs table covering the cutoff and the atom types (n_types %d, rtab_n %d)", who,
               A.n_types, A.rtab_n);
  // one wavefront per (row, slice): the grid holds 8 n_rows workgroups
  E2V2_REQUIRE(A.n_rows < (1 << 27), "%s: %d rows exceed the slice grid", who, A.n_rows);
  return 0;
}

E2V2_API int e2v2_deg_fwd(const e2v2_deg_args* args, float* x0, hipStream_t s) {
  const e2v2_deg_args& A = *args;
  if (int rc = check_deg_table(A, "deg_fwd")) return rc;
  if (A.n_rows == 0) return 0;
  hipLaunchKernelGGL(k_deg_fwd_sl, dim3((unsigned)A.n_rows * kDSl), dim3(kWave), 0, s, A, x0);
  E2V2_LAUNCHED("k_deg_fwd_sl");
  return 0;
}

E2V2_API size_t e2v2_deg_bwd_workspace(int64_t n_edges) {
  return n_edges > 0 ? (size_t)n_edges * kDSl * sizeof(float4) : 0;
}

E2V2_API int e2v2_deg_bwd(const e2v2_deg_args* args, const float* grad_x0, float* ddvec, float* ddist,
                          void* workspace, size_t workspace_bytes, hipStream_t s) {
  const e2v2_deg_args& A = *args;
  if (int rc = check_deg_table(A, "deg_bwd")) return rc;
  if (A.n_rows == 0) return 0;
  const size_t need = e2v2_deg_bwd_workspace(A.n_edges);
  E2V2_REQUIRE(workspace_bytes >= need && (need == 0 || workspace) &&
                   reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
               "deg_bwd: workspace of %zu bytes (16-byte aligned) needed, got %zu", need, workspace_bytes);
  float4* part = static_cast<float4*>(workspace);
  hipLaunchKernelGGL(k_deg_bwd_sl, dim3((unsigned)A.n_rows * kDSl), dim3(kWave), 0, s, A, grad_x0, part);
  E2V2_LAUNCHED("k_deg_bwd_sl");
  return launch_edge_part_sum(reinterpret_cast<const float*>(part), A.n_edges, ddvec, ddist, s, kDSl);
}

E2V2_API int e2v2_deg_hidden_fwd(const e2v2_deg_args* args, float* hs, hipStream_t s) {
  E2V2_REQUIRE(args && hs && ((uintptr_t)hs & 15) == 0, "deg_hidden_fwd: null argument or hs not 16-byte aligned");
  const e2v2_deg_args& A = *args;
  if (int rc = check_deg_table(A, "deg_hidden_fwd", kDH)) return rc;
  if (A.n_rows == 0) return 0;
  hipLaunchKernelGGL(k_degh_fwd_sl, dim3((unsigned)A.n_rows * DegSl<true>::NS), dim3(kWave), 0, s, A, hs);
  E2V2_LAUNCHED("k_degh_fwd_sl");
  return 0;
}

E2V2_API int e2v2_deg_hidden_bwd(const e2v2_deg_args* args, const float* grad_h, const float* grad_s, float* ddvec,
                                 float* ddist, void* workspace, size_t workspace_bytes, hipStream_t s) {
  E2V2_REQUIRE(args, "deg_hidden_bwd: null arguments");
  const e2v2_deg_args& A = *args;
  if (int rc = check_deg_table(A, "deg_hidden_bwd", kDH)) return rc;
  if (A.n_rows == 0) return 0;
  E2V2_REQUIRE(grad_h && grad_s && ddvec && ddist && ((uintptr_t)grad_h & 15) == 0,
               "deg_hidden_bwd: null operand or grad_h not 16-byte aligned");
  const size_t need = e2v2_deg_bwd_workspace(A.n_edges);
  E2V2_REQUIRE(workspace_bytes >= need && (need == 0 || workspace) &&
                   reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
               "deg_hidden_bwd: workspace of %zu bytes (16-byte aligned) needed, got %zu", need, workspace_bytes);
  float4* part = static_cast<float4*>(workspace);
  hipLaunchKernelGGL(k_degh_bwd_sl, dim3((unsigned)A.n_rows * DegSl<true>::NS), dim3(kWave), 0, s, A, grad_h,
                     grad_s, part);
  E2V2_LAUNCHED("k_degh_bwd_sl");
  return launch_edge_part_sum(reinterpret_cast<const float*>(part), A.n_edges, ddvec, ddist, s, DegSl<true>::NS);
}

E2V2_API int e2v2_deg_bias_grad(const float* grad_x0, const float* b3, int32_t n, float* grad_s, hipStream_t s) {
  E2V2_REQUIRE(n >= 0 && n < (1 << 27), "deg_bias_grad: n=%d", n);
  if (n == 0) return 0;
  E2V2_REQUIRE(grad_x0 && b3 && grad_s && ((uintptr_t)grad_x0 & 15) == 0 && ((uintptr_t)b3 & 15) == 0,
               "deg_bias_grad: null or unaligned operand (16 bytes)");
  const int64_t rows = 9 * (int64_t)n;
  hipLaunchKernelGGL(k_deg_bias_grad, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, grad_x0, b3, n, grad_s);
  E2V2_LAUNCHED("k_deg_bias_grad");
  return 0;
}

E2V2_API int e2v2_edge_to_pos(int n_atoms, const int32_t* row_ptr, const int32_t* key_ptr, const int32_t* key_eid,
                              const float* dvec, const float* dist, const float* ddvec, const float* ddist,
                              float* dpos, hipStream_t s) {
  if (n_atoms == 0) return 0;
  const int blocks = (int)std::min<int64_t>(((int64_t)n_atoms + kPosWaves - 1) / kPosWaves, 1 << 20);
  hipLaunchKernelGGL(k_edge_to_pos, dim3(blocks), dim3(64 * kPosWaves), 0, s, n_atoms, row_ptr, key_ptr, key_eid,
                     dvec, dist, ddvec, ddist, dpos);
  E2V2_LAUNCHED("k_edge_to_pos");
  return 0;
}
