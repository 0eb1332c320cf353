// Edge-degree embedding (src/molfm/models/e2former/e2former.py:689-753) and
// the edge -> position gradient assembly.
//
// Forward, one wavefront per query atom i (lane owns channels 4 lane .. + 3):
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

// dY/du for u = (x, y, z) given dL/dY -> dL/du
__device__ __forceinline__ void raw_sh2_bwd(float x, float y, float z, const float (&g)[9], float& gx, float& gy,
                                            float& gz) {
  const float s3 = 1.7320508075688772f;
  gx = g[1] + s3 * z * g[4] + s3 * y * g[5] - x * g[6] - s3 * x * g[8];
  gy = g[2] + s3 * x * g[5] + 2.f * y * g[6] + s3 * z * g[7];
  gz = g[3] + s3 * x * g[4] - z * g[6] + s3 * y * g[7] + s3 * z * g[8];
}

__device__ __forceinline__ int l_of(int m) { return m == 0 ? 0 : (m < 4 ? 1 : 2); }

__device__ __forceinline__ RadialTab make_deg_tab(const e2v2_deg_args& A) {
  RadialTab R;
  R.tab = A.rtab; R.n_types = A.n_types; R.n_nodes = A.rtab_n; R.nc = kDegC; R.inv_h = 1.0f / A.rtab_h;
  return R;
}

// Four consecutive channels of profile l from rows r0 .. r0 + 2 at both nodes (node block p):
// the quintic Hermite interpolant.
__device__ __forceinline__ floatx4 deg_interp(const float* p, const Hermite5& H, int r0) {
  const floatx4 f0 = *reinterpret_cast<const floatx4*>(p + r0 * kDegC);
  const floatx4 f1 = *reinterpret_cast<const floatx4*>(p + (r0 + 1) * kDegC);
  const floatx4 f2 = *reinterpret_cast<const floatx4*>(p + (r0 + 2) * kDegC);
  const floatx4 g0 = *reinterpret_cast<const floatx4*>(p + (4 + r0) * kDegC);
  const floatx4 g1 = *reinterpret_cast<const floatx4*>(p + (5 + r0) * kDegC);
  const floatx4 g2 = *reinterpret_cast<const floatx4*>(p + (6 + r0) * kDegC);
  floatx4 v;
#pragma unroll
  for (int u = 0; u < 4; ++u) v[u] = herm_value(H, f0[u], f1[u], f2[u], g0[u], g1[u], g2[u]);
  return v;
}

// One wavefront per query atom; lane owns channels 4 lane .. 4 lane + 3 (16-byte
// loads of each edge's table rows); the edge's SH, envelope and table node are
// wave-uniform.
constexpr int kDegWaves = 4;

__global__ __launch_bounds__(64 * kDegWaves) void k_deg_fwd(e2v2_deg_args A, float* __restrict__ x0) {
  const int w = (int)(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int i = xcd_row(blockIdx.x, (A.n_rows + kDegWaves - 1) / kDegWaves) * kDegWaves + w;
  if (i >= A.n_rows) return;
  const int b = A.row_ptr[i], n = A.row_ptr[i + 1] - b;
  Envelope env;
  env.rc = A.rc; env.a = A.env_a; env.b = A.env_b; env.c = A.env_c;
  const RadialTab R = make_deg_tab(A);
  const int ti = A.atom_type[i];
  floatx4 acc[9];
#pragma unroll
  for (int m = 0; m < 9; ++m) acc[m] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int c = 4 * lane;
  for (int el = 0; el < n; ++el) {
    const int64_t e = (int64_t)b + el;
    const float d = A.dist[e];
    const float nrm = fmaxf(d, 1e-12f);
    float Y[9];
    raw_sh2(A.dvec[3 * e] / nrm, A.dvec[3 * e + 1] / nrm, A.dvec[3 * e + 2] / nrm, Y);
    float p, dp;
    env.eval(d, p, dp);
    float t;
    const float* tb = R.tab + radial_node(R, ti * R.n_types + A.atom_type[A.col[e]], d, t) + c;
    const Hermite5 H = hermite5(t);
    const floatx4 fa = deg_interp(tb, H, 0);
    const floatx4 fb = deg_interp(tb + kDC, H, 0);
    const floatx4 fc = deg_interp(tb + 2 * kDC, H, 0);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float f0 = fa[u] * p, f1 = fb[u] * p, f2 = fc[u] * p;
      acc[0][u] = fmaf(Y[0], f0, acc[0][u]);
#pragma unroll
      for (int m = 1; m < 4; ++m) acc[m][u] = fmaf(Y[m], f1, acc[m][u]);
#pragma unroll
      for (int m = 4; m < 9; ++m) acc[m][u] = fmaf(Y[m], f2, acc[m][u]);
    }
  }
#pragma unroll
  for (int m = 0; m < 9; ++m) {
    floatx4 o;
#pragma unroll
    for (int u = 0; u < 4; ++u) o[u] = acc[m][u] / A.avg;
    *reinterpret_cast<floatx4*>(x0 + ((size_t)m * A.n_rows + i) * kDC + c) = o;
  }
}

// One workgroup per query atom; one wave per edge, lane owns channels 4 lane .. + 3.
// Per edge: dfea_l[c] = p/avg sum_{m in l} Y_m G0[m][i][c]; dL/dd = sum_{l,c} dfea_l[c]
// (p' fea_l[c] / p + fea_l'[c]) (envelope and profile derivative) and dL/dY -> dL/ddvec.
__global__ __launch_bounds__(256) void k_deg_bwd(e2v2_deg_args A, const float* __restrict__ G0,
                                                 float* __restrict__ ddv, float* __restrict__ dd) {
  const int i = xcd_row(blockIdx.x, A.n_rows), t = threadIdx.x, lane = t & 63, wave = t >> 6;
  if (i >= A.n_rows) return;
  const int b = A.row_ptr[i], n = A.row_ptr[i + 1] - b;
  Envelope env;
  env.rc = A.rc; env.a = A.env_a; env.b = A.env_b; env.c = A.env_c;
  const RadialTab R = make_deg_tab(A);
  const int ti = A.atom_type[i];
  const int c = 4 * lane;
  floatx4 g[9];
#pragma unroll
  for (int m = 0; m < 9; ++m) {
    const floatx4 v = *reinterpret_cast<const floatx4*>(G0 + ((size_t)m * A.n_rows + i) * kDC + c);
#pragma unroll
    for (int u = 0; u < 4; ++u) g[m][u] = v[u] / A.avg;
  }
  for (int el = wave; el < n; el += 4) {
    const int64_t e = (int64_t)b + el;
    const float d = A.dist[e];
    const float nrm = fmaxf(d, 1e-12f);
    const float ux = A.dvec[3 * e] / nrm, uy = A.dvec[3 * e + 1] / nrm, uz = A.dvec[3 * e + 2] / nrm;
    float Y[9];
    raw_sh2(ux, uy, uz, Y);
    float p, dpdd;
    env.eval(d, p, dpdd);
    float tt;
    const float* tb = R.tab + radial_node(R, ti * R.n_types + A.atom_type[A.col[e]], d, tt) + c;
    const Hermite5 H = hermite5(tt);
    float dsh[9];
#pragma unroll
    for (int m = 0; m < 9; ++m) dsh[m] = 0.f;
    float s_val = 0.f, s_der = 0.f;   // sum dfea_l fea_l / p and sum dfea_l fea_l' / p
    // one degree block l (rows m0 .. m0 + 2l) at compile-time indices (the arrays stay in registers)
    auto block = [&](auto lc) {
      constexpr int l = decltype(lc)::value, m0 = l * l, m1 = (l + 1) * (l + 1);
      const floatx4 f = deg_interp(tb + l * kDC, H, 0);
      const floatx4 fd = deg_interp(tb + l * kDC, H, 1);
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
    s_val = wave_sum(s_val);
    s_der = wave_sum(s_der);
#pragma unroll
    for (int m = 1; m < 9; ++m) dsh[m] = wave_sum(dsh[m]);
    if (lane == 0) {
      float gx, gy, gz;
      raw_sh2_bwd(ux, uy, uz, dsh, gx, gy, gz);
      // u = v / |v|:  dv = (du - u (u . du)) / |v|
      const float ud = ux * gx + uy * gy + uz * gz;
      ddv[3 * e] = (gx - ux * ud) / nrm;
      ddv[3 * e + 1] = (gy - uy * ud) / nrm;
      ddv[3 * e + 2] = (gz - uz * ud) / nrm;
      dd[e] = s_val * dpdd + p * s_der * R.inv_h;
    }
  }
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

static int check_deg_table(const e2v2_deg_args& A, const char* who) {
  E2V2_REQUIRE(A.channels == kDC, "%s: built for C=%d, got %d", who, kDC, A.channels);
  E2V2_REQUIRE(A.rtab && A.atom_type && A.col && A.n_types >= 1 && A.n_types <= E2V2_MAX_TYPES && A.rtab_n >= 2 &&
                   A.rtab_h > 0.f && (double)A.rc * (1.0 / A.rtab_h) <= (double)(A.rtab_n - 1),
               "%s: needs the gbf_projs table covering the cutoff and the atom types (n_types %d, rtab_n %d)", who,
               A.n_types, A.rtab_n);
  return 0;
}

E2V2_API int e2v2_deg_fwd(const e2v2_deg_args* args, float* x0, hipStream_t s) {
  const e2v2_deg_args& A = *args;
  if (int rc = check_deg_table(A, "deg_fwd")) return rc;
  if (A.n_rows == 0) return 0;
  hipLaunchKernelGGL(k_deg_fwd, dim3(xcd_grid((A.n_rows + kDegWaves - 1) / kDegWaves)), dim3(64 * kDegWaves), 0, s,
                     A, x0);
  E2V2_LAUNCHED("k_deg_fwd");
  return 0;
}

E2V2_API int e2v2_deg_bwd(const e2v2_deg_args* args, const float* grad_x0, float* ddvec, float* ddist,
                          hipStream_t s) {
  const e2v2_deg_args& A = *args;
  if (int rc = check_deg_table(A, "deg_bwd")) return rc;
  if (A.n_rows == 0) return 0;
  hipLaunchKernelGGL(k_deg_bwd, dim3(xcd_grid(A.n_rows)), dim3(256), 0, s, A, grad_x0, ddvec, ddist);
  E2V2_LAUNCHED("k_deg_bwd");
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
