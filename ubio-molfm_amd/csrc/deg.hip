// Edge-degree embedding (src/molfm/models/e2former/e2former.py:689-753) and
// the edge -> position gradient assembly.
//
// Forward, one workgroup per query atom i (thread per channel c):
//   x0[i, m, c] = (1/avg) sum_e Y_m(dvec_e / |dvec_e|) * fea_e[l(m), c] * p(d_e)
// with Y the e3nn raw real spherical harmonics of degree <= 2 (unit norm per
// l block) and fea the three radial-MLP outputs [E, 3, 256].
// Backward: dL/ddvec and dL/dd per edge, and optionally dfea (the MLP
// backward can form dfea from G0 itself: e2v2_mlp_bwd_deg).
#include <algorithm>
#include "common.h"
#include "../../include/e2v2.h"

namespace e2v2 {

constexpr int kDC = 256;

// dY/du for u = (x, y, z) given dL/dY -> dL/du
__device__ __forceinline__ void raw_sh2_bwd(float x, float y, float z, const float (&g)[9], float& gx, float& gy,
                                            float& gz) {
  const float s3 = 1.7320508075688772f;
  gx = g[1] + s3 * z * g[4] + s3 * y * g[5] - x * g[6] - s3 * x * g[8];
  gy = g[2] + s3 * x * g[5] + 2.f * y * g[6] + s3 * z * g[7];
  gz = g[3] + s3 * x * g[4] - z * g[6] + s3 * y * g[7] + s3 * z * g[8];
}

__device__ __forceinline__ int l_of(int m) { return m == 0 ? 0 : (m < 4 ? 1 : 2); }

// One wavefront per query atom; lane owns channels 4 lane .. 4 lane + 3 (16-byte
// loads of each edge's three feature rows); the edge's SH and envelope are
// wave-uniform.
constexpr int kDegWaves = 4;

__global__ __launch_bounds__(64 * kDegWaves) void k_deg_fwd(e2v2_deg_args A, float* __restrict__ x0) {
  const int w = (int)(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int i = xcd_row(blockIdx.x, (A.n_rows + kDegWaves - 1) / kDegWaves) * kDegWaves + w;
  if (i >= A.n_rows) return;
  const int b = A.row_ptr[i], n = A.row_ptr[i + 1] - b;
  Envelope env;
  env.rc = A.rc; env.a = A.env_a; env.b = A.env_b; env.c = A.env_c;
  floatx4 acc[9];
#pragma unroll
  for (int m = 0; m < 9; ++m) acc[m] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int c = 4 * lane;
#pragma unroll 2
  for (int el = 0; el < n; ++el) {
    const int64_t e = (int64_t)b + el;
    const float d = A.dist[e];
    const float nrm = fmaxf(d, 1e-12f);
    float Y[9];
    raw_sh2(A.dvec[3 * e] / nrm, A.dvec[3 * e + 1] / nrm, A.dvec[3 * e + 2] / nrm, Y);
    float p, dp;
    env.eval(d, p, dp);
    const float* f = A.fea + e * (3 * kDC) + c;
    const floatx4 fa = *reinterpret_cast<const floatx4*>(f);
    const floatx4 fb = *reinterpret_cast<const floatx4*>(f + kDC);
    const floatx4 fc = *reinterpret_cast<const floatx4*>(f + 2 * kDC);
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

// one workgroup per query atom; one wave per edge, lane owns channels lane + 64 q
__global__ __launch_bounds__(256) void k_deg_bwd(e2v2_deg_args A, const float* __restrict__ G0,
                                                 float* __restrict__ dfea, float* __restrict__ ddv,
                                                 float* __restrict__ dd) {
  const int i = xcd_row(blockIdx.x, A.n_rows), t = threadIdx.x, lane = t & 63, wave = t >> 6;
  if (i >= A.n_rows) return;
  const int b = A.row_ptr[i], n = A.row_ptr[i + 1] - b;
  Envelope env;
  env.rc = A.rc; env.a = A.env_a; env.b = A.env_b; env.c = A.env_c;
  float g[4][9];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int m = 0; m < 9; ++m) g[q][m] = G0[((size_t)m * A.n_rows + i) * kDC + lane + 64 * q] / A.avg;
  for (int el = wave; el < n; el += 4) {
    const int64_t e = (int64_t)b + el;
    const float d = A.dist[e];
    const float nrm = fmaxf(d, 1e-12f);
    const float ux = A.dvec[3 * e] / nrm, uy = A.dvec[3 * e + 1] / nrm, uz = A.dvec[3 * e + 2] / nrm;
    float Y[9];
    raw_sh2(ux, uy, uz, Y);
    float p, dpdd;
    env.eval(d, p, dpdd);
    float dsh[9];
#pragma unroll
    for (int m = 0; m < 9; ++m) dsh[m] = 0.f;
    float dp = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = lane + 64 * q;
      const float* f = A.fea + e * (3 * kDC) + c;
      const float f0 = f[0], f1 = f[kDC], f2 = f[2 * kDC];
      // d(edge_fea_l) = sum_{m in l} Y_m g_m
      const float d0 = Y[0] * g[q][0];
      const float d1 = Y[1] * g[q][1] + Y[2] * g[q][2] + Y[3] * g[q][3];
      const float d2 = Y[4] * g[q][4] + Y[5] * g[q][5] + Y[6] * g[q][6] + Y[7] * g[q][7] + Y[8] * g[q][8];
      if (dfea) {  // NULL when the MLP backward forms these from G0 itself
        float* df = dfea + e * (3 * kDC) + c;
        df[0] = d0 * p;
        df[kDC] = d1 * p;
        df[2 * kDC] = d2 * p;
      }
      dp = fmaf(d0, f0, dp);
      dp = fmaf(d1, f1, dp);
      dp = fmaf(d2, f2, dp);
      const float e0 = f0 * p, e1 = f1 * p, e2 = f2 * p;
      dsh[0] = fmaf(g[q][0], e0, dsh[0]);
#pragma unroll
      for (int m = 1; m < 4; ++m) dsh[m] = fmaf(g[q][m], e1, dsh[m]);
#pragma unroll
      for (int m = 4; m < 9; ++m) dsh[m] = fmaf(g[q][m], e2, dsh[m]);
    }
    dp = wave_sum(dp);
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
      dd[e] = dp * dpdd;
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

E2V2_API int e2v2_deg_fwd(const e2v2_deg_args* args, float* x0, hipStream_t s) {
  const e2v2_deg_args& A = *args;
  E2V2_REQUIRE(A.channels == kDC, "deg_fwd: built for C=%d, got %d", kDC, A.channels);
  if (A.n_rows == 0) return 0;
  hipLaunchKernelGGL(k_deg_fwd, dim3(xcd_grid((A.n_rows + kDegWaves - 1) / kDegWaves)), dim3(64 * kDegWaves), 0, s,
                     A, x0);
  E2V2_LAUNCHED("k_deg_fwd");
  return 0;
}

E2V2_API int e2v2_deg_bwd(const e2v2_deg_args* args, const float* grad_x0, float* dfea, float* ddvec, float* ddist,
                          hipStream_t s) {
  const e2v2_deg_args& A = *args;
  E2V2_REQUIRE(A.channels == kDC, "deg_bwd: built for C=%d, got %d", kDC, A.channels);
  if (A.n_rows == 0) return 0;
  hipLaunchKernelGGL(k_deg_bwd, dim3(xcd_grid(A.n_rows)), dim3(256), 0, s, A, grad_x0, dfea, ddvec, ddist);
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
