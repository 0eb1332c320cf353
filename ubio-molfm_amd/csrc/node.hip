// Per-node kernels on the m-major node layout x[9][N][C] (C = 256, l <= 2):
//  * rms_norm_sh  = EquivariantRMSNormArraySphericalHarmonicsV2_BL
//    (src/molfm/models/e2former/module_utils.py:1663-1772: centre the l = 0 row,
//    degree-balanced mean square over all (m, c), affine per l, bias on l = 0)
//  * Gate_s3 activation (module_utils.py:2694-2746) given the gate logits
//    sc[N][3C] = gates(x[0]).
// Backward passes return input gradients only (weights are constants for force
// evaluation) and recompute the statistics.
#include <type_traits>

#include "common.h"
#include "../../include/e2v2.h"

namespace e2v2 {

constexpr int kNC = 256;

__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

__device__ __forceinline__ int lof(int m) { return m == 0 ? 0 : (m < 4 ? 1 : 2); }

// balance weight of row m: 1 / ((2l+1) (lmax+1))
__device__ __forceinline__ float bal(int m) {
  const int l = lof(m);
  return 1.0f / ((2.0f * l + 1.0f) * 3.0f);
}

// y = rms_norm_sh(x), or with delta: xs = x + delta (the residual add of the
// producing block, written out) and y = rms_norm_sh(xs)
__global__ __launch_bounds__(256) void k_rmsnorm_fwd(const float* __restrict__ x, const float* __restrict__ delta,
                                                     const float* __restrict__ w, const float* __restrict__ b,
                                                     float* __restrict__ xs, float* __restrict__ y, int n,
                                                     float eps) {
  __shared__ float red[4];
  const int i = blockIdx.x, c = threadIdx.x;
  const size_t st = (size_t)n * kNC;
  const float* xp = x + (size_t)i * kNC + c;
  float f[9];
#pragma unroll
  for (int m = 0; m < 9; ++m) f[m] = xp[m * st];
  if (delta) {
    const float* dp = delta + (size_t)i * kNC + c;
    float* sp = xs + (size_t)i * kNC + c;
#pragma unroll
    for (int m = 0; m < 9; ++m) {
      f[m] += dp[m * st];
      sp[m * st] = f[m];
    }
  }
  const float mean0 = block_sum256(f[0], red) * (1.0f / kNC);
  f[0] -= mean0;
  float ss = 0.f;
#pragma unroll
  for (int m = 0; m < 9; ++m) ss = fmaf(bal(m), f[m] * f[m], ss);
  const float S = block_sum256(ss, red) * (1.0f / kNC);
  const float r = 1.0f / sqrtf(S + eps);
  float* yp = y + (size_t)i * kNC + c;
#pragma unroll
  for (int m = 0; m < 9; ++m) {
    float v = f[m] * (r * w[lof(m) * kNC + c]);
    if (m == 0) v += b[c];
    yp[m * st] = v;
  }
}

__global__ __launch_bounds__(256) void k_rmsnorm_bwd(const float* __restrict__ x, const float* __restrict__ w,
                                                     const float* __restrict__ gy, const float* __restrict__ gres,
                                                     float* __restrict__ gx, int n, float eps) {
  __shared__ float red[4];
  const int i = blockIdx.x, c = threadIdx.x;
  const size_t st = (size_t)n * kNC;
  const float* xp = x + (size_t)i * kNC + c;
  const float* gp = gy + (size_t)i * kNC + c;
  float f[9], g[9];
#pragma unroll
  for (int m = 0; m < 9; ++m) {
    f[m] = xp[m * st];
    g[m] = gp[m * st];
  }
  const float mean0 = block_sum256(f[0], red) * (1.0f / kNC);
  f[0] -= mean0;
  float ss = 0.f, dr = 0.f;
#pragma unroll
  for (int m = 0; m < 9; ++m) {
    ss = fmaf(bal(m), f[m] * f[m], ss);
    g[m] *= w[lof(m) * kNC + c];      // dL/d(f r) per element
    dr = fmaf(g[m], f[m], dr);
  }
  const float S = block_sum256(ss, red) * (1.0f / kNC);
  const float DR = block_sum256(dr, red);
  const float r = 1.0f / sqrtf(S + eps);
  const float dS = -0.5f * r * r * r * DR;
  float gf[9];
#pragma unroll
  for (int m = 0; m < 9; ++m) gf[m] = g[m] * r + dS * 2.0f * bal(m) * f[m] * (1.0f / kNC);
  const float gmean0 = block_sum256(gf[0], red) * (1.0f / kNC);
  gf[0] -= gmean0;
  float* op = gx + (size_t)i * kNC + c;
  if (gres) {  // gradient of a residual branch that reads x directly
    const float* rp = gres + (size_t)i * kNC + c;
#pragma unroll
    for (int m = 0; m < 9; ++m) op[m * st] = gf[m] + rp[m * st];
  } else {
#pragma unroll
    for (int m = 0; m < 9; ++m) op[m * st] = gf[m];
  }
}

__global__ void k_gate_fwd(const float* __restrict__ sc, const float* __restrict__ x, float* __restrict__ y, int n,
                           float k1, float k2) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)n * kNC) return;
  const int i = (int)(idx / kNC), c = (int)(idx % kNC);
  const size_t st = (size_t)n * kNC;
  const float* s = sc + (size_t)i * 3 * kNC;
  y[idx] = silu(s[c]) * k1;
  const float g1 = sigmoidf_(s[kNC + c]) * k2, g2 = sigmoidf_(s[2 * kNC + c]) * k2;
#pragma unroll
  for (int m = 1; m < 9; ++m) y[idx + m * st] = (m < 4 ? g1 : g2) * x[idx + m * st];
}

__global__ void k_gate_bwd(const float* __restrict__ sc, const float* __restrict__ x, const float* __restrict__ gy,
                           float* __restrict__ gsc, float* __restrict__ gx, int n, float k1, float k2) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)n * kNC) return;
  const int i = (int)(idx / kNC), c = (int)(idx % kNC);
  const size_t st = (size_t)n * kNC;
  const float* s = sc + (size_t)i * 3 * kNC;
  float* gs = gsc + (size_t)i * 3 * kNC;
  const float s0 = s[c];
  const float sg0 = sigmoidf_(s0);
  gs[c] = gy[idx] * k1 * sg0 * (1.0f + s0 * (1.0f - sg0));
  gx[idx] = 0.f;
  const float sg1 = sigmoidf_(s[kNC + c]), sg2 = sigmoidf_(s[2 * kNC + c]);
  float a1 = 0.f, a2 = 0.f;
#pragma unroll
  for (int m = 1; m < 9; ++m) {
    const float g = gy[idx + m * st];
    if (m < 4) {
      a1 = fmaf(g, x[idx + m * st], a1);
      gx[idx + m * st] = g * sg1 * k2;
    } else {
      a2 = fmaf(g, x[idx + m * st], a2);
      gx[idx + m * st] = g * sg2 * k2;
    }
  }
  gs[kNC + c] = a1 * k2 * sg1 * (1.0f - sg1);
  gs[2 * kNC + c] = a2 * k2 * sg2 * (1.0f - sg2);
}

// Derivative of the Gate_s3 backward (k_gate_bwd) for the training path's second differentiation:
// given the upstream gradients qsc [N][768] on gsc and qx [9][N][256] on gx (each may be NULL: zero),
// with s_l the logits of degree l at (i, c), sg_l = sigmoid(s_l), sg'_l = sg_l (1 - sg_l),
// sg''_l = sg'_l (1 - 2 sg_l), silu'(s) = sg (1 + s (1 - sg)), silu''(s) = sg (1 - sg) (2 + s (1 - 2 sg)):
//   dgy_0 = q_0 k1 silu'(s_0),   dgy_m = k2 (q_l sg'_l x_m + qx_m sg_l)   (m >= 1, l = l(m)),
//   dx_0 = 0,                     dx_m = k2 q_l sg'_l gy_m,
//   dsc_0 = q_0 k1 silu''(s_0) gy_0,   dsc_l = k2 (q_l sg''_l sum_{m in l} gy_m x_m + sg'_l sum_{m in l} qx_m gy_m).
__global__ void k_gate_bwd2(const float* __restrict__ sc, const float* __restrict__ x, const float* __restrict__ gy,
                            const float* __restrict__ qsc, const float* __restrict__ qx, float* __restrict__ dgy,
                            float* __restrict__ dsc, float* __restrict__ dx, int n, float k1, float k2) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)n * kNC) return;
  const int i = (int)(idx / kNC), c = (int)(idx % kNC);
  const size_t st = (size_t)n * kNC;
  const size_t srow = (size_t)i * 3 * kNC;
  float sl[3], sg[3], d1[3], q[3];
#pragma unroll
  for (int l = 0; l < 3; ++l) {
    sl[l] = sc[srow + l * kNC + c];
    sg[l] = sigmoidf_(sl[l]);
    d1[l] = sg[l] * (1.0f - sg[l]);
    q[l] = qsc ? qsc[srow + l * kNC + c] : 0.f;
  }
  const float g0 = gy[idx];
  dgy[idx] = q[0] * k1 * (sg[0] * (1.0f + sl[0] * (1.0f - sg[0])));
  dx[idx] = 0.f;
  dsc[srow + c] = q[0] * k1 * (d1[0] * (2.0f + sl[0] * (1.0f - 2.0f * sg[0]))) * g0;
  float gxs[3] = {0.f, 0.f, 0.f}, qgs[3] = {0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 1; m < 9; ++m) {
    const int l = m < 4 ? 1 : 2;
    const float g = gy[idx + m * st], xv = x[idx + m * st];
    const float qv = qx ? qx[idx + m * st] : 0.f;
    dgy[idx + m * st] = k2 * (q[l] * d1[l] * xv + qv * sg[l]);
    dx[idx + m * st] = k2 * q[l] * d1[l] * g;
    gxs[l] = fmaf(g, xv, gxs[l]);
    qgs[l] = fmaf(qv, g, qgs[l]);
  }
#pragma unroll
  for (int l = 1; l < 3; ++l)
    dsc[srow + l * kNC + c] = k2 * (q[l] * (d1[l] * (1.0f - 2.0f * sg[l])) * gxs[l] + d1[l] * qgs[l]);
}

// ---- rms_norm_sh on the training path, where the forces are differentiated once more.  Per node
// (f = x with row 0 centred over the channels, r = (S + eps)^-1/2, S = <bal f^2> over the channels and
// summed over the rows, P = gy w, C = 256):
//   first order   gx = centred_0(r P - (r^3 / C) (sum P f) bal f), dw_l = sum_nodes sum_{m in l} gy f r,
//                 db = sum_nodes gy_0;
//   second order  (upstream qx, qw, qb on gx, dw, db; q = centred_0(qx), Qw = qw of the row's degree,
//                 A = sum q P, B = sum q bal f, G = sum P f, T = sum gy Qw f, k = r^3 / C)
//                 u = r q - k B f,  dgy = w u + r Qw f + [m = 0] qb,  d(w)_l = sum_nodes sum_{m in l} gy u,
//                 dx = centred_0(-k (P B + G q bal) + r gy Qw - (A - 3 r^2 G B / C + T) k bal f).
// One workgroup per node (thread = channel), nodes strided over n_part workgroups; each writes its
// parameter sums to part [n_part][4 or 3][256] (summed over workgroups by the caller, in fixed order).
template <int K>
__device__ __forceinline__ void block_sums256(float (&v)[K], float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < K; ++k) v[k] = wave_sum(v[k]);
  __syncthreads();
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < K; ++k) red[wave * K + k] = v[k];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < K; ++k) v[k] = red[k] + red[K + k] + red[2 * K + k] + red[3 * K + k];
}

__global__ __launch_bounds__(256) void k_rmsnorm_bwd_param(const float* __restrict__ x, const float* __restrict__ w,
                                                           const float* __restrict__ gy, float* __restrict__ gx,
                                                           float* __restrict__ part, int n, float eps) {
  __shared__ float red[4];
  const int c = threadIdx.x;
  const size_t st = (size_t)n * kNC;
  float aw[3] = {0.f, 0.f, 0.f}, ab = 0.f;
  for (int i = blockIdx.x; i < n; i += gridDim.x) {
    const float* xp = x + (size_t)i * kNC + c;
    const float* gp = gy + (size_t)i * kNC + c;
    float f[9], g[9];
#pragma unroll
    for (int m = 0; m < 9; ++m) {
      f[m] = xp[m * st];
      g[m] = gp[m * st];
    }
    ab += g[0];
    const float mean0 = block_sum256(f[0], red) * (1.0f / kNC);
    f[0] -= mean0;
    float ss = 0.f, dr = 0.f;
#pragma unroll
    for (int m = 0; m < 9; ++m) {
      ss = fmaf(bal(m), f[m] * f[m], ss);
      dr = fmaf(g[m] * w[lof(m) * kNC + c], f[m], dr);
    }
    const float S = block_sum256(ss, red) * (1.0f / kNC);
    const float DR = block_sum256(dr, red);
    const float r = 1.0f / sqrtf(S + eps);
    const float dS = -0.5f * r * r * r * DR;
    float gf[9];
#pragma unroll
    for (int m = 0; m < 9; ++m) {
      aw[lof(m)] = fmaf(g[m], f[m] * r, aw[lof(m)]);
      gf[m] = (g[m] * w[lof(m) * kNC + c]) * r + dS * 2.0f * bal(m) * f[m] * (1.0f / kNC);
    }
    const float gmean0 = block_sum256(gf[0], red) * (1.0f / kNC);
    gf[0] -= gmean0;
    float* op = gx + (size_t)i * kNC + c;
#pragma unroll
    for (int m = 0; m < 9; ++m) op[m * st] = gf[m];
  }
  float* pp = part + (size_t)blockIdx.x * 4 * kNC + c;
  pp[0] = aw[0];
  pp[kNC] = aw[1];
  pp[2 * kNC] = aw[2];
  pp[3 * kNC] = ab;
}

__global__ __launch_bounds__(256) void k_rmsnorm_bwd2(const float* __restrict__ x, const float* __restrict__ w,
                                                      const float* __restrict__ gy, const float* __restrict__ qx,
                                                      const float* __restrict__ qw, const float* __restrict__ qb,
                                                      float* __restrict__ dgy, float* __restrict__ dx,
                                                      float* __restrict__ part, int n, float eps) {
  __shared__ float red[4 * 4];
  const int c = threadIdx.x;
  const size_t st = (size_t)n * kNC;
  float wc[3], qwc[3], aw[3] = {0.f, 0.f, 0.f};
#pragma unroll
  for (int l = 0; l < 3; ++l) {
    wc[l] = w[l * kNC + c];
    qwc[l] = qw ? qw[l * kNC + c] : 0.f;
  }
  const float qbc = qb ? qb[c] : 0.f;
  for (int i = blockIdx.x; i < n; i += gridDim.x) {
    const size_t base = (size_t)i * kNC + c;
    float f[9], g[9], q[9];
#pragma unroll
    for (int m = 0; m < 9; ++m) {
      f[m] = x[base + m * st];
      g[m] = gy[base + m * st];
      q[m] = qx ? qx[base + m * st] : 0.f;
    }
    float mv[2] = {f[0], q[0]};
    block_sums256<2>(mv, red);
    f[0] -= mv[0] * (1.0f / kNC);
    q[0] -= mv[1] * (1.0f / kNC);
    float sv[4] = {0.f, 0.f, 0.f, 0.f};   // S, then A, B, G, T
    float ss = 0.f;
#pragma unroll
    for (int m = 0; m < 9; ++m) {
      const int l = lof(m);
      const float P = g[m] * wc[l];
      ss = fmaf(bal(m), f[m] * f[m], ss);
      sv[0] = fmaf(q[m], P, sv[0]);
      sv[1] = fmaf(q[m] * bal(m), f[m], sv[1]);
      sv[2] = fmaf(P, f[m], sv[2]);
      sv[3] = fmaf(g[m] * qwc[l], f[m], sv[3]);
    }
    block_sums256<4>(sv, red);
    const float S = block_sum256(ss, red) * (1.0f / kNC);
    const float r = 1.0f / sqrtf(S + eps);
    const float A = sv[0], B = sv[1], G = sv[2], T = sv[3];
    const float k3 = r * r * r * (1.0f / kNC);
    const float dLdr = A - 3.0f * r * r * (1.0f / kNC) * G * B + T;
    float Gf[9];
#pragma unroll
    for (int m = 0; m < 9; ++m) {
      const int l = lof(m);
      const float P = g[m] * wc[l];
      const float u = r * q[m] - k3 * B * f[m];
      dgy[base + m * st] = wc[l] * u + r * qwc[l] * f[m] + (m == 0 ? qbc : 0.f);
      aw[l] = fmaf(g[m], u, aw[l]);
      Gf[m] = -k3 * (P * B + G * q[m] * bal(m)) + r * g[m] * qwc[l] - dLdr * k3 * bal(m) * f[m];
    }
    const float gm0 = block_sum256(Gf[0], red) * (1.0f / kNC);
    Gf[0] -= gm0;
#pragma unroll
    for (int m = 0; m < 9; ++m) dx[base + m * st] = Gf[m];
  }
  float* pp = part + (size_t)blockIdx.x * 3 * kNC + c;
  pp[0] = aw[0];
  pp[kNC] = aw[1];
  pp[2 * kNC] = aw[2];
}

}  // namespace e2v2

using namespace e2v2;

E2V2_API int e2v2_gate_bwd2(const float* sc, const float* x, const float* gy, const float* qsc, const float* qx,
                            float* dgy, float* dsc, float* dx, int n, float k1, float k2, hipStream_t s) {
  E2V2_REQUIRE(n >= 0, "gate_bwd2: n %d", n);
  if (n == 0) return 0;
  const int64_t tot = (int64_t)n * e2v2::kNC;
  hipLaunchKernelGGL(e2v2::k_gate_bwd2, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s, sc, x, gy, qsc, qx, dgy,
                     dsc, dx, n, k1, k2);
  E2V2_LAUNCHED("k_gate_bwd2");
  return 0;
}

E2V2_API int e2v2_rmsnorm_bwd_param(const float* x, const float* w, const float* gy, float* gx, float* part, int n,
                                    int n_part, float eps, hipStream_t s) {
  E2V2_REQUIRE(n >= 0 && n_part > 0 && n_part <= 65535, "rmsnorm_bwd_param: n %d, n_part %d", n, n_part);
  hipLaunchKernelGGL(e2v2::k_rmsnorm_bwd_param, dim3((unsigned)n_part), dim3(256), 0, s, x, w, gy, gx, part, n, eps);
  E2V2_LAUNCHED("k_rmsnorm_bwd_param");
  return 0;
}

E2V2_API int e2v2_rmsnorm_bwd2(const float* x, const float* w, const float* gy, const float* qx, const float* qw,
                               const float* qb, float* dgy, float* dx, float* part, int n, int n_part, float eps,
                               hipStream_t s) {
  E2V2_REQUIRE(n >= 0 && n_part > 0 && n_part <= 65535, "rmsnorm_bwd2: n %d, n_part %d", n, n_part);
  hipLaunchKernelGGL(e2v2::k_rmsnorm_bwd2, dim3((unsigned)n_part), dim3(256), 0, s, x, w, gy, qx, qw, qb, dgy, dx,
                     part, n, eps);
  E2V2_LAUNCHED("k_rmsnorm_bwd2");
  return 0;
}

E2V2_API int e2v2_rmsnorm_fwd(const float* x, const float* w, const float* b, float* y, int n, float eps,
                              hipStream_t s) {
  return e2v2_add_rmsnorm_fwd(x, nullptr, w, b, nullptr, y, n, eps, s);
}

E2V2_API int e2v2_add_rmsnorm_fwd(const float* x, const float* delta, const float* w, const float* b, float* xs,
                                  float* y, int n, float eps, hipStream_t s) {
  E2V2_REQUIRE(!delta || xs, "add_rmsnorm_fwd: the sum x + delta needs an output buffer");
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_rmsnorm_fwd, dim3(n), dim3(256), 0, s, x, delta, w, b, xs, y, n, eps);
  E2V2_LAUNCHED("k_rmsnorm_fwd");
  return 0;
}

E2V2_API int e2v2_rmsnorm_bwd(const float* x, const float* w, const float* gy, const float* gres, float* gx,
                              int n, float eps, hipStream_t s) {
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_rmsnorm_bwd, dim3(n), dim3(256), 0, s, x, w, gy, gres, gx, n, eps);
  E2V2_LAUNCHED("k_rmsnorm_bwd");
  return 0;
}

E2V2_API int e2v2_gate_fwd(const float* sc, const float* x, float* y, int n, float k1, float k2, hipStream_t s) {
  if (n == 0) return 0;
  const int64_t tot = (int64_t)n * kNC;
  hipLaunchKernelGGL(k_gate_fwd, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s, sc, x, y, n, k1, k2);
  E2V2_LAUNCHED("k_gate_fwd");
  return 0;
}

E2V2_API int e2v2_gate_bwd(const float* sc, const float* x, const float* gy, float* gsc, float* gx, int n, float k1,
                           float k2, hipStream_t s) {
  if (n == 0) return 0;
  const int64_t tot = (int64_t)n * kNC;
  hipLaunchKernelGGL(k_gate_bwd, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s, sc, x, gy, gsc, gx, n, k1, k2);
  E2V2_LAUNCHED("k_gate_bwd");
  return 0;
}

// ---- Q/K scalarisation of SO3_Linear2Scalar_e2former (module_utils.py:2241-2266):
// y [9][N][4*hid] holds (q_a, q_b, k_a, k_b) of the fused projection; for X in {q, k}:
//   h_X[n][l*hid + c] = sum_{m in l} X_a[m][n][c] * X_b[m][n][c]        -> hq, hk [N][3*hid]
namespace e2v2 {
__global__ void k_pairdot_fwd(const float* __restrict__ y, float* __restrict__ hq, float* __restrict__ hk, int n,
                              int hid) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)n * hid) return;
  const int i = (int)(idx / hid), c = (int)(idx % hid);
  const size_t st = (size_t)n * 4 * hid;
  const float* p = y + (size_t)i * 4 * hid + c;
  float q[3] = {0.f, 0.f, 0.f}, k[3] = {0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < 9; ++m) {
    const int l = m == 0 ? 0 : (m < 4 ? 1 : 2);
    const float* r = p + m * st;
    q[l] = fmaf(r[0], r[hid], q[l]);
    k[l] = fmaf(r[2 * hid], r[3 * hid], k[l]);
  }
#pragma unroll
  for (int l = 0; l < 3; ++l) {
    hq[(size_t)i * 3 * hid + l * hid + c] = q[l];
    hk[(size_t)i * 3 * hid + l * hid + c] = k[l];
  }
}

__global__ void k_pairdot_bwd(const float* __restrict__ y, const float* __restrict__ ghq,
                              const float* __restrict__ ghk, float* __restrict__ gy, int n, int hid) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)n * hid) return;
  const int i = (int)(idx / hid), c = (int)(idx % hid);
  const size_t st = (size_t)n * 4 * hid;
  const float* p = y + (size_t)i * 4 * hid + c;
  float* g = gy + (size_t)i * 4 * hid + c;
  float gq[3], gk[3];
#pragma unroll
  for (int l = 0; l < 3; ++l) {
    gq[l] = ghq[(size_t)i * 3 * hid + l * hid + c];
    gk[l] = ghk[(size_t)i * 3 * hid + l * hid + c];
  }
#pragma unroll
  for (int m = 0; m < 9; ++m) {
    const int l = m == 0 ? 0 : (m < 4 ? 1 : 2);
    const float* r = p + m * st;
    float* o = g + m * st;
    const float qa = r[0], qb = r[hid], ka = r[2 * hid], kb = r[3 * hid];
    o[0] = gq[l] * qb;
    o[hid] = gq[l] * qa;
    o[2 * hid] = gk[l] * kb;
    o[3 * hid] = gk[l] * ka;
  }
}
}  // namespace e2v2

E2V2_API int e2v2_pairdot_fwd(const float* y, float* hq, float* hk, int n, int hid, hipStream_t s) {
  if (n == 0) return 0;
  const int64_t tot = (int64_t)n * hid;
  hipLaunchKernelGGL(e2v2::k_pairdot_fwd, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s, y, hq, hk, n, hid);
  E2V2_LAUNCHED("k_pairdot_fwd");
  return 0;
}

E2V2_API int e2v2_pairdot_bwd(const float* y, const float* ghq, const float* ghk, float* gy, int n, int hid,
                              hipStream_t s) {
  if (n == 0) return 0;
  const int64_t tot = (int64_t)n * hid;
  hipLaunchKernelGGL(e2v2::k_pairdot_bwd, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, s, y, ghq, ghk, gy, n,
                     hid);
  E2V2_LAUNCHED("k_pairdot_bwd");
  return 0;
}

// ---- LayerNorm + SiLU of the Q/K head (final_linear of SO3_Linear2Scalar_e2former,
// module_utils.py:2230-2233,2268): y = silu(LN(x) * g + b) on rows x[N][w], one
// wavefront per row (w a multiple of 64, at most 1024: w / 64 values per lane).
// The forward keeps (mean, rstd) per row; the backward recomputes the rest.
namespace e2v2 {
constexpr int kLnMaxPerLane = 16;

__global__ __launch_bounds__(256) void k_ln_silu_fwd(const float* __restrict__ x, const float* __restrict__ g,
                                                     const float* __restrict__ b, float* __restrict__ y,
                                                     float* __restrict__ stats, int n, int w, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (row >= n) return;
  const int nq = w >> 6;
  const float* xr = x + (size_t)row * w;
  float v[kLnMaxPerLane];
  float s = 0.f;
#pragma unroll
  for (int q = 0; q < kLnMaxPerLane; ++q) {
    v[q] = q < nq ? xr[q * 64 + lane] : 0.f;
    s += v[q];
  }
  const float mean = wave_sum(s) / (float)w;
  float s2 = 0.f;
#pragma unroll
  for (int q = 0; q < kLnMaxPerLane; ++q) {
    const float d = q < nq ? v[q] - mean : 0.f;
    s2 = fmaf(d, d, s2);
  }
  const float rstd = 1.0f / sqrtf(wave_sum(s2) / (float)w + eps);
  float* yr = y + (size_t)row * w;
#pragma unroll
  for (int q = 0; q < kLnMaxPerLane; ++q) {
    if (q < nq) {
      const int c = q * 64 + lane;
      const float a = (v[q] - mean) * rstd * g[c] + b[c];
      yr[c] = a / (1.0f + expf(-a));
    }
  }
  if (lane == 0) {
    stats[2 * (size_t)row] = mean;
    stats[2 * (size_t)row + 1] = rstd;
  }
}

__global__ __launch_bounds__(256) void k_ln_silu_bwd(const float* __restrict__ x, const float* __restrict__ g,
                                                     const float* __restrict__ b, const float* __restrict__ stats,
                                                     const float* __restrict__ gy, float* __restrict__ gx, int n,
                                                     int w) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (row >= n) return;
  const int nq = w >> 6;
  const float mean = stats[2 * (size_t)row], rstd = stats[2 * (size_t)row + 1];
  const float* xr = x + (size_t)row * w;
  const float* gr = gy + (size_t)row * w;
  float nv[kLnMaxPerLane], dn[kLnMaxPerLane];
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int q = 0; q < kLnMaxPerLane; ++q) {
    nv[q] = 0.f;
    dn[q] = 0.f;
    if (q < nq) {
      const int c = q * 64 + lane;
      nv[q] = (xr[c] - mean) * rstd;
      const float a = nv[q] * g[c] + b[c];
      const float sg = 1.0f / (1.0f + expf(-a));
      dn[q] = gr[c] * sg * (1.0f + a * (1.0f - sg)) * g[c];
      s1 += dn[q];
      s2 = fmaf(dn[q], nv[q], s2);
    }
  }
  const float m1 = wave_sum(s1) / (float)w, m2 = wave_sum(s2) / (float)w;
  float* o = gx + (size_t)row * w;
#pragma unroll
  for (int q = 0; q < kLnMaxPerLane; ++q)
    if (q < nq) o[q * 64 + lane] = rstd * (dn[q] - m1 - nv[q] * m2);
}
}  // namespace e2v2

// ---- LayerNorm + SiLU of the RadialProfile nets on the training path
// (module_utils.py:2151-2178: Linear -> LayerNorm -> SiLU per hidden layer), where
// the forces are differentiated once more: the first-order pass also returns the
// affine parameters' gradients, and the second-order pass differentiates that
// first-order pass.  Per row (z = xh g + b, xh = (x - mean) rstd, s = sigmoid(z),
// s1 = silu'(z) = s (1 + z (1 - s)), s2 = silu''(z) = s (1 - s) (2 + z (1 - 2 s))):
//   first order   gz = gy s1, u = gz g, gx = rstd (u - <u> - xh <u xh>),
//                 dg = sum_rows gz xh, db = sum_rows gz;
//   second order  (upstream qx, qg, qb on gx, dg, db; <.> the row mean over w)
//                 A = rstd (qx - <qx> - xh <qx xh>), P = g A + qg xh + qb,
//                 dgy = P s1, Z = P gy s2, c = <u xh>, m = <qx xh>,
//                 R = sum qx (u - <u> - xh c),
//                 X = -rstd (c qx + m u) + qg gz + Z g,
//                 dx = rstd (X - <X> - xh <X xh>) - R rstd^2 xh / w,
//                 d(g) = sum_rows (gz A + Z xh), d(b) = sum_rows Z.
// One wavefront per row, rows strided over n_part blocks of 4 wavefronts; each
// block writes its parameter sums to row blockIdx.x of part_* [n_part][w] (summed
// over blocks by the caller: the order is fixed, so results repeat bitwise).
namespace e2v2 {
template <int NQ>
__device__ __forceinline__ void ln_block_partials(float (&acc_a)[NQ], float (&acc_b)[NQ], float* part_a,
                                                  float* part_b) {
  constexpr int W = NQ * 64;
  __shared__ float red[2][4][W];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    red[0][wave][q * 64 + lane] = acc_a[q];
    red[1][wave][q * 64 + lane] = acc_b[q];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 2 * W; i += 256) {
    const int k = i / W, c = i % W;
    const float v = ((red[k][0][c] + red[k][1][c]) + red[k][2][c]) + red[k][3][c];
    (k ? part_b : part_a)[(size_t)blockIdx.x * W + c] = v;
  }
}

template <int NQ>
__global__ __launch_bounds__(256) void k_ln_silu_bwd_param(const float* __restrict__ x, const float* __restrict__ g,
                                                           const float* __restrict__ b,
                                                           const float* __restrict__ stats,
                                                           const float* __restrict__ gy, float* __restrict__ gx,
                                                           float* __restrict__ part_g, float* __restrict__ part_b,
                                                           int n) {
  constexpr int W = NQ * 64;
  const int lane = threadIdx.x & 63;
  float gc[NQ], bc[NQ], ag[NQ], ab[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    gc[q] = g[q * 64 + lane];
    bc[q] = b[q * 64 + lane];
    ag[q] = 0.f;
    ab[q] = 0.f;
  }
  for (int row = blockIdx.x * 4 + (int)(threadIdx.x >> 6); row < n; row += gridDim.x * 4) {
    const float mean = stats[2 * (size_t)row], rstd = stats[2 * (size_t)row + 1];
    const float* xr = x + (size_t)row * W;
    const float* gr = gy + (size_t)row * W;
    float xh[NQ], u[NQ];
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int c = q * 64 + lane;
      xh[q] = (xr[c] - mean) * rstd;
      const float z = xh[q] * gc[q] + bc[q];
      const float sg = 1.0f / (1.0f + expf(-z));
      const float gz = gr[c] * sg * (1.0f + z * (1.0f - sg));
      ag[q] = fmaf(gz, xh[q], ag[q]);
      ab[q] += gz;
      u[q] = gz * gc[q];
      s1 += u[q];
      s2 = fmaf(u[q], xh[q], s2);
    }
    const float m1 = wave_sum(s1) / (float)W, m2 = wave_sum(s2) / (float)W;
    float* o = gx + (size_t)row * W;
#pragma unroll
    for (int q = 0; q < NQ; ++q) o[q * 64 + lane] = rstd * (u[q] - m1 - xh[q] * m2);
  }
  ln_block_partials<NQ>(ag, ab, part_g, part_b);
}

template <int NQ>
__global__ __launch_bounds__(256) void k_ln_silu_bwd2(const float* __restrict__ x, const float* __restrict__ g,
                                                      const float* __restrict__ b, const float* __restrict__ stats,
                                                      const float* __restrict__ gy, const float* __restrict__ qx,
                                                      const float* __restrict__ qg, const float* __restrict__ qb,
                                                      float* __restrict__ dgy, float* __restrict__ dx,
                                                      float* __restrict__ part_g, float* __restrict__ part_b, int n) {
  constexpr int W = NQ * 64;
  constexpr float kInvW = 1.0f / (float)W;
  const int lane = threadIdx.x & 63;
  float gc[NQ], bc[NQ], qgc[NQ], qbc[NQ], ag[NQ], ab[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int c = q * 64 + lane;
    gc[q] = g[c];
    bc[q] = b[c];
    qgc[q] = qg ? qg[c] : 0.f;
    qbc[q] = qb ? qb[c] : 0.f;
    ag[q] = 0.f;
    ab[q] = 0.f;
  }
  for (int row = blockIdx.x * 4 + (int)(threadIdx.x >> 6); row < n; row += gridDim.x * 4) {
    const float mean = stats[2 * (size_t)row], rstd = stats[2 * (size_t)row + 1];
    const size_t base = (size_t)row * W;
    float xh[NQ], gz[NQ], u[NQ], qv[NQ], s1d[NQ], gzs2[NQ];
    float su = 0.f, sux = 0.f, sq = 0.f, sqx = 0.f, squ = 0.f;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int c = q * 64 + lane;
      xh[q] = (x[base + c] - mean) * rstd;
      const float z = xh[q] * gc[q] + bc[q];
      const float sg = 1.0f / (1.0f + expf(-z));
      const float gyv = gy[base + c];
      s1d[q] = sg * (1.0f + z * (1.0f - sg));
      gz[q] = gyv * s1d[q];
      gzs2[q] = gyv * (sg * (1.0f - sg) * (2.0f + z * (1.0f - 2.0f * sg)));
      u[q] = gz[q] * gc[q];
      qv[q] = qx ? qx[base + c] : 0.f;
      su += u[q];
      sux = fmaf(u[q], xh[q], sux);
      sq += qv[q];
      sqx = fmaf(qv[q], xh[q], sqx);
      squ = fmaf(qv[q], u[q], squ);
    }
    su = wave_sum(su);
    sux = wave_sum(sux);
    sq = wave_sum(sq);
    sqx = wave_sum(sqx);
    squ = wave_sum(squ);
    const float ubar = su * kInvW, c_ = sux * kInvW, qbar = sq * kInvW, m = sqx * kInvW;
    const float R = squ - ubar * sq - c_ * sqx;
    float X[NQ];
    float t1 = 0.f, t2 = 0.f;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int c = q * 64 + lane;
      const float A = rstd * (qv[q] - qbar - xh[q] * m);
      const float P = gc[q] * A + qgc[q] * xh[q] + qbc[q];
      dgy[base + c] = P * s1d[q];
      const float Z = P * gzs2[q];
      X[q] = -rstd * (c_ * qv[q] + m * u[q]) + qgc[q] * gz[q] + Z * gc[q];
      ag[q] += gz[q] * A + Z * xh[q];
      ab[q] += Z;
      t1 += X[q];
      t2 = fmaf(X[q], xh[q], t2);
    }
    const float mX = wave_sum(t1) * kInvW, mXx = wave_sum(t2) * kInvW;
    const float rr = R * rstd * rstd * kInvW;
#pragma unroll
    for (int q = 0; q < NQ; ++q) dx[base + q * 64 + lane] = rstd * (X[q] - mX - xh[q] * mXx) - rr * xh[q];
  }
  ln_block_partials<NQ>(ag, ab, part_g, part_b);
}

template <typename F>
int ln_width_dispatch(int w, F&& f) {
  switch (w) {
    case 64: return f(std::integral_constant<int, 1>{});
    case 128: return f(std::integral_constant<int, 2>{});
    case 192: return f(std::integral_constant<int, 3>{});
    case 256: return f(std::integral_constant<int, 4>{});
    case 384: return f(std::integral_constant<int, 6>{});
    case 512: return f(std::integral_constant<int, 8>{});
    default: return -1;
  }
}
}  // namespace e2v2

E2V2_API int e2v2_ln_silu_bwd_param(const float* x, const float* g, const float* b, const float* stats,
                                    const float* gy, float* gx, float* part_g, float* part_b, int n, int w,
                                    int n_part, hipStream_t s) {
  E2V2_REQUIRE(n >= 0 && n_part > 0 && n_part <= 65535, "ln_silu_bwd_param: n %d, n_part %d", n, n_part);
  const int rc = e2v2::ln_width_dispatch(w, [&](auto nq) {
    hipLaunchKernelGGL(e2v2::k_ln_silu_bwd_param<decltype(nq)::value>, dim3((unsigned)n_part), dim3(256), 0, s, x,
                       g, b, stats, gy, gx, part_g, part_b, n);
    return 0;
  });
  E2V2_REQUIRE(rc == 0, "ln_silu_bwd_param: width %d (64, 128, 192, 256, 384 or 512)", w);
  E2V2_LAUNCHED("k_ln_silu_bwd_param");
  return 0;
}

E2V2_API int e2v2_ln_silu_bwd2(const float* x, const float* g, const float* b, const float* stats, const float* gy,
                               const float* qx, const float* qg, const float* qb, float* dgy, float* dx,
                               float* part_g, float* part_b, int n, int w, int n_part, hipStream_t s) {
  E2V2_REQUIRE(n >= 0 && n_part > 0 && n_part <= 65535, "ln_silu_bwd2: n %d, n_part %d", n, n_part);
  const int rc = e2v2::ln_width_dispatch(w, [&](auto nq) {
    hipLaunchKernelGGL(e2v2::k_ln_silu_bwd2<decltype(nq)::value>, dim3((unsigned)n_part), dim3(256), 0, s, x, g, b,
                       stats, gy, qx, qg, qb, dgy, dx, part_g, part_b, n);
    return 0;
  });
  E2V2_REQUIRE(rc == 0, "ln_silu_bwd2: width %d (64, 128, 192, 256, 384 or 512)", w);
  E2V2_LAUNCHED("k_ln_silu_bwd2");
  return 0;
}

E2V2_API int e2v2_ln_silu_fwd(const float* x, const float* g, const float* b, float* y, float* stats, int n, int w,
                              float eps, hipStream_t s) {
  E2V2_REQUIRE(w > 0 && w % 64 == 0 && w <= 64 * e2v2::kLnMaxPerLane, "ln_silu_fwd: width %d", w);
  if (n == 0) return 0;
  hipLaunchKernelGGL(e2v2::k_ln_silu_fwd, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, x, g, b, y, stats, n, w,
                     eps);
  E2V2_LAUNCHED("k_ln_silu_fwd");
  return 0;
}

E2V2_API int e2v2_ln_silu_bwd(const float* x, const float* g, const float* b, const float* stats, const float* gy,
                              float* gx, int n, int w, hipStream_t s) {
  E2V2_REQUIRE(w > 0 && w % 64 == 0 && w <= 64 * e2v2::kLnMaxPerLane, "ln_silu_bwd: width %d", w);
  if (n == 0) return 0;
  hipLaunchKernelGGL(e2v2::k_ln_silu_bwd, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, x, g, b, stats, gy, gx, n,
                     w);
  E2V2_LAUNCHED("k_ln_silu_bwd");
  return 0;
}
