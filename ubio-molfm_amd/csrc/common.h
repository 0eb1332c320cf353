// Shared helpers for the e2v2 HIP library (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>
#include <math.h>

#define E2V2_API extern "C" __attribute__((visibility("default")))

namespace e2v2 {

int set_error(int code, const char* fmt, ...);
// ddv[e] = sum_s part[s][e].xyz, dd[e] = sum_s part[s][e].w over n_sl (<= 8) slices in slice order (deg.hip)
int launch_edge_part_sum(const float* part, int64_t n_edges, float* ddv, float* dd, hipStream_t st, int n_sl = 8);

#define E2V2_TRY_HIP(expr)                                                          \
  do {                                                                              \
    hipError_t e_ = (expr);                                                         \
    if (e_ != hipSuccess)                                                           \
      return ::e2v2::set_error((int)e_, "%s failed: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

#define E2V2_LAUNCHED(name)                                                         \
  do {                                                                              \
    hipError_t e_ = hipGetLastError();                                              \
    if (e_ != hipSuccess)                                                           \
      return ::e2v2::set_error((int)e_, "launch of %s failed: %s", name, hipGetErrorString(e_)); \
  } while (0)

#define E2V2_REQUIRE(cond, ...)                                                     \
  do {                                                                              \
    if (!(cond)) return ::e2v2::set_error(-1, __VA_ARGS__);                         \
  } while (0)

constexpr int kWave = 64;

typedef float floatx4 __attribute__((ext_vector_type(4)));

// The one fp32 distance expression shared with the CPU oracle:
// d = sqrt((dx*dx + dy*dy) + dz*dz), every op rounded to fp32 (no FMA
// contraction; __builtin_sqrtf is correctly rounded under HIP's default
// -fhip-fp32-correctly-rounded-divide-sqrt).
__device__ __forceinline__ float exact_dist(float dx, float dy, float dz) {
#pragma clang fp contract(off)
  float xx = dx * dx;
  float yy = dy * dy;
  float zz = dz * dz;
  float s = (xx + yy) + zz;
  return __builtin_sqrtf(s);
}

// img = pos_j + off; dv = pos_i - img (component-wise, rounded)
__device__ __forceinline__ void exact_edge(const float* pi, const float* pj, const float* off,
                                           float& dx, float& dy, float& dz) {
#pragma clang fp contract(off)
  float ix = pj[0] + off[0];
  float iy = pj[1] + off[1];
  float iz = pj[2] + off[2];
  dx = pi[0] - ix;
  dy = pi[1] - iy;
  dz = pi[2] - iz;
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Sum over each row of 16 lanes, left in every lane of the row, by four DPP
// steps (lane ^ 1, lane ^ 2 via quad permutes; ^ 7 within 8 and ^ 15 within
// 16 via the half-row and row mirrors) instead of LDS-crossbar shuffles.
template <int kCtrl>
__device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_row_sum16(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);  // row_half_mirror
  v += dpp_mov<0x140>(v);  // row_mirror
  return v;
}

// Workgroups are dispatched round-robin over the 8 XCDs of an MI355X (each with
// its own L2).  Give every XCD a contiguous range of rows so that spatially
// adjacent rows (atoms are Morton-ordered by the host) share one L2.
constexpr int kXcd = 8;
__host__ __device__ __forceinline__ int xcd_grid(int n) { return ((n + kXcd - 1) / kXcd) * kXcd; }
__device__ __forceinline__ int xcd_row(int b, int n) {
  const int per = (n + kXcd - 1) / kXcd;
  return (b % kXcd) * per + b / kXcd;
}

// Streaming (non-temporal) global accesses for data touched once per kernel:
// per-edge weights, row gradients, outputs.  They are marked for early L2
// eviction so the 4 MB L2 of each XCD keeps the neighbour features that
// many rows gather.
template <typename T>
__device__ __forceinline__ T ntload(const T* p) { return __builtin_nontemporal_load(p); }
template <typename T>
__device__ __forceinline__ void ntstore(T v, T* p) { __builtin_nontemporal_store(v, p); }

// Native transcendental instructions (v_exp_f32 = 2^x, v_rcp_f32, v_rsq_f32),
// one VALU op each and accurate to about 1 ulp, in place of the libm
// sequences (range reduction, IEEE division) that dominate the VALU budget of
// the per-edge MLP epilogues.  exp(x) = 2^(x log2 e): the rounding of the
// product adds |x| * 6e-8 relative error, below fp32 rounding of the inputs
// for the |x| < 20 that carry weight here.
constexpr float kLog2e = 1.4426950408889634f;
__device__ __forceinline__ float fexp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }
__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float frcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float frsq(float x) { return __builtin_amdgcn_rsqf(x); }

__device__ __forceinline__ float sigmoidf_(float x) { return frcp(1.0f + fexp(-x)); }
__device__ __forceinline__ float silu(float x) { return x * sigmoidf_(x); }

// e3nn's raw real spherical harmonics of degree <= 2 at a unit vector (x, y, z)
// (each l block of unit norm up to the l = 0 scale), as used by the edge-degree
// embedding (src/molfm/models/e2former/e2former.py:719-726).
__device__ __forceinline__ void raw_sh2(float x, float y, float z, float (&Y)[9]) {
  const float s3 = 1.7320508075688772f;
  Y[0] = 1.f;
  Y[1] = x; Y[2] = y; Y[3] = z;
  Y[4] = s3 * x * z;
  Y[5] = s3 * x * y;
  Y[6] = y * y - 0.5f * (x * x + z * z);
  Y[7] = s3 * y * z;
  Y[8] = s3 / 2.0f * (z * z - x * x);
}

// Distance envelope of the attention weights.  kind 0: the polynomial of exponent 5,
// p = 1 + r^5 (a + r (b + c r)), r = d / rc, 0 for r >= 1 (module_utils.py:1946-1954);
// kind 1: the smooth bell (1 - t^2)^2, t = (2 d - (lo + hi)) / (hi - lo) clamped to
// [-1, 1], hi = max(rc, lo + 1e-8) (module_utils.py:1956-1985, exponent 2).
struct Envelope {
  float rc, a, b, c;
  float lo = 0.f;   // lower end of the bell
  template <bool kBell = false>
  __device__ __forceinline__ void eval(float d, float& p, float& dp_dd) const {
    if constexpr (kBell) {
      const float hi = fmaxf(rc, lo + 1e-8f);
      const float t = (2.0f * d - (lo + hi)) / (hi - lo);
      if (t > -1.0f && t < 1.0f) {
        const float u = 1.0f - t * t;
        p = u * u;
        dp_dd = -8.0f * u * t / (hi - lo);
      } else {
        p = 0.0f;
        dp_dd = 0.0f;
      }
      return;
    }
    float r = d / rc;
    if (r < 1.0f) {
      float r2 = r * r, r4 = r2 * r2, r5 = r4 * r;
      p = 1.0f + r5 * (a + r * (b + c * r));
      dp_dd = r4 * (5.0f * a + r * (6.0f * b + 7.0f * c * r)) / rc;
    } else {
      p = 0.0f;
      dp_dd = 0.0f;
    }
  }
};

}  // namespace e2v2
