// Device-side evaluation of radial-profile tables (built by radial.hip).
//
// A RadialProfile over x_edge = [rbf(d), tgt[z_i], src[z_j]]
// (src/molfm/models/e2former/module_utils.py:2151-2178 with the GaussianSmearing
// basis of module_utils.py:1853-1869) is, for a fixed pair of atom types, a
// smooth function of the edge distance d alone.  The table holds, per type
// pair p = type(i) * n_types + type(j) and node n (d = n h, h a power of two),
// four rows of nc channels: h^k d^k f / dd^k for k = 0..3.  Values come from
// the quintic Hermite interpolant of rows 0..2 on the node interval, the
// derivative from the same interpolant of rows 1..3 (divided by h).
#pragma once
#include "common.h"

namespace e2v2 {

struct Hermite5 {
  float a0, a1, a2, b0, b1, b2;
};

// Quintic Hermite basis on t in [0, 1] for node values and h-, h^2-scaled
// first and second derivatives at both ends.
__device__ __forceinline__ Hermite5 hermite5(float t) {
  const float t2 = t * t, t3 = t2 * t, t4 = t3 * t, t5 = t4 * t;
  Hermite5 H;
  H.a0 = 1.f - 10.f * t3 + 15.f * t4 - 6.f * t5;
  H.a1 = t - 6.f * t3 + 8.f * t4 - 3.f * t5;
  H.a2 = 0.5f * (t2 - 3.f * t3 + 3.f * t4 - t5);
  H.b0 = 10.f * t3 - 15.f * t4 + 6.f * t5;
  H.b1 = -4.f * t3 + 7.f * t4 - 3.f * t5;
  H.b2 = 0.5f * (t3 - 2.f * t4 + t5);
  return H;
}

// Table of one kernel launch: tab [n_pairs][n_nodes][4][nc]; pair_slot [n_types^2] maps the type pair
// (a, b) = (query atom's type, source atom's type) to its table slot (NULL: slot a n_types + b, all pairs)
struct RadialTab {
  const float* tab;
  int32_t n_types, n_nodes, nc;
  float inv_h;   // 1 / h (exact: h is a power of two)
  const int32_t* pair_slot = nullptr;
};

// Table slot of the type pair (a, b).  The host builds a slot for every pair that an edge can join (the
// products of each graph's own type set); a pair without one (no such edge exists) reads slot 0.
__device__ __forceinline__ int tab_pair(const RadialTab& R, int a, int b) {
  const int ab = a * R.n_types + b;
  return R.pair_slot ? max(R.pair_slot[ab], 0) : ab;
}

// Offset (floats) of node n of the interval holding d for pair p, and the
// fraction t in [0, 1] (d / h, its floor and fraction are exact in fp32).
// u is clamped to [0, n_nodes - 2] (a NaN distance gives the last interval), so no
// distance reads outside the pair's nodes.
__device__ __forceinline__ int64_t radial_node(const RadialTab& R, int pair, float d, float& t) {
  const float u = fmaxf(fminf(d * R.inv_h, (float)(R.n_nodes - 2)), 0.0f);
  const float fn = floorf(u);
  t = u - fn;
  return ((int64_t)pair * R.n_nodes + (int64_t)fn) * (4 * R.nc);
}

// Offset (floats) of node n of the interval holding d for pair p in a slice-major
// table ([pairs][n_slices][nodes][4][w]) of slice `slice`, and the fraction t.
__device__ __forceinline__ int64_t radial_node_sliced(const RadialTab& R, int pair, int slice, int n_slices, int w,
                                                      float d, float& t) {
  const float u = fmaxf(fminf(d * R.inv_h, (float)(R.n_nodes - 2)), 0.0f);
  const float fn = floorf(u);
  t = u - fn;
  return (((int64_t)pair * n_slices + slice) * R.n_nodes + (int64_t)fn) * (4 * w);
}

// Interpolated value of channel c from its six node rows (f0, f1, f2 at n and at n + 1)
__device__ __forceinline__ float herm_value(const Hermite5& H, float f0, float f1, float f2, float g0, float g1,
                                            float g2) {
  return H.a0 * f0 + H.a1 * f1 + H.a2 * f2 + H.b0 * g0 + H.b1 * g1 + H.b2 * g2;
}

}  // namespace e2v2
