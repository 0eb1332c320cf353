// Radial profiles as distance tables, built in float64.
//
// RadialProfile [K0 + 2 E -> 128 -> LN -> SiLU -> 128 -> LN -> SiLU -> 256]
// (src/molfm/models/e2former/module_utils.py:2151-2178) applied to
// x_edge = [rbf(d), tgt[z_i], src[z_j]] (e2former.py:258-266 for fc_easy,
// e2former.py:709-733 for the degree embedding's gbf_projs) with the Gaussian
// basis rbf_k(d) = exp(coeff (d - mu_k)^2) (module_utils.py:1853-1869) is, for
// one pair of atom types, a function of the scalar distance d only.  Every
// (type pair, node d = n h) gets the truncated Taylor series of the profile
// output in delta = d - n h to third order, propagated exactly through each op
// in float64 ("jets": value and three derivatives), and stored as the rows
// h^k d^k f/dd^k, k = 0..3, of the table the edge kernels interpolate
// (quintic Hermite, radial.h).  e2v2_radial_table_check evaluates the profile
// at every interval midpoint and reports the interpolation error, so the host
// can halve h until the table meets its tolerance.
#include <cmath>

#include "common.h"
#include "radial.h"
#include "../../include/e2v2.h"

namespace e2v2 {

constexpr int kRH = 128;   // hidden width of the profiles
constexpr int kRO = 256;   // output width of one profile
constexpr int kNB = 256;   // Gaussian basis functions

struct Jet {
  double c[4];
};

__device__ __forceinline__ Jet jconst(double v) { return Jet{{v, 0.0, 0.0, 0.0}}; }

__device__ __forceinline__ Jet jmul(const Jet& a, const Jet& b) {
  Jet r;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    double s = 0.0;
#pragma unroll
    for (int j = 0; j <= k; ++j) s += a.c[j] * b.c[k - j];
    r.c[k] = s;
  }
  return r;
}

// y = exp(a): y' = y a'  ->  k y_k = sum_{j=1..k} j a_j y_{k-j}
__device__ __forceinline__ Jet jexp(const Jet& a) {
  Jet y;
  y.c[0] = exp(a.c[0]);
#pragma unroll
  for (int k = 1; k < 4; ++k) {
    double s = 0.0;
#pragma unroll
    for (int j = 1; j <= k; ++j) s += j * a.c[j] * y.c[k - j];
    y.c[k] = s / k;
  }
  return y;
}

// y = a^p: a y' = p a' y  ->  k a_0 y_k = sum_{j=1..k} (p j - (k - j)) a_j y_{k-j}
__device__ __forceinline__ Jet jpow(const Jet& a, double p) {
  Jet y;
  y.c[0] = pow(a.c[0], p);
#pragma unroll
  for (int k = 1; k < 4; ++k) {
    double s = 0.0;
#pragma unroll
    for (int j = 1; j <= k; ++j) s += (p * j - (k - j)) * a.c[j] * y.c[k - j];
    y.c[k] = s / (k * a.c[0]);
  }
  return y;
}

// silu(a) = a sigma(a); sigma' = sigma (1 - sigma) a'  ->  k s_k = sum_j j a_j u_{k-j}, u = s - s^2
__device__ __forceinline__ Jet jsilu(const Jet& a) {
  Jet s, u;
  const double a0 = a.c[0];
  s.c[0] = a0 >= 0.0 ? 1.0 / (1.0 + exp(-a0)) : exp(a0) / (1.0 + exp(a0));
  u.c[0] = s.c[0] - s.c[0] * s.c[0];
#pragma unroll
  for (int k = 1; k < 4; ++k) {
    double acc = 0.0;
#pragma unroll
    for (int j = 1; j <= k; ++j) acc += j * a.c[j] * u.c[k - j];
    s.c[k] = acc / k;
    double sq = 0.0;
#pragma unroll
    for (int j = 0; j <= k; ++j) sq += s.c[j] * s.c[k - j];
    u.c[k] = s.c[k] - sq;
  }
  return jmul(a, s);
}

// Sum over the 128 threads of the block, every order at once (fixed order).
__device__ __forceinline__ Jet block_sum128(Jet v, double (*red)[4]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int k = 0; k < 4; ++k) red[t][k] = v.c[k];
  __syncthreads();
  for (int s = kRH / 2; s > 0; s >>= 1) {
    if (t < s) {
#pragma unroll
      for (int k = 0; k < 4; ++k) red[t][k] += red[t + s][k];
    }
    __syncthreads();
  }
  Jet r;
#pragma unroll
  for (int k = 0; k < 4; ++k) r.c[k] = red[0][k];
  __syncthreads();
  return r;
}

// LayerNorm(128) with affine (g, b), eps 1e-5, of this thread's channel
__device__ __forceinline__ Jet jlayernorm(const Jet& x, double g, double b, double (*red)[4]) {
  Jet mean = block_sum128(x, red);
#pragma unroll
  for (int k = 0; k < 4; ++k) mean.c[k] *= 1.0 / kRH;
  Jet u;
#pragma unroll
  for (int k = 0; k < 4; ++k) u.c[k] = x.c[k] - mean.c[k];
  Jet var = block_sum128(jmul(u, u), red);
#pragma unroll
  for (int k = 0; k < 4; ++k) var.c[k] *= 1.0 / kRH;
  var.c[0] += 1e-5;
  const Jet r = jpow(var, -0.5);
  Jet n = jmul(u, r);
#pragma unroll
  for (int k = 0; k < 4; ++k) n.c[k] *= g;
  n.c[0] += b;
  return n;
}

// Output jets of one profile at d = d0 (type pair (ta, tb)) for channels t and t + 128, and hid, the jet of
// hidden channel t (the second SiLU's output, the last Linear's input).
__device__ void profile_jets(const e2v2_radial_net& W, const float* __restrict__ mu, double coeff, int za, int zb,
                             double d0, Jet (&out)[2], Jet& hid) {
  __shared__ double rbf_s[kNB][4];
  __shared__ double hid_s[kRH][4];
  __shared__ double red[kRH][4];
  const int t = threadIdx.x;
  for (int k = t; k < kNB; k += kRH) {   // rbf_k(d0 + delta) = exp(coeff (x + delta)^2), x = d0 - mu_k
    const double x = d0 - (double)mu[k];
    const Jet a{{coeff * x * x, 2.0 * coeff * x, coeff, 0.0}};
    const Jet y = jexp(a);
#pragma unroll
    for (int q = 0; q < 4; ++q) rbf_s[k][q] = y.c[q];
  }
  __syncthreads();
  // Linear1: rbf block + the constant type blocks and bias
  const float* w1 = W.w1 + (size_t)t * W.ld_w1;
  Jet z = jconst((double)W.b1[t]);
  for (int k = 0; k < kNB; ++k) {
    const double w = (double)w1[k];
#pragma unroll
    for (int q = 0; q < 4; ++q) z.c[q] += w * rbf_s[k][q];
  }
  const float* tg = W.tgt + (size_t)za * W.n_emb;
  const float* sr = W.src + (size_t)zb * W.n_emb;
  double cst = 0.0;
  for (int e = 0; e < W.n_emb; ++e)
    cst += (double)w1[kNB + e] * (double)tg[e] + (double)w1[kNB + W.n_emb + e] * (double)sr[e];
  z.c[0] += cst;
  Jet s1 = jsilu(jlayernorm(z, (double)W.g1[t], (double)W.be1[t], red));
#pragma unroll
  for (int q = 0; q < 4; ++q) hid_s[t][q] = s1.c[q];
  __syncthreads();
  // Linear2
  const float* w2 = W.w2 + (size_t)t * kRH;
  z = jconst((double)W.b2[t]);
  for (int j = 0; j < kRH; ++j) {
    const double w = (double)w2[j];
#pragma unroll
    for (int q = 0; q < 4; ++q) z.c[q] += w * hid_s[j][q];
  }
  __syncthreads();
  const Jet s2 = jsilu(jlayernorm(z, (double)W.g2[t], (double)W.be2[t], red));
  hid = s2;
#pragma unroll
  for (int q = 0; q < 4; ++q) hid_s[t][q] = s2.c[q];
  __syncthreads();
  // Linear3: outputs t and t + 128
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int o = t + h * kRH;
    const float* w3 = W.w3 + (size_t)o * kRH;
    Jet y = jconst((double)W.b3[o]);
    for (int j = 0; j < kRH; ++j) {
      const double w = (double)w3[j];
#pragma unroll
      for (int q = 0; q < 4; ++q) y.c[q] += w * hid_s[j][q];
    }
    out[h] = y;
  }
  __syncthreads();
}

// Table position of output channel o of a profile (e2v2_radial_layout)
__device__ __forceinline__ int layout_pos(const e2v2_radial_layout& Lo, int o) {
  return Lo.col0 + ((o % Lo.split) / Lo.block) * Lo.block_stride + (o / Lo.split) * Lo.split_stride + o % Lo.block;
}
// Index of (pair p, node n, row k, channel position pos) in a table of nc positions per row
__device__ __forceinline__ int64_t tab_index(const e2v2_radial_layout& Lo, int p, int n_nodes, int n, int k, int nc,
                                             int pos) {
  if (Lo.slice_width == 0) return (((int64_t)p * n_nodes + n) * 4 + k) * nc + pos;
  const int w = Lo.slice_width, ns = nc / w;
  return ((((int64_t)p * ns + pos / w) * n_nodes + n) * 4 + k) * w + pos % w;
}

// Rows h^k f^(k) = h^k k! c_k of the jets
__device__ __forceinline__ void jet_rows(const Jet& y, double h, double (&r)[4]) {
  r[0] = y.c[0];
  r[1] = h * y.c[1];
  r[2] = h * h * 2.0 * y.c[2];
  r[3] = h * h * h * 6.0 * y.c[3];
}

// one block per (node, pair); writes the profile's 256 output channels (kHid: its 128 hidden channels, the last
// Linear's input) of rows k = 0..3 at their layout positions (pair slot p holds the type pair
// pair_ab[p] = a n_types + b; pair_ab NULL: p itself)
template <bool kHid>
__global__ __launch_bounds__(kRH) void k_radial_table(e2v2_radial_net W, const float* __restrict__ mu, double coeff,
                                                      const int32_t* __restrict__ type_z, int n_types,
                                                      const int32_t* __restrict__ pair_ab, int n_nodes,
                                                      double h, float* __restrict__ tab, int nc,
                                                      e2v2_radial_layout Lo) {
  const int n = blockIdx.x, p = blockIdx.y;
  const int ab = pair_ab ? pair_ab[p] : p;
  const int za = type_z[ab / n_types], zb = type_z[ab % n_types];
  Jet y[2], hid;
  profile_jets(W, mu, coeff, za, zb, (double)n * h, y, hid);
#pragma unroll
  for (int hh = 0; hh < (kHid ? 1 : 2); ++hh) {
    double r[4];
    jet_rows(kHid ? hid : y[hh], h, r);
    const int o = layout_pos(Lo, threadIdx.x + hh * kRH);
#pragma unroll
    for (int k = 0; k < 4; ++k) tab[tab_index(Lo, p, n_nodes, n, k, nc, o)] = (float)r[k];
  }
}

// Interpolation error at the midpoint of every node interval: err[0] = max |f - f~|,
// err[1] = max |f|, err[2] = max h |f' - f~'|, err[3] = max h |f'| (float bits; non-negative
// floats order like their bit patterns, so the unsigned atomic max is exact and deterministic).
// kHid: the table holds the hidden channels; the error is that of the profile's output formed from them,
// f~ = W3 h~ + b3 (in float64 from the fp32 interpolants h~, h~'), against the float64 output.
template <bool kHid>
__global__ __launch_bounds__(kRH) void k_radial_check(e2v2_radial_net W, const float* __restrict__ mu, double coeff,
                                                      const int32_t* __restrict__ type_z, int n_types,
                                                      const int32_t* __restrict__ pair_ab, int n_nodes,
                                                      double h, const float* __restrict__ tab, int nc,
                                                      e2v2_radial_layout Lo, uint32_t* __restrict__ err) {
  __shared__ float hv_s[kRH], hd_s[kRH];
  const int n = blockIdx.x, p = blockIdx.y;
  const int ab = pair_ab ? pair_ab[p] : p;
  const int za = type_z[ab / n_types], zb = type_z[ab % n_types];
  Jet y[2], hid;
  profile_jets(W, mu, coeff, za, zb, ((double)n + 0.5) * h, y, hid);
  const Hermite5 H = hermite5(0.5f);
  if constexpr (kHid) {
    const int o = layout_pos(Lo, threadIdx.x);
    float a[4], b[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      a[k] = tab[tab_index(Lo, p, n_nodes, n, k, nc, o)];
      b[k] = tab[tab_index(Lo, p, n_nodes, n + 1, k, nc, o)];
    }
    hv_s[threadIdx.x] = herm_value(H, a[0], a[1], a[2], b[0], b[1], b[2]);
    hd_s[threadIdx.x] = herm_value(H, a[1], a[2], a[3], b[1], b[2], b[3]);
    __syncthreads();
  }
  float e_v = 0.f, m_v = 0.f, e_d = 0.f, m_d = 0.f;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    float v, dv;
    if constexpr (kHid) {
      const int oc = threadIdx.x + hh * kRH;
      const float* w3 = W.w3 + (size_t)oc * kRH;
      double sv = (double)W.b3[oc], sd = 0.0;
      for (int j = 0; j < kRH; ++j) {
        sv += (double)w3[j] * (double)hv_s[j];
        sd += (double)w3[j] * (double)hd_s[j];
      }
      v = (float)sv;
      dv = (float)sd;
    } else {
      const int o = layout_pos(Lo, threadIdx.x + hh * kRH);
      float a[4], b[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        a[k] = tab[tab_index(Lo, p, n_nodes, n, k, nc, o)];
        b[k] = tab[tab_index(Lo, p, n_nodes, n + 1, k, nc, o)];
      }
      v = herm_value(H, a[0], a[1], a[2], b[0], b[1], b[2]);
      dv = herm_value(H, a[1], a[2], a[3], b[1], b[2], b[3]);
    }
    e_v = fmaxf(e_v, (float)fabs((double)v - y[hh].c[0]));
    m_v = fmaxf(m_v, (float)fabs(y[hh].c[0]));
    e_d = fmaxf(e_d, (float)fabs((double)dv - h * y[hh].c[1]));
    m_d = fmaxf(m_d, (float)fabs(h * y[hh].c[1]));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    e_v = fmaxf(e_v, __shfl_xor(e_v, o, kWave));
    m_v = fmaxf(m_v, __shfl_xor(m_v, o, kWave));
    e_d = fmaxf(e_d, __shfl_xor(e_d, o, kWave));
    m_d = fmaxf(m_d, __shfl_xor(m_d, o, kWave));
  }
  if ((threadIdx.x & (kWave - 1)) == 0) {
    atomicMax(err + 0, __float_as_uint(e_v));
    atomicMax(err + 1, __float_as_uint(m_v));
    atomicMax(err + 2, __float_as_uint(e_d));
    atomicMax(err + 3, __float_as_uint(m_d));
  }
}

// Per-edge evaluation of a plain-layout table ([pairs][nodes][4][nc]): one
// wavefront per edge, lanes over channels.  The forward interpolates rows 0..2
// (values), the backward rows 1..3 (h-scaled derivatives) and sums
// grad[e][c] f_c'(d) over the channels in a fixed order (lane partials, then a
// butterfly), so the result does not depend on the launch.  e_end (NULL: n_edges)
// bounds the edges on the device: in a capacity build the slots from row_ptr[n_rows]
// on hold no edge (their row, column and distance were never written), and they
// get zeros without reading them.
constexpr int kEvWaves = 4;

__device__ __forceinline__ bool past_end(int64_t e, const int32_t* __restrict__ e_end) {
  return e_end != nullptr && e >= (int64_t)*e_end;
}

__global__ __launch_bounds__(64 * kEvWaves) void k_radial_eval(RadialTab R, const int32_t* __restrict__ atom_type,
                                                               const int32_t* __restrict__ edge_row,
                                                               const int32_t* __restrict__ col,
                                                               const float* __restrict__ dist, int64_t n_edges,
                                                               const int32_t* __restrict__ e_end,
                                                               float* __restrict__ out) {
  const int64_t e = (int64_t)blockIdx.x * kEvWaves + (threadIdx.x >> 6);
  if (e >= n_edges) return;
  const int lane = threadIdx.x & 63;
  if (past_end(e, e_end)) {
    for (int c = lane; c < R.nc; c += 64) out[e * R.nc + c] = 0.f;
    return;
  }
  const int pair = tab_pair(R, atom_type[edge_row[e]], atom_type[col[e]]);
  float t;
  const float* a = R.tab + radial_node(R, pair, dist[e], t);
  const float* b = a + 4 * R.nc;
  const Hermite5 H = hermite5(t);
  const int nc = R.nc;
  for (int c = lane; c < nc; c += 64)
    out[e * nc + c] = herm_value(H, a[c], a[nc + c], a[2 * nc + c], b[c], b[nc + c], b[2 * nc + c]);
}

__global__ __launch_bounds__(64 * kEvWaves) void k_radial_eval_bwd(RadialTab R, const int32_t* __restrict__ atom_type,
                                                                   const int32_t* __restrict__ edge_row,
                                                                   const int32_t* __restrict__ col,
                                                                   const float* __restrict__ dist, int64_t n_edges,
                                                                   const int32_t* __restrict__ e_end,
                                                                   const float* __restrict__ grad,
                                                                   float* __restrict__ ddist) {
  const int64_t e = (int64_t)blockIdx.x * kEvWaves + (threadIdx.x >> 6);
  if (e >= n_edges) return;
  const int lane = threadIdx.x & 63;
  if (past_end(e, e_end)) {
    if (lane == 0) ddist[e] = 0.f;
    return;
  }
  const int pair = tab_pair(R, atom_type[edge_row[e]], atom_type[col[e]]);
  float t;
  const float* a = R.tab + radial_node(R, pair, dist[e], t);
  const float* b = a + 4 * R.nc;
  const Hermite5 H = hermite5(t);
  const int nc = R.nc;
  float acc = 0.f;
  for (int c = lane; c < nc; c += 64)
    acc = fmaf(grad[e * nc + c],
               herm_value(H, a[nc + c], a[2 * nc + c], a[3 * nc + c], b[nc + c], b[2 * nc + c], b[3 * nc + c]), acc);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, kWave);
  if (lane == 0) ddist[e] = acc * R.inv_h;
}

}  // namespace e2v2

using namespace e2v2;

static int check_net(const e2v2_radial_net* W, const char* who) {
  E2V2_REQUIRE(W && W->w1 && W->b1 && W->g1 && W->be1 && W->w2 && W->b2 && W->g2 && W->be2 && W->w3 && W->b3 &&
                   W->tgt && W->src,
               "%s: incomplete radial profile weights", who);
  E2V2_REQUIRE(W->n_emb > 0 && W->ld_w1 == kNB + 2 * W->n_emb,
               "%s: Linear1 must read [rbf(256) | tgt(n_emb) | src(n_emb)] (ld_w1 %d, n_emb %d)", who, W->ld_w1,
               W->n_emb);
  return 0;
}

E2V2_API int e2v2_radial_table_size(float rc, float rbf_coeff, int32_t refine, int32_t* n_nodes, float* h) {
  E2V2_REQUIRE(rc > 0.f && rbf_coeff < 0.f && n_nodes && h && refine >= -3 && refine <= 6,
               "radial_table_size: need rc > 0, rbf_coeff < 0, -3 <= refine <= 6");
  const double sigma = std::sqrt(-0.5 / (double)rbf_coeff);
  const double hh = std::ldexp(1.0, (int)std::floor(std::log2(0.2 * sigma)) - refine);
  const double n = std::floor((double)rc / hh) + 2.0;
  E2V2_REQUIRE(n <= 1 << 20, "radial_table_size: %.0f nodes (rc %g, width %g) is too many", n, (double)rc, sigma);
  *n_nodes = (int32_t)n;
  *h = (float)hh;
  return 0;
}

// Every channel of the profile (n_ch: its 256 outputs or 128 hidden channels) lands inside the row, at a
// distinct position.
static int check_layout(const e2v2_radial_layout* Lo, int32_t nc, const char* who, int n_ch = kRO) {
  E2V2_REQUIRE(Lo, "%s: no channel layout", who);
  E2V2_REQUIRE(nc >= n_ch && nc <= 4 * kRO && Lo->split >= 1 && n_ch % Lo->split == 0 && Lo->block >= 1 &&
                   Lo->split % Lo->block == 0 && Lo->col0 >= 0 && Lo->block_stride >= 0 && Lo->split_stride >= 0 &&
                   Lo->slice_width >= 0 && (Lo->slice_width == 0 || nc % Lo->slice_width == 0),
               "%s: bad channel layout (nc %d, col0 %d, split %d, block %d, slice width %d)", who, nc, Lo->col0,
               Lo->split, Lo->block, Lo->slice_width);
  uint64_t used[4 * kRO / 64] = {};
  for (int o = 0; o < n_ch; ++o) {
    const int64_t p = (int64_t)Lo->col0 + (int64_t)((o % Lo->split) / Lo->block) * Lo->block_stride +
                      (int64_t)(o / Lo->split) * Lo->split_stride + o % Lo->block;
    E2V2_REQUIRE(p >= 0 && p < nc, "%s: channel %d maps to position %lld outside rows of %d", who, o, (long long)p,
                 nc);
    E2V2_REQUIRE(!((used[p / 64] >> (p % 64)) & 1), "%s: two channels map to position %lld", who, (long long)p);
    used[p / 64] |= 1ull << (p % 64);
  }
  return 0;
}

// pair slots: n_pairs of them, pair_ab [n_pairs] (device) the type pair a n_types + b of each, or NULL for all
// n_types^2 pairs in order
static int check_pairs(int32_t n_types, const int32_t* pair_ab, int32_t n_pairs, const char* who) {
  E2V2_REQUIRE(n_types >= 1 && n_types <= E2V2_MAX_TYPES, "%s: %d atom types (1 .. %d)", who, n_types,
               E2V2_MAX_TYPES);
  E2V2_REQUIRE(n_pairs >= 1 && n_pairs <= E2V2_MAX_PAIRS && (pair_ab || n_pairs == n_types * n_types),
               "%s: %d table pairs for %d types (1 .. %d; all n_types^2 without a pair list)", who, n_pairs, n_types,
               E2V2_MAX_PAIRS);
  return 0;
}

template <bool kHid>
static int radial_table_launch(const e2v2_radial_net* net, const float* rbf_offset, float rbf_coeff,
                               const int32_t* type_z, int32_t n_types, const int32_t* pair_ab, int32_t n_pairs,
                               int32_t n_nodes, float h, float* tab, int32_t nc, const e2v2_radial_layout* layout,
                               hipStream_t s, const char* who) {
  if (int rc = check_net(net, who)) return rc;
  if (int rc = check_pairs(n_types, pair_ab, n_pairs, who)) return rc;
  E2V2_REQUIRE(rbf_offset && type_z && tab && n_nodes >= 2 && h > 0.f, "%s: bad arguments (n_types %d, n_nodes %d)",
               who, n_types, n_nodes);
  if (int rc = check_layout(layout, nc, who, kHid ? kRH : kRO)) return rc;
  hipLaunchKernelGGL(k_radial_table<kHid>, dim3((unsigned)n_nodes, (unsigned)n_pairs), dim3(kRH), 0, s, *net,
                     rbf_offset, (double)rbf_coeff, type_z, n_types, pair_ab, n_nodes, (double)h, tab, nc, *layout);
  E2V2_LAUNCHED("k_radial_table");
  return 0;
}

template <bool kHid>
static int radial_check_launch(const e2v2_radial_net* net, const float* rbf_offset, float rbf_coeff,
                               const int32_t* type_z, int32_t n_types, const int32_t* pair_ab, int32_t n_pairs,
                               int32_t n_nodes, float h, const float* tab, int32_t nc,
                               const e2v2_radial_layout* layout, uint32_t* err, hipStream_t s, const char* who) {
  if (int rc = check_net(net, who)) return rc;
  if (int rc = check_pairs(n_types, pair_ab, n_pairs, who)) return rc;
  E2V2_REQUIRE(rbf_offset && type_z && tab && err && n_nodes >= 2, "%s: bad arguments", who);
  if (int rc = check_layout(layout, nc, who, kHid ? kRH : kRO)) return rc;
  hipLaunchKernelGGL(k_radial_check<kHid>, dim3((unsigned)(n_nodes - 1), (unsigned)n_pairs), dim3(kRH), 0, s,
                     *net, rbf_offset, (double)rbf_coeff, type_z, n_types, pair_ab, n_nodes, (double)h, tab, nc,
                     *layout, err);
  E2V2_LAUNCHED("k_radial_check");
  return 0;
}

E2V2_API int e2v2_radial_table(const e2v2_radial_net* net, const float* rbf_offset, float rbf_coeff,
                               const int32_t* type_z, int32_t n_types, const int32_t* pair_ab, int32_t n_pairs,
                               int32_t n_nodes, float h, float* tab, int32_t nc, const e2v2_radial_layout* layout,
                               hipStream_t s) {
  return radial_table_launch<false>(net, rbf_offset, rbf_coeff, type_z, n_types, pair_ab, n_pairs, n_nodes, h, tab,
                                    nc, layout, s, "radial_table");
}

E2V2_API int e2v2_radial_table_check(const e2v2_radial_net* net, const float* rbf_offset, float rbf_coeff,
                                     const int32_t* type_z, int32_t n_types, const int32_t* pair_ab, int32_t n_pairs,
                                     int32_t n_nodes, float h, const float* tab, int32_t nc,
                                     const e2v2_radial_layout* layout, uint32_t* err, hipStream_t s) {
  return radial_check_launch<false>(net, rbf_offset, rbf_coeff, type_z, n_types, pair_ab, n_pairs, n_nodes, h, tab,
                                    nc, layout, err, s, "radial_table_check");
}

E2V2_API int e2v2_radial_hidden_table(const e2v2_radial_net* net, const float* rbf_offset, float rbf_coeff,
                                      const int32_t* type_z, int32_t n_types, const int32_t* pair_ab,
                                      int32_t n_pairs, int32_t n_nodes, float h, float* tab, int32_t nc,
                                      const e2v2_radial_layout* layout, hipStream_t s) {
  return radial_table_launch<true>(net, rbf_offset, rbf_coeff, type_z, n_types, pair_ab, n_pairs, n_nodes, h, tab,
                                   nc, layout, s, "radial_hidden_table");
}

E2V2_API int e2v2_radial_hidden_table_check(const e2v2_radial_net* net, const float* rbf_offset, float rbf_coeff,
                                            const int32_t* type_z, int32_t n_types, const int32_t* pair_ab,
                                            int32_t n_pairs, int32_t n_nodes, float h, const float* tab, int32_t nc,
                                            const e2v2_radial_layout* layout, uint32_t* err, hipStream_t s) {
  return radial_check_launch<true>(net, rbf_offset, rbf_coeff, type_z, n_types, pair_ab, n_pairs, n_nodes, h, tab,
                                   nc, layout, err, s, "radial_hidden_table_check");
}

static int radial_eval_check(const float* tab, int32_t n_types, int32_t n_nodes, float h, int32_t nc,
                             const int32_t* atom_type, const int32_t* edge_row, const int32_t* col, const float* dist,
                             int64_t n_edges, const char* who) {
  E2V2_REQUIRE(n_edges >= 0 && (n_edges == 0 || (tab && atom_type && edge_row && col && dist)) && n_types >= 1 &&
                   n_types <= E2V2_MAX_TYPES && n_nodes >= 2 && h > 0.f && nc >= 1 && nc <= 4096,
               "%s: bad arguments (n_types %d, n_nodes %d, nc %d)", who, n_types, n_nodes, nc);
  return 0;
}

E2V2_API int e2v2_radial_eval(const float* tab, int32_t n_types, const int32_t* pair_slot, int32_t n_nodes, float h,
                              int32_t nc, const int32_t* atom_type, const int32_t* edge_row, const int32_t* col,
                              const float* dist, int64_t n_edges, const int32_t* e_end, float* out,
                              hipStream_t s) {
  if (int rc = radial_eval_check(tab, n_types, n_nodes, h, nc, atom_type, edge_row, col, dist, n_edges,
                                 "radial_eval"))
    return rc;
  if (n_edges == 0) return 0;
  E2V2_REQUIRE(out, "radial_eval: out is NULL");
  const RadialTab R{tab, n_types, n_nodes, nc, 1.0f / h, pair_slot};
  hipLaunchKernelGGL(k_radial_eval, dim3((unsigned)((n_edges + kEvWaves - 1) / kEvWaves)), dim3(64 * kEvWaves), 0, s,
                     R, atom_type, edge_row, col, dist, n_edges, e_end, out);
  E2V2_LAUNCHED("k_radial_eval");
  return 0;
}

E2V2_API int e2v2_radial_eval_bwd(const float* tab, int32_t n_types, const int32_t* pair_slot, int32_t n_nodes,
                                  float h, int32_t nc, const int32_t* atom_type, const int32_t* edge_row,
                                  const int32_t* col, const float* dist, int64_t n_edges, const int32_t* e_end,
                                  const float* grad, float* ddist, hipStream_t s) {
  if (int rc = radial_eval_check(tab, n_types, n_nodes, h, nc, atom_type, edge_row, col, dist, n_edges,
                                 "radial_eval_bwd"))
    return rc;
  if (n_edges == 0) return 0;
  E2V2_REQUIRE(grad && ddist, "radial_eval_bwd: grad or ddist is NULL");
  const RadialTab R{tab, n_types, n_nodes, nc, 1.0f / h, pair_slot};
  hipLaunchKernelGGL(k_radial_eval_bwd, dim3((unsigned)((n_edges + kEvWaves - 1) / kEvWaves)), dim3(64 * kEvWaves),
                     0, s, R, atom_type, edge_row, col, dist, n_edges, e_end, grad, ddist);
  E2V2_LAUNCHED("k_radial_eval_bwd");
  return 0;
}
