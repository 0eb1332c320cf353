// Sparse equivariant attention of one E2Former-V2 layer on the query CSR.
//
// Forward (one workgroup per query atom i, online segmented softmax):
//   a_e[h]   = gate_e[h] * <q_i[h]/sqrt(D), k_j[h]>
//   m[h]     = max_e a_e[h];  e_e = exp(a_e - m) p(d_e);  s = sum_e e_e
//   w_e[h]   = e_e ih_e[h] / (s + 1e-3) / max(d_e, 1e-6)
//   out[t,c] = sum_e w_e[h(c)] sum_{r,k} T[t,r,k] v_j[r,c] dvec_e[k]     (h(c) = c % 128)
// which equals the reference's gather-scale-scatter of the merged node-frame
// tensor followed by the SO(2) unrotation, h_a - h_b before forward_linear
// (src/molfm/models/e2former/e2former.py:327-433,
//  wigner6j/so2_tensor_product.py:341-385): TP(v, r_i) - TP(v, r_j) = TP(v, r_ij).
// gate and inputhead of every edge are the fc_easy radial profile of
// (d, z_i, z_j), interpolated from its per-type-pair distance table (radial.h)
// where they are used; no per-edge tensor is read from or written to memory
// except the column pass's inputs below.
// Backward: row pass (dq, w, dqk, dvec/ddist with the profile's distance
// derivative; the softmax row terms come from D_h = sum_{c in h} sum_t G[t,c]
// out[t,c]) and a column pass over the key CSR (dv_j, dk_j) with no atomics.
#include "common.h"
#include "radial.h"
#include "tp_table.h"
#include "../../include/e2v2.h"

namespace e2v2 {

constexpr int kH = 128, kD = 8, kC = 256, kNV = 9, kNT = 20, kCH = 32, kCHB = 16;
constexpr float kEps = 1e-3f;
// Channel groups of the clustered kernels: group g holds heads 32g..32g+31 and
// their 64 channels (c and c + 128 share head c % 128).  Lane l of a wave owns
// channel 32g + l (l < 32) or 128 + 32g + l - 32, i.e. head 32g + l % 32, and
// dims 4 (l / 32) .. +3 of that head's q / k.
constexpr int kGroups = 4, kGroupHeads = kH / kGroups;
__device__ __forceinline__ int group_channel(int g, int lane) {
  return (lane < 32) ? (kGroupHeads * g + lane) : (kH + kGroupHeads * g + lane - 32);
}
// (cluster, group) of a workgroup: the workgroups of one XCD (blockIdx % 8) run
// its contiguous range of clusters group by group, so its L2 holds one group's
// quarter of the gathered rows at a time.
__device__ __forceinline__ bool cluster_group(int n_cl, int& cl, int& grp) {
  const int per = (n_cl + kXcd - 1) / kXcd;
  const int seq = blockIdx.x / kXcd, x = blockIdx.x % kXcd;
  grp = seq / per;
  cl = x * per + seq % per;
  return grp < kGroups && cl < n_cl;
}

__device__ __forceinline__ Envelope make_env(const e2v2_attn_args& A) {
  Envelope E;
  E.rc = A.rc; E.a = A.env_a; E.b = A.env_b; E.c = A.env_c;
  return E;
}

// the fc_easy table: channels h (gate) and 128 + h (inputhead) of each row
constexpr int kTabC = 2 * kH;
__device__ __forceinline__ RadialTab make_tab(const e2v2_attn_args& A) {
  RadialTab R;
  R.tab = A.rtab; R.n_types = A.n_types; R.n_nodes = A.rtab_n; R.nc = kTabC; R.inv_h = 1.0f / A.rtab_h;
  return R;
}

// Node activations q, k, v, the output rows and their gradient are stored as TS
// (float, or __bf16 in the bf16 mode); every load widens to fp32 and all
// arithmetic, softmax statistics and reductions are fp32.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float f32(float x) { return x; }
__device__ __forceinline__ float f32(__bf16 x) { return (float)x; }

__device__ __forceinline__ void load8(const float* p, float (&v)[8]) {
  const float4 a = reinterpret_cast<const float4*>(p)[0];
  const float4 b = reinterpret_cast<const float4*>(p)[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
__device__ __forceinline__ void load8(const __bf16* p, float (&v)[8]) {
  const bf16x8 a = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (float)a[i];
}
__device__ __forceinline__ void load4(const float* p, float (&v)[4]) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
}
__device__ __forceinline__ void load4(const __bf16* p, float (&v)[4]) {
  const bf16x4 a = *reinterpret_cast<const bf16x4*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = (float)a[i];
}
// One activation through a 32-bit load of the aligned word that holds it: the
// gathers of the column pass then schedule like their fp32 form (16-bit loads
// are issued one edge at a time); the word lies inside the tensor because rows
// have an even number of elements.
__device__ __forceinline__ float ld_word(const float* p) { return *p; }
__device__ __forceinline__ float ld_word(const __bf16* p) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t w = *reinterpret_cast<const uint32_t*>(a & ~uintptr_t(3));
  return __uint_as_float((a & 2) ? (w & 0xffff0000u) : (w << 16));
}
__device__ __forceinline__ void store_act(float v, float* p) { ntstore(v, p); }
__device__ __forceinline__ void store_act(float v, __bf16* p) { *p = (__bf16)v; }

// <q_s, k_j[h]> with q_s already divided by sqrt(D), as the sum of the two
// half-dots over dims 0..3 and 4..7: the clustered kernels hold one half per
// lane and add the partner lane's, and every pass must round a logit the same
// way (the softmax max is matched bitwise in the backward).
__device__ __forceinline__ float half_dot(const float* q, const float* k) {
  float s = q[0] * k[0];
#pragma unroll
  for (int d = 1; d < 4; ++d) s = fmaf(q[d], k[d], s);
  return s;
}
template <typename TS>
__device__ __forceinline__ float qk_dot(const float (&qs)[kD], const TS* __restrict__ kp) {
  float k[kD];
  load8(kp, k);
  return half_dot(qs, k) + half_dot(qs + 4, k + 4);
}

template <typename TS>
__device__ __forceinline__ void load_qs(const e2v2_attn_args& A, int i, int h, float (&qs)[kD]) {
  float q[kD];
  load8(static_cast<const TS*>(A.q) + ((size_t)i * kH + h) * kD, q);
#pragma unroll
  for (int d = 0; d < kD; ++d) qs[d] = q[d] / A.q_div;
}

struct ChunkEdges {
  int64_t toff[kCH];   // table offset of the edge's lower node
  int j[kCH];
  float dv[kCH][3];
  float p[kCH];
  float dp[kCH];
  float R[kCH];
  float rR[kCH];
  float d[kCH];
  float tt[kCH];       // fraction of the distance in its node interval
};

__device__ __forceinline__ void load_chunk(const e2v2_attn_args& A, const Envelope& env, const RadialTab& R, int ti,
                                           int e0, int nc, ChunkEdges& ce) {
  const int t = threadIdx.x;
  if (t < nc) {
    const int64_t e = (int64_t)e0 + t;
    const int j = A.col[e];
    ce.j[t] = j;
    ce.dv[t][0] = A.dvec[3 * e];
    ce.dv[t][1] = A.dvec[3 * e + 1];
    ce.dv[t][2] = A.dvec[3 * e + 2];
    const float d = A.dist[e];
    ce.d[t] = d;
    float p, dp;
    env.eval(d, p, dp);
    ce.p[t] = p;
    ce.dp[t] = dp;
    ce.R[t] = fmaxf(d, 1e-6f);
    ce.rR[t] = 1.0f / ce.R[t];
    float tt;
    ce.toff[t] = radial_node(R, ti * R.n_types + A.atom_type[j], d, tt);
    ce.tt[t] = tt;
  }
}

template <typename TS>
__global__ __launch_bounds__(256) void k_attn_fwd(e2v2_attn_args A, TS* __restrict__ out, float* __restrict__ mrow,
                                                  float* __restrict__ srow, int32_t* __restrict__ cnt) {
  const TS* __restrict__ Kp = static_cast<const TS*>(A.k);
  const TS* __restrict__ Vp = static_cast<const TS*>(A.v);
  __shared__ float a_s[kCH][kH];
  __shared__ float coef_s[kCH][kH];
  __shared__ float scale_s[kH];
  __shared__ float inv_s[kH];
  __shared__ ChunkEdges ce;
  const int i = xcd_row(blockIdx.x, A.n_rows), t = threadIdx.x;
  if (i >= A.n_rows) return;
  const int h = t & (kH - 1), half = t >> 7;
  const int b = A.row_ptr[i], n = A.row_ptr[i + 1] - b;
  const Envelope env = make_env(A);
  const RadialTab R = make_tab(A);
  const int ti = A.atom_type[i];
  float qs[kD];
  load_qs<TS>(A, i, h, qs);
  float m_run = -INFINITY, s_run = 0.f;
  int c_run = 0;
  float acc[kNV][3];
#pragma unroll
  for (int r = 0; r < kNV; ++r) acc[r][0] = acc[r][1] = acc[r][2] = 0.f;
  const int hc = t & (kH - 1);  // head of channel c = t
  for (int c0 = 0; c0 < n; c0 += kCH) {
    const int nc = min(kCH, n - c0);
    load_chunk(A, env, R, ti, b + c0, nc, ce);
    __syncthreads();
    for (int el = half; el < nc; el += 2) {
      const float qk = qk_dot(qs, Kp + ((size_t)ce.j[el] * kH + h) * kD);
      // gate (channel h) and inputhead (channel 128 + h): rows 0..2 at the two nodes
      const float* tb = R.tab + ce.toff[el] + h;
      const Hermite5 Hw = hermite5(ce.tt[el]);
      constexpr int nb = 4 * kTabC;
      const float gate = herm_value(Hw, tb[0], tb[kTabC], tb[2 * kTabC], tb[nb], tb[nb + kTabC], tb[nb + 2 * kTabC]);
      const float* tb2 = tb + kH;
      const float ih = herm_value(Hw, tb2[0], tb2[kTabC], tb2[2 * kTabC], tb2[nb], tb2[nb + kTabC],
                                  tb2[nb + 2 * kTabC]);
      a_s[el][h] = gate * qk;
      coef_s[el][h] = ih;   // input head, scaled below
    }
    __syncthreads();
    if (t < kH) {
      float cm = -INFINITY;
      for (int el = 0; el < nc; ++el) cm = fmaxf(cm, a_s[el][h]);
      const float m_new = fmaxf(m_run, cm);
      const float sc = (m_run == -INFINITY) ? 0.f : expf(m_run - m_new);
      int cc = 0;
      for (int el = 0; el < nc; ++el) cc += (a_s[el][h] == m_new);
      c_run = (m_new == m_run) ? c_run + cc : cc;
      s_run *= sc;
      for (int el = 0; el < nc; ++el) {
        const float ex = expf(a_s[el][h] - m_new);
        const float ee = ex * ce.p[el];
        s_run += ee;
        coef_s[el][h] = (ee * coef_s[el][h]) * ce.rR[el];
      }
      m_run = m_new;
      scale_s[h] = sc;
    }
    __syncthreads();
    {
      const float sc = scale_s[hc];
      if (sc != 1.f) {
#pragma unroll
        for (int r = 0; r < kNV; ++r) {
          acc[r][0] *= sc; acc[r][1] *= sc; acc[r][2] *= sc;
        }
      }
      for (int el = 0; el < nc; ++el) {
        const float w = coef_s[el][hc];
        const float wx = w * ce.dv[el][0], wy = w * ce.dv[el][1], wz = w * ce.dv[el][2];
        const TS* vp = Vp + (size_t)ce.j[el] * kC + t;
        const size_t vs = (size_t)A.n_rows * kC;
        float vv[kNV];
#pragma unroll
        for (int r = 0; r < kNV; ++r) vv[r] = f32(vp[r * vs]);
#pragma unroll
        for (int r = 0; r < kNV; ++r) {
          acc[r][0] = fmaf(vv[r], wx, acc[r][0]);
          acc[r][1] = fmaf(vv[r], wy, acc[r][1]);
          acc[r][2] = fmaf(vv[r], wz, acc[r][2]);
        }
      }
    }
    __syncthreads();
  }
  if (t < kH) {
    inv_s[h] = 1.0f / (s_run + kEps);
    mrow[(size_t)i * kH + h] = m_run;
    srow[(size_t)i * kH + h] = s_run;
    cnt[(size_t)i * kH + h] = c_run;
  }
  __syncthreads();
  const float inv = inv_s[hc];
  float o[kNT];
#pragma unroll
  for (int q = 0; q < kNT; ++q) o[q] = 0.f;
#pragma unroll
  for (int z = 0; z < kTpNnz; ++z) o[kTp[z].t] = fmaf(kTp[z].c, acc[kTp[z].r][kTp[z].k], o[kTp[z].t]);
  TS* op = out + (size_t)i * kC + t;
  const size_t os = (size_t)A.n_rows * kC;
#pragma unroll
  for (int q = 0; q < kNT; ++q) store_act(o[q] * inv, op + q * os);
}

// dA[r][k] = sum_t T[t][r][k] g[t] for one channel
__device__ __forceinline__ void tp_transpose(const float (&g)[kNT], float (&dA)[kNV][3]) {
#pragma unroll
  for (int r = 0; r < kNV; ++r) dA[r][0] = dA[r][1] = dA[r][2] = 0.f;
#pragma unroll
  for (int z = 0; z < kTpNnz; ++z) dA[kTp[z].r][kTp[z].k] = fmaf(kTp[z].c, g[kTp[z].t], dA[kTp[z].r][kTp[z].k]);
}

// Column pass, one channel per thread (the fp32 form: a 4-byte gather per lane
// is as cheap per byte for the address unit as a pair load): for every source
// atom j, sum over its key-CSR edges (ascending edge id) -> dv_j and dk_j.
// Edge metadata of a 32-edge chunk is staged in LDS so the per-edge gathers of
// grad rows do not wait on index loads; two edges are processed per iteration
// to overlap their 20-row gathers.
template <typename TS>
__global__ __launch_bounds__(256) void k_attn_bwd_col_ch(e2v2_attn_args A, const TS* __restrict__ G,
                                                      const float* __restrict__ w_e, const float* __restrict__ dqk_e,
                                                      float* __restrict__ dv_out, float* __restrict__ dk_out) {
  constexpr int CC = 32;
  __shared__ int ci[CC];
  __shared__ float cdv[CC][3];
  __shared__ float cw[CC][kH];
  __shared__ float cq[CC][kH];
  const int j = xcd_row(blockIdx.x, A.n_rows), t = threadIdx.x;
  if (j >= A.n_rows) return;
  const int c = t, hc = t & (kH - 1);
  const int hk = t >> 1, d0 = 4 * (t & 1);
  const size_t os = (size_t)A.n_rows * kC;
  float av[kNV];
#pragma unroll
  for (int r = 0; r < kNV; ++r) av[r] = 0.f;
  float ak[4] = {0.f, 0.f, 0.f, 0.f};
  const int p0 = A.key_ptr[j], p1 = A.key_ptr[j + 1];
  const TS* __restrict__ Qp = static_cast<const TS*>(A.q);
  for (int c0 = p0; c0 < p1; c0 += CC) {
    const int nc = min(CC, p1 - c0);
    if (t < nc) {
      const int64_t e = A.key_eid[c0 + t];
      ci[t] = A.edge_row[e];
      cdv[t][0] = A.dvec[3 * e];
      cdv[t][1] = A.dvec[3 * e + 1];
      cdv[t][2] = A.dvec[3 * e + 2];
    }
    // per-edge head weights: w and dqk rows are 512 B each; 2 edges x 128 heads per pass
    for (int idx = t; idx < nc * kH; idx += 256) {
      const int el = idx >> 7, h = idx & (kH - 1);
      const int64_t e = A.key_eid[c0 + el];
      cw[el][h] = ntload(w_e + e * kH + h);
      cq[el][h] = ntload(dqk_e + e * kH + h);
    }
    __syncthreads();
    // dv_j[r] += sum_k dA[r][k] (w dvec_k), dA = T^T G_i[:, c]; dk_j += dqk q_i (scaled by 1/sqrt(D) once at the end)
    auto edge = [&](int el, const float (&g)[kNT], const float (&q)[4]) {
      float dA[kNV][3];
      tp_transpose(g, dA);
      const float w = cw[el][hc];
      const float wx = w * cdv[el][0], wy = w * cdv[el][1], wz = w * cdv[el][2];
#pragma unroll
      for (int r = 0; r < kNV; ++r) av[r] = fmaf(dA[r][2], wz, fmaf(dA[r][1], wy, fmaf(dA[r][0], wx, av[r])));
      const float dqv = cq[el][hk];
#pragma unroll
      for (int d = 0; d < 4; ++d) ak[d] = fmaf(dqv, q[d], ak[d]);
    };
    int el = 0;
    for (; el + 1 < nc; el += 2) {
      const int i0 = ci[el], i1 = ci[el + 1];
      float g0[kNT], g1[kNT];
#pragma unroll
      for (int z = 0; z < kNT; ++z) {
        g0[z] = ld_word(G + (size_t)i0 * kC + z * os + c);
        g1[z] = ld_word(G + (size_t)i1 * kC + z * os + c);
      }
      float qa[4], qb[4];
      load4(Qp + ((size_t)i0 * kH + hk) * kD + d0, qa);
      load4(Qp + ((size_t)i1 * kH + hk) * kD + d0, qb);
      edge(el, g0, qa);
      edge(el + 1, g1, qb);
    }
    if (el < nc) {
      const int i0 = ci[el];
      float g0[kNT];
#pragma unroll
      for (int z = 0; z < kNT; ++z) g0[z] = ld_word(G + (size_t)i0 * kC + z * os + c);
      float qa[4];
      load4(Qp + ((size_t)i0 * kH + hk) * kD + d0, qa);
      edge(el, g0, qa);
    }
    __syncthreads();
  }
#pragma unroll
  for (int r = 0; r < kNV; ++r) ntstore(av[r], dv_out + (size_t)j * kC + r * os + c);
#pragma unroll
  for (int d = 0; d < 4; ++d) ntstore(ak[d] / A.q_div, dk_out + ((size_t)j * kH + hk) * kD + d0 + d);
}

// Column pass, channel pairs (the bf16 form: one 4-byte word carries two
// channels): for every source atom j, sum over its key-CSR edges (ascending
// edge id) -> dv_j and dk_j, no atomics.  Thread t owns the channel pair
// (2u, 2u + 1), u = t % 128, and the chunk's edges of parity t / 128: every
// gather instruction moves two channels per lane (the gathers, not the bytes,
// bound this pass).  The two parities' partial sums are added once per column
// in LDS (fixed order: deterministic).  Edge metadata of 32-edge chunks is
// staged in LDS.
__device__ __forceinline__ void ld_pair(const float* p, float& a, float& b) {
  const float2 v = *reinterpret_cast<const float2*>(p);
  a = v.x;
  b = v.y;
}
__device__ __forceinline__ void ld_pair(const __bf16* p, float& a, float& b) {
  const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xffff0000u);
}

template <typename TS>
__global__ __launch_bounds__(256) void k_attn_bwd_col_pair(e2v2_attn_args A, const TS* __restrict__ G,
                                                           const float* __restrict__ w_e,
                                                           const float* __restrict__ dqk_e, float* __restrict__ dv_out,
                                                           float* __restrict__ dk_out) {
  constexpr int CC = 32;
  __shared__ int ci[CC];
  __shared__ float cdv[CC][3];
  __shared__ float cwq[2 * CC * kH];          // per-chunk w | dqk; after the loop, the parity partial sums
  float (*cw)[kH] = reinterpret_cast<float (*)[kH]>(cwq);
  float (*cq)[kH] = reinterpret_cast<float (*)[kH]>(cwq + CC * kH);
  float (*red_v)[kC] = reinterpret_cast<float (*)[kC]>(cwq);
  float (*red_k)[kD] = reinterpret_cast<float (*)[kD]>(cwq + kNV * kC);
  static_assert(kNV * kC + kH * kD <= 2 * CC * kH, "partial sums fit the chunk buffers");
  const int j = xcd_row(blockIdx.x, A.n_rows), t = threadIdx.x;
  if (j >= A.n_rows) return;
  const int u = t & (kH - 1), par = t >> 7;
  const int c0 = 2 * u;                                     // channels c0, c0 + 1
  const int h0 = c0 & (kH - 1), h1 = (c0 + 1) & (kH - 1);   // their heads
  const size_t os = (size_t)A.n_rows * kC;
  float av0[kNV], av1[kNV];
#pragma unroll
  for (int r = 0; r < kNV; ++r) av0[r] = av1[r] = 0.f;
  float ak[kD];
#pragma unroll
  for (int d = 0; d < kD; ++d) ak[d] = 0.f;
  const int p0 = A.key_ptr[j], p1 = A.key_ptr[j + 1];
  const TS* __restrict__ Qp = static_cast<const TS*>(A.q);
  // dv[r] += sum_k dA[r][k] (w dvec_k), dA = T^T G_i[:, c]
  auto channel = [&](int el, const float (&g)[kNT], int h, float (&av)[kNV]) {
    float dA[kNV][3];
    tp_transpose(g, dA);
    const float w = cw[el][h];
    const float wx = w * cdv[el][0], wy = w * cdv[el][1], wz = w * cdv[el][2];
#pragma unroll
    for (int r = 0; r < kNV; ++r) av[r] = fmaf(dA[r][2], wz, fmaf(dA[r][1], wy, fmaf(dA[r][0], wx, av[r])));
  };
  for (int c0e = p0; c0e < p1; c0e += CC) {
    const int nc = min(CC, p1 - c0e);
    if (t < nc) {
      const int64_t e = A.key_eid[c0e + t];
      ci[t] = A.edge_row[e];
      cdv[t][0] = A.dvec[3 * e];
      cdv[t][1] = A.dvec[3 * e + 1];
      cdv[t][2] = A.dvec[3 * e + 2];
    }
    // per-edge head weights: w and dqk rows are 512 B each; 2 edges x 128 heads per pass
    for (int idx = t; idx < nc * kH; idx += 256) {
      const int el = idx >> 7, h = idx & (kH - 1);
      const int64_t e = A.key_eid[c0e + el];
      cw[el][h] = ntload(w_e + e * kH + h);
      cq[el][h] = ntload(dqk_e + e * kH + h);
    }
    __syncthreads();
    for (int el = par; el < nc; el += 2) {
      const int i = ci[el];
      float ga[kNT], gb[kNT];
#pragma unroll
      for (int z = 0; z < kNT; ++z) ld_pair(G + (size_t)i * kC + z * os + c0, ga[z], gb[z]);
      float q[kD];
      load8(Qp + ((size_t)i * kH + u) * kD, q);
      channel(el, ga, h0, av0);
      channel(el, gb, h1, av1);
      const float dqv = cq[el][u];
#pragma unroll
      for (int d = 0; d < kD; ++d) ak[d] = fmaf(dqv, q[d], ak[d]);
    }
    __syncthreads();
  }
  if (par) {
#pragma unroll
    for (int r = 0; r < kNV; ++r) {
      red_v[r][c0] = av0[r];
      red_v[r][c0 + 1] = av1[r];
    }
#pragma unroll
    for (int d = 0; d < kD; ++d) red_k[u][d] = ak[d];
  }
  __syncthreads();
  if (!par) {
#pragma unroll
    for (int r = 0; r < kNV; ++r) {
      const float2 v = make_float2(av0[r] + red_v[r][c0], av1[r] + red_v[r][c0 + 1]);
      *reinterpret_cast<float2*>(dv_out + (size_t)j * kC + r * os + c0) = v;
    }
    float* kp = dk_out + ((size_t)j * kH + u) * kD;
#pragma unroll
    for (int d = 0; d < kD; ++d) kp[d] = (ak[d] + red_k[u][d]) / A.q_div;
  }
}

// Column pass over clusters of R consecutive key-CSR columns and one of four
// channel groups (G and q in fp32 or bf16, sums in fp32).  Group g holds the 64 channels of heads 32g..32g+31
// (c and c + 128 share a head); the workgroups of one XCD run group by group,
// so its L2 holds a quarter of each neighbour row at a time and the gathered
// rows of a column window stay resident.  Wave w applies the slots s = w mod 4
// of each chunk (lane = channel of the group; for dk lane = (head, half of the
// head's dims)); the four waves' partial sums are added once per cluster in
// LDS in a fixed order.  Every slot's G_i and q_i are loaded once and applied
// to each column of the cluster that it joins.

template <int R, typename TS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void k_attn_bwd_col_grp(e2v2_attn_args A, const TS* __restrict__ G,
                                                          const float* __restrict__ w_e,
                                                          const float* __restrict__ dqk_e, float* __restrict__ dv_out,
                                                          float* __restrict__ dk_out) {
  constexpr int S = 32;                        // slots per staged chunk
  __shared__ int ci[S];
  __shared__ int ce[S][R];
  __shared__ float cdv[S][R][3];
  __shared__ float red[2][R][kNV + 4][kWave];  // per-wave partial sums, added in two rounds
  const int n_cl = (A.n_rows + R - 1) / R;
  int cl, grp;
  if (!cluster_group(n_cl, cl, grp)) return;
  const int t = threadIdx.x, lane = t & (kWave - 1), wave = t >> 6;
  const int c = group_channel(grp, lane);
  const int hc = c & (kH - 1);
  const int hk = kGroupHeads * grp + (lane >> 1), d0 = 4 * (lane & 1);
  const int j0 = cl * R, nj = min(R, A.n_rows - j0);
  const size_t os = (size_t)A.n_rows * kC;
  const int64_t base = A.key_ptr[j0];
  const int ns = A.col_n_slots[cl];
  const int32_t* __restrict__ smem = A.col_slot_member + base;
  const int32_t* __restrict__ sedge = A.col_slot_edge + base * R;
  const TS* __restrict__ Qp = static_cast<const TS*>(A.q);
  float av[R][kNV];
  float ak[R][4];
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int z = 0; z < kNV; ++z) av[r][z] = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) ak[r][d] = 0.f;
  }
  struct Loads {
    TS g[kNT];   // converted to fp32 in apply()
    float q[4];
    float w[R];
    float dq[R];
  };
  auto issue = [&](int sl, Loads& L) {
    const int i = ci[sl];
#pragma unroll
    for (int z = 0; z < kNT; ++z) L.g[z] = G[(size_t)i * kC + z * os + c];
    load4(Qp + ((size_t)i * kH + hk) * kD + d0, L.q);
    // unconditional (an absent edge reads edge 0, unused): every slot issues the
    // same loads, so the wait before apply() counts only the older slot's
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t e = max(ce[sl][r], 0);
      L.w[r] = ntload(w_e + e * kH + hc);
      L.dq[r] = ntload(dqk_e + e * kH + hk);
    }
  };
  auto apply = [&](int sl, const Loads& L) {
    float g[kNT], dA[kNV][3];
#pragma unroll
    for (int z = 0; z < kNT; ++z) g[z] = static_cast<float>(L.g[z]);
    tp_transpose(g, dA);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (ce[sl][r] >= 0) {
        const float w = L.w[r];
        const float wx = w * cdv[sl][r][0], wy = w * cdv[sl][r][1], wz = w * cdv[sl][r][2];
#pragma unroll
        for (int z = 0; z < kNV; ++z)
          av[r][z] = fmaf(dA[z][2], wz, fmaf(dA[z][1], wy, fmaf(dA[z][0], wx, av[r][z])));
#pragma unroll
        for (int d = 0; d < 4; ++d) ak[r][d] = fmaf(L.dq[r], L.q[d], ak[r][d]);
      }
    }
  };
  for (int s0 = 0; s0 < ns; s0 += S) {
    const int nc = min(S, ns - s0);
    if (t < nc) ci[t] = smem[s0 + t];
    for (int idx = t; idx < nc * R; idx += 256) {
      const int sl = idx / R, r = idx % R;
      const int e = sedge[(int64_t)(s0 + sl) * R + r];
      ce[sl][r] = e;
      if (e >= 0) {
        cdv[sl][r][0] = A.dvec[3 * (int64_t)e];
        cdv[sl][r][1] = A.dvec[3 * (int64_t)e + 1];
        cdv[sl][r][2] = A.dvec[3 * (int64_t)e + 2];
      }
    }
    __syncthreads();
    int sl = wave;
    if (sl < nc) {
      Loads La, Lb;
      issue(sl, La);
      for (; sl + 8 < nc; sl += 8) {
        issue(sl + 4, Lb);
        apply(sl, La);
        issue(sl + 8, La);
        apply(sl + 4, Lb);
      }
      if (sl + 4 < nc) {
        issue(sl + 4, Lb);
        apply(sl, La);
        apply(sl + 4, Lb);
      } else {
        apply(sl, La);
      }
    }
    __syncthreads();
  }
  // (w0 + w2) + (w1 + w3)
  auto put = [&](int b) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int z = 0; z < kNV; ++z) red[b][r][z][lane] = av[r][z];
#pragma unroll
      for (int d = 0; d < 4; ++d) red[b][r][kNV + d][lane] = ak[r][d];
    }
  };
  auto add = [&](int b) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int z = 0; z < kNV; ++z) av[r][z] += red[b][r][z][lane];
#pragma unroll
      for (int d = 0; d < 4; ++d) ak[r][d] += red[b][r][kNV + d][lane];
    }
  };
  if (wave >= 2) put(wave - 2);
  __syncthreads();
  if (wave < 2) add(wave);
  __syncthreads();
  if (wave == 1) put(0);
  __syncthreads();
  if (wave == 0) {
    add(0);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r < nj) {
        const int j = j0 + r;
#pragma unroll
        for (int z = 0; z < kNV; ++z) ntstore(av[r][z], dv_out + (size_t)j * kC + z * os + c);
#pragma unroll
        for (int d = 0; d < 4; ++d) ntstore(ak[r][d] / A.q_div, dk_out + ((size_t)j * kH + hk) * kD + d0 + d);
      }
    }
  }
}

// Sums of four values over the 64 lanes of a wave; every lane of row k (lanes
// 16k .. 16k + 15) returns the sum of value k.  A swap across the wave halves
// (lanes < 32 keep values 0 and 1, lanes >= 32 values 2 and 3), a swap across
// the two rows of each half (even rows keep the first, odd rows the second),
// then four DPP steps within each row of 16.
__device__ __forceinline__ float wave_sum4(float v0, float v1, float v2, float v3, int lane) {
  const bool hi = (lane & 32) != 0, odd = (lane & 16) != 0;
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v0), __float_as_uint(v2), false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v1), __float_as_uint(v3), false, false);
  // lane < 32: a[1] = v0 of lane + 32; lane >= 32: a[0] = v2 of lane - 32 (b likewise for v1, v3)
  const float x = hi ? v2 + __uint_as_float(a[0]) : v0 + __uint_as_float(a[1]);
  const float y = hi ? v3 + __uint_as_float(b[0]) : v1 + __uint_as_float(b[1]);
  const auto c = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  // even row: c[1] = x of the odd row beside it; odd row: c[0] = y of the even row
  const float z = odd ? y + __uint_as_float(c[0]) : x + __uint_as_float(c[1]);
  return dpp_row_sum16(z);
}

// One edge's gathered operands for a head, kept in the storage type until the
// edge is applied (bf16: half the staging registers of converted values).
template <typename TS>
struct HeadEdge {
  TS k[kD];
  TS v0[kNV], v1[kNV];
  float tg[8], ti[8];   // table rows 0..3 at the lower and upper node: gate, inputhead
};
__device__ __forceinline__ void load8_raw(const float* p, float (&v)[8]) { load8(p, v); }
__device__ __forceinline__ void load8_raw(const __bf16* p, __bf16 (&v)[8]) {
  const bf16x8 a = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = a[i];
}

// Backward row pass, one workgroup per query row; thread t owns head h = t % 128
// with both of its channels (h, h + 128) and the row's edges of parity t / 128.
// The edge index is uniform per wave (scalar loads of the edge record), and
// the gathers of the next edge (k_j, v_j and the head's gate / inputhead table
// rows) are issued before the current one is applied.  Per edge a thread
// interpolates the head's gate and inputhead and their distance derivatives,
// recomputes its logit and weight, forms u = dA^T v_j for both channels
// (dA = T^T G_i) and with it the head's dL/dw, runs the softmax / gate /
// distance backward for its head (the profile's part dL/dgate gate' +
// dL/dih ih' included) and accumulates dq from the k_j row it already holds,
// so nothing crosses threads but the per-edge sums over heads (dL/d dvec,
// dL/dd): the 64 heads of a wave by lane swaps and DPP (wave_sum4), the two
// waves of a parity in LDS, added in a fixed order once per chunk of up to 128
// edges.  The head-independent edge terms (column, distance, envelope, 1/d,
// dvec, table node and fraction) are formed once per edge at the start of a
// chunk and read from LDS.
template <typename TS>
__global__ __launch_bounds__(256) void k_attn_bwd_row_hp(e2v2_attn_args A, const TS* __restrict__ G,
                                                         const TS* __restrict__ O, const float* __restrict__ mrow,
                                                         const float* __restrict__ srow,
                                                         const int32_t* __restrict__ cnt,
                                                         float* __restrict__ ddv, float* __restrict__ dd,
                                                         float* __restrict__ dq, float* __restrict__ w_out,
                                                         float* __restrict__ dqk_out) {
  constexpr int CH = 64;                      // edges per parity and reduction chunk
  __shared__ float part[2 * CH][2][4];
  __shared__ float dq_s[kH][kD];
  __shared__ float4 er_a[2 * CH];             // per edge of the chunk: p, dp/dd, 1/max(d, 1e-6), d
  __shared__ float4 er_b[2 * CH];             // dvec, column (int bits)
  __shared__ int64_t er_toff[2 * CH];         // table offset of the lower node
  __shared__ float er_t[2 * CH];              // fraction in the node interval
  const int i = xcd_row(blockIdx.x, A.n_rows), t = threadIdx.x;
  if (i >= A.n_rows) return;
  const RadialTab R = make_tab(A);
  const int ti = A.atom_type[i];
  const int h = t & (kH - 1), par = t >> 7, lane = t & (kWave - 1), wsub = (t >> 6) & 1;
  const TS* __restrict__ Kp = static_cast<const TS*>(A.k);
  const TS* __restrict__ Vp = static_cast<const TS*>(A.v);
  const size_t os = (size_t)A.n_rows * kC;
  const int b = A.row_ptr[i], n = A.row_ptr[i + 1] - b;
  const Envelope env = make_env(A);
  // per-row prologue: dA of both channels, D_h, softmax statistics of head h
  float dA0[kNV][3], dA1[kNV][3];
  float inv, dsum, dmc, m;
  {
    float g0[kNT], g1[kNT];
    float Dh = 0.f;
#pragma unroll
    for (int z = 0; z < kNT; ++z) {
      g0[z] = f32(G[(size_t)i * kC + z * os + h]);
      g1[z] = f32(G[(size_t)i * kC + z * os + h + kH]);
    }
    // D_h = sum over the head's channels and the 20 rows, summed as channel h then h + 128
    float d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int z = 0; z < kNT; ++z) {
      d0 = fmaf(g0[z], f32(O[(size_t)i * kC + z * os + h]), d0);
      d1 = fmaf(g1[z], f32(O[(size_t)i * kC + z * os + h + kH]), d1);
    }
    Dh = d1 + d0;
    tp_transpose(g0, dA0);
    tp_transpose(g1, dA1);
    m = mrow[(size_t)i * kH + h];
    const float s = srow[(size_t)i * kH + h];
    const int cn = cnt[(size_t)i * kH + h];
    inv = 1.0f / (s + kEps);
    dsum = Dh * inv;
    dmc = cn > 0 ? (-Dh * kEps * inv) / (float)cn : 0.f;
  }
  float qs[kD];
  load_qs<TS>(A, i, h, qs);
  float dqa[kD];
#pragma unroll
  for (int d = 0; d < kD; ++d) dqa[d] = 0.f;
  using L = HeadEdge<TS>;
  int c0 = 0;  // first edge of the current chunk
  auto issue = [&](int el, L& X) {
    const int64_t e = (int64_t)b + el;
    const int j = __float_as_int(er_b[el - c0].w);
    // 32-bit per-lane byte offsets from wave-uniform bases (n_rows * kH * kD *
    // sizeof(TS) < 2^32 is checked by the host)
    const uint32_t kof = ((uint32_t)j * kH + h) * (kD * sizeof(TS));
    load8_raw(reinterpret_cast<const TS*>(reinterpret_cast<const char*>(Kp) + kof), X.k);
    const uint32_t vof = ((uint32_t)j * kC + h) * sizeof(TS);
#pragma unroll
    for (int r = 0; r < kNV; ++r) {
      const char* vb = reinterpret_cast<const char*>(Vp + r * os);
      X.v0[r] = *reinterpret_cast<const TS*>(vb + vof);
      X.v1[r] = *reinterpret_cast<const TS*>(vb + vof + kH * sizeof(TS));
    }
    const float* tb = R.tab + er_toff[el - c0] + h;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      X.tg[q] = tb[q * kTabC];
      X.tg[4 + q] = tb[(4 + q) * kTabC];
      X.ti[q] = tb[q * kTabC + kH];
      X.ti[4 + q] = tb[(4 + q) * kTabC + kH];
    }
  };
  auto apply = [&](int el, int slot, const L& X) {
    const int64_t e = (int64_t)b + el;
    const float4 ea = er_a[slot], eb = er_b[slot];
    const float pe = ea.x, dpe = ea.y, rR = ea.z, d = ea.w;
    const float dvx = eb.x, dvy = eb.y, dvz = eb.z;
    const Hermite5 Hw = hermite5(er_t[slot]);
    const float gate = herm_value(Hw, X.tg[0], X.tg[1], X.tg[2], X.tg[4], X.tg[5], X.tg[6]);
    const float ih = herm_value(Hw, X.ti[0], X.ti[1], X.ti[2], X.ti[4], X.ti[5], X.ti[6]);
    const float gate_d = herm_value(Hw, X.tg[1], X.tg[2], X.tg[3], X.tg[5], X.tg[6], X.tg[7]) * R.inv_h;
    const float ih_d = herm_value(Hw, X.ti[1], X.ti[2], X.ti[3], X.ti[5], X.ti[6], X.ti[7]) * R.inv_h;
    float kf[kD];
#pragma unroll
    for (int q = 0; q < kD; ++q) kf[q] = f32(X.k[q]);
    const float qk = half_dot(qs, kf) + half_dot(qs + 4, kf + 4);
    const float a = gate * qk;
    const float ex = expf(a - m);
    const float ee = ex * pe;
    const float alpha = (ee * ih) * inv;
    const float w = alpha * rR;
    float U[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      float u0 = 0.f, u1 = 0.f;
#pragma unroll
      for (int r = 0; r < kNV; ++r) {
        u0 = fmaf(dA0[r][k], f32(X.v0[r]), u0);
        u1 = fmaf(dA1[r][k], f32(X.v1[r]), u1);
      }
      U[k] = u0 + u1;
    }
    const float dw = U[0] * dvx + U[1] * dvy + U[2] * dvz;
    const float dalpha = dw * rR;
    const float dR = (d > 1e-6f) ? -dalpha * alpha * rR : 0.f;
    const float dih = dalpha * ee * inv;
    const float de = dalpha * ih * inv - dsum;
    float da = de * ee;
    if (a == m) da += dmc;
    const float dpv = de * ex;
    const float dqk = da * gate;
    ntstore(w, w_out + e * kH + h);
    ntstore(dqk, dqk_out + e * kH + h);
#pragma unroll
    for (int q = 0; q < kD; ++q) dqa[q] = fmaf(dqk, kf[q], dqa[q]);
    // dL/dd of this head: envelope, 1/d, and the profile (dL/dgate gate' + dL/dih ih')
    const float ddh = fmaf(da * qk, gate_d, fmaf(dih, ih_d, fmaf(dpv, dpe, dR)));
    // sums over the 64 heads of this wave; lane 16k holds the sum of value k
    const float sum = wave_sum4(w * U[0], w * U[1], w * U[2], ddh, lane);
    if ((lane & 15) == 0) part[slot][wsub][lane >> 4] = sum;
  };
  for (c0 = 0; c0 < n; c0 += 2 * CH) {
    const int nc = min(2 * CH, n - c0);
    if (t < nc) {
      const int64_t e = (int64_t)b + c0 + t;
      const float d = A.dist[e];
      float pe, dpe;
      env.eval(d, pe, dpe);
      er_a[t] = make_float4(pe, dpe, 1.0f / fmaxf(d, 1e-6f), d);
      const int j = A.col[e];
      er_b[t] = make_float4(A.dvec[3 * e], A.dvec[3 * e + 1], A.dvec[3 * e + 2], __int_as_float(j));
      float tt;
      er_toff[t] = radial_node(R, ti * R.n_types + A.atom_type[j], d, tt);
      er_t[t] = tt;
    }
    __syncthreads();
    {
      L Xa, Xb;
      int el = par;
      if (el < nc) {
        issue(c0 + el, Xa);
        for (; el + 4 < nc; el += 4) {
          issue(c0 + el + 2, Xb);
          apply(c0 + el, el, Xa);
          issue(c0 + el + 4, Xa);
          apply(c0 + el + 2, el + 2, Xb);
        }
        if (el + 2 < nc) {
          issue(c0 + el + 2, Xb);
          apply(c0 + el, el, Xa);
          apply(c0 + el + 2, el + 2, Xb);
        } else {
          apply(c0 + el, el, Xa);
        }
      }
    }
    __syncthreads();
    if (t < nc) {
      const int64_t e = (int64_t)b + c0 + t;
      ddv[3 * e] = part[t][0][0] + part[t][1][0];
      ddv[3 * e + 1] = part[t][0][1] + part[t][1][1];
      ddv[3 * e + 2] = part[t][0][2] + part[t][1][2];
      dd[e] = part[t][0][3] + part[t][1][3];
    }
    __syncthreads();
  }
  if (par) {
#pragma unroll
    for (int q = 0; q < kD; ++q) dq_s[h][q] = dqa[q];
  }
  __syncthreads();
  if (!par) {
#pragma unroll
    for (int q = 0; q < kD; ++q) dq[((size_t)i * kH + h) * kD + q] = (dqa[q] + dq_s[h][q]) / A.q_div;
  }
}

}  // namespace e2v2

using namespace e2v2;

static int check_table(const e2v2_attn_args& A, const char* who);

E2V2_API int e2v2_attn_fwd(const e2v2_attn_args* args, void* out, float* mrow, float* srow, int32_t* cnt,
                           hipStream_t s) {
  const e2v2_attn_args& A = *args;
  E2V2_REQUIRE(A.n_heads == kH && A.head_dim == kD && A.channels == kC,
               "attn_fwd: built for H=%d D=%d C=%d, got H=%d D=%d C=%d", kH, kD, kC, A.n_heads, A.head_dim,
               A.channels);
  if (A.n_rows == 0) return 0;
  if (int rc = check_table(A, "attn_fwd")) return rc;
  const dim3 grid(xcd_grid(A.n_rows));
  if (A.act_bf16) {
    hipLaunchKernelGGL(k_attn_fwd<__bf16>, grid, dim3(256), 0, s, A, static_cast<__bf16*>(out), mrow, srow, cnt);
  } else {
    hipLaunchKernelGGL(k_attn_fwd<float>, grid, dim3(256), 0, s, A, static_cast<float*>(out), mrow, srow, cnt);
  }
  E2V2_LAUNCHED("k_attn_fwd");
  return 0;
}

template <typename TS>
static int attn_bwd_launch(const e2v2_attn_args& A, const TS* G, const TS* O, const float* mrow, const float* srow,
                           const int32_t* cnt, float* ddvec, float* ddist, float* dq, float* dk, float* dv,
                           float* w_edge, float* dqk_edge, hipStream_t s) {
  const dim3 grid(xcd_grid(A.n_rows));
  hipLaunchKernelGGL(k_attn_bwd_row_hp<TS>, grid, dim3(256), 0, s, A, G, O, mrow, srow, cnt, ddvec, ddist, dq,
                     w_edge, dqk_edge);
  E2V2_LAUNCHED("k_attn_bwd_row");
  if (A.col_slot_member) {
    const int n_cl = (A.n_rows + 3) / 4;
    hipLaunchKernelGGL((k_attn_bwd_col_grp<4, TS>), dim3(xcd_grid(n_cl) * kGroups), dim3(256), 0, s, A, G, w_edge,
                       dqk_edge, dv, dk);
  } else if constexpr (sizeof(TS) == 2) {
    hipLaunchKernelGGL(k_attn_bwd_col_pair<TS>, grid, dim3(256), 0, s, A, G, w_edge, dqk_edge, dv, dk);
  } else {
    hipLaunchKernelGGL(k_attn_bwd_col_ch<TS>, grid, dim3(256), 0, s, A, G, w_edge, dqk_edge, dv, dk);
  }
  E2V2_LAUNCHED("k_attn_bwd_col");
  return 0;
}

static int check_table(const e2v2_attn_args& A, const char* who) {
  E2V2_REQUIRE(A.rtab && A.atom_type && A.n_types >= 1 && A.n_types <= E2V2_MAX_TYPES && A.rtab_n >= 2 &&
                   A.rtab_h > 0.f,
               "%s: needs the fc_easy table and atom types (n_types %d, rtab_n %d)", who, A.n_types, A.rtab_n);
  E2V2_REQUIRE((double)A.rc * (1.0 / A.rtab_h) <= (double)(A.rtab_n - 1),
               "%s: table of %d nodes (h %g) does not cover the cutoff %g", who, A.rtab_n, (double)A.rtab_h,
               (double)A.rc);
  return 0;
}

E2V2_API int e2v2_attn_bwd(const e2v2_attn_args* args, const void* grad_out, const void* out, const float* mrow,
                           const float* srow, const int32_t* cnt, float* ddvec, float* ddist, float* dq, float* dk,
                           float* dv, float* w_edge, float* dqk_edge, hipStream_t s) {
  const e2v2_attn_args& A = *args;
  E2V2_REQUIRE(A.n_heads == kH && A.head_dim == kD && A.channels == kC,
               "attn_bwd: built for H=%d D=%d C=%d", kH, kD, kC);
  E2V2_REQUIRE(!A.col_slot_member || (A.col_span == 4 && A.col_slot_edge && A.col_n_slots),
               "attn_bwd: column clusters need span 4 and all three slot arrays (span %d)", A.col_span);
  if (A.n_rows == 0) return 0;
  // the row pass gathers k_j and v_j through 32-bit byte offsets within one row block
  E2V2_REQUIRE((uint64_t)A.n_rows * kH * kD * (A.act_bf16 ? 2 : 4) < (1ull << 32),
               "attn_bwd: %d rows exceed the 32-bit gather offsets of the row pass", A.n_rows);
  if (int rc = check_table(A, "attn_bwd")) return rc;
  if (A.act_bf16)
    return attn_bwd_launch(A, static_cast<const __bf16*>(grad_out), static_cast<const __bf16*>(out), mrow, srow,
                           cnt, ddvec, ddist, dq, dk, dv, w_edge, dqk_edge, s);
  return attn_bwd_launch(A, static_cast<const float*>(grad_out), static_cast<const float*>(out), mrow, srow, cnt,
                         ddvec, ddist, dq, dk, dv, w_edge, dqk_edge, s);
}
