// Sparse equivariant attention of one E2Former-V2 layer on the query CSR.
//
// Forward (online segmented softmax per query atom i and head h):
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
// where they are used.
//
// Head slices: the 128 heads form 8 slices of 16.  The forward and the
// backward row pass run one wavefront per (query row, slice), slice =
// blockIdx % 8; workgroups are dispatched round-robin over the 8 XCDs, so XCD
// s runs every row of slice s in Morton order and its L2 holds slice s of the
// table and of the gathered k and v rows (a whole layer's table does not fit
// one XCD's 4 MB L2; one slice of its frequent type pairs does).  Channels of
// v, out, their gradients and the table are stored in slice order (position
// p holds the first or second channel of head pos_head(p); the header's
// E2V2_POS0 / E2V2_POS1), so a slice is one 128-byte run of every row.
// Backward, one head group (32 heads, two slices) at a time: row pass (dq, the
// group's edge weights w and dL/dqk, dvec/ddist partials per slice with the
// profile's distance derivative; the softmax row terms come from
// D_h = sum_{c in h} sum_t G[t,c] out[t,c]) and the group's column pass over the
// key CSR (dv_j, dk_j) with no atomics; then the slice partials are added per
// edge in slice order.
#include <type_traits>

#include "common.h"
#include "radial.h"
#include "tp_table.h"
#include "../../include/e2v2.h"

namespace e2v2 {

constexpr int kH = 128, kD = 8, kC = 256, kNV = 9, kNT = 20;
static_assert(kNT == kTpRows, "the coupling table's output rows");
constexpr float kEps = 1e-3f;
// Slice order of channel positions: position p holds the first (p % 32 < 16,
// model channel h) or second (model channel 128 + h) channel of head
// h = pos_head(p); slice s = p / 32 holds heads 16 s .. 16 s + 15.  In the
// fc_easy table the first channel of a head is its gate, the second its
// inputhead.
constexpr int kSl = 8, kSlH = kH / kSl, kSlC = kC / kSl;
__device__ __forceinline__ int pos_head(int p) { return ((p >> 5) << 4) | (p & 15); }
// Channel groups of the clustered column pass: group g holds heads
// 32 g .. 32 g + 31, i.e. the 64 positions 64 g .. 64 g + 63 (slices 2 g and
// 2 g + 1).  Lane l of a wave owns position 64 g + l, and dims 4 (l % 2) .. +3
// of head 32 g + l / 2 for dk.
constexpr int kGroups = 4, kGroupHeads = kH / kGroups, kGroupC = kC / kGroups;
// kernel variants (template bits): zero-order aggregation, bell envelope, the caller's gate, and the weight
// form: the segmented softmax (neither bit), or alpha = act(a) ih p with act softplus or sigmoid
// (tp_type "+softplus" / "+sigmoid", e2former.py:123-124, 329-334: no row maximum or sum)
constexpr int kModeZero = 1, kModeBell = 2, kModeExt = 4, kModeSoftplus = 8, kModeSigmoid = 16;
constexpr int kModeAct = kModeSoftplus | kModeSigmoid;

// The non-softmax weight activations and their derivatives: softplus as torch's F.softplus (beta 1,
// threshold 20: the identity above it), the logistic sigmoid.
template <int kAct>
__device__ __forceinline__ void weight_act(float a, float& f, float& df) {
  if constexpr (kAct == kModeSoftplus) {
    if (a > 20.f) {
      f = a;
      df = 1.f;
    } else {
      const float e = expf(a);
      f = log1pf(e);
      df = e / (1.f + e);
    }
  } else {
    const float sg = 1.f / (1.f + expf(-a));
    f = sg;
    df = sg * (1.f - sg);
  }
}
__device__ __forceinline__ Envelope make_env(const e2v2_attn_args& A) {
  Envelope E;
  E.rc = A.rc; E.a = A.env_a; E.b = A.env_b; E.c = A.env_c;
  E.lo = A.env_lo;
  return E;
}

// the fc_easy table: 256 channels per row in slice order (gate, inputhead of each head)
constexpr int kTabC = 2 * kH;
__device__ __forceinline__ RadialTab make_tab(const e2v2_attn_args& A) {
  RadialTab R;
  R.tab = A.rtab; R.n_types = A.n_types; R.n_nodes = A.rtab_n; R.nc = kTabC; R.inv_h = 1.0f / A.rtab_h;
  R.pair_slot = A.pair_slot;
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


// One edge's gathered operands for a head, kept in the storage type until the
// edge is applied (bf16: half the staging registers of converted values).
template <typename TS>
struct HeadEdge {
  TS k[kD];
  TS v0[kNV], v1[kNV];
  float tg[8], ti[8];   // table rows 0..3 at the lower and upper node: gate, inputhead
  float gx;             // the caller's gate (external-gate mode)
};
__device__ __forceinline__ void load8_raw(const float* p, float (&v)[8]) { load8(p, v); }
__device__ __forceinline__ void load8_raw(const __bf16* p, __bf16 (&v)[8]) {
  const bf16x8 a = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = a[i];
}


// Buffer resource over [base, base + bytes): vector loads at a 32-bit byte
// offset plus a wave-uniform scalar offset, no per-lane address arithmetic.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float buf_act(float*, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ float buf_act(__bf16*, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0) << 16);
}

// Forward, one wavefront per (query row i, slice s), i = blockIdx / 8,
// s = blockIdx % 8.  Per chunk of up to 32 edges: lane t < nc forms edge t's
// gather offsets, dvec, envelope, 1/d, table node and Hermite weights in LDS;
// lane (sub, hh) = (lane / 16, lane % 16) computes the logits of head 16 s + hh
// for the chunk's edges sub, sub + 4, ... (gate and inputhead interpolated from
// the slice-major table; a partial chunk repeats its last edge and masks it)
// and the head's online-softmax update (chunk max, count of maxima and sum
// combined over the four subs by lane swaps, the same order in every lane) and
// stages the edge weights ee ih / d; then lane (par, u) = (lane / 32, lane % 32)
// accumulates position 32 s + u over the chunk's edges of parity par (27
// accumulators: 9 rows of v times xyz).  In both loops the next edge's gathers
// are issued before the current edge is applied.  The two parities are added
// once per row in LDS, the coupling table is applied and the slice's 20
// output rows are written.
// kMode: bit kModeZero the zero-order aggregation (else first order), bit kModeBell the bell envelope (else
// the polynomial), bit kModeExt the caller's gate per (edge, head) (else the table's gate rows)
template <typename TS, int kMode>
__global__ __launch_bounds__(64) void k_attn_fwd_sl(e2v2_attn_args A, TS* __restrict__ out, float* __restrict__ mrow,
                                                    float* __restrict__ srow, int32_t* __restrict__ cnt) {
  constexpr bool kZ = kMode & kModeZero, kBell = kMode & kModeBell, kExt = kMode & kModeExt;
  constexpr int kAct = kMode & kModeAct;
  constexpr int CH = 32;               // edges per chunk
  __shared__ uint32_t ckof[CH];        // byte offsets of the edge's k row (head 16 s) and v rows (position 32 s)
  __shared__ uint32_t cvof[CH];
  __shared__ float4 cg[CH];            // dvec, envelope p
  __shared__ float crR[CH];            // 1 / max(d, 1e-6)
  __shared__ int64_t ctoff[CH];        // slice-s table offset of the lower node
  __shared__ float chw[6][CH];         // quintic Hermite weights of the edge's fraction in its node interval
  __shared__ float a_s[CH][kSlH];      // logits per (edge, head)
  __shared__ float coef_s[CH][kSlH];   // inputhead, then ee ih / d per (edge, head)
  __shared__ float sc_s[kSlH];         // rescale of the running sums per head
  __shared__ float red[kNV * 3][kSlC];
  const int s = blockIdx.x % kSl, i = blockIdx.x / kSl;
  if (i >= A.n_rows) return;
  const int lane = threadIdx.x;
  const int hh = lane & (kSlH - 1), sub = lane >> 4;
  const int u = lane & (kSlC - 1), par = lane >> 5, hu = u & (kSlH - 1);
  const int h = kSlH * s + hh;
  const int pu = kSlC * s + u;
  // gathers at 32-bit byte offsets: k through its base (n_rows * kH * kD * sizeof(TS) < 2^32 and
  // 9 n_rows * kC * sizeof(TS) < 2^32 are checked by the host), v through a buffer resource
  const char* __restrict__ Kb = static_cast<const char*>(A.k) + (size_t)hh * kD * sizeof(TS);
  const uint32_t vsb = (uint32_t)A.n_rows * kC * sizeof(TS);
  const __amdgpu_buffer_rsrc_t Vr = buf_rsrc(A.v, kNV * vsb);   // uniform base; the lane's column in voffset
  const uint32_t ub = (uint32_t)u * sizeof(TS);
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
  struct LogitIn {
    TS k[kD];
    float t[12];   // gate rows 0..2 at the two nodes, then inputhead
    float g;       // the caller's gate (external-gate mode)
  };
  for (int c0 = 0; c0 < n; c0 += CH) {
    const int nc = min(CH, n - c0);
    if (lane < nc) {
      const int64_t e = (int64_t)b + c0 + lane;
      const int j = A.col[e];
      const float d = A.dist[e];
      float p, dp;
      env.template eval<kBell>(d, p, dp);
      ckof[lane] = ((uint32_t)j * kH + kSlH * s) * (kD * sizeof(TS));
      cvof[lane] = ((uint32_t)j * kC + kSlC * s) * sizeof(TS);
      cg[lane] = make_float4(A.dvec[3 * e], A.dvec[3 * e + 1], A.dvec[3 * e + 2], p);
      crR[lane] = 1.0f / fmaxf(d, 1e-6f);
      float tt;
      ctoff[lane] = radial_node_sliced(R, tab_pair(R, ti, A.atom_type[j]), s, kSl, kSlC, d, tt);
      const Hermite5 Hw = hermite5(tt);
      chw[0][lane] = Hw.a0; chw[1][lane] = Hw.a1; chw[2][lane] = Hw.a2;
      chw[3][lane] = Hw.b0; chw[4][lane] = Hw.b1; chw[5][lane] = Hw.b2;
    }
    __syncthreads();
    // logits of head h for the edges sub, sub + 4, ... of the chunk (a missing edge repeats the last one and
    // is not stored)
    auto lload = [&](int k, LogitIn& X) {
      const int el = min(sub + 4 * k, nc - 1);
      load8_raw(reinterpret_cast<const TS*>(Kb + ckof[el]), X.k);
      // slice-s table: gate of head hh in column hh, inputhead in column 16 + hh; rows 0..2 at the two nodes
      const float* tg = R.tab + ctoff[el] + hh;
      constexpr int rs = kSlC, nb = 4 * kSlC;
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        if constexpr (!kExt) {
          X.t[q] = tg[q * rs];
          X.t[3 + q] = tg[nb + q * rs];
        }
        X.t[6 + q] = tg[kSlH + q * rs];
        X.t[9 + q] = tg[kSlH + nb + q * rs];
      }
      if constexpr (kExt) X.g = A.ext_gate[((int64_t)b + c0 + el) * kH + h];
    };
    auto lapply = [&](int k, const LogitIn& X) {
      const int el = sub + 4 * k;
      if (el >= nc) return;
      float kf[kD];
#pragma unroll
      for (int q = 0; q < kD; ++q) kf[q] = f32(X.k[q]);
      const float qk = half_dot(qs, kf) + half_dot(qs + 4, kf + 4);
      Hermite5 Hw;
      Hw.a0 = chw[0][el]; Hw.a1 = chw[1][el]; Hw.a2 = chw[2][el];
      Hw.b0 = chw[3][el]; Hw.b1 = chw[4][el]; Hw.b2 = chw[5][el];
      const float gate = kExt ? X.g : herm_value(Hw, X.t[0], X.t[1], X.t[2], X.t[3], X.t[4], X.t[5]);
      a_s[el][hh] = gate * qk;
      coef_s[el][hh] = herm_value(Hw, X.t[6], X.t[7], X.t[8], X.t[9], X.t[10], X.t[11]);
    };
    {
      const int ke = (nc + 3) / 4;   // logit steps of this chunk (the subs of a step share it)
      LogitIn Xa, Xb;
      lload(0, Xa);
      int k = 0;
      for (; k + 2 < ke; k += 2) {
        lload(k + 1, Xb);
        lapply(k, Xa);
        lload(k + 2, Xa);
        lapply(k + 1, Xb);
      }
      if (k + 1 < ke) {
        lload(k + 1, Xb);
        lapply(k, Xa);
        lapply(k + 1, Xb);
      } else {
        lapply(k, Xa);
      }
    }
    if constexpr (kAct != 0) {
      // alpha = act(a) ih p: no statistics, nothing to rescale
      for (int el = sub; el < nc; el += 4) {
        float f, df;
        weight_act<kAct>(a_s[el][hh], f, df);
        const float ee = f * cg[el].w;
        coef_s[el][hh] = kZ ? ee * coef_s[el][hh] : (ee * coef_s[el][hh]) * crR[el];
      }
      if (sub == 0) sc_s[hh] = 1.f;
    } else {
    // online softmax of head h over the chunk (each lane reads back the logits it wrote)
    float cm = -INFINITY;
    for (int el = sub; el < nc; el += 4) cm = fmaxf(cm, a_s[el][hh]);
    cm = fmaxf(cm, __shfl_xor(cm, 16, kWave));
    cm = fmaxf(cm, __shfl_xor(cm, 32, kWave));
    const float m_new = fmaxf(m_run, cm);
    const float sc = (m_run == -INFINITY) ? 0.f : fexp(m_run - m_new);
    int cc = 0;
    float ls = 0.f;
    for (int el = sub; el < nc; el += 4) {
      const float av = a_s[el][hh];
      cc += (av == m_new);
      const float ee = fexp(av - m_new) * cg[el].w;
      ls += ee;
      coef_s[el][hh] = kZ ? ee * coef_s[el][hh] : (ee * coef_s[el][hh]) * crR[el];
    }
    cc += __shfl_xor(cc, 16, kWave);
    cc += __shfl_xor(cc, 32, kWave);
    ls += __shfl_xor(ls, 16, kWave);
    ls += __shfl_xor(ls, 32, kWave);
    c_run = (m_new == m_run) ? c_run + cc : cc;
    s_run = s_run * sc + ls;
    m_run = m_new;
    if (sub == 0) sc_s[hh] = sc;
    }
    __syncthreads();
    // value aggregation of position 32 s + u over the edges of parity par
    const float scu = sc_s[hu];
    if (scu != 1.f) {
#pragma unroll
      for (int r = 0; r < kNV; ++r) {
        acc[r][0] *= scu; acc[r][1] *= scu; acc[r][2] *= scu;
      }
    }
    auto vload = [&](int el, float (&vv)[kNV]) {
      const uint32_t vof = cvof[el] + ub;
#pragma unroll
      for (int r = 0; r < kNV; ++r) vv[r] = buf_act(static_cast<TS*>(nullptr), Vr, vof, (uint32_t)r * vsb);
    };
    auto vapply = [&](int el, const float (&vv)[kNV]) {
      const float w = coef_s[el][hu];
      if constexpr (kZ) {
#pragma unroll
        for (int r = 0; r < kNV; ++r) acc[r][0] = fmaf(vv[r], w, acc[r][0]);
      } else {
        const float4 g = cg[el];
        const float wx = w * g.x, wy = w * g.y, wz = w * g.z;
#pragma unroll
        for (int r = 0; r < kNV; ++r) {
          acc[r][0] = fmaf(vv[r], wx, acc[r][0]);
          acc[r][1] = fmaf(vv[r], wy, acc[r][1]);
          acc[r][2] = fmaf(vv[r], wz, acc[r][2]);
        }
      }
    };
    int el = par;
    if (el < nc) {
      float va[kNV], vb[kNV];
      vload(el, va);
      for (; el + 4 < nc; el += 4) {
        vload(el + 2, vb);
        vapply(el, va);
        vload(el + 4, va);
        vapply(el + 2, vb);
      }
      if (el + 2 < nc) {
        vload(el + 2, vb);
        vapply(el, va);
        vapply(el + 2, vb);
      } else {
        vapply(el, va);
      }
    }
    __syncthreads();
  }
  if (par) {
#pragma unroll
    for (int r = 0; r < kNV; ++r) {
      red[3 * r][u] = acc[r][0]; red[3 * r + 1][u] = acc[r][1]; red[3 * r + 2][u] = acc[r][2];
    }
  }
  __syncthreads();
  if (!par) {
#pragma unroll
    for (int r = 0; r < kNV; ++r) {
      acc[r][0] += red[3 * r][u]; acc[r][1] += red[3 * r + 1][u]; acc[r][2] += red[3 * r + 2][u];
    }
    // this lane (sub = u / 16, hh = u % 16) holds the statistics of head 16 s + hu
    const float inv = kAct ? 1.0f : 1.0f / (s_run + kEps);   // (no normalisation for the act forms)
    if constexpr (kZ) {
      // zero order: the aggregated rows themselves, m-major [9][N][C]
      const size_t os = (size_t)A.n_rows * kC;
#pragma unroll
      for (int r = 0; r < kNV; ++r) store_act(acc[r][0] * inv, out + r * os + (size_t)i * kC + pu);
    } else {
      float o[kNT];
#pragma unroll
      for (int q = 0; q < kNT; ++q) o[q] = 0.f;
#pragma unroll
      for (int z = 0; z < kTpNnz; ++z) o[kTp[z].t] = fmaf(kTp[z].c, acc[kTp[z].r][kTp[z].k], o[kTp[z].t]);
      const size_t nr = (size_t)A.n_rows;
#pragma unroll
      for (int q = 0; q < kNT; ++q)
        store_act(o[q] * inv, out + nr * kRowA[q] + (size_t)i * kRowLd[q] + kRowCol[q] + pu);
    }
  }
  if (lane < kSlH) {
    mrow[(size_t)i * kH + h] = kAct ? 0.f : m_run;
    srow[(size_t)i * kH + h] = s_run;
    cnt[(size_t)i * kH + h] = c_run;
  }
}

// dA[r][k] = sum_t T[t][r][k] g[t] for one channel
__device__ __forceinline__ void tp_transpose(const float (&g)[kNT], float (&dA)[kNV][3]) {
#pragma unroll
  for (int r = 0; r < kNV; ++r) dA[r][0] = dA[r][1] = dA[r][2] = 0.f;
#pragma unroll
  for (int z = 0; z < kTpNnz; ++z) dA[kTp[z].r][kTp[z].k] = fmaf(kTp[z].c, g[kTp[z].t], dA[kTp[z].r][kTp[z].k]);
}

// Column pass of channel group g (heads 32 g .. 32 g + 31, positions 64 g .. 64 g
// + 63; G and q in fp32 or bf16, sums in fp32) over clusters of R consecutive
// key-CSR columns: the workgroups of one XCD run a contiguous range of clusters,
// so the gathered rows of a column window stay in its L2.  Wave w applies the
// slots s = w mod 4 of each chunk (lane = channel of the group; for dk lane =
// (head, half of the head's dims)); the four waves' partial sums are added once
// per cluster in LDS in a fixed order.  Every slot's G_i and q_i are loaded once
// and applied to each column of the cluster that it joins.  With kSlots the
// slots come from e2v2_cluster_slots (R = 4); without, R = 1 and the slots of
// column j are its key-CSR edges.  w_g and dqk_g hold the group's 32 heads per
// edge ([E][32]), written by the row pass of the same group.
template <int R, typename TS, bool kSlots, int kMode>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(sizeof(TS) == 4 ? 2 : 3))) void k_attn_bwd_col_grp(
    e2v2_attn_args A, const TS* __restrict__ G, const float* __restrict__ w_g, const float* __restrict__ dqk_g,
    float* __restrict__ dv_out, float* __restrict__ dk_out, int grp) {
  constexpr bool kZ = kMode & kModeZero;
  static_assert(kSlots || R == 1, "columns without slots are clusters of one");
  constexpr int S = 32;                        // slots per staged chunk
  __shared__ int ci[S];
  __shared__ int ce[S][R];
  __shared__ float cdv[S][R][3];
  __shared__ float red[2][R][kNV + 4][kWave];  // per-wave partial sums, added in two rounds
  const int n_cl = (A.n_rows + R - 1) / R;
  const int cl = xcd_row(blockIdx.x, n_cl);
  if (cl >= n_cl) return;
  const int t = threadIdx.x, lane = t & (kWave - 1), wave = t >> 6;
  const int c = kGroupC * grp + lane;   // channel position
  const int hc = pos_head(c) - kGroupHeads * grp;                     // its head within the group
  const int hkg = lane >> 1, hk = kGroupHeads * grp + hkg, d0 = 4 * (lane & 1);
  const int j0 = cl * R, nj = min(R, A.n_rows - j0);
  const size_t os = (size_t)A.n_rows * kC;
  const int64_t base = A.key_ptr[j0];
  const int ns = kSlots ? A.col_n_slots[cl] : A.key_ptr[j0 + 1] - (int)base;
  const int32_t* __restrict__ smem = kSlots ? A.col_slot_member + base : nullptr;
  const int32_t* __restrict__ sedge = kSlots ? A.col_slot_edge + base * R : nullptr;
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
  constexpr int NG = kZ ? kNV : kNT;   // rows of the output gradient
  struct Loads {
    TS g[NG];   // converted to fp32 in apply()
    float q[4];
    float w[R];
    float dq[R];
  };
  auto issue = [&](int sl, Loads& L) {
    const int i = ci[sl];
#pragma unroll
    for (int z = 0; z < NG; ++z)
      L.g[z] = kZ ? G[z * os + (size_t)i * kC + c]
                  : G[(size_t)A.n_rows * kRowA[z] + (size_t)i * kRowLd[z] + kRowCol[z] + c];
    load4(Qp + ((size_t)i * kH + hk) * kD + d0, L.q);
    // unconditional (an absent edge reads edge 0, unused): every slot issues the
    // same loads, so the wait before apply() counts only the older slot's
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t e = max(ce[sl][r], 0);
      L.w[r] = ntload(w_g + e * kGroupHeads + hc);
      L.dq[r] = ntload(dqk_g + e * kGroupHeads + hkg);
    }
  };
  auto apply = [&](int sl, const Loads& L) {
    float g[NG], dA[kNV][3];
#pragma unroll
    for (int z = 0; z < NG; ++z) g[z] = static_cast<float>(L.g[z]);
    if constexpr (!kZ) tp_transpose(g, dA);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (ce[sl][r] >= 0) {
        const float w = L.w[r];
        if constexpr (kZ) {
#pragma unroll
          for (int z = 0; z < kNV; ++z) av[r][z] = fmaf(g[z], w, av[r][z]);
        } else {
          const float wx = w * cdv[sl][r][0], wy = w * cdv[sl][r][1], wz = w * cdv[sl][r][2];
#pragma unroll
          for (int z = 0; z < kNV; ++z)
            av[r][z] = fmaf(dA[z][2], wz, fmaf(dA[z][1], wy, fmaf(dA[z][0], wx, av[r][z])));
        }
#pragma unroll
        for (int d = 0; d < 4; ++d) ak[r][d] = fmaf(L.dq[r], L.q[d], ak[r][d]);
      }
    }
  };
  for (int s0 = 0; s0 < ns; s0 += S) {
    const int nc = min(S, ns - s0);
    if (t < nc) ci[t] = kSlots ? smem[s0 + t] : A.edge_row[A.key_eid[base + s0 + t]];
    for (int idx = t; idx < nc * R; idx += 256) {
      const int sl = idx / R, r = idx % R;
      const int e = kSlots ? sedge[(int64_t)(s0 + sl) * R + r] : A.key_eid[base + s0 + sl];
      ce[sl][r] = e;
      if (!kZ && e >= 0) {
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

// Sums over the 16 lanes of each row of the wave of four values: quad q of the
// row (lanes 4 q .. 4 q + 3) returns the sum of value q.  Lanes 0..7 of a row
// keep values 0, 1 and lanes 8..15 values 2, 3, each adding its partner's
// (lane ^ 8: row rotation by 8); then within each half row lanes 0..3 keep the
// first and lanes 4..7 the second (partner 7 - lane: half-row mirror); two
// quad permutes finish the sums.  Fixed order, the same in every row.
__device__ __forceinline__ float row_sum4(float v0, float v1, float v2, float v3, int lane) {
  const bool hi8 = (lane & 8) != 0, hi4 = (lane & 4) != 0;
  const float k0 = hi8 ? v2 : v0, k1 = hi8 ? v3 : v1;
  const float s0 = hi8 ? v0 : v2, s1 = hi8 ? v1 : v3;
  const float x0 = k0 + dpp_mov<0x128>(s0);   // row_ror:8
  const float x1 = k1 + dpp_mov<0x128>(s1);
  float y = (hi4 ? x1 : x0) + dpp_mov<0x141>(hi4 ? x0 : x1);   // row_half_mirror
  y += dpp_mov<0x4E>(y);   // quad_perm [2,3,0,1]
  y += dpp_mov<0xB1>(y);   // quad_perm [1,0,3,2]
  return y;
}

// Backward row pass, one wavefront per (query row i, slice s) as in the
// forward.  Lane (sub, hh) owns head h = 16 s + hh with both of its channel
// positions and the row's edges sub, sub + 4, ...  Per edge it interpolates the
// head's gate and inputhead and their distance derivatives, recomputes the
// logit and weight, forms u = dA^T v_j for both channels (dA = T^T G_i, formed
// once per row) and with it the head's dL/dw, runs the softmax / gate /
// distance backward (dL/dgate gate' + dL/dih ih' included; the softmax row
// terms from D_h and the exact amax gradient split over ties), accumulates dq
// from the k_j row it already holds and writes the edge's w and dL/dqk for the
// column pass.  The sums over the slice's 16 heads of dL/d dvec and dL/dd are
// formed within each 16-lane row (row_sum4) and written as the slice's partial
// part[s][e][0..3].  The head-independent terms of up to 64 edges (column,
// distance, envelope, 1/d, dvec, table node and fraction) are formed once per
// chunk in LDS, and the next edge's gathers are issued before the current one
// is applied.
template <typename TS, int kMode>
__global__ __launch_bounds__(64) void k_attn_bwd_row_sl(e2v2_attn_args A, const TS* __restrict__ G,
                                                        const TS* __restrict__ O, const float* __restrict__ mrow,
                                                        const float* __restrict__ srow,
                                                        const int32_t* __restrict__ cnt, float* __restrict__ part,
                                                        float* __restrict__ dq, float* __restrict__ w_out,
                                                        float* __restrict__ dqk_out, int grp) {
  constexpr bool kZ = kMode & kModeZero, kBell = kMode & kModeBell, kExt = kMode & kModeExt;
  constexpr int kAct = kMode & kModeAct;
  constexpr int CH = 64;
  __shared__ float4 er_a[CH];      // p, dp/dd, 1/max(d, 1e-6), d
  __shared__ float4 er_b[CH];      // dvec, column (int bits)
  __shared__ int64_t er_toff[CH];  // slice-s table offset of the lower node
  __shared__ float er_hw[6][CH];   // quintic Hermite weights of the fraction in the node interval
  // slice 2 grp on the even XCDs (blockIdx % 8 = 0, 2, 4, 6), 2 grp + 1 on the odd ones; the four XCDs of a
  // slice take contiguous quarters of the rows, each in order, so an XCD's rows stay spatially compact
  const int x = blockIdx.x % kXcd, quarter = (A.n_rows + 3) / 4;
  const int s = 2 * grp + (x & 1), i = (x >> 1) * quarter + (int)(blockIdx.x / kXcd);
  if (blockIdx.x / kXcd >= (unsigned)quarter || i >= A.n_rows) return;
  const int lane = threadIdx.x, hh = lane & (kSlH - 1), sub = lane >> 4;
  const int h = kSlH * s + hh;
  const int hg = h - kGroupHeads * grp;   // head within the group (w, dqk columns)
  const int p0 = kSlC * s + hh, p1 = p0 + kSlH;   // the head's two channel positions
  const RadialTab R = make_tab(A);
  const int ti = A.atom_type[i];
  const TS* __restrict__ Kp = static_cast<const TS*>(A.k);
  const TS* __restrict__ Vp = static_cast<const TS*>(A.v);
  const size_t os = (size_t)A.n_rows * kC;
  const int b = A.row_ptr[i], n = A.row_ptr[i + 1] - b;
  const Envelope env = make_env(A);
  // per-row prologue: dA of both channels, D_h, softmax statistics of head h
  float dA0[kNV][3], dA1[kNV][3];
  float inv, dsum, dmc, m;
  {
    constexpr int NG = kZ ? kNV : kNT;   // output rows: 9 (zero order) or the 20 l3-grouped ones
    float g0[NG], g1[NG];
    const size_t nr = (size_t)A.n_rows;
    auto row_at = [&](int z) -> size_t {
      return kZ ? z * os + (size_t)i * kC : nr * kRowA[z] + (size_t)i * kRowLd[z] + kRowCol[z];
    };
#pragma unroll
    for (int z = 0; z < NG; ++z) {
      const size_t rz = row_at(z);
      g0[z] = f32(G[rz + p0]);
      g1[z] = f32(G[rz + p1]);
    }
    // D_h = sum over the head's two channels and the output rows, summed as the first channel then the second
    // (the softmax row term; the act forms have none)
    float d0 = 0.f, d1 = 0.f;
    if constexpr (kAct == 0) {
#pragma unroll
      for (int z = 0; z < NG; ++z) {
        const size_t rz = row_at(z);
        d0 = fmaf(g0[z], f32(O[rz + p0]), d0);
        d1 = fmaf(g1[z], f32(O[rz + p1]), d1);
      }
    }
    const float Dh = d1 + d0;
    if constexpr (kZ) {
      // zero order: u = G_i . v_j per channel, dA = G itself (component 0)
#pragma unroll
      for (int r = 0; r < kNV; ++r) {
        dA0[r][0] = g0[r]; dA0[r][1] = dA0[r][2] = 0.f;
        dA1[r][0] = g1[r]; dA1[r][1] = dA1[r][2] = 0.f;
      }
    } else {
      tp_transpose(g0, dA0);
      tp_transpose(g1, dA1);
    }
    if constexpr (kAct != 0) {
      m = 0.f; inv = 1.f; dsum = 0.f; dmc = 0.f;
    } else {
      m = mrow[(size_t)i * kH + h];
      const float sr = srow[(size_t)i * kH + h];
      const int cn = cnt[(size_t)i * kH + h];
      inv = 1.0f / (sr + kEps);
      dsum = Dh * inv;
      dmc = cn > 0 ? (-Dh * kEps * inv) / (float)cn : 0.f;
    }
  }
  float qs[kD];
  load_qs<TS>(A, i, h, qs);
  float dqa[kD];
#pragma unroll
  for (int d = 0; d < kD; ++d) dqa[d] = 0.f;
  using L = HeadEdge<TS>;
  int c0 = 0;  // first edge of the current chunk
  auto issue = [&](int sl, L& X) {
    const int j = __float_as_int(er_b[sl].w);
    // 32-bit per-lane byte offsets from wave-uniform bases (n_rows * kH * kD * sizeof(TS) < 2^32, which
    // bounds the v offsets too, is checked by the host)
    const uint32_t kof = ((uint32_t)j * kH + h) * (kD * sizeof(TS));
    load8_raw(reinterpret_cast<const TS*>(reinterpret_cast<const char*>(Kp) + kof), X.k);
    const uint32_t vof = ((uint32_t)j * kC + p0) * sizeof(TS);
#pragma unroll
    for (int r = 0; r < kNV; ++r) {
      const char* vb = reinterpret_cast<const char*>(Vp + r * os);
      X.v0[r] = *reinterpret_cast<const TS*>(vb + vof);
      X.v1[r] = *reinterpret_cast<const TS*>(vb + vof + kSlH * sizeof(TS));
    }
    // slice-s table: gate of head hh in column hh, inputhead in column 16 + hh; rows 0..3 at the two nodes
    const float* tb = R.tab + er_toff[sl] + hh;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if constexpr (!kExt) {
        X.tg[q] = tb[q * kSlC];
        X.tg[4 + q] = tb[(4 + q) * kSlC];
      }
      X.ti[q] = tb[q * kSlC + kSlH];
      X.ti[4 + q] = tb[(4 + q) * kSlC + kSlH];
    }
    if constexpr (kExt) X.gx = A.ext_gate[((int64_t)b + c0 + sl) * kH + h];
  };
  auto apply = [&](int sl, const L& X) {
    const int64_t e = (int64_t)b + c0 + sl;
    const float4 ea = er_a[sl], eb = er_b[sl];
    const float pe = ea.x, dpe = ea.y, rR = ea.z, d = ea.w;
    const float dvx = eb.x, dvy = eb.y, dvz = eb.z;
    Hermite5 Hw;
    Hw.a0 = er_hw[0][sl]; Hw.a1 = er_hw[1][sl]; Hw.a2 = er_hw[2][sl];
    Hw.b0 = er_hw[3][sl]; Hw.b1 = er_hw[4][sl]; Hw.b2 = er_hw[5][sl];
    const float gate = kExt ? X.gx : herm_value(Hw, X.tg[0], X.tg[1], X.tg[2], X.tg[4], X.tg[5], X.tg[6]);
    const float ih = herm_value(Hw, X.ti[0], X.ti[1], X.ti[2], X.ti[4], X.ti[5], X.ti[6]);
    const float gate_d =
        kExt ? 0.f : herm_value(Hw, X.tg[1], X.tg[2], X.tg[3], X.tg[5], X.tg[6], X.tg[7]) * R.inv_h;
    const float ih_d = herm_value(Hw, X.ti[1], X.ti[2], X.ti[3], X.ti[5], X.ti[6], X.ti[7]) * R.inv_h;
    float kf[kD];
#pragma unroll
    for (int q = 0; q < kD; ++q) kf[q] = f32(X.k[q]);
    const float qk = half_dot(qs, kf) + half_dot(qs + 4, kf + 4);
    const float a = gate * qk;
    // softmax: ex = exp(a - m), d ex/da = ex; act forms: ex = act(a), d ex/da = act'(a)
    float ex, dex;
    if constexpr (kAct != 0) {
      weight_act<kAct>(a, ex, dex);
    } else {
      ex = fexp(a - m);
      dex = ex;
    }
    const float ee = ex * pe;
    const float alpha = (ee * ih) * inv;
    const float w = kZ ? alpha : alpha * rR;
    float U[3];
#pragma unroll
    for (int k = 0; k < (kZ ? 1 : 3); ++k) {
      float u0 = 0.f, u1 = 0.f;
#pragma unroll
      for (int r = 0; r < kNV; ++r) {
        u0 = fmaf(dA0[r][k], f32(X.v0[r]), u0);
        u1 = fmaf(dA1[r][k], f32(X.v1[r]), u1);
      }
      U[k] = u0 + u1;
    }
    if constexpr (kZ) U[1] = U[2] = 0.f;
    // zero order: the weight is alpha itself and the output does not depend on dvec directly
    const float dw = kZ ? U[0] : U[0] * dvx + U[1] * dvy + U[2] * dvz;
    const float dalpha = kZ ? dw : dw * rR;
    const float dR = (!kZ && d > 1e-6f) ? -dalpha * alpha * rR : 0.f;
    const float dih = dalpha * ee * inv;
    const float de = dalpha * ih * inv - dsum;
    float da = de * (dex * pe);
    if (kAct == 0 && a == m) da += dmc;
    const float dpv = de * ex;
    const float dqk = da * gate;
    ntstore(w, w_out + e * kGroupHeads + hg);
    ntstore(dqk, dqk_out + e * kGroupHeads + hg);
    if constexpr (kExt) ntstore(da * qk, A.ext_dgate + e * kH + h);   // dL/dgate
#pragma unroll
    for (int q = 0; q < kD; ++q) dqa[q] = fmaf(dqk, kf[q], dqa[q]);
    // dL/dd of this head: envelope, 1/d, and the profile (dL/dgate gate' + dL/dih ih')
    // (external gate: its distance dependence is the caller's)
    const float ddh = kExt ? fmaf(dih, ih_d, fmaf(dpv, dpe, dR)) : fmaf(da * qk, gate_d, fmaf(dih, ih_d, fmaf(dpv, dpe, dR)));
    // sums over the slice's 16 heads (this row of 16 lanes); quad q holds value q
    const float sum = row_sum4(kZ ? 0.f : w * U[0], w * U[1], w * U[2], ddh, lane);
    if ((lane & 3) == 0) part[((size_t)s * A.n_edges + e) * 4 + (hh >> 2)] = sum;
  };
  for (c0 = 0; c0 < n; c0 += CH) {
    const int nc = min(CH, n - c0);
    if (lane < nc) {
      const int64_t e = (int64_t)b + c0 + lane;
      const float d = A.dist[e];
      float pe, dpe;
      env.template eval<kBell>(d, pe, dpe);
      er_a[lane] = make_float4(pe, dpe, 1.0f / fmaxf(d, 1e-6f), d);
      const int j = A.col[e];
      er_b[lane] = make_float4(A.dvec[3 * e], A.dvec[3 * e + 1], A.dvec[3 * e + 2], __int_as_float(j));
      float tt;
      er_toff[lane] = radial_node_sliced(R, tab_pair(R, ti, A.atom_type[j]), s, kSl, kSlC, d, tt);
      const Hermite5 Hw = hermite5(tt);
      er_hw[0][lane] = Hw.a0; er_hw[1][lane] = Hw.a1; er_hw[2][lane] = Hw.a2;
      er_hw[3][lane] = Hw.b0; er_hw[4][lane] = Hw.b1; er_hw[5][lane] = Hw.b2;
    }
    __syncthreads();
    {
      // the 16 lanes of a row share their edges (sub), so the row sums see whole rows
      L Xa, Xb;
      int el = sub;
      if (el < nc) {
        issue(el, Xa);
        for (; el + 8 < nc; el += 8) {
          issue(el + 4, Xb);
          apply(el, Xa);
          issue(el + 8, Xa);
          apply(el + 4, Xb);
        }
        if (el + 4 < nc) {
          issue(el + 4, Xb);
          apply(el, Xa);
          apply(el + 4, Xb);
        } else {
          apply(el, Xa);
        }
      }
    }
    __syncthreads();
  }
  // dq of head h: the four subs added in a fixed order
#pragma unroll
  for (int q = 0; q < kD; ++q) {
    dqa[q] += __shfl_xor(dqa[q], 16, kWave);
    dqa[q] += __shfl_xor(dqa[q], 32, kWave);
  }
  if (sub == 0) {
#pragma unroll
    for (int q = 0; q < kD; ++q) dq[((size_t)i * kH + h) * kD + q] = dqa[q] / A.q_div;
  }
}

}  // namespace e2v2

using namespace e2v2;

// kernel variant of the arguments (combinations checked by check_table): the bell only with zero order
static int kernel_mode(const e2v2_attn_args& A) {
  return (A.zero_order ? kModeZero : 0) | (A.env_kind ? kModeBell : 0) | (A.ext_gate ? kModeExt : 0) |
         (A.weight_act == 1 ? kModeSoftplus : A.weight_act == 2 ? kModeSigmoid : 0);
}

// Calls f(integral_constant<int, mode>) for the instantiated variants: {0, Z, Z|B, E, E|Z, E|Z|B} with each of
// the three weight forms.
template <int kA, typename F>
static int with_shape(int mode, F&& f) {
  switch (mode & ~kModeAct) {
    case 0: return f(std::integral_constant<int, kA>{});
    case kModeZero: return f(std::integral_constant<int, kA | kModeZero>{});
    case kModeZero | kModeBell: return f(std::integral_constant<int, kA | kModeZero | kModeBell>{});
    case kModeExt: return f(std::integral_constant<int, kA | kModeExt>{});
    case kModeExt | kModeZero: return f(std::integral_constant<int, kA | kModeExt | kModeZero>{});
    case kModeExt | kModeZero | kModeBell:
      return f(std::integral_constant<int, kA | kModeExt | kModeZero | kModeBell>{});
    default: return ::e2v2::set_error(-1, "attention variant %d is not built", mode);
  }
}

template <typename F>
static int with_mode(int mode, F&& f) {
  switch (mode & kModeAct) {
    case 0: return with_shape<0>(mode, f);
    case kModeSoftplus: return with_shape<kModeSoftplus>(mode, f);
    case kModeSigmoid: return with_shape<kModeSigmoid>(mode, f);
    default: return ::e2v2::set_error(-1, "attention variant %d is not built", mode);
  }
}

static int check_table(const e2v2_attn_args& A, const char* who) {
  E2V2_REQUIRE((A.zero_order == 0 || A.zero_order == 1) && (A.env_kind == 0 || A.env_kind == 1) &&
                   (A.env_kind == 0 || (A.zero_order == 1 && A.env_lo >= 0.f && A.env_lo < A.rc)),
               "%s: zero_order %d with envelope kind %d (lo %g, rc %g) is not supported (the bell envelope is "
               "built for the zero-order layers)", who, A.zero_order, A.env_kind, (double)A.env_lo, (double)A.rc);
  E2V2_REQUIRE(A.weight_act >= 0 && A.weight_act <= 2, "%s: weight form %d (0 softmax, 1 softplus, 2 sigmoid)",
               who, A.weight_act);
  E2V2_REQUIRE(A.rtab && A.atom_type && A.n_types >= 1 && A.n_types <= E2V2_MAX_TYPES && A.rtab_n >= 2 &&
                   A.rtab_h > 0.f,
               "%s: needs the fc_easy table and atom types (n_types %d, rtab_n %d)", who, A.n_types, A.rtab_n);
  E2V2_REQUIRE((double)A.rc * (1.0 / A.rtab_h) <= (double)(A.rtab_n - 1),
               "%s: table of %d nodes (h %g) does not cover the cutoff %g", who, A.rtab_n, (double)A.rtab_h,
               (double)A.rc);
  // one wavefront per (row, slice): the grid holds 8 n_rows workgroups
  E2V2_REQUIRE(A.n_rows < (1 << 27), "%s: %d rows exceed the slice grid", who, A.n_rows);
  // the forward and the row pass gather k_j and v_j through 32-bit byte offsets (v: all 9 rows)
  E2V2_REQUIRE((uint64_t)A.n_rows * kH * kD * (A.act_bf16 ? 2 : 4) < (1ull << 32) &&
                   (uint64_t)A.n_rows * kNV * kC * (A.act_bf16 ? 2 : 4) < (1ull << 32),
               "%s: %d rows exceed the 32-bit gather offsets", who, A.n_rows);
  return 0;
}

E2V2_API int e2v2_attn_fwd(const e2v2_attn_args* args, void* out, float* mrow, float* srow, int32_t* cnt,
                           hipStream_t s) {
  const e2v2_attn_args& A = *args;
  E2V2_REQUIRE(A.n_heads == kH && A.head_dim == kD && A.channels == kC,
               "attn_fwd: built for H=%d D=%d C=%d, got H=%d D=%d C=%d", kH, kD, kC, A.n_heads, A.head_dim,
               A.channels);
  if (A.n_rows == 0) return 0;
  if (int rc = check_table(A, "attn_fwd")) return rc;
  const dim3 grid((unsigned)A.n_rows * kSl);
  return with_mode(kernel_mode(A), [&](auto md) -> int {
    constexpr int kM = decltype(md)::value;
    if (A.act_bf16)
      hipLaunchKernelGGL((k_attn_fwd_sl<__bf16, kM>), grid, dim3(kWave), 0, s, A, static_cast<__bf16*>(out), mrow,
                         srow, cnt);
    else
      hipLaunchKernelGGL((k_attn_fwd_sl<float, kM>), grid, dim3(kWave), 0, s, A, static_cast<float*>(out), mrow,
                         srow, cnt);
    E2V2_LAUNCHED("k_attn_fwd_sl");
    return 0;
  });
}

// workspace of e2v2_attn_bwd: w [E][32] and dL/dqk [E][32] of one head group, handed from that group's row
// pass to its column pass, and the slice partials of dL/d dvec, dL/dd [8][E][4]
static size_t bwd_ws_floats(int64_t n_edges) { return (size_t)n_edges * (2 * kGroupHeads + 4 * kSl); }

E2V2_API size_t e2v2_attn_bwd_workspace(int64_t n_edges) {
  return n_edges > 0 ? bwd_ws_floats(n_edges) * sizeof(float) : 0;
}

// The four head groups in turn: the row pass of the group's two slices, then its column pass (clusters when
// given, else one column per workgroup); finally the slice partials are added per edge.
template <typename TS, int kMode>
static int attn_bwd_launch(const e2v2_attn_args& A, const TS* G, const TS* O, const float* mrow, const float* srow,
                           const int32_t* cnt, float* ddvec, float* ddist, float* dq, float* dk, float* dv,
                           float* ws, hipStream_t s) {
  const int64_t E = A.n_edges;
  float* w_g = ws;
  float* dqk_g = ws + (size_t)E * kGroupHeads;
  float* part = ws + (size_t)E * 2 * kGroupHeads;
  for (int g = 0; g < kGroups; ++g) {
    hipLaunchKernelGGL((k_attn_bwd_row_sl<TS, kMode>), dim3((unsigned)((A.n_rows + 3) / 4) * kXcd), dim3(kWave), 0, s, A, G, O,
                       mrow, srow, cnt, part, dq, w_g, dqk_g, g);
    E2V2_LAUNCHED("k_attn_bwd_row_sl");
    if (A.col_slot_member) {
      const int n_cl = (A.n_rows + 3) / 4;
      hipLaunchKernelGGL((k_attn_bwd_col_grp<4, TS, true, kMode & kModeZero>), dim3(xcd_grid(n_cl)), dim3(256), 0, s, A, G, w_g, dqk_g,
                         dv, dk, g);
    } else {
      hipLaunchKernelGGL((k_attn_bwd_col_grp<1, TS, false, kMode & kModeZero>), dim3(xcd_grid(A.n_rows)), dim3(256), 0, s, A, G, w_g,
                         dqk_g, dv, dk, g);
    }
    E2V2_LAUNCHED("k_attn_bwd_col_grp");
  }
  return launch_edge_part_sum(part, E, ddvec, ddist, s);
}

E2V2_API int e2v2_attn_bwd(const e2v2_attn_args* args, const void* grad_out, const void* out, const float* mrow,
                           const float* srow, const int32_t* cnt, float* ddvec, float* ddist, float* dq, float* dk,
                           float* dv, void* workspace, size_t workspace_bytes, hipStream_t s) {
  const e2v2_attn_args& A = *args;
  E2V2_REQUIRE(A.n_heads == kH && A.head_dim == kD && A.channels == kC,
               "attn_bwd: built for H=%d D=%d C=%d", kH, kD, kC);
  E2V2_REQUIRE(!A.col_slot_member || (A.col_span == 4 && A.col_slot_edge && A.col_n_slots),
               "attn_bwd: column clusters need span 4 and all three slot arrays (span %d)", A.col_span);
  if (A.n_rows == 0) return 0;
  if (int rc = check_table(A, "attn_bwd")) return rc;
  const size_t need = e2v2_attn_bwd_workspace(A.n_edges);
  E2V2_REQUIRE(workspace_bytes >= need && (need == 0 || workspace) &&
                   reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
               "attn_bwd: workspace of %zu bytes (16-byte aligned) needed, got %zu", need, workspace_bytes);
  float* ws = static_cast<float*>(workspace);
  const auto* Gb = static_cast<const __bf16*>(grad_out);
  const auto* Ob = static_cast<const __bf16*>(out);
  const auto* Gf = static_cast<const float*>(grad_out);
  const auto* Of = static_cast<const float*>(out);
  E2V2_REQUIRE(!A.ext_gate || A.ext_dgate, "attn_bwd: the external gate needs ext_dgate for its gradient");
  return with_mode(kernel_mode(A), [&](auto md) -> int {
    constexpr int kM = decltype(md)::value;
    if (A.act_bf16) return attn_bwd_launch<__bf16, kM>(A, Gb, Ob, mrow, srow, cnt, ddvec, ddist, dq, dk, dv, ws, s);
    return attn_bwd_launch<float, kM>(A, Gf, Of, mrow, srow, cnt, ddvec, ddist, dq, dk, dv, ws, s);
  });
}
