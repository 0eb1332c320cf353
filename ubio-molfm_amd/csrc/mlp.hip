// Edge radial MLP (RadialProfile [K0 + types -> 128 -> LN -> SiLU -> 128 -> LN
// -> SiLU -> OUT], src/molfm/models/e2former/module_utils.py:2151-2178) fused
// with the Gaussian RBF of the edge distance (module_utils.py:1853-1869).
//
// Linear1 splits as W1 [rbf | tgt | src] x = W1r rbf(d) + (W1t tgt[z_i] + b1) +
// W1s src[z_j].  The type terms are per-type tables.  W1r rbf(d) depends on the
// scalar distance alone: it is tabulated per profile with its first three
// derivatives (float64, node spacing h a power of two, about 0.17 of the
// Gaussian width) and evaluated by quintic Hermite interpolation -- the
// interpolation error, ~f^(6) h^6 / 46080, is ~1e-8 of the values, below the
// fp32 rounding of the 256-term product it replaces.  The backward's
// dL/dd = sum_c dz1[c] d/dd (W1r rbf(d))[c] is a 128-term dot with the
// interpolated derivative.  Linear2 and Linear3 run as MFMA GEMMs on 32-edge
// tiles (fp32 16x16x4, or bf16 16x16x32 operands with fp32 accumulation).  The
// forward saves the normalised LayerNorm inputs (n1, n2) and their rstd; the
// backward uses them (no recompute) and returns only dL/d(distance).
//
// Latency structure: each tile is a chain of GEMMs separated by LayerNorms, so
// every global access on that chain is issued a stage ahead of its use.
// LayerNorm affine parameters live in LDS for the whole block; the bf16 kernels
// load a GEMM's entire per-wave B panel into registers while the previous stage
// computes; the backward prefetches the saved LayerNorm inputs before the GEMM
// whose output they normalise.
#include <algorithm>
#include <cmath>

#include <type_traits>
#include "common.h"
#include "../../include/e2v2.h"

namespace e2v2 {

constexpr int kT = 32;          // edges per tile
constexpr int kH = 128;         // hidden width
constexpr int kLdX = 258;       // fp32 LDS row stride for K=256 tiles (== 2 mod 32: conflict-free A reads)
constexpr int kLdY = 130;       // fp32 LDS row stride for K=128 tiles (== 2 mod 32)
constexpr int kLdXb = 264;      // bf16 row stride of K=256 tiles (16-byte aligned rows)
constexpr int kLdYb = 136;      // bf16 row stride of K=128 tiles
constexpr int kPFNarrow = 8;    // fp32 GEMM: k-steps (of 4) per register-prefetched B chunk, N <= 128
constexpr int kPFWide = 4;      //   and for N = 256 (same register footprint)
constexpr int kTabRow = 4 * kH; // floats per table node: value and h, h^2, h^3 scaled derivatives
constexpr float kFarDist = 1e18f;  // distance of padding rows (finite)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// ---------------------------------------------------------------------------
// fp32 GEMM: C[32][N] = A[32][K] x B[K][N].  Wave w owns columns
// [w*N/4, (w+1)*N/4).  acc[rt][ct] holds the 16x16 tile (rows rt*16.., cols
// w*N/4 + ct*16..); lane l holds rows 4*(l/16)+r, col l%16.  Within each block
// of 16 k the four k-steps s take k = 16 blk + 4 (l/16) + s, so a lane's B values
// for a block are four consecutive k of one column: B is stored lane-packed,
// one float4 per (wave, ct, blk, lane), B[16 blk + 4 (l/16) + s][w N/4 + 16 ct + l%16]
// at ((w (N/64) + ct) (K/16) + blk) 64 + l (16-byte loads, a wave's 1 KB contiguous).
// afn(k, a0, a1) supplies A[l%16][k] and A[16 + l%16][k].  B is streamed in chunks
// held in registers one chunk ahead (the fp32 MFMA time per chunk covers the load).
// The first B chunk of a GEMM, loaded ahead (before the stage that precedes the
// GEMM) so that its L2 round trip overlaps that stage.
template <int N>
struct BChunk {
  floatx4 v[(N > 128 ? kPFWide : kPFNarrow) / 4][N / 64];
};

template <int K, int N>
__device__ __forceinline__ const floatx4* b_lane_ptr(const float* __restrict__ B) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  return reinterpret_cast<const floatx4*>(B) + (size_t)wave * (N / 64) * (K / 16) * 64 + lane;
}

template <int K, int N>
__device__ __forceinline__ void load_first_chunk(const float* __restrict__ B, BChunk<N>& c) {
  constexpr int kBl = (N > 128 ? kPFWide : kPFNarrow) / 4;
  const floatx4* Bp = b_lane_ptr<K, N>(B);
#pragma unroll
  for (int b = 0; b < kBl; ++b)
#pragma unroll
    for (int ct = 0; ct < N / 64; ++ct) c.v[b][ct] = Bp[(ct * (K / 16) + b) * 64];
}

template <int K, int N, bool kPin, typename AFn>
__device__ __forceinline__ void gemm32f(AFn afn, const float* __restrict__ B, const BChunk<N>& first,
                                        floatx4 (&acc)[2][N / 64]) {
  constexpr int CT = N / 64;
  constexpr int kPF = N > 128 ? kPFWide : kPFNarrow;   // k-steps per chunk (kPF / 4 blocks of 16 k)
  constexpr int kBl = kPF / 4;
  constexpr int NCH = K / (4 * kPF);
  const int lane = threadIdx.x & 63;
  const int lk = lane >> 4;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) acc[rt][ct] = floatx4{0.f, 0.f, 0.f, 0.f};
  const floatx4* Bp = b_lane_ptr<K, N>(B);
  floatx4 bc[kBl][CT], bn[kBl][CT];
#pragma unroll
  for (int b = 0; b < kBl; ++b)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) bc[b][ct] = first.v[b][ct];
  __builtin_amdgcn_s_setprio(1);   // MFMA-ready waves issue ahead of epilogue work of other waves
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    if (ch + 1 < NCH) {
#pragma unroll
      for (int b = 0; b < kBl; ++b)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) bn[b][ct] = Bp[(ct * (K / 16) + (ch + 1) * kBl + b) * 64];
    }
    // kPin: keep the next chunk's loads here, a chunk of MFMAs ahead of their use
    // (the scheduler would otherwise sink them next to the first use and wait on
    // them); costs registers, so kernels under a 128-VGPR cap leave it off
    if constexpr (kPin) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < kPF; ++s) {
      float a0, a1;
      afn(16 * (ch * kBl + s / 4) + 4 * lk + (s & 3), a0, a1);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        acc[0][ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, bc[s / 4][ct][s & 3], acc[0][ct], 0, 0, 0);
        acc[1][ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, bc[s / 4][ct][s & 3], acc[1][ct], 0, 0, 0);
      }
    }
    if (ch + 1 < NCH) {
#pragma unroll
      for (int b = 0; b < kBl; ++b)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) bc[b][ct] = bn[b][ct];
    }
  }
  __builtin_amdgcn_s_setprio(0);
}

// A from an LDS tile with row stride lda; the first B chunk already loaded
template <int K, int N, bool kPin = false>
__device__ __forceinline__ void gemm32(const float* A, int lda, const float* __restrict__ B,
                                       const BChunk<N>& first, floatx4 (&acc)[2][N / 64]) {
  const int li = threadIdx.x & 15;
  const float* A0 = A + li * lda;
  const float* A1 = A + (16 + li) * lda;
  gemm32f<K, N, kPin>([&](int k, float& a0, float& a1) { a0 = A0[k]; a1 = A1[k]; }, B, first, acc);
}

// ---------------------------------------------------------------------------
// bf16 GEMM on a register-resident B panel.  Bt is B^T row-major [N][K]; the
// panel holds this wave's N/4 columns for all K (lane l: column l%16 of each
// 16-column group, k values 8*(l/16)..+7 of each 32-k step), i.e. K/8 * N/64
// VGPRs: 64 for K=256,N=128 or K=128,N=256.
template <int K, int N>
struct Panel {
  bf16x8 v[K / 32][N / 64];
};

template <int K, int N>
__device__ __forceinline__ void load_panel(Panel<K, N>& P, const __bf16* __restrict__ Bt) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const __bf16* p = Bt + (size_t)(wave * (N / 4) + (lane & 15)) * K + 8 * (lane >> 4);
#pragma unroll
  for (int ks = 0; ks < K / 32; ++ks)
#pragma unroll
    for (int ct = 0; ct < N / 64; ++ct)
      P.v[ks][ct] = *reinterpret_cast<const bf16x8*>(p + (size_t)ct * 16 * K + ks * 32);
}

template <int K, int N>
__device__ __forceinline__ void gemm_panel(const __bf16* A, int lda, const Panel<K, N>& P,
                                           floatx4 (&acc)[2][N / 64]) {
  const int lane = threadIdx.x & 63;
  const int li = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int ct = 0; ct < N / 64; ++ct) acc[rt][ct] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < K / 32; ++ks) {
    const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(A + li * lda + ks * 32 + 8 * lg);
    const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(A + (16 + li) * lda + ks * 32 + 8 * lg);
#pragma unroll
    for (int ct = 0; ct < N / 64; ++ct) {
      acc[0][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, P.v[ks][ct], acc[0][ct], 0, 0, 0);
      acc[1][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, P.v[ks][ct], acc[1][ct], 0, 0, 0);
    }
  }
}

// ---------------------------------------------------------------------------
// Accumulator tile <-> LDS / global.  Lane l of wave w holds rows
// rt*16 + 4*(l/16) + r and columns w*N/4 + ct*16 + l%16.
__device__ __forceinline__ int acc_row(int rt, int r) { return rt * 16 + 4 * ((threadIdx.x & 63) >> 4) + r; }
template <int N>
__device__ __forceinline__ int acc_col0() { return (threadIdx.x >> 6) * (N / 4) + (threadIdx.x & 15); }

template <int N>
__device__ __forceinline__ void store_acc(const floatx4 (&acc)[2][N / 64], float* Y, int ldy,
                                          const float (&bias)[N / 64]) {
  const int c0 = acc_col0<N>();
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float* y = Y + acc_row(rt, r) * ldy + c0;
#pragma unroll
      for (int ct = 0; ct < N / 64; ++ct) y[ct * 16] = acc[rt][ct][r] + bias[ct];
    }
}

template <int N>
__device__ __forceinline__ void load_bias(const float* __restrict__ b, float (&bias)[N / 64]) {
  const int c0 = acc_col0<N>();
#pragma unroll
  for (int ct = 0; ct < N / 64; ++ct) bias[ct] = b ? b[c0 + ct * 16] : 0.f;
}

// LayerNorm affine parameters of one profile, staged in LDS for the block
struct LnParams {
  float g1[kH], b1[kH], g2[kH], b2[kH];
};

__device__ __forceinline__ void load_ln_params(const e2v2_mlp_weights& W, LnParams& p) {
  const int t = threadIdx.x;      // threads 256 and up (larger blocks) load nothing
  if (t < kH) {
    p.g1[t] = W.g1[t];
    p.b1[t] = W.be1[t];
  } else if (t < 2 * kH) {
    p.g2[t - kH] = W.g2[t - kH];
    p.b2[t - kH] = W.be2[t - kH];
  }
}

// Row-wise LayerNorm(128) + SiLU of the fp32 rows of Y (8 threads per row),
// written to the next GEMM's A operand (fp32 in place, or bf16).  Rows below
// nsave also store the normalised (pre-affine) values and rstd.  Thread sub of
// a row owns columns ln_col(sub, q) = 4 sub + 32 (q / 4) + q % 4: for each q / 4
// the row's 8 threads cover 128 contiguous bytes, so the saved rows are written
// (and read back by the backward) as whole cache lines with 16-byte accesses.
__device__ __forceinline__ int ln_col(int sub, int q) { return 4 * sub + 32 * (q >> 2) + (q & 3); }

template <typename OutT>
__device__ __forceinline__ void ln_silu_rows(const float* Y, int ldy, OutT* Z, int ldz, const float* g,
                                             const float* b, float* __restrict__ nrm, int ldn,
                                             float* __restrict__ rstd_out, int rstd_stride, int nsave) {
  const int row = threadIdx.x >> 3, sub = threadIdx.x & 7;
  const float* y = Y + row * ldy;
  float v[16];
  float s = 0.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    v[q] = y[ln_col(sub, q)];
    s += v[q];
  }
  s += __shfl_xor(s, 1, 64);
  s += __shfl_xor(s, 2, 64);
  s += __shfl_xor(s, 4, 64);
  const float mean = s * (1.0f / kH);
  float s2 = 0.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const float dlt = v[q] - mean;
    s2 += dlt * dlt;
  }
  s2 += __shfl_xor(s2, 1, 64);
  s2 += __shfl_xor(s2, 2, 64);
  s2 += __shfl_xor(s2, 4, 64);
  const float rstd = frsq(s2 * (1.0f / kH) + 1e-5f);
  const bool save = nrm != nullptr && row < nsave;
  OutT* z = Z + row * ldz;
  float nv[16];
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int c = ln_col(sub, q);
    nv[q] = (v[q] - mean) * rstd;
    z[c] = (OutT)silu(nv[q] * g[c] + b[c]);
  }
  if (save) {
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4)
      *reinterpret_cast<floatx4*>(nrm + (size_t)row * ldn + ln_col(sub, 4 * q4)) =
          floatx4{nv[4 * q4], nv[4 * q4 + 1], nv[4 * q4 + 2], nv[4 * q4 + 3]};
    if (sub == 0) rstd_out[(size_t)row * rstd_stride] = rstd;
  }
}

// Saved LayerNorm input of this thread's row (8 threads per row, 16 columns each)
struct SavedRow {
  float n[16];
  float rstd;
};

__device__ __forceinline__ void load_saved_row(const float* __restrict__ nrm, int ldn,
                                               const float* __restrict__ rstd, int rstd_stride, int nvalid,
                                               SavedRow& sr) {
  const int row = threadIdx.x >> 3, sub = threadIdx.x & 7;
  const bool ok = row < nvalid;
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    const floatx4 v = ok ? *reinterpret_cast<const floatx4*>(nrm + (size_t)row * ldn + ln_col(sub, 4 * q4))
                         : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) sr.n[4 * q4 + i] = v[i];
  }
  sr.rstd = ok ? rstd[(size_t)row * rstd_stride] : 0.f;
}

// dz = LN-backward(SiLU-backward(dy)) of the fp32 rows of Y, written to Z
template <typename OutT>
__device__ __forceinline__ void ln_silu_bwd_rows(const float* Y, int ldy, OutT* Z, int ldz, const SavedRow& sr,
                                                 const float* g, const float* b) {
  const int row = threadIdx.x >> 3, sub = threadIdx.x & 7;
  const float* y = Y + row * ldy;
  float dn[16];
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int c = ln_col(sub, q);
    const float a = sr.n[q] * g[c] + b[c];
    const float sg = sigmoidf_(a);
    const float da = y[c] * sg * (1.0f + a * (1.0f - sg));
    dn[q] = da * g[c];
    s1 += dn[q];
    s2 += dn[q] * sr.n[q];
  }
  s1 += __shfl_xor(s1, 1, 64); s1 += __shfl_xor(s1, 2, 64); s1 += __shfl_xor(s1, 4, 64);
  s2 += __shfl_xor(s2, 1, 64); s2 += __shfl_xor(s2, 2, 64); s2 += __shfl_xor(s2, 4, 64);
  const float m1 = s1 * (1.0f / kH), m2 = s2 * (1.0f / kH);
  OutT* z = Z + row * ldz;
#pragma unroll
  for (int q = 0; q < 16; ++q) z[ln_col(sub, q)] = (OutT)(sr.rstd * (dn[q] - m1 - sr.n[q] * m2));
}

// ---------------------------------------------------------------------------
struct TileEdges {
  float d[kT];          // padding rows hold kFarDist
  int zi[kT], zj[kT];
};

__device__ __forceinline__ void load_tile_edges(const e2v2_mlp_args& A, int64_t e0, TileEdges& te) {
  const int t = threadIdx.x;
  if (t < kT) {
    const int64_t e = e0 + t;
    const bool v = e < A.n_edges;
    te.d[t] = v ? A.dist[e] : kFarDist;
    te.zi[t] = v ? A.node_type[A.edge_row[e]] : 0;
    te.zj[t] = v ? A.node_type[A.col[e]] : 0;
  }
}

// dOut of the backward as the edge-degree embedding's gradient, formed per tile
// instead of read from a stored [E][3][256] tensor:
//   dOut[e, l, c] = p(d_e) / avg * sum_{m in l} Y_m(u_e) G0[m][i_e][c]
// (the transpose of the CSR outer-product reduce of e2former.py:719-741, Y the
// raw spherical harmonics of the unit edge vector, p the envelope).
struct DegTile {
  float y[kT][9];
  float pa[kT];         // p(d) / avg; 0 on padding rows
  int row[kT];
};

__device__ __forceinline__ void load_deg_tile(const e2v2_mlp_args& A, const e2v2_deg_args& D, int64_t e0,
                                              DegTile& dt) {
  const int t = threadIdx.x;
  if (t < kT) {
    const int64_t e = e0 + t;
    if (e < A.n_edges) {
      const float d = D.dist[e];
      const float nrm = fmaxf(d, 1e-12f);
      float Y[9];
      raw_sh2(D.dvec[3 * e] / nrm, D.dvec[3 * e + 1] / nrm, D.dvec[3 * e + 2] / nrm, Y);
#pragma unroll
      for (int m = 0; m < 9; ++m) dt.y[t][m] = Y[m];
      Envelope env;
      env.rc = D.rc; env.a = D.env_a; env.b = D.env_b; env.c = D.env_c;
      float p, dp;
      env.eval(d, p, dp);
      dt.pa[t] = p / D.avg;
      dt.row[t] = A.edge_row[e];
    } else {
#pragma unroll
      for (int m = 0; m < 9; ++m) dt.y[t][m] = 0.f;
      dt.pa[t] = 0.f;
      dt.row[t] = 0;
    }
  }
}

// Four consecutive channels (4 c4 .. 4 c4 + 3) of dOut row `row`, profile m: a
// dense load, or (kDeg) the degree-embedding gradient of profile l = m.
template <bool kDeg>
__device__ __forceinline__ floatx4 dout4(const float* __restrict__ dout, int ld_dout, int64_t e0, int row,
                                         int nvalid, int m, int c4, const float* __restrict__ g0, int n_rows,
                                         const DegTile& dt) {
  floatx4 v = {0.f, 0.f, 0.f, 0.f};
  if (row >= nvalid) return v;
  if constexpr (kDeg) {
    const floatx4* gp = reinterpret_cast<const floatx4*>(g0 + (size_t)dt.row[row] * 256) + c4;
    const size_t gs = (size_t)n_rows * 64;   // one m-row of g0, in floatx4
    // the 2l + 1 rows of profile l = m, loaded together
    auto acc = [&](int q0, auto nq) {
      floatx4 g[decltype(nq)::value];
#pragma unroll
      for (int q = 0; q < decltype(nq)::value; ++q) g[q] = gp[(q0 + q) * gs];
#pragma unroll
      for (int q = 0; q < decltype(nq)::value; ++q) {
        const float y = dt.y[row][q0 + q];
        v[0] = fmaf(y, g[q][0], v[0]); v[1] = fmaf(y, g[q][1], v[1]);
        v[2] = fmaf(y, g[q][2], v[2]); v[3] = fmaf(y, g[q][3], v[3]);
      }
    };
    if (m == 0) acc(0, std::integral_constant<int, 1>{});
    else if (m == 1) acc(1, std::integral_constant<int, 3>{});
    else acc(4, std::integral_constant<int, 5>{});
    const float pa = dt.pa[row];
    v[0] *= pa; v[1] *= pa; v[2] *= pa; v[3] *= pa;
    return v;
  } else {
    return reinterpret_cast<const floatx4*>(dout + (e0 + row) * ld_dout + m * 256)[c4];
  }
}

// ---------------------------------------------------------------------------
// Linear1's rbf block from its table.  Quintic Hermite basis on t in [0, 1]:
// node values and h-, h^2-scaled derivatives at both ends.
struct Hermite5 {
  float a0, a1, a2, b0, b1, b2;
};

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

// Interval of distance d: d / h is exact (h is a power of two), so are its floor
// and fraction; padding rows clamp to the last interval.
__device__ __forceinline__ const float* table_interval(const e2v2_mlp_weights& W, float d, float& t) {
  const float u = fminf(d * (1.0f / W.rtab_h), (float)(W.rtab_n - 2));
  const float fn = floorf(u);
  t = u - fn;
  return W.rtab + (size_t)(int)fn * kTabRow;
}

// Y[row][c] = W1r rbf(d_row) + ttgt[z_i][c] + tsrc[z_j][c] (the pre-LayerNorm
// activation of Linear1); thread t owns row t/8 and 16 consecutive columns.
__device__ __forceinline__ void linear1_rows(const e2v2_mlp_weights& W, const TileEdges& te, float* Y, int ldy) {
  const int row = threadIdx.x >> 3, c0 = (threadIdx.x & 7) * 16;
  float t;
  const float* p = table_interval(W, te.d[row], t) + c0;
  const Hermite5 H = hermite5(t);
  const float* tt = W.ttgt + te.zi[row] * kH + c0;
  const float* ts = W.tsrc + te.zj[row] * kH + c0;
  float* y = Y + row * ldy + c0;
#pragma unroll 2
  for (int q = 0; q < 4; ++q) {
    const floatx4 f0 = reinterpret_cast<const floatx4*>(p + 4 * q)[0];
    const floatx4 f1 = reinterpret_cast<const floatx4*>(p + kH + 4 * q)[0];
    const floatx4 f2 = reinterpret_cast<const floatx4*>(p + 2 * kH + 4 * q)[0];
    const floatx4 g0 = reinterpret_cast<const floatx4*>(p + kTabRow + 4 * q)[0];
    const floatx4 g1 = reinterpret_cast<const floatx4*>(p + kTabRow + kH + 4 * q)[0];
    const floatx4 g2 = reinterpret_cast<const floatx4*>(p + kTabRow + 2 * kH + 4 * q)[0];
    const floatx4 a = reinterpret_cast<const floatx4*>(tt + 4 * q)[0];
    const floatx4 b = reinterpret_cast<const floatx4*>(ts + 4 * q)[0];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float f = H.a0 * f0[i] + H.a1 * f1[i] + H.a2 * f2[i] + H.b0 * g0[i] + H.b1 * g1[i] + H.b2 * g2[i];
      y[4 * q + i] = f + a[i] + b[i];
    }
  }
}

// sum_c Z[row][c] d/dd (W1r rbf(d_row))[c], complete in each of the row's 8 threads
__device__ __forceinline__ float linear1_dd(const e2v2_mlp_weights& W, const TileEdges& te, const float* Z, int ldz) {
  const int row = threadIdx.x >> 3, c0 = (threadIdx.x & 7) * 16;
  float t;
  const float* p = table_interval(W, te.d[row], t) + c0;
  const Hermite5 H = hermite5(t);
  const float* z = Z + row * ldz + c0;
  float s = 0.f;
#pragma unroll 2
  for (int q = 0; q < 4; ++q) {
    const floatx4 f1 = reinterpret_cast<const floatx4*>(p + kH + 4 * q)[0];
    const floatx4 f2 = reinterpret_cast<const floatx4*>(p + 2 * kH + 4 * q)[0];
    const floatx4 f3 = reinterpret_cast<const floatx4*>(p + 3 * kH + 4 * q)[0];
    const floatx4 g1 = reinterpret_cast<const floatx4*>(p + kTabRow + kH + 4 * q)[0];
    const floatx4 g2 = reinterpret_cast<const floatx4*>(p + kTabRow + 2 * kH + 4 * q)[0];
    const floatx4 g3 = reinterpret_cast<const floatx4*>(p + kTabRow + 3 * kH + 4 * q)[0];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float hd = H.a0 * f1[i] + H.a1 * f2[i] + H.a2 * f3[i] + H.b0 * g1[i] + H.b1 * g2[i] + H.b2 * g3[i];
      s = fmaf(z[4 * q + i], hd, s);
    }
  }
  s += __shfl_xor(s, 1, 64);
  s += __shfl_xor(s, 2, 64);
  s += __shfl_xor(s, 4, 64);
  return s * (1.0f / W.rtab_h);
}

// Table builder: one block per node n, thread c; float64 sums over the 256 centres of
// h^k d^k/dd^k exp(c (d - mu)^2) W1r[c][mu] at d = n h.
__global__ __launch_bounds__(kH) void k_rbf_table(const float* __restrict__ w1, int ldw1,
                                                  const float* __restrict__ mu, float coeff, float h,
                                                  float* __restrict__ rtab) {
  const int n = blockIdx.x, c = threadIdx.x;
  const double d = (double)n * (double)h, cf = (double)coeff, hh = (double)h;
  double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
  for (int j = 0; j < 256; ++j) {
    const double x = d - (double)mu[j];
    const double r = exp(cf * x * x);
    const double w = (double)w1[(size_t)c * ldw1 + j];
    s0 += w * r;
    s1 += w * (2.0 * cf * x) * r;
    s2 += w * (2.0 * cf + 4.0 * cf * cf * x * x) * r;
    s3 += w * (12.0 * cf * cf * x + 8.0 * cf * cf * cf * x * x * x) * r;
  }
  float* o = rtab + (size_t)n * kTabRow + c;
  o[0] = (float)s0;
  o[kH] = (float)(hh * s1);
  o[2 * kH] = (float)(hh * hh * s2);
  o[3 * kH] = (float)(hh * hh * hh * s3);
}

// GEMM-3 epilogue: out[e0 + row][m * 256 + c] = acc + b3[c] for the valid rows.
// The tile goes through LDS (O, row stride kLdO; the caller has synchronised so
// the buffer is free) and leaves as whole rows, one 16-byte store per lane and
// 1 KB per wave instruction (the accumulator layout would write 64-byte pieces).
constexpr int kLdO = 260;
__device__ __forceinline__ void store_out(const floatx4 (&acc)[2][4], const float (&b3)[4], float* O,
                                          float* __restrict__ out, int ld_out, int64_t e0, int nvalid, int m) {
  const int c0 = acc_col0<256>();
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float* o = O + acc_row(rt, r) * kLdO + c0;
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) o[ct * 16] = acc[rt][ct][r] + b3[ct];
    }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int rr = 0; rr < kT / 4; ++rr) {
    const int row = wave + 4 * rr;
    if (row < nvalid) {
      const float* src = O + row * kLdO + 4 * lane;
      *reinterpret_cast<floatx4*>(out + (e0 + row) * (int64_t)ld_out + m * 256 + 4 * lane) =
          floatx4{src[0], src[1], src[2], src[3]};
    }
  }
}

// ---------------------------------------------------------------------------
// fp32 kernels
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 8))) void k_mlp_fwd(
    e2v2_mlp_args A, float* __restrict__ out, int ld_out) {
  extern __shared__ float sm[];
  float* Y = sm;                    // [32][130]: Linear1/2 outputs, LayerNorm in place
  __shared__ TileEdges te;
  __shared__ LnParams lp;
  const int m = blockIdx.y;
  const e2v2_mlp_weights& W = A.w[m];
  const int64_t e0 = (int64_t)blockIdx.x * kT;
  const int nvalid = (int)min<int64_t>(kT, A.n_edges - e0);
  float* sn = A.save_n ? A.save_n + ((size_t)m * A.n_edges + e0) * (2 * kH) : nullptr;
  float* sr = A.save_r ? A.save_r + ((size_t)m * A.n_edges + e0) * 2 : nullptr;
  float b2[2], b3[4];
  load_bias<kH>(W.b2, b2);
  load_bias<256>(W.b3, b3);
  load_tile_edges(A, e0, te);
  load_ln_params(W, lp);
  BChunk<kH> f2;
  load_first_chunk<kH, kH>(W.w2t, f2);      // in flight during Linear1 and LayerNorm 1
  __syncthreads();
  linear1_rows(W, te, Y, kLdY);
  __syncthreads();
  ln_silu_rows(Y, kLdY, Y, kLdY, lp.g1, lp.b1, sn, 2 * kH, sr, 2, nvalid);
  __syncthreads();
  BChunk<256> f3;
  {
    floatx4 acc[2][2];
    gemm32<kH, kH, true>(Y, kLdY, W.w2t, f2, acc);
    load_first_chunk<kH, 256>(W.w3t, f3);  // in flight during LayerNorm 2
    __syncthreads();
    store_acc<kH>(acc, Y, kLdY, b2);
  }
  __syncthreads();
  ln_silu_rows(Y, kLdY, Y, kLdY, lp.g2, lp.b2, sn ? sn + kH : nullptr, 2 * kH, sr ? sr + 1 : nullptr, 2, nvalid);
  __syncthreads();
  floatx4 acc[2][4];
  gemm32<kH, 256, true>(Y, kLdY, W.w3t, f3, acc);
  __syncthreads();
  store_out(acc, b3, sm, out, ld_out, e0, nvalid, m);
}

template <bool kDeg>
__device__ __forceinline__ void mlp_bwd_body(e2v2_mlp_args A, const float* __restrict__ dout, int ld_dout,
                                             float* __restrict__ dd, int accumulate, e2v2_deg_args D,
                                             const float* __restrict__ g0) {
  extern __shared__ float sm[];
  float* X = sm;                    // [32][258]: dOut tile; after GEMM a, the [32][130] LayerNorm rows
  float* Y = sm;
  __shared__ TileEdges te;
  __shared__ LnParams lp;
  __shared__ DegTile dt;
  // degree mode: each XCD takes a contiguous range of tiles, so the node-gradient
  // rows that neighbouring tiles share stay in one L2
  const int64_t n_tiles = (A.n_edges + kT - 1) / kT;
  const int64_t tile = kDeg ? (int64_t)xcd_row(blockIdx.x, (int)n_tiles) : (int64_t)blockIdx.x;
  if (tile >= n_tiles) return;
  const int64_t e0 = tile * kT;
  const int nvalid = (int)min<int64_t>(kT, A.n_edges - e0);
  const float zero2[2] = {0.f, 0.f};
  load_tile_edges(A, e0, te);
  if constexpr (kDeg) load_deg_tile(A, D, e0, dt);
  __syncthreads();
  float dd_row = 0.f;
  for (int m = 0; m < A.n_mlp; ++m) {
    const e2v2_mlp_weights& W = A.w[m];
    const float* sn = A.save_n + ((size_t)m * A.n_edges + e0) * (2 * kH);
    const float* srs = A.save_r + ((size_t)m * A.n_edges + e0) * 2;
    load_ln_params(W, lp);
    BChunk<kH> fa;
    load_first_chunk<256, kH>(W.w3, fa);       // in flight during the dOut tile load
    for (int idx = threadIdx.x; idx < kT * 64; idx += 256) {   // dOut tile, 16-byte loads
      const int row = idx >> 6, c4 = idx & 63;
      const floatx4 v = dout4<kDeg>(dout, ld_dout, e0, row, nvalid, m, c4, g0, D.n_rows, dt);
      float* xr = X + row * kLdX + 4 * c4;
      xr[0] = v[0]; xr[1] = v[1]; xr[2] = v[2]; xr[3] = v[3];
    }
    SavedRow s2;
    load_saved_row(sn + kH, 2 * kH, srs + 1, 2, nvalid, s2);
    __syncthreads();
    BChunk<kH> fb;
    {  // dy2 = dOut . W3   (W3 [256][128] row-major = B[K=256][N=128])
      floatx4 acc[2][2];
      gemm32<256, kH>(X, kLdX, W.w3, fa, acc);
      load_first_chunk<kH, kH>(W.w2, fb);     // in flight during the LayerNorm-2 backward
      __syncthreads();
      store_acc<kH>(acc, Y, kLdY, zero2);
    }
    SavedRow s1;
    load_saved_row(sn, 2 * kH, srs, 2, nvalid, s1);
    __syncthreads();
    ln_silu_bwd_rows(Y, kLdY, Y, kLdY, s2, lp.g2, lp.b2);
    __syncthreads();
    {  // dy1 = dz2 . W2   (W2 [128][128])
      floatx4 acc[2][2];
      gemm32<kH, kH>(Y, kLdY, W.w2, fb, acc);
      __syncthreads();
      store_acc<kH>(acc, Y, kLdY, zero2);
    }
    __syncthreads();
    ln_silu_bwd_rows(Y, kLdY, Y, kLdY, s1, lp.g1, lp.b1);
    __syncthreads();
    dd_row += linear1_dd(W, te, Y, kLdY);
    __syncthreads();
  }
  const int row = threadIdx.x >> 3;
  if ((threadIdx.x & 7) == 0 && row < nvalid) {
    const int64_t e = e0 + row;
    dd[e] = accumulate ? dd[e] + dd_row : dd_row;
  }
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void k_mlp_bwd(
    e2v2_mlp_args A, const float* __restrict__ dout, int ld_dout, float* __restrict__ dd, int accumulate) {
  mlp_bwd_body<false>(A, dout, ld_dout, dd, accumulate, e2v2_deg_args{}, nullptr);
}
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void k_mlp_bwd_deg(
    e2v2_mlp_args A, float* __restrict__ dd, int accumulate, e2v2_deg_args D, const float* __restrict__ g0) {
  mlp_bwd_body<true>(A, nullptr, 0, dd, accumulate, D, g0);
}

// ---------------------------------------------------------------------------
// bf16-operand kernels (fp32 accumulation; LayerNorm, SiLU, tables, saved
// statistics and all outputs stay fp32).  B panels come as B^T row-major
// [N][K] in bf16.
// four waves per SIMD (126 VGPRs, no spills; the compiler picks 160 with accumulation
// registers otherwise and three waves): 5% faster.  The backward kernels spill at four.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void k_mlp_fwd_bf16(e2v2_mlp_args A, float* __restrict__ out, int ld_out) {
  extern __shared__ float sm[];
  float* Yf = sm;                                              // [32][130] fp32
  __bf16* Yb = reinterpret_cast<__bf16*>(Yf + kT * kLdY);      // [32][136] bf16
  __bf16* Zb = Yb + kT * kLdYb;                                // [32][136] bf16
  __shared__ TileEdges te;
  __shared__ LnParams lp;
  const int m = blockIdx.y;
  const e2v2_mlp_weights& W = A.w[m];
  const int64_t e0 = (int64_t)blockIdx.x * kT;
  const int nvalid = (int)min<int64_t>(kT, A.n_edges - e0);
  float* sn = A.save_n ? A.save_n + ((size_t)m * A.n_edges + e0) * (2 * kH) : nullptr;
  float* sr = A.save_r ? A.save_r + ((size_t)m * A.n_edges + e0) * 2 : nullptr;
  Panel<kH, kH> P2;
  load_panel(P2, static_cast<const __bf16*>(W.w2b));
  float b2[2], b3[4];
  load_bias<kH>(W.b2, b2);
  load_bias<256>(W.b3, b3);
  load_tile_edges(A, e0, te);
  load_ln_params(W, lp);
  __syncthreads();
  linear1_rows(W, te, Yf, kLdY);
  __syncthreads();
  ln_silu_rows(Yf, kLdY, Yb, kLdYb, lp.g1, lp.b1, sn, 2 * kH, sr, 2, nvalid);
  __syncthreads();
  Panel<kH, 256> P3;
  {
    floatx4 acc[2][2];
    gemm_panel(Yb, kLdYb, P2, acc);
    load_panel(P3, static_cast<const __bf16*>(W.w3b));
    store_acc<kH>(acc, Yf, kLdY, b2);
  }
  __syncthreads();
  ln_silu_rows(Yf, kLdY, Zb, kLdYb, lp.g2, lp.b2, sn ? sn + kH : nullptr, 2 * kH, sr ? sr + 1 : nullptr, 2,
               nvalid);
  __syncthreads();
  floatx4 acc[2][4];
  gemm_panel(Zb, kLdYb, P3, acc);
  __syncthreads();
  store_out(acc, b3, sm, out, ld_out, e0, nvalid, m);
}

template <bool kDeg>
__device__ __forceinline__ void mlp_bwd_bf16_body(e2v2_mlp_args A, const float* __restrict__ dout, int ld_dout,
                                                  float* __restrict__ dd, int accumulate, e2v2_deg_args D,
                                                  const float* __restrict__ g0) {
  extern __shared__ float sm[];
  __bf16* Xb = reinterpret_cast<__bf16*>(sm);                 // [32][264] bf16
  float* Yf = sm + (kT * kLdXb) / 2;                           // [32][130] fp32
  __bf16* Yb = reinterpret_cast<__bf16*>(Yf + kT * kLdY);      // [32][136] bf16
  __shared__ TileEdges te;
  __shared__ LnParams lp;
  __shared__ DegTile dt;
  // degree mode: each XCD takes a contiguous range of tiles, so the node-gradient
  // rows that neighbouring tiles share stay in one L2
  const int64_t n_tiles = (A.n_edges + kT - 1) / kT;
  const int64_t tile = kDeg ? (int64_t)xcd_row(blockIdx.x, (int)n_tiles) : (int64_t)blockIdx.x;
  if (tile >= n_tiles) return;
  const int64_t e0 = tile * kT;
  const int nvalid = (int)min<int64_t>(kT, A.n_edges - e0);
  const float zero2[2] = {0.f, 0.f};
  load_tile_edges(A, e0, te);
  if constexpr (kDeg) load_deg_tile(A, D, e0, dt);
  __syncthreads();
  float dd_row = 0.f;
  for (int m = 0; m < A.n_mlp; ++m) {
    const e2v2_mlp_weights& W = A.w[m];
    const float* sn = A.save_n + ((size_t)m * A.n_edges + e0) * (2 * kH);
    const float* srs = A.save_r + ((size_t)m * A.n_edges + e0) * 2;
    Panel<256, kH> Pa;
    load_panel(Pa, static_cast<const __bf16*>(W.w3tb));
    load_ln_params(W, lp);
    for (int idx = threadIdx.x; idx < kT * 64; idx += 256) {
      const int row = idx >> 6, c4 = idx & 63;
      const floatx4 v = dout4<kDeg>(dout, ld_dout, e0, row, nvalid, m, c4, g0, D.n_rows, dt);
      __bf16* xr = Xb + row * kLdXb + 4 * c4;
      xr[0] = (__bf16)v[0]; xr[1] = (__bf16)v[1]; xr[2] = (__bf16)v[2]; xr[3] = (__bf16)v[3];
    }
    SavedRow s2;
    load_saved_row(sn + kH, 2 * kH, srs + 1, 2, nvalid, s2);
    __syncthreads();
    Panel<kH, kH> Pb;
    {  // dy2 = dOut . W3   (B^T = W3^T [128][256])
      floatx4 acc[2][2];
      gemm_panel(Xb, kLdXb, Pa, acc);
      load_panel(Pb, static_cast<const __bf16*>(W.w2tb));
      store_acc<kH>(acc, Yf, kLdY, zero2);
    }
    SavedRow s1;
    load_saved_row(sn, 2 * kH, srs, 2, nvalid, s1);
    __syncthreads();
    ln_silu_bwd_rows(Yf, kLdY, Yb, kLdYb, s2, lp.g2, lp.b2);
    __syncthreads();
    {  // dy1 = dz2 . W2   (B^T = W2^T)
      floatx4 acc[2][2];
      gemm_panel(Yb, kLdYb, Pb, acc);
      store_acc<kH>(acc, Yf, kLdY, zero2);
    }
    __syncthreads();
    ln_silu_bwd_rows(Yf, kLdY, Yf, kLdY, s1, lp.g1, lp.b1);
    __syncthreads();
    dd_row += linear1_dd(W, te, Yf, kLdY);
    __syncthreads();
  }
  const int row = threadIdx.x >> 3;
  if ((threadIdx.x & 7) == 0 && row < nvalid) {
    const int64_t e = e0 + row;
    dd[e] = accumulate ? dd[e] + dd_row : dd_row;
  }
}

__global__ __launch_bounds__(256) void k_mlp_bwd_bf16(e2v2_mlp_args A, const float* __restrict__ dout, int ld_dout,
                                                      float* __restrict__ dd, int accumulate) {
  mlp_bwd_bf16_body<false>(A, dout, ld_dout, dd, accumulate, e2v2_deg_args{}, nullptr);
}
__global__ __launch_bounds__(256) void k_mlp_bwd_deg_bf16(e2v2_mlp_args A, float* __restrict__ dd, int accumulate,
                                                          e2v2_deg_args D, const float* __restrict__ g0) {
  mlp_bwd_bf16_body<true>(A, nullptr, 0, dd, accumulate, D, g0);
}

}  // namespace e2v2

using namespace e2v2;

static size_t mlp_lds_fwd() { return sizeof(float) * kT * kLdO; }
static size_t mlp_lds_bwd() { return sizeof(float) * kT * kLdX; }
static size_t mlp_lds_fwd_bf16() {
  return std::max(sizeof(float) * kT * kLdY + 2 * sizeof(__bf16) * kT * kLdYb, sizeof(float) * kT * kLdO);
}
static size_t mlp_lds_bwd_bf16() { return sizeof(__bf16) * (kT * kLdXb + kT * kLdYb) + sizeof(float) * kT * kLdY; }

static int check_tables(const e2v2_mlp_args& A, const char* who) {
  for (int m = 0; m < A.n_mlp; ++m)
    E2V2_REQUIRE(A.w[m].rtab != nullptr && A.w[m].rtab_n >= 2 && A.w[m].rtab_h > 0.f,
                 "%s: profile %d has no rbf-block table (e2v2_mlp_rbf_table)", who, m);
  return 0;
}

E2V2_API int e2v2_mlp_rbf_table_size(float rc, float rbf_coeff, int32_t* n_nodes, float* h) {
  E2V2_REQUIRE(rc > 0.f && rbf_coeff < 0.f && n_nodes && h, "mlp_rbf_table_size: need rc > 0, rbf_coeff < 0");
  const double sigma = std::sqrt(-0.5 / (double)rbf_coeff);
  const double hh = std::ldexp(1.0, (int)std::floor(std::log2(0.2 * sigma)));
  const double n = std::floor((double)rc / hh) + 2.0;
  E2V2_REQUIRE(n <= 1 << 20, "mlp_rbf_table_size: %.0f nodes (rc %g, width %g) is too many", n, (double)rc, sigma);
  *n_nodes = (int32_t)n;
  *h = (float)hh;
  return 0;
}

E2V2_API int e2v2_mlp_rbf_table(const float* w1, int ldw1, const float* rbf_offset, float rbf_coeff, int32_t n_nodes,
                                float h, float* rtab, hipStream_t s) {
  E2V2_REQUIRE(w1 && rbf_offset && rtab && ldw1 >= 256 && n_nodes >= 2 && h > 0.f,
               "mlp_rbf_table: bad arguments (ldw1 %d, n_nodes %d)", ldw1, n_nodes);
  hipLaunchKernelGGL(k_rbf_table, dim3((unsigned)n_nodes), dim3(kH), 0, s, w1, ldw1, rbf_offset, rbf_coeff, h, rtab);
  E2V2_LAUNCHED("k_rbf_table");
  return 0;
}

E2V2_API int e2v2_mlp_fwd(const e2v2_mlp_args* args, float* out, int ld_out, hipStream_t s) {
  const e2v2_mlp_args& A = *args;
  E2V2_REQUIRE(A.n_mlp >= 1 && A.n_mlp <= E2V2_MAX_MLP, "mlp_fwd: n_mlp %d out of range", A.n_mlp);
  E2V2_REQUIRE(ld_out >= 256 * A.n_mlp, "mlp_fwd: ld_out %d < 256*n_mlp", ld_out);
  if (A.n_edges == 0) return 0;
  if (int rc = check_tables(A, "mlp_fwd")) return rc;
  dim3 grid((unsigned)((A.n_edges + kT - 1) / kT), (unsigned)A.n_mlp);
  if (A.compute_bf16) {
    for (int m = 0; m < A.n_mlp; ++m)
      E2V2_REQUIRE(A.w[m].w2b && A.w[m].w3b, "mlp_fwd: bf16 weights missing for profile %d", m);
    hipLaunchKernelGGL(k_mlp_fwd_bf16, grid, dim3(256), mlp_lds_fwd_bf16(), s, A, out, ld_out);
    E2V2_LAUNCHED("k_mlp_fwd_bf16");
    return 0;
  }
  hipLaunchKernelGGL(k_mlp_fwd, grid, dim3(256), mlp_lds_fwd(), s, A, out, ld_out);
  E2V2_LAUNCHED("k_mlp_fwd");
  return 0;
}

static int mlp_bwd_launch(const e2v2_mlp_args& A, const float* dout, int ld_dout, float* dd, int accumulate,
                          const e2v2_deg_args* D, const float* g0, hipStream_t s) {
  E2V2_REQUIRE(A.n_mlp >= 1 && A.n_mlp <= E2V2_MAX_MLP, "mlp_bwd: n_mlp %d out of range", A.n_mlp);
  E2V2_REQUIRE(A.save_n != nullptr && A.save_r != nullptr,
               "mlp_bwd: needs the normalised activations saved by e2v2_mlp_fwd (save_n, save_r)");
  if (A.n_edges == 0) return 0;
  if (int rc = check_tables(A, "mlp_bwd")) return rc;
  dim3 grid((unsigned)((A.n_edges + kT - 1) / kT));
  if (A.compute_bf16) {
    for (int m = 0; m < A.n_mlp; ++m)
      E2V2_REQUIRE(A.w[m].w3tb && A.w[m].w2tb, "mlp_bwd: bf16 weights missing for profile %d", m);
    if (D) {
      hipLaunchKernelGGL(k_mlp_bwd_deg_bf16, dim3((unsigned)xcd_grid((int)((A.n_edges + kT - 1) / kT))), dim3(256),
                         mlp_lds_bwd_bf16(), s, A, dd, accumulate, *D, g0);
      E2V2_LAUNCHED("k_mlp_bwd_deg_bf16");
    } else {
      hipLaunchKernelGGL(k_mlp_bwd_bf16, grid, dim3(256), mlp_lds_bwd_bf16(), s, A, dout, ld_dout, dd, accumulate);
      E2V2_LAUNCHED("k_mlp_bwd_bf16");
    }
    return 0;
  }
  const dim3 grid_deg((unsigned)xcd_grid((int)((A.n_edges + kT - 1) / kT)));
  if (D) {
    hipLaunchKernelGGL(k_mlp_bwd_deg, grid_deg, dim3(256), mlp_lds_bwd(), s, A, dd, accumulate, *D, g0);
    E2V2_LAUNCHED("k_mlp_bwd_deg");
  } else {
    hipLaunchKernelGGL(k_mlp_bwd, grid, dim3(256), mlp_lds_bwd(), s, A, dout, ld_dout, dd, accumulate);
    E2V2_LAUNCHED("k_mlp_bwd");
  }
  return 0;
}

E2V2_API int e2v2_mlp_bwd(const e2v2_mlp_args* args, const float* dout, int ld_dout, float* dd, int accumulate,
                          hipStream_t s) {
  E2V2_REQUIRE(ld_dout >= 256 * args->n_mlp && ld_dout % 4 == 0, "mlp_bwd: bad ld_dout %d", ld_dout);
  return mlp_bwd_launch(*args, dout, ld_dout, dd, accumulate, nullptr, nullptr, s);
}

E2V2_API int e2v2_mlp_bwd_deg(const e2v2_mlp_args* args, const e2v2_deg_args* deg, const float* grad_x0, float* dd,
                              int accumulate, hipStream_t s) {
  E2V2_REQUIRE(args->n_mlp == 3 && deg && grad_x0 && deg->channels == 256 && deg->n_edges == args->n_edges,
               "mlp_bwd_deg: needs the three l-profiles of the degree embedding (n_mlp %d) and its edges",
               args->n_mlp);
  return mlp_bwd_launch(*args, nullptr, 0, dd, accumulate, deg, grad_x0, s);
}
