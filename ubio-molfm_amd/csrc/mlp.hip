// Edge radial MLP (RadialProfile [K0 + types -> 128 -> LN -> SiLU -> 128 -> LN
// -> SiLU -> OUT], src/molfm/models/e2former/module_utils.py:2151-2178) fused
// with the Gaussian RBF of the edge distance (module_utils.py:1853-1869).
//
// The first Linear is split: W1 [rbf | tgt | src] x = W1r rbf + (W1t tgt[z_i] + b1)
// + W1s src[z_j]; the two type terms arrive as per-type tables.  The RBF tile
// lives in LDS only; the MLP runs as fp32 MFMA 16x16x4 GEMMs on 32-edge tiles.
// The forward saves the normalised LayerNorm inputs (n1, n2) and their rstd;
// the backward uses them (no recompute) and returns only dL/d(distance).
#include "common.h"
#include "../../include/e2v2.h"

namespace e2v2 {

constexpr int kT = 32;          // edges per tile
constexpr int kK0 = 256;        // rbf basis
constexpr int kH = 128;         // hidden width
constexpr int kLdX = 258;       // LDS row stride for K=256 tiles (== 2 mod 32: conflict-free A reads)
constexpr int kLdY = 130;       // LDS row stride for K=128 tiles (== 2 mod 32)
constexpr int kPF = 8;          // k-steps (of 4) per register-prefetched B chunk

// C[32][N] = A[32][K] (LDS, row stride lda) x B[K][N] (global, row stride ldb).
// Wave w owns columns [w*N/4, (w+1)*N/4).  acc[rt][ct] holds the 16x16 tile
// (rows rt*16.., cols w*N/4 + ct*16..); lane l holds rows 4*(l/16)+r, col l%16.
// B is streamed in chunks of 32 k-rows held in registers one chunk ahead.
template <int K, int N>
__device__ __forceinline__ void gemm32(const float* A, int lda, const float* __restrict__ B, int ldb,
                                       floatx4 (&acc)[2][N / 64]) {
  constexpr int CT = N / 64;
  constexpr int NCH = K / (4 * kPF);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15, lk = lane >> 4;
  const int cbase = wave * (N / 4);
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) acc[rt][ct] = floatx4{0.f, 0.f, 0.f, 0.f};
  const float* Bp = B + (size_t)lk * ldb + cbase + li;
  float bc[kPF][CT], bn[kPF][CT];
#pragma unroll
  for (int s = 0; s < kPF; ++s)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) bc[s][ct] = Bp[(size_t)(4 * s) * ldb + ct * 16];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    if (ch + 1 < NCH) {
#pragma unroll
      for (int s = 0; s < kPF; ++s)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) bn[s][ct] = Bp[(size_t)((ch + 1) * 4 * kPF + 4 * s) * ldb + ct * 16];
    }
#pragma unroll
    for (int s = 0; s < kPF; ++s) {
      const int k0 = ch * 4 * kPF + 4 * s;
      const float a0 = A[li * lda + k0 + lk];
      const float a1 = A[(16 + li) * lda + k0 + lk];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        acc[0][ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, bc[s][ct], acc[0][ct], 0, 0, 0);
        acc[1][ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, bc[s][ct], acc[1][ct], 0, 0, 0);
      }
    }
    if (ch + 1 < NCH) {
#pragma unroll
      for (int s = 0; s < kPF; ++s)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) bc[s][ct] = bn[s][ct];
    }
  }
}

template <int N>
__device__ __forceinline__ void acc_coord(int rt, int ct, int r, int& row, int& c) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  row = rt * 16 + 4 * (lane >> 4) + r;
  c = wave * (N / 4) + ct * 16 + (lane & 15);
}

template <int N>
__device__ __forceinline__ void store_acc(const floatx4 (&acc)[2][N / 64], float* Y, int ldy,
                                          const float* __restrict__ bias) {
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int ct = 0; ct < N / 64; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        int row, c;
        acc_coord<N>(rt, ct, r, row, c);
        Y[row * ldy + c] = acc[rt][ct][r] + (bias ? bias[c] : 0.f);
      }
}

// Row-wise LayerNorm(128) + SiLU on Y (in place), 8 threads per row.  Rows
// below nsave also store the normalised (pre-affine) values and rstd.
__device__ __forceinline__ void ln_silu_rows(float* Y, int ldy, const float* __restrict__ g,
                                             const float* __restrict__ b, float* nrm, int ldn, float* rstd_out,
                                             int rstd_stride, int nsave) {
  const int row = threadIdx.x >> 3, sub = threadIdx.x & 7;
  float* y = Y + row * ldy;
  float v[16];
  float s = 0.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    v[q] = y[sub + 8 * q];
    s += v[q];
  }
  s += __shfl_xor(s, 1, 64);
  s += __shfl_xor(s, 2, 64);
  s += __shfl_xor(s, 4, 64);
  const float mean = s * (1.0f / kH);
  float s2 = 0.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    float dlt = v[q] - mean;
    s2 += dlt * dlt;
  }
  s2 += __shfl_xor(s2, 1, 64);
  s2 += __shfl_xor(s2, 2, 64);
  s2 += __shfl_xor(s2, 4, 64);
  const float rstd = 1.0f / sqrtf(s2 * (1.0f / kH) + 1e-5f);
  const bool save = nrm != nullptr && row < nsave;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int c = sub + 8 * q;
    float n = (v[q] - mean) * rstd;
    if (save) nrm[(size_t)row * ldn + c] = n;
    float a = n * g[c] + b[c];
    y[c] = silu(a);
  }
  if (save && sub == 0) rstd_out[(size_t)row * rstd_stride] = rstd;
}

// dz = LN-backward(SiLU-backward(dy)) given the saved normalised input and rstd (global).
__device__ __forceinline__ void ln_silu_bwd_rows(float* Y, int ldy, const float* __restrict__ nrm, int ldn,
                                                 const float* __restrict__ rstd, int rstd_stride, int nvalid,
                                                 const float* __restrict__ g, const float* __restrict__ b) {
  const int row = threadIdx.x >> 3, sub = threadIdx.x & 7;
  float* y = Y + row * ldy;
  const bool ok = row < nvalid;
  float dn[16], nn[16];
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int c = sub + 8 * q;
    float n = ok ? nrm[(size_t)row * ldn + c] : 0.f;
    float a = n * g[c] + b[c];
    float sg = sigmoidf_(a);
    float da = y[c] * sg * (1.0f + a * (1.0f - sg));
    dn[q] = da * g[c];
    nn[q] = n;
    s1 += dn[q];
    s2 += dn[q] * n;
  }
  s1 += __shfl_xor(s1, 1, 64); s1 += __shfl_xor(s1, 2, 64); s1 += __shfl_xor(s1, 4, 64);
  s2 += __shfl_xor(s2, 1, 64); s2 += __shfl_xor(s2, 2, 64); s2 += __shfl_xor(s2, 4, 64);
  const float m1 = s1 * (1.0f / kH), m2 = s2 * (1.0f / kH);
  const float r = ok ? rstd[(size_t)row * rstd_stride] : 0.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) y[sub + 8 * q] = r * (dn[q] - m1 - nn[q] * m2);
}

struct TileEdges {
  float d[kT];
  int zi[kT], zj[kT];
  int valid[kT];
};

__device__ __forceinline__ void load_tile_edges(const e2v2_mlp_args& A, int64_t e0, TileEdges& te) {
  const int t = threadIdx.x;
  if (t < kT) {
    const int64_t e = e0 + t;
    const bool v = e < A.n_edges;
    te.valid[t] = v;
    te.d[t] = v ? A.dist[e] : 0.f;
    te.zi[t] = v ? A.node_type[A.edge_row[e]] : 0;
    te.zj[t] = v ? A.node_type[A.col[e]] : 0;
  }
}

// rbf tile: X[r][k] = exp(coeff * (d_r - mu_k)^2); thread t owns basis k = t
__device__ __forceinline__ void rbf_tile(const e2v2_mlp_args& A, const TileEdges& te, float* X) {
  const int k = threadIdx.x;
  const float mu = A.rbf_offset[k];
#pragma unroll 4
  for (int r = 0; r < kT; ++r) {
    float x = te.d[r] - mu;
    X[r * kLdX + k] = te.valid[r] ? expf(A.rbf_coeff * (x * x)) : 0.f;
  }
}

__global__ __launch_bounds__(256) void k_mlp_fwd(e2v2_mlp_args A, float* __restrict__ out, int ld_out) {
  extern __shared__ float sm[];
  float* X = sm;                    // [32][258]: rbf tile, then h2 / y2 with stride kLdY
  float* Y = X + kT * kLdX;         // [32][130]
  __shared__ TileEdges te;
  const int m = blockIdx.y;
  const e2v2_mlp_weights& W = A.w[m];
  const int64_t e0 = (int64_t)blockIdx.x * kT;
  const int nvalid = (int)min<int64_t>(kT, A.n_edges - e0);
  float* sn = A.save_n ? A.save_n + ((size_t)m * A.n_edges + e0) * (2 * kH) : nullptr;
  float* sr = A.save_r ? A.save_r + ((size_t)m * A.n_edges + e0) * 2 : nullptr;
  load_tile_edges(A, e0, te);
  __syncthreads();
  rbf_tile(A, te, X);
  __syncthreads();
  {
    floatx4 acc[2][2];
    gemm32<kK0, kH>(X, kLdX, W.w1t, kH, acc);
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          int row, c;
          acc_coord<kH>(rt, ct, r, row, c);
          Y[row * kLdY + c] = acc[rt][ct][r] + W.ttgt[te.zi[row] * kH + c] + W.tsrc[te.zj[row] * kH + c];
        }
  }
  __syncthreads();
  ln_silu_rows(Y, kLdY, W.g1, W.be1, sn, 2 * kH, sr, 2, nvalid);
  __syncthreads();
  {
    floatx4 acc[2][2];
    gemm32<kH, kH>(Y, kLdY, W.w2t, kH, acc);
    store_acc<kH>(acc, X, kLdY, W.b2);
  }
  __syncthreads();
  ln_silu_rows(X, kLdY, W.g2, W.be2, sn ? sn + kH : nullptr, 2 * kH, sr ? sr + 1 : nullptr, 2, nvalid);
  __syncthreads();
  floatx4 acc[2][4];
  gemm32<kH, 256>(X, kLdY, W.w3t, 256, acc);
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        int row, c;
        acc_coord<256>(rt, ct, r, row, c);
        if (row < nvalid) out[(e0 + row) * ld_out + m * 256 + c] = acc[rt][ct][r] + W.b3[c];
      }
}

__global__ __launch_bounds__(256) void k_mlp_bwd(e2v2_mlp_args A, const float* __restrict__ dout, int ld_dout,
                                                 float* __restrict__ dd, int accumulate) {
  extern __shared__ float sm[];
  float* X = sm;                    // [32][258]
  float* Y = X + kT * kLdX;         // [32][130]
  __shared__ TileEdges te;
  __shared__ float part[4][kT];
  const int64_t e0 = (int64_t)blockIdx.x * kT;
  const int nvalid = (int)min<int64_t>(kT, A.n_edges - e0);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  load_tile_edges(A, e0, te);
  __syncthreads();
  float dd_lane[2][4];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int r = 0; r < 4; ++r) dd_lane[rt][r] = 0.f;
  for (int m = 0; m < A.n_mlp; ++m) {
    const e2v2_mlp_weights& W = A.w[m];
    const float* sn = A.save_n + ((size_t)m * A.n_edges + e0) * (2 * kH);
    const float* sr = A.save_r + ((size_t)m * A.n_edges + e0) * 2;
    for (int idx = threadIdx.x; idx < kT * 64; idx += 256) {   // dOut tile, float4 loads
      const int row = idx >> 6, c4 = idx & 63;
      float4 v = row < nvalid ? reinterpret_cast<const float4*>(dout + (e0 + row) * ld_dout + m * 256)[c4]
                              : float4{0.f, 0.f, 0.f, 0.f};
      float* xr = X + row * kLdX + 4 * c4;
      xr[0] = v.x; xr[1] = v.y; xr[2] = v.z; xr[3] = v.w;
    }
    __syncthreads();
    {  // dy2 = dOut . W3   (W3 [256][128] row-major = B[K=256][N=128])
      floatx4 acc[2][2];
      gemm32<256, kH>(X, kLdX, W.w3, kH, acc);
      store_acc<kH>(acc, Y, kLdY, nullptr);
    }
    __syncthreads();
    ln_silu_bwd_rows(Y, kLdY, sn + kH, 2 * kH, sr + 1, 2, nvalid, W.g2, W.be2);
    __syncthreads();
    {  // dy1 = dz2 . W2   (W2 [128][128]) -> X with stride kLdY
      floatx4 acc[2][2];
      gemm32<kH, kH>(Y, kLdY, W.w2, kH, acc);
      store_acc<kH>(acc, X, kLdY, nullptr);
    }
    __syncthreads();
    ln_silu_bwd_rows(X, kLdY, sn, 2 * kH, sr, 2, nvalid, W.g1, W.be1);
    __syncthreads();
    {  // drbf = dz1 . W1r  (W1 [128][ldw1], rbf columns 0..255); dd += sum_k drbf * rbf * 2c(d - mu)
      floatx4 acc[2][4];
      gemm32<kH, 256>(X, kLdY, W.w1, W.ldw1, acc);
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            int row, c;
            acc_coord<256>(rt, ct, r, row, c);
            float x = te.d[row] - A.rbf_offset[c];
            float rb = expf(A.rbf_coeff * (x * x));
            dd_lane[rt][r] += acc[rt][ct][r] * rb * (2.0f * A.rbf_coeff * x);
          }
    }
    __syncthreads();
  }
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = dd_lane[rt][r];
      v += __shfl_xor(v, 1, 64);
      v += __shfl_xor(v, 2, 64);
      v += __shfl_xor(v, 4, 64);
      v += __shfl_xor(v, 8, 64);
      if ((lane & 15) == 0) part[wave][rt * 16 + 4 * (lane >> 4) + r] = v;
    }
  __syncthreads();
  if (threadIdx.x < nvalid) {
    float v = part[0][threadIdx.x] + part[1][threadIdx.x] + part[2][threadIdx.x] + part[3][threadIdx.x];
    int64_t e = e0 + threadIdx.x;
    dd[e] = accumulate ? dd[e] + v : v;
  }
}


// ---------------------------------------------------------------------------
// bf16-operand variant (weights in bf16, fp32 accumulation): GEMMs on
// v_mfma_f32_16x16x32_bf16; LayerNorm, SiLU, tables, saved statistics and all
// outputs stay fp32.  B operands come as B^T row-major [N][K] in bf16 so each
// lane loads its 8 consecutive k values with one 16-byte load.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
constexpr int kLdXb = 264;   // bf16 row stride of K=256 tiles (multiple of 8)
constexpr int kLdYb = 136;   // bf16 row stride of K=128 tiles

template <int K, int N>
__device__ __forceinline__ void gemm32_bf16(const __bf16* A, int lda, const __bf16* __restrict__ Bt, int ldb,
                                            floatx4 (&acc)[2][N / 64]) {
  constexpr int CT = N / 64;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int cbase = wave * (N / 4);
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) acc[rt][ct] = floatx4{0.f, 0.f, 0.f, 0.f};
  bf16x8 bc[CT], bn[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct)
    bc[ct] = *reinterpret_cast<const bf16x8*>(Bt + (size_t)(cbase + ct * 16 + li) * ldb + 8 * lg);
#pragma unroll
  for (int k0 = 0; k0 < K; k0 += 32) {
    if (k0 + 32 < K) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
        bn[ct] = *reinterpret_cast<const bf16x8*>(Bt + (size_t)(cbase + ct * 16 + li) * ldb + k0 + 32 + 8 * lg);
    }
    const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(A + li * lda + k0 + 8 * lg);
    const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(A + (16 + li) * lda + k0 + 8 * lg);
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      acc[0][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bc[ct], acc[0][ct], 0, 0, 0);
      acc[1][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bc[ct], acc[1][ct], 0, 0, 0);
    }
    if (k0 + 32 < K) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) bc[ct] = bn[ct];
    }
  }
}

// LayerNorm(128) + SiLU of the fp32 rows in Yf; writes the bf16 activation to Yb
__device__ __forceinline__ void ln_silu_rows_bf16(const float* Yf, int ldf, __bf16* Yb, int ldb,
                                                  const float* __restrict__ g, const float* __restrict__ b,
                                                  float* nrm, int ldn, float* rstd_out, int rstd_stride, int nsave) {
  const int row = threadIdx.x >> 3, sub = threadIdx.x & 7;
  const float* y = Yf + row * ldf;
  float v[16];
  float s = 0.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) { v[q] = y[sub + 8 * q]; s += v[q]; }
  s += __shfl_xor(s, 1, 64); s += __shfl_xor(s, 2, 64); s += __shfl_xor(s, 4, 64);
  const float mean = s * (1.0f / kH);
  float s2 = 0.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) { float dl = v[q] - mean; s2 += dl * dl; }
  s2 += __shfl_xor(s2, 1, 64); s2 += __shfl_xor(s2, 2, 64); s2 += __shfl_xor(s2, 4, 64);
  const float rstd = 1.0f / sqrtf(s2 * (1.0f / kH) + 1e-5f);
  const bool save = nrm != nullptr && row < nsave;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int c = sub + 8 * q;
    const float n = (v[q] - mean) * rstd;
    if (save) nrm[(size_t)row * ldn + c] = n;
    Yb[row * ldb + c] = (__bf16)silu(n * g[c] + b[c]);
  }
  if (save && sub == 0) rstd_out[(size_t)row * rstd_stride] = rstd;
}

// SiLU/LN backward on fp32 rows of Yf -> bf16 rows of Yb
__device__ __forceinline__ void ln_silu_bwd_rows_bf16(const float* Yf, int ldf, __bf16* Yb, int ldb,
                                                      const float* __restrict__ nrm, int ldn,
                                                      const float* __restrict__ rstd, int rstd_stride, int nvalid,
                                                      const float* __restrict__ g, const float* __restrict__ b) {
  const int row = threadIdx.x >> 3, sub = threadIdx.x & 7;
  const float* y = Yf + row * ldf;
  const bool ok = row < nvalid;
  float dn[16], nn[16];
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int c = sub + 8 * q;
    const float n = ok ? nrm[(size_t)row * ldn + c] : 0.f;
    const float a = n * g[c] + b[c];
    const float sg = sigmoidf_(a);
    const float da = y[c] * sg * (1.0f + a * (1.0f - sg));
    dn[q] = da * g[c];
    nn[q] = n;
    s1 += dn[q];
    s2 += dn[q] * n;
  }
  s1 += __shfl_xor(s1, 1, 64); s1 += __shfl_xor(s1, 2, 64); s1 += __shfl_xor(s1, 4, 64);
  s2 += __shfl_xor(s2, 1, 64); s2 += __shfl_xor(s2, 2, 64); s2 += __shfl_xor(s2, 4, 64);
  const float m1 = s1 * (1.0f / kH), m2 = s2 * (1.0f / kH);
  const float r = ok ? rstd[(size_t)row * rstd_stride] : 0.f;
#pragma unroll
  for (int q = 0; q < 16; ++q) Yb[row * ldb + sub + 8 * q] = (__bf16)(r * (dn[q] - m1 - nn[q] * m2));
}

template <int N>
__device__ __forceinline__ void store_acc_f32(const floatx4 (&acc)[2][N / 64], float* Y, int ldy,
                                              const float* __restrict__ bias) {
  store_acc<N>(acc, Y, ldy, bias);
}

__global__ __launch_bounds__(256) void k_mlp_fwd_bf16(e2v2_mlp_args A, float* __restrict__ out, int ld_out) {
  extern __shared__ float sm[];
  __bf16* Xb = reinterpret_cast<__bf16*>(sm);                 // [32][264] bf16
  float* Yf = sm + (kT * kLdXb) / 2;                           // [32][130] fp32
  __bf16* Yb = reinterpret_cast<__bf16*>(Yf + kT * kLdY);      // [32][136] bf16
  __shared__ TileEdges te;
  const int m = blockIdx.y;
  const e2v2_mlp_weights& W = A.w[m];
  const __bf16* w1b = static_cast<const __bf16*>(W.w1b);
  const __bf16* w2b = static_cast<const __bf16*>(W.w2b);
  const __bf16* w3b = static_cast<const __bf16*>(W.w3b);
  const int64_t e0 = (int64_t)blockIdx.x * kT;
  const int nvalid = (int)min<int64_t>(kT, A.n_edges - e0);
  float* sn = A.save_n ? A.save_n + ((size_t)m * A.n_edges + e0) * (2 * kH) : nullptr;
  float* sr = A.save_r ? A.save_r + ((size_t)m * A.n_edges + e0) * 2 : nullptr;
  load_tile_edges(A, e0, te);
  __syncthreads();
  {
    const int k = threadIdx.x;
    const float mu = A.rbf_offset[k];
#pragma unroll 4
    for (int r = 0; r < kT; ++r) {
      const float x = te.d[r] - mu;
      Xb[r * kLdXb + k] = (__bf16)(te.valid[r] ? expf(A.rbf_coeff * (x * x)) : 0.f);
    }
  }
  __syncthreads();
  {
    floatx4 acc[2][2];
    gemm32_bf16<kK0, kH>(Xb, kLdXb, w1b, kK0, acc);
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          int row, c;
          acc_coord<kH>(rt, ct, r, row, c);
          Yf[row * kLdY + c] = acc[rt][ct][r] + W.ttgt[te.zi[row] * kH + c] + W.tsrc[te.zj[row] * kH + c];
        }
  }
  __syncthreads();
  ln_silu_rows_bf16(Yf, kLdY, Yb, kLdYb, W.g1, W.be1, sn, 2 * kH, sr, 2, nvalid);
  __syncthreads();
  {
    floatx4 acc[2][2];
    gemm32_bf16<kH, kH>(Yb, kLdYb, w2b, kH, acc);
    store_acc_f32<kH>(acc, Yf, kLdY, W.b2);
  }
  __syncthreads();
  ln_silu_rows_bf16(Yf, kLdY, Xb, kLdYb, W.g2, W.be2, sn ? sn + kH : nullptr, 2 * kH, sr ? sr + 1 : nullptr, 2,
                    nvalid);
  __syncthreads();
  floatx4 acc[2][4];
  gemm32_bf16<kH, 256>(Xb, kLdYb, w3b, kH, acc);
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        int row, c;
        acc_coord<256>(rt, ct, r, row, c);
        if (row < nvalid) out[(e0 + row) * ld_out + m * 256 + c] = acc[rt][ct][r] + W.b3[c];
      }
}

__global__ __launch_bounds__(256) void k_mlp_bwd_bf16(e2v2_mlp_args A, const float* __restrict__ dout, int ld_dout,
                                                      float* __restrict__ dd, int accumulate) {
  extern __shared__ float sm[];
  __bf16* Xb = reinterpret_cast<__bf16*>(sm);                 // [32][264] bf16
  float* Yf = sm + (kT * kLdXb) / 2;                           // [32][130] fp32
  __bf16* Yb = reinterpret_cast<__bf16*>(Yf + kT * kLdY);      // [32][136] bf16
  __shared__ TileEdges te;
  __shared__ float part[4][kT];
  const int64_t e0 = (int64_t)blockIdx.x * kT;
  const int nvalid = (int)min<int64_t>(kT, A.n_edges - e0);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  load_tile_edges(A, e0, te);
  __syncthreads();
  float dd_lane[2][4];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int r = 0; r < 4; ++r) dd_lane[rt][r] = 0.f;
  for (int m = 0; m < A.n_mlp; ++m) {
    const e2v2_mlp_weights& W = A.w[m];
    const __bf16* w3tb = static_cast<const __bf16*>(W.w3tb);
    const __bf16* w2tb = static_cast<const __bf16*>(W.w2tb);
    const __bf16* w1rtb = static_cast<const __bf16*>(W.w1rtb);
    const float* sn = A.save_n + ((size_t)m * A.n_edges + e0) * (2 * kH);
    const float* sr = A.save_r + ((size_t)m * A.n_edges + e0) * 2;
    for (int idx = threadIdx.x; idx < kT * 64; idx += 256) {
      const int row = idx >> 6, c4 = idx & 63;
      float4 v = row < nvalid ? reinterpret_cast<const float4*>(dout + (e0 + row) * ld_dout + m * 256)[c4]
                              : float4{0.f, 0.f, 0.f, 0.f};
      __bf16* xr = Xb + row * kLdXb + 4 * c4;
      xr[0] = (__bf16)v.x; xr[1] = (__bf16)v.y; xr[2] = (__bf16)v.z; xr[3] = (__bf16)v.w;
    }
    __syncthreads();
    {  // dy2 = dOut . W3   (B^T = W3^T [128][256])
      floatx4 acc[2][2];
      gemm32_bf16<256, kH>(Xb, kLdXb, w3tb, 256, acc);
      store_acc_f32<kH>(acc, Yf, kLdY, nullptr);
    }
    __syncthreads();
    ln_silu_bwd_rows_bf16(Yf, kLdY, Yb, kLdYb, sn + kH, 2 * kH, sr + 1, 2, nvalid, W.g2, W.be2);
    __syncthreads();
    {  // dy1 = dz2 . W2   (B^T = W2^T)
      floatx4 acc[2][2];
      gemm32_bf16<kH, kH>(Yb, kLdYb, w2tb, kH, acc);
      store_acc_f32<kH>(acc, Yf, kLdY, nullptr);
    }
    __syncthreads();
    ln_silu_bwd_rows_bf16(Yf, kLdY, Xb, kLdYb, sn, 2 * kH, sr, 2, nvalid, W.g1, W.be1);
    __syncthreads();
    {  // drbf = dz1 . W1r   (B^T = W1r^T [256][128])
      floatx4 acc[2][4];
      gemm32_bf16<kH, 256>(Xb, kLdYb, w1rtb, kH, acc);
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            int row, c;
            acc_coord<256>(rt, ct, r, row, c);
            float x = te.d[row] - A.rbf_offset[c];
            float rb = expf(A.rbf_coeff * (x * x));
            dd_lane[rt][r] += acc[rt][ct][r] * rb * (2.0f * A.rbf_coeff * x);
          }
    }
    __syncthreads();
  }
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = dd_lane[rt][r];
      v += __shfl_xor(v, 1, 64);
      v += __shfl_xor(v, 2, 64);
      v += __shfl_xor(v, 4, 64);
      v += __shfl_xor(v, 8, 64);
      if ((lane & 15) == 0) part[wave][rt * 16 + 4 * (lane >> 4) + r] = v;
    }
  __syncthreads();
  if (threadIdx.x < nvalid) {
    float v = part[0][threadIdx.x] + part[1][threadIdx.x] + part[2][threadIdx.x] + part[3][threadIdx.x];
    int64_t e = e0 + threadIdx.x;
    dd[e] = accumulate ? dd[e] + v : v;
  }
}

}  // namespace e2v2

using namespace e2v2;

static size_t mlp_lds() { return sizeof(float) * (kT * kLdX + kT * kLdY); }
static size_t mlp_lds_bf16() { return sizeof(__bf16) * (kT * kLdXb + kT * kLdYb) + sizeof(float) * kT * kLdY; }

E2V2_API int e2v2_mlp_fwd(const e2v2_mlp_args* args, float* out, int ld_out, hipStream_t s) {
  const e2v2_mlp_args& A = *args;
  E2V2_REQUIRE(A.n_mlp >= 1 && A.n_mlp <= E2V2_MAX_MLP, "mlp_fwd: n_mlp %d out of range", A.n_mlp);
  E2V2_REQUIRE(ld_out >= 256 * A.n_mlp, "mlp_fwd: ld_out %d < 256*n_mlp", ld_out);
  if (A.n_edges == 0) return 0;
  dim3 grid((unsigned)((A.n_edges + kT - 1) / kT), (unsigned)A.n_mlp);
  if (A.compute_bf16) {
    for (int m = 0; m < A.n_mlp; ++m)
      E2V2_REQUIRE(A.w[m].w1b && A.w[m].w2b && A.w[m].w3b, "mlp_fwd: bf16 weights missing for profile %d", m);
    hipLaunchKernelGGL(k_mlp_fwd_bf16, grid, dim3(256), mlp_lds_bf16(), s, A, out, ld_out);
    E2V2_LAUNCHED("k_mlp_fwd_bf16");
    return 0;
  }
  static bool attr = false;
  if (!attr) {
    E2V2_TRY_HIP(hipFuncSetAttribute((const void*)k_mlp_fwd, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)mlp_lds()));
    attr = true;
  }
  hipLaunchKernelGGL(k_mlp_fwd, grid, dim3(256), mlp_lds(), s, A, out, ld_out);
  E2V2_LAUNCHED("k_mlp_fwd");
  return 0;
}

E2V2_API int e2v2_mlp_bwd(const e2v2_mlp_args* args, const float* dout, int ld_dout, float* dd, int accumulate,
                          hipStream_t s) {
  const e2v2_mlp_args& A = *args;
  E2V2_REQUIRE(A.n_mlp >= 1 && A.n_mlp <= E2V2_MAX_MLP, "mlp_bwd: n_mlp %d out of range", A.n_mlp);
  E2V2_REQUIRE(ld_dout >= 256 * A.n_mlp && ld_dout % 4 == 0, "mlp_bwd: bad ld_dout %d", ld_dout);
  E2V2_REQUIRE(A.save_n != nullptr && A.save_r != nullptr,
               "mlp_bwd: needs the normalised activations saved by e2v2_mlp_fwd (save_n, save_r)");
  if (A.n_edges == 0) return 0;
  dim3 grid((unsigned)((A.n_edges + kT - 1) / kT));
  if (A.compute_bf16) {
    for (int m = 0; m < A.n_mlp; ++m)
      E2V2_REQUIRE(A.w[m].w3tb && A.w[m].w2tb && A.w[m].w1rtb, "mlp_bwd: bf16 weights missing for profile %d", m);
    hipLaunchKernelGGL(k_mlp_bwd_bf16, grid, dim3(256), mlp_lds_bf16(), s, A, dout, ld_dout, dd, accumulate);
    E2V2_LAUNCHED("k_mlp_bwd_bf16");
    return 0;
  }
  static bool attr = false;
  if (!attr) {
    E2V2_TRY_HIP(hipFuncSetAttribute((const void*)k_mlp_bwd, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)mlp_lds()));
    attr = true;
  }
  hipLaunchKernelGGL(k_mlp_bwd, grid, dim3(256), mlp_lds(), s, A, dout, ld_dout, dd, accumulate);
  E2V2_LAUNCHED("k_mlp_bwd");
  return 0;
}
