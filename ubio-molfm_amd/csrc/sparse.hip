// Segment (CSR) kernels behind the reference's op-level sparse edge functions
// (src/molfm/models/e2former/triton_dr/): edge-indexed dot products, their
// grouped reductions (the QK logits, the value aggregation and both of their
// gradients), the segmented alpha sum, row gathers and the edge-degree outer
// product with its gradient.  A segment layout is the reference's
// (row_ptr [R+1], col_index, alpha_index): slot p of row r carries edge
// alpha_index[p] and its partner row col_index[p].  Every row is summed in
// slot order by one workgroup (deterministic, no atomics).  Tensors are fp32
// with explicit element strides, so [R, H, D] and [M, C, H] operands share
// the kernels.  Slots whose partner row or edge id is out of range are skipped
// and row bounds are clamped to the slot arrays, so malformed metadata cannot
// make a kernel read or write outside its operands.  The attention and degree
// paths of the model run fused in attn.hip and deg.hip; these serve callers of
// the reference's op-level interfaces.
#include "common.h"
#include "../../include/e2v2.h"

namespace e2v2 {

constexpr int kSegThreads = 256;
constexpr int kSegMaxD = 16;   // d per thread of the h-fast segmented reduction
constexpr int kSegMaxA = 24;   // d of a segmented dot held in registers

struct SegRow {
  int p0, p1;
};

__device__ __forceinline__ SegRow seg_row(const e2v2_segments& S, int r) {
  const int64_t n = S.n_slots;
  int64_t a = S.row_ptr[r], b = S.row_ptr[r + 1];
  a = a < 0 ? 0 : (a > n ? n : a);
  b = b < a ? a : (b > n ? n : b);
  return {(int)a, (int)b};
}

__device__ __forceinline__ bool slot_ok(const e2v2_segments& S, int c, int e) {
  return c >= 0 && c < S.n_cols && e >= 0 && (int64_t)e < S.n_edges;
}

// Slots of one row staged in LDS (edge id and partner row, -1 for a skipped slot) when the row has at most
// kSegStage of them; longer rows read the slot arrays directly.
constexpr int kSegStage = 512;

__device__ __forceinline__ bool stage_row(const e2v2_segments& S, const SegRow& R, bool with_col, int* se, int* sc) {
  const int np = R.p1 - R.p0;
  if (np > kSegStage) return false;
  for (int t = threadIdx.x; t < np; t += kSegThreads) {
    const int p = R.p0 + t;
    const int e = S.alpha_index[p], c = with_col ? S.col_index[p] : 0;
    const bool ok = e >= 0 && (int64_t)e < S.n_edges && (!with_col || (c >= 0 && c < S.n_cols));
    se[t] = ok ? e : -1;
    sc[t] = ok ? c : 0;
  }
  __syncthreads();
  return true;
}

// out[alpha_index[p], h] = sum_d A[r, h, d] B[col_index[p], h, d] for the slots p of row r
__global__ __launch_bounds__(kSegThreads) void k_seg_dot(e2v2_segments S, const float* __restrict__ A, int64_t sa_r,
                                                         int64_t sa_h, int64_t sa_d, const float* __restrict__ B,
                                                         int64_t sb_r, int64_t sb_h, int64_t sb_d, int H, int D,
                                                         float* __restrict__ out, int64_t so_e, int64_t so_h) {
  __shared__ int se[kSegStage], sc[kSegStage];
  const int r = blockIdx.x;
  const SegRow R = seg_row(S, r);
  const bool staged = stage_row(S, R, true, se, sc);
  const unsigned n = (unsigned)(R.p1 - R.p0) * (unsigned)H;
  const float* a = A + (int64_t)r * sa_r;
  // H dividing the block: thread t keeps head t % H for every slot it takes (t / H, + 256 / H, ...), so its
  // A row stays in registers; each slot's B row is loaded whole before the products (summed in d order)
  if (kSegThreads % H == 0 && D <= kSegMaxA) {
    const int h = (int)threadIdx.x % H, ks = kSegThreads / H, np = R.p1 - R.p0;
    const float* ah = a + (int64_t)h * sa_h;
    float ar[kSegMaxA];
#pragma unroll
    for (int j = 0; j < kSegMaxA; ++j) ar[j] = j < D ? ah[(int64_t)j * sa_d] : 0.f;
    for (int k = (int)threadIdx.x / H; k < np; k += ks) {
      int c, e;
      if (staged) {
        e = se[k];
        c = sc[k];
        if (e < 0) continue;
      } else {
        const int p = R.p0 + k;
        c = S.col_index[p];
        e = S.alpha_index[p];
        if (!slot_ok(S, c, e)) continue;
      }
      const float* b = B + (int64_t)c * sb_r + (int64_t)h * sb_h;
      float y[kSegMaxA];
#pragma unroll
      for (int j = 0; j < kSegMaxA; ++j) y[j] = j < D ? b[(int64_t)j * sb_d] : 0.f;
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < kSegMaxA; ++j)
        if (j < D) s = fmaf(ar[j], y[j], s);
      out[(int64_t)e * so_e + (int64_t)h * so_h] = s;
    }
    return;
  }
  // unit-stride rows of 16-byte aligned groups of four: float4 loads (the same products, summed in d order)
  const bool v4 = sa_d == 1 && sb_d == 1 && (D & 3) == 0 && ((sa_r | sa_h | sb_r | sb_h) & 3) == 0 &&
                  (((uintptr_t)A | (uintptr_t)B) & 15) == 0;
  for (unsigned idx = threadIdx.x; idx < n; idx += kSegThreads) {
    const int k = (int)(idx / (unsigned)H), h = (int)(idx % (unsigned)H);
    int c, e;
    if (staged) {
      e = se[k];
      c = sc[k];
      if (e < 0) continue;
    } else {
      const int p = R.p0 + k;
      c = S.col_index[p];
      e = S.alpha_index[p];
      if (!slot_ok(S, c, e)) continue;
    }
    const float* b = B + (int64_t)c * sb_r + (int64_t)h * sb_h;
    const float* ah = a + (int64_t)h * sa_h;
    float s = 0.f;
    if (v4) {
      for (int d = 0; d < D; d += 4) {
        const float4 x = *reinterpret_cast<const float4*>(ah + d), y = *reinterpret_cast<const float4*>(b + d);
        s = fmaf(x.x, y.x, s);
        s = fmaf(x.y, y.y, s);
        s = fmaf(x.z, y.z, s);
        s = fmaf(x.w, y.w, s);
      }
    } else {
      // four d steps' loads issued before their products (the same order of the sum)
      int d = 0;
      for (; d + 4 <= D; d += 4) {
        float x[4], y[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          x[u] = ah[(int64_t)(d + u) * sa_d];
          y[u] = b[(int64_t)(d + u) * sb_d];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) s = fmaf(x[u], y[u], s);
      }
      for (; d < D; ++d) s = fmaf(ah[(int64_t)d * sa_d], b[(int64_t)d * sb_d], s);
    }
    out[(int64_t)e * so_e + (int64_t)h * so_h] = s;
  }
}

// out[r, h, d] = sum_{p in row r} W[alpha_index[p], h] X[col_index[p], h, d]; X NULL: the plain
// sum of W (D = 1).  Threads walk (h, d) with the operand's unit-stride index fastest.
__global__ __launch_bounds__(kSegThreads) void k_seg_reduce(e2v2_segments S, const float* __restrict__ W,
                                                            int64_t sw_e, int64_t sw_h, const float* __restrict__ X,
                                                            int64_t sx_r, int64_t sx_h, int64_t sx_d, int H, int D,
                                                            bool h_fast, float* __restrict__ out, int64_t so_r,
                                                            int64_t so_h, int64_t so_d) {
  __shared__ int se[kSegStage], sc[kSegStage];
  const int r = blockIdx.x;
  const SegRow R = seg_row(S, r);
  const bool staged = stage_row(S, R, X != nullptr, se, sc);
  const int np = R.p1 - R.p0;
  // h-fast X with H dividing the block: thread (g, h) = (t / H, t % H) owns d = g, g + G, ... (G = 256 / H,
  // at most kSegMaxD of them) and loads W[e, h] once per slot for all of them; the sums keep slot order
  const int G = (X && h_fast && kSegThreads % H == 0) ? kSegThreads / H : 0;
  if (staged && G > 0 && (D + G - 1) / G <= kSegMaxD) {
    const int t = threadIdx.x, h = t % H, g = t / H;
    const int nd = g < D ? (D - g + G - 1) / G : 0;
    const float* wh = W + (int64_t)h * sw_h;
    const float* xh = X + (int64_t)h * sx_h + (int64_t)g * sx_d;
    const int64_t xs = (int64_t)G * sx_d;
    float acc[kSegMaxD];
#pragma unroll
    for (int j = 0; j < kSegMaxD; ++j) acc[j] = 0.f;
    int k = 0;
    for (; k + 2 <= np; k += 2) {   // two slots' loads in flight
      float w[2], x[2][kSegMaxD];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int e = se[k + u];
        w[u] = e >= 0 ? wh[(int64_t)e * sw_e] : 0.f;
        const float* xr = xh + (int64_t)sc[k + u] * sx_r;
#pragma unroll
        for (int j = 0; j < kSegMaxD; ++j) x[u][j] = (e >= 0 && j < nd) ? xr[j * xs] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        if (se[k + u] < 0) continue;
#pragma unroll
        for (int j = 0; j < kSegMaxD; ++j)
          if (j < nd) acc[j] = fmaf(w[u], x[u][j], acc[j]);
      }
    }
    if (k < np && se[k] >= 0) {
      const float w = wh[(int64_t)se[k] * sw_e];
      const float* xr = xh + (int64_t)sc[k] * sx_r;
#pragma unroll
      for (int j = 0; j < kSegMaxD; ++j)
        if (j < nd) acc[j] = fmaf(w, xr[j * xs], acc[j]);
    }
#pragma unroll
    for (int j = 0; j < kSegMaxD; ++j)
      if (j < nd) out[(int64_t)r * so_r + (int64_t)h * so_h + (int64_t)(g + j * G) * so_d] = acc[j];
    return;
  }
  for (int idx = threadIdx.x; idx < H * D; idx += kSegThreads) {
    const int h = h_fast ? idx % H : idx / D, d = h_fast ? idx / H : idx % D;
    const float* wh = W + (int64_t)h * sw_h;
    const float* xh = X ? X + (int64_t)h * sx_h + (int64_t)d * sx_d : nullptr;
    float s = 0.f;
    if (staged) {
      // four slots' loads in flight at a time (a skipped slot loads nothing and adds nothing); the sum keeps
      // slot order
      int k = 0;
      for (; k + 4 <= np; k += 4) {
        int e[4];
        float w[4], x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          e[u] = se[k + u];
          w[u] = e[u] >= 0 ? wh[(int64_t)e[u] * sw_e] : 0.f;
          x[u] = (xh && e[u] >= 0) ? xh[(int64_t)sc[k + u] * sx_r] : 1.f;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (e[u] >= 0) s = xh ? fmaf(w[u], x[u], s) : s + w[u];
      }
      for (; k < np; ++k) {
        const int e = se[k];
        if (e < 0) continue;
        const float w = wh[(int64_t)e * sw_e];
        s = xh ? fmaf(w, xh[(int64_t)sc[k] * sx_r], s) : s + w;
      }
    } else {
      for (int p = R.p0; p < R.p1; ++p) {
        const int e = S.alpha_index[p];
        if (e < 0 || (int64_t)e >= S.n_edges) continue;
        const float w = wh[(int64_t)e * sw_e];
        if (X) {
          const int c = S.col_index[p];
          if (c < 0 || c >= S.n_cols) continue;
          s = fmaf(w, xh[(int64_t)c * sx_r], s);
        } else {
          s += w;
        }
      }
    }
    out[(int64_t)r * so_r + (int64_t)h * so_h + (int64_t)d * so_d] = s;
  }
}

// out[e, k] = in[index[e], k] (rows of K contiguous floats; an index outside [0, n_in) gives a zero row)
__global__ void k_gather_rows(const float* __restrict__ in, int64_t n_in, const int32_t* __restrict__ index,
                              int64_t n, int K, float* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n * K) return;
  const int64_t e = t / K;
  const int64_t i = index[e];
  out[t] = (i >= 0 && i < n_in) ? in[i * K + t % K] : 0.f;
}

// out[r, l, h] = sum_{p in row r} sh[e, l] fea[e, h], e = alpha_index[p]
__global__ __launch_bounds__(kSegThreads) void k_outer_reduce(e2v2_segments S, const float* __restrict__ sh,
                                                              const float* __restrict__ fea, int L, int H,
                                                              float* __restrict__ out) {
  const int r = blockIdx.x;
  const SegRow R = seg_row(S, r);
  for (int idx = threadIdx.x; idx < L * H; idx += kSegThreads) {
    const int l = idx / H, h = idx % H;
    float s = 0.f;
    for (int p = R.p0; p < R.p1; ++p) {
      const int64_t e = S.alpha_index[p];
      if (e < 0 || e >= S.n_edges) continue;
      s = fmaf(sh[e * L + l], fea[e * H + h], s);
    }
    out[(int64_t)r * L * H + idx] = s;
  }
}

// dsh[e, l] = sum_h g[q[e], l, h] fea[e, h]  (q[e] outside [0, n_rows): 0)
__global__ void k_outer_dsh(const float* __restrict__ g, int n_rows, const float* __restrict__ fea,
                            const int32_t* __restrict__ qidx, int64_t n_edges, int L, int H, float* __restrict__ dsh) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_edges * L) return;
  const int64_t e = t / L;
  const int l = (int)(t % L);
  const int q = qidx[e];
  float s = 0.f;
  if (q >= 0 && q < n_rows) {
    const float* gr = g + ((int64_t)q * L + l) * H;
    const float* f = fea + e * H;
    for (int h = 0; h < H; ++h) s = fmaf(gr[h], f[h], s);
  }
  dsh[t] = s;
}

// The same, one wavefront per edge for H <= 256 channels in groups of four and L <= kOuterL: lane t owns
// channels 4 t .. 4 t + 3 of fea[e] (loaded once) and of each g row; per l the lanes' partial dots are added
// by a fixed-order wave sum.
constexpr int kOuterL = 9, kOuterWaves = 4;
__global__ __launch_bounds__(64 * kOuterWaves) void k_outer_dsh_w(const float* __restrict__ g, int n_rows,
                                                                 const float* __restrict__ fea,
                                                                 const int32_t* __restrict__ qidx, int64_t n_edges,
                                                                 int L, int H, float* __restrict__ dsh) {
  const int64_t e = (int64_t)blockIdx.x * kOuterWaves + (threadIdx.x >> 6);
  if (e >= n_edges) return;
  const int lane = threadIdx.x & 63, c = 4 * lane;
  const int q = qidx[e];
  const bool ok = q >= 0 && q < n_rows, in = c < H;
  float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
  if (ok && in) f = *reinterpret_cast<const float4*>(fea + e * H + c);
#pragma unroll
  for (int l = 0; l < kOuterL; ++l) {
    if (l >= L) break;
    float v = 0.f;
    if (ok && in) {
      const float4 x = *reinterpret_cast<const float4*>(g + ((int64_t)q * L + l) * H + c);
      v = x.x * f.x;
      v = fmaf(x.y, f.y, v);
      v = fmaf(x.z, f.z, v);
      v = fmaf(x.w, f.w, v);
    }
    v = wave_sum(v);
    if (lane == 0) dsh[e * L + l] = v;
  }
}

// dfea[e, h] = sum_l g[q[e], l, h] sh[e, l]  (q[e] outside [0, n_rows): 0)
__global__ void k_outer_dfea(const float* __restrict__ g, int n_rows, const float* __restrict__ sh,
                             const int32_t* __restrict__ qidx, int64_t n_edges, int L, int H,
                             float* __restrict__ dfea) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_edges * H) return;
  const int64_t e = t / H;
  const int h = (int)(t % H);
  const int q = qidx[e];
  float s = 0.f;
  if (q >= 0 && q < n_rows) {
    const float* gr = g + (int64_t)q * L * H + h;
    const float* s_e = sh + e * L;
    for (int l = 0; l < L; ++l) s = fmaf(gr[(int64_t)l * H], s_e[l], s);
  }
  dfea[t] = s;
}

static inline unsigned blocks_of(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

static int check_segments(const e2v2_segments* S, bool need_col, const char* what) {
  E2V2_REQUIRE(S != nullptr, "%s: null segment layout", what);
  E2V2_REQUIRE(S->n_rows >= 0 && S->n_slots >= 0 && S->n_edges >= 0 && S->n_cols >= 0,
               "%s: negative size (rows %d, cols %d, slots %lld, edges %lld)", what, S->n_rows, S->n_cols,
               (long long)S->n_slots, (long long)S->n_edges);
  E2V2_REQUIRE(S->n_slots < (1ll << 31), "%s: %lld slots exceed the 32-bit slot index", what,
               (long long)S->n_slots);
  E2V2_REQUIRE(S->n_rows == 0 || S->row_ptr, "%s: null row_ptr", what);
  E2V2_REQUIRE(S->n_slots == 0 || (S->alpha_index && (!need_col || S->col_index)),
               "%s: null col_index / alpha_index", what);
  return 0;
}

// Per-edge contraction of a query node's irreps with the edge's spherical
// harmonics, l by l: x0[e][l][c] = sum_{m in l} Y[e][m] xn[m][row(e)][c] (the
// x_0_extra of the QKdot_alpha / QKdotS_alpha gates, e2former.py:271-277 and
// 288-296), for lmax = 2 (9 m-rows, 3 l-blocks) and C <= 256 channels.  One
// wavefront per query row (edges of a row contiguous, CSR row_ptr), lanes over
// channels (up to four each), the row's node values held in registers.  The
// backward of the same row forms dxn[m][i][c] = sum_e Y[e][m] g[e][l(m)][c]
// in registers (no atomics) and dY[e][m] = sum_c g[e][l(m)][c] xn[m][i][c] by a
// fixed-order butterfly over the lanes.
constexpr int kShWaves = 4, kShPer = 4;

__device__ __forceinline__ int sh_l(int m) { return m == 0 ? 0 : (m < 4 ? 1 : 2); }

__global__ __launch_bounds__(64 * kShWaves) void k_sh_contract(const float* __restrict__ Y,
                                                               const float* __restrict__ xn,
                                                               const int32_t* __restrict__ row_ptr, int32_t n_rows,
                                                               int32_t C, float* __restrict__ x0) {
  const int i = blockIdx.x * kShWaves + (threadIdx.x >> 6);
  if (i >= n_rows) return;
  const int lane = threadIdx.x & 63;
  const size_t ms = (size_t)n_rows * C;
  float xr[kShPer][9];
#pragma unroll
  for (int q = 0; q < kShPer; ++q) {
    const int c = lane + 64 * q;
#pragma unroll
    for (int m = 0; m < 9; ++m) xr[q][m] = c < C ? xn[m * ms + (size_t)i * C + c] : 0.f;
  }
  const int b = row_ptr[i], n = row_ptr[i + 1] - b;
  for (int k = 0; k < n; ++k) {
    const int64_t e = (int64_t)b + k;
    float y[9];
#pragma unroll
    for (int m = 0; m < 9; ++m) y[m] = Y[e * 9 + m];
#pragma unroll
    for (int q = 0; q < kShPer; ++q) {
      const int c = lane + 64 * q;
      if (c < C) {
        float* o = x0 + (size_t)e * 3 * C + c;
        o[0] = y[0] * xr[q][0];
        o[C] = fmaf(y[3], xr[q][3], fmaf(y[2], xr[q][2], y[1] * xr[q][1]));
        o[2 * C] = fmaf(y[8], xr[q][8], fmaf(y[7], xr[q][7], fmaf(y[6], xr[q][6], fmaf(y[5], xr[q][5],
                   y[4] * xr[q][4]))));
      }
    }
  }
}

__global__ __launch_bounds__(64 * kShWaves) void k_sh_contract_bwd(const float* __restrict__ Y,
                                                                   const float* __restrict__ xn,
                                                                   const int32_t* __restrict__ row_ptr,
                                                                   int32_t n_rows, int32_t C,
                                                                   const float* __restrict__ g,
                                                                   float* __restrict__ dY, float* __restrict__ dxn) {
  const int i = blockIdx.x * kShWaves + (threadIdx.x >> 6);
  if (i >= n_rows) return;
  const int lane = threadIdx.x & 63;
  const size_t ms = (size_t)n_rows * C;
  float xr[kShPer][9], dx[kShPer][9];
#pragma unroll
  for (int q = 0; q < kShPer; ++q) {
    const int c = lane + 64 * q;
#pragma unroll
    for (int m = 0; m < 9; ++m) {
      xr[q][m] = c < C ? xn[m * ms + (size_t)i * C + c] : 0.f;
      dx[q][m] = 0.f;
    }
  }
  const int b = row_ptr[i], n = row_ptr[i + 1] - b;
  for (int k = 0; k < n; ++k) {
    const int64_t e = (int64_t)b + k;
    float y[9], p[9];
#pragma unroll
    for (int m = 0; m < 9; ++m) {
      y[m] = Y[e * 9 + m];
      p[m] = 0.f;
    }
#pragma unroll
    for (int q = 0; q < kShPer; ++q) {
      const int c = lane + 64 * q;
      const float* gp = g + (size_t)e * 3 * C + c;
      const float gl[3] = {c < C ? gp[0] : 0.f, c < C ? gp[C] : 0.f, c < C ? gp[2 * C] : 0.f};
#pragma unroll
      for (int m = 0; m < 9; ++m) {
        dx[q][m] = fmaf(y[m], gl[sh_l(m)], dx[q][m]);
        p[m] = fmaf(gl[sh_l(m)], xr[q][m], p[m]);
      }
    }
#pragma unroll
    for (int m = 0; m < 9; ++m) {
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) p[m] += __shfl_xor(p[m], o, kWave);
    }
    if (lane < 9) {
      float v = p[0];
#pragma unroll
      for (int m = 1; m < 9; ++m) v = lane == m ? p[m] : v;
      dY[e * 9 + lane] = v;
    }
  }
#pragma unroll
  for (int q = 0; q < kShPer; ++q) {
    const int c = lane + 64 * q;
    if (c < C) {
#pragma unroll
      for (int m = 0; m < 9; ++m) dxn[m * ms + (size_t)i * C + c] = dx[q][m];
    }
  }
}

}  // namespace e2v2

using namespace e2v2;

E2V2_API int e2v2_seg_dot(const e2v2_segments* S, const float* A, const int64_t* a_strides, const float* B,
                          const int64_t* b_strides, int H, int D, float* out, const int64_t* out_strides,
                          hipStream_t s) {
  if (int rc = check_segments(S, true, "seg_dot")) return rc;
  E2V2_REQUIRE(H >= 1 && D >= 1 && a_strides && b_strides && out_strides, "seg_dot: bad sizes (H %d, D %d)", H, D);
  if (S->n_rows == 0 || S->n_slots == 0) return 0;
  E2V2_REQUIRE(A && B && out, "seg_dot: null operand");
  E2V2_REQUIRE((int64_t)S->n_slots * H < (1ll << 32), "seg_dot: rows of up to 2^32 / H slots");
  hipLaunchKernelGGL(k_seg_dot, dim3(S->n_rows), dim3(kSegThreads), 0, s, *S, A, a_strides[0], a_strides[1],
                     a_strides[2], B, b_strides[0], b_strides[1], b_strides[2], H, D, out, out_strides[0],
                     out_strides[1]);
  E2V2_LAUNCHED("k_seg_dot");
  return 0;
}

E2V2_API int e2v2_seg_reduce(const e2v2_segments* S, const float* W, const int64_t* w_strides, const float* X,
                             const int64_t* x_strides, int H, int D, float* out, const int64_t* out_strides,
                             hipStream_t s) {
  if (int rc = check_segments(S, X != nullptr, "seg_reduce")) return rc;
  E2V2_REQUIRE(H >= 1 && D >= 1 && (int64_t)H * D < (1ll << 31) && w_strides && out_strides &&
                   (X == nullptr || x_strides),
               "seg_reduce: bad sizes (H %d, D %d)", H, D);
  E2V2_REQUIRE(X != nullptr || D == 1, "seg_reduce: a plain sum (X NULL) has D = 1");
  if (S->n_rows == 0) return 0;
  E2V2_REQUIRE(W && out, "seg_reduce: null operand");
  const int64_t z = 0;
  const bool h_fast = X ? (x_strides[1] <= x_strides[2]) : true;
  hipLaunchKernelGGL(k_seg_reduce, dim3(S->n_rows), dim3(kSegThreads), 0, s, *S, W, w_strides[0], w_strides[1], X,
                     X ? x_strides[0] : z, X ? x_strides[1] : z, X ? x_strides[2] : z, H, D, h_fast, out,
                     out_strides[0], out_strides[1], out_strides[2]);
  E2V2_LAUNCHED("k_seg_reduce");
  return 0;
}

E2V2_API int e2v2_gather_rows(const float* in, int64_t n_in, const int32_t* index, int64_t n, int K, float* out,
                              hipStream_t s) {
  E2V2_REQUIRE(n >= 0 && n_in >= 0 && K >= 1, "gather_rows: bad sizes (n %lld, K %d)", (long long)n, K);
  if (n == 0) return 0;
  E2V2_REQUIRE(in && index && out, "gather_rows: null pointer");
  hipLaunchKernelGGL(k_gather_rows, dim3(blocks_of(n * K, 256)), dim3(256), 0, s, in, n_in, index, n, K, out);
  E2V2_LAUNCHED("k_gather_rows");
  return 0;
}

E2V2_API int e2v2_outer_reduce(const e2v2_segments* S, const float* sh, const float* fea, int L, int H, float* out,
                               hipStream_t s) {
  if (int rc = check_segments(S, false, "outer_reduce")) return rc;
  E2V2_REQUIRE(L >= 1 && H >= 1 && (int64_t)L * H < (1ll << 31), "outer_reduce: bad sizes (L %d, H %d)", L, H);
  if (S->n_rows == 0) return 0;
  E2V2_REQUIRE(sh && fea && out, "outer_reduce: null operand");
  hipLaunchKernelGGL(k_outer_reduce, dim3(S->n_rows), dim3(kSegThreads), 0, s, *S, sh, fea, L, H, out);
  E2V2_LAUNCHED("k_outer_reduce");
  return 0;
}

E2V2_API int e2v2_outer_bwd(const float* grad, int n_rows, const float* sh, const float* fea,
                            const int32_t* query_index, int64_t n_edges, int L, int H, float* dsh, float* dfea,
                            hipStream_t s) {
  E2V2_REQUIRE(n_rows >= 0 && n_edges >= 0 && L >= 1 && H >= 1, "outer_bwd: bad sizes (E %lld, L %d, H %d)",
               (long long)n_edges, L, H);
  if (n_edges == 0) return 0;
  E2V2_REQUIRE(grad && query_index && (dsh == nullptr || fea) && (dfea == nullptr || sh),
               "outer_bwd: null operand");
  if (dsh) {
    if (H <= 256 && H % 4 == 0 && L <= kOuterL && ((uintptr_t)grad & 15) == 0 && ((uintptr_t)fea & 15) == 0) {
      hipLaunchKernelGGL(k_outer_dsh_w, dim3(blocks_of(n_edges, kOuterWaves)), dim3(64 * kOuterWaves), 0, s, grad,
                         n_rows, fea, query_index, n_edges, L, H, dsh);
      E2V2_LAUNCHED("k_outer_dsh_w");
    } else {
      hipLaunchKernelGGL(k_outer_dsh, dim3(blocks_of(n_edges * L, 256)), dim3(256), 0, s, grad, n_rows, fea,
                         query_index, n_edges, L, H, dsh);
      E2V2_LAUNCHED("k_outer_dsh");
    }
  }
  if (dfea) {
    hipLaunchKernelGGL(k_outer_dfea, dim3(blocks_of(n_edges * H, 256)), dim3(256), 0, s, grad, n_rows, sh,
                       query_index, n_edges, L, H, dfea);
    E2V2_LAUNCHED("k_outer_dfea");
  }
  return 0;
}

E2V2_API int e2v2_sh_contract(const float* Y, const float* xn, const int32_t* row_ptr, int32_t n_rows, int32_t C,
                              float* x0, hipStream_t s) {
  E2V2_REQUIRE(n_rows >= 0 && C >= 1 && C <= 64 * kShPer && (n_rows == 0 || (Y && xn && row_ptr && x0)),
               "sh_contract: bad arguments (n_rows %d, C %d; C must be 1..%d)", n_rows, C, 64 * kShPer);
  if (n_rows == 0) return 0;
  hipLaunchKernelGGL(k_sh_contract, dim3((unsigned)((n_rows + kShWaves - 1) / kShWaves)), dim3(64 * kShWaves), 0, s,
                     Y, xn, row_ptr, n_rows, C, x0);
  E2V2_LAUNCHED("k_sh_contract");
  return 0;
}

E2V2_API int e2v2_sh_contract_bwd(const float* Y, const float* xn, const int32_t* row_ptr, int32_t n_rows, int32_t C,
                                  const float* g, float* dY, float* dxn, hipStream_t s) {
  E2V2_REQUIRE(n_rows >= 0 && C >= 1 && C <= 64 * kShPer &&
                   (n_rows == 0 || (Y && xn && row_ptr && g && dY && dxn)),
               "sh_contract_bwd: bad arguments (n_rows %d, C %d; C must be 1..%d)", n_rows, C, 64 * kShPer);
  if (n_rows == 0) return 0;
  hipLaunchKernelGGL(k_sh_contract_bwd, dim3((unsigned)((n_rows + kShWaves - 1) / kShWaves)), dim3(64 * kShWaves), 0,
                     s, Y, xn, row_ptr, n_rows, C, g, dY, dxn);
  E2V2_LAUNCHED("k_sh_contract_bwd");
  return 0;
}
