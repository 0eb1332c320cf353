// Q/K projection of E2Former's attention as fp32 MFMA GEMMs with the
// SO3_Linear2Scalar m-contraction fused in
// (module_utils.py:2198-2272 SO3_Linear2Scalar_e2former, called for the query
// and key inputs at e2former.py:300-303).
//
// Forward, per m-row m of degree l = l(m) and node n:
//   y[m][n][o] = sum_k x[m][n][k] W_l[o][k] (+ bias[o] on m = 0),
//   o over [q_a | q_b | k_a | k_b] (hid columns each),
//   hq[n][l hid + c] = sum_{m in l} y[m][n][c] y[m][n][hid + c]   (hk likewise from k_a, k_b).
// y is kept for the backward.  The contraction is formed on the GEMM's
// accumulators: a wavefront owns the a- and b-columns of the same 32 channels,
// whose 32x32 MFMA accumulator tiles have identical lane layouts.
//
// Backward: gx[m][n][k] = sum_o gy[m][n][o] W_l[o][k] with gy (the m-contraction's
// gradient, gy[m][n][c] = ghq[n][l hid + c] y[m][n][hid + c] etc.) formed while the
// A operand is staged, so it is never written; optionally + sum_j gv[m][n][j] Wv_l[j][k]
// (the value projection's input gradient, same x) as further K stages.
//
// Tiling: 128 nodes x 128 GEMM columns per workgroup, eight wavefronts of 32 x 64
// (4 x 2; two 32x32 tiles of v_mfma_f32_32x32x2f32 each, at most 128 VGPRs so that
// two workgroups, four waves per SIMD, share a CU), K staged through LDS 32 at a
// time in two buffers (32 KB each).  In LDS a row keeps its 32 k as eight 16-byte granules,
// granule g of row r at slot g ^ (r & 7), so the eight lanes of a 128-byte
// ds_read_b128 phase read eight different bank groups.  An MFMA k-step s of an
// 8-k group takes k = 4 (lane / 32) + s in both operands: one 16-byte LDS read per
// operand and group.
#include "common.h"

namespace e2v2 {
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kPjRows = 128;                    // nodes per workgroup
constexpr int kPjCols = 128;                    // GEMM columns per workgroup
constexpr int kPjK = 32;                        // K per LDS stage (16 or 32)
constexpr int kPjG = kPjK / 4;                  // 16-byte granules per row and stage
constexpr int kPjT = 512;                       // threads per workgroup (8 waves, 4 x 2)
constexpr int kPjPer = kPjRows * kPjG / kPjT;    // granules per thread and operand
constexpr int kPjStage = (kPjRows + kPjCols) * kPjK;  // floats per stage buffer

__device__ __forceinline__ int pj_l(int m) { return m == 0 ? 0 : (m < 4 ? 1 : 2); }
// LDS float offset of granule g of row r: 128-byte lines of 8 granules (one row of
// 32 k, or two rows of 16 k) with the granule slot XOR-ed by the line index
__device__ __forceinline__ int pj_slot(int r, int g) {
  if (kPjK == 32) return r * 32 + ((g ^ (r & 7)) << 2);
  return (r >> 1) * 32 + (((((r & 1) << 2) | g) ^ ((r >> 1) & 7)) << 2);
}

// kPjK k of one stage: 8-k groups, each four k-steps on the wave's 1 x 2 tiles (rows
// 32 wr.., columns 64 wc + 32 j..).
__device__ __forceinline__ void pj_mma(const float* __restrict__ As, const float* __restrict__ Bs,
                                       floatx16 (&acc)[2], int wr, int wc, int lane) {
  const int r0 = wr * 32 + (lane & 31), c0 = wc * 64 + (lane & 31), h = lane >> 5;
#pragma unroll
  for (int grp = 0; grp < kPjK / 8; ++grp) {
    const floatx4 a = *reinterpret_cast<const floatx4*>(As + pj_slot(r0, 2 * grp + h));
    floatx4 b[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) b[j] = *reinterpret_cast<const floatx4*>(Bs + pj_slot(c0 + 32 * j, 2 * grp + h));
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b[j][s], acc[j], 0, 0, 0);
  }
}

__device__ __forceinline__ void pj_zero(floatx16 (&acc)[2]) {
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
}

__device__ __forceinline__ void pj_zero(floatx16 (&acc)[2][2]) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
}

// Row of accumulator register r of a 32x32 tile for this lane (column = lane & 31).
__device__ __forceinline__ int pj_acc_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// ---------------------------------------------------------------------------
// Forward.  Workgroup tile: nodes row0 .. row0+127, channel pairs p0 .. p0+63
// (pair p < hid: q channel p; else k channel p - hid).  LDS B column cl:
// wave column wc = cl / 64, a/b = (cl / 32) & 1, pair p0 + 32 wc + (cl & 31).
__device__ __forceinline__ int pj_pair_col(int p, int ab, int hid) {
  return p < hid ? (ab ? hid + p : p) : (ab ? 2 * hid + p : hid + p);
}

__global__ __launch_bounds__(kPjT) __attribute__((amdgpu_waves_per_eu(4))) void k_qk_proj_fwd(const float* __restrict__ x, const float* __restrict__ w,
                                                        const float* __restrict__ bias, float* __restrict__ y,
                                                        float* __restrict__ hq, float* __restrict__ hk, int n,
                                                        int hid, int c) {
  __shared__ __attribute__((aligned(16))) float lds[2 * kPjStage];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6, wr = wv >> 1, wc = wv & 1;
  const int n_cb = (2 * hid) / 64, n_rb = (n + kPjRows - 1) / kPjRows, n_tiles = n_rb * n_cb;
  // three groups of xcd_grid(n_tiles) workgroups, l = 2, 1, 0 (5, 3, 1 m-rows of work):
  // the long tiles are dispatched first, the short ones fill the tail
  const int grp = blockIdx.x / xcd_grid(n_tiles), L = 2 - grp;
  const int tile = xcd_row(blockIdx.x - grp * xcd_grid(n_tiles), n_tiles);
  if (tile >= n_tiles) return;
  const int row0 = (tile / n_cb) * kPjRows, p0 = (tile % n_cb) * 64;
  const int O = 4 * hid, nk = c / kPjK, m0 = L * L, n_it = (2 * L + 1) * nk;

  // staging assignment: granule g of rows / columns t / kPjG + (kPjT / kPjG) i
  const int g = t % kPjG;
  int a_row[kPjPer], b_col[kPjPer];
#pragma unroll
  for (int i = 0; i < kPjPer; ++i) {
    a_row[i] = row0 + t / kPjG + (kPjT / kPjG) * i;
    const int cl = t / kPjG + (kPjT / kPjG) * i;
    b_col[i] = pj_pair_col(p0 + 32 * (cl >> 6) + (cl & 31), (cl >> 5) & 1, hid);
  }
  // 32-bit element offsets from wave-uniform bases (per m / per l)
  uint32_t a_off[kPjPer], b_off[kPjPer];
#pragma unroll
  for (int i = 0; i < kPjPer; ++i) {
    a_off[i] = (uint32_t)a_row[i] * c + 4 * g;
    b_off[i] = (uint32_t)b_col[i] * c + 4 * g;
  }
  struct Regs { floatx4 a[kPjPer], b[kPjPer]; };
  const float* wl = w + (size_t)L * O * c;
  auto load = [&](int it, Regs& R) {
    const int m = m0 + it / nk, k0 = (it % nk) * kPjK;
    const float* xm = x + (size_t)m * n * c + k0;
    const float* wk = wl + k0;
#pragma unroll
    for (int i = 0; i < kPjPer; ++i) {
      R.a[i] = a_row[i] < n ? *reinterpret_cast<const floatx4*>(xm + a_off[i]) : floatx4{0.f, 0.f, 0.f, 0.f};
      R.b[i] = *reinterpret_cast<const floatx4*>(wk + b_off[i]);
    }
  };
  auto store = [&](int it, const Regs& R) {
    float* As = lds + (it & 1) * kPjStage;
    float* Bs = As + kPjRows * kPjK;
#pragma unroll
    for (int i = 0; i < kPjPer; ++i) {
      const int r = t / kPjG + (kPjT / kPjG) * i;
      *reinterpret_cast<floatx4*>(As + pj_slot(r, g)) = R.a[i];
      *reinterpret_cast<floatx4*>(Bs + pj_slot(r, g)) = R.b[i];
    }
  };

  // epilogue coordinates: this lane's pair and its a/b output columns; the lane's
  // first accumulator row is erow, register (i, r) adds pj_acc_row(r, 0) + 32 i
  const int p = p0 + 32 * wc + (lane & 31);
  const int oa = pj_pair_col(p, 0, hid), ob = pj_pair_col(p, 1, hid);
  const int erow = row0 + wr * 32 + 4 * (lane >> 5);
  const uint32_t y_off = (uint32_t)erow * O + oa, h_off = (uint32_t)erow * 3 * hid + (p < hid ? p : p - hid);
  float* hbase = p < hid ? hq : hk;
  const float ba = bias ? bias[oa] : 0.f, bb = bias ? bias[ob] : 0.f;

  floatx16 acc[2];   // the a- and b-columns of the wave's 32 channels
  pj_zero(acc);
  float s[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) s[r] = 0.f;

  // stages: LDS buffer it & 1; the next stage's global loads are in flight during the MFMAs
  Regs R;
  load(0, R);
  store(0, R);
  __syncthreads();
  for (int it = 0; it < n_it; ++it) {
    if (it + 1 < n_it) load(it + 1, R);
    const float* As = lds + (it & 1) * kPjStage;
    pj_mma(As, As + kPjRows * kPjK, acc, wr, wc, lane);
    if (it % nk == nk - 1) {
      const int m = m0 + it / nk;
      const float a0 = m == 0 ? ba : 0.f, b0 = m == 0 ? bb : 0.f;
      float* ym = y + (size_t)m * n * O;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int dr = pj_acc_row(r, 0);
        const float va = acc[0][r] + a0, vb = acc[1][r] + b0;
        s[r] = fmaf(va, vb, s[r]);
        if (erow + dr < n) {
          float* yr = ym + (size_t)dr * O;
          yr[y_off] = va;
          yr[y_off + (ob - oa)] = vb;
        }
      }
      pj_zero(acc);
      if (it == n_it - 1) {
        float* hl = hbase + L * hid;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dr = pj_acc_row(r, 0);
          if (erow + dr < n) hl[(size_t)dr * 3 * hid + h_off] = s[r];
          s[r] = 0.f;
        }
      }
    }
    if (it + 1 < n_it) store(it + 1, R);
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Backward.  Workgroup tile: m-row m, nodes row0 .. row0+127, input channels
// k0 .. k0+127.  K stages: the 4 hid columns of gy (formed from y and ghq/ghk),
// then the cv columns of gv when given.
__global__ __launch_bounds__(kPjT) __attribute__((amdgpu_waves_per_eu(4))) void k_qk_proj_bwd(const float* __restrict__ y, const float* __restrict__ ghq,
                                                        const float* __restrict__ ghk,
                                                        const float* __restrict__ wt,
                                                        const float* __restrict__ gv,
                                                        const float* __restrict__ wvt, float* __restrict__ gx,
                                                        int n, int hid, int c, int cv) {
  __shared__ __attribute__((aligned(16))) float lds[2 * kPjStage];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6, wr = wv >> 1, wc = wv & 1;
  const int n_cb = c / kPjCols, n_rb = (n + kPjRows - 1) / kPjRows;
  const int n_tiles = 9 * n_rb * n_cb;
  const int tile = xcd_row(blockIdx.x, n_tiles);
  if (tile >= n_tiles) return;
  const int m = tile / (n_rb * n_cb), rem = tile % (n_rb * n_cb);
  const int row0 = (rem / n_cb) * kPjRows, col0 = (rem % n_cb) * kPjCols, l = pj_l(m);
  const int O = 4 * hid, nkq = O / kPjK, n_it = nkq + (gv ? cv / kPjK : 0);

  const int g = t % kPjG;
  int a_row[kPjPer];
  uint32_t y_off[kPjPer], g_off[kPjPer], v_off[kPjPer], b_off[kPjPer], bv_off[kPjPer];
#pragma unroll
  for (int i = 0; i < kPjPer; ++i) {
    a_row[i] = row0 + t / kPjG + (kPjT / kPjG) * i;
    y_off[i] = (uint32_t)a_row[i] * O + 4 * g;
    g_off[i] = (uint32_t)a_row[i] * 3 * hid + 4 * g;
    v_off[i] = (uint32_t)a_row[i] * cv + 4 * g;
    b_off[i] = (uint32_t)(col0 + t / kPjG + (kPjT / kPjG) * i) * O + 4 * g;
    bv_off[i] = (uint32_t)(col0 + t / kPjG + (kPjT / kPjG) * i) * cv + 4 * g;
  }
  const float* ym = y + (size_t)m * n * O;
  const float* wt_m = wt + (size_t)m * c * O;
  struct Regs { floatx4 a[kPjPer], b[kPjPer], g[kPjPer]; };  // g: the gradient factor of a gy stage (multiplied in when staged)
  auto load = [&](int it, Regs& R) {
    if (it < nkq) {
      const int j0 = it * kPjK, q = j0 / hid;
      const float* yp = ym + (q & 1 ? j0 - hid : j0 + hid);            // the other factor's columns
      const float* gs = (q < 2 ? ghq : ghk) + l * hid + (j0 - q * hid);  // channel within the quarter
      const float* wp = wt_m + j0;
#pragma unroll
      for (int i = 0; i < kPjPer; ++i) {
        const bool ok = a_row[i] < n;
        R.a[i] = ok ? *reinterpret_cast<const floatx4*>(yp + y_off[i]) : floatx4{0.f, 0.f, 0.f, 0.f};
        R.g[i] = ok ? *reinterpret_cast<const floatx4*>(gs + g_off[i]) : floatx4{0.f, 0.f, 0.f, 0.f};
        R.b[i] = *reinterpret_cast<const floatx4*>(wp + b_off[i]);
      }
    } else {
      const int j0 = (it - nkq) * kPjK;
      const float* vp = gv + (size_t)m * n * cv + j0;
      const float* wp = wvt + (size_t)m * c * cv + j0;
#pragma unroll
      for (int i = 0; i < kPjPer; ++i) {
        R.a[i] = a_row[i] < n ? *reinterpret_cast<const floatx4*>(vp + v_off[i]) : floatx4{0.f, 0.f, 0.f, 0.f};
        R.g[i] = floatx4{1.f, 1.f, 1.f, 1.f};
        R.b[i] = *reinterpret_cast<const floatx4*>(wp + bv_off[i]);
      }
    }
  };
  auto store = [&](int it, const Regs& R) {
    float* As = lds + (it & 1) * kPjStage;
    float* Bs = As + kPjRows * kPjK;
#pragma unroll
    for (int i = 0; i < kPjPer; ++i) {
      const int r = t / kPjG + (kPjT / kPjG) * i;
      *reinterpret_cast<floatx4*>(As + pj_slot(r, g)) = R.a[i] * R.g[i];
      *reinterpret_cast<floatx4*>(Bs + pj_slot(r, g)) = R.b[i];
    }
  };

  floatx16 acc[2];
  pj_zero(acc);
  // stages: LDS buffer it & 1; the next stage's global loads are in flight during the MFMAs
  Regs R;
  load(0, R);
  store(0, R);
  __syncthreads();
  for (int it = 0; it < n_it; ++it) {
    if (it + 1 < n_it) load(it + 1, R);
    const float* As = lds + (it & 1) * kPjStage;
    pj_mma(As, As + kPjRows * kPjK, acc, wr, wc, lane);
    if (it + 1 < n_it) store(it + 1, R);
    __syncthreads();
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = row0 + wr * 32 + pj_acc_row(r, lane);
    if (row < n) {
      float* gr = gx + ((size_t)m * n + row) * c + col0 + wc * 64 + (lane & 31);
      gr[0] = acc[0][r];
      gr[32] = acc[1][r];
    }
  }
}

// ---------------------------------------------------------------------------
// bf16 operands (bf16 compute mode): the same tiling on v_mfma_f32_32x32x16_bf16.
// A stage holds 64 k, again 128-byte rows of eight 16-byte granules (8 bf16 each,
// same XOR swizzle); an MFMA step takes 16 k, granule 2 s + lane / 32 of both
// operands.  Activations are read in fp32 and rounded to bf16 as they are staged
// (no separate cast pass); the forward keeps y in bf16 for the backward, hq / hk
// are formed from the fp32 accumulators.  The backward uses the eight-wave 32 x 64
// layout of the fp32 kernels; the forward keeps four waves of 64 x 64 (256 threads,
// two workgroups per CU): on eight waves its staging registers and per-pair sums no
// longer fit in 128 VGPRs and it spills.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
constexpr int kPbK = 64;   // bf16 K per LDS stage

__device__ __forceinline__ int pb_slot(int r, int g) { return r * 8 + (g ^ (r & 7)); }  // in granules

__device__ __forceinline__ bf16x8 pb_round(floatx4 a, floatx4 b) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[i] = (__bf16)a[i];
    r[4 + i] = (__bf16)b[i];
  }
  return r;
}

// 64x64 wave tile (forward, four waves of 256 threads)
__device__ __forceinline__ void pb_mma64(const bf16x8* __restrict__ As, const bf16x8* __restrict__ Bs,
                                       floatx16 (&acc)[2][2], int wr, int wc, int lane) {
  const int r0 = wr * 64 + (lane & 31), c0 = wc * 64 + (lane & 31), h = lane >> 5;
#pragma unroll
  for (int ks = 0; ks < kPbK / 16; ++ks) {
    bf16x8 a[2], b[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      a[i] = As[pb_slot(r0 + 32 * i, 2 * ks + h)];
      b[i] = Bs[pb_slot(c0 + 32 * i, 2 * ks + h)];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
  }
}

// 32x64 wave tile (backward, eight waves of 512 threads)
__device__ __forceinline__ void pb_mma(const bf16x8* __restrict__ As, const bf16x8* __restrict__ Bs,
                                       floatx16 (&acc)[2], int wr, int wc, int lane) {
  const int r0 = wr * 32 + (lane & 31), c0 = wc * 64 + (lane & 31), h = lane >> 5;
#pragma unroll
  for (int ks = 0; ks < kPbK / 16; ++ks) {
    const bf16x8 a = As[pb_slot(r0, 2 * ks + h)];
    bf16x8 b[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) b[j] = Bs[pb_slot(c0 + 32 * j, 2 * ks + h)];
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b[j], acc[j], 0, 0, 0);
  }
}

__global__ __launch_bounds__(256, 2) void k_qk_proj_fwd_bf16(const float* __restrict__ x,
                                                             const __bf16* __restrict__ w,
                                                             const float* __restrict__ bias,
                                                             __bf16* __restrict__ y, float* __restrict__ hq,
                                                             float* __restrict__ hk, int n, int hid, int c) {
  __shared__ __attribute__((aligned(16))) bf16x8 lds[2 * (kPjRows + kPjCols) * 8];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6, wr = wv >> 1, wc = wv & 1;
  const int n_cb = (2 * hid) / 64, n_rb = (n + kPjRows - 1) / kPjRows, n_tiles = n_rb * n_cb;
  const int grp = blockIdx.x / xcd_grid(n_tiles), L = 2 - grp;
  const int tile = xcd_row(blockIdx.x - grp * xcd_grid(n_tiles), n_tiles);
  if (tile >= n_tiles) return;
  const int row0 = (tile / n_cb) * kPjRows, p0 = (tile % n_cb) * 64;
  const int O = 4 * hid, nk = c / kPbK, m0 = L * L, n_it = (2 * L + 1) * nk;

  const int g = t & 7;   // granule of rows / columns (t >> 3) + 32 i
  int a_row[4];
  uint32_t a_off[4], b_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a_row[i] = row0 + (t >> 3) + 32 * i;
    const int cl = (t >> 3) + 32 * i;
    a_off[i] = (uint32_t)a_row[i] * c + 8 * g;
    b_off[i] = (uint32_t)pj_pair_col(p0 + 32 * (cl >> 6) + (cl & 31), (cl >> 5) & 1, hid) * c + 8 * g;
  }
  struct Regs { floatx4 a[4][2]; bf16x8 b[4]; };
  const __bf16* wl = w + (size_t)L * O * c;
  auto load = [&](int it, Regs& R) {
    const int m = m0 + it / nk, k0 = (it % nk) * kPbK;
    const float* xm = x + (size_t)m * n * c + k0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool ok = a_row[i] < n;
      R.a[i][0] = ok ? *reinterpret_cast<const floatx4*>(xm + a_off[i]) : floatx4{0.f, 0.f, 0.f, 0.f};
      R.a[i][1] = ok ? *reinterpret_cast<const floatx4*>(xm + a_off[i] + 4) : floatx4{0.f, 0.f, 0.f, 0.f};
      R.b[i] = *reinterpret_cast<const bf16x8*>(wl + k0 + b_off[i]);
    }
  };
  auto store = [&](int it, const Regs& R) {
    bf16x8* As = lds + (it & 1) * (kPjRows + kPjCols) * 8;
    bf16x8* Bs = As + kPjRows * 8;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = (t >> 3) + 32 * i;
      As[pb_slot(r, g)] = pb_round(R.a[i][0], R.a[i][1]);
      Bs[pb_slot(r, g)] = R.b[i];
    }
  };

  const int p = p0 + 32 * wc + (lane & 31);
  const int oa = pj_pair_col(p, 0, hid), ob = pj_pair_col(p, 1, hid);
  const int erow = row0 + wr * 64 + 4 * (lane >> 5);
  const uint32_t y_off = (uint32_t)erow * O + oa, h_off = (uint32_t)erow * 3 * hid + (p < hid ? p : p - hid);
  float* hbase = p < hid ? hq : hk;
  const float ba = bias ? bias[oa] : 0.f, bb = bias ? bias[ob] : 0.f;

  floatx16 acc[2][2];
  pj_zero(acc);
  float s[2][16];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) s[i][r] = 0.f;
  Regs R;
  load(0, R);
  store(0, R);
  __syncthreads();
  for (int it = 0; it < n_it; ++it) {
    if (it + 1 < n_it) load(it + 1, R);
    const bf16x8* As = lds + (it & 1) * (kPjRows + kPjCols) * 8;
    pb_mma64(As, As + kPjRows * 8, acc, wr, wc, lane);
    if (it % nk == nk - 1) {
      const int m = m0 + it / nk;
      const float a0 = m == 0 ? ba : 0.f, b0 = m == 0 ? bb : 0.f;
      __bf16* ym = y + (size_t)m * n * O;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dr = 32 * i + pj_acc_row(r, 0);
          const float va = acc[i][0][r] + a0, vb = acc[i][1][r] + b0;
          s[i][r] = fmaf(va, vb, s[i][r]);
          if (erow + dr < n) {
            __bf16* yr = ym + (size_t)dr * O;
            yr[y_off] = (__bf16)va;
            yr[y_off + (ob - oa)] = (__bf16)vb;
          }
        }
      pj_zero(acc);
      if (it == n_it - 1) {
        float* hl = hbase + L * hid;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int dr = 32 * i + pj_acc_row(r, 0);
            if (erow + dr < n) hl[(size_t)dr * 3 * hid + h_off] = s[i][r];
          }
      }
    }
    if (it + 1 < n_it) store(it + 1, R);
    __syncthreads();
  }
}

// Backward with bf16 operands: gy formed in fp32 from the bf16 y and ghq / ghk and
// rounded as it is staged; wt / wvt are per degree l: [3][C][4 hid] and [3][C][cv].
__global__ __launch_bounds__(kPjT) __attribute__((amdgpu_waves_per_eu(4))) void k_qk_proj_bwd_bf16(const __bf16* __restrict__ y,
                                                             const float* __restrict__ ghq,
                                                             const float* __restrict__ ghk,
                                                             const __bf16* __restrict__ wt,
                                                             const float* __restrict__ gv,
                                                             const __bf16* __restrict__ wvt, float* __restrict__ gx,
                                                             int n, int hid, int c, int cv) {
  __shared__ __attribute__((aligned(16))) bf16x8 lds[2 * (kPjRows + kPjCols) * 8];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6, wr = wv >> 1, wc = wv & 1;
  const int n_cb = c / kPjCols, n_rb = (n + kPjRows - 1) / kPjRows;
  const int n_tiles = 9 * n_rb * n_cb;
  const int tile = xcd_row(blockIdx.x, n_tiles);
  if (tile >= n_tiles) return;
  const int m = tile / (n_rb * n_cb), rem = tile % (n_rb * n_cb);
  const int row0 = (rem / n_cb) * kPjRows, col0 = (rem % n_cb) * kPjCols, l = pj_l(m);
  const int O = 4 * hid, nkq = O / kPbK, n_it = nkq + (gv ? cv / kPbK : 0);

  const int g = t & 7;
  const int r_base = row0 + (t >> 3);                  // staged rows r_base + 64 i, i < 2
  const uint32_t c_base = (uint32_t)(col0 + (t >> 3));  // staged columns c_base + 64 i
  const __bf16* ym = y + (size_t)m * n * O;
  const __bf16* wt_l = wt + (size_t)l * c * O;
  // a: the fp32 factor (g or gv); yb: 8 bf16 of y as four 32-bit words
  struct Regs { floatx4 a[2][2]; uint4 yb[2]; bf16x8 b[2]; };
  auto load = [&](int it, Regs& R) {
    if (it < nkq) {
      const int j0 = it * kPbK, q = j0 / hid;
      const __bf16* yp = ym + (q & 1 ? j0 - hid : j0 + hid) + 8 * g;
      const float* gs = (q < 2 ? ghq : ghk) + l * hid + (j0 - q * hid) + 8 * g;
      const __bf16* wp = wt_l + j0 + 8 * g;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int row = r_base + 64 * i;
        const bool ok = row < n;
        // rows past n read row n - 1 of y (their gradient factor is 0)
        R.yb[i] = *reinterpret_cast<const uint4*>(yp + (uint32_t)min(row, n - 1) * O);
        const float* gr = gs + (uint32_t)row * 3 * hid;
        R.a[i][0] = ok ? *reinterpret_cast<const floatx4*>(gr) : floatx4{0.f, 0.f, 0.f, 0.f};
        R.a[i][1] = ok ? *reinterpret_cast<const floatx4*>(gr + 4) : floatx4{0.f, 0.f, 0.f, 0.f};
        R.b[i] = *reinterpret_cast<const bf16x8*>(wp + (c_base + 64 * i) * O);
      }
    } else {
      const int j0 = (it - nkq) * kPbK;
      const float* vp = gv + (size_t)m * n * cv + j0 + 8 * g;
      const __bf16* wp = wvt + (size_t)l * c * cv + j0 + 8 * g;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int row = r_base + 64 * i;
        const bool ok = row < n;
        const float* vr = vp + (uint32_t)row * cv;
        R.a[i][0] = ok ? *reinterpret_cast<const floatx4*>(vr) : floatx4{0.f, 0.f, 0.f, 0.f};
        R.a[i][1] = ok ? *reinterpret_cast<const floatx4*>(vr + 4) : floatx4{0.f, 0.f, 0.f, 0.f};
        R.b[i] = *reinterpret_cast<const bf16x8*>(wp + (c_base + 64 * i) * cv);
      }
    }
  };
  auto store = [&](int it, const Regs& R) {
    bf16x8* As = lds + (it & 1) * (kPjRows + kPjCols) * 8;
    bf16x8* Bs = As + kPjRows * 8;
    const bool gy_stage = it < nkq;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = (t >> 3) + 64 * i;
      floatx4 lo = R.a[i][0], hi = R.a[i][1];
      if (gy_stage) {   // bf16 -> fp32: the 16 bits are the fp32's upper half
        const uint4 w = R.yb[i];
        lo *= floatx4{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                      __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u)};
        hi *= floatx4{__uint_as_float(w.z << 16), __uint_as_float(w.z & 0xffff0000u),
                      __uint_as_float(w.w << 16), __uint_as_float(w.w & 0xffff0000u)};
      }
      As[pb_slot(r, g)] = pb_round(lo, hi);
      Bs[pb_slot(r, g)] = R.b[i];
    }
  };

  floatx16 acc[2];
  pj_zero(acc);
  Regs R;
  load(0, R);
  store(0, R);
  __syncthreads();
  for (int it = 0; it < n_it; ++it) {
    if (it + 1 < n_it) load(it + 1, R);
    const bf16x8* As = lds + (it & 1) * (kPjRows + kPjCols) * 8;
    pb_mma(As, As + kPjRows * 8, acc, wr, wc, lane);
    if (it + 1 < n_it) store(it + 1, R);
    __syncthreads();
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = row0 + wr * 32 + pj_acc_row(r, lane);
    if (row < n) {
      float* gr = gx + ((size_t)m * n + row) * c + col0 + wc * 64 + (lane & 31);
      gr[0] = acc[0][r];
      gr[32] = acc[1][r];
    }
  }
}

// Staging and epilogue offsets are 32-bit element offsets from per-m bases.
__host__ inline bool pj_offsets_fit(int n, int width) {
  return (uint64_t)(n + kPjRows) * (uint64_t)width < (1ull << 32);
}
}  // namespace e2v2

E2V2_API int e2v2_qk_proj_fwd(const float* x, const float* w, const float* bias, float* y, float* hq, float* hk,
                              int n, int hid, int c, hipStream_t s) {
  using namespace e2v2;
  E2V2_REQUIRE(hid > 0 && hid % 64 == 0, "qk_proj_fwd: hid=%d must be a positive multiple of 64", hid);
  E2V2_REQUIRE(c > 0 && c % kPjK == 0, "qk_proj_fwd: C=%d must be a positive multiple of %d", c, kPjK);
  E2V2_REQUIRE(n >= 0 && pj_offsets_fit(n, 4 * hid) && pj_offsets_fit(n, c), "qk_proj_fwd: n=%d too large", n);
  if (n == 0) return 0;
  const int tiles = ((n + kPjRows - 1) / kPjRows) * (2 * hid / 64);
  hipLaunchKernelGGL(k_qk_proj_fwd, dim3(3 * xcd_grid(tiles)), dim3(kPjT), 0, s, x, w, bias, y, hq, hk, n, hid, c);
  E2V2_LAUNCHED("k_qk_proj_fwd");
  return 0;
}

E2V2_API int e2v2_qk_proj_bwd(const float* y, const float* ghq, const float* ghk, const float* wt, const float* gv,
                              const float* wvt, float* gx, int n, int hid, int c, int cv, hipStream_t s) {
  using namespace e2v2;
  E2V2_REQUIRE(hid > 0 && hid % kPjK == 0, "qk_proj_bwd: hid=%d must be a positive multiple of %d", hid, kPjK);
  E2V2_REQUIRE(c > 0 && c % kPjCols == 0, "qk_proj_bwd: C=%d must be a positive multiple of %d", c, kPjCols);
  E2V2_REQUIRE(!gv || (wvt && cv > 0 && cv % kPjK == 0), "qk_proj_bwd: value gradient needs Wv^T and Cv %% %d == 0",
               kPjK);
  E2V2_REQUIRE(n >= 0 && pj_offsets_fit(n, 4 * hid) && pj_offsets_fit(n, c) && pj_offsets_fit(n, cv),
               "qk_proj_bwd: n=%d too large", n);
  if (n == 0) return 0;
  const int tiles = 9 * ((n + kPjRows - 1) / kPjRows) * (c / kPjCols);
  hipLaunchKernelGGL(k_qk_proj_bwd, dim3(xcd_grid(tiles)), dim3(kPjT), 0, s, y, ghq, ghk, wt, gv, wvt, gx, n, hid, c,
                     cv);
  E2V2_LAUNCHED("k_qk_proj_bwd");
  return 0;
}

E2V2_API int e2v2_qk_proj_fwd_bf16(const float* x, const void* w, const float* bias, void* y, float* hq, float* hk,
                                   int n, int hid, int c, hipStream_t s) {
  using namespace e2v2;
  E2V2_REQUIRE(hid > 0 && hid % 64 == 0, "qk_proj_fwd_bf16: hid=%d must be a positive multiple of 64", hid);
  E2V2_REQUIRE(c > 0 && c % kPbK == 0, "qk_proj_fwd_bf16: C=%d must be a positive multiple of %d", c, kPbK);
  E2V2_REQUIRE(n >= 0 && pj_offsets_fit(n, 4 * hid) && pj_offsets_fit(n, c), "qk_proj_fwd_bf16: n=%d too large", n);
  if (n == 0) return 0;
  const int tiles = ((n + kPjRows - 1) / kPjRows) * (2 * hid / 64);
  hipLaunchKernelGGL(k_qk_proj_fwd_bf16, dim3(3 * xcd_grid(tiles)), dim3(256), 0, s, x,
                     static_cast<const __bf16*>(w), bias, static_cast<__bf16*>(y), hq, hk, n, hid, c);
  E2V2_LAUNCHED("k_qk_proj_fwd_bf16");
  return 0;
}

E2V2_API int e2v2_qk_proj_bwd_bf16(const void* y, const float* ghq, const float* ghk, const void* wt, const float* gv,
                                   const void* wvt, float* gx, int n, int hid, int c, int cv, hipStream_t s) {
  using namespace e2v2;
  E2V2_REQUIRE(hid > 0 && hid % kPbK == 0, "qk_proj_bwd_bf16: hid=%d must be a positive multiple of %d", hid, kPbK);
  E2V2_REQUIRE(c > 0 && c % kPjCols == 0, "qk_proj_bwd_bf16: C=%d must be a positive multiple of %d", c, kPjCols);
  E2V2_REQUIRE(!gv || (wvt && cv > 0 && cv % kPbK == 0),
               "qk_proj_bwd_bf16: value gradient needs Wv^T and Cv %% %d == 0", kPbK);
  E2V2_REQUIRE(n >= 0 && pj_offsets_fit(n, 4 * hid) && pj_offsets_fit(n, c) && pj_offsets_fit(n, cv),
               "qk_proj_bwd_bf16: n=%d too large", n);
  if (n == 0) return 0;
  const int tiles = 9 * ((n + kPjRows - 1) / kPjRows) * (c / kPjCols);
  hipLaunchKernelGGL(k_qk_proj_bwd_bf16, dim3(xcd_grid(tiles)), dim3(kPjT), 0, s, static_cast<const __bf16*>(y), ghq,
                     ghk, static_cast<const __bf16*>(wt), gv, static_cast<const __bf16*>(wvt), gx, n, hid, c, cv);
  E2V2_LAUNCHED("k_qk_proj_bwd_bf16");
  return 0;
}
