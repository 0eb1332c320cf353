// fp32 GEMMs of the per-node dense layers on bf16 MFMA (v_mfma_f32_32x32x16_bf16)
// by an exact three-piece split of both operands:
//   x = x0 + x1 + x2 + r,  x0 = bf16(x), x1 = bf16(x - x0), x2 = bf16(x - x0 - x1)
// (round to nearest even at each step; every subtraction is exact in fp32, and
// |x1| <= 2^-8 |x|, |x2| <= 2^-16 |x|, |r| <= 2^-24 |x|).  A product a b is
// formed from the six piece products of order <= 2,
//   a0 b0 + (a0 b1 + a1 b0) + (a0 b2 + a1 b1 + a2 b0),
// each exact in fp32 (8-bit x 8-bit significands) and accumulated in fp32 by the
// MFMA (one rounding per instruction of 16 products: 6 per 16 k, against 8 for an
// fp32 GEMM on v_mfma_f32_32x32x2_f32).  The neglected terms (a1 b2, a2 b1, a2 b2
// and the split remainders) are at most about 3 * 2^-24 |a b| per product.
// Measured against float64, the error is below that of the fp32 MFMA GEMM of the
// same operands; the bf16 MFMA rate is 16x the fp32 one on gfx950, so the six
// products cost 3/8 of the fp32 MFMA time.
//
// Layers (paths relative to the reference repository): SO3_Linear_e2former
// (src/molfm/models/e2former/module_utils.py:2010-2052) and hence
// FeedForwardNetwork_s3 (module_utils.py:2755-2797), the value projection
// (e2former.py:300-303) and proj_first (e2former.py:215-219, 433); forward_linear
// of SO2_TP_givenl2 (wigner6j/so2_tensor_product.py:276-290); the final_linear
// of SO3_Linear2Scalar_e2former (module_utils.py:2230-2233); the gate logits of
// Gate_s3 (module_utils.py:2694-2746); and the input gradients of each.
//
// C[b][m][n] = sum_k A[b][m][k] W_{widx[b]}[n][k] (+ bias[n] for b < bias_batches)
// (+ R[b][m][n]).  A is fp32 row-major (k contiguous).  The weights are packed once
// per weight version by e2v2_gemm_pack: split into the three bf16 pieces and laid
// out per (weight, 128-column tile, 16-k stage) as the 12 KB LDS image of that
// stage (three pieces of 256 16-byte granules in the swizzled slot order below),
// so that a stage is copied to LDS by contiguous 16-byte direct loads.
//
// Tiling: 128 x 128 per workgroup of four wavefronts (each 32 rows x 128 columns:
// four 32x32 MFMA tiles, one fp32 accumulator each), K in stages of 16 through
// two LDS buffers (20 KB each: A as fp32, 8 KB; the three B pieces, 12 KB), three
// workgroups per CU (135 VGPRs).  Both operands reach LDS by buffer loads with the
// LDS destination (no staging registers; rows past m read as zero through the
// buffer's bound).  A wavefront splits its A fragment of the next stage while the
// 24 MFMAs of the current one run (B by piece: b0 with a0, a1, a2; b1 with a0,
// a1; b2 with a0).  Outputs are written with ordinary stores, so that they stay
// in the L2 / Infinity Cache for the kernel that consumes them.
// In LDS (64 banks of 4 bytes: a 16-byte granule's bank group is its index mod 16)
// an A row keeps its 16 k as four granules, granule g of row r in slot
// g ^ ((r / 4) & 3); a B piece keeps a column's 16 k as two granules, granule g of
// column c in slot g ^ ((c / 8) & 1): the rows (columns) that 8 or 16 consecutive
// lanes read land in distinct bank groups.
#include "gemm_core.h"

namespace e2v2 {
namespace {

__device__ __forceinline__ int gemm_tiles(const e2v2_gemm_args& G) {
  return G.batch * ((G.m + kGM - 1) / kGM) * (G.n / kGN);
}

// Gate_s3 (module_utils.py:2694-2746) applied to the A operand as it is read:
// batch 0 reads silu(s[i][kk]) k1 from the gate logits themselves, batch b >= 1
// reads a[b][i][kk] sigmoid(s[i][k widx[b] + kk]) k2 (the same products, rounded
// the same way, as the gate kernel's output).
struct GateOp {
  const float* s;
  int64_t ld;
  float k1, k2;
};

// Epilogue of a tile: C = acc (+ bias) (+ R), fp32 or bf16 (rounded once).
__device__ __forceinline__ void gemm_store(const e2v2_gemm_args& G, int bi, int nt, int row0, int wv, int lane,
                                           const floatx16 (&acc)[4]) {
  const bool with_bias = G.bias && bi < G.bias_batches;
  float* cb = static_cast<float*>(G.c) + (G.c_bf16 ? 0 : (int64_t)bi * G.c_bs);
  __bf16* cbh = static_cast<__bf16*>(G.c) + (G.c_bf16 ? (int64_t)bi * G.c_bs : 0);
  const float* rb = G.r ? G.r + (int64_t)bi * G.r_bs : nullptr;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int col = nt * kGN + 32 * j + (lane & 31);
    const float bv = with_bias ? G.bias[(int64_t)bi * G.bias_bs + col] : 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = row0 + wv * 32 + acc_row(r, lane);
      if (row < G.m) {
        float v = acc[j][r];
        if (with_bias) v += bv;
        if (rb) v += rb[(size_t)row * G.ldr + col];
        if (G.c_bf16)
          cbh[(size_t)row * G.ldc + col] = (__bf16)v;
        else
          cb[(size_t)row * G.ldc + col] = v;
      }
    }
  }
}

// One 128 x 128 output tile (batch-major, then row tile, then column tile).  kP operand pieces; kAB: A is
// bf16 in memory (G.a_bf16); C is written as bf16 when G.c_bf16 (rounded once, from the fp32 sum).
template <int kP, bool kAB, bool kGate>
__device__ __forceinline__ void gemm_tile(const e2v2_gemm_args& G, int tile, char* lds, const GateOp& gt) {
  static_assert(!(kAB && kGate), "the gated operand is fp32");
  constexpr int SB = g_stage_bytes(kP, kAB);
  const int t = threadIdx.x, lane = t & 63, wv = __builtin_amdgcn_readfirstlane(t >> 6), h = lane >> 5;
  const int n_mt = (G.m + kGM - 1) / kGM, n_nt = G.n / kGN;
  const int nt = tile % n_nt, mt = (tile / n_nt) % n_mt, bi = tile / (n_nt * n_mt);
  const int row0 = mt * kGM, nks = G.k / kGK;
  const bool g0 = kGate && bi == 0;                      // batch 0 of a gated call: silu of the logits
  const int lda = g0 ? (int)gt.ld : (int)G.lda;
  __amdgpu_buffer_rsrc_t ar;
  uint32_t a_voff[kGAi / 4];
  if constexpr (kAB) {
    ar = rows_rsrc_bf(static_cast<const __bf16*>(G.a) + (int64_t)bi * G.a_bs, row0, G.m, lda);
    a_voff[0] = abf_offset(wv, lane, lda);
  } else {
    ar = rows_rsrc(g0 ? gt.s : static_cast<const float*>(G.a) + (int64_t)bi * G.a_bs, row0, G.m, lda);
    a_offsets(wv, lane, lda, a_voff);
  }
  const __amdgpu_buffer_rsrc_t br = b_rsrc<kP>(G.b, G.widx[bi], n_nt, nt, nks);
  const int ra = wv * 32 + (lane & 31);
  // gate logits of this lane's A values (row ra, k 8 h .. +7 of each stage), one stage ahead
  // (32-bit byte offsets from the uniform base: (m + 128) ld_s 4 < 2^31 is checked by the host)
  const char* sb = reinterpret_cast<const char*>(gt.s);
  const bool mok = kGate && !g0 && row0 + ra < G.m;
  const uint32_t moff = mok ? (uint32_t)(((uint32_t)(row0 + ra) * (uint32_t)gt.ld + (uint32_t)(G.k * G.widx[bi]) +
                                          8u * h) * 4u)
                            : 0u;
  floatx4 mv0 = {0.f, 0.f, 0.f, 0.f}, mv1 = {0.f, 0.f, 0.f, 0.f};
  if (mok) {
    mv0 = *reinterpret_cast<const floatx4*>(sb + moff);
    mv1 = *reinterpret_cast<const floatx4*>(sb + moff + 16u);
  }
  floatx16 acc[4];
  kloop<kP, kAB>(lds, SB, nks, lane,
        [&](int ks, int buf) {
          if constexpr (kAB) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ar, (lds_void*)(lds + buf * SB + wv * 1024), 16,
                                                     a_voff[0] + (uint32_t)(ks * kGK) * 2u, 0, 0, 0);
          } else {
            load_a(ar, a_voff, (uint32_t)(ks * kGK) * 4u, lds + buf * SB, wv);
          }
          load_b<kP>(br, ks, lds + buf * SB + a_stage_bytes(kAB), wv, lane);
        },
        [&](int ks, int buf, AFrag& f) {
          if constexpr (kAB) {
            f.b = reinterpret_cast<const bf16x8*>(lds + buf * SB)[abf_slot(ra, h)];
            return;
          } else {
            const floatx4* As = reinterpret_cast<const floatx4*>(lds + buf * SB);
            f.x0 = As[a_slot(ra, 2 * h)];
            f.x1 = As[a_slot(ra, 2 * h + 1)];
            if constexpr (kGate) {
              if (g0) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  f.x0[e] = silu(f.x0[e]) * gt.k1;
                  f.x1[e] = silu(f.x1[e]) * gt.k1;
                }
              } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  f.x0[e] = sigmoidf_(mv0[e]) * gt.k2 * f.x0[e];
                  f.x1[e] = sigmoidf_(mv1[e]) * gt.k2 * f.x1[e];
                }
                if (mok && ks + 1 < nks) {
                  const uint32_t o = moff + (uint32_t)(ks + 1) * (kGK * 4u);
                  mv0 = *reinterpret_cast<const floatx4*>(sb + o);
                  mv1 = *reinterpret_cast<const floatx4*>(sb + o + 16u);
                }
              }
            }
          }
        },
        acc);

  gemm_store(G, bi, nt, row0, wv, lane, acc);
}

// One tile of an fp32-A GEMM on kloop_r (A into registers two stages ahead, B through three LDS buffers of
// 12 KB (kP = 3): 36 KB and at most 128 VGPRs, four workgroups per CU).
template <int kP>
__device__ __forceinline__ void gemm_tile_r(const e2v2_gemm_args& G, int tile) {
  constexpr int BB = b_stage_bytes(kP);
  __shared__ __attribute__((aligned(16))) char B0[BB];
  __shared__ __attribute__((aligned(16))) char B1[BB];
  __shared__ __attribute__((aligned(16))) char B2[BB];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n_mt = (G.m + kGM - 1) / kGM, n_nt = G.n / kGN;
  const int nt = tile % n_nt, mt = (tile / n_nt) % n_mt, bi = tile / (n_nt * n_mt);
  const int row0 = mt * kGM, nks = G.k / kGK;
  const __amdgpu_buffer_rsrc_t ar =
      rows_rsrc(static_cast<const float*>(G.a) + (int64_t)bi * G.a_bs, row0, G.m, (int)G.lda);
  const __amdgpu_buffer_rsrc_t br = b_rsrc<kP>(G.b, G.widx[bi], n_nt, nt, nks);
  const uint32_t aoff = (uint32_t)((wv * 32 + (lane & 31)) * (int)G.lda + 8 * (lane >> 5)) * 4u;
  floatx16 acc[4];
  kloop_r<kP>(B0, B1, B2, nks, lane,
              [&](int ks, char* Bs) { load_b<kP>(br, ks, Bs, wv, lane); },
              [&](int ks, floatx4 (&x)[2]) { load_a_regs(ar, aoff, ks, x); }, acc);
  gemm_store(G, bi, nt, row0, wv, lane, acc);
}

// fp32 A, three pieces
__global__ __launch_bounds__(kGT, 4) void k_gemm_s3(e2v2_gemm_args G) {
  const int n_tiles = gemm_tiles(G);
  const int tile = xcd_row(blockIdx.x, n_tiles);
  if (tile >= n_tiles) return;
  gemm_tile_r<3>(G, tile);
}
// one piece (the bf16 mode), A fp32 or bf16 (kAB), on kloop: with one MFMA product per stage these GEMMs are
// bound by their operand and output traffic, and the two-buffer loop at up to five workgroups per CU was
// measured faster for an fp32 A than kloop_r (55.8 against 64.1 us per call at cfg 4)
template <bool kAB>
__global__ __launch_bounds__(kGT, 3) void k_gemm_s3_p1(e2v2_gemm_args G) {
  __shared__ __attribute__((aligned(16))) char lds[2 * g_stage_bytes(1, kAB)];
  const int n_tiles = gemm_tiles(G);
  const int tile = xcd_row(blockIdx.x, n_tiles);
  if (tile >= n_tiles) return;
  gemm_tile<1, kAB, false>(G, tile, lds, GateOp{});
}

template <int kP>
__global__ __launch_bounds__(kGT, 3) void k_gemm_s3_gate(e2v2_gemm_args G, GateOp gt) {
  __shared__ __attribute__((aligned(16))) char lds[2 * g_stage_bytes(kP, false)];
  const int n_tiles = gemm_tiles(G);
  const int tile = xcd_row(blockIdx.x, n_tiles);
  if (tile >= n_tiles) return;
  gemm_tile<kP, false, true>(G, tile, lds, gt);
}

// Independent GEMMs in one launch: group g owns workgroups block0[g] ..
// block0[g + 1] - 1 (xcd_grid of its tile count, in the order given, so the
// caller puts the longest tiles first), its tiles spread over the XCDs as in a
// launch of its own.  The group is selected with constant indices so that its
// arguments stay in the kernel-argument segment.  The groups share the operand
// pieces and A's storage type (the output's may differ).
constexpr int kGGroups = 4;
struct GemmGroups {
  e2v2_gemm_args g[kGGroups];
  int block0[kGGroups + 1];
  int n;
};

__global__ __launch_bounds__(kGT, 4) void k_gemm_s3_grp(GemmGroups P) {
  const int b = blockIdx.x;
#pragma unroll
  for (int gi = 0; gi < kGGroups; ++gi) {
    if (gi < P.n && b >= P.block0[gi] && b < P.block0[gi + 1]) {
      const int n_tiles = gemm_tiles(P.g[gi]);
      const int tile = xcd_row(b - P.block0[gi], n_tiles);
      if (tile < n_tiles) gemm_tile_r<3>(P.g[gi], tile);
      return;
    }
  }
}
template <bool kAB>
__global__ __launch_bounds__(kGT, 3) void k_gemm_s3_grp_p1(GemmGroups P) {
  __shared__ __attribute__((aligned(16))) char lds[2 * g_stage_bytes(1, kAB)];
  const int b = blockIdx.x;
#pragma unroll
  for (int gi = 0; gi < kGGroups; ++gi) {
    if (gi < P.n && b >= P.block0[gi] && b < P.block0[gi + 1]) {
      const int n_tiles = gemm_tiles(P.g[gi]);
      const int tile = xcd_row(b - P.block0[gi], n_tiles);
      if (tile < n_tiles) gemm_tile<1, kAB, false>(P.g[gi], tile, lds, GateOp{});
      return;
    }
  }
}

// ---------------------------------------------------------------------------
// Q/K projection of SO3_Linear2Scalar_e2former (module_utils.py:2198-2266, query
// and key at e2former.py:300-303) with its m-contraction, on the split GEMM.
// Pairs p < 2 hid: the query pairs (q_a, q_b) = (weight, weight2) columns p, then
// the key pairs; hq[n][l hid + p] = sum_{m in l} y[m][n][a(p)] y[m][n][b(p)].
// Forward: the packed weight's 128-column tile t holds the a-columns of pairs
// 64 t .. +63 then their b-columns, so a wavefront's tiles j and j + 2 hold the
// a- and b-values of the same 32 pairs in the same accumulator layout; a
// workgroup runs the m-rows of its degree l in turn and adds a b to its pair
// sums.  y is kept for the backward in the paired order:
//   y[m][n][16 (p / 8) + 8 ab + p % 8]  (ab = 0: a-column, 1: b-column)
// so that within every 16-k stage of the backward the partner of column k is k ^ 8.
__device__ __forceinline__ int pair_pos(int p, int ab) { return 16 * (p >> 3) + 8 * ab + (p & 7); }

template <int kP, bool kYB>
__global__ __launch_bounds__(kGT, 2) void k_qk_s3_fwd(const float* __restrict__ x, const void* __restrict__ wp,
                                                      const float* __restrict__ bias, void* __restrict__ y,
                                                      float* __restrict__ hq, float* __restrict__ hk, int n,
                                                      int hid, int c) {
  constexpr int SB = g_stage_bytes(kP, false);
  __shared__ __attribute__((aligned(16))) char lds[2 * SB];
  const int t = threadIdx.x, lane = t & 63, wv = __builtin_amdgcn_readfirstlane(t >> 6), h = lane >> 5;
  const int n_mt = (n + kGM - 1) / kGM, n_pt = 2 * hid / 64, tiles = n_mt * n_pt;
  // three groups of xcd_grid(tiles) workgroups, l = 2, 1, 0 (5, 3, 1 m-rows): long tiles first
  const int grp = blockIdx.x / xcd_grid(tiles), L = 2 - grp;
  const int tile = xcd_row(blockIdx.x - grp * xcd_grid(tiles), tiles);
  if (tile >= tiles) return;
  const int mt = tile / n_pt, pt = tile % n_pt, row0 = mt * kGM, nks = c / kGK, O = 4 * hid;
  uint32_t a_voff[kGAi / 4];
  a_offsets(wv, lane, c, a_voff);
  const __amdgpu_buffer_rsrc_t br = b_rsrc<kP>(wp, L, n_pt, pt, nks);
  const int ra = wv * 32 + (lane & 31);
  float s[2][16];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) s[j][r] = 0.f;
  for (int m = L * L; m < (L + 1) * (L + 1); ++m) {
    if (m != L * L) __syncthreads();      // every wavefront is done with the previous row's LDS stages
    const __amdgpu_buffer_rsrc_t ar = rows_rsrc(x + (size_t)m * n * c, row0, n, c);
    floatx16 acc[4];
    kloop<kP, false>(lds, SB, nks, lane,
          [&](int ks, int buf) {
            load_a(ar, a_voff, (uint32_t)(ks * kGK) * 4u, lds + buf * SB, wv);
            load_b<kP>(br, ks, lds + buf * SB + kGAg * 16, wv, lane);
          },
          [&](int, int buf, AFrag& f) {
            const floatx4* As = reinterpret_cast<const floatx4*>(lds + buf * SB);
            f.x0 = As[a_slot(ra, 2 * h)];
            f.x1 = As[a_slot(ra, 2 * h + 1)];
          },
          acc);
    // y kept for the backward: fp32, or bf16 (kYB, the bf16 mode: rounded once; the contraction below uses
    // the fp32 sums)
    float* ym = static_cast<float*>(y) + (kYB ? 0 : (size_t)m * n * O);
    __bf16* ymb = static_cast<__bf16*>(y) + (kYB ? (size_t)m * n * O : 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int p = 64 * pt + 32 * (j & 1) + (lane & 31), ab = j >> 1;
      const float bv = m == 0 && bias ? bias[128 * pt + 32 * j + (lane & 31)] : 0.f;
      const int col = pair_pos(p, ab);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = row0 + wv * 32 + acc_row(r, lane);
        acc[j][r] += bv;
        if (row < n) {
          if constexpr (kYB)
            ymb[(size_t)row * O + col] = (__bf16)acc[j][r];
          else
            ym[(size_t)row * O + col] = acc[j][r];
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[j][r] = fmaf(acc[j][r], acc[j + 2][r], s[j][r]);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int p = 64 * pt + 32 * j + (lane & 31);
    float* out = p < hid ? hq + L * hid + p : hk + L * hid + (p - hid);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = row0 + wv * 32 + acc_row(r, lane);
      if (row < n) out[(size_t)row * 3 * hid] = s[j][r];
    }
  }
}

// Backward: gx[m][n][k] = sum_o gy[m][n][o] W_l[o][k] + sum_j gv[m][n][j] Wv_l[j][k]
// with gy at a- / b-column of pair p = g(n, l, p) times the partner's y
// (g = ghq or ghk at [n][l hid + p']), formed as the A operand is read: the stage
// holds y[m] of 8 pairs (a then b columns: the partner granules are those of the
// other half) and their 8 g values (a G tile of 128 rows x 8 fp32 after the B
// pieces, granule g of row r in slot g ^ ((r / 8) & 1)).  The packed weight is
// [W_l (rows in the paired order) ; Wv_l]^T per l: the value projection's input
// gradient enters as cv / 16 further stages with A = gv[m].
__host__ __device__ constexpr int qk_bwd_stage_bytes(int kP) { return g_stage_bytes(kP, false) + 128 * 8 * 4; }
__device__ __forceinline__ int g_slot(int r, int g) { return r * 2 + (g ^ ((r >> 3) & 1)); }

template <int kP, bool kYB>
__global__ __launch_bounds__(kGT, 2) void k_qk_s3_bwd(const void* __restrict__ y, const float* __restrict__ ghq,
                                                      const float* __restrict__ ghk, const void* __restrict__ wp,
                                                      const float* __restrict__ gv, float* __restrict__ gx, int n,
                                                      int hid, int c, int cv) {
  constexpr int SB = g_stage_bytes(kP, false), kGStageQ = qk_bwd_stage_bytes(kP);   // + the G tile: 4 KB
  __shared__ __attribute__((aligned(16))) char lds[2 * kGStageQ];
  const int t = threadIdx.x, lane = t & 63, wv = __builtin_amdgcn_readfirstlane(t >> 6), h = lane >> 5;
  const int n_mt = (n + kGM - 1) / kGM, n_ct = c / kGN, tiles = 9 * n_mt * n_ct;
  const int tile = xcd_row(blockIdx.x, tiles);
  if (tile >= tiles) return;
  const int ct = tile % n_ct, mt = (tile / n_ct) % n_mt, m = tile / (n_ct * n_mt);
  const int l = m == 0 ? 0 : (m < 4 ? 1 : 2);
  const int O = 4 * hid, row0 = mt * kGM, nk1 = O / kGK, nks = nk1 + (gv ? cv / kGK : 0);
  const int nks_w = nk1 + cv / kGK;                                // stages of the packed weight
  uint32_t y_voff[kGAi / 4], v_voff[kGAi / 4];
  a_offsets(wv, lane, O, y_voff);
  a_offsets(wv, lane, cv, v_voff);
  const uint32_t yb_voff = abf_offset(wv, lane, O);      // bf16 y: one granule (8 values) per lane and stage
  const __amdgpu_buffer_rsrc_t yr =
      kYB ? rows_rsrc_bf(static_cast<const __bf16*>(y) + (size_t)m * n * O, row0, n, O)
          : rows_rsrc(static_cast<const float*>(y) + (size_t)m * n * O, row0, n, O);
  const __amdgpu_buffer_rsrc_t vr = gv ? rows_rsrc(gv + (size_t)m * n * cv, row0, n, cv) : yr;
  const __amdgpu_buffer_rsrc_t qr = rows_rsrc(ghq, row0, n, 3 * hid), kr = rows_rsrc(ghk, row0, n, 3 * hid);
  constexpr int kBS = b_stage_granules(kP) * 16;
  const char* wbase = static_cast<const char*>(wp) + ((size_t)l * n_ct + ct) * (size_t)nks_w * kBS;
  const __amdgpu_buffer_rsrc_t br =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(wbase), (short)0, nks_w * kBS, 0x00020000);
  // G tile load: one instruction per wavefront, LDS granules 64 wv .. +63 = rows 32 wv + lane / 2, slot lane % 2
  const int g_r = 32 * wv + (lane >> 1);
  const uint32_t g_voff = (uint32_t)(g_r * 3 * hid + 4 * ((lane & 1) ^ ((g_r >> 3) & 1))) * 4u;
  const int ra = wv * 32 + (lane & 31);
  floatx16 acc[4];
  kloop<kP, false>(lds, kGStageQ, nks, lane,
        [&](int ks, int buf) {
          char* As = lds + buf * kGStageQ;
          if (ks < nk1) {
            if constexpr (kYB)
              __builtin_amdgcn_raw_ptr_buffer_load_lds(yr, (lds_void*)(As + wv * 1024), 16,
                                                       yb_voff + (uint32_t)(ks * kGK) * 2u, 0, 0, 0);
            else
              load_a(yr, y_voff, (uint32_t)(ks * kGK) * 4u, As, wv);
            const int p0 = 8 * ks;                                     // first pair of the stage
            const uint32_t goff = (uint32_t)(l * hid + (p0 < hid ? p0 : p0 - hid)) * 4u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(p0 < hid ? qr : kr, (lds_void*)(As + SB + wv * 1024), 16,
                                                     g_voff + goff, 0, 0, 0);
          } else {
            load_a(vr, v_voff, (uint32_t)((ks - nk1) * kGK) * 4u, As, wv);
          }
          load_b<kP>(br, ks, As + kGAg * 16, wv, lane);
        },
        [&](int ks, int buf, AFrag& f) {
          const floatx4* As = reinterpret_cast<const floatx4*>(lds + buf * kGStageQ);
          if (ks < nk1) {
            const floatx4* Gs = reinterpret_cast<const floatx4*>(lds + buf * kGStageQ + SB);
            if constexpr (kYB) {
              // the partner's eight bf16 values (the other half of the stage: granule 1 - h), widened exactly
              const bf16x8 yb = reinterpret_cast<const bf16x8*>(lds + buf * kGStageQ)[abf_slot(ra, 1 - h)];
              const floatx4 g0 = Gs[g_slot(ra, 0)], g1 = Gs[g_slot(ra, 1)];
#pragma unroll
              for (int u = 0; u < 4; ++u) {
                f.x0[u] = (float)yb[u] * g0[u];
                f.x1[u] = (float)yb[4 + u] * g1[u];
              }
            } else {
              f.x0 = As[a_slot(ra, 2 - 2 * h)] * Gs[g_slot(ra, 0)];
              f.x1 = As[a_slot(ra, 3 - 2 * h)] * Gs[g_slot(ra, 1)];
            }
          } else {
            f.x0 = As[a_slot(ra, 2 * h)];
            f.x1 = As[a_slot(ra, 2 * h + 1)];
          }
        },
        acc);
  float* gm = gx + (size_t)m * n * c;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int col = ct * kGN + 32 * j + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = row0 + wv * 32 + acc_row(r, lane);
      if (row < n) gm[(size_t)row * c + col] = acc[j][r];
    }
  }
}

// Pack: one thread per (weight, column tile, stage, LDS granule): the granule's
// eight k of its column, split into the three pieces (or rounded to the first alone).
__global__ __launch_bounds__(256) void k_gemm_pack(const float* __restrict__ w, int64_t ld_n, int64_t ld_k,
                                                   int64_t w_stride, int n_w, int n, int k, int pieces,
                                                   bf16x8* __restrict__ out) {
  const int n_nt = n / kGN, nks = k / kGK;
  const int64_t total = (int64_t)n_w * n_nt * nks * kGBg;
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= total) return;
  const int q = (int)(id % kGBg);
  const int64_t st = id / kGBg;                  // (weight, column tile, stage)
  const int ks = (int)(st % nks), nt = (int)((st / nks) % n_nt), wi = (int)(st / ((int64_t)nks * n_nt));
  // invert b_slot: LDS granule q -> (column c, granule g)
  const int c = q / kGBc, g = (q % kGBc) ^ ((c >> 3) & 1);
  const float* src = w + wi * w_stride + (int64_t)(nt * kGN + c) * ld_n + (int64_t)(ks * kGK + 8 * g) * ld_k;
  floatx4 x0, x1;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x0[i] = src[i * ld_k];
    x1[i] = src[(4 + i) * ld_k];
  }
  bf16x8* dst = out + st * b_stage_granules(pieces) + q;
  if (pieces == 3) {
    bf16x8 p[3];
    split8(x0, x1, p);
    dst[0] = p[0];
    dst[kGBg] = p[1];
    dst[2 * kGBg] = p[2];
  } else {
    bf16x8 p[1];
    round8(x0, x1, p);
    dst[0] = p[0];
  }
}
}  // namespace
}  // namespace e2v2

E2V2_API int64_t e2v2_gemm_packed_bytes(int n_w, int n, int k, int pieces) {
  using namespace e2v2;
  if (n_w <= 0 || n <= 0 || k <= 0 || n % kGN || k % kGK || (pieces != 1 && pieces != 3)) return -1;
  return (int64_t)n_w * (n / kGN) * (k / kGK) * b_stage_granules(pieces) * 16;
}

E2V2_API int e2v2_gemm_pack(const float* w, int64_t ld_n, int64_t ld_k, int64_t w_stride, int n_w, int n, int k,
                            int pieces, void* packed, hipStream_t s) {
  using namespace e2v2;
  E2V2_REQUIRE(pieces == 1 || pieces == 3, "gemm_pack: %d pieces (1 or 3)", pieces);
  E2V2_REQUIRE(n_w > 0 && n_w <= 16, "gemm_pack: %d weights (1 .. 16)", n_w);
  E2V2_REQUIRE(n > 0 && n % kGN == 0, "gemm_pack: n=%d must be a positive multiple of %d", n, kGN);
  E2V2_REQUIRE(k > 0 && k % kGK == 0, "gemm_pack: k=%d must be a positive multiple of %d", k, kGK);
  E2V2_REQUIRE(w && packed, "gemm_pack: null pointer");
  const int64_t total = (int64_t)n_w * (n / kGN) * (k / kGK) * kGBg;
  hipLaunchKernelGGL(k_gemm_pack, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, w, ld_n, ld_k, w_stride, n_w,
                     n, k, pieces, static_cast<bf16x8*>(packed));
  E2V2_LAUNCHED("k_gemm_pack");
  return 0;
}

namespace e2v2 {
namespace {
int check_gemm_args(const e2v2_gemm_args& G) {
  E2V2_REQUIRE(G.batch > 0 && G.batch <= 16, "gemm_s3: batch=%d (1 .. 16)", G.batch);
  E2V2_REQUIRE(G.m >= 0 && G.n > 0 && G.n % kGN == 0 && G.k > 0 && G.k % kGK == 0,
               "gemm_s3: m=%d, n=%d (multiple of %d), k=%d (multiple of %d)", G.m, G.n, kGN, G.k, kGK);
  E2V2_REQUIRE(G.a && G.b && G.c, "gemm_s3: null operand");
  E2V2_REQUIRE((G.pieces == 1 || G.pieces == 3) && (G.a_bf16 == 0 || G.a_bf16 == 1) &&
                   (G.c_bf16 == 0 || G.c_bf16 == 1) && (!G.a_bf16 || G.pieces == 1),
               "gemm_s3: %d pieces with a_bf16 %d, c_bf16 %d (a bf16 A needs one piece)", G.pieces, G.a_bf16,
               G.c_bf16);
  const int ea = G.a_bf16 ? 2 : 4;                     // bytes per A element; granules of 16 bytes
  E2V2_REQUIRE(G.lda >= G.k && G.lda % (16 / ea) == 0 && ((uintptr_t)G.a & 15) == 0,
               "gemm_s3: A needs lda >= k, 16-byte rows (lda %% %d == 0) and 16-byte alignment", 16 / ea);
  E2V2_REQUIRE(G.ldc >= G.n && (!G.r || G.ldr >= G.n), "gemm_s3: ldc / ldr below n");
  E2V2_REQUIRE((uint64_t)(G.m + kGM) * (uint64_t)G.lda * ea < (1ull << 31), "gemm_s3: A batch too large (m=%d)", G.m);
  E2V2_REQUIRE((uint64_t)(G.k / kGK) * b_stage_granules(G.pieces) * 16u < (1ull << 31), "gemm_s3: k=%d too large",
               G.k);
  E2V2_REQUIRE(G.n_w > 0 && G.n_w <= 16, "gemm_s3: n_w=%d (1 .. 16)", G.n_w);
  for (int b = 0; b < G.batch; ++b)
    E2V2_REQUIRE(G.widx[b] >= 0 && G.widx[b] < G.n_w, "gemm_s3: widx[%d]=%d outside 0 .. %d", b, G.widx[b], G.n_w - 1);
  return 0;
}
int host_tiles(const e2v2_gemm_args& G) { return G.batch * ((G.m + kGM - 1) / kGM) * (G.n / kGN); }
}  // namespace
}  // namespace e2v2

E2V2_API int e2v2_gemm_s3(const e2v2_gemm_args* g, hipStream_t s) {
  using namespace e2v2;
  E2V2_REQUIRE(g, "gemm_s3: null arguments");
  const e2v2_gemm_args& G = *g;
  if (int rc = check_gemm_args(G)) return rc;
  if (G.m == 0) return 0;
  const dim3 grid(xcd_grid(host_tiles(G)));
  if (G.pieces == 3)
    hipLaunchKernelGGL(k_gemm_s3, grid, dim3(kGT), 0, s, G);
  else if (G.a_bf16)
    hipLaunchKernelGGL((k_gemm_s3_p1<true>), grid, dim3(kGT), 0, s, G);
  else
    hipLaunchKernelGGL((k_gemm_s3_p1<false>), grid, dim3(kGT), 0, s, G);
  E2V2_LAUNCHED("k_gemm_s3");
  return 0;
}

E2V2_API int e2v2_gemm_s3_gated(const e2v2_gemm_args* g, const float* s, int64_t ld_s, float k1, float k2,
                                hipStream_t st) {
  using namespace e2v2;
  E2V2_REQUIRE(g, "gemm_s3_gated: null arguments");
  const e2v2_gemm_args& G = *g;
  if (int rc = check_gemm_args(G)) return rc;
  E2V2_REQUIRE(s && ((uintptr_t)s & 15) == 0 && ld_s % 4 == 0,
               "gemm_s3_gated: the gate logits need 16-byte alignment and ld_s %% 4 == 0");
  E2V2_REQUIRE(!G.a_bf16, "gemm_s3_gated: the gated operand is fp32");
  for (int b = 0; b < G.batch; ++b)
    E2V2_REQUIRE((int64_t)G.k * (G.widx[b] + 1) <= ld_s, "gemm_s3_gated: batch %d reads logit columns past ld_s=%lld",
                 b, (long long)ld_s);
  E2V2_REQUIRE((uint64_t)(G.m + kGM) * (uint64_t)ld_s * 4u < (1ull << 31), "gemm_s3_gated: logits too large (m=%d)",
               G.m);
  if (G.m == 0) return 0;
  if (G.pieces == 3)
    hipLaunchKernelGGL((k_gemm_s3_gate<3>), dim3(xcd_grid(host_tiles(G))), dim3(kGT), 0, st, G,
                       GateOp{s, ld_s, k1, k2});
  else
    hipLaunchKernelGGL((k_gemm_s3_gate<1>), dim3(xcd_grid(host_tiles(G))), dim3(kGT), 0, st, G,
                       GateOp{s, ld_s, k1, k2});
  E2V2_LAUNCHED("k_gemm_s3_gate");
  return 0;
}

E2V2_API int e2v2_gemm_s3_grouped(const e2v2_gemm_args* groups, int n_groups, hipStream_t s) {
  using namespace e2v2;
  E2V2_REQUIRE(groups && n_groups >= 1 && n_groups <= kGGroups, "gemm_s3_grouped: %d groups (1 .. %d)", n_groups,
               kGGroups);
  GemmGroups P{};
  P.block0[0] = 0;
  for (int i = 0; i < n_groups; ++i) {
    if (int rc = check_gemm_args(groups[i])) return rc;
    E2V2_REQUIRE(groups[i].pieces == groups[0].pieces && groups[i].a_bf16 == groups[0].a_bf16,
                 "gemm_s3_grouped: the groups must share the operand pieces and A's storage type");
    P.g[i] = groups[i];
    P.block0[i + 1] = P.block0[i] + xcd_grid(host_tiles(groups[i]));
    E2V2_REQUIRE(P.block0[i + 1] >= P.block0[i], "gemm_s3_grouped: too many tiles");
  }
  for (int i = n_groups; i < kGGroups; ++i) P.block0[i + 1] = P.block0[n_groups];
  P.n = n_groups;
  if (P.block0[n_groups] == 0) return 0;
  const dim3 grid(P.block0[n_groups]);
  if (groups[0].pieces == 3)
    hipLaunchKernelGGL(k_gemm_s3_grp, grid, dim3(kGT), 0, s, P);
  else if (groups[0].a_bf16)
    hipLaunchKernelGGL((k_gemm_s3_grp_p1<true>), grid, dim3(kGT), 0, s, P);
  else
    hipLaunchKernelGGL((k_gemm_s3_grp_p1<false>), grid, dim3(kGT), 0, s, P);
  E2V2_LAUNCHED("k_gemm_s3_grp");
  return 0;
}

// hq, hk [n][3 hid] and the kept y [9][n][4 hid] (paired order) from x [9][n][c];
// wp: the three per-l weights packed with their columns in the tile-paired order
// (n = 4 hid, k = c), bias [4 hid] in the same order (m = 0 rows only; may be NULL).
E2V2_API int e2v2_qk_proj_fwd_s3(const float* x, const void* wp, const float* bias, void* y, float* hq, float* hk,
                                 int n, int hid, int c, int pieces, int y_bf16, hipStream_t s) {
  using namespace e2v2;
  E2V2_REQUIRE(pieces == 1 || pieces == 3, "qk_proj_fwd_s3: %d pieces (1 or 3)", pieces);
  E2V2_REQUIRE(y_bf16 == 0 || (y_bf16 == 1 && pieces == 1), "qk_proj_fwd_s3: bf16 y (%d) with one piece only",
               y_bf16);
  E2V2_REQUIRE(hid > 0 && hid % 64 == 0, "qk_proj_fwd_s3: hid=%d must be a positive multiple of 64", hid);
  E2V2_REQUIRE(c > 0 && c % kGK == 0, "qk_proj_fwd_s3: C=%d must be a positive multiple of %d", c, kGK);
  E2V2_REQUIRE(x && wp && y && hq && hk, "qk_proj_fwd_s3: null operand");
  E2V2_REQUIRE(((uintptr_t)x & 15) == 0, "qk_proj_fwd_s3: x must be 16-byte aligned");
  E2V2_REQUIRE(n >= 0 && (uint64_t)(n + kGM) * (uint64_t)c * 4u < (1ull << 31) &&
                   (uint64_t)(n + kGM) * 4u * hid < (1ull << 32), "qk_proj_fwd_s3: n=%d too large", n);
  if (n == 0) return 0;
  const int tiles = ((n + kGM - 1) / kGM) * (2 * hid / 64);
  const dim3 grid(3 * xcd_grid(tiles));
  if (pieces == 3)
    hipLaunchKernelGGL((k_qk_s3_fwd<3, false>), grid, dim3(kGT), 0, s, x, wp, bias, y, hq, hk, n, hid, c);
  else if (y_bf16)
    hipLaunchKernelGGL((k_qk_s3_fwd<1, true>), grid, dim3(kGT), 0, s, x, wp, bias, y, hq, hk, n, hid, c);
  else
    hipLaunchKernelGGL((k_qk_s3_fwd<1, false>), grid, dim3(kGT), 0, s, x, wp, bias, y, hq, hk, n, hid, c);
  E2V2_LAUNCHED("k_qk_s3_fwd");
  return 0;
}

// gx [9][n][c] from y (paired order), ghq, ghk [n][3 hid] and, when gv != NULL,
// gv [9][n][cv]; wp: per l the packed [W_l (rows in the paired order) ; Wv_l]^T
// (n = c, k = 4 hid + cv).
E2V2_API int e2v2_qk_proj_bwd_s3(const void* y, const float* ghq, const float* ghk, const void* wp, const float* gv,
                                 float* gx, int n, int hid, int c, int cv, int pieces, int y_bf16, hipStream_t s) {
  using namespace e2v2;
  E2V2_REQUIRE(pieces == 1 || pieces == 3, "qk_proj_bwd_s3: %d pieces (1 or 3)", pieces);
  E2V2_REQUIRE(y_bf16 == 0 || (y_bf16 == 1 && pieces == 1), "qk_proj_bwd_s3: bf16 y (%d) with one piece only",
               y_bf16);
  E2V2_REQUIRE(hid > 0 && hid % 64 == 0, "qk_proj_bwd_s3: hid=%d must be a positive multiple of 64", hid);
  E2V2_REQUIRE(c > 0 && c % kGN == 0, "qk_proj_bwd_s3: C=%d must be a positive multiple of %d", c, kGN);
  E2V2_REQUIRE(cv > 0 && cv % kGK == 0, "qk_proj_bwd_s3: Cv=%d must be a positive multiple of %d", cv, kGK);
  E2V2_REQUIRE(y && ghq && ghk && wp && gx, "qk_proj_bwd_s3: null operand");
  E2V2_REQUIRE(((uintptr_t)y & 15) == 0 && ((uintptr_t)ghq & 15) == 0 && ((uintptr_t)ghk & 15) == 0 &&
                   ((uintptr_t)gv & 15) == 0 && hid % 4 == 0, "qk_proj_bwd_s3: operands must be 16-byte aligned");
  E2V2_REQUIRE(n >= 0 && (uint64_t)(n + kGM) * 4u * hid * 4u < (1ull << 31) &&
                   (uint64_t)(n + kGM) * (uint64_t)cv * 4u < (1ull << 31), "qk_proj_bwd_s3: n=%d too large", n);
  if (n == 0) return 0;
  const int tiles = 9 * ((n + kGM - 1) / kGM) * (c / kGN);
  const dim3 grid(xcd_grid(tiles));
  if (pieces == 3)
    hipLaunchKernelGGL((k_qk_s3_bwd<3, false>), grid, dim3(kGT), 0, s, y, ghq, ghk, wp, gv, gx, n, hid, c, cv);
  else if (y_bf16)
    hipLaunchKernelGGL((k_qk_s3_bwd<1, true>), grid, dim3(kGT), 0, s, y, ghq, ghk, wp, gv, gx, n, hid, c, cv);
  else
    hipLaunchKernelGGL((k_qk_s3_bwd<1, false>), grid, dim3(kGT), 0, s, y, ghq, ghk, wp, gv, gx, n, hid, c, cv);
  E2V2_LAUNCHED("k_qk_s3_bwd");
  return 0;
}
