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
#include "common.h"
#include "../../include/e2v2.h"

namespace e2v2 {
namespace {
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef uint32_t uint32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kGM = 128, kGN = 128, kGK = 16, kGT = 256;
constexpr int kGAr = kGK / 4;                       // A granules (4 fp32) per row and stage
constexpr int kGBc = kGK / 8;                       // B granules (8 bf16) per column, piece and stage
constexpr int kGAg = kGM * kGAr;                    // A granules per stage: 512
constexpr int kGBg = kGN * kGBc;                    // granules per B piece and stage: 256
constexpr int kGStage = 16 * (kGAg + 3 * kGBg);     // bytes per LDS buffer: 20 KB
constexpr int kGBStage = 3 * kGBg;                  // packed granules per (weight, column tile, stage)
constexpr int kGAi = kGAg / 64, kGBi = kGBStage / 64;   // wave-wide LDS-direct loads per stage: 8 (A), 12 (B)

__device__ __forceinline__ int a_slot(int r, int g) { return r * kGAr + (g ^ ((r >> 2) & 3)); }       // granules
__host__ __device__ __forceinline__ int b_slot(int c, int g) { return c * kGBc + (g ^ ((c >> 3) & 1)); }

// Row of accumulator register r of a 32x32 tile for this lane (column = lane & 31).
__device__ __forceinline__ int acc_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// Two fp32 values -> one dword of two bf16 (round to nearest even; a in the low half).
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((float2v){a, b}, bf16x2));
}
__device__ __forceinline__ float lo_f(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float hi_f(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// Eight fp32 values -> their three bf16 pieces, two values per conversion; the
// remainders are formed from the packed pieces by shifts / masks (exact).
__device__ __forceinline__ void split8(const floatx4& x0, const floatx4& x1, bf16x8 (&p)[3]) {
  uint32_t u[3][4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float x = q < 2 ? x0[2 * q] : x1[2 * q - 4], y = q < 2 ? x0[2 * q + 1] : x1[2 * q - 3];
    const uint32_t h = pk_bf16(x, y);
    const float rx = x - lo_f(h), ry = y - hi_f(h);
    const uint32_t m = pk_bf16(rx, ry);
    u[0][q] = h;
    u[1][q] = m;
    u[2][q] = pk_bf16(rx - lo_f(m), ry - hi_f(m));
  }
#pragma unroll
  for (int k = 0; k < 3; ++k) p[k] = __builtin_bit_cast(bf16x8, (uint32x4){u[k][0], u[k][1], u[k][2], u[k][3]});
}

__global__ __launch_bounds__(kGT, 3) void k_gemm_s3(e2v2_gemm_args G) {
  __shared__ __attribute__((aligned(16))) char lds[2 * kGStage];
  const int t = threadIdx.x, lane = t & 63, wv = __builtin_amdgcn_readfirstlane(t >> 6), h = lane >> 5;
  const int n_mt = (G.m + kGM - 1) / kGM, n_nt = G.n / kGN, n_tiles = G.batch * n_mt * n_nt;
  const int tile = xcd_row(blockIdx.x, n_tiles);
  if (tile >= n_tiles) return;
  const int nt = tile % n_nt, mt = (tile / n_nt) % n_mt, bi = tile / (n_nt * n_mt);
  const int row0 = mt * kGM, nks = G.k / kGK;

  // A: buffer over this batch's rows row0 .. m-1 (reads past m return zero).  Load
  // instruction ii (= wv, wv + 4) fills LDS granules 64 ii .. +63, i.e. rows
  // 16 ii + lane / 4, slot lane % 4, from the source granule that belongs there.
  const float* abase = G.a + (size_t)bi * G.a_bs + (size_t)row0 * G.lda;
  const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(abase), (short)0, (int)((uint32_t)(G.m - row0) * (uint32_t)G.lda * 4u), 0x00020000);
  uint32_t a_voff[kGAi / 4];
#pragma unroll
  for (int i = 0; i < kGAi / 4; ++i) {
    const int r = (wv + 4 * i) * 16 + (lane >> 2), sl = lane & 3;
    a_voff[i] = (uint32_t)(r * G.lda + 4 * (sl ^ ((r >> 2) & 3))) * 4u;
  }
  // B: contiguous packed stages of this weight and column tile
  const char* bbase = static_cast<const char*>(G.b) + ((size_t)G.widx[bi] * n_nt + nt) * (size_t)nks * kGBStage * 16;
  const __amdgpu_buffer_rsrc_t br =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(bbase), (short)0, nks * kGBStage * 16, 0x00020000);

  auto load = [&](int ks, int buf) {
    char* As = lds + buf * kGStage;
    char* Bs = As + kGAg * 16;
    const uint32_t koff = (uint32_t)(ks * kGK) * 4u;
#pragma unroll
    for (int i = 0; i < kGAi / 4; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ar, (lds_void*)(As + (wv + 4 * i) * 1024), 16, a_voff[i] + koff, 0, 0, 0);
    const uint32_t bst = (uint32_t)ks * kGBStage * 16u;
#pragma unroll
    for (int i = 0; i < kGBi / 4; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(br, (lds_void*)(Bs + (wv + 4 * i) * 1024), 16,
                                               bst + (uint32_t)((wv + 4 * i) * 1024 + 16 * lane), 0, 0, 0);
  };
  // wavefront wv: rows 32 wv .. +31 of the tile, all 128 columns (four 32x32 tiles j)
  const int ra = wv * 32 + (lane & 31);
  auto a_lds = [&](int buf) { return reinterpret_cast<const floatx4*>(lds + buf * kGStage); };
  auto b_lds = [&](int buf) { return reinterpret_cast<const bf16x8*>(lds + buf * kGStage + kGAg * 16); };

  floatx16 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;

  // Stage ks sits in buffer ks & 1; stage ks + 2 is loaded into it once every
  // wavefront has read it.  The A fragment of stage ks + 1 is split while the
  // MFMAs of stage ks run.
  load(0, 0);
  if (nks > 1) load(1, 1);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  bf16x8 a_cur[3];
  split8(a_lds(0)[a_slot(ra, 2 * h)], a_lds(0)[a_slot(ra, 2 * h + 1)], a_cur);
  for (int ks = 0; ks < nks; ++ks) {
    const int buf = ks & 1;
    bf16x8 b[3][4];
#pragma unroll
    for (int p = 0; p < 3; ++p)
#pragma unroll
      for (int j = 0; j < 4; ++j) b[p][j] = b_lds(buf)[p * kGBg + b_slot(32 * j + (lane & 31), h)];
    if (ks + 1 < nks) {
      __builtin_amdgcn_s_waitcnt(0);      // stage ks + 1 landed; this wavefront's reads of buf are done
      __syncthreads();
      if (ks + 2 < nks) load(ks + 2, buf);
    }
    // (after the last stage this reads the other buffer's stale A: a value never used)
    const floatx4 x0 = a_lds(buf ^ 1)[a_slot(ra, 2 * h)], x1 = a_lds(buf ^ 1)[a_slot(ra, 2 * h + 1)];
    constexpr int kPa[6] = {0, 1, 2, 0, 1, 0}, kPb[6] = {0, 0, 0, 1, 1, 2};
#pragma unroll
    for (int q = 0; q < 6; ++q)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_cur[kPa[q]], b[kPb[q]][j], acc[j], 0, 0, 0);
    split8(x0, x1, a_cur);
  }

  // epilogue: C = acc (+ bias) (+ R)
  const bool with_bias = G.bias && bi < G.bias_batches;
  float* cb = G.c + (size_t)bi * G.c_bs;
  const float* rb = G.r ? G.r + (size_t)bi * G.r_bs : nullptr;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int col = nt * kGN + 32 * j + (lane & 31);
    const float bv = with_bias ? G.bias[col] : 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = row0 + wv * 32 + acc_row(r, lane);
      if (row < G.m) {
        float v = acc[j][r];
        if (with_bias) v += bv;
        if (rb) v += rb[(size_t)row * G.ldr + col];
        cb[(size_t)row * G.ldc + col] = v;
      }
    }
  }
}

// Pack: one thread per (weight, column tile, stage, LDS granule): the granule's
// eight k of its column, split into the three pieces.
__global__ __launch_bounds__(256) void k_gemm_pack(const float* __restrict__ w, int64_t ld_n, int64_t ld_k,
                                                   int64_t w_stride, int n_w, int n, int k, bf16x8* __restrict__ out) {
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
  bf16x8 p[3];
  split8(x0, x1, p);
  bf16x8* dst = out + st * kGBStage + q;
  dst[0] = p[0];
  dst[kGBg] = p[1];
  dst[2 * kGBg] = p[2];
}
}  // namespace
}  // namespace e2v2

E2V2_API int64_t e2v2_gemm_packed_bytes(int n_w, int n, int k) {
  using namespace e2v2;
  if (n_w <= 0 || n <= 0 || k <= 0 || n % kGN || k % kGK) return -1;
  return (int64_t)n_w * (n / kGN) * (k / kGK) * kGBStage * 16;
}

E2V2_API int e2v2_gemm_pack(const float* w, int64_t ld_n, int64_t ld_k, int64_t w_stride, int n_w, int n, int k,
                            void* packed, hipStream_t s) {
  using namespace e2v2;
  E2V2_REQUIRE(n_w > 0 && n_w <= 16, "gemm_pack: %d weights (1 .. 16)", n_w);
  E2V2_REQUIRE(n > 0 && n % kGN == 0, "gemm_pack: n=%d must be a positive multiple of %d", n, kGN);
  E2V2_REQUIRE(k > 0 && k % kGK == 0, "gemm_pack: k=%d must be a positive multiple of %d", k, kGK);
  E2V2_REQUIRE(w && packed, "gemm_pack: null pointer");
  const int64_t total = (int64_t)n_w * (n / kGN) * (k / kGK) * kGBg;
  hipLaunchKernelGGL(k_gemm_pack, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, w, ld_n, ld_k, w_stride, n_w,
                     n, k, static_cast<bf16x8*>(packed));
  E2V2_LAUNCHED("k_gemm_pack");
  return 0;
}

E2V2_API int e2v2_gemm_s3(const e2v2_gemm_args* g, hipStream_t s) {
  using namespace e2v2;
  E2V2_REQUIRE(g, "gemm_s3: null arguments");
  const e2v2_gemm_args& G = *g;
  E2V2_REQUIRE(G.batch > 0 && G.batch <= 16, "gemm_s3: batch=%d (1 .. 16)", G.batch);
  E2V2_REQUIRE(G.m >= 0 && G.n > 0 && G.n % kGN == 0 && G.k > 0 && G.k % kGK == 0,
               "gemm_s3: m=%d, n=%d (multiple of %d), k=%d (multiple of %d)", G.m, G.n, kGN, G.k, kGK);
  E2V2_REQUIRE(G.a && G.b && G.c, "gemm_s3: null operand");
  E2V2_REQUIRE(G.lda >= G.k && G.lda % 4 == 0 && ((uintptr_t)G.a & 15) == 0,
               "gemm_s3: A needs lda >= k, lda %% 4 == 0 and 16-byte alignment");
  E2V2_REQUIRE(G.ldc >= G.n && (!G.r || G.ldr >= G.n), "gemm_s3: ldc / ldr below n");
  E2V2_REQUIRE((uint64_t)(G.m + kGM) * (uint64_t)G.lda * 4u < (1ull << 31), "gemm_s3: A batch too large (m=%d)", G.m);
  E2V2_REQUIRE((uint64_t)(G.k / kGK) * kGBStage * 16u < (1ull << 31), "gemm_s3: k=%d too large", G.k);
  E2V2_REQUIRE(G.n_w > 0 && G.n_w <= 16, "gemm_s3: n_w=%d (1 .. 16)", G.n_w);
  for (int b = 0; b < G.batch; ++b)
    E2V2_REQUIRE(G.widx[b] >= 0 && G.widx[b] < G.n_w, "gemm_s3: widx[%d]=%d outside 0 .. %d", b, G.widx[b], G.n_w - 1);
  if (G.m == 0) return 0;
  const int tiles = G.batch * ((G.m + kGM - 1) / kGM) * (G.n / kGN);
  hipLaunchKernelGGL(k_gemm_s3, dim3(xcd_grid(tiles)), dim3(kGT), 0, s, G);
  E2V2_LAUNCHED("k_gemm_s3");
  return 0;
}
