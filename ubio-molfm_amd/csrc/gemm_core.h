// Shared pieces of the split-bf16 GEMM kernels (gemm.hip, qkdot.hip): tile constants, the exact
// three-piece split of eight fp32 values, the LDS-direct operand loads and slot swizzles, and the
// pipelined K loop.  The scheme itself is described at the top of gemm.hip.
#pragma once
#include <type_traits>

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
constexpr int kGAi = kGAg / 64;                     // wave-wide LDS-direct loads of an fp32 A stage: 8
// Operand pieces kP: 3 (the exact split above, six products) or 1 (bf16 operands: x0 alone, one product,
// the bf16 mode's GEMM).  A kept as bf16 in memory (kAB) is its own single piece: 8 bf16 per granule, two
// granules per row and stage (4 KB).
__host__ __device__ constexpr int a_stage_bytes(bool kAB) { return kAB ? kGM * kGK * 2 : 16 * kGAg; }
__host__ __device__ constexpr int g_stage_bytes(int kP, bool kAB) { return a_stage_bytes(kAB) + 16 * kP * kGBg; }
__host__ __device__ constexpr int b_stage_granules(int kP) { return kP * kGBg; }   // per (weight, column tile, stage)
constexpr int kGStage = g_stage_bytes(3, false);    // largest LDS buffer: 20 KB

__device__ __forceinline__ int a_slot(int r, int g) { return r * kGAr + (g ^ ((r >> 2) & 3)); }       // granules
__device__ __forceinline__ int abf_slot(int r, int g) { return r * 2 + (g ^ ((r >> 3) & 1)); }       // bf16 A
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

// Eight fp32 values -> their bf16 roundings (the first piece alone).
__device__ __forceinline__ void round8(const floatx4& x0, const floatx4& x1, bf16x8 (&p)[1]) {
  p[0] = __builtin_bit_cast(bf16x8, (uint32x4){pk_bf16(x0[0], x0[1]), pk_bf16(x0[2], x0[3]),
                                               pk_bf16(x1[0], x1[1]), pk_bf16(x1[2], x1[3])});
}
template <int kP>
__device__ __forceinline__ void split_pieces(const floatx4& x0, const floatx4& x1, bf16x8 (&p)[kP]) {
  if constexpr (kP == 3) split8(x0, x1, p);
  else round8(x0, x1, p);
}

// LDS-direct load offsets of an fp32 A tile of 128 rows (row stride lda floats):
// this wavefront's two loads per stage (ii = wv, wv + 4) fill LDS granules
// 64 ii .. +63, i.e. rows 16 ii + lane / 4, slot lane % 4, from the source
// granule that belongs there; byte offsets from the tile's first row.
__device__ __forceinline__ void a_offsets(int wv, int lane, int lda, uint32_t (&voff)[kGAi / 4]) {
#pragma unroll
  for (int i = 0; i < kGAi / 4; ++i) {
    const int r = (wv + 4 * i) * 16 + (lane >> 2), sl = lane & 3;
    voff[i] = (uint32_t)(r * lda + 4 * (sl ^ ((r >> 2) & 3))) * 4u;
  }
}
// Buffer resource over rows row0 .. m-1 of a row-major fp32 matrix (reads past
// row m - 1 return zero).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const float* base, int row0, int m, int ld) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base + (size_t)row0 * ld), (short)0,
                                           (int)((uint32_t)(m - row0) * (uint32_t)ld * 4u), 0x00020000);
}
__device__ __forceinline__ void load_a(__amdgpu_buffer_rsrc_t r, const uint32_t (&voff)[kGAi / 4], uint32_t koff,
                                       char* As, int wv) {
#pragma unroll
  for (int i = 0; i < kGAi / 4; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(As + (wv + 4 * i) * 1024), 16, voff[i] + koff, 0, 0, 0);
}
// bf16 A (row stride lda elements): this wavefront's one load per stage fills LDS granules 64 wv .. +63,
// i.e. rows 32 wv + lane / 2, slot lane % 2, from the source granule that belongs there (byte offset from
// the tile's first row; the stage's k offset is 32 ks bytes).
__device__ __forceinline__ uint32_t abf_offset(int wv, int lane, int lda) {
  const int r = 32 * wv + (lane >> 1), sl = lane & 1;
  return (uint32_t)(r * lda + 8 * (sl ^ ((r >> 3) & 1))) * 2u;
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc_bf(const __bf16* base, int row0, int m, int ld) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<__bf16*>(base + (size_t)row0 * ld), (short)0,
                                           (int)((uint32_t)(m - row0) * (uint32_t)ld * 2u), 0x00020000);
}
// The packed B stage ks (kP 4 KB pieces, contiguous from the weight's column-tile base).
template <int kP>
__device__ __forceinline__ void load_b(__amdgpu_buffer_rsrc_t r, int ks, char* Bs, int wv, int lane) {
  const uint32_t bst = (uint32_t)ks * b_stage_granules(kP) * 16u;
#pragma unroll
  for (int i = 0; i < kP; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(Bs + (wv + 4 * i) * 1024), 16,
                                             bst + (uint32_t)((wv + 4 * i) * 1024 + 16 * lane), 0, 0, 0);
}
template <int kP>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t b_rsrc(const void* packed, int w, int n_nt, int nt, int nks) {
  const size_t stage = (size_t)b_stage_granules(kP) * 16;
  const char* base = static_cast<const char*>(packed) + ((size_t)w * n_nt + nt) * (size_t)nks * stage;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), (short)0, (int)(nks * stage), 0x00020000);
}

// A fragment of one stage for this lane (row 32 wv + lane % 32, k 8 (lane / 32) .. +7): eight fp32 values
// (x0, x1) to split into the pieces, or, for a bf16 A, the granule itself (b).
struct AFrag {
  floatx4 x0, x1;
  bf16x8 b;
};

// The pipelined K loop of every kernel here: stage ks sits in LDS buffer ks & 1
// (A at offset 0, the kP B pieces after it, any extra region after them);
// stage ks + 2 is loaded into it (load(ks, buf)) once every wavefront has read
// it.  read_a(ks, buf, f) gives this lane's A fragment of stage ks; it is split
// (or rounded, kP = 1) while the MFMAs of the previous stage run: 24 for kP = 3
// (B by piece: b0 with a0, a1, a2; b1 with a0, a1; b2 with a0), 4 for kP = 1.
// The wavefront accumulates rows 32 wv .. +31 of the tile over all 128 columns
// (four 32x32 tiles j).
template <int kP, bool kAB, typename Load, typename ReadA>
__device__ __forceinline__ void kloop(const char* lds, int stage_bytes, int nks, int lane, Load&& load,
                                      ReadA&& read_a, floatx16 (&acc)[4]) {
  static_assert(kP == 1 || kP == 3, "one or three operand pieces");
  static_assert(!kAB || kP == 1, "a bf16 A operand is one piece");
  const int h = lane >> 5;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
  load(0, 0);
  if (nks > 1) load(1, 1);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  bf16x8 a_cur[kP];
  auto pieces = [&](const AFrag& f) {
    if constexpr (kAB) a_cur[0] = f.b;
    else split_pieces<kP>(f.x0, f.x1, a_cur);
  };
  {
    AFrag f;
    read_a(0, 0, f);
    pieces(f);
  }
  for (int ks = 0; ks < nks; ++ks) {
    const int buf = ks & 1;
    const bf16x8* Bs = reinterpret_cast<const bf16x8*>(lds + buf * stage_bytes + a_stage_bytes(kAB));
    bf16x8 b[kP][4];
#pragma unroll
    for (int p = 0; p < kP; ++p)
#pragma unroll
      for (int j = 0; j < 4; ++j) b[p][j] = Bs[p * kGBg + b_slot(32 * j + (lane & 31), h)];
    if (ks + 1 < nks) {
      __builtin_amdgcn_s_waitcnt(0);      // stage ks + 1 landed; this wavefront's reads of buf are done
      __syncthreads();
      if (ks + 2 < nks) load(ks + 2, buf);
    }
    // (after the last stage this reads the other buffer's stale contents: values never used)
    AFrag f;
    read_a(ks + 1, buf ^ 1, f);
    if constexpr (kP == 3) {
      constexpr int kPa[6] = {0, 1, 2, 0, 1, 0}, kPb[6] = {0, 0, 0, 1, 1, 2};
#pragma unroll
      for (int q = 0; q < 6; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_cur[kPa[q]], b[kPb[q]][j], acc[j], 0, 0, 0);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_cur[0], b[0][j], acc[j], 0, 0, 0);
    }
    pieces(f);
  }
}

// The K loop of the fp32-A GEMMs whose A rows belong to one wavefront each (a wavefront's 32 rows are read by
// no other): A goes from memory straight into registers (load_a(ks, x): this lane's eight values of stage ks,
// row 32 wv + lane % 32, k 8 (lane / 32) .. +7), two stages ahead in a ring of three; the kP B pieces go
// through three LDS buffers (B0, B1, B2: separate objects, so that the compiler's waits for the LDS-direct
// loads of one buffer do not hold the reads of another), filled by load_b(ks, buffer) two stages ahead.  Per
// stage: wait for the stage's own loads (vmcnt: the next stage's kP + 2 may stay in flight), one barrier
// (every wavefront's share of the stage has landed and every wavefront is done with the buffer of stage
// ks - 1, which the loads of stage ks + 2 then fill), the B fragments from LDS, the split of A, the MFMAs.
// The steady state issues a stage's loads in every step (no branch between the loads and the waits); the
// last stages run with the loads past the end left out.  The products and their order are those of kloop.
template <int kP, typename LoadB, typename LoadA>
__device__ __forceinline__ void kloop_r(char* B0, char* B1, char* B2, int nks, int lane, LoadB&& load_b_,
                                        LoadA&& load_a_, floatx16 (&acc)[4]) {
  static_assert(kP == 1 || kP == 3, "one or three operand pieces");
  const int h = lane >> 5;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
  floatx4 av[3][2];
  auto load = [&](int ks, auto slot) {
    constexpr int sl = decltype(slot)::value;
    load_b_(ks, sl == 0 ? B0 : sl == 1 ? B1 : B2);
    load_a_(ks, av[sl]);
  };
  auto step = [&](int ks, auto slot, auto steady) {
    constexpr int sl = decltype(slot)::value, sl2 = (sl + 2) % 3;
    constexpr bool kU = decltype(steady)::value;
    // s_waitcnt immediate (gfx9): vmcnt in bits 3:0 (and 15:14), expcnt 6:4 and lgkmcnt 11:8 at their
    // maxima (no wait).  Per stage a wavefront issues kP LDS-direct B loads and two A loads.
    if (kU || ks + 1 < nks) __builtin_amdgcn_s_waitcnt(0x0F70 | (kP + 2));   // vmcnt(kP + 2)
    else __builtin_amdgcn_s_waitcnt(0x0F70);                                // vmcnt(0)
    // a plain s_barrier: __syncthreads()'s release fence would also wait for the loads of stage ks + 1
    asm volatile("s_barrier" ::: "memory");
    if (kU || ks + 2 < nks) load(ks + 2, std::integral_constant<int, sl2>{});
    const bf16x8* Bs = reinterpret_cast<const bf16x8*>(sl == 0 ? B0 : sl == 1 ? B1 : B2);
    bf16x8 b[kP][4];
#pragma unroll
    for (int p = 0; p < kP; ++p)
#pragma unroll
      for (int j = 0; j < 4; ++j) b[p][j] = Bs[p * kGBg + b_slot(32 * j + (lane & 31), h)];
    bf16x8 a[kP];
    split_pieces<kP>(av[sl][0], av[sl][1], a);
    if constexpr (kP == 3) {
      constexpr int kPa[6] = {0, 1, 2, 0, 1, 0}, kPb[6] = {0, 0, 0, 1, 1, 2};
#pragma unroll
      for (int q = 0; q < 6; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[kPa[q]], b[kPb[q]][j], acc[j], 0, 0, 0);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0][j], acc[j], 0, 0, 0);
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  load(0, I0{});
  if (nks > 1) load(1, I1{});
  int ks = 0;
  for (; ks + 5 <= nks; ks += 3) {   // every step here issues stage ks + 2 <= nks - 1
    step(ks, I0{}, std::true_type{});
    step(ks + 1, I1{}, std::true_type{});
    step(ks + 2, I2{}, std::true_type{});
  }
  for (; ks < nks; ks += 3) {
    step(ks, I0{}, std::false_type{});
    if (ks + 1 < nks) step(ks + 1, I1{}, std::false_type{});
    if (ks + 2 < nks) step(ks + 2, I2{}, std::false_type{});
  }
}
// This lane's eight A values of stage ks from a buffer resource over the tile's rows (rows past m read as
// zero): byte offset aoff of the lane's row and k 8 (lane / 32), plus 64 bytes per stage.
__device__ __forceinline__ void load_a_regs(__amdgpu_buffer_rsrc_t r, uint32_t aoff, int ks, floatx4 (&x)[2]) {
  const uint32_t o = aoff + (uint32_t)ks * (kGK * 4u);
  x[0] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, o, 0, 0));
  x[1] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, o + 16u, 0, 0));
}
constexpr int b_stage_bytes(int kP) { return 16 * kP * kGBg; }

}  // namespace
}  // namespace e2v2
