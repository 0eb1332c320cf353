// Periodic radius graph: cell-list binning -> per-row count -> exclusive scan
// -> fill -> per-row sort by (distance, j, shift) -> key CSR (transpose).
//
// Replaces CellExpander.expand_includeself + construct_radius_neighbor
// (src/molfm/models/e2former/module_utils.py:1065-1274,3119-3242) and the
// CSR metadata of prepare_sparse_qk_edge_index_metadata
// (src/molfm/models/e2former/triton_dr/triton_sparse_qk_autograd.py:601-652).
#include <mutex>

#include "common.h"
#include "../../include/e2v2.h"

namespace e2v2 {

__global__ void k_fill_i32(int32_t* __restrict__ p, int32_t v, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = v;
}

__global__ void k_fill_f32(float* __restrict__ p, float v, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = v;
}

// Single-workgroup exclusive scan: out[0..n] with out[n] = total;
// stats[0] = total, stats[1] = max(in).
__global__ __launch_bounds__(1024) void k_scan_i32(const int32_t* __restrict__ in, int n,
                                                   int32_t* __restrict__ out, int32_t* __restrict__ stats) {
  __shared__ int64_t part[1024];
  __shared__ int32_t pmax[1024];
  const int t = threadIdx.x;
  const int per = (n + 1023) / 1024;
  const int b = t * per;
  const int e = min(n, b + per);
  int64_t s = 0;
  int32_t mx = 0;
  for (int i = b; i < e; ++i) {
    s += in[i];
    mx = max(mx, in[i]);
  }
  part[t] = s;
  pmax[t] = mx;
  __syncthreads();
  // Hillis-Steele inclusive scan over 1024 partials
  for (int o = 1; o < 1024; o <<= 1) {
    int64_t v = (t >= o) ? part[t - o] : 0;
    int32_t m = (t >= o) ? pmax[t - o] : 0;
    __syncthreads();
    part[t] += v;
    pmax[t] = max(pmax[t], m);
    __syncthreads();
  }
  int64_t run = part[t] - s;
  for (int i = b; i < e; ++i) {
    out[i] = (int32_t)run;
    run += in[i];
  }
  if (t == 1023) {
    out[n] = (int32_t)part[1023];
    stats[0] = (int32_t)part[1023];
    stats[1] = pmax[1023];
  }
}

__device__ __forceinline__ int bin_coord(float x, float lo, float h, int dim) {
  int b = (int)floorf((x - lo) / h);
  return min(max(b, 0), dim - 1);
}

// An atom outside its graph's grid box (possible only with a caller-supplied box):
// the cell search tolerates atoms up to the bin margin (0.01 A) outside, so one
// further out than 1e-3 A is flagged in stats[2] for the host to rebuild with
// the atoms' own bounding box.
__device__ __forceinline__ bool outside_box(float x, float lo, float h, int dim) {
  return !(x >= lo - 1e-3f && x <= lo + h * (float)dim + 1e-3f);
}

__global__ void k_bin_assign(e2v2_nbr_plan P) {
  int a = blockIdx.x * blockDim.x + threadIdx.x;
  if (a >= P.n_atoms) return;
  int g = P.atom_graph[a];
  const float* p = P.pos + 3 * a;
  int bx = bin_coord(p[0], P.grid_lo[3 * g + 0], P.grid_h[3 * g + 0], P.grid_dim[3 * g + 0]);
  int by = bin_coord(p[1], P.grid_lo[3 * g + 1], P.grid_h[3 * g + 1], P.grid_dim[3 * g + 1]);
  int bz = bin_coord(p[2], P.grid_lo[3 * g + 2], P.grid_h[3 * g + 2], P.grid_dim[3 * g + 2]);
  bool out = false;
#pragma unroll
  for (int d = 0; d < 3; ++d) out |= outside_box(p[d], P.grid_lo[3 * g + d], P.grid_h[3 * g + d], P.grid_dim[3 * g + d]);
  if (out) atomicOr(&P.stats[2], 1);
  int bin = P.bin_base[g] + (bx * P.grid_dim[3 * g + 1] + by) * P.grid_dim[3 * g + 2] + bz;
  P.atom_bin[a] = bin;
  atomicAdd(&P.bin_count[bin], 1);
}

__global__ void k_bin_fill(e2v2_nbr_plan P, int32_t* __restrict__ cursor) {
  int a = blockIdx.x * blockDim.x + threadIdx.x;
  if (a >= P.n_atoms) return;
  int bin = P.atom_bin[a];
  int slot = P.bin_start[bin] + atomicAdd(&cursor[bin], 1);
  P.bin_atoms[slot] = a;
}

constexpr float kBinMargin = 1e-2f;

// Does any atom of graph g lie strictly within rc of the image img?
__device__ bool image_has_inner(const e2v2_nbr_plan& P, int g, const float* img) {
  const float lo0 = P.grid_lo[3 * g], lo1 = P.grid_lo[3 * g + 1], lo2 = P.grid_lo[3 * g + 2];
  const float h0 = P.grid_h[3 * g], h1 = P.grid_h[3 * g + 1], h2 = P.grid_h[3 * g + 2];
  const int d0 = P.grid_dim[3 * g], d1 = P.grid_dim[3 * g + 1], d2 = P.grid_dim[3 * g + 2];
  const float r = P.rc + kBinMargin;
  int x0 = (int)floorf((img[0] - r - lo0) / h0), x1 = (int)floorf((img[0] + r - lo0) / h0);
  int y0 = (int)floorf((img[1] - r - lo1) / h1), y1 = (int)floorf((img[1] + r - lo1) / h1);
  int z0 = (int)floorf((img[2] - r - lo2) / h2), z1 = (int)floorf((img[2] + r - lo2) / h2);
  x0 = max(x0, 0); y0 = max(y0, 0); z0 = max(z0, 0);
  x1 = min(x1, d0 - 1); y1 = min(y1, d1 - 1); z1 = min(z1, d2 - 1);
  const float zero[3] = {0.f, 0.f, 0.f};
  for (int bx = x0; bx <= x1; ++bx)
    for (int by = y0; by <= y1; ++by)
      for (int bz = z0; bz <= z1; ++bz) {
        int bin = P.bin_base[g] + (bx * d1 + by) * d2 + bz;
        for (int s = P.bin_start[bin]; s < P.bin_start[bin + 1]; ++s) {
          int k = P.bin_atoms[s];
          float dx, dy, dz;
          exact_edge(P.pos + 3 * k, img, zero, dx, dy, dz);
          if (exact_dist(dx, dy, dz) < P.rc) return true;
        }
      }
  return false;
}

// Visit every edge i <- (j, s) of atom i with one wavefront.  For each shift the
// bins within rc + margin of pos_i - off span at most 3 bins per direction
// (bin edge h >= rc + margin), so they form at most 3 x 3 columns of
// z-consecutive bins, i.e. at most 9 contiguous runs of bin_atoms.  The runs are
// concatenated and dealt out 64 candidates per round.  (A fourth bin that fp32
// rounding of the bin range could add starts beyond q + rc + margin, so it holds
// no edge.)  emit(ok, j, s, dx, dy, dz, d) is called by every lane of the wave in
// each round (ok false on lanes without an edge) and may use wave-wide ballots.
template <class Emit>
__device__ void visit_edges_wave(const e2v2_nbr_plan& P, int i, Emit&& emit) {
  const int lane = threadIdx.x & 63;
  const int g = P.atom_graph[i];
  const bool periodic = P.graph_periodic[g] != 0;
  const float pi[3] = {P.pos[3 * i], P.pos[3 * i + 1], P.pos[3 * i + 2]};
  const float lo0 = P.grid_lo[3 * g], lo1 = P.grid_lo[3 * g + 1], lo2 = P.grid_lo[3 * g + 2];
  const float h0 = P.grid_h[3 * g], h1 = P.grid_h[3 * g + 1], h2 = P.grid_h[3 * g + 2];
  const int d0 = P.grid_dim[3 * g], d1 = P.grid_dim[3 * g + 1], d2 = P.grid_dim[3 * g + 2];
  const int bbase = P.bin_base[g];
  const float r = P.rc + kBinMargin;
  for (int s = P.graph_shift_ptr[g]; s < P.graph_shift_ptr[g + 1]; ++s) {
    const float* off = P.shift_off + 3 * s;
    const float q0 = pi[0] - off[0], q1 = pi[1] - off[1], q2 = pi[2] - off[2];
    int x0 = (int)floorf((q0 - r - lo0) / h0), x1 = (int)floorf((q0 + r - lo0) / h0);
    if (x1 < 0 || x0 > d0 - 1) continue;
    int y0 = (int)floorf((q1 - r - lo1) / h1), y1 = (int)floorf((q1 + r - lo1) / h1);
    if (y1 < 0 || y0 > d1 - 1) continue;
    int z0 = (int)floorf((q2 - r - lo2) / h2), z1 = (int)floorf((q2 + r - lo2) / h2);
    if (z1 < 0 || z0 > d2 - 1) continue;
    x0 = max(x0, 0); y0 = max(y0, 0); z0 = max(z0, 0);
    x1 = min(min(x1, d0 - 1), x0 + 2); y1 = min(min(y1, d1 - 1), y0 + 2); z1 = min(min(z1, d2 - 1), z0 + 2);
    // run r = (a, b) holds bins (x0 + a, y0 + b, z0..z1); pre = inclusive prefix of
    // run lengths, base = run start - exclusive prefix
    int pre[9], base[9];
    int total = 0;
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
      for (int b = 0; b < 3; ++b) {
        int st = 0, len = 0;
        if (x0 + a <= x1 && y0 + b <= y1) {
          const int bin = bbase + ((x0 + a) * d1 + (y0 + b)) * d2;
          st = P.bin_start[bin + z0];
          len = P.bin_start[bin + z1 + 1] - st;
        }
        base[3 * a + b] = st - total;
        total += len;
        pre[3 * a + b] = total;
      }
    for (int c0 = 0; c0 < total; c0 += 64) {
      const int c = c0 + lane;
      bool ok = false;
      int j = 0;
      float dx = 0.f, dy = 0.f, dz = 0.f, d = 0.f;
      if (c < total) {
        int t = 0;
#pragma unroll
        for (int q = 8; q >= 0; --q)
          if (c < pre[q]) t = base[q] + c;
        j = P.bin_atoms[t];
        exact_edge(pi, P.pos + 3 * j, off, dx, dy, dz);
        d = exact_dist(dx, dy, dz);
        ok = d >= P.rmin && d <= P.rc && (P.src_include == nullptr || P.src_include[j] != 0);
        if (ok && periodic && !(d < P.rc)) {
          float img[3];
          {
#pragma clang fp contract(off)
            img[0] = P.pos[3 * j] + off[0];
            img[1] = P.pos[3 * j + 1] + off[1];
            img[2] = P.pos[3 * j + 2] + off[2];
          }
          ok = image_has_inner(P, g, img);
        }
      }
      emit(ok, j, s, dx, dy, dz, d);
    }
  }
}

// lanes below this one whose bit is set in m
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

constexpr int kNbrWaves = 4;  // atoms (wavefronts) per workgroup of the count and fill kernels

__global__ __launch_bounds__(64 * kNbrWaves) void k_nbr_count(e2v2_nbr_plan P, int32_t* __restrict__ row_count) {
  for (int i = blockIdx.x * kNbrWaves + (int)(threadIdx.x >> 6); i < P.n_atoms; i += gridDim.x * kNbrWaves) {
    int c = 0;
    visit_edges_wave(P, i, [&](bool ok, int, int, float, float, float, float) { c += __popcll(__ballot(ok)); });
    if ((threadIdx.x & 63) == 0) row_count[i] = c;
  }
}

__global__ __launch_bounds__(64 * kNbrWaves) void k_nbr_fill(e2v2_nbr_plan P, const int32_t* __restrict__ row_ptr,
                                                            int32_t* __restrict__ col, int32_t* __restrict__ shift,
                                                            float* __restrict__ dvec, float* __restrict__ dist,
                                                            uint64_t* __restrict__ key) {
  for (int i = blockIdx.x * kNbrWaves + (int)(threadIdx.x >> 6); i < P.n_atoms; i += gridDim.x * kNbrWaves) {
    int o = row_ptr[i];
    const int o_end = row_ptr[i + 1];
    const int g = P.atom_graph[i];
    const int a0 = P.graph_atom_ptr[g];
    const int s0 = P.graph_shift_ptr[g];
    const int ns = P.graph_shift_ptr[g + 1] - s0;
    visit_edges_wave(P, i, [&](bool ok, int j, int s, float dx, float dy, float dz, float d) {
      const uint64_t m = __ballot(ok);
      const int p = o + lanes_below(m);
      if (ok && p < o_end) {  // count and fill share one traversal; never write past the row
        col[p] = j;
        shift[p] = s;
        dvec[3 * p] = dx;
        dvec[3 * p + 1] = dy;
        dvec[3 * p + 2] = dz;
        dist[p] = d;
        uint32_t lo = (uint32_t)(j - a0) * (uint32_t)ns + (uint32_t)(s - s0);
        key[p] = ((uint64_t)__float_as_uint(d) << 32) | (uint64_t)lo;
      }
      o += __popcll(m);
    });
  }
}

// Bitonic sort of one segment per workgroup (length <= kMaxSeg), returning
// the sorted order as source positions.
constexpr int kMaxSeg = 4096;

__device__ void segment_sort(const uint64_t* __restrict__ key, int b, int n, uint64_t* sk, int32_t* sv) {
  int p2 = 1;
  while (p2 < n) p2 <<= 1;
  for (int t = threadIdx.x; t < p2; t += blockDim.x) {
    sk[t] = (t < n) ? key[b + t] : ~0ull;
    sv[t] = (t < n) ? t : 0x7fffffff;
  }
  __syncthreads();
  for (int k = 2; k <= p2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int t = threadIdx.x; t < p2; t += blockDim.x) {
        int x = t ^ j;
        if (x > t) {
          bool up = ((t & k) == 0);
          uint64_t a = sk[t], c = sk[x];
          int32_t va = sv[t], vc = sv[x];
          bool gt = (a > c) || (a == c && va > vc);
          if (gt == up) {
            sk[t] = c; sk[x] = a;
            sv[t] = vc; sv[x] = va;
          }
        }
      }
      __syncthreads();
    }
  }
}

// One wavefront per row (column); LDS holds cap keys and positions (cap = the
// longest row rounded up to a power of two, sized by the host).
extern __shared__ uint64_t seg_lds[];

__global__ __launch_bounds__(64) void k_sort_rows(const int32_t* __restrict__ row_ptr,
                                                  const uint64_t* __restrict__ key,
                                                  const int32_t* __restrict__ tcol, const int32_t* __restrict__ tshift,
                                                  const float* __restrict__ tdv, const float* __restrict__ td,
                                                  int32_t* __restrict__ col, int32_t* __restrict__ shift,
                                                  float* __restrict__ dvec, float* __restrict__ dist, int cap) {
  uint64_t* sk = seg_lds;
  int32_t* sv = reinterpret_cast<int32_t*>(seg_lds + cap);
  const int r = blockIdx.x;
  const int b = row_ptr[r], n_row = row_ptr[r + 1] - b, n = min(n_row, cap);
  if (n_row == 0) return;
  segment_sort(key, b, n, sk, sv);
  // A row longer than cap exists only in a capacity build that overflowed (the caller
  // rebuilds the list): its first cap entries are sorted and the rest copied unsorted, so
  // that every entry of the row is still one of its edges for the kernels that read it.
  for (int t = threadIdx.x; t < n_row; t += blockDim.x) {
    int src = t < n ? b + sv[t] : b + t, dst = b + t;
    col[dst] = tcol[src];
    shift[dst] = tshift[src];
    dvec[3 * dst] = tdv[3 * src];
    dvec[3 * dst + 1] = tdv[3 * src + 1];
    dvec[3 * dst + 2] = tdv[3 * src + 2];
    dist[dst] = td[src];
  }
}

// Capacity build: stats = {E, longest row} of the scan; rows are clamped to the
// first cap_edges edge slots and stats[3] = 1 when the list needs more edges or a
// longer row than the caller sized for (the list is then truncated).
__global__ void k_cap_rows(int32_t* __restrict__ row_ptr, int n_rows, int64_t cap_edges, int cap_row,
                           int32_t* __restrict__ stats) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i == 0) stats[3] = ((int64_t)stats[0] > cap_edges || stats[1] > cap_row) ? 1 : 0;
  if (i <= n_rows) row_ptr[i] = (int32_t)min((int64_t)row_ptr[i], cap_edges);
}

// edge -> row index
__global__ void k_edge_rows(const int32_t* __restrict__ row_ptr, int n_rows, int32_t* __restrict__ edge_row) {
  int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= n_rows) return;
  for (int e = row_ptr[r]; e < row_ptr[r + 1]; ++e) edge_row[e] = r;
}

// e_end (NULL: n_edges) bounds the edges on the device: the query CSR's row_ptr[n_rows],
// which is below n_edges in a capacity build (arrays sized for more edges than exist)
__global__ void k_col_count(const int32_t* __restrict__ col, int64_t n_edges, const int32_t* __restrict__ e_end,
                            int32_t* __restrict__ cnt) {
  int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n_edges || (e_end && e >= *e_end)) return;
  atomicAdd(&cnt[col[e]], 1);
}

__global__ void k_col_fill(const int32_t* __restrict__ col, int64_t n_edges, const int32_t* __restrict__ e_end,
                           const int32_t* __restrict__ key_ptr, int32_t* __restrict__ cursor,
                           uint64_t* __restrict__ tkey) {
  int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n_edges || (e_end && e >= *e_end)) return;
  int j = col[e];
  int slot = key_ptr[j] + atomicAdd(&cursor[j], 1);
  tkey[slot] = (uint64_t)e;
}

// In-place ascending sort of n distinct keys in global memory by one workgroup,
// for segments longer than the LDS sort holds.  Bitonic network in the form
// whose comparators all put the minimum at the lower index (first step of each
// merge pairs t with t ^ (k - 1), later steps t with t ^ j), so positions past
// n act as +infinity and their comparators are skipped.
__device__ void sort_global(uint64_t* __restrict__ k, int n) {
  int p2 = 1;
  while (p2 < n) p2 <<= 1;
  for (int kk = 2; kk <= p2; kk <<= 1) {
    for (int j = kk >> 1; j > 0; j >>= 1) {
      for (int t = threadIdx.x; t < p2; t += blockDim.x) {
        const int x = (j == (kk >> 1)) ? (t ^ (kk - 1)) : (t ^ j);
        if (x > t && x < n) {
          const uint64_t a = k[t], c = k[x];
          if (a > c) {
            k[t] = c;
            k[x] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Columns of any length: up to cap in LDS, longer ones in place in global
// memory (tkey is scratch), so the host needs no column-length check.
__global__ __launch_bounds__(64) void k_sort_cols(const int32_t* __restrict__ key_ptr,
                                                  uint64_t* __restrict__ tkey,
                                                  int32_t* __restrict__ key_eid, int cap) {
  uint64_t* sk = seg_lds;
  int32_t* sv = reinterpret_cast<int32_t*>(seg_lds + cap);
  const int r = blockIdx.x;
  const int b = key_ptr[r], n = key_ptr[r + 1] - b;
  if (n == 0) return;
  if (n > cap) {
    sort_global(tkey + b, n);
    for (int t = threadIdx.x; t < n; t += blockDim.x) key_eid[b + t] = (int32_t)tkey[b + t];
    return;
  }
  segment_sort(tkey, b, n, sk, sv);
  for (int t = threadIdx.x; t < n; t += blockDim.x) key_eid[b + t] = (int32_t)sk[t];
}

// Clusters of `span` consecutive segments of a CSR (rows of the query CSR, or
// columns of the key CSR).  The edge kernels process one cluster per
// workgroup and load the features of a neighbour atom once for every segment
// of the cluster that it joins, so each distinct (member atom, occurrence)
// pair of a cluster becomes one slot: slot_member = the atom, slot_edge[span] =
// for every segment of the cluster the edge joining it to that atom (-1 when
// absent).  Occurrence k > 0 exists only when one segment holds the same atom
// more than once (periodic images).  Slots are sorted by (atom, occurrence)
// and stored from the cluster's first item on (a cluster never has more slots
// than items).  A cluster with more than kMaxClusterItems items keeps one
// slot per item in CSR order (correct, without the reuse).
constexpr int kMaxClusterItems = 4096;

__global__ __launch_bounds__(256) void k_cluster_slots(const int32_t* __restrict__ seg_ptr, int n_seg, int span,
                                                       const int32_t* __restrict__ member,
                                                       const int32_t* __restrict__ item_eid,
                                                       int32_t* __restrict__ slot_member,
                                                       int32_t* __restrict__ slot_edge,
                                                       int32_t* __restrict__ n_slots) {
  __shared__ uint64_t sk[kMaxClusterItems];
  __shared__ int32_t gbase[kMaxClusterItems];
  __shared__ int32_t part[256];
  const int cl = blockIdx.x, t = threadIdx.x;
  const int s0 = cl * span, s1 = min(s0 + span, n_seg);
  const int b = seg_ptr[s0], n = seg_ptr[s1] - b;
  auto eid_of = [&](int p) { return item_eid ? item_eid[p] : p; };
  if (n > kMaxClusterItems) {
    for (int q = t; q < n; q += 256) {
      const int p = b + q;
      int sg = 0;
      while (sg + 1 < s1 - s0 && seg_ptr[s0 + sg + 1] <= p) ++sg;
      const int e = eid_of(p);
      slot_member[p] = member[e];
      for (int r = 0; r < span; ++r) slot_edge[(int64_t)p * span + r] = (r == sg) ? e : -1;
    }
    if (t == 0) n_slots[cl] = n;
    return;
  }
  // keys (member, segment, position) sorted ascending
  int p2 = 1;
  while (p2 < n) p2 <<= 1;
  for (int q = t; q < p2; q += 256) {
    uint64_t k = ~0ull;
    if (q < n) {
      const int p = b + q;
      int sg = 0;
      while (sg + 1 < s1 - s0 && seg_ptr[s0 + sg + 1] <= p) ++sg;
      k = ((uint64_t)(uint32_t)member[eid_of(p)] << 32) | ((uint64_t)sg << 16) | (uint64_t)q;
    }
    sk[q] = k;
  }
  __syncthreads();
  for (int k = 2; k <= p2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int q = t; q < p2; q += 256) {
        const int x = q ^ j;
        if (x > q) {
          const uint64_t a = sk[q], c = sk[x];
          if ((a > c) == ((q & k) == 0)) {
            sk[q] = c;
            sk[x] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  // per item: occurrence = rank among equal (member, segment); per member group: slot count
  // = 1 + max occurrence, written at the group's first item
  auto occ_of = [&](int q) {
    int o = 0;
    while (q - o - 1 >= 0 && (sk[q - o - 1] >> 16) == (sk[q] >> 16)) ++o;
    return o;
  };
  constexpr int kPer = kMaxClusterItems / 256;
  int local = 0;
  for (int z = 0; z < kPer; ++z) {
    const int q = t * kPer + z;
    int cnt = 0;
    if (q < n && (q == 0 || (sk[q - 1] >> 32) != (sk[q] >> 32))) {
      int mx = 0;
      for (int u = q; u < n && (sk[u] >> 32) == (sk[q] >> 32); ++u) mx = max(mx, occ_of(u));
      cnt = mx + 1;
    }
    gbase[q] = cnt;
    local += cnt;
  }
  part[t] = local;
  __syncthreads();
  __shared__ int total;
  if (t == 0) {
    int acc = 0;
    for (int u = 0; u < 256; ++u) {
      const int v = part[u];
      part[u] = acc;
      acc += v;
    }
    total = acc;
    n_slots[cl] = acc;
  }
  __syncthreads();
  int run = part[t];
  for (int z = 0; z < kPer; ++z) {
    const int q = t * kPer + z;
    const int v = gbase[q];
    gbase[q] = run;
    run += v;
  }
  __syncthreads();
  // group heads initialise their slots, then every item writes its edge
  for (int q = t; q < n; q += 256) {
    if (q == 0 || (sk[q - 1] >> 32) != (sk[q] >> 32)) {
      // exclusive scan: the item after a group head carries the head's base + count
      const int cnt = ((q + 1 < n) ? gbase[q + 1] : total) - gbase[q];
      for (int o = 0; o < cnt; ++o) {
        const int64_t sl = (int64_t)b + gbase[q] + o;
        slot_member[sl] = (int32_t)(sk[q] >> 32);
        for (int r = 0; r < span; ++r) slot_edge[sl * span + r] = -1;
      }
    }
  }
  __syncthreads();
  for (int q = t; q < n; q += 256) {
    int g = q;
    while (g > 0 && (sk[g - 1] >> 32) == (sk[q] >> 32)) --g;
    const int sg = (int)((sk[q] >> 16) & 0xffff);
    const int pos = (int)(sk[q] & 0xffff);
    const int64_t sl = (int64_t)b + gbase[g] + occ_of(q);
    slot_edge[sl * span + sg] = eid_of(b + pos);
  }
}

// keep the first k entries of each row (rows already sorted by distance)
__global__ void k_topk_count(const int32_t* __restrict__ row_ptr, int n_rows, int k, int32_t* __restrict__ cnt) {
  int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= n_rows) return;
  cnt[r] = min(row_ptr[r + 1] - row_ptr[r], k);
}

__global__ void k_topk_compact(const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ new_ptr, int n_rows,
                               const int32_t* __restrict__ col, const int32_t* __restrict__ shift,
                               const float* __restrict__ dvec, const float* __restrict__ dist,
                               int32_t* __restrict__ ocol, int32_t* __restrict__ oshift,
                               float* __restrict__ odv, float* __restrict__ od) {
  int r = blockIdx.x;
  int b = row_ptr[r], nb = new_ptr[r], n = new_ptr[r + 1] - nb;
  for (int t = threadIdx.x; t < n; t += blockDim.x) {
    ocol[nb + t] = col[b + t];
    oshift[nb + t] = shift[b + t];
    odv[3 * (nb + t)] = dvec[3 * (b + t)];
    odv[3 * (nb + t) + 1] = dvec[3 * (b + t) + 1];
    odv[3 * (nb + t) + 2] = dvec[3 * (b + t) + 2];
    od[nb + t] = dist[b + t];
  }
}

// LDS capacity (power of two, 64 .. kMaxSeg) of the per-segment sorts for segments of up to n items
static inline int seg_cap(int n) {
  int c = 64;
  while (c < n && c < kMaxSeg) c <<= 1;
  return c;
}
static inline size_t seg_lds_bytes(int cap) { return (size_t)cap * (sizeof(uint64_t) + sizeof(int32_t)); }

// 30-bit Morton (Z-order) key of each atom within its graph's bounding box:
// key = graph << 32 | interleave(q_x, q_y, q_z), q = clamp((pos - lo) / span * 1023, 0, 1023)
// truncated, graphs given by gid (NULL: one graph).
__device__ __forceinline__ uint64_t spread_bits10(uint64_t v) {
  v &= 0x3FF;
  v = (v | (v << 16)) & 0x030000FF;
  v = (v | (v << 8)) & 0x0300F00F;
  v = (v | (v << 4)) & 0x030C30C3;
  v = (v | (v << 2)) & 0x09249249;
  return v;
}

__global__ void k_morton_keys(const float* __restrict__ pos, const int32_t* __restrict__ gid,
                              const float* __restrict__ lo, const float* __restrict__ span, int n,
                              uint64_t* __restrict__ key) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int g = gid ? gid[i] : 0;
  uint64_t code = 0;
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    const float u = (pos[3 * i + d] - lo[3 * g + d]) / span[3 * g + d] * 1023.0f;
    code |= spread_bits10((uint64_t)fminf(fmaxf(u, 0.0f), 1023.0f)) << d;
  }
  key[i] = ((uint64_t)(uint32_t)g << 32) | code;
}

static inline unsigned blocks_for(int64_t n, int bs) {
  int64_t b = (n + bs - 1) / bs;
  return (unsigned)(b < 1 ? 1 : (b > 1048576 ? 1048576 : b));
}

// ---------------------------------------------------------------------------
// Segment metadata of an edge list in any order (COO -> CSR): entries of row r
// in ascending edge order (a stable sort by row).  Row indices outside
// [0, n_rows) are counted in *bad and left out.
__global__ void k_coo_count(const int32_t* __restrict__ row, int64_t n, int n_rows, int32_t* __restrict__ cnt,
                            int32_t* __restrict__ bad) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n) return;
  const int r = row[e];
  if (r < 0 || r >= n_rows) {
    atomicAdd(bad, 1);
    return;
  }
  atomicAdd(&cnt[r], 1);
}

__global__ void k_gather_i32(const int32_t* __restrict__ src, const int32_t* __restrict__ index, int64_t n,
                             int32_t* __restrict__ out) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n) return;
  out[p] = src[index[p]];
}

// ---------------------------------------------------------------------------
// Query -> source pairs of padded batches by direct distance evaluation (the
// reference's dense construct_radius_neighbor form): query q of graph b meets
// every one of the l2 padded source positions of b.  A pair is kept when
// min_dist <= d <= max_dist (a NaN distance fails both) and the source is
// included; each row is sorted by (distance, source slot) and cut to its k
// nearest.
__device__ __forceinline__ bool pair_dist(const e2v2_pair_plan& P, int q, int b, int k, float& d) {
#pragma clang fp contract(off)
  const float* a = P.qpos + 3 * (int64_t)q;
  const float* c = P.spos + ((int64_t)b * P.l2 + k) * 3;
  d = exact_dist(a[0] - c[0], a[1] - c[1], a[2] - c[2]);
  const bool inc = P.include == nullptr || P.include[(int64_t)b * P.l2 + k] != 0;
  return inc && d >= P.min_dist && d <= P.max_dist;
}

__global__ __launch_bounds__(64 * kNbrWaves) void k_pair_count(e2v2_pair_plan P, int32_t* __restrict__ row_count) {
  const int lane = threadIdx.x & 63;
  for (int q = blockIdx.x * kNbrWaves + (int)(threadIdx.x >> 6); q < P.n_query; q += gridDim.x * kNbrWaves) {
    const int b = P.qgraph[q];
    int c = 0;
    for (int k0 = 0; k0 < P.l2; k0 += 64) {
      const int k = k0 + lane;
      float d;
      const bool ok = k < P.l2 && pair_dist(P, q, b, k, d);
      c += __popcll(__ballot(ok));
    }
    if (lane == 0) row_count[q] = c;
  }
}

__global__ __launch_bounds__(64 * kNbrWaves) void k_pair_fill(e2v2_pair_plan P, const int32_t* __restrict__ row_ptr,
                                                             uint64_t* __restrict__ key) {
  const int lane = threadIdx.x & 63;
  for (int q = blockIdx.x * kNbrWaves + (int)(threadIdx.x >> 6); q < P.n_query; q += gridDim.x * kNbrWaves) {
    const int b = P.qgraph[q];
    int o = row_ptr[q];
    const int o_end = row_ptr[q + 1];
    for (int k0 = 0; k0 < P.l2; k0 += 64) {
      const int k = k0 + lane;
      float d = 0.f;
      const bool ok = k < P.l2 && pair_dist(P, q, b, k, d);
      const uint64_t m = __ballot(ok);
      const int p = o + lanes_below(m);
      if (ok && p < o_end) key[p] = ((uint64_t)__float_as_uint(d) << 32) | (uint64_t)(uint32_t)k;
      o += __popcll(m);
    }
  }
}

// module_utils.py:1946-1954 (kind 0, exponent 5) and :1956-1985 (kind 1, exponent 2), fp32, unfused
__device__ __forceinline__ float pair_envelope(const e2v2_pair_plan& P, float d) {
#pragma clang fp contract(off)
  if (P.poly == 0) {
    const float r = d / P.max_dist;
    if (!(r < 1.0f)) return 0.0f;
    const float r2 = r * r, r4 = r2 * r2, r5 = r4 * r;
    return 1.0f + r5 * (-21.0f + r * (35.0f + -15.0f * r));
  }
  const float lo = P.min_dist, hi = fmaxf(P.max_dist, P.min_dist + 1e-8f);
  float t = (2.0f * d - (lo + hi)) / (hi - lo);
  t = fminf(fmaxf(t, -1.0f), 1.0f);
  const float u = 1.0f - t * t;
  return u * u;
}

// One workgroup per query row: sort its keys (LDS up to cap, longer rows in place in
// global memory) and write the first new_ptr[q+1] - new_ptr[q] of them.
__global__ __launch_bounds__(64) void k_pair_emit(e2v2_pair_plan P, const int32_t* __restrict__ row_ptr,
                                                  const int32_t* __restrict__ new_ptr, uint64_t* __restrict__ key,
                                                  int cap, int64_t* __restrict__ query_idx,
                                                  int64_t* __restrict__ neighbor_idx, float* __restrict__ edge_vec,
                                                  float* __restrict__ dist, float* __restrict__ poly) {
#pragma clang fp contract(off)
  uint64_t* sk = seg_lds;
  int32_t* sv = reinterpret_cast<int32_t*>(seg_lds + cap);
  const int q = blockIdx.x;
  const int b0 = row_ptr[q], n = row_ptr[q + 1] - b0;
  const int o0 = new_ptr[q], nk = new_ptr[q + 1] - o0;
  if (n == 0 || nk == 0) return;
  const bool in_lds = n <= cap;
  if (in_lds)
    segment_sort(key, b0, n, sk, sv);
  else
    sort_global(key + b0, n);
  const int g = P.qgraph[q];
  const float* a = P.qpos + 3 * (int64_t)q;
  for (int t = threadIdx.x; t < nk; t += blockDim.x) {
    const uint64_t kv = in_lds ? sk[t] : key[b0 + t];
    const int k = (int)(uint32_t)kv;
    const float d = __uint_as_float((uint32_t)(kv >> 32));
    int64_t j = (int64_t)P.sbase[g] + k;
    if (j > (int64_t)P.n_flat - 1) j = (int64_t)P.n_flat - 1;
    const int64_t o = o0 + t;
    query_idx[o] = q;
    neighbor_idx[o] = j;
    const float* c = P.sflat + 3 * j;
    edge_vec[3 * o] = a[0] - c[0];
    edge_vec[3 * o + 1] = a[1] - c[1];
    edge_vec[3 * o + 2] = a[2] - c[2];
    dist[o] = d;
    poly[o] = pair_envelope(P, d);
  }
}

// ---------------------------------------------------------------------------
// No-allocation variant of e2v2_nbr_bin + e2v2_nbr_count: the bin workspace lives
// in this file-scope device array instead of the plan's workspace buffers.  In
// host code `scratch` only names the symbol; its device address (one copy per
// GPU) comes from hipGetSymbolAddress, taken once per device on first use.
constexpr int64_t kNoAllocAtoms = E2V2_NOALLOC_MAX_ATOMS;
constexpr int64_t kNoAllocBins = E2V2_NOALLOC_MAX_BINS;
// atom_bin [atoms] | bin_atoms [atoms] | bin_count [bins] | bin_start [bins + 1]
constexpr int64_t kScratchInts = 2 * kNoAllocAtoms + 2 * kNoAllocBins + 1;
static __device__ __align__(256) int32_t scratch[kScratchInts];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static int32_t* g_scratch_ptr[kMaxDevices] = {};

static int scratch_for_current_device(int32_t** out) {
  int dev = 0;
  E2V2_TRY_HIP(hipGetDevice(&dev));
  E2V2_REQUIRE(dev >= 0 && dev < kMaxDevices, "nbr_count_noalloc: device %d beyond the %d supported", dev,
               kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    E2V2_TRY_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    E2V2_REQUIRE(p != nullptr, "nbr_count_noalloc: no device address for the scratch array on device %d", dev);
    g_scratch_ptr[dev] = static_cast<int32_t*>(p);
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace e2v2

using namespace e2v2;

E2V2_API int e2v2_fill_i32(int32_t* p, int32_t v, int64_t n, hipStream_t s) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(k_fill_i32, dim3(blocks_for(n, 256)), dim3(256), 0, s, p, v, n);
  E2V2_LAUNCHED("k_fill_i32");
  return 0;
}

E2V2_API int e2v2_fill_f32(float* p, float v, int64_t n, hipStream_t s) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(k_fill_f32, dim3(blocks_for(n, 256)), dim3(256), 0, s, p, v, n);
  E2V2_LAUNCHED("k_fill_f32");
  return 0;
}

E2V2_API int e2v2_scan_i32(const int32_t* in, int n, int32_t* out, int32_t* stats, hipStream_t s) {
  E2V2_REQUIRE(n >= 0, "scan: negative length %d", n);
  hipLaunchKernelGGL(k_scan_i32, dim3(1), dim3(1024), 0, s, in, n, out, stats);
  E2V2_LAUNCHED("k_scan_i32");
  return 0;
}

E2V2_API int e2v2_nbr_bin(const e2v2_nbr_plan* plan, hipStream_t s) {
  const e2v2_nbr_plan& P = *plan;
  E2V2_REQUIRE(P.n_atoms >= 0 && P.n_bins > 0, "nbr_bin: bad sizes (atoms %d, bins %d)", P.n_atoms, P.n_bins);
  int rc = e2v2_fill_i32(P.bin_count, 0, P.n_bins, s);
  if (rc) return rc;
  if (P.n_atoms == 0) return e2v2_fill_i32(P.bin_start, 0, (int64_t)P.n_bins + 1, s);
  hipLaunchKernelGGL(k_bin_assign, dim3(blocks_for(P.n_atoms, 256)), dim3(256), 0, s, P);
  E2V2_LAUNCHED("k_bin_assign");
  // bin_start = exclusive scan of counts; the count buffer becomes the fill cursor
  hipLaunchKernelGGL(k_scan_i32, dim3(1), dim3(1024), 0, s, P.bin_count, P.n_bins, P.bin_start, P.stats);
  E2V2_LAUNCHED("k_scan_i32");
  rc = e2v2_fill_i32(P.bin_count, 0, P.n_bins, s);
  if (rc) return rc;
  hipLaunchKernelGGL(k_bin_fill, dim3(blocks_for(P.n_atoms, 256)), dim3(256), 0, s, P, P.bin_count);
  E2V2_LAUNCHED("k_bin_fill");
  return 0;
}

E2V2_API int e2v2_nbr_count(const e2v2_nbr_plan* plan, int32_t* row_count, int32_t* row_ptr, hipStream_t s) {
  const e2v2_nbr_plan& P = *plan;
  if (P.n_atoms > 0) {
    hipLaunchKernelGGL(k_nbr_count, dim3(blocks_for(P.n_atoms, kNbrWaves)), dim3(64 * kNbrWaves), 0, s, P,
                       row_count);
    E2V2_LAUNCHED("k_nbr_count");
  }
  hipLaunchKernelGGL(k_scan_i32, dim3(1), dim3(1024), 0, s, row_count, P.n_atoms, row_ptr, P.stats);
  E2V2_LAUNCHED("k_scan_i32");
  return 0;
}

E2V2_API int e2v2_nbr_fill(const e2v2_nbr_plan* plan, const int32_t* row_ptr, int64_t n_edges, int max_row,
                           int32_t* tmp_col, int32_t* tmp_shift, float* tmp_dvec, float* tmp_dist, uint64_t* tmp_key,
                           int32_t* col, int32_t* shift, float* dvec, float* dist, hipStream_t s) {
  const e2v2_nbr_plan& P = *plan;
  E2V2_REQUIRE(max_row <= kMaxSeg, "nbr_fill: a row has %d neighbours; the per-row sort supports at most %d",
               max_row, kMaxSeg);
  if (P.n_atoms == 0 || n_edges == 0) return 0;
  hipLaunchKernelGGL(k_nbr_fill, dim3(blocks_for(P.n_atoms, kNbrWaves)), dim3(64 * kNbrWaves), 0, s, P, row_ptr,
                     tmp_col, tmp_shift, tmp_dvec, tmp_dist, tmp_key);
  E2V2_LAUNCHED("k_nbr_fill");
  const int cap = seg_cap(max_row);
  hipLaunchKernelGGL(k_sort_rows, dim3(P.n_atoms), dim3(64), seg_lds_bytes(cap), s, row_ptr, tmp_key, tmp_col,
                     tmp_shift, tmp_dvec, tmp_dist, col, shift, dvec, dist, cap);
  E2V2_LAUNCHED("k_sort_rows");
  return 0;
}

E2V2_API int e2v2_nbr_cap(int32_t* row_ptr, int n_rows, int64_t cap_edges, int cap_row, int32_t* stats,
                          hipStream_t s) {
  E2V2_REQUIRE(row_ptr && stats && n_rows >= 0, "nbr_cap: null row_ptr / stats or negative row count");
  E2V2_REQUIRE(cap_edges >= 0 && cap_edges < (1ll << 31) && cap_row > 0 && cap_row <= kMaxSeg,
               "nbr_cap: capacity %lld edges / %d per row outside the supported range", (long long)cap_edges, cap_row);
  hipLaunchKernelGGL(k_cap_rows, dim3(blocks_for(n_rows + 1, 256)), dim3(256), 0, s, row_ptr, n_rows, cap_edges,
                     cap_row, stats);
  E2V2_LAUNCHED("k_cap_rows");
  return 0;
}

E2V2_API int e2v2_nbr_topk(const int32_t* row_ptr, int n_rows, int k, int32_t* cnt, int32_t* new_ptr, int32_t* stats,
                           const int32_t* col, const int32_t* shift, const float* dvec, const float* dist,
                           int32_t* ocol, int32_t* oshift, float* odv, float* od, int phase, hipStream_t s) {
  if (phase == 0) {
    if (n_rows > 0) {
      hipLaunchKernelGGL(k_topk_count, dim3(blocks_for(n_rows, 256)), dim3(256), 0, s, row_ptr, n_rows, k, cnt);
      E2V2_LAUNCHED("k_topk_count");
    }
    hipLaunchKernelGGL(k_scan_i32, dim3(1), dim3(1024), 0, s, cnt, n_rows, new_ptr, stats);
    E2V2_LAUNCHED("k_scan_i32");
    return 0;
  }
  if (n_rows == 0) return 0;
  hipLaunchKernelGGL(k_topk_compact, dim3(n_rows), dim3(128), 0, s, row_ptr, new_ptr, n_rows, col, shift, dvec, dist,
                     ocol, oshift, odv, od);
  E2V2_LAUNCHED("k_topk_compact");
  return 0;
}

E2V2_API int e2v2_morton_keys(const float* pos, const int32_t* gid, const float* lo, const float* span, int n,
                              int64_t* key, hipStream_t s) {
  E2V2_REQUIRE(n >= 0, "morton_keys: negative count %d", n);
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_morton_keys, dim3(blocks_for(n, 256)), dim3(256), 0, s, pos, gid, lo, span, n,
                     reinterpret_cast<uint64_t*>(key));
  E2V2_LAUNCHED("k_morton_keys");
  return 0;
}

E2V2_API int e2v2_cluster_slots(const int32_t* seg_ptr, int32_t n_seg, const int32_t* member,
                                const int32_t* item_eid, int32_t span, int32_t* slot_member, int32_t* slot_edge,
                                int32_t* n_slots, hipStream_t s) {
  E2V2_REQUIRE(span >= 1 && span <= 16, "cluster_slots: span must be 1..16, got %d", span);
  if (n_seg <= 0) return 0;
  const int n_cl = (n_seg + span - 1) / span;
  hipLaunchKernelGGL(k_cluster_slots, dim3(n_cl), dim3(256), 0, s, seg_ptr, n_seg, span, member, item_eid,
                     slot_member, slot_edge, n_slots);
  E2V2_LAUNCHED("k_cluster_slots");
  return 0;
}

E2V2_API int e2v2_csr_transpose(const int32_t* row_ptr, const int32_t* col, int n_rows, int n_cols, int64_t n_edges,
                                int32_t* edge_row, int32_t* key_cnt, int32_t* key_ptr, int32_t* stats,
                                uint64_t* tmp_key, int32_t* key_eid, int phase, hipStream_t s) {
  // phase 0: edge_row, column counts and key_ptr (stats = {E, max column}, informational)
  // phase 1: fill and sort each column by edge id (any column length)
  if (phase == 0) {
    if (n_rows > 0 && n_edges > 0) {
      hipLaunchKernelGGL(k_edge_rows, dim3(blocks_for(n_rows, 256)), dim3(256), 0, s, row_ptr, n_rows, edge_row);
      E2V2_LAUNCHED("k_edge_rows");
    }
    int rc = e2v2_fill_i32(key_cnt, 0, n_cols, s);
    if (rc) return rc;
    if (n_edges > 0) {
      hipLaunchKernelGGL(k_col_count, dim3(blocks_for(n_edges, 256)), dim3(256), 0, s, col, n_edges,
                         row_ptr + n_rows, key_cnt);
      E2V2_LAUNCHED("k_col_count");
    }
    hipLaunchKernelGGL(k_scan_i32, dim3(1), dim3(1024), 0, s, key_cnt, n_cols, key_ptr, stats);
    E2V2_LAUNCHED("k_scan_i32");
    return 0;
  }
  if (n_edges == 0) return 0;
  int rc = e2v2_fill_i32(key_cnt, 0, n_cols, s);
  if (rc) return rc;
  hipLaunchKernelGGL(k_col_fill, dim3(blocks_for(n_edges, 256)), dim3(256), 0, s, col, n_edges, row_ptr + n_rows,
                     key_ptr, key_cnt, tmp_key);
  E2V2_LAUNCHED("k_col_fill");
  // columns of up to 256 edges sort in LDS (at liquid density and a 6 A cutoff a column
  // holds about 90), longer ones in place in global memory
  const int cap = 256;
  hipLaunchKernelGGL(k_sort_cols, dim3(n_cols), dim3(64), seg_lds_bytes(cap), s, key_ptr, tmp_key, key_eid, cap);
  E2V2_LAUNCHED("k_sort_cols");
  return 0;
}

E2V2_API int e2v2_nbr_count_noalloc(const e2v2_nbr_plan* plan, int32_t* row_count, int32_t* row_ptr,
                                    int32_t* stats_out, hipStream_t s) {
  E2V2_REQUIRE(plan && row_ptr && stats_out && (row_count || plan->n_atoms == 0),
               "nbr_count_noalloc: plan, row_count, row_ptr and stats_out are required");
  const e2v2_nbr_plan& P0 = *plan;
  E2V2_REQUIRE(P0.n_atoms >= 0 && P0.n_atoms <= kNoAllocAtoms && P0.n_bins > 0 && P0.n_bins <= kNoAllocBins,
               "nbr_count_noalloc: %d atoms / %d bins exceed the static scratch (at most %lld atoms, %lld bins)",
               P0.n_atoms, P0.n_bins, (long long)kNoAllocAtoms, (long long)kNoAllocBins);
  int32_t* sc = nullptr;
  if (int rc = scratch_for_current_device(&sc)) return rc;
  e2v2_nbr_plan P = P0;
  P.atom_bin = sc;
  P.bin_atoms = sc + kNoAllocAtoms;
  P.bin_count = sc + 2 * kNoAllocAtoms;
  P.bin_start = P.bin_count + kNoAllocBins;
  P.stats = stats_out;
  // the outside flag accumulates by atomic OR: start from zero (a fill kernel, not a memset)
  if (int rc = e2v2_fill_i32(stats_out, 0, 3, s)) return rc;
  if (int rc = e2v2_nbr_bin(&P, s)) return rc;
  return e2v2_nbr_count(&P, row_count, row_ptr, s);
}

E2V2_API int e2v2_segment_metadata(const int32_t* row_index, const int32_t* other_index, int64_t n_edges, int n_rows,
                                   int32_t* row_ptr, int32_t* col_index, int32_t* alpha_index, int32_t* cnt,
                                   uint64_t* tmp_key, int32_t* stats, int phase, hipStream_t s) {
  E2V2_REQUIRE(n_edges >= 0 && n_edges < (1ll << 31) && n_rows >= 0,
               "segment_metadata: bad sizes (%lld edges, %d rows)", (long long)n_edges, n_rows);
  E2V2_REQUIRE(row_ptr && stats && (cnt || n_rows == 0), "segment_metadata: null row_ptr / stats / cnt");
  if (phase == 0) {
    if (int rc = e2v2_fill_i32(cnt, 0, n_rows, s)) return rc;
    if (int rc = e2v2_fill_i32(stats + 2, 0, 1, s)) return rc;
    if (n_edges > 0) {
      E2V2_REQUIRE(row_index, "segment_metadata: null row_index");
      hipLaunchKernelGGL(k_coo_count, dim3(blocks_for(n_edges, 256)), dim3(256), 0, s, row_index, n_edges, n_rows,
                         cnt, stats + 2);
      E2V2_LAUNCHED("k_coo_count");
    }
    hipLaunchKernelGGL(k_scan_i32, dim3(1), dim3(1024), 0, s, cnt, n_rows, row_ptr, stats);
    E2V2_LAUNCHED("k_scan_i32");
    return 0;
  }
  // phase 1: only after phase 0 reported no out-of-range row (stats[2] == 0)
  if (n_edges == 0) return 0;
  E2V2_REQUIRE(n_rows > 0, "segment_metadata: %lld edges but no row", (long long)n_edges);
  E2V2_REQUIRE(row_index && other_index && col_index && alpha_index && tmp_key, "segment_metadata: null pointer");
  if (int rc = e2v2_fill_i32(cnt, 0, n_rows, s)) return rc;
  hipLaunchKernelGGL(k_col_fill, dim3(blocks_for(n_edges, 256)), dim3(256), 0, s, row_index, n_edges,
                     (const int32_t*)nullptr, row_ptr, cnt,
                     tmp_key);
  E2V2_LAUNCHED("k_col_fill");
  const int cap = 256;
  hipLaunchKernelGGL(k_sort_cols, dim3(n_rows), dim3(64), seg_lds_bytes(cap), s, row_ptr, tmp_key, alpha_index, cap);
  E2V2_LAUNCHED("k_sort_cols");
  hipLaunchKernelGGL(k_gather_i32, dim3(blocks_for(n_edges, 256)), dim3(256), 0, s, other_index, alpha_index,
                     n_edges, col_index);
  E2V2_LAUNCHED("k_gather_i32");
  return 0;
}

static int check_pair_plan(const e2v2_pair_plan* P) {
  E2V2_REQUIRE(P != nullptr, "pair search: null plan");
  E2V2_REQUIRE(P->n_query >= 0 && P->n_graphs >= 0 && P->l2 >= 0 && P->n_flat >= 0,
               "pair search: negative size (queries %d, graphs %d, l2 %d, flat %d)", P->n_query, P->n_graphs, P->l2,
               P->n_flat);
  E2V2_REQUIRE(P->poly == 0 || P->poly == 1, "pair search: envelope kind %d (0 polynomial, 1 bell)", P->poly);
  E2V2_REQUIRE(P->n_query == 0 || (P->qpos && P->qgraph && P->n_graphs > 0), "pair search: null query arrays");
  E2V2_REQUIRE(P->l2 == 0 || P->spos, "pair search: null source positions");
  return 0;
}

E2V2_API int e2v2_pair_count(const e2v2_pair_plan* plan, int32_t* row_count, int32_t* row_ptr, int32_t* stats,
                             hipStream_t s) {
  if (int rc = check_pair_plan(plan)) return rc;
  E2V2_REQUIRE(row_ptr && stats && (row_count || plan->n_query == 0), "pair_count: null output");
  const e2v2_pair_plan& P = *plan;
  if (P.n_query > 0) {
    hipLaunchKernelGGL(k_pair_count, dim3(blocks_for(P.n_query, kNbrWaves)), dim3(64 * kNbrWaves), 0, s, P,
                       row_count);
    E2V2_LAUNCHED("k_pair_count");
  }
  hipLaunchKernelGGL(k_scan_i32, dim3(1), dim3(1024), 0, s, row_count, P.n_query, row_ptr, stats);
  E2V2_LAUNCHED("k_scan_i32");
  return 0;
}

E2V2_API int e2v2_pair_emit(const e2v2_pair_plan* plan, const int32_t* row_ptr, int64_t n_pairs, int max_row,
                            const int32_t* new_ptr, uint64_t* tmp_key, int64_t* query_idx, int64_t* neighbor_idx,
                            float* edge_vec, float* dist, float* poly, hipStream_t s) {
  if (int rc = check_pair_plan(plan)) return rc;
  const e2v2_pair_plan& P = *plan;
  E2V2_REQUIRE(n_pairs >= 0 && n_pairs < (1ll << 31) && max_row >= 0, "pair_emit: bad sizes (%lld pairs, row %d)",
               (long long)n_pairs, max_row);
  if (n_pairs == 0 || P.n_query == 0) return 0;
  E2V2_REQUIRE(P.n_flat > 0 && P.sflat && P.sbase, "pair_emit: pairs found but no flattened source nodes");
  E2V2_REQUIRE(row_ptr && new_ptr && tmp_key && query_idx && neighbor_idx && edge_vec && dist && poly,
               "pair_emit: null pointer");
  hipLaunchKernelGGL(k_pair_fill, dim3(blocks_for(P.n_query, kNbrWaves)), dim3(64 * kNbrWaves), 0, s, P, row_ptr,
                     tmp_key);
  E2V2_LAUNCHED("k_pair_fill");
  const int cap = seg_cap(max_row);
  hipLaunchKernelGGL(k_pair_emit, dim3(P.n_query), dim3(64), seg_lds_bytes(cap), s, P, row_ptr, new_ptr, tmp_key,
                     cap, query_idx, neighbor_idx, edge_vec, dist, poly);
  E2V2_LAUNCHED("k_pair_emit");
  return 0;
}
